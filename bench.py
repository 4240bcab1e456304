"""Benchmark of the batched token sampler on one MI355X: ONE JSON line.

Headline (`value`): batch 1024 x vocab 128256 fp32 logits ~ N(0, 3^2),
repetition penalty 1.15 over a per-row history of 256 uniform ids, greedy
argmax with lowest-id tie-break.  A step is one synchronous pz_sample_batch
call (the kernels plus the ids' return to the host); logits and histories are
resident in HBM before timing starts.

The same line carries
  workloads    c1 one sequence x 49152, repetition + top-k 40 + top-p 0.95,
                  one row per call (the reference's loop), 500 fresh rows
               c2 64 x 128256, temperature 0.7 + top-p 0.9, 5 spikes per row
               c3 256 x 151936, presence/frequency + top-k 20 + top-p 0.8
               c5 speculative verification, 32 sequences x 4 drafts x 128256
  batch_sweep  greedy (as the headline), top-p (as c2) and the plain
               categorical draw (c2's logits at T 1.0, top-p 1.0: the HTTP
               default) at vocab 128256, batch 1, 8, 64, 256, 1024
  attention    the reference softmax over attention scores (the tn_softmax of
               attention.c:210), 32 heads x valid context 128, 4096, 32768
  lm_head      the bf16 LM head producing the logits (parallel_matmul_bf16,
               vocab 128256 x hidden 2560), alone and with greedy argmax fused
               into its epilogue, batch 1, 8, 32
each with rows/s (wall clock of synchronous calls), the kernels' time per
launch from HIP events on the sampler's own stream, algorithmic GB/s and the
fraction of the 8 TB/s HBM peak, and parity with the oracle (ids; draws
within 1e-5 of a CDF boundary counted apart).  The timed loops rotate over
enough distinct batches that one pass reads more than the 256 MB Infinity
Cache holds, so the GB/s figures are HBM figures.

CPU baseline: the oracle (oracle/pz_oracle.c, the clean-room restatement of
the reference sampler) built on this host with the reference's release flags
(-O3 -march=native), on a bounded sample of each workload: one thread
(`cpu_baseline`, the reference's own threading) and N threads
(`cpu_baseline_ncore`, N stated).  The temperature form follows the host:
x * (1/T) where the CPU has AVX-512 (the reference's build there), else x / T;
the GPU sampler uses the same form.
"""
import argparse
import json
import os
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "project-zero_amd"))

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20
BOUNDARY = 1e-5
METRIC = "sampled rows/s at vocab 128256, batch 1-1024; achieved HBM GB/s vs peak"

WORKLOAD_TEXT = {
    "c4": "repetition 1.15 (H=256 uniform ids) + greedy argmax, batch 1024 x vocab 128256, "
          "N(0,3^2) logits",
    "c2": "temperature 0.7 + top-p 0.9, batch 64 x vocab 128256, N(0,2^2) + 5 spikes/row",
    "c3": "presence 0.5 / frequency 0.3 (512 Zipf(1.1) ids) + top-k 20 + top-p 0.8, "
          "batch 256 x vocab 151936, 2.5*Gumbel logits",
    "c1": "repetition 1.1 (H=64) + T 0.8 + top-k 40 + top-p 0.95, one sequence x vocab 49152, "
          "one row per call",
    "c5": "speculative verification, 32 sequences x 4 drafts x vocab 128256 (+ bonus row), "
          "tau 0.8",
}
KERNELS = {
    "c4": "k_greedy",
    "c2": "k_topp_front + k_topp_walkf + k_topp_fallback",
    "c3": "k_topk",
    "c1": "k_topk",
    "c5": "k_spec_stat + k_spec_rec + k_spec_walk + k_spec_vest + "
          "k_spec_vrec + k_spec_vwalk",
}
SWEEP_B = (1, 8, 64, 256, 1024)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="all",
                    choices=["all", "sweep", "attn", "lmhead"] + sorted(WORKLOAD_TEXT),
                    help="all (default): the headline, every workload and the sweep; "
                         "one name: that workload alone (profiling runs)")
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baseline and the parity checks")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--sweep", default="all",
                    help="comma-separated sweep kinds (greedy, top_p, categorical) or all")
    ap.add_argument("--batches", default=None,
                    help="comma-separated sweep batch sizes (default 1,8,64,256,1024)")
    ap.add_argument("--cpu-seconds", type=float, default=3.0,
                    help="CPU time of each baseline sample (per thread count)")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---------------------------------------------------------------------------
# the oracle: CPU baseline and checker
# ---------------------------------------------------------------------------
class Cpu:
    """The oracle built for this host, its thread count and temperature form."""

    def __init__(self, enabled):
        self.enabled = enabled
        self.build = "not built"
        self.po = None
        self.threads = max(1, min(16, os.cpu_count() or 1))
        if not enabled:
            return
        out = os.path.join(tempfile.mkdtemp(prefix="pzorc_"), "libpzoracle.so")
        r = subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "native",
                            f"NATIVE_OUT={out}"], capture_output=True, text=True)
        if r.returncode == 0 and os.path.exists(out):
            os.environ["PZ_ORACLE_LIB"] = out
            self.build = "gcc -std=c99 -O3 -march=native -ffp-contract=off (built on this host)"
        else:
            log(f"native oracle build failed, using the shipped x86-64-v3 build: {r.stderr[-300:]}")
            self.build = "gcc -std=c99 -O3 -march=x86-64-v3 -ffp-contract=off (shipped build)"
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import pz_oracle as po
        self.po = po
        self.avx512 = po.host_has_avx512()

    def temp_mode(self):
        import pzsample as pz
        if self.po is None:
            return pz.PZ_TEMP_MUL_RECIP
        return pz.PZ_TEMP_MUL_RECIP if self.avx512 else pz.PZ_TEMP_DIV

    def oparams(self, params):
        po = self.po
        return [po.params(p.temperature, p.top_k, p.top_p, p.rep_penalty, p.presence_penalty,
                          p.frequency_penalty) for p in params]

    def rows(self, x, params, u, hist, lo, hi):
        return self.po.sample_batch(x[lo:hi], self.oparams(params),
                                    u=None if u is None else u[lo:hi],
                                    hist=None if hist is None else hist[lo:hi],
                                    temp_mode=self.temp_mode())

    def parity(self, x, params, u, hist, gpu_ids, n_rows=None):
        """Oracle ids of the first n_rows rows (threads over row blocks) and
        the comparison, boundary rows apart."""
        import numpy as np
        from concurrent.futures import ThreadPoolExecutor
        B = x.shape[0] if n_rows is None else n_rows
        n = min(self.threads, B)
        cuts = [B * i // n for i in range(n + 1)]
        with ThreadPoolExecutor(n) as ex:
            parts = list(ex.map(lambda i: self.rows(x, params, u, hist, cuts[i], cuts[i + 1]),
                                range(n)))
        ids = np.concatenate([p[0] for p in parts])
        dd = np.concatenate([p[2] for p in parts])
        dc = np.concatenate([p[3] for p in parts])
        bnd = np.minimum(dd, dc) < BOUNDARY
        bad = ids != np.asarray(gpu_ids[:B])
        return {"rows": int(B), "boundary_rows": int(bnd.sum()),
                "mismatches_nonboundary": int((bad & ~bnd).sum()),
                "mismatches_boundary": int((bad & bnd).sum())}

    def ref_baseline(self, x, params, draw_seed, gpu_ids, budget):
        """The reference's own sampler (oracle/_ref: src/sampling/*.c
        compiled from their sources) on rows that are exactly one reference
        call -- apply_temperature + sample_top_p, each row's RNG state seeded
        as the workload's uniforms were (so it draws the same u) -- timed on
        one thread over a bounded sample; its ids are compared with the
        GPU's.  None when the reference build is absent."""
        import ctypes
        import numpy as np
        po = self.po
        ref = po.ref(self.avx512) if po is not None else None
        if ref is None or len(params) != 1 or params[0].top_k > 0:
            return None
        p = params[0]
        if not (0.0 < p.top_p < 1.0) or p.temperature < 1e-6 or p.rep_penalty != 1.0 or \
                p.presence_penalty != 0.0 or p.frequency_penalty != 0.0:
            return None
        B, V = x.shape
        work = np.empty(V, np.float32)
        st = ctypes.c_ulonglong(0)
        ids = []
        t0 = time.perf_counter()
        rows = 0
        while rows < B and (rows < 4 or time.perf_counter() - t0 < budget):
            work[:] = x[rows]
            ref.rng_seed(ctypes.byref(st), (int(draw_seed) ^ (rows + 1)) & ((1 << 64) - 1))
            ref.apply_temperature(work.ctypes.data, V, float(p.temperature))
            ids.append(ref.sample_top_p(work.ctypes.data, V, float(p.top_p), ctypes.byref(st)))
            rows += 1
        dt = time.perf_counter() - t0
        match = int((np.array(ids) == np.asarray(gpu_ids[:rows])).sum())
        return {"value": rows / dt, "unit": "rows/s", "cores": 1, "kind": "reference",
                "sample": f"the first {rows} of {B} rows ({dt:.1f} s): apply_temperature + "
                          "sample_top_p per row, row copied first (temperature works in place)",
                "build": "gcc -std=c99 -O3 -march=x86-64-v4 (or -v3 without AVX-512) of the "
                         "reference's src/sampling/*.c and src/math/softmax.c (oracle/Makefile ref)",
                "ids_equal_to_gpu": f"{match} of {rows}"}

    def baseline(self, x, params, u, hist, budget, unit="rows/s"):
        """Rows/s of the oracle on a bounded sample of the batch: one
        thread, then self.threads threads each sampling the same rows."""
        from concurrent.futures import ThreadPoolExecutor
        B = x.shape[0]
        probe = min(B, 4)
        t0 = time.perf_counter()
        self.rows(x, params, u, hist, 0, probe)
        per_row = (time.perf_counter() - t0) / probe
        rows = int(max(1, min(B, budget / max(per_row, 1e-9))))
        reps = max(1, int(budget / max(per_row * rows, 1e-9))) if rows == B else 1
        t0 = time.perf_counter()
        for _ in range(reps):
            self.rows(x, params, u, hist, 0, rows)
        dt1 = time.perf_counter() - t0
        what = f"{reps} x the full {B}-row batch" if rows == B else f"the first {rows} of {B} rows"
        one = {"value": rows * reps / dt1, "unit": unit, "cores": 1, "kind": "port",
               "sample": f"{what} ({rows * reps} rows, {dt1:.1f} s)", "build": self.build}
        N = self.threads
        t0 = time.perf_counter()
        with ThreadPoolExecutor(N) as ex:
            list(ex.map(lambda _: self.rows(x, params, u, hist, 0, rows), range(N)))
        dtn = time.perf_counter() - t0
        ncore = {"value": N * rows / dtn, "unit": unit, "cores": N, "kind": "port",
                 "sample": f"{N} threads x the first {rows} rows ({N * rows} rows, {dtn:.1f} s)",
                 "build": self.build}
        return one, ncore


# ---------------------------------------------------------------------------
# GPU timing
# ---------------------------------------------------------------------------
def events_ms(torch, stream_ptr, launches, per_call=False):
    """Average time per launch of the kernels the callables in `launches`
    enqueue (one launch each), from HIP events on the sampler's stream: one
    pair around the whole back-to-back sequence, or with per_call (calls that
    wait for their own results) one pair around each call's kernels."""
    ext = torch.cuda.ExternalStream(stream_ptr)
    launches[0]()
    torch.cuda.synchronize()
    if not per_call:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(ext)
        for f in launches:
            f()
        e1.record(ext)
        e1.synchronize()
        return e0.elapsed_time(e1) / len(launches)
    total = 0.0
    for f in launches:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(ext)
        f()
        e1.record(ext)
        e1.synchronize()
        total += e0.elapsed_time(e1)
    return total / len(launches)


def rotation(batch_bytes):
    """Distinct batches the timed loop cycles through: more than the
    Infinity Cache holds."""
    return max(1, -(-int(1.2 * MALL_BYTES) // int(batch_bytes)))


def roofline(bytes_per_launch, kern_ms, traffic, kernel):
    achieved = bytes_per_launch / (kern_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
            "traffic_source": "profiles/traffic.json (rocprofv3 --pmc DRAM requests of the same "
                              "kernels on this workload, calibrated on a copy)" if traffic
                              else None, "kernel": kernel,
            "kernel_us": kern_ms * 1e3, "algorithmic_bytes_per_launch": int(bytes_per_launch)}


def traffic_for(workload):
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            t = json.load(f)
        return t.get(workload, {}).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def run_batched(args, torch, cpu, name):
    """c2, c3, c4: one synchronous call per step over rotating batches."""
    import numpy as np
    import pzsample as pz
    import workloads as wl
    build = wl.BUILDERS[name]
    w0 = build()
    B, V = w0["logits"].shape
    nrot = rotation(B * w0["bytes_per_row"])
    log(f"{name}: {nrot} distinct batches of {B} x {V}")
    ws = [w0] + [build(seed=wl.SEEDS[name] + 977 * k) for k in range(1, nrot)]
    H = w0["hist"].shape[1] if w0["hist"] is not None else 0
    dev = torch.device("cuda:0")
    t_x = [torch.from_numpy(w["logits"]).to(dev) for w in ws]
    t_h = [torch.from_numpy(w["hist"]).to(dev) if H else None for w in ws]
    t_u = [torch.from_numpy(w["u"]).to(dev) if w["u"] is not None else None for w in ws]
    t_ids = torch.empty(B, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    params = w0["params"]
    s = pz.Sampler(B, V, max_hist=max(H, 1), temp_mode=cpu.temp_mode())
    # arguments marshalled once (pzsample Sampler.caller): a step costs the
    # library call, as a C serving loop pays it
    fast = s.caller(B, V, V, params, H=H)
    d_x = [t.data_ptr() for t in t_x]
    d_h = [t.data_ptr() if t is not None else None for t in t_h]

    def step(k):
        return fast(d_x[k], ws[k]["u"], d_h[k])

    for t in range(args.warmup):
        step(t % nrot)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(args.steps):
        step(t % nrot)
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ids0 = step(0).copy()

    def launch(k):
        return lambda: s.sample_async(t_x[k], B, V, V, params, t_u[k], t_ids, d_hist=t_h[k], H=H)
    kern = events_ms(torch, s.stream, [launch(t % nrot) for t in range(max(args.steps, 20))])
    s.close()
    bpl = w0["bytes_per_row"] * B
    r = {"workload": WORKLOAD_TEXT[name], "batch": B, "vocab": V, "hist": H,
         "distinct_batches": nrot, "ms_per_step": ms, "value": B / (ms * 1e-3), "unit": "rows/s",
         "roofline": roofline(bpl, kern, traffic_for(name), KERNELS[name])}
    if cpu.enabled:
        log(f"{name}: parity and cpu baseline")
        r["parity"] = cpu.parity(w0["logits"], params, w0["u"], w0["hist"], ids0)
        r["cpu_baseline"], r["cpu_baseline_ncore"] = cpu.baseline(
            w0["logits"], params, w0["u"], w0["hist"], args.cpu_seconds)
        if "draw_seed" in w0:
            rb = cpu.ref_baseline(w0["logits"], params, w0["draw_seed"], ids0, args.cpu_seconds)
            if rb is not None:
                # the reference's own code is the baseline where one call is the chain
                r["cpu_baseline_port"] = r["cpu_baseline"]
                r["cpu_baseline"] = rb
    del t_x, t_h, t_u
    torch.cuda.empty_cache()
    return r


def run_c1(args, torch, cpu):
    """One row per call, the reference's loop: 500 fresh rows, each call
    synchronous (the id returns to the host before the next).  The calls go
    through a caller with its arguments marshalled once (pzsample
    Sampler.caller), so the time is the library's, as a C loop would see
    it."""
    import numpy as np
    import pzsample as pz
    import workloads as wl
    w = wl.build_c1()
    x, hist, u = w["logits"], w["hist"], w["u"]
    R, V = x.shape
    H = hist.shape[1]
    dev = torch.device("cuda:0")
    t_x = torch.from_numpy(x).to(dev)
    t_h = torch.from_numpy(hist).to(dev)
    t_u = torch.from_numpy(u).to(dev)
    t_ids = torch.empty(R, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    params = w["params"]
    s = pz.Sampler(1, V, max_hist=H, temp_mode=cpu.temp_mode())
    dx, dh, du, di = t_x.data_ptr(), t_h.data_ptr(), t_u.data_ptr(), t_ids.data_ptr()
    ids = np.empty(R, np.int32)

    fast = s.caller(1, V, V, params, H=H)

    def call(r):
        return fast(dx + 4 * V * r, u[r:r + 1], dh + 4 * H * r)[0]

    for r in range(min(args.warmup * 10, R)):
        call(r)
    t0 = time.perf_counter()
    for r in range(R):
        ids[r] = call(r)
    ms = (time.perf_counter() - t0) * 1e3 / R

    def launch(r):
        return lambda: s.sample_async(dx + 4 * V * r, 1, V, V, params, du + 4 * r, di + 4 * r,
                                      d_hist=dh + 4 * H * r, H=H)
    kern = events_ms(torch, s.stream, [launch(r) for r in range(R)])
    s.close()
    r = {"workload": WORKLOAD_TEXT["c1"], "batch": 1, "vocab": V, "hist": H, "calls": R,
         "ms_per_step": ms, "value": 1.0 / (ms * 1e-3), "unit": "rows/s",
         "roofline": roofline(w["bytes_per_row"], kern, traffic_for("c1"), KERNELS["c1"])}
    if cpu.enabled:
        log("c1: parity and cpu baseline")
        r["parity"] = cpu.parity(x, params, u, hist, ids)
        r["cpu_baseline"], r["cpu_baseline_ncore"] = cpu.baseline(x, params, u, hist,
                                                                  args.cpu_seconds)
        r["gpu_call_over_cpu_row"] = r["cpu_baseline"]["value"] / r["value"]
    return r


def run_c5(args, torch, cpu):
    import numpy as np
    import pzsample as pz
    import workloads as wl
    w0 = wl.build_c5()
    B, K, V = w0["B"], w0["K"], w0["V"]
    nrot = rotation(w0["bytes_per_seq"] * B)
    log(f"c5: {nrot} distinct batches")
    ws = [w0] + [wl.build_c5(seed=wl.SEEDS["c5"] + 977 * k) for k in range(1, nrot)]
    dev = torch.device("cuda:0")
    t_t = [torch.from_numpy(w["target"]).to(dev) for w in ws]
    t_d = [torch.from_numpy(w["draft"]).to(dev) for w in ws]
    torch.cuda.synchronize()
    s = pz.Sampler(B, V, temp_mode=cpu.temp_mode())

    def call(k):
        w = ws[k]
        return s.spec_verify(t_t[k], t_d[k], B, K, V, V, w["has_bonus"], w["tau"],
                             w["draft_ids"], w["u_acc"], w["u_res"])

    for t in range(args.warmup):
        call(t % nrot)
    t0 = time.perf_counter()
    for t in range(args.steps):
        call(t % nrot)
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    acc0, out0 = call(0)
    # the kernels' time: the same verifications enqueued back to back through
    # the device-resident entry point (inputs already in HBM), bracketed by
    # events on the sampler's stream
    d_in = [(torch.from_numpy(np.ascontiguousarray(w["draft_ids"], np.int32)).to(dev),
             torch.from_numpy(np.ascontiguousarray(w["u_acc"], np.float32)).to(dev),
             torch.from_numpy(np.ascontiguousarray(w["u_res"], np.float32)).to(dev)) for w in ws]
    d_acc = torch.empty(B, dtype=torch.int32, device=dev)
    d_out = torch.empty((B, K + 1), dtype=torch.int32, device=dev)
    torch.cuda.synchronize()

    def launch(k):
        w = ws[k]
        s.spec_verify_async(t_t[k], t_d[k], B, K, V, V, w["has_bonus"], w["tau"], *d_in[k],
                            d_acc, d_out)

    kern = events_ms(torch, s.stream,
                     [(lambda k=t % nrot: launch(k)) for t in range(max(args.steps, 20))])
    s.close()
    bpl = w0["bytes_per_seq"] * B
    r = {"workload": WORKLOAD_TEXT["c5"], "batch": B, "drafts": K, "vocab": V,
         "distinct_batches": nrot, "ms_per_step": ms, "value": B / (ms * 1e-3),
         "unit": "sequences/s", "roofline": roofline(bpl, kern, traffic_for("c5"), KERNELS["c5"])}
    if cpu.enabled:
        log("c5: parity and cpu baseline")
        po = cpu.po
        tm = cpu.temp_mode()
        acc, out, dist = po.spec_verify(w0["target"], w0["draft"], K, w0["has_bonus"],
                                        w0["tau"], w0["draft_ids"], w0["u_acc"], w0["u_res"],
                                        temp_mode=tm)
        bnd = dist < BOUNDARY
        bad = (acc != acc0) | (out != out0).any(axis=1)
        r["parity"] = {"sequences": B, "boundary_sequences": int(bnd.sum()),
                       "mismatches_nonboundary": int((bad & ~bnd).sum()),
                       "mismatches_boundary": int((bad & bnd).sum())}
        from concurrent.futures import ThreadPoolExecutor

        def verify(lo, hi):
            return po.spec_verify(w0["target"][lo:hi], w0["draft"][lo:hi], K, w0["has_bonus"],
                                  w0["tau"], w0["draft_ids"][lo:hi], w0["u_acc"][lo:hi],
                                  w0["u_res"][lo:hi], temp_mode=tm)
        t1 = time.perf_counter()
        verify(0, 1)
        per_seq = time.perf_counter() - t1
        nseq = int(max(1, min(B, args.cpu_seconds / max(per_seq, 1e-9))))
        t0 = time.perf_counter()
        verify(0, nseq)
        dt1 = time.perf_counter() - t0
        N = cpu.threads
        t0 = time.perf_counter()
        with ThreadPoolExecutor(N) as ex:
            list(ex.map(lambda _: verify(0, nseq), range(N)))
        dtn = time.perf_counter() - t0
        r["cpu_baseline"] = {"value": nseq / dt1, "unit": "sequences/s", "cores": 1,
                             "kind": "port", "sample": f"the first {nseq} of {B} sequences "
                             f"({dt1:.1f} s)", "build": cpu.build}
        r["cpu_baseline_ncore"] = {"value": N * nseq / dtn, "unit": "sequences/s", "cores": N,
                                   "kind": "port", "sample": f"{N} threads x the first {nseq} "
                                   f"sequences ({dtn:.1f} s)", "build": cpu.build}
    del t_t, t_d
    torch.cuda.empty_cache()
    return r


def run_sweep(args, torch, cpu):
    """Greedy (headline chain), top-p (c2 chain) and the categorical draw at
    vocab 128256 over a 1024-row pool (525 MB, beyond the Infinity Cache):
    step t of batch B reads rows [tB mod 1024, +B)."""
    import numpy as np
    import pzsample as pz
    import workloads as wl
    V, P = 128256, 1024
    out = {"vocab": V, "pool_rows": P, "greedy": [], "top_p": [], "categorical": []}
    dev = torch.device("cuda:0")
    kinds = (("greedy", wl.build_c4), ("top_p", wl.build_c2), ("categorical", wl.build_cat))
    for kind, build in kinds:
        if args.sweep != "all" and kind not in args.sweep.split(","):
            continue
        w = build(B=P, V=V)
        x, hist, u = w["logits"], w["hist"], w["u"]
        H = hist.shape[1] if hist is not None else 0
        t_x = torch.from_numpy(x).to(dev)
        t_h = torch.from_numpy(hist).to(dev) if H else None
        t_u = torch.from_numpy(u).to(dev) if u is not None else None
        t_ids = torch.empty(P, dtype=torch.int32, device=dev)
        torch.cuda.synchronize()
        params = w["params"]
        for B in (SWEEP_B if not args.batches else [int(b) for b in args.batches.split(",")]):
            s = pz.Sampler(B, V, max_hist=max(H, 1), temp_mode=cpu.temp_mode())
            steps = 100 if B <= 64 else (40 if B <= 256 else 20)
            dx = t_x.data_ptr()
            dh = t_h.data_ptr() if H else None
            du = t_u.data_ptr() if t_u is not None else None

            def off(t):
                return (t * B) % P

            def call(t):
                o = off(t)
                return s.sample(dx + 4 * V * o, B, V, V, params,
                                u=None if u is None else u[o:o + B],
                                d_hist=None if dh is None else dh + 4 * H * o, H=H)[0]
            for t in range(3):
                call(t)
            t0 = time.perf_counter()
            for t in range(steps):
                call(t)
            ms = (time.perf_counter() - t0) * 1e3 / steps
            ids0 = call(0).copy()

            def launch(t):
                o = off(t)
                return lambda: s.sample_async(dx + 4 * V * o, B, V, V, params,
                                              None if du is None else du + 4 * o,
                                              t_ids.data_ptr(),
                                              d_hist=None if dh is None else dh + 4 * H * o, H=H)
            kern = events_ms(torch, s.stream, [launch(t) for t in range(steps)])
            s.close()
            gbs = B * w["bytes_per_row"] / (kern * 1e-3) / 1e9
            e = {"batch": B, "rows_per_s": B / (ms * 1e-3), "ms_per_step": ms,
                 "kernel_us": kern * 1e3, "achieved_gbs": gbs, "frac": gbs / HBM_PEAK_GBS}
            if cpu.enabled:
                e["parity"] = cpu.parity(x, params, u, hist, ids0, n_rows=min(B, 64))
            out[kind].append(e)
            log(f"sweep {kind} B={B}: {e['rows_per_s']:.0f} rows/s, kernels {kern * 1e3:.1f} us, "
                f"{gbs:.0f} GB/s")
        del t_x, t_h, t_u
        torch.cuda.empty_cache()
    return out


def run_attention(args, torch, cpu):
    """pz_attn_softmax over [32 heads, ctx] N(0, 3^2) scores, ctx rotating
    over distinct score blocks past the Infinity Cache; bytes per launch =
    one read and one write of every score."""
    import ctypes
    import numpy as np
    import pzsample as pz
    heads = 32
    out = {"heads": heads, "entries": []}
    dev = torch.device("cuda:0")
    s = pz.Sampler(1, 16)
    for ctx in (128, 4096, 32768):
        blk = heads * ctx * 4
        nrot = rotation(2 * blk)
        rng = np.random.default_rng(ctx)
        x = (rng.standard_normal((nrot * heads, ctx)) * 3.0).astype(np.float32)
        t_x = torch.from_numpy(x).to(dev)
        t_o = torch.empty_like(t_x)
        torch.cuda.synchronize()
        dx, do = t_x.data_ptr(), t_o.data_ptr()

        def launch(t):
            k = (t % nrot) * heads
            return lambda: s.lib.pz_attn_softmax(s.h, dx + 4 * ctx * k, ctx, do + 4 * ctx * k,
                                                 ctx, heads, ctx, None)
        steps = 200 if ctx <= 4096 else 50
        kern = events_ms(torch, s.stream, [launch(t) for t in range(steps)])
        gbs = 2 * blk / (kern * 1e-3) / 1e9
        e = {"ctx": ctx, "kernel_us": kern * 1e3, "achieved_gbs": gbs, "frac": gbs / HBM_PEAK_GBS,
             "distinct_blocks": nrot,
             "kernel": ("k_attn_wave" if ctx <= 1024 else "k_attn_row" if ctx <= 8192 else
                        "k_attn_stat + k_attn_rec + k_attn_walk + k_attn_write (row split)")}
        if cpu.enabled:
            s.sync()
            got = t_o[:heads].cpu().numpy()
            want = x[:heads].copy()
            o = cpu.po.oracle()
            for r in range(heads):
                o.orc_softmax(want[r].ctypes.data_as(ctypes.c_void_p), ctx)
            e["parity"] = {"rows": heads, "rows_not_bit_identical":
                           int((got.view(np.uint32) != want.view(np.uint32)).any(axis=1).sum())}
        out["entries"].append(e)
        log(f"attention ctx={ctx}: {kern * 1e3:.1f} us, {gbs:.0f} GB/s")
        del t_x, t_o
        torch.cuda.empty_cache()
    s.close()
    return out


def run_lm_head(args, torch, cpu):
    """pz_lm_head_bf16 and pz_lm_head_argmax_bf16 at vocab 128256 x hidden
    2560 (656 MB of bf16 weights: every launch streams them from HBM).
    Bytes per launch: the weights once per weight pass, the activations, and
    (unfused) the logits written."""
    import numpy as np
    import pzsample as pz
    V, n = 128256, 2560
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(0x1E0)
    # bf16 bit patterns of small positive weights
    w = torch.from_numpy(rng.integers(0x3c00, 0x3d00, (V, n), dtype=np.uint16).view(np.int16)).to(dev)
    out = {"vocab": V, "hidden": n, "weight_bytes": V * n * 2, "entries": []}
    s = pz.Sampler(32, V)
    for B in (1, 8, 32):
        x = torch.from_numpy(rng.standard_normal((B, n), dtype=np.float32)).to(dev)
        logits = torch.empty((B, V), dtype=torch.float32, device=dev)
        ids = torch.empty(B, dtype=torch.int32, device=dev)
        torch.cuda.synchronize()
        dw, dx, dl, di = w.data_ptr(), x.data_ptr(), logits.data_ptr(), ids.data_ptr()
        steps = 30
        t_un = events_ms(torch, s.stream, [lambda: s.lib.pz_lm_head_bf16(
            s.h, dw, V, n, dx, B, n, dl, V)] * steps)
        t_fu = events_ms(torch, s.stream, [lambda: s.lib.pz_lm_head_argmax_bf16(
            s.h, dw, V, n, dx, B, n, di)] * steps)
        # batch 4 and up: the matrix-core kernel, one weight pass per 32 rows;
        # below, the vector kernel's single tile
        passes = -(-B // 32) if B >= 4 else 1
        b_un = passes * V * n * 2 + B * n * 4 + B * V * 4
        b_fu = passes * V * n * 2 + B * n * 4 + B * 4
        e = {"batch": B, "weight_passes": passes,
             "engine": "bf16 MFMA, activations in three bf16 parts" if B >= 4 else "fp32 FMA",
             "unfused_us": t_un * 1e3, "unfused_gbs": b_un / (t_un * 1e-3) / 1e9,
             "fused_us": t_fu * 1e3, "fused_gbs": b_fu / (t_fu * 1e-3) / 1e9}
        e["unfused_frac"] = e["unfused_gbs"] / HBM_PEAK_GBS
        e["fused_frac"] = e["fused_gbs"] / HBM_PEAK_GBS
        if cpu.enabled:
            s.sync()
            lg = logits.cpu().numpy()
            o = cpu.po.oracle()
            want = [o.orc_argmax(np.ascontiguousarray(r).ctypes.data_as(cpu.po._P), V) for r in lg]
            e["fused_ids_equal_argmax_of_unfused_logits"] = bool(
                (ids.cpu().numpy() == np.array(want)).all())
        out["entries"].append(e)
        log(f"lm head B={B}: unfused {t_un * 1e3:.1f} us ({e['unfused_gbs']:.0f} GB/s), fused "
            f"{t_fu * 1e3:.1f} us ({e['fused_gbs']:.0f} GB/s)")
        del x, logits, ids
    s.close()
    del w
    torch.cuda.empty_cache()
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU (one process, one device); "
                                   "rows shard across GPUs with no exchange, so no multi-GPU "
                                   "figure is produced: run --gpus 1"}))
        sys.exit(2)
    import torch

    cpu = Cpu(not args.no_cpu)
    if args.workload == "attn":
        print(json.dumps({"attention": run_attention(args, torch, cpu)}), flush=True)
        return
    if args.workload == "lmhead":
        print(json.dumps({"lm_head": run_lm_head(args, torch, cpu)}), flush=True)
        return
    head = "c4" if args.workload in ("all", "sweep") else args.workload
    runners = {"c1": run_c1, "c5": run_c5}
    log(f"headline {head}")
    h = runners.get(head, lambda a, t, c: run_batched(a, t, c, head))(args, torch, cpu)
    log(f"{head}: step {h['ms_per_step'] * 1e3:.1f} us, kernels "
        f"{h['roofline']['kernel_us']:.1f} us, frac {h['roofline']['frac']:.3f}")
    config = {"workload": h["workload"], "batch": h["batch"], "vocab": h["vocab"]}
    for k in ("hist", "drafts", "distinct_batches", "calls"):
        if k in h:
            config[k] = h[k]
    line = {
        "metric": METRIC,
        "value": h["value"],
        "unit": h["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": h["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded generators in project-zero_amd/synth)",
        "config": config,
        "roofline": h["roofline"],
    }
    for k in ("cpu_baseline", "cpu_baseline_ncore", "parity"):
        if k in h:
            line[k] = h[k]
    if cpu.enabled:
        line["temperature_form"] = "x*(1/T)" if cpu.avx512 else "x/T"
    if args.workload == "all":
        line["workloads"] = {}
        for name in ("c1", "c2", "c3", "c5"):
            log(f"workload {name}")
            r = runners.get(name, lambda a, t, c, n=name: run_batched(a, t, c, n))(args, torch,
                                                                                   cpu)
            line["workloads"][name] = r
            log(f"{name}: step {r['ms_per_step'] * 1e3:.1f} us, kernels "
                f"{r['roofline']['kernel_us']:.1f} us, frac {r['roofline']['frac']:.3f}")
    if args.workload in ("all", "sweep") and not args.no_sweep:
        line["batch_sweep"] = run_sweep(args, torch, cpu)
    if args.workload == "all":
        line["attention"] = run_attention(args, torch, cpu)
        line["lm_head"] = run_lm_head(args, torch, cpu)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
