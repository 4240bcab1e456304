"""Top-p (nucleus) sampling on the GPU against the oracle.

The GPU reproduces the reference's sequential fp32 normaliser and cumulative
sums exactly (integer-state emulation), so every row's id and p(chosen) must
be identical to the oracle's -- boundary rows included.  The oracle's
boundary classification (draw or cut-off mass within 1e-5 of a CDF edge) is
still computed and printed, and the stated 1e-5 bar on p is asserted too."""
import numpy as np
import pytest

import pz_oracle as po
import pzsample as pz
import workloads as wl
from conftest import to_dev

pytestmark = pytest.mark.gpu

P_TOL = 1e-5


def orc(p):
    return po.params(p.temperature, p.top_k, p.top_p, p.rep_penalty, p.presence_penalty,
                     p.frequency_penalty)


def same_p(a, b):
    return (a == b) | (np.isnan(a) & np.isnan(b))


def oracle_rows(x, params, u, hist=None, temp_mode=pz.PZ_TEMP_MUL_RECIP, threads=16):
    """The oracle over row blocks on several threads (its buffers are per
    thread), for batches whose rows take seconds on one core."""
    from concurrent.futures import ThreadPoolExecutor
    B = x.shape[0]
    n = max(1, min(threads, B))
    cuts = [B * i // n for i in range(n + 1)]
    op = [orc(q) for q in params]

    def part(i):
        lo, hi = cuts[i], cuts[i + 1]
        return po.sample_batch(x[lo:hi], op if len(op) == 1 else op[lo:hi],
                               u=None if u is None else u[lo:hi],
                               hist=None if hist is None else hist[lo:hi], temp_mode=temp_mode)
    with ThreadPoolExecutor(n) as ex:
        parts = list(ex.map(part, range(n)))
    return tuple(np.concatenate([q[i] for q in parts]) for i in range(4))


def check(torch, x, params, u, hist=None, temp_mode=pz.PZ_TEMP_MUL_RECIP, label="", ld=None):
    B, V = x.shape
    print(f"case {label} B={B} V={V}", flush=True)
    if ld is not None and ld > V:
        full = np.zeros((B, ld), np.float32)
        full[:, :V] = x
        d_x = to_dev(torch, full)
    else:
        ld = V
        d_x = to_dev(torch, np.ascontiguousarray(x))
    H = hist.shape[1] if hist is not None else 0
    d_h = to_dev(torch, np.ascontiguousarray(hist)) if hist is not None else None
    with pz.Sampler(B, V, max_hist=max(H, 1), temp_mode=temp_mode) as s:
        ids, p = s.sample(d_x, B, V, ld, params, u=u, d_hist=d_h, H=H, want_p=True)
    want, pw, dd, dc = oracle_rows(x, params, u, hist=hist, temp_mode=temp_mode)
    boundary = (dd < 1e-5) | (dc < 1e-5)
    bad = ids != want
    print(f"  rows={B} boundary={int(boundary.sum())} mismatches={int(bad.sum())}", flush=True)
    assert not bad.any(), (label, np.nonzero(bad)[0][:8], ids[bad][:8], want[bad][:8],
                           boundary[bad][:8])
    assert same_p(p, pw).all(), (label, np.nonzero(~same_p(p, pw))[0][:8])
    fin = np.isfinite(pw)
    assert np.all(np.abs(p[fin] - pw[fin]) <= P_TOL)
    return ids, p, want


def test_c2_full_size(torch_cuda):
    """64 x 128256, N(0, 2^2) + 5 spikes per row, T 0.7, top-p 0.9."""
    w = wl.build_c2()
    check(torch_cuda, w["logits"], w["params"], w["u"], label="c2")


def test_c2_more_rows(torch_cuda):
    w = wl.build_c2(B=256, seed=0xC2 + 7)
    check(torch_cuda, w["logits"], w["params"], w["u"], label="c2 x256")


def test_c2_batch_1024(torch_cuda):
    """The top of the metric's batch range: 1024 x 128256 in one call (the
    front launch runs 8192 workgroups in several rounds, each row's slices
    meeting through the workspace); every row against the oracle."""
    w = wl.build_c2(B=1024, seed=0xC2 + 11)
    check(torch_cuda, w["logits"], w["params"], w["u"], label="c2 x1024")


@pytest.mark.parametrize("V", [1, 3, 5, 1000, 4099, 49152, 151936, 200000])
@pytest.mark.parametrize("top_p", [0.5, 0.9, 0.99])
def test_sizes(torch_cuda, V, top_p):
    B = 6
    x = pz.synth_normal(B, V, 2.5, 300 + V)
    u = pz.synth_draws(B, 17 + V)
    check(torch_cuda, x, [pz.row_params(temperature=0.8, top_p=top_p)], u,
          label=f"V={V} p={top_p}")


def test_flat_and_broad_rows_use_the_fallback(torch_cuda):
    """Nuclei larger than the LDS buffer: all-equal logits (every p ties, id
    order decides), a very broad row at top_p 0.999, a two-level row."""
    B, V = 4, 128256
    x = pz.synth_normal(B, V, 0.3, 41)
    x[0, :] = 1.5
    x[2, ::2] = 3.0
    x[3, :1000] = 9.0
    u = pz.synth_draws(B, 42)
    check(torch_cuda, x, [pz.row_params(temperature=1.0, top_p=0.999)], u, label="broad")
    check(torch_cuda, x, [pz.row_params(temperature=1.0, top_p=0.9)], u, label="broad 0.9")


def test_selected_bins_beyond_the_gather(torch_cuda):
    """Rows 377, 796 and 977 of the 1024-row c2 pool: the nucleus bins picked
    from the e histogram hold 8.3K-8.8K candidates (nuclei of 7.3K-7.7K),
    past the 8192-key gather, so the fallback sorts the gated candidates;
    two ordinary rows beside them."""
    w = wl.build_c2(B=1024)
    pick = [377, 796, 977, 0, 1]
    x = np.ascontiguousarray(w["logits"][pick])
    u = np.ascontiguousarray(w["u"][pick])
    check(torch_cuda, x, w["params"], u, label="c2 pool rows past the gather")


def test_degenerate_rows(torch_cuda):
    B, V = 8, 5000
    x = pz.synth_normal(B, V, 2.0, 51)
    x[0, 0] = np.nan             # max is NaN -> argmax -> 0
    x[1, 7] = np.nan             # NaN elsewhere is never a candidate
    x[2, :] = -np.inf            # max -inf -> first element
    x[3, 100] = np.inf           # max +inf -> first +inf
    x[3, 200] = np.inf
    x[4, :] = -np.inf
    x[4, 3] = np.nan
    x[5, :] = 0.0
    x[5, 0] = -0.0
    x[6, :] = np.round(x[6, :])  # heavy ties
    x[7, :] = -1e30
    x[7, 10] = -1e30 + 1e24
    u = pz.synth_draws(B, 52)
    ids, p, want = check(torch_cuda, x, [pz.row_params(temperature=1.0, top_p=0.9)], u,
                         label="degenerate")
    assert ids[0] == 0 and ids[2] == 0 and ids[3] == 100


def test_penalties_then_top_p(torch_cuda):
    B, V = 32, 32000
    x = pz.synth_normal(B, V, 3.0, 61)
    hist = pz.synth_zipf_ids(B, 128, V, 1.1, 62)
    u = pz.synth_draws(B, 63)
    for prm in (pz.row_params(temperature=0.9, top_p=0.8, rep_penalty=1.3),
                pz.row_params(temperature=1.2, top_p=0.95, presence_penalty=0.5,
                              frequency_penalty=0.3)):
        check(torch_cuda, x, [prm], u, hist=hist, label="penalties")


def test_temperature_division_form(torch_cuda):
    B, V = 16, 49152
    x = pz.synth_normal(B, V, 3.0, 71)
    u = pz.synth_draws(B, 72)
    for mode in (pz.PZ_TEMP_MUL_RECIP, pz.PZ_TEMP_DIV):
        check(torch_cuda, x, [pz.row_params(temperature=0.7, top_p=0.9)], u, temp_mode=mode,
              label=f"temp form {mode}")


def test_vocab_guard_takes_argmax(torch_cuda):
    """V > 200000: the reference's static buffer guard returns argmax of the
    tempered row (top_p.c:33-34)."""
    B, V = 4, 200001
    x = pz.synth_normal(B, V, 2.0, 81)
    x[1, 5] = x[1, 9] = 50.0
    u = pz.synth_draws(B, 82)
    ids, p, want = check(torch_cuda, x, [pz.row_params(temperature=0.7, top_p=0.9)], u,
                         label="guard")
    assert ids[1] == 5 and (p == 1.0).all()


def test_uniform_edges(torch_cuda):
    B, V = 4, 20000
    x = pz.synth_normal(B, V, 2.0, 91)
    for uval in (0.0, 1.0, 0.9999999):
        u = np.full(B, uval, np.float32)
        check(torch_cuda, x, [pz.row_params(temperature=1.0, top_p=0.9)], u, label=f"u={uval}")


def test_strided_rows_and_mixed_modes(torch_cuda):
    B, V = 24, 12345
    x = pz.synth_normal(B, V, 2.0, 101)
    u = pz.synth_draws(B, 102)
    prms = []
    for b in range(B):
        prms.append([pz.row_params(temperature=0.0),
                     pz.row_params(temperature=0.9, top_p=0.85),
                     pz.row_params(temperature=1.0, top_k=30, top_p=0.9)][b % 3])
    check(torch_cuda, x, prms, u, label="mixed strided", ld=12347)


@pytest.mark.parametrize("top_p", [0.3, 0.9, 1.0])
def test_short_lists(torch_cuda, top_p):
    """Rows with 1 to 72 candidates (every other logit 30 below the maximum,
    outside the reference's max - 20 window): lists of one wave and just
    past it, the cumulative cut inside the list or (top_p 1.0) never
    reached, draws at u = 0 and u = 1 among them."""
    B, V = 72, 5000
    rng = np.random.default_rng(0x5107 + int(top_p * 10))
    x = np.full((B, V), -30.0, np.float32)
    for b in range(B):
        k = b + 1
        pos = rng.choice(V, size=k, replace=False)
        x[b, pos] = rng.normal(0.0, 1.5, size=k).astype(np.float32)
    u = pz.synth_draws(B, 0x5108)
    u[0], u[1], u[70] = 0.0, 1.0, 1.0
    check(torch_cuda, x, [pz.row_params(temperature=1.0, top_p=top_p)], u,
          label=f"short lists p={top_p}")


def test_cutoff_inside_the_first_segment_of_a_long_list(torch_cuda):
    """A long gathered list (3000 candidates spread over the nucleus bins
    behind 200 large ones) whose cumulative reaches top_p within its first
    256 sorted keys (row 0: about 33 past the large ones) or well past them
    (row 1), so the cut-off walk stops inside the list's first segment,
    whose sum comes with the walk's set-up, or after it."""
    B, V = 2, 128256
    rng = np.random.default_rng(77)
    x = np.full((B, V), -30.0, np.float32)
    for b, gap in ((0, 4.9), (1, 4.5)):  # cut-offs near 233 and 956
        big = rng.choice(V, 200, replace=False)
        rest = np.setdiff1d(np.arange(V), big)
        small = rng.choice(rest, 3000, replace=False)
        x[b, small] = (1.0 + rng.uniform(-0.3, 0.3, 3000)).astype(np.float32)
        x[b, big] = (1.0 + gap + rng.uniform(-1e-3, 1e-3, 200)).astype(np.float32)
    u = pz.synth_draws(B, 78)
    check(torch_cuda, x, [pz.row_params(temperature=1.0, top_p=0.9)], u, label="long list")
    check(torch_cuda, x, [pz.row_params(temperature=1.0, top_p=0.9)], np.array([0.999, 0.0], np.float32),
          label="long list, u at the ends")
