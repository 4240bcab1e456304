"""pz_sample_step: decode steps with per-row xorshift64* states on the device
and the EOS check.  After every step the ids, each row's RNG state and the
EOS flags must equal the oracle's (orc_sample_step, whose state handling is
pinned against the reference's own sample_top_p / sample_top_k in
tests/test_oracle_step.py)."""
import numpy as np
import pytest

import pz_oracle as po
import pzsample as pz
import workloads as wl
from conftest import to_dev

pytestmark = pytest.mark.gpu


def orc_params(p):
    return po.params(temperature=p.temperature, top_k=p.top_k, top_p=p.top_p,
                     rep_penalty=p.rep_penalty, presence_penalty=p.presence_penalty,
                     frequency_penalty=p.frequency_penalty)


def run_steps(torch, s, batches, params, seeds, eos, hist=None, n_steps=None, workers=8,
              label=""):
    """Runs n_steps steps, step t on batches[t % len(batches)]; compares
    ids, states and EOS flags with the oracle after each step."""
    n_steps = len(batches) if n_steps is None else n_steps
    B, V = batches[0].shape
    d_batches = [to_dev(torch, x) for x in batches]
    H = 0
    d_hist = None
    if hist is not None:
        H = hist.shape[-1]
    d_state = to_dev(torch, seeds.view(np.int64)).view(torch.int64)
    d_ids = torch.full((B,), -5, dtype=torch.int32, device="cuda")
    d_eos = torch.full((B,), 7, dtype=torch.uint8, device="cuda")
    want_state = seeds.copy()
    oparams = [orc_params(p) for p in params]
    s.set_eos(eos)
    draws = 0
    eos_hits = 0
    for t in range(n_steps):
        x = batches[t % len(batches)]
        h = None
        if hist is not None:
            h = hist[t % len(hist)] if hist.ndim == 3 else hist
            d_hist = to_dev(torch, np.ascontiguousarray(h))
        torch.cuda.synchronize()
        s.sample_step(d_batches[t % len(batches)], B, V, V, params, d_state, d_ids, d_eos=d_eos,
                      d_hist=d_hist, H=H)
        s.sync()
        ids, flags, drew = po.sample_step(x, oparams, want_state, hist=h, eos=eos,
                                          workers=workers)
        got_ids = d_ids.cpu().numpy()
        got_state = d_state.cpu().numpy().view(np.uint64)
        got_eos = d_eos.cpu().numpy()
        assert (got_ids == ids).all(), (label, t, np.nonzero(got_ids != ids)[0][:8])
        assert (got_state == want_state).all(), (label, t, np.nonzero(got_state != want_state)[0])
        assert (got_eos == flags).all(), (label, t)
        draws += int(drew.sum())
        eos_hits += int(flags.sum())
    print(f"{label}: {n_steps} steps x {B} rows, {draws} draws, {eos_hits} EOS flags", flush=True)
    return draws, eos_hits


def eos_from_trace(x_rows, prm, seed, hist, picks):
    """EOS ids that the run will meet: the oracle's ids at a few steps."""
    st = np.array([seed], np.uint64)
    out = []
    for t in range(max(picks) + 1):
        ids, _, _ = po.sample_step(x_rows[t:t + 1], [prm], st, hist=hist[t:t + 1])
        if t in picks:
            out.append(int(ids[0]))
    return out


def test_c1_500_steps_one_row_per_call(torch_cuda):
    w = wl.build_c1()
    x, hist = w["logits"], w["hist"]
    prm = w["params"][0]
    print("case step c1 500 steps", flush=True)
    eos = eos_from_trace(x, orc_params(prm), 42, hist, {5, 77, 312}) + [49151, 0]
    batches = [x[t:t + 1] for t in range(x.shape[0])]
    with pz.Sampler(1, x.shape[1], max_hist=hist.shape[1]) as s:
        draws, hits = run_steps(torch_cuda, s, batches, [prm], np.array([42], np.uint64), eos,
                                hist=hist[:, None, :], workers=1, label="c1")
    assert draws == 500  # the chain draws every step
    assert hits >= 3


def test_c2_64_steps(torch_cuda):
    w = wl.build_c2()
    x = w["logits"]
    # four distinct batches (the base one and row rotations of it); each row
    # walks its own state
    batches = [np.ascontiguousarray(np.roll(x, r, axis=0)) for r in (0, 1, 2, 3)]
    seeds = (np.arange(64, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15)) | np.uint64(1)
    print("case step c2 64 steps", flush=True)
    with pz.Sampler(64, x.shape[1]) as s:
        draws, _ = run_steps(torch_cuda, s, batches, w["params"], seeds, [5, 17], n_steps=64,
                             label="c2")
    assert draws == 64 * 64


def test_mixed_rows_that_do_not_draw(torch_cuda):
    """Per-row modes with rows that must not draw: greedy, top-p with a NaN
    first value (argmax before the draw), plus categorical, top-k and chain
    rows with penalties; 32 steps over 4 batches."""
    B, V, H = 8, 4096, 32
    rng = np.random.default_rng(0xE05)
    batches = []
    for k in range(4):
        x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
        x[2, 0] = np.nan           # top-p row: never draws
        if k % 2:
            x[6, 0] = np.nan       # top-p row: draws on even batches only
        batches.append(x)
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    hist[3, :4] = 0
    params = [pz.row_params(temperature=0.0, rep_penalty=1.3),
              pz.row_params(temperature=0.8, top_p=0.9),
              pz.row_params(temperature=0.8, top_p=0.9),
              pz.row_params(temperature=0.7, top_p=0.9, presence_penalty=0.5,
                            frequency_penalty=0.3),
              pz.row_params(temperature=0.9),
              pz.row_params(temperature=0.8, top_k=40),
              pz.row_params(temperature=0.8, top_p=0.9),
              pz.row_params(temperature=0.8, top_k=50, top_p=0.9, rep_penalty=1.1)]
    seeds = np.arange(1, B + 1, dtype=np.uint64) * np.uint64(1000003)
    # the greedy row's id on the first batch is an EOS id: flagged every 4th step
    g, _ = po.sample_row(batches[0][0], orc_params(params[0]), hist=hist[0])
    print("case step mixed 32 steps", flush=True)
    with pz.Sampler(B, V, max_hist=H) as s:
        draws, hits = run_steps(torch_cuda, s, batches, params, seeds, [3, 4095, g], hist=hist,
                                n_steps=32, label="mixed")
    # rows 0 and 2 never draw, row 6 on half the steps, the other five always
    assert draws == 32 * 5 + 16
    assert hits >= 8


def test_top_p_above_vocabulary_guard_does_not_draw(torch_cuda):
    B, V = 2, 200001
    rng = np.random.default_rng(0xE06)
    batches = [(rng.standard_normal((B, V)) * 2).astype(np.float32) for _ in range(2)]
    seeds = np.array([7, 8], np.uint64)
    print("case step guard", flush=True)
    with pz.Sampler(B, V) as s:
        draws, _ = run_steps(torch_cuda, s, batches, [pz.row_params(temperature=0.7, top_p=0.9)],
                             seeds, [], n_steps=4, label="guard")
    assert draws == 0
