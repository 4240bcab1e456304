"""Plain categorical draw (softmax + ascending-id CDF, generate.c:157-169) on
the GPU against the oracle: the normaliser and the CDF are reproduced with
the reference's sequential fp32 rounding, so ids and p(chosen) must be
identical on every row."""
import numpy as np
import pytest

import pz_oracle as po
import pzsample as pz
from conftest import to_dev

pytestmark = pytest.mark.gpu


def orc(p):
    return po.params(p.temperature, p.top_k, p.top_p, p.rep_penalty, p.presence_penalty,
                     p.frequency_penalty)


def check(torch, x, params, u, hist=None, temp_mode=pz.PZ_TEMP_MUL_RECIP, label=""):
    B, V = x.shape
    print(f"case {label} B={B} V={V}", flush=True)
    d_x = to_dev(torch, np.ascontiguousarray(x))
    H = hist.shape[1] if hist is not None else 0
    d_h = to_dev(torch, np.ascontiguousarray(hist)) if hist is not None else None
    with pz.Sampler(B, V, max_hist=max(H, 1), temp_mode=temp_mode) as s:
        ids, p = s.sample(d_x, B, V, V, params, u=u, d_hist=d_h, H=H, want_p=True)
    want, pw, dd, _ = po.sample_batch(x, [orc(q) for q in params], u=u, hist=hist,
                                      temp_mode=temp_mode)
    bad = ids != want
    print(f"  boundary={int((dd < 1e-5).sum())} mismatches={int(bad.sum())}", flush=True)
    assert not bad.any(), (label, np.nonzero(bad)[0][:8], ids[bad][:8], want[bad][:8])
    same = (p == pw) | (np.isnan(p) & np.isnan(pw))
    assert same.all(), (label, np.nonzero(~same)[0][:8])
    return ids, p


def test_full_vocab_batch(torch_cuda):
    B, V = 256, 128256
    x = pz.synth_normal(B, V, 3.0, 0xCA7)
    u = pz.synth_draws(B, 0xCA8)
    check(torch_cuda, x, [pz.row_params(temperature=1.0)], u, label="256x128256")


@pytest.mark.parametrize("V", [1, 2, 7, 4096, 4097, 49152, 151936, 262144])
def test_sizes(torch_cuda, V):
    B = 5
    x = pz.synth_normal(B, V, 2.0, 500 + V)
    u = pz.synth_draws(B, 600 + V)
    check(torch_cuda, x, [pz.row_params(temperature=0.8)], u, label=f"V={V}")


def test_top_p_one_and_zero_take_the_plain_path(torch_cuda):
    B, V = 8, 32000
    x = pz.synth_normal(B, V, 2.0, 77)
    u = pz.synth_draws(B, 78)
    for tp in (1.0, 0.0, 1.5):
        check(torch_cuda, x, [pz.row_params(temperature=0.9, top_p=tp)], u, label=f"top_p={tp}")


def test_early_stop_with_many_specials_after(torch_cuda):
    """Rows whose mass grows geometrically with the id (x_i = i ln2 / 1024:
    the CDF doubles every 1024 ids) drawn with tiny uniforms: the draw stops
    about 30 binade crossings before the row's end, more special segments
    after the stop than the walk's ring holds.  The walk's producers must
    stop with it (every kernel ends) and the ids match the oracle."""
    B, V = 4, 128256
    i = np.arange(V, dtype=np.float64)
    x = np.empty((B, V), np.float32)
    x[0] = (i * np.log(2.0) / 1024).astype(np.float32)
    x[1] = x[0]
    x[2] = (i * np.log(2.0) / 256).astype(np.float32)
    x[3] = x[0]
    u = np.array([2.0 ** -30, 2.0 ** -20, 1e-9, 0.5], np.float32)
    ids, _ = check(torch_cuda, x, [pz.row_params(temperature=1.0)], u, label="ramps")
    assert ids[0] < V - 25 * 1024 and ids[2] < V - 25 * 256, ids


def test_degenerate_rows(torch_cuda):
    B, V = 7, 3000
    x = pz.synth_normal(B, V, 2.0, 88)
    x[0, 0] = np.nan            # NaN max -> V-1
    x[1, 17] = np.nan           # NaN anywhere -> sum NaN -> V-1
    x[2, 5] = np.inf            # +inf max -> NaN term -> V-1
    x[3, :] = -np.inf           # -inf max -> V-1
    x[4, :] = 0.0               # uniform
    x[5, :] = -1e4              # very negative, finite
    x[5, 1234] = -1e4 + 30
    x[6, ::3] = -np.inf         # -inf entries contribute 0
    u = pz.synth_draws(B, 89)
    ids, _ = check(torch_cuda, x, [pz.row_params(temperature=1.0)], u, label="degenerate")
    assert ids[0] == ids[1] == ids[2] == ids[3] == V - 1


def test_uniform_edges(torch_cuda):
    B, V = 4, 10000
    x = pz.synth_normal(B, V, 3.0, 99)
    for uval in (0.0, 1.0, 0.99999994, 0.5):
        check(torch_cuda, x, [pz.row_params(temperature=1.0)], np.full(B, uval, np.float32),
              label=f"u={uval}")


def test_penalties_and_temperature_forms(torch_cuda):
    B, V = 32, 50000
    x = pz.synth_normal(B, V, 3.0, 111)
    hist = pz.synth_uniform_ids(B, 200, V, 112)
    u = pz.synth_draws(B, 113)
    for mode in (pz.PZ_TEMP_MUL_RECIP, pz.PZ_TEMP_DIV):
        check(torch_cuda, x, [pz.row_params(temperature=0.7, rep_penalty=1.2,
                                             presence_penalty=0.3, frequency_penalty=0.2)],
              u, hist=hist, temp_mode=mode, label=f"pen temp {mode}")


@pytest.mark.parametrize("B", [1, 64, 1024])
def test_default_chain_batches(torch_cuda, B):
    """The HTTP default (T 1.0, top-p 1.0: softmax + CDF draw) over spiked
    N(0, 2^2) rows at vocab 128256, from batch 1 to 1024 (the bench's sweep):
    every row against the oracle (on several threads: its buffers are per
    thread)."""
    from concurrent.futures import ThreadPoolExecutor
    import workloads as wl
    w = wl.build_cat(B=B, seed=0xCA + B)
    x, params, u = w["logits"], w["params"], w["u"]
    print(f"case categorical default chain B={B}", flush=True)
    d_x = to_dev(torch_cuda, x)
    with pz.Sampler(B, x.shape[1]) as s:
        ids, p = s.sample(d_x, B, x.shape[1], x.shape[1], params, u=u, want_p=True)
    n = min(16, B)
    cuts = [B * i // n for i in range(n + 1)]
    with ThreadPoolExecutor(n) as ex:
        parts = list(ex.map(lambda i: po.sample_batch(x[cuts[i]:cuts[i + 1]], [orc(params[0])],
                                                      u=u[cuts[i]:cuts[i + 1]]), range(n)))
    want = np.concatenate([q[0] for q in parts])
    pw = np.concatenate([q[1] for q in parts])
    assert (ids == want).all(), (np.nonzero(ids != want)[0][:8], ids[:4], want[:4])
    assert (p == pw).all()
