"""LM head on the device (pz_lm_head_bf16) and its fused greedy epilogue
(pz_lm_head_argmax_bf16).

Logits: against the exact product (float64 of the same bf16 weights and fp32
activations), within the fp32 summation bound the header states:
|gpu - exact| <= n * 2^-24 * sum_j |w_ij x_bj| (any order of n fp32 adds and
products is inside it).  Fused ids: bit for bit the reference argmax
(orc_argmax, argmax.c:3-13) of the unfused kernel's logits, and the ids the
batched sampler's greedy path gives on those logits."""
import numpy as np
import pytest

import pz_oracle as po
import pzsample as pz
from conftest import to_dev

pytestmark = pytest.mark.gpu


def bf16_bits(a):
    """fp32 -> bf16 bit patterns, round to nearest even."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_to_f64(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def weights(V, n, seed, scale=0.02):
    rng = np.random.default_rng(seed)
    return bf16_bits(rng.standard_normal((V, n), dtype=np.float32) * scale)


def exact(wb, x):
    """float64 product and the summation bound, row blocks of W."""
    V = wb.shape[0]
    B = x.shape[0]
    xd = x.astype(np.float64)
    out = np.empty((B, V))
    bound = np.empty((B, V))
    step = max(1, (1 << 25) // wb.shape[1])  # 256 MiB of float64 per block
    for r0 in range(0, V, step):
        wd = bf16_to_f64(wb[r0:r0 + step])
        out[:, r0:r0 + step] = xd @ wd.T
        bound[:, r0:r0 + step] = np.abs(xd) @ np.abs(wd).T
    return out, bound


def run(torch, wb, x, s, offset=0):
    V, n = wb.shape
    B = x.shape[0]
    if offset:
        flat = np.zeros(V * n + offset, np.uint16)
        flat[offset:] = wb.ravel()
        d_flat = to_dev(torch, flat.view(np.int16))
        d_w = d_flat.data_ptr() + 2 * offset
    else:
        d_flat = to_dev(torch, wb.view(np.int16))
        d_w = d_flat.data_ptr()
    d_x = to_dev(torch, x)
    d_l = torch.full((B, V), -7.0, dtype=torch.float32, device="cuda")
    d_i = torch.full((B,), -9, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    s.lm_head(d_w, V, n, d_x, B, n, d_l, V)
    s.lm_head_argmax(d_w, V, n, d_x, B, n, d_i)
    s.sync()
    logits = d_l.cpu().numpy()
    ids = d_i.cpu().numpy()
    # the batched sampler's greedy path on the same device logits
    gids, _ = s.sample(d_l, B, V, V, [pz.row_params(temperature=0.0)])
    del d_flat
    return logits, ids, gids


def check(label, wb, x, logits, ids, gids, check_logits=True):
    n = wb.shape[1]
    if check_logits:
        ex, bound = exact(wb, x)
        err = np.abs(logits.astype(np.float64) - ex)
        tol = n * 2.0 ** -24 * bound + 1e-30
        worst = float((err / tol).max())
        print(f"{label}: max |err| / bound = {worst:.4f}, max |err| = {err.max():.3e}", flush=True)
        assert (err <= tol).all(), label
    o = po.oracle()
    want = np.array([o.orc_argmax(np.ascontiguousarray(r).ctypes.data_as(po._P), r.size)
                     for r in logits], np.int32)
    assert (ids == want).all(), (label, ids, want)
    assert (gids == ids).all(), (label, gids, ids)


@pytest.mark.parametrize("B", [1, 3, 8, 17])
def test_lm_head_batches(torch_cuda, B):
    V, n = 32000, 2048
    print(f"case lmhead V={V} n={n} B={B}", flush=True)
    wb = weights(V, n, 0x1A0 + B)
    x = np.random.default_rng(B).standard_normal((B, n), dtype=np.float32)
    with pz.Sampler(32, V) as s:
        check(f"B{B}", wb, x, *run(torch_cuda, wb, x, s))


def test_lm_head_full_vocab(torch_cuda):
    """BitNet b1.58-2B-4T shape: vocab 128256, hidden 2560, one sequence."""
    V, n = 128256, 2560
    print(f"case lmhead full V={V} n={n}", flush=True)
    wb = weights(V, n, 0x1B0)
    x = np.random.default_rng(7).standard_normal((1, n), dtype=np.float32)
    with pz.Sampler(4, V) as s:
        check("full", wb, x, *run(torch_cuda, wb, x, s))


@pytest.mark.parametrize("n,offset", [(2050, 0), (2048, 1), (37, 0), (24576, 0)])
def test_lm_head_odd_shapes(torch_cuda, n, offset):
    """n not a multiple of 8 and a weight pointer off 16-byte alignment (the
    element-load path), a tiny n, and the largest n the LDS tile holds."""
    V = 4099
    print(f"case lmhead n={n} offset={offset}", flush=True)
    wb = weights(V, n, 0x1C0 + n)
    x = np.random.default_rng(n).standard_normal((5, n), dtype=np.float32)
    with pz.Sampler(8, V) as s:
        check(f"n{n}o{offset}", wb, x, *run(torch_cuda, wb, x, s, offset=offset))


def test_fused_argmax_ties_and_nan(torch_cuda):
    V, n = 3000, 512
    rng = np.random.default_rng(0x1D0)
    w = rng.standard_normal((V, n), dtype=np.float32) * 0.01
    x = rng.standard_normal((4, n), dtype=np.float32)
    # rows 1500 and 700 identical and dominant for x[0]: equal logits, lowest id
    w[1500] = np.sign(x[0]) * 0.5
    w[700] = w[1500]
    # x[1] NaN: every logit NaN, argmax returns 0
    x[1, 3] = np.nan
    # an inf weight in row 0: logit 0 is -inf for x[0] and x[3], NaN for
    # x[2] (inf times a zero activation)
    w[0, 5] = np.inf
    x[0, 5] = -1.0
    x[2, 5] = 0.0
    # x[3] zero but for that one activation, which meets a zero weight in
    # every other row: logit 0 = -inf, every other logit +0 or -0, so the
    # first of them (id 1) wins
    w[1:, 5] = 0.0
    x[3] = 0.0
    x[3, 5] = -1.0
    wb = bf16_bits(w)
    print("case lmhead ties and nan", flush=True)
    with pz.Sampler(8, V) as s:
        logits, ids, gids = run(torch_cuda, wb, x, s)
    assert ids[0] == 700
    assert ids[1] == 0 and np.isnan(logits[1]).all()
    assert np.isnan(logits[2, 0]) and ids[2] == 0
    assert ids[3] == 1
    check("ties", wb, x, logits, ids, gids, check_logits=False)
