"""pz_attn_softmax: the reference softmax (softmax.c:4-23) over attention
scores, one row per head over its valid context (attention.c:210 and the
three other tn_softmax call sites).  Every written probability must be
bit-identical to the oracle's softmax of the row's first len entries, and
nothing past len may be written."""
import ctypes

import numpy as np
import pytest

import pz_oracle as po
import pzsample as pz
from conftest import to_dev

pytestmark = pytest.mark.gpu

HEADS = 32
SENTINEL = np.float32(-12345.0)


def oracle_rows(x, lens):
    out = np.full_like(x, SENTINEL)
    o = po.oracle()
    for r in range(x.shape[0]):
        n = int(lens[r])
        assert 0 <= n <= x.shape[1]
        if n == 0:
            continue
        row = x[r, :n].copy()  # the oracle works in place
        o.orc_softmax(row.ctypes.data_as(ctypes.c_void_p), n)
        out[r, :n] = row
    return out


def scores(rows, n, seed, sigma=3.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((rows, n)) * sigma).astype(np.float32)


def check(got, want, lens, label):
    for r in range(got.shape[0]):
        n = int(lens[r])
        g, w = got[r, :n], want[r, :n]
        gn, wn = np.isnan(g), np.isnan(w)
        assert (gn == wn).all(), (label, r)
        assert (g[~gn].view(np.uint32) == w[~wn].view(np.uint32)).all(), (
            label, r, np.nonzero(g.view(np.uint32) != w.view(np.uint32))[0][:5])
        assert (got[r, n:] == SENTINEL).all(), (label, r, "wrote past the row")


def run(torch, x, lens=None, ld_out=None, in_place=False, label=""):
    rows, n = x.shape
    ld_out = n if ld_out is None else ld_out
    # the lengths the kernel uses: min(len, n), nothing for len <= 0 (the
    # raw lengths go to the device)
    L = np.full(rows, n, np.int32) if lens is None else np.clip(lens, 0, n).astype(np.int32)
    want = oracle_rows(x, L)
    d_x = to_dev(torch, x)
    d_len = to_dev(torch, lens) if lens is not None else None
    with pz.Sampler(1, 16) as s:
        if in_place:
            d_o = d_x
            # entries past each row's length keep the input: mark them
            for r in range(rows):
                d_o[r, int(L[r]):] = float(SENTINEL)
            torch.cuda.synchronize()
            s.attn_softmax(d_x, d_o, rows, n, n, n, d_len)
        else:
            d_o = torch.full((rows, ld_out), float(SENTINEL), dtype=torch.float32, device="cuda")
            s.attn_softmax(d_x, d_o, rows, n, n, ld_out, d_len)
        s.sync()
    got = d_o.cpu().numpy()[:, :n]
    check(got, want, L, label)
    if ld_out > n:
        assert (d_o.cpu().numpy()[:, n:] == SENTINEL).all()


@pytest.mark.parametrize("ctx", [1, 7, 128, 255, 256, 257, 1000, 1024, 1025, 2048, 4096, 4097,
                                 32768, 32769])
def test_heads_by_context(torch_cuda, ctx):
    print(f"case attn heads={HEADS} ctx={ctx}", flush=True)
    run(torch_cuda, scores(HEADS, ctx, 0xA0 + ctx), label=f"ctx{ctx}")


@pytest.mark.parametrize("n", [300, 4096, 9000])
def test_ragged_valid_context(torch_cuda, n):
    """Per-row lengths (a batch of sequences at different positions),
    including empty rows and lengths above n (clamped)."""
    rows = 3 * HEADS
    rng = np.random.default_rng(n)
    lens = rng.integers(-2, n + 3, rows).astype(np.int32)
    lens[:4] = [0, 1, n, n + 100]
    print(f"case attn ragged n={n}", flush=True)
    run(torch_cuda, scores(rows, n, 0xB0 + n, sigma=5.0), lens=lens, label=f"ragged{n}")


@pytest.mark.parametrize("n", [129, 4096, 5000])
def test_in_place_and_padded_output(torch_cuda, n):
    print(f"case attn in-place n={n}", flush=True)
    x = scores(HEADS, n, 0xC0 + n)
    run(torch_cuda, x, in_place=True, label=f"inplace{n}")
    run(torch_cuda, x, ld_out=n + 3, label=f"padded{n}")  # misaligned output rows


@pytest.mark.parametrize("n", [700, 5000, 9000])
def test_special_values(torch_cuda, n):
    """NaN first / later, +inf, all -inf, -inf entries, ties, tiny and huge
    spreads (sums that leave and re-enter binades); rows of one wave (700),
    of one workgroup (5000) and split over workgroups (9000)."""
    x = scores(16, n, 0xD0 + n)
    x[0, 0] = np.nan
    x[1, 99] = np.nan
    x[2, 5] = np.inf
    x[3, :] = -np.inf
    x[4, ::3] = -np.inf
    x[5, :] = 0.5
    x[6, :] = np.round(x[6, :])
    x[7, :] *= 40.0
    x[8, :] *= 1e-6
    x[9, 0] = 80.0
    x[10, :] = -80.0 + x[10, :] * 1e-3
    x[11, 10] = -0.0
    x[11, 11] = 0.0
    print(f"case attn special n={n}", flush=True)
    run(torch_cuda, x, label=f"special{n}")
