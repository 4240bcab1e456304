"""Top-k and top-k -> top-p chain on the GPU against the oracle.

Selection is bit-exact (same k ids in the same order); the k-slot softmax,
cut-off and draw use the reference's sequential fp32 sums, so ids and
p(chosen) are expected to be identical to the oracle's; the 1e-5 tolerance
on p is the stated bar, and rows whose draw lies within 1e-5 of a CDF
boundary are counted separately (they must still match here)."""
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


def check(torch, x, params, u, hist=None, temp_mode=pz.PZ_TEMP_MUL_RECIP, label=""):
    B, V = x.shape
    print(f"case {label} B={B} V={V}", flush=True)
    d_x = to_dev(torch, np.ascontiguousarray(x))
    H = hist.shape[1] if hist is not None else 0
    d_h = to_dev(torch, np.ascontiguousarray(hist)) if hist is not None else None
    with pz.Sampler(B, V, max_hist=max(H, 1), temp_mode=temp_mode) as s:
        ids, p = s.sample(d_x, B, V, V, params, u=u, d_hist=d_h, H=H, want_p=True)
    want, pw, dd, dc = po.sample_batch(x, [orc(q) for q in params], u=u, hist=hist,
                                       temp_mode=temp_mode)
    boundary = (dd < 1e-5) | (dc < 1e-5)
    bad = ids != want
    assert not (bad & ~boundary).any(), (label, np.nonzero(bad)[0][:8], ids[bad][:8], want[bad][:8])
    assert not bad.any(), f"{label}: {bad.sum()} boundary rows differ"
    assert np.all(np.abs(p - pw) <= P_TOL), label
    return ids, p, want, pw


def test_c3_full_size(torch_cuda):
    w = wl.build_c3()
    ids, p, want, pw = check(torch_cuda, w["logits"], w["params"], w["u"], w["hist"], label="c3")
    assert (p == pw).all()  # same sequential arithmetic: bitwise equal


def test_c1_steps_as_batch(torch_cuda):
    w = wl.build_c1(steps=500)
    ids, p, want, pw = check(torch_cuda, w["logits"], w["params"], w["u"], w["hist"], label="c1")
    assert (p == pw).all()


@pytest.mark.parametrize("k", [1, 2, 20, 40, 1024, 5000])
@pytest.mark.parametrize("top_p", [1.0, 0.9])
def test_k_sweep(torch_cuda, k, top_p):
    B, V = 24, 32000
    x = pz.synth_normal(B, V, 2.5, 100 + k)
    u = pz.synth_draws(B, 7 + k)
    check(torch_cuda, x, [pz.row_params(temperature=0.9, top_k=k, top_p=top_p)], u,
          label=f"k={k} p={top_p}")


def test_ties_and_degenerate_rows(torch_cuda):
    B, V = 12, 20000
    x = (np.round(pz.synth_normal(B, V, 1.0, 5) * 2) / 2).astype(np.float32)  # heavy ties
    x[0, :] = 1.0                    # all equal -> lowest ids, forces the rescan path
    x[1, :] = -np.inf                # no value above -1e30 -> id -1
    x[2, :] = -np.inf
    x[2, 777] = 3.0                  # fewer than k valid values
    x[3, ::2] = np.nan               # NaN never enters
    x[4, :] = np.arange(V, dtype=np.float32) * 1e-3   # ascending: adversarial order
    x[5, :] = -np.arange(V, dtype=np.float32) * 1e-3  # descending
    x[6, :] = -2e30                  # below -1e30: never admitted
    x[6, 10:20] = 0.0
    x[7, 0] = -0.0
    x[7, 1:] = 0.0
    u = pz.synth_draws(B, 99)
    ids, *_ = check(torch_cuda, x, [pz.row_params(temperature=1.0, top_k=40, top_p=0.95)], u,
                    label="degenerate")
    assert ids[1] == -1
    ids2, *_ = check(torch_cuda, x, [pz.row_params(temperature=1.0, top_k=5)], u,
                     label="degenerate k5")
    assert ids2[0] in range(5) and ids2[2] == 777


def test_temperature_division_form(torch_cuda):
    B, V = 64, 49152
    x = pz.synth_normal(B, V, 3.0, 11)
    u = pz.synth_draws(B, 12)
    for mode in (pz.PZ_TEMP_MUL_RECIP, pz.PZ_TEMP_DIV):
        check(torch_cuda, x, [pz.row_params(temperature=0.8, top_k=40, top_p=0.95)], u,
              temp_mode=mode, label=f"temp form {mode}")


def test_mixed_modes_in_one_batch(torch_cuda):
    B, V = 32, 8192
    x = pz.synth_normal(B, V, 2.0, 21)
    u = pz.synth_draws(B, 22)
    hist = pz.synth_uniform_ids(B, 64, V, 23)
    prms = []
    for b in range(B):
        if b % 3 == 0:
            prms.append(pz.row_params(temperature=0.0, rep_penalty=1.2))
        elif b % 3 == 1:
            prms.append(pz.row_params(temperature=0.7, top_k=10, presence_penalty=0.4))
        else:
            prms.append(pz.row_params(temperature=1.1, top_k=50, top_p=0.7, frequency_penalty=0.2))
    check(torch_cuda, x, prms, u, hist=hist, label="mixed")


def test_uniform_one_and_zero(torch_cuda):
    """u = 1.0 (rng_float can return it) takes the fallback slot; u = 0 the first."""
    B, V = 4, 5000
    x = pz.synth_normal(B, V, 2.0, 3)
    for uval in (0.0, 1.0, 0.999999):
        u = np.full(B, uval, np.float32)
        check(torch_cuda, x, [pz.row_params(temperature=1.0, top_k=30, top_p=0.9)], u,
              label=f"u={uval}")
        check(torch_cuda, x, [pz.row_params(temperature=1.0, top_k=30)], u, label=f"u={uval} k")


@pytest.mark.parametrize("B,V", [(1, 49152), (3, 128256), (8, 4097), (1, 4096), (2, 151936),
                                 (1, 300000)])
@pytest.mark.parametrize("k,top_p", [(1, 1.0), (40, 0.95), (64, 0.9), (65, 1.0), (100, 1.0),
                                     (300, 0.8)])
def test_small_batch_rows_split_over_workgroups(torch_cuda, B, V, k, top_p):
    """Small batches take the split kernel (each 4096-id range selects its own
    top k, the last workgroup of the row merges) whenever the ranges' k
    candidates fit its merge buffer and the row has at most 64 ranges (V =
    300000 has 74: one workgroup per row); k <= 64 merges sorted range lists
    in registers, larger k the ranges' supersets.  Penalties, ties across
    range boundaries and rows with fewer than k valid values included."""
    rng = np.random.default_rng(V + k)
    x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
    x[0, 4090:4102] = 9.0                      # a tie straddling a range boundary
    if B > 1:
        x[1, :] = -np.inf                      # no valid value: every slot stays -1
        x[1, ::997] = 1.0                      # ... but a few valid ones, fewer than k
    if B > 2:
        x[2, 5] = np.nan
    H = 64
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    hist[0, :4] = [4090, 4095, 4096, 4101]     # penalised members of the tie
    params = [pz.row_params(temperature=0.8, top_k=k, top_p=top_p, rep_penalty=1.3)]
    check(torch_cuda, x, params, pz.synth_draws(B, V * 7 + k), hist=hist,
          label=f"split B={B} V={V} k={k}")


@pytest.mark.parametrize("V", [49152, 128256])
@pytest.mark.parametrize("k", [40, 64, 100])
def test_split_rows_of_equal_values(torch_cuda, V, k):
    """Every value of a range in one key bin (a constant row: the range's k
    are its k lowest ids, chosen by the exact select), a row of two levels
    whose upper level is spread thinly over the ranges, and a row whose
    ranges each hold a single valid value."""
    B = 3
    x = np.full((B, V), 0.5, np.float32)
    x[1, ::1531] = 2.0
    x[2, :] = -np.inf
    x[2, 4095::4096] = np.linspace(-1.0, 1.0, len(range(4095, V, 4096)), dtype=np.float32)
    params = [pz.row_params(temperature=1.0, top_k=k, top_p=0.9)]
    check(torch_cuda, x, params, pz.synth_draws(B, V + k), label=f"equal V={V} k={k}")
