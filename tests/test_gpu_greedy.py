"""Greedy path on the GPU (through the C ABI) against the oracle.

Greedy selection and penalty indexing must be bit-exact: every row's id must
equal the oracle's (argmax.c:3-13 on the penalised row)."""
import numpy as np
import pytest

import pz_oracle as po
import pzsample as pz
import workloads as wl
from conftest import to_dev

pytestmark = pytest.mark.gpu


def run_gpu(torch, x, params, hist=None, max_hist=2048, ld=None):
    B, V = x.shape[0], x.shape[1] if ld is None else ld
    xv = x if ld is None else x
    d_x = to_dev(torch, np.ascontiguousarray(xv))
    d_h = to_dev(torch, np.ascontiguousarray(hist)) if hist is not None else None
    H = hist.shape[1] if hist is not None else 0
    with pz.Sampler(B, x.shape[1], max_hist=max_hist) as s:
        ids, p = s.sample(d_x, B, x.shape[1] if ld is None else ld, x.shape[1], params,
                          u=None, d_hist=d_h, H=H, want_p=True)
    return ids, p


def orc_params(p):
    return po.params(p.temperature, p.top_k, p.top_p, p.rep_penalty, p.presence_penalty,
                     p.frequency_penalty)


def test_c4_full_size_bit_exact(torch_cuda):
    """1024 x 128256, repetition 1.15 over 256 uniform ids, greedy."""
    w = wl.build_c4()
    print("case c4 1024x128256 H=256", flush=True)
    ids, p = run_gpu(torch_cuda, w["logits"], w["params"], w["hist"])
    want, _, _, _ = po.sample_batch(w["logits"], [orc_params(q) for q in w["params"]],
                                    hist=w["hist"])
    assert (ids == want).all(), np.nonzero(ids != want)[0][:10]
    assert (p == 1.0).all()
    # the penalty changed the answer on some rows (so the test exercises it)
    plain, _, _, _ = po.sample_batch(w["logits"], [po.params(temperature=0.0)])
    assert (plain != want).sum() > 0


@pytest.mark.parametrize("V", [1, 3, 4, 5, 1000, 4099, 49152, 151936])
def test_sizes_and_tails(torch_cuda, V):
    x = pz.synth_normal(7, V, 3.0, 1000 + V)
    hist = pz.synth_uniform_ids(7, 16, V, 77)
    for prm in (pz.row_params(temperature=0.0),
                pz.row_params(temperature=0.0, rep_penalty=1.3),
                pz.row_params(temperature=0.0, presence_penalty=0.5, frequency_penalty=0.3)):
        ids, _ = run_gpu(torch_cuda, x, [prm], hist)
        want, _, _, _ = po.sample_batch(x, [orc_params(prm)], hist=hist)
        assert (ids == want).all(), (V, prm.rep_penalty)


def test_ties_lowest_id(torch_cuda):
    V = 128256
    x = np.round(pz.synth_normal(64, V, 1.0, 5)).astype(np.float32)  # massive ties
    x[3, :] = 2.0
    x[4, 10] = x[4, 20] = x[4, 5000] = 100.0
    x[5, 0] = -0.0
    x[5, 1:] = 0.0 - 1.0
    x[5, 77] = 0.0  # -0.0 at id 0 equals +0.0 at id 77 -> 0
    ids, _ = run_gpu(torch_cuda, x, [pz.row_params(temperature=0.0)])
    want, _, _, _ = po.sample_batch(x, [po.params(temperature=0.0)])
    assert (ids == want).all()
    assert ids[3] == 0 and ids[4] == 10 and ids[5] == 0


@pytest.mark.parametrize("V", [4000, 8192, 128256])
def test_nan_and_inf_rows(torch_cuda, V):
    """V=4000 takes one workgroup per row, the others split rows; with and
    without a penalty history (a history id's -inf stays -inf)."""
    x = pz.synth_normal(6, V, 1.0, 9)
    x[0, 0] = np.nan                 # NaN at 0 -> 0
    x[1, 5] = np.nan                 # NaN elsewhere is skipped
    x[2, :] = -np.inf                # nothing beats -inf -> 0
    x[3, :] = np.nan
    x[4, 100] = np.inf
    x[5, 1:] = -np.inf
    hist = pz.synth_uniform_ids(6, 32, V, 10)
    hist[:, 0] = 5
    for prm in (pz.row_params(temperature=0.0), pz.row_params(temperature=0.0, rep_penalty=1.2),
                pz.row_params(temperature=0.0, presence_penalty=0.5, frequency_penalty=0.3)):
        ids, _ = run_gpu(torch_cuda, x, [prm], hist)
        want, _, _, _ = po.sample_batch(x, [orc_params(prm)], hist=hist)
        assert (ids == want).all(), (V, prm.rep_penalty, ids, want)


def test_penalty_edge_ids(torch_cuda):
    """Duplicates apply once, out-of-range ids are ignored, id 0 and V-1."""
    V = 1000
    x = np.zeros((4, V), np.float32)
    x[:, 0] = 5.0
    x[:, V - 1] = 4.9
    x[:, 500] = 4.0
    hist = np.array([[0, 0, 0, 0], [-1, V, 10**9, 0], [V - 1, 0, 0, V - 1], [7, 7, 7, 7]], np.int32)
    prm = [pz.row_params(temperature=0.0, rep_penalty=1.5)]
    ids, _ = run_gpu(torch_cuda, x, prm, hist)
    want, _, _, _ = po.sample_batch(x, [po.params(temperature=0.0, rep_penalty=1.5)], hist=hist)
    assert (ids == want).all()
    # 5/1.5 = 3.33 < 4.9 (once, not three times) ; out-of-range ids ignored
    assert list(ids) == [V - 1, V - 1, 500, 0]


def test_strided_unaligned_rows(torch_cuda):
    """ld > V and ld % 4 != 0 take the scalar path."""
    B, V, ld = 9, 3001, 3003
    full = pz.synth_normal(B, ld, 2.0, 31)
    d_x = to_dev(torch_cuda, full)
    with pz.Sampler(B, V) as s:
        ids, _ = s.sample(d_x, B, V, ld, [pz.row_params(temperature=0.0)])
    want, _, _, _ = po.sample_batch(np.ascontiguousarray(full[:, :V]), [po.params(temperature=0.0)])
    assert (ids == want).all()


def test_per_row_params_and_errors(torch_cuda):
    B, V = 16, 2048
    x = pz.synth_normal(B, V, 3.0, 3)
    hist = pz.synth_uniform_ids(B, 32, V, 4)
    prms = [pz.row_params(temperature=0.0, rep_penalty=1.0 + 0.1 * b) for b in range(B)]
    ids, _ = run_gpu(torch_cuda, x, prms, hist)
    want, _, _, _ = po.sample_batch(x, [orc_params(p) for p in prms], hist=hist)
    assert (ids == want).all()
    d_x = to_dev(torch_cuda, x)
    with pz.Sampler(8, V) as s:
        with pytest.raises(pz.PzError) as e:
            s.sample(d_x, B, V, V, [pz.row_params(temperature=0.0)])
        assert e.value.code == pz.PZ_ERANGE


def split_plan(V, n_rows, target_wg=512, min_chunk=4096, max_split=128):
    """The launcher's rule (pz_greedy.hip, greedy_split): workgroups per row
    and ids per range, a multiple of 1024."""
    S = min(-(-target_wg // n_rows), V // min_chunk, max_split)
    if S < 2:
        return 1, V
    c = -(-V // S)
    c = (c + 1023) & ~1023
    return -(-V // c), c


@pytest.mark.parametrize("B", [1, 8, 64, 128, 256])
def test_split_rows_small_batches(torch_cuda, B):
    """Small batches split each row over workgroups (ranges of a multiple of
    1024 ids) and merge the ranges' bests: ids stay bit-exact, with ties and
    history ids placed on both sides of the range boundaries."""
    V = 128256
    x = pz.synth_normal(B, V, 3.0, 4000 + B)
    hist = pz.synth_uniform_ids(B, 256, V, 4100 + B)
    S, chunk = split_plan(V, B)
    assert S > 1
    b24 = chunk * (S // 2)  # a boundary between two ranges in the middle of the row
    x[0, b24 - 1] = x[0, b24] = 50.0                    # tie across the boundary -> b24 - 1
    if B > 1:
        x[1, :] = -1.0
        x[1, b24 - 1], x[1, b24] = -0.0, 0.0            # -0.0 == +0.0 -> b24 - 1
    if B > 2:
        x[2, 5000::7000] = 60.0                         # one tie in many ranges -> 5000
        x[2, V - 1] = 60.0
    if B > 3:
        x[3, 0] = np.nan                                # NaN at x[0] -> 0
    if B > 4:
        x[4, :] = -np.inf                               # nothing beats -inf -> 0
        x[4, V - 1] = np.nan
    if B > 5:
        x[5, b24 - 1] = 40.0                            # penalised away (history below)
        x[5, b24] = 39.0
        hist[5, :4] = [b24 - 1, b24 - 1, V, -3]
    if B > 6:
        x[6, V - 1] = 70.0                              # the last id, in the last range
    for prm in (pz.row_params(temperature=0.0),
                pz.row_params(temperature=0.0, rep_penalty=1.15),
                pz.row_params(temperature=0.0, presence_penalty=0.5, frequency_penalty=0.3)):
        print(f"case split greedy B={B} rep={prm.rep_penalty} pres={prm.presence_penalty}",
              flush=True)
        ids, p = run_gpu(torch_cuda, x, [prm], hist)
        want, _, _, _ = po.sample_batch(x, [orc_params(prm)], hist=hist)
        assert (ids == want).all(), (np.nonzero(ids != want)[0][:10], ids[:8], want[:8])
        assert (p == 1.0).all()
    assert want[0] == b24 - 1


@pytest.mark.parametrize("V", [8192, 8193, 12291, 20481, 20482, 20483, 49152, 151936])
def test_split_rows_range_tails(torch_cuda, V):
    """Vocabularies whose last range holds 1-3 ids (or a partial float4)."""
    B = 3
    S, chunk = split_plan(V, B)
    assert S > 1
    x = pz.synth_normal(B, V, 2.0, 4200 + V)
    x[1, V - 1] = 30.0
    x[2, V - 3:] = 30.0
    hist = pz.synth_uniform_ids(B, 64, V, 4300 + V)
    hist[2, 0] = V - 3
    for prm in (pz.row_params(temperature=0.0), pz.row_params(temperature=0.0, rep_penalty=1.3)):
        ids, _ = run_gpu(torch_cuda, x, [prm], hist)
        want, _, _, _ = po.sample_batch(x, [orc_params(prm)], hist=hist)
        assert (ids == want).all(), (V, ids, want)
