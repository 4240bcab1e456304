"""Speculative-draft verification on the GPU against the oracle: accepted
lengths and every output id must be identical (the softmax normalisers, the
residual mass and both CDFs use the reference's sequential fp32 rounding)."""
import numpy as np
import pytest

import pz_oracle as po
import pzsample as pz
import workloads as wl
from conftest import to_dev

pytestmark = pytest.mark.gpu


def run(torch, target, draft, draft_ids, u_acc, u_res, tau, has_bonus,
        temp_mode=pz.PZ_TEMP_MUL_RECIP, label=""):
    B, K, V = draft.shape
    print(f"case {label} B={B} K={K} V={V} bonus={has_bonus}", flush=True)
    d_t = to_dev(torch, np.ascontiguousarray(target))
    d_d = to_dev(torch, np.ascontiguousarray(draft))
    with pz.Sampler(B, V, temp_mode=temp_mode) as s:
        acc, out = s.spec_verify(d_t, d_d, B, K, V, V, has_bonus, tau, draft_ids, u_acc, u_res)
    wacc, wout, dist = po.spec_verify(target, draft, K, has_bonus, tau, draft_ids, u_acc, u_res,
                                      temp_mode=temp_mode)
    print(f"  accepted={acc.tolist()[:16]} boundary={int((dist < 1e-5).sum())}", flush=True)
    assert (acc == wacc).all(), (label, acc, wacc)
    bad = (out != wout).any(axis=1)
    assert not bad.any(), (label, np.nonzero(bad)[0][:8], out[bad][:4], wout[bad][:4])
    return acc, out


def test_c5_full_size(torch_cuda):
    w = wl.build_c5()
    run(torch_cuda, w["target"], w["draft"], w["draft_ids"], w["u_acc"], w["u_res"], w["tau"],
        True, label="c5")


def test_c5_without_bonus_and_other_seeds(torch_cuda):
    w = wl.build_c5(has_bonus=False, seed=0xC5 + 11)
    run(torch_cuda, w["target"], w["draft"], w["draft_ids"], w["u_acc"], w["u_res"], w["tau"],
        False, label="no bonus")
    w = wl.build_c5(B=16, K=7, V=32000, seed=0xC5 + 12)
    run(torch_cuda, w["target"], w["draft"], w["draft_ids"], w["u_acc"], w["u_res"], w["tau"],
        True, label="K=7")


def test_forced_paths(torch_cuda):
    """draft == target accepts everything (u < 1) and reaches the bonus row;
    u_acc == 1 then rejects with Z == 0 (draw from p); invalid draft ids
    reject; a large gap forces the residual."""
    B, K, V = 6, 3, 20000
    rng = np.random.default_rng(5)
    target = pz.synth_normal(B * (K + 1), V, 2.5, 77).reshape(B, K + 1, V)
    draft = np.ascontiguousarray(target[:, :K, :]).copy()
    draft[3] += pz.synth_normal(K, V, 3.0, 78).reshape(K, V)
    draft_ids = rng.integers(0, V, size=(B, K)).astype(np.int32)
    draft_ids[2, 0] = -1
    draft_ids[4, 1] = V
    u_acc = pz.synth_draws(B * K, 79).reshape(B, K)
    u_acc[1, :] = 1.0
    u_acc[5, 2] = 0.0
    u_res = pz.synth_draws(B, 80)
    u_res[0] = 1.0
    acc, out = run(torch_cuda, target, draft, draft_ids, u_acc, u_res, 0.8, True, label="forced")
    assert acc[0] == K and acc[1] == 0 and acc[2] == 0


def test_residual_draw_stops_early_after_many_specials(torch_cuda):
    """The residual draw resumes from the first walk's recorded states: with
    p growing geometrically with the id (target x_i = i ln2 / 1024), q
    concentrated on the low ids (draft = the reversed ramp) and u_res tiny,
    it stops about 30 binade crossings before the row's end, past the
    specials the walk's ring still holds.  Both drafts are rejected (low
    p(d) / q(d)); accepted lengths and tokens match the oracle."""
    B, K, V = 2, 1, 128256
    i = np.arange(V, dtype=np.float64)
    ramp = (i * np.log(2.0) / 1024).astype(np.float32)
    target = np.stack([ramp, ramp]).reshape(B, K, V).astype(np.float32)
    target = np.concatenate([target, target], axis=1)  # + the bonus row
    draft = np.stack([ramp[::-1], ramp[::-1]]).reshape(B, K, V).copy()
    draft_ids = np.array([[5], [1000]], np.int32)
    u_acc = np.array([[0.5], [0.5]], np.float32)
    u_res = np.array([2.0 ** -30, 2.0 ** -22], np.float32)
    acc, out = run(torch_cuda, target, draft, draft_ids, u_acc, u_res, 1.0, True,
                   label="early residual stop")
    assert (acc == 0).all() and (out[:, 0] < V - 20 * 1024).all(), (acc, out)


def test_degenerate_rows(torch_cuda):
    B, K, V = 4, 2, 5000
    target = pz.synth_normal(B * (K + 1), V, 2.0, 91).reshape(B, K + 1, V)
    draft = np.ascontiguousarray(target[:, :K, :]) + 0.1
    target[0, 0, 10] = np.nan       # p NaN at the first position -> V-1
    draft[1, 0, 3] = np.nan         # q NaN -> Z == 0 -> draw from p
    target[2, 2, :] = -np.inf       # degenerate bonus row
    draft[2] = target[2, :K]        # accept both drafts
    target[3, 0, 7] = np.inf
    draft_ids = np.array([[1, 2], [3, 4], [5, 6], [7, 8]], np.int32)
    draft_ids[2] = [int(np.argmax(target[2, 0])), int(np.argmax(target[2, 1]))]
    u_acc = np.full((B, K), 0.5, np.float32)
    u_res = pz.synth_draws(B, 92)
    run(torch_cuda, target, draft, draft_ids, u_acc, u_res, 1.0, True, label="degenerate")


@pytest.mark.parametrize("V", [1, 3, 4097, 151936])
def test_sizes_and_temperature_forms(torch_cuda, V):
    w = wl.build_c5(B=5, K=3, V=V, seed=0xC5 + V)
    for mode in (pz.PZ_TEMP_MUL_RECIP, pz.PZ_TEMP_DIV):
        run(torch_cuda, w["target"], w["draft"], w["draft_ids"], w["u_acc"], w["u_res"], 0.7,
            True, temp_mode=mode, label=f"V={V} mode={mode}")


def test_nan_temperature(torch_cuda):
    """A NaN temperature is not clamped (temperature.c:10 tests T < 1e-6):
    every p and q is NaN, so each draft is rejected and the token falls back
    exactly as the oracle's does."""
    w = wl.build_c5(B=4, K=2, V=3000, seed=0xC5 + 21)
    run(torch_cuda, w["target"], w["draft"], w["draft_ids"], w["u_acc"], w["u_res"],
        float("nan"), True, label="nan tau")


def test_async_matches_sync_over_repeated_calls(torch_cuda):
    """pz_spec_verify_async (device inputs and outputs, no wait) gives the
    synchronous call's results, call after call on one sampler, including a
    smaller batch after a larger one."""
    torch = torch_cuda
    for label, B, K, V, seed in (("c5 shape", 32, 4, 128256, 0xC5 + 21),
                                 ("smaller", 8, 2, 50000, 0xC5 + 22)):
        w = wl.build_c5(B=B, K=K, V=V, seed=seed)
        print(f"case async {label} B={B} K={K} V={V}", flush=True)
        d_t = to_dev(torch, np.ascontiguousarray(w["target"]))
        d_d = to_dev(torch, np.ascontiguousarray(w["draft"]))
        d_ids = to_dev(torch, np.ascontiguousarray(w["draft_ids"], np.int32))
        d_ua = to_dev(torch, np.ascontiguousarray(w["u_acc"], np.float32))
        d_ur = to_dev(torch, np.ascontiguousarray(w["u_res"], np.float32))
        with pz.Sampler(32, 128256) as s:
            acc, out = s.spec_verify(d_t, d_d, B, K, V, V, True, w["tau"], w["draft_ids"],
                                     w["u_acc"], w["u_res"])
            for rep in range(3):
                d_acc = torch.full((B,), -7, dtype=torch.int32, device="cuda")
                d_out = torch.full((B, K + 1), -7, dtype=torch.int32, device="cuda")
                s.spec_verify_async(d_t, d_d, B, K, V, V, True, w["tau"], d_ids, d_ua, d_ur,
                                    d_acc, d_out)
                s.sync()
                assert (d_acc.cpu().numpy() == acc).all(), (label, rep)
                assert (d_out.cpu().numpy() == out).all(), (label, rep)
        wacc, wout, _ = po.spec_verify(w["target"], w["draft"], K, True, w["tau"], w["draft_ids"],
                                       w["u_acc"], w["u_res"])
        assert (acc == wacc).all() and (out == wout).all(), label


@pytest.mark.parametrize("has_bonus", [True, False])
def test_greedy_drafts(torch_cuda, has_bonus):
    """Greedy drafting (q one-hot at each draft, no draft rows): the draft
    ids are the draft rows' argmax, with invalid ids, a draft the target
    gives p = 1 (u = 1.0 then rejects with Z == 0) and u = 0 mixed in."""
    w = wl.build_c5(B=32, K=4, seed=0xC5 + 21, has_bonus=has_bonus)
    B, K, V, tau = w["B"], w["K"], w["V"], w["tau"]
    target = w["target"].copy()
    ids = np.argmax(w["draft"], axis=2).astype(np.int32)
    ids[2, 0] = -1
    ids[5, 2] = V
    target[7, 0, :] = -1e30
    target[7, 0, ids[7, 0]] = 0.0  # p(d) == 1
    u_acc = w["u_acc"].copy()
    u_acc[7, 0] = 1.0
    u_acc[9, :] = 0.0
    print(f"case greedy drafts B={B} K={K} V={V} bonus={has_bonus}", flush=True)
    d_t = to_dev(torch_cuda, np.ascontiguousarray(target))
    with pz.Sampler(B, V) as s:
        acc, out = s.spec_verify(d_t, None, B, K, V, V, has_bonus, tau, ids, u_acc, w["u_res"])
    wacc, wout, _ = po.spec_verify(target, None, K, has_bonus, tau, ids, u_acc, w["u_res"])
    assert (acc == wacc).all(), (acc, wacc)
    assert (out == wout).all(), np.nonzero((out != wout).any(axis=1))[0]
    assert acc[7] == 0 and acc[9] == K and acc[2] == 0
