"""Pins for the oracle functions the reference has no code for, and for the
inline categorical draw it never tests (CPU only).

  a5  categorical draw (generate.c:157-169): hand-computed CDF cases
      including the V-1 fallback, and the draw frequencies over a grid of
      uniforms against float64 probabilities;
  a8/a9 penalties: hand-computed exact cases (sign rule, once per distinct
      id, ids out of range, counts) and a vectorised np.bincount formulation
      on random histories;
  a10 top-k -> top-p chain: reduces to top-k outside (0, 1); against a
      float64 model (lexsort, softmax, cumulative cut-off, draw) away from
      rounding boundaries;
  a11 speculative verification: draft == target accepts everything, a
      rejected draft is never resampled, and the first emitted token is
      distributed as the target softmax (Leviathan et al. 2023, Thm. 1),
      checked by simulation on a 5-token vocabulary.
"""
import ctypes

import numpy as np
import pytest

import pz_oracle as po

_P = ctypes.c_void_p


def ptr(a):
    return a.ctypes.data_as(_P)


# ---------------------------------------------------------------------- a5
@pytest.mark.parametrize("probs,r,want", [
    ([0.25, 0.25, 0.5], 0.0, 0),
    ([0.25, 0.25, 0.5], 0.2499999, 0),
    ([0.25, 0.25, 0.5], 0.25, 1),      # r < cdf is strict
    ([0.25, 0.25, 0.5], 0.5, 2),
    ([0.25, 0.25, 0.5], 0.99, 2),
    ([0.25, 0.25, 0.5], 1.0, 2),       # never r < cdf: fallback V-1
    ([0.5, 0.5, 0.0], 1.0, 2),         # fallback is V-1 even with p = 0 there
    ([0.0, 0.5, 0.0, 0.5], 0.0, 1),    # zero-probability ids are skipped
    ([0.0, 0.5, 0.0, 0.5], 0.5, 3),
])
def test_categorical_hand_cases(probs, r, want):
    p = np.array(probs, np.float32)
    assert po.oracle().orc_categorical(ptr(p), p.size, ctypes.c_float(r), None) == want


def test_categorical_frequencies_match_probabilities():
    rng = np.random.default_rng(3)
    o = po.oracle()
    for V in (5, 37):
        x = (rng.standard_normal(V) * 2).astype(np.float32)
        p = x.copy()
        o.orc_softmax(ptr(p), V)
        N = 20000
        counts = np.zeros(V)
        for j in range(N):
            counts[o.orc_categorical(ptr(p), V, ctypes.c_float((j + 0.5) / N), None)] += 1
        ref = np.exp(x.astype(np.float64) - x.max())
        ref /= ref.sum()
        assert np.max(np.abs(counts / N - ref)) < 3.0 / N + 1e-5


# ------------------------------------------------------------------- a8/a9
def test_penalties_hand_case():
    x = np.array([2.0, -2.0, 3.0, 4.0, 1.0], np.float32)
    hist = np.array([0, 1, 1, 1, 7, -1, 2], np.int32)
    po.oracle().orc_penalties(ptr(x), 5, ptr(hist), hist.size, ctypes.c_float(2.0),
                              ctypes.c_float(0.25), ctypes.c_float(0.5))
    # id 0: 2/2 - (1*0.5 + 0.25); id 1: -2*2 - (3*0.5 + 0.25); id 2: 3/2 - 0.75
    assert x.tolist() == [0.25, -5.75, 0.75, 4.0, 1.0]


def test_repetition_applies_once_and_keeps_zero():
    x = np.array([0.0, 1.0, 2.0, 4.0], np.float32)
    hist = np.array([3, 3, 3, 0, 0], np.int32)
    po.oracle().orc_penalties(ptr(x), 4, ptr(hist), hist.size, ctypes.c_float(2.0),
                              ctypes.c_float(0.0), ctypes.c_float(0.0))
    assert x.tolist() == [0.0, 1.0, 2.0, 2.0]


def test_penalties_against_bincount_formulation():
    rng = np.random.default_rng(11)
    o = po.oracle()
    for trial in range(20):
        V = int(rng.integers(1, 3000))
        x = (rng.standard_normal(V) * 3).astype(np.float32)
        H = int(rng.integers(1, 600))
        hist = rng.integers(-5, V + 5, size=H).astype(np.int32)
        rep, pres, freq = (np.float32(rng.uniform(0.5, 2.0)), np.float32(rng.uniform(0, 1)),
                           np.float32(rng.uniform(0, 1)))
        got = x.copy()
        o.orc_penalties(ptr(got), V, ptr(hist), H, ctypes.c_float(rep), ctypes.c_float(pres),
                        ctypes.c_float(freq))
        valid = hist[(hist >= 0) & (hist < V)]
        cnt = np.bincount(valid, minlength=V)
        hit = cnt > 0
        v = np.where(x > 0, x / rep, x * rep).astype(np.float32)
        t = (cnt.astype(np.float32) * freq).astype(np.float32) + pres
        want = np.where(hit, (v - t.astype(np.float32)).astype(np.float32), x)
        assert (got.view(np.uint32) == want.view(np.uint32)).all(), trial


# --------------------------------------------------------------------- a10
def chain_f64(x, k, top_p, u):
    """float64 model of the chain: top-k by (value desc, id asc), softmax over
    the k values, cumulative cut-off at top_p, draw u * truncated mass.
    Returns (id, distance of the draw / cut-off from a boundary)."""
    order = np.lexsort((np.arange(x.size), -x.astype(np.float64)))[:k]
    v = x[order].astype(np.float64)
    e = np.exp(v - v[0])
    p = e / e.sum()
    cum = np.cumsum(p)
    cut = int(np.searchsorted(cum, top_p, side="left")) + 1
    cut = min(cut, k)
    trunc = cum[cut - 1]
    r = u * trunc
    j = int(np.searchsorted(cum[:cut], r, side="right"))
    j = min(j, cut - 1) if r < trunc else 0
    dist = min(np.min(np.abs(cum - top_p)), np.min(np.abs(cum[:cut] - r)), abs(r))
    return int(order[j]), dist


def test_chain_reduces_to_top_k_outside_unit_interval():
    rng = np.random.default_rng(5)
    o = po.oracle()
    for _ in range(50):
        V = int(rng.integers(2, 500))
        x = (rng.standard_normal(V) * 2).astype(np.float32)
        k = int(rng.integers(1, 60))
        u = np.float32(rng.uniform())
        want = o.orc_top_k(ptr(x), V, k, ctypes.c_float(u), None)
        for tp in (1.0, 1.5, 0.0, -0.5):
            assert o.orc_chain(ptr(x), V, k, ctypes.c_float(tp), ctypes.c_float(u), None) == want


def test_chain_against_float64_model():
    rng = np.random.default_rng(6)
    o = po.oracle()
    checked = 0
    for _ in range(400):
        V = int(rng.integers(2, 2000))
        x = (rng.standard_normal(V) * rng.uniform(0.3, 3)).astype(np.float32)
        k = int(rng.integers(1, min(V, 200) + 1))
        tp = float(rng.uniform(0.05, 0.99))
        u = float(np.float32(rng.uniform()))
        want, dist = chain_f64(x, k, np.float32(tp), u)
        if dist < 1e-5:
            continue  # fp32 rounding may legitimately decide these
        got = o.orc_chain(ptr(x), V, k, ctypes.c_float(tp), ctypes.c_float(u), None)
        assert got == want, (V, k, tp, u)
        checked += 1
    assert checked > 300


# --------------------------------------------------------------------- a11
def softmax64(x, tau):
    z = x.astype(np.float64) / tau
    e = np.exp(z - z.max())
    return e / e.sum()


def test_spec_accepts_everything_when_draft_equals_target():
    rng = np.random.default_rng(7)
    B, K, V = 6, 3, 50
    target = (rng.standard_normal((B, K + 1, V)) * 2).astype(np.float32)
    draft = np.ascontiguousarray(target[:, :K, :])
    ids = rng.integers(0, V, size=(B, K)).astype(np.int32)
    ua = rng.uniform(0, 0.999, size=(B, K)).astype(np.float32)
    ur = rng.uniform(size=B).astype(np.float32)
    acc, out, _ = po.spec_verify(target, draft, K, True, 0.8, ids, ua, ur)
    assert (acc == K).all()
    assert (out[:, :K] == ids).all() and (out[:, K] >= 0).all()


def test_spec_rejected_draft_is_never_resampled():
    rng = np.random.default_rng(8)
    B, K, V = 64, 2, 40
    target = (rng.standard_normal((B, K, V)) * 2).astype(np.float32)
    draft = (target + rng.standard_normal((B, K, V)) * 1.5).astype(np.float32)
    ids = rng.integers(0, V, size=(B, K)).astype(np.int32)
    ua = rng.uniform(size=(B, K)).astype(np.float32)
    ur = rng.uniform(size=B).astype(np.float32)
    acc, out, _ = po.spec_verify(target, draft, K, False, 1.0, ids, ua, ur)
    rej = acc < K
    assert rej.any()
    b = np.nonzero(rej)[0]
    assert (out[b, acc[b]] != ids[b, acc[b]]).all()


def test_spec_first_token_is_distributed_as_target():
    """Speculative sampling emits the target distribution whatever q is."""
    rng = np.random.default_rng(9)
    V, tau, N = 5, 0.8, 40000
    t_row = np.array([1.0, 0.2, -0.5, 2.0, 0.0], np.float32)
    d_row = np.array([0.1, 1.5, 0.3, 0.5, -1.0], np.float32)
    q = softmax64(d_row, tau)
    p = softmax64(t_row, tau)
    target = np.broadcast_to(t_row, (N, 1, V)).copy()
    draft = np.broadcast_to(d_row, (N, 1, V)).copy()
    ids = rng.choice(V, size=(N, 1), p=q).astype(np.int32)
    ua = rng.uniform(size=(N, 1)).astype(np.float32)
    ur = rng.uniform(size=N).astype(np.float32)
    acc, out, _ = po.spec_verify(target, draft, 1, False, tau, ids, ua, ur)
    freq = np.bincount(out[:, 0], minlength=V) / N
    sigma = np.sqrt(p * (1 - p) / N)
    assert np.all(np.abs(freq - p) < 5 * sigma + 1e-4), (freq, p)
    # and the acceptance rate is sum(min(p, q))
    assert abs(acc.mean() - np.minimum(p, q).sum()) < 5 * np.sqrt(0.25 / N)
