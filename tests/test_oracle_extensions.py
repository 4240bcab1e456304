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
      checked by simulation on a 5-token vocabulary; greedy (one-hot)
      drafts against a float64 model of the rule and by the same theorem;
  f3  the speculative decode loop: the first token each round commits is
      distributed as the target softmax (chi-square over 20000 seeded
      sequences, drawn and greedy drafts), and EOS stops (the EOS is not
      committed; a stopped sequence's state stays as it is).
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


# ------------------------------------------------- a11: greedy (one-hot) drafts
def test_spec_greedy_drafts_closed_form():
    """q one-hot at the draft: accepted iff u < p(d); on rejection the token
    comes from p with p(d) removed (float64 model, away from boundaries)."""
    rng = np.random.default_rng(11)
    B, K, V, tau = 200, 3, 30, 0.9
    target = (rng.standard_normal((B, K + 1, V)) * 1.5).astype(np.float32)
    ids = rng.integers(-1, V, size=(B, K)).astype(np.int32)  # -1: never accepted
    ua = rng.uniform(size=(B, K)).astype(np.float32)
    ur = rng.uniform(size=B).astype(np.float32)
    acc, out, _ = po.spec_verify(target, None, K, True, tau, ids, ua, ur)
    checked = 0
    for b in range(B):
        j = 0
        while j < K:
            d = ids[b, j]
            p = softmax64(target[b, j], tau)
            if d < 0 or not ua[b, j] < p[d]:
                break
            j += 1
        if any(abs(float(ua[b, i]) - softmax64(target[b, i], tau)[ids[b, i]]) < 1e-5
               for i in range(min(j + 1, K)) if ids[b, i] >= 0):
            continue  # too close to the acceptance boundary for a float64 model
        assert acc[b] == j, (b, acc[b], j)
        assert (out[b, :j] == ids[b, :j]).all()
        if j < K:
            r = softmax64(target[b, j], tau)
            if ids[b, j] >= 0:
                r[ids[b, j]] = 0.0
            cdf = np.cumsum(r)
            x = ur[b] * cdf[-1]
            if np.min(np.abs(cdf - x)) < 1e-5:
                continue
            assert out[b, j] == int(np.searchsorted(cdf, x, side="right")), b
            assert out[b, j] != ids[b, j]
        checked += 1
    assert checked > B // 2


def test_spec_greedy_draft_first_token_is_distributed_as_target():
    """With a fixed (greedy) draft the emitted token is still distributed as
    the target softmax: accepted with probability p(d), else drawn from p
    without d."""
    rng = np.random.default_rng(12)
    V, tau, N = 5, 0.8, 40000
    t_row = np.array([1.0, 0.2, -0.5, 2.0, 0.0], np.float32)
    p = softmax64(t_row, tau)
    target = np.broadcast_to(t_row, (N, 1, V)).copy()
    ids = np.full((N, 1), 3, np.int32)  # the draft model's argmax
    ua = rng.uniform(size=(N, 1)).astype(np.float32)
    ur = rng.uniform(size=N).astype(np.float32)
    acc, out, _ = po.spec_verify(target, None, 1, False, tau, ids, ua, ur)
    freq = np.bincount(out[:, 0], minlength=V) / N
    sigma = np.sqrt(p * (1 - p) / N)
    assert np.all(np.abs(freq - p) < 5 * sigma + 1e-4), (freq, p)
    assert abs(acc.mean() - p[3]) < 5 * np.sqrt(0.25 / N)


class FixedModels:
    """Draft and target models whose logits ignore the context (fixed rows),
    with the cache bookkeeping of a real pair (positions checked)."""

    def __init__(self, B, lens, d_row, t_row):
        self.d, self.t = d_row, t_row
        self.len = [np.asarray(lens, np.int64) - 1, np.asarray(lens, np.int64) - 1]

    def draft(self, tok, pos):
        assert (np.asarray(pos) == self.len[0]).all()
        self.len[0] = np.asarray(pos) + 1
        return np.broadcast_to(self.d, (len(tok), self.d.size)).copy()

    def target(self, tok, pos):
        assert (np.asarray(pos) == self.len[1]).all()
        B, n = np.asarray(tok).shape
        self.len[1] = np.asarray(pos) + n
        return np.broadcast_to(self.t, (B, n, self.t.size)).copy()

    def rollback(self, m, pos):
        assert (np.asarray(pos) <= self.len[m]).all()
        self.len[m] = np.asarray(pos).copy()


@pytest.mark.parametrize("greedy", [False, True])
def test_spec_decode_first_committed_token_is_distributed_as_target(greedy):
    """The loop (draft draws or greedy drafts, the uniforms' order, the
    verification, the commit): over many sequences with their own RNG
    seeds, the first token each round commits follows softmax(target/tau)."""
    V, K, tau, N = 6, 2, 0.9, 20000
    t_row = np.array([0.5, 1.8, -0.3, 1.0, 0.0, -1.2], np.float32)
    d_row = np.array([1.2, 0.4, 0.2, 1.5, -0.5, 0.0], np.float32)
    p = softmax64(t_row, tau)
    lens = np.ones(N, np.int64)
    tokens = np.zeros((N, 1 + K + 1), np.int32)
    ds = (np.arange(1, N + 1, dtype=np.uint64) * np.uint64(7919)) | np.uint64(1)
    vs = (np.arange(1, N + 1, dtype=np.uint64) * np.uint64(104729)) ^ np.uint64(5)
    m = FixedModels(N, lens, d_row, t_row)
    acc = po.spec_decode(m, N, K, V, tau, tokens, lens, 1, ds, vs, greedy_draft=greedy)
    first = tokens[:, 1]
    freq = np.bincount(first, minlength=V) / N
    # chi-square against p (5 degrees of freedom; 0.1 % critical value 20.5)
    chi2 = float(((freq - p) ** 2 / p).sum() * N)
    assert chi2 < 20.5, (chi2, freq, p)
    assert (lens == 1 + acc[0] + 1).all()
    if greedy:
        assert (acc[0] >= 0).all()
        assert (ds == (np.arange(1, N + 1, dtype=np.uint64) * np.uint64(7919)) | np.uint64(1)).all()


def test_spec_decode_stops_at_eos():
    """A sequence stops at the first committed EOS id (not committed); later
    rounds leave its tokens, length and RNG states alone."""
    V, K, tau, B = 8, 3, 0.7, 64
    t_row = np.array([0.0, 3.0, 0.0, 1.0, 0.0, 0.0, 0.0, 0.0], np.float32)
    d_row = np.array([0.0, 3.0, 0.0, 0.8, 0.0, 0.0, 0.0, 0.0], np.float32)
    rounds = 6
    max_len = 1 + (rounds + 1) * (K + 1)
    lens = np.ones(B, np.int64)
    tokens = np.zeros((B, max_len), np.int32)
    ds = (np.arange(1, B + 1, dtype=np.uint64) * np.uint64(7919)) | np.uint64(1)
    vs = (np.arange(1, B + 1, dtype=np.uint64) * np.uint64(104729)) ^ np.uint64(5)
    done = np.zeros(B, np.uint8)
    m = FixedModels(B, lens, d_row, t_row)
    acc = po.spec_decode(m, B, K, V, tau, tokens, lens, rounds, ds, vs, eos=[3], done=done)
    assert done.any() and not done.all()
    for b in range(B):
        seq = tokens[b, 1:lens[b]]
        assert 3 not in seq  # the EOS is never committed
        if not done[b]:
            assert (acc[:, b] >= 0).all()
            assert lens[b] == 1 + sum(int(a) + 1 for a in acc[:, b])
    # sequences that stopped before the last round keep their state there
    later = np.nonzero(acc[-1] < 0)[0]
    assert later.size > 0
    ds2, vs2, tok2, len2 = ds.copy(), vs.copy(), tokens.copy(), lens.copy()
    po.spec_decode(m, B, K, V, tau, tokens, lens, 1, ds, vs, eos=[3], done=done)
    assert (ds[later] == ds2[later]).all() and (vs[later] == vs2[later]).all()
    assert (lens[later] == len2[later]).all() and (tokens[later] == tok2[later]).all()
