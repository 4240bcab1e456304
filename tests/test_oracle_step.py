"""The oracle's decode step (orc_sample_step): per-row RNG states advance
exactly where the reference's samplers consume a uniform, and EOS flags.

Pinned against the reference sampler compiled from its own sources
(oracle/_ref): sample_top_p and sample_top_k take the RNG state themselves,
so their returned id AND the state they leave behind are compared with the
oracle's, including the two argmax returns of top_p.c that come before the
draw (V > 200000, :33-34; NaN first logit, :68-69).  Greedy and the inline
categorical block of generate.c (not a compiled function of the reference)
are pinned by the closed form: zero draws and one draw."""
import ctypes

import numpy as np
import pytest

import pz_oracle as po

_P = ctypes.c_void_p


def one_draw(seed):
    s = ctypes.c_ulonglong(seed)
    po.oracle().orc_rng_float(ctypes.byref(s))
    return s.value


def step1(x, prm, seed, hist=None, eos=()):
    st = np.array([seed], np.uint64)
    ids, flags, drew = po.sample_step(x[None, :], [prm], st, hist=hist, eos=eos)
    return int(ids[0]), int(st[0]), bool(drew[0]), int(flags[0])


def ref_top_p(r, x, T, p, seed):
    y = x.copy()
    r.apply_temperature(y.ctypes.data_as(_P), y.size, ctypes.c_float(T))
    s = ctypes.c_ulonglong(seed)
    rid = r.sample_top_p(y.ctypes.data_as(_P), y.size, ctypes.c_float(p), ctypes.byref(s))
    return rid, s.value


def ref_top_k(r, x, T, k, seed):
    y = x.copy()
    r.apply_temperature(y.ctypes.data_as(_P), y.size, ctypes.c_float(T))
    s = ctypes.c_ulonglong(seed)
    rid = r.sample_top_k(y.ctypes.data_as(_P), y.size, k, ctypes.byref(s))
    return rid, s.value


def top_p_rows():
    rng = np.random.default_rng(77)
    rows = []
    for V in (1, 5, 300, 4096):
        rows.append(("normal", (rng.standard_normal(V) * 3).astype(np.float32)))
    x = (rng.standard_normal(500) * 2).astype(np.float32)
    x[0] = np.nan
    rows.append(("nan_first", x))                 # top_p.c:68-69: argmax, no draw
    x = (rng.standard_normal(500) * 2).astype(np.float32)
    x[7] = np.nan
    rows.append(("nan_later", x))                 # a later NaN never wins the max: draws
    rows.append(("all_minus_inf", np.full(64, -np.inf, np.float32)))
    x = (rng.standard_normal(64)).astype(np.float32)
    x[3] = np.inf
    rows.append(("plus_inf", x))
    rows.append(("above_guard", (rng.standard_normal(200001)).astype(np.float32)))  # :33-34
    rows.append(("at_guard", (rng.standard_normal(200000)).astype(np.float32)))
    return rows


@pytest.mark.skipif(po.ref(True) is None, reason="oracle/_ref not built here")
@pytest.mark.parametrize("name,x", top_p_rows(), ids=[n for n, _ in top_p_rows()])
def test_top_p_state_matches_reference(name, x):
    r = po.ref(True)
    for seed in (1, 42, 0x9E3779B97F4A7C15):
        want_id, want_state = ref_top_p(r, x, 0.7, 0.9, seed)
        rid, state, drew, _ = step1(x, po.params(temperature=0.7, top_p=0.9), seed)
        assert rid == want_id, (name, seed)
        assert state == want_state, (name, seed)
        assert drew == (want_state != seed)
    if name in ("nan_first", "above_guard"):
        assert not drew
    else:
        assert drew


@pytest.mark.skipif(po.ref(True) is None, reason="oracle/_ref not built here")
def test_top_k_state_matches_reference():
    r = po.ref(True)
    rng = np.random.default_rng(78)
    for trial in range(30):
        V = int(rng.integers(1, 5000))
        x = (rng.standard_normal(V) * rng.uniform(0.5, 4)).astype(np.float32)
        if trial == 3:
            x[:] = -np.inf  # every slot keeps -1: returns -1, still draws
        k = int(rng.integers(1, 70))  # top_k > 0 selects sample_top_k (generate order)
        seed = int(rng.integers(1, 2**63))
        want_id, want_state = ref_top_k(r, x, 0.8, k, seed)
        rid, state, drew, _ = step1(x, po.params(temperature=0.8, top_k=k), seed)
        assert (rid, state) == (want_id, want_state), trial
        assert drew


def test_greedy_never_draws_categorical_and_chain_draw_once():
    rng = np.random.default_rng(79)
    x = (rng.standard_normal(3000) * 3).astype(np.float32)
    hist = rng.integers(0, 3000, (1, 32)).astype(np.int32)
    for seed in (1, 5, 2**40 + 3):
        _, st, drew, _ = step1(x, po.params(temperature=0.0, rep_penalty=1.3), seed, hist)
        assert st == seed and not drew
        _, st, drew, _ = step1(x, po.params(temperature=1e-7), seed)
        assert st == seed and not drew
        rid, st, drew, _ = step1(x, po.params(temperature=0.9), seed)
        assert st == one_draw(seed) and drew
        # the id is the categorical draw with that one uniform
        s = ctypes.c_ulonglong(seed)
        u = po.oracle().orc_rng_float(ctypes.byref(s))
        want, _ = po.sample_row(x, po.params(temperature=0.9), u=u)
        assert rid == want
        _, st, drew, _ = step1(x, po.params(temperature=0.8, top_k=40, top_p=0.95,
                                            rep_penalty=1.1), seed, hist)
        assert st == one_draw(seed) and drew


def test_state_sequence_over_steps_is_the_reference_stream():
    """A row that draws every step walks the plain rng_float sequence of its
    seed (golden sequence of tests/golden/rng.json's generator)."""
    rng = np.random.default_rng(80)
    seed = 12345
    st = np.array([seed], np.uint64)
    s = ctypes.c_ulonglong(seed)
    for step in range(50):
        x = (rng.standard_normal(700) * 2).astype(np.float32)
        po.sample_step(x[None, :], [po.params(temperature=0.8, top_p=0.9)], st)
        po.oracle().orc_rng_float(ctypes.byref(s))
        assert int(st[0]) == s.value, step


def test_penalised_nan_first_value_skips_the_draw():
    """A NaN first value made by the penalty (inf - inf) is what top_p.c sees
    after the chain's earlier stages: no draw."""
    x = np.zeros(100, np.float32)
    x[0] = np.inf
    hist = np.array([[0, 0, 5]], np.int32)
    prm = po.params(temperature=0.7, top_p=0.9, frequency_penalty=np.inf)
    _, st, drew, _ = step1(x, prm, 99, hist)
    assert not drew and st == 99


def test_eos_flags():
    rng = np.random.default_rng(81)
    B, V = 6, 64
    x = (rng.standard_normal((B, V)) * 0.1).astype(np.float32)
    for b in range(B):
        x[b, b * 3] = 50.0  # greedy picks id 3b
    st = np.arange(1, B + 1, dtype=np.uint64)
    ids, flags, drew = po.sample_step(x, [po.params(temperature=0.0)], st, eos=[3, 12, 999])
    assert list(ids) == [0, 3, 6, 9, 12, 15]
    assert list(flags) == [0, 1, 0, 0, 1, 0]
    assert not drew.any() and list(st) == list(range(1, B + 1))
