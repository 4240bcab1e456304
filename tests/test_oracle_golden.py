"""The CPU oracle against the reference sampler itself.

Pins: the golden fixtures written by tests/golden/make_golden.py from the
reference's own C sources (compiled by oracle/Makefile), the known answers of
the reference's tests/test_sampling.c, and -- when oracle/_ref is built --
a direct comparison with the reference binary on fresh seeded rows.
"""
import ctypes
import hashlib
import json
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import pz_oracle as po  # noqa: E402
from make_golden import gen_rows  # noqa: E402

_P = ctypes.c_void_p
GOLD = os.path.join(HERE, "golden")


def load(name):
    with open(os.path.join(GOLD, name + ".json")) as f:
        return json.load(f)


def f32bits(v):
    return int(np.float32(v).view(np.uint32))


def orc_u(seed):
    o = po.oracle()
    s = ctypes.c_ulonglong()
    o.orc_rng_seed(ctypes.byref(s), seed)
    return o.orc_rng_float(ctypes.byref(s))


def test_rng_golden():
    o = po.oracle()
    for case in load("rng"):
        s = ctypes.c_ulonglong()
        o.orc_rng_seed(ctypes.byref(s), case["seed"])
        draws = [f32bits(o.orc_rng_float(ctypes.byref(s))) for _ in range(256)]
        assert draws == case["draws_f32bits"], case["seed"]
        assert s.value == case["state_after"]


def test_rng_closed_form():
    """xorshift64* by hand for one step (rng.c:11-16) and the seed-0 rule (:5)."""
    o = po.oracle()
    s = ctypes.c_ulonglong()
    o.orc_rng_seed(ctypes.byref(s), 0)
    assert s.value == 1
    x = 1
    x ^= x >> 12
    x = (x ^ (x << 25)) & (2**64 - 1)
    x ^= x >> 27
    want = np.float32(np.float32((x * 0x2545F4914F6CDD1D % 2**64) >> 33) / np.float32(2**31))
    assert o.orc_rng_float(ctypes.byref(s)) == want
    assert s.value == x


def test_rng_can_return_one():
    """(float)(k) rounds to 2^31 for k >= 2^31 - 64, so rng_float returns 1.0f."""
    assert np.float32(2**31 - 64) == np.float32(2**31)
    assert np.float32(2**31 - 65) < np.float32(2**31)


@pytest.mark.parametrize("vals,want", [
    ([1.0, 3.0, 2.0, 0.5], 1),      # tests/test_sampling.c:76-80
    ([10.0, 3.0, 2.0, 0.5], 0),     # :82-86
    ([1.0, 2.0, 3.0, 100.0], 3),    # :88-92
    ([-5.0, -1.0, -3.0, -2.0], 1),  # :94-98
    ([42.0], 0),                    # :100-104
    ([2.0, 5.0, 5.0, 1.0], 1),      # tie -> lowest id (strict '>' in argmax.c:7)
    ([np.nan, 5.0, 7.0], 0),        # NaN at x[0] is never replaced (argmax.c:5)
    ([1.0, np.nan, 0.5], 0),
    ([-np.inf, -np.inf], 0),
    ([-0.0, 0.0], 0),               # -0 == +0 under '>'
])
def test_argmax_known_answers(vals, want):
    x = np.array(vals, np.float32)
    assert po.oracle().orc_argmax(x.ctypes.data_as(_P), len(x)) == want


def test_argmax_golden():
    o = po.oracle()
    for c in load("argmax"):
        x = gen_rows(c["kind"], c["rows"], c["V"], c["seed"], **c["kw"])
        got = [o.orc_argmax(x[i].ctypes.data_as(_P), c["V"]) for i in range(c["rows"])]
        assert got == c["ids"]


def test_temperature_golden():
    o = po.oracle()
    for c in load("temperature"):
        x = gen_rows("normal", c["rows"], c["V"], c["seed"], sigma=3.0)
        mode = po.TEMP_MUL_RECIP if c["form"] == "mul_recip" else po.TEMP_DIV
        for i in range(c["rows"]):
            o.orc_apply_temperature(x[i].ctypes.data_as(_P), c["V"], c["T"], mode)
        assert hashlib.sha256(x.tobytes()).hexdigest() == c["sha256"], (c["T"], c["form"])


def test_temperature_forms_differ():
    """The two builds of temperature.c disagree on some inputs at T=0.8, so
    the form is a real parameter (it is pinned per form above)."""
    x = gen_rows("normal", 1, 49152, 7, sigma=3.0)[0]
    a, b = x.copy(), x.copy()
    o = po.oracle()
    o.orc_apply_temperature(a.ctypes.data_as(_P), len(a), 0.8, po.TEMP_MUL_RECIP)
    o.orc_apply_temperature(b.ctypes.data_as(_P), len(b), 0.8, po.TEMP_DIV)
    frac = np.mean(a != b)
    assert 0.05 < frac < 0.3


def test_softmax_golden():
    o = po.oracle()
    for c in load("softmax"):
        x = gen_rows("normal", c["rows"], c["V"], c["seed"], sigma=c["sigma"])
        for i in range(c["rows"]):
            o.orc_softmax(x[i].ctypes.data_as(_P), c["V"])
        assert hashlib.sha256(x.tobytes()).hexdigest() == c["sha256"]
        assert [f32bits(x[i, 0]) for i in range(c["rows"])] == c["p0_f32bits"]
        # The reference's sequential fp32 sum drops terms below half an ulp of
        # the running sum, so its normaliser is low and the probabilities sum
        # slightly above 1 at large V (4e-5 at V=49152): tolerance scales with V.
        tol = 1e-5 if c["V"] <= 1000 else 2e-4
        assert np.all(np.abs(x.sum(axis=1, dtype=np.float64) - 1.0) < tol)


def test_softmax_known_answers():
    """tests/test_math.c:70-88 and tests/audit_math.c:19-33."""
    o = po.oracle()
    x = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    o.orc_softmax(x.ctypes.data_as(_P), 4)
    assert abs(float(x.sum()) - 1.0) < 1e-5 and x[3] > x[2] > x[1]
    x = np.array([1000.0, 1001.0, 999.0], np.float32)
    o.orc_softmax(x.ctypes.data_as(_P), 3)
    assert abs(float(x.sum()) - 1.0) < 1e-5 and x[1] > x[0]
    x = np.array([1e10, 1e10, 10.0, -1e10, -1e10, 0, 0, 0], np.float32)
    o.orc_softmax(x.ctypes.data_as(_P), 8)
    assert not np.isnan(x).any()
    assert abs(x[0] - 0.5) < 1e-4 and abs(x[1] - 0.5) < 1e-4 and x[2] < 1e-4


def test_top_k_golden():
    o = po.oracle()
    for c in load("top_k"):
        x = gen_rows(c["kind"], c["rows"], c["V"], c["seed"], **c["kw"])
        got = []
        for i in range(c["rows"]):
            u = orc_u(c["draw_seed_base"] * (i + 1) + c["k"])
            got.append(o.orc_top_k(x[i].ctypes.data_as(_P), c["V"], c["k"], u, None))
        assert got == c["ids"], (c["kind"], c["k"])


def test_top_p_golden():
    for c in load("top_p"):
        x = gen_rows(c["kind"], c["rows"], c["V"], c["seed"], **c["kw"])
        got = []
        for i in range(c["rows"]):
            u = orc_u(c["draw_seed_base"] * (i + 1) + int(c["top_p"] * 1000))
            rid, _ = po.sample_row(x[i], po.params(temperature=c["T"], top_p=c["top_p"]), u=u)
            got.append(rid)
        assert got == c["ids"], (c["kind"], c["top_p"])


def test_top_k_reference_tests():
    """Known answers of tests/test_sampling.c:195-245 and test_bugfixes.c:34-92."""
    o = po.oracle()
    x = np.array([1.0, 5.0, 3.0, 2.0], np.float32)
    for t in range(20):
        assert o.orc_top_k(x.ctypes.data_as(_P), 4, 1, orc_u(42 + t), None) == 1
    x = np.array([1.0, 10.0, 100.0, 0.1], np.float32)
    for t in range(50):
        assert o.orc_top_k(x.ctypes.data_as(_P), 4, 2, orc_u(42 + t), None) in (1, 2)
    x = np.arange(32, dtype=np.float32)
    assert 0 <= o.orc_top_k(x.ctypes.data_as(_P), 32, 5000, orc_u(42), None) < 32
    for k in (0, -5):
        assert 0 <= o.orc_top_k(x.ctypes.data_as(_P), 32, k, orc_u(1), None) < 32
    # no logit above -1e30: every slot keeps index -1 (top_k.c:29-32)
    x = np.full(8, -np.inf, np.float32)
    assert o.orc_top_k(x.ctypes.data_as(_P), 8, 3, 0.5, None) == -1


def test_top_p_reference_tests():
    """tests/test_sampling.c:155-189."""
    x = np.array([-100.0, 100.0, -100.0, -100.0], np.float32)
    for t in range(20):
        rid, _ = po.sample_row(x, po.params(temperature=1.0, top_p=0.5), u=orc_u(42 + t))
        assert rid == 1
    seen = set()
    o = po.oracle()
    s = ctypes.c_ulonglong()
    o.orc_rng_seed(ctypes.byref(s), 42)
    for t in range(200):
        u = o.orc_rng_float(ctypes.byref(s))
        info = po.OrcInfo()
        z = np.zeros(4, np.float32)
        rid = o.orc_top_p(z.ctypes.data_as(_P), 4, 1.0, u, ctypes.byref(info))
        seen.add(rid)
    assert len(seen) >= 3


@pytest.mark.skipif(po.ref(True) is None, reason="oracle/_ref not built here")
def test_oracle_equals_reference_binary_fresh_rows():
    """Fresh seeds (not in the fixtures): restatement == compiled reference."""
    r = po.ref(True)
    o = po.oracle()
    rng = np.random.default_rng(123)
    for trial in range(40):
        V = int(rng.integers(1, 3000))
        x = (rng.standard_normal(V) * rng.uniform(0.1, 8)).astype(np.float32)
        if trial % 5 == 0:
            x = np.round(x).astype(np.float32)  # ties
        seed = int(rng.integers(1, 2**63))
        # argmax
        assert r.sample_argmax(x.ctypes.data_as(_P), V) == o.orc_argmax(x.ctypes.data_as(_P), V)
        # top-k
        k = int(rng.integers(-2, 60))
        s = ctypes.c_ulonglong(seed)
        want = r.sample_top_k(x.copy().ctypes.data_as(_P), V, k, ctypes.byref(s))
        assert o.orc_top_k(x.ctypes.data_as(_P), V, k, orc_u(seed), None) == want
        # temperature + top-p
        T = float(rng.uniform(0.3, 1.5))
        p = float(rng.uniform(0.05, 0.999))
        y = x.copy()
        r.apply_temperature(y.ctypes.data_as(_P), V, ctypes.c_float(T))
        s = ctypes.c_ulonglong(seed)
        want = r.sample_top_p(y.ctypes.data_as(_P), V, ctypes.c_float(p), ctypes.byref(s))
        rid, _ = po.sample_row(x, po.params(temperature=T, top_p=p), u=orc_u(seed))
        assert rid == want
