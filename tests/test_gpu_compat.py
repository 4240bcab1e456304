"""The reference-compatible symbols (include/pz_sampling_compat.h) and the
device softmax / temperature operations, on the GPU, against the oracle and
-- when oracle/_ref was built from the reference sources -- against the
reference sampler itself.  Ids, rows and the RNG state after each call must
be identical."""
import ctypes

import numpy as np
import pytest

import pz_oracle as po
import pzsample as pz
from conftest import to_dev

pytestmark = pytest.mark.gpu
_P = ctypes.c_void_p


def ptr(a):
    return a.ctypes.data_as(_P)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def lib(torch_cuda):
    return pz.load()


def rows(n, V, seed):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        x = (rng.standard_normal(V) * rng.uniform(0.5, 4)).astype(np.float32)
        if i % 4 == 1:
            x = np.round(x).astype(np.float32)
        out.append(x)
    return out


def test_rng_matches_reference(lib):
    o = po.oracle()
    for seed in (0, 1, 42, 12345, 2**63 + 5):
        a = ctypes.c_ulonglong()
        b = ctypes.c_ulonglong()
        lib.rng_seed(ctypes.byref(a), seed)
        o.orc_rng_seed(ctypes.byref(b), seed)
        for _ in range(100):
            assert bits(lib.rng_float(ctypes.byref(a))) == bits(o.orc_rng_float(ctypes.byref(b)))
        assert a.value == b.value


def test_argmax_and_temperature(lib):
    o = po.oracle()
    for x in rows(12, 5000, 1):
        assert lib.sample_argmax(ptr(x), x.size) == o.orc_argmax(ptr(x), x.size)
    x = rows(1, 100, 2)[0]
    x[0] = np.nan
    assert lib.sample_argmax(ptr(x), x.size) == 0
    for mode in (pz.PZ_TEMP_MUL_RECIP, pz.PZ_TEMP_DIV):
        lib.pz_compat_set_temp_mode(mode)
        for T in (0.7, 0.8, 1.3, 1e-9):
            x = rows(1, 9999, 3)[0]
            y = x.copy()
            lib.apply_temperature(ptr(x), x.size, ctypes.c_float(T))
            o.orc_apply_temperature(ptr(y), y.size, ctypes.c_float(T), mode)
            assert (bits(x) == bits(y)).all(), (mode, T)
    lib.pz_compat_set_temp_mode(pz.PZ_TEMP_MUL_RECIP)
    assert lib.pz_compat_last_status() == 0


@pytest.mark.parametrize("top_p", [0.5, 0.9, 0.99, 1.0, 0.0, 1.5])
def test_top_p_same_ids_and_rng_state(lib, top_p):
    o = po.oracle()
    for i, x in enumerate(rows(6, 20000, 10)):
        a = ctypes.c_ulonglong(1000 + i)
        b = ctypes.c_ulonglong(1000 + i)
        got = lib.sample_top_p(ptr(x.copy()), x.size, ctypes.c_float(top_p), ctypes.byref(a))
        u = o.orc_rng_float(ctypes.byref(b))
        want = o.orc_top_p(ptr(x), x.size, ctypes.c_float(top_p), ctypes.c_float(u), None)
        assert got == want and a.value == b.value, (i, got, want)


def test_top_p_paths_that_skip_the_draw(lib):
    """NaN maximum and the vocabulary guard return argmax without drawing."""
    x = rows(1, 300, 4)[0]
    x[0] = np.nan
    s = ctypes.c_ulonglong(77)
    assert lib.sample_top_p(ptr(x), x.size, ctypes.c_float(0.9), ctypes.byref(s)) == 0
    assert s.value == 77
    big = rows(1, 200001, 5)[0]
    big[123456] = 50.0
    assert lib.sample_top_p(ptr(big), big.size, ctypes.c_float(0.9), ctypes.byref(s)) == 123456
    assert s.value == 77


@pytest.mark.parametrize("k", [-1, 0, 1, 2, 40, 1024, 2000, 30000])
def test_top_k_same_ids_and_rng_state(lib, k):
    o = po.oracle()
    for i, x in enumerate(rows(5, 25000, 20)):
        a = ctypes.c_ulonglong(50 + i)
        b = ctypes.c_ulonglong(50 + i)
        got = lib.sample_top_k(ptr(x.copy()), x.size, k, ctypes.byref(a))
        u = o.orc_rng_float(ctypes.byref(b))
        want = o.orc_top_k(ptr(x), x.size, k, ctypes.c_float(u), None)
        assert got == want and a.value == b.value, (k, i, got, want)


def test_tn_softmax_bit_exact(lib):
    o = po.oracle()
    for V in (1, 7, 4096, 50000, 151936):
        for x in rows(3, V, V):
            y = x.copy()
            lib.pz_tn_softmax(ptr(x), V)
            o.orc_softmax(ptr(y), V)
            assert (bits(x) == bits(y)).all(), V
    x = rows(1, 1000, 6)[0]
    x[500] = np.nan
    lib.pz_tn_softmax(ptr(x), x.size)
    assert np.isnan(x).all()


def test_device_softmax_and_temperature(torch_cuda):
    o = po.oracle()
    B, V = 16, 128256
    x = pz.synth_normal(B, V, 3.0, 31)
    d_in = to_dev(torch_cuda, x)
    d_out = torch_cuda.empty_like(d_in)
    with pz.Sampler(B, V) as s:
        for mode in (pz.PZ_TEMP_MUL_RECIP, pz.PZ_TEMP_DIV):
            s.set_temp_mode(mode)
            s.softmax(d_in, d_out, B, V, V, V, temperature=0.8)
            s.sync()
            got = d_out.cpu().numpy()
            want = x.copy()
            for b in range(B):
                o.orc_apply_temperature(ptr(want[b]), V, ctypes.c_float(0.8), mode)
                o.orc_softmax(ptr(want[b]), V)
            assert (bits(got) == bits(want)).all(), mode
        s.set_temp_mode(pz.PZ_TEMP_MUL_RECIP)
        d_t = d_in.clone()
        s.temperature(d_t, B, V, V, 0.7)
        s.sync()
        want = x.copy()
        for b in range(B):
            o.orc_apply_temperature(ptr(want[b]), V, ctypes.c_float(0.7), 0)
        assert (bits(d_t.cpu().numpy()) == bits(want)).all()


def test_nan_temperature_is_not_clamped(lib, torch_cuda):
    """temperature.c:10 clamps with T < 1e-6, which a NaN fails: the row
    becomes NaN (x * (1/NaN) or x / NaN), and so does its softmax."""
    o = po.oracle()
    nan = ctypes.c_float(float("nan"))
    for mode in (pz.PZ_TEMP_MUL_RECIP, pz.PZ_TEMP_DIV):
        lib.pz_compat_set_temp_mode(mode)
        x = rows(1, 4099, 8)[0]
        y = x.copy()
        lib.apply_temperature(ptr(x), x.size, nan)
        o.orc_apply_temperature(ptr(y), y.size, nan, mode)
        assert np.isnan(y).all() and np.isnan(x).all(), mode
    lib.pz_compat_set_temp_mode(pz.PZ_TEMP_MUL_RECIP)
    B, V = 3, 5003
    x = pz.synth_normal(B, V, 2.0, 77)
    d_in = to_dev(torch_cuda, x)
    d_out = torch_cuda.empty_like(d_in)
    with pz.Sampler(B, V) as s:
        s.softmax(d_in, d_out, B, V, V, V, temperature=float("nan"))
        s.sync()
        got = d_out.cpu().numpy()
    want = x.copy()
    for b in range(B):
        o.orc_apply_temperature(ptr(want[b]), V, nan, 0)
        o.orc_softmax(ptr(want[b]), V)
    assert np.isnan(want).all() and np.isnan(got).all()


def test_against_reference_binary(lib):
    r = po.ref(True)
    if r is None:
        pytest.skip("oracle/_ref (the reference sampler built from its sources) is not present")
    for i, x in enumerate(rows(8, 30000, 40)):
        a = ctypes.c_ulonglong(9 + i)
        b = ctypes.c_ulonglong(9 + i)
        assert lib.sample_top_p(ptr(x.copy()), x.size, ctypes.c_float(0.9), ctypes.byref(a)) == \
            r.sample_top_p(ptr(x.copy()), x.size, ctypes.c_float(0.9), ctypes.byref(b))
        assert lib.sample_top_k(ptr(x.copy()), x.size, 40, ctypes.byref(a)) == \
            r.sample_top_k(ptr(x.copy()), x.size, 40, ctypes.byref(b))
        assert a.value == b.value
        y1, y2 = x.copy(), x.copy()
        lib.pz_tn_softmax(ptr(y1), x.size)
        r.softmax(ptr(y2), x.size)
        assert (bits(y1) == bits(y2)).all()
