"""The hardware-exp estimate used by the records pass (pz_fast_exp) stays
within the relative error bound the exact-increment test assumes (2^-16),
checked on every fp32 input in [-104, 0] against the glibc-identical pz_expf.
A larger error would let an increment be decided from a wrong estimate."""
import ctypes
import os

import pytest

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "libpzcheck.so")


def test_fast_exp_error_bound(torch_cuda):
    lib = ctypes.CDLL(LIB)
    rel = ctypes.c_float()
    bad = ctypes.c_uint()
    assert lib.pzcheck_exp_bound(ctypes.byref(rel), ctypes.byref(bad)) == 0
    print(f"max relative error {rel.value:.3e} (2^{__import__('math').log2(max(rel.value, 1e-45)):.2f}),"
          f" subnormal-range violations {bad.value}")
    assert rel.value < 2.0 ** -16
    assert bad.value == 0
