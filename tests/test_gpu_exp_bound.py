"""The hardware-exp estimate used by the records pass (pz_fast_exp) stays
within the relative error bound the exact-increment test assumes,
(|d| + 2) * 2^-23 for exp(d), checked on every fp32 input in [-104, 0]
against the glibc-identical pz_expf.  A larger error would let an increment
be decided from a wrong estimate."""
import ctypes
import os

import pytest

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "libpzcheck.so")


def test_fast_exp_error_bound(torch_cuda):
    lib = ctypes.CDLL(LIB)
    rel = ctypes.c_float()
    bad = ctypes.c_uint()
    ratio = ctypes.c_float()
    assert lib.pzcheck_exp_bound(ctypes.byref(rel), ctypes.byref(bad), ctypes.byref(ratio)) == 0
    print(f"max relative error {rel.value:.3e} (2^{__import__('math').log2(max(rel.value, 1e-45)):.2f}),"
          f" max error / ((|d| + 2) 2^-23) = {ratio.value:.3f},"
          f" subnormal-range violations {bad.value}")
    assert rel.value < 2.0 ** -16
    assert ratio.value <= 1.0
    assert bad.value == 0


@pytest.mark.parametrize("lo,hi,stride", [
    (0x80000000, 0xC2D00000, 1),   # every fp32 in [-104, -0]: the sampler's exponents
    (0xC2D00000, 0xFF800000, 97),  # the underflowing tail down to -inf (sampled)
    (0x00000000, 0x42B20000, 13),  # positive arguments up to 89 (sampled)
])
def test_gpu_expf_is_bit_identical_to_libm(torch_cuda, lo, hi, stride):
    """pz_expf (the GPU's exponential, a restatement of glibc's table-driven
    expf) against the host libm expf the reference links, compared through an
    order-independent 64-bit hash of every (input, result) pair."""
    import pz_oracle as po
    lib = ctypes.CDLL(LIB)
    lib.pzcheck_expf_hash.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                      ctypes.POINTER(ctypes.c_uint64)]
    g = ctypes.c_uint64()
    assert lib.pzcheck_expf_hash(lo, hi, stride, ctypes.byref(g)) == 0
    h = po.oracle().orc_expf_hash(lo, hi, stride)
    print(f"range {lo:#x}..{hi:#x} stride {stride}: gpu {g.value:#018x} libm {h:#018x}")
    assert g.value == h
