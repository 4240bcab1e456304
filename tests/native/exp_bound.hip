// GPU check of the estimate behind the records pass: for every fp32 d in
// [-104, 0], pz_fast_exp(d) must lie within (|d| + 2) * 2^-23 (relative) of
// the exact pz_expf(d) whenever expf(d) is a normal number, and stay below
// 2^-120 when it is not.  Test infrastructure (tests/test_gpu_exp_bound.py); built by
// tests/native/Makefile.
#include <hip/hip_runtime.h>

#include "pz_rowpass.h"

__global__ void k_exp_bound(uint32_t lo_bits, uint32_t count, unsigned int* out) {
  const uint32_t stride = gridDim.x * blockDim.x;
  float worst = 0.0f, worst_ratio = 0.0f;
  unsigned int small_bad = 0;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    const float d = __uint_as_float(lo_bits + i);  // 0x80000000 + i: -0 ... more negative
    const float e = pz_expf(d);
    const float a = pz_fast_exp(d);
    if (e >= 0x1p-126f) {
      // relative error in double (exact for these fp32 values), and its
      // ratio to the bound (|d| + 2) * 2^-23 the records pass relies on
      const double rel = fabs((double)a - (double)e) / (double)e;
      worst = fmaxf(worst, (float)rel);
      worst_ratio = fmaxf(worst_ratio, (float)(rel / (((double)fabsf(d) + 2.0) * 0x1p-23)));
    } else if (!(a < 0x1p-120f)) {
      small_bad++;
    }
  }
  atomicMax(&out[0], __float_as_uint(worst));
  atomicMax(&out[2], __float_as_uint(worst_ratio));
  if (small_bad) atomicAdd(&out[1], small_bad);
}

extern "C" int pzcheck_exp_bound(float* max_rel, unsigned int* n_bad_small, float* max_ratio) {
  unsigned int* d = nullptr;
  if (hipMalloc(&d, 12) != hipSuccess) return -1;
  if (hipMemset(d, 0, 12) != hipSuccess) return -1;
  const uint32_t lo = 0x80000000u;                           // -0.0
  const uint32_t hi = __builtin_bit_cast(uint32_t, -104.0f);  // 0xc2d00000
  const uint32_t count = hi - lo + 1u;
  hipLaunchKernelGGL(k_exp_bound, dim3(16384), dim3(256), 0, 0, lo, count, d);
  unsigned int h[3] = {0, 0, 0};
  if (hipMemcpy(h, d, 12, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  hipFree(d);
  *max_rel = __builtin_bit_cast(float, h[0]);
  *n_bad_small = h[1];
  *max_ratio = __builtin_bit_cast(float, h[2]);
  return 0;
}

// The same hash as oracle/pz_oracle.c orc_expf_hash, of the GPU's pz_expf.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z ^= z >> 33;
  z *= 0xff51afd7ed558ccdULL;
  z ^= z >> 33;
  z *= 0xc4ceb9fe1a85ec53ULL;
  z ^= z >> 33;
  return z;
}

__global__ void k_expf_hash(uint32_t lo, uint64_t n, uint32_t stride,
                            unsigned long long* out) {
  unsigned long long h = 0;
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
       i += (uint64_t)gridDim.x * blockDim.x) {
    const uint32_t b = lo + (uint32_t)(i * stride);
    const float r = pz_expf(__uint_as_float(b));
    h += mix64(((uint64_t)__float_as_uint(r) << 32) | b);
  }
  atomicAdd(out, h);
}

extern "C" int pzcheck_expf_hash(uint32_t lo, uint32_t hi, uint32_t stride, uint64_t* hash) {
  unsigned long long* d = nullptr;
  if (hipMalloc(&d, 8) != hipSuccess) return -1;
  if (hipMemset(d, 0, 8) != hipSuccess) return -1;
  const uint64_t n = ((uint64_t)hi - lo) / stride + 1;
  hipLaunchKernelGGL(k_expf_hash, dim3(16384), dim3(256), 0, 0, lo, n, stride, d);
  unsigned long long h = 0;
  if (hipMemcpy(&h, d, 8, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  hipFree(d);
  *hash = h;
  return 0;
}
