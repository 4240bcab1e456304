// pz_seq.h -- strictly sequential fp32 sums inside one wave.
//
// The reference accumulates probabilities one by one in fp32
// (top_k.c:53-56, top_p.c:80-105, generate.c:162-168); over a short list
// (the k survivors of top-k) the GPU reproduces those sums exactly by walking
// the lanes in order with v_readlane, so every rounding step is the same.
#pragma once
#include <hip/hip_runtime.h>

__device__ __forceinline__ float pz_readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// s + v[lane 0] + v[lane 1] + ... + v[lane n-1], left to right (n clamped to
// 64).  Wave-uniform result.
__device__ __forceinline__ float pz_seq_sum_lanes(float s, float v, int n) {
  if (n > 64) n = 64;
  for (int j = 0; j < n; j++) s = s + pz_readlane_f(v, j);
  return s;
}

// Inclusive sequential prefix: lane j receives s + v[0] + ... + v[j] summed
// left to right; lanes >= n receive the total over the first n lanes.
__device__ __forceinline__ float pz_seq_scan_lanes(float s, float v, int n) {
  if (n > 64) n = 64;
  const int lane = threadIdx.x & 63;
  float mine = 0.0f;
  for (int j = 0; j < n; j++) {
    s = s + pz_readlane_f(v, j);
    if (lane == j) mine = s;
  }
  return lane < n ? mine : s;
}
