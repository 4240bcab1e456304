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

// Inclusive sequential prefix: lane j receives ((s + v[0]) + v[1]) + ... +
// v[j], the additions of a left-to-right loop started at s, in its order;
// lanes >= n receive the total over the first n lanes (n clamped to 64,
// wave-uniform).  A systolic chain of DPP adds: lane 0 holds s + v[0], and
// at every step each lane j > 0 adds its v[j] to lane j-1's value of the
// step before (wave_shr:1), so lane j holds its final value from step j on
// and keeps it through further steps; the steps run in groups of eight with
// no branch inside a group.  s must not be -0.0 (lane 0 receives +0.0 from
// the shift), which no sum started at +0.0 is.
__device__ __forceinline__ float pz_seq_scan_lanes(float s, float v, int n) {
  if (n > 64) n = 64;
  if (n <= 0) return s;
  const int lane = threadIdx.x & 63;
  const float w = lane == 0 ? s + v : v;
  float c = w;
  for (int g = 1; g < n; g += 8) {
#pragma unroll
    for (int t = 0; t < 8; t++)
      c = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(c), 0x138, 0xf, 0xf,
                                                     true)) + w;
  }
  const float tot = pz_readlane_f(c, n - 1);
  return lane < n ? c : tot;
}

// s + v[lane 0] + v[lane 1] + ... + v[lane n-1], left to right (n clamped to
// 64; s not -0.0).  Wave-uniform result.
__device__ __forceinline__ float pz_seq_sum_lanes(float s, float v, int n) {
  if (n > 64) n = 64;
  if (n <= 0) return s;
  return pz_readlane_f(pz_seq_scan_lanes(s, v, n), n - 1);
}

// The sequential fp32 sum, from +0.0, of the 256 terms a wave holds in id
// order (lane l: t[0..3] = terms 4l .. 4l+3), in every lane: the DPP chain
// of pz_seq_scan_lanes with each lane's four terms added in turn, 64 steps
// (lane j holds ((x + t0) + t1) + t2) + t3 over lane j-1's value x from step
// j on).  Terms must not be -0.0 where every term before them is zero.
__device__ __forceinline__ float pz_seq_sum_seg4(const float (&t)[4]) {
  float c = 0.0f;
  for (int s = 0; s < 64; s += 8) {
#pragma unroll
    for (int u = 0; u < 8; u++) {
      c = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(c), 0x138, 0xf, 0xf,
                                                     true)) + t[0];
      c = c + t[1];
      c = c + t[2];
      c = c + t[3];
    }
  }
  return pz_readlane_f(c, 63);
}
