// pz_sort.h -- in-workgroup bitonic sort of 64-bit composite keys.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pz_device.h"

// Descending bitonic sort of buf[0..N) (N a power of two) by all BLOCK
// threads of the workgroup.  buf is an LDS (pz_lds_u64*) or global
// (uint64_t*) pointer; global buffers must be owned by the workgroup (every
// stage ends in a workgroup barrier, which also orders the workgroup's
// global accesses).
template <int BLOCK, class Ptr>
__device__ __forceinline__ void pz_bitonic_desc(Ptr buf, int N) {
  for (int size = 2; size <= N; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < (N >> 1); i += BLOCK) {
        const int lo = ((i & ~(stride - 1)) << 1) | (i & (stride - 1));  // stride: power of two
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t a = buf[lo], b = buf[hi];
        if ((a < b) == desc) {
          buf[lo] = b;
          buf[hi] = a;
        }
      }
      __syncthreads();
    }
  }
}

// ---- wave-wide bitonic merges of 64-entry lists held one entry per lane

// The value lane (l ^ D) holds, D a power of two below 64, by VALU lane
// moves only: DPP within rows of 16 lanes for D = 1, 2 (quad_perm [1,0,3,2],
// [2,3,0,1]), 4 (row_shl:4 where bit 2 of the lane is clear, row_shr:4
// where it is set) and 8 (row_ror:8); gfx950's v_permlane16_swap and
// v_permlane32_swap for 16 and 32 (with both operands the value itself,
// lanes with bit D set find the partner's value in the first result and
// the others in the second).
__device__ __forceinline__ uint32_t pz_lane_xor_u32_16(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return (threadIdx.x & 16u) ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t pz_lane_xor_u32_32(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (threadIdx.x & 32u) ? r[0] : r[1];
}

template <int D>
__device__ __forceinline__ uint64_t pz_lane_xor_u64(uint64_t v) {
  const int lo = (int)(uint32_t)v, hi = (int)(uint32_t)(v >> 32);
  int a, b;
  if constexpr (D == 1 || D == 2 || D == 8) {
    constexpr int ctrl = D == 1 ? 0xb1 : (D == 2 ? 0x4e : 0x128);
    a = __builtin_amdgcn_update_dpp(0, lo, ctrl, 0xf, 0xf, false);
    b = __builtin_amdgcn_update_dpp(0, hi, ctrl, 0xf, 0xf, false);
  } else if constexpr (D == 4) {
    const int al = __builtin_amdgcn_update_dpp(0, lo, 0x104, 0xf, 0xf, false);  // lane + 4
    const int bl = __builtin_amdgcn_update_dpp(0, hi, 0x104, 0xf, 0xf, false);
    const int ar = __builtin_amdgcn_update_dpp(0, lo, 0x114, 0xf, 0xf, false);  // lane - 4
    const int br = __builtin_amdgcn_update_dpp(0, hi, 0x114, 0xf, 0xf, false);
    const bool up = (threadIdx.x & 4u) != 0u;
    a = up ? ar : al;
    b = up ? br : bl;
  } else if constexpr (D == 16) {
    a = (int)pz_lane_xor_u32_16((uint32_t)lo);
    b = (int)pz_lane_xor_u32_16((uint32_t)hi);
  } else {
    static_assert(D == 32, "lane distance");
    a = (int)pz_lane_xor_u32_32((uint32_t)lo);
    b = (int)pz_lane_xor_u32_32((uint32_t)hi);
  }
  return ((uint64_t)(uint32_t)b << 32) | (uint32_t)a;
}

// The value lane 63 - l holds (a list's order reversed).
__device__ __forceinline__ uint64_t pz_lane_rev_u64(uint64_t v) {
  const int addr = (63 - (int)(threadIdx.x & 63u)) << 2;
  const int a = __builtin_amdgcn_ds_bpermute(addr, (int)(uint32_t)v);
  const int b = __builtin_amdgcn_ds_bpermute(addr, (int)(uint32_t)(v >> 32));
  return ((uint64_t)(uint32_t)b << 32) | (uint32_t)a;
}

// One half-cleaner of a bitonic sequence over the wave: lanes l and l ^ D
// exchange so that the lower lane holds the larger (desc) or the smaller.
template <int D>
__device__ __forceinline__ uint64_t pz_half_clean_u64(uint64_t c, bool desc) {
  const uint64_t o = pz_lane_xor_u64<D>(c);
  const bool keep_max = ((threadIdx.x & (unsigned)D) == 0u) == desc;
  const bool take = keep_max ? o > c : o < c;
  return take ? o : c;
}

// a sorted descending over the lanes, b ascending: the 64 largest of the
// 128, sorted descending (desc) or ascending.  max(a, b) lane by lane is the
// upper half of the first half-cleaner of the 128-entry bitonic sequence
// a ++ b, itself bitonic; six half-cleaners sort it.
__device__ __forceinline__ uint64_t pz_wave_merge_u64(uint64_t a, uint64_t b, bool desc) {
  uint64_t c = a > b ? a : b;
  c = pz_half_clean_u64<32>(c, desc);
  c = pz_half_clean_u64<16>(c, desc);
  c = pz_half_clean_u64<8>(c, desc);
  c = pz_half_clean_u64<4>(c, desc);
  c = pz_half_clean_u64<2>(c, desc);
  c = pz_half_clean_u64<1>(c, desc);
  return c;
}
