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
