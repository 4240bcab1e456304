// pz_lmhead.hip -- the LM head producing the sampler's logits on the device,
// and the same product with greedy argmax fused into its epilogue.
//
// Reference: src/transformer/forward.c:102-168 runs the classifier
// parallel_matmul_bf16 (src/math/parallel_matmul.c:283-414):
//   logits[i] = sum_j bf16(W[i, j]) * x[j]
// with W [V, n] row-major bf16 (the upper half of an fp32; widening is a
// 16-bit shift), x the fp32 final-norm activations and fp32 accumulation.
// Here B activation rows are done at once: logits[b, i] = W[i, :] . x[b, :].
//
// Layout and schedule (HBM-bound: W is read once per batch tile, 2 bytes per
// weight):
//   * a workgroup of 4 waves owns 64 consecutive rows of W; the batch tile of
//     x (BT rows x n fp32) is staged in LDS once per workgroup;
//   * a wave takes 4 rows of W at a time; lane l covers elements
//     512 c + 8 l .. +7 of every row (one 16-byte load per row per c), so a
//     wave keeps 4 x n/512 loads in flight;
//   * each lane accumulates with fused multiply-adds in a fixed order (c,
//     then the 8 elements), and a DPP tree sums the 64 lanes.
// The order differs from the reference's AVX-512 accumulators, so logits
// agree with an exact product to fp32 rounding, not bit for bit; the fused
// argmax sees exactly the values the unfused kernel writes, because both are
// the same template.
//
// Fused epilogue (greedy, src/sampling/argmax.c:3-13): the first maximum by
// strict '>' is the largest value with the lowest id among equals, NaN never
// winning, and a NaN logit at id 0 returns 0.  Each workgroup reduces its
// rows to one 64-bit key per batch row -- the order key of the value above,
// ~id below -- and takes the atomic maximum in global memory; the workgroup
// that owns id 0 records whether logit 0 is NaN.  A finishing kernel turns
// keys into ids and clears them for the next call.
#include <hip/hip_runtime.h>

#include "../../include/pz_sampler.h"
#include "pz_device.h"
#include "pz_sampler_impl.h"

namespace {

constexpr int LM_WAVES = 4;
constexpr int LM_RW = 4;                        // rows per wave step
constexpr int LM_ROWS = 64;                     // rows per workgroup
constexpr int LM_STEPS = LM_ROWS / (LM_WAVES * LM_RW);
constexpr size_t LM_LDS_MAX = 96 * 1024;        // x tile budget

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// The 8 weights of one 16-byte load (little-endian: element 2k is the low
// half of word k).
__device__ __forceinline__ void widen8(const uint4 q, float (&w)[8]) {
  w[0] = __uint_as_float(q.x << 16);
  w[1] = __uint_as_float(q.x & 0xffff0000u);
  w[2] = __uint_as_float(q.y << 16);
  w[3] = __uint_as_float(q.y & 0xffff0000u);
  w[4] = __uint_as_float(q.z << 16);
  w[5] = __uint_as_float(q.z & 0xffff0000u);
  w[6] = __uint_as_float(q.w << 16);
  w[7] = __uint_as_float(q.w & 0xffff0000u);
}

__device__ __forceinline__ uint64_t argmax_key(float v, int id) {
  return ((uint64_t)pz_key(v) << 32) | (uint64_t)(0xffffffffu - (uint32_t)id);
}

// MODE 0: write logits.  MODE 1: argmax keys.  VEC: n % 8 == 0 and W 16-byte
// aligned (one 16-byte load per 8 weights), else element loads.
template <int BT, int MODE, bool VEC>
__global__ __launch_bounds__(64 * LM_WAVES) void k_lmhead(
    const uint16_t* __restrict__ W, int V, int n, const float* __restrict__ X, long ldx, int nb,
    float* __restrict__ logits, long ld, unsigned long long* __restrict__ keys,
    uint8_t* __restrict__ nan0) {
  extern __shared__ __align__(16) float xs[];  // [BT][n]
  __shared__ unsigned long long best_sh[LM_WAVES][BT];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int b = 0; b < BT; b++)
    for (int j = tid; j < n; j += 64 * LM_WAVES)
      xs[b * n + j] = b < nb ? X[(size_t)b * ldx + j] : 0.0f;
  __syncthreads();
  unsigned long long best[BT];
#pragma unroll
  for (int b = 0; b < BT; b++) best[b] = 0ull;
  const int nchunk = (n + 511) >> 9;
  for (int step = 0; step < LM_STEPS; step++) {
    const int r0 = blockIdx.x * LM_ROWS + (step * LM_WAVES + w) * LM_RW;
    if (r0 >= V) break;  // whole wave
    float acc[LM_RW][BT];
#pragma unroll
    for (int r = 0; r < LM_RW; r++)
#pragma unroll
      for (int b = 0; b < BT; b++) acc[r][b] = 0.0f;
    for (int c = 0; c < nchunk; c++) {
      const int k = c * 512 + lane * 8;
      float wv[LM_RW][8];
#pragma unroll
      for (int r = 0; r < LM_RW; r++) {
        const int row = r0 + r < V ? r0 + r : V - 1;  // rows past V: a valid row, result unused
        const uint16_t* wr = W + (size_t)row * n;
        if (VEC) {
          uint4 q = make_uint4(0u, 0u, 0u, 0u);
          if (k < n) q = *reinterpret_cast<const uint4*>(wr + k);
          widen8(q, wv[r]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; e++) wv[r][e] = k + e < n ? bf16_to_f32(wr[k + e]) : 0.0f;
        }
      }
#pragma unroll
      for (int b = 0; b < BT; b++) {
        float xv[8];
#pragma unroll
        for (int e = 0; e < 8; e++) xv[e] = k + e < n ? xs[b * n + k + e] : 0.0f;
#pragma unroll
        for (int r = 0; r < LM_RW; r++)
#pragma unroll
          for (int e = 0; e < 8; e++) acc[r][b] = __builtin_fmaf(wv[r][e], xv[e], acc[r][b]);
      }
    }
#pragma unroll
    for (int r = 0; r < LM_RW; r++) {
      const int row = r0 + r;
#pragma unroll
      for (int b = 0; b < BT; b++) {
        const float v = pz_wave_sum(acc[r][b]);  // uniform
        if (row < V && b < nb) {
          if (MODE == 0) {
            if (lane == 0) logits[(size_t)b * ld + row] = v;
          } else {
            if (row == 0 && lane == 0) nan0[b] = v != v ? 1 : 0;
            if (!(v != v)) {
              const unsigned long long kk = argmax_key(v, row);
              best[b] = kk > best[b] ? kk : best[b];
            }
          }
        }
      }
    }
  }
  if (MODE == 1) {
    if (lane == 0)
#pragma unroll
      for (int b = 0; b < BT; b++) best_sh[w][b] = best[b];
    __syncthreads();
    if (tid < BT && tid < nb) {
      unsigned long long m = best_sh[0][tid];
      for (int i = 1; i < LM_WAVES; i++) m = best_sh[i][tid] > m ? best_sh[i][tid] : m;
      if (m) atomicMax(&keys[tid], m);
    }
  }
}

// Keys to ids (argmax.c:3-13); clears the keys for the next call.
__global__ void k_lmhead_finish(int B, unsigned long long* keys, const uint8_t* nan0,
                                int32_t* ids) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const unsigned long long k = keys[b];
  // logit 0 NaN: argmax.c returns 0; no key at all means every logit was NaN,
  // logit 0 among them
  ids[b] = nan0[b] || !k ? 0 : (int32_t)(0xffffffffu - (uint32_t)(k & 0xffffffffull));
  keys[b] = 0ull;
}

template <int BT, int MODE>
int launch_tile(pz_sampler* s, const uint16_t* d_w, int V, int n, const float* x, long ldx, int nb,
                float* out, long ld, unsigned long long* keys, uint8_t* nan0) {
  const bool vec = n % 8 == 0 && ((uintptr_t)d_w & 15) == 0;
  auto k = vec ? k_lmhead<BT, MODE, true> : k_lmhead<BT, MODE, false>;
  const size_t lds = (size_t)BT * n * sizeof(float);
  if (lds > 65536)
    PZ_HIP(s, hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)lds));
  const int grid = (V + LM_ROWS - 1) / LM_ROWS;
  hipLaunchKernelGGL(k, dim3(grid), dim3(64 * LM_WAVES), lds, s->stream, d_w, V, n, x, ldx, nb,
                     out, ld, keys, nan0);
  PZ_HIP(s, hipGetLastError());
  return PZ_OK;
}

// Batch tile: the largest of 8, 4, 2, 1 not above B whose x tile fits the
// LDS budget (0: n too large even for one row).
int tile_for(int B, int n) {
  for (int bt = 8; bt >= 1; bt >>= 1)
    if (bt <= B && (size_t)bt * n * sizeof(float) <= LM_LDS_MAX) return bt;
  return (size_t)n * sizeof(float) <= LM_LDS_MAX ? 1 : 0;
}

template <int MODE>
int run(pz_sampler* s, const uint16_t* d_w, int V, int n, const float* d_x, int B, long ldx,
        float* d_logits, long ld) {
  const int bt = tile_for(B, n);
  if (!bt) return fail(s, PZ_ENOTSUP, "n=%d: the activation row does not fit in LDS", n);
  for (int b0 = 0; b0 < B; b0 += bt) {
    const int nb = B - b0 < bt ? B - b0 : bt;
    const float* x = d_x + (size_t)b0 * ldx;
    float* out = MODE == 0 ? d_logits + (size_t)b0 * ld : nullptr;
    unsigned long long* keys = s->d_lmh_keys + b0;
    uint8_t* nan0 = s->d_lmh_nan + b0;
    int rc;
    switch (bt) {
      case 8: rc = launch_tile<8, MODE>(s, d_w, V, n, x, ldx, nb, out, ld, keys, nan0); break;
      case 4: rc = launch_tile<4, MODE>(s, d_w, V, n, x, ldx, nb, out, ld, keys, nan0); break;
      case 2: rc = launch_tile<2, MODE>(s, d_w, V, n, x, ldx, nb, out, ld, keys, nan0); break;
      default: rc = launch_tile<1, MODE>(s, d_w, V, n, x, ldx, nb, out, ld, keys, nan0); break;
    }
    if (rc != PZ_OK) return rc;
  }
  return PZ_OK;
}

int check(pz_sampler* s, const uint16_t* d_w, int V, int n, const float* d_x, int B, long ldx) {
  if (!d_w || !d_x || V <= 0 || n <= 0 || B < 0 || ldx < n)
    return fail(s, PZ_EINVAL, "bad LM head shape");
  if (B > s->max_batch) return fail(s, PZ_ERANGE, "B=%d > max_batch=%d", B, s->max_batch);
  return PZ_OK;
}

}  // namespace

extern "C" int pz_lm_head_bf16(pz_sampler* s, const uint16_t* d_w, int V, int n, const float* d_x,
                               int B, long ldx, float* d_logits, long ld) {
  if (!s) return PZ_EINVAL;
  const int rc = check(s, d_w, V, n, d_x, B, ldx);
  if (rc != PZ_OK) return rc;
  if (!d_logits || ld < V) return fail(s, PZ_EINVAL, "bad logits buffer");
  if (B == 0) return PZ_OK;
  PZ_HIP(s, hipSetDevice(s->device));
  return run<0>(s, d_w, V, n, d_x, B, ldx, d_logits, ld);
}

extern "C" int pz_lm_head_argmax_bf16(pz_sampler* s, const uint16_t* d_w, int V, int n,
                                      const float* d_x, int B, long ldx, int32_t* d_ids) {
  if (!s) return PZ_EINVAL;
  const int rc = check(s, d_w, V, n, d_x, B, ldx);
  if (rc != PZ_OK) return rc;
  if (!d_ids) return fail(s, PZ_EINVAL, "null ids");
  if (B == 0) return PZ_OK;
  PZ_HIP(s, hipSetDevice(s->device));
  const int r = run<1>(s, d_w, V, n, d_x, B, ldx, nullptr, 0);
  if (r != PZ_OK) return r;
  hipLaunchKernelGGL(k_lmhead_finish, dim3((B + 255) / 256), dim3(256), 0, s->stream, B,
                     s->d_lmh_keys, s->d_lmh_nan, d_ids);
  PZ_HIP(s, hipGetLastError());
  return PZ_OK;
}
