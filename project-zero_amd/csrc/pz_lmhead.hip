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
// Batch 4 and up run on the matrix cores (k_lmhead_mfma, below).  Batches of
// 1 to 3 use the vector kernel.
//
// Vector kernel layout and schedule (HBM-bound: W is read once per batch
// tile, 2 bytes per weight):
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

// ---- batch >= 4: bf16 MFMA ---------------------------------------------------
// logits[b, i] = W[i, :] . x[b, :] as a GEMM on the matrix cores.  Each fp32
// activation is split into three bf16 parts, x = x0 + x1 + x2 (its 24
// significant bits in three 8-bit pieces, by truncation: exact for finite x;
// an infinite or NaN x keeps x0 = x and zero parts), so every bf16 x bf16
// product is exact in fp32 and the sum of the three part-products per weight
// is the fp32-accumulated product the reference forms -- the order of the
// fp32 additions differs (as it does in the VALU kernel), inside the same
// summation bound.  A weight of +-inf would meet a zero part (inf * 0 = NaN
// where the reference has +-inf): rows holding one are flagged while they
// stream and recomputed with fp32 fused multiply-adds in the epilogue.
//   * v_mfma_f32_16x16x32_bf16: A = 16 rows of W x 32 k (lane l: row l % 16,
//     its 8 k of group l / 16, one 16-byte load), B = 32 k x 16 batch rows of
//     one part (the same k per lane from LDS), D = 16 rows x 16 batch rows
//     (lane l: batch row l % 16, rows 4 (l / 16) .. +3);
//   * a workgroup of 8 waves owns LMM_ROWS = 256 rows of W (2 tiles of 16 per
//     wave; two workgroups per CU, one loading while the other computes),
//     walks k in chunks of LMM_KC: the chunk's activation parts of the
//     batch tile (16 NT rows) in LDS, each wave's W loads for the chunk all in
//     flight (8 per tile), three parts x NT MFMAs per 32 k and tile;
//   * W is read once per batch tile of 16 NT rows; the activations once per
//     workgroup.
// MODE 1 (argmax keys) as in k_lmhead.
typedef __bf16 lm_bf16x8 __attribute__((ext_vector_type(8)));
typedef float lm_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t lm_u32x4 __attribute__((ext_vector_type(4)));
constexpr int LMM_WAVES = 8;
constexpr int LMM_TILES = 2;                       // 16-row tiles per wave
constexpr int LMM_ROWS = LMM_WAVES * LMM_TILES * 16;  // 256 (two workgroups per CU)
constexpr int LMM_KC = 128;                        // k per LDS chunk
constexpr int LMM_KS = LMM_KC / 32;                // MFMA k-steps per chunk
constexpr int LMM_PAD = 8;                         // bf16 of padding per LDS row (banks)
constexpr int LMM_RS = LMM_KC + LMM_PAD;           // LDS row stride in bf16

__device__ __forceinline__ float lm_bf16_f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// A 16-byte load of 8 weights holds an infinite or NaN one.
__device__ __forceinline__ bool lm_nonfinite8(const lm_u32x4 q) {
  bool r = false;
#pragma unroll
  for (int c = 0; c < 4; c++)
    r |= ((q[c] & 0x7f800000u) == 0x7f800000u) | ((q[c] & 0x7f80u) == 0x7f80u);
  return r;
}

// Keys of the fused argmax spread over LMM_SLOTS slots per batch row (one
// per workgroup index modulo LMM_SLOTS, each on its own cache line), so the
// workgroups' atomics do not all meet on the batch's few words.
constexpr int LMM_SLOTS = 16;

// One chunk's activations: 16 NT batch rows x LMM_KC, loaded into registers
// (XPT per thread), then split into the three bf16 parts in LDS.
template <int NT>
struct LmX {
  static constexpr int XPT = 16 * NT * LMM_KC / (64 * LMM_WAVES);
  float v[XPT];
};

template <int NT>
__device__ __forceinline__ void lm_x_load(LmX<NT>& xr, const float* __restrict__ X, long ldx,
                                          int nb, int n, int k0) {
#pragma unroll
  for (int q = 0; q < LmX<NT>::XPT; q++) {
    const int i = (int)threadIdx.x + q * 64 * LMM_WAVES;
    const int b = i / LMM_KC, kk = i - b * LMM_KC;
    xr.v[q] = b < nb && k0 + kk < n ? X[(size_t)b * ldx + k0 + kk] : 0.0f;
  }
}

template <int NT>
__device__ __forceinline__ void lm_x_store(const LmX<NT>& xr, uint16_t* xs) {
#pragma unroll
  for (int q = 0; q < LmX<NT>::XPT; q++) {
    const int i = (int)threadIdx.x + q * 64 * LMM_WAVES;
    const int b = i / LMM_KC, kk = i - b * LMM_KC;
    const float x = xr.v[q];
    const uint32_t ux = __float_as_uint(x);
    const bool fin = (ux & 0x7f800000u) != 0x7f800000u;
    // (a NaN whose payload sits in the low bits stays a NaN)
    const uint16_t h0 = fin || !(ux & 0x7fffffu) ? (uint16_t)(ux >> 16) : (uint16_t)0x7fc0u;
    const float r0 = fin ? x - lm_bf16_f(h0) : 0.0f;  // exact: x's low 16 significand bits
    const uint16_t h1 = (uint16_t)(__float_as_uint(r0) >> 16);
    const float r1 = r0 - lm_bf16_f(h1);  // exact: at most 8 significant bits left
    const uint16_t h2 = (uint16_t)(__float_as_uint(r1) >> 16);
    xs[(0 * 16 * NT + b) * LMM_RS + kk] = h0;
    xs[(1 * 16 * NT + b) * LMM_RS + kk] = h1;
    xs[(2 * 16 * NT + b) * LMM_RS + kk] = h2;
  }
}

__device__ __forceinline__ void lm_w_load(lm_u32x4 (&a)[LMM_TILES][LMM_KS],
                                          const uint16_t* const (&wr)[LMM_TILES], int n, int k0,
                                          int g) {
#pragma unroll
  for (int t = 0; t < LMM_TILES; t++)
#pragma unroll
    for (int s = 0; s < LMM_KS; s++) {
      const int k = k0 + 32 * s + 8 * g;
      a[t][s] = k < n ? *reinterpret_cast<const lm_u32x4*>(wr[t] + k) : lm_u32x4{0u, 0u, 0u, 0u};
    }
}

template <int NT>
__device__ __forceinline__ void lm_mfma(const lm_u32x4 (&a)[LMM_TILES][LMM_KS],
                                        const uint16_t* xs, lm_f32x4 (&acc)[LMM_TILES][NT],
                                        uint32_t& bad, int m, int g) {
#pragma unroll
  for (int s = 0; s < LMM_KS; s++) {
    lm_bf16x8 bx[3][NT];
#pragma unroll
    for (int p = 0; p < 3; p++)
#pragma unroll
      for (int j = 0; j < NT; j++)
        bx[p][j] = *reinterpret_cast<const lm_bf16x8*>(
            &xs[(p * 16 * NT + j * 16 + m) * LMM_RS + 32 * s + 8 * g]);
#pragma unroll
    for (int t = 0; t < LMM_TILES; t++) {
      bad |= lm_nonfinite8(a[t][s]) ? 1u << t : 0u;
      const lm_bf16x8 av = __builtin_bit_cast(lm_bf16x8, a[t][s]);
#pragma unroll
      for (int j = 0; j < NT; j++) {
        // the largest part first: the small ones add to an accumulator of
        // the product's own size
        acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bx[2][j], acc[t][j], 0, 0, 0);
        acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bx[1][j], acc[t][j], 0, 0, 0);
        acc[t][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bx[0][j], acc[t][j], 0, 0, 0);
      }
    }
  }
}

// One chunk step of the pipeline: the next chunk's activations and weights
// are loaded (activations first: converting them waits only for them) and
// its activation parts stored in the other LDS buffer while this chunk's
// MFMAs run; one barrier per chunk.
template <int NT>
__device__ __forceinline__ void lm_step(int k0, int n, const float* __restrict__ X, long ldx,
                                        int nb, const uint16_t* const (&wr)[LMM_TILES],
                                        const lm_u32x4 (&cur)[LMM_TILES][LMM_KS],
                                        lm_u32x4 (&nxt)[LMM_TILES][LMM_KS], const uint16_t* xs_cur,
                                        uint16_t* xs_nxt, lm_f32x4 (&acc)[LMM_TILES][NT],
                                        uint32_t& bad, int m, int g) {
  const bool more = k0 + LMM_KC < n;
  LmX<NT> xr;
  if (more) {
    lm_x_load<NT>(xr, X, ldx, nb, n, k0 + LMM_KC);
    lm_w_load(nxt, wr, n, k0 + LMM_KC, g);
    lm_x_store<NT>(xr, xs_nxt);
  }
  lm_mfma<NT>(cur, xs_cur, acc, bad, m, g);
  __syncthreads();
}

template <int NT, int MODE>
__global__ __launch_bounds__(64 * LMM_WAVES) __attribute__((amdgpu_waves_per_eu(4))) void k_lmhead_mfma(
    const uint16_t* __restrict__ W, int V, int n, const float* __restrict__ X, long ldx, int nb,
    float* __restrict__ logits, long ld, unsigned long long* __restrict__ keys, int kstride,
    uint8_t* __restrict__ nan0) {
  // the activation parts of two chunks (this one and the next): [2][3][16 NT][LMM_RS] bf16
  __shared__ __align__(16) uint16_t xs[2][3 * 16 * NT * LMM_RS];
  __shared__ unsigned long long best_sh[LMM_WAVES][16 * NT];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int m = lane & 15, g = lane >> 4;
  const int wrow0 = blockIdx.x * LMM_ROWS + w * LMM_TILES * 16;  // the wave's first row
  lm_f32x4 acc[LMM_TILES][NT];
#pragma unroll
  for (int t = 0; t < LMM_TILES; t++)
#pragma unroll
    for (int j = 0; j < NT; j++) acc[t][j] = lm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // this lane's W rows (clamped into range: rows past V compute unused values)
  const uint16_t* wr[LMM_TILES];
#pragma unroll
  for (int t = 0; t < LMM_TILES; t++) {
    const int r = wrow0 + t * 16 + m;
    wr[t] = W + (size_t)(r < V ? r : V - 1) * n;
  }
  uint32_t bad = 0;  // bit t: this lane's row of tile t holds a non-finite weight
  if (NT == 1) {
    // two chunks' weights in registers: the next chunk's loads overlap this
    // chunk's MFMAs
    lm_u32x4 a0[LMM_TILES][LMM_KS], a1[LMM_TILES][LMM_KS];
    {
      LmX<NT> xr;
      lm_x_load<NT>(xr, X, ldx, nb, n, 0);
      lm_w_load(a0, wr, n, 0, g);
      lm_x_store<NT>(xr, xs[0]);
    }
    __syncthreads();
    for (int k0 = 0; k0 < n; k0 += 2 * LMM_KC) {
      lm_step<NT>(k0, n, X, ldx, nb, wr, a0, a1, xs[0], xs[1], acc, bad, m, g);
      if (k0 + LMM_KC >= n) break;
      lm_step<NT>(k0 + LMM_KC, n, X, ldx, nb, wr, a1, a0, xs[1], xs[0], acc, bad, m, g);
    }
  } else {
    // 32 batch rows: one chunk's weights in registers (two would spill at
    // two workgroups per CU), every load of a chunk in flight before its
    // MFMAs
    for (int k0 = 0; k0 < n; k0 += LMM_KC) {
      lm_u32x4 a[LMM_TILES][LMM_KS];
      LmX<NT> xr;
      lm_x_load<NT>(xr, X, ldx, nb, n, k0);
      lm_w_load(a, wr, n, k0, g);
      __syncthreads();  // the previous chunk's MFMAs are done with the LDS
      lm_x_store<NT>(xr, xs[0]);
      __syncthreads();
      lm_mfma<NT>(a, xs[0], acc, bad, m, g);
    }
  }
  // rows with a non-finite weight: fp32 fused multiply-adds over k (lanes),
  // in every batch row, into the lanes that hold them (rare: a loop per row)
#pragma unroll
  for (int t = 0; t < LMM_TILES; t++) {
    uint64_t rows_bad = __ballot((bad >> t) & 1u) ;
    // lanes l, l + 16, l + 32, l + 48 share a row: fold the groups
    const uint32_t rb = (uint32_t)(rows_bad | (rows_bad >> 16) | (rows_bad >> 32) | (rows_bad >> 48)) &
                        0xffffu;
    for (uint32_t mm = rb; mm; mm &= mm - 1u) {
      const int r16 = (int)__builtin_ctz(mm);
      const int row = wrow0 + t * 16 + r16;
      if (row >= V) break;
      const uint16_t* wrow = W + (size_t)row * n;
      for (int b = 0; b < nb && b < 16 * NT; b++) {
        float d = 0.0f;
        for (int k = lane; k < n; k += 64)
          d = __builtin_fmaf(lm_bf16_f(wrow[k]), X[(size_t)b * ldx + k], d);
        d = pz_wave_sum(d);
        if (g == (r16 >> 2) && m == (b & 15))
#pragma unroll
          for (int j = 0; j < NT; j++)
            if (j == (b >> 4))
#pragma unroll
              for (int i = 0; i < 4; i++)
                if (i == (r16 & 3)) acc[t][j][i] = d;
      }
    }
  }
  // epilogue: lane l holds batch row 16 j + l % 16, rows 4 (l / 16) + i of each tile
  unsigned long long best[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) best[j] = 0ull;
#pragma unroll
  for (int t = 0; t < LMM_TILES; t++)
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const int b = 16 * j + m;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = wrow0 + t * 16 + 4 * g + i;
        const float v = acc[t][j][i];
        if (row < V && b < nb) {
          if (MODE == 0) {
            logits[(size_t)b * ld + row] = v;
          } else {
            if (row == 0) nan0[b] = v != v ? 1 : 0;
            if (!(v != v)) {
              const unsigned long long kk = argmax_key(v, row);
              best[j] = kk > best[j] ? kk : best[j];
            }
          }
        }
      }
    }
  if (MODE == 1) {
    // the maximum key per batch row: over the four lane groups, then the waves
#pragma unroll
    for (int j = 0; j < NT; j++) {
#pragma unroll
      for (int off = 16; off < 64; off <<= 1) {
        const unsigned long long o = __shfl_xor(best[j], off, 64);
        best[j] = o > best[j] ? o : best[j];
      }
      if (g == 0) best_sh[w][16 * j + m] = best[j];
    }
    __syncthreads();
    if (tid < 16 * NT && tid < nb) {
      unsigned long long mx = best_sh[0][tid];
      for (int i = 1; i < LMM_WAVES; i++) mx = best_sh[i][tid] > mx ? best_sh[i][tid] : mx;
      if (mx) atomicMax(&keys[(size_t)(blockIdx.x % LMM_SLOTS) * kstride + tid], mx);
    }
  }
}

template <int NT, int MODE>
int launch_mfma(pz_sampler* s, const uint16_t* d_w, int V, int n, const float* x, long ldx,
                int nb, float* out, long ld, unsigned long long* keys, uint8_t* nan0) {
  const int grid = (V + LMM_ROWS - 1) / LMM_ROWS;
  hipLaunchKernelGGL((k_lmhead_mfma<NT, MODE>), dim3(grid), dim3(64 * LMM_WAVES), 0, s->stream,
                     d_w, V, n, x, ldx, nb, out, ld, keys, s->max_batch, nan0);
  PZ_HIP(s, hipGetLastError());
  return PZ_OK;
}

// Keys to ids (argmax.c:3-13); clears the keys for the next call.  The
// matrix-core kernel spreads each row's key over LMM_SLOTS slots (stride
// kstride); the others use slot 0 only (the rest stay zero).
__global__ void k_lmhead_finish(int B, unsigned long long* keys, int kstride, const uint8_t* nan0,
                                int32_t* ids) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  unsigned long long k = 0ull;
  for (int sl = 0; sl < LMM_SLOTS; sl++) {
    const unsigned long long o = keys[(size_t)sl * kstride + b];
    k = o > k ? o : k;
    if (sl) keys[(size_t)sl * kstride + b] = 0ull;
  }
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
  // batch 4 and up: the matrix cores, batch tiles of 32 (or 16), W 16-byte
  // aligned with rows of a multiple of 8 weights
  if (B >= 4 && n % 8 == 0 && ((uintptr_t)d_w & 15) == 0) {
    for (int b0 = 0; b0 < B; b0 += 32) {
      const int nb = B - b0 < 32 ? B - b0 : 32;
      const float* x = d_x + (size_t)b0 * ldx;
      float* out = MODE == 0 ? d_logits + (size_t)b0 * ld : nullptr;
      unsigned long long* keys = s->d_lmh_keys + b0;
      uint8_t* nan0 = s->d_lmh_nan + b0;
      const int rc = nb > 16 ? launch_mfma<2, MODE>(s, d_w, V, n, x, ldx, nb, out, ld, keys, nan0)
                             : launch_mfma<1, MODE>(s, d_w, V, n, x, ldx, nb, out, ld, keys, nan0);
      if (rc != PZ_OK) return rc;
    }
    return PZ_OK;
  }
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
                     s->d_lmh_keys, s->max_batch, s->d_lmh_nan, d_ids);
  PZ_HIP(s, hipGetLastError());
  return PZ_OK;
}
