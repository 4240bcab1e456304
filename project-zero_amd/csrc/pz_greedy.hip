// pz_greedy.hip -- batched greedy sampling: virtual penalties + argmax.
//
// Reference semantics: sample_argmax (src/sampling/argmax.c:3-13): the first
// maximum wins (strict '>' scan from x[0]), so ties go to the lowest id and a
// NaN at x[0] returns 0.  Penalties (repetition / presence / frequency) are
// applied without writing the row: the streaming pass skips the history's ids
// (an LDS bitmap marks them) and a second, tiny pass over the history takes
// their penalised values.  The argmax of the union under (value desc, id asc)
// is the argmax of the penalised row.  The row in HBM is read once with
// 128-bit non-temporal loads, plus one gathered load per history entry.
//
// Layout: one workgroup per row, BLOCK threads, each thread walks float4
// groups tid, tid+BLOCK, ... in ascending id order.  Two register sets of U
// float4 alternate: one set's loads are in flight while the other is
// compared, and the first set is issued before the history bitmap is built.
#include "pz_device.h"
#include "pz_launch.h"

namespace {

template <int BLOCK, int U>
__device__ __forceinline__ void gr_load(const pz_f4* x4, int n4, int base, pz_f4 (&v)[U]) {
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int i4 = base + u * BLOCK + (int)threadIdx.x;
    v[u] = __builtin_nontemporal_load(&x4[i4 < n4 ? i4 : n4 - 1]);  // unconditional
  }
}

template <int U>
__device__ __forceinline__ void gr_drain(const pz_f4 (&v)[U]) {
#pragma unroll
  for (int u = 0; u < U; u++) {
    asm volatile("" ::"v"(v[u].x));
    asm volatile("" ::"v"(v[u].w));
  }
}

// Running best over one register set, per float4: m = max of its four
// values (history ids masked to -inf when PEN), and the first float4 of the
// thread whose m beats bv (strict '>') is kept with its values, so the id is
// resolved once at the end.  Groups past the row end hold copies of the
// row's last float4 (clamped loads): a copy ties its original, which the
// owning thread holds at a lower index, so it never wins the reduction.
struct GrBest {
  float bv;     // best value
  int b4;       // its float4 index (0x7fffffff: none)
  pz_f4 bx;     // that float4's values, as compared
};

// lo: the id of x4[0] (0 for a whole row, a multiple of 32 for a range).
template <int BLOCK, int U, bool TEMPER, bool PEN>
__device__ __forceinline__ void gr_group(const PzPenalty& P, const pz_row_params_dev& prm,
                                         int lo, int n4, int base, const pz_f4 (&v)[U],
                                         GrBest& B) {
  const int tid = threadIdx.x;
  uint32_t nib[U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int i4 = base + u * BLOCK + tid;
    nib[u] = PEN ? pz_pen_nibble(P, lo + ((i4 < n4 ? i4 : n4 - 1) << 2)) : 0u;
  }
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int i4 = base + u * BLOCK + tid;
    pz_f4 e = v[u];
    if (TEMPER) {
      e.x = pz_temper(e.x, prm);
      e.y = pz_temper(e.y, prm);
      e.z = pz_temper(e.z, prm);
      e.w = pz_temper(e.w, prm);
    }
    if (PEN) {  // history ids -> -inf (their penalised values join later)
      const uint32_t ninf = 0xff800000u;
      const uint32_t m0 = 0u - (nib[u] & 1u), m1 = 0u - ((nib[u] >> 1) & 1u);
      const uint32_t m2 = 0u - ((nib[u] >> 2) & 1u), m3 = 0u - ((nib[u] >> 3) & 1u);
      e.x = __uint_as_float((__float_as_uint(e.x) & ~m0) | (ninf & m0));
      e.y = __uint_as_float((__float_as_uint(e.y) & ~m1) | (ninf & m1));
      e.z = __uint_as_float((__float_as_uint(e.z) & ~m2) | (ninf & m2));
      e.w = __uint_as_float((__float_as_uint(e.w) & ~m3) | (ninf & m3));
    }
    const float m = fmaxf(fmaxf(e.x, e.y), fmaxf(e.z, e.w));  // NaNs drop out
    const bool take = m > B.bv;
    B.bv = take ? m : B.bv;
    B.b4 = take ? i4 : B.b4;
    B.bx.x = take ? e.x : B.bx.x;
    B.bx.y = take ? e.y : B.bx.y;
    B.bx.z = take ? e.z : B.bx.z;
    B.bx.w = take ? e.w : B.bx.w;
  }
}

// One exit only (the loop condition): a break in the middle of the loop body
// makes the compiler merge paths on which the other set's loads are still
// in flight, and it then drains every load at the loop head.
template <int BLOCK, int U, bool TEMPER, bool PEN>
__device__ __forceinline__ void gr_stream(const PzPenalty& P, const pz_row_params_dev& prm,
                                          int lo, const pz_f4* x4, int n4, pz_f4 (&a)[U],
                                          pz_f4 (&b)[U], GrBest& B) {
  constexpr int STEP = BLOCK * U;
  const int ng = (n4 + STEP - 1) / STEP;
  int g = 0;
  for (; g + 1 < ng; g += 2) {
    gr_load<BLOCK, U>(x4, n4, (g + 1) * STEP, b);
    gr_group<BLOCK, U, TEMPER, PEN>(P, prm, lo, n4, g * STEP, a, B);
    __builtin_amdgcn_sched_barrier(0);
    gr_load<BLOCK, U>(x4, n4, (g + 2) * STEP, a);
    gr_group<BLOCK, U, TEMPER, PEN>(P, prm, lo, n4, (g + 1) * STEP, b, B);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (g < ng) gr_group<BLOCK, U, TEMPER, PEN>(P, prm, lo, n4, g * STEP, a, B);
  gr_drain(a);
  gr_drain(b);
}

// TEMPER: the launch's rows are top-p rows above the reference's vocabulary
// guard, which take the argmax of the tempered row (top_p.c:33-34, after
// apply_temperature).  PEN: some row of the launch has an active penalty;
// every row then builds the bitmap (all zero where the row has none).
template <int BLOCK, int U, bool VEC, bool TEMPER, bool PEN>
__global__ __launch_bounds__(BLOCK) void k_greedy(
    const float* __restrict__ logits, long ld, int V,
    const int32_t* __restrict__ rows, const pz_row_params_dev* __restrict__ params,
    int n_params, const int32_t* __restrict__ hist, int H, int hcap,
    int32_t* __restrict__ ids_out, float* __restrict__ p_out) {
  extern __shared__ __align__(16) char lds[];
  __shared__ float red_v[BLOCK / PZ_WAVE];
  __shared__ int red_i[BLOCK / PZ_WAVE];

  const int row = pz_row_of(rows, blockIdx.x);
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const float* x = logits + (long)row * ld;
  const int32_t* hrow = hist ? hist + (long)row * H : nullptr;
  const int tid = threadIdx.x;
  const pz_f4* x4 = reinterpret_cast<const pz_f4*>(x);
  const int n4 = VEC ? V >> 2 : 0;  // VEC launches have V >= 4, so n4 >= 1

  // Prologue ordered for the in-order load counter: the history id of one
  // entry per thread first, then the first register set and x[0], so that
  // the bitmap insert waits for the id only; the entry's logit is gathered
  // after the insert and is not waited for until the history pass.
  int hid0 = -1;
  if (hrow && tid < H) hid0 = hrow[tid];
  pz_f4 a[U], b[U];
  if (VEC) gr_load<BLOCK, U>(x4, n4, 0, a);  // unconditional within the launch
  const float x0 = tid == 0 ? x[0] : 0.0f;
  __builtin_amdgcn_sched_barrier(0);

  PzPenalty P;
  pz_penalty_setup<BLOCK>(P, lds, V, hcap, PEN && hrow != nullptr && H > 0, prm);
  float hx0 = 0.0f;
  if (PEN) {
    if (!P.active) {  // the set-up clears the tables of active rows only
      pz_lds_u32* bm = (pz_lds_u32*)lds;
      for (int w = tid; w < ((V + 31) >> 5); w += BLOCK) bm[w] = 0u;
    }
    __syncthreads();
    if (P.active) {
      if (tid < H) {
        pz_penalty_insert(P, lds, V, hid0, nullptr, nullptr);
        hx0 = x[hid0 >= 0 && hid0 < V ? hid0 : 0];
      }
      for (int j = tid + BLOCK; j < H; j += BLOCK)
        pz_penalty_insert(P, lds, V, hrow[j], nullptr, nullptr);
    }
    __syncthreads();
  }

  constexpr bool temper = TEMPER;
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  if (VEC) {
    GrBest B;
    B.bv = -__builtin_inff();
    B.b4 = 0x7fffffff;
    B.bx = pz_f4{0.0f, 0.0f, 0.0f, 0.0f};
    gr_stream<BLOCK, U, TEMPER, PEN>(P, prm, 0, x4, n4, a, b, B);
    if (B.b4 != 0x7fffffff) {  // the first of the float4's values equal to the best
      bv = B.bv;
      bi = (B.b4 << 2) + (B.bx.x == bv ? 0 : B.bx.y == bv ? 1 : B.bx.z == bv ? 2 : 3);
    }
  }
  for (int i = (n4 << 2) + tid; i < V; i += BLOCK) {
    if (P.active && pz_pen_member(P, i)) continue;  // taken by the history pass
    float e = x[i];
    if (temper) e = pz_temper(e, prm);
    if (e > bv) { bv = e; bi = i; }
  }

  // the history's ids with their penalised values; duplicates give equal
  // (value, id) pairs
  if (P.active) {
    for (int j = tid; j < H; j += BLOCK) {
      const int id = j == tid ? hid0 : hrow[j];
      if (id < 0 || id >= V) continue;
      float e = pz_penalize_inline(j == tid ? hx0 : x[id], id, P.rep, P.pres, P.freq, P.hcap,
                                   P.hkey, P.hcnt);
      if (temper) e = pz_temper(e, prm);
      // -inf never enters (as in the stream): a row whose maximum is -inf
      // returns id 0, where the reference's scan starts
      if (e > -__builtin_inff()) pz_argmax_combine(bv, bi, e, id);
    }
  }

  pz_block_argmax<BLOCK>(bv, bi, red_v, red_i);
  if (tid == 0) {
    float y0 = x0;
    if (P.active && pz_pen_member(P, 0)) y0 = pz_penalize(P, y0, 0);
    if (temper) y0 = pz_temper(y0, prm);
    // argmax.c:4-5 starts from x[0]: a NaN there is never replaced; and if
    // nothing beats -inf the scan also ends on index 0.
    if (y0 != y0 || bi == 0x7fffffff) bi = 0;
    ids_out[row] = bi;
    if (p_out) p_out[row] = 1.0f;
  }
}


// Small batches: each row split over gridDim.x workgroups of `chunk` ids
// (a multiple of 1024, so a range starts 16-byte aligned and on a bitmap
// word).  Workgroup (s, b) streams the ids [s*chunk, min(V, (s+1)*chunk)) of
// its row with the loop above, its penalty tables covering that range only,
// and posts its best as the key (pz_key(v) << 32) | ~id -- the larger key is
// the larger value, then the lower id, exactly the order of argmax.c's
// strict '>' scan.  Every posted word is nonzero: 1 means no candidate (below
// every value's key), and the range holding id 0 posts all ones (above every
// value's key) when y[0] is NaN, which returns id 0.  The workgroup that
// arrives last takes the largest word (pz_sp_post_last).  words: the row's
// meeting words (zero between launches); arrive: zero between launches.
template <int BLOCK, int U, bool TEMPER, bool PEN>
__global__ __launch_bounds__(BLOCK) void k_greedy_split(
    const float* __restrict__ logits, long ld, int V, int chunk,
    const int32_t* __restrict__ rows, const pz_row_params_dev* __restrict__ params,
    int n_params, const int32_t* __restrict__ hist, int H, int hcap,
    int32_t* __restrict__ ids_out, float* __restrict__ p_out, uint64_t* __restrict__ words,
    int wstride, uint32_t* __restrict__ arrive, uint32_t cap) {
  extern __shared__ __align__(16) char lds[];
  __shared__ float red_v[BLOCK / PZ_WAVE];
  __shared__ int red_i[BLOCK / PZ_WAVE];

  const int sl = blockIdx.x, S = gridDim.x;
  const int row = pz_row_of(rows, blockIdx.y);
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const int lo = sl * chunk;
  const int hi = lo + chunk < V ? lo + chunk : V;
  const float* x = logits + (long)row * ld;
  const int32_t* hrow = hist ? hist + (long)row * H : nullptr;
  const int tid = threadIdx.x;
  const pz_f4* x4 = reinterpret_cast<const pz_f4*>(x + lo);
  const int n4 = (hi - lo) >> 2;  // 0 only for a last range of 1-3 ids

  int hid0 = -1;
  if (hrow && tid < H) hid0 = hrow[tid];
  pz_f4 a[U], b[U];
  if (n4 > 0) gr_load<BLOCK, U>(x4, n4, 0, a);
  const float x0 = (sl == 0 && tid == 0) ? x[0] : 0.0f;
  __builtin_amdgcn_sched_barrier(0);

  PzPenalty P;
  pz_penalty_setup_range<BLOCK>(P, lds, lo, hi, hcap, PEN && hrow != nullptr && H > 0, prm);
  float hx0 = 0.0f;
  const bool hin0 = hid0 >= lo && hid0 < hi;
  if (PEN) {
    if (!P.active) {
      pz_lds_u32* bm = (pz_lds_u32*)lds;
      for (int w = tid; w < ((hi - lo + 31) >> 5); w += BLOCK) bm[w] = 0u;
    }
    __syncthreads();
    if (P.active) {
      if (tid < H && hin0) {
        pz_penalty_insert(P, lds, V, hid0, nullptr, nullptr);
        hx0 = x[hid0];
      }
      for (int j = tid + BLOCK; j < H; j += BLOCK)
        pz_penalty_insert(P, lds, V, hrow[j], nullptr, nullptr);  // skips ids out of range
    }
    __syncthreads();
  }

  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  if (n4 > 0) {
    GrBest B;
    B.bv = -__builtin_inff();
    B.b4 = 0x7fffffff;
    B.bx = pz_f4{0.0f, 0.0f, 0.0f, 0.0f};
    gr_stream<BLOCK, U, TEMPER, PEN>(P, prm, lo, x4, n4, a, b, B);
    if (B.b4 != 0x7fffffff) {
      bv = B.bv;
      bi = lo + (B.b4 << 2) + (B.bx.x == bv ? 0 : B.bx.y == bv ? 1 : B.bx.z == bv ? 2 : 3);
    }
  }
  for (int i = lo + (n4 << 2) + tid; i < hi; i += BLOCK) {
    if (P.active && pz_pen_member(P, i)) continue;
    float e = x[i];
    if (TEMPER) e = pz_temper(e, prm);
    if (e > bv) { bv = e; bi = i; }
  }
  if (P.active) {
    for (int j = tid; j < H; j += BLOCK) {
      const int id = j == tid ? hid0 : hrow[j];
      if (id < lo || id >= hi) continue;
      float e = pz_penalize_inline(j == tid ? hx0 : x[id], id, P.rep, P.pres, P.freq, P.hcap,
                                   P.hkey, P.hcnt);
      if (TEMPER) e = pz_temper(e, prm);
      if (e > -__builtin_inff()) pz_argmax_combine(bv, bi, e, id);
    }
  }

  pz_block_argmax<BLOCK>(bv, bi, red_v, red_i);
  if (tid >= PZ_WAVE) return;  // wave 0 posts and, in the last workgroup, merges
  uint64_t* w = words + (size_t)row * wstride;
  int last = 0;
  if (tid == 0) {
    uint64_t key = bi == 0x7fffffff ? 1ull
                                    : ((uint64_t)pz_key(bv) << 32) | (uint32_t)~(uint32_t)bi;
    if (sl == 0) {
      float y0 = x0;
      if (P.active && pz_pen_member(P, 0)) y0 = pz_penalize(P, y0, 0);
      if (TEMPER) y0 = pz_temper(y0, prm);
      if (y0 != y0) key = ~0ull;  // argmax.c:4-5: a NaN x[0] is never replaced
    }
    last = pz_sp_post_last(w, sl, key, arrive, row, S);
  }
  if (!__builtin_amdgcn_readfirstlane(last)) return;
  uint64_t k = 1ull;
  bool seen = true;
  for (int j = tid; j < S; j += PZ_WAVE) {
    const uint64_t o = pz_poll_u64(&w[j], cap);
    seen = seen && o != 0ull;
    k = o > k ? o : k;
    __hip_atomic_store(&w[j], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo32 = (uint32_t)__shfl_xor((int)(uint32_t)k, off, PZ_WAVE);
    const uint32_t hi32 = (uint32_t)__shfl_xor((int)(uint32_t)(k >> 32), off, PZ_WAVE);
    const uint64_t o = ((uint64_t)hi32 << 32) | lo32;
    k = o > k ? o : k;
  }
  const bool all_seen = __builtin_amdgcn_ballot_w64(!seen) == 0ull;
  if (tid == 0) {
    // no candidate (every value NaN or -inf): the scan ends on index 0
    ids_out[row] = !all_seen ? PZ_ID_FAILED : (k == 1ull || k == ~0ull) ? 0
                                                                      : (int32_t)~(uint32_t)k;
    if (p_out) p_out[row] = 1.0f;
    __hip_atomic_store(&arrive[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

constexpr int GREEDY_BLOCK = 256;
constexpr int GREEDY_U = 4;

// Rows split over workgroups while a launch has fewer than GREEDY_SPLIT_WG
// workgroups' worth of rows: ranges of at least GREEDY_MIN_CHUNK ids.
#ifndef GREEDY_SPLIT_WG
#define GREEDY_SPLIT_WG 512
#endif
#ifndef GREEDY_MIN_CHUNK
#define GREEDY_MIN_CHUNK 4096
#endif
constexpr int GREEDY_MAX_SPLIT = 128;
#ifndef GREEDY_SPLIT_BLOCK
#define GREEDY_SPLIT_BLOCK 256
#endif
#ifndef GREEDY_SPLIT_U
#define GREEDY_SPLIT_U 4
#endif

// Workgroups per row (1: one workgroup owns the row) and the ids of each.
static int greedy_split(int V, int n_rows, int* chunk) {
  int S = (GREEDY_SPLIT_WG + n_rows - 1) / n_rows;
  const int smax = V / GREEDY_MIN_CHUNK;
  if (S > smax) S = smax;
  if (S > GREEDY_MAX_SPLIT) S = GREEDY_MAX_SPLIT;
  if (S < 2) return 1;
  int c = (V + S - 1) / S;
  c = (c + 1023) & ~1023;
  *chunk = c;
  return (V + c - 1) / c;
}

template <bool TEMPER>
static int launch_argmax(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  if (n_rows <= 0) return 0;
  constexpr size_t kStatic = 2 * (GREEDY_BLOCK / PZ_WAVE) * 4;
  const bool vec = (L.ld % 4 == 0) && (((uintptr_t)L.logits & 15) == 0) && L.V >= 4;
  int chunk = 0;
  const int S = vec && L.ws.meet && L.ws.arrive ? greedy_split(L.V, n_rows, &chunk) : 1;
  if (S > 1 && S <= 2 * L.ws.smax) {
    const size_t lds = L.pen_any ? pz_penalty_lds_bytes(chunk, L.hcap) : 0;
    constexpr size_t kStaticS = 2 * (GREEDY_SPLIT_BLOCK / PZ_WAVE) * 4;
    if (lds + kStaticS > (size_t)L.max_lds) return -2;
    auto k = L.pen_any ? k_greedy_split<GREEDY_SPLIT_BLOCK, GREEDY_SPLIT_U, TEMPER, true>
                       : k_greedy_split<GREEDY_SPLIT_BLOCK, GREEDY_SPLIT_U, TEMPER, false>;
    if (lds > 65536 && hipFuncSetAttribute((const void*)k,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds) != hipSuccess)
      return -1;
    hipLaunchKernelGGL(k, dim3(S, n_rows), dim3(GREEDY_SPLIT_BLOCK), lds, L.stream, L.logits,
                       L.ld,
                       L.V, chunk, d_rows, L.params, L.n_params, L.hist, L.H, L.hcap, L.ids,
                       L.p_out, L.ws.meet, 2 * L.ws.smax, L.ws.arrive, L.wait_polls);
    return hipGetLastError() == hipSuccess ? 0 : -1;
  }
  const size_t lds = L.pen_any ? pz_penalty_lds_bytes(L.V, L.hcap) : 0;
  // static LDS: the block argmax scratch (2 words per wave)
  if (lds + kStatic > (size_t)L.max_lds) return -2;
  dim3 grid(n_rows), block(GREEDY_BLOCK);
  auto k = vec ? (L.pen_any ? k_greedy<GREEDY_BLOCK, GREEDY_U, true, TEMPER, true>
                            : k_greedy<GREEDY_BLOCK, GREEDY_U, true, TEMPER, false>)
               : (L.pen_any ? k_greedy<GREEDY_BLOCK, GREEDY_U, false, TEMPER, true>
                            : k_greedy<GREEDY_BLOCK, GREEDY_U, false, TEMPER, false>);
  if (lds > 65536 && hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)lds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(k, grid, block, lds, L.stream, L.logits, L.ld, L.V, d_rows, L.params,
                     L.n_params, L.hist, L.H, L.hcap, L.ids, L.p_out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int pz_launch_greedy(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  return launch_argmax<false>(L, n_rows, d_rows);
}

int pz_launch_greedy_tempered(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  return launch_argmax<true>(L, n_rows, d_rows);
}

size_t pz_greedy_lds_bytes(int V, int hcap) { return pz_penalty_lds_bytes(V, hcap); }
