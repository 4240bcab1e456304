// pz_device.h -- device-side building blocks shared by the sampling kernels
// (gfx950 / CDNA4, wave64).  Compiled with -ffp-contract=off so every fp32
// expression rounds exactly as the reference's gcc -std=c99 build does.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pz_params.h"

#define PZ_WAVE 64

// Native 128-bit vector (HIP's float4 is a struct; the builtins want this).
typedef float pz_f4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Row addressing.  A launch either covers rows 0..n-1 or the rows named in a
// device row list (used when a batch mixes sampling modes).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int pz_row_of(const int32_t* rows, int b) {
  return rows ? rows[b] : b;
}

__device__ __forceinline__ const pz_row_params_dev& pz_params_of(
    const pz_row_params_dev* p, int n_params, int row) {
  return p[n_params == 1 ? 0 : row];
}

// ---------------------------------------------------------------------------
// expf bit-identical to glibc 2.35's expf (the libm the reference links,
// called at top_k.c:54, top_p.c:59, softmax.c:14).  Method: x*N/ln2 = k + r,
// N = 32, 2^(k/N) from a 32-entry table of 2^(i/32) (stored minus i<<47 so
// the exponent can be added as an integer), 2^(r/N) by a cubic in double,
// one final rounding to fp32 (Szabolcs Nagy's table-driven expf, as published
// in ARM optimized-routines and adopted by glibc 2.27).  The fused
// multiply-adds are written out explicitly; the sequence was checked bit for
// bit against the host libm on every fp32 input in (-103.9, 88.7).
// ---------------------------------------------------------------------------
__constant__ static const uint64_t pz_exp2_tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,
    0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
    0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,
    0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,
    0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
    0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,
    0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,
    0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
    0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// The method with the table read through `tab` (the constant table, or a
// copy of it in LDS for latency-bound callers).
template <class Tab>
__device__ __forceinline__ float pz_expf_tab(float x, Tab tab) {
  const uint32_t ux = __float_as_uint(x);
  const uint32_t abstop = (ux >> 20) & 0x7ff;
  if (__builtin_expect(abstop >= 0x42b, 0)) {  // |x| >= 88 or non-finite
    if (ux == 0xff800000u) return 0.0f;           // -inf
    if (abstop >= 0x7f8) return x + x;            // +inf, nan
    if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
  const double Shift = 0x1.8p+52;
  const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const double xd = (double)x;
  double kd = __builtin_fma(InvLn2N, xd, Shift);
  const uint64_t ki = (uint64_t)__double_as_longlong(kd);
  kd = kd - Shift;
  const double r = __builtin_fma(InvLn2N, xd, -kd);
  uint64_t t = tab[ki & 31];
  t += ki << 47;
  const double s = __longlong_as_double((long long)t);
  const double z = __builtin_fma(C0, r, C1);
  const double r2 = r * r;
  double y = __builtin_fma(C2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

__device__ __forceinline__ float pz_expf_inline(float x) { return pz_expf_tab(x, pz_exp2_tab); }

typedef __attribute__((address_space(3))) uint64_t pz_lds_u64;

// A workgroup's LDS copy of the table (read at LDS latency instead of a
// global-memory round trip on the serial paths).  Threads 0..31 fill it; the
// caller puts a barrier between the fill and the first use.
__device__ __forceinline__ void pz_etab_fill(pz_lds_u64* t) {
  if (threadIdx.x < 32) t[threadIdx.x] = pz_exp2_tab[threadIdx.x];
}

// Out of line, with the table in LDS.
__device__ __noinline__ float pz_expf_l(float x, const pz_lds_u64* tab) {
  return pz_expf_tab(x, tab);
}

// x_c for a per-lane c in 0..3.  The values pass through an empty asm
// first: a select between elements of one array would otherwise become a
// load at a per-lane index, which puts the array in scratch memory.
__device__ __forceinline__ uint32_t pz_sel4(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3,
                                            int c) {
  asm volatile("" : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3));
  const uint32_t lo = (c & 1) ? x1 : x0, hi = (c & 1) ? x3 : x2;
  return (c & 2) ? hi : lo;
}
__device__ __forceinline__ float pz_sel4f(float x0, float x1, float x2, float x3, int c) {
  return __uint_as_float(pz_sel4(__float_as_uint(x0), __float_as_uint(x1), __float_as_uint(x2),
                                 __float_as_uint(x3), c));
}

// Workgroup barrier that orders LDS only: the waves' global stores still
// in flight stay in flight (__syncthreads waits for every one of them to
// complete first).  Only where no thread reads global memory another wave
// of the workgroup wrote before the barrier.
__device__ __forceinline__ void pz_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Out of line: the exact exponential sits on paths that are rare next to the
// streaming passes, and inlining it into every one of them multiplies the
// kernels' code size beyond the instruction cache.
__device__ __noinline__ float pz_expf(float x) { return pz_expf_inline(x); }

// ---------------------------------------------------------------------------
// Order key: monotone uint32 image of an fp32 value (larger value -> larger
// key), with -0.0 folded onto +0.0 so the two compare equal exactly as the
// reference's float '>' does.  NaN is never passed in.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pz_key(float v) {
  uint32_t u = __float_as_uint(v);
  if (u == 0x80000000u) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float pz_unkey(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// ---------------------------------------------------------------------------
// Penalty context built in LDS from one row's history (repetition penalty:
// membership bitmap; presence/frequency: id -> count hash, linear probing).
// The penalty is applied virtually while a kernel streams the row: the
// logits in HBM are never written.
// ---------------------------------------------------------------------------
// LDS-qualified pointers: lookups compile to ds_read (counted by lgkmcnt
// only), so they never force a wait on the row's outstanding HBM loads the
// way generic (flat) accesses would.
typedef __attribute__((address_space(3))) uint32_t pz_lds_u32;
typedef __attribute__((address_space(3))) int32_t pz_lds_i32;

// The tables cover the ids [base, lim): the whole row (base 0, lim V) for a
// workgroup that owns a row, or its slice for one of several workgroups that
// share a row (base a multiple of 32).
struct PzPenalty {
  const pz_lds_u32* bitmap;  // ceil((lim-base)/32) words, bit i-base set <=> id i in history
  const pz_lds_i32* hkey;    // hash keys (-1 = empty), hcap entries
  const pz_lds_i32* hcnt;    // counts
  int hcap;           // power of two, 0 when counts are not needed
  int base, lim;      // ids held: [base, lim)
  float rep, pres, freq;
  bool active;
};

// Bytes of LDS the penalty context needs (for n ids).
__host__ __device__ inline size_t pz_penalty_lds_bytes(int n, int hcap) {
  size_t words = ((size_t)n + 31) / 32;
  return words * 4 + (size_t)hcap * 8;
}

__device__ __forceinline__ uint32_t pz_hash(uint32_t id) {
  return (id * 0x9E3779B1u) >> 7;
}

// Set-up half of the build for the ids [base, lim): fills P and clears the
// tables (no barrier).
template <int BLOCK>
__device__ __forceinline__ void pz_penalty_setup_range(PzPenalty& P, char* lds, int base, int lim,
                                                       int hcap, bool has_hist,
                                                       const pz_row_params_dev& prm) {
  const int tid = threadIdx.x;
  P.active = has_hist && (prm.rep_penalty != 1.0f || prm.presence_penalty != 0.0f ||
                          prm.frequency_penalty != 0.0f);
  P.rep = prm.rep_penalty;
  P.pres = prm.presence_penalty;
  P.freq = prm.frequency_penalty;
  P.base = base;
  P.lim = lim;
  const int words = (lim - base + 31) >> 5;
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(lds);
  int32_t* hkey = reinterpret_cast<int32_t*>(lds + (size_t)words * 4);
  int32_t* hcnt = hkey + hcap;
  P.bitmap = (const pz_lds_u32*)bitmap;
  P.hkey = (const pz_lds_i32*)hkey;
  P.hcnt = (const pz_lds_i32*)hcnt;
  P.hcap = (prm.presence_penalty != 0.0f || prm.frequency_penalty != 0.0f) ? hcap : 0;
  if (!P.active) return;
  for (int w = tid; w < words; w += BLOCK) bitmap[w] = 0u;
  for (int j = tid; j < P.hcap; j += BLOCK) { hkey[j] = -1; hcnt[j] = 0; }
}

template <int BLOCK>
__device__ __forceinline__ void pz_penalty_setup(PzPenalty& P, char* lds, int V, int hcap,
                                                 bool has_hist, const pz_row_params_dev& prm) {
  pz_penalty_setup_range<BLOCK>(P, lds, 0, V, hcap, has_hist, prm);
}

// Inserts one history id (after the set-up and a barrier).  With dlist !=
// nullptr every distinct valid id is also appended once to dlist, *dcount
// counting them (zeroed by the caller before the set-up barrier).  Ids
// outside [0, V) are ignored (the penalty's definition), and so are ids
// outside the tables' [base, lim).
__device__ __forceinline__ void pz_penalty_insert(const PzPenalty& P, char* lds, int V, int id,
                                                  int32_t* dlist, int* dcount) {
  if (id < 0 || id >= V || id < P.base || id >= P.lim) return;
  const int words = (P.lim - P.base + 31) >> 5;
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(lds);
  int32_t* hkey = reinterpret_cast<int32_t*>(lds + (size_t)words * 4);
  int32_t* hcnt = hkey + P.hcap;
  const uint32_t bit = 1u << (id & 31);
  const uint32_t before = atomicOr(&bitmap[(id - P.base) >> 5], bit);
  if (dlist && !(before & bit)) dlist[atomicAdd(dcount, 1)] = id;
  if (P.hcap) {
    const uint32_t mask = (uint32_t)P.hcap - 1u;
    uint32_t s = pz_hash((uint32_t)id) & mask;
    while (true) {
      const int prev = atomicCAS(&hkey[s], -1, id);
      if (prev == -1 || prev == id) { atomicAdd(&hcnt[s], 1); break; }
      s = (s + 1) & mask;
    }
  }
}

// Builds the tables of the ids [base, lim) of a row of V from its history.
template <int BLOCK>
__device__ __forceinline__ void pz_penalty_build_range(PzPenalty& P, char* lds, int V, int base,
                                                       int lim, int hcap,
                                                       const int32_t* hist_row, int H,
                                                       const pz_row_params_dev& prm) {
  pz_penalty_setup_range<BLOCK>(P, lds, base, lim, hcap, hist_row != nullptr && H > 0, prm);
  if (!P.active) return;
  __syncthreads();
  for (int j = threadIdx.x; j < H; j += BLOCK)
    pz_penalty_insert(P, lds, V, hist_row[j], nullptr, nullptr);
  __syncthreads();
}

template <int BLOCK>
__device__ __forceinline__ void pz_penalty_build(PzPenalty& P, char* lds, int V, int hcap,
                                                 const int32_t* hist_row, int H,
                                                 const pz_row_params_dev& prm) {
  pz_penalty_build_range<BLOCK>(P, lds, V, 0, V, hcap, hist_row, H, prm);
}

// Penalised value of a history member (caller checked the bitmap bit).
// Repetition first (x>0 ? x/rep : x*rep, each distinct id once), then
// t = (float)c*freq; t = t + pres; x = x - t.
__device__ __forceinline__ float pz_penalize_inline(float x, int id, float rep, float pres,
                                                   float freq, int hcap, const pz_lds_i32* hkey,
                                                   const pz_lds_i32* hcnt) {
  x = x > 0.0f ? x / rep : x * rep;
  if (hcap) {
    const uint32_t mask = (uint32_t)hcap - 1u;
    uint32_t s = pz_hash((uint32_t)id) & mask;
    while (hkey[s] != id) s = (s + 1) & mask;
    const int c = hcnt[s];
    float t = (float)c * freq;
    t = t + pres;
    x = x - t;
  }
  return x;
}

// Out of line for the streaming passes (only history members take it;
// inlined at every element of every unrolled pass it bloats the kernels),
// with every operand passed by value.
__device__ __noinline__ float pz_penalize_v(float x, int id, float rep, float pres, float freq,
                                            int hcap, const pz_lds_i32* hkey,
                                            const pz_lds_i32* hcnt) {
  return pz_penalize_inline(x, id, rep, pres, freq, hcap, hkey, hcnt);
}

__device__ __forceinline__ float pz_penalize(const PzPenalty& P, float x, int id) {
  return pz_penalize_v(x, id, P.rep, P.pres, P.freq, P.hcap, P.hkey, P.hcnt);
}

// 4-bit membership nibble for the aligned group of 4 ids starting at i
// (i in [base, lim), base a multiple of 32).
__device__ __forceinline__ uint32_t pz_pen_nibble(const PzPenalty& P, int i) {
  return (P.bitmap[(i - P.base) >> 5] >> (i & 31)) & 0xfu;
}

__device__ __forceinline__ bool pz_pen_member(const PzPenalty& P, int i) {
  return (P.bitmap[(i - P.base) >> 5] >> (i & 31)) & 1u;
}

// Temperature (temperature.c:8-25): x*(1/T) for the AVX-512 build, x/T for
// the scalar build.  inv_t is 1.0f/T rounded on the host, t is T clamped.
__device__ __forceinline__ float pz_temper(float x, const pz_row_params_dev& p) {
  return p.temp_div ? x / p.temp : x * p.inv_temp;
}

// Correctly rounded x / t, out of line (the division form is the reference's
// scalar-build temperature, temperature.c:22-23).
__device__ __noinline__ float pz_div(float x, float t) { return x / t; }

// The same, with the row's parameters held in registers.
struct PzTemp {
  float t, inv;
  int div;
  __device__ __forceinline__ static PzTemp of(const pz_row_params_dev& p) {
    PzTemp r;
    r.t = p.temp;
    r.inv = p.inv_temp;
    r.div = p.temp_div;
    return r;
  }
  __device__ __forceinline__ float apply(float x) const { return div ? pz_div(x, t) : x * inv; }
  // Four values with one choice of form (values past a row's end are
  // transformed too; callers ignore them).
  __device__ __forceinline__ void apply4(float (&y)[4]) const {
    if (div) {
#pragma unroll
      for (int c = 0; c < 4; c++) y[c] = pz_div(y[c], t);
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++) y[c] = y[c] * inv;
    }
  }
};

// Value the sampling chain sees for raw logit x of id i: penalties (when the
// row has any), then temperature.
__device__ __forceinline__ float pz_transform(const PzPenalty& P, const pz_row_params_dev& prm,
                                              float x, int i) {
  if (P.active && pz_pen_member(P, i)) x = pz_penalize(P, x, i);
  return pz_temper(x, prm);
}
__device__ __forceinline__ float pz_transform(const PzPenalty& P, const PzTemp& T, float x,
                                              int i) {
  if (P.active && pz_pen_member(P, i)) x = pz_penalize(P, x, i);
  return T.apply(x);
}

// ---------------------------------------------------------------------------
// (value, id) argmax combine with lowest-id tie-break.  NaN values never
// enter (the caller filters with x > best).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void pz_argmax_combine(float& bv, int& bi, float ov, int oi) {
  if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}

__device__ __forceinline__ void pz_wave_argmax(float& bv, int& bi) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, PZ_WAVE);
    const int oi = __shfl_xor(bi, off, PZ_WAVE);
    pz_argmax_combine(bv, bi, ov, oi);
  }
}

// Block-wide argmax; result valid in every thread.  scratch: 2*BLOCK/64 words.
template <int BLOCK>
__device__ void pz_block_argmax(float& bv, int& bi, float* sv, int* si) {
  pz_wave_argmax(bv, bi);
  const int lane = threadIdx.x & (PZ_WAVE - 1), wid = threadIdx.x / PZ_WAVE;
  if (lane == 0) { sv[wid] = bv; si[wid] = bi; }
  __syncthreads();
  if (threadIdx.x < PZ_WAVE) {
    constexpr int NW = BLOCK / PZ_WAVE;
    bv = lane < NW ? sv[lane] : -__builtin_inff();
    bi = lane < NW ? si[lane] : 0x7fffffff;
    pz_wave_argmax(bv, bi);
    if (lane == 0) { sv[0] = bv; si[0] = bi; }
  }
  __syncthreads();
  bv = sv[0];
  bi = si[0];
  __syncthreads();
}

// Wave-wide reductions with DPP (row shifts + row broadcasts: no LDS round
// trip).  The inclusive scan leaves the total in lane 63.
#define PZ_DPPF(v, ident, ctrl, rmask)                                                   \
  __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(ident), __float_as_int(v), \
                                             (ctrl), (rmask), 0xf, false))

__device__ __forceinline__ float pz_wave_sum(float v) {
  v += PZ_DPPF(v, 0.0f, 0x111, 0xf);
  v += PZ_DPPF(v, 0.0f, 0x112, 0xf);
  v += PZ_DPPF(v, 0.0f, 0x114, 0xf);
  v += PZ_DPPF(v, 0.0f, 0x118, 0xf);
  v += PZ_DPPF(v, 0.0f, 0x142, 0xa);
  v += PZ_DPPF(v, 0.0f, 0x143, 0xc);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float pz_wave_max(float v) {
  const float ninf = -__builtin_inff();
  v = fmaxf(v, PZ_DPPF(v, ninf, 0x111, 0xf));
  v = fmaxf(v, PZ_DPPF(v, ninf, 0x112, 0xf));
  v = fmaxf(v, PZ_DPPF(v, ninf, 0x114, 0xf));
  v = fmaxf(v, PZ_DPPF(v, ninf, 0x118, 0xf));
  v = fmaxf(v, PZ_DPPF(v, ninf, 0x142, 0xa));
  v = fmaxf(v, PZ_DPPF(v, ninf, 0x143, 0xc));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
