// pz_exact.h -- exact, parallel evaluation of a sequential fp32 sum of
// non-negative terms:  s = 0; for i: s = fl(s + v_i)  (round to nearest even).
//
// The reference accumulates every normaliser and CDF this way, one term at a
// time in fp32 (src/math/softmax.c:12-16, src/sampling/top_p.c:57-65 and
// :80-105, src/transformer/generate.c:162-168).  With ~10^5 terms that sum
// loses mass to swamping (up to ~3e-4 relative on a 128K-vocab row), so an
// accurate parallel sum does not reproduce the reference's probabilities.
//
// Method.  While s stays inside one binade [2^E, 2^(E+1)) every fp32 value
// there is a multiple of the grid G = ulp(s), so
//     fl(s + v) = s + G * rne(v / G)
// and the sequential sum is an INTEGER sum of per-term increments
// inc(v) = rne(v / G), which can be scanned in parallel.  The two exceptions
// are handled one element at a time with a real fp32 add:
//   * a term that makes s leave its binade (the integer state reaches 2^24, or
//     the term alone is at least 2^24 G), after which the grid doubles;
//   * a term sitting exactly halfway between two grid points (a tie), whose
//     rounding depends on the parity of the running state.
// The state is (n, g): s = n * 2^(g - 150) with g = max(biased exponent, 1),
// n < 2^24 (n >= 2^23 when g > 1).  Subnormals and the first normal binade
// share g = 1, whose grid is 2^-149 for both.
//
// The scalar part compiles for host and device, so the CPU tests can check
// pz_acc_add against plain fp32 addition.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define PZ_HD __host__ __device__ __forceinline__
#else
#define PZ_HD static inline
#endif

PZ_HD uint32_t pz_fbits(float f) { return __builtin_bit_cast(uint32_t, f); }
PZ_HD float pz_bitsf(uint32_t u) { return __builtin_bit_cast(float, u); }

struct PzAcc {
  uint32_t n;  // integer state, < 2^24
  uint32_t g;  // grid exponent: s = n * 2^(g - 150), g >= 1
};

enum { PZ_INC_PLAIN = 0, PZ_INC_TIE = 1, PZ_INC_BIG = 2 };

PZ_HD PzAcc pz_acc_of(float s) {
  const uint32_t b = pz_fbits(s);
  const uint32_t e = b >> 23;
  const uint32_t g = e > 1u ? e : 1u;
  PzAcc a;
  a.n = b - ((g - 1u) << 23);
  a.g = g;
  return a;
}

PZ_HD float pz_acc_value_ng(uint32_t n, uint32_t g) { return pz_bitsf(((g - 1u) << 23) + n); }
PZ_HD float pz_acc_value(PzAcc a) { return pz_acc_value_ng(a.n, a.g); }

// Increment of a term v >= 0 (finite) at grid exponent g.  *cls is PLAIN
// (the increment is exact), TIE (v / G is exactly m + 1/2: the increment is m
// and the caller rounds by parity) or BIG (v alone is >= 2^24 G: the sum
// certainly leaves the binade; the increment is 0 and meaningless).
PZ_HD uint32_t pz_inc(float v, uint32_t g, uint32_t* cls) {
  // branch-free: k = g - (the term's exponent) is the right shift that puts
  // the term on the grid; shifts are clamped below 32 (k > 25 rounds to 0)
  const uint32_t b = pz_fbits(v);
  const uint32_t ev = b >> 23;
  const uint32_t mv = (b & 0x7fffffu) | (ev ? 0x800000u : 0u);
  const uint32_t evb = ev ? ev : 1u;
  const bool big = evb > g;
  const uint32_t k = big ? 0u : g - evb;
  const uint32_t ks = k > 26u ? 26u : k;
  const uint32_t mask = (2u << (ks > 0u ? ks - 1u : 0u)) - 1u;  // the low k bits (k >= 1)
  const uint32_t half = ks > 0u ? 1u << (ks - 1u) : 0u;
  const uint32_t rem = mv & mask;
  const bool far = k > 25u;
  const bool tie = !big && !far && k > 0u && rem == half;
  const uint32_t up = (k > 0u && rem > half) ? 1u : 0u;
  *cls = big ? PZ_INC_BIG : (tie ? PZ_INC_TIE : PZ_INC_PLAIN);
  return big || far ? 0u : (mv >> ks) + up;
}

// s = fl(s + v) on the integer state, v >= 0 finite.
PZ_HD PzAcc pz_acc_add(PzAcc a, float v) {
  if (a.g >= 255u) return a;  // +inf stays +inf
  uint32_t cls;
  uint32_t inc = pz_inc(v, a.g, &cls);
  if (cls != PZ_INC_BIG) {
    if (cls == PZ_INC_TIE) inc += (a.n + inc) & 1u;
    const uint32_t m = a.n + inc;
    if (m < (1u << 24)) {
      PzAcc r;
      r.n = m;
      r.g = a.g;
      return r;
    }
  }
  // the sum leaves the binade: one real fp32 add (round to nearest even)
  return pz_acc_of(pz_acc_value(a) + v);
}

#if defined(__HIPCC__) || defined(__HIP__)
#include <hip/hip_runtime.h>

// ---------------------------------------------------------------------------
// Wave64 building blocks (DPP row shifts + row broadcasts, gfx9 family).
// ---------------------------------------------------------------------------
#define PZ_DPP(v, ctrl, rmask) \
  ((uint32_t)__builtin_amdgcn_update_dpp(0, (int)(v), (ctrl), (rmask), 0xf, false))

// Inclusive prefix sum over the 64 lanes (lane 0 first).
__device__ __forceinline__ uint32_t pz_wave_scan_u32(uint32_t v) {
  v += PZ_DPP(v, 0x111, 0xf);  // row_shr:1
  v += PZ_DPP(v, 0x112, 0xf);  // row_shr:2
  v += PZ_DPP(v, 0x114, 0xf);  // row_shr:4
  v += PZ_DPP(v, 0x118, 0xf);  // row_shr:8
  v += PZ_DPP(v, 0x142, 0xa);  // row_bcast:15 -> rows 1, 3
  v += PZ_DPP(v, 0x143, 0xc);  // row_bcast:31 -> rows 2, 3
  return v;
}

__device__ __forceinline__ uint32_t pz_readlane_u32(uint32_t v, int lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}
__device__ __forceinline__ float pz_readlane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ uint32_t pz_wave_sum_u32(uint32_t v) {
  return pz_readlane_u32(pz_wave_scan_u32(v), 63);
}

// Inclusive prefix sum of floats over the lanes (any rounding: used only for
// estimates).
__device__ __forceinline__ float pz_wave_scan_f32(float v) {
#define PZ_DPPF_(v, ctrl, rmask) \
  __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), (ctrl), (rmask), 0xf, false))
  v += PZ_DPPF_(v, 0x111, 0xf);
  v += PZ_DPPF_(v, 0x112, 0xf);
  v += PZ_DPPF_(v, 0x114, 0xf);
  v += PZ_DPPF_(v, 0x118, 0xf);
  v += PZ_DPPF_(v, 0x142, 0xa);
  v += PZ_DPPF_(v, 0x143, 0xc);
#undef PZ_DPPF_
  return v;
}

// Comparison used to stop an accumulation: GT stops at the first element
// whose running sum is > thr (the reference's `r < cdf`), GE at the first
// whose running sum is >= thr (top_p.c:83 `cumulative >= top_p`).
enum { PZ_STOP_NONE = 0, PZ_STOP_GT = 1, PZ_STOP_GE = 2 };

__device__ __forceinline__ bool pz_stop_hit(float s, float thr, int mode) {
  return mode == PZ_STOP_GT ? (thr < s) : (mode == PZ_STOP_GE ? (s >= thr) : false);
}

// The same accumulation as pz_wave_accumulate over elements [start, 256) of
// the 4 per lane a wave holds, by real fp32 adds in id order: a systolic DPP
// chain in which, at each of 64 steps, every lane adds its four terms in
// turn to its predecessor's value of the step before (wave_shr:1; the terms
// before start count as 0, and lane 0 starts from the state's value), so
// lane j holds its running sums from step j on.  With a stop mode, or cum,
// each lane's four running sums are formed again from its predecessor's
// final value -- the same adds.  A fixed 256 dependent adds: for segments
// whose exceptional terms (ties, binade exits, terms as large as the sum)
// are too many to take one at a time.  Returns the first hit index, or -1;
// cum receives the running sums up to the hit.
__device__ __forceinline__ int pz_wave_chain4(PzAcc& st, const float (&v)[4], int start, float thr,
                                              int stop_mode, float* cum) {
  const int lane = threadIdx.x & 63;
  const float s = pz_acc_value(st);
  float t[4];
#pragma unroll
  for (int c = 0; c < 4; c++) t[c] = 4 * lane + c >= start ? v[c] : 0.0f;
  // lane 0's first term carries the state (the shift gives lane 0 a +0.0,
  // and +0.0 + x == x for the non-negative sums here)
  const float a0 = lane == 0 ? s + t[0] : t[0];
  float c = 0.0f;
  for (int q = 0; q < 64; q += 8) {
#pragma unroll
    for (int u = 0; u < 8; u++) {
      c = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(c), 0x138, 0xf, 0xf,
                                                     true)) + a0;
      c = c + t[1];
      c = c + t[2];
      c = c + t[3];
    }
  }
  if (stop_mode != PZ_STOP_NONE || cum) {
    const float p = __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(c), 0x138, 0xf, 0xf, true));
    float pc[4];
    pc[0] = p + a0;
    pc[1] = pc[0] + t[1];
    pc[2] = pc[1] + t[2];
    pc[3] = pc[2] + t[3];
    int hit = 256;
    if (stop_mode != PZ_STOP_NONE) {
      uint32_t m = 0;
#pragma unroll
      for (int e = 0; e < 4; e++)
        m |= (4 * lane + e >= start && pz_stop_hit(pc[e], thr, stop_mode) ? 1u : 0u) << e;
      const uint64_t ball = __ballot(m != 0u);
      if (ball) {
        const int L = (int)__builtin_ctzll(ball);
        hit = 4 * L + (int)__builtin_ctz(pz_readlane_u32(m, L));
      }
    }
    if (cum) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int idx = 4 * lane + e;
        if (idx >= start && idx <= hit) cum[idx] = pc[e];
      }
    }
    if (hit < 256) {
      const int L = hit >> 2, e = hit & 3;
      float h = pz_readlane_f32(pc[0], L);
#pragma unroll
      for (int q = 1; q < 4; q++) {
        const float x = pz_readlane_f32(pc[q], L);
        h = q == e ? x : h;
      }
      st = pz_acc_of(h);
      return hit;
    }
  }
  st = pz_acc_of(pz_readlane_f32(c, 63));
  return -1;
}

// Exact sequential accumulation of the 64*C terms a wave holds, lane-major
// (element index lane*C + c), starting at element `start`.  st is
// wave-uniform and is advanced past the processed terms.  With a stop mode,
// returns the index of the first element whose running sum hits thr (st is
// then the sum including it); otherwise, or when nothing hits, returns -1.
// cum (optional, LDS or global) receives every processed running sum.
template <int C>
__device__ __forceinline__ int pz_wave_accumulate(PzAcc& st, const float (&v)[C], int start, float thr,
                                  int stop_mode, float* cum) {
  const int lane = threadIdx.x & 63;
  int pos = start;
  int rounds = 0;
  static_assert(C == 4, "four terms per lane");
  while (pos < 64 * C) {
    // past the first event: the rest of the segment by the chain of real adds
    if (++rounds > 1) return pz_wave_chain4(st, v, pos, thr, stop_mode, cum);
    // increments at the current grid; a flagged term (tie or big) ends the
    // lane's run of plain terms
    uint32_t inc[C];
    uint32_t flag = 0;
#pragma unroll
    for (int c = 0; c < C; c++) {
      uint32_t cls;
      const uint32_t i = pz_inc(v[c], st.g, &cls);
      const bool valid = lane * C + c >= pos;
      const bool f = valid && cls != PZ_INC_PLAIN;
      inc[c] = valid && !f ? i : 0u;
      flag |= (f ? 1u : 0u) << c;
    }
    const int first_flag = flag ? (int)__builtin_ctz(flag) : C;
    uint32_t lsum = 0;
#pragma unroll
    for (int c = 0; c < C; c++) lsum += c < first_flag ? inc[c] : 0u;
    const uint32_t incl = pz_wave_scan_u32(lsum);
    const uint32_t excl = incl - lsum;
    // this lane's first event: a binade exit, a stop hit, or the flagged
    // term (selects, no branches)
    uint32_t run = st.n + excl;
    int ev = first_flag, ev_kind = first_flag < C ? 1 : 0;
    uint32_t ev_n = 0;
    bool open = true;  // no exit or hit yet among the terms before the flag
#pragma unroll
    for (int c = 0; c < C; c++) {
      const bool live = open && c < first_flag;
      const uint32_t nr = run + inc[c];
      const bool cross = live && nr >= (1u << 24);
      const bool hit = live && !cross && stop_mode != PZ_STOP_NONE && lane * C + c >= pos &&
                       pz_stop_hit(pz_acc_value_ng(nr, st.g), thr, stop_mode);
      ev_n = cross ? run : (hit ? nr : ev_n);
      ev = cross || hit ? c : ev;
      ev_kind = cross ? 1 : (hit ? 2 : ev_kind);
      run = live && !cross ? nr : run;
      open = open && !cross && !hit;
    }
    if (open) ev_n = run;  // the flagged term's state: every term before it
    const uint64_t ball = __ballot(ev < C);
    const int L = ball ? (int)__builtin_ctzll(ball) : 64;
    if (cum) {
      // running sums of the terms before the first event (plus a stop hit)
      uint32_t r2 = st.n + excl;
#pragma unroll
      for (int c = 0; c < C; c++) {
        const int idx = lane * C + c;
        if (idx < pos) continue;
        const bool valid = lane < L || (lane == L && (c < ev || (c == ev && ev_kind == 2)));
        if (!valid) continue;
        r2 += inc[c];
        cum[idx] = pz_acc_value_ng(r2, st.g);
      }
    }
    if (!ball) {
      st.n += pz_readlane_u32(incl, 63);
      return -1;
    }
    const int cL = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(ev, L));
    const int kind = __builtin_amdgcn_readlane(ev_kind, L);
    const int idx = L * C + cL;
    st.n = pz_readlane_u32(ev_n, L);
    if (kind == 2) return idx;
    // term cL of lane L: read every c and select (an index into v[] by the
    // run-time cL would put the array in scratch memory)
    float vv = pz_readlane_f32(v[0], L);
#pragma unroll
    for (int c = 1; c < C; c++) {
      const float vc = pz_readlane_f32(v[c], L);
      vv = c == cL ? vc : vv;
    }
    st = pz_acc_add(st, vv);
    const float sv = pz_acc_value(st);
    if (cum && lane == 0) cum[idx] = sv;
    if (stop_mode != PZ_STOP_NONE && pz_stop_hit(sv, thr, stop_mode)) return idx;
    pos = idx + 1;
  }
  return -1;
}

// Grid exponent of the binade an estimate s >= 0 falls in.
__device__ __forceinline__ uint32_t pz_grid_of(float s) {
  const uint32_t e = __float_as_uint(s) >> 23;
  return e > 1u ? e : 1u;
}
#endif
