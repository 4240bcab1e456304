// pz_rowpass.h -- streaming passes of one 1024-thread workgroup over one
// logits row, shared by the kernels whose normaliser or CDF is a full-row
// sequential fp32 sum (top-p, plain categorical, speculative verification).
//
// Layout: the row is walked in tiles of 4096 elements, one 128-bit load per
// thread per tile; thread t of a tile holds elements 4t..4t+3.  A segment is
// one wave's 256-element slice of a tile (segment k = tile*16 + wave), the
// unit at which the exact-sum records (pz_exact.h) are kept.
//
// Passes:
//   pass 1   the row maximum (and NaN / y[0] checks): the compulsory HBM read;
//   records  per chunk of 4 tiles: the exact terms are computed once, their
//            fp32 segment sums estimate the running sum, from which each
//            segment's binade is predicted; the segment's integer increment
//            sum is then recorded at that grid (and at the grid below when
//            the estimate sits within 1% above a power of two).  Segments
//            whose terms need element-wise treatment (ties, terms as large
//            as the running sum) keep their terms in an LDS cache;
//   walk     one wave scans the records in order with the exact state and
//            accumulates element by element wherever a record does not
//            apply (pz_rec_walk).
#pragma once
#include "pz_device.h"
#include "pz_exact.h"

constexpr int PZ_RB = 1024;           // threads per row workgroup
constexpr int PZ_TILE = PZ_RB * 4;    // elements per tile
constexpr int PZ_SEG = 256;           // elements per segment
constexpr int PZ_SEGS_PER_TILE = PZ_RB / 64;
constexpr int PZ_REC_CHUNK = 4;       // tiles per record chunk (= 64 segments)
constexpr int PZ_REC_SLOTS = 32;      // dirty segments whose terms stay in LDS

__host__ __device__ inline int pz_tiles(int V) { return (V + PZ_TILE - 1) / PZ_TILE; }
__host__ __device__ inline int pz_nseg(int V) { return pz_tiles(V) * PZ_SEGS_PER_TILE; }

// First element of this thread's 4 in tile t, and of this lane's 4 in segment k.
__device__ __forceinline__ int pz_tile_e0(int t) { return t * PZ_TILE + 4 * (int)threadIdx.x; }
__device__ __forceinline__ int pz_seg_e0(int k) {
  return (k >> 4) * PZ_TILE + (k & 15) * PZ_SEG + 4 * ((int)threadIdx.x & 63);
}

// Raw logits of elements e0..e0+3 (e0 a multiple of 4).  Returns how many
// are < V; the others hold unspecified values.  The vector form always loads
// (from the last in-bounds float4 when e0 is past the row: rows are 16-byte
// aligned with ld a multiple of 4, so that float4 lies inside the row's ld
// elements), which keeps the loads unconditional and lets the compiler keep
// many in flight.
template <bool VEC, bool NT>
__device__ __forceinline__ int pz_load4(const float* __restrict__ x, int V, int e0, float (&r)[4]) {
  int n = V - e0;
  n = n < 0 ? 0 : (n > 4 ? 4 : n);
  if (VEC) {
    const int last4 = (V - 1) & ~3;
    const pz_f4* p = reinterpret_cast<const pz_f4*>(x + (e0 < last4 ? e0 : last4));
    const pz_f4 v = NT ? __builtin_nontemporal_load(p) : *p;
    r[0] = v.x;
    r[1] = v.y;
    r[2] = v.z;
    r[3] = v.w;
    return n;
  }
#pragma unroll
  for (int c = 0; c < 4; c++) r[c] = c < n ? x[e0 + c] : 0.0f;
  return n;
}

// One row as the sampling chain sees it: y_i = temperature(penalties(x_i)).
template <bool VEC>
struct PzRow {
  const float* x;
  int V;
  PzPenalty P;
  PzTemp T;

  // raw logits of elements e0..e0+3 (count < V returned), then the chain
  __device__ __forceinline__ int load(int e0, float (&y)[4]) const {
    return pz_load4<VEC, false>(x, V, e0, y);
  }
  // (the history members among the four from one bitmap read, then the
  // temperature on all four: values past the row's end are ignored by the
  // callers)
  __device__ __forceinline__ void apply(int e0, int n, float (&y)[4]) const {
    if (P.active && n > 0) {
      const uint32_t nib = pz_pen_nibble(P, e0) & ((1u << n) - 1u);
      if (nib) {
#pragma unroll
        for (int c = 0; c < 4; c++)
          if ((nib >> c) & 1u) y[c] = pz_penalize(P, y[c], e0 + c);
      }
    }
    T.apply4(y);
  }
  __device__ __forceinline__ int get(int e0, float (&y)[4]) const {
    const int n = load(e0, y);
    apply(e0, n, y);
    return n;
  }
};

// A plain row scaled by temperature only (speculative verification).
template <bool VEC>
struct PzTempRow {
  const float* x;
  int V;
  PzTemp T;

  __device__ __forceinline__ int load(int e0, float (&y)[4]) const {
    return pz_load4<VEC, false>(x, V, e0, y);
  }
  __device__ __forceinline__ void apply(int e0, int n, float (&y)[4]) const {
    (void)e0;
    (void)n;  // values past the row's end are transformed too and ignored
    T.apply4(y);
  }
  __device__ __forceinline__ int get(int e0, float (&y)[4]) const {
    const int n = load(e0, y);
    apply(e0, n, y);
    return n;
  }
};

struct PzPass1Shared {
  float red[PZ_RB / 64];
  int any_nan;
  float y0;
};

// Pass 1 (the one compulsory HBM read of the row): the row maximum (NaN
// ignored, as the reference's strict '>' scans do), whether any y is NaN,
// and y[0].  Returns the maximum in every thread.
template <int U, class Row>
__device__ __forceinline__ float pz_pass1(const Row& row, int ntiles, PzPass1Shared& S) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (tid == 0) S.any_nan = 0;
  float tmax = -__builtin_inff();
  bool nan = false;
  for (int t0 = 0; t0 < ntiles; t0 += U) {
    float r[U][4];
    int nv[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      nv[u] = 0;
      if (t0 + u < ntiles) nv[u] = row.load(pz_tile_e0(t0 + u), r[u]);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int t = t0 + u;
      if (t >= ntiles) continue;
      row.apply(pz_tile_e0(t), nv[u], r[u]);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        if (c >= nv[u]) continue;
        const float y = r[u][c];
        if (y != y) nan = true;
        else tmax = fmaxf(tmax, y);
      }
      if (t == 0 && tid == 0) S.y0 = r[u][0];
    }
  }
  tmax = pz_wave_max(tmax);
  if (__ballot(nan) && lane == 0) S.any_nan = 1;
  if (lane == 0) S.red[w] = tmax;
  __syncthreads();
  float M = S.red[0];
#pragma unroll
  for (int i = 1; i < PZ_RB / 64; i++) M = fmaxf(M, S.red[i]);
  return M;
}

// ---------------------------------------------------------------------------
// Exact-sum records
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) float pz_lds_f32;
typedef __attribute__((address_space(3))) pz_f4 pz_lds_f4;

// Sentinel gf of a segment without a record (the walk regenerates it).
constexpr uint32_t PZ_NO_RECORD = 0xffffffffu;
// gf = grid | DIRTY (record at grid unusable) | HAS2 (record at grid - 1) |
// DIRTY2 (that one unusable) | XING (the estimate leaves the binade inside
// the segment)
constexpr uint32_t PZ_GF_DIRTY = 0x100u, PZ_GF_HAS2 = 0x200u, PZ_GF_DIRTY2 = 0x400u,
                   PZ_GF_XING = 0x800u;

struct PzRec {
  pz_lds_u32* d;      // [nseg] increment sum at the predicted grid
  pz_lds_u32* d2;     // [nseg] increment sum at the grid below
  pz_lds_u32* gf;     // [nseg] grid and flags
  pz_lds_f32* a;      // [nseg] estimate of the segment's sum
  pz_lds_i32* slot;   // [nseg] LDS cache slot of the segment's terms, or -1
  pz_lds_f32* cache;  // [PZ_REC_SLOTS][256]
};

__host__ __device__ inline size_t pz_rec_bytes(int V) {
  return (size_t)pz_nseg(V) * 20 + (size_t)PZ_REC_SLOTS * PZ_SEG * 4;
}

// Carves the record arrays out of LDS at base (16-byte aligned).
__device__ __forceinline__ PzRec pz_rec_at(char* base, int nseg) {
  PzRec R;
  R.cache = (pz_lds_f32*)base;
  char* p = base + (size_t)PZ_REC_SLOTS * PZ_SEG * 4;
  R.d = (pz_lds_u32*)p;
  R.d2 = R.d + nseg;
  R.gf = R.d2 + nseg;
  R.a = (pz_lds_f32*)(R.gf + nseg);
  R.slot = (pz_lds_i32*)(R.a + nseg);
  return R;
}

struct PzRecShared {
  int slots_used;
  int stop;
  int hit;
  float sum;
};

// Predicted grid (and whether to record the grid below too) of a segment
// whose running sum is estimated to start at s.
__device__ __forceinline__ uint32_t pz_predict_gf(float s) {
  const uint32_t g = pz_grid_of(s);
  const bool near = g > 1u && (__float_as_uint(s) & 0x7fffffu) < 83886u;  // < 1% above 2^E
  return g | (near ? PZ_GF_HAS2 : 0u);
}

template <class X>
__device__ __forceinline__ void pz_rec_segment(const X& x, const typename X::Raw& raw,
                                               const float (&a)[4], uint32_t gf, int k,
                                               const PzRec& R, PzRecShared& S) {
  const int lane = threadIdx.x & 63;
  const uint32_t g = gf & 0xffu;
  const bool has2 = (gf & PZ_GF_HAS2) != 0;
  uint32_t s1 = 0, s2 = 0;
  bool d1 = false, d2 = false;
  x.inc4(raw, a, g, s1, d1);
  if (has2) {
    x.inc4(raw, a, g - 1u, s2, d2);
    s2 = pz_wave_sum_u32(s2);
  }
  s1 = pz_wave_sum_u32(s1);
  const bool D1 = __ballot(d1) != 0;
  const bool D2 = has2 && __ballot(d2) != 0;
  int slot = -1;
  if ((D1 && (!has2 || D2)) || (gf & PZ_GF_XING)) {
    // the walk will go through this segment element by element: keep what
    // it needs in LDS
    if (lane == 0) slot = atomicAdd(&S.slots_used, 1);
    slot = __builtin_amdgcn_readfirstlane(slot);
    if (slot >= PZ_REC_SLOTS) slot = -1;
    if (slot >= 0) x.cache_put(R.cache + slot * PZ_SEG, raw, a);
  }
  if (lane == 0) {
    R.d[k] = s1;
    R.d2[k] = s2;
    R.gf[k] = (gf & (0xffu | PZ_GF_HAS2 | PZ_GF_XING)) | (D1 ? PZ_GF_DIRTY : 0u) |
              (D2 ? PZ_GF_DIRTY2 : 0u);
    R.slot[k] = slot;
  }
}

// Records pass over the row's terms (see the header).  X provides
//   typename Raw;                  per-thread data of 4 elements
//   int  load(e0, Raw&)            issues the loads, returns the count < V
//   void prep(e0, n, Raw&, a[4])   finishes the element data, estimates the
//                                  terms (relative error < 2^-16)
//   void observe(e0, Raw&, a[4])   per-kernel side work (histograms, ...)
//   void inc4(Raw&, a[4], g, s&, dirty&)  adds the exact increments of the
//                                  four terms at grid g to s; sets dirty on a
//                                  tie or a big term
//   void cache_put(lds, Raw&, a[4]) / cache_terms(lds, v[4])
//                                  keep / rebuild a segment's exact terms
//   void seg(k, v[4])              exact terms of segment k from memory
// Recording stops after the chunk in which the estimated running sum passes
// stop_after; later segments get PZ_NO_RECORD.  Every thread calls it; it
// ends with the records complete (after a barrier).
template <class X>
__device__ __forceinline__ void pz_record_pass(X& x, int ntiles, const PzRec& R, PzRecShared& S,
                                               float stop_after) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nseg = ntiles * PZ_SEGS_PER_TILE;
  constexpr int U = PZ_REC_CHUNK;
  if (tid == 0) {
    S.slots_used = 0;
    S.stop = 0;
  }
  float carry = 0.0f;  // wave 0: estimated running sum at the chunk start
  int t0 = 0;
  for (; t0 < ntiles; t0 += U) {
    typename X::Raw raw[U];
    int nv[U];
    float a[U][4];
#pragma unroll
    for (int u = 0; u < U; u++) {
      nv[u] = 0;
      if (t0 + u < ntiles) nv[u] = x.load(pz_tile_e0(t0 + u), raw[u]);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int t = t0 + u;
      if (t >= ntiles) continue;
      const int e0 = pz_tile_e0(t);
      x.prep(e0, nv[u], raw[u], a[u]);
      x.observe(e0, raw[u], a[u]);
      const float sa = pz_wave_sum((a[u][0] + a[u][1]) + (a[u][2] + a[u][3]));
      if (lane == 0) R.a[t * PZ_SEGS_PER_TILE + w] = sa;
    }
    __syncthreads();
    if (w == 0) {
      // U * 16 == 64 segments per chunk: one lane each
      const int k = t0 * PZ_SEGS_PER_TILE + lane;
      const bool in = k < nseg;
      const float sa = in ? R.a[k] : 0.0f;
      const float incl = pz_wave_scan_f32(sa);
      const float start = carry + (incl - sa), end = carry + incl;
      if (in)
        R.gf[k] = pz_predict_gf(start) | (pz_grid_of(end) != pz_grid_of(start) ? PZ_GF_XING : 0u);
      carry += pz_readlane_f32(incl, 63);
      if (lane == 0 && carry > stop_after) S.stop = 1;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int t = t0 + u;
      if (t >= ntiles) continue;
      const int k = t * PZ_SEGS_PER_TILE + w;
      pz_rec_segment(x, raw[u], a[u], R.gf[k], k, R, S);
    }
    if (S.stop) {
      t0 += U;
      break;
    }
  }
  for (int k = t0 * PZ_SEGS_PER_TILE + tid; k < nseg; k += PZ_RB) {
    R.gf[k] = PZ_NO_RECORD;
    R.slot[k] = -1;
  }
  __syncthreads();
}

// Walk over the records in order (one wave): a record is used when it was
// made at the state's grid and is clean; the state then only advances by an
// integer (checked to stay in the binade).  Any other segment is accumulated
// element by element from its cached or regenerated terms.  With a stop mode
// returns the element index of the first hit, else -1.
template <class X>
__device__ __forceinline__ int pz_rec_walk(PzAcc& st, const PzRec& R, int nseg, float thr,
                                           int stop_mode, const X& x) {
  const int lane = threadIdx.x & 63;
  int k0 = 0;
  while (k0 < nseg) {
    const int k = k0 + lane;
    uint32_t d = 0;
    bool ok = false;
    if (k < nseg) {
      const uint32_t gf = R.gf[k];
      if (gf != PZ_NO_RECORD) {
        const uint32_t g = gf & 0xffu;
        if (g == st.g && !(gf & PZ_GF_DIRTY)) {
          ok = true;
          d = R.d[k];
        } else if ((gf & PZ_GF_HAS2) && g - 1u == st.g && !(gf & PZ_GF_DIRTY2)) {
          ok = true;
          d = R.d2[k];
        }
      }
    }
    const uint32_t incl = pz_wave_scan_u32(d);
    const uint32_t nend = st.n + incl;
    bool bad = false;
    if (k < nseg) {
      bad = !ok || nend >= (1u << 24) ||
            (stop_mode != PZ_STOP_NONE &&
             pz_stop_hit(pz_acc_value_ng(nend, st.g), thr, stop_mode));
    }
    const uint64_t ball = __ballot(bad);
    if (!ball) {
      st.n += pz_readlane_u32(incl, 63);
      k0 += 64;
      continue;
    }
    const int L = (int)__builtin_ctzll(ball);
    const int kb = k0 + L;
    st.n += pz_readlane_u32(incl - d, L);
    float v[4];
    const int slot = R.slot[kb];
    if (slot >= 0) x.cache_terms(R.cache + slot * PZ_SEG, v);
    else x.seg(kb, v);
    const int f = pz_wave_accumulate<4>(st, v, 0, thr, stop_mode, nullptr);
    if (f >= 0) return kb * PZ_SEG + f;
    k0 = kb + 1;
  }
  return -1;
}

// Estimate of expf(d) with the hardware exp2.  Its relative error grows with
// |d|: the fp32 product d*log2(e) carries an absolute error of about
// |d| * 2^-23 in the exponent, plus v_exp_f32's own.  The bound used below,
// (|d| + 2) * 2^-23, is checked on every fp32 d in [-104, 0] where expf(d)
// is normal.  Only used where pz_inc_from_estimate can prove the rounding it
// decides.
__device__ __forceinline__ float pz_fast_exp(float d) {
  return __builtin_amdgcn_exp2f(d * 1.44269504088896341f);
}

// Increment of a term at grid g from an estimate a of expf(d) (times a
// factor rounded once more, for probabilities) when that settles the
// rounding; otherwise sets *exact (the caller then evaluates the term
// exactly).  The estimate's relative error is below (|d| + 3) * 2^-23; the
// test uses twice that.  Grids below 2^-100 (only at the very start of a
// row) always take the exact path, so estimates that underflow cannot
// matter; so do terms of 2^20 grid steps or more, whose fraction fp32 no
// longer resolves against the bound.
// Branch-free (selects only): the value returned is meaningful only where
// *exact is false.  a == 0 gives t = 0, fr = 0, no exact evaluation and 0.
__device__ __forceinline__ uint32_t pz_inc_from_estimate(float a, float d, uint32_t g,
                                                         bool* exact) {
  const uint32_t gc = g < 50u ? 50u : g;
  const float t = a * __uint_as_float((277u - gc) << 23);  // a / 2^(g - 150), exact
  // the nearest integer and the distance to it: a fraction at least the
  // margin away from one half rounds to that integer (round to nearest)
  const float r = __builtin_rintf(t);
  const float eps = (fabsf(d) + 3.0f) * 0x1p-22f;
  *exact = (g < 50u) | (t >= 1048576.0f) | (0.5f - fabsf(t - r) <= t * eps + 0x1p-20f);
  return (uint32_t)fminf(r, 1048576.0f);
}

// Terms of one row: e = expf(y - M) for y >= thr (0 otherwise), times inv
// when as_p.  Raw holds the elements' y (-inf past the row).
template <class Row>
struct PzExpTerms {
  typedef float Raw[4];
  Row R;
  float M, thr, inv;
  bool as_p;
  const pz_lds_u64* et;  // the workgroup's LDS copy of the expf table
  __device__ __forceinline__ int load(int e0, Raw& r) const { return R.load(e0, r); }
  __device__ __forceinline__ float exact_term(float y) const {
    const float e = y >= thr ? pz_expf_l(y - M, et) : 0.0f;
    return as_p ? e * inv : e;
  }
  __device__ __forceinline__ void prep(int e0, int n, Raw& r, float (&a)[4]) const {
    R.apply(e0, n, r);
    if (n < 4) {  // (only at the row's end)
#pragma unroll
      for (int c = 0; c < 4; c++)
        if (c >= n) r[c] = -__builtin_inff();
    }
    if (thr == -__builtin_inff()) {
      // no threshold: every term is estimated (exp2(-inf) = 0 past the end;
      // the callers without a threshold have no NaN row here)
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float e = pz_fast_exp(r[c] - M);
        a[c] = as_p ? e * inv : e;
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float e = r[c] >= thr ? pz_fast_exp(r[c] - M) : 0.0f;
        a[c] = as_p ? e * inv : e;
      }
    }
  }
  __device__ __forceinline__ void observe(int, const Raw&, const float (&)[4]) {}
  // The estimates settle most terms; the rest are evaluated exactly, one per
  // lane per round, so a wave calls the exact exponential once per round
  // rather than once per term position that any lane needed.  (A term the
  // estimate settles is neither a tie nor big: both fail its test.)
  __device__ __forceinline__ void inc4(const Raw& y, const float (&a)[4], uint32_t g,
                                       uint32_t& s, bool& dirty) const {
    uint32_t need = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {  // (selects: no exec-mask branches per term)
      bool ex;
      const uint32_t i = pz_inc_from_estimate(a[c], y[c] - M, g, &ex);
      need |= (ex ? 1u : 0u) << c;
      s += ex ? 0u : i;
    }
    while (__ballot(need != 0u)) {
      if (need) {
        const int c = __builtin_ctz(need);
        need &= need - 1u;
        uint32_t cls;
        s += pz_inc(exact_term(pz_sel4f(y[0], y[1], y[2], y[3], c)), g, &cls);
        dirty |= cls != PZ_INC_PLAIN;
      }
    }
  }
  // The cache keeps the exact terms, evaluated here by the segment's whole
  // wave in the parallel pass, so the serial walk only reads them.
  __device__ __forceinline__ void cache_put(pz_lds_f32* base, const Raw& y,
                                            const float (&)[4]) const {
    pz_f4 q;
    q.x = exact_term(y[0]);
    q.y = exact_term(y[1]);
    q.z = exact_term(y[2]);
    q.w = exact_term(y[3]);
    ((pz_lds_f4*)base)[threadIdx.x & 63] = q;
  }
  __device__ __forceinline__ void cache_terms(const pz_lds_f32* base, float (&v)[4]) const {
    const pz_f4 q = ((const pz_lds_f4*)base)[threadIdx.x & 63];
    v[0] = q.x;
    v[1] = q.y;
    v[2] = q.z;
    v[3] = q.w;
  }
  __device__ __forceinline__ void seg(int k, float (&v)[4]) const {
    Raw r;
    const int e0 = pz_seg_e0(k);
    const int n = R.get(e0, r);
#pragma unroll
    for (int c = 0; c < 4; c++) v[c] = c < n ? exact_term(r[c]) : 0.0f;
  }
};

// The reference's softmax normaliser (softmax.c:12-16; top_p.c:57-65 with
// thr = max - 20): exact sequential fp32 sum of the terms in ascending id.
// Called by every thread; returns the sum in every thread.
template <class X>
__device__ __forceinline__ float pz_exact_sum(X& x, int ntiles, const PzRec& R,
                                              PzRecShared& S) {
  pz_record_pass(x, ntiles, R, S, __builtin_inff());
  if (threadIdx.x < 64) {
    PzAcc st;
    st.n = 0;
    st.g = 1;
    pz_rec_walk(st, R, ntiles * PZ_SEGS_PER_TILE, 0.0f, PZ_STOP_NONE, x);
    if (threadIdx.x == 0) S.sum = pz_acc_value(st);
  }
  __syncthreads();
  return S.sum;
}

// The reference's categorical draw (generate.c:162-168): cdf += term in
// ascending id, the first index with r < cdf (-1 if none below V).  Called
// by every thread; returns the index in every thread.
template <class X>
__device__ __forceinline__ int pz_exact_draw(X& x, int V, int ntiles, float r, const PzRec& R,
                                             PzRecShared& S) {
  pz_record_pass(x, ntiles, R, S, r + 0.01f);
  if (threadIdx.x < 64) {
    PzAcc st;
    st.n = 0;
    st.g = 1;
    int hit = pz_rec_walk(st, R, ntiles * PZ_SEGS_PER_TILE, r, PZ_STOP_GT, x);
    if (hit >= V) hit = -1;  // padding terms are 0 and never raise the CDF
    if (threadIdx.x == 0) S.hit = hit;
  }
  __syncthreads();
  return S.hit;
}
