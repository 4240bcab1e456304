// pz_split.h -- one logits row shared by several workgroups, for the
// samplers whose normaliser or CDF is a full-row sequential fp32 sum
// (top-p, softmax + categorical draw, softmax output, speculative
// verification).
//
// A row of V logits is cut into segments of 256 ids (segment k holds ids
// 256k .. 256k+255: one wave, 4 per lane) and into slices of `spw`
// consecutive segments, one 1024-thread workgroup each, so a batch smaller
// than the CU count still spreads over the whole chip.  The passes are
// separate launches on one stream, so each one sees everything the previous
// ones wrote:
//
//   stat     (the compulsory HBM read) per slice its maximum and NaN flag,
//            and -- when the terms have no threshold -- per segment its
//            maximum m_k and s_k = sum exp(y - m_k) (hardware exp2: an
//            estimate of the segment's mass in units of exp(y - m_k)).
//   estimate (top-p only: its terms drop y < M - 20, which the stat pass
//            cannot know) per segment the estimated mass of its terms.
//   records  (L2 / Infinity Cache) each workgroup reduces the slice maxima
//            to the row maximum M, sums the estimates of the segments before
//            its own to predict the binade the exact running sum sits in at
//            each of its segments (pz_predict_gf), and records per segment
//            the integer increment sums of the exact terms at that binade
//            (pz_exact.h) in global memory.
//   walk     one workgroup per row stages the records in LDS; its waves
//            evaluate in parallel the exact terms of the segments the records
//            cannot serve (dirty ones, binade crossings) together with their
//            increment prefixes; then one wave walks the row in id order:
//            runs of clean records advance the integer state in one step
//            each, a crossing is located in its segment with one ballot
//            over the precomputed prefixes and taken with one real fp32 add.
//            The result is the reference's sequential fp32 sum, bit for bit.
// The passes that follow (top-p nucleus, CDF draw, softmax output,
// speculative residual) reuse the records and the walk with other terms.
#pragma once
#include "pz_device.h"
#include "pz_exact.h"
#include "pz_rowpass.h"

constexpr int PZ_SP_BLOCK = 1024;              // threads per workgroup
constexpr int PZ_SP_WAVES = PZ_SP_BLOCK / 64;  // 16
constexpr int PZ_SP_SEG = 256;                 // ids per segment
constexpr int PZ_SP_NC = 32;                   // special segments the walk pre-evaluates
constexpr int PZ_SP_TARGET_WG = 512;           // workgroups a launch aims for (2 per CU)
constexpr int PZ_SP_U = 4;                     // segments a wave loads per step

// Row flags (from the slices' maxima and NaN flags).
enum {
  PZ_RS_NAN = 1,      // some y is NaN
  PZ_RS_Y0NAN = 2,    // y[0] is NaN
  PZ_RS_NONFIN = 4,   // the NaN-free maximum is +-inf (or there is no value at all)
};

// Per-row values handed from pass to pass (device scratch, 64 bytes).
struct PzRowState {
  float M;          // maximum of the NaN-free y (-inf if none)
  float y0;         // y[0]
  uint32_t flags;   // PZ_RS_*
  float sum;        // exact sequential normaliser
  float inv;        // 1.0f / sum
  float f[3];       // pass-specific values
  int32_t i[8];     // pass-specific values
};

struct PzSplitWs {
  PzRowState* rs;     // [rows]
  uint32_t* arrive;   // [rows] arrival counters, zero between launches
  float* slice_m;     // [rows][smax] slice maxima (NaN-free)
  uint32_t* slice_f;  // [rows][smax] slice NaN flags
  float* seg_m;       // [rows][nsc] segment maxima (stat pass)
  float* seg_s;       // [rows][nsc] segment mass estimates
  uint32_t* rec;      // [rows][3][nsc] records: increments at g, at g - 1, grid+flags
  uint32_t* hist;     // [hslots][PZ_TOPP_NB] top-p mass histograms (or null)
  uint64_t* keys;     // [rows][capg] top-p candidates (or null)
  int nsc;            // segments per row the buffers hold
  int smax;           // slices per row the buffers hold
  int capg;           // top-p candidates per row the buffers hold
  int hslots;         // histogram slots (workgroups of one launch)
};

// Top-p mass histogram: bins of 1/64 binade over e in [2^-29, 1] (candidate
// terms are >= expf(-20) ~ 2^-28.9); smaller values land in bin 0.
constexpr int PZ_TOPP_NB_BASE = 98 << 6;
constexpr int PZ_TOPP_NB = (127 << 6) - PZ_TOPP_NB_BASE + 1;

__host__ __device__ inline int pz_sp_nseg(int V) { return (V + PZ_SP_SEG - 1) / PZ_SP_SEG; }

struct PzSplitPlan {
  int nseg;  // segments per row
  int spw;   // segments per workgroup (a multiple of 16 unless the row is shorter)
  int S;     // workgroups per row
};

// Slices so that a launch of nrows rows has about PZ_SP_TARGET_WG
// workgroups, each wave holding at least one segment, at most smax slices.
inline PzSplitPlan pz_split_plan(int V, int nrows, int smax) {
  PzSplitPlan p;
  p.nseg = pz_sp_nseg(V);
  int S = (PZ_SP_TARGET_WG + nrows - 1) / (nrows > 0 ? nrows : 1);
  const int smax_seg = (p.nseg + PZ_SP_WAVES - 1) / PZ_SP_WAVES;
  if (S > smax_seg) S = smax_seg;
  if (S > smax) S = smax;
  if (S < 1) S = 1;
  int spw = (p.nseg + S - 1) / S;
  spw = (spw + PZ_SP_WAVES - 1) / PZ_SP_WAVES * PZ_SP_WAVES;
  p.spw = spw;
  p.S = (p.nseg + spw - 1) / spw;
  return p;
}

// Bytes of a workspace for `rows` rows of up to V ids (top-p buffers when
// capg > 0); with base != nullptr also carves it.
inline size_t pz_split_ws_layout(int rows, int V, int capg, void* base, PzSplitWs* out) {
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  const int nsc = pz_sp_nseg(V);
  const int smax = (nsc + PZ_SP_WAVES - 1) / PZ_SP_WAVES;
  const int hslots = capg > 0 ? PZ_SP_TARGET_WG + rows : 0;
  const size_t R = (size_t)rows;
  size_t off = 0;
  const size_t o_rs = off;   off = up(off + R * sizeof(PzRowState));
  const size_t o_arr = off;  off = up(off + R * 4);
  const size_t o_sm = off;   off = up(off + R * smax * 4);
  const size_t o_sf = off;   off = up(off + R * smax * 4);
  const size_t o_segm = off; off = up(off + R * nsc * 4);
  const size_t o_segs = off; off = up(off + R * nsc * 4);
  const size_t o_rec = off;  off = up(off + R * 3 * nsc * 4);
  const size_t o_hist = off; off = up(off + (size_t)hslots * PZ_TOPP_NB * 4);
  const size_t o_keys = off; off = up(off + R * (size_t)(capg > 0 ? capg : 0) * 8);
  if (base && out) {
    char* b = static_cast<char*>(base);
    out->rs = reinterpret_cast<PzRowState*>(b + o_rs);
    out->arrive = reinterpret_cast<uint32_t*>(b + o_arr);
    out->slice_m = reinterpret_cast<float*>(b + o_sm);
    out->slice_f = reinterpret_cast<uint32_t*>(b + o_sf);
    out->seg_m = reinterpret_cast<float*>(b + o_segm);
    out->seg_s = reinterpret_cast<float*>(b + o_segs);
    out->rec = reinterpret_cast<uint32_t*>(b + o_rec);
    out->hist = hslots ? reinterpret_cast<uint32_t*>(b + o_hist) : nullptr;
    out->keys = capg > 0 ? reinterpret_cast<uint64_t*>(b + o_keys) : nullptr;
    out->nsc = nsc;
    out->smax = smax;
    out->capg = capg > 0 ? capg : 0;
    out->hslots = hslots;
  }
  return off;
}

#if defined(__HIPCC__) || defined(__HIP__)

__device__ __forceinline__ uint32_t* pz_sp_rec_d(const PzSplitWs& ws, int row) {
  return ws.rec + (size_t)row * 3 * ws.nsc;
}
__device__ __forceinline__ uint32_t* pz_sp_rec_d2(const PzSplitWs& ws, int row) {
  return ws.rec + (size_t)row * 3 * ws.nsc + ws.nsc;
}
__device__ __forceinline__ uint32_t* pz_sp_rec_gf(const PzSplitWs& ws, int row) {
  return ws.rec + (size_t)row * 3 * ws.nsc + 2 * ws.nsc;
}

// The slice of this workgroup: segments [k0, k1).
struct PzSlice {
  int k0, k1;
};
__device__ __forceinline__ PzSlice pz_sp_slice(int nseg, int spw) {
  PzSlice s;
  s.k0 = (int)blockIdx.x * spw;
  s.k1 = s.k0 + spw < nseg ? s.k0 + spw : nseg;
  return s;
}

// Ids [lo, hi) of a slice (for its penalty tables).
__device__ __forceinline__ int pz_sp_lo(const PzSlice& s) { return s.k0 * PZ_SP_SEG; }
__device__ __forceinline__ int pz_sp_hi(const PzSlice& s, int V) {
  const int h = s.k1 * PZ_SP_SEG;
  return h < V ? h : V;
}

// "Last workgroup" of a row (top-p's final sort): every thread's global
// writes, a workgroup barrier, then thread 0's agent-scope release increment
// of the row's counter (one L2 write-back per workgroup); the workgroup that
// brings it to S acquires (one invalidation, which serves the whole
// workgroup through the second barrier), continues, and re-zeroes the
// counter for the next launch.  No workgroup ever waits for another, so
// the pattern cannot deadlock whatever the residency.  (A fence in every
// thread instead would write back and invalidate the L2 once per wave.)
__device__ __forceinline__ bool pz_sp_arrive(uint32_t* arrive, int row, int S, int* flag_sh) {
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(&arrive[row], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = prev == (uint32_t)(S - 1);
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    *flag_sh = last;
  }
  __syncthreads();
  return *flag_sh != 0;
}

__device__ __forceinline__ void pz_sp_rearm(uint32_t* arrive, int row) {
  if (threadIdx.x == 0)
    __hip_atomic_store(&arrive[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct PzSpShared {
  float red[PZ_SP_WAVES];
  float M;
  uint32_t any;
  int flag;
  int cnt;
  float carry;
  int list[PZ_SP_NC];
};

// ---------------------------------------------------------------------------
// Stat pass over the slice.  Row: get(e0, y) gives y of ids e0..e0+3 after
// the row's chain (penalties, temperature) and their count below V.  With
// est, also the segments' maxima and relative masses.  Every thread calls
// it; S.any must be zero on entry.
// ---------------------------------------------------------------------------
template <class Row>
__device__ __forceinline__ void pz_sp_stat_slice(const Row& R, int row, const PzSlice& sl,
                                                 const PzSplitWs& ws, PzSpShared& S, bool est) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  float smax = -__builtin_inff();
  bool nan = false;
  float* seg_m = ws.seg_m + (size_t)row * ws.nsc;
  float* seg_s = ws.seg_s + (size_t)row * ws.nsc;
  // PZ_SP_U segments per wave per step: their loads are all in flight
  // before the first is used
  for (int kb = sl.k0 + w; kb < sl.k1; kb += PZ_SP_U * PZ_SP_WAVES) {
    float y[PZ_SP_U][4];
    int n[PZ_SP_U];
#pragma unroll
    for (int u = 0; u < PZ_SP_U; u++)
      n[u] = R.load((kb + u * PZ_SP_WAVES) * PZ_SP_SEG + 4 * lane, y[u]);
#pragma unroll
    for (int u = 0; u < PZ_SP_U; u++) {
      const int k = kb + u * PZ_SP_WAVES;
      if (k >= sl.k1) break;
      const int e0 = k * PZ_SP_SEG + 4 * lane;
      R.apply(e0, n[u], y[u]);
      float m = -__builtin_inff();
#pragma unroll
      for (int c = 0; c < 4; c++) {
        if (c >= n[u]) continue;
        if (y[u][c] != y[u][c]) nan = true;
        else m = fmaxf(m, y[u][c]);
      }
      m = pz_wave_max(m);
      if (est) {
        float t = 0.0f;
        if (m > -__builtin_inff() && m < __builtin_inff()) {
#pragma unroll
          for (int c = 0; c < 4; c++)  // NaN fails '>'
            if (c < n[u] && y[u][c] > -__builtin_inff()) t += pz_fast_exp(y[u][c] - m);
        }
        t = pz_wave_sum(t);
        if (lane == 0) {
          seg_m[k] = m;
          seg_s[k] = t;
        }
      }
      smax = fmaxf(smax, m);
    }
  }
  if (__ballot(nan) && lane == 0) atomicOr(&S.any, 1u);
  if (lane == 0) S.red[w] = smax;
  __syncthreads();
  if (tid == 0) {
    float mm = S.red[0];
    for (int i = 1; i < PZ_SP_WAVES; i++) mm = fmaxf(mm, S.red[i]);
    ws.slice_m[(size_t)row * ws.smax + blockIdx.x] = mm;
    ws.slice_f[(size_t)row * ws.smax + blockIdx.x] = S.any;
    if (blockIdx.x == 0) {
      float y[4];
      R.get(0, y);
      ws.rs[row].y0 = y[0];
    }
  }
}

// Row maximum and flags from the S slices the stat pass left (every thread
// calls it; results in S.M and S.any; a barrier inside).
__device__ __forceinline__ void pz_sp_row_stat(int row, int S_row, const PzSplitWs& ws,
                                               PzSpShared& S) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    float M = -__builtin_inff();
    uint32_t f = 0;
    for (int s = lane; s < S_row; s += 64) {
      M = fmaxf(M, ws.slice_m[(size_t)row * ws.smax + s]);
      f |= ws.slice_f[(size_t)row * ws.smax + s];
    }
    M = pz_wave_max(M);
    const bool anyf = __ballot(f != 0) != 0;
    if (lane == 0) {
      const float y0 = ws.rs[row].y0;
      uint32_t flags = anyf ? PZ_RS_NAN : 0u;
      if (y0 != y0) flags |= PZ_RS_Y0NAN;
      if (!(M > -__builtin_inff() && M < __builtin_inff())) flags |= PZ_RS_NONFIN;
      S.M = M;
      S.any = flags;
    }
  }
  __syncthreads();
}

// Estimated mass of segment k in units of exp(y - M): from the stat pass's
// (m_k, s_k), or (top-p) the estimate pass's absolute value.
struct PzEstRel {
  const float* m;
  const float* s;
  float M;
  __device__ __forceinline__ float operator()(int k) const {
    const float mk = m[k];
    return mk > -__builtin_inff() ? s[k] * pz_fast_exp(mk - M) : 0.0f;
  }
};
struct PzEstAbs {
  const float* s;
  __device__ __forceinline__ float operator()(int k) const { return s[k]; }
};

// Estimated running sum at the start of segment k0 (sum of the estimates of
// segments [0, k0), any rounding).  Every thread calls it; a barrier inside.
template <class Est>
__device__ __forceinline__ float pz_sp_prefix(const Est& est, int k0, PzSpShared& S) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  float t = 0.0f;
  for (int k = tid; k < k0; k += PZ_SP_BLOCK) t += est(k);
  t = pz_wave_sum(t);
  __syncthreads();
  if (lane == 0) S.red[w] = t;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < PZ_SP_WAVES; i++) tot += S.red[i];
  __syncthreads();
  return tot;
}

// Predicted grid and flags of the slice's segments, from the running-sum
// estimate at the slice start (carry) and the segments' estimates: each
// wave predicts the segments it will record (k = k0 + w + 16 j) after a scan
// over the slice.  Writes rec_gf.  Every thread calls it; barriers inside.
template <class Est>
__device__ __forceinline__ void pz_sp_predict(const Est& est, float carry, int row,
                                              const PzSlice& sl, const PzSplitWs& ws,
                                              PzSpShared& S) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  uint32_t* gf = pz_sp_rec_gf(ws, row);
  if (tid == 0) S.carry = carry;
  __syncthreads();
  for (int c0 = sl.k0; c0 < sl.k1; c0 += PZ_SP_BLOCK) {
    const int k = c0 + tid;
    const float e = k < sl.k1 ? est(k) : 0.0f;
    const float incl = pz_wave_scan_f32(e);
    if (lane == 63) S.red[w] = incl;
    __syncthreads();
    float off = S.carry;
    for (int i = 0; i < w; i++) off += S.red[i];
    const float start = off + (incl - e), end = off + incl;
    if (k < sl.k1)
      gf[k] = pz_predict_gf(start) | (pz_grid_of(end) != pz_grid_of(start) ? PZ_GF_XING : 0u);
    __syncthreads();
    if (tid == PZ_SP_BLOCK - 1) S.carry = end;
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Records pass over the slice's segments.  X provides (as for
// pz_record_pass): typename Raw; load(e0, Raw&) -> count < V;
// prep(e0, n, Raw&, a[4]); observe(e0, Raw&, a[4]);
// inc(Raw&, a[4], c, g, cls*).  The predicted grid and flags of segment k
// are in rec_gf (pz_sp_predict); PZ_NO_RECORD skips a segment.
// ---------------------------------------------------------------------------
template <class X>
__device__ __forceinline__ void pz_sp_records(X& x, int row, const PzSlice& sl,
                                              const PzSplitWs& ws) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t* rd = pz_sp_rec_d(ws, row);
  uint32_t* rd2 = pz_sp_rec_d2(ws, row);
  uint32_t* rgf = pz_sp_rec_gf(ws, row);
  for (int kb = sl.k0 + w; kb < sl.k1; kb += PZ_SP_U * PZ_SP_WAVES) {
  typename X::Raw raws[PZ_SP_U];
  int ns[PZ_SP_U];
#pragma unroll
  for (int u = 0; u < PZ_SP_U; u++)
    ns[u] = x.load((kb + u * PZ_SP_WAVES) * PZ_SP_SEG + 4 * lane, raws[u]);
#pragma unroll
  for (int u = 0; u < PZ_SP_U; u++) {
    const int k = kb + u * PZ_SP_WAVES;
    if (k >= sl.k1) break;
    const uint32_t gf = rgf[k];
    if (gf == PZ_NO_RECORD) continue;
    const int e0 = k * PZ_SP_SEG + 4 * lane;
    typename X::Raw& raw = raws[u];
    const int n = ns[u];
    float a[4];
    x.prep(e0, n, raw, a);
    x.observe(e0, raw, a);
    const uint32_t g = gf & 0xffu;
    const bool has2 = (gf & PZ_GF_HAS2) != 0;
    uint32_t s1 = 0, s2 = 0;
    bool d1 = false, d2 = false;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      uint32_t cls;
      s1 += x.inc(raw, a, c, g, &cls);
      d1 |= cls != PZ_INC_PLAIN;
    }
    if (has2) {
#pragma unroll
      for (int c = 0; c < 4; c++) {
        uint32_t cls;
        s2 += x.inc(raw, a, c, g - 1u, &cls);
        d2 |= cls != PZ_INC_PLAIN;
      }
      s2 = pz_wave_sum_u32(s2);
    }
    s1 = pz_wave_sum_u32(s1);
    const bool D1 = __ballot(d1) != 0;
    const bool D2 = has2 && __ballot(d2) != 0;
    if (lane == 0) {
      rd[k] = s1;
      rd2[k] = s2;
      rgf[k] = (gf & (0xffu | PZ_GF_HAS2 | PZ_GF_XING)) | (D1 ? PZ_GF_DIRTY : 0u) |
               (D2 ? PZ_GF_DIRTY2 : 0u);
    }
  }
  }
}

// ---------------------------------------------------------------------------
// The walk.
// ---------------------------------------------------------------------------
typedef uint32_t pz_u4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) pz_u4 pz_lds_u4;
typedef __attribute__((address_space(3))) uint8_t pz_lds_u8;

struct PzWalk {
  pz_lds_u32* d;      // [nseg] increments at the record's grid
  pz_lds_u32* d2;     // [nseg] increments at the grid below (HAS2)
  pz_lds_u32* gf;     // [nseg] grid and flags
  pz_lds_u32* pd;     // [nseg + 1] exclusive prefix of d (mod 2^32)
  pz_lds_i32* slot;   // [nseg] pre-evaluated slot, or -1
  pz_lds_f32* terms;  // [nc][256] exact terms
  pz_lds_u32* pa;     // [nc][256] inclusive increment prefix at the slot's grid g0
  pz_lds_u32* pb;     // [nc][256] the same at g0 + 1
  pz_lds_u8* fa;      // [nc][64] per lane: flagged (tie / big) terms at g0, one bit each
  pz_lds_u8* fb;      // [nc][64] the same at g0 + 1
  pz_lds_i32* g0;     // [nc]
  int nseg, nc;
};

// LDS of the walk for a row of nseg segments with nc pre-evaluated special
// segments: six words per segment plus the prefix's extra word; per special
// segment its terms, two increment prefixes, two flag masks and its grid.
__host__ __device__ inline size_t pz_sp_walk_lds(int nseg, int nc) {
  return (size_t)nseg * 24 + 32 + (size_t)nc * (3 * PZ_SP_SEG * 4 + 2 * 64 + 4);
}

// Special segments the walk can pre-evaluate within max_lds bytes (0 if the
// records alone do not fit).
inline int pz_sp_walk_nc(int nseg, size_t max_lds) {
  for (int nc = PZ_SP_NC; nc >= 1; nc--)
    if (pz_sp_walk_lds(nseg, nc) <= max_lds) return nc;
  return 0;
}

// The walk's state is wave-uniform; saying so lets the compiler keep it in
// scalar registers and branch on it with scalar instructions.
__device__ __forceinline__ void pz_sp_uni(PzAcc& st) {
  st.n = (uint32_t)__builtin_amdgcn_readfirstlane((int)st.n);
  st.g = (uint32_t)__builtin_amdgcn_readfirstlane((int)st.g);
}

__device__ __forceinline__ bool pz_sp_clean(uint32_t gf) {
  return gf != PZ_NO_RECORD && !(gf & (PZ_GF_DIRTY | PZ_GF_XING));
}

// Inclusive prefix pv of the increments at grid g of the 256 terms a wave
// holds (lane l: terms 4l..4l+3) and this lane's flag bits (tie / big).
// Flagged terms contribute their floor (tie) or 0 (big).
__device__ __forceinline__ void pz_sp_prefix4(const float (&v)[4], uint32_t g, uint32_t (&pv)[4],
                                              uint32_t& flags) {
  uint32_t inc[4], sum = 0;
  flags = 0;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    uint32_t cls;
    inc[c] = pz_inc(v[c], g, &cls);
    flags |= (cls != PZ_INC_PLAIN ? 1u : 0u) << c;
    sum += inc[c];
  }
  uint32_t run = pz_wave_scan_u32(sum) - sum;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    run += inc[c];
    pv[c] = run;
  }
}

// Element i of a lane-major 4-per-lane array (wave-uniform i).
__device__ __forceinline__ uint32_t pz_sp_elem(const uint32_t (&a)[4], int i) {
  const int c = i & 3;
  const uint32_t x = c == 0 ? a[0] : (c == 1 ? a[1] : (c == 2 ? a[2] : a[3]));
  return pz_readlane_u32(x, i >> 2);
}
__device__ __forceinline__ float pz_sp_elemf(const float (&a)[4], int i) {
  const int c = i & 3;
  const float x = c == 0 ? a[0] : (c == 1 ? a[1] : (c == 2 ? a[2] : a[3]));
  return pz_readlane_f32(x, i >> 2);
}

// Stages the row's records in LDS and pre-evaluates up to nc special
// segments (dirty, crossing, or without a record) in id order: exact terms
// (X::seg) and increment prefixes and flags at the record's grid and the
// next.  Every thread calls it.
template <class X>
__device__ __forceinline__ PzWalk pz_sp_walk_setup(const X& x, int row, int nseg, int nc,
                                                   const PzSplitWs& ws, char* lds,
                                                   PzSpShared& S) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  PzWalk W;
  W.nseg = nseg;
  W.nc = nc;
  char* p = lds;
  W.terms = (pz_lds_f32*)p;    p += (size_t)nc * PZ_SP_SEG * 4;
  W.pa = (pz_lds_u32*)p;       p += (size_t)nc * PZ_SP_SEG * 4;
  W.pb = (pz_lds_u32*)p;       p += (size_t)nc * PZ_SP_SEG * 4;
  W.fa = (pz_lds_u8*)p;        p += (size_t)nc * 64;
  W.fb = (pz_lds_u8*)p;        p += (size_t)nc * 64;
  W.g0 = (pz_lds_i32*)p;       p += (size_t)nc * 4;
  W.d = (pz_lds_u32*)p;        p += (size_t)nseg * 4;
  W.d2 = (pz_lds_u32*)p;       p += (size_t)nseg * 4;
  W.gf = (pz_lds_u32*)p;       p += (size_t)nseg * 4;
  W.pd = (pz_lds_u32*)p;       p += (size_t)(nseg + 1) * 4;
  W.slot = (pz_lds_i32*)p;
  const uint32_t* rd = pz_sp_rec_d(ws, row);
  const uint32_t* rd2 = pz_sp_rec_d2(ws, row);
  const uint32_t* rgf = pz_sp_rec_gf(ws, row);
  // records, their prefix, and the special segments in id order
  uint32_t base = 0;  // prefix carried over the chunks (thread-uniform)
  int sbase = 0;      // specials found in earlier chunks
  for (int c0 = 0; c0 < nseg; c0 += PZ_SP_BLOCK) {
    const int k = c0 + tid;
    uint32_t d = 0, gf = PZ_NO_RECORD;
    if (k < nseg) {
      d = rd[k];
      gf = rgf[k];
      W.d[k] = d;
      W.d2[k] = rd2[k];
      W.gf[k] = gf;
    }
    const bool special = k < nseg && !pz_sp_clean(gf);
    // exclusive prefix of d and rank of the special segments (workgroup scans)
    const uint32_t incl = pz_wave_scan_u32(d);
    const uint64_t sb = __ballot(special);
    __syncthreads();
    if (lane == 63) S.list[w] = (int)incl;  // wave totals (list[] is free until the end)
    if (lane == 0) S.red[w] = __int_as_float(__popcll(sb));
    __syncthreads();
    uint32_t off = base;
    int soff = sbase;
    for (int i = 0; i < w; i++) {
      off += (uint32_t)S.list[i];
      soff += __float_as_int(S.red[i]);
    }
    uint32_t tot = 0;
    int stot = 0;
    for (int i = 0; i < PZ_SP_WAVES; i++) {
      tot += (uint32_t)S.list[i];
      stot += __float_as_int(S.red[i]);
    }
    if (k < nseg) {
      W.pd[k] = off + incl - d;
      const int rank = soff + __popcll(sb & ((1ull << lane) - 1ull));
      W.slot[k] = special && rank < nc ? rank : -1;
    }
    base += tot;
    sbase += stot;
    __syncthreads();
  }
  if (tid == 0) W.pd[nseg] = base;
  __syncthreads();
  // the list of pre-evaluated segments
  for (int k = tid; k < nseg; k += PZ_SP_BLOCK) {
    const int s = W.slot[k];
    if (s >= 0) S.list[s] = k;
  }
  if (tid == 0) S.cnt = sbase < nc ? sbase : nc;
  __syncthreads();
  const int n_pre = S.cnt;
  for (int j = w; j < n_pre; j += PZ_SP_WAVES) {
    const int k = S.list[j];
    float v[4];
    x.seg(k, v);
    pz_f4 q;
    q.x = v[0];
    q.y = v[1];
    q.z = v[2];
    q.w = v[3];
    ((pz_lds_f4*)(W.terms + j * PZ_SP_SEG))[lane] = q;
    const uint32_t gf = W.gf[k];
    const uint32_t g = gf == PZ_NO_RECORD ? 1u : (gf & 0xffu);
    uint32_t pa[4], pb[4], fa, fb;
    pz_sp_prefix4(v, g, pa, fa);
    pz_sp_prefix4(v, g + 1u, pb, fb);
    pz_u4 a4, b4;
    a4.x = pa[0]; a4.y = pa[1]; a4.z = pa[2]; a4.w = pa[3];
    b4.x = pb[0]; b4.y = pb[1]; b4.z = pb[2]; b4.w = pb[3];
    ((pz_lds_u4*)(W.pa + j * PZ_SP_SEG))[lane] = a4;
    ((pz_lds_u4*)(W.pb + j * PZ_SP_SEG))[lane] = b4;
    W.fa[j * 64 + lane] = (uint8_t)fa;
    W.fb[j * 64 + lane] = (uint8_t)fb;
    if (lane == 0) W.g0[j] = (int)g;
  }
  __syncthreads();
  return W;
}

// Sequential fp32 accumulation of the segment's terms from position start,
// one real add each, by the whole wave in lockstep (terms read from their
// lanes): for stretches where nearly every term is an event, e.g. the start
// of a row.  Returns the first hit index or -1.
template <int MODE>
__device__ __forceinline__ int pz_sp_serial(PzAcc& st, const float (&v)[4], int start, float thr) {
  float s = pz_acc_value(st);
  int i = start;
  for (; i < PZ_SP_SEG && (i & 15); i++) {
    const float sn = s + pz_sp_elemf(v, i);
    if (MODE != PZ_STOP_NONE && pz_stop_hit(sn, thr, MODE)) {
      st = pz_acc_of(sn);
      return i;
    }
    s = sn;
  }
  // 16 terms per step: the reads of four lanes' terms are independent of
  // the chain of adds and issue ahead of it
  for (int l = i >> 2; l < 64; l += 4) {
    float x[16];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      x[4 * j + 0] = pz_readlane_f32(v[0], l + j);
      x[4 * j + 1] = pz_readlane_f32(v[1], l + j);
      x[4 * j + 2] = pz_readlane_f32(v[2], l + j);
      x[4 * j + 3] = pz_readlane_f32(v[3], l + j);
    }
    if (MODE == PZ_STOP_NONE) {
#pragma unroll
      for (int j = 0; j < 16; j++) s = s + x[j];
    } else {
#pragma unroll
      for (int j = 0; j < 16; j++) {
        const float sn = s + x[j];
        if (pz_stop_hit(sn, thr, MODE)) {
          st = pz_acc_of(sn);
          return 4 * l + j;
        }
        s = sn;
      }
    }
  }
  st = pz_acc_of(s);
  return -1;
}

// One segment element by element from the state st: each event (a term that
// leaves the binade, a tie, a term as large as the sum, a stop hit) is found
// with one ballot over the increment prefix at the state's grid -- P at g0,
// Q at g0 + 1, recomputed from the terms at any other grid -- and taken with
// one exact add (pz_acc_add).  Dense events go to the serial loop.  Returns
// the first hit index or -1.
template <int MODE>
__device__ __forceinline__ int pz_sp_events(PzAcc& st, const float (&v)[4], uint32_t g0,
                                            uint32_t (&P)[4], uint32_t fP, uint32_t (&Q)[4],
                                            uint32_t fQ, float thr) {
  const int lane = threadIdx.x & 63;
  int pos = 0;
  pz_sp_uni(st);
  g0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)g0);
  for (int nev = 0; pos < PZ_SP_SEG; nev++) {
    if (nev >= 8 || (st.n == 0u && st.g == 1u)) return pz_sp_serial<MODE>(st, v, pos, thr);
    if (st.g != g0 && st.g != g0 + 1u) {
      g0 = st.g;
      pz_sp_prefix4(v, g0, P, fP);
      pz_sp_prefix4(v, g0 + 1u, Q, fQ);
    }
    const bool hi = st.g != g0;
    uint32_t a[4];
#pragma unroll
    for (int c = 0; c < 4; c++) a[c] = hi ? Q[c] : P[c];
    const uint32_t fl4 = hi ? fQ : fP;
    const uint32_t base = pos > 0 ? pz_sp_elem(a, pos - 1) : 0u;
    if (pos > 0) {
      // after an event: the rest of the segment in one step when it holds no
      // flagged term, stays in the binade and (sums only grow) ends below
      // the stop
      const uint64_t fb =
          __ballot(fl4 != 0u && 4 * lane + 31 - (int)__builtin_clz(fl4) >= pos);
      const uint32_t rest = pz_sp_elem(a, PZ_SP_SEG - 1) - base;
      if (!fb && rest < (1u << 24) - st.n &&
          !(MODE != PZ_STOP_NONE &&
            pz_stop_hit(pz_acc_value_ng(st.n + rest, st.g), thr, MODE))) {
        st.n += rest;
        return -1;
      }
    }
    const uint32_t room = (1u << 24) - st.n;  // a prefix >= room leaves the binade
    int ev = 4, kind = 0;
#pragma unroll
    for (int c = 3; c >= 0; c--) {
      const int i = 4 * lane + c;
      const bool live = i >= pos;
      const bool fl = live && ((fl4 >> c) & 1u);
      const uint32_t dd = a[c] - base;
      const bool cross = live && !fl && dd >= room;
      const bool hit = MODE != PZ_STOP_NONE && live && !fl && !cross &&
                       pz_stop_hit(pz_acc_value_ng(st.n + dd, st.g), thr, MODE);
      if (fl || cross || hit) {
        ev = c;
        kind = hit ? 2 : (cross ? 1 : 3);
      }
    }
    const uint64_t ball = __ballot(ev < 4);
    if (!ball) {
      st.n += pz_sp_elem(a, PZ_SP_SEG - 1) - base;
      return -1;
    }
    const int L = (int)__builtin_ctzll(ball);
    const int i = 4 * L + __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(ev, L));
    const int kd = __builtin_amdgcn_readfirstlane(__builtin_amdgcn_readlane(kind, L));
    if (kd == 2) {
      st.n += pz_sp_elem(a, i) - base;
      return i;
    }
    if (i > pos) st.n += pz_sp_elem(a, i - 1) - base;
    const float t = pz_sp_elemf(v, i);
    // a plain term that leaves the binade: one real add; a tie or a term as
    // large as the sum: the exact step
    st = kd == 1 ? pz_acc_of(pz_acc_value(st) + t) : pz_acc_add(st, t);
    pz_sp_uni(st);
    if (MODE != PZ_STOP_NONE && pz_stop_hit(pz_acc_value(st), thr, MODE)) return i;
    pos = i + 1;
  }
  return -1;
}

// The walk (one wave): the exact sequential sum of the row's terms in id
// order, from state 0.  With a stop mode returns the element index of the
// first hit (st = the sum including it), else -1 (st = the whole sum).  X
// provides seg(k, v[4]) for segments evaluated during the walk.
template <int MODE, class X>
__device__ __forceinline__ int pz_sp_walk(PzAcc& st, const PzWalk& W, float thr, const X& x) {
  const int lane = threadIdx.x & 63;
  st.n = 0;
  st.g = 1;
  int k = 0;
  const int nseg = W.nseg;
  while (k < nseg) {
    // runs of clean records at the state's grid: 64 segments per step
    {
      const int kk = k + lane;
      bool bad = true;
      if (kk < nseg) {
        const uint32_t gf = W.gf[kk];
        const uint32_t upto = W.pd[kk + 1] - W.pd[k];  // d of [k, kk]
        bad = !pz_sp_clean(gf) || (gf & 0xffu) != st.g || upto >= (1u << 24) - st.n ||
              (MODE != PZ_STOP_NONE &&
               pz_stop_hit(pz_acc_value_ng(st.n + upto, st.g), thr, MODE));
      }
      const uint64_t ball = __ballot(bad);
      const int L = ball ? (int)__builtin_ctzll(ball) : 64;
      const int kb = k + L;
      st.n += W.pd[kb < nseg ? kb : nseg] - W.pd[k];
      pz_sp_uni(st);
      if (kb >= nseg) break;
      k = kb;
      if (L == 64) continue;
    }
    // segment k cannot be taken from its primary record
    const uint32_t gf = W.gf[k];
    if (gf != PZ_NO_RECORD && (gf & PZ_GF_HAS2) && !(gf & (PZ_GF_DIRTY2 | PZ_GF_XING)) &&
        (gf & 0xffu) - 1u == st.g) {
      const uint32_t d2 = W.d2[k];
      if (d2 < (1u << 24) - st.n &&
          !(MODE != PZ_STOP_NONE && pz_stop_hit(pz_acc_value_ng(st.n + d2, st.g), thr, MODE))) {
        st.n += d2;
        pz_sp_uni(st);
        k++;
        continue;
      }
    }
    const int s = W.slot[k];
    float v[4];
    uint32_t P[4], Q[4], fP, fQ, g0;
    if (s >= 0) {
      // everything the segment needs, in one round of LDS reads
      const pz_f4 q = ((const pz_lds_f4*)(W.terms + s * PZ_SP_SEG))[lane];
      const pz_u4 a4 = ((const pz_lds_u4*)(W.pa + s * PZ_SP_SEG))[lane];
      const pz_u4 b4 = ((const pz_lds_u4*)(W.pb + s * PZ_SP_SEG))[lane];
      fP = W.fa[s * 64 + lane];
      fQ = W.fb[s * 64 + lane];
      g0 = (uint32_t)W.g0[s];
      v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
      P[0] = a4.x; P[1] = a4.y; P[2] = a4.z; P[3] = a4.w;
      Q[0] = b4.x; Q[1] = b4.y; Q[2] = b4.z; Q[3] = b4.w;
    } else {
      x.seg(k, v);
      g0 = st.g;
      pz_sp_prefix4(v, g0, P, fP);
      pz_sp_prefix4(v, g0 + 1u, Q, fQ);
    }
    const int r = pz_sp_events<MODE>(st, v, g0, P, fP, Q, fQ, thr);
    if (r >= 0) return k * PZ_SP_SEG + r;
    k++;
  }
  return -1;
}

#endif
