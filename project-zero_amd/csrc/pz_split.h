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

// Slice kernels run PZ_SP_TARGET_WG workgroups of PZ_SP_BLOCK threads: two
// per CU only if a wave keeps to 64 VGPRs (8 waves per SIMD); past that the
// launch runs in two rounds.
#define PZ_SP_TWO_PER_CU __attribute__((amdgpu_waves_per_eu(8)))

// Row flags (from the slices' maxima and NaN flags).
enum {
  PZ_RS_NAN = 1,      // some y is NaN
  PZ_RS_Y0NAN = 2,    // y[0] is NaN
  PZ_RS_NONFIN = 4,   // the NaN-free maximum is +-inf (or there is no value at all)
  PZ_RS_FAILED = 8,   // a wait between the row's workgroups gave up
};

// Per-row values handed from pass to pass (device scratch, 64 bytes).
struct PzRowState {
  float M;          // maximum of the NaN-free y (-inf if none)
  float y0;         // y[0]
  uint32_t flags;   // PZ_RS_*
  float sum;        // exact sequential normaliser
  float inv;        // 1.0f / sum
  uint32_t s0;      // sequential sum of segment 0's terms from 0 (bits), where a pass
                    // posts it for the walk (0xffffffff: not posted)
  float f[3];       // pass-specific values
  int32_t i[8];     // pass-specific values
};

struct PzSplitWs {
  PzRowState* rs;     // [rows]
  uint32_t* arrive;   // [rows] arrival counters, zero between launches
  uint64_t* meet;     // [rows][2][smax] values the workgroups of a row hand each
                      // other within a launch (bit 63: written), zero between
                      // launches
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

// Segments of a row slice the top-p front launch keeps in LDS (64 KiB).
constexpr int PZ_SP_FRONT_SEGS = 64;

// Bytes of a workspace for `rows` rows of up to V ids (top-p buffers when
// capg > 0); with base != nullptr also carves it.  front_hist: histogram
// slots for the top-p front launch at any batch (every row's slices at
// once), else for one round of workgroups.
inline size_t pz_split_ws_layout(int rows, int V, int capg, void* base, PzSplitWs* out,
                                 bool front_hist = false) {
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  const int nsc = pz_sp_nseg(V);
  const int smax = (nsc + PZ_SP_WAVES - 1) / PZ_SP_WAVES;
  const int sfront = (nsc + PZ_SP_FRONT_SEGS - 1) / PZ_SP_FRONT_SEGS;
  const int hslots =
      capg > 0 ? PZ_SP_TARGET_WG + rows * (front_hist && sfront > 1 ? sfront : 1) : 0;
  const size_t R = (size_t)rows;
  size_t off = 0;
  const size_t o_rs = off;   off = up(off + R * sizeof(PzRowState));
  const size_t o_arr = off;  off = up(off + R * 4);
  const size_t o_meet = off; off = up(off + R * 2 * smax * 8);
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
    out->meet = reinterpret_cast<uint64_t*>(b + o_meet);
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
__device__ __forceinline__ PzSlice pz_sp_slice_at(int idx, int nseg, int spw) {
  PzSlice s;
  s.k0 = idx * spw;
  s.k1 = s.k0 + spw < nseg ? s.k0 + spw : nseg;
  return s;
}
__device__ __forceinline__ PzSlice pz_sp_slice(int nseg, int spw) {
  return pz_sp_slice_at((int)blockIdx.x, nseg, spw);
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

// Polls a word published by another workgroup of the launch with an
// agent-scope relaxed atomic load (coherent across the XCDs' L2s) until it
// is nonzero, at most PZ_POLL_CAP times; returns 0 if it never was.
#ifndef PZ_POLL_CAP
#define PZ_POLL_CAP (1u << 22)
#endif
__device__ __forceinline__ uint64_t pz_poll_u64(const uint64_t* w, uint32_t cap = PZ_POLL_CAP) {
  uint64_t v = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (uint32_t n = 1; v == 0ull && n < cap; n++) {
    __builtin_amdgcn_s_sleep(1);
    v = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return v;
}

// "Last workgroup merges" for one nonzero 64-bit word per workgroup, with no
// L2 write-back or invalidation (an agent-scope release/acquire pair costs
// one of each per workgroup, which stalls every other workgroup's stream on
// that XCD's L2).  Thread 0 of each of the row's S workgroups stores its
// word w[sl] with an agent-scope relaxed atomic store, then counts itself in
// at arrive[row]; the call returns true in thread 0 of the workgroup whose
// increment brings the counter to S (false everywhere else).  That
// workgroup then reads the words with pz_poll_u64: every other workgroup
// issued its store before its increment, so each poll ends as soon as that
// store lands -- the waiting workgroup is the last one, so no wait depends
// on a workgroup that has not run.  The merging wave clears the words and
// the counter (zero between launches).
__device__ __forceinline__ bool pz_sp_post_last(uint64_t* w, int sl, uint64_t word,
                                                uint32_t* arrive, int row, int S) {
  __hip_atomic_store(&w[sl], word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t prev =
      __hip_atomic_fetch_add(&arrive[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return prev == (uint32_t)(S - 1);
}

__device__ __forceinline__ void pz_sp_rearm(uint32_t* arrive, int row) {
  if (threadIdx.x == 0)
    __hip_atomic_store(&arrive[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct PzSpShared {
  float red[PZ_SP_WAVES];
  uint32_t red2[PZ_SP_WAVES];
  float M;
  uint32_t any;
  int flag;
  int cnt;
  int tail_end;
  float carry;
  uint32_t s0;  // a first-segment sum handed to the walk's set-up (bits)
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
      if (n[u] < 4) {  // (only at the row's end: nothing past it counts)
#pragma unroll
        for (int c = 0; c < 4; c++)
          if (c >= n[u]) y[u][c] = -__builtin_inff();
      }
      // (fmaxf passes over a NaN)
      float m = -__builtin_inff();
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float v = y[u][c];
        nan |= v != v;
        m = fmaxf(m, v);
      }
      m = pz_wave_max(m);
      if (est) {
        // exp2(-inf) = 0 past the end; a NaN makes the row's flags say so,
        // and the callers that ask for estimates skip such rows
        float t = 0.0f;
        if (m > -__builtin_inff() && m < __builtin_inff()) {
#pragma unroll
          for (int c = 0; c < 4; c++) t += pz_fast_exp(y[u][c] - m);
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
  // (LDS only: the segments' stores stay in flight; one wave reduces the
  // waves' maxima, one LDS load per lane)
  pz_lds_barrier();
  const float mm = w == 0 ? pz_wave_max(lane < PZ_SP_WAVES ? S.red[lane] : -__builtin_inff())
                          : 0.0f;
  if (tid == 0) {
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
  const float tot = pz_wave_sum(lane < PZ_SP_WAVES ? S.red[lane] : 0.0f);
  __syncthreads();
  return tot;
}

// Predicted grid and flags of the slice's segments, from the running-sum
// estimate at the slice start (carry) and the segments' estimates: each
// wave predicts the segments it will record (k = k0 + w + 16 j) after a scan
// over the slice.  Writes rec_gf, and with lgf also lgf[k - k0] (a slice of
// at most PZ_SP_BLOCK segments), which pz_sp_records then reads instead:
// the barriers inside order LDS only.  Every thread calls it.
template <class Est>
__device__ __forceinline__ void pz_sp_predict(const Est& est, float carry, int row,
                                              const PzSlice& sl, const PzSplitWs& ws,
                                              PzSpShared& S, pz_lds_u32* lgf = nullptr) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  uint32_t* gf = pz_sp_rec_gf(ws, row);
  auto barrier = [&] {
    if (lgf) pz_lds_barrier();
    else __syncthreads();
  };
  if (sl.k1 - sl.k0 <= 64) {
    // one segment per lane of wave 0 (the same scan and sums as below with
    // a single wave), one barrier
    if (w == 0) {
      const int k = sl.k0 + lane;
      const float e = k < sl.k1 ? est(k) : 0.0f;
      const float incl = pz_wave_scan_f32(e);
      const float start = (carry + 0.0f) + (incl - e), end = (carry + 0.0f) + incl;
      if (k < sl.k1) {
        const uint32_t v =
            pz_predict_gf(start) | (pz_grid_of(end) != pz_grid_of(start) ? PZ_GF_XING : 0u);
        gf[k] = v;
        if (lgf) lgf[k - sl.k0] = v;
      }
      if (lane == 63) S.carry = end;
    }
    barrier();
    return;
  }
  if (tid == 0) S.carry = carry;
  barrier();
  for (int c0 = sl.k0; c0 < sl.k1; c0 += PZ_SP_BLOCK) {
    const int k = c0 + tid;
    const float e = k < sl.k1 ? est(k) : 0.0f;
    const float incl = pz_wave_scan_f32(e);
    if (lane == 63) S.red[w] = incl;
    barrier();
    // (the waves before this one: a wave reduction, one LDS load per lane)
    const float off = S.carry + pz_wave_sum(lane < w ? S.red[lane] : 0.0f);
    const float start = off + (incl - e), end = off + incl;
    if (k < sl.k1) {
      const uint32_t v =
          pz_predict_gf(start) | (pz_grid_of(end) != pz_grid_of(start) ? PZ_GF_XING : 0u);
      gf[k] = v;
      if (lgf) lgf[k - sl.k0] = v;
    }
    barrier();
    if (tid == PZ_SP_BLOCK - 1) S.carry = end;
    barrier();
  }
}

// ---------------------------------------------------------------------------
// Records pass over the slice's segments.  X provides (as for
// pz_record_pass): typename Raw; load(e0, Raw&) -> count < V;
// prep(e0, n, Raw&, a[4]); observe(e0, Raw&, a[4]);
// inc4(Raw&, a[4], g, s&, dirty&).  The predicted grid and flags of segment k
// are in rec_gf, or lgf[k - k0] (pz_sp_predict); PZ_NO_RECORD skips a segment.
// skip_xing: segments predicted to cross a binade are skipped too (their
// grid word, written by the prediction, already makes them specials, whose
// increments the walk never reads) -- only for terms whose observer does
// nothing.
// ---------------------------------------------------------------------------
template <class X>
__device__ __forceinline__ void pz_sp_records(X& x, int row, const PzSlice& sl,
                                              const PzSplitWs& ws,
                                              const pz_lds_u32* lgf = nullptr,
                                              bool skip_xing = false) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  uint32_t* rd = pz_sp_rec_d(ws, row);
  uint32_t* rd2 = pz_sp_rec_d2(ws, row);
  uint32_t* rgf = pz_sp_rec_gf(ws, row);
  for (int kb = sl.k0 + w; kb < sl.k1; kb += PZ_SP_U * PZ_SP_WAVES) {
  typename X::Raw raws[PZ_SP_U];
  int ns[PZ_SP_U];
  uint32_t gfs[PZ_SP_U];  // every grid word in flight before the first is used
#pragma unroll
  for (int u = 0; u < PZ_SP_U; u++) {
    const int k = kb + u * PZ_SP_WAVES;
    ns[u] = x.load(k * PZ_SP_SEG + 4 * lane, raws[u]);
    gfs[u] = k < sl.k1 ? (lgf ? lgf[k - sl.k0] : rgf[k]) : PZ_NO_RECORD;
  }
#pragma unroll
  for (int u = 0; u < PZ_SP_U; u++) {
    const int k = kb + u * PZ_SP_WAVES;
    if (k >= sl.k1) break;
    const uint32_t gf = gfs[u];
    if (gf == PZ_NO_RECORD || (skip_xing && (gf & PZ_GF_XING))) continue;
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
    x.inc4(raw, a, g, s1, d1);
    if (has2) {
      x.inc4(raw, a, g - 1u, s2, d2);
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
// Front pass: stat and records of a slice in one launch, the slice read once
// (HBM) into LDS with the row's chain applied.  The row's S workgroups meet
// twice through the row's meeting words (ws.meet, zero between launches):
// for the row maximum (meet 1: slice maximum, NaN and y[0] flags) and for
// the estimated mass of the slices before each one (meet 2).  Each workgroup
// posts a word (value and a written bit; no fence) and wave 0 polls the S
// words with agent-scope atomic loads, at most `cap` times.  A row's
// workgroups are consecutive in the launch order and each posts everything
// it owes before it waits, so with the row's S <= 64 workgroups resident
// together the waits end; one that gives up posts what it still owes and
// marks the row failed (rs.i[7], cleared by the walk launch).  Writes what
// the stat pass writes (slice maxima and flags, y[0]; the segments' maxima,
// and their masses as absolute estimates in units of exp(y - M)) and the
// records of the terms exp(y - M), y >= M + thr_rel, at the predicted grids.
// Returns whether the row is settled here (degenerate or failed).
// ---------------------------------------------------------------------------
struct PzLdsRow {
  const pz_lds_f32* y;
  int lo, V;
  __device__ __forceinline__ int load(int e0, float (&r)[4]) const {
    int n = V - e0;
    n = n < 0 ? 0 : (n > 4 ? 4 : n);
    const pz_f4 q = *(const pz_lds_f4*)(y + (e0 - lo));
    r[0] = q.x;
    r[1] = q.y;
    r[2] = q.z;
    r[3] = q.w;
    return n;
  }
  __device__ __forceinline__ void apply(int, int, float (&)[4]) const {}
  __device__ __forceinline__ int get(int e0, float (&r)[4]) const { return load(e0, r); }
};

struct PzSliceEst {
  const float* s;
  int k0;
  __device__ __forceinline__ float operator()(int k) const { return s[k - k0]; }
};

constexpr int PZ_FRONT_SEGS = 64;  // segments of a slice held in LDS

struct PzFrontShared {
  float sest[PZ_FRONT_SEGS];
  uint32_t sgf[PZ_FRONT_SEGS];
  int fail;
};

__device__ __forceinline__ void pz_sp_mark_failed(const PzSplitWs& ws, int row) {
  __hip_atomic_store(&ws.rs[row].i[7], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls the first n words of w (lane i: w[i]) until every one has its
// written bit, at most cap times (wave 0).  Returns false if it gave up.
__device__ __forceinline__ bool pz_sp_meet(const uint64_t* w, int n, uint32_t cap, uint64_t& v) {
  const int lane = threadIdx.x & 63;
  v = 1ull << 63;
  for (uint32_t t = 1;; t++) {
    if (lane < n) v = __hip_atomic_load(&w[lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__ballot((v >> 63) == 0) == 0) return true;
    if (t >= cap) return false;
    __builtin_amdgcn_s_sleep(1);
  }
}

template <class Row>
__device__ __forceinline__ bool pz_sp_front(const Row& R, int row, const PzSlice& sl, int S,
                                            float thr_rel, const PzSplitWs& ws,
                                            PzSpShared& SS, PzFrontShared& F, pz_lds_f32* ybuf,
                                            const pz_lds_u64* et, uint32_t cap) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lo = pz_sp_lo(sl);
  const int V = R.V;
  uint64_t* meet = ws.meet + (size_t)row * 2 * ws.smax;
  float* seg_m = ws.seg_m + (size_t)row * ws.nsc;
  float* seg_s = ws.seg_s + (size_t)row * ws.nsc;
  // 1. the slice, once: chain applied, into LDS; segment and slice maxima
  float smx = -__builtin_inff();
  bool nan = false;
  for (int kb = sl.k0 + w; kb < sl.k1; kb += PZ_SP_U * PZ_SP_WAVES) {
    float y[PZ_SP_U][4];
    int n[PZ_SP_U];
#pragma unroll
    for (int uu = 0; uu < PZ_SP_U; uu++)
      n[uu] = R.load((kb + uu * PZ_SP_WAVES) * PZ_SP_SEG + 4 * lane, y[uu]);
#pragma unroll
    for (int uu = 0; uu < PZ_SP_U; uu++) {
      const int k = kb + uu * PZ_SP_WAVES;
      if (k >= sl.k1) break;
      const int e0 = k * PZ_SP_SEG + 4 * lane;
      R.apply(e0, n[uu], y[uu]);
      if (n[uu] < 4) {  // (only at the row's end: -inf past it)
#pragma unroll
        for (int c = 0; c < 4; c++)
          if (c >= n[uu]) y[uu][c] = -__builtin_inff();
      }
      // (fmaxf passes over a NaN)
      float m = -__builtin_inff();
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float v = y[uu][c];
        nan |= v != v;
        m = fmaxf(m, v);
      }
      pz_f4 q;
      q.x = y[uu][0];
      q.y = y[uu][1];
      q.z = y[uu][2];
      q.w = y[uu][3];
      *(pz_lds_f4*)(ybuf + (e0 - lo)) = q;
      m = pz_wave_max(m);
      if (lane == 0) seg_m[k] = m;
      smx = fmaxf(smx, m);
    }
  }
  if (__ballot(nan) && lane == 0) atomicOr(&SS.any, 1u);
  if (lane == 0) SS.red[w] = smx;
  pz_lds_barrier();
  const float mm = w == 0 ? pz_wave_max(lane < PZ_SP_WAVES ? SS.red[lane] : -__builtin_inff())
                          : 0.0f;
  if (tid == 0) {
    uint32_t f = SS.any;
    ws.slice_m[(size_t)row * ws.smax + blockIdx.x] = mm;
    ws.slice_f[(size_t)row * ws.smax + blockIdx.x] = f;
    if (blockIdx.x == 0) {
      ws.rs[row].y0 = ybuf[0];
      if (ybuf[0] != ybuf[0]) f |= PZ_RS_Y0NAN;
    }
    // meet 1: every slice's maximum and flags
    __hip_atomic_store(&meet[blockIdx.x],
                       (1ull << 63) | ((uint64_t)f << 32) | (uint64_t)__float_as_uint(mm),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (w == 0) {
    uint64_t v;
    if (!pz_sp_meet(meet, S, cap, v) && lane == 0) F.fail = 1;
    const float M = pz_wave_max(lane < S ? __uint_as_float((uint32_t)v) : -__builtin_inff());
    const bool anyf = __ballot(lane < S && (((uint32_t)(v >> 32) & PZ_RS_NAN) != 0)) != 0;
    const bool y0nan = __ballot(lane < S && (((uint32_t)(v >> 32) & PZ_RS_Y0NAN) != 0)) != 0;
    if (lane == 0) {
      uint32_t flags = anyf ? PZ_RS_NAN : 0u;
      if (y0nan) flags |= PZ_RS_Y0NAN;
      if (!(M > -__builtin_inff() && M < __builtin_inff())) flags |= PZ_RS_NONFIN;
      SS.M = M;
      SS.any = flags;
    }
  }
  pz_lds_barrier();
  const bool degen = (SS.any & (PZ_RS_NAN | PZ_RS_Y0NAN | PZ_RS_NONFIN)) != 0;
  if (F.fail || degen) {
    // what the others may wait for: no mass; the failure mark
    if (tid == 0) {
      __hip_atomic_store(&meet[ws.smax + blockIdx.x], 1ull << 63, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      if (F.fail) pz_sp_mark_failed(ws, row);
    }
    return true;
  }
  const float M = SS.M, thr = M + thr_rel;
  // 2. the estimated mass of each segment's terms
  // (the slice in LDS holds -inf past the row's end, whose terms are 0, and
  // no NaN: such a row has left at meeting 1)
  for (int k = sl.k0 + w; k < sl.k1; k += PZ_SP_WAVES) {
    const int e0 = k * PZ_SP_SEG + 4 * lane;
    const pz_f4 q = *(const pz_lds_f4*)(ybuf + (e0 - lo));
    const float y[4] = {q.x, q.y, q.z, q.w};
    float t = 0.0f;
    if (thr == -__builtin_inff()) {
#pragma unroll
      for (int c = 0; c < 4; c++) t += pz_fast_exp(y[c] - M);
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++)
        if (y[c] >= thr) t += pz_fast_exp(y[c] - M);
    }
    t = pz_wave_sum(t);
    if (lane == 0) {
      F.sest[k - sl.k0] = t;
      seg_s[k] = t;
    }
  }
  pz_lds_barrier();
  static_assert(PZ_FRONT_SEGS <= 64, "one estimate per lane");
  const float tot = w == 0 ? pz_wave_sum(lane < sl.k1 - sl.k0 ? F.sest[lane] : 0.0f) : 0.0f;
  if (tid == 0)  // meet 2: every slice's estimated mass
    __hip_atomic_store(&meet[ws.smax + blockIdx.x], (1ull << 63) | (uint64_t)__float_as_uint(tot),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (w == 0) {
    uint64_t v;
    if (!pz_sp_meet(meet + ws.smax, (int)blockIdx.x, cap, v) && lane == 0) F.fail = 1;
    const float carry = pz_wave_sum(lane < (int)blockIdx.x ? __uint_as_float((uint32_t)v) : 0.0f);
    if (lane == 0) SS.carry = carry;
  }
  pz_lds_barrier();
  if (F.fail) {
    if (tid == 0) pz_sp_mark_failed(ws, row);
    return true;
  }
  pz_sp_predict(PzSliceEst{F.sest, sl.k0}, SS.carry, row, sl, ws, SS, (pz_lds_u32*)F.sgf);
  // 3. records from LDS
  PzExpTerms<PzLdsRow> X;
  X.R.y = ybuf;
  X.R.lo = lo;
  X.R.V = V;
  X.M = M;
  X.thr = thr;
  X.inv = 1.0f;
  X.as_p = false;
  X.et = et;
  pz_sp_records(X, row, sl, ws, (const pz_lds_u32*)F.sgf, true);
  return false;
}

// Clears the row's meeting words (every thread of the walk's workgroup;
// plain stores, which the launch boundary makes visible to the next launch).
__device__ __forceinline__ void pz_sp_clear_meet(const PzSplitWs& ws, int row) {
  for (int i = threadIdx.x; i < 2 * ws.smax; i += blockDim.x)
    ws.meet[(size_t)row * 2 * ws.smax + i] = 0ull;
}

// Front-pass plan: the split plan's slices capped at PZ_FRONT_SEGS segments.
inline PzSplitPlan pz_front_plan(int V, int nrows, int smax) {
  PzSplitPlan p = pz_split_plan(V, nrows, smax);
  if (p.spw > PZ_FRONT_SEGS) {
    p.spw = PZ_FRONT_SEGS;
    p.S = (p.nseg + p.spw - 1) / p.spw;
  }
  return p;
}

// ---------------------------------------------------------------------------
// The walk.
// ---------------------------------------------------------------------------
typedef uint32_t pz_u4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) pz_u4 pz_lds_u4;
typedef __attribute__((address_space(3))) uint8_t pz_lds_u8;
typedef __attribute__((address_space(3))) uint16_t pz_lds_u16h;

// One slot of the walk's ring, every part at a fixed offset from the slot's
// base, so that a slot is read through one address: the exact terms, the
// inclusive increment prefix at the slot's grid g0 and at g1 (the grid the
// segment is expected to end in), per lane the flag bits at g0 (low byte)
// and g1 (high byte), then four scalars (g0; g1 | first tie at g0 << 8 |
// (last flagged at g1 + 1) << 17; the prefix at g0 at the first tie; the
// parity corrections of the later ties at g0).  The flag bytes hold per
// term (low nibble) whether it is flagged (a tie or big) and (high nibble)
// whether it is a tie.
constexpr int PZ_SLOT_PA = PZ_SP_SEG * 4;
constexpr int PZ_SLOT_PB = 2 * PZ_SP_SEG * 4;
constexpr int PZ_SLOT_FL = 3 * PZ_SP_SEG * 4;
constexpr int PZ_SLOT_SC = PZ_SLOT_FL + 64 * 2;
constexpr int PZ_SP_SLOT = PZ_SLOT_SC + 16;  // bytes per slot (a multiple of 16)
static_assert(PZ_SP_SLOT % 16 == 0, "slots stay 16-byte aligned");

constexpr uint32_t PZ_WALK_DONE = 0xffffffffu;  // consumed: the walk is over

struct PzWalk {
  pz_lds_u32* d;      // [nseg] increments at the record's grid
  pz_lds_u32* d2;     // [nseg] increments at the grid below (HAS2)
  pz_lds_u32* gf;     // [nseg] grid and flags
  pz_lds_u32* pd;     // [nseg + 1] exclusive prefix of d (mod 2^32)
  pz_lds_u32* chp;    // [nseg + 1] exclusive prefix count of grid changes between
                      //            neighbouring clean segments
  pz_lds_i32* spk;    // [nseg] the special segments in id order
  // Ring of nc pre-evaluated specials: special j sits in slot j % nc once
  // rdy[slot] == j + 1; a producer rewrites a slot only after the walker has
  // consumed the special before (consumed > j - nc).
  pz_lds_u8* ring;    // [nc][PZ_SP_SLOT] the slots
  pz_lds_u32* rdy;    // [nc] special + 1 held by the slot (0: none yet)
  pz_lds_u32* consumed;  // specials the walker has read out of the ring (PZ_WALK_DONE:
                         // the walk is over, the producers stop)
  pz_lds_u32* s0;     // the sequential fp32 sum of segment 0's terms from 0 (bits), when
                      // segment 0 is special 0 (else 0xffffffff)
  int nseg, nc, n_spec;
  bool pre0;  // s0 came with the set-up: segment 0 has no ring slot
};

// LDS of the walk for a row of nseg segments with a ring of nc pre-evaluated
// specials: six words per segment plus the prefixes' extra words and the
// ring's counter; per slot its terms, two increment prefixes, two flag masks
// and four scalars, and its ready word.
__host__ __device__ inline size_t pz_sp_walk_lds(int nseg, int nc) {
  return (size_t)nseg * 24 + 64 + (size_t)nc * PZ_SP_SLOT +
         (((size_t)nc * 4 + 15) & ~(size_t)15);
}

// Ring slots of the walk within max_lds bytes (0 when fewer than two fit:
// the ring's hand-over needs two).
inline int pz_sp_walk_nc(int nseg, size_t max_lds) {
  for (int nc = PZ_SP_NC; nc >= 2; nc--)
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

// Element i of a lane-major 4-per-lane array (wave-uniform i): the four
// registers of lane i / 4 read into scalars, then scalar selects (a select
// between registers on a uniform index compiles to branches).
__device__ __forceinline__ uint32_t pz_sp_elem(const uint32_t (&a)[4], int i) {
  const int l = i >> 2, c = i & 3;
  const uint32_t x0 = pz_readlane_u32(a[0], l), x1 = pz_readlane_u32(a[1], l);
  const uint32_t x2 = pz_readlane_u32(a[2], l), x3 = pz_readlane_u32(a[3], l);
  const uint32_t lo = (c & 1) ? x1 : x0, hi = (c & 1) ? x3 : x2;
  return (c & 2) ? hi : lo;
}
__device__ __forceinline__ float pz_sp_elemf(const float (&a)[4], int i) {
  const uint32_t u[4] = {__float_as_uint(a[0]), __float_as_uint(a[1]), __float_as_uint(a[2]),
                         __float_as_uint(a[3])};
  return __uint_as_float(pz_sp_elem(u, i));
}

// Index of the first element (lane-major, 4 per lane) whose predicate holds,
// or PZ_SP_SEG: one ballot per register column and scalar minima.
__device__ __forceinline__ int pz_sp_first4(bool p0, bool p1, bool p2, bool p3) {
  const uint64_t b0 = __ballot(p0), b1 = __ballot(p1), b2 = __ballot(p2), b3 = __ballot(p3);
  const int i0 = b0 ? 4 * (int)__builtin_ctzll(b0) : 1024;
  const int i1 = b1 ? 4 * (int)__builtin_ctzll(b1) + 1 : 1024;
  const int i2 = b2 ? 4 * (int)__builtin_ctzll(b2) + 2 : 1024;
  const int i3 = b3 ? 4 * (int)__builtin_ctzll(b3) + 3 : 1024;
  const int m01 = i0 < i1 ? i0 : i1, m23 = i2 < i3 ? i2 : i3;
  const int m = m01 < m23 ? m01 : m23;
  return m < PZ_SP_SEG ? m : PZ_SP_SEG;
}

// Inclusive prefix pv of the increments at grid g (as pz_sp_prefix4), with
// this lane's flag bits (tie or big) and, apart, its tie bits.
__device__ __forceinline__ void pz_sp_prefix4t(const float (&v)[4], uint32_t g, uint32_t (&pv)[4],
                                               uint32_t& flags, uint32_t& ties) {
  uint32_t inc[4], sum = 0;
  flags = 0;
  ties = 0;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    uint32_t cls;
    inc[c] = pz_inc(v[c], g, &cls);
    flags |= (cls != PZ_INC_PLAIN ? 1u : 0u) << c;
    ties |= (cls == PZ_INC_TIE ? 1u : 0u) << c;
    sum += inc[c];
  }
  uint32_t run = pz_wave_scan_u32(sum) - sum;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    run += inc[c];
    pv[c] = run;
  }
}

// Exclusive maximum over the lanes below (0 for lane 0).
__device__ __forceinline__ uint32_t pz_wave_excl_max_u32(uint32_t v) {
#define PZ_MAXDPP_(x, ctrl, rmask)                                                      \
  {                                                                                     \
    const uint32_t o = PZ_DPP(x, ctrl, rmask);                                          \
    x = o > x ? o : x;                                                                  \
  }
  PZ_MAXDPP_(v, 0x111, 0xf);  // row_shr:1
  PZ_MAXDPP_(v, 0x112, 0xf);  // row_shr:2
  PZ_MAXDPP_(v, 0x114, 0xf);  // row_shr:4
  PZ_MAXDPP_(v, 0x118, 0xf);  // row_shr:8
  PZ_MAXDPP_(v, 0x142, 0xa);  // row_bcast:15
  PZ_MAXDPP_(v, 0x143, 0xc);  // row_bcast:31
#undef PZ_MAXDPP_
  // lane l takes lane l - 1's inclusive maximum (wave_shr:1; lane 0 gets 0)
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x138, 0xf, 0xf, true);
}

// The segment's terms added to the state one at a time in id order with real
// fp32 adds -- the sequential sum itself, by the wave's DPP chain
// (pz_wave_chain4) -- for every segment the one-step forms do not take.
// Returns the index of a stop hit (st = the sum including that term) or -1
// (st = the sum over the segment).
template <int MODE>
__device__ __forceinline__ int pz_sp_chain(PzAcc& st, const float (&v)[4], float thr) {
  const int r = pz_wave_chain4(st, v, 0, thr, MODE, nullptr);
  pz_sp_uni(st);
  return r;
}

// A special segment in the walker's registers: its terms, the increment
// prefixes at its two grids, and per lane the flag bits (tie or big; low
// nibble) and tie bits (high nibble) at each.
struct PzSpSeg {
  float v[4];
  uint32_t P[4], Q[4];
  uint32_t fa, fb;
  uint32_t g0, sinfo, pt1, tc;  // as PzSpInfo (wave-uniform)
};

// Its scalars: the grids g0 (of P) and g1 (of Q), the first tie at g0 (256:
// none), the last flagged term at g1 plus one (0: none), P at the first tie
// and the parity corrections of the later ties at g0.  From a state n at
// g0 with no term leaving the binade and no big term, the ties at g0 give
// n + P[255] + ((n + pt1) & 1) + tc: round-half-even leaves the state even
// after the first tie, so only that one depends on n.
struct PzSpInfo {
  uint32_t g0, sinfo, pt1, tc;
};

__device__ __forceinline__ void pz_sp_prep(const float (&v)[4], uint32_t g0, uint32_t g1,
                                           PzSpSeg& d, PzSpInfo& inf) {
  uint32_t fP, tP, fQ, tQ;
  pz_sp_prefix4t(v, g0, d.P, fP, tP);
  pz_sp_prefix4t(v, g1, d.Q, fQ, tQ);
#pragma unroll
  for (int c = 0; c < 4; c++) d.v[c] = v[c];
  d.fa = fP | (tP << 4);
  d.fb = fQ | (tQ << 4);
  const uint64_t bt = __ballot(tP != 0u), bq = __ballot(fQ != 0u);
  uint32_t ft = PZ_SP_SEG, lq1 = 0;
  if (bt) {
    const int L = (int)__builtin_ctzll(bt);
    ft = 4u * L + (uint32_t)__builtin_ctz(pz_readlane_u32(tP, L));
  }
  if (bq) {
    const int L = 63 - (int)__builtin_clzll(bq);
    lq1 = 4u * L + 32u - (uint32_t)__builtin_clz(pz_readlane_u32(fQ, L));
  }
  // each later tie's correction: the parity of the prefix since the tie
  // before it (the previous tie's prefix + 1 by a max-scan: 0 = none yet)
  uint32_t last = 0;
#pragma unroll
  for (int c = 0; c < 4; c++) last = ((tP >> c) & 1u) ? d.P[c] + 1u : last;
  uint32_t prev = pz_wave_excl_max_u32(last), corr = 0;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    if ((tP >> c) & 1u) {
      if (prev) corr += (d.P[c] - (prev - 1u)) & 1u;
      prev = d.P[c] + 1u;
    }
  }
  inf.g0 = g0;
  inf.sinfo = g1 | (ft << 8) | (lq1 << 17);
  inf.pt1 = ft < (uint32_t)PZ_SP_SEG ? pz_sp_elem(d.P, (int)ft) : 0u;
  inf.tc = pz_wave_sum_u32(corr);
}

// The walk's LDS layout for nseg segments and nc ring slots at lds.
__device__ __forceinline__ PzWalk pz_sp_walk_layout(char* lds, int nseg, int nc) {
  PzWalk W;
  W.nseg = nseg;
  W.nc = nc;
  char* p = lds;
  W.ring = (pz_lds_u8*)p;      p += (size_t)nc * PZ_SP_SLOT;
  W.rdy = (pz_lds_u32*)p;      p += ((size_t)nc * 4 + 15) & ~(size_t)15;
  W.consumed = (pz_lds_u32*)p; p += 16;
  W.s0 = W.consumed + 1;
  W.d = (pz_lds_u32*)p;        p += (size_t)nseg * 4;
  W.d2 = (pz_lds_u32*)p;       p += (size_t)nseg * 4;
  W.gf = (pz_lds_u32*)p;       p += (size_t)nseg * 4;
  W.pd = (pz_lds_u32*)p;       p += (size_t)(nseg + 1) * 4;
  W.chp = (pz_lds_u32*)p;      p += (size_t)(nseg + 1) * 4;
  W.spk = (pz_lds_i32*)p;
  W.n_spec = 0;
  W.pre0 = false;
  return W;
}

// The second half of the set-up for records already in LDS (W.d, W.d2,
// W.gf of a layout from pz_sp_walk_layout, written before a barrier):
// prefixes, the special list, the ring and its producers.  s0_pre: the
// sequential fp32 sum of segment 0's terms from 0 (bits) when the caller
// has it already (0xffffffff: the producers add it up); segment 0 then
// gets no ring slot and the walker starts from that sum at once.
template <class X>
__device__ __forceinline__ PzWalk pz_sp_walk_start(const X& x, PzWalk W, PzSpShared& S,
                                                   int n_producers = -1,
                                                   uint32_t s0_pre = 0xffffffffu) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nt = (int)blockDim.x, nw = nt >> 6;
  if (n_producers < 0) n_producers = nw - 1;
  const int nseg = W.nseg, nc = W.nc;
  if (nseg <= 64) {
    // one segment per lane of wave 0, one barrier: the record prefix, the
    // grid changes and the special list by wave scans and ballots (lanes
    // past the row hold d = 0, so lane 63's prefix is the total)
    pz_lds_u32* nsp = W.consumed + 2;  // the special count, for every wave
    if (w == 0) {
      const int k = lane;
      uint32_t d = 0, gf = PZ_NO_RECORD, gfp = PZ_NO_RECORD;
      if (k < nseg) {
        d = W.d[k];
        gf = W.gf[k];
        if (k > 0) gfp = W.gf[k - 1];
      }
      const bool special = k < nseg && !pz_sp_clean(gf);
      const bool chg =
          k < nseg && pz_sp_clean(gf) && pz_sp_clean(gfp) && ((gf ^ gfp) & 0xffu) != 0u;
      const uint32_t incl = pz_wave_scan_u32(d);
      const uint64_t sb = __ballot(special);
      const uint64_t cb = __ballot(chg);
      const uint64_t below = (1ull << lane) - 1ull;
      if (k < nseg) {
        W.pd[k] = incl - d;
        W.chp[k] = (uint32_t)__popcll(cb & below);
        if (special) W.spk[__popcll(sb & below)] = k;
      }
      if (lane == 63) {
        W.pd[nseg] = incl;
        W.chp[nseg] = (uint32_t)__popcll(cb);
        *W.consumed = 0u;
        *W.s0 = s0_pre;
        *nsp = (uint32_t)__popcll(sb);
      }
    }
    if (tid < nc) W.rdy[tid] = 0u;
    __syncthreads();
    W.n_spec = (int)*nsp;
  } else {
    // records, their prefix, the grid changes between clean neighbours, and
    // the special segments in id order
    uint32_t base = 0;  // prefix carried over the chunks (thread-uniform)
    int sbase = 0;      // specials found in earlier chunks
    uint32_t cbase = 0; // grid changes in earlier chunks
    for (int c0 = 0; c0 < nseg; c0 += nt) {
      const int k = c0 + tid;
      uint32_t d = 0, gf = PZ_NO_RECORD, gfp = PZ_NO_RECORD;
      if (k < nseg) {
        d = W.d[k];
        gf = W.gf[k];
        if (k > 0) gfp = W.gf[k - 1];
      }
      const bool special = k < nseg && !pz_sp_clean(gf);
      const bool chg = k < nseg && pz_sp_clean(gf) && pz_sp_clean(gfp) && ((gf ^ gfp) & 0xffu) != 0u;
      // exclusive prefixes of d and of the grid changes, and the rank of the
      // special segments (workgroup scans)
      const uint32_t incl = pz_wave_scan_u32(d);
      const uint64_t sb = __ballot(special);
      const uint64_t cb = __ballot(chg);
      // (the caller's barrier orders the first chunk's writes of S after
      // earlier uses of it; later chunks wait for the reads of the last)
      if (c0 > 0) __syncthreads();
      if (lane == 63) S.list[w] = (int)incl;  // wave totals
      if (lane == 0) {
        S.red[w] = __int_as_float(__popcll(sb));
        S.red2[w] = (uint32_t)__popcll(cb);
      }
      __syncthreads();
      // the waves' totals, one per lane: inclusive scans, read at this wave
      // (exclusive) and at the last (the chunk's totals), mod 2^32
      const bool in_w = lane < nw;
      const uint32_t lt = in_w ? (uint32_t)S.list[lane] : 0u;
      const uint32_t ls = in_w ? (uint32_t)__float_as_int(S.red[lane]) : 0u;
      const uint32_t lc = in_w ? S.red2[lane] : 0u;
      const uint32_t it = pz_wave_scan_u32(lt), is = pz_wave_scan_u32(ls),
                     ic = pz_wave_scan_u32(lc);
      const uint32_t off = base + pz_readlane_u32(it - lt, w);
      const int soff = sbase + (int)pz_readlane_u32(is - ls, w);
      const uint32_t coff = cbase + pz_readlane_u32(ic - lc, w);
      const uint64_t below = (1ull << lane) - 1ull;
      if (k < nseg) {
        W.pd[k] = off + incl - d;
        W.chp[k] = coff + (uint32_t)__popcll(cb & below);
        if (special) W.spk[soff + __popcll(sb & below)] = k;
      }
      base += pz_readlane_u32(it, nw - 1);
      sbase += (int)pz_readlane_u32(is, nw - 1);
      cbase += pz_readlane_u32(ic, nw - 1);
    }
    if (tid == 0) {
      W.pd[nseg] = base;
      W.chp[nseg] = cbase;
      *W.consumed = 0u;
      *W.s0 = s0_pre;
    }
    if (tid < nc) W.rdy[tid] = 0u;
    W.n_spec = sbase;
    __syncthreads();
  }
  W.pre0 = s0_pre != 0xffffffffu;
  // Waves 1 .. n_producers pre-evaluate the specials in id order into the
  // ring, while wave 0 (the walker) starts at once.  The walker waits only
  // for the special it needs next; the producer of that special handles its
  // specials in increasing order and waits only until special j - nc is
  // consumed, which it is by then -- so every wait ends.
  // A walk that stops early (a stop hit) marks itself over
  // (PZ_WALK_DONE), which ends every producer's wait and loop.
  for (int j = w - 1; w > 0 && w <= n_producers && j < W.n_spec; j += n_producers) {
    uint32_t c = __hip_atomic_load((uint32_t*)W.consumed, __ATOMIC_ACQUIRE,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
    if (j >= nc)
      while (c <= (uint32_t)(j - nc)) {
        __builtin_amdgcn_s_sleep(1);
        c = __hip_atomic_load((uint32_t*)W.consumed, __ATOMIC_ACQUIRE,
                              __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    if (c == PZ_WALK_DONE) break;
    const int k = W.spk[j];
    if (j == 0 && k == 0 && W.pre0) continue;  // summed before the walk: no slot
    const int sl = j % nc;
    pz_lds_u8* sb = W.ring + (size_t)sl * PZ_SP_SLOT;
    float v[4];
    x.seg(k, v);
    const uint32_t gf = W.gf[k];
    const uint32_t g = gf == PZ_NO_RECORD ? 1u : (gf & 0xffu);
    // the grid the segment is expected to end in: a mid-binade start plus
    // the segment's terms (a term as large as the sum lifts it several
    // binades at once)
    const float sum = pz_wave_sum((v[0] + v[1]) + (v[2] + v[3]));
    const float start = g > 1u ? 1.5f * __uint_as_float(g << 23) : 0.0f;  // 1.5 * 2^(g - 127)
    const uint32_t ge = pz_grid_of(start + sum);
    PzSpSeg d;
    PzSpInfo inf;
    pz_sp_prep(v, g, ge > g + 1u ? ge : g + 1u, d, inf);
    pz_f4 q;
    q.x = v[0];
    q.y = v[1];
    q.z = v[2];
    q.w = v[3];
    ((pz_lds_f4*)sb)[lane] = q;
    pz_u4 a4, b4;
    a4.x = d.P[0]; a4.y = d.P[1]; a4.z = d.P[2]; a4.w = d.P[3];
    b4.x = d.Q[0]; b4.y = d.Q[1]; b4.z = d.Q[2]; b4.w = d.Q[3];
    ((pz_lds_u4*)(sb + PZ_SLOT_PA))[lane] = a4;
    ((pz_lds_u4*)(sb + PZ_SLOT_PB))[lane] = b4;
    ((pz_lds_u16h*)(sb + PZ_SLOT_FL))[lane] = (uint16_t)((d.fa & 0xffu) | ((d.fb & 0xffu) << 8));
    if (lane == 0) {
      pz_u4 sc;
      sc.x = g; sc.y = inf.sinfo; sc.z = inf.pt1; sc.w = inf.tc;
      *(pz_lds_u4*)(sb + PZ_SLOT_SC) = sc;
    }
    if (j == 0 && k == 0) {
      // the row's first segment from a zero sum, where nearly every term
      // leaves the binade: its plain sequential fp32 sum (the wave's chain
      // of real adds), for the walker to take in one step
      PzAcc z;
      z.n = 0u;
      z.g = 1u;
      pz_sp_chain<PZ_STOP_NONE>(z, v, 0.0f);
      if (lane == 0) *W.s0 = __float_as_uint(pz_acc_value(z));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane == 0)
      __hip_atomic_store((uint32_t*)&W.rdy[sl], (uint32_t)(j + 1), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  return W;
}

// A row's records loaded ahead into registers (thread k: segment k, for rows
// of at most blockDim.x segments; else off), so that their latency passes
// while the kernel does other set-up work; pz_sp_walk_setup stores them.
struct PzRecAhead {
  uint32_t d, d2, gf;
  bool on;
};

__device__ __forceinline__ PzRecAhead pz_sp_rec_ahead(const PzSplitWs& ws, int row, int nseg) {
  PzRecAhead a;
  a.on = nseg <= (int)blockDim.x;
  a.d = 0u;
  a.d2 = 0u;
  a.gf = PZ_NO_RECORD;
  const int k = threadIdx.x;
  if (a.on && k < nseg) {
    a.d = pz_sp_rec_d(ws, row)[k];
    a.d2 = pz_sp_rec_d2(ws, row)[k];
    a.gf = pz_sp_rec_gf(ws, row)[k];
  }
  return a;
}

// Stages the row's records in LDS, lists every special segment (dirty,
// crossing, or without a record) in id order, and starts the pre-evaluation
// of the specials into the ring: exact terms (X::seg) and increment
// prefixes and flags at the record's grid and the grid the segment is
// expected to end in.  Every thread calls it; it returns without a final
// barrier: waves 1 .. n_producers keep filling the ring while the walker
// (wave 0) consumes it (pz_sp_load_slot), the other waves may go on to other
// work.  Any block size that is a multiple of 64, up to 1024.  s0_pre as for
// pz_sp_walk_start; ahead: the records already loaded (pz_sp_rec_ahead).
template <class X>
__device__ __forceinline__ PzWalk pz_sp_walk_setup(const X& x, int row, int nseg, int nc,
                                                   const PzSplitWs& ws, char* lds,
                                                   PzSpShared& S, int n_producers = -1,
                                                   uint32_t s0_pre = 0xffffffffu,
                                                   const PzRecAhead* ahead = nullptr) {
  PzWalk W = pz_sp_walk_layout(lds, nseg, nc);
  if (ahead && ahead->on) {
    const int k = threadIdx.x;
    if (k < nseg) {
      W.d[k] = ahead->d;
      W.d2[k] = ahead->d2;
      W.gf[k] = ahead->gf;
    }
  } else {
    const uint32_t* rd = pz_sp_rec_d(ws, row);
    const uint32_t* rd2 = pz_sp_rec_d2(ws, row);
    const uint32_t* rgf = pz_sp_rec_gf(ws, row);
    for (int k = threadIdx.x; k < nseg; k += blockDim.x) {
      W.d[k] = rd[k];
      W.d2[k] = rd2[k];
      W.gf[k] = rgf[k];
    }
  }
  __syncthreads();
  return pz_sp_walk_start(x, W, S, n_producers, s0_pre);
}

// The common special segment in one step: at the state's grid no tie or big
// term comes before the first term that leaves the binade, that term is
// taken with one real fp32 add, and the rest of the segment fits the next
// binade without a flagged term (the prefixes only grow, so the rest's
// total decides).  Also a segment with no event at all.  Needs st.g == the
// grid of P; Q is the prefix at the grid above.  Returns false, leaving st
// alone, for anything else (and for a stop hit anywhere in the segment),
// which the caller hands to pz_sp_chain.
template <int MODE>
__device__ __forceinline__ bool pz_sp_fast(PzAcc& st, const float (&v)[4], const uint32_t (&P)[4],
                                           uint32_t fP, const uint32_t (&Q)[4], uint32_t fQ,
                                           float thr) {
  const int lane = threadIdx.x & 63;
  const uint32_t room = (1u << 24) - st.n;
  bool e[4];
#pragma unroll
  for (int c = 0; c < 4; c++) e[c] = ((fP >> c) & 1u) != 0u || P[c] >= room;
  const int i = pz_sp_first4(e[0], e[1], e[2], e[3]);
  PzAcc a;
  if (i >= PZ_SP_SEG) {
    a.n = st.n + pz_readlane_u32(P[3], 63);
    a.g = st.g;
  } else {
    if ((pz_readlane_u32(fP, i >> 2) >> (i & 3)) & 1u) return false;  // a tie or a big term first
    const uint32_t before = i > 0 ? pz_sp_elem(P, i - 1) : 0u;
    a = pz_acc_of(pz_acc_value_ng(st.n + before, st.g) + pz_sp_elemf(v, i));
    if (a.g != st.g + 1u) return false;
    // the terms after i at the next grid: none flagged, their sum inside it
    const uint32_t qi = pz_sp_elem(Q, i);
    const uint64_t later = __ballot(fQ != 0u && 4 * lane + 31 - (int)__builtin_clz(fQ) > i);
    const uint32_t rest = pz_readlane_u32(Q[3], 63) - qi;
    if (later || rest >= (1u << 24) - a.n) return false;
    a.n += rest;
  }
  if (MODE != PZ_STOP_NONE && pz_stop_hit(pz_acc_value(a), thr, MODE)) return false;
  st.n = (uint32_t)__builtin_amdgcn_readfirstlane((int)a.n);
  st.g = (uint32_t)__builtin_amdgcn_readfirstlane((int)a.g);
  return true;
}

// A pre-evaluated special segment in one step (sinfo, pt1, tc as in
// PzSpInfo; the state at g0, the grid of P): with no term leaving the
// binade and no big term, the segment's increments plus its ties' parity
// corrections; else, when no tie comes first, the first term that leaves
// the binade (or the big term) taken with one real fp32 add and the rest of
// the segment at g1, which must hold no flagged term after it and fit the
// binade.  Returns false, leaving st alone, for anything else (and for a
// stop hit anywhere in the segment).
template <int MODE>
__device__ __forceinline__ bool pz_sp_fast_pre(PzAcc& st, const PzSpSeg& d, uint32_t sinfo,
                                               uint32_t pt1, uint32_t tc, float thr) {
  const uint32_t g1 = sinfo & 0xffu, ft = (sinfo >> 8) & 0x1ffu, lq1 = (sinfo >> 17) & 0x1ffu;
  const uint32_t room = (1u << 24) - st.n;
  const uint32_t big = (d.fa & ~(d.fa >> 4)) & 15u;  // flagged and not a tie
  uint32_t m = 0;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    const uint32_t reach = (d.P[c] >> 31) | (((d.P[c] - room) >> 31) ^ 1u);
    m |= (((big >> c) & 1u) | reach) << c;
  }
  const uint64_t ball = __ballot(m != 0u);
  PzAcc a;
  if (!ball) {
    uint32_t nn = st.n + pz_readlane_u32(d.P[3], 63);
    if (ft < (uint32_t)PZ_SP_SEG) {
      nn += ((st.n + pt1) & 1u) + tc;
      if (nn >= (1u << 24)) return false;
    }
    a.n = nn;
    a.g = st.g;
  } else {
    const int c = (int)__builtin_ctz(m | 16u);
    const uint32_t before = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)d.P[3], 0x138, 0xf, 0xf, true);
    const uint32_t prv = pz_sel4(before, d.P[0], d.P[1], d.P[2], c);
    const float tv = pz_sel4f(d.v[0], d.v[1], d.v[2], d.v[3], c & 3);
    const uint32_t qv = pz_sel4(d.Q[0], d.Q[1], d.Q[2], d.Q[3], c & 3);
    const int L = (int)__builtin_ctzll(ball);
    const uint32_t i = 4u * L + (uint32_t)__builtin_amdgcn_readlane(c, L);
    if (ft <= i) return false;  // a tie first
    const uint32_t prev = pz_readlane_u32(prv, L), qi = pz_readlane_u32(qv, L);
    a = pz_acc_of(pz_acc_value_ng(st.n + prev, st.g) + pz_readlane_f32(tv, L));
    const uint32_t rest = pz_readlane_u32(d.Q[3], 63) - qi;
    if (a.g != g1 || lq1 > i + 1u || rest >= (1u << 24) - a.n) return false;
    a.n += rest;
  }
  if (MODE != PZ_STOP_NONE && pz_stop_hit(pz_acc_value(a), thr, MODE)) return false;
  st.n = (uint32_t)__builtin_amdgcn_readfirstlane((int)a.n);
  st.g = (uint32_t)__builtin_amdgcn_readfirstlane((int)a.g);
  return true;
}

// Whether special j is in the ring (acquire).
__device__ __forceinline__ bool pz_sp_slot_ready(const PzWalk& W, int j) {
  return __hip_atomic_load((uint32_t*)&W.rdy[j % W.nc], __ATOMIC_ACQUIRE,
                           __HIP_MEMORY_SCOPE_WORKGROUP) == (uint32_t)(j + 1);
}

// How many specials from j1 on (slot s1, the next ones in the following
// slots) are in the ring: lane i reads the ready word of special j1 + i,
// one LDS round trip for up to nc specials (acquire: their data is read
// after).  A special seen there stays until the walker has consumed it.
__device__ __forceinline__ int pz_sp_ready_count(const PzWalk& W, int j1, int s1) {
  const int lane = threadIdx.x & 63;
  bool rdy = false;
  if (lane < W.nc) {
    int s = s1 + lane;
    s = s >= W.nc ? s - W.nc : s;
    rdy = __hip_atomic_load((uint32_t*)&W.rdy[s], __ATOMIC_RELAXED,
                            __HIP_MEMORY_SCOPE_WORKGROUP) == (uint32_t)(j1 + lane + 1);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  const uint64_t nb = ~__ballot(rdy);
  return nb ? (int)__builtin_ctzll(nb) : 64;
}

// The pre-evaluated data of the special in slot s (one round of LDS reads),
// once in the ring.
__device__ __forceinline__ void pz_sp_load_slot_at(const PzWalk& W, int s, PzSpSeg& d) {
  const int lane = threadIdx.x & 63;
  const pz_lds_u8* sb = W.ring + (size_t)s * PZ_SP_SLOT;
  const pz_u4 sc = *(const pz_lds_u4*)(sb + PZ_SLOT_SC);
  d.g0 = sc.x;
  d.sinfo = sc.y;
  d.pt1 = sc.z;
  d.tc = sc.w;
  const pz_f4 q = ((const pz_lds_f4*)sb)[lane];
  const pz_u4 a4 = ((const pz_lds_u4*)(sb + PZ_SLOT_PA))[lane];
  const pz_u4 b4 = ((const pz_lds_u4*)(sb + PZ_SLOT_PB))[lane];
  const uint32_t fl = ((const pz_lds_u16h*)(sb + PZ_SLOT_FL))[lane];
  d.fa = fl & 0xffu;
  d.fb = fl >> 8;
  d.v[0] = q.x; d.v[1] = q.y; d.v[2] = q.z; d.v[3] = q.w;
  d.P[0] = a4.x; d.P[1] = a4.y; d.P[2] = a4.z; d.P[3] = a4.w;
  d.Q[0] = b4.x; d.Q[1] = b4.y; d.Q[2] = b4.z; d.Q[3] = b4.w;
}

// The same for special j, waiting until it is in the ring.
__device__ __forceinline__ void pz_sp_load_slot(const PzWalk& W, int j, PzSpSeg& d) {
  while (!pz_sp_slot_ready(W, j)) __builtin_amdgcn_s_sleep(1);
  pz_sp_load_slot_at(W, j % W.nc, d);
}

// Lane i of the walker: the clean run before special j0 + i (its end, the
// sum of its records, their common grid or 0) and the special's own record
// (grid and flags, the increment at the grid below); the run after the last
// special ends at nseg.
struct PzRunLanes {
  int k;
  uint32_t D, G, gf, d2;
};
__device__ __forceinline__ PzRunLanes pz_sp_run_lanes(const PzWalk& W, int j0) {
  const int j = j0 + (int)(threadIdx.x & 63);
  PzRunLanes r;
  r.k = 0;
  r.D = 0;
  r.G = 0;
  r.gf = PZ_NO_RECORD;
  r.d2 = 0;
  if (j <= W.n_spec) {
    const int a = j == 0 ? 0 : W.spk[j - 1] + 1;
    const int b = j < W.n_spec ? W.spk[j] : W.nseg;
    r.k = b;
    if (b > a) {
      r.D = W.pd[b] - W.pd[a];
      const bool one_grid = b == a + 1 || W.chp[b] == W.chp[a + 1];
      r.G = one_grid ? (W.gf[a] & 0xffu) : 0u;
    }
    if (j < W.n_spec) {
      r.gf = W.gf[b];
      r.d2 = W.d2[b];
    }
  }
  return r;
}

// The record at the grid below (HAS2) when the state sits there: gf, d2 of
// the segment.  Returns true when it served the segment.
template <int MODE>
__device__ __forceinline__ bool pz_sp_has2(PzAcc& st, uint32_t gf, uint32_t d2, float thr) {
  if (gf != PZ_NO_RECORD && (gf & PZ_GF_HAS2) && !(gf & (PZ_GF_DIRTY2 | PZ_GF_XING)) &&
      (gf & 0xffu) - 1u == st.g && d2 < (1u << 24) - st.n &&
      !(MODE != PZ_STOP_NONE && pz_stop_hit(pz_acc_value_ng(st.n + d2, st.g), thr, MODE))) {
    st.n += d2;
    pz_sp_uni(st);
    return true;
  }
  return false;
}

// Segment k from the state st when its primary record cannot serve it and
// it has no pre-evaluated slot: the record at the grid below (HAS2), else
// its exact terms (X::seg) through pz_sp_fast or the chain.  Returns the
// index of a stop hit in the segment, or -1.
template <int MODE, class X>
__device__ __forceinline__ int pz_sp_special(PzAcc& st, const PzWalk& W, float thr, const X& x,
                                             int k) {
  if (pz_sp_has2<MODE>(st, W.gf[k], W.d2[k], thr)) return -1;
  float v[4];
  uint32_t P[4], Q[4], fP, fQ;
  x.seg(k, v);
  const uint32_t g0 = st.g;
  pz_sp_prefix4(v, g0, P, fP);
  pz_sp_prefix4(v, g0 + 1u, Q, fQ);
  if (pz_sp_fast<MODE>(st, v, P, fP, Q, fQ, thr)) return -1;
  return pz_sp_chain<MODE>(st, v, thr);
}

// Segments [k, kend) one record at a time: runs of clean records at the
// state's grid advance 64 segments per step, any other segment goes through
// pz_sp_special.  Returns the element index of a stop hit, or -1.
template <int MODE, class X>
__device__ __forceinline__ int pz_sp_walk_range(PzAcc& st, const PzWalk& W, float thr,
                                                const X& x, int k, int kend) {
  const int lane = threadIdx.x & 63;
  while (k < kend) {
    {
      const int kk = k + lane;
      bool bad = true;
      if (kk < kend) {
        const uint32_t gf = W.gf[kk];
        const uint32_t upto = W.pd[kk + 1] - W.pd[k];  // d of [k, kk]
        bad = !pz_sp_clean(gf) || (gf & 0xffu) != st.g || upto >= (1u << 24) - st.n ||
              (MODE != PZ_STOP_NONE &&
               pz_stop_hit(pz_acc_value_ng(st.n + upto, st.g), thr, MODE));
      }
      const uint64_t ball = __ballot(bad);
      const int L = ball ? (int)__builtin_ctzll(ball) : 64;
      const int kb = k + L;
      st.n += W.pd[kb < kend ? kb : kend] - W.pd[k];
      pz_sp_uni(st);
      if (kb >= kend) break;
      k = kb;
      if (L == 64) continue;
    }
    const int r = pz_sp_special<MODE>(st, W, thr, x, k);
    if (r >= 0) return k * PZ_SP_SEG + r;
    k++;
  }
  return -1;
}

// States of a walk after each listed special (lane j: after special j), so
// a later walk over the same terms with a higher stop can resume from the
// last one below its stop instead of from state 0.
struct PzWalkCk {
  uint32_t n = 0, g = 0;  // per lane
  int cnt = 0;            // specials recorded
};

// The walk (one wave): the exact sequential sum of the row's terms in id
// order, from state 0.  With a stop mode returns the element index of the
// first hit (st = the sum including it), else -1 (st = the whole sum).  X
// provides seg(k, v[4]) for segments evaluated during the walk.
//
// It goes from listed special to listed special: the clean run before each
// one is a single step when its records share the state's grid and neither
// leave the binade nor reach the stop (sums only grow, so the run's total
// decides); otherwise that run goes record by record (pz_sp_walk_range).
// The runs' and the specials' scalars sit in the wave's lanes (lane j: run
// and special j), and each special's pre-evaluated data loads while the one
// before is processed, so a step waits on no LDS read.
//
// With rec, the state after each listed special is recorded there; with
// from (a record of an earlier walk over the same terms whose sums never
// met this walk's stop before the point it resumes from), the walk starts at
// the last recorded state that does not meet the stop -- the sums only grow,
// so no hit lies before it.  A resumed walk does not read the ring (the
// earlier walk has released its slots to the producers): it evaluates its
// specials itself (pz_sp_special).
template <int MODE, class X>
__device__ __forceinline__ int pz_sp_walk_run(PzAcc& st, const PzWalk& W, float thr, const X& x,
                                              PzWalkCk* rec, const PzWalkCk* from) {
  const int lane = threadIdx.x & 63;
  const bool ring = from == nullptr;
  st.n = 0;
  st.g = 1;
  const int np = W.n_spec;
  int k = 0, j0 = 0;
  if (from && from->cnt > 0) {
    const bool hit = lane < from->cnt &&
                     (MODE == PZ_STOP_NONE ||
                      pz_stop_hit(pz_acc_value_ng(from->n, from->g), thr, MODE));
    const uint64_t hb = __ballot(hit);
    const int h = hb ? (int)__builtin_ctzll(hb) : from->cnt;  // first record at or past the stop
    if (h > 0) {
      st.n = pz_readlane_u32(from->n, h - 1);
      st.g = pz_readlane_u32(from->g, h - 1);
      k = W.spk[h - 1] + 1;
      j0 = h;
    }
  }
  int base = j0 & ~63;  // specials of the lanes
  PzRunLanes m = pz_sp_run_lanes(W, base);
  // (the run lanes settle before the loop's ring loads are issued, so no use
  // of them waits for those)
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
  PzSpSeg nxt;
  bool have = false;     // nxt holds special j
  int ready_to = j0;     // the specials below it are known to be in the ring
  int slot = j0 % W.nc;  // special j's slot
  for (int j = j0;; j++) {
    if (j - base == 64) {
      base = j;
      m = pz_sp_run_lanes(W, base);
      __builtin_amdgcn_s_waitcnt(0xc07f);
    }
    const int jl = j - base;
    const int b = __builtin_amdgcn_readlane(m.k, jl);
    const int slot1 = slot + 1 == W.nc ? 0 : slot + 1;  // special j + 1's slot
    PzSpSeg cur = nxt;
    // segment 0 summed before the walk has no slot: taken from s0, or (a
    // stop within it) evaluated here
    const bool self0 = ring && j == 0 && b == 0 && W.pre0;
    if (ring) {
      if (j < np && !have && !self0) pz_sp_load_slot(W, j, cur);
      // the slots of the specials before j are released to the producers
      // (their reads are done: special j's data came in with the last step's
      // loads; special j's slot stays, the serial path reads its terms
      // there), then the next special's loads, when it is already in the
      // ring, overlap this step (no fence waits for them).  The producer of
      // special j + 1 needs consumed > j + 1 - nc, which holds with nc >= 2.
      // Which specials are in the ring is read for several at once, again
      // when the walk gets past them.
      if (j < np) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0)
          __hip_atomic_store((uint32_t*)W.consumed, (uint32_t)j, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      if (j + 1 < np && j + 1 >= ready_to)
        ready_to = j + 1 + pz_sp_ready_count(W, j + 1, slot1);
      have = j + 1 < np && j + 1 < ready_to;
      if (have) pz_sp_load_slot_at(W, slot1, nxt);
    }
    if (k < b) {
      const uint32_t D = pz_readlane_u32(m.D, jl), G = pz_readlane_u32(m.G, jl);
      if (G == st.g && D < (1u << 24) - st.n &&
          !(MODE != PZ_STOP_NONE && pz_stop_hit(pz_acc_value_ng(st.n + D, st.g), thr, MODE))) {
        st.n += D;
      } else {
        const int r = pz_sp_walk_range<MODE>(st, W, thr, x, k, b);
        if (r >= 0) return r;
      }
      pz_sp_uni(st);
    }
    k = b;
    if (j >= np) break;
    // special b
    bool taken = false;
    if (j == 0 && b == 0 && st.n == 0u && st.g == 1u) {
      // the first segment from a zero sum, pre-added (sums only grow: when
      // its total does not meet the stop, no term of it does)
      const uint32_t s0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)*W.s0);
      if (s0 != 0xffffffffu &&
          !(MODE != PZ_STOP_NONE && pz_stop_hit(__uint_as_float(s0), thr, MODE))) {
        st = pz_acc_of(__uint_as_float(s0));
        pz_sp_uni(st);
        taken = true;
      }
    }
    if (!taken && (!ring || self0)) {
      const int r = pz_sp_special<MODE>(st, W, thr, x, b);
      if (r >= 0) return b * PZ_SP_SEG + r;
    } else if (!taken &&
               !pz_sp_has2<MODE>(st, pz_readlane_u32(m.gf, jl), pz_readlane_u32(m.d2, jl), thr)) {
      const uint32_t g0 = cur.g0, si = cur.sinfo;
      if (!(st.g == g0 && pz_sp_fast_pre<MODE>(st, cur, si, cur.pt1, cur.tc, thr))) {
        const int r = pz_sp_chain<MODE>(st, cur.v, thr);
        if (r >= 0) return b * PZ_SP_SEG + r;
      }
    }
    k = b + 1;
    slot = slot1;
    if (rec && j < 64) {
      rec->n = lane == j ? st.n : rec->n;
      rec->g = lane == j ? st.g : rec->g;
      rec->cnt = j + 1;
    }
  }
  return -1;
}

// The walk, then (a walk that reads the ring) the mark that it is over: a
// walk that stopped early leaves specials its producers would otherwise
// wait to write, so every producer's wait ends and its loop stops, and the
// workgroup's next barrier is reached whatever the stop.  One walk reads
// the ring per set-up; later walks over the same set-up resume from its
// recorded states (from).
template <int MODE, class X>
__device__ __forceinline__ int pz_sp_walk(PzAcc& st, const PzWalk& W, float thr, const X& x,
                                          PzWalkCk* rec = nullptr,
                                          const PzWalkCk* from = nullptr) {
  const int r = pz_sp_walk_run<MODE>(st, W, thr, x, rec, from);
  if (from == nullptr) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if ((threadIdx.x & 63) == 0)
      __hip_atomic_store((uint32_t*)W.consumed, PZ_WALK_DONE, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  return r;
}

#endif
