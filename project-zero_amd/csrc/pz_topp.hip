// pz_topp.hip -- batched top-p (nucleus) sampling, bit-exact with the
// reference's fp32 arithmetic.
//
// Reference semantics (src/sampling/top_p.c:30-108), applied after penalties
// and temperature:
//   * V > 200000 -> argmax (:33-34);  maximum by strict '>' from x[0] (:37-41);
//   * candidates x >= max - 20 (:53-58), e = expf(x - max), a sequential fp32
//     sum in ascending id order (:57-65); no candidate -> argmax (:68-69);
//   * p = e * (1/sum) (:72-74); stable sort by p descending (:77), so equal p
//     stay in ascending id;
//   * cut-off: first i with sequential cumulative >= top_p, else all (:80-88);
//     trunc_sum = the same sequential sum (:91-93); r = u * trunc_sum;
//     first i < cut-off with r < cdf, else slot 0 (:96-105).
//
// Design: every row is split over S workgroups (pz_split.h), launches
//   k_topp_stat    (HBM) slice maxima;
//   k_topp_est     (L2)  estimated candidate mass per segment;
//   k_topp_rec     (L2)  exact e = expf(x - max) (glibc-identical pz_expf)
//                  of every candidate -> integer segment records at the
//                  predicted binades + a mass histogram of e per workgroup;
//   k_topp_walk    one workgroup per row walks the records (the exact
//                  normaliser) while its spare waves merge the histograms
//                  and pick the smallest set of top bins whose estimated
//                  mass clears top_p with margin; in the same launch S
//                  workgroups per row then gather the candidates of those
//                  bins as (e, ~id) keys -- with p = e * (1/sum) a prefix of
//                  the reference's sort order, so the gather does not wait
//                  for the normaliser;
//   k_topp_nucleus (one workgroup per row) keys to p, sorted in LDS
//                  (counting sort by p bin, rank inside a bin), the exact
//                  cumulative to the cut-off and the draw;
//   k_topp_fallback rows whose selected set does not fit in LDS, or whose
//                  cumulative does not reach top_p inside it: every
//                  candidate sorted in a global scratch slot.
#include <limits.h>

#include <atomic>

#include "pz_device.h"
#include "pz_exact.h"
#include "pz_launch.h"
#include "pz_rowpass.h"
#include "pz_seq.h"
#include "pz_sort.h"
#include "pz_split.h"

namespace {

constexpr int TOPP_CAP_MAX = 12288;
// Lists whose bins are too large for the rank count are bitonic-sorted whole
// in LDS up to this many keys (beyond: the fallback).
constexpr int TOPP_BITONIC_MAX = 8192;
// Gathered lists of at least TOPP_BINSORT_MIN keys are ordered by a counting
// sort over PBINS bins of p (1/128 binade each, 32 binades below 1.0) and a
// rank count inside each bin; smaller ones by a bitonic sort.
constexpr int PBINS = 4 * PZ_RB;
constexpr int TOPP_BINSORT_MIN = 1024;
constexpr int TOPP_BIN_MAX = 256;  // larger bins: bitonic sort

// Row states (PzRowState::i[0]).
constexpr int TP_OPEN = 0, TP_DONE = 1;
// PzRowState fields used here: f[0] p threshold, f[1] gate on y - M,
// i[1] every candidate gathered, i[2] gathered count, i[3] overflow,
// i[4] candidates in the selected bins.

__device__ __forceinline__ int ebin(float e) {
  const int b = (int)(__float_as_uint(e) >> 17) - PZ_TOPP_NB_BASE;
  return b < 0 ? 0 : (b >= PZ_TOPP_NB ? PZ_TOPP_NB - 1 : b);
}
__device__ __forceinline__ float ebin_lo(int b) {
  return __uint_as_float((uint32_t)(b + PZ_TOPP_NB_BASE) << 17);
}
__device__ __forceinline__ float ebin_mid(int b) {
  return __uint_as_float(((uint32_t)(b + PZ_TOPP_NB_BASE) << 17) | 0x10000u);
}

__device__ __forceinline__ uint64_t topp_key(float p, int id) {
  return ((uint64_t)__float_as_uint(p) << 32) | (uint64_t)(0xffffffffu - (uint32_t)id);
}
__device__ __forceinline__ int key_id(uint64_t k) { return (int)(0xffffffffu - (uint32_t)k); }
// A gathered (e, ~id) key as (p, ~id): p = e * (1 / sum), top_p.c:72-74.
__device__ __forceinline__ uint64_t topp_pkey(uint64_t ekey, float inv) {
  const float p = __uint_as_float((uint32_t)(ekey >> 32)) * inv;
  return ((uint64_t)__float_as_uint(p) << 32) | (ekey & 0xffffffffull);
}
__device__ __forceinline__ float key_p(uint64_t k) { return __uint_as_float((uint32_t)(k >> 32)); }

struct ToppShared {
  int merged;  // waves done merging the histograms
  uint32_t wtot[PZ_RB / 64];
  uint32_t bmax;
  float sum;
  int bsel;
  uint32_t nsel;
  int cutoff;
  int first;
};

// Wave-aggregated append of up to one key per lane into buf (capacity cap).
template <class CountPtr>
__device__ __forceinline__ void append_key(CountPtr count, int* over, uint64_t* buf, int cap,
                                           bool want, uint64_t key) {
  const uint64_t ball = __ballot(want);
  if (!ball) return;
  const int lane = threadIdx.x & 63;
  const int leader = (int)__builtin_ctzll(ball);
  int base = 0;
  if (lane == leader) base = atomicAdd(count, __popcll(ball));
  base = __shfl(base, leader, 64);
  if (want) {
    const int slot = base + __popcll(ball & ((1ull << lane) - 1ull));
    if (slot < cap) buf[slot] = key;
    else *over = 1;
  }
}

// Reference cumulative/draw over a descending key list (wave 0 computes the
// cut-off, thread 0 draws).  keys/cum may be LDS or global.  all_gathered:
// the list holds every candidate (then a cumulative that never reaches top_p
// keeps all of them, top_p.c:81).  Returns the cut-off, or -1 when the
// list is a strict prefix whose cumulative stays below top_p.
__device__ __forceinline__ int nucleus_cutoff(const uint64_t* keys, float* cum, int m, float top_p,
                                              bool all_gathered, int* cutoff_sh) {
  const int tid = threadIdx.x, lane = tid & 63;
  if (tid < 64) {
    PzAcc st;
    st.n = 0;
    st.g = 1;
    int cutoff = -1;
    for (int j0 = 0; j0 < m; j0 += 256) {
      // lane l holds keys j0 + 4l .. j0 + 4l + 3 (terms past m are 0; cum
      // has room: cap and the fallback slots are multiples of 256)
      float v[4];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int j = j0 + 4 * lane + c;
        v[c] = j < m ? key_p(keys[j]) : 0.0f;
      }
      const int f = pz_wave_accumulate<4>(st, v, 0, top_p, PZ_STOP_GE, cum + j0);
      if (f >= 0) {
        cutoff = j0 + f + 1;
        break;
      }
    }
    if (cutoff < 0 && all_gathered) cutoff = m;
    if (lane == 0) *cutoff_sh = cutoff;
  }
  __syncthreads();
  return *cutoff_sh;
}

__device__ __forceinline__ void nucleus_draw(const uint64_t* keys, const float* cum, int cutoff,
                                             float uu, int32_t* id_out, float* p_out) {
  const float trunc_sum = cum[cutoff - 1];
  const float r = uu * trunc_sum;
  int lo = 0, hi = cutoff;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (r < cum[mid]) hi = mid;
    else lo = mid + 1;
  }
  const int pick = lo < cutoff ? lo : 0;
  const uint64_t k = keys[pick];
  *id_out = key_id(k);
  if (p_out) *p_out = key_p(k);
}

typedef __attribute__((address_space(3))) uint16_t pz_lds_u16;
typedef __attribute__((address_space(3))) uint32_t pz_lds_u32b;

// p bin of a key, 0 for p in [1, 2) (p <= 1), growing as p falls.
__device__ __forceinline__ int pbin(uint64_t key) {
  const int q = 0x3f80 - (int)(key >> 48);  // bits(p) >> 16
  return q < PBINS - 1 ? q : PBINS - 1;
}

// Exclusive starts of the PBINS bin counts in bcnt, by every thread of a
// PZ_SP_BLOCK workgroup (thread t owns bins 4t .. 4t+3): bstart[b] = bcnt[b]
// = the start of bin b (bcnt turns into the bins' cursors).  T.bmax must be
// 0 on entry; returns the largest bin count.
__device__ __forceinline__ uint32_t topp_bin_starts(pz_lds_u32b* bcnt, pz_lds_u32b* bstart,
                                                    ToppShared& T) {
  static_assert(PBINS == 4 * PZ_SP_BLOCK, "four bins per thread");
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  uint32_t c[4], local = 0, mx = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    c[j] = bcnt[4 * tid + j];
    local += c[j];
    mx = c[j] > mx ? c[j] : mx;
  }
  const uint32_t incl = pz_wave_scan_u32(local);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t o = __shfl_xor(mx, off, 64);
    mx = o > mx ? o : mx;
  }
  if (lane == 63) T.wtot[w] = incl;
  if (lane == 0) atomicMax(&T.bmax, mx);
  __syncthreads();
  uint32_t run = incl - local;
  for (int j = 0; j < w; j++) run += T.wtot[j];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    bstart[4 * tid + j] = run;
    bcnt[4 * tid + j] = run;  // cursor
    run += c[j];
  }
  __syncthreads();
  return T.bmax;
}

// Candidate terms with the e histogram (LDS, PZ_TOPP_NB bins) as observer.
template <class Row>
struct ToppTermsR : PzExpTerms<Row> {
  pz_lds_u32b* ehist;
  __device__ __forceinline__ void observe(int, const float (&)[4], const float (&a)[4]) {
#pragma unroll
    for (int c = 0; c < 4; c++)
      if (a[c] > 0.0f) atomicAdd((uint32_t*)&ehist[ebin(a[c])], 1u);
  }
};
template <bool VEC>
using ToppTerms = ToppTermsR<PzRow<VEC>>;

// A workgroup's slice of the row with the chain already applied, in LDS
// (ids from lo on): a row for the records pass that only reads LDS.
struct ToppLdsRow {
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

// Estimated mass of the slice's segments, from LDS (k from k0 on).
struct ToppSliceEst {
  const float* s;
  int k0;
  __device__ __forceinline__ float operator()(int k) const { return s[k - k0]; }
};

// The row's chain with penalty tables for the ids [lo, hi).
template <bool VEC>
__device__ __forceinline__ PzRow<VEC> topp_row(const float* logits, long ld, int row, int V,
                                              const pz_row_params_dev& prm, char* lds, int lo,
                                              int hi, int hcap, const int32_t* hist, int H) {
  PzRow<VEC> R;
  R.x = logits + (long)row * ld;
  R.V = V;
  R.T = PzTemp::of(prm);
  pz_penalty_build_range<PZ_SP_BLOCK>(R.P, lds, V, lo, hi, hcap,
                                      hist ? hist + (long)row * H : nullptr, H, prm);
  return R;
}

#define TOPP_ARGS                                                                            \
  const float *__restrict__ logits, long ld, int V, const int32_t *__restrict__ rows,        \
      const pz_row_params_dev *__restrict__ params, int n_params,                            \
      const int32_t *__restrict__ hist, int H, int hcap, int nseg, int spw, int S,           \
      PzSplitWs ws, const float *__restrict__ u, int32_t *__restrict__ ids_out,             \
      float *__restrict__ p_out, pz_scratch sc

// Rows the stat pass settles: y[0] NaN (the reference's maximum is NaN, no
// candidate passes, argmax of a row starting with NaN -> 0) and an infinite
// or absent maximum (every e is expf(NaN): the first y == max).
__device__ __forceinline__ bool topp_degenerate(uint32_t flags) {
  return (flags & (PZ_RS_Y0NAN | PZ_RS_NONFIN)) != 0;
}

// ---- pass 1 (HBM): slice maxima -------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_topp_stat(TOPP_ARGS) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  const int row = pz_row_of(rows, blockIdx.y);
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const PzSlice sl = pz_sp_slice(nseg, spw);
  if (threadIdx.x == 0) {
    SS.any = 0u;
    if (blockIdx.x == 0) ws.rs[row].i[5] = 0;  // the nucleus bins of this launch: not yet picked
    // the fallback queue, empty for this launch's later kernels (the one
    // before, k_topp_fallback, has read it: launches on a stream run in order)
    if (blockIdx.x == 0 && blockIdx.y == 0) sc.counters[0] = 0;
  }
  const PzRow<VEC> R =
      topp_row<VEC>(logits, ld, row, V, prm, lds, pz_sp_lo(sl), pz_sp_hi(sl, V), hcap, hist, H);
  __syncthreads();
  pz_sp_stat_slice(R, row, sl, ws, SS, false);
}

// ---- pass 2 (L2): estimated mass of the candidates per segment, and each --
// segment's maximum (the gather skips segments below its gate)
template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_topp_est(TOPP_ARGS) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  const int row = pz_row_of(rows, blockIdx.y);
  pz_sp_row_stat(row, S, ws, SS);
  if (topp_degenerate(SS.any)) return;
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const PzSlice sl = pz_sp_slice(nseg, spw);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const PzRow<VEC> R =
      topp_row<VEC>(logits, ld, row, V, prm, lds, pz_sp_lo(sl), pz_sp_hi(sl, V), hcap, hist, H);
  const float M = SS.M, thr = M - 20.0f;
  float* seg_s = ws.seg_s + (size_t)row * ws.nsc;
  float* seg_m = ws.seg_m + (size_t)row * ws.nsc;
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
      R.apply(k * PZ_SP_SEG + 4 * lane, n[u], y[u]);
      float t = 0.0f, mx = -__builtin_inff();
#pragma unroll
      for (int c = 0; c < 4; c++) {  // (selects)
        const float v = y[u][c];
        const bool ok = c < n[u];
        const float e = pz_fast_exp(v - M);
        t += ok && v >= thr ? e : 0.0f;
        mx = fmaxf(mx, ok && v == v ? v : -__builtin_inff());  // NaN-free maximum
      }
      t = pz_wave_sum(t);
      mx = pz_wave_max(mx);
      if (lane == 0) {
        seg_s[k] = t;
        seg_m[k] = mx;
      }
    }
  }
}

// Nucleus bins from the row's merged e histogram (one wave), given its
// estimated total mass and count: the smallest set of top bins whose
// estimated mass clears top_p by more than the histogram's resolution (a
// bin's mass is known to within half its width, 0.55 %).  bsel 0 keeps every
// candidate.  (Any choice gives the reference's result: the nucleus checks
// that its cut-off lies inside the gathered set, else the fallback runs.)
__device__ __forceinline__ void topp_select_bins(const pz_lds_u32b* ehist, float tot,
                                                 uint32_t ncand, float top_p, int* bsel_out,
                                                 uint32_t* nsel_out) {
  const int lane = threadIdx.x & 63;
  const float goal = (top_p * 1.012f + 3e-4f) * tot;
  float carry = 0.0f;
  uint32_t ccarry = 0;
  int bsel = 0;
  uint32_t nsel = ncand;
  for (int b0 = PZ_TOPP_NB - 1; b0 >= 0; b0 -= 64) {
    const int b = b0 - lane;
    float m = 0.0f;
    uint32_t c = 0;
    if (b >= 0) {
      c = ehist[b];
      m = (float)c * ebin_mid(b);
    }
    const float incl = pz_wave_scan_f32(m);
    const uint32_t cincl = pz_wave_scan_u32(c);
    const uint64_t ball = __ballot(b >= 0 && carry + incl >= goal);
    if (ball) {
      const int L = (int)__builtin_ctzll(ball);
      bsel = b0 - L;
      nsel = ccarry + pz_readlane_u32(cincl, L);
      break;
    }
    carry += pz_readlane_f32(incl, 63);
    ccarry += pz_readlane_u32(cincl, 63);
  }
  *bsel_out = bsel;
  *nsel_out = nsel;
}

// ---- pass 3 (L2): records of the exact candidate terms + mass histogram ---
template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_topp_rec(TOPP_ARGS, int pen_bytes) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ uint64_t etab[32];
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  pz_etab_fill((pz_lds_u64*)etab);
  const int row = pz_row_of(rows, blockIdx.y);
  pz_sp_row_stat(row, S, ws, SS);
  if (topp_degenerate(SS.any)) return;
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const int tid = threadIdx.x;
  const PzSlice sl = pz_sp_slice(nseg, spw);
  const float M = SS.M;
  pz_lds_u32b* ehist = (pz_lds_u32b*)(lds + pen_bytes);
  for (int i = tid; i < PZ_TOPP_NB; i += PZ_SP_BLOCK) ehist[i] = 0u;
  const PzEstAbs est{ws.seg_s + (size_t)row * ws.nsc};
  const float carry = pz_sp_prefix(est, sl.k0, SS);
  pz_sp_predict(est, carry, row, sl, ws, SS);
  ToppTerms<VEC> X;
  X.R = topp_row<VEC>(logits, ld, row, V, prm, lds, pz_sp_lo(sl), pz_sp_hi(sl, V), hcap, hist, H);
  X.M = M;
  X.thr = M - 20.0f;
  X.inv = 1.0f;
  X.as_p = false;
  X.et = et;
  X.ehist = ehist;
  __syncthreads();
  pz_sp_records(X, row, sl, ws);  // (every segment: the observer fills the histogram)
  __syncthreads();
  uint32_t* gh = ws.hist + ((size_t)blockIdx.y * S + blockIdx.x) * PZ_TOPP_NB;
  for (int i = tid; i < PZ_TOPP_NB; i += PZ_SP_BLOCK) gh[i] = ehist[i];
}

// ---- passes 1-3, the nucleus bins and the gather in one launch ------------
// For slices that fit in LDS.  Each workgroup reads its slice once and keeps
// it, the chain applied, in LDS; the row's S workgroups meet twice (for the
// row maximum, then for the estimated mass before each slice), and the
// estimates, the records, the e histogram and the gather all come from LDS.
// At a meeting each workgroup posts one 64-bit word (value and a written
// bit, so no fence orders it: a fence at agent scope writes back or
// invalidates the whole L2) and wave 0 polls the row's S words.  The
// histograms are exchanged the same way, one word per bin (written bit and
// the count).  A row's workgroups are consecutive in the launch order, each
// posts everything it owes before its first wait, and the S <= 64 of them
// fit on the device together, so every workgroup a wait depends on gets
// dispatched: the waits end.  Each wait is bounded all the same (`cap`
// polls): one that gives up posts what its workgroup still owes, marks the
// row failed (rs.i[7]) and leaves; the walk launch then returns
// PZ_ID_FAILED for the row.  (The walk launch, which follows, clears the
// words and the mark on every path.)  Every workgroup of a row merges the same histograms into the same
// nucleus bins (a fixed-order reduction), gathers its slice's candidates of
// those bins as (e, ~id) keys into the row's list (count: ws.arrive[row],
// plus TOPP_GOVER when a wave's staging overflows), and workgroup 0 records
// the bins' gate in the row state.
constexpr int TOPP_FRONT_SEGS = PZ_SP_FRONT_SEGS;  // segments of a slice held in LDS
constexpr uint32_t TOPP_HWRITTEN = 0x80000000u;
constexpr int TOPP_GOVER = 1 << 30;      // added to a row's count when its gather overflowed
constexpr int TOPP_STAGE = PZ_SP_SEG / 2;  // keys a 256-term segment of LDS stages (8 B each)

__device__ __forceinline__ uint32_t topp_hword(uint32_t count) { return TOPP_HWRITTEN | count; }

// The row's nucleus-bin selection as one word (rs.i[6], zero between
// launches): written bit, the lowest bin kept (11 bits; TOPP_SEL_FAILED: a
// wait gave up) and the candidates in the kept bins (20 bits, saturated:
// only its comparison with the list capacity matters).
constexpr uint32_t TOPP_SEL_FAILED = 0x7ffu;
__device__ __forceinline__ uint32_t topp_sel_word(uint32_t bsel, uint32_t nsel) {
  return TOPP_HWRITTEN | (bsel << 20) | (nsel < 0xfffffu ? nsel : 0xfffffu);
}

// Marks the row failed: a wait between its workgroups gave up (read and
// cleared by the walk launch).
__device__ __forceinline__ void topp_mark_failed(const PzSplitWs& ws, int row) {
  __hip_atomic_store(&ws.rs[row].i[7], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Nucleus bins of the row from its S published histograms (every thread; a
// barrier inside): the merged counts in ehist, then wave 0's fixed-order
// total and selection (every workgroup of the row gets the same bins).
// bsel < 0: a bin's wait gave up (the row is failed).
struct ToppSel {
  int bsel;
  uint32_t nsel;
};
__device__ __forceinline__ ToppSel topp_front_select(const uint32_t* hrow, int S, uint32_t cap,
                                                     pz_lds_u32b* ehist, float top_p,
                                                     ToppSel* sel_sh, float* part_sh,
                                                     int* fail_sh) {
  static_assert(PZ_TOPP_NB <= 2 * PZ_SP_BLOCK, "two bins per thread");
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const uint32_t want = TOPP_HWRITTEN;
  const uint32_t mask = TOPP_HWRITTEN;
  const int i0 = tid, i1 = tid + PZ_SP_BLOCK;
  uint32_t c0 = 0, c1 = 0;
  bool gave_up = false;
  for (int s0 = 0; s0 < S; s0 += 8) {
    uint32_t v0[8], v1[8];
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const uint32_t* h = hrow + (size_t)(s0 + q) * PZ_TOPP_NB;
      const bool in = s0 + q < S;
      v0[q] = in ? __hip_atomic_load(&h[i0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : want;
      v1[q] = in && i1 < PZ_TOPP_NB
                  ? __hip_atomic_load(&h[i1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                  : want;
    }
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const uint32_t* h = hrow + (size_t)(s0 + q) * PZ_TOPP_NB;
      for (uint32_t n = 1; (v0[q] & mask) != want && n < cap; n++) {
        __builtin_amdgcn_s_sleep(1);
        v0[q] = __hip_atomic_load(&h[i0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      for (uint32_t n = 1; (v1[q] & mask) != want && n < cap; n++) {
        __builtin_amdgcn_s_sleep(1);
        v1[q] = __hip_atomic_load(&h[i1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      gave_up |= (v0[q] & mask) != want || (v1[q] & mask) != want;
      c0 += v0[q] & 0x7fffffffu;
      c1 += v1[q] & 0x7fffffffu;
    }
  }
  ehist[i0] = c0;
  if (i1 < PZ_TOPP_NB) ehist[i1] = c1;
  if (tid == 0) sel_sh->bsel = INT_MAX;  // (the first crossing, as a position from the top)
  if (gave_up) *fail_sh = 1;
  pz_lds_barrier();
  if (*fail_sh) {
    ToppSel r;
    r.bsel = -1;
    r.nsel = 0;
    return r;
  }
  // The bins from the top down, two per thread (positions 2 tid, 2 tid + 1
  // are bins NB-1-2 tid, NB-2-2 tid): the estimated mass and count above
  // each one by a workgroup scan in a fixed order, so every workgroup of
  // the row finds the same bins.  The first position whose running mass
  // reaches the goal (as topp_select_bins): the lowest bin kept.
  const int bh = PZ_TOPP_NB - 1 - 2 * tid, bl = bh - 1;
  const uint32_t nh = bh >= 0 ? ehist[bh] : 0u, nl = bl >= 0 ? ehist[bl] : 0u;
  const float mh = bh >= 0 ? (float)nh * ebin_mid(bh) : 0.0f;
  const float ml = bl >= 0 ? (float)nl * ebin_mid(bl) : 0.0f;
  const float pm = mh + ml;
  const uint32_t pn = nh + nl;
  const float incl = pz_wave_scan_f32(pm);
  const uint32_t cincl = pz_wave_scan_u32(pn);
  if (lane == 63) {
    part_sh[w] = incl;
    part_sh[PZ_SP_WAVES + w] = __uint_as_float(cincl);
  }
  pz_lds_barrier();
  const float pw = lane < PZ_SP_WAVES ? part_sh[lane] : 0.0f;
  const uint32_t cw = lane < PZ_SP_WAVES ? __float_as_uint(part_sh[PZ_SP_WAVES + lane]) : 0u;
  const float tot = pz_wave_sum(pw);
  const uint32_t ncand = pz_wave_sum_u32(cw);
  const float wpre = pz_wave_sum(lane < w ? pw : 0.0f);
  const uint32_t cpre = pz_wave_sum_u32(lane < w ? cw : 0u);
  const float goal = (top_p * 1.012f + 3e-4f) * tot;
  const float cum_h = wpre + (incl - pm) + mh, cum_l = cum_h + ml;
  const int pos = bh >= 0 && cum_h >= goal ? 2 * tid : (bl >= 0 && cum_l >= goal ? 2 * tid + 1 : INT_MAX);
  // (positions grow with the lane: the wave's first crossing is its lowest)
  const uint64_t crossed = __ballot(pos != INT_MAX);
  if (crossed && lane == (int)__builtin_ctzll(crossed)) atomicMin(&sel_sh->bsel, pos);
  pz_lds_barrier();
  const int fp = sel_sh->bsel;
  ToppSel r;
  if (fp == INT_MAX) {  // never reached: every bin
    r.bsel = 0;
    r.nsel = ncand;
  } else {
    r.bsel = PZ_TOPP_NB - 1 - fp;
    if ((fp >> 1) == tid) sel_sh->nsel = cpre + (cincl - pn) + nh + ((fp & 1) ? nl : 0u);
    pz_lds_barrier();
    r.nsel = sel_sh->nsel;
  }
  return r;
}

template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_topp_front(TOPP_ARGS,
                                                                             int pen_bytes,
                                                                             uint32_t cap) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ uint64_t etab[32];
  __shared__ float sest[TOPP_FRONT_SEGS];
  __shared__ ToppSel sel_sh;
  __shared__ float part_sh[2 * PZ_SP_WAVES];
  __shared__ int wcnt[PZ_SP_WAVES];
  __shared__ uint32_t sgf[TOPP_FRONT_SEGS];  // the slice's predicted grids
  __shared__ int fail_sh;                     // a wait of this workgroup gave up
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  pz_etab_fill((pz_lds_u64*)etab);
  const int row = pz_row_of(rows, blockIdx.y);
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // this workgroup's slice: rotated by the row's place in the launch, so that
  // the slices' roles (slice 0 goes on past meeting 2 at once, the last one
  // merges the histograms) spread over the XCDs, which receive consecutive
  // workgroups in turn
  const int sx = (int)((blockIdx.x + blockIdx.y) % (unsigned)S);
  const PzSlice sl = pz_sp_slice_at(sx, nseg, spw);
  const int lo = pz_sp_lo(sl);
  pz_lds_u32b* ehist = (pz_lds_u32b*)(lds + pen_bytes);
  pz_lds_f32* ybuf = (pz_lds_f32*)(lds + (((size_t)pen_bytes + PZ_TOPP_NB * 4 + 15) & ~(size_t)15));
  uint64_t* meet = ws.meet + (size_t)row * 2 * ws.smax;
  if (tid == 0) {
    SS.any = 0u;
    fail_sh = 0;
  }
  // the fallback queue, empty for k_topp_walkf (the k_topp_fallback before
  // has read it: launches on a stream run in order)
  if (tid == 0 && blockIdx.x == 0 && blockIdx.y == 0) sc.counters[0] = 0;
  for (int i = tid; i < PZ_TOPP_NB; i += PZ_SP_BLOCK) ehist[i] = 0u;
  const PzRow<VEC> R =
      topp_row<VEC>(logits, ld, row, V, prm, lds, lo, pz_sp_hi(sl, V), hcap, hist, H);
  __syncthreads();
  // 1. the slice, once: chain applied, into LDS; segment and slice maxima
  float* seg_m = ws.seg_m + (size_t)row * ws.nsc;
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
      if (lane == 0) seg_m[k] = m;  // (NaN-free; the fallback skips segments by it)
      smx = fmaxf(smx, m);
    }
  }
  if (__ballot(nan) && lane == 0) atomicOr(&SS.any, 1u);
  if (lane == 0) SS.red[w] = smx;
  pz_lds_barrier();
  // (reductions over LDS words by a wave, not one thread's loop: every load
  // of a serial loop waits out the LDS latency)
  const float mm = w == 0 ? pz_wave_max(lane < PZ_SP_WAVES ? SS.red[lane] : -__builtin_inff())
                          : 0.0f;
  if (tid == 0) {
    uint32_t f = SS.any;
    ws.slice_m[(size_t)row * ws.smax + sx] = mm;
    ws.slice_f[(size_t)row * ws.smax + sx] = f;
    if (sx == 0) {
      ws.rs[row].y0 = ybuf[0];
      if (ybuf[0] != ybuf[0]) f |= PZ_RS_Y0NAN;
    }
    // meet 1: every slice's maximum and flags
    __hip_atomic_store(&meet[sx],
                       (1ull << 63) | ((uint64_t)f << 32) | (uint64_t)__float_as_uint(mm),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (w == 0) {
    uint64_t v = 1ull << 63;
    for (uint32_t n = 1;; n++) {
      if (lane < S) v = __hip_atomic_load(&meet[lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__ballot((v >> 63) == 0) == 0) break;
      if (n >= cap) {
        if (lane == 0) fail_sh = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
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
  if (fail_sh) {
    // meet 1 gave up: post what the others wait for (an empty histogram, no
    // mass), mark the row and leave
    uint32_t* gh = ws.hist + ((size_t)blockIdx.y * S + sx) * PZ_TOPP_NB;
    for (int i = tid; i < PZ_TOPP_NB; i += PZ_SP_BLOCK)
      __hip_atomic_store(&gh[i], topp_hword(0u), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
      __hip_atomic_store(&meet[ws.smax + sx], 1ull << 63, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      if (sx == S - 1)  // the others wait for its selection
        __hip_atomic_store(&ws.rs[row].i[6], (int)topp_sel_word(TOPP_SEL_FAILED, 0u),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      topp_mark_failed(ws, row);
    }
    return;
  }
  const bool degen = topp_degenerate(SS.any);
  const float M = SS.M, thr = M - 20.0f;
  // segment 0's values, for its sum after the records (wave 1 of slice 0),
  // held in registers: the gather stages keys over the slice in LDS, and the
  // row's last slice reaches it without a barrier after its records
  pz_f4 seg0 = {0.0f, 0.0f, 0.0f, 0.0f};
  if (sx == 0 && w == 1) seg0 = *(const pz_lds_f4*)(ybuf + 4 * lane);
  // 2. the estimated candidate mass of each segment (as k_topp_est) and the
  // histogram of the estimated e (the nucleus bins), the slice's total for
  // the slices after it
  if (!degen) {
    for (int k = sl.k0 + w; k < sl.k1; k += PZ_SP_WAVES) {
      const int e0 = k * PZ_SP_SEG + 4 * lane;
      int n = V - e0;
      n = n < 0 ? 0 : (n > 4 ? 4 : n);
      const pz_f4 q = *(const pz_lds_f4*)(ybuf + (e0 - lo));
      const float y[4] = {q.x, q.y, q.z, q.w};
      float t = 0.0f;
#pragma unroll
      for (int c = 0; c < 4; c++)
        if (c < n && y[c] >= thr) {
          const float ee = pz_fast_exp(y[c] - M);
          t += ee;
          atomicAdd((uint32_t*)&ehist[ebin(ee)], 1u);
        }
      t = pz_wave_sum(t);
      if (lane == 0) sest[k - sl.k0] = t;
    }
  }
  pz_lds_barrier();
  uint32_t* hrow = ws.hist + (size_t)blockIdx.y * S * PZ_TOPP_NB;
  if (!degen) {
    uint32_t* gh = hrow + (size_t)sx * PZ_TOPP_NB;
    for (int i = tid; i < PZ_TOPP_NB; i += PZ_SP_BLOCK)
      __hip_atomic_store(&gh[i], topp_hword(ehist[i]), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  static_assert(TOPP_FRONT_SEGS <= 64, "one estimate per lane");
  const float tot =
      w == 0 && !degen ? pz_wave_sum(lane < sl.k1 - sl.k0 ? sest[lane] : 0.0f) : 0.0f;
  if (tid == 0) {
    // meet 2: every slice's estimated mass
    __hip_atomic_store(&meet[ws.smax + sx], (1ull << 63) | (uint64_t)__float_as_uint(tot),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (degen) return;  // (every workgroup of the row; the words are cleared all the same)
  if (w == 0) {
    uint64_t v = 1ull << 63;
    for (uint32_t n = 1;; n++) {
      if (lane < sx)
        v = __hip_atomic_load(&meet[ws.smax + lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (__ballot((v >> 63) == 0) == 0) break;
      if (n >= cap) {
        if (lane == 0) fail_sh = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    // the estimated mass before this slice
    const float carry = pz_wave_sum(lane < sx ? __uint_as_float((uint32_t)v) : 0.0f);
    if (lane == 0) SS.carry = carry;
  }
  pz_lds_barrier();
  if (fail_sh) {  // (this workgroup's histogram and meet-2 word are posted)
    if (tid == 0) topp_mark_failed(ws, row);
    if (sx == S - 1 && tid == 0)  // the others wait for its selection
      __hip_atomic_store(&ws.rs[row].i[6], (int)topp_sel_word(TOPP_SEL_FAILED, 0u),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  // 4. the nucleus bins: the last slice merges the row's histograms (every
  // one is posted, bin by bin, before its workgroup's meet-2 word, so the
  // polls end at once) and posts the selection for the others, which take
  // it after their records -- one workgroup per row reads the S histograms
  ToppSel sel;
  if (sx == S - 1) {
    sel = topp_front_select(hrow, S, cap, ehist, prm.top_p, &sel_sh, part_sh, &fail_sh);
    if (tid == 0)
      __hip_atomic_store(&ws.rs[row].i[6],
                         (int)topp_sel_word(sel.bsel < 0 ? TOPP_SEL_FAILED : (uint32_t)sel.bsel,
                                            sel.nsel),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  pz_sp_predict(ToppSliceEst{sest, sl.k0}, SS.carry, row, sl, ws, SS, (pz_lds_u32*)sgf);
  // 3. records from LDS (as k_topp_rec)
  PzExpTerms<ToppLdsRow> X;
  X.R.y = ybuf;
  X.R.lo = lo;
  X.R.V = V;
  X.M = M;
  X.thr = thr;
  X.inv = 1.0f;
  X.as_p = false;
  X.et = et;
  pz_sp_records(X, row, sl, ws, (const pz_lds_u32*)sgf, true);
  if (sx == 0 && w == 1) {
    // the row's first segment, summed for the walk (wave 1: wave 0's first
    // thread waits for the selection meanwhile)
    const int e0 = 4 * lane;
    const int n = V - e0 < 0 ? 0 : (V - e0 > 4 ? 4 : V - e0);
    const pz_f4 q = seg0;
    const float t[4] = {0 < n ? X.exact_term(q.x) : 0.0f, 1 < n ? X.exact_term(q.y) : 0.0f,
                        2 < n ? X.exact_term(q.z) : 0.0f, 3 < n ? X.exact_term(q.w) : 0.0f};
    const float s0 = pz_seq_sum_seg4(t);
    if (lane == 0) ws.rs[row].s0 = __float_as_uint(s0);
  }
  if (sx != S - 1) {
    if (tid == 0) {
      uint32_t v = 0;
      for (uint32_t t = 1;; t++) {
        v = (uint32_t)__hip_atomic_load(&ws.rs[row].i[6], __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
        if ((v & TOPP_HWRITTEN) || t >= cap) break;
        __builtin_amdgcn_s_sleep(1);
      }
      const uint32_t b = (v >> 20) & 0x7ffu;
      sel_sh.bsel = !(v & TOPP_HWRITTEN) || b == TOPP_SEL_FAILED ? -1 : (int)b;
      sel_sh.nsel = v & 0xfffffu;
    }
    pz_lds_barrier();
    sel = sel_sh;
  }
  if (sel.bsel < 0) {
    if (tid == 0) topp_mark_failed(ws, row);
    return;
  }
  const bool all = sel.bsel == 0;
  const float e_gate = all ? 0.0f : ebin_lo(sel.bsel);
  const float dgate = all ? -__builtin_inff() : __logf(e_gate) - 0.01f;
  if (sx == 0 && tid == 0) {
    PzRowState& rs = ws.rs[row];
    rs.M = M;
    rs.f[0] = e_gate;
    rs.f[1] = dgate;
    rs.i[1] = all ? 1 : 0;
    rs.i[4] = (int)sel.nsel;
  }
  if (sel.nsel > (uint32_t)ws.capg) return;  // too many for the LDS sort: the fallback
  // 5. the gather: candidates with e >= e_lo = e_gate (1 - 2^-21) (a superset
  // gate on y - M first; exact e per candidate).  Any e below that bound has
  // fl(e * inv) < fl(e_gate * inv) (two roundings of 2^-24 cannot close a
  // 2^-21 gap), so every candidate with p >= fl(e_gate * inv) is gathered.
  // Each wave stages its keys over its own segments of the LDS slice (read
  // into registers first), then the workgroup appends them with one atomic.
  const float e_lo = e_gate * (1.0f - 0x1p-21f);
  constexpr int WSEG = TOPP_FRONT_SEGS / PZ_SP_WAVES;  // segments a wave owns (k0 + w + 16 j)
  float yv[WSEG][4];
  int nv[WSEG];
  int cap_w = 0;  // keys the wave can stage: TOPP_STAGE per segment it owns
#pragma unroll
  for (int j = 0; j < WSEG; j++) {
    const int k = sl.k0 + w + PZ_SP_WAVES * j;
    nv[j] = 0;
    if (k < sl.k1) {
      cap_w += TOPP_STAGE;
      const int e0 = k * PZ_SP_SEG + 4 * lane;
      int n = V - e0;
      nv[j] = n < 0 ? 0 : (n > 4 ? 4 : n);
      const pz_f4 q = *(const pz_lds_f4*)(ybuf + (e0 - lo));
      yv[j][0] = q.x;
      yv[j][1] = q.y;
      yv[j][2] = q.z;
      yv[j][3] = q.w;
    }
  }
  asm volatile("" ::: "memory");  // the wave's reads of its segments come before its staging
  int cnt = 0;  // keys this wave staged (wave-uniform)
  bool over = false;
#pragma unroll
  for (int j = 0; j < WSEG; j++) {
    const int k = sl.k0 + w + PZ_SP_WAVES * j;
    if (k >= sl.k1) break;
    const int e0 = k * PZ_SP_SEG + 4 * lane;
    uint32_t want = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const bool wnt = (c < nv[j]) & (yv[j][c] >= thr) & ((yv[j][c] - M) >= dgate);
      want |= (wnt ? 1u : 0u) << c;
    }
    while (__ballot(want != 0u)) {
      bool take = false;
      uint64_t key = 0;
      if (want) {
        const uint32_t c = (uint32_t)__builtin_ctz(want);
        want &= want - 1u;
        const float yy = pz_sel4f(yv[j][0], yv[j][1], yv[j][2], yv[j][3], (int)c);
        const float e = pz_expf_l(yy - M, et);
        take = e >= e_lo;
        key = topp_key(e, e0 + (int)c);
      }
      const uint64_t ball = __ballot(take);
      if (take) {
        const int slot = cnt + __popcll(ball & ((1ull << lane) - 1ull));
        if (slot < cap_w) {
          // slot q of the wave: segment k0 + w + 16 (q / TOPP_STAGE), key q % TOPP_STAGE
          const int ks = sl.k0 + w + PZ_SP_WAVES * (slot / TOPP_STAGE);
          ((pz_lds_u64*)(ybuf + (ks - sl.k0) * PZ_SP_SEG))[slot % TOPP_STAGE] = key;
        }
      }
      cnt += __popcll(ball);
    }
  }
  if (cnt > cap_w) {
    over = true;
    cnt = cap_w;
  }
  if (lane == 0) wcnt[w] = cnt | (over ? TOPP_GOVER : 0);
  pz_lds_barrier();
  // every wave reads the 16 counts once (one lane each): its offset among
  // the workgroup's keys, and (wave 0) the total and the overflow flag
  const int wc = lane < PZ_SP_WAVES ? wcnt[lane] : 0;
  const uint32_t before = pz_wave_sum_u32(lane < w ? (uint32_t)(wc & (TOPP_GOVER - 1)) : 0u);
  if (w == 0) {
    const uint32_t gtot = pz_wave_sum_u32((uint32_t)(wc & (TOPP_GOVER - 1)));
    const bool ov = __ballot((wc & TOPP_GOVER) != 0) != 0;
    if (lane == 0) {
      SS.cnt = gtot > 0 ? (int)atomicAdd(&ws.arrive[row], gtot) : 0;
      if (ov) atomicOr(&ws.arrive[row], (uint32_t)TOPP_GOVER);
    }
  }
  pz_lds_barrier();
  const int base = (SS.cnt & (TOPP_GOVER - 1)) + (int)before;
  uint64_t* gkeys = ws.keys + (size_t)row * ws.capg;
  for (int q = lane; q < cnt; q += 64) {
    if (base + q >= ws.capg) break;  // (the count tells the walk the list overflowed)
    const int ks = sl.k0 + w + PZ_SP_WAVES * (q / TOPP_STAGE);
    gkeys[base + q] = ((const pz_lds_u64*)(ybuf + (ks - sl.k0) * PZ_SP_SEG))[q % TOPP_STAGE];
  }
}

// Gather of one slice: candidates with e >= e_lo (1 - 2^-21) (a superset
// gate on y - M first, 0.01 below the bin edge; each possible candidate's
// exact e one per lane per trip), staged as (e, ~id) keys in LDS (lkeys,
// capacity lcap; one LDS atomic per wave and trip) and appended to the row's
// list with one global atomic per workgroup.  Any e below that bound has
// fl(e * inv) < fl(e_lo * inv) (two roundings of 2^-24 cannot close a 2^-21
// gap), so every candidate with p >= p_lo = fl(e_lo * inv) is gathered.
template <bool VEC>
__device__ __forceinline__ void topp_gather_slice(TOPP_ARGS, int row, int slice, int gspw,
                                                  char* lds, pz_lds_u64* lkeys, int lcap,
                                                  const pz_lds_u64* et, PzSpShared& SS,
                                                  uint32_t cap) {
  __shared__ int ready_sh;
  pz_sp_row_stat(row, S, ws, SS);
  if (topp_degenerate(SS.any)) return;
  // the row's nucleus bins, picked by the walking workgroup of this launch
  // (it has a lower block index, so it was dispatched first, and it waits on
  // nothing here: the wait ends; bounded all the same -- a gather that gives
  // up marks the row failed, which the nucleus launch reports)
  // (relaxed polls -- an acquire per poll would invalidate the L2 the walks
  // read from -- then one acquire)
  if (threadIdx.x == 0) {
    int ready = 0;
    for (uint32_t n = 1;; n++) {
      ready = __hip_atomic_load(&ws.rs[row].i[5], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (ready != 0 || n >= cap) break;
      __builtin_amdgcn_s_sleep(8);
    }
    if (ready) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    else topp_mark_failed(ws, row);
    ready_sh = ready;
  }
  __syncthreads();
  if (!ready_sh) return;
  const PzRowState rs0 = ws.rs[row];
  if (rs0.i[0] == TP_DONE) return;
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const PzSlice sl = pz_sp_slice_at(slice, nseg, gspw);
  const float M = rs0.M, thr = M - 20.0f;
  const float e_lo = rs0.f[0] * (1.0f - 0x1p-21f), dgate = rs0.f[1];
  PzRowState& rs = ws.rs[row];
  uint64_t* gkeys = ws.keys + (size_t)row * ws.capg;
  const float* seg_m = ws.seg_m + (size_t)row * ws.nsc;
  const PzRow<VEC> R =
      topp_row<VEC>(logits, ld, row, V, prm, lds, pz_sp_lo(sl), pz_sp_hi(sl, V), hcap, hist, H);
  if (threadIdx.x == 0) {
    SS.cnt = 0;
    SS.flag = 0;
  }
  __syncthreads();  // the penalty tables, the staging count
  for (int kb = sl.k0 + w; kb < sl.k1; kb += PZ_SP_U * PZ_SP_WAVES) {
    float ys[PZ_SP_U][4];
    int ns[PZ_SP_U];
#pragma unroll
    for (int u = 0; u < PZ_SP_U; u++) {
      // a segment whose maximum is below the gate holds no candidate
      const int k = kb + u * PZ_SP_WAVES;
      ns[u] = k < sl.k1 && !(seg_m[k] - M < dgate)
                  ? R.load(k * PZ_SP_SEG + 4 * lane, ys[u]) : 0;
    }
#pragma unroll
    for (int u = 0; u < PZ_SP_U; u++) {
      const int k = kb + u * PZ_SP_WAVES;
      if (k >= sl.k1) break;
      const int e0 = k * PZ_SP_SEG + 4 * lane;
      float (&y)[4] = ys[u];
      const int n = ns[u];
      R.apply(e0, n, y);
      uint32_t want = 0;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const bool wnt = (c < n) & (y[c] >= thr) & ((y[c] - M) >= dgate);
        want |= (wnt ? 1u : 0u) << c;
      }
      while (__ballot(want != 0u)) {
        bool take = false;
        uint64_t key = 0;
        if (want) {
          const uint32_t j = (uint32_t)__builtin_ctz(want);
          want &= want - 1u;
          const float yy = j == 0 ? y[0] : (j == 1 ? y[1] : (j == 2 ? y[2] : y[3]));
          const float e = pz_expf_l(yy - M, et);
          take = e >= e_lo;
          key = topp_key(e, e0 + (int)j);
        }
        const uint64_t ball = __ballot(take);
        if (ball) {
          const int leader = (int)__builtin_ctzll(ball);
          int base = 0;
          if (lane == leader) base = atomicAdd(&SS.cnt, __popcll(ball));
          base = __builtin_amdgcn_readlane(base, leader);
          if (take) {
            const int slot = base + __popcll(ball & ((1ull << lane) - 1ull));
            if (slot < lcap) lkeys[slot] = key;
            else SS.flag = 1;
          }
        }
      }
    }
  }
  __syncthreads();
  const int n = SS.cnt < lcap ? SS.cnt : lcap;
  if (threadIdx.x == 0) {
    SS.carry = __int_as_float(n > 0 ? atomicAdd(&rs.i[2], n) : 0);
    if (SS.flag) rs.i[3] = 1;
  }
  __syncthreads();
  const int base = __float_as_int(SS.carry);
  bool over = false;
  for (int i = threadIdx.x; i < n; i += PZ_SP_BLOCK) {
    if (base + i < ws.capg) gkeys[base + i] = lkeys[i];
    else over = true;
  }
  if (over) rs.i[3] = 1;
}

// ---- pass 4: the exact normaliser (one workgroup per row) beside the ------
// gather (gS workgroups per row, slices of gspw segments), in one launch:
// blocks [0, rows) walk, blocks [rows, rows + rows * gS) gather.  A gather
// block waits only for its row's nucleus bins, which the walking block picks
// early; the gather keys carry e, not p, so nothing waits for the
// normaliser.  Each block takes a CU of its own (the walk's LDS), so gS is
// sized for the gather to run in one round beside the walks.
template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) void k_topp_walk(TOPP_ARGS, int pen_bytes, int nc,
                                                          int n_rows, int gS, int gspw,
                                                          int goff, int lcap, uint32_t cap) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ int first_sh, merged_sh;
  __shared__ float sum_sh, tot_sh;
  __shared__ uint32_t ncand_sh;
  __shared__ uint64_t etab[32];
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  pz_etab_fill((pz_lds_u64*)etab);
  if ((int)blockIdx.x >= n_rows) {
    const int g = (int)blockIdx.x - n_rows;
    topp_gather_slice<VEC>(logits, ld, V, rows, params, n_params, hist, H, hcap, nseg, spw, S,
                           ws, u, ids_out, p_out, sc, pz_row_of(rows, g / gS), g % gS, gspw,
                           lds, (pz_lds_u64*)(lds + goff), lcap, et, SS, cap);
    return;
  }
  const int row = pz_row_of(rows, blockIdx.x);
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const int tid = threadIdx.x;
  // k_topp_front's meetings are over: clear the row's words
  for (int i = tid; i < 2 * ws.smax; i += PZ_SP_BLOCK)
    __hip_atomic_store(&ws.meet[(size_t)row * 2 * ws.smax + i], 0ull, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  pz_sp_row_stat(row, S, ws, SS);
  const float M = SS.M;
  const uint32_t flags = SS.any;
  PzRowState& rs = ws.rs[row];
  const PzRow<VEC> R = topp_row<VEC>(logits, ld, row, V, prm, lds, 0, V, hcap, hist, H);
  __syncthreads();  // the expf table
  if (flags & PZ_RS_Y0NAN) {
    if (tid == 0) {
      ids_out[row] = 0;
      if (p_out) p_out[row] = 1.0f;
      rs.i[0] = TP_DONE;
    }
    return;
  }
  if (flags & PZ_RS_NONFIN) {
    if (tid == 0) first_sh = INT_MAX;
    __syncthreads();
    int mine = INT_MAX;
    for (int e0 = 4 * tid; e0 < V; e0 += 4 * PZ_SP_BLOCK) {
      float y[4];
      const int n = R.get(e0, y);
      for (int c = 0; c < n; c++)
        if (y[c] == M && e0 + c < mine) mine = e0 + c;
    }
    atomicMin(&first_sh, mine);
    __syncthreads();
    if (tid == 0) {
      ids_out[row] = first_sh;
      if (p_out) p_out[row] = __builtin_nanf("");
      rs.i[0] = TP_DONE;
    }
    return;
  }
  PzExpTerms<PzRow<VEC>> X;
  X.R = R;
  X.M = M;
  X.thr = M - 20.0f;
  X.inv = 1.0f;
  X.as_p = false;
  X.et = et;
  pz_lds_u32b* ehist = (pz_lds_u32b*)(lds + pen_bytes);
  const size_t walk_off = ((size_t)pen_bytes + PZ_TOPP_NB * 4 + 15) & ~(size_t)15;
  const int w = tid >> 6;
  if (tid == 0) {
    merged_sh = 0;
    tot_sh = 0.0f;
    ncand_sh = 0u;
  }
  // waves 1..7 pre-evaluate the walk's specials while waves 8..15 merge the
  // row's histograms and wave 8 picks the nucleus bins for this launch's
  // gather
  const PzWalk W = pz_sp_walk_setup(X, row, nseg, nc, ws, lds + walk_off, SS, 7);
  if (w == 0) {
    PzAcc st;
    pz_sp_walk<PZ_STOP_NONE>(st, W, 0.0f, X);
    if (tid == 0) sum_sh = pz_acc_value(st);
  } else if (w >= 8) {
    // merged histogram (every load of a bin issued before its sum), with
    // the estimated total mass and count on the side
    const uint32_t* hrow = ws.hist + (size_t)blockIdx.x * S * PZ_TOPP_NB;
    float tot = 0.0f;
    uint32_t ncand = 0;
    for (int i = tid - 512; i < PZ_TOPP_NB; i += PZ_SP_BLOCK - 512) {
      uint32_t c = 0;
      int s2 = 0;
      for (; s2 + 4 <= S; s2 += 4) {
        const uint32_t c0 = hrow[(size_t)s2 * PZ_TOPP_NB + i];
        const uint32_t c1 = hrow[(size_t)(s2 + 1) * PZ_TOPP_NB + i];
        const uint32_t c2 = hrow[(size_t)(s2 + 2) * PZ_TOPP_NB + i];
        const uint32_t c3 = hrow[(size_t)(s2 + 3) * PZ_TOPP_NB + i];
        c += (c0 + c1) + (c2 + c3);
      }
      for (; s2 < S; s2++) c += hrow[(size_t)s2 * PZ_TOPP_NB + i];
      ehist[i] = c;
      tot += (float)c * ebin_mid(i);
      ncand += c;
    }
    tot = pz_wave_sum(tot);
    ncand = pz_wave_sum_u32(ncand);
    if ((tid & 63) == 0) {
      atomicAdd(&tot_sh, tot);
      atomicAdd(&ncand_sh, ncand);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if ((tid & 63) == 0)
      __hip_atomic_fetch_add(&merged_sh, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (w == 8) {
      while (__hip_atomic_load(&merged_sh, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < 8)
        __builtin_amdgcn_s_sleep(1);
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      int bsel;
      uint32_t nsel;
      topp_select_bins(ehist, tot_sh, ncand_sh, prm.top_p, &bsel, &nsel);
      if (tid == 512) {
        const bool all = bsel == 0;
        const float e_lo = ebin_lo(bsel);
        rs.M = M;
        rs.f[0] = all ? 0.0f : e_lo;
        rs.f[1] = all ? -__builtin_inff() : __logf(e_lo) - 0.01f;
        rs.i[1] = all ? 1 : 0;
        rs.i[2] = 0;
        rs.i[3] = 0;
        rs.i[4] = (int)nsel;
        if (nsel > (uint32_t)ws.capg) {
          // the selected set cannot fit: straight to the fallback
          const int q = atomicAdd(&sc.counters[0], 1);
          sc.fb_list[q] = row;
          rs.i[0] = TP_DONE;
        } else {
          rs.i[0] = TP_OPEN;
        }
        __hip_atomic_store(&rs.i[5], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    rs.sum = sum_sh;
    rs.inv = 1.0f / sum_sh;  // top_p.c:72
  }
}

// The sorted probabilities (p of bkeys[perm[j]], j < m, 0 past m) for the
// walk over the sorted list.
struct SortedSeg {
  const pz_lds_u64* bkeys;
  const pz_lds_u16* perm;
  int m;
  __device__ __forceinline__ uint64_t key(int j) const { return bkeys[perm[j]]; }
  __device__ __forceinline__ void seg(int k, float (&v)[4]) const {
    const int j0 = k * PZ_SP_SEG + 4 * ((int)threadIdx.x & 63);
#pragma unroll
    for (int c = 0; c < 4; c++) v[c] = j0 + c < m ? key_p(bkeys[perm[j0 + c]]) : 0.0f;
  }
};
// The same over a sorted key list in global memory.
struct GSortedSeg {
  const uint64_t* keys;
  int m;
  __device__ __forceinline__ uint64_t key(int j) const { return keys[j]; }
  __device__ __forceinline__ void seg(int k, float (&v)[4]) const {
    const int j0 = k * PZ_SP_SEG + 4 * ((int)threadIdx.x & 63);
#pragma unroll
    for (int c = 0; c < 4; c++) v[c] = j0 + c < m ? key_p(keys[j0 + c]) : 0.0f;
  }
};

// The cut-off and the draw over a list X of m keys sorted by (p desc, id
// asc), by every thread of the workgroup: records of the list (the row's
// record area, free once the row's normaliser is known), an exact-sum walk
// to the first running sum >= top_p -- the cut-off and the truncated mass
// (top_p.c:80-93) -- and a second walk, resumed from the first one's
// checkpoints, to the first running sum > u * trunc_sum (:96-105).  all: the
// list holds every candidate (a cumulative that never reaches top_p keeps
// all, :81); otherwise a cut-off term below p_lo, or none inside the list,
// means the list is too short.  Returns the picked index or -1 (too short).
template <class X>
__device__ __forceinline__ int nucleus_pick(const X& xs, int m, int row0, float top_p, float uu,
                                            bool all, float p_lo, int nc, char* region,
                                            const PzSplitWs& ws0, PzSpShared& SS, int* pick_sh,
                                            char* lrec = nullptr) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nsl = (m + PZ_SP_SEG - 1) / PZ_SP_SEG;
  // the list's segment estimates and records: in LDS when the caller has
  // room for them (lrec, 16 bytes per segment), else the row's global ones
  PzSplitWs ws = ws0;
  int row = row0;
  if (lrec) {
    ws.seg_s = reinterpret_cast<float*>(lrec);
    ws.rec = reinterpret_cast<uint32_t*>(lrec + (size_t)nsl * 4);
    ws.nsc = nsl;
    row = 0;
  }
  float* est = ws.seg_s + (size_t)row * ws.nsc;
  for (int k = w; k < nsl; k += PZ_SP_WAVES) {
    float v[4];
    xs.seg(k, v);
    const float t = pz_wave_sum((v[0] + v[1]) + (v[2] + v[3]));
    // (segment 0: also its sequential sum from zero, for the first walk)
    const float s0 = k == 0 ? pz_seq_sum_seg4(v) : 0.0f;
    if (lane == 0) {
      est[k] = t;
      if (k == 0) SS.s0 = __float_as_uint(s0);
    }
  }
  __syncthreads();
  PzSlice sl;
  sl.k0 = 0;
  sl.k1 = nsl;
  pz_sp_predict(PzEstAbs{est}, 0.0f, row, sl, ws, SS);
  {
    uint32_t* rd = pz_sp_rec_d(ws, row);
    uint32_t* rd2 = pz_sp_rec_d2(ws, row);
    uint32_t* rgf = pz_sp_rec_gf(ws, row);
    for (int k = w; k < nsl; k += PZ_SP_WAVES) {
      float v[4];
      xs.seg(k, v);
      const uint32_t gf = rgf[k];
      const uint32_t g = gf & 0xffu;
      const bool has2 = (gf & PZ_GF_HAS2) != 0;
      uint32_t s1 = 0, s2 = 0;
      bool d1 = false, d2 = false;
#pragma unroll
      for (int cc = 0; cc < 4; cc++) {
        uint32_t cls;
        s1 += pz_inc(v[cc], g, &cls);
        d1 |= cls != PZ_INC_PLAIN;
        if (has2) {
          s2 += pz_inc(v[cc], g - 1u, &cls);
          d2 |= cls != PZ_INC_PLAIN;
        }
      }
      s1 = pz_wave_sum_u32(s1);
      s2 = pz_wave_sum_u32(s2);
      const bool D1 = __ballot(d1) != 0, D2 = has2 && __ballot(d2) != 0;
      if (lane == 0) {
        rd[k] = s1;
        rd2[k] = s2;
        rgf[k] = gf | (D1 ? PZ_GF_DIRTY : 0u) | (D2 ? PZ_GF_DIRTY2 : 0u);
      }
    }
  }
  __syncthreads();
  const PzWalk W = pz_sp_walk_setup(xs, row, nsl, nc, ws, region, SS, -1, SS.s0);
  if (w == 0) {
    PzAcc st;
    PzWalkCk ck;
    const int hit = pz_sp_walk<PZ_STOP_GE>(st, W, top_p, xs, &ck);
    int cutoff = hit >= 0 && hit < m ? hit + 1 : -1;
    if (cutoff < 0 && all) cutoff = m;  // st then holds the whole sum
    if (cutoff > 0 && !all && !(key_p(xs.key(cutoff - 1)) >= p_lo)) cutoff = -1;
    int pick = -1;
    if (cutoff > 0) {
      const float r = uu * pz_acc_value(st);  // trunc_sum: the cumulative at the cut-off
      PzAcc s2;
      const int d = pz_sp_walk<PZ_STOP_GT>(s2, W, r, xs, nullptr, &ck);
      pick = d >= 0 && d < cutoff ? d : 0;
    }
    if (lane == 0) *pick_sh = pick;
  }
  __syncthreads();
  return *pick_sh;
}

// ---- pass 6 (one workgroup per row): order, cut-off and draw ------------
// The gathered keys are counted into bins of p (1/128 binade) straight from
// global memory and scattered into LDS in bin order; each key's rank inside
// its bin (independent reads, no chains) gives the (p desc, id asc) order;
// the cumulative over that order is an exact-sum walk (records of the
// sorted list, pz_sp_walk): first running sum >= top_p is the cut-off and
// its sum the truncated mass (top_p.c:80-93); a second walk over the same
// records stops at the first running sum > r (:96-105).
template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) void k_topp_nucleus(TOPP_ARGS, int cap, int nc) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ ToppShared T;
  const int row = pz_row_of(rows, blockIdx.x);
  const PzRowState rs0 = ws.rs[row];
  if (rs0.i[7]) {
    // a gather's wait gave up: the list is incomplete (a row the walk
    // settled, or queued for the fallback, keeps that result)
    if (threadIdx.x == 0) {
      ws.rs[row].i[7] = 0;
      if (rs0.i[0] != TP_DONE) {
        ids_out[row] = PZ_ID_FAILED;
        if (p_out) p_out[row] = __builtin_nanf("");
      }
    }
    return;
  }
  if (rs0.i[0] == TP_DONE) return;
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const int tid = threadIdx.x;
  const int m = rs0.i[2];
  const bool all = rs0.i[1] != 0;
  const uint64_t* gkeys = ws.keys + (size_t)row * ws.capg;
  const float inv = rs0.inv;
  // Every candidate with p >= p_lo = fl(e_lo * inv) was gathered (p is
  // monotone in e; the gather keeps a margin below e_lo), so the sorted list
  // is the reference's order down to p_lo, and a cut-off whose last term
  // lies at or above p_lo only ever saw reference terms (else: the fallback).
  const float p_lo = rs0.f[0] * inv;
  bool done = false, sorted = false;  // sorted: the whole list, cut-off checked
  if (rs0.i[3] == 0 && m <= cap && m > 0) {
    pz_lds_u64* bkeys = (pz_lds_u64*)lds;                          // [cap]
    pz_lds_u16* perm = (pz_lds_u16*)(lds + (size_t)cap * 8);       // [cap]
    char* region = lds + (((size_t)cap * 10 + 15) & ~(size_t)15);  // bins, then the walk
    pz_lds_u32b* bcnt = (pz_lds_u32b*)region;
    pz_lds_u32b* bstart = bcnt + PBINS;
    if (m < TOPP_BINSORT_MIN) {
      // small lists: bitonic sort of the keys, then the lane-ordered walks
      int N = 1;
      while (N < m) N <<= 1;
      for (int i = tid; i < N; i += PZ_SP_BLOCK) bkeys[i] = i < m ? topp_pkey(gkeys[i], inv) : 0ull;
      __syncthreads();
      pz_bitonic_desc<PZ_SP_BLOCK>(bkeys, N);
      uint64_t* kk = reinterpret_cast<uint64_t*>(lds);
      float* cum = reinterpret_cast<float*>(region);
      const int cutoff = nucleus_cutoff(kk, cum, m, prm.top_p, all, &T.cutoff);
      if (cutoff > 0 && (all || key_p(kk[cutoff - 1]) >= p_lo)) {
        if (tid == 0)
          nucleus_draw(kk, cum, cutoff, u[row], &ids_out[row], p_out ? &p_out[row] : nullptr);
        done = true;
      }
      sorted = true;
    } else {
      for (int i = tid; i < PBINS; i += PZ_SP_BLOCK) bcnt[i] = 0u;
      if (tid == 0) T.bmax = 0u;
      __syncthreads();
      for (int i = tid; i < m; i += PZ_SP_BLOCK)
        atomicAdd((uint32_t*)&bcnt[pbin(topp_pkey(gkeys[i], inv))], 1u);
      __syncthreads();
      const bool binned = topp_bin_starts(bcnt, bstart, T) <= (uint32_t)TOPP_BIN_MAX;
      if (binned) {
        for (int i = tid; i < m; i += PZ_SP_BLOCK) {
          const uint64_t key = topp_pkey(gkeys[i], inv);
          const uint32_t pos = atomicAdd((uint32_t*)&bcnt[pbin(key)], 1u);
          bkeys[pos] = key;
        }
        __syncthreads();
        // rank inside the bin: every comparison independent of the others
        for (int j = tid; j < m; j += PZ_SP_BLOCK) {
          const uint64_t key = bkeys[j];
          const int q = pbin(key);
          const uint32_t b0 = bstart[q], b1 = bcnt[q];
          uint32_t r = 0, x = b0;
          for (; x + 4 <= b1; x += 4) {
            const uint64_t k0 = bkeys[x], k1 = bkeys[x + 1], k2 = bkeys[x + 2], k3 = bkeys[x + 3];
            r += (k0 > key ? 1u : 0u) + (k1 > key ? 1u : 0u) + (k2 > key ? 1u : 0u) +
                 (k3 > key ? 1u : 0u);
          }
          for (; x < b1; x++) r += bkeys[x] > key ? 1u : 0u;
          perm[b0 + r] = (uint16_t)j;
        }
        __syncthreads();
        SortedSeg X;
        X.bkeys = bkeys;
        X.perm = perm;
        X.m = m;
        nucleus_pick(X, m, row, prm.top_p, u[row], all, p_lo, nc, region, ws, SS, &T.cutoff);
        if (T.cutoff >= 0) {
          if (tid == 0) {
            const uint64_t k = bkeys[perm[T.cutoff]];
            ids_out[row] = key_id(k);
            if (p_out) p_out[row] = key_p(k);
          }
          done = true;
        }
        sorted = true;
      } else if (m <= TOPP_BITONIC_MAX) {
        // a bin too large for the rank count: bitonic sort of the whole list
        __syncthreads();
        int N = 1;
        while (N < m) N <<= 1;
        for (int i = tid; i < N; i += PZ_SP_BLOCK) bkeys[i] = i < m ? topp_pkey(gkeys[i], inv) : 0ull;
        __syncthreads();
        pz_bitonic_desc<PZ_SP_BLOCK>(bkeys, N);
        uint64_t* kk = reinterpret_cast<uint64_t*>(lds);
        float* cum = reinterpret_cast<float*>(region);
        const int cutoff = nucleus_cutoff(kk, cum, m, prm.top_p, all, &T.cutoff);
        if (cutoff > 0 && (all || key_p(kk[cutoff - 1]) >= p_lo)) {
          if (tid == 0)
            nucleus_draw(kk, cum, cutoff, u[row], &ids_out[row], p_out ? &p_out[row] : nullptr);
          done = true;
        }
        sorted = true;
      }
    }
  }
  if (!done && tid == 0) {
    if (sorted) {
      // the whole gathered list was sorted: the cut-off lies past it
      ws.rs[row].f[0] = 0.0f;
      ws.rs[row].i[1] = 1;
    }
    const int q = atomicAdd(&sc.counters[0], 1);
    sc.fb_list[q] = row;
  }
}

// Fallback, one workgroup per queued row at a time (rows whose selected set
// overflowed the gather or the nucleus kernel's LDS, or whose cut-off lies
// outside it): the candidates with e at or above the row's gate -- every
// candidate when the gate is 0 -- as (p, ~id) keys in the workgroup's global
// slot; a counting sort by p bin into the second slot, then each key's rank
// inside its bin (bins above TOPP_BIN_MAX keys: a bitonic sort in LDS; a bin
// beyond the LDS buffer: one global bitonic sort of the whole list) back into
// the first, which then holds the reference's order; then nucleus_pick.  A
// gated list too short for the cut-off is gathered again with gate 0.
constexpr int FB_NC = 8;                                // pre-evaluated segments of its walk
constexpr int FB_U = 8;                                 // segments a wave loads at once
constexpr int FB_LBUF = 8192;                           // keys of its LDS bin sort
constexpr int FB_BIG = 1024;  // bins above TOPP_BIN_MAX it lists (slot_n / 257 < FB_BIG)
// bins, starts, the big-bin list and its chunk starts
constexpr size_t FB_HEAD = (size_t)PBINS * 8 + (size_t)FB_BIG * 8 + 16;

// One pass of the fallback over row with the given gate (the workgroup's
// slot: blockIdx.x).  Returns false when the gated list is too short for the
// cut-off.  (Inlined: a kernel that calls a function launches slower, even
// when the queue is empty.)
template <bool VEC>
__device__ __forceinline__ bool fb_pass(const float* __restrict__ logits, long ld, int V,
                                     const pz_row_params_dev* __restrict__ params, int n_params,
                                     const int32_t* __restrict__ hist, int H, int hcap, int nseg,
                                     const PzSplitWs& ws, const float* __restrict__ u,
                                     int32_t* __restrict__ ids_out, float* __restrict__ p_out,
                                     const pz_scratch& sc, int row, float gate, int slot,
                                     float M, float inv, float rdgate) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ ToppShared T;
  __shared__ uint64_t etab[32];
  __shared__ int nbig, nchunks;
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  uint64_t* keys = sc.fb_keys + (size_t)slot * sc.slot_n;
  uint64_t* keys2 = sc.fb_keys2 + (size_t)slot * sc.slot_n;
  // after the gather: bin counts (then cursors, then ends), bin starts, the
  // big-bin list, then the LDS sort buffer or the walk
  pz_lds_u32b* bcnt = (pz_lds_u32b*)lds;
  pz_lds_u32b* bstart = bcnt + PBINS;
  pz_lds_u32b* big = bstart + PBINS;
  pz_lds_u32b* chs = big + FB_BIG;
  char* region = lds + FB_HEAD;
  pz_lds_u64* sbuf = (pz_lds_u64*)region;
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const float thr = M - 20.0f;
  const float* seg_m = ws.seg_m + (size_t)row * ws.nsc;
  __syncthreads();  // the previous pass's LDS is free
  pz_etab_fill((pz_lds_u64*)etab);
  const bool all = gate == 0.0f;
  // gathered: every e >= e_lo, so every p >= p_lo = fl(gate * inv) (p is
  // monotone in e); dgate skips the expf of terms far below the gate
  const float e_lo = gate * (1.0f - 0x1p-21f), p_lo = gate * inv;
  const float dgate = all ? -__builtin_inff() : rdgate;
  const PzRow<VEC> R = topp_row<VEC>(logits, ld, row, V, prm, lds, 0, V, hcap, hist, H);
  if (tid == 0) SS.cnt = 0;
  __syncthreads();
  // each wave: segments w + 16 j; which of its next 64 hold a term at or
  // above the gate, from one load per lane, then FB_U row loads in flight
  for (int kb = w; kb < nseg; kb += 64 * PZ_SP_WAVES) {
    const int kl = kb + lane * PZ_SP_WAVES;
    uint64_t todo = __ballot(kl < nseg && !(seg_m[kl < nseg ? kl : 0] - M < dgate));
    while (todo) {
      int ks[FB_U], ns[FB_U];
      float ys[FB_U][4];
#pragma unroll
      for (int uu = 0; uu < FB_U; uu++) {
        ks[uu] = -1;
        ns[uu] = 0;
        if (todo) {
          const int j = (int)__builtin_ctzll(todo);
          todo &= todo - 1ull;
          ks[uu] = kb + j * PZ_SP_WAVES;
          ns[uu] = R.load(ks[uu] * PZ_SP_SEG + 4 * lane, ys[uu]);
        }
      }
#pragma unroll
      for (int uu = 0; uu < FB_U; uu++) {
        if (ks[uu] < 0) break;
        const int e0 = ks[uu] * PZ_SP_SEG + 4 * lane;
        float (&y)[4] = ys[uu];
        const int n = ns[uu];
        R.apply(e0, n, y);
        uint32_t want = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const bool wnt = (c < n) & (y[c] >= thr) & ((y[c] - M) >= dgate);
          want |= (wnt ? 1u : 0u) << c;
        }
        while (__ballot(want != 0u)) {
          bool take = false;
          uint64_t key = 0;
          if (want) {
            const uint32_t j = (uint32_t)__builtin_ctz(want);
            want &= want - 1u;
            const float yy = j == 0 ? y[0] : (j == 1 ? y[1] : (j == 2 ? y[2] : y[3]));
            const float e = pz_expf_l(yy - M, et);
            take = e >= e_lo;
            key = topp_key(e * inv, e0 + (int)j);  // top_p.c:72-74
          }
          const uint64_t ball = __ballot(take);
          if (ball) {
            const int leader = (int)__builtin_ctzll(ball);
            int base = 0;
            if (lane == leader) base = atomicAdd(&SS.cnt, __popcll(ball));
            base = __builtin_amdgcn_readlane(base, leader);
            // (slot_n >= V: every candidate fits)
            if (take) keys[base + __popcll(ball & ((1ull << lane) - 1ull))] = key;
          }
        }
      }
    }
  }
  __syncthreads();  // the keys, their count; the penalty tables are free
  const int m = SS.cnt;
  for (int i = tid; i < PBINS; i += PZ_SP_BLOCK) bcnt[i] = 0u;
  if (tid == 0) {
    T.bmax = 0u;
    nbig = 0;
  }
  __syncthreads();
  for (int i = tid; i < m; i += PZ_SP_BLOCK) atomicAdd((uint32_t*)&bcnt[pbin(keys[i])], 1u);
  __syncthreads();
  const uint32_t bmax = topp_bin_starts(bcnt, bstart, T);
  if (bmax > (uint32_t)FB_LBUF) {
    // a bin beyond the LDS buffer: the whole list by one global bitonic sort
    int N = 1;
    while (N < m) N <<= 1;
    for (int i = m + tid; i < N; i += PZ_SP_BLOCK) keys[i] = 0ull;
    __syncthreads();
    pz_bitonic_desc<PZ_SP_BLOCK>(keys, N);
  } else {
    for (int i = tid; i < m; i += PZ_SP_BLOCK) {
      const uint64_t key = keys[i];
      keys2[atomicAdd((uint32_t*)&bcnt[pbin(key)], 1u)] = key;
    }
    __syncthreads();  // bcnt[b]: the end of bin b
    // rank inside the bin: every comparison independent of the others
    for (int j = tid; j < m; j += PZ_SP_BLOCK) {
      const uint64_t key = keys2[j];
      const int b = pbin(key);
      const uint32_t b0 = bstart[b], b1 = bcnt[b];
      if (b1 - b0 > (uint32_t)TOPP_BIN_MAX) continue;
      uint32_t r = 0, x = b0;
      for (; x + 4 <= b1; x += 4) {
        const uint64_t k0 = keys2[x], k1 = keys2[x + 1], k2 = keys2[x + 2], k3 = keys2[x + 3];
        r += (k0 > key ? 1u : 0u) + (k1 > key ? 1u : 0u) + (k2 > key ? 1u : 0u) +
             (k3 > key ? 1u : 0u);
      }
      for (; x < b1; x++) r += keys2[x] > key ? 1u : 0u;
      keys[b0 + r] = key;
    }
    // the big bins (above TOPP_BIN_MAX keys, so fewer than FB_BIG of them),
    // listed in bin order and sorted in LDS in chunks of consecutive big bins
    // of up to FB_LBUF keys: keys are ordered between bins, so a chunk's
    // sorted union is its bins' sorted lists one after the other
    if (bmax > (uint32_t)TOPP_BIN_MAX) {
      for (int r = 0; r < PBINS; r += PZ_SP_BLOCK) {
        const int b = r + tid;
        const bool isbig = bcnt[b] - bstart[b] > (uint32_t)TOPP_BIN_MAX;
        const uint64_t ball = __ballot(isbig);
        if (lane == 0) T.wtot[w] = (uint32_t)__popcll(ball);
        __syncthreads();
        uint32_t base = (uint32_t)nbig;
        for (int j = 0; j < w; j++) base += T.wtot[j];
        if (isbig) big[base + __popcll(ball & ((1ull << lane) - 1ull))] = (uint32_t)b;
        __syncthreads();
        if (tid == 0) {
          uint32_t t = 0;
          for (int j = 0; j < PZ_SP_WAVES; j++) t += T.wtot[j];
          nbig += (int)t;
        }
        __syncthreads();
      }
      if (tid == 0) {
        int nch = 0;
        uint32_t acc = 0;
        for (int i = 0; i < nbig; i++) {
          const uint32_t c = bcnt[big[i]] - bstart[big[i]];
          if (i == 0 || acc + c > (uint32_t)FB_LBUF) {
            chs[nch++] = (uint32_t)i;
            acc = 0;
          }
          acc += c;
        }
        chs[nch] = (uint32_t)nbig;
        nchunks = nch;
      }
      __syncthreads();
      for (int k = 0; k < nchunks; k++) {
        const int i0 = (int)chs[k], i1 = (int)chs[k + 1];
        int off = 0;
        for (int i = i0; i < i1; i++) {
          const uint32_t b0 = bstart[big[i]];
          const int c = (int)(bcnt[big[i]] - b0);
          for (int j = tid; j < c; j += PZ_SP_BLOCK) sbuf[off + j] = keys2[b0 + j];
          off += c;
        }
        int N = 1;
        while (N < off) N <<= 1;
        for (int j = off + tid; j < N; j += PZ_SP_BLOCK) sbuf[j] = 0ull;
        __syncthreads();
        pz_bitonic_desc<PZ_SP_BLOCK>(sbuf, N);
        off = 0;
        for (int i = i0; i < i1; i++) {
          const uint32_t b0 = bstart[big[i]];
          const int c = (int)(bcnt[big[i]] - b0);
          for (int j = tid; j < c; j += PZ_SP_BLOCK) keys[b0 + j] = sbuf[off + j];
          off += c;
        }
        __syncthreads();
      }
    }
  }
  __syncthreads();  // keys: the sorted list
  GSortedSeg X;
  X.keys = keys;
  X.m = m;
  const int pick =
      nucleus_pick(X, m, row, prm.top_p, u[row], all, p_lo, FB_NC, region, ws, SS, &T.cutoff);
  if (pick >= 0 || all) {
    if (tid == 0) {
      const uint64_t k = keys[pick > 0 ? pick : 0];
      ids_out[row] = key_id(k);
      if (p_out) p_out[row] = key_p(k);
    }
    return true;
  }
  return false;
}

template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) void k_topp_fallback(
    const float* __restrict__ logits, long ld, int V,
    const pz_row_params_dev* __restrict__ params, int n_params,
    const int32_t* __restrict__ hist, int H, int hcap, int nseg, PzSplitWs ws,
    const float* __restrict__ u, int32_t* __restrict__ ids_out, float* __restrict__ p_out,
    pz_scratch sc) {
  // (the queue is emptied by the first kernel of the next launch)
  const int n_fb = sc.counters[0];
  for (int q = blockIdx.x; q < n_fb; q += gridDim.x) {
    const int row = sc.fb_list[q];
    const PzRowState rs0 = ws.rs[row];
    const float gate = rs0.i[1] ? 0.0f : rs0.f[0];
    if (!fb_pass<VEC>(logits, ld, V, params, n_params, hist, H, hcap, nseg, ws, u, ids_out,
                      p_out, sc, row, gate, blockIdx.x, rs0.M, rs0.inv, rs0.f[1]))
      fb_pass<VEC>(logits, ld, V, params, n_params, hist, H, hcap, nseg, ws, u, ids_out, p_out,
                   sc, row, 0.0f, blockIdx.x, rs0.M, rs0.inv,
                   rs0.f[1]);  // the cut-off lies past the gated list
  }
}

// ---- walk, nucleus and fallback in one launch (after k_topp_front) --------
// One workgroup per row.  Wave 0 walks the records (the exact normaliser)
// while waves 1..7 pre-evaluate its specials and waves 8..15 sort the keys
// k_topp_front gathered, by e: a counting sort over PBINS bins of e and each
// key's rank inside its bin (bins above TOPP_BIN_MAX keys: a bitonic sort
// of p keys after the walk).  With the normaliser, e keys become p keys
// (p = e * (1/sum) is monotone in e, so the order holds except inside runs
// of equal p, which are put back in ascending id), and the same workgroup
// finds the cut-off and the draw; rows whose list overflowed, or whose
// cut-off lies below the gathered bins, are queued for k_topp_fallback
// (which follows; the fallback pass in this launch would spill its
// registers).
constexpr int WF_SORT = PZ_SP_BLOCK / 2;  // threads of the sort (waves 8..15)
constexpr int WF_KR = 16;                  // keys per sort thread held in registers

__host__ __device__ inline int pz_pow2_ceil(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}
// Offset of the keys in the fused walk's sort LDS (packed bins, then the
// order): at least 4 * TOPP_BITONIC_MAX bytes before them, for the bitonic
// path's running sums.
__host__ __device__ inline size_t wf_keys_off(int cap) {
  const size_t o = ((size_t)PBINS * 4 + (size_t)cap * 2 + 15) & ~(size_t)15;
  return o > (size_t)TOPP_BITONIC_MAX * 4 ? o : (size_t)TOPP_BITONIC_MAX * 4;
}

// Barrier of waves 8..15 (a monotonic LDS counter: generation g ends when it
// reaches 8 g).  It orders LDS only (the sort's data): the waves' stores
// that clear the row's words stay in flight.
__device__ __forceinline__ void wf_sub_barrier(int* ctr, int& gen) {
  gen++;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  if ((threadIdx.x & 63) == 0)
    __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < 8 * gen)
    __builtin_amdgcn_s_sleep(1);
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Bin of an e key for the fused walk's counting sort: PBINS bins spread
// over the row's e range [e_min, 1] (e = expf(y - max) <= 1), the finest
// power-of-two width that keeps them within PBINS, so a short range gets
// narrow bins and the ranks inside them take few comparisons.  Bins grow as
// e falls (keys below e_min, none expected, share the last).
__device__ __forceinline__ int wf_shift(float e_min) {
  const uint32_t span = 0x3f800000u - (__float_as_uint(e_min) < 0x3f800000u ? __float_as_uint(e_min) : 0x3f800000u);
  int s = 0;
  while ((span >> s) >= (uint32_t)PBINS) s++;
  return s;
}
__device__ __forceinline__ int wf_bin(uint64_t key, int shift) {
  const uint32_t b = (uint32_t)(key >> 32);  // bits(e)
  const uint32_t q = (0x3f800000u - (b < 0x3f800000u ? b : 0x3f800000u)) >> shift;
  return q < (uint32_t)PBINS - 1u ? (int)q : PBINS - 1;
}

template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) void k_topp_walkf(TOPP_ARGS, int pen_bytes, int nc,
                                                           int sort_off, int cap, int nc6) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ ToppShared T;
  __shared__ float sum_sh;
  __shared__ int m_sh, sb_ctr, path_sh;
  __shared__ uint64_t etab[32];
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  pz_etab_fill((pz_lds_u64*)etab);
  const int row = pz_row_of(rows, blockIdx.x);
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  // k_topp_front's meetings and histograms are over: the row's words are
  // cleared by waves 8..15 during the walk (plain stores: the end of this
  // launch makes them visible to the next), or here by every thread on the
  // rows that return early
  uint32_t* hrow = ws.hist + (size_t)blockIdx.x * S * PZ_TOPP_NB;
  auto clear_words = [&](int t0, int nt) {
    for (int i = t0; i < 2 * ws.smax; i += nt) ws.meet[(size_t)row * 2 * ws.smax + i] = 0ull;
    for (int i = t0; i < S * PZ_TOPP_NB; i += nt) hrow[i] = 0u;
  };
  // the nucleus bins (k_topp_front, workgroup 0): loaded at once, beside the
  // row's maxima below, and the row's records for the walk
  const PzRowState rs0 = ws.rs[row];
  const PzRecAhead ra = pz_sp_rec_ahead(ws, row, nseg);
  if (tid == 0) {
    // the gathered count, re-armed for the next call, and the selection word
    m_sh = (int)ws.arrive[row];
    ws.arrive[row] = 0u;
    ws.rs[row].i[6] = 0;
    sb_ctr = 0;
    path_sh = 0;
  }
  if (rs0.i[7]) {  // a wait of k_topp_front gave up on this row
    clear_words(tid, PZ_SP_BLOCK);
    if (tid == 0) {
      ws.rs[row].i[7] = 0;
      ids_out[row] = PZ_ID_FAILED;
      if (p_out) p_out[row] = __builtin_nanf("");
    }
    return;
  }
  pz_sp_row_stat(row, S, ws, SS);
  const float M = SS.M;
  const uint32_t flags = SS.any;
  const PzRow<VEC> R = topp_row<VEC>(logits, ld, row, V, prm, lds, 0, V, hcap, hist, H);
  __syncthreads();  // the expf table, the penalty tables, m
  if (flags & (PZ_RS_Y0NAN | PZ_RS_NONFIN)) clear_words(tid, PZ_SP_BLOCK);
  if (flags & PZ_RS_Y0NAN) {
    if (tid == 0) {
      ids_out[row] = 0;
      if (p_out) p_out[row] = 1.0f;
    }
    return;
  }
  if (flags & PZ_RS_NONFIN) {
    if (tid == 0) T.first = INT_MAX;
    __syncthreads();
    int mine = INT_MAX;
    for (int e0 = 4 * tid; e0 < V; e0 += 4 * PZ_SP_BLOCK) {
      float y[4];
      const int n = R.get(e0, y);
      for (int c = 0; c < n; c++)
        if (y[c] == M && e0 + c < mine) mine = e0 + c;
    }
    atomicMin(&T.first, mine);
    __syncthreads();
    if (tid == 0) {
      ids_out[row] = T.first;
      if (p_out) p_out[row] = __builtin_nanf("");
    }
    return;
  }
  const bool all = rs0.i[1] != 0;
  const float e_gate = rs0.f[0];
  const int m = m_sh;
  // the list: sorted here when it fits (else the fallback)
  const bool listed = (uint32_t)rs0.i[4] <= (uint32_t)ws.capg && m > 0 && m <= cap;
  PzExpTerms<PzRow<VEC>> X;
  X.R = R;
  X.M = M;
  X.thr = M - 20.0f;
  X.inv = 1.0f;
  X.as_p = false;
  X.et = et;
  char* region = lds + pen_bytes;  // the walk's LDS, free again after it
  // the sort's LDS: bin counts and starts packed two per word (every count
  // fits 16 bits: cap < 65536), the order, the keys
  pz_lds_u32b* bcnt = (pz_lds_u32b*)(lds + sort_off);
  pz_lds_u32b* bstart = bcnt + PBINS / 2;
  pz_lds_u16* perm = (pz_lds_u16*)(bstart + PBINS / 2);
  pz_lds_u64* bkeys = (pz_lds_u64*)(lds + sort_off + wf_keys_off(cap));
  const uint64_t* gkeys = ws.keys + (size_t)row * ws.capg;
  // (segment 0's sum: posted by the front launch)
  const PzWalk W = pz_sp_walk_setup(X, row, nseg, nc, ws, region, SS, 7, rs0.s0, &ra);
  if (w == 0) {
    PzAcc st;
    pz_sp_walk<PZ_STOP_NONE>(st, W, 0.0f, X);
    if (tid == 0) sum_sh = pz_acc_value(st);
  } else if (w >= 8) {
    const int tt = tid - (PZ_SP_BLOCK - WF_SORT);
    clear_words(tt, WF_SORT);
  }
  if (w >= 8 && listed) {
    // counting sort of the e keys by bin, then the rank inside each bin
    // (every gathered e is >= e_gate (1 - 2^-21), or >= expf(-20) > 2^-29)
    const int tt = tid - (PZ_SP_BLOCK - WF_SORT);
    const int shw = wf_shift(all ? 0x1p-29f : e_gate * (1.0f - 0x1p-21f));
    int gen = 0;
    // a list of at most WF_KR keys per thread is loaded once, every load in
    // flight together, and both passes read the registers; a longer one is
    // read twice, four keys' loads in flight per thread and trip
    const bool inreg = m <= WF_KR * WF_SORT;
    uint64_t kr[WF_KR];
    if (inreg) {
#pragma unroll
      for (int r = 0; r < WF_KR; r++) kr[r] = tt + r * WF_SORT < m ? gkeys[tt + r * WF_SORT] : 0ull;
    }
    for (int i = tt; i < PBINS / 2; i += WF_SORT) bcnt[i] = 0u;
    if (tt == 0) T.bmax = 0u;
    wf_sub_barrier(&sb_ctr, gen);
    if (inreg) {
#pragma unroll
      for (int r = 0; r < WF_KR; r++)
        if (tt + r * WF_SORT < m) {
          const int q = wf_bin(kr[r], shw);
          atomicAdd((uint32_t*)&bcnt[q >> 1], 1u << (16 * (q & 1)));
        }
    } else {
      for (int i0 = tt; i0 < m; i0 += 4 * WF_SORT) {
        uint64_t kq[4];
#pragma unroll
        for (int r = 0; r < 4; r++) kq[r] = i0 + r * WF_SORT < m ? gkeys[i0 + r * WF_SORT] : 0ull;
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (i0 + r * WF_SORT < m) {
            const int q = wf_bin(kq[r], shw);
            atomicAdd((uint32_t*)&bcnt[q >> 1], 1u << (16 * (q & 1)));
          }
      }
    }
    wf_sub_barrier(&sb_ctr, gen);
    // exclusive bin starts: thread tt owns bins 8 tt .. 8 tt + 7 (words 4 tt ..)
    constexpr int BPT = PBINS / WF_SORT;
    uint32_t c[BPT], local = 0, mx = 0;
#pragma unroll
    for (int j = 0; j < BPT; j++) {
      c[j] = (bcnt[(BPT * tt + j) >> 1] >> (16 * (j & 1))) & 0xffffu;
      local += c[j];
      mx = c[j] > mx ? c[j] : mx;
    }
    const uint32_t incl = pz_wave_scan_u32(local);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint32_t o = __shfl_xor(mx, off, 64);
      mx = o > mx ? o : mx;
    }
    const int sw = w - 8;
    if (lane == 63) T.wtot[sw] = incl;
    if (lane == 0) atomicMax(&T.bmax, mx);
    wf_sub_barrier(&sb_ctr, gen);
    uint32_t run = incl - local;
    for (int j = 0; j < sw; j++) run += T.wtot[j];
#pragma unroll
    for (int j = 0; j < BPT; j += 2) {
      const uint32_t s0 = run, s1 = run + c[j];
      bstart[(BPT * tt + j) >> 1] = s0 | (s1 << 16);
      bcnt[(BPT * tt + j) >> 1] = s0 | (s1 << 16);  // cursors
      run = s1 + c[j + 1];
    }
    wf_sub_barrier(&sb_ctr, gen);
    if (inreg) {
#pragma unroll
      for (int r = 0; r < WF_KR; r++)
        if (tt + r * WF_SORT < m) {
          const int q = wf_bin(kr[r], shw);
          const uint32_t old = atomicAdd((uint32_t*)&bcnt[q >> 1], 1u << (16 * (q & 1)));
          bkeys[(old >> (16 * (q & 1))) & 0xffffu] = kr[r];
        }
    } else {
      for (int i0 = tt; i0 < m; i0 += 4 * WF_SORT) {
        uint64_t kq[4];
#pragma unroll
        for (int r = 0; r < 4; r++) kq[r] = i0 + r * WF_SORT < m ? gkeys[i0 + r * WF_SORT] : 0ull;
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (i0 + r * WF_SORT < m) {
            const int q = wf_bin(kq[r], shw);
            const uint32_t old = atomicAdd((uint32_t*)&bcnt[q >> 1], 1u << (16 * (q & 1)));
            bkeys[(old >> (16 * (q & 1))) & 0xffffu] = kq[r];
          }
      }
    }
    wf_sub_barrier(&sb_ctr, gen);
    if (T.bmax <= (uint32_t)TOPP_BIN_MAX) {
      for (int j = tt; j < m; j += WF_SORT) {
        const uint64_t key = bkeys[j];
        const int q = wf_bin(key, shw);
        const uint32_t b0 = (bstart[q >> 1] >> (16 * (q & 1))) & 0xffffu;
        const uint32_t b1 = (bcnt[q >> 1] >> (16 * (q & 1))) & 0xffffu;
        uint32_t r = 0, x = b0;
        for (; x + 4 <= b1; x += 4) {
          const uint64_t k0 = bkeys[x], k1 = bkeys[x + 1], k2 = bkeys[x + 2], k3 = bkeys[x + 3];
          r += (k0 > key ? 1u : 0u) + (k1 > key ? 1u : 0u) + (k2 > key ? 1u : 0u) +
               (k3 > key ? 1u : 0u);
        }
        for (; x < b1; x++) r += bkeys[x] > key ? 1u : 0u;
        perm[b0 + r] = (uint16_t)j;
      }
      if (tt == 0) path_sh = 1;  // sorted through perm
    } else if (tt == 0) {
      path_sh = 2;  // a bin too large: bitonic sort after the walk
    }
  }
  __syncthreads();
  const float sum = sum_sh;
  const float inv = 1.0f / sum;  // top_p.c:72
  if (tid == 0) {
    ws.rs[row].sum = sum;
    ws.rs[row].inv = inv;
  }
  const int path = path_sh;
  const float p_lo = e_gate * inv;
  bool done = false, whole = false;  // whole: the list was sorted, its cut-off lies past it
  if (listed && path == 1) {
    for (int i = tid; i < m; i += PZ_SP_BLOCK) bkeys[i] = topp_pkey(bkeys[i], inv);
    __syncthreads();
    // runs of equal p (distinct e can round to one p) back in ascending id:
    // each thread checks 8 consecutive positions, the p of those and of
    // their two neighbours loaded at once (-1 outside the list: no p equals
    // it); only a run longer than one goes on key by key
    constexpr int CH = 8;
    for (int j0 = tid * CH; j0 < m; j0 += PZ_SP_BLOCK * CH) {
      float pv[CH + 2];  // p at positions j0 - 1 .. j0 + CH
      uint32_t ix[CH + 2];
#pragma unroll
      for (int c = 0; c < CH + 2; c++) {
        const int jj = j0 - 1 + c;
        ix[c] = jj >= 0 && jj < m ? (uint32_t)perm[jj] : 0u;
      }
#pragma unroll
      for (int c = 0; c < CH + 2; c++) {
        const int jj = j0 - 1 + c;
        pv[c] = jj >= 0 && jj < m ? key_p(bkeys[ix[c]]) : -1.0f;
      }
#pragma unroll
      for (int c = 1; c <= CH; c++) {
        const int j = j0 - 1 + c;
        if (j >= m || pv[c - 1] == pv[c] || pv[c + 1] != pv[c]) continue;
        const float pj = pv[c];
        int e = j + 1;
        while (e < m && key_p(bkeys[perm[e]]) == pj) e++;
        for (int a = j + 1; a < e; a++) {  // insertion sort of perm[j, e) by key, descending
          const uint16_t pa = perm[a];
          const uint64_t ka = bkeys[pa];
          int b = a;
          while (b > j && bkeys[perm[b - 1]] < ka) {
            perm[b] = perm[b - 1];
            b--;
          }
          perm[b] = pa;
        }
      }
    }
    __syncthreads();
    if (m <= 64) {
      // a list of one wave: each lane holds one p, and the reference's loops
      // run as written over them (top_p.c:80-93 the cumulative to the first
      // sum >= top_p, :96-105 the first cumulative > u * trunc_sum), every
      // add a plain fp32 add in list order
      if (w == 0) {
        const float pl = lane < m ? key_p(bkeys[perm[lane]]) : 0.0f;
        auto p_at = [&](int j) {
          return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pl), j));
        };
        float cum = 0.0f;
        int cutoff = -1;
        for (int j = 0; j < m; j++) {
          cum = cum + p_at(j);
          if (cum >= prm.top_p) {
            cutoff = j + 1;
            break;
          }
        }
        if (cutoff < 0 && all) cutoff = m;  // cum: the whole sum
        if (cutoff > 0 && (all || p_at(cutoff - 1) >= p_lo)) {
          const float r = u[row] * cum;  // cum: the cumulative at the cut-off
          float c2 = 0.0f;
          int pick = 0;
          for (int j = 0; j < cutoff; j++) {
            c2 = c2 + p_at(j);
            if (c2 > r) {
              pick = j;
              break;
            }
          }
          if (lane == 0) {
            const uint64_t k = bkeys[perm[pick]];
            ids_out[row] = key_id(k);
            if (p_out) p_out[row] = key_p(k);
          }
          done = true;
        }
      }
    } else if (m < TOPP_BINSORT_MIN) {
      // a short list: contiguous keys and the lane-ordered walks
      uint64_t* kk = reinterpret_cast<uint64_t*>(region);
      float* cum = reinterpret_cast<float*>(region + (size_t)TOPP_BINSORT_MIN * 8);
      for (int j = tid; j < m; j += PZ_SP_BLOCK) kk[j] = bkeys[perm[j]];
      __syncthreads();
      const int cutoff = nucleus_cutoff(kk, cum, m, prm.top_p, all, &T.cutoff);
      if (cutoff > 0 && (all || key_p(kk[cutoff - 1]) >= p_lo)) {
        if (tid == 0)
          nucleus_draw(kk, cum, cutoff, u[row], &ids_out[row], p_out ? &p_out[row] : nullptr);
        done = true;
      }
    } else {
      SortedSeg Xs;
      Xs.bkeys = bkeys;
      Xs.perm = perm;
      Xs.m = m;
      // (the bins are free: the list's records go there)
      nucleus_pick(Xs, m, row, prm.top_p, u[row], all, p_lo, nc6, region, ws, SS, &T.cutoff,
                   lds + sort_off);
      if (T.cutoff >= 0) {
        if (tid == 0) {
          const uint64_t k = bkeys[perm[T.cutoff]];
          ids_out[row] = key_id(k);
          if (p_out) p_out[row] = key_p(k);
        }
        done = true;
      }
    }
    whole = true;
  } else if (listed && path == 2 && m <= TOPP_BITONIC_MAX && pz_pow2_ceil(m) <= cap) {
    const int N = pz_pow2_ceil(m);
    for (int i = tid; i < N; i += PZ_SP_BLOCK)
      bkeys[i] = i < m ? topp_pkey(bkeys[i], inv) : 0ull;
    __syncthreads();
    pz_bitonic_desc<PZ_SP_BLOCK>(bkeys, N);
    uint64_t* kk = reinterpret_cast<uint64_t*>(lds + sort_off + wf_keys_off(cap));  // bkeys
    // the running sums over the bins and the order (free here): m <= 8192 floats
    float* cum = reinterpret_cast<float*>(lds + sort_off);
    const int cutoff = nucleus_cutoff(kk, cum, m, prm.top_p, all, &T.cutoff);
    if (cutoff > 0 && (all || key_p(kk[cutoff - 1]) >= p_lo)) {
      if (tid == 0)
        nucleus_draw(kk, cum, cutoff, u[row], &ids_out[row], p_out ? &p_out[row] : nullptr);
      done = true;
    }
    whole = true;
  }
  if (done || tid != 0) return;
  // the fallback: every candidate at or above the gate (all of them when the
  // whole gathered list was sorted without reaching the cut-off)
  if (whole) {
    ws.rs[row].f[0] = 0.0f;
    ws.rs[row].i[1] = 1;
  }
  const int q = atomicAdd(&sc.counters[0], 1);
  sc.fb_list[q] = row;
}

// LDS of the fallback: the penalty tables during the gather, then the bins
// and the sort buffer or the walk over up to slot_n keys.
size_t topp_fallback_bytes(size_t pen_full, int slot_n) {
  const size_t sortb = (size_t)FB_LBUF * 8;
  const size_t walk = pz_sp_walk_lds((slot_n + PZ_SP_SEG - 1) / PZ_SP_SEG, FB_NC);
  const size_t after = FB_HEAD + (sortb > walk ? sortb : walk);
  return pen_full > after ? pen_full : after;
}

size_t pen_region(const pz_launch& L, int n_ids) {
  return L.pen_any ? (pz_penalty_lds_bytes(n_ids, L.hcap) + 15) & ~(size_t)15 : 0;
}

size_t max_sz(size_t a, size_t b) { return a > b ? a : b; }

// LDS of the nucleus kernel for lists of up to cap keys with nc
// pre-evaluated segments: keys and their order, then the bins / the running
// sums of the small-list path / the walk over the sorted list.
size_t topp_nucleus_bytes(int cap, int nc) {
  const size_t head = ((size_t)cap * 10 + 15) & ~(size_t)15;
  const size_t bins = (size_t)PBINS * 8;
  const size_t cum = (size_t)(cap < TOPP_BITONIC_MAX ? cap : TOPP_BITONIC_MAX) * 4;
  const size_t walk = pz_sp_walk_lds((cap + PZ_SP_SEG - 1) / PZ_SP_SEG, nc);
  return head + max_sz(max_sz(bins, cum), walk);
}

template <bool VEC>
int launch_topp_t(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  const PzSplitWs& ws = L.ws;
  const PzSplitPlan pl = pz_split_plan(L.V, n_rows, ws.smax);
  if ((size_t)n_rows * pl.S > (size_t)ws.hslots || pl.nseg > ws.nsc) return -2;
  const size_t fixed = 4096;  // static LDS of the kernels
  const size_t pen_slice = pen_region(L, pl.spw * PZ_SP_SEG), pen_full = pen_region(L, L.V);
  // slice passes: the slice's penalty tables (+ the histogram)
  const size_t lds1 = pen_slice;
  const size_t lds2 = pen_slice + PZ_TOPP_NB * 4;
  // walk: the row's penalty tables, the merged histogram, the walk's arrays
  // (the gather blocks of the same launch use the first pen_slice bytes)
  const size_t walk_off = (pen_full + PZ_TOPP_NB * 4 + 15) & ~(size_t)15;
  if (walk_off + fixed >= (size_t)L.max_lds) return -2;
  const int nc = pz_sp_walk_nc(pl.nseg, (size_t)L.max_lds - walk_off - fixed);
  if (nc < 1) return -2;
  const size_t lds3 = walk_off + pz_sp_walk_lds(pl.nseg, nc);
  // nucleus: the largest list (and its walk) that fits
  // (pre-evaluated segments of its walk: as many as fit, 4 to 16)
  int cap = TOPP_CAP_MAX < ws.capg ? TOPP_CAP_MAX : ws.capg;
  int nc6 = 16;
  while (topp_nucleus_bytes(cap, nc6) + fixed > (size_t)L.max_lds) {
    if (nc6 > 4) nc6--;
    else if (cap > 256) {
      cap >>= 1;
      nc6 = 16;
    } else {
      break;
    }
  }
  const size_t lds4 = topp_nucleus_bytes(cap, nc6);
  if (lds4 + fixed > (size_t)L.max_lds || pen_full + fixed > (size_t)L.max_lds) return -2;
  const size_t lds5 = topp_fallback_bytes(pen_full, L.sc.slot_n);
  if (lds5 + fixed > (size_t)L.max_lds || L.sc.slot_n / (TOPP_BIN_MAX + 1) >= FB_BIG) return -2;
  // passes 1-3, the bins and the gather in one launch when a slice fits in
  // LDS beside its tables (two workgroups per CU), then the walk, the
  // nucleus and the fallback in one more (the keys' sort beside the walk:
  // the largest list that fits, a power of two for its bitonic path)
  // the front launch's slices: the plan's, or -- when a batch is large
  // enough that the plan's slices exceed LDS -- TOPP_FRONT_SEGS segments,
  // the rows then running in several rounds of workgroups (every row's
  // histogram slots at once)
  PzSplitPlan pf = pl;
  if (pf.spw > TOPP_FRONT_SEGS) {
    pf.spw = TOPP_FRONT_SEGS;
    pf.S = (pl.nseg + pf.spw - 1) / pf.spw;
  }
  const size_t pen_slice_f = pen_region(L, pf.spw * PZ_SP_SEG);
  const size_t lds_front = ((pen_slice_f + PZ_TOPP_NB * 4 + 15) & ~(size_t)15) +
                           (size_t)pf.spw * PZ_SP_SEG * sizeof(float);
  const size_t wf_walk_off = (pen_full + 15) & ~(size_t)15;
  int wf_cap = 0, wf_nc = 0;
  size_t wf_sort_off = 0;
  for (int c = TOPP_CAP_MAX; c >= 2048 && !wf_cap; c -= 1024) {
    if (c > ws.capg) continue;
    for (int n = 16; n >= 4; n--) {
      const size_t so = (wf_walk_off + pz_sp_walk_lds(pl.nseg, n) + 15) & ~(size_t)15;
      if (so + wf_keys_off(c) + (size_t)c * 8 + fixed <= (size_t)L.max_lds) {
        wf_cap = c;
        wf_nc = n;
        wf_sort_off = so;
        break;
      }
    }
  }
  const size_t lds_wf = wf_sort_off + wf_keys_off(wf_cap) + (size_t)wf_cap * 8;
  // (the front launch's waits end because a row's S workgroups can all be
  // resident at once: S <= 64 and, on a device or partition with few CUs,
  // at most one per CU)
  const bool front = (size_t)n_rows * pf.S <= (size_t)ws.hslots && pf.S <= 64 &&
                     (L.n_cu <= 0 || pf.S <= L.n_cu) &&
                     2 * (lds_front + fixed) <= (size_t)L.max_lds && wf_cap > 0 &&
                     lds_wf + fixed <= (size_t)L.max_lds;
  if (front) {
    auto kf = k_topp_front<VEC>;
    auto kw = k_topp_walkf<VEC>;
    if ((lds_front > 65536 &&
         hipFuncSetAttribute((const void*)kf, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)lds_front) != hipSuccess) ||
        (lds_wf > 65536 &&
         hipFuncSetAttribute((const void*)kw, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)lds_wf) != hipSuccess))
      return -1;
    hipLaunchKernelGGL(kf, dim3(pf.S, n_rows), dim3(PZ_SP_BLOCK), lds_front, L.stream, L.logits,
                       L.ld, L.V, d_rows, L.params, L.n_params, L.hist, L.H, L.hcap, pf.nseg,
                       pf.spw, pf.S, ws, L.u, L.ids, L.p_out, L.sc, (int)pen_slice_f,
                       L.wait_polls);
    hipLaunchKernelGGL(kw, dim3(n_rows), dim3(PZ_SP_BLOCK), lds_wf, L.stream, L.logits, L.ld,
                       L.V, d_rows, L.params, L.n_params, L.hist, L.H, L.hcap, pf.nseg, pf.spw,
                       pf.S, ws, L.u, L.ids, L.p_out, L.sc, (int)wf_walk_off, wf_nc,
                       (int)wf_sort_off, wf_cap, wf_nc);
    auto fbk = k_topp_fallback<VEC>;
    if (lds5 > 65536 && hipFuncSetAttribute((const void*)fbk,
                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                            (int)lds5) != hipSuccess)
      return -1;
    const int fb_grid = n_rows < L.sc.fb_slots ? n_rows : L.sc.fb_slots;
    hipLaunchKernelGGL(fbk, dim3(fb_grid), dim3(PZ_SP_BLOCK), lds5, L.stream, L.logits, L.ld,
                       L.V, L.params, L.n_params, L.hist, L.H, L.hcap, pl.nseg, ws, L.u, L.ids,
                       L.p_out, L.sc);
    return hipGetLastError() == hipSuccess ? 0 : -1;
  }
  auto k1 = k_topp_stat<VEC>;
  auto k1e = k_topp_est<VEC>;
  auto k2 = k_topp_rec<VEC>;
  auto k3 = k_topp_walk<VEC>;
  auto k4 = k_topp_nucleus<VEC>;
  auto fb = k_topp_fallback<VEC>;
  const void* fns[6] = {(const void*)k1, (const void*)k1e, (const void*)k2, (const void*)k3,
                        (const void*)k4, (const void*)fb};
  const size_t need[6] = {lds1, lds1, lds2, lds3, lds4, lds5};
  for (int i = 0; i < 6; i++)
    if (need[i] > 65536 && hipFuncSetAttribute(fns[i], hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)need[i]) != hipSuccess)
      return -1;
  const dim3 grid(pl.S, n_rows), block(PZ_SP_BLOCK);
  // gather blocks per row: the CUs the walks leave free, in one round
  const int cus = PZ_SP_TARGET_WG / 2;
  int gS = n_rows < cus ? (cus - n_rows) / n_rows : 1;
  gS = gS < 1 ? 1 : (gS > pl.S ? pl.S : gS);
  const int gspw = (pl.nseg + gS - 1) / gS;
  // a gather block's LDS: its slice's penalty tables, then staged keys
  const size_t goff = (pen_region(L, gspw * PZ_SP_SEG) + 15) & ~(size_t)15;
  int lcap = (int)((lds3 - goff) / 8);
  lcap = lcap < ws.capg ? lcap : ws.capg;
#define TOPP_PASS L.logits, L.ld, L.V, d_rows, L.params, L.n_params, L.hist, L.H, L.hcap, \
                  pl.nseg, pl.spw, pl.S, ws, L.u, L.ids, L.p_out, L.sc
  hipLaunchKernelGGL(k1, grid, block, lds1, L.stream, TOPP_PASS);
  hipLaunchKernelGGL(k1e, grid, block, lds1, L.stream, TOPP_PASS);
  hipLaunchKernelGGL(k2, grid, block, lds2, L.stream, TOPP_PASS, (int)pen_slice);
  hipLaunchKernelGGL(k3, dim3(n_rows * (1 + gS)), block, lds3, L.stream, TOPP_PASS,
                     (int)pen_full, nc, n_rows, gS, gspw, (int)goff, lcap, L.wait_polls);
  hipLaunchKernelGGL(k4, dim3(n_rows), block, lds4, L.stream, TOPP_PASS, cap, nc6);
#undef TOPP_PASS
  const int fb_grid = n_rows < L.sc.fb_slots ? n_rows : L.sc.fb_slots;
  hipLaunchKernelGGL(fb, dim3(fb_grid), block, lds5, L.stream, L.logits, L.ld, L.V, L.params,
                     L.n_params, L.hist, L.H, L.hcap, pl.nseg, ws, L.u, L.ids, L.p_out, L.sc);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

int pz_launch_topp(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  if (n_rows <= 0) return 0;
  if (L.V > PZ_TOPP_MAX_V) return pz_launch_greedy_tempered(L, n_rows, d_rows);  // top_p.c:33-34
  const bool vec = (L.ld % 4 == 0) && (((uintptr_t)L.logits & 15) == 0);
  return vec ? launch_topp_t<true>(L, n_rows, d_rows) : launch_topp_t<false>(L, n_rows, d_rows);
}
