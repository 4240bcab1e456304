// pz_topk.hip -- batched top-k sampling, optionally chained with top-p.
//
// Reference semantics (src/sampling/top_k.c:8-73):
//   * selection: the k largest values above -1e30, ties to the lower id,
//     sorted by (value desc, id asc); unfilled slots are (-1e30, -1);
//   * softmax over the k values: e = expf(v - v0), a sequential fp32 sum,
//     p = e / sum (a true division);
//   * draw: first slot with r < cdf (sequential), fallback slot 0.
// Chain (0 < top_p < 1): cut-off, truncated mass and draw of
// src/sampling/top_p.c:79-105 over those k sorted probabilities.
//
// Design (one workgroup per row, 1024 threads):
//   0. The loads of the first tiles, the history ids and the expf table are
//      issued before anything else, so their latency overlaps the set-up.
//   1. Penalty tables in LDS (membership bitmap, id -> count hash); the
//      streaming pass reads one bitmap word per four ids and penalises the
//      rare history members in registers.
//   2. LDS histogram of the order keys of the first tile (a sample of the
//      row) -> a lower bound on the row's k-th largest (key, id).
//   3. One software-pipelined streaming pass (128-bit loads, the next group
//      of tiles in flight while the current one is processed).  The bound is
//      carried back through the temperature to the raw logits (the
//      temperature map is monotone), so each element costs one compare; the
//      few candidates that pass are keyed and appended to an LDS buffer with
//      one LDS atomic per wave.  On overflow the buffer's k-th largest is a
//      tighter bound and the row is streamed again (from L2 / Infinity
//      Cache).
//   4. Radix select (11-bit digits over the candidates' actual range, LDS
//      histograms) of the exact k-th largest candidate, compaction of the k
//      survivors, and their order: a rank count for small k, a bitonic sort
//      otherwise.
//   5. Wave 0 evaluates the k-slot softmax (expf from an LDS copy of its
//      table), cut-off and draw with the exact sequential fp32 sums of the
//      reference (lane-ordered scans).
//
// Small batches (a few rows: one sequence per call, as the reference's loop
// runs) split each row over workgroups instead (k_topk_split): workgroup s
// takes ids [4096 s, 4096 s + 4096), keys every valid element of that range
// into LDS (penalty tables built for the range only) and selects the range's
// own k largest (key, id); the row's top k are among the union of these.
// The ranges' candidates meet in the row's workspace and the workgroup that
// arrives last merges them and runs steps 4-5.
#include "pz_device.h"
#include "pz_exact.h"
#include "pz_launch.h"
#include "pz_rowpass.h"
#include "pz_seq.h"
#include "pz_sort.h"
#include "pz_split.h"

namespace {

constexpr int TOPK_BLOCK = 1024;
constexpr int TOPK_CAP = 4096;    // candidate buffer entries (8 B each)
constexpr int TOPK_MAXK = 1024;   // top_k.c:11-17 clamps k to 1024
constexpr int HBINS = 2048;       // 11-bit digit
constexpr int TK_U = 4;           // tiles per load group
constexpr int TK_RANK_MAX = 128;  // survivors ordered by a rank count up to this many
constexpr int TK_WM = 64;          // split rows with k up to this: sorted range lists, wave merges
constexpr int TK_WM_WAVES = 4;     // waves merging the lists (16 each: at most 64 ranges)

struct TopkShared {
  uint32_t hist[HBINS];     // sample / radix histograms (kept zeroed), then p and cdf
  uint64_t top[TOPK_MAXK];  // the k survivors
  uint64_t etab[32];        // expf table
  uint64_t thr;             // candidates are the (key, ~id) >= thr
  uint64_t maxc;            // largest candidate appended
  uint64_t base;            // radix select state
  float rlo, rhi;           // the pass bound in raw logits (TkRaw)
  int ridmax;
  int need;
  int done;
  int count;  // candidates appended (may exceed TOPK_CAP)
  int ntop;   // survivors
  int nbin;   // entries of the k-th bin (tk_select_bin)
  uint32_t bin;
};

typedef __attribute__((address_space(3))) uint32_t tk_lds_u32;
typedef __attribute__((address_space(3))) float tk_lds_f32;

__device__ __forceinline__ uint64_t comp_of(uint32_t key, int id) {
  return ((uint64_t)key << 32) | (uint32_t)(0xffffffffu - (uint32_t)id);
}

__device__ __forceinline__ int id_of(uint64_t c) { return (int)(0xffffffffu - (uint32_t)c); }

template <bool DIV>
__device__ __forceinline__ float tk_temper(float x, const PzTemp& T) {
  return DIV ? x / T.t : x * T.inv;
}

// Order key of y + 0.0f (pz_key without the -0.0 test: the addition has
// already folded -0.0 onto +0.0).
__device__ __forceinline__ uint32_t tk_key(float y) {
  const uint32_t u = __float_as_uint(y);
  return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}

// Smallest raw logit x (in key order) whose tempered value reaches f:
// temper(x) >= f  <=>  x >= tk_raw_bound(f) for every non-NaN x, since
// x -> fl(x * inv) and x -> fl(x / t) are monotone non-decreasing.  A 64-way
// search by one wave over the keys of [-inf, +inf] (six rounds); NaN
// (nothing passes) when f is NaN.  Wave-uniform result.
template <bool DIV>
__device__ __forceinline__ float tk_raw_bound(float f, const PzTemp& T) {
  if (!(f <= __builtin_inff())) return __builtin_nanf("");
  const uint32_t lane = threadIdx.x & 63;
  // invariant: temper(unkey(lo)) < f <= temper(unkey(hi)); -inf < f always
  uint32_t lo = 0x007fffffu, hi = 0xff800000u;  // keys of -inf and +inf
  while (hi - lo > 1u) {
    const uint64_t span = hi - lo;
    // lane l tests lo + ceil(span * (l + 1) / 64), the last lane tests hi
    const uint32_t m = lo + (uint32_t)((span * (lane + 1) + 63) >> 6);
    const uint64_t ok = __ballot(tk_temper<DIV>(pz_unkey(m), T) >= f);
    const int j = (int)__builtin_ctzll(ok);  // lane 63 (m == hi) always passes
    const uint32_t mj = __builtin_amdgcn_readlane(m, j);
    const uint32_t mp = j > 0 ? __builtin_amdgcn_readlane(m, j - 1) : lo;
    hi = mj;
    lo = mp;
  }
  return pz_unkey(hi);
}

// The pass bound (key, ~id) >= thr, with y > -1e30, in raw logits:
//   plain (~id part 0):  key(y) >= K                    <=>  x >= lo
//   composite:           key(y) > K, or key(y) == K and id <= idmax
//                                                       <=>  x >= hi, or x >= lo and id <= idmax
struct TkRaw {
  float lo, hi;
  int idmax;
};

template <bool DIV>
__device__ __forceinline__ TkRaw tk_raw_of(uint64_t thr, const PzTemp& T) {
  const uint32_t kk = (uint32_t)(thr >> 32);
  const float fk = pz_unkey(kk);
  const float valid = __uint_as_float(0xf149f2c9u);  // smallest float > -1e30f
  TkRaw r;
  r.lo = tk_raw_bound<DIV>(fk > valid ? fk : valid, T);
  r.hi = r.lo;
  r.idmax = (int)(0xffffffffu - (uint32_t)thr);
  if ((uint32_t)thr != 0u) {
    // composite bounds come from real candidates: fk is above -1e30, not NaN
    r.hi = fk < __builtin_inff() ? tk_raw_bound<DIV>(pz_unkey(kk + 1u), T)
                                 : __builtin_nanf("");
  }
  return r;
}

// Wave 0 publishes the raw form of a new pass bound.
template <bool DIV>
__device__ __forceinline__ void tk_publish(TopkShared& S, uint64_t thr, const PzTemp& T) {
  const TkRaw r = tk_raw_of<DIV>(thr, T);
  if ((threadIdx.x & 63) == 0) {
    S.thr = thr;
    S.rlo = r.lo;
    S.rhi = r.hi;
    S.ridmax = r.idmax;
  }
}

// Loads tiles t0..t0+TK_U-1 of the row (tiles past the end re-load the last
// one, so every load is unconditional and in bounds).
template <bool VEC>
__device__ __forceinline__ void tk_load(const float* x, int V, int t0, int ntiles,
                                        float (&a)[TK_U][4]) {
#pragma unroll
  for (int u = 0; u < TK_U; u++) {
    const int t = t0 + u < ntiles ? t0 + u : ntiles - 1;
    (void)pz_load4<VEC, false>(x, V, pz_tile_e0(t), a[u]);
  }
}

// Reads every register of a group, so that loads still in flight when a
// streaming pass ends are waited for there, not at the next pass's first
// use of the registers (which would stall every iteration of its loop).
__device__ __forceinline__ void tk_drain(const float (&a)[TK_U][4]) {
#pragma unroll
  for (int u = 0; u < TK_U; u++)
#pragma unroll
    for (int c = 0; c < 4; c++) asm volatile("" ::"v"(a[u][c]));
}

// Wave-cooperative search over a 2048-bin histogram (bin 2047 = largest
// digit): the bin holding the need-th largest element, with above = the
// count in larger bins.  Returns false when the histogram holds fewer than
// need.  The histogram is zeroed afterwards (same wave, program order).
__device__ __forceinline__ bool tk_find_bin(tk_lds_u32* hist, uint32_t need, uint32_t& bin,
                                            uint32_t& above, uint32_t& cnt) {
  const int lane = threadIdx.x & 63;
  tk_lds_u32* h = hist + 32 * lane;  // lane l owns bins [32l, 32l+32)
  // each lane walks its bins from a rotated start, so the 64 lanes' reads
  // of one step fall in different LDS banks
  uint32_t own = 0;
#pragma unroll
  for (int j = 0; j < 32; j++) own += h[(j + lane) & 31];
  const uint32_t incl = pz_wave_scan_u32(own);
  const uint32_t total = pz_readlane_u32(incl, 63);
  bool found = false;
  if (total >= need) {
    const uint32_t abv = total - incl;  // bins of lanes > l
    const uint64_t b = __ballot(abv < need && abv + own >= need);
    const int l = (int)__builtin_ctzll(b);
    const uint32_t above_l = pz_readlane_u32(abv, l);
    // lanes 0..31 take the 32 bins of lane l, largest first
    const uint32_t hj = lane < 32 ? hist[32 * l + 31 - lane] : 0u;
    const uint32_t sj = pz_wave_scan_u32(hj);
    const uint64_t f = __ballot(lane < 32 && above_l + sj >= need);
    const int fl = (int)__builtin_ctzll(f);
    bin = (uint32_t)(32 * l + 31 - fl);
    cnt = pz_readlane_u32(hj, fl);
    above = above_l + pz_readlane_u32(sj, fl) - cnt;
    found = true;
  }
#pragma unroll
  for (int j = 0; j < 32; j++) h[(j + lane) & 31] = 0u;
  return found;
}

// Exact radix select over buf[0..n) (distinct composite keys, all in
// [base, maxc], n >= k >= 1): returns thr such that exactly k entries are
// >= thr.  Digits are 11-bit slices of (c - base) over the live range, so
// the first pass already resolves the candidates' actual spread.  S.hist is
// zero on entry and on exit.
template <int BLOCK>
__device__ uint64_t tk_select(TopkShared& S, const pz_lds_u64* buf, int n, int k, uint64_t base,
                              uint64_t maxc) {
  const int tid = threadIdx.x;
  uint32_t need = (uint32_t)k;
  const uint64_t span = maxc - base;
  int w = span == 0 ? 0 : 64 - __builtin_clzll(span);  // range [base, base + 2^w)
  if (w == 0) return base;
  for (;;) {
    const int bits = w >= 11 ? 11 : w;
    const int sh = w - bits;
    for (int i = tid; i < n; i += BLOCK) {
      const uint64_t d = buf[i] - base;
      if (w >= 64 || (d >> w) == 0) atomicAdd(&S.hist[(uint32_t)(d >> sh)], 1u);
    }
    __syncthreads();
    if (tid < PZ_WAVE) {
      uint32_t bin = 0, above = 0, cnt = 0;
      tk_find_bin((tk_lds_u32*)S.hist, need, bin, above, cnt);
      if (tid == 0) {
        S.base = base + ((uint64_t)bin << sh);
        S.need = (int)(need - above);
        S.done = sh == 0 || cnt == need - above;
      }
    }
    __syncthreads();
    base = S.base;
    need = (uint32_t)S.need;
    w = sh;
    if (S.done) return base;
  }
}

// Number of the n entries of a[] greater than c: eight independent LDS
// reads per step (a sequential loop would wait for each read in turn).
__device__ __forceinline__ int tk_rank(const pz_lds_u64* a, int n, uint64_t c) {
  int r0 = 0, r1 = 0, r2 = 0, r3 = 0, j = 0;
  for (; j + 8 <= n; j += 8) {
    const uint64_t x0 = a[j], x1 = a[j + 1], x2 = a[j + 2], x3 = a[j + 3];
    const uint64_t x4 = a[j + 4], x5 = a[j + 5], x6 = a[j + 6], x7 = a[j + 7];
    r0 += (x0 > c) + (x4 > c);
    r1 += (x1 > c) + (x5 > c);
    r2 += (x2 > c) + (x6 > c);
    r3 += (x3 > c) + (x7 > c);
  }
  for (; j < n; j++) r0 += a[j] > c ? 1 : 0;
  return (r0 + r1) + (r2 + r3);
}

// The same contract as tk_select (exactly k entries of buf[0..n) are >=
// the result; n > k >= 1, entries distinct; base == ~0 when the entries'
// range is not known) in one histogram pass: the bin
// of the top 11 key bits holding the k-th largest is found, and the entries
// of that bin are ranked against each other (one per thread, every
// comparison independent).  A bin of more than BLOCK entries (long runs of
// equal values) takes the radix select.  S.hist is zero on entry and exit.
template <int BLOCK>
__device__ uint64_t tk_select_bin(TopkShared& S, const pz_lds_u64* buf, int n, int k,
                                  uint64_t base, uint64_t maxc) {
  const int tid = threadIdx.x;
  for (int i = tid; i < n; i += BLOCK) atomicAdd(&S.hist[(uint32_t)(buf[i] >> 53)], 1u);
  __syncthreads();
  if (tid < PZ_WAVE) {
    uint32_t bin = 0, above = 0, cnt = 0;
    tk_find_bin((tk_lds_u32*)S.hist, (uint32_t)k, bin, above, cnt);  // zeroes S.hist
    if (tid == 0) {
      S.bin = bin;
      S.need = k - (int)above;
      S.nbin = (int)cnt;
      S.ntop = 0;
    }
  }
  __syncthreads();
  const uint32_t bin = S.bin;
  const int need = S.need, cnt = S.nbin;
  if (cnt > BLOCK || cnt > HBINS / 2) {
    if (base == ~0ull) {  // range not known: the entries' smallest and largest
      if (tid == 0) {
        S.base = ~0ull;
        S.maxc = 0ull;
      }
      __syncthreads();
      for (int i = tid; i < n; i += BLOCK) {
        atomicMin(&S.base, buf[i]);
        atomicMax(&S.maxc, buf[i]);
      }
      __syncthreads();
      base = S.base;
      maxc = S.maxc;
    }
    return tk_select<BLOCK>(S, buf, n, k, base, maxc);
  }
  // the bin's entries, listed in the (zero) histogram's words
  pz_lds_u64* list = (pz_lds_u64*)S.hist;
  for (int i = tid; i < n; i += BLOCK) {
    const uint64_t c = buf[i];
    if ((uint32_t)(c >> 53) == bin) list[atomicAdd(&S.ntop, 1)] = c;
  }
  __syncthreads();
  if (tid < cnt) {
    const uint64_t c = list[tid];
    const int r = tk_rank(list, cnt, c);
    if (r == need - 1) S.base = c;
  }
  __syncthreads();
  const uint64_t thr = S.base;
  for (int j = tid; j < 2 * cnt; j += BLOCK) S.hist[j] = 0u;
  __syncthreads();
  return thr;
}

// Element j (0..15) of a group's registers: a[j >> 2][j & 3] by selects
// (indexing the register array by a run-time value would go through scratch).
__device__ __forceinline__ float tk_pick(const float (&a)[TK_U][4], uint32_t j) {
  float r[TK_U];
#pragma unroll
  for (int u = 0; u < TK_U; u++) {
    const float lo = (j & 1u) ? a[u][1] : a[u][0];
    const float hi = (j & 1u) ? a[u][3] : a[u][2];
    r[u] = (j & 2u) ? hi : lo;
  }
  const float lo = (j & 4u) ? r[1] : r[0];
  const float hi = (j & 4u) ? r[3] : r[2];
  return (j & 8u) ? hi : lo;
}

// Processes one group of tiles: history members take their penalised logit
// in place (rare lanes, a divergent branch), then every element passing the
// raw bound is keyed and appended to buf, with one LDS atomic per wave and
// one loop trip per candidate of the busiest lane.  lmax tracks the lane's
// largest appended candidate.
template <bool DIV, bool COMP>
__device__ __forceinline__ void tk_group(TopkShared& S, pz_lds_u64* buf, const PzPenalty& P,
                                         const PzTemp& T, int V, int t0, int ntiles,
                                         float (&a)[TK_U][4], const TkRaw& rb, uint64_t& lmax) {
  const int lane = threadIdx.x & (PZ_WAVE - 1);
  uint32_t vm[TK_U];
#pragma unroll
  for (int u = 0; u < TK_U; u++) {
    const int lim = t0 + u < ntiles ? V - pz_tile_e0(t0 + u) : 0;  // row elements in the float4
    vm[u] = lim >= 4 ? 0xfu : (lim > 0 ? (1u << lim) - 1u : 0u);
  }
  const int e00 = pz_tile_e0(t0);
  if (P.active) {
    // the four bitmap reads are issued together (clamped into the bitmap;
    // bits of elements past the end are masked by vm)
    uint32_t pb = 0;
#pragma unroll
    for (int u = 0; u < TK_U; u++) {
      const int e0 = pz_tile_e0(t0 + u);
      pb |= ((P.bitmap[(e0 < V ? e0 : V - 1) >> 5] >> (e0 & 31)) & vm[u]) << (4 * u);
    }
    while (pb) {  // one trip per history member of the busiest lane
      const uint32_t j = (uint32_t)__builtin_ctz(pb);
      pb &= pb - 1u;
      const int id = e00 + (int)(j >> 2) * PZ_TILE + (int)(j & 3u);
      const float y = pz_penalize_inline(tk_pick(a, j), id, P.rep, P.pres, P.freq, P.hcap,
                                         P.hkey, P.hcnt);
#pragma unroll
      for (int u = 0; u < TK_U; u++)
#pragma unroll
        for (int c = 0; c < 4; c++) a[u][c] = j == (uint32_t)(4 * u + c) ? y : a[u][c];
    }
  }
  uint32_t want = 0;
#pragma unroll
  for (int u = 0; u < TK_U; u++) {
    const int e0 = pz_tile_e0(t0 + u);
    uint32_t nib = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float xv = a[u][c];
      const bool w = COMP ? (xv >= rb.hi) | ((xv >= rb.lo) & (e0 + c <= rb.idmax))
                          : xv >= rb.lo;
      nib |= (w ? 1u : 0u) << c;
    }
    want |= (nib & vm[u]) << (4 * u);
  }
  if (__ballot(want != 0u) == 0) return;
  const uint32_t cnt = (uint32_t)__builtin_popcount(want);
  const uint32_t incl = pz_wave_scan_u32(cnt);
  const uint32_t total = pz_readlane_u32(incl, 63);
  int base = 0;
  if (lane == 0) base = atomicAdd(&S.count, (int)total);
  base = __builtin_amdgcn_readfirstlane(base);
  int slot = base + (int)(incl - cnt);
  while (want) {
    const uint32_t j = (uint32_t)__builtin_ctz(want);
    want &= want - 1u;
    const int id = e00 + (int)(j >> 2) * PZ_TILE + (int)(j & 3u);
    const uint64_t cc = comp_of(tk_key(tk_temper<DIV>(tk_pick(a, j), T) + 0.0f), id);
    if (slot < TOPK_CAP) buf[slot] = cc;
    lmax = cc > lmax ? cc : lmax;
    slot++;
  }
}

// One streaming pass over the row.  The first group is in a on entry.
// sched_barrier keeps each group's loads below the processing of the group
// whose registers they reuse (hoisted above it, the loaded values would need
// registers of their own and copies at every iteration); the next group's
// loads are issued unconditionally (past the end they re-read the last
// tile), so the wait before each group counts exactly the group behind it.
template <bool VEC, bool DIV, bool COMP>
__device__ __forceinline__ void tk_pass(TopkShared& S, pz_lds_u64* buf, const PzPenalty& P,
                                        const PzTemp& T, const float* x, int V, int ntiles,
                                        float (&a)[TK_U][4], float (&b)[TK_U][4],
                                        const TkRaw& rb, uint64_t& lmax) {
  for (int t0 = 0;; t0 += 2 * TK_U) {
    tk_load<VEC>(x, V, t0 + TK_U, ntiles, b);
    tk_group<DIV, COMP>(S, buf, P, T, V, t0, ntiles, a, rb, lmax);
    if (t0 + TK_U >= ntiles) break;
    __builtin_amdgcn_sched_barrier(0);
    tk_load<VEC>(x, V, t0 + 2 * TK_U, ntiles, a);
    tk_group<DIV, COMP>(S, buf, P, T, V, t0 + TK_U, ntiles, b, rb, lmax);
    if (t0 + 2 * TK_U >= ntiles) break;
    __builtin_amdgcn_sched_barrier(0);
  }
  tk_drain(a);
  tk_drain(b);
}

__device__ __forceinline__ void tk_draw(TopkShared& S, const pz_lds_u64* res, int m, int k,
                                        const pz_row_params_dev& prm, float uu, int row,
                                        int32_t* __restrict__ ids_out,
                                        float* __restrict__ p_out);

// The k survivors of buf[0..n) (distinct candidates in [base, maxc]) in
// order, then the k-slot softmax, top-p cut-off and draw of row `row` (wave
// 0; uu is the row's uniform in thread 0).  Every thread calls it.
template <int BLOCK>
__device__ __forceinline__ void tk_finish(TopkShared& S, pz_lds_u64* buf, int n, int k,
                                          uint64_t base, uint64_t maxc,
                                          const pz_row_params_dev& prm, float uu, int row,
                                          int32_t* __restrict__ ids_out,
                                          float* __restrict__ p_out) {
  const int tid = threadIdx.x;
  const uint64_t thr = n > k ? tk_select_bin<BLOCK>(S, buf, n, k, base, maxc) : 0ull;
  if (tid == 0) S.ntop = 0;
  __syncthreads();
  for (int i = tid; i < n; i += BLOCK) {
    const uint64_t c = buf[i];
    if (c >= thr) S.top[atomicAdd(&S.ntop, 1)] = c;
  }
  __syncthreads();
  const int m = S.ntop;  // min(n, k)
  const pz_lds_u64* res;
  if (m <= TK_RANK_MAX) {
    // rank = number of survivors above; all distinct
    const pz_lds_u64* top = (const pz_lds_u64*)S.top;
    if (tid < m) {
      const uint64_t c = top[tid];
      buf[tk_rank(top, m, c)] = c;
    }
    res = buf;
  } else {
    int N = 1;
    while (N < m) N <<= 1;
    pz_lds_u64* top = (pz_lds_u64*)S.top;
    for (int i = m + tid; i < N; i += BLOCK) top[i] = 0ull;  // below any key
    __syncthreads();
    pz_bitonic_desc<BLOCK>(top, N);
    res = top;
  }
  __syncthreads();
  tk_draw(S, res, m, k, prm, uu, row, ids_out, p_out);
}

// ---- 5. softmax over k slots, cut-off and draw (wave 0) of the m <= k
// survivors res[0..m) in order (unfilled slots are (-1e30, -1)).
__device__ __forceinline__ void tk_draw(TopkShared& S, const pz_lds_u64* res, int m, int k,
                                        const pz_row_params_dev& prm, float uu, int row,
                                        int32_t* __restrict__ ids_out,
                                        float* __restrict__ p_out) {
  const int tid = threadIdx.x;
  const int lane = tid & (PZ_WAVE - 1);
  // pv holds the
  // probabilities, cv their sequential cumulative sums (the cut-off scan of
  // top_p.c:80-88 and the draw's cdf add the same terms in the same order).
  // Lane l owns slots l, l+64, ... of pv; cv is read across lanes only after
  // the scan that wrote it (same wave, program order).
  if (tid < PZ_WAVE) {
    tk_lds_f32* pv = (tk_lds_f32*)S.hist;             // k <= 1024 probabilities
    tk_lds_f32* cv = (tk_lds_f32*)S.hist + TOPK_MAXK;  // and cumulative sums
    const pz_lds_u64* et = (const pz_lds_u64*)S.etab;
    const float v0 = m > 0 ? pz_unkey((uint32_t)(res[0] >> 32)) : -1e30f;
    // e_i = expf(v_i - v0), then the sequential sum
    float sum = 0.0f;
    for (int c0 = 0; c0 < k; c0 += PZ_WAVE) {
      const int i = c0 + lane;
      float e = 0.0f;
      if (i < k) {
        const float v = i < m ? pz_unkey((uint32_t)(res[i] >> 32)) : -1e30f;
        e = pz_expf_tab(v - v0, et);
        pv[i] = e;
      }
      sum = pz_seq_sum_lanes(sum, e, k - c0);
    }
    float cum = 0.0f;
    for (int c0 = 0; c0 < k; c0 += PZ_WAVE) {
      const int i = c0 + lane;
      float p = 0.0f;
      if (i < k) p = pv[i] / sum;
      const float cs = pz_seq_scan_lanes(cum, p, k - c0);
      if (i < k) {
        pv[i] = p;
        cv[i] = cs;
      }
      cum = pz_readlane_f(cs, PZ_WAVE - 1);
    }
    const float ur = pz_readlane_f(uu, 0);
    const bool chain = prm.top_p > 0.0f && prm.top_p < 1.0f;
    int cutoff = k;
    float r = ur;
    if (chain) {
      // first slot with cum >= top_p; the truncated mass is the sequential
      // sum of the same slots (top_p.c:91-93), i.e. cum there
      int found = -1;
      for (int c0 = 0; c0 < k && found < 0; c0 += PZ_WAVE) {
        const int i = c0 + lane;
        const uint64_t hit = __ballot(i < k && cv[i] >= prm.top_p);
        if (hit) found = c0 + __ffsll((long long)hit) - 1;
      }
      if (found >= 0) cutoff = found + 1;
      r = ur * cv[cutoff - 1];  // every lane reads the same word
    }
    // draw: first slot < cutoff with r < cdf, else slot 0
    int pick = 0;
    for (int c0 = 0; c0 < cutoff; c0 += PZ_WAVE) {
      const int i = c0 + lane;
      const uint64_t hit = __ballot(i < cutoff && r < cv[i]);
      if (hit) {
        pick = c0 + __ffsll((long long)hit) - 1;
        break;
      }
    }
    if (lane == 0) {
      ids_out[row] = pick < m ? id_of(res[pick]) : -1;
      if (p_out) p_out[row] = pv[pick];
    }
  }
}

template <int BLOCK, bool VEC, bool DIV>
__global__ __launch_bounds__(BLOCK) void k_topk(
    const float* __restrict__ logits, long ld, int V, const int32_t* __restrict__ rows,
    const pz_row_params_dev* __restrict__ params, int n_params,
    const int32_t* __restrict__ hist, int H, int hcap, size_t pen_bytes,
    const float* __restrict__ u, int32_t* __restrict__ ids_out, float* __restrict__ p_out) {
  extern __shared__ __align__(16) char lds[];
  __shared__ TopkShared S;
  const int row = pz_row_of(rows, blockIdx.x);
  const int tid = threadIdx.x;
  const int lane = tid & (PZ_WAVE - 1);
  const float* x = logits + (long)row * ld;
  const int ntiles = pz_tiles(V);
  const int32_t* hrow = hist ? hist + (long)row * H : nullptr;

  // ---- 0. history ids, expf table and the first group of tiles in flight
  const int hid = (hrow && tid < H) ? hrow[tid] : -1;
  const uint64_t tab = tid < 32 ? pz_exp2_tab[tid] : 0ull;
  float a[TK_U][4], b[TK_U][4];
  tk_load<VEC>(x, V, 0, ntiles, a);
  float uu = 0.0f;
  if (tid == 0) uu = u[row];

  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  pz_lds_u64* buf = (pz_lds_u64*)(lds + pen_bytes);

  // ---- 1. penalty tables and the penalised values of the distinct history ids
  PzPenalty P;
  pz_penalty_setup<BLOCK>(P, lds, V, hcap, hrow != nullptr && H > 0, prm);
  for (int j = tid; j < HBINS; j += BLOCK) S.hist[j] = 0u;
  if (tid == 0) {
    S.count = 0;
    S.maxc = 0ull;
  }
  if (tid < 32) S.etab[tid] = tab;
  __syncthreads();
  if (P.active) {
    pz_penalty_insert(P, lds, V, hid, nullptr, nullptr);
    for (int j = tid + BLOCK; j < H; j += BLOCK)
      pz_penalty_insert(P, lds, V, hrow[j], nullptr, nullptr);
    __syncthreads();
  }
  const PzTemp T = PzTemp::of(prm);
  const int k = prm.top_k;

  // ---- 2. the first tile as a sample -> lower bound on the k-th key
  {
    const int e0 = pz_tile_e0(0);
    const uint32_t pen = (P.active && e0 < V) ? pz_pen_nibble(P, e0) : 0u;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float y = tk_temper<DIV>(a[0][c], T);
      if (e0 + c < V && y > -1e30f && !((pen >> c) & 1u))
        atomicAdd(&S.hist[pz_key(y) >> 21], 1u);
    }
  }
  __syncthreads();
  if (tid < PZ_WAVE) {
    uint32_t bin = 0, above = 0, cnt = 0;
    // fewer than k valid in the sample: keep every valid value
    const bool found = tk_find_bin((tk_lds_u32*)S.hist, (uint32_t)k, bin, above, cnt);
    tk_publish<DIV>(S, found ? (uint64_t)(bin << 21) << 32 : 0ull, T);
  }
  __syncthreads();

  // ---- 3. stream the row, rescanning with a tighter bound on overflow
  uint64_t bd;
  for (;;) {
    bd = S.thr;
    TkRaw rb;
    rb.lo = S.rlo;
    rb.hi = S.rhi;
    rb.idmax = S.ridmax;
    uint64_t lmax = 0ull;
    if ((uint32_t)bd == 0u)
      tk_pass<VEC, DIV, false>(S, buf, P, T, x, V, ntiles, a, b, rb, lmax);
    else
      tk_pass<VEC, DIV, true>(S, buf, P, T, x, V, ntiles, a, b, rb, lmax);
    // one LDS atomic per wave for the largest candidate
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint64_t o = __shfl_xor(lmax, off, PZ_WAVE);
      lmax = o > lmax ? o : lmax;
    }
    if (lane == 0 && lmax != 0ull) atomicMax(&S.maxc, lmax);
    __syncthreads();
    if (S.count <= TOPK_CAP) break;
    // the buffer holds TOPK_CAP >= k candidates of the row: its k-th largest
    // (key, id) bounds the row's k-th largest from below
    const uint64_t thr = tk_select_bin<BLOCK>(S, buf, TOPK_CAP, k, bd, S.maxc);
    if (tid < PZ_WAVE) tk_publish<DIV>(S, thr, T);
    if (tid == 0) {
      S.count = 0;
      S.maxc = 0ull;
    }
    tk_load<VEC>(x, V, 0, ntiles, a);
    __syncthreads();
  }

  // ---- 4./5. the k survivors in order, softmax, cut-off and draw
  tk_finish<BLOCK>(S, buf, S.count, k, bd, S.maxc, prm, uu, row, ids_out, p_out);
}



// Uniforms of a small batch passed by value.
struct PzUArg {
  float v[8];
  int n;  // rows 0..n-1 take v[row]
};

// One row split over gridDim.x <= 64 workgroups of 4096 ids (one tile) each.
// cand: the row's candidate area (`room` entries per workgroup, room >= k;
// for k <= TK_WM exactly the range's min(n, k) largest, in descending
// order, else a superset of its k largest), counts: entries each workgroup
// wrote ([rows][gridDim.x]); arrive: the rows' arrival counters (zero
// between launches).
template <int BLOCK, bool VEC, bool DIV>
__global__ __launch_bounds__(BLOCK) void k_topk_split(
    const float* __restrict__ logits, long ld, int V, const int32_t* __restrict__ rows,
    const pz_row_params_dev* __restrict__ params, int n_params,
    const int32_t* __restrict__ hist, int H, int hcap, size_t pen_bytes,
    const float* __restrict__ u, int32_t* __restrict__ ids_out, float* __restrict__ p_out,
    uint64_t* __restrict__ cand, int capg, int room, uint32_t* __restrict__ counts,
    uint32_t* __restrict__ arrive, PzUArg ua) {
  static_assert(BLOCK >= TK_WM_WAVES * PZ_WAVE && TK_WM_WAVES * 16 == PZ_WAVE, "merge waves");
  extern __shared__ __align__(16) char lds[];
  __shared__ TopkShared S;
  __shared__ int last_sh;
  const int sl = blockIdx.x, S_row = gridDim.x;
  const int row = pz_row_of(rows, blockIdx.y);
  const int tid = threadIdx.x;
  const int lane = tid & (PZ_WAVE - 1);
  const float* x = logits + (long)row * ld;
  const int32_t* hrow = hist ? hist + (long)row * H : nullptr;
  const int lo = sl * PZ_TILE;
  const int hi = lo + PZ_TILE < V ? lo + PZ_TILE : V;
  const int e0 = lo + 4 * tid;
  float a[4];
  const int n = pz_load4<VEC, false>(x, hi, e0, a);
  const uint64_t tab = tid < 32 ? pz_exp2_tab[tid] : 0ull;
  // the uniform: from the launch's arguments for the first rows of a small
  // batch (no memory read on the merge's path), else from u
  float uu = 0.0f;
  if (tid == 0) uu = row < ua.n ? ua.v[row] : u[row];
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  pz_lds_u64* buf = (pz_lds_u64*)(lds + pen_bytes);
  PzPenalty P;
  pz_penalty_setup_range<BLOCK>(P, lds, lo, hi, hcap, hrow != nullptr && H > 0, prm);
  for (int j = tid; j < HBINS; j += BLOCK) S.hist[j] = 0u;
  if (tid == 0) {
    S.count = 0;
    S.maxc = 0ull;
    S.base = ~0ull;
  }
  if (tid < 32) S.etab[tid] = tab;
  __syncthreads();
  if (P.active) {
    for (int j = tid; j < H; j += BLOCK) pz_penalty_insert(P, lds, V, hrow[j], nullptr, nullptr);
    __syncthreads();
  }
  const PzTemp T = PzTemp::of(prm);
  const int k = prm.top_k;
  // every valid element of the range (y > -1e30, NaN never), keyed
  uint64_t cc[4];
  uint32_t want = 0;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    float y = a[c];
    if (c < n && P.active && pz_pen_member(P, e0 + c)) y = pz_penalize(P, y, e0 + c);
    y = tk_temper<DIV>(y, T);
    cc[c] = comp_of(tk_key(y + 0.0f), e0 + c);
    if (c < n && y > -1e30f) want |= 1u << c;
  }
  {
    const uint32_t cnt = (uint32_t)__builtin_popcount(want);
    const uint32_t incl = pz_wave_scan_u32(cnt);
    const uint32_t total = pz_readlane_u32(incl, 63);
    int base = 0;
    if (lane == 0 && total) base = atomicAdd(&S.count, (int)total);
    base = __builtin_amdgcn_readfirstlane(base);
    int slot = base + (int)(incl - cnt);
#pragma unroll
    for (int c = 0; c < 4; c++)
      if ((want >> c) & 1u) buf[slot++] = cc[c];
  }
  __syncthreads();
  // a superset of this range's k largest: every key in the bins (top 11 key
  // bits) from the one holding the k-th largest up, when that fits the
  // range's room, else exactly the k largest
  const int nc = S.count;
  uint64_t thr = 0ull;
  if (nc > k) {
    for (int i = tid; i < nc; i += BLOCK) atomicAdd(&S.hist[(uint32_t)(buf[i] >> 53)], 1u);
    __syncthreads();
    if (tid < PZ_WAVE) {
      uint32_t bin = 0, above = 0, cnt = 0;
      tk_find_bin((tk_lds_u32*)S.hist, (uint32_t)k, bin, above, cnt);  // zeroes S.hist
      if (tid == 0) {
        S.bin = bin;
        S.nbin = (int)(above + cnt);
      }
    }
    __syncthreads();
    // k <= TK_WM: up to TK_RANK_MAX entries are ranked below, else room bounds them
    const int lim = k <= TK_WM ? TK_RANK_MAX : room;
    thr = S.nbin <= lim ? (uint64_t)S.bin << 53
                        : tk_select_bin<BLOCK>(S, buf, nc, k, ~0ull, 0ull);
  }
  uint64_t* out = cand + (size_t)row * capg + (size_t)sl * room;
  if (tid == 0) S.ntop = 0;
  __syncthreads();
  if (k <= TK_WM) {
    // the range's min(nc, k) largest, in descending order: the survivors
    // (at most TK_RANK_MAX) each placed by its rank among them (keys distinct)
    for (int i = tid; i < nc; i += BLOCK) {
      const uint64_t c = buf[i];
      if (c >= thr) S.top[atomicAdd(&S.ntop, 1)] = c;
    }
    __syncthreads();
    const int nt = S.ntop;
    if (tid < nt) {
      const uint64_t c = S.top[tid];
      const int r = tk_rank((const pz_lds_u64*)S.top, nt, c);
      if (r < k) out[r] = c;
    }
    if (tid == 0) counts[(size_t)row * S_row + sl] = (uint32_t)(nt < k ? nt : k);
  } else {
    for (int i = tid; i < nc; i += BLOCK) {
      const uint64_t c = buf[i];
      if (c >= thr) out[atomicAdd(&S.ntop, 1)] = c;
    }
    __syncthreads();
    if (tid == 0) counts[(size_t)row * S_row + sl] = (uint32_t)S.ntop;
  }
  // the last workgroup of the row merges the ranges' candidates
  if (!pz_sp_arrive(arrive, row, S_row, &last_sh)) return;
  if (tid == 0) {
    S.count = 0;
    S.maxc = 0ull;
    S.base = ~0ull;
  }
  __syncthreads();
  const uint64_t* all = cand + (size_t)row * capg;
  // the ranges' counts and their prefix (at most 64 ranges: one wave)
  __shared__ int off[65];
  if (tid < PZ_WAVE) {
    const int c = tid < S_row ? (int)counts[(size_t)row * S_row + tid] : 0;
    off[tid + 1] = (int)pz_wave_scan_u32((uint32_t)c);
    if (tid == 0) off[0] = 0;
  }
  __syncthreads();
  const int total = off[S_row];  // at most TOPK_CAP: S * room entries
  if (k <= TK_WM) {
    // every list is its range's largest (at most 64) in descending order:
    // wave w merges lists w, w + 4, ... (slot j holds list w + 4j, read
    // descending in even slots and ascending in odd ones) by a tree of wave
    // merges whose left inputs are descending and right inputs ascending,
    // then wave 0 merges the four waves' lists the same way
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint64_t mine = 0ull;
    if (wv < TK_WM_WAVES) {
      uint64_t r[16];
#pragma unroll
      for (int j = 0; j < 16; j++) {
        const int i = wv + TK_WM_WAVES * j;
        const int cnt = i < S_row ? off[i + 1] - off[i] : 0;
        const int e = (j & 1) ? 63 - lane : lane;
        r[j] = e < cnt ? all[(size_t)i * room + e] : 0ull;
      }
      const int nl = S_row > wv ? (S_row - wv + TK_WM_WAVES - 1) / TK_WM_WAVES : 0;
#pragma unroll
      for (int s = 1; s < 16; s <<= 1) {
#pragma unroll
        for (int p = 0; p < 16 / (2 * s); p++) {
          const bool desc = (p & 1) == 0;
          if ((2 * p + 1) * s < nl)
            r[p] = pz_wave_merge_u64(r[2 * p], r[2 * p + 1], desc);
          else if (2 * p * s < nl)  // the left subtree alone: descending
            r[p] = desc ? r[2 * p] : pz_lane_rev_u64(r[2 * p]);
          else
            r[p] = 0ull;
        }
      }
      mine = r[0];
      if (wv > 0) S.top[wv * PZ_WAVE + lane] = mine;
    }
    __syncthreads();
    pz_sp_rearm(arrive, row);
    const int m = total < k ? total : k;
    if (tid < PZ_WAVE) {
      const pz_lds_u64* t = (const pz_lds_u64*)S.top;
      const uint64_t w1 = t[PZ_WAVE + 63 - lane], w2 = t[2 * PZ_WAVE + lane];
      const uint64_t w3 = t[3 * PZ_WAVE + 63 - lane];
      const uint64_t m01 = pz_wave_merge_u64(mine, w1, true);
      const uint64_t m23 = pz_wave_merge_u64(w2, w3, false);
      const uint64_t fin = pz_wave_merge_u64(m01, m23, true);
      if (lane < m) S.top[lane] = fin;
    }
    __syncthreads();
    tk_draw(S, (const pz_lds_u64*)S.top, m, k, prm, uu, row, ids_out, p_out);
    return;
  }
  // up to four entries per thread, their loads issued together
  uint64_t got[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int f = tid + q * BLOCK;
    got[q] = 0ull;
    if (f < total) {
      int si = 0;
      while (off[si + 1] <= f) si++;
      got[q] = all[(size_t)si * room + (f - off[si])];
    }
  }
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int f = tid + q * BLOCK;
    if (f < total) buf[f] = got[q];
  }
  __syncthreads();
  pz_sp_rearm(arrive, row);
  tk_finish<BLOCK>(S, buf, total, k, ~0ull, 0ull, prm, uu, row, ids_out, p_out);
}

}  // namespace

// Rows split over workgroups when the launch would otherwise occupy few CUs
// and the ranges' candidates fit one merge buffer.
constexpr int TOPK_SPLIT_MAX_WG = 256;

template <bool VEC, bool DIV>
static int launch_topk_split_t(const pz_launch& L, int n_rows, const int32_t* d_rows, int S,
                               int kmax) {
  const size_t pen =
      L.pen_any ? (pz_penalty_lds_bytes(PZ_TILE, L.hcap) + 15) & ~(size_t)15 : 0;
  const size_t lds = pen + (size_t)TOPK_CAP * 8;
  if ((int)(lds + sizeof(TopkShared) + 16) > L.max_lds) return -2;
  auto kern = k_topk_split<TOPK_BLOCK, VEC, DIV>;
  if (lds > 65536 &&
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return -1;
  // each range's room in the candidate area: the merge buffer (and the
  // row's area) split evenly, at least kmax (the caller checked S * kmax)
  int room = TOPK_CAP / S;
  if (room > L.ws.capg / S) room = L.ws.capg / S;
  if (room < kmax) return -2;
  PzUArg ua;
  ua.n = 0;
  if (L.h_u && L.B <= 8) {
    for (int b = 0; b < L.B; b++) ua.v[b] = L.h_u[b];
    ua.n = L.B;
  }
  hipLaunchKernelGGL(kern, dim3(S, n_rows), dim3(TOPK_BLOCK), lds, L.stream, L.logits, L.ld,
                     L.V, d_rows, L.params, L.n_params, L.hist, L.H, L.hcap, pen, L.u, L.ids,
                     L.p_out, L.ws.keys, L.ws.capg, room, L.ws.slice_f, L.ws.arrive, ua);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <bool VEC, bool DIV>
static int launch_topk_t(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  const size_t pen = L.pen_any ? (pz_penalty_lds_bytes(L.V, L.hcap) + 15) & ~(size_t)15 : 0;
  const size_t lds = pen + (size_t)TOPK_CAP * 8;
  if ((int)(lds + sizeof(TopkShared)) > L.max_lds) return -2;
  auto kern = k_topk<TOPK_BLOCK, VEC, DIV>;
  if (lds > 65536 &&
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(kern, dim3(n_rows), dim3(TOPK_BLOCK), lds, L.stream, L.logits, L.ld, L.V,
                     d_rows, L.params, L.n_params, L.hist, L.H, L.hcap, pen, L.u, L.ids,
                     L.p_out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int pz_launch_topk(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  if (n_rows <= 0) return 0;
  const bool vec = (L.ld % 4 == 0) && (((uintptr_t)L.logits & 15) == 0);
  // the largest k among the rows decides whether the split's merge fits
  // (k is resolved per row on the host: the host passes it as kmax)
  const int S = pz_tiles(L.V);
  // at most 64 ranges: the merge scans their counts in one wave
  if (S >= 2 && S <= PZ_WAVE && (long)S * n_rows <= TOPK_SPLIT_MAX_WG && L.kmax > 0 &&
      (long)S * L.kmax <= TOPK_CAP && (long)S * L.kmax <= L.ws.capg && L.ws.keys) {
    if (L.temp_div)
      return vec ? launch_topk_split_t<true, true>(L, n_rows, d_rows, S, L.kmax)
                 : launch_topk_split_t<false, true>(L, n_rows, d_rows, S, L.kmax);
    return vec ? launch_topk_split_t<true, false>(L, n_rows, d_rows, S, L.kmax)
               : launch_topk_split_t<false, false>(L, n_rows, d_rows, S, L.kmax);
  }
  if (L.temp_div)
    return vec ? launch_topk_t<true, true>(L, n_rows, d_rows)
               : launch_topk_t<false, true>(L, n_rows, d_rows);
  return vec ? launch_topk_t<true, false>(L, n_rows, d_rows)
             : launch_topk_t<false, false>(L, n_rows, d_rows);
}
