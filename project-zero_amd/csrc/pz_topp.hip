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
// Design (one 1024-thread workgroup per row):
//   pass 1  (HBM)   row maximum + per-segment estimates of the normaliser;
//   pass 2  (L2)    exact e = expf(x - max) (glibc-identical pz_expf) of every
//                   candidate -> integer segment records at the predicted
//                   binade (pz_exact.h) + an LDS histogram of e (1/128
//                   binade bins);
//   walk    (wave 0) the exact sequential normaliser; meanwhile wave 1 picks,
//                   from the histogram, the smallest set of top bins whose
//                   estimated mass clears top_p with margin;
//   pass 3  (L2)    gathers the candidates with p >= p(threshold) into LDS as
//                   (p, ~id) keys -- a prefix of the reference's sort order;
//   sort + exact cumulative walk + draw (binary search over the stored sums).
// A row whose selected set does not fit in LDS, or whose exact cumulative
// does not reach top_p inside it, is queued for the fallback kernel, which
// sorts every candidate of the row in its global scratch slot.
#include <limits.h>

#include "pz_device.h"
#include "pz_exact.h"
#include "pz_launch.h"
#include "pz_rowpass.h"
#include "pz_sort.h"

namespace {

// Histogram of e in (0, 1]: bins of 1/128 binade, e >= 2^-29 (candidates are
// >= expf(-20) ~ 2.06e-9); smaller values fall in bin 0.
constexpr int EBIN_BASE = 98 << 7;
constexpr int EBINS = (127 << 7) - EBIN_BASE + 1;
constexpr int TOPP_CAP_MAX = 8192;
constexpr int EBINS_BYTES = ((EBINS * 4 + 15) / 16) * 16;
// Gathered lists of at least TOPP_BINSORT_MIN keys are ordered by a counting
// sort over PBINS bins of p (1/128 binade each, 32 binades below 1.0) and a
// rank count inside each bin; smaller ones by a bitonic sort.
constexpr int PBINS = 4 * PZ_RB;
constexpr int TOPP_BINSORT_MIN = 1024;
constexpr int TOPP_BIN_MAX = 256;  // larger bins: bitonic sort

__device__ __forceinline__ int ebin(float e) {
  const int b = (int)(__float_as_uint(e) >> 16) - EBIN_BASE;
  return b < 0 ? 0 : (b >= EBINS ? EBINS - 1 : b);
}
__device__ __forceinline__ float ebin_lo(int b) {
  return __uint_as_float((uint32_t)(b + EBIN_BASE) << 16);
}
__device__ __forceinline__ float ebin_mid(int b) {
  return __uint_as_float(((uint32_t)(b + EBIN_BASE) << 16) | 0x8000u);
}

__device__ __forceinline__ uint64_t topp_key(float p, int id) {
  return ((uint64_t)__float_as_uint(p) << 32) | (uint64_t)(0xffffffffu - (uint32_t)id);
}
__device__ __forceinline__ int key_id(uint64_t k) { return (int)(0xffffffffu - (uint32_t)k); }
__device__ __forceinline__ float key_p(uint64_t k) { return __uint_as_float((uint32_t)(k >> 32)); }

struct ToppShared {
  PzPass1Shared p1;
  uint32_t wtot[PZ_RB / 64];
  uint32_t bmax;
  float sum;
  int bsel;
  uint32_t nsel;
  int count;
  int over;
  int cutoff;
  int first;
};

// Wave-aggregated append of up to one key per lane into buf (capacity cap).
__device__ __forceinline__ void append_key(int* count, int* over, uint64_t* buf, int cap,
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

__device__ __forceinline__ void nucleus_draw(const uint64_t* keys, const float* cum, int cutoff, float uu,
                             int32_t* id_out, float* p_out) {
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

// The (p desc, id asc) order of keys[0..m) without moving them: a counting
// sort by p bin into perm1 (any order inside a bin), then each key's rank
// inside its bin puts its slot at its sorted position in perm2.  Returns
// false, having done nothing usable, when a bin holds more than
// TOPP_BIN_MAX keys.  Every thread calls it.
__device__ __forceinline__ bool binned_order(const pz_lds_u64* keys, int m, pz_lds_u16* perm1,
                                             pz_lds_u16* perm2, pz_lds_u32b* bcnt,
                                             pz_lds_u32b* bstart, ToppShared& S) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int i = tid; i < PBINS; i += PZ_RB) bcnt[i] = 0u;
  if (tid == 0) S.bmax = 0u;
  __syncthreads();
  for (int i = tid; i < m; i += PZ_RB) atomicAdd((uint32_t*)&bcnt[pbin(keys[i])], 1u);
  __syncthreads();
  // exclusive scan over the bins; thread t owns bins 4t .. 4t+3
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
  if (lane == 63) S.wtot[w] = incl;
  if (lane == 0) atomicMax(&S.bmax, mx);
  __syncthreads();
  uint32_t run = incl - local;
  for (int j = 0; j < w; j++) run += S.wtot[j];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    bstart[4 * tid + j] = run;
    bcnt[4 * tid + j] = run;  // cursor
    run += c[j];
  }
  __syncthreads();
  if (S.bmax > (uint32_t)TOPP_BIN_MAX) return false;
  for (int i = tid; i < m; i += PZ_RB) {
    const uint32_t pos = atomicAdd((uint32_t*)&bcnt[pbin(keys[i])], 1u);
    perm1[pos] = (uint16_t)i;
  }
  __syncthreads();
  for (int j = tid; j < m; j += PZ_RB) {
    const int i = perm1[j];
    const uint64_t key = keys[i];
    const int q = pbin(key);
    const uint32_t b0 = bstart[q], b1 = bcnt[q];
    uint32_t r = 0;
    for (uint32_t x = b0; x < b1; x++) r += keys[perm1[x]] > key ? 1u : 0u;
    perm2[b0 + r] = (uint16_t)i;
  }
  __syncthreads();
  return true;
}

// The sorted probabilities (p of keys[perm[j]], j < m) as the terms of an
// exact-sum records pass: the values are exact, so every increment is too.
struct SortedTerms {
  typedef float Raw[4];
  const pz_lds_u64* keys;
  const pz_lds_u16* perm;
  int m;
  __device__ __forceinline__ int load(int e0, Raw& r) const {
#pragma unroll
    for (int c = 0; c < 4; c++) r[c] = e0 + c < m ? key_p(keys[perm[e0 + c]]) : 0.0f;
    const int n = m - e0;
    return n < 0 ? 0 : (n > 4 ? 4 : n);
  }
  __device__ __forceinline__ void prep(int, int, Raw& r, float (&a)[4]) const {
#pragma unroll
    for (int c = 0; c < 4; c++) a[c] = r[c];
  }
  __device__ __forceinline__ void observe(int, const Raw&, const float (&)[4]) {}
  __device__ __forceinline__ uint32_t inc(const Raw&, const float (&a)[4], int c, uint32_t g,
                                          uint32_t* cls) const {
    return pz_inc(a[c], g, cls);
  }
  __device__ __forceinline__ void cache_put(pz_lds_f32* base, const Raw& r,
                                            const float (&)[4]) const {
    pz_f4 q;
    q.x = r[0];
    q.y = r[1];
    q.z = r[2];
    q.w = r[3];
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
    load(pz_seg_e0(k), r);
#pragma unroll
    for (int c = 0; c < 4; c++) v[c] = r[c];
  }
};

// Cut-off and draw over the order in perm2 (top_p.c:80-105) with exact-sum
// records of the sorted probabilities: the cumulative walk stops at the
// first running sum >= top_p (the cut-off; its sum is the truncated mass),
// a second walk over the same records at the first running sum > r.
// Returns the picked sorted position, or -1 when the list is a strict prefix
// whose cumulative stays below top_p.  Every thread calls it; rec is LDS of
// pz_rec_bytes(m) bytes.
__device__ __forceinline__ int binned_pick(const pz_lds_u64* keys, const pz_lds_u16* perm2, int m,
                                           float top_p, bool all_gathered, float uu, char* rec,
                                           PzRecShared& RS, int* sh) {
  SortedTerms X;
  X.keys = keys;
  X.perm = perm2;
  X.m = m;
  const int ntiles = pz_tiles(m), nseg = ntiles * PZ_SEGS_PER_TILE;
  const PzRec REC = pz_rec_at(rec, nseg);
  pz_record_pass(X, ntiles, REC, RS, __builtin_inff());
  if (threadIdx.x < 64) {
    PzAcc st;
    st.n = 0;
    st.g = 1;
    const int hit = pz_rec_walk(st, REC, nseg, top_p, PZ_STOP_GE, X);
    int pick = -1;
    int cutoff = hit >= 0 && hit < m ? hit + 1 : -1;
    if (cutoff < 0 && all_gathered) cutoff = m;  // st then holds the whole sum
    if (cutoff > 0) {
      const float r = uu * pz_acc_value(st);  // trunc_sum: the cumulative at the cut-off
      PzAcc s2;
      s2.n = 0;
      s2.g = 1;
      const int d = pz_rec_walk(s2, REC, nseg, r, PZ_STOP_GT, X);
      pick = d >= 0 && d < cutoff ? d : 0;
    }
    if (threadIdx.x == 0) *sh = pick;
  }
  __syncthreads();
  return *sh;
}

// Candidate terms with the e histogram as observer.
template <bool VEC>
struct ToppTerms : PzExpTerms<PzRow<VEC>> {
  uint32_t* ehist;
  __device__ __forceinline__ void observe(int, const float (&)[4], const float (&a)[4]) {
#pragma unroll
    for (int c = 0; c < 4; c++)
      if (a[c] > 0.0f) atomicAdd(&ehist[ebin(a[c])], 1u);
  }
};

template <bool VEC>
__global__ __launch_bounds__(PZ_RB) void k_topp(
    const float* __restrict__ logits, long ld, int V, const int32_t* __restrict__ rows,
    const pz_row_params_dev* __restrict__ params, int n_params,
    const int32_t* __restrict__ hist, int H, int hcap, int pen_bytes, int cap,
    const float* __restrict__ u, int32_t* __restrict__ ids_out, float* __restrict__ p_out,
    pz_scratch sc) {
  extern __shared__ __align__(16) char lds[];
  __shared__ ToppShared S;
  __shared__ PzRecShared RS;
  __shared__ uint64_t etab[32];
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  pz_etab_fill((pz_lds_u64*)etab);  // ordered by pz_pass1's barriers
  const int row = pz_row_of(rows, blockIdx.x);
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

  PzRow<VEC> R;
  R.x = logits + (long)row * ld;
  R.V = V;
  R.T = PzTemp::of(prm);
  pz_penalty_build<PZ_RB>(R.P, lds, V, hcap, hist ? hist + (long)row * H : nullptr, H, prm);

  const int ntiles = pz_tiles(V), nseg = ntiles * PZ_SEGS_PER_TILE;
  char* reg = lds + pen_bytes;
  // phase A: records + e histogram; phase B (overlaid): gathered keys + sums
  uint32_t* ehist = reinterpret_cast<uint32_t*>(reg);
  const PzRec REC = pz_rec_at(reg + EBINS_BYTES, nseg);
  uint64_t* keys = reinterpret_cast<uint64_t*>(reg);
  float* cum = reinterpret_cast<float*>(keys + cap);

  for (int i = tid; i < EBINS; i += PZ_RB) ehist[i] = 0u;

  // ---- pass 1: maximum
  const float M = pz_pass1<8>(R, ntiles, S.p1);
  const float y0 = S.p1.y0;
  if (y0 != y0) {
    // max_val = NaN: no candidate passes, argmax of a row starting with NaN -> 0
    if (tid == 0) {
      ids_out[row] = 0;
      if (p_out) p_out[row] = 1.0f;
    }
    return;
  }
  if (!(M > -__builtin_inff() && M < __builtin_inff())) {
    // every e is expf(NaN): the sort leaves candidates in id order and no
    // comparison succeeds -> the first candidate, i.e. the first y == max
    if (tid == 0) S.first = INT_MAX;
    __syncthreads();
    int mine = INT_MAX;
    for (int t = 0; t < ntiles; t++) {
      float y[4];
      const int e0 = pz_tile_e0(t);
      const int n = R.get(e0, y);
      for (int c = 0; c < n; c++)
        if (y[c] == M && e0 + c < mine) mine = e0 + c;
    }
    atomicMin(&S.first, mine);
    __syncthreads();
    if (tid == 0) {
      ids_out[row] = S.first;
      if (p_out) p_out[row] = __builtin_nanf("");
    }
    return;
  }
  const float thr = M - 20.0f;

  // ---- records of the exact candidate terms (+ e histogram)
  ToppTerms<VEC> X;
  X.R = R;
  X.M = M;
  X.thr = thr;
  X.inv = 1.0f;
  X.as_p = false;
  X.et = et;
  X.ehist = ehist;
  pz_record_pass(X, ntiles, REC, RS, __builtin_inff());

  // ---- exact normaliser (wave 0) || nucleus bin selection (wave 1)
  if (w == 0) {
    PzAcc st;
    st.n = 0;
    st.g = 1;
    pz_rec_walk(st, REC, nseg, 0.0f, PZ_STOP_NONE, X);
    if (lane == 0) S.sum = pz_acc_value(st);
  } else if (w == 1) {
    float tot = 0.0f;
    uint32_t ncand = 0;
    for (int b = lane; b < EBINS; b += 64) {
      const uint32_t c = ehist[b];
      tot += (float)c * ebin_mid(b);
      ncand += c;
    }
    tot = pz_wave_sum(tot);
    ncand = pz_wave_sum_u32(ncand);
    const float goal = (prm.top_p * 1.006f + 2e-4f) * tot;
    float carry = 0.0f;
    uint32_t ccarry = 0;
    int bsel = 0;
    uint32_t nsel = ncand;
    for (int b0 = EBINS - 1; b0 >= 0; b0 -= 64) {
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
    if (lane == 0) {
      S.bsel = bsel;
      S.nsel = nsel;
    }
  }
  if (tid == 0) {
    S.count = 0;
    S.over = 0;
  }
  __syncthreads();

  const float inv = 1.0f / S.sum;  // top_p.c:72
  const bool all = S.bsel == 0;
  bool fallback = S.nsel > (uint32_t)cap;
  if (!fallback) {
    // ---- pass 3: gather every candidate with p >= p_thr (a prefix of the
    // (p desc, id asc) order) into LDS.  A cheap gate on y - M picks the
    // lanes' possible candidates (a superset: 0.01 below the bin edge); the
    // exact p of those is evaluated one candidate per lane per trip, and the
    // survivors are appended with one LDS atomic per wave per trip.
    const float e_lo = ebin_lo(S.bsel);
    const float p_thr = all ? 0.0f : e_lo * inv;
    const float dgate = all ? -__builtin_inff() : __logf(e_lo) - 0.01f;
    constexpr int U2 = 8;
    for (int t0 = 0; t0 < ntiles; t0 += U2) {
      float y[U2][4];
      int nv[U2];
#pragma unroll
      for (int uu = 0; uu < U2; uu++) {
        const int t = t0 + uu < ntiles ? t0 + uu : ntiles - 1;  // unconditional loads
        const int nl = R.load(pz_tile_e0(t), y[uu]);
        nv[uu] = t0 + uu < ntiles ? nl : 0;
      }
      uint32_t want = 0;
#pragma unroll
      for (int uu = 0; uu < U2; uu++) {
        const int e0 = pz_tile_e0(t0 + uu);
        R.apply(e0, nv[uu], y[uu]);
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const float yy = y[uu][c];
          const bool w = (c < nv[uu]) & (yy >= thr) & ((yy - M) >= dgate);
          want |= (w ? 1u : 0u) << (4 * uu + c);
        }
      }
      const int e00 = pz_tile_e0(t0);
      while (__ballot(want != 0u)) {
        bool take = false;
        uint64_t key = 0;
        if (want) {
          const uint32_t j = (uint32_t)__builtin_ctz(want);
          want &= want - 1u;
          float yy = y[0][0];
#pragma unroll
          for (int uu = 0; uu < U2; uu++)
#pragma unroll
            for (int c = 0; c < 4; c++)
              if (j == (uint32_t)(4 * uu + c)) yy = y[uu][c];
          const float p = pz_expf_l(yy - M, et) * inv;
          take = p >= p_thr;
          key = topp_key(p, e00 + (int)(j >> 2) * PZ_TILE + (int)(j & 3u));
        }
        append_key(&S.count, &S.over, keys, cap, take, key);
      }
    }
    __syncthreads();
    fallback = S.over != 0;
  }
  if (!fallback) {
    const int m = S.count;
    pz_lds_u64* lkeys = (pz_lds_u64*)keys;
    pz_lds_u16* perm1 = (pz_lds_u16*)cum;  // the running-sum area holds two u16 orders
    pz_lds_u16* perm2 = perm1 + cap;
    pz_lds_u32b* bcnt = (pz_lds_u32b*)(cum + cap);
    pz_lds_u32b* bstart = bcnt + PBINS;
    if (m >= TOPP_BINSORT_MIN && binned_order(lkeys, m, perm1, perm2, bcnt, bstart, S)) {
      // the bin arrays are free again: they hold the records of the sorted list
      const int pick = binned_pick(lkeys, perm2, m, prm.top_p, all, u[row], (char*)bcnt, RS,
                                   &S.cutoff);
      if (pick >= 0) {
        if (tid == 0) {
          const uint64_t k = lkeys[perm2[pick]];
          ids_out[row] = key_id(k);
          if (p_out) p_out[row] = key_p(k);
        }
        return;
      }
    } else {
      int N = 1;
      while (N < m) N <<= 1;
      for (int i = m + tid; i < N; i += PZ_RB) keys[i] = 0ull;
      __syncthreads();
      pz_bitonic_desc<PZ_RB>(lkeys, N);
      const int cutoff = nucleus_cutoff(keys, cum, m, prm.top_p, all, &S.cutoff);
      if (cutoff > 0) {
        if (tid == 0)
          nucleus_draw(keys, cum, cutoff, u[row], &ids_out[row], p_out ? &p_out[row] : nullptr);
        return;
      }
    }
  }
  // ---- queue the row for the fallback kernel
  if (tid == 0) {
    float* st = sc.row_stat + 4 * (long)row;
    st[0] = M;
    st[1] = inv;
    const int q = atomicAdd(&sc.counters[0], 1);
    sc.fb_list[q] = row;
  }
}

// Fallback: every candidate of the row, sorted in the workgroup's global
// scratch slot, then the same cumulative and draw.
template <bool VEC>
__global__ __launch_bounds__(PZ_RB) void k_topp_fallback(
    const float* __restrict__ logits, long ld, int V,
    const pz_row_params_dev* __restrict__ params, int n_params,
    const int32_t* __restrict__ hist, int H, int hcap, const float* __restrict__ u,
    int32_t* __restrict__ ids_out, float* __restrict__ p_out, pz_scratch sc) {
  extern __shared__ __align__(16) char lds[];
  __shared__ int count, over, cutoff_sh;
  __shared__ uint64_t etab[32];
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  pz_etab_fill((pz_lds_u64*)etab);
  __syncthreads();
  const int tid = threadIdx.x;
  const int n_fb = sc.counters[0];
  uint64_t* keys = sc.fb_keys + (size_t)blockIdx.x * sc.slot_n;
  float* cum = sc.fb_cum + (size_t)blockIdx.x * sc.slot_n;
  for (int q = blockIdx.x; q < n_fb; q += gridDim.x) {
    const int row = sc.fb_list[q];
    const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
    PzRow<VEC> R;
    R.x = logits + (long)row * ld;
    R.V = V;
    R.T = PzTemp::of(prm);
    pz_penalty_build<PZ_RB>(R.P, lds, V, hcap, hist ? hist + (long)row * H : nullptr, H, prm);
    const float M = sc.row_stat[4 * (long)row];
    const float inv = sc.row_stat[4 * (long)row + 1];
    const float thr = M - 20.0f;
    if (tid == 0) {
      count = 0;
      over = 0;
    }
    __syncthreads();
    const int ntiles = pz_tiles(V);
    for (int t = 0; t < ntiles; t++) {
      float y[4];
      const int e0 = pz_tile_e0(t);
      const int n = R.get(e0, y);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const bool want = c < n && y[c] >= thr;
        uint64_t key = 0;
        if (want) key = topp_key(pz_expf_l(y[c] - M, et) * inv, e0 + c);
        append_key(&count, &over, keys, sc.slot_n, want, key);
      }
    }
    __syncthreads();
    const int m = count;
    int N = 1;
    while (N < m) N <<= 1;
    for (int i = m + tid; i < N; i += PZ_RB) keys[i] = 0ull;
    __syncthreads();
    pz_bitonic_desc<PZ_RB>(keys, N);
    const int cutoff = nucleus_cutoff(keys, cum, m, prm.top_p, true, &cutoff_sh);
    if (tid == 0) nucleus_draw(keys, cum, cutoff, u[row], &ids_out[row], p_out ? &p_out[row] : nullptr);
    __syncthreads();
  }
  // the last workgroup out re-arms the queue for the next launch (every
  // workgroup has read counters[0] before it counts itself done)
  if (tid == 0) {
    __threadfence();
    if (atomicAdd(&sc.counters[1], 1) == (int)gridDim.x - 1) {
      atomicExch(&sc.counters[0], 0);
      atomicExch(&sc.counters[1], 0);
    }
  }
}

size_t topp_region_bytes(int V, int cap) {
  const size_t a = (size_t)EBINS_BYTES + pz_rec_bytes(V);
  // keys, running sums (or two u16 orders), then bin counts and starts or
  // the records of the sorted list
  const size_t bins = (size_t)PBINS * 8, recs = pz_rec_bytes(cap);
  const size_t b = (size_t)cap * 12 + (bins > recs ? bins : recs);
  return a > b ? a : b;
}

template <bool VEC>
int launch_topp_t(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  const int pen = L.pen_any ? (int)((pz_penalty_lds_bytes(L.V, L.hcap) + 15) & ~(size_t)15) : 0;
  const int fixed = (int)sizeof(ToppShared) + 64;
  int cap = TOPP_CAP_MAX;
  while (cap > 256 && pen + topp_region_bytes(L.V, cap) + fixed > (size_t)L.max_lds) cap >>= 1;
  const size_t lds = pen + topp_region_bytes(L.V, cap);
  if (lds + fixed > (size_t)L.max_lds) return -2;
  auto kern = k_topp<VEC>;
  auto fb = k_topp_fallback<VEC>;
  if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return -1;
  if (pen > 65536 && hipFuncSetAttribute((const void*)fb, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         pen) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(kern, dim3(n_rows), dim3(PZ_RB), lds, L.stream, L.logits, L.ld, L.V, d_rows,
                     L.params, L.n_params, L.hist, L.H, L.hcap, pen, cap, L.u, L.ids, L.p_out,
                     L.sc);
  const int fb_grid = n_rows < L.sc.fb_slots ? n_rows : L.sc.fb_slots;
  hipLaunchKernelGGL(fb, dim3(fb_grid), dim3(PZ_RB), (size_t)pen, L.stream, L.logits, L.ld,
                     L.V, L.params, L.n_params, L.hist, L.H, L.hcap, L.u, L.ids, L.p_out, L.sc);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

int pz_launch_topp(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  if (n_rows <= 0) return 0;
  if (L.V > PZ_TOPP_MAX_V) return pz_launch_greedy_tempered(L, n_rows, d_rows);  // top_p.c:33-34
  const bool vec = (L.ld % 4 == 0) && (((uintptr_t)L.logits & 15) == 0);
  return vec ? launch_topp_t<true>(L, n_rows, d_rows) : launch_topp_t<false>(L, n_rows, d_rows);
}
