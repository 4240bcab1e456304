// pz_attn.hip -- the reference softmax over attention scores: many short
// rows, one per (sequence, head), each over its valid context.
//
// The call sites (src/transformer/attention.c:210, mla_attention.c:282,
// qwen35_attention.c:156, qwen3moe_attention.c:136) all run
// tn_softmax(att, valid_ctx) per head: softmax.c:4-23, i.e. the maximum by
// strict '>' from x[0], e = expf(x - max), a sequential fp32 sum in index
// order, x *= 1/sum.  Rows of up to 4096 scores take one wave each (four rows
// per 256-thread workgroup): the row sits in the wave's registers, 4
// consecutive scores per lane per 256-score segment, so the maximum, the
// exponentials, the exact sum and the write need no LDS beyond the exp
// table.  The sum is the exact sequential one (pz_exact.h): every segment
// through the integer state -- a segment with at most one binade exit and
// no tie before it in one step (pz_sp_fast) -- else, and for the first
// segment, by its 256 real fp32 adds in order (the DPP chain, pz_sp_chain).  Rows of more than
// ATTN_WAVE_SHORT scores (and up to ATTN_ROW_MAX) take one 1024-thread
// workgroup each instead (k_attn_row): its 16 waves estimate every 256-score
// segment's mass, predict the binade the running sum sits in at each
// segment, record the segments' integer increment sums there in LDS, and
// pre-evaluate the segments the records cannot serve while wave 0 walks the
// row (pz_split.h) -- the serial work left is one step per segment.  Longer
// rows use the one-workgroup-per-row softmax (pz_softmax.hip).
#include <hip/hip_runtime.h>

#include "../../include/pz_sampler.h"
#include "pz_device.h"
#include "pz_exact.h"
#include "pz_sampler_impl.h"
#include "pz_seq.h"
#include "pz_split.h"

namespace {

constexpr int ATTN_WAVES = 4;               // rows per workgroup
constexpr int ATTN_WAVE_MAX = 16 * 256;     // longest row of the wave kernel
#ifndef ATTN_WAVE_SHORT
#define ATTN_WAVE_SHORT 1024                // longer rows: one workgroup each
#endif

// One 256-term segment added to the running sum st (the whole wave, lane l
// holding terms 4l .. 4l+3): the one-step form when no tie or big term comes
// before the term that leaves the binade, else the sequential chain of real
// fp32 adds (always from a zero sum).  Out
// of line so the unrolled segment loop holds one copy.
__device__ __noinline__ PzAcc attn_seg_sum(PzAcc st, float a, float b, float c, float d) {
  const float v[4] = {a, b, c, d};
  if (st.n == 0u && st.g == 1u) {
    pz_sp_chain<PZ_STOP_NONE>(st, v, 0.0f);
  } else {
    uint32_t P[4], Q[4], fP, fQ;
    const uint32_t g0 = st.g;
    pz_sp_prefix4(v, g0, P, fP);
    pz_sp_prefix4(v, g0 + 1u, Q, fQ);
    if (!pz_sp_fast<PZ_STOP_NONE>(st, v, P, fP, Q, fQ, 0.0f)) pz_sp_chain<PZ_STOP_NONE>(st, v, 0.0f);
  }
  pz_sp_uni(st);
  return st;
}

// Row of NSEG segments (256 scores each, lane l: scores 256s + 4l .. +3).
template <int NSEG, bool VEC_IN, bool VEC_OUT>
__global__ __launch_bounds__(64 * ATTN_WAVES) void k_attn_wave(const float* in, long ld_in,
                                                              float* out, long ld_out,
                                                              int n_rows, int n,
                                                              const int32_t* lens) {
  __shared__ uint64_t etab[32];
  pz_etab_fill((pz_lds_u64*)etab);
  __syncthreads();
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * ATTN_WAVES + (threadIdx.x >> 6);
  if (row >= n_rows) return;  // whole waves
  int len = lens ? lens[row] : n;
  len = len < n ? len : n;
  if (len <= 0) return;  // softmax.c with size 0 writes nothing
  const float* x = in + (size_t)row * ld_in;
  float v[NSEG][4];
  bool nan_seen = false;
  float m = -__builtin_inff();
#pragma unroll
  for (int s = 0; s < NSEG; s++) {
    const int i0 = s * 256 + 4 * lane;
    if (VEC_IN && i0 + 3 < len) {
      const pz_f4 q = *reinterpret_cast<const pz_f4*>(x + i0);
      v[s][0] = q.x;
      v[s][1] = q.y;
      v[s][2] = q.z;
      v[s][3] = q.w;
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++) v[s][c] = i0 + c < len ? x[i0 + c] : -__builtin_inff();
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      nan_seen |= v[s][c] != v[s][c];
      m = fmaxf(m, v[s][c]);
    }
  }
  // softmax.c:6-9: a NaN anywhere makes the sum NaN (a NaN x[0] is the
  // maximum itself, a later one a NaN term), and so does an infinite
  // maximum (inf - inf, or -inf - -inf); every output is then NaN
  const bool any_nan = __ballot(nan_seen) != 0ull;
  const float M = pz_wave_max(m);
  float* o = out + (size_t)row * ld_out;
  if (any_nan || !(M > -__builtin_inff() && M < __builtin_inff())) {
    for (int i = lane; i < len; i += 64) o[i] = __builtin_nanf("");
    return;
  }
  // terms e = expf(x - M) (glibc's expf, bit for bit); 0 past the row
#pragma unroll
  for (int s = 0; s < NSEG; s++)
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int i = s * 256 + 4 * lane + c;
      v[s][c] = i < len ? pz_expf_tab(v[s][c] - M, et) : 0.0f;
    }
  // the sequential fp32 sum (softmax.c:12-16)
  PzAcc st;
  st.n = 0;
  st.g = 1;
  const int nseg = (len + 255) >> 8;
#pragma unroll
  for (int s = 0; s < NSEG; s++)
    if (s < nseg) st = attn_seg_sum(st, v[s][0], v[s][1], v[s][2], v[s][3]);
  const float inv = 1.0f / pz_acc_value(st);  // softmax.c:19
#pragma unroll
  for (int s = 0; s < NSEG; s++) {
    const int i0 = s * 256 + 4 * lane;
    if (VEC_OUT && i0 + 3 < len) {
      pz_f4 q;
      q.x = v[s][0] * inv;
      q.y = v[s][1] * inv;
      q.z = v[s][2] * inv;
      q.w = v[s][3] * inv;
      *reinterpret_cast<pz_f4*>(o + i0) = q;
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++)
        if (i0 + c < len) o[i0 + c] = v[s][c] * inv;
    }
  }
}

template <int NSEG>
int launch_wave(pz_sampler* s, const float* d_in, long ld_in, float* d_out, long ld_out,
                int n_rows, int n, const int32_t* d_len) {
  const bool vi = (ld_in % 4 == 0) && (((uintptr_t)d_in & 15) == 0);
  const bool vo = (ld_out % 4 == 0) && (((uintptr_t)d_out & 15) == 0);
  auto k = vi ? (vo ? k_attn_wave<NSEG, true, true> : k_attn_wave<NSEG, true, false>)
              : (vo ? k_attn_wave<NSEG, false, true> : k_attn_wave<NSEG, false, false>);
  const int blocks = (n_rows + ATTN_WAVES - 1) / ATTN_WAVES;
  hipLaunchKernelGGL(k, dim3(blocks), dim3(64 * ATTN_WAVES), 0, s->stream, d_in, ld_in, d_out,
                     ld_out, n_rows, n, d_len);
  PZ_HIP(s, hipGetLastError());
  return PZ_OK;
}


// ---- one workgroup per row ----------------------------------------------------
constexpr int AR_BLOCK = 1024;
constexpr int AR_WAVES = AR_BLOCK / 64;
constexpr int ATTN_ROW_MAX = 128 * 256;  // longest row of k_attn_row (128 segments)

// Row r's scores as the walk reads them: V = the row's valid length.
struct AttnRow {
  const float* x;
  int V;
  bool vec;
  __device__ __forceinline__ int load(int e0, float (&y)[4]) const {
    return vec ? pz_load4<true, false>(x, V, e0, y) : pz_load4<false, false>(x, V, e0, y);
  }
  __device__ __forceinline__ void apply(int, int, float (&)[4]) const {}
  __device__ __forceinline__ int get(int e0, float (&y)[4]) const { return load(e0, y); }
};

struct AttnShared {
  float est[128];
  float red[AR_WAVES];
  uint32_t bad[AR_WAVES];
  float carry;
  float sum;
  uint32_t s0;  // segment 0's sequential sum (bits), or 0xffffffff
};

// NSW: segments per wave (rows of up to 16 NSW segments); each wave holds
// its segments' scores (segments w, w + 16, ...) in registers through the
// records, and reads them once more for the probabilities.
template <int NSW, bool VEC_IN, bool VEC_OUT>
__global__ __launch_bounds__(AR_BLOCK) void k_attn_row(const float* in, long ld_in, float* out,
                                                      long ld_out, int n_rows, int n,
                                                      const int32_t* lens, int nc) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ AttnShared A;
  __shared__ uint64_t etab[32];
  pz_etab_fill((pz_lds_u64*)etab);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int row = blockIdx.x;
  int len = lens ? lens[row] : n;
  len = len < n ? len : n;
  if (len <= 0) return;  // softmax.c with size 0 writes nothing (every thread)
  const int nseg = (len + 255) >> 8;
  AttnRow R;
  R.x = in + (size_t)row * ld_in;
  R.V = len;
  R.vec = VEC_IN;
  float* o = out + (size_t)row * ld_out;
  // 1. the wave's segments into registers (every load in flight at once),
  // the maximum and the NaN check
  float y[NSW][4];
  int cnt[NSW];
#pragma unroll
  for (int j = 0; j < NSW; j++) {
    const int k = w + AR_WAVES * j;
    cnt[j] = k < nseg ? R.load(k * PZ_SP_SEG + 4 * lane, y[j]) : 0;
  }
  float m = -__builtin_inff();
  bool nan = false;
#pragma unroll
  for (int j = 0; j < NSW; j++)
#pragma unroll
    for (int c = 0; c < 4; c++) {
      if (c >= cnt[j]) continue;
      nan |= y[j][c] != y[j][c];
      m = fmaxf(m, y[j][c]);
    }
  m = pz_wave_max(m);
  const bool wnan = __ballot(nan) != 0ull;
  if (lane == 0) {
    A.red[w] = m;
    A.bad[w] = wnan ? 1u : 0u;
  }
  __syncthreads();
  float M = -__builtin_inff();
  bool bad = false;
#pragma unroll
  for (int i = 0; i < AR_WAVES; i++) {
    M = fmaxf(M, A.red[i]);
    bad |= A.bad[i] != 0u;
  }
  // softmax.c:6-9: a NaN anywhere, or an infinite maximum, makes every
  // output NaN (as k_attn_wave)
  if (bad || !(M > -__builtin_inff() && M < __builtin_inff())) {
    for (int i = tid; i < len; i += AR_BLOCK) o[i] = __builtin_nanf("");
    return;
  }
  // 2. each segment's estimated mass (hardware exp)
#pragma unroll
  for (int j = 0; j < NSW; j++) {
    const int k = w + AR_WAVES * j;
    if (k >= nseg) break;
    float t = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++)
      if (c < cnt[j]) t += pz_fast_exp(y[j][c] - M);
    t = pz_wave_sum(t);
    if (lane == 0) A.est[k] = t;
  }
  __syncthreads();
  // 3. the predicted grid of each segment: the binade of the estimated
  // running sum at its start (and whether the segment leaves it)
  PzWalk W = pz_sp_walk_layout(lds, nseg, nc);
  if (w == 0) {
    float carry = 0.0f;
    for (int c0 = 0; c0 < nseg; c0 += 64) {
      const int k = c0 + lane;
      const float e = k < nseg ? A.est[k] : 0.0f;
      const float incl = pz_wave_scan_f32(e);
      const float start = carry + (incl - e), end = carry + incl;
      if (k < nseg)
        W.gf[k] = pz_predict_gf(start) | (pz_grid_of(end) != pz_grid_of(start) ? PZ_GF_XING : 0u);
      carry += pz_readlane_f32(incl, 63);
    }
  }
  __syncthreads();
  // 4. records at the predicted grids, in LDS (segments predicted to cross
  // a binade are specials: no record)
  PzExpTerms<AttnRow> X;
  X.R = R;
  X.M = M;
  X.thr = -__builtin_inff();
  X.inv = 1.0f;
  X.as_p = false;
  X.et = (const pz_lds_u64*)etab;
#pragma unroll
  for (int j = 0; j < NSW; j++) {
    const int k = w + AR_WAVES * j;
    if (k >= nseg) break;
    const uint32_t gf = W.gf[k];
    if (gf & PZ_GF_XING) {
      if (lane == 0) {
        W.d[k] = 0u;
        W.d2[k] = 0u;
      }
      continue;
    }
    float raw[4] = {y[j][0], y[j][1], y[j][2], y[j][3]};
    float a[4];
    X.prep(k * PZ_SP_SEG + 4 * lane, cnt[j], raw, a);
    const uint32_t g = gf & 0xffu;
    const bool has2 = (gf & PZ_GF_HAS2) != 0;
    uint32_t s1 = 0, s2 = 0;
    bool d1 = false, d2 = false;
    X.inc4(raw, a, g, s1, d1);
    if (has2) {
      X.inc4(raw, a, g - 1u, s2, d2);
      s2 = pz_wave_sum_u32(s2);
    }
    s1 = pz_wave_sum_u32(s1);
    const bool D1 = __ballot(d1) != 0;
    const bool D2 = has2 && __ballot(d2) != 0;
    if (lane == 0) {
      W.d[k] = s1;
      W.d2[k] = s2;
      W.gf[k] = (gf & (0xffu | PZ_GF_HAS2 | PZ_GF_XING)) | (D1 ? PZ_GF_DIRTY : 0u) |
                (D2 ? PZ_GF_DIRTY2 : 0u);
    }
  }
  // wave 0 has no record to make for segment 0 when it is predicted to
  // cross binades (from a zero sum it nearly always is): it adds up that
  // segment's exact terms in id order meanwhile, so the walk starts from
  // that sum without waiting for a producer to load and add the segment
  if (w == 0) {
    uint32_t s0 = 0xffffffffu;
    if (W.gf[0] & PZ_GF_XING) {
      float t[4];
#pragma unroll
      for (int c = 0; c < 4; c++) t[c] = c < cnt[0] ? X.exact_term(y[0][c]) : 0.0f;
      s0 = __float_as_uint(pz_seq_sum_seg4(t));
    }
    if (lane == 0) A.s0 = s0;
  }
  __syncthreads();
  // 5. the walk: wave 0, waves 1..15 pre-evaluating its specials
  W = pz_sp_walk_start(X, W, SS, -1, A.s0);
  if (w == 0) {
    PzAcc st;
    pz_sp_walk<PZ_STOP_NONE>(st, W, 0.0f, X);
    if (lane == 0) A.sum = pz_acc_value(st);
  }
  __syncthreads();
  // 6. p = e * (1 / sum) (softmax.c:19-22), every exact term again: the
  // scores reloaded (all loads in flight at once; holding them across the
  // walk would spill)
  const float inv = 1.0f / A.sum;
#pragma unroll
  for (int j = 0; j < NSW; j++) {
    const int k = w + AR_WAVES * j;
    cnt[j] = k < nseg ? R.load(k * PZ_SP_SEG + 4 * lane, y[j]) : 0;
  }
#pragma unroll
  for (int j = 0; j < NSW; j++) {
    const int k = w + AR_WAVES * j;
    if (k >= nseg) break;
    float v[4];
#pragma unroll
    for (int c = 0; c < 4; c++) v[c] = c < cnt[j] ? X.exact_term(y[j][c]) * inv : 0.0f;
    const int i0 = k * PZ_SP_SEG + 4 * lane;
    if (VEC_OUT && i0 + 3 < len) {
      pz_f4 q;
      q.x = v[0];
      q.y = v[1];
      q.z = v[2];
      q.w = v[3];
      *reinterpret_cast<pz_f4*>(o + i0) = q;
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++)
        if (i0 + c < len) o[i0 + c] = v[c];
    }
  }
}

template <int NSW>
int launch_row_t(pz_sampler* s, const float* d_in, long ld_in, float* d_out, long ld_out,
                 int n_rows, int n, const int32_t* d_len, int nc, size_t lds) {
  const bool vi = (ld_in % 4 == 0) && (((uintptr_t)d_in & 15) == 0);
  const bool vo = (ld_out % 4 == 0) && (((uintptr_t)d_out & 15) == 0);
  auto k = vi ? (vo ? k_attn_row<NSW, true, true> : k_attn_row<NSW, true, false>)
              : (vo ? k_attn_row<NSW, false, true> : k_attn_row<NSW, false, false>);
  if (lds > 65536 && hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)lds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(k, dim3(n_rows), dim3(AR_BLOCK), lds, s->stream, d_in, ld_in, d_out, ld_out,
                     n_rows, n, d_len, nc);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_row(pz_sampler* s, const float* d_in, long ld_in, float* d_out, long ld_out,
               int n_rows, int n, const int32_t* d_len) {
  const int nseg = (n + 255) / 256;
  const size_t fixed = sizeof(PzSpShared) + sizeof(AttnShared) + 512;
  const int nc = pz_sp_walk_nc(nseg, (size_t)s->max_lds - fixed);
  if (nc < 2) return -2;
  const size_t lds = pz_sp_walk_lds(nseg, nc);
  const int nsw = (nseg + AR_WAVES - 1) / AR_WAVES;
  if (nsw <= 1) return launch_row_t<1>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len, nc, lds);
  if (nsw <= 2) return launch_row_t<2>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len, nc, lds);
  if (nsw <= 4) return launch_row_t<4>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len, nc, lds);
  return launch_row_t<8>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len, nc, lds);
}

// ---- long rows split over workgroups -----------------------------------------
// Rows of more than ATTN_SPLIT_MIN scores: the row-split passes of
// pz_split.h over the rows' own lengths -- slice maxima and segment
// estimates (k_attn_stat), the integer increment records at the predicted
// grids (k_attn_rec), one workgroup per row for the exact sum (k_attn_walk),
// then every probability (k_attn_write) -- so the per-element work runs on
// every CU rather than one per row.  Each pass reads the row again (L2 /
// Infinity Cache: a few MB).
#ifndef ATTN_SPLIT_MIN
#define ATTN_SPLIT_MIN 8192
#endif

struct AttnSplit {
  const float* in;
  long ld_in;
  float* out;
  long ld_out;
  int n;
  const int32_t* lens;
  PzSplitWs ws;
  int nseg, spw, S, nc;
};

__device__ __forceinline__ int attn_len(const AttnSplit& A, int row) {
  const int len = A.lens ? A.lens[row] : A.n;
  return len < A.n ? len : A.n;  // (<= 0: the row is left alone)
}

template <bool VI>
__device__ __forceinline__ AttnRow attn_row(const AttnSplit& A, int row, int len) {
  AttnRow R;
  R.x = A.in + (size_t)row * A.ld_in;
  R.V = len;
  R.vec = VI;
  return R;
}

__device__ __forceinline__ bool attn_bad(uint32_t flags) {
  return (flags & (PZ_RS_NAN | PZ_RS_NONFIN)) != 0;  // softmax.c:6-9: NaN everywhere
}

template <bool VI>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_attn_stat(AttnSplit A) {
  __shared__ PzSpShared SS;
  const int row = blockIdx.y, len = attn_len(A, row);
  if (len <= 0) return;
  if (threadIdx.x == 0) SS.any = 0u;
  __syncthreads();
  pz_sp_stat_slice(attn_row<VI>(A, row, len), row, pz_sp_slice(A.nseg, A.spw), A.ws, SS, true);
}

template <bool VI>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_attn_rec(AttnSplit A) {
  __shared__ PzSpShared SS;
  __shared__ uint64_t etab[32];
  pz_etab_fill((pz_lds_u64*)etab);
  const int row = blockIdx.y, len = attn_len(A, row);
  if (len <= 0) return;
  pz_sp_row_stat(row, A.S, A.ws, SS);
  if (attn_bad(SS.any)) return;
  const PzSlice sl = pz_sp_slice(A.nseg, A.spw);
  const PzEstRel est{A.ws.seg_m + (size_t)row * A.ws.nsc, A.ws.seg_s + (size_t)row * A.ws.nsc,
                     SS.M};
  const float carry = pz_sp_prefix(est, sl.k0, SS);
  pz_sp_predict(est, carry, row, sl, A.ws, SS);
  PzExpTerms<AttnRow> X;
  X.R = attn_row<VI>(A, row, len);
  X.M = SS.M;
  X.thr = -__builtin_inff();
  X.inv = 1.0f;
  X.as_p = false;
  X.et = (const pz_lds_u64*)etab;
  pz_sp_records(X, row, sl, A.ws, nullptr, true);
  if (sl.k0 == 0 && threadIdx.x < 64) {
    // the row's first segment summed from zero (the DPP chain of real adds),
    // for the walk to start from instead of waiting for a producer
    float v[4];
    X.seg(0, v);
    PzAcc z;
    z.n = 0u;
    z.g = 1u;
    pz_sp_chain<PZ_STOP_NONE>(z, v, 0.0f);
    if (threadIdx.x == 0) A.ws.rs[row].s0 = __float_as_uint(pz_acc_value(z));
  }
}

// One workgroup per row: wave 0 walks, waves 1..15 pre-evaluate its specials.
template <bool VI>
__global__ __launch_bounds__(PZ_SP_BLOCK) void k_attn_walk(AttnSplit A) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ uint64_t etab[32];
  __shared__ float sum_sh;
  pz_etab_fill((pz_lds_u64*)etab);
  const int row = blockIdx.x, len = attn_len(A, row);
  if (len <= 0) return;
  const PzRecAhead ra = pz_sp_rec_ahead(A.ws, row, A.nseg);  // in flight beside the maxima
  const uint32_t s0 = A.ws.rs[row].s0;  // segment 0's sum (k_attn_rec)
  pz_sp_row_stat(row, A.S, A.ws, SS);
  PzRowState& rs = A.ws.rs[row];
  if (attn_bad(SS.any)) {
    if (threadIdx.x == 0) {
      rs.M = SS.M;
      rs.flags = SS.any;
    }
    return;
  }
  PzExpTerms<AttnRow> X;
  X.R = attn_row<VI>(A, row, len);
  X.M = SS.M;
  X.thr = -__builtin_inff();
  X.inv = 1.0f;
  X.as_p = false;
  X.et = (const pz_lds_u64*)etab;
  const PzWalk W = pz_sp_walk_setup(X, row, A.nseg, A.nc, A.ws, lds, SS, -1, s0, &ra);
  if (threadIdx.x < 64) {
    PzAcc st;
    pz_sp_walk<PZ_STOP_NONE>(st, W, 0.0f, X);
    if (threadIdx.x == 0) sum_sh = pz_acc_value(st);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    rs.M = SS.M;
    rs.flags = SS.any;
    rs.sum = sum_sh;
    rs.inv = 1.0f / sum_sh;  // softmax.c:19-22
  }
}

// p = e * (1 / sum) for every score of the slice (NaN on degenerate rows).
template <bool VI, bool VO>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_attn_write(AttnSplit A) {
  __shared__ uint64_t etab[32];
  pz_etab_fill((pz_lds_u64*)etab);
  const int row = blockIdx.y, len = attn_len(A, row);
  if (len <= 0) return;
  const PzRowState rs = A.ws.rs[row];
  const bool bad = attn_bad(rs.flags);
  PzExpTerms<AttnRow> X;
  X.R = attn_row<VI>(A, row, len);
  X.M = rs.M;
  X.thr = -__builtin_inff();
  X.inv = 1.0f;
  X.as_p = false;
  X.et = (const pz_lds_u64*)etab;
  __syncthreads();  // the expf table
  float* o = A.out + (size_t)row * A.ld_out;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const PzSlice sl = pz_sp_slice(A.nseg, A.spw);
  for (int k = sl.k0 + w; k < sl.k1; k += PZ_SP_WAVES) {
    const int i0 = k * PZ_SP_SEG + 4 * lane;
    if (i0 >= len) continue;
    float y[4];
    X.R.load(i0, y);
    float v[4];
#pragma unroll
    for (int c = 0; c < 4; c++) v[c] = bad ? __builtin_nanf("") : X.exact_term(y[c]) * rs.inv;
    if (VO && i0 + 3 < len) {
      pz_f4 q;
      q.x = v[0];
      q.y = v[1];
      q.z = v[2];
      q.w = v[3];
      *reinterpret_cast<pz_f4*>(o + i0) = q;
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++)
        if (i0 + c < len) o[i0 + c] = v[c];
    }
  }
}

template <bool VI, bool VO>
int launch_split_t(pz_sampler* s, const AttnSplit& A, int n_rows, size_t walk_lds) {
  auto kw = k_attn_walk<VI>;
  if (walk_lds > 65536 && hipFuncSetAttribute((const void*)kw,
                                              hipFuncAttributeMaxDynamicSharedMemorySize,
                                              (int)walk_lds) != hipSuccess)
    return -1;
  const dim3 grid(A.S, n_rows), block(PZ_SP_BLOCK);
  hipLaunchKernelGGL(k_attn_stat<VI>, grid, block, 0, s->stream, A);
  hipLaunchKernelGGL(k_attn_rec<VI>, grid, block, 0, s->stream, A);
  hipLaunchKernelGGL(kw, dim3(n_rows), block, walk_lds, s->stream, A);
  hipLaunchKernelGGL((k_attn_write<VI, VO>), grid, block, 0, s->stream, A);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_split(pz_sampler* s, const float* d_in, long ld_in, float* d_out, long ld_out,
                 int n_rows, int n, const int32_t* d_len) {
  const size_t bytes = pz_split_ws_layout(n_rows, n, 0, nullptr, nullptr);
  if (s->attn_dev_bytes < bytes) {
    // (earlier launches on the stream may still use the old workspace)
    if (hipStreamSynchronize(s->stream) != hipSuccess) return -1;
    (void)hipFree(s->attn_dev);
    s->attn_dev = nullptr;
    s->attn_dev_bytes = 0;
    if (hipMalloc(&s->attn_dev, bytes) != hipSuccess) return -3;
    s->attn_dev_bytes = bytes;
  }
  AttnSplit A;
  A.in = d_in;
  A.ld_in = ld_in;
  A.out = d_out;
  A.ld_out = ld_out;
  A.n = n;
  A.lens = d_len;
  pz_split_ws_layout(n_rows, n, 0, s->attn_dev, &A.ws);
  const PzSplitPlan pl = pz_split_plan(n, n_rows, A.ws.smax);
  A.nseg = pl.nseg;
  A.spw = pl.spw;
  A.S = pl.S;
  const size_t fixed = 4096;
  int nc = pz_sp_walk_nc(pl.nseg, (size_t)s->max_lds / 2 - fixed);
  if (nc < 12) nc = pz_sp_walk_nc(pl.nseg, (size_t)s->max_lds - fixed);
  if (nc < 2) return -2;
  A.nc = nc;
  const size_t walk_lds = pz_sp_walk_lds(pl.nseg, nc);
  const bool vi = (ld_in % 4 == 0) && (((uintptr_t)d_in & 15) == 0);
  const bool vo = (ld_out % 4 == 0) && (((uintptr_t)d_out & 15) == 0);
  if (vi) return vo ? launch_split_t<true, true>(s, A, n_rows, walk_lds)
                    : launch_split_t<true, false>(s, A, n_rows, walk_lds);
  return vo ? launch_split_t<false, true>(s, A, n_rows, walk_lds)
            : launch_split_t<false, false>(s, A, n_rows, walk_lds);
}

}  // namespace

extern "C" int pz_attn_softmax(pz_sampler* s, const float* d_in, long ld_in, float* d_out,
                               long ld_out, int n_rows, int n, const int32_t* d_len) {
  if (!s) return PZ_EINVAL;
  if (!d_in || !d_out || n_rows < 0 || n < 0 || ld_in < n || ld_out < n)
    return fail(s, PZ_EINVAL, "bad attention softmax shape");
  if (n_rows == 0 || n == 0) return PZ_OK;
  PZ_HIP(s, hipSetDevice(s->device));
  if (n > ATTN_SPLIT_MIN) {
    const int rc = launch_split(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len);
    if (rc == 0) return PZ_OK;
    if (rc == -3) return fail(s, PZ_ENOMEM, "attention softmax workspace");
    if (rc != -2) return fail(s, PZ_EDEVICE, "attention softmax launch failed");
  }
  if (n > ATTN_WAVE_SHORT && n <= ATTN_ROW_MAX) {
    const int rc = launch_row(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len);
    if (rc == 0) return PZ_OK;
    if (rc != -2) return fail(s, PZ_EDEVICE, "attention softmax launch failed");
  }
  if (n > ATTN_WAVE_MAX) {
    PzTemp one;  // scores are softmaxed as they are: x * 1.0f == x
    one.t = 1.0f;
    one.inv = 1.0f;
    one.div = 0;
    return pz_launch_softmax_rows(s, d_in, ld_in, d_out, ld_out, n_rows, n, one, d_len);
  }
  const int nseg = (n + 255) / 256;
  if (nseg <= 1) return launch_wave<1>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len);
  if (nseg <= 2) return launch_wave<2>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len);
  if (nseg <= 4) return launch_wave<4>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len);
  if (nseg <= 8) return launch_wave<8>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len);
  return launch_wave<16>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len);
}
