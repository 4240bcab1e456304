// pz_spec.hip -- speculative-draft verification on the GPU (accept/reject and
// residual resampling), with the reference's fp32 softmax arithmetic.
//
// The reference has no speculative decoding (docs/architecture/
// IMPLEMENTATION_PLAN.md:1664-1693 is a plan only); the rule follows
// Leviathan et al. 2023, Alg. 1, built from the reference's own pieces:
//   p = softmax(target_j / T), q = softmax(draft_j / T) with
//   apply_temperature (temperature.c:8-25) and softmax.c:4-23;
//   draft d_j is accepted iff u_acc < p(d_j) / q(d_j) (q(d_j) == 0 rejects);
//   with greedy drafting (IMPLEMENTATION_PLAN.md:1680) q is one-hot at the
//   draft instead (no draft rows: accept iff u_acc < p(d_j));
//   at the first rejection r(x) = max(0, p(x) - q(x)) (fp32 difference),
//   Z = sequential fp32 sum of r in ascending id, and the token is the first
//   x with u_res * Z < cdf_r(x) (the last x with r(x) > 0 if none); when
//   Z == 0 it is drawn from p with generate.c:157-169.  With every draft
//   accepted and a bonus target row, the bonus token is drawn from p_K with
//   u_res the same way.
//
// Launches (rows split over several workgroups, pz_split.h):
//   k_spec_stat   every target and draft row: maximum, segment estimates;
//   k_spec_rec    their exact-term records;
//   k_spec_walk   one workgroup per row: the exact softmax normaliser;
//   k_spec_vest   per sequence: the acceptance tests (one draft per lane of
//                 wave 0 in each workgroup; the first posts the outcome and
//                 the row the token is drawn from), then the estimated
//                 residual (or p) mass per segment;
//   k_spec_vrec   its exact-term records;
//   k_spec_vwalk  one workgroup per sequence: Z and the residual draw (or the
//                 categorical draw from p), the output row.
#include <limits.h>
#include <string.h>

#include <chrono>

#include "pz_device.h"
#include "pz_exact.h"
#include "pz_launch.h"
#include "pz_rowpass.h"
#include "pz_sampler_impl.h"
#include "pz_split.h"

namespace {

// Sequence outcomes after the acceptance tests.
enum { SQ_DONE = 0, SQ_RES = 1, SQ_CAT = 2 };

struct SpecSeq {
  int mode;   // SQ_*
  int js;     // accepted drafts
  int qt, qd; // target / draft row of the draw (logits row indices; qd < 0: one-hot q)
  int last;   // residual: the last x with r(x) > 0
  int dr;     // the rejected draft (one-hot q)
  int pad[2];
};

struct SpecArgs {
  const float* target;  // [B, KT, ld]
  const float* draft;   // [B, K, ld]
  long ld;
  int V, B, K, KT, NT, NR, has_bonus;
  int onehot;  // greedy drafts: q one-hot at the draft, no draft rows (NR == NT)
  PzTemp T;
  const int32_t* draft_ids;  // [B, K]
  const float* u_acc;        // [B, K]
  const float* u_res;        // [B]
  int32_t* acc_len;          // [B]
  int32_t* ids_out;          // [B, K+1]
  SpecSeq* seq;              // [B]
  PzSplitWs ws;              // rows [0, NR): logits rows; [NR, NR + B): sequences
  int nseg, spw, S, nc;
  __device__ __forceinline__ const float* row(int q) const {
    return q < NT ? target + (long)q * ld : draft + (long)(q - NT) * ld;
  }
};

// p(x) of one element of a row whose softmax statistics are (M, inv).
template <bool VEC>
__device__ __forceinline__ float prob_at(const PzTempRow<VEC>& R, int x, float M, float inv) {
  return pz_expf(R.T.apply(R.x[x]) - M) * inv;
}

// Residual terms r(x) = max(0, p(x) - q(x)) of a target/draft row pair (or,
// with oh, of the target row and q one-hot at the draft ohd), evaluated
// exactly in prep; the observer tracks the last x with r(x) > 0.
template <bool VEC>
struct ResidualTerms {
  struct Raw {
    float t[4];
    float d[4];
  };
  PzTempRow<VEC> T, D;
  float MT, invT, MD, invD;
  bool oh;     // q one-hot at ohd (greedy drafts) rather than the draft row's softmax
  int ohd;     // (an id outside [0, V): q == 0 everywhere)
  int lastpos;
  const pz_lds_u64* et;  // the workgroup's LDS copy of the expf table
  __device__ __forceinline__ int load(int e0, Raw& r) const {
    const int n = T.load(e0, r.t);
    if (!oh) D.load(e0, r.d);
    return n;
  }
  __device__ __forceinline__ void residual(int e0, int n, Raw& r, float (&v)[4]) const {
    T.apply(e0, n, r.t);
    if (!oh) D.apply(e0, n, r.d);
#pragma unroll
    for (int c = 0; c < 4; c++) {
      float res = 0.0f;
      if (c < n) {
        const float p = pz_expf_tab(r.t[c] - MT, et) * invT;
        const float qq = !oh ? pz_expf_tab(r.d[c] - MD, et) * invD
                             : (e0 + c == ohd ? 1.0f : 0.0f);
        const float t = p - qq;
        res = t > 0.0f ? t : 0.0f;
      }
      v[c] = res;
    }
  }
  __device__ __forceinline__ void prep(int e0, int n, Raw& r, float (&a)[4]) const {
    residual(e0, n, r, a);
  }
  __device__ __forceinline__ void observe(int e0, const Raw&, const float (&a)[4]) {
#pragma unroll
    for (int c = 0; c < 4; c++)
      if (a[c] > 0.0f) lastpos = e0 + c;
  }
  __device__ __forceinline__ void inc4(const Raw&, const float (&a)[4], uint32_t g, uint32_t& s,
                                       bool& dirty) const {
#pragma unroll
    for (int c = 0; c < 4; c++) {
      uint32_t cls;
      s += pz_inc(a[c], g, &cls);
      dirty |= cls != PZ_INC_PLAIN;
    }
  }
  __device__ __forceinline__ void seg(int k, float (&v)[4]) const {
    Raw r;
    const int e0 = pz_seg_e0(k);
    const int n = load(e0, r);
    residual(e0, n, r, v);
  }
};

template <bool VEC>
__device__ __forceinline__ PzTempRow<VEC> temp_row(const SpecArgs& A, int q) {
  PzTempRow<VEC> R;
  R.x = A.row(q);
  R.V = A.V;
  R.T = A.T;
  return R;
}

// Softmax of a row is degenerate (every p NaN) when any y is NaN or the
// maximum is not finite (softmax.c:4-23 then sums a NaN).
__device__ __forceinline__ bool spec_bad(uint32_t flags) {
  return (flags & (PZ_RS_NAN | PZ_RS_NONFIN)) != 0;
}

// ---- every logits row: maximum and segment estimates (HBM) ----------------
template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_spec_stat(SpecArgs A) {
  __shared__ PzSpShared SS;
  const int q = blockIdx.y;
  if (threadIdx.x == 0) SS.any = 0u;
  __syncthreads();
  const PzSlice sl = pz_sp_slice(A.nseg, A.spw);
  pz_sp_stat_slice(temp_row<VEC>(A, q), q, sl, A.ws, SS, true);
}

// ---- their records ---------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_spec_rec(SpecArgs A) {
  __shared__ PzSpShared SS;
  __shared__ uint64_t etab[32];
  pz_etab_fill((pz_lds_u64*)etab);
  const int q = blockIdx.y;
  pz_sp_row_stat(q, A.S, A.ws, SS);
  if (spec_bad(SS.any)) return;
  const PzSlice sl = pz_sp_slice(A.nseg, A.spw);
  const PzEstRel est{A.ws.seg_m + (size_t)q * A.ws.nsc, A.ws.seg_s + (size_t)q * A.ws.nsc, SS.M};
  const float carry = pz_sp_prefix(est, sl.k0, SS);
  pz_sp_predict(est, carry, q, sl, A.ws, SS);
  PzExpTerms<PzTempRow<VEC>> X;
  X.R = temp_row<VEC>(A, q);
  X.M = SS.M;
  X.thr = -__builtin_inff();
  X.inv = 1.0f;
  X.as_p = false;
  X.et = (const pz_lds_u64*)etab;
  pz_sp_records(X, q, sl, A.ws, nullptr, true);
}

// ---- one workgroup per row: the exact normaliser -----------------------------
// 512 threads: one wave walks, the others stage and pre-evaluate, and two
// workgroups share a CU with room for the walk's registers.
constexpr int SPEC_WALK_BLOCK = 512;
template <bool VEC>
__global__ __launch_bounds__(SPEC_WALK_BLOCK) void k_spec_walk(SpecArgs A) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ uint64_t etab[32];
  __shared__ float sum_sh;
  pz_etab_fill((pz_lds_u64*)etab);
  const int q = blockIdx.x;
  const PzRecAhead ra = pz_sp_rec_ahead(A.ws, q, A.nseg);  // in flight beside the maxima
  pz_sp_row_stat(q, A.S, A.ws, SS);
  PzRowState& rs = A.ws.rs[q];
  if (spec_bad(SS.any)) {
    if (threadIdx.x == 0) {
      rs.M = SS.M;
      rs.flags = SS.any;
      rs.inv = __builtin_nanf("");
    }
    return;
  }
  PzExpTerms<PzTempRow<VEC>> X;
  X.R = temp_row<VEC>(A, q);
  X.M = SS.M;
  X.thr = -__builtin_inff();
  X.inv = 1.0f;
  X.as_p = false;
  X.et = (const pz_lds_u64*)etab;
  const PzWalk W = pz_sp_walk_setup(X, q, A.nseg, A.nc, A.ws, lds, SS, -1, 0xffffffffu, &ra);
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

// ---- acceptance tests of a sequence (one wave) ----------------------------
template <bool VEC>
__device__ __forceinline__ SpecSeq spec_accept(const SpecArgs& A, int b, bool post) {
  const int lane = threadIdx.x & 63;
  const PzRowState* rs = A.ws.rs;
  bool accept = false;
  if (lane < A.K) {
    const int qt = b * A.KT + lane, qd = A.NT + b * A.K + lane;
    const int d = A.draft_ids[b * A.K + lane];
    if (d >= 0 && d < A.V) {
      const float pd = prob_at(temp_row<VEC>(A, qt), d, rs[qt].M, rs[qt].inv);
      const float qv = A.onehot ? 1.0f : prob_at(temp_row<VEC>(A, qd), d, rs[qd].M, rs[qd].inv);
      accept = qv > 0.0f && A.u_acc[b * A.K + lane] < pd / qv;
    }
  }
  SpecSeq s;
  memset(&s, 0, sizeof(s));
  // a row whose front wait gave up fails the whole sequence
  bool failed = false;
  for (int j = lane; j < A.KT; j += 64) failed |= (rs[b * A.KT + j].flags & PZ_RS_FAILED) != 0;
  if (!A.onehot)
    for (int j = lane; j < A.K; j += 64)
      failed |= (rs[A.NT + b * A.K + j].flags & PZ_RS_FAILED) != 0;
  if (__ballot(failed)) {
    s.mode = SQ_DONE;
    if (post && lane == 0) {
      A.seq[b] = s;
      A.acc_len[b] = PZ_ID_FAILED;
      for (int j = 0; j <= A.K; j++) A.ids_out[(long)b * (A.K + 1) + j] = PZ_ID_FAILED;
    }
    return s;
  }
  const uint64_t rej = __ballot(lane < A.K && !accept);
  const int js = rej ? (int)__builtin_ctzll(rej) : A.K;
  s.js = js;
  s.last = -1;
  s.qt = s.qd = -1;
  s.dr = -1;
  int tok = -1;
  s.mode = SQ_DONE;
  if (js < A.K) {
    const int qt = b * A.KT + js, qd = A.NT + b * A.K + js;
    if (spec_bad(rs[qt].flags)) {
      tok = A.V - 1;  // p is NaN everywhere: r == 0, and the p-draw falls back
    } else if (!A.onehot && spec_bad(rs[qd].flags)) {
      s.mode = SQ_CAT;  // q is NaN: every p - q fails t > 0, Z == 0
      s.qt = qt;
    } else {
      s.mode = SQ_RES;
      s.qt = qt;
      s.qd = A.onehot ? -1 : qd;
      s.dr = A.draft_ids[b * A.K + js];
    }
  } else if (A.has_bonus) {
    const int qt = b * A.KT + A.K;
    if (spec_bad(rs[qt].flags)) tok = A.V - 1;
    else {
      s.mode = SQ_CAT;
      s.qt = qt;
    }
  }
  if (post && lane == 0) {
    A.seq[b] = s;
    if (s.mode == SQ_DONE) {
      A.acc_len[b] = js;
      for (int j = 0; j <= A.K; j++)
        A.ids_out[(long)b * (A.K + 1) + j] =
            j < js ? A.draft_ids[b * A.K + j] : (j == js ? tok : -1);
    }
  }
  return s;
}

template <bool VEC>
__device__ __forceinline__ ResidualTerms<VEC> residual_terms(const SpecArgs& A, const SpecSeq& s,
                                                             const pz_lds_u64* et) {
  ResidualTerms<VEC> X;
  X.T = temp_row<VEC>(A, s.qt);
  X.oh = s.qd < 0;
  X.ohd = s.dr;
  X.D = s.qd < 0 ? X.T : temp_row<VEC>(A, s.qd);
  X.MT = A.ws.rs[s.qt].M;
  X.invT = A.ws.rs[s.qt].inv;
  X.MD = s.qd < 0 ? 0.0f : A.ws.rs[s.qd].M;
  X.invD = s.qd < 0 ? 0.0f : A.ws.rs[s.qd].inv;
  X.lastpos = -1;
  X.et = et;
  return X;
}

template <bool VEC>
__device__ __forceinline__ PzExpTerms<PzTempRow<VEC>> p_terms(const SpecArgs& A, int qt,
                                                              const pz_lds_u64* et) {
  PzExpTerms<PzTempRow<VEC>> X;
  X.R = temp_row<VEC>(A, qt);
  X.M = A.ws.rs[qt].M;
  X.thr = -__builtin_inff();
  X.inv = A.ws.rs[qt].inv;
  X.as_p = true;
  X.et = et;
  return X;
}

// ---- per sequence: estimated mass of the draw's terms per segment ----------
template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_spec_vest(SpecArgs A) {
  __shared__ SpecSeq s_sh;
  const int b = blockIdx.y, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // the sequence's acceptance tests, by wave 0 of each of its workgroups
  // (the same reads and ballots in each); the first posts the outcome for
  // the launches after it, and the output row when the sequence is done
  if (w == 0) {
    const SpecSeq sq = spec_accept<VEC>(A, b, blockIdx.x == 0);
    if (lane == 0) s_sh = sq;
  }
  __syncthreads();
  const SpecSeq s = s_sh;
  if (s.mode == SQ_DONE) return;
  const PzSlice sl = pz_sp_slice(A.nseg, A.spw);
  const PzTempRow<VEC> T = temp_row<VEC>(A, s.qt);
  const float MT = A.ws.rs[s.qt].M, invT = A.ws.rs[s.qt].inv;
  float MD = 0.0f, invD = 0.0f;
  PzTempRow<VEC> D = T;
  const bool two = s.mode == SQ_RES && s.qd >= 0;  // q from a draft row (else one-hot)
  if (two) {
    D = temp_row<VEC>(A, s.qd);
    MD = A.ws.rs[s.qd].M;
    invD = A.ws.rs[s.qd].inv;
  }
  float* est = A.ws.seg_s + (size_t)(A.NR + b) * A.ws.nsc;
  for (int kb = sl.k0 + w; kb < sl.k1; kb += PZ_SP_U * PZ_SP_WAVES) {
    float yts[PZ_SP_U][4], yds[PZ_SP_U][4];
    int ns[PZ_SP_U];
#pragma unroll
    for (int u = 0; u < PZ_SP_U; u++) {
      const int e0 = (kb + u * PZ_SP_WAVES) * PZ_SP_SEG + 4 * lane;
      ns[u] = T.load(e0, yts[u]);
      if (two) D.load(e0, yds[u]);
    }
#pragma unroll
    for (int u = 0; u < PZ_SP_U; u++) {
      const int k = kb + u * PZ_SP_WAVES;
      if (k >= sl.k1) break;
      const int e0 = k * PZ_SP_SEG + 4 * lane;
      const int n = ns[u];
      float (&yt)[4] = yts[u];
      float (&yd)[4] = yds[u];
      T.apply(e0, n, yt);
      float t = 0.0f;
      if (two) {
        D.apply(e0, n, yd);
#pragma unroll
        for (int c = 0; c < 4; c++) {
          if (c >= n) continue;
          const float r = pz_fast_exp(yt[c] - MT) * invT - pz_fast_exp(yd[c] - MD) * invD;
          t += r > 0.0f ? r : 0.0f;
        }
      } else if (s.mode == SQ_RES) {  // one-hot q: p, less 1 at the draft
#pragma unroll
        for (int c = 0; c < 4; c++) {
          if (c >= n) continue;
          const float r = pz_fast_exp(yt[c] - MT) * invT - (e0 + c == s.dr ? 1.0f : 0.0f);
          t += r > 0.0f ? r : 0.0f;
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; c++)
          if (c < n) t += pz_fast_exp(yt[c] - MT) * invT;
      }
      t = pz_wave_sum(t);
      if (lane == 0) est[k] = t;
    }
  }
}

// ---- per sequence: records of the draw's terms ----------------------------
template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) void k_spec_vrec(SpecArgs A) {
  __shared__ PzSpShared SS;
  __shared__ uint64_t etab[32];
  __shared__ int last_sh;
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  pz_etab_fill((pz_lds_u64*)etab);
  const int b = blockIdx.y;
  const SpecSeq s = A.seq[b];
  if (s.mode == SQ_DONE) return;
  if (threadIdx.x == 0) last_sh = -1;
  const int r = A.NR + b;
  const PzSlice sl = pz_sp_slice(A.nseg, A.spw);
  const PzEstAbs est{A.ws.seg_s + (size_t)r * A.ws.nsc};
  const float carry = pz_sp_prefix(est, sl.k0, SS);
  pz_sp_predict(est, carry, r, sl, A.ws, SS);
  if (s.mode == SQ_RES) {
    ResidualTerms<VEC> X = residual_terms<VEC>(A, s, et);
    pz_sp_records(X, r, sl, A.ws);
    if (X.lastpos >= 0) atomicMax(&last_sh, X.lastpos);
    __syncthreads();
    if (threadIdx.x == 0 && last_sh >= 0) atomicMax(&A.seq[b].last, last_sh);
  } else {
    PzExpTerms<PzTempRow<VEC>> X = p_terms<VEC>(A, s.qt, et);
    pz_sp_records(X, r, sl, A.ws, nullptr, true);
  }
}

// ---- one workgroup per sequence: Z and the draw -------------------------------
struct VwalkShared {
  float Z;
  int hit;
};

template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) void k_spec_vwalk(SpecArgs A) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ PzRecShared RS;
  __shared__ VwalkShared VS;
  __shared__ uint64_t etab[32];
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  pz_etab_fill((pz_lds_u64*)etab);
  const int b = blockIdx.x;
  const int r = A.NR + b;
  const PzRecAhead ra = pz_sp_rec_ahead(A.ws, r, A.nseg);  // in flight beside the sequence's
  const SpecSeq s = A.seq[b];
  if (s.mode == SQ_DONE) return;
  const float ur = A.u_res[b];
  int tok;
  if (s.mode == SQ_RES) {
    const ResidualTerms<VEC> X = residual_terms<VEC>(A, s, et);
    const PzWalk W = pz_sp_walk_setup(X, r, A.nseg, A.nc, A.ws, lds, SS, -1, 0xffffffffu, &ra);
    if (threadIdx.x < 64) {
      PzAcc st;
      PzWalkCk ck;
      pz_sp_walk<PZ_STOP_NONE>(st, W, 0.0f, X, &ck);
      const float Z = pz_acc_value(st);
      int hit = -1;
      if (Z > 0.0f) {
        // the same sequence of adds: the CDF of r, stop at ur * Z < cdf,
        // resumed from the last state of the first walk below the stop
        PzAcc s2;
        hit = pz_sp_walk<PZ_STOP_GT>(s2, W, ur * Z, X, nullptr, &ck);
        if (hit >= A.V) hit = -1;
      }
      if (threadIdx.x == 0) {
        VS.Z = Z;
        VS.hit = hit;
      }
    }
    __syncthreads();
    if (VS.Z > 0.0f) {
      tok = VS.hit >= 0 ? VS.hit : A.seq[b].last;
    } else {
      // Z == 0: categorical draw from p of the target row (generate.c:157-169),
      // with records built by this workgroup alone (a rare path)
      PzExpTerms<PzTempRow<VEC>> Xp = p_terms<VEC>(A, s.qt, et);
      const int ntiles = pz_tiles(A.V);
      const PzRec REC = pz_rec_at(lds, ntiles * PZ_SEGS_PER_TILE);
      const int hit = pz_exact_draw(Xp, A.V, ntiles, ur, REC, RS);
      tok = hit >= 0 ? hit : A.V - 1;
    }
  } else {
    const PzExpTerms<PzTempRow<VEC>> X = p_terms<VEC>(A, s.qt, et);
    const PzWalk W = pz_sp_walk_setup(X, r, A.nseg, A.nc, A.ws, lds, SS, -1, 0xffffffffu, &ra);
    if (threadIdx.x < 64) {
      PzAcc st;
      int hit = pz_sp_walk<PZ_STOP_GT>(st, W, ur, X);
      if (hit >= A.V) hit = -1;
      if (threadIdx.x == 0) VS.hit = hit;
    }
    __syncthreads();
    tok = VS.hit >= 0 ? VS.hit : A.V - 1;
  }
  if (threadIdx.x == 0) {
    const int js = s.js;
    A.acc_len[b] = js;
    for (int j = 0; j <= A.K; j++)
      A.ids_out[(long)b * (A.K + 1) + j] = j < js ? A.draft_ids[b * A.K + j] : (j == js ? tok : -1);
  }
}

size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

// Outputs not yet written (no accepted length or id takes this value).
constexpr int32_t kSpecPending = INT32_MIN;

// Waits until every accepted length and output id has arrived in the mapped
// buffer (true), or gives up after two seconds (false).  Each value is one
// 4-byte store, so watching all of them needs no fence on the device side;
// it returns several microseconds sooner than a stream synchronisation.
bool wait_spec(volatile const int32_t* acc, int B, volatile const int32_t* out, int n) {
  const auto t0 = std::chrono::steady_clock::now();
  unsigned spins = 0;
  for (int i = 0; i < n; i++) {
    while (out[i] == kSpecPending || (i < B && acc[i] == kSpecPending))
      if ((++spins & 0xffffu) == 0 &&
          std::chrono::steady_clock::now() - t0 > std::chrono::seconds(2))
        return false;
  }
  return true;
}

template <bool VEC>
int launch_spec(pz_sampler* s, SpecArgs& A) {
  const size_t fixed = 4096;
  // stat and records over the NR rows: about two rounds of workgroups (fewer,
  // larger slices leave a second round mostly empty; more add overhead)
  const PzSplitPlan pl = pz_split_plan(A.V, (A.NR + 1) / 2, A.ws.smax);
  const PzSplitPlan pv = pz_split_plan(A.V, A.B, A.ws.smax);
  if (pl.nseg > A.ws.nsc) return -2;
  // two walking workgroups per CU fit when each takes at most half the LDS
  int nc = pz_sp_walk_nc(pl.nseg, (size_t)s->max_lds / 2 - fixed);
  if (nc < 12) nc = pz_sp_walk_nc(pl.nseg, (size_t)s->max_lds - fixed);
  if (nc < 1) return -2;
  const size_t walk = pz_sp_walk_lds(pl.nseg, nc);
  const size_t rec = pz_rec_bytes(A.V);  // the Z == 0 path's records
  const size_t lds_vw = walk > rec ? walk : rec;
  if (lds_vw + fixed > (size_t)s->max_lds) return -2;
  A.nseg = pl.nseg;
  A.nc = nc;
  auto kw = k_spec_walk<VEC>;
  auto kv = k_spec_vwalk<VEC>;
  if (walk > 65536 && hipFuncSetAttribute((const void*)kw,
                                          hipFuncAttributeMaxDynamicSharedMemorySize,
                                          (int)walk) != hipSuccess)
    return -1;
  if (lds_vw > 65536 && hipFuncSetAttribute((const void*)kv,
                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                            (int)lds_vw) != hipSuccess)
    return -1;
  const dim3 block(PZ_SP_BLOCK);
  A.spw = pl.spw;
  A.S = pl.S;
  hipLaunchKernelGGL(k_spec_stat<VEC>, dim3(pl.S, A.NR), block, 0, s->stream, A);
  hipLaunchKernelGGL(k_spec_rec<VEC>, dim3(pl.S, A.NR), block, 0, s->stream, A);
  hipLaunchKernelGGL(kw, dim3(A.NR), dim3(SPEC_WALK_BLOCK), walk, s->stream, A);
  A.spw = pv.spw;
  A.S = pv.S;
  hipLaunchKernelGGL(k_spec_vest<VEC>, dim3(pv.S, A.B), block, 0, s->stream, A);
  hipLaunchKernelGGL(k_spec_vrec<VEC>, dim3(pv.S, A.B), block, 0, s->stream, A);
  hipLaunchKernelGGL(kv, dim3(A.B), block, lds_vw, s->stream, A);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Checks the arguments, sizes the sequences' state and the row-split
// workspace (device scratch, grown when needed, after a stream
// synchronisation) and enqueues the launches on the sampler's stream.  The
// inputs and outputs are device-visible addresses (device memory or mapped
// pinned memory).
int spec_enqueue(pz_sampler* s, const float* d_target, const float* d_draft, int B, int K, int V,
                 long ld, int has_bonus, float temperature, const int32_t* ids_in,
                 const float* uacc_in, const float* ures_in, int32_t* acc_out,
                 int32_t* out_ids) {
  const int KT = K + (has_bonus ? 1 : 0);
  const bool onehot = d_draft == nullptr;  // greedy drafts: no draft rows
  const int NR = B * KT + (onehot ? 0 : B * K);
  const size_t o_seq = 0;
  const size_t o_ws = up256(o_seq + (size_t)B * sizeof(SpecSeq));
  const size_t dev_bytes = o_ws + pz_split_ws_layout(NR + B, V, 0, nullptr, nullptr);
  if (s->spec_dev_bytes < dev_bytes) {
    PZ_HIP(s, hipStreamSynchronize(s->stream));
    (void)hipFree(s->spec_dev);
    s->spec_dev = nullptr;
    s->spec_dev_bytes = 0;
    if (hipMalloc(&s->spec_dev, dev_bytes) != hipSuccess)
      return fail(s, PZ_ENOMEM, "spec scratch of %zu bytes", dev_bytes);
    s->spec_dev_bytes = dev_bytes;
  }
  char* d = static_cast<char*>(s->spec_dev);
  float T = temperature;
  if (T < 1e-6f) T = 1e-6f;  // temperature.c:10 (a NaN temperature stays NaN)
  SpecArgs A;
  memset(&A, 0, sizeof(A));
  A.target = d_target;
  A.draft = d_draft;
  A.ld = ld;
  A.V = V;
  A.B = B;
  A.K = K;
  A.KT = KT;
  A.NT = B * KT;
  A.NR = NR;
  A.has_bonus = has_bonus ? 1 : 0;
  A.onehot = onehot ? 1 : 0;
  A.T.t = T;
  A.T.inv = 1.0f / T;
  A.T.div = s->temp_mode == PZ_TEMP_DIV;
  A.draft_ids = ids_in;
  A.u_acc = uacc_in;
  A.u_res = ures_in;
  A.acc_len = acc_out;
  A.ids_out = out_ids;
  A.seq = reinterpret_cast<SpecSeq*>(d + o_seq);
  pz_split_ws_layout(NR + B, V, 0, d + o_ws, &A.ws);
  const bool vec = (ld % 4 == 0) && (((uintptr_t)d_target & 15) == 0) &&
                   (((uintptr_t)d_draft & 15) == 0);
  const int rc = vec ? launch_spec<true>(s, A) : launch_spec<false>(s, A);
  if (rc == -2) return fail(s, PZ_ENOTSUP, "V=%d needs more LDS than the device has", V);
  if (rc != 0) return fail(s, PZ_EDEVICE, "spec launch failed: %s",
                           hipGetErrorString(hipGetLastError()));
  return PZ_OK;
}

int spec_check(pz_sampler* s, int B, int K, int V, long ld) {
  if (B < 0 || K < 1 || K > 64 || V < 1 || ld < V) return fail(s, PZ_EINVAL, "bad spec shape");
  if (B > s->max_batch) return fail(s, PZ_ERANGE, "B=%d > max_batch=%d", B, s->max_batch);
  if (V > s->max_vocab) return fail(s, PZ_ERANGE, "V=%d > max_vocab=%d", V, s->max_vocab);
  return PZ_OK;
}

}  // namespace

namespace {

// greedy: drafts are the draft model's argmax (q one-hot; no draft logits)
int verify_async(pz_sampler* s, bool greedy, const float* d_target, const float* d_draft, int B,
                 int K, int V, long ld, int has_bonus, float temperature,
                 const int32_t* d_draft_ids, const float* d_u_acc, const float* d_u_res,
                 int32_t* d_acc_len_out, int32_t* d_ids_out) {
  if (!s) return PZ_EINVAL;
  int rc = spec_check(s, B, K, V, ld);
  if (rc != PZ_OK || B == 0) return rc;
  if (!d_target || (!greedy && !d_draft) || !d_draft_ids || !d_u_acc || !d_u_res ||
      !d_acc_len_out || !d_ids_out)
    return fail(s, PZ_EINVAL, "null spec argument");
  if (greedy) d_draft = nullptr;
  PZ_HIP(s, hipSetDevice(s->device));
  return spec_enqueue(s, d_target, d_draft, B, K, V, ld, has_bonus, temperature, d_draft_ids,
                      d_u_acc, d_u_res, d_acc_len_out, d_ids_out);
}

int verify_sync(pz_sampler* s, bool greedy, const float* d_target, const float* d_draft, int B,
                int K, int V, long ld, int has_bonus, float temperature,
                const int32_t* draft_ids, const float* u_acc, const float* u_res,
                int32_t* acc_len_out, int32_t* ids_out) {
  if (!s) return PZ_EINVAL;
  int rc = spec_check(s, B, K, V, ld);
  if (rc != PZ_OK || B == 0) return rc;
  if (!d_target || (!greedy && !d_draft) || !draft_ids || !u_acc || !u_res || !acc_len_out ||
      !ids_out)
    return fail(s, PZ_EINVAL, "null spec argument");
  if (greedy) d_draft = nullptr;
  PZ_HIP(s, hipSetDevice(s->device));
  // the inputs and outputs in mapped, coherent pinned memory: the kernels
  // read and write them there, no copies
  const size_t o_ids = 0;
  const size_t o_uacc = up256(o_ids + (size_t)B * K * 4);
  const size_t o_ures = up256(o_uacc + (size_t)B * K * 4);
  const size_t o_acc = up256(o_ures + (size_t)B * 4);
  const size_t o_out = up256(o_acc + (size_t)B * 4);
  const size_t io_bytes = up256(o_out + (size_t)B * (K + 1) * 4);
  if (s->spec_host_bytes < io_bytes) {
    PZ_HIP(s, hipStreamSynchronize(s->stream));
    s->spec_busy = false;
    (void)hipHostFree(s->spec_host);
    s->spec_host = nullptr;
    s->spec_zc = nullptr;
    s->spec_host_bytes = 0;
    void* z = nullptr;
    if (hipHostMalloc(&s->spec_host, io_bytes, hipHostMallocMapped | hipHostMallocCoherent) !=
            hipSuccess ||
        hipHostGetDevicePointer(&z, s->spec_host, 0) != hipSuccess)
      return fail(s, PZ_ENOMEM, "spec staging of %zu bytes", io_bytes);
    s->spec_zc = z;
    s->spec_host_bytes = io_bytes;
  }
  // A call returns once every output is back (wait_spec), and the kernels
  // write each sequence's outputs after their last read of its inputs: the
  // staging area is free here unless the previous call failed.
  if (s->spec_busy) {
    PZ_HIP(s, hipStreamSynchronize(s->stream));
    s->spec_busy = false;
  }
  char* h = static_cast<char*>(s->spec_host);
  char* z = static_cast<char*>(s->spec_zc);
  memcpy(h + o_ids, draft_ids, (size_t)B * K * 4);
  memcpy(h + o_uacc, u_acc, (size_t)B * K * 4);
  memcpy(h + o_ures, u_res, (size_t)B * 4);
  volatile int32_t* h_acc = reinterpret_cast<volatile int32_t*>(h + o_acc);
  volatile int32_t* h_out = reinterpret_cast<volatile int32_t*>(h + o_out);
  for (int b = 0; b < B; b++) h_acc[b] = kSpecPending;
  for (int i = 0; i < B * (K + 1); i++) h_out[i] = kSpecPending;
  s->spec_busy = true;
  rc = spec_enqueue(s, d_target, d_draft, B, K, V, ld, has_bonus, temperature,
                    reinterpret_cast<const int32_t*>(z + o_ids),
                    reinterpret_cast<const float*>(z + o_uacc),
                    reinterpret_cast<const float*>(z + o_ures),
                    reinterpret_cast<int32_t*>(z + o_acc), reinterpret_cast<int32_t*>(z + o_out));
  if (rc != PZ_OK) return rc;
  if (!wait_spec(h_acc, B, h_out, B * (K + 1))) {
    PZ_HIP(s, hipStreamSynchronize(s->stream));
    for (int i = 0; i < B * (K + 1); i++)
      if (h_out[i] == kSpecPending || (i < B && h_acc[i] == kSpecPending))
        return fail(s, PZ_EDEVICE, "speculative verification returned no result");
  }
  s->spec_busy = false;
  memcpy(acc_len_out, h + o_acc, (size_t)B * 4);
  memcpy(ids_out, h + o_out, (size_t)B * (K + 1) * 4);
  for (int b = 0; b < B; b++)
    if (acc_len_out[b] == PZ_ID_FAILED)
      return fail(s, PZ_EDEVICE, "sequence %d: a wait between workgroups gave up", b);
  return PZ_OK;
}

}  // namespace

extern "C" int pz_spec_verify_async(pz_sampler* s, const float* d_target, const float* d_draft,
                                    int B, int K, int V, long ld, int has_bonus,
                                    float temperature, const int32_t* d_draft_ids,
                                    const float* d_u_acc, const float* d_u_res,
                                    int32_t* d_acc_len_out, int32_t* d_ids_out) {
  return verify_async(s, false, d_target, d_draft, B, K, V, ld, has_bonus, temperature, d_draft_ids,
                      d_u_acc, d_u_res, d_acc_len_out, d_ids_out);
}

extern "C" int pz_spec_verify(pz_sampler* s, const float* d_target, const float* d_draft, int B,
                              int K, int V, long ld, int has_bonus, float temperature,
                              const int32_t* draft_ids, const float* u_acc, const float* u_res,
                              int32_t* acc_len_out, int32_t* ids_out) {
  return verify_sync(s, false, d_target, d_draft, B, K, V, ld, has_bonus, temperature, draft_ids, u_acc,
                     u_res, acc_len_out, ids_out);
}

extern "C" int pz_spec_verify_greedy_async(pz_sampler* s, const float* d_target, int B, int K,
                                           int V, long ld, int has_bonus, float temperature,
                                           const int32_t* d_draft_ids, const float* d_u_acc,
                                           const float* d_u_res, int32_t* d_acc_len_out,
                                           int32_t* d_ids_out) {
  return verify_async(s, true, d_target, nullptr, B, K, V, ld, has_bonus, temperature, d_draft_ids,
                      d_u_acc, d_u_res, d_acc_len_out, d_ids_out);
}

extern "C" int pz_spec_verify_greedy(pz_sampler* s, const float* d_target, int B, int K, int V,
                                     long ld, int has_bonus, float temperature,
                                     const int32_t* draft_ids, const float* u_acc,
                                     const float* u_res, int32_t* acc_len_out,
                                     int32_t* ids_out) {
  return verify_sync(s, true, d_target, nullptr, B, K, V, ld, has_bonus, temperature, draft_ids, u_acc,
                     u_res, acc_len_out, ids_out);
}
