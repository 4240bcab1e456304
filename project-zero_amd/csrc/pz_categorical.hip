// pz_categorical.hip -- batched full-vocabulary categorical draw, bit-exact
// with the reference's plain sampling path.
//
// Reference semantics (src/transformer/generate.c:157-169 after
// apply_temperature, with tn_softmax = src/math/softmax.c:4-23):
//   max by strict '>' from x[0]; e_i = expf(x_i - max) with a sequential fp32
//   sum in ascending id; p_i = e_i * (1/sum); then r = rng_float(),
//   cdf += p_i in ascending id, the first i with r < cdf, fallback V-1.
// A NaN anywhere in the row, or an infinite maximum, makes the sum NaN: no
// comparison succeeds and the draw is V-1.
//
// Row-split design (the default, any batch): each row is cut into slices of
// segments over several workgroups (pz_split.h):
//   k_cat_front  (HBM)  each slice read once into LDS: its maximum and NaN
//                       flag, the row's workgroups meet for the row maximum,
//                       then the segments' mass estimates, a second meeting
//                       for the mass before the slice, and the exact
//                       e = expf(y - M) terms' records at the predicted
//                       grids (pz_sp_front);
//     (or, for slices that do not fit: k_cat_stat (HBM) maxima and
//     estimates, k_cat_rec (L2) the records)
//   k_cat_walk          one workgroup per row walks them: the exact
//                       sequential normaliser, inv = 1 / sum;
//   k_cat_prec   (L2)   the records of p = e * inv at the CDF's predicted
//                       grids (estimates: the stat pass's times inv);
//   k_cat_draw          one workgroup per row walks the CDF of p to the
//                       first cdf > r, the id (V-1 when none).
// One-workgroup design (k_categorical, rows whose workspace does not fit):
//   pass 1 (HBM)  maximum and NaN check;
//   pass 2 (L2)   exact e (glibc-identical pz_expf) -> integer segment records
//                 at predicted binades; wave 0 walks them: exact sum;
//   pass 3 (L2)   exact p = e * inv -> records for the CDF, only as far as the
//                 estimated CDF says the draw can reach; wave 0 walks them with
//                 the stop rule r < cdf and resolves the hit segment element by
//                 element.
#include "pz_device.h"
#include "pz_exact.h"
#include "pz_launch.h"
#include "pz_rowpass.h"
#include "pz_split.h"

namespace {

struct CatShared {
  PzPass1Shared p1;
  PzRecShared r;
};

template <bool VEC>
__global__ __launch_bounds__(PZ_RB) void k_categorical(
    const float* __restrict__ logits, long ld, int V, const int32_t* __restrict__ rows,
    const pz_row_params_dev* __restrict__ params, int n_params,
    const int32_t* __restrict__ hist, int H, int hcap, int pen_bytes,
    const float* __restrict__ u, int32_t* __restrict__ ids_out, float* __restrict__ p_out) {
  extern __shared__ __align__(16) char lds[];
  __shared__ CatShared S;
  __shared__ uint64_t etab[32];
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  pz_etab_fill((pz_lds_u64*)etab);  // ordered by pz_pass1's barriers
  const int row = pz_row_of(rows, blockIdx.x);
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const int tid = threadIdx.x;

  PzRow<VEC> R;
  R.x = logits + (long)row * ld;
  R.V = V;
  R.T = PzTemp::of(prm);
  pz_penalty_build<PZ_RB>(R.P, lds, V, hcap, hist ? hist + (long)row * H : nullptr, H, prm);

  const int ntiles = pz_tiles(V), nseg = ntiles * PZ_SEGS_PER_TILE;
  const PzRec REC = pz_rec_at(lds + pen_bytes, nseg);

  const float M = pz_pass1<8>(R, ntiles, S.p1);
  if (S.p1.any_nan || !(M > -__builtin_inff() && M < __builtin_inff())) {
    if (tid == 0) {
      ids_out[row] = V - 1;
      if (p_out) p_out[row] = __builtin_nanf("");
    }
    return;
  }
  PzExpTerms<PzRow<VEC>> X;
  X.R = R;
  X.M = M;
  X.thr = -__builtin_inff();
  X.inv = 1.0f;
  X.as_p = false;
  X.et = et;
  const float sum = pz_exact_sum(X, ntiles, REC, S.r);
  const float inv = 1.0f / sum;  // softmax.c:19-22
  X.inv = inv;
  X.as_p = true;
  const int hit = pz_exact_draw(X, V, ntiles, u[row], REC, S.r);
  if (tid == 0) {
    const int id = hit >= 0 ? hit : V - 1;  // generate.c:161
    ids_out[row] = id;
    if (p_out) {
      float yy[4];
      const int e0 = id & ~3;
      R.get(e0, yy);
      float y = yy[0];
#pragma unroll
      for (int c = 1; c < 4; c++)
        if (e0 + c == id) y = yy[c];
      p_out[row] = pz_expf_l(y - M, et) * inv;
    }
  }
}

template <bool VEC>
int launch_cat_t(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  const int pen = L.pen_any ? (int)((pz_penalty_lds_bytes(L.V, L.hcap) + 15) & ~(size_t)15) : 0;
  const size_t lds = pen + pz_rec_bytes(L.V);
  if (lds + sizeof(CatShared) + 64 > (size_t)L.max_lds) return -2;
  auto kern = k_categorical<VEC>;
  if (lds > 65536 && hipFuncSetAttribute((const void*)kern,
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)lds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(kern, dim3(n_rows), dim3(PZ_RB), lds, L.stream, L.logits, L.ld, L.V, d_rows,
                     L.params, L.n_params, L.hist, L.H, L.hcap, pen, L.u, L.ids, L.p_out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}


// ---- row-split path --------------------------------------------------------
struct CatArgs {
  const float* logits;
  long ld;
  int V;
  const int32_t* rows;
  const pz_row_params_dev* params;
  int n_params;
  const int32_t* hist;
  int H, hcap;
  const float* u;
  int32_t* ids_out;
  float* p_out;
  PzSplitWs ws;
  int nseg, spw, S, nc;
  int est_abs;  // seg_s holds the front pass's absolute estimates
};

template <bool VEC>
__device__ __forceinline__ PzRow<VEC> cat_row(const CatArgs& A, int row, char* lds, int lo,
                                              int hi) {
  PzRow<VEC> R;
  const pz_row_params_dev& prm = pz_params_of(A.params, A.n_params, row);
  R.x = A.logits + (long)row * A.ld;
  R.V = A.V;
  R.T = PzTemp::of(prm);
  const int32_t* hrow = A.hist ? A.hist + (long)row * A.H : nullptr;
  pz_penalty_build_range<PZ_SP_BLOCK>(R.P, lds, A.V, lo, hi, A.hcap, hrow, A.H, prm);
  return R;
}

// softmax.c:4-23 gives NaN everywhere when any y is NaN or the maximum is not
// finite: the draw then falls back to V-1 (generate.c:161)
__device__ __forceinline__ bool cat_bad(uint32_t flags) {
  return (flags & (PZ_RS_NAN | PZ_RS_NONFIN | PZ_RS_FAILED)) != 0;
}

// Stat and records in one read of each slice (pen_bytes: the slice's penalty
// tables, then the slice).
template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_cat_front(CatArgs A,
                                                                            int pen_bytes,
                                                                            uint32_t cap) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ PzFrontShared F;
  __shared__ uint64_t etab[32];
  pz_etab_fill((pz_lds_u64*)etab);
  const int row = pz_row_of(A.rows, blockIdx.y);
  const PzSlice sl = pz_sp_slice(A.nseg, A.spw);
  if (threadIdx.x == 0) {
    SS.any = 0u;
    F.fail = 0;
  }
  const PzRow<VEC> R = cat_row<VEC>(A, row, lds, pz_sp_lo(sl), pz_sp_hi(sl, A.V));
  __syncthreads();
  pz_sp_front(R, row, sl, A.S, -__builtin_inff(), A.ws, SS, F, (pz_lds_f32*)(lds + pen_bytes),
              (const pz_lds_u64*)etab, cap);
}

template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_cat_stat(CatArgs A) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  const int row = pz_row_of(A.rows, blockIdx.y);
  const PzSlice sl = pz_sp_slice(A.nseg, A.spw);
  if (threadIdx.x == 0) SS.any = 0u;
  const PzRow<VEC> R = cat_row<VEC>(A, row, lds, pz_sp_lo(sl), pz_sp_hi(sl, A.V));
  __syncthreads();
  pz_sp_stat_slice(R, row, sl, A.ws, SS, true);
}

template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_cat_rec(CatArgs A) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ uint64_t etab[32];
  pz_etab_fill((pz_lds_u64*)etab);
  const int row = pz_row_of(A.rows, blockIdx.y);
  pz_sp_row_stat(row, A.S, A.ws, SS);
  if (cat_bad(SS.any)) return;
  const PzSlice sl = pz_sp_slice(A.nseg, A.spw);
  const PzEstRel est{A.ws.seg_m + (size_t)row * A.ws.nsc, A.ws.seg_s + (size_t)row * A.ws.nsc,
                     SS.M};
  const float carry = pz_sp_prefix(est, sl.k0, SS);
  pz_sp_predict(est, carry, row, sl, A.ws, SS);
  PzExpTerms<PzRow<VEC>> X;
  X.R = cat_row<VEC>(A, row, lds, pz_sp_lo(sl), pz_sp_hi(sl, A.V));
  X.M = SS.M;
  X.thr = -__builtin_inff();
  X.inv = 1.0f;
  X.as_p = false;
  X.et = (const pz_lds_u64*)etab;
  __syncthreads();
  pz_sp_records(X, row, sl, A.ws, nullptr, true);
}

// Estimated p mass of segment k: the e estimate times inv (abs: the front
// pass's estimates in units of exp(y - M), else the stat pass's relative
// ones).
struct CatEstP {
  PzEstRel e;
  float inv;
  int abs;
  __device__ __forceinline__ float operator()(int k) const {
    return (abs ? e.s[k] : e(k)) * inv;
  }
};

// One workgroup per row (512 threads: two per CU with room for the walk's
// LDS): the exact normaliser.  pen_bytes: the row's penalty tables, then the
// walk's arrays.
constexpr int CAT_WALK_BLOCK = 512;
template <bool VEC>
__global__ __launch_bounds__(CAT_WALK_BLOCK) void k_cat_walk(CatArgs A, int pen_bytes) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ uint64_t etab[32];
  __shared__ float sum_sh;
  pz_etab_fill((pz_lds_u64*)etab);
  const int row = pz_row_of(A.rows, blockIdx.x);
  const PzRecAhead ra = pz_sp_rec_ahead(A.ws, row, A.nseg);  // in flight beside the maxima
  PzRowState& rs = A.ws.rs[row];
  const int failed = rs.i[7];
  pz_sp_clear_meet(A.ws, row);  // the front launch's meetings are over
  pz_sp_row_stat(row, A.S, A.ws, SS);
  if (failed || cat_bad(SS.any)) {
    if (threadIdx.x == 0) {
      rs.M = SS.M;
      rs.flags = SS.any | (failed ? PZ_RS_FAILED : 0u);
      rs.inv = __builtin_nanf("");
      rs.i[7] = 0;
    }
    return;
  }
  const pz_row_params_dev& prm = pz_params_of(A.params, A.n_params, row);
  PzExpTerms<PzRow<VEC>> X;
  X.R.x = A.logits + (long)row * A.ld;
  X.R.V = A.V;
  X.R.T = PzTemp::of(prm);
  pz_penalty_build_range<CAT_WALK_BLOCK>(X.R.P, lds, A.V, 0, A.V, A.hcap,
                                         A.hist ? A.hist + (long)row * A.H : nullptr, A.H, prm);
  X.M = SS.M;
  X.thr = -__builtin_inff();
  X.inv = 1.0f;
  X.as_p = false;
  X.et = (const pz_lds_u64*)etab;
  __syncthreads();
  const PzWalk W =
      pz_sp_walk_setup(X, row, A.nseg, A.nc, A.ws, lds + pen_bytes, SS, -1, 0xffffffffu, &ra);
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

template <bool VEC>
__global__ __launch_bounds__(PZ_SP_BLOCK) PZ_SP_TWO_PER_CU void k_cat_prec(CatArgs A) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ uint64_t etab[32];
  pz_etab_fill((pz_lds_u64*)etab);
  const int row = pz_row_of(A.rows, blockIdx.y);
  const PzRowState rs = A.ws.rs[row];
  if (cat_bad(rs.flags)) return;
  const PzSlice sl = pz_sp_slice(A.nseg, A.spw);
  const CatEstP est{{A.ws.seg_m + (size_t)row * A.ws.nsc, A.ws.seg_s + (size_t)row * A.ws.nsc,
                     rs.M},
                    rs.inv, A.est_abs};
  const float carry = pz_sp_prefix(est, sl.k0, SS);
  pz_sp_predict(est, carry, row, sl, A.ws, SS);
  PzExpTerms<PzRow<VEC>> X;
  X.R = cat_row<VEC>(A, row, lds, pz_sp_lo(sl), pz_sp_hi(sl, A.V));
  X.M = rs.M;
  X.thr = -__builtin_inff();
  X.inv = rs.inv;
  X.as_p = true;
  X.et = (const pz_lds_u64*)etab;
  __syncthreads();
  pz_sp_records(X, row, sl, A.ws, nullptr, true);
}

// One workgroup per row (as the normaliser walk): the CDF of p in ascending
// id to the first cdf > r (generate.c:162-168), V-1 when none (:161).
template <bool VEC>
__global__ __launch_bounds__(CAT_WALK_BLOCK) void k_cat_draw(CatArgs A, int pen_bytes) {
  extern __shared__ __align__(16) char lds[];
  __shared__ PzSpShared SS;
  __shared__ uint64_t etab[32];
  __shared__ int hit_sh;
  pz_etab_fill((pz_lds_u64*)etab);
  const int row = pz_row_of(A.rows, blockIdx.x);
  const PzRecAhead ra = pz_sp_rec_ahead(A.ws, row, A.nseg);  // in flight beside the row state
  const PzRowState rs = A.ws.rs[row];
  if (cat_bad(rs.flags)) {
    if (threadIdx.x == 0) {
      A.ids_out[row] = (rs.flags & PZ_RS_FAILED) ? PZ_ID_FAILED : A.V - 1;
      if (A.p_out) A.p_out[row] = __builtin_nanf("");
    }
    return;
  }
  const pz_row_params_dev& prm = pz_params_of(A.params, A.n_params, row);
  PzExpTerms<PzRow<VEC>> X;
  X.R.x = A.logits + (long)row * A.ld;
  X.R.V = A.V;
  X.R.T = PzTemp::of(prm);
  pz_penalty_build_range<CAT_WALK_BLOCK>(X.R.P, lds, A.V, 0, A.V, A.hcap,
                                      A.hist ? A.hist + (long)row * A.H : nullptr, A.H, prm);
  X.M = rs.M;
  X.thr = -__builtin_inff();
  X.inv = rs.inv;
  X.as_p = true;
  X.et = (const pz_lds_u64*)etab;
  const float r = A.u[row];
  __syncthreads();
  const PzWalk W =
      pz_sp_walk_setup(X, row, A.nseg, A.nc, A.ws, lds + pen_bytes, SS, -1, 0xffffffffu, &ra);
  if (threadIdx.x < 64) {
    PzAcc st;
    int hit = pz_sp_walk<PZ_STOP_GT>(st, W, r, X);
    if (hit >= A.V) hit = -1;
    if (threadIdx.x == 0) hit_sh = hit;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int id = hit_sh >= 0 ? hit_sh : A.V - 1;
    A.ids_out[row] = id;
    if (A.p_out) {
      float yy[4];
      const int e0 = id & ~3;
      X.R.get(e0, yy);
      float y = yy[0];
#pragma unroll
      for (int c = 1; c < 4; c++)
        if (e0 + c == id) y = yy[c];
      A.p_out[row] = X.exact_term(y);
    }
  }
}

template <bool VEC>
int launch_cat_split(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  const PzSplitWs& ws = L.ws;
  if (!ws.rs || !ws.rec) return -2;
  // the front pass when its workgroups run in one round (at larger batches
  // the rounds wait on each other's meetings: the separate stat and records
  // passes are quicker), a slice fits in LDS beside its tables (two
  // workgroups per CU) and a row's slices fit the device together
  const PzSplitPlan pf = pz_front_plan(L.V, n_rows, ws.smax);
  const size_t pen_f = L.pen_any
                           ? (pz_penalty_lds_bytes(pf.spw * PZ_SP_SEG, L.hcap) + 15) & ~(size_t)15
                           : 0;
  const size_t lds_front = pen_f + (size_t)pf.spw * PZ_SP_SEG * 4;
  const bool front = (long)n_rows * pf.S <= PZ_SP_TARGET_WG && pf.S <= 64 &&
                     (L.n_cu <= 0 || pf.S <= L.n_cu) && ws.meet &&
                     2 * (lds_front + 4096) <= (size_t)L.max_lds;
  const PzSplitPlan pl = front ? pf : pz_split_plan(L.V, n_rows, ws.smax);
  if (pl.nseg > ws.nsc || pl.S > ws.smax) return -2;
  const size_t fixed = 4096;
  auto pen = [&](int n) {
    return L.pen_any ? (pz_penalty_lds_bytes(n, L.hcap) + 15) & ~(size_t)15 : (size_t)0;
  };
  const size_t pen_slice = pen(pl.spw * PZ_SP_SEG), pen_full = pen(L.V);
  // the normaliser walk: two workgroups per CU when the walk fits in half the LDS
  int nc = pz_sp_walk_nc(pl.nseg, (size_t)L.max_lds / 2 - fixed - pen_full);
  if (nc < 12) nc = pz_sp_walk_nc(pl.nseg, (size_t)L.max_lds - fixed - pen_full);
  if (nc < 1) return -2;
  const size_t lds_walk = pen_full + pz_sp_walk_lds(pl.nseg, nc);
  if (pen_slice + fixed > (size_t)L.max_lds || lds_walk + fixed > (size_t)L.max_lds) return -2;
  CatArgs A;
  A.logits = L.logits;
  A.ld = L.ld;
  A.V = L.V;
  A.rows = d_rows;
  A.params = L.params;
  A.n_params = L.n_params;
  A.hist = L.hist;
  A.H = L.H;
  A.hcap = L.hcap;
  A.u = L.u;
  A.ids_out = L.ids;
  A.p_out = L.p_out;
  A.ws = ws;
  A.nseg = pl.nseg;
  A.spw = pl.spw;
  A.S = pl.S;
  A.nc = nc;
  A.est_abs = front ? 1 : 0;
  const void* big[2] = {(const void*)k_cat_walk<VEC>, (const void*)k_cat_draw<VEC>};
  for (int i = 0; i < 2; i++)
    if (lds_walk > 65536 &&
        hipFuncSetAttribute(big[i], hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_walk) !=
            hipSuccess)
      return -1;
  const dim3 grid(pl.S, n_rows), block(PZ_SP_BLOCK);
  if (front) {
    auto kf = k_cat_front<VEC>;
    if (lds_front > 65536 &&
        hipFuncSetAttribute((const void*)kf, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds_front) != hipSuccess)
      return -1;
    hipLaunchKernelGGL(kf, grid, block, lds_front, L.stream, A, (int)pen_f, L.wait_polls);
  } else {
    hipLaunchKernelGGL(k_cat_stat<VEC>, grid, block, pen_slice, L.stream, A);
    hipLaunchKernelGGL(k_cat_rec<VEC>, grid, block, pen_slice, L.stream, A);
  }
  hipLaunchKernelGGL(k_cat_walk<VEC>, dim3(n_rows), dim3(CAT_WALK_BLOCK), lds_walk, L.stream, A,
                     (int)pen_full);
  hipLaunchKernelGGL(k_cat_prec<VEC>, grid, block, pen_slice, L.stream, A);
  hipLaunchKernelGGL(k_cat_draw<VEC>, dim3(n_rows), dim3(CAT_WALK_BLOCK), lds_walk, L.stream, A,
                     (int)pen_full);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

int pz_launch_categorical(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  if (n_rows <= 0) return 0;
  const bool vec = (L.ld % 4 == 0) && (((uintptr_t)L.logits & 15) == 0);
  const int rc = vec ? launch_cat_split<true>(L, n_rows, d_rows)
                     : launch_cat_split<false>(L, n_rows, d_rows);
  if (rc != -2) return rc;
  return vec ? launch_cat_t<true>(L, n_rows, d_rows) : launch_cat_t<false>(L, n_rows, d_rows);
}
