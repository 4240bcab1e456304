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
// Design (one 1024-thread workgroup per row):
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

}  // namespace

int pz_launch_categorical(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  if (n_rows <= 0) return 0;
  const bool vec = (L.ld % 4 == 0) && (((uintptr_t)L.logits & 15) == 0);
  return vec ? launch_cat_t<true>(L, n_rows, d_rows) : launch_cat_t<false>(L, n_rows, d_rows);
}
