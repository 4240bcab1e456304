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
//   pass 1 (HBM)  maximum, NaN check, per-segment estimates;
//   pass 2 (L2)   exact e (glibc-identical pz_expf) -> integer segment records
//                 at the predicted binade; wave 0 walks them: exact sum;
//   pass 3 (L2)   exact p = e * inv -> records for the CDF, only over the
//                 segments the estimated CDF says the draw can reach; wave 0
//                 walks them with the stop rule r < cdf and resolves the hit
//                 segment element by element.
#include "pz_device.h"
#include "pz_exact.h"
#include "pz_launch.h"
#include "pz_rowpass.h"

namespace {

struct CatShared {
  PzPass1Shared p1;
  PzDrawShared d;
};

template <bool VEC>
__global__ __launch_bounds__(PZ_RB) void k_categorical(
    const float* __restrict__ logits, long ld, int V, const int32_t* __restrict__ rows,
    const pz_row_params_dev* __restrict__ params, int n_params,
    const int32_t* __restrict__ hist, int H, int hcap, int pen_bytes,
    const float* __restrict__ u, int32_t* __restrict__ ids_out, float* __restrict__ p_out) {
  extern __shared__ __align__(16) char lds[];
  __shared__ CatShared S;
  const int row = pz_row_of(rows, blockIdx.x);
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const int tid = threadIdx.x;

  PzRow<VEC> R;
  R.x = logits + (long)row * ld;
  R.V = V;
  R.prm = &prm;
  pz_penalty_build<PZ_RB>(R.P, lds, V, hcap, hist ? hist + (long)row * H : nullptr, H, prm);

  const int ntiles = pz_tiles(V), nseg = ntiles * PZ_SEGS_PER_TILE;
  float* seg_m = reinterpret_cast<float*>(lds + pen_bytes);
  float* seg_s = seg_m + nseg;
  uint32_t* seg_d = reinterpret_cast<uint32_t*>(seg_s + nseg);
  uint32_t* seg_gf = seg_d + nseg;

  const float M = pz_pass1<8>(R, ntiles, seg_m, seg_s, S.p1);
  if (S.p1.any_nan || !(M > -__builtin_inff() && M < __builtin_inff())) {
    if (tid == 0) {
      ids_out[row] = V - 1;
      if (p_out) p_out[row] = __builtin_nanf("");
    }
    return;
  }
  const float sum = pz_exact_normaliser<4>(R, ntiles, M, -__builtin_inff(), seg_m, seg_s,
                                           seg_d, seg_gf, S.d);
  const float inv = 1.0f / sum;  // softmax.c:19-22
  const int hit = pz_exact_cdf_draw<4>(R, V, ntiles, M, inv, u[row], seg_m, seg_s, seg_d,
                                       seg_gf, S.d);
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
      p_out[row] = pz_expf(y - M) * inv;
    }
  }
}

template <bool VEC>
int launch_cat_t(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  const int pen = L.pen_any ? (int)((pz_penalty_lds_bytes(L.V, L.hcap) + 15) & ~(size_t)15) : 0;
  const size_t lds = pen + (size_t)pz_nseg(L.V) * 16;
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
