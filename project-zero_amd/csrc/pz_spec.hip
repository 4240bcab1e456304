// pz_spec.hip -- speculative-draft verification on the GPU (accept/reject and
// residual resampling), with the reference's fp32 softmax arithmetic.
//
// The reference has no speculative decoding (docs/architecture/
// IMPLEMENTATION_PLAN.md:1664-1693 is a plan only); the rule follows
// Leviathan et al. 2023, Alg. 1, built from the reference's own pieces:
//   p = softmax(target_j / T), q = softmax(draft_j / T) with
//   apply_temperature (temperature.c:8-25) and softmax.c:4-23;
//   draft d_j is accepted iff u_acc < p(d_j) / q(d_j) (q(d_j) == 0 rejects);
//   at the first rejection r(x) = max(0, p(x) - q(x)) (fp32 difference),
//   Z = sequential fp32 sum of r in ascending id, and the token is the first
//   x with u_res * Z < cdf_r(x) (the last x with r(x) > 0 if none); when
//   Z == 0 it is drawn from p with generate.c:157-169.  With every draft
//   accepted and a bonus target row, the bonus token is drawn from p_K with
//   u_res the same way.
//
// Kernels:
//   k_spec_rows    one workgroup per logits row (all target rows, then all
//                  draft rows): maximum, exact softmax normaliser, NaN/inf
//                  degeneracy; target rows also store their pass-1
//                  estimates for a later CDF draw.
//   k_spec_verify  one workgroup per sequence: acceptance tests (two logits
//                  per draft), then the residual (exact Z and draw) or the
//                  bonus / Z == 0 categorical draw.
#include <string.h>

#include "pz_device.h"
#include "pz_exact.h"
#include "pz_launch.h"
#include "pz_rowpass.h"
#include "pz_sampler_impl.h"

namespace {

struct SpecRowsShared {
  PzPass1Shared p1;
  PzDrawShared d;
};

template <bool VEC>
__global__ __launch_bounds__(PZ_RB) void k_spec_rows(
    const float* __restrict__ target, const float* __restrict__ draft, long ld, int V, int B,
    int K, int KT, const pz_row_params_dev* __restrict__ prm, float* __restrict__ stats,
    float* __restrict__ seg_store) {
  extern __shared__ __align__(16) char lds[];
  __shared__ SpecRowsShared S;
  const int q = blockIdx.x, tid = threadIdx.x;
  const int NT = B * KT;
  PzTempRow<VEC> R;
  R.x = q < NT ? target + (long)q * ld : draft + (long)(q - NT) * ld;
  R.V = V;
  R.prm = prm;
  const int ntiles = pz_tiles(V), nseg = ntiles * PZ_SEGS_PER_TILE;
  float* seg_m = reinterpret_cast<float*>(lds);
  float* seg_s = seg_m + nseg;
  uint32_t* seg_d = reinterpret_cast<uint32_t*>(seg_s + nseg);
  uint32_t* seg_gf = seg_d + nseg;

  const float M = pz_pass1<8>(R, ntiles, seg_m, seg_s, S.p1);
  const bool bad = S.p1.any_nan || !(M > -__builtin_inff() && M < __builtin_inff());
  float inv = __builtin_nanf("");
  if (!bad) {
    const float sum = pz_exact_normaliser<4>(R, ntiles, M, -__builtin_inff(), seg_m, seg_s,
                                             seg_d, seg_gf, S.d);
    inv = 1.0f / sum;
  }
  if (tid == 0) {
    stats[4 * (long)q] = M;
    stats[4 * (long)q + 1] = inv;
    stats[4 * (long)q + 2] = bad ? 1.0f : 0.0f;
  }
  if (q < NT) {
    float* dst = seg_store + (long)q * nseg * 2;
    for (int k = tid; k < nseg; k += PZ_RB) {
      dst[k] = seg_m[k];
      dst[nseg + k] = seg_s[k];
    }
  }
}

// p(x) of one element of a row whose softmax statistics are (M, inv).
template <bool VEC>
__device__ __forceinline__ float prob_at(const PzTempRow<VEC>& R, int x, float M, float inv) {
  return pz_expf(pz_temper(R.x[x], *R.prm) - M) * inv;
}

// Residual terms r(x) = max(0, p(x) - q(x)) of elements e0..e0+3.
template <bool VEC, bool EXACT>
struct ResidualRow {
  PzTempRow<VEC> T, D;
  float MT, invT, MD, invD;
  __device__ __forceinline__ void terms(int e0, float (&v)[4]) const {
    float yt[4], yd[4];
    const int n = T.get(e0, yt);
    D.get(e0, yd);
#pragma unroll
    for (int c = 0; c < 4; c++) {
      float r = 0.0f;
      if (c < n) {
        const float p = EXACT ? pz_expf(yt[c] - MT) * invT : __expf(yt[c] - MT) * invT;
        const float qq = EXACT ? pz_expf(yd[c] - MD) * invD : __expf(yd[c] - MD) * invD;
        const float t = p - qq;
        r = t > 0.0f ? t : 0.0f;
      }
      v[c] = r;
    }
  }
  __device__ __forceinline__ void operator()(int k, float (&v)[4]) const { terms(pz_seg_e0(k), v); }
};

struct SpecVerifyShared {
  PzDrawShared d;
  int jstar;
  int last;
  float Z;
  int hit;
};

template <bool VEC>
__global__ __launch_bounds__(PZ_RB) void k_spec_verify(
    const float* __restrict__ target, const float* __restrict__ draft, long ld, int V, int B,
    int K, int KT, int has_bonus, const pz_row_params_dev* __restrict__ prm,
    const float* __restrict__ stats, const float* __restrict__ seg_store,
    const int32_t* __restrict__ draft_ids, const float* __restrict__ u_acc,
    const float* __restrict__ u_res, int32_t* __restrict__ acc_len,
    int32_t* __restrict__ ids_out) {
  extern __shared__ __align__(16) char lds[];
  __shared__ SpecVerifyShared S;
  const int b = blockIdx.x, tid = threadIdx.x, w = tid >> 6;
  const int NT = B * KT;
  const int ntiles = pz_tiles(V), nseg = ntiles * PZ_SEGS_PER_TILE;
  float* seg_m = reinterpret_cast<float*>(lds);
  float* seg_s = seg_m + nseg;
  uint32_t* seg_d = reinterpret_cast<uint32_t*>(seg_s + nseg);
  uint32_t* seg_gf = seg_d + nseg;

  // ---- acceptance tests, in draft order, up to the first rejection
  if (tid == 0) {
    int j = 0;
    for (; j < K; j++) {
      const int qt = b * KT + j, qd = NT + b * K + j;
      const int d = draft_ids[b * K + j];
      bool accept = false;
      if (d >= 0 && d < V) {
        PzTempRow<VEC> RT{target + (long)qt * ld, V, prm};
        PzTempRow<VEC> RD{draft + (long)(qd - NT) * ld, V, prm};
        const float pd = prob_at(RT, d, stats[4 * qt], stats[4 * qt + 1]);
        const float qv = prob_at(RD, d, stats[4 * qd], stats[4 * qd + 1]);
        accept = qv > 0.0f && u_acc[b * K + j] < pd / qv;
      }
      if (!accept) break;
    }
    S.jstar = j;
    S.last = 0;
  }
  __syncthreads();
  const int js = S.jstar;
  const float ur = u_res[b];
  int tok = -1;
  int cat_row = -1;  // target row to draw from with the categorical rule
  if (js < K) {
    const int qt = b * KT + js, qd = NT + b * K + js;
    const bool badT = stats[4 * qt + 2] != 0.0f, badD = stats[4 * qd + 2] != 0.0f;
    if (badT) {
      tok = V - 1;  // p is NaN everywhere: r == 0, and the p-draw falls back
    } else if (badD) {
      cat_row = qt;  // q is NaN: every p - q fails t > 0, Z == 0
    } else {
      ResidualRow<VEC, false> A;
      ResidualRow<VEC, true> E;
      A.T = PzTempRow<VEC>{target + (long)qt * ld, V, prm};
      A.D = PzTempRow<VEC>{draft + (long)(qd - NT) * ld, V, prm};
      A.MT = stats[4 * qt];
      A.invT = stats[4 * qt + 1];
      A.MD = stats[4 * qd];
      A.invD = stats[4 * qd + 1];
      E.T = A.T;
      E.D = A.D;
      E.MT = A.MT;
      E.invT = A.invT;
      E.MD = A.MD;
      E.invD = A.invD;
      // pass A: per-segment estimates of the residual mass
      for (int t = 0; t < ntiles; t++) {
        float v[4];
        A.terms(pz_tile_e0(t), v);
        const float s = pz_wave_sum(v[0] + v[1] + v[2] + v[3]);
        if ((tid & 63) == 0) {
          seg_m[t * PZ_SEGS_PER_TILE + w] = 0.0f;
          seg_s[t * PZ_SEGS_PER_TILE + w] = s;
        }
      }
      __syncthreads();
      if (w == 0) pz_predict_grids(seg_m, seg_s, nseg, 0.0f, 1.0f, seg_gf);
      __syncthreads();
      // pass B: exact residual terms -> records, and the last positive term
      int lastpos = -1;
      for (int t = 0; t < ntiles; t++) {
        float v[4];
        const int e0 = pz_tile_e0(t);
        E.terms(e0, v);
#pragma unroll
        for (int c = 0; c < 4; c++)
          if (v[c] > 0.0f) lastpos = e0 + c;
        const int k = t * PZ_SEGS_PER_TILE + w;
        pz_segment_record(v, seg_gf[k], true, seg_d, seg_gf, k);
      }
      if (lastpos > 0) atomicMax(&S.last, lastpos);
      __syncthreads();
      if (w == 0) {
        PzAcc st;
        st.n = 0;
        st.g = 1;
        pz_wave_walk(st, seg_d, seg_gf, nseg, 0.0f, PZ_STOP_NONE, E);
        const float Z = pz_acc_value(st);
        int hit = -1;
        if (Z > 0.0f) {
          PzAcc s2;
          s2.n = 0;
          s2.g = 1;
          hit = pz_wave_walk(s2, seg_d, seg_gf, nseg, ur * Z, PZ_STOP_GT, E);
          if (hit >= V) hit = -1;
        }
        if (tid == 0) {
          S.Z = Z;
          S.hit = hit;
        }
      }
      __syncthreads();
      if (S.Z > 0.0f) tok = S.hit >= 0 ? S.hit : S.last;
      else cat_row = qt;
    }
  } else if (has_bonus) {
    const int qt = b * KT + K;
    if (stats[4 * qt + 2] != 0.0f) tok = V - 1;
    else cat_row = qt;
  }
  if (cat_row >= 0) {
    // categorical draw from p of a target row (generate.c:157-169)
    const float* src = seg_store + (long)cat_row * nseg * 2;
    for (int k = tid; k < nseg; k += PZ_RB) {
      seg_m[k] = src[k];
      seg_s[k] = src[nseg + k];
    }
    __syncthreads();
    PzTempRow<VEC> RT{target + (long)cat_row * ld, V, prm};
    const int hit = pz_exact_cdf_draw<4>(RT, V, ntiles, stats[4 * cat_row],
                                         stats[4 * cat_row + 1], ur, seg_m, seg_s, seg_d,
                                         seg_gf, S.d);
    tok = hit >= 0 ? hit : V - 1;
  }
  if (tid == 0) {
    acc_len[b] = js;
    for (int j = 0; j <= K; j++)
      ids_out[(long)b * (K + 1) + j] = j < js ? draft_ids[b * K + j] : (j == js ? tok : -1);
  }
}

size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

template <bool VEC>
int launch_spec(pz_sampler* s, const float* d_target, const float* d_draft, long ld, int V,
                int B, int K, int KT, int has_bonus, const pz_row_params_dev* d_prm,
                float* d_stats, float* d_seg, const int32_t* d_ids_in, const float* d_uacc,
                const float* d_ures, int32_t* d_acc, int32_t* d_ids_out) {
  const size_t lds = (size_t)pz_nseg(V) * 16;
  if (lds + 256 > (size_t)s->max_lds) return -2;
  auto k1 = k_spec_rows<VEC>;
  auto k2 = k_spec_verify<VEC>;
  if (lds > 65536) {
    if (hipFuncSetAttribute((const void*)k1, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess ||
        hipFuncSetAttribute((const void*)k2, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return -1;
  }
  const int NR = B * KT + B * K;
  hipLaunchKernelGGL(k1, dim3(NR), dim3(PZ_RB), lds, s->stream, d_target, d_draft, ld, V, B, K,
                     KT, d_prm, d_stats, d_seg);
  hipLaunchKernelGGL(k2, dim3(B), dim3(PZ_RB), lds, s->stream, d_target, d_draft, ld, V, B, K, KT,
                     has_bonus, d_prm, d_stats, d_seg, d_ids_in, d_uacc, d_ures, d_acc,
                     d_ids_out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

extern "C" int pz_spec_verify(pz_sampler* s, const float* d_target, const float* d_draft, int B,
                              int K, int V, long ld, int has_bonus, float temperature,
                              const int32_t* draft_ids, const float* u_acc, const float* u_res,
                              int32_t* acc_len_out, int32_t* ids_out) {
  if (!s) return PZ_EINVAL;
  if (B < 0 || K < 1 || V < 1 || ld < V) return fail(s, PZ_EINVAL, "bad spec shape");
  if (B == 0) return PZ_OK;
  if (!d_target || !d_draft || !draft_ids || !u_acc || !u_res || !acc_len_out || !ids_out)
    return fail(s, PZ_EINVAL, "null spec argument");
  if (B > s->max_batch) return fail(s, PZ_ERANGE, "B=%d > max_batch=%d", B, s->max_batch);
  if (V > s->max_vocab) return fail(s, PZ_ERANGE, "V=%d > max_vocab=%d", V, s->max_vocab);
  PZ_HIP(s, hipSetDevice(s->device));
  const int KT = K + (has_bonus ? 1 : 0);
  const int NR = B * KT + B * K;
  const int nseg = pz_nseg(V);

  // one input block and one output block, identical layout host and device
  const size_t o_prm = 0;
  const size_t o_ids = up256(o_prm + sizeof(pz_row_params_dev));
  const size_t o_uacc = up256(o_ids + (size_t)B * K * 4);
  const size_t o_ures = up256(o_uacc + (size_t)B * K * 4);
  const size_t in_bytes = up256(o_ures + (size_t)B * 4);
  const size_t o_acc = in_bytes;
  const size_t o_out = up256(o_acc + (size_t)B * 4);
  const size_t io_bytes = up256(o_out + (size_t)B * (K + 1) * 4);
  const size_t o_stats = io_bytes;
  const size_t o_seg = up256(o_stats + (size_t)NR * 16);
  const size_t dev_bytes = up256(o_seg + (size_t)B * KT * nseg * 8);

  if (s->spec_dev_bytes < dev_bytes || s->spec_host_bytes < io_bytes) {
    PZ_HIP(s, hipStreamSynchronize(s->stream));
    if (s->spec_dev_bytes < dev_bytes) {
      (void)hipFree(s->spec_dev);
      s->spec_dev = nullptr;
      s->spec_dev_bytes = 0;
      if (hipMalloc(&s->spec_dev, dev_bytes) != hipSuccess)
        return fail(s, PZ_ENOMEM, "spec scratch of %zu bytes", dev_bytes);
      s->spec_dev_bytes = dev_bytes;
    }
    if (s->spec_host_bytes < io_bytes) {
      (void)hipHostFree(s->spec_host);
      s->spec_host = nullptr;
      s->spec_host_bytes = 0;
      if (hipHostMalloc(&s->spec_host, io_bytes, 0) != hipSuccess)
        return fail(s, PZ_ENOMEM, "spec staging of %zu bytes", io_bytes);
      s->spec_host_bytes = io_bytes;
    }
  }
  // earlier work on the stream may still read the staging area
  PZ_HIP(s, hipStreamSynchronize(s->stream));
  char* h = static_cast<char*>(s->spec_host);
  char* d = static_cast<char*>(s->spec_dev);
  pz_row_params_dev prm;
  memset(&prm, 0, sizeof(prm));
  float T = temperature;
  if (!(T >= 1e-6f)) T = 1e-6f;  // temperature.c:10
  prm.temp = T;
  prm.inv_temp = 1.0f / T;
  prm.temp_div = s->temp_mode == PZ_TEMP_DIV;
  prm.mode = PZ_MODE_CATEGORICAL;
  prm.rep_penalty = 1.0f;
  memcpy(h + o_prm, &prm, sizeof(prm));
  memcpy(h + o_ids, draft_ids, (size_t)B * K * 4);
  memcpy(h + o_uacc, u_acc, (size_t)B * K * 4);
  memcpy(h + o_ures, u_res, (size_t)B * 4);
  PZ_HIP(s, hipMemcpyAsync(d, h, in_bytes, hipMemcpyHostToDevice, s->stream));
  const bool vec = (ld % 4 == 0) && (((uintptr_t)d_target & 15) == 0) &&
                   (((uintptr_t)d_draft & 15) == 0);
  auto launch = vec ? launch_spec<true> : launch_spec<false>;
  const int rc = launch(s, d_target, d_draft, ld, V, B, K, KT, has_bonus ? 1 : 0,
                        reinterpret_cast<const pz_row_params_dev*>(d + o_prm),
                        reinterpret_cast<float*>(d + o_stats), reinterpret_cast<float*>(d + o_seg),
                        reinterpret_cast<const int32_t*>(d + o_ids),
                        reinterpret_cast<const float*>(d + o_uacc),
                        reinterpret_cast<const float*>(d + o_ures),
                        reinterpret_cast<int32_t*>(d + o_acc),
                        reinterpret_cast<int32_t*>(d + o_out));
  if (rc == -2) return fail(s, PZ_ENOTSUP, "V=%d needs more LDS than the device has", V);
  if (rc != 0) return fail(s, PZ_EDEVICE, "spec launch failed: %s",
                           hipGetErrorString(hipGetLastError()));
  PZ_HIP(s, hipMemcpyAsync(h + o_acc, d + o_acc, io_bytes - in_bytes, hipMemcpyDeviceToHost,
                           s->stream));
  PZ_HIP(s, hipStreamSynchronize(s->stream));
  memcpy(acc_len_out, h + o_acc, (size_t)B * 4);
  memcpy(ids_out, h + o_out, (size_t)B * (K + 1) * 4);
  return PZ_OK;
}
