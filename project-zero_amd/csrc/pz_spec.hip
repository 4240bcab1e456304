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
//   k_spec_rows_*  one workgroup per logits row (all target rows, then all
//                  draft rows): maximum, exact softmax normaliser, NaN/inf
//                  degeneracy.
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
  PzRecShared r;
};

template <bool VEC>
__device__ __forceinline__ void spec_rows_body(
    const float* __restrict__ target, const float* __restrict__ draft, long ld, int V, int B,
    int K, int KT, const pz_row_params_dev* __restrict__ prm, float* __restrict__ stats) {
  extern __shared__ __align__(16) char lds[];
  __shared__ SpecRowsShared S;
  __shared__ uint64_t etab[32];
  pz_etab_fill((pz_lds_u64*)etab);  // ordered by pz_pass1's barriers
  const int q = blockIdx.x, tid = threadIdx.x;
  const int NT = B * KT;
  PzTempRow<VEC> R;
  R.x = q < NT ? target + (long)q * ld : draft + (long)(q - NT) * ld;
  R.V = V;
  R.T = PzTemp::of(*prm);
  const int ntiles = pz_tiles(V);
  const PzRec REC = pz_rec_at(lds, ntiles * PZ_SEGS_PER_TILE);

  const float M = pz_pass1<8>(R, ntiles, S.p1);
  const bool bad = S.p1.any_nan || !(M > -__builtin_inff() && M < __builtin_inff());
  float inv = __builtin_nanf("");
  if (!bad) {
    PzExpTerms<PzTempRow<VEC>> X;
    X.R = R;
    X.M = M;
    X.thr = -__builtin_inff();
    X.inv = 1.0f;
    X.as_p = false;
    X.et = (const pz_lds_u64*)etab;
    inv = 1.0f / pz_exact_sum(X, ntiles, REC, S.r);
  }
  if (tid == 0) {
    stats[4 * (long)q] = M;
    stats[4 * (long)q + 1] = inv;
    stats[4 * (long)q + 2] = bad ? 1.0f : 0.0f;
  }
}

__global__ __launch_bounds__(PZ_RB) void k_spec_rows_v(
    const float* __restrict__ target, const float* __restrict__ draft, long ld, int V, int B,
    int K, int KT, const pz_row_params_dev* __restrict__ prm, float* __restrict__ stats) {
  spec_rows_body<true>(target, draft, ld, V, B, K, KT, prm, stats);
}
__global__ __launch_bounds__(PZ_RB) void k_spec_rows_s(
    const float* __restrict__ target, const float* __restrict__ draft, long ld, int V, int B,
    int K, int KT, const pz_row_params_dev* __restrict__ prm, float* __restrict__ stats) {
  spec_rows_body<false>(target, draft, ld, V, B, K, KT, prm, stats);
}

// p(x) of one element of a row whose softmax statistics are (M, inv).
template <bool VEC>
__device__ __forceinline__ float prob_at(const PzTempRow<VEC>& R, int x, float M, float inv,
                                        const pz_lds_u64* et) {
  return pz_expf_l(R.T.apply(R.x[x]) - M, et) * inv;
}

// Residual terms r(x) = max(0, p(x) - q(x)) of a target/draft row pair,
// evaluated exactly in prep; the observer tracks the last x with r(x) > 0.
template <bool VEC>
struct ResidualTerms {
  struct Raw {
    float t[4];
    float d[4];
  };
  PzTempRow<VEC> T, D;
  float MT, invT, MD, invD;
  int lastpos;
  const pz_lds_u64* et;  // the workgroup's LDS copy of the expf table
  __device__ __forceinline__ int load(int e0, Raw& r) const {
    T.load(e0, r.t);
    return D.load(e0, r.d);
  }
  __device__ __forceinline__ void residual(int e0, int n, Raw& r, float (&v)[4]) const {
    T.apply(e0, n, r.t);
    D.apply(e0, n, r.d);
#pragma unroll
    for (int c = 0; c < 4; c++) {
      float res = 0.0f;
      if (c < n) {
        const float p = pz_expf_tab(r.t[c] - MT, et) * invT;
        const float qq = pz_expf_tab(r.d[c] - MD, et) * invD;
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
  __device__ __forceinline__ uint32_t inc(const Raw&, const float (&a)[4], int c, uint32_t g,
                                          uint32_t* cls) const {
    return pz_inc(a[c], g, cls);
  }
  __device__ __forceinline__ void cache_put(pz_lds_f32* base, const Raw&,
                                            const float (&a)[4]) const {
    pz_f4 q;
    q.x = a[0];
    q.y = a[1];
    q.z = a[2];
    q.w = a[3];
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
    const int e0 = pz_seg_e0(k);
    const int n = load(e0, r);
    residual(e0, n, r, v);
  }
};

struct SpecVerifyShared {
  PzRecShared r;
  int jstar;
  int last;
  float Z;
  int hit;
};

template <bool VEC>
__global__ __launch_bounds__(PZ_RB) void k_spec_verify(
    const float* __restrict__ target, const float* __restrict__ draft, long ld, int V, int B,
    int K, int KT, int has_bonus, const pz_row_params_dev* __restrict__ prm,
    const float* __restrict__ stats, const int32_t* __restrict__ draft_ids,
    const float* __restrict__ u_acc, const float* __restrict__ u_res,
    int32_t* __restrict__ acc_len, int32_t* __restrict__ ids_out) {
  extern __shared__ __align__(16) char lds[];
  __shared__ SpecVerifyShared S;
  __shared__ uint64_t etab[32];
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  pz_etab_fill((pz_lds_u64*)etab);
  __syncthreads();
  const int b = blockIdx.x, tid = threadIdx.x;
  const int NT = B * KT;
  const int ntiles = pz_tiles(V), nseg = ntiles * PZ_SEGS_PER_TILE;
  const PzRec REC = pz_rec_at(lds, nseg);
  const PzTemp TT = PzTemp::of(*prm);

  // ---- acceptance tests, in draft order, up to the first rejection
  if (tid == 0) {
    int j = 0;
    for (; j < K; j++) {
      const int qt = b * KT + j, qd = NT + b * K + j;
      const int d = draft_ids[b * K + j];
      bool accept = false;
      if (d >= 0 && d < V) {
        PzTempRow<VEC> RT{target + (long)qt * ld, V, TT};
        PzTempRow<VEC> RD{draft + (long)(qd - NT) * ld, V, TT};
        const float pd = prob_at(RT, d, stats[4 * qt], stats[4 * qt + 1], et);
        const float qv = prob_at(RD, d, stats[4 * qd], stats[4 * qd + 1], et);
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
      ResidualTerms<VEC> X;
      X.T = PzTempRow<VEC>{target + (long)qt * ld, V, TT};
      X.D = PzTempRow<VEC>{draft + (long)(qd - NT) * ld, V, TT};
      X.MT = stats[4 * qt];
      X.invT = stats[4 * qt + 1];
      X.MD = stats[4 * qd];
      X.invD = stats[4 * qd + 1];
      X.lastpos = -1;
      X.et = et;
      pz_record_pass(X, ntiles, REC, S.r, __builtin_inff());
      if (X.lastpos > 0) atomicMax(&S.last, X.lastpos);
      if (tid < 64) {
        PzAcc st;
        st.n = 0;
        st.g = 1;
        pz_rec_walk(st, REC, nseg, 0.0f, PZ_STOP_NONE, X);
        const float Z = pz_acc_value(st);
        int hit = -1;
        if (Z > 0.0f) {
          // the same sequence of adds: the CDF of r, stop at ur * Z < cdf
          PzAcc s2;
          s2.n = 0;
          s2.g = 1;
          hit = pz_rec_walk(s2, REC, nseg, ur * Z, PZ_STOP_GT, X);
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
    PzExpTerms<PzTempRow<VEC>> X;
    X.R = PzTempRow<VEC>{target + (long)cat_row * ld, V, TT};
    X.M = stats[4 * cat_row];
    X.thr = -__builtin_inff();
    X.inv = stats[4 * cat_row + 1];
    X.as_p = true;
    X.et = et;
    const int hit = pz_exact_draw(X, V, ntiles, ur, REC, S.r);
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
                float* d_stats, const int32_t* d_ids_in, const float* d_uacc,
                const float* d_ures, int32_t* d_acc, int32_t* d_ids_out) {
  const size_t lds = pz_rec_bytes(V);
  if (lds + 256 > (size_t)s->max_lds) return -2;
  auto k1 = VEC ? k_spec_rows_v : k_spec_rows_s;
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
                     KT, d_prm, d_stats);
  hipLaunchKernelGGL(k2, dim3(B), dim3(PZ_RB), lds, s->stream, d_target, d_draft, ld, V, B, K, KT,
                     has_bonus, d_prm, d_stats, d_ids_in, d_uacc, d_ures, d_acc,
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
  const size_t dev_bytes = up256(o_stats + (size_t)NR * 16);

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
  if (T < 1e-6f) T = 1e-6f;  // temperature.c:10 (a NaN temperature stays NaN)
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
                        reinterpret_cast<float*>(d + o_stats),
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
