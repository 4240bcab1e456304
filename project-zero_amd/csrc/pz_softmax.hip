// pz_softmax.hip -- batched apply_temperature and softmax on device rows,
// bit-exact with the reference.
//
//   apply_temperature (src/sampling/temperature.c:8-25): T < 1e-6 -> 1e-6,
//     x *= 1/T (AVX-512 build) or x /= T (scalar build), in place.
//   softmax (src/math/softmax.c:4-23, the tn_softmax slot of
//     include/math/simd_dispatch.h:23,47): max by strict '>', e = expf(x -
//     max) with a sequential fp32 sum in ascending order, x *= 1/sum.  Any
//     NaN, or an infinite maximum, makes the sum NaN and every output NaN.
// The softmax runs one 1024-thread workgroup per row: pass 1 (max), the
// exact-sum records and walk (pz_rowpass.h), then one write pass.  Rows may
// have their own lengths (attention scores, pz_attn.hip).
#include "pz_device.h"
#include "pz_exact.h"
#include "pz_launch.h"
#include "pz_rowpass.h"
#include "pz_sampler_impl.h"

namespace {

__global__ void k_temperature(float* __restrict__ x, long ld, int V, int B, PzTemp T) {
  const long n = (long)B * V;
  for (long i = blockIdx.x * (long)blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x) {
    const long r = i / V, c = i - r * V;
    float* p = x + r * ld + c;
    *p = T.apply(*p);
  }
}

struct SoftmaxShared {
  PzPass1Shared p1;
  PzRecShared r;
};

template <bool VEC>
__global__ __launch_bounds__(PZ_RB) void k_softmax(const float* in, long ld_in, float* out,
                                                   long ld_out, int Vmax, PzTemp T,
                                                   const int32_t* lens) {
  extern __shared__ __align__(16) char lds[];
  __shared__ SoftmaxShared S;
  __shared__ uint64_t etab[32];
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  pz_etab_fill((pz_lds_u64*)etab);  // ordered by pz_pass1's barriers
  const int row = blockIdx.x, tid = threadIdx.x;
  // the row's length: every thread reads the same value, so the early return
  // below is uniform over the workgroup
  const int V = lens ? (lens[row] < Vmax ? lens[row] : Vmax) : Vmax;
  if (V <= 0) return;
  PzTempRow<VEC> R;
  R.x = in + (long)row * ld_in;
  R.V = V;
  R.T = T;
  const int ntiles = pz_tiles(V);
  const PzRec REC = pz_rec_at(lds, ntiles * PZ_SEGS_PER_TILE);
  float* o = out + (long)row * ld_out;

  const float M = pz_pass1<8>(R, ntiles, S.p1);
  if (S.p1.any_nan || !(M > -__builtin_inff() && M < __builtin_inff())) {
    for (int i = tid; i < V; i += PZ_RB) o[i] = __builtin_nanf("");
    return;
  }
  PzExpTerms<PzTempRow<VEC>> X;
  X.R = R;
  X.M = M;
  X.thr = -__builtin_inff();
  X.inv = 1.0f;
  X.as_p = false;
  X.et = et;
  const float inv = 1.0f / pz_exact_sum(X, ntiles, REC, S.r);
  // every read of the row is done: the write pass may overwrite it (in == out)
  for (int t = 0; t < ntiles; t++) {
    float y[4];
    const int e0 = pz_tile_e0(t);
    const int n = R.get(e0, y);
#pragma unroll
    for (int c = 0; c < 4; c++)
      if (c < n) o[e0 + c] = pz_expf_tab(y[c] - M, et) * inv;
  }
}

PzTemp temp_of(pz_sampler* s, float temperature) {
  float T = temperature;
  if (T < 1e-6f) T = 1e-6f;  // temperature.c:10 (a NaN temperature stays NaN)
  PzTemp t;
  t.t = T;
  t.inv = 1.0f / T;
  t.div = s->temp_mode == PZ_TEMP_DIV;
  return t;
}

}  // namespace

int pz_launch_softmax_rows(pz_sampler* s, const float* d_in, long ld_in, float* d_out,
                           long ld_out, int B, int V, PzTemp T, const int32_t* d_len) {
  const size_t lds = pz_rec_bytes(V);
  if (lds + sizeof(SoftmaxShared) + 64 > (size_t)s->max_lds)
    return fail(s, PZ_ENOTSUP, "V=%d needs more LDS than the device has", V);
  const bool vec = (ld_in % 4 == 0) && (((uintptr_t)d_in & 15) == 0);
  auto kern = vec ? k_softmax<true> : k_softmax<false>;
  if (lds > 65536)
    PZ_HIP(s, hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)lds));
  hipLaunchKernelGGL(kern, dim3(B), dim3(PZ_RB), lds, s->stream, d_in, ld_in, d_out, ld_out, V,
                     T, d_len);
  PZ_HIP(s, hipGetLastError());
  return PZ_OK;
}

extern "C" int pz_temperature_batch(pz_sampler* s, float* d_x, long ld, int B, int V,
                                    float temperature) {
  if (!s) return PZ_EINVAL;
  if (!d_x || B < 0 || V < 0 || ld < V) return fail(s, PZ_EINVAL, "bad temperature shape");
  if ((long)B * V == 0) return PZ_OK;
  PZ_HIP(s, hipSetDevice(s->device));
  const long n = (long)B * V;
  const int blocks = (int)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
  hipLaunchKernelGGL(k_temperature, dim3(blocks), dim3(256), 0, s->stream, d_x, ld, V, B,
                     temp_of(s, temperature));
  PZ_HIP(s, hipGetLastError());
  return PZ_OK;
}

extern "C" int pz_softmax_batch(pz_sampler* s, const float* d_in, long ld_in, float* d_out,
                                long ld_out, int B, int V, float temperature) {
  if (!s) return PZ_EINVAL;
  if (!d_in || !d_out || B < 0 || V <= 0 || ld_in < V || ld_out < V)
    return fail(s, PZ_EINVAL, "bad softmax shape");
  if (B == 0) return PZ_OK;
  PZ_HIP(s, hipSetDevice(s->device));
  return pz_launch_softmax_rows(s, d_in, ld_in, d_out, ld_out, B, V, temp_of(s, temperature),
                                nullptr);
}
