// pz_step.hip -- one decode step with the RNG and the EOS check on the
// device (pz_sample_step, pz_sampler_set_eos).
//
// The reference keeps one xorshift64* state per generation
// (src/transformer/generate.c:125-126), draws from it inside the sampler it
// dispatches to (generate.c:151-169), and after sampling compares the id
// with the model's EOS ids (generate.c:198-211).  Here the states are a
// device array, one per row, and a step is three launches on the sampler's
// stream: the draw (k_step_draw, one thread per row), the batched sampler
// reading the uniforms it wrote, and the EOS flags (k_step_eos).
#include <hip/hip_runtime.h>

#include <string.h>

#include "../../include/pz_sampler.h"
#include "pz_device.h"
#include "pz_launch.h"
#include "pz_params.h"
#include "pz_sampler_impl.h"

namespace {

// rng.c:8-17: xorshift64*; the product's upper 31 bits over 2^31.  The
// value is below 2^31, so converting it through uint32 (v_cvt_f32_u32,
// round to nearest even) equals the reference's 64-bit int -> float
// conversion; the division by 2^31 is exact.
__device__ __forceinline__ float step_rng_float(uint64_t& s) {
  s ^= s >> 12;
  s ^= s << 25;
  s ^= s >> 27;
  const uint32_t hi = (uint32_t)((s * 0x2545F4914F6CDD1DULL) >> 33);
  return (float)hi / 2147483648.0f;
}

// The value the chain sees for id 0 of row b (penalties as the kernels
// apply them, then temperature): top_p.c starts its maximum at the row's
// first element, so a NaN there leaves no candidate and the row returns
// argmax without drawing (top_p.c:37-41, 53-58, 68-69).
__device__ float step_first_value(const float* row, const int32_t* hist_row, int H,
                                  const pz_row_params_dev& p) {
  float x = row[0];
  const bool active = hist_row != nullptr && H > 0 &&
                      (p.rep_penalty != 1.0f || p.presence_penalty != 0.0f ||
                       p.frequency_penalty != 0.0f);
  if (active) {
    int c = 0;
    for (int j = 0; j < H; j++) c += hist_row[j] == 0;
    if (c > 0) {
      x = x > 0.0f ? x / p.rep_penalty : x * p.rep_penalty;
      if (p.presence_penalty != 0.0f || p.frequency_penalty != 0.0f) {
        float t = (float)c * p.frequency_penalty;
        t = t + p.presence_penalty;
        x = x - t;
      }
    }
  }
  return p.temp_div ? x / p.temp : x * p.inv_temp;
}

// One thread per row: draws the row's uniform exactly when the reference
// would -- never for greedy rows (generate.c:151-152), never for top-p rows
// that take argmax first (vocabulary above 200000, top_p.c:33-34, or a NaN
// first value), once for every other row (top_k.c:62, top_p.c:96,
// generate.c:159) -- and advances its state only then.
__global__ void k_step_draw(const float* logits, long ld, int V, int B,
                            const pz_row_params_dev* params, int n_params, const int32_t* hist,
                            int H, uint64_t* state, float* u) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const pz_row_params_dev p = params[n_params == 1 ? 0 : b];
  bool draws = p.mode != PZ_MODE_GREEDY;
  if (draws && p.mode == PZ_MODE_TOPP) {
    if (V > PZ_TOPP_MAX_V) {
      draws = false;
    } else {
      const float y0 = step_first_value(logits + (size_t)b * ld,
                                        hist ? hist + (size_t)b * H : nullptr, H, p);
      draws = !(y0 != y0);
    }
  }
  float r = 0.0f;
  if (draws) {
    uint64_t s = state[b];
    r = step_rng_float(s);
    state[b] = s;
  }
  u[b] = r;
}

// generate.c:198-211: the row's id against the EOS list.
__global__ void k_step_eos(const int32_t* ids, int B, const int32_t* eos, int n_eos,
                           uint8_t* flags) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int32_t id = ids[b];
  uint8_t f = 0;
  for (int e = 0; e < n_eos; e++) f |= (uint8_t)(eos[e] == id);
  flags[b] = f;
}

}  // namespace

int pz_launch_step_draw(const pz_launch& L, int B, uint64_t* d_state, float* d_u) {
  const int block = 256;
  hipLaunchKernelGGL(k_step_draw, dim3((B + block - 1) / block), dim3(block), 0, L.stream,
                     L.logits, L.ld, L.V, B, L.params, L.n_params, L.hist, L.H, d_state, d_u);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int pz_launch_step_eos(hipStream_t st, const int32_t* d_ids, int B, const int32_t* d_eos,
                       int n_eos, uint8_t* d_flags) {
  const int block = 256;
  hipLaunchKernelGGL(k_step_eos, dim3((B + block - 1) / block), dim3(block), 0, st, d_ids, B,
                     d_eos, n_eos, d_flags);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int pz_sampler_set_eos(pz_sampler* s, const int32_t* eos_ids, int n_eos) {
  if (!s) return PZ_EINVAL;
  if (n_eos < 0 || (n_eos > 0 && !eos_ids)) return fail(s, PZ_EINVAL, "bad EOS list");
  if (n_eos > PZ_MAX_EOS) return fail(s, PZ_ERANGE, "n_eos=%d > %d", n_eos, PZ_MAX_EOS);
  PZ_HIP(s, hipSetDevice(s->device));
  // the stream may still run a step that reads the old list
  PZ_HIP(s, hipStreamSynchronize(s->stream));
  if (n_eos > 0)
    PZ_HIP(s, hipMemcpy(s->d_eos, eos_ids, (size_t)n_eos * sizeof(int32_t),
                        hipMemcpyHostToDevice));
  if (n_eos > 0) memcpy(s->h_eos, eos_ids, (size_t)n_eos * sizeof(int32_t));
  s->n_eos = n_eos;
  return PZ_OK;
}

extern "C" int pz_sample_step(pz_sampler* s, const float* d_logits, int B, int V, long ld,
                              const pz_row_params* params, int n_params, const int32_t* d_hist,
                              int H, uint64_t* d_state, int32_t* d_ids_out, float* d_p_out,
                              uint8_t* d_eos_out) {
  if (!s) return PZ_EINVAL;
  if (!d_state) return fail(s, PZ_EINVAL, "null RNG states");
  PZ_HIP(s, hipSetDevice(s->device));
  PzStepHooks hooks;
  hooks.state = d_state;
  hooks.eos_out = d_eos_out;
  return pz_dispatch_params(s, d_logits, B, V, ld, params, n_params, d_hist, H, nullptr,
                            d_ids_out, d_p_out, &hooks);
}
