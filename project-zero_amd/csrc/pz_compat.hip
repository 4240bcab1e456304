// pz_compat.hip -- the reference sampler's own C symbols
// (include/sampling/sampling.h:12-50, include/sampling/rng.h:14-21) and a
// tn_softmax-compatible function, served by the same HIP kernels as the
// batched API, so the objects of src/sampling can be replaced at link time.
//
// Each call takes the host row the reference takes, copies it to the
// device, runs a batch-1 launch and returns the id (or copies the row back
// for the in-place functions).  State lives in a per-thread context (one
// sampler, stream and row buffer per host thread), so unlike the reference's
// static top-p buffer (top_p.c:22-28) the calls are safe from several
// threads.  The reference has no error returns: a device failure makes the
// id calls return -1 (the value top_k.c already returns when no logit
// exceeds -1e30) and is reported by pz_compat_last_status().
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/pz_sampler.h"
#include "../../include/pz_sampling_compat.h"
#include "pz_launch.h"
#include "pz_sampler_impl.h"

namespace {

struct CompatCtx {
  pz_sampler* s = nullptr;
  int vmax = 0;
  float* d_row = nullptr;
  // the uniform in and the id out: coherent pinned host memory the kernels
  // use directly (z_*: the device's addresses of the same words)
  float* h_u = nullptr;
  int32_t* h_id = nullptr;
  const float* z_u = nullptr;
  int32_t* z_id = nullptr;
  int temp_mode = PZ_TEMP_MUL_RECIP;
  int status = PZ_OK;
  void release() {
    (void)hipFree(d_row);
    (void)hipHostFree(h_u);
    (void)hipHostFree(h_id);
    d_row = nullptr;
    h_u = nullptr;
    h_id = nullptr;
    pz_sampler_destroy(s);
    s = nullptr;
  }
  ~CompatCtx() {
    if (s) release();
  }
};

thread_local CompatCtx g_ctx;

int compat_device() {
  const char* e = getenv("PZ_COMPAT_DEVICE");
  return e ? atoi(e) : 0;
}

// Makes sure the context can take a row of V logits.
int ensure(int V) {
  CompatCtx& c = g_ctx;
  if (c.s && V <= c.vmax) return PZ_OK;
  int vmax = c.vmax > 0 ? c.vmax : 1;
  while (vmax < V) vmax *= 2;
  if (c.s) c.release();
  c.vmax = 0;
  int rc = pz_sampler_create(&c.s, 1, vmax, 0, compat_device());
  if (rc != PZ_OK) return rc;
  pz_sampler_set_temp_mode(c.s, c.temp_mode);
  const unsigned zc = hipHostMallocMapped | hipHostMallocCoherent;
  void *zu = nullptr, *zi = nullptr;
  if (hipMalloc((void**)&c.d_row, (size_t)vmax * sizeof(float)) != hipSuccess ||
      hipHostMalloc((void**)&c.h_u, sizeof(float), zc) != hipSuccess ||
      hipHostMalloc((void**)&c.h_id, sizeof(int32_t), zc) != hipSuccess)
    return PZ_ENOMEM;
  if (hipHostGetDevicePointer(&zu, c.h_u, 0) != hipSuccess ||
      hipHostGetDevicePointer(&zi, c.h_id, 0) != hipSuccess)
    return PZ_EDEVICE;
  c.z_u = static_cast<const float*>(zu);
  c.z_id = static_cast<int32_t*>(zi);
  c.vmax = vmax;
  return PZ_OK;
}

// One row through the kernel of `mode` (params already clamped like the
// reference), with uniform u.  Returns the id, -1 on failure.
int run_row(const float* logits, int V, int mode, float temperature, int top_k, float top_p,
            float u) {
  CompatCtx& c = g_ctx;
  c.status = ensure(V);
  if (c.status != PZ_OK) return -1;
  pz_sampler* s = c.s;
  *c.h_u = u;  // the previous call drained the stream
  if (hipMemcpyAsync(c.d_row, logits, (size_t)V * sizeof(float), hipMemcpyHostToDevice,
                     s->stream) != hipSuccess) {
    c.status = PZ_EDEVICE;
    return -1;
  }
  pz_row_params_dev& p = s->res_params[0];
  memset(&p, 0, sizeof(p));
  p.mode = mode;
  p.temp = temperature;
  p.inv_temp = 1.0f / temperature;
  p.temp_div = s->temp_mode == PZ_TEMP_DIV;
  p.top_k = top_k;
  p.top_p = top_p;
  p.rep_penalty = 1.0f;
  c.status = pz_dispatch_resolved(s, c.d_row, 1, V, V, 1, nullptr, 0, false, false, c.z_u,
                                  c.z_id, nullptr);
  // drained on every path: the next call rewrites h_u
  if (hipStreamSynchronize(s->stream) != hipSuccess && c.status == PZ_OK) c.status = PZ_EDEVICE;
  if (c.status == PZ_OK && *c.h_id == PZ_ID_FAILED) c.status = PZ_EDEVICE;
  return c.status == PZ_OK ? *c.h_id : -1;
}

// In-place row operation: copy in, op, copy back.
template <class Op>
void inplace_row(float* x, int V, Op op) {
  CompatCtx& c = g_ctx;
  if (V <= 0) return;
  c.status = ensure(V);
  if (c.status != PZ_OK) return;
  pz_sampler* s = c.s;
  if (hipMemcpyAsync(c.d_row, x, (size_t)V * sizeof(float), hipMemcpyHostToDevice, s->stream) !=
      hipSuccess) {
    c.status = PZ_EDEVICE;
    return;
  }
  c.status = op(s, c.d_row);
  if (c.status != PZ_OK) return;
  if (hipMemcpyAsync(x, c.d_row, (size_t)V * sizeof(float), hipMemcpyDeviceToHost, s->stream) !=
          hipSuccess ||
      hipStreamSynchronize(s->stream) != hipSuccess)
    c.status = PZ_EDEVICE;
}

}  // namespace

extern "C" {

// rng.c:3-6: seed 0 becomes 1.
void rng_seed(unsigned long long* state, unsigned long long seed) { *state = seed ? seed : 1ULL; }

// rng.c:8-17: xorshift64*, upper 31 bits of the product over 2^31 (the
// int -> float conversion rounds to nearest, so the result can be 1.0f).
float rng_float(unsigned long long* state) {
  unsigned long long x = *state;
  x ^= x >> 12;
  x ^= x << 25;
  x ^= x >> 27;
  *state = x;
  return (float)((x * 0x2545F4914F6CDD1DULL) >> 33) / 2147483648.0f;
}

// argmax.c:3-13: first maximum (strict '>').
int sample_argmax(const float* logits, int vocab_size) {
  if (vocab_size <= 0) return 0;
  return run_row(logits, vocab_size, PZ_MODE_GREEDY, 1.0f, 1, 1.0f, 0.0f);
}

// temperature.c:8-25, in place.
void apply_temperature(float* logits, int vocab_size, float temperature) {
  inplace_row(logits, vocab_size, [&](pz_sampler* s, float* d) {
    return pz_temperature_batch(s, d, vocab_size, 1, vocab_size, temperature);
  });
}

// top_p.c:30-108.  The vocabulary guard and the NaN-maximum case return
// argmax before the reference draws its uniform, so the state only
// advances when the reference's does.
int sample_top_p(float* logits, int vocab_size, float top_p, unsigned long long* rng_state) {
  if (vocab_size <= 0) return 0;
  if (vocab_size > PZ_TOPP_MAX_V || logits[0] != logits[0]) return sample_argmax(logits, vocab_size);
  const float u = rng_float(rng_state);
  return run_row(logits, vocab_size, PZ_MODE_TOPP, 1.0f, 1, top_p, u);
}

// top_k.c:8-73 (k clamped to [1, min(V, 1024)], :11-17).
int sample_top_k(float* logits, int vocab_size, int k, unsigned long long* rng_state) {
  if (vocab_size <= 0) return 0;
  if (k > vocab_size) k = vocab_size;
  if (k <= 0) k = 1;
  if (k > 1024) k = 1024;
  const float u = rng_float(rng_state);
  return run_row(logits, vocab_size, PZ_MODE_TOPK, 1.0f, k, 1.0f, u);
}

// softmax.c:4-23 in place, the signature of tn_softmax_fn.
void pz_tn_softmax(float* x, int size) {
  inplace_row(x, size, [&](pz_sampler* s, float* d) {
    return pz_softmax_batch(s, d, size, d, size, 1, size, 1.0f);
  });
}

void pz_compat_set_temp_mode(int mode) {
  if (mode != PZ_TEMP_MUL_RECIP && mode != PZ_TEMP_DIV) return;
  g_ctx.temp_mode = mode;
  if (g_ctx.s) pz_sampler_set_temp_mode(g_ctx.s, mode);
}

int pz_compat_last_status(void) { return g_ctx.status; }

}  // extern "C"
