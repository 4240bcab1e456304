// pz_sampler.hip -- host side of the C ABI (include/pz_sampler.h).
//
// Replaces the per-step hand-off of src/transformer/generate.c:143-174: the
// engine keeps [B, V] logits in HBM and this dispatcher resolves each row's
// sampling mode once (generate.c:151-169 order), groups rows by mode, and
// launches one batched kernel per group on the sampler's stream.  Only ids
// (and p(chosen)) travel back.
#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <chrono>
#include <new>

#include "../../include/pz_sampler.h"
#include "pz_launch.h"
#include "pz_params.h"
#include "pz_sampler_impl.h"

namespace {

constexpr int kTopKMax = 1024;  // top_k.c:6
constexpr int kMaxHist = 2048;
// An id no kernel writes (ids are -1 .. V-1): marks rows still pending.
constexpr int32_t kIdPending = INT32_MIN;

int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

}  // namespace


size_t pz_scratch_layout(int max_batch, int max_vocab, int max_slots, void* base,
                         pz_scratch* out) {
  auto up = [](size_t v) { return (v + 255) & ~(size_t)255; };
  int vt = max_vocab < PZ_TOPP_MAX_V ? max_vocab : PZ_TOPP_MAX_V;
  int slot = 256;  // a power of two >= every candidate list (one segment at least)
  while (slot < vt) slot <<= 1;
  const size_t B = (size_t)max_batch;
  // the fallback sorts at most one queued row per slot at a time: a sampler
  // for max_batch rows never needs more than max_batch slots
  const size_t slots = (size_t)(max_batch < max_slots ? max_batch : max_slots);
  size_t off = 0;
  const size_t o_stat = off; off = up(off + B * 4 * sizeof(float));
  const size_t o_list = off; off = up(off + B * sizeof(int32_t));
  const size_t o_cnt = off;  off = up(off + PZ_COUNTERS * sizeof(int32_t));
  const size_t o_keys = off; off = up(off + slots * slot * sizeof(uint64_t));
  const size_t o_keys2 = off; off = up(off + slots * slot * sizeof(uint64_t));
  if (base && out) {
    char* b = static_cast<char*>(base);
    out->row_stat = reinterpret_cast<float*>(b + o_stat);
    out->fb_list = reinterpret_cast<int32_t*>(b + o_list);
    out->counters = reinterpret_cast<int32_t*>(b + o_cnt);
    out->fb_keys = reinterpret_cast<uint64_t*>(b + o_keys);
    out->fb_keys2 = reinterpret_cast<uint64_t*>(b + o_keys2);
    out->slot_n = slot;
    out->fb_slots = (int)slots;
  }
  return off;
}

extern "C" int pz_sampler_create(pz_sampler** out, int max_batch, int max_vocab,
                                 int max_hist, int device) {
  if (!out || max_batch <= 0 || max_vocab <= 0 || max_hist < 0) return PZ_EINVAL;
  if (max_hist > kMaxHist) return PZ_ERANGE;
  *out = nullptr;
  pz_sampler* s = new (std::nothrow) pz_sampler();
  if (!s) return PZ_ENOMEM;
  s->device = device;
  s->max_batch = max_batch;
  s->max_vocab = max_vocab;
  s->max_hist = max_hist;
  int rc = PZ_OK;
  auto bail = [&](int code) {
    pz_sampler_destroy(s);
    return code;
  };
  if (hipSetDevice(device) != hipSuccess) return bail(PZ_EDEVICE);
  if (hipDeviceGetAttribute(&s->max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock,
                            device) != hipSuccess ||
      hipDeviceGetAttribute(&s->n_cu, hipDeviceAttributeMultiprocessorCount, device) !=
          hipSuccess)
    return bail(PZ_EDEVICE);
  if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess)
    return bail(PZ_EDEVICE);
  if (hipEventCreateWithFlags(&s->staged, hipEventDisableTiming) != hipSuccess)
    return bail(PZ_EDEVICE);
  const size_t B = (size_t)max_batch;
  const unsigned zc = hipHostMallocMapped | hipHostMallocCoherent;
  if (hipHostMalloc((void**)&s->h_params, B * sizeof(pz_row_params_dev), 0) != hipSuccess ||
      hipHostMalloc((void**)&s->h_rows, B * sizeof(int32_t), 0) != hipSuccess ||
      hipHostMalloc((void**)&s->h_u, B * sizeof(float), zc) != hipSuccess ||
      hipHostMalloc((void**)&s->h_ids, B * sizeof(int32_t), zc) != hipSuccess ||
      hipHostMalloc((void**)&s->h_p, B * sizeof(float), zc) != hipSuccess)
    return bail(PZ_ENOMEM);
  void *zu = nullptr, *zi = nullptr, *zp = nullptr;
  if (hipHostGetDevicePointer(&zu, s->h_u, 0) != hipSuccess ||
      hipHostGetDevicePointer(&zi, s->h_ids, 0) != hipSuccess ||
      hipHostGetDevicePointer(&zp, s->h_p, 0) != hipSuccess)
    return bail(PZ_EDEVICE);
  s->z_u = static_cast<const float*>(zu);
  s->z_ids = static_cast<int32_t*>(zi);
  s->z_p = static_cast<float*>(zp);
  if (hipMalloc((void**)&s->d_params, B * sizeof(pz_row_params_dev)) != hipSuccess ||
      hipMalloc((void**)&s->d_rows, B * sizeof(int32_t)) != hipSuccess ||
      hipMalloc((void**)&s->d_u_step, B * sizeof(float)) != hipSuccess ||
      hipMalloc((void**)&s->d_eos, PZ_MAX_EOS * sizeof(int32_t)) != hipSuccess ||
      hipMalloc((void**)&s->d_lmh_keys, 16 * B * sizeof(unsigned long long)) != hipSuccess ||
      hipMalloc((void**)&s->d_lmh_nan, B) != hipSuccess)
    return bail(PZ_ENOMEM);
  // the fused LM head's argmax keys: 16 slots per row (zero between calls)
  if (hipMemset(s->d_lmh_keys, 0, 16 * B * sizeof(unsigned long long)) != hipSuccess)
    return bail(PZ_EDEVICE);
  s->res_params = new (std::nothrow) pz_row_params_dev[B];
  if (!s->res_params) return bail(PZ_ENOMEM);
  s->scratch_bytes = pz_scratch_layout(max_batch, max_vocab, PZ_FB_SLOTS, nullptr, nullptr);
  if (hipMalloc(&s->d_scratch, s->scratch_bytes) != hipSuccess) return bail(PZ_ENOMEM);
  pz_scratch_layout(max_batch, max_vocab, PZ_FB_SLOTS, s->d_scratch, &s->sc);
  // queue counters start at zero; the fallback kernel re-zeroes them after
  // each launch that read them
  if (hipMemset(s->sc.counters, 0, PZ_COUNTERS * sizeof(int32_t)) != hipSuccess)
    return bail(PZ_EDEVICE);
  s->split_bytes =
      pz_split_ws_layout(max_batch, max_vocab, PZ_TOPP_CAPG, nullptr, nullptr, true);
  if (hipMalloc(&s->d_split, s->split_bytes) != hipSuccess) return bail(PZ_ENOMEM);
  pz_split_ws_layout(max_batch, max_vocab, PZ_TOPP_CAPG, s->d_split, &s->ws, true);
  // arrival counters start at zero; every pass's last workgroup re-zeroes
  // its row's
  if (hipMemset(s->d_split, 0, s->split_bytes) != hipSuccess) return bail(PZ_EDEVICE);
  *out = s;
  return rc;
}

extern "C" void pz_sampler_destroy(pz_sampler* s) {
  if (!s) return;
  // Teardown: errors here have no caller to report to.
  if (s->stream) (void)hipStreamSynchronize(s->stream);
  (void)hipFree(s->d_params);
  (void)hipFree(s->d_rows);
  (void)hipFree(s->d_u_step);
  (void)hipFree(s->d_eos);
  (void)hipFree(s->d_lmh_keys);
  (void)hipFree(s->d_lmh_nan);
  (void)hipFree(s->d_scratch);
  (void)hipFree(s->d_split);
  (void)hipFree(s->spec_dev);
  (void)hipFree(s->attn_dev);
  (void)hipHostFree(s->spec_host);
  (void)hipHostFree(s->h_params);
  (void)hipHostFree(s->h_rows);
  (void)hipHostFree(s->h_u);
  (void)hipHostFree(s->h_ids);
  (void)hipHostFree(s->h_p);
  if (s->staged) (void)hipEventDestroy(s->staged);
  if (s->stream) (void)hipStreamDestroy(s->stream);
  delete[] s->res_params;
  delete s;
}

extern "C" int pz_sampler_set_temp_mode(pz_sampler* s, int mode) {
  if (!s || (mode != PZ_TEMP_MUL_RECIP && mode != PZ_TEMP_DIV)) return PZ_EINVAL;
  s->temp_mode = mode;
  return PZ_OK;
}

extern "C" int pz_sampler_set_wait_bound(pz_sampler* s, uint32_t polls) {
  if (!s) return PZ_EINVAL;
  s->wait_polls = polls ? polls : PZ_POLL_CAP;
  return PZ_OK;
}

extern "C" const char* pz_sampler_last_error(const pz_sampler* s) {
  return s ? s->err : "null sampler";
}

extern "C" void* pz_sampler_stream(pz_sampler* s) { return s ? (void*)s->stream : nullptr; }

extern "C" int pz_sampler_sync(pz_sampler* s) {
  if (!s) return PZ_EINVAL;
  PZ_HIP(s, hipStreamSynchronize(s->stream));
  return PZ_OK;
}

// Resolves one row's host parameters into the kernel form (mode decided as
// generate.c:151-169; clamps of temperature.c:10 and top_k.c:11-17).
pz_row_params_dev pz_resolve_row(const pz_row_params& p, int V, int temp_mode) {
  pz_row_params_dev d;
  memset(&d, 0, sizeof(d));
  d.rep_penalty = p.rep_penalty;
  d.presence_penalty = p.presence_penalty;
  d.frequency_penalty = p.frequency_penalty;
  d.top_p = p.top_p;
  float T = p.temperature;
  if (T <= 0.0f || T < 1e-6f) {
    d.mode = PZ_MODE_GREEDY;
    T = 1.0f;
  } else if (p.top_k > 0) {
    d.mode = PZ_MODE_TOPK;
  } else if (p.top_p < 1.0f && p.top_p > 0.0f) {
    d.mode = PZ_MODE_TOPP;
  } else {
    d.mode = PZ_MODE_CATEGORICAL;
  }
  if (T < 1e-6f) T = 1e-6f;
  d.temp = T;
  d.inv_temp = 1.0f / T;
  d.temp_div = temp_mode == PZ_TEMP_DIV;
  int k = p.top_k;
  if (k > V) k = V;
  if (k <= 0) k = 1;
  if (k > kTopKMax) k = kTopKMax;
  d.top_k = k;
  return d;
}

bool pz_penalty_active(const pz_row_params& p) {
  return p.rep_penalty != 1.0f || p.presence_penalty != 0.0f || p.frequency_penalty != 0.0f;
}

bool pz_needs_counts(const pz_row_params& p) {
  return p.presence_penalty != 0.0f || p.frequency_penalty != 0.0f;
}

int pz_hash_capacity(bool counts_any, int H) {
  return counts_any ? next_pow2(2 * (H > 0 ? H : 1)) : 0;
}

void pz_group_rows(const pz_row_params_dev* res, int B, int n_params, int count[PZ_MODE_COUNT],
                   int offset[PZ_MODE_COUNT], int* modes_present) {
  for (int m = 0; m < PZ_MODE_COUNT; m++) count[m] = 0;
  for (int b = 0; b < B; b++) count[res[n_params == 1 ? 0 : b].mode]++;
  int acc = 0, present = 0;
  for (int m = 0; m < PZ_MODE_COUNT; m++) {
    offset[m] = acc;
    acc += count[m];
    present += count[m] > 0;
  }
  *modes_present = present;
}

int pz_max_top_k(const pz_row_params_dev* res, int B, int n_params) {
  int kmax = 0;
  for (int b = 0; b < (n_params == 1 ? 1 : B); b++)
    if (res[b].mode == PZ_MODE_TOPK && res[b].top_k > kmax) kmax = res[b].top_k;
  return kmax;
}

void pz_fill_rows(const pz_row_params_dev* res, int B, int n_params,
                  const int offset[PZ_MODE_COUNT], int32_t* rows) {
  int fill[PZ_MODE_COUNT];
  memcpy(fill, offset, sizeof(fill));
  for (int b = 0; b < B; b++) rows[fill[res[n_params == 1 ? 0 : b].mode]++] = b;
}

typedef int (*pz_launcher)(const pz_launch&, int, const int32_t*);

int pz_launch_modes(const pz_launch& L, const int count[PZ_MODE_COUNT],
                    const int offset[PZ_MODE_COUNT], int modes_present, const int32_t* d_rows,
                    int* failed_mode) {
  static const pz_launcher launchers[PZ_MODE_COUNT] = {
      pz_launch_greedy, pz_launch_categorical, pz_launch_topk, pz_launch_topp};
  for (int m = 0; m < PZ_MODE_COUNT; m++) {
    if (!count[m]) continue;
    const int32_t* rows = modes_present > 1 ? d_rows + offset[m] : nullptr;
    const int rc = launchers[m](L, count[m], rows);
    if (rc != 0) {
      *failed_mode = m;
      return rc;
    }
  }
  return 0;
}

// Common body of the sync, async and step entry points.  Stages params (and,
// when the batch mixes modes, a mode-grouped row list) through pinned memory
// and launches one kernel per mode present.
int pz_dispatch_params(pz_sampler* s, const float* d_logits, int B, int V, long ld,
                       const pz_row_params* params, int n_params, const int32_t* d_hist,
                       int H, const float* d_u, int32_t* d_ids, float* d_p,
                       const PzStepHooks* hooks) {
  if (!s) return PZ_EINVAL;
  if (!d_logits || !params || B < 0 || V <= 0 || ld < V) return fail(s, PZ_EINVAL, "bad logits/shape");
  if (n_params != 1 && n_params != B) return fail(s, PZ_EINVAL, "n_params must be 1 or B");
  if (B > s->max_batch) return fail(s, PZ_ERANGE, "B=%d > max_batch=%d", B, s->max_batch);
  if (V > s->max_vocab) return fail(s, PZ_ERANGE, "V=%d > max_vocab=%d", V, s->max_vocab);
  if (H < 0 || H > s->max_hist) return fail(s, PZ_ERANGE, "H=%d > max_hist=%d", H, s->max_hist);
  if (H > 0 && !d_hist) return fail(s, PZ_EINVAL, "H>0 needs d_hist");
  if (!d_ids) return fail(s, PZ_EINVAL, "null ids");
  if (B == 0) return PZ_OK;

  bool pen_any = false, counts_any = false;
  pz_row_params_dev* res = s->res_params;
  for (int i = 0; i < n_params; i++) {
    res[i] = pz_resolve_row(params[i], V, s->temp_mode);
    if (H > 0 && pz_penalty_active(params[i])) {
      pen_any = true;
      counts_any |= pz_needs_counts(params[i]);
    }
  }
  return pz_dispatch_resolved(s, d_logits, B, V, ld, n_params, d_hist, H, pen_any, counts_any,
                              d_u, d_ids, d_p, hooks);
}

int pz_dispatch_resolved(pz_sampler* s, const float* d_logits, int B, int V, long ld,
                         int n_params, const int32_t* d_hist, int H, bool pen_any,
                         bool counts_any, const float* d_u, int32_t* d_ids, float* d_p,
                         const PzStepHooks* hooks) {
  int count[PZ_MODE_COUNT], offset[PZ_MODE_COUNT], modes_present = 0;
  pz_row_params_dev* res = s->res_params;
  pz_group_rows(res, B, n_params, count, offset, &modes_present);
  if (hooks) d_u = s->d_u_step;  // written by the step's draw kernel
  if (!d_u) {
    for (int b = 0; b < B; b++)
      if (res[n_params == 1 ? 0 : b].mode != PZ_MODE_GREEDY)
        return fail(s, PZ_EINVAL, "sampling rows need uniforms");
  }
  // Parameters (and the row grouping they imply) usually repeat from step to
  // step: upload only when they changed, so back-to-back calls queue their
  // kernels without a host wait.
  const bool same = s->staged_n == n_params && s->staged_B == B &&
                    memcmp(s->h_params, res, (size_t)n_params * sizeof(pz_row_params_dev)) == 0;
  if (!same) {
    // The previous staging copy must have left pinned memory first.
    PZ_HIP(s, hipEventSynchronize(s->staged));
    memcpy(s->h_params, res, (size_t)n_params * sizeof(pz_row_params_dev));
    if (modes_present > 1) {
      pz_fill_rows(res, B, n_params, offset, s->h_rows);
      PZ_HIP(s, hipMemcpyAsync(s->d_rows, s->h_rows, (size_t)B * sizeof(int32_t),
                               hipMemcpyHostToDevice, s->stream));
    }
    PZ_HIP(s, hipMemcpyAsync(s->d_params, s->h_params,
                             (size_t)n_params * sizeof(pz_row_params_dev),
                             hipMemcpyHostToDevice, s->stream));
    PZ_HIP(s, hipEventRecord(s->staged, s->stream));
    s->staged_n = n_params;
    s->staged_B = B;
  }

  pz_launch L;
  L.logits = d_logits;
  L.ld = ld;
  L.V = V;
  L.params = s->d_params;
  L.n_params = n_params;
  L.hist = H > 0 ? d_hist : nullptr;
  L.H = H;
  L.pen_any = pen_any;
  L.temp_div = s->temp_mode == PZ_TEMP_DIV;
  L.hcap = pz_hash_capacity(counts_any, H);
  L.u = d_u;
  L.h_u = hooks ? nullptr : s->call_u;
  L.B = B;
  L.ids = d_ids;
  L.p_out = d_p;
  L.sc = s->sc;
  L.ws = s->ws;
  L.kmax = pz_max_top_k(res, B, n_params);
  L.max_lds = s->max_lds;
  L.wait_polls = s->wait_polls;
  L.n_cu = s->n_cu;
  L.stream = s->stream;

  if (hooks && pz_launch_step_draw(L, B, hooks->state, s->d_u_step) != 0)
    return fail(s, PZ_EDEVICE, "launch of the step draw failed");
  int m = -1;
  const int rc = pz_launch_modes(L, count, offset, modes_present, s->d_rows, &m);
  if (rc == -2) return fail(s, PZ_ENOTSUP, "sampling mode %d not supported for V=%d", m, V);
  if (rc != 0) return fail(s, PZ_EDEVICE, "launch of mode %d failed: %s", m,
                           hipGetErrorString(hipGetLastError()));
  if (hooks && hooks->eos_out &&
      pz_launch_step_eos(s->stream, d_ids, B, s->d_eos, s->n_eos, hooks->eos_out) != 0)
    return fail(s, PZ_EDEVICE, "launch of the EOS check failed");
  return PZ_OK;
}

extern "C" int pz_sample_batch_async(pz_sampler* s, const float* d_logits, int B, int V,
                                     long ld, const pz_row_params* params, int n_params,
                                     const int32_t* d_hist, int H, const float* d_u,
                                     int32_t* d_ids_out, float* d_p_out) {
  if (!s) return PZ_EINVAL;
  PZ_HIP(s, hipSetDevice(s->device));
  return pz_dispatch_params(s, d_logits, B, V, ld, params, n_params, d_hist, H, d_u, d_ids_out,
                            d_p_out, nullptr);
}

// Waits until the kernels have written all B ids into the coherent pinned
// buffer (true), or gives up after two seconds (false).  Every sampling
// kernel writes each row's id exactly once, after its last read of the row's
// inputs (the uniform included), so once every id is back the call's host
// buffers are free again, and later launches queue behind this call's in
// stream order.  Watching the ids return is several microseconds quicker
// than a stream synchronisation.
static bool wait_ids(pz_sampler* s, int B) {
  volatile const int32_t* h = s->h_ids;
  const auto t0 = std::chrono::steady_clock::now();
  for (int b = 0; b < B; b++) {
    unsigned spins = 0;
    while (h[b] == kIdPending)
      if ((++spins & 0xffffu) == 0 &&
          std::chrono::steady_clock::now() - t0 > std::chrono::seconds(2))
        return false;
  }
  return true;
}

extern "C" int pz_sample_batch(pz_sampler* s, const float* d_logits, int B, int V, long ld,
                               const pz_row_params* params, int n_params,
                               const int32_t* d_hist, int H, const float* u,
                               int32_t* ids_out, float* p_out) {
  if (!s) return PZ_EINVAL;
  if (!ids_out) return fail(s, PZ_EINVAL, "null ids_out");
  if (B > s->max_batch) return fail(s, PZ_ERANGE, "B=%d > max_batch=%d", B, s->max_batch);
  if (B <= 0) return B == 0 ? PZ_OK : fail(s, PZ_EINVAL, "B<0");
  PZ_HIP(s, hipSetDevice(s->device));
  // A synchronous call returns once its kernels have read h_u and written
  // h_ids (see wait_ids), and asynchronous calls never touch h_u / h_ids /
  // h_p: the buffers are free here.
  const float* d_u = nullptr;
  if (u) {
    memcpy(s->h_u, u, (size_t)B * sizeof(float));
    d_u = s->z_u;
  }
  for (int b = 0; b < B; b++) s->h_ids[b] = kIdPending;
  s->call_u = u ? s->h_u : nullptr;
  int rc = pz_dispatch_params(s, d_logits, B, V, ld, params, n_params, d_hist, H, d_u,
                              s->z_ids, p_out ? s->z_p : nullptr, nullptr);
  s->call_u = nullptr;
  if (rc != PZ_OK) {
    (void)hipStreamSynchronize(s->stream);  // kernels already queued may use the buffers
    return rc;
  }
  // p(chosen) is written after the id: with it requested, wait for the stream
  if (p_out || !wait_ids(s, B)) {
    PZ_HIP(s, hipStreamSynchronize(s->stream));
    for (int b = 0; b < B; b++)
      if (s->h_ids[b] == kIdPending) return fail(s, PZ_EDEVICE, "row %d returned no id", b);
  }
  memcpy(ids_out, s->h_ids, (size_t)B * sizeof(int32_t));
  if (p_out) memcpy(p_out, s->h_p, (size_t)B * sizeof(float));
  for (int b = 0; b < B; b++)
    if (ids_out[b] == PZ_ID_FAILED)
      return fail(s, PZ_EDEVICE, "row %d: a wait between the row's workgroups gave up", b);
  return PZ_OK;
}

extern "C" int pz_device_alloc(void** ptr, size_t bytes, int device) {
  if (!ptr) return PZ_EINVAL;
  if (hipSetDevice(device) != hipSuccess) return PZ_EDEVICE;
  return hipMalloc(ptr, bytes) == hipSuccess ? PZ_OK : PZ_ENOMEM;
}

extern "C" int pz_device_free(void* ptr) {
  return hipFree(ptr) == hipSuccess ? PZ_OK : PZ_EDEVICE;
}

extern "C" int pz_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  return hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice) == hipSuccess ? PZ_OK : PZ_EDEVICE;
}

extern "C" int pz_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  return hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost) == hipSuccess ? PZ_OK : PZ_EDEVICE;
}
