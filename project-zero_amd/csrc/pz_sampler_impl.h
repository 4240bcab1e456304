// pz_sampler_impl.h -- the sampler object behind the opaque pz_sampler
// handle of include/pz_sampler.h (shared by the host-side sources).
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/pz_sampler.h"
#include "pz_launch.h"
#include "pz_params.h"

struct pz_sampler {
  int device = 0;
  int max_batch = 0, max_vocab = 0, max_hist = 0;
  int temp_mode = PZ_TEMP_MUL_RECIP;
  int max_lds = 0;
  int n_cu = 0;                       // compute units of the device
  uint32_t wait_polls = PZ_POLL_CAP;  // bound of the waits between workgroups
  hipStream_t stream = nullptr;
  hipEvent_t staged = nullptr;  // guards reuse of the pinned staging area

  // pinned host staging and their device mirrors
  pz_row_params_dev* h_params = nullptr;
  pz_row_params_dev* d_params = nullptr;
  int32_t* h_rows = nullptr;
  int32_t* d_rows = nullptr;
  // uniforms in, ids and p out of the synchronous call: coherent pinned host
  // memory that the kernels read and write directly (z_*: the device's
  // addresses of the same buffers), so a call needs no copy commands
  float* h_u = nullptr;
  const float* z_u = nullptr;
  int32_t* h_ids = nullptr;
  int32_t* z_ids = nullptr;
  float* h_p = nullptr;
  float* z_p = nullptr;

  void* d_scratch = nullptr;
  size_t scratch_bytes = 0;
  pz_scratch sc{};
  // workspace of the row-split passes (rows up to max_batch, ids up to
  // max_vocab, top-p candidate lists)
  void* d_split = nullptr;
  size_t split_bytes = 0;
  PzSplitWs ws{};

  // decode steps with device-side draws: the uniforms the draw kernel
  // writes (max_batch) and the EOS ids (PZ_MAX_EOS, n_eos in use)
  float* d_u_step = nullptr;
  int32_t* d_eos = nullptr;
  int n_eos = 0;
  int32_t h_eos[PZ_MAX_EOS] = {0};  // host copy of the list (the speculative loop's stops)

  // fused LM head + argmax: per-row argmax keys (zero between calls) and
  // the NaN flag of logit 0 (max_batch each)
  unsigned long long* d_lmh_keys = nullptr;
  uint8_t* d_lmh_nan = nullptr;

  const float* call_u = nullptr;  // the synchronous call's host uniforms, during the call

  pz_row_params_dev* res_params = nullptr;  // host work area (max_batch)
  int staged_n = -1, staged_B = -1;         // what d_params / d_rows hold

  // speculative verification: device scratch and pinned staging, grown on
  // demand by pz_spec_verify
  void* spec_dev = nullptr;
  size_t spec_dev_bytes = 0;
  void* attn_dev = nullptr;  // the row-split attention softmax's workspace (grown on demand)
  size_t attn_dev_bytes = 0;
  void* spec_host = nullptr;   // mapped, coherent pinned inputs and outputs
  void* spec_zc = nullptr;     // its device address
  size_t spec_host_bytes = 0;
  bool spec_busy = false;      // a call's kernels may still read spec_host

  char err[512] = {0};
};

static inline int fail(pz_sampler* s, int code, const char* fmt, ...) {
  if (s) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(s->err, sizeof(s->err), fmt, ap);
    va_end(ap);
  }
  return code;
}

#define PZ_HIP(s, expr)                                                      \
  do {                                                                       \
    hipError_t e_ = (expr);                                                  \
    if (e_ != hipSuccess)                                                    \
      return fail((s), PZ_EDEVICE, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

// Kernel form of one row's parameters (mode, clamps, reciprocal temperature).
pz_row_params_dev pz_resolve_row(const pz_row_params& p, int V, int temp_mode);
bool pz_penalty_active(const pz_row_params& p);
bool pz_needs_counts(const pz_row_params& p);
// LDS hash capacity for presence / frequency counts over H history ids.
int pz_hash_capacity(bool counts_any, int H);
// Rows per mode and each mode's offset in a mode-grouped row list.
void pz_group_rows(const pz_row_params_dev* res, int B, int n_params, int count[PZ_MODE_COUNT],
                   int offset[PZ_MODE_COUNT], int* modes_present);
// Largest top_k among the top-k rows (0 when there are none).
int pz_max_top_k(const pz_row_params_dev* res, int B, int n_params);
// The mode-grouped row list (B entries).
void pz_fill_rows(const pz_row_params_dev* res, int B, int n_params,
                  const int offset[PZ_MODE_COUNT], int32_t* rows);
// One launch per mode present; d_rows (device, the grouped list) is read only
// when more than one mode is present.  Returns 0, or the failing launcher's
// code with *failed_mode set.
int pz_launch_modes(const pz_launch& L, const int count[PZ_MODE_COUNT],
                    const int offset[PZ_MODE_COUNT], int modes_present, const int32_t* d_rows,
                    int* failed_mode);

// Extra work of a decode step (pz_sample_step): the per-row draws from
// device RNG states before sampling, the EOS flags after.
struct PzStepHooks {
  uint64_t* state;   // device [B] xorshift64* states
  uint8_t* eos_out;  // device [B] flags, or nullptr
};
int pz_launch_step_draw(const pz_launch& L, int B, uint64_t* d_state, float* d_u);
int pz_launch_step_eos(hipStream_t st, const int32_t* d_ids, int B, const int32_t* d_eos,
                       int n_eos, uint8_t* d_flags);

// Resolves host parameters and samples (the body of the pz_sample_* entry
// points); hooks != nullptr makes it a decode step (d_u is then ignored).
int pz_dispatch_params(pz_sampler* s, const float* d_logits, int B, int V, long ld,
                       const pz_row_params* params, int n_params, const int32_t* d_hist,
                       int H, const float* d_u, int32_t* d_ids, float* d_p,
                       const PzStepHooks* hooks);

// The reference softmax of B device rows, one workgroup per row, after the
// temperature T; row r holds min(d_len[r], V) entries (all V when d_len is
// nullptr).
int pz_launch_softmax_rows(pz_sampler* s, const float* d_in, long ld_in, float* d_out,
                           long ld_out, int B, int V, PzTemp T, const int32_t* d_len);

// Launches the kernels for B rows whose kernel parameters are already in
// s->res_params (n_params entries).  Used by the public entry points after
// resolving pz_row_params, and by the reference-compatible calls, which set
// a row's mode directly.
int pz_dispatch_resolved(pz_sampler* s, const float* d_logits, int B, int V, long ld,
                         int n_params, const int32_t* d_hist, int H, bool pen_any,
                         bool counts_any, const float* d_u, int32_t* d_ids, float* d_p,
                         const PzStepHooks* hooks = nullptr);
