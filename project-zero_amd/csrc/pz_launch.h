// pz_launch.h -- what the host dispatcher hands each kernel launcher.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "pz_params.h"
#include "pz_sampler.h"
#include "pz_split.h"

// Device scratch owned by a sampler (carved from one allocation).
constexpr int PZ_FB_SLOTS = 32;        // rows the top-p fallback kernel sorts at once
constexpr int PZ_COUNTERS = 64;        // words of pz_scratch::counters
constexpr int PZ_TOPP_MAX_V = 200000;  // top_p.c:27 (larger rows take argmax)
constexpr int PZ_TOPP_CAPG = 12288;    // top-p candidates a row can gather for the LDS sort

struct pz_scratch {
  float* row_stat;    // [max_batch][4] per-row values handed between kernels
  int32_t* fb_list;   // [max_batch] rows queued for the top-p fallback
  int32_t* counters;  // [PZ_COUNTERS] queue counters: [0] rows queued for the top-p
                      // fallback (emptied by a top-p launch's first kernel)
  uint64_t* fb_keys;  // [fb_slots][slot_n] sort buffers of the fallback
  uint64_t* fb_keys2; // [fb_slots][slot_n] its second buffer (keys in bin order)
  int slot_n;         // power of two >= min(max_vocab, PZ_TOPP_MAX_V)
  int fb_slots;       // min(PZ_FB_SLOTS, max_batch) sort slots
};

// Bytes of scratch for max_batch rows of up to max_vocab ids with at most
// max_slots fallback sort slots; with base != nullptr also fills *out with
// the carved pointers.
size_t pz_scratch_layout(int max_batch, int max_vocab, int max_slots, void* base,
                         pz_scratch* out);

struct pz_launch {
  const float* logits;  // device [B, ld] fp32, caller-owned, read-only
  long ld;              // row stride in elements
  int V;                // vocabulary size
  const pz_row_params_dev* params;  // device, n_params entries
  int n_params;         // 1 (shared) or B
  const int32_t* hist;  // device [B, H] or nullptr
  int H;
  int hcap;             // LDS hash capacity for presence/frequency counts (0: none)
  bool pen_any;         // any row has an active penalty
  bool temp_div;        // temperature as x / T (scalar build) rather than x * (1/T)
  const float* u;       // device [B] uniforms
  const float* h_u = nullptr;  // host copy of the same uniforms, when the caller has one
  int B = 0;            // rows of the call
  int32_t* ids;         // device [B] sampled ids
  float* p_out;         // device [B] p(chosen) or nullptr
  pz_scratch sc;         // device scratch owned by the sampler
  PzSplitWs ws;          // workspace of the row-split passes
  int kmax = 0;         // largest top_k among the launch's top-k rows (0: unknown)
  int max_lds;          // max dynamic LDS per workgroup on this device
  uint32_t wait_polls = PZ_POLL_CAP;  // bound of a wait between workgroups, in polls
  int n_cu = 0;                       // compute units of the device
  hipStream_t stream;
};

int pz_launch_greedy(const pz_launch& L, int n_rows, const int32_t* d_rows);
// Argmax of the tempered row (top-p rows above the vocabulary guard).
int pz_launch_greedy_tempered(const pz_launch& L, int n_rows, const int32_t* d_rows);
int pz_launch_topk(const pz_launch& L, int n_rows, const int32_t* d_rows);
int pz_launch_topp(const pz_launch& L, int n_rows, const int32_t* d_rows);
int pz_launch_categorical(const pz_launch& L, int n_rows, const int32_t* d_rows);
