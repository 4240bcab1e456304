// pz_launch.h -- what the host dispatcher hands each kernel launcher.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "pz_params.h"

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
  const float* u;       // device [B] uniforms
  int32_t* ids;         // device [B] sampled ids
  float* p_out;         // device [B] p(chosen) or nullptr
  void* scratch;        // device scratch owned by the sampler
  size_t scratch_bytes;
  int max_lds;          // max dynamic LDS per workgroup on this device
  hipStream_t stream;
};

int pz_launch_greedy(const pz_launch& L, int n_rows, const int32_t* d_rows);
int pz_launch_topk(const pz_launch& L, int n_rows, const int32_t* d_rows);
int pz_launch_topp(const pz_launch& L, int n_rows, const int32_t* d_rows);
int pz_launch_categorical(const pz_launch& L, int n_rows, const int32_t* d_rows);
