// pz_params.h -- per-row sampling parameters as the kernels read them.
// Resolved on the host from pz_row_params (include/pz_sampler.h): the
// sampling mode is decided once per row, temperature is clamped and its
// reciprocal rounded exactly as src/sampling/temperature.c:10-12 does.
#pragma once
#include <stdint.h>

enum {
  PZ_MODE_GREEDY = 0,       // generate.c:151-152 (T < 1e-6)
  PZ_MODE_CATEGORICAL = 1,  // generate.c:157-169 (softmax + ascending CDF)
  PZ_MODE_TOPK = 2,         // top_k.c, chained with top-p when 0<p<1
  PZ_MODE_TOPP = 3,         // top_p.c:30-108
  PZ_MODE_COUNT = 4
};

typedef struct {
  float temp;      // temperature after the 1e-6 clamp
  float inv_temp;  // 1.0f / temp (fp32 division on the host)
  int32_t temp_div;  // 1: x / temp (scalar build), 0: x * inv_temp (AVX-512 build)
  int32_t mode;
  int32_t top_k;   // clamped to [1, min(V, 1024)] (top_k.c:11-17)
  float top_p;
  float rep_penalty;
  float presence_penalty;
  float frequency_penalty;
  int32_t pad_;
} pz_row_params_dev;
