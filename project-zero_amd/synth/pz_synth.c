/*
 * pz_synth.c -- deterministic synthetic workloads for the sampling path.
 *
 * Host-only C99 generators for seeded fp32 logits rows, token histories and
 * per-row uniform draws.  Every row has its own stream, seeded as
 * base_seed ^ (row + 1) * 0x9E3779B97F4A7C15, so rows can be generated in
 * parallel (OpenMP) and any subset of rows can be regenerated bit-identically.
 *
 *   normal : splitmix64 -> 53-bit uniform -> Box-Muller in double -> fp32
 *   gumbel : scale * -log(-log(u)) in double -> fp32
 *   zipf   : inverse CDF over ranks 1..V with weight rank^-s, id = rank - 1
 *   draws  : xorshift64* rng_float (src/sampling/rng.c:8-17) seeded with
 *            seed ^ (b + 1) through rng_seed (rng.c:3-6)
 *
 * Not part of the sampler ABI: tests and bench.py use it to build inputs.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define GOLDEN 0x9E3779B97F4A7C15ULL

static uint64_t splitmix64(uint64_t *s) {
  uint64_t z = (*s += GOLDEN);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

/* uniform in [0,1) with 53 random bits */
static double unif(uint64_t *s) {
  return (double)(splitmix64(s) >> 11) * (1.0 / 9007199254740992.0);
}

/* uniform in (0,1] */
static double unif_pos(uint64_t *s) { return 1.0 - unif(s); }

static uint64_t row_seed(uint64_t base, long row) {
  return base ^ ((uint64_t)(row + 1) * GOLDEN);
}

/* out[r*ld + i] = mean + sigma * N(0,1), i < V */
void pz_synth_normal(float *out, int rows, int V, long ld, double mean,
                     double sigma, uint64_t seed) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; r++) {
    uint64_t s = row_seed(seed, r);
    float *o = out + r * ld;
    int i = 0;
    for (; i + 1 < V; i += 2) {
      double u1 = unif_pos(&s), u2 = unif(&s);
      double rad = sqrt(-2.0 * log(u1));
      double th = 6.283185307179586 * u2;
      o[i] = (float)(mean + sigma * rad * cos(th));
      o[i + 1] = (float)(mean + sigma * rad * sin(th));
    }
    if (i < V) {
      double u1 = unif_pos(&s), u2 = unif(&s);
      o[i] = (float)(mean + sigma * sqrt(-2.0 * log(u1)) *
                                cos(6.283185307179586 * u2));
    }
  }
}

/* out[r*ld + i] = scale * Gumbel(0,1) */
void pz_synth_gumbel(float *out, int rows, int V, long ld, double scale,
                     uint64_t seed) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; r++) {
    uint64_t s = row_seed(seed, r);
    float *o = out + r * ld;
    for (int i = 0; i < V; i++) {
      double u = unif(&s);
      if (u <= 0.0) u = 0x1p-53;
      o[i] = (float)(scale * -log(-log(u)));
    }
  }
}

/* Adds U[lo,hi) to n_spikes DISTINCT uniform ids per row; ids written to
 * spike_ids[r*n_spikes + j] when non-NULL. */
void pz_synth_spikes(float *out, int rows, int V, long ld, int n_spikes,
                     double lo, double hi, uint64_t seed, int32_t *spike_ids) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; r++) {
    uint64_t s = row_seed(seed, r);
    int32_t picked[64];
    int m = n_spikes < 64 ? n_spikes : 64;
    for (int j = 0; j < m;) {
      int id = (int)(unif(&s) * V);
      if (id >= V) id = V - 1;
      int dup = 0;
      for (int t = 0; t < j; t++) dup |= picked[t] == id;
      if (dup) continue;
      picked[j] = id;
      double add = lo + (hi - lo) * unif(&s);
      out[r * ld + id] = (float)((double)out[r * ld + id] + add);
      if (spike_ids) spike_ids[r * n_spikes + j] = id;
      j++;
    }
  }
}

/* draft = target + sigma * N(0,1), elementwise over [rows, V] */
void pz_synth_perturb(float *dst, const float *src, int rows, int V, long ld,
                      double sigma, uint64_t seed) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; r++) {
    uint64_t s = row_seed(seed, r);
    const float *a = src + r * ld;
    float *o = dst + r * ld;
    for (int i = 0; i < V; i++) {
      double u1 = unif_pos(&s), u2 = unif(&s);
      double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
      o[i] = (float)((double)a[i] + sigma * z);
    }
  }
}

/* ids[r*H + j] uniform in [0, V) */
void pz_synth_uniform_ids(int32_t *ids, int rows, int H, int V, uint64_t seed) {
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; r++) {
    uint64_t s = row_seed(seed, r);
    for (int j = 0; j < H; j++) {
      int id = (int)(unif(&s) * V);
      ids[r * H + j] = id >= V ? V - 1 : id;
    }
  }
}

/* ids[r*H + j] ~ Zipf(s) over ranks 1..V, id = rank - 1 */
int pz_synth_zipf_ids(int32_t *ids, int rows, int H, int V, double s_exp,
                      uint64_t seed) {
  double *cdf = (double *)malloc((size_t)V * sizeof(double));
  if (!cdf) return -1;
  double acc = 0.0;
  for (int k = 0; k < V; k++) {
    acc += pow((double)(k + 1), -s_exp);
    cdf[k] = acc;
  }
#pragma omp parallel for schedule(static)
  for (long r = 0; r < rows; r++) {
    uint64_t st = row_seed(seed, r);
    for (int j = 0; j < H; j++) {
      double t = unif(&st) * acc;
      int lo = 0, hi = V - 1;
      while (lo < hi) {
        int mid = lo + (hi - lo) / 2;
        if (cdf[mid] > t) hi = mid; else lo = mid + 1;
      }
      ids[r * H + j] = lo;
    }
  }
  free(cdf);
  return 0;
}

/* xorshift64* draw of src/sampling/rng.c:8-17 */
static float rng_float_(unsigned long long *state) {
  unsigned long long x = *state;
  x ^= x >> 12;
  x ^= x << 25;
  x ^= x >> 27;
  *state = x;
  return (float)((x * 0x2545F4914F6CDD1DULL) >> 33) / 2147483648.0f;
}

/* u[b] = first rng_float after rng_seed(seed ^ (b + 1)) */
void pz_synth_draws(float *u, int n, uint64_t seed) {
  for (int b = 0; b < n; b++) {
    unsigned long long st = seed ^ (uint64_t)(b + 1);
    if (!st) st = 1;
    u[b] = rng_float_(&st);
  }
}

/* Draft token ids sampled from q = softmax(D / tau) with the ascending-id
 * categorical rule (generate.c:157-169), uniforms from pz_synth_draws. */
void pz_synth_draft_ids(int32_t *ids, const float *draft, int rows, int V,
                        long ld, float tau, uint64_t seed) {
  float *w = (float *)malloc((size_t)V * sizeof(float));
  if (!w) return;
  float inv = 1.0f / tau;
  for (long r = 0; r < rows; r++) {
    const float *d = draft + r * ld;
    float mx = d[0] * inv;
    for (int i = 0; i < V; i++) {
      w[i] = d[i] * inv;
      if (w[i] > mx) mx = w[i];
    }
    float sum = 0.0f;
    for (int i = 0; i < V; i++) { w[i] = expf(w[i] - mx); sum += w[i]; }
    float is = 1.0f / sum;
    unsigned long long st = seed ^ (uint64_t)(r + 1);
    if (!st) st = 1;
    float u = rng_float_(&st);
    float cdf = 0.0f;
    int pick = V - 1;
    for (int i = 0; i < V; i++) {
      cdf += w[i] * is;
      if (u < cdf) { pick = i; break; }
    }
    ids[r] = pick;
  }
  free(w);
}
