/*
 * dropin.c -- a C99 host program that uses libpzsample.so exactly where the
 * reference's objects of src/sampling would sit: it includes only
 * pz_sampling_compat.h and links -lpzsample.  Test infrastructure, built by
 * tests/native/Makefile and run by tests/test_gpu_dropin.py.
 *
 *   dropin kat                 known-answer checks of the sampler API, the
 *                              properties tests/test_sampling.c:24-245 checks
 *                              (argmax ties and ranges, power-of-two
 *                              temperatures, top-p and top-k ranges and
 *                              restrictions, RNG range / reproducibility);
 *                              prints one line per failure and a summary,
 *                              exit status 0 when all pass.
 *   dropin dispatch IN OUT     the sampling block of generate.c:145-169 on
 *                              each row of IN (its own seeded RNG state),
 *                              writing the id and the final state per row.
 *
 * IN:  int32 rows, int32 V, then per row {float T, float top_p, int32 top_k,
 *      uint64 seed}, then rows x V float logits.   OUT: per row {int32 id,
 *      uint64 state}.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "pz_sampling_compat.h"

static int n_checks = 0, n_failed = 0;

static void check(int ok, const char *what) {
  n_checks++;
  if (!ok) {
    n_failed++;
    printf("FAIL: %s\n", what);
  }
}

static int argmax_of(const float *x, int n) {
  float a[16];
  memcpy(a, x, (size_t)n * sizeof(float));
  return sample_argmax(a, n);
}

static void kat_argmax(void) {
  const float mid[] = {0.5f, 2.5f, -1.0f, 1.0f};
  const float first[] = {9.0f, 1.0f, 2.0f};
  const float last[] = {0.0f, 1.0f, 2.0f, 7.0f};
  const float neg[] = {-3.0f, -0.5f, -2.0f};
  const float one[] = {-4.0f};
  const float tie[] = {1.0f, 6.0f, 6.0f, 6.0f};
  check(argmax_of(mid, 4) == 1, "argmax picks the largest logit");
  check(argmax_of(first, 3) == 0, "argmax at the first element");
  check(argmax_of(last, 4) == 3, "argmax at the last element");
  check(argmax_of(neg, 3) == 1, "argmax over negative logits");
  check(argmax_of(one, 1) == 0, "argmax of one logit");
  check(argmax_of(tie, 4) == 1, "argmax ties go to the lowest id");
}

static void kat_temperature(void) {
  float x[] = {2.0f, -4.0f, 6.0f, 0.0f};
  const float half[] = {1.0f, -2.0f, 3.0f, 0.0f};
  apply_temperature(x, 4, 2.0f);
  check(memcmp(x, half, sizeof(x)) == 0, "T = 2 halves every logit");
  float y[] = {1.5f, -2.25f, 3.0f};
  const float y0[] = {1.5f, -2.25f, 3.0f};
  apply_temperature(y, 3, 1.0f);
  check(memcmp(y, y0, sizeof(y)) == 0, "T = 1 leaves logits unchanged");
  float z[] = {1.0f, 2.0f, 3.0f};
  apply_temperature(z, 3, 0.5f);
  check(z[0] == 2.0f && z[1] == 4.0f && z[2] == 6.0f, "T = 0.5 doubles every logit");
  float w[] = {0.3f, 1.7f, -0.2f, 1.1f};
  apply_temperature(w, 4, 0.37f);
  check(argmax_of(w, 4) == 1, "temperature keeps the argmax");
}

static void kat_top_p(void) {
  unsigned long long st;
  rng_seed(&st, 7);
  int all_peak = 1;
  for (int t = 0; t < 50; t++) {
    float x[] = {0.0f, 20.0f, 0.5f, -1.0f};
    all_peak &= sample_top_p(x, 4, 0.9f, &st) == 1;
  }
  check(all_peak, "top-p returns the dominant logit");
  int seen[4] = {0, 0, 0, 0}, in_range = 1;
  rng_seed(&st, 11);
  for (int t = 0; t < 200; t++) {
    float x[] = {1.0f, 1.1f, 0.9f, 1.05f};
    const int id = sample_top_p(x, 4, 0.99f, &st);
    if (id < 0 || id > 3) in_range = 0; else seen[id] = 1;
  }
  check(in_range, "top-p ids lie in the vocabulary");
  check(seen[0] + seen[1] + seen[2] + seen[3] >= 3, "top-p of a flat row reaches most ids");
}

static void kat_top_k(void) {
  unsigned long long st;
  rng_seed(&st, 3);
  int is_argmax = 1, in_range = 1, top2 = 1;
  for (int t = 0; t < 50; t++) {
    float x[] = {0.1f, 3.0f, 2.9f, -1.0f, 0.0f, 1.0f, 2.0f, 0.5f};
    is_argmax &= sample_top_k(x, 8, 1, &st) == 1;
    const int id = sample_top_k(x, 8, 5, &st);
    in_range &= id >= 0 && id < 8;
    const int id2 = sample_top_k(x, 8, 2, &st);
    top2 &= id2 == 1 || id2 == 2;
  }
  check(is_argmax, "top-k with k = 1 is argmax");
  check(in_range, "top-k ids lie in the vocabulary");
  check(top2, "top-k with k = 2 picks one of the two largest");
  float y[] = {0.2f, 0.4f};
  const int id = sample_top_k(y, 2, 10, &st);
  check(id >= 0 && id < 2, "top-k clamps k to the vocabulary");
}

static void kat_rng(void) {
  unsigned long long a, b;
  rng_seed(&a, 42);
  int in01 = 1;
  for (int t = 0; t < 1000; t++) {
    const float v = rng_float(&a);
    in01 &= v >= 0.0f && v < 1.0f;
  }
  check(in01, "rng_float lies in [0, 1)");
  rng_seed(&a, 12345);
  rng_seed(&b, 12345);
  int same = 1;
  for (int t = 0; t < 100; t++) same &= rng_float(&a) == rng_float(&b);
  check(same, "one seed gives one sequence");
  rng_seed(&a, 111);
  rng_seed(&b, 222);
  int differ = 0;
  for (int t = 0; t < 10; t++) differ |= rng_float(&a) != rng_float(&b);
  check(differ, "different seeds give different sequences");
  rng_seed(&a, 0);
  const float v = rng_float(&a);
  check(v >= 0.0f && v < 1.0f, "seed 0 still gives a valid draw");
}

/* generate.c:145-169 with sample_top_k in front of top-p when top_k > 0 */
static int sample_row(float *x, int V, float T, float top_p, int top_k, unsigned long long *st) {
  if (T <= 0.0f || T < 1e-6f) return sample_argmax(x, V);
  apply_temperature(x, V, T);
  if (top_k > 0) return sample_top_k(x, V, top_k, st);
  if (top_p < 1.0f && top_p > 0.0f) return sample_top_p(x, V, top_p, st);
  pz_tn_softmax(x, V);
  const float r = rng_float(st);
  float cdf = 0.0f;
  for (int i = 0; i < V; i++) {
    cdf += x[i];
    if (r < cdf) return i;
  }
  return V - 1;
}

static int dispatch(const char *in_path, const char *out_path) {
  FILE *in = fopen(in_path, "rb"), *out = fopen(out_path, "wb");
  if (!in || !out) return 2;
  int32_t rows, V;
  if (fread(&rows, 4, 1, in) != 1 || fread(&V, 4, 1, in) != 1 || rows <= 0 || V <= 0) return 2;
  struct {
    float T, top_p;
    int32_t top_k;
    uint64_t seed;
  } *prm = malloc((size_t)rows * sizeof(*prm));
  float *x = malloc((size_t)V * sizeof(float));
  if (!prm || !x) return 2;
  for (int r = 0; r < rows; r++) {
    if (fread(&prm[r].T, 4, 1, in) != 1 || fread(&prm[r].top_p, 4, 1, in) != 1 ||
        fread(&prm[r].top_k, 4, 1, in) != 1 || fread(&prm[r].seed, 8, 1, in) != 1)
      return 2;
  }
  for (int r = 0; r < rows; r++) {
    if (fread(x, 4, (size_t)V, in) != (size_t)V) return 2;
    unsigned long long st;
    rng_seed(&st, prm[r].seed);
    const int32_t id = sample_row(x, V, prm[r].T, prm[r].top_p, prm[r].top_k, &st);
    const uint64_t s = st;
    fwrite(&id, 4, 1, out);
    fwrite(&s, 8, 1, out);
  }
  free(prm);
  free(x);
  fclose(in);
  return fclose(out) == 0 && pz_compat_last_status() == 0 ? 0 : 3;
}

int main(int argc, char **argv) {
  if (argc >= 2 && strcmp(argv[1], "kat") == 0) {
    kat_argmax();
    kat_temperature();
    kat_top_p();
    kat_top_k();
    kat_rng();
    printf("%d of %d checks passed\n", n_checks - n_failed, n_checks);
    return n_failed == 0 && pz_compat_last_status() == 0 ? 0 : 1;
  }
  if (argc == 4 && strcmp(argv[1], "dispatch") == 0) return dispatch(argv[2], argv[3]);
  fprintf(stderr, "usage: dropin kat | dropin dispatch IN OUT\n");
  return 2;
}
