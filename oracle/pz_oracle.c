/*
 * pz_oracle.c -- CPU oracle for the token-sampling path (TEST INFRASTRUCTURE).
 *
 * A clean-room C99 restatement of the Project Zero sampler semantics.  It is
 * the checker for the HIP product and the timed CPU baseline; it is never
 * linked into the product.  Build: oracle/Makefile (gcc -std=c99 -O3
 * -ffp-contract=off, libm expf, no -ffast-math).
 */
#include "pz_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define ORC_TOPK_MAX 1024      /* top_k.c:6 */
#define ORC_TOPP_MAX_V 200000  /* top_p.c:27 */

float orc_expf(float x) { return expf(x); }

/* Order-independent hash of libm expf over the fp32 bit patterns lo..hi
 * (every stride-th one), for the exhaustive comparison with the GPU's
 * exponential: sum over inputs of a 64-bit finaliser of (result, input). */
static uint64_t mix64(uint64_t z) {
  z ^= z >> 33;
  z *= 0xff51afd7ed558ccdULL;
  z ^= z >> 33;
  z *= 0xc4ceb9fe1a85ec53ULL;
  z ^= z >> 33;
  return z;
}

uint64_t orc_expf_hash(uint32_t lo, uint32_t hi, uint32_t stride) {
  uint64_t h = 0;
  const uint64_t n = ((uint64_t)hi - lo) / stride + 1;
#pragma omp parallel for reduction(+ : h) schedule(static)
  for (int64_t i = 0; i < (int64_t)n; i++) {
    const uint32_t b = lo + (uint32_t)((uint64_t)i * stride);
    float x, r;
    uint32_t rb;
    memcpy(&x, &b, 4);
    r = expf(x);
    memcpy(&rb, &r, 4);
    h += mix64(((uint64_t)rb << 32) | b);
  }
  return h;
}

static void info_reset(orc_info *info) {
  if (!info) return;
  info->p_chosen = 1.0f;
  info->dist_draw = FLT_MAX;
  info->dist_cut = FLT_MAX;
  info->cutoff = 0;
  info->n_cand = 0;
  info->trunc_sum = 0.0f;
  info->norm_sum = 0.0f;
  info->path = ORC_PATH_ARGMAX;
}

static float fminf_(float a, float b) { return a < b ? a : b; }

/* Distance of r from the CDF partial sums bracketing slot j: the draw picked
 * slot j because lo <= r < hi. */
static float draw_dist(float r, float lo, float hi) {
  return fminf_(r - lo, hi - r);
}

/* ---- a1: src/sampling/rng.c:3-6 (seed 0 -> 1) and :8-17 (xorshift64*) -- */
void orc_rng_seed(unsigned long long *state, unsigned long long seed) {
  *state = seed ? seed : 1ULL;
}

float orc_rng_float(unsigned long long *state) {
  unsigned long long s = *state;
  s ^= s >> 12;
  s ^= s << 25;
  s ^= s >> 27;
  *state = s;
  /* upper 31 bits of the xorshift64* product, int->float rounds to nearest
   * (so the result can be exactly 1.0f), then an exact division by 2^31 */
  return (float)((s * 0x2545F4914F6CDD1DULL) >> 33) / 2147483648.0f;
}

/* ---- a2: src/sampling/argmax.c:3-13 -- first maximum, strict '>' ------- */
int orc_argmax(const float *x, int n) {
  int best = 0;
  float bv = x[0];
  for (int i = 1; i < n; i++)
    if (x[i] > bv) { bv = x[i]; best = i; }
  return best;
}

/* ---- a3: src/sampling/temperature.c:8-25 ------------------------------- */
void orc_apply_temperature(float *x, int n, float temperature, int mode) {
  if (temperature < 1e-6f) temperature = 1e-6f;          /* :10 */
  if (mode == ORC_TEMP_MUL_RECIP) {
    float inv = 1.0f / temperature;                        /* :12 */
    for (int i = 0; i < n; i++) x[i] *= inv;               /* :15-20 */
  } else {
    for (int i = 0; i < n; i++) x[i] /= temperature;       /* :22-23 */
  }
}

/* ---- a4: src/math/softmax.c:4-23 (== softmax_avx512.c:20-64 bitwise) -- */
static float softmax_sum(float *x, int n) {
  float mx = x[0];
  for (int i = 1; i < n; i++)
    if (x[i] > mx) mx = x[i];                              /* :6-9 */
  float sum = 0.0f;
  for (int i = 0; i < n; i++) {                            /* :12-16 */
    x[i] = expf(x[i] - mx);
    sum += x[i];
  }
  float inv = 1.0f / sum;                                  /* :19-22 */
  for (int i = 0; i < n; i++) x[i] *= inv;
  return sum;
}

void orc_softmax(float *x, int n) { (void)softmax_sum(x, n); }

/* ---- a5: src/transformer/generate.c:157-169 ---------------------------- */
int orc_categorical(const float *probs, int n, float r, orc_info *info) {
  float cdf = 0.0f;
  int next = n - 1;                                        /* :161 fallback */
  float lo = 0.0f;
  int hit = 0;
  for (int i = 0; i < n; i++) {                            /* :162-168 */
    lo = cdf;
    cdf += probs[i];
    if (r < cdf) { next = i; hit = 1; break; }
  }
  if (info) {
    info->path = ORC_PATH_CATEGORICAL;
    info->p_chosen = probs[next];
    info->dist_draw = hit ? draw_dist(r, lo, cdf) : r - cdf;
  }
  return next;
}

/* Top-k selection of top_k.c:29-48: keeps the k largest values that exceed
 * -1e30, ties resolved to the lower id (strict '>' insertion), list sorted by
 * (value desc, id asc); unfilled slots hold (-1e30, -1).  Returns k after the
 * clamps of top_k.c:11-17. */
static int topk_select(const float *x, int n, int k, float *vals, int *idx) {
  if (k > n) k = n;
  if (k <= 0) k = 1;
  if (k > ORC_TOPK_MAX) k = ORC_TOPK_MAX;
  for (int i = 0; i < k; i++) { idx[i] = -1; vals[i] = -1e30f; }
  for (int i = 0; i < n; i++) {
    if (x[i] > vals[k - 1]) {
      int j = k - 1;
      while (j > 0 && x[i] > vals[j - 1]) {
        vals[j] = vals[j - 1];
        idx[j] = idx[j - 1];
        j--;
      }
      vals[j] = x[i];
      idx[j] = i;
    }
  }
  return k;
}

/* Softmax over the selected values as top_k.c:50-59 (expf(v - v0), a
 * sequential sum, then a true division). */
static void topk_softmax(float *vals, int k) {
  float mx = vals[0];
  float sum = 0.0f;
  for (int i = 0; i < k; i++) {
    vals[i] = expf(vals[i] - mx);
    sum += vals[i];
  }
  for (int i = 0; i < k; i++) vals[i] /= sum;
}

/* ---- a6: src/sampling/top_k.c:8-73 ------------------------------------- */
int orc_top_k(const float *x, int n, int k, float u, orc_info *info) {
  float vals[ORC_TOPK_MAX];
  int idx[ORC_TOPK_MAX];
  k = topk_select(x, n, k, vals, idx);
  topk_softmax(vals, k);
  float r = u;                                             /* :62 */
  float cdf = 0.0f, lo = 0.0f;
  for (int i = 0; i < k; i++) {                            /* :63-69 */
    lo = cdf;
    cdf += vals[i];
    if (r < cdf) {
      if (info) {
        info->path = ORC_PATH_TOPK;
        info->cutoff = k;
        info->p_chosen = vals[i];
        info->dist_draw = draw_dist(r, lo, cdf);
      }
      return idx[i];
    }
  }
  if (info) {                                              /* :71-72 */
    info->path = ORC_PATH_TOPK;
    info->cutoff = k;
    info->p_chosen = vals[0];
    info->dist_draw = r - cdf;
  }
  return idx[0];
}

/* ---- a7: src/sampling/top_p.c:30-108 ----------------------------------- */
typedef struct { float prob; int index; } orc_pi;

/* (prob desc, index asc): the order glibc's stable qsort leaves the
 * ascending-id candidate list in under compare_prob_desc (top_p.c:12-20). */
static int cmp_pi(const void *a, const void *b) {
  const orc_pi *x = (const orc_pi *)a, *y = (const orc_pi *)b;
  if (x->prob > y->prob) return -1;
  if (x->prob < y->prob) return 1;
  return (x->index > y->index) - (x->index < y->index);
}

static __thread orc_pi *g_cand = NULL;  /* grows on demand; one per thread */
static __thread int g_cand_cap = 0;

static orc_pi *cand_buf(int n) {
  if (n > g_cand_cap) {
    free(g_cand);
    g_cand = (orc_pi *)malloc((size_t)n * sizeof(orc_pi));
    g_cand_cap = g_cand ? n : 0;
  }
  return g_cand;
}

/* Nucleus cut-off, truncated mass and draw over a list already sorted by
 * (prob desc, index asc): top_p.c:79-105. */
static int nucleus_draw(const orc_pi *c, int n, float top_p, float u,
                        orc_info *info) {
  float cumulative = 0.0f, prev = 0.0f;
  int cutoff = n;
  for (int i = 0; i < n; i++) {                            /* :80-88 */
    prev = cumulative;
    cumulative += c[i].prob;
    if (cumulative >= top_p) { cutoff = i + 1; break; }
  }
  float trunc_sum = 0.0f;
  for (int i = 0; i < cutoff; i++) trunc_sum += c[i].prob; /* :91-93 */
  float r = u * trunc_sum;                                 /* :96 */
  float cdf = 0.0f, lo = 0.0f;
  int result = c[0].index;                                 /* :98 */
  float pch = c[0].prob, dd = -1.0f;
  for (int i = 0; i < cutoff; i++) {                       /* :99-105 */
    lo = cdf;
    cdf += c[i].prob;
    if (r < cdf) {
      result = c[i].index;
      pch = c[i].prob;
      dd = draw_dist(r, lo, cdf);
      break;
    }
  }
  if (dd < 0.0f) dd = r - cdf;
  if (info) {
    info->cutoff = cutoff;
    info->trunc_sum = trunc_sum;
    info->p_chosen = pch;
    info->dist_draw = dd;
    if (cutoff < n || cumulative >= top_p) {
      float d1 = fabsf(cumulative - top_p);
      float d0 = fabsf(prev - top_p);
      info->dist_cut = fminf_(d0, d1);
    } else {
      info->dist_cut = fabsf(top_p - cumulative);
    }
  }
  return result;
}

int orc_top_p(const float *x, int n, float top_p, float u, orc_info *info) {
  if (n > ORC_TOPP_MAX_V) {                                /* :33-34 */
    if (info) info->path = ORC_PATH_TOPP_ARGMAX;
    return orc_argmax(x, n);
  }
  float mx = x[0];                                         /* :37-41 */
  for (int i = 1; i < n; i++)
    if (x[i] > mx) mx = x[i];
  float thr = mx - 20.0f;                                  /* :53 */
  orc_pi *c = cand_buf(n);
  int m = 0;
  float sum = 0.0f;
  for (int i = 0; i < n; i++) {                            /* :57-65 */
    if (x[i] >= thr) {
      float e = expf(x[i] - mx);
      c[m].prob = e;
      c[m].index = i;
      sum += e;
      m++;
    }
  }
  if (m == 0) {                                            /* :68-69 */
    if (info) info->path = ORC_PATH_TOPP_ARGMAX;
    return orc_argmax(x, n);
  }
  float inv = 1.0f / sum;                                  /* :72-74 */
  for (int i = 0; i < m; i++) c[i].prob *= inv;
  qsort(c, (size_t)m, sizeof(orc_pi), cmp_pi);             /* :77 */
  int id = nucleus_draw(c, m, top_p, u, info);
  if (info) {
    info->path = ORC_PATH_TOPP;
    info->n_cand = m;
    info->norm_sum = sum;
  }
  return id;
}

/* ---- a8/a9: penalties (build-defined) ---------------------------------
 * Repetition (CTRL, Keskar et al. 2019; sign-aware form): every DISTINCT id h
 * of the history in [0, n): x[h] = x[h] > 0 ? x[h] / rep : x[h] * rep.
 * Then presence/frequency (OpenAI convention) with c = count of h:
 * t = (float)c * freq; t = t + pres; x[h] = x[h] - t   (each step rounded).
 * Ids outside [0, n) are ignored. */
void orc_penalties(float *x, int n, const int32_t *hist, int h,
                   float rep, float pres, float freq) {
  if (!hist || h <= 0) return;
  int *cnt = (int *)calloc((size_t)n, sizeof(int));
  if (!cnt) abort();
  for (int j = 0; j < h; j++) {
    int id = hist[j];
    if (id >= 0 && id < n) cnt[id]++;
  }
  for (int j = 0; j < h; j++) {
    int id = hist[j];
    if (id < 0 || id >= n || cnt[id] <= 0) continue;
    int c = cnt[id];
    cnt[id] = 0; /* apply once per distinct id */
    float v = x[id];
    v = v > 0.0f ? v / rep : v * rep;
    float t = (float)c * freq;
    t = t + pres;
    v = v - t;
    x[id] = v;
  }
  free(cnt);
}

/* ---- a10: top-k -> top-p chain (build-defined) -------------------------
 * Selection and softmax of top_k.c (a6), then the cut-off, truncated mass and
 * draw of top_p.c:79-105 over those k sorted probabilities; no second sort,
 * no max-20 prefilter.  With top_p outside (0,1) this is exactly a6. */
int orc_chain(const float *x, int n, int k, float top_p, float u,
              orc_info *info) {
  if (!(top_p > 0.0f && top_p < 1.0f)) return orc_top_k(x, n, k, u, info);
  float vals[ORC_TOPK_MAX];
  int idx[ORC_TOPK_MAX];
  k = topk_select(x, n, k, vals, idx);
  topk_softmax(vals, k);
  orc_pi c[ORC_TOPK_MAX];
  for (int i = 0; i < k; i++) { c[i].prob = vals[i]; c[i].index = idx[i]; }
  int id = nucleus_draw(c, k, top_p, u, info);
  if (info) info->path = ORC_PATH_CHAIN;
  return id;
}

/* ---- per-row dispatch: generate.c:145-169 plus the extensions ---------- */
static __thread float *g_row = NULL;  /* one per thread */
static __thread int g_row_cap = 0;

int orc_sample_row(const float *x, int n, const orc_params *prm,
                   const int32_t *hist, int h, float u, int temp_mode,
                   orc_info *info) {
  info_reset(info);
  if (n > g_row_cap) {
    free(g_row);
    g_row = (float *)malloc((size_t)n * sizeof(float));
    g_row_cap = g_row ? n : 0;
    if (!g_row) abort();
  }
  float *w = g_row;
  memcpy(w, x, (size_t)n * sizeof(float));
  if (hist && h > 0 &&
      (prm->rep_penalty != 1.0f || prm->presence_penalty != 0.0f ||
       prm->frequency_penalty != 0.0f))
    orc_penalties(w, n, hist, h, prm->rep_penalty, prm->presence_penalty,
                  prm->frequency_penalty);
  float T = prm->temperature;
  if (T <= 0.0f || T < 1e-6f) {                            /* :151-152 */
    if (info) info->path = ORC_PATH_ARGMAX;
    return orc_argmax(w, n);
  }
  orc_apply_temperature(w, n, T, temp_mode);               /* :154 */
  if (prm->top_k > 0) return orc_chain(w, n, prm->top_k, prm->top_p, u, info);
  if (prm->top_p < 1.0f && prm->top_p > 0.0f)              /* :155-156 */
    return orc_top_p(w, n, prm->top_p, u, info);
  float s = softmax_sum(w, n);                             /* :158 */
  int id = orc_categorical(w, n, u, info);                 /* :159-169 */
  if (info) info->norm_sum = s;
  return id;
}

void orc_sample_batch(const float *x, int rows, int n, long ld,
                      const orc_params *params, int n_params,
                      const int32_t *hist, int h, const float *u, int temp_mode,
                      int32_t *ids, float *p_chosen, float *dist_draw,
                      float *dist_cut) {
  for (int b = 0; b < rows; b++) {
    orc_info info;
    const orc_params *prm = &params[n_params == 1 ? 0 : b];
    ids[b] = orc_sample_row(x + (long)b * ld, n, prm,
                            hist ? hist + (long)b * h : NULL, h, u[b],
                            temp_mode, &info);
    if (p_chosen) p_chosen[b] = info.p_chosen;
    if (dist_draw) dist_draw[b] = info.dist_draw;
    if (dist_cut) dist_cut[b] = info.dist_cut;
  }
}

/* One decode step.  The uniform is drawn from a copy of the row's state and
 * the copy is kept only when the path taken is one where the reference
 * consumes it: rng_float sits after sample_top_p's two argmax returns
 * (top_p.c:33-34, 68-69, draw at :96), unconditionally in sample_top_k
 * (top_k.c:62) and in the categorical block (generate.c:159); greedy rows
 * never reach a sampler (generate.c:151-152).  EOS as generate.c:201-205
 * (the caller's list holds eos_token_id when it is > 0). */
void orc_sample_step(const float *x, int rows, int n, long ld,
                     const orc_params *params, int n_params,
                     const int32_t *hist, int h, unsigned long long *state,
                     int temp_mode, const int32_t *eos, int n_eos,
                     int32_t *ids, uint8_t *eos_flag, int32_t *drew) {
  for (int b = 0; b < rows; b++) {
    orc_info info;
    const orc_params *prm = &params[n_params == 1 ? 0 : b];
    unsigned long long s = state[b];
    const float u = orc_rng_float(&s);
    ids[b] = orc_sample_row(x + (long)b * ld, n, prm, hist ? hist + (long)b * h : NULL, h, u,
                            temp_mode, &info);
    const int draws = info.path != ORC_PATH_ARGMAX && info.path != ORC_PATH_TOPP_ARGMAX;
    if (draws) state[b] = s;
    if (drew) drew[b] = draws;
    int f = 0;
    for (int e = 0; e < n_eos; e++) f |= eos[e] == ids[b];
    if (eos_flag) eos_flag[b] = (uint8_t)f;
  }
}

/* ---- a11: speculative verification (build-defined) ---------------------
 * Leviathan et al. 2023 (Alg. 1) / Chen et al. 2023.  For draft position j:
 * p = softmax(T_j / tau), q = softmax(D_j / tau) (a3 + a4).  Accept d_j iff
 * u_acc < p(d_j) / q(d_j) (fp32 division; q(d_j) == 0 rejects).  On the first
 * rejection: r(x) = max(0, p(x) - q(x)) with the difference rounded to fp32,
 * Z = sum of r in ascending id (fp32, sequential); if Z > 0 the token is the
 * first x with u_res * Z < cdf_r(x), falling back to the last x with
 * r(x) > 0; if Z == 0 the token is drawn from p with the a5 rule.  When every
 * draft is accepted and a bonus target row is present, the bonus token is
 * drawn from p_K with the a5 rule and u_res.
 * draft == NULL: greedy drafting (IMPLEMENTATION_PLAN.md:1680), q is one-hot
 * at the draft (q(d_j) = 1, 0 elsewhere; an id outside [0, n) has q = 0): so
 * d_j is accepted iff u_acc < p(d_j), and r = p with r(d_j) = 0. */
static float spec_softmax(const float *logits, int n, float tau, int mode,
                          float *out) {
  memcpy(out, logits, (size_t)n * sizeof(float));
  orc_apply_temperature(out, n, tau, mode);
  return softmax_sum(out, n);
}

void orc_spec_verify(const float *target, const float *draft, int B, int K,
                     int n, int has_bonus, float temperature, int temp_mode,
                     const int32_t *draft_ids, const float *u_acc,
                     const float *u_res, int32_t *acc_len, int32_t *out_ids,
                     float *dist) {
  float *p = (float *)malloc((size_t)n * sizeof(float));
  float *q = (float *)malloc((size_t)n * sizeof(float));
  if (!p || !q) abort();
  const int KT = K + (has_bonus ? 1 : 0);
  for (int b = 0; b < B; b++) {
    int32_t *o = out_ids + (long)b * (K + 1);
    for (int j = 0; j <= K; j++) o[j] = -1;
    float dmin = FLT_MAX;
    int j = 0;
    for (; j < K; j++) {
      const float *T = target + ((long)b * KT + j) * n;
      const float *D = draft ? draft + ((long)b * K + j) * n : NULL;
      int d = draft_ids[(long)b * K + j];
      spec_softmax(T, n, temperature, temp_mode, p);
      if (draft) {
        spec_softmax(D, n, temperature, temp_mode, q);
      } else {
        memset(q, 0, (size_t)n * sizeof(float));
        if (d >= 0 && d < n) q[d] = 1.0f;
      }
      float ua = u_acc[(long)b * K + j];
      int accept = 0;
      if (d >= 0 && d < n && q[d] > 0.0f) {
        float ratio = p[d] / q[d];
        accept = ua < ratio;
        float dd = fabsf(ua - ratio);
        if (dd < dmin) dmin = dd;
      }
      if (accept) { o[j] = d; continue; }
      /* first rejection: residual resample */
      float Z = 0.0f;
      for (int x = 0; x < n; x++) {
        float t = p[x] - q[x];
        q[x] = t > 0.0f ? t : 0.0f;   /* q now holds r(x) */
        Z += q[x];
      }
      int tok;
      if (Z > 0.0f) {
        float r = u_res[b] * Z;
        float cdf = 0.0f, lo = 0.0f;
        tok = -1;
        int last = 0;
        for (int x = 0; x < n; x++) {
          if (q[x] > 0.0f) last = x;
          lo = cdf;
          cdf += q[x];
          if (r < cdf) { tok = x; break; }
        }
        float dd;
        if (tok < 0) { tok = last; dd = r - cdf; }
        else dd = draw_dist(r, lo, cdf);
        if (dd < dmin) dmin = dd;
      } else {
        orc_info inf;
        info_reset(&inf);
        tok = orc_categorical(p, n, u_res[b], &inf);
        if (inf.dist_draw < dmin) dmin = inf.dist_draw;
      }
      o[j] = tok;
      break;
    }
    acc_len[b] = j;
    if (j == K && has_bonus) {
      const float *T = target + ((long)b * KT + K) * n;
      spec_softmax(T, n, temperature, temp_mode, p);
      orc_info inf;
      info_reset(&inf);
      o[K] = orc_categorical(p, n, u_res[b], &inf);
      if (inf.dist_draw < dmin) dmin = inf.dist_draw;
    }
    if (dist) dist[b] = dmin;
  }
  free(p);
  free(q);
}
