/*
 * pz_oracle.h -- CPU oracle for the token-sampling path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain C99 restatement of the Project
 * Zero reference sampler (src/sampling/ *.c, src/math/softmax.c and the
 * sampling block of src/transformer/generate.c:145-169) plus the
 * build-defined extensions the reference lacks (penalties, the top-k -> top-p
 * chain, speculative verification).  Only tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py may load it, and only as the checker or
 * the timed CPU baseline.  The product (libpzsample.so) never calls it.
 *
 * Every sum is taken sequentially in fp32 in the order the reference uses,
 * and every exponential goes through the host libm expf, exactly like the
 * reference.  Each function names the reference lines it follows.
 *
 * Parity pins (what checks each function; tests/test_oracle_golden.py,
 * tests/test_oracle_extensions.py):
 *   orc_rng_*            golden sequences from the compiled reference (FIX),
 *                        closed form of xorshift64* (CF)
 *   orc_argmax           reference KATs (tests/test_sampling.c:76-104) +
 *                        compiled reference (KAT, FIX)
 *   orc_apply_temperature compiled reference, both forms (FIX)
 *   orc_softmax          compiled reference softmax.c (FIX) + reference
 *                        KATs (test_math.c:70-88, audit_math.c:19-33)
 *   orc_categorical      hand-computed CDF cases incl. the V-1 fallback (CF)
 *                        + draw frequencies vs float64 probabilities (INV)
 *   orc_top_k            compiled reference top_k.c (FIX) + reference tests
 *   orc_top_p            compiled reference top_p.c (FIX) + reference tests
 *   orc_penalties        hand-computed exact cases (CF) + a np.bincount
 *                        formulation on random histories (BF)
 *   orc_chain            equals orc_top_k outside (0,1) (INV) + float64
 *                        model away from rounding boundaries (BF)
 *   orc_spec_verify      draft == target accepts all (CF), rejected drafts
 *                        never resampled (INV), emitted token distributed as
 *                        the target softmax (INV, simulation)
 */
#ifndef PZ_ORACLE_H
#define PZ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- a1: RNG (src/sampling/rng.c:3-17) -------------------------------- */
void  orc_rng_seed(unsigned long long *state, unsigned long long seed);
float orc_rng_float(unsigned long long *state);

/* ---- a2: greedy (src/sampling/argmax.c:3-13) --------------------------- */
int orc_argmax(const float *x, int n);

/* ---- a3: temperature (src/sampling/temperature.c:8-25) ----------------- */
#define ORC_TEMP_MUL_RECIP 0 /* AVX-512 build: x *= 1.0f/T  (:11-20) */
#define ORC_TEMP_DIV       1 /* scalar build:  x /= T       (:22-23) */
void orc_apply_temperature(float *x, int n, float temperature, int mode);

/* ---- a4: stable softmax (src/math/softmax.c:4-23) ---------------------- */
void orc_softmax(float *x, int n);

/* Draw diagnostics shared by every sampler below.  dist_draw is the distance
 * of the draw r from the nearer CDF partial sum around the chosen slot;
 * dist_cut (top-p only) is the distance of the cumulative mass at and just
 * before the cut-off from top_p.  Both are FLT_MAX when not applicable. */
typedef struct {
  float p_chosen;   /* probability of the chosen token in the draw distribution */
  float dist_draw;
  float dist_cut;
  int   cutoff;     /* top-p: number of tokens kept; top-k: k after clamping */
  int   n_cand;     /* top-p: candidates after the max-20 filter */
  float trunc_sum;  /* top-p / chain: truncated mass */
  float norm_sum;   /* softmax / top-p: the sequential normaliser */
  int   path;       /* ORC_PATH_* actually taken */
} orc_info;

#define ORC_PATH_ARGMAX      0
#define ORC_PATH_CATEGORICAL 1
#define ORC_PATH_TOPK        2
#define ORC_PATH_TOPP        3
#define ORC_PATH_CHAIN       4
#define ORC_PATH_TOPP_ARGMAX 5 /* top-p fell back to argmax (V>200000 or n==0) */

/* ---- a5: inline categorical draw (src/transformer/generate.c:157-169) -- */
int orc_categorical(const float *probs, int n, float r, orc_info *info);

/* ---- a6: top-k (src/sampling/top_k.c:8-73), uniform passed in --------- */
int orc_top_k(const float *x, int n, int k, float u, orc_info *info);

/* ---- a7: top-p (src/sampling/top_p.c:30-108), uniform passed in ------- */
int orc_top_p(const float *x, int n, float top_p, float u, orc_info *info);

/* ---- a8/a9: penalties (build-defined; absent from the reference) ------- */
void orc_penalties(float *x, int n, const int32_t *hist, int h,
                   float rep, float pres, float freq);

/* ---- a10: top-k -> top-p chain (build-defined) ------------------------- */
int orc_chain(const float *x, int n, int k, float top_p, float u, orc_info *info);

/* ---- per-row dispatch: generate.c:145-169 extended with a8-a10 -------- */
typedef struct {
  float temperature;
  int   top_k;
  float top_p;
  float rep_penalty;
  float presence_penalty;
  float frequency_penalty;
} orc_params;

/* Samples one row.  x is copied (the row is not modified). */
int orc_sample_row(const float *x, int n, const orc_params *prm,
                   const int32_t *hist, int h, float u, int temp_mode,
                   orc_info *info);

/* Batched driver over [rows, n] with leading dimension ld.  params has
 * n_params entries (1 = shared by every row).  hist is [rows, h] or NULL.
 * Outputs ids[rows] and, when non-NULL, p_chosen/dist_draw/dist_cut[rows]. */
void orc_sample_batch(const float *x, int rows, int n, long ld,
                      const orc_params *params, int n_params,
                      const int32_t *hist, int h, const float *u, int temp_mode,
                      int32_t *ids, float *p_chosen, float *dist_draw,
                      float *dist_cut);

/* One decode step with per-row RNG states and the EOS check
 * (generate.c:125-126 state, :145-169 dispatch, :198-211 EOS).  Row b draws
 * orc_rng_float(&state[b]) only where the reference's sampler consumes a
 * uniform: not for argmax (:151-152), not when top-p returns argmax first
 * (top_p.c:33-34, 68-69); once otherwise (top_k.c:62, top_p.c:96,
 * generate.c:159).  eos_flag[b] = ids[b] is in eos[0..n_eos). */
void orc_sample_step(const float *x, int rows, int n, long ld,
                     const orc_params *params, int n_params,
                     const int32_t *hist, int h, unsigned long long *state,
                     int temp_mode, const int32_t *eos, int n_eos,
                     int32_t *ids, uint8_t *eos_flag, int32_t *drew);

/* ---- a11: speculative verification (build-defined) ---------------------
 * target [B, K+has_bonus, n], draft [B, K, n] logits; draft_ids [B, K];
 * u_acc [B, K]; u_res [B].  draft == NULL: greedy drafts, q one-hot at each
 * draft id (accept iff u < p(d); residual max(0, p - [i == d])).
 * Outputs acc_len[B] and out_ids[B, K+1]
 * (accepted drafts, then the resampled or bonus token; -1 pads).
 * dist[B] receives the minimum boundary distance over the tests taken. */
void orc_spec_verify(const float *target, const float *draft, int B, int K,
                     int n, int has_bonus, float temperature, int temp_mode,
                     const int32_t *draft_ids, const float *u_acc,
                     const float *u_res, int32_t *acc_len, int32_t *out_ids,
                     float *dist);

/* Exposed for the expf-agreement tests. */
float orc_expf(float x);
uint64_t orc_expf_hash(uint32_t lo_bits, uint32_t hi_bits, uint32_t stride);

#ifdef __cplusplus
}
#endif
#endif /* PZ_ORACLE_H */
