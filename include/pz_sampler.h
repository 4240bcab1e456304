/*
 * pz_sampler.h -- C ABI of libpzsample.so, the MI355X (gfx950) token sampler.
 *
 * Two surfaces:
 *   1. A batched, device-resident API (pz_*): [B, V] fp32 logits stay in HBM,
 *      only int32 ids (and optionally p(chosen)) come back.  This replaces the
 *      per-step hand-off at src/transformer/generate.c:143-174, where
 *      transformer_forward() returns one host row of logits and the sampling
 *      block picks one id.
 *   2. The reference's own sampler symbols (pz_sampling_compat.h), so the
 *      objects of src/sampling can be swapped for this library at link time.
 *
 * Conventions: every pz_* call returns 0 (PZ_OK) or a negative PZ_E* code,
 * mirroring the project's TernaryError convention (include/core/error.h:4-31);
 * no exception or longjmp crosses the ABI.  A pz_sampler owns one HIP stream,
 * its scratch memory and pinned staging buffers; use one per host thread (the
 * reference sampler, by contrast, is non-reentrant: src/sampling/top_p.c:22-28).
 */
#ifndef PZ_SAMPLER_H
#define PZ_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Symbols of the ABI (this header and pz_sampling_compat.h) are the only
 * ones the library exports. */
#ifndef PZ_API
#define PZ_API __attribute__((visibility("default")))
#endif

#define PZ_OK       0
#define PZ_EINVAL  (-1) /* bad argument (NULL pointer, negative size, ...)    */
#define PZ_ENOMEM  (-2) /* device or pinned allocation failed                 */
#define PZ_EDEVICE (-3) /* HIP runtime error (launch, copy, sync)             */
#define PZ_ERANGE  (-4) /* size above what the sampler was created for        */
#define PZ_ENOTSUP (-5) /* request the build does not support                 */

/* Id written for a row whose kernels gave up a bounded wait between the
 * workgroups that share the row (a device that did not run them together);
 * ids are otherwise -1 .. V-1.  The synchronous calls return PZ_EDEVICE. */
#define PZ_ID_FAILED (-2)

/* Temperature forms of src/sampling/temperature.c: the AVX-512 build
 * multiplies by 1.0f/T (:11-20), the scalar build divides by T (:22-23).
 * The default is PZ_TEMP_MUL_RECIP (reference built with -march=native on an
 * AVX-512 host, the case on MI355X servers). */
#define PZ_TEMP_MUL_RECIP 0
#define PZ_TEMP_DIV       1

typedef struct pz_sampler pz_sampler;

/* Per-row sampling parameters.  Dispatch mirrors generate.c:145-169:
 *   temperature <= 0 or < 1e-6          -> greedy argmax (argmax.c:3-13)
 *   else temperature is applied, then
 *     top_k > 0                         -> top-k (top_k.c:8-73), chained with
 *                                          top-p over the k survivors when
 *                                          0 < top_p < 1
 *     else 0 < top_p < 1                -> top-p (top_p.c:30-108)
 *     else                              -> softmax + ascending-id categorical
 *                                          draw (generate.c:157-169)
 * Penalties (absent from the reference; applied before temperature, only to
 * ids of the row's history): repetition x>0 ? x/rep : x*rep once per distinct
 * id (1.0 = off), then x -= (float)count*frequency + presence (0 = off). */
typedef struct {
  float temperature;
  int32_t top_k;
  float top_p;
  float rep_penalty;
  float presence_penalty;
  float frequency_penalty;
} pz_row_params;

/* Creates a sampler on `device` for batches of up to max_batch rows of up to
 * max_vocab logits and histories of up to max_hist ids (max_hist <= 2048). */
PZ_API int pz_sampler_create(pz_sampler **out, int max_batch, int max_vocab,
                      int max_hist, int device);
PZ_API void pz_sampler_destroy(pz_sampler *s);

/* PZ_TEMP_MUL_RECIP or PZ_TEMP_DIV. */
PZ_API int pz_sampler_set_temp_mode(pz_sampler *s, int mode);

/* Bound of every wait between the workgroups that share a row inside one
 * launch, in polls of the awaited word (0 restores the default, 2^22 polls:
 * tenths of a second).  The waits end by themselves on a device that runs a
 * row's workgroups together; one that reaches the bound gives up, every
 * kernel still exits, and the row's id is PZ_ID_FAILED (the synchronous
 * calls return PZ_EDEVICE).  A bound of a few polls makes rows fail on
 * purpose, which tests that path. */
PZ_API int pz_sampler_set_wait_bound(pz_sampler *s, uint32_t polls);

/* Last error message of this sampler ("" when none). */
PZ_API const char *pz_sampler_last_error(const pz_sampler *s);

/* The sampler's hipStream_t (as void*) for callers that order their own work
 * against it. */
PZ_API void *pz_sampler_stream(pz_sampler *s);

/* Samples B rows.  d_logits: device [B, ld] fp32 (ld >= V), caller-owned and
 * not modified.  params: host, n_params = 1 (shared) or B entries.  d_hist:
 * device [B, H] int32 token history (NULL when H == 0); ids outside [0, V)
 * are ignored.  u: host [B] uniforms in [0, 1] (at least B floats are
 * read), one per row, exactly as
 * rng_float() would return them (unused by greedy rows).  ids_out: host [B].
 * p_out: host [B] or NULL, receives p(chosen) in the distribution the draw
 * used (1.0 for greedy).  Synchronous on the sampler's stream. */
PZ_API int pz_sample_batch(pz_sampler *s, const float *d_logits, int B, int V,
                    long ld, const pz_row_params *params, int n_params,
                    const int32_t *d_hist, int H, const float *u,
                    int32_t *ids_out, float *p_out);

/* Asynchronous form: uniforms, ids and p are device pointers ([B] each,
 * d_p_out may be NULL); the work is enqueued on the sampler's stream and the
 * call returns without waiting.  params stay host-side (they select the
 * kernels).  Wait with pz_sampler_sync(). */
PZ_API int pz_sample_batch_async(pz_sampler *s, const float *d_logits, int B, int V,
                          long ld, const pz_row_params *params, int n_params,
                          const int32_t *d_hist, int H, const float *d_u,
                          int32_t *d_ids_out, float *d_p_out);

PZ_API int pz_sampler_sync(pz_sampler *s);

/* One decode step with the RNG and the EOS check on the device, replacing
 * the per-generation state of generate.c:125-126 (rng_seed / rng_float,
 * src/sampling/rng.c:3-17), the sampling block of generate.c:145-169 and the
 * EOS test of generate.c:198-211 for B rows at once.
 *   d_state: device [B] xorshift64* states, one per row, caller-owned and
 *   seeded as rng_seed does (seed 0 becomes 1).  Row b draws
 *   u = rng_float(&d_state[b]) exactly when the reference would: never for a
 *   greedy row, never for a top-p row that returns argmax before drawing
 *   (V > 200000, top_p.c:33-34; a NaN first value after penalties and
 *   temperature, top_p.c:68-69), once for every other row.  The state
 *   advances only when the row draws.
 *   d_eos_out: device [B] uint8 or NULL; 1 when the sampled id is in the
 *   sampler's EOS list (pz_sampler_set_eos), else 0.
 * Other arguments as pz_sample_batch_async.  Asynchronous on the sampler's
 * stream. */
PZ_API int pz_sample_step(pz_sampler *s, const float *d_logits, int B, int V, long ld,
                          const pz_row_params *params, int n_params,
                          const int32_t *d_hist, int H, uint64_t *d_state,
                          int32_t *d_ids_out, float *d_p_out, uint8_t *d_eos_out);

/* The EOS ids pz_sample_step checks (host list, copied; at most PZ_MAX_EOS):
 * the model's eos_token_id when it is > 0 plus the tokenizer's eos_list,
 * as generate.c:201-205 tests them.  Waits for the sampler's stream. */
#define PZ_MAX_EOS 64
PZ_API int pz_sampler_set_eos(pz_sampler *s, const int32_t *eos_ids, int n_eos);

/* Allocation-free form of pz_sample_batch_async.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops that forbid hipMalloc).  It takes no
 * sampler: the kernels' scratch (row parameters, row lists, the top-p
 * workspace) is one static device array per GPU, about 24 MiB, held until the
 * process ends; its address is looked up on the first call on a device.
 * Arguments as pz_sample_batch_async (device pointers for uniforms, ids and
 * p), plus the device, the hipStream_t as void* (NULL: the null stream) and
 * the temperature form (PZ_TEMP_MUL_RECIP or PZ_TEMP_DIV).  Limits:
 * B <= PZ_NOALLOC_MAX_BATCH, V <= PZ_NOALLOC_MAX_VOCAB,
 * H <= PZ_NOALLOC_MAX_HIST (PZ_ERANGE beyond, before anything is enqueued).
 * Every call on one GPU shares that GPU's array, which keeps the last call's
 * contents: calls that overlap on one GPU (other streams, other host threads)
 * race, so order them on one stream.  Errors are reported by return code
 * only.  Asynchronous on `stream`; the caller's current device is left as it
 * was.  A call can be captured into a HIP graph (it enqueues kernels only,
 * no copies or memsets) once a first call on the device has run outside the
 * capture; replays keep the captured arguments. */
#define PZ_NOALLOC_MAX_BATCH 64
#define PZ_NOALLOC_MAX_VOCAB 262144
#define PZ_NOALLOC_MAX_HIST 2048
PZ_API int pz_sample_batch_noalloc(int device, void *stream, int temp_mode,
                                   const float *d_logits, int B, int V, long ld,
                                   const pz_row_params *params, int n_params,
                                   const int32_t *d_hist, int H, const float *d_u,
                                   int32_t *d_ids_out, float *d_p_out);

/* Speculative-draft verification (Leviathan et al. 2023, Alg. 1; absent from
 * the reference, whose plan is docs/architecture/IMPLEMENTATION_PLAN.md:
 * 1664-1693).  For each sequence b and draft position j < K:
 *   p = softmax(target[b,j] / temperature), q = softmax(draft[b,j] / temperature)
 *   (temperature as apply_temperature, softmax as src/math/softmax.c:4-23);
 *   accept draft_ids[b,j] iff u_acc[b,j] < p(d)/q(d) (q(d) == 0 rejects).
 * On the first rejection a token is drawn from r = max(0, p - q) (ascending-id
 * CDF of r, threshold u_res[b] * sum(r)); when sum(r) == 0 it is drawn from p
 * with the categorical rule of generate.c:157-169.  If every draft is accepted
 * and has_bonus, a bonus token is drawn from p of target row K with u_res[b].
 *   1 <= K <= 64 drafts per sequence.
 *   d_target: device [B, K + has_bonus, ld] fp32;  d_draft: device [B, K, ld]
 *   draft_ids, u_acc: host [B, K];  u_res: host [B]
 *   acc_len_out: host [B] accepted count;  ids_out: host [B, K+1] accepted
 *   drafts followed by the resampled / bonus token, -1 pads. */
PZ_API int pz_spec_verify(pz_sampler *s, const float *d_target, const float *d_draft,
                   int B, int K, int V, long ld, int has_bonus,
                   float temperature, const int32_t *draft_ids,
                   const float *u_acc, const float *u_res,
                   int32_t *acc_len_out, int32_t *ids_out);

/* pz_spec_verify with device-resident inputs and outputs, enqueued on the
 * sampler's stream without waiting (a decode loop that keeps everything on
 * the device; the same kernels and results).  d_draft_ids, d_u_acc: device
 * [B, K]; d_u_res: device [B]; d_acc_len_out: device [B]; d_ids_out: device
 * [B, K+1].  The input buffers must stay unchanged until the stream has run
 * the call; calls on one sampler are ordered on its stream. */
PZ_API int pz_spec_verify_async(pz_sampler *s, const float *d_target, const float *d_draft,
                                int B, int K, int V, long ld, int has_bonus,
                                float temperature, const int32_t *d_draft_ids,
                                const float *d_u_acc, const float *d_u_res,
                                int32_t *d_acc_len_out, int32_t *d_ids_out);

/* Verification of greedy drafts (IMPLEMENTATION_PLAN.md:1680: the draft
 * model's argmax, q one-hot at each draft; no draft logits): draft j is
 * accepted iff u_acc < p(d_j), and on the first rejection the residual is p
 * with p(d_j) replaced by 0 (max(0, p - q), fp32); otherwise as
 * pz_spec_verify / pz_spec_verify_async. */
PZ_API int pz_spec_verify_greedy(pz_sampler *s, const float *d_target, int B, int K, int V,
                                 long ld, int has_bonus, float temperature,
                                 const int32_t *draft_ids, const float *u_acc,
                                 const float *u_res, int32_t *acc_len_out, int32_t *ids_out);
PZ_API int pz_spec_verify_greedy_async(pz_sampler *s, const float *d_target, int B, int K,
                                       int V, long ld, int has_bonus, float temperature,
                                       const int32_t *d_draft_ids, const float *d_u_acc,
                                       const float *d_u_res, int32_t *d_acc_len_out,
                                       int32_t *d_ids_out);

/* The models of a speculative decode (docs/architecture/
 * IMPLEMENTATION_PLAN.md:1675-1693), supplied by the caller, who owns their
 * weights and KV caches.  Every call gets the sampler's stream (as void*)
 * and returns 0 on success.
 *   draft_step:     one token per sequence: d_tokens device [B], pos host [B]
 *                   (the position each token takes); writes the draft
 *                   model's logits of row b at d_logits + b * ld (device).
 *   target_forward: n tokens per sequence: d_tokens device [B, n] at
 *                   positions pos[b] .. pos[b] + n - 1; writes logits
 *                   [B, n, V] (row j of sequence b at d_logits + (b*n+j)*ld).
 *   kv_rollback:    kv_cache_rollback (plan 18.3): model 0 (draft) or 1
 *                   (target) keeps, for each sequence b, only the cache
 *                   positions < pos[b] (host [B]); later forwards overwrite
 *                   the rest. */
typedef struct {
  void *ctx;
  int (*draft_step)(void *ctx, const int32_t *d_tokens, const int32_t *pos, int B,
                    float *d_logits, long ld, void *stream);
  int (*target_forward)(void *ctx, const int32_t *d_tokens, const int32_t *pos, int B, int n,
                        float *d_logits, long ld, void *stream);
  int (*kv_rollback)(void *ctx, int model, const int32_t *pos, int B);
} pz_spec_models;

/* The speculative decode loop (plan 18.2) for B sequences, `rounds` rounds.
 * tokens: host [B, max_len], sequence b holding len[b] >= 1 committed tokens
 * (its caches cover positions < len[b] - 1: the last token is the next
 * round's input).  Per round and sequence: K draft steps, each draft drawn
 * on the device from q = softmax(draft / tau) with the categorical rule of
 * generate.c:157-169 and the sequence's draft RNG state (d_draft_state,
 * device [B], as pz_sample_step); one draft step more so the draft cache
 * covers the last draft; one target forward over the input and the K drafts;
 * pz_spec_verify with K + 1 uniforms drawn on the host from the sequence's
 * verification state (verify_state, host [B]: K acceptance uniforms, then
 * the residual one); the accepted drafts and the resampled or bonus token
 * appended to tokens (len[b] grows by accepted + 1); both caches rolled back
 * to the new length - 1.  accepted_out: host [rounds, B] accepted counts, or
 * NULL.  1 <= K <= 64; every sequence must have room for rounds * (K + 1)
 * more tokens.  Synchronous. */
PZ_API int pz_spec_decode(pz_sampler *s, const pz_spec_models *m, int B, int K, int V,
                          float tau, int32_t *tokens, int32_t *len, int max_len, int rounds,
                          uint64_t *d_draft_state, uint64_t *verify_state,
                          int32_t *accepted_out);

/* pz_spec_decode with options (a NULL opts is pz_spec_decode):
 *   greedy_draft: each draft is the draft model's argmax (argmax.c:3-13, no
 *     draw, the draft RNG states stay as they are) and the verification
 *     takes q one-hot at the draft (pz_spec_verify_greedy), as the plan's
 *     greedy drafting (IMPLEMENTATION_PLAN.md:1680).
 *   stop_at_eos: the committed tokens of a round are scanned in order and
 *     the first id of the sampler's EOS list (pz_sampler_set_eos) ends the
 *     sequence as generate.c:198-211 ends generation: the EOS itself is not
 *     committed, both caches keep only what precedes it, and in later rounds
 *     the sequence's tokens, length, RNG states and caches stay as they are
 *     (its accepted count reads -1).
 * done: host [B] flags or NULL; sequences flagged on entry take no part,
 * and a sequence that stops is flagged on return. */
typedef struct {
  int greedy_draft;
  int stop_at_eos;
} pz_spec_opts;
PZ_API int pz_spec_decode_opts(pz_sampler *s, const pz_spec_models *m,
                               const pz_spec_opts *opts, int B, int K, int V, float tau,
                               int32_t *tokens, int32_t *len, int max_len, int rounds,
                               uint64_t *d_draft_state, uint64_t *verify_state,
                               int32_t *accepted_out, uint8_t *done);

/* The reference's temperature (src/sampling/temperature.c:8-25) over device
 * rows [B, ld], in place, on the sampler's stream (asynchronous). */
PZ_API int pz_temperature_batch(pz_sampler *s, float *d_x, long ld, int B, int V,
                                float temperature);

/* The reference's softmax (src/math/softmax.c:4-23, the tn_softmax slot)
 * of temperature-scaled device rows: d_out[b, i] = p_i, bit-identical to
 * the reference (sequential fp32 normaliser).  d_in and d_out may be the same
 * buffer.  Asynchronous on the sampler's stream. */
PZ_API int pz_softmax_batch(pz_sampler *s, const float *d_in, long ld_in, float *d_out,
                            long ld_out, int B, int V, float temperature);

/* The reference softmax (src/math/softmax.c:4-23) over attention scores,
 * the tn_softmax(att, valid_ctx) of src/transformer/attention.c:210,
 * mla_attention.c:282, qwen35_attention.c:156 and qwen3moe_attention.c:136,
 * for many rows at once (one per sequence and head).  Row r of d_in
 * [n_rows, ld_in] holds len_r = min(d_len[r], n) scores (d_len: device
 * int32 [n_rows], or NULL for len_r = n); d_out[r, 0 .. len_r) receives the
 * probabilities, bit-identical to the reference, and entries from len_r on
 * are not written (a row with len_r <= 0 is left alone).  d_in and d_out may
 * be the same buffer.  Rows of up to 4096 scores run one wave each, longer
 * ones one workgroup each.  Asynchronous on the sampler's stream. */
PZ_API int pz_attn_softmax(pz_sampler *s, const float *d_in, long ld_in, float *d_out,
                           long ld_out, int n_rows, int n, const int32_t *d_len);

/* The LM head on the device: the classifier product of
 * src/transformer/forward.c:102-168 as parallel_matmul_bf16 computes it
 * (src/math/parallel_matmul.c:283-414), for B activation rows at once:
 *   d_logits[b, i] = sum_j bf16(d_w[i, j]) * d_x[b, j]
 * d_w: device [V, n] bf16 bit patterns (uint16), row-major as the model's
 * wcls; d_x: device [B, ldx] fp32 final-norm activations; fp32
 * accumulation.  The summation order is not the reference's SIMD order, so
 * logits equal the exact product to fp32 rounding (|error| <= n * 2^-24 *
 * sum_j |w_ij x_bj|), not bit for bit.  B <= max_batch; n * 4 bytes must fit
 * in 96 KiB (n <= 24576).  Asynchronous on the sampler's stream. */
PZ_API int pz_lm_head_bf16(pz_sampler *s, const uint16_t *d_w, int V, int n,
                           const float *d_x, int B, long ldx, float *d_logits, long ld);

/* The same product with greedy sampling (sample_argmax, argmax.c:3-13: the
 * first maximum, a NaN logit 0 giving 0) fused into its epilogue: d_ids[b]
 * is the argmax of exactly the logits pz_lm_head_bf16 writes, and no logits
 * are written.  Asynchronous on the sampler's stream. */
PZ_API int pz_lm_head_argmax_bf16(pz_sampler *s, const uint16_t *d_w, int V, int n,
                                  const float *d_x, int B, long ldx, int32_t *d_ids);

/* Device memory helpers for C hosts (hipMalloc / hipFree / hipMemcpy). */
PZ_API int pz_device_alloc(void **ptr, size_t bytes, int device);
PZ_API int pz_device_free(void *ptr);
PZ_API int pz_memcpy_h2d(void *dst, const void *src, size_t bytes);
PZ_API int pz_memcpy_d2h(void *dst, const void *src, size_t bytes);

#ifdef __cplusplus
}
#endif
#endif /* PZ_SAMPLER_H */
