/*
 * pz_sampling_compat.h -- the Project Zero sampler's own C symbols, exported
 * by libpzsample.so so the objects of src/sampling (and the tn_softmax slot)
 * can be replaced at link time.  Same signatures and semantics as the
 * reference; each call copies the host row to the GPU, runs the batch-1 form
 * of the batched kernels and returns the id (or copies the row back).
 *
 * Differences a caller can observe:
 *   - the calls are thread-safe (one device context per host thread), where
 *     the reference's sample_top_p is not (src/sampling/top_p.c:22-28);
 *   - a device failure returns -1 from the id calls (and leaves in-place rows
 *     untouched); pz_compat_last_status() reports it.  The reference cannot
 *     fail.
 * The temperature form is the AVX-512 build's x * (1/T) unless
 * pz_compat_set_temp_mode(PZ_TEMP_DIV) selects the scalar build's x / T
 * (src/sampling/temperature.c:11-23).  PZ_COMPAT_DEVICE picks the GPU.
 */
#ifndef PZ_SAMPLING_COMPAT_H
#define PZ_SAMPLING_COMPAT_H

#include "pz_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

/* include/sampling/sampling.h:12 -- first maximum, ties to the lowest id. */
PZ_API int sample_argmax(const float *logits, int vocab_size);

/* include/sampling/sampling.h:23 -- in place; T < 1e-6 is clamped. */
PZ_API void apply_temperature(float *logits, int vocab_size, float temperature);

/* include/sampling/sampling.h:36-37 -- nucleus sampling; draws one uniform
 * from *rng_state exactly when the reference does. */
PZ_API int sample_top_p(float *logits, int vocab_size, float top_p,
                        unsigned long long *rng_state);

/* include/sampling/sampling.h:49-50 -- top-k sampling (k clamped to
 * [1, min(V, 1024)]); draws one uniform from *rng_state. */
PZ_API int sample_top_k(float *logits, int vocab_size, int k,
                        unsigned long long *rng_state);

/* include/sampling/rng.h:14,21 -- xorshift64* (host arithmetic). */
PZ_API void rng_seed(unsigned long long *state, unsigned long long seed);
PZ_API float rng_float(unsigned long long *state);

/* The tn_softmax slot (include/math/simd_dispatch.h:23,47; typedef
 * void (*tn_softmax_fn)(float *x, int size)): in-place softmax of
 * src/math/softmax.c:4-23.  Assign tn_softmax = pz_tn_softmax after
 * tn_simd_init(). */
PZ_API void pz_tn_softmax(float *x, int size);

/* PZ_TEMP_MUL_RECIP (default) or PZ_TEMP_DIV for this thread's calls. */
PZ_API void pz_compat_set_temp_mode(int mode);

/* PZ_OK or the PZ_E* code of this thread's last call. */
PZ_API int pz_compat_last_status(void);

#ifdef __cplusplus
}
#endif
#endif /* PZ_SAMPLING_COMPAT_H */
