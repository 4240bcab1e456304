// pz_specdec.hip -- the speculative decode loop around the device
// verification (pz_spec_decode), with the models and their KV caches
// supplied by the caller.
//
// Reference plan: docs/architecture/IMPLEMENTATION_PLAN.md:1675-1693 (the
// speculative generation loop, 18.2, and kv_cache_rollback, 18.3; neither is
// implemented in the reference).  One round for B sequences, each with its
// last committed token x at position p (the caches hold positions < p):
//   1. draft:  K single-token steps.  Step j forwards x (j = 0) or the draft
//      d_{j-1} at position p + j and gives q_j; d_j is drawn from
//      q_j = softmax(draft_j / tau) with the ascending-id categorical rule
//      of generate.c:157-169, on the device, from the sequence's draft RNG
//      state (pz_sample_step).  A (K+1)-th step forwards d_{K-1} at p + K so
//      the draft cache covers every draft; its logits are not used.
//   2. target: one forward of [x, d_0 .. d_{K-1}] at p .. p+K gives p_0 .. p_K.
//   3. verify: pz_spec_verify with the round's uniforms drawn on the host
//      from the sequence's verification state (K acceptance uniforms, then
//      the residual one; all K+1 are drawn every round).
//   4. commit: the a accepted drafts and the resampled (or bonus) token are
//      appended; both caches are rolled back to p + a + 1 (they keep x and
//      the accepted drafts; the next round forwards the new token there).
// Options (pz_spec_decode_opts):
//   greedy drafts (IMPLEMENTATION_PLAN.md:1680): d_j is the draft model's
//      argmax (argmax.c:3-13, no draw), q is one-hot at d_j in the
//      verification (pz_spec_verify_greedy: accept iff u < p(d_j));
//   EOS stops (generate.c:198-211): the committed tokens are scanned in
//      order and the first id of the sampler's EOS list ends the sequence
//      -- it is not committed, the caches keep what precedes it, and later
//      rounds leave the sequence, its RNG states and its caches as they are.
#include <hip/hip_runtime.h>

#include <string.h>

#include <vector>

#include "../../include/pz_sampler.h"
#include "../../include/pz_sampling_compat.h"
#include "pz_sampler_impl.h"

namespace {

struct DevBuf {
  void* p = nullptr;
  ~DevBuf() { (void)hipFree(p); }
};

}  // namespace

extern "C" int pz_spec_decode_opts(pz_sampler* s, const pz_spec_models* m,
                                   const pz_spec_opts* opts, int B, int K, int V, float tau,
                                   int32_t* tokens, int32_t* len, int max_len, int rounds,
                                   uint64_t* d_draft_state, uint64_t* verify_state,
                                   int32_t* accepted_out, uint8_t* done) {
  if (!s) return PZ_EINVAL;
  const bool greedy = opts && opts->greedy_draft;
  const bool stop_eos = opts && opts->stop_at_eos && s->n_eos > 0;
  if (!m || !m->draft_step || !m->target_forward || !m->kv_rollback || !tokens || !len ||
      !d_draft_state || !verify_state || B < 0 || V <= 0 || rounds < 0)
    return fail(s, PZ_EINVAL, "bad speculative decode arguments");
  if (K < 1 || K > 64) return fail(s, PZ_EINVAL, "K=%d outside [1, 64]", K);
  if (B > s->max_batch) return fail(s, PZ_ERANGE, "B=%d > max_batch=%d", B, s->max_batch);
  if (V > s->max_vocab) return fail(s, PZ_ERANGE, "V=%d > max_vocab=%d", V, s->max_vocab);
  for (int b = 0; b < B; b++) {
    if (len[b] < 1) return fail(s, PZ_EINVAL, "sequence %d is empty", b);
    if ((long)len[b] + (long)rounds * (K + 1) > max_len)
      return fail(s, PZ_ERANGE, "sequence %d would outgrow max_len=%d", b, max_len);
  }
  if (B == 0 || rounds == 0) return PZ_OK;
  PZ_HIP(s, hipSetDevice(s->device));
  const size_t BV = (size_t)B * V;
  DevBuf q, p, junk, tok, ids, tt, ds0;
  if (hipMalloc(&q.p, BV * K * sizeof(float)) != hipSuccess ||
      hipMalloc(&ds0.p, (size_t)B * sizeof(uint64_t)) != hipSuccess ||
      hipMalloc(&p.p, BV * (K + 1) * sizeof(float)) != hipSuccess ||
      hipMalloc(&junk.p, BV * sizeof(float)) != hipSuccess ||
      hipMalloc(&tok.p, (size_t)B * sizeof(int32_t)) != hipSuccess ||
      hipMalloc(&ids.p, (size_t)B * K * sizeof(int32_t)) != hipSuccess ||
      hipMalloc(&tt.p, (size_t)B * (K + 1) * sizeof(int32_t)) != hipSuccess)
    return fail(s, PZ_ENOMEM, "speculative decode buffers");
  float* d_q = static_cast<float*>(q.p);      // [B, K, V] draft logits
  float* d_p = static_cast<float*>(p.p);      // [B, K+1, V] target logits
  int32_t* d_tok = static_cast<int32_t*>(tok.p);
  int32_t* d_ids = static_cast<int32_t*>(ids.p);  // [K, B] drafts
  int32_t* d_tt = static_cast<int32_t*>(tt.p);    // [B, K+1] target tokens
  std::vector<int32_t> h_tok(B), pos0(B), posj(B), h_ids((size_t)K * B), draft_ids((size_t)B * K),
      h_tt((size_t)B * (K + 1)), acc(B), out((size_t)B * (K + 1)), pos_new(B);
  std::vector<float> u_acc((size_t)B * K), u_res(B);
  std::vector<uint8_t> fin(B, 0);  // stopped sequences
  if (done)
    for (int b = 0; b < B; b++) fin[b] = done[b] ? 1 : 0;
  uint64_t* d_ds0 = static_cast<uint64_t*>(ds0.p);
  pz_row_params prm;
  memset(&prm, 0, sizeof(prm));
  prm.temperature = greedy ? 0.0f : tau;  // greedy drafts: argmax, no draw
  prm.top_k = 0;
  prm.top_p = 1.0f;
  prm.rep_penalty = 1.0f;
  void* st = (void*)s->stream;
  for (int r = 0; r < rounds; r++) {
    for (int b = 0; b < B; b++) {
      pos0[b] = len[b] - 1;
      h_tok[b] = tokens[(size_t)b * max_len + len[b] - 1];
    }
    PZ_HIP(s, hipMemcpyAsync(d_tok, h_tok.data(), (size_t)B * sizeof(int32_t),
                             hipMemcpyHostToDevice, s->stream));
    bool any_fin = false;
    for (int b = 0; b < B; b++) any_fin |= fin[b] != 0;
    if (any_fin && !greedy)  // the stopped sequences' draft states, restored after the draws
      PZ_HIP(s, hipMemcpyAsync(d_ds0, d_draft_state, (size_t)B * sizeof(uint64_t),
                               hipMemcpyDeviceToDevice, s->stream));
    // 1. draft steps and their draws
    for (int j = 0; j <= K; j++) {
      for (int b = 0; b < B; b++) posj[b] = pos0[b] + j;
      const int32_t* in = j == 0 ? d_tok : d_ids + (size_t)(j - 1) * B;
      float* out_l = j < K ? d_q + (size_t)j * V : static_cast<float*>(junk.p);
      const long ld = j < K ? (long)K * V : (long)V;
      if (m->draft_step(m->ctx, in, posj.data(), B, out_l, ld, st) != 0)
        return fail(s, PZ_EDEVICE, "draft model step %d of round %d failed", j, r);
      if (j < K) {
        const int rc = pz_sample_step(s, out_l, B, V, ld, &prm, 1, nullptr, 0, d_draft_state,
                                      d_ids + (size_t)j * B, nullptr, nullptr);
        if (rc != PZ_OK) return rc;
      }
    }
    if (any_fin && !greedy)
      for (int b = 0; b < B; b++)
        if (fin[b])
          PZ_HIP(s, hipMemcpyAsync(d_draft_state + b, d_ds0 + b, sizeof(uint64_t),
                                   hipMemcpyDeviceToDevice, s->stream));
    PZ_HIP(s, hipMemcpyAsync(h_ids.data(), d_ids, (size_t)K * B * sizeof(int32_t),
                             hipMemcpyDeviceToHost, s->stream));
    PZ_HIP(s, hipStreamSynchronize(s->stream));
    // 2. the target's forward over [x, d_0 .. d_{K-1}]
    for (int b = 0; b < B; b++) {
      h_tt[(size_t)b * (K + 1)] = h_tok[b];
      for (int j = 0; j < K; j++) {
        const int32_t d = h_ids[(size_t)j * B + b];
        draft_ids[(size_t)b * K + j] = d;
        h_tt[(size_t)b * (K + 1) + 1 + j] = d;
      }
    }
    PZ_HIP(s, hipMemcpyAsync(d_tt, h_tt.data(), (size_t)B * (K + 1) * sizeof(int32_t),
                             hipMemcpyHostToDevice, s->stream));
    if (m->target_forward(m->ctx, d_tt, pos0.data(), B, K + 1, d_p, (long)V, st) != 0)
      return fail(s, PZ_EDEVICE, "target model forward of round %d failed", r);
    // 3. verification
    for (int b = 0; b < B; b++) {
      if (fin[b]) {  // a stopped sequence draws nothing
        for (int j = 0; j < K; j++) u_acc[(size_t)b * K + j] = 0.0f;
        u_res[b] = 0.0f;
        continue;
      }
      unsigned long long vs = verify_state[b];
      for (int j = 0; j < K; j++) u_acc[(size_t)b * K + j] = rng_float(&vs);
      u_res[b] = rng_float(&vs);
      verify_state[b] = vs;
    }
    const int rc =
        greedy ? pz_spec_verify_greedy(s, d_p, B, K, V, (long)V, 1, tau, draft_ids.data(),
                                       u_acc.data(), u_res.data(), acc.data(), out.data())
               : pz_spec_verify(s, d_p, d_q, B, K, V, (long)V, 1, tau, draft_ids.data(),
                                u_acc.data(), u_res.data(), acc.data(), out.data());
    if (rc != PZ_OK) return rc;
    // 4. commit and roll the caches back
    for (int b = 0; b < B; b++) {
      if (fin[b]) {
        pos_new[b] = pos0[b];
        if (accepted_out) accepted_out[(size_t)r * B + b] = -1;
        continue;
      }
      const int a = acc[b];
      int n = a + 1;  // tokens committed: up to the first EOS, which is not
      for (int i = 0; stop_eos && i <= a && n == a + 1; i++) {
        const int32_t t = out[(size_t)b * (K + 1) + i];
        for (int e = 0; e < s->n_eos; e++)
          if (t == s->h_eos[e]) {
            n = i;
            fin[b] = 1;
            break;
          }
      }
      for (int i = 0; i < n; i++)
        tokens[(size_t)b * max_len + len[b] + i] = out[(size_t)b * (K + 1) + i];
      len[b] += n;
      pos_new[b] = pos0[b] + n;
      if (accepted_out) accepted_out[(size_t)r * B + b] = a;
    }
    if (m->kv_rollback(m->ctx, 0, pos_new.data(), B) != 0 ||
        m->kv_rollback(m->ctx, 1, pos_new.data(), B) != 0)
      return fail(s, PZ_EDEVICE, "KV cache rollback of round %d failed", r);
  }
  if (done)
    for (int b = 0; b < B; b++) done[b] = fin[b];
  return PZ_OK;
}

extern "C" int pz_spec_decode(pz_sampler* s, const pz_spec_models* m, int B, int K, int V,
                              float tau, int32_t* tokens, int32_t* len, int max_len, int rounds,
                              uint64_t* d_draft_state, uint64_t* verify_state,
                              int32_t* accepted_out) {
  return pz_spec_decode_opts(s, m, nullptr, B, K, V, tau, tokens, len, max_len, rounds,
                             d_draft_state, verify_state, accepted_out, nullptr);
}
