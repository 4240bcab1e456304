// A toy draft/target model pair with KV caches, for the speculative decode
// loop's tests (never linked into the product library).  Test
// infrastructure: built by tests/native/Makefile, driven by
// tests/test_gpu_specdec.py.
//
// Each model's "cache" of sequence b is a chain of 64-bit prefix hashes:
// hash[0] = seed ^ b, hash[p+1] = mix(hash[p] ^ (token_p + 1) * K1).  The
// forward of token t at position p requires the cache to hold exactly the
// positions < p (else it counts an error), appends t, and produces the
// logits of row seed hash[p+1]:
//   draft   logit[v] = (u24(seed, v) - 2^23) * 2^-21                  in [-4, 4)
//   target  logit[v] = draft logit[v] + ((u24(seed', v) >> 3) - 2^20) * 2^-21
// with u24 the top 24 bits of a 64-bit hash: every value is a multiple of
// 2^-21 below 5 in magnitude, so the fp32 sum is exact on any machine and a
// numpy restatement reproduces the logits bit for bit.  A logit depends on
// the whole cached prefix, so a cache that is not rolled back correctly
// changes every later logit.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <string.h>

#include <vector>

namespace {

constexpr uint64_t K1 = 0x9E3779B97F4A7C15ull;
constexpr uint64_t K2 = 0xD1B54A32D192ED03ull;

__host__ __device__ inline uint64_t mix64(uint64_t z) {
  z ^= z >> 33;
  z *= 0xff51afd7ed558ccdULL;
  z ^= z >> 33;
  z *= 0xc4ceb9fe1a85ec53ULL;
  z ^= z >> 33;
  return z;
}

__global__ void k_toy_logits(const uint64_t* seeds, int rows, int V, float* out, long ld,
                             int target) {
  const int r = blockIdx.y;
  if (r >= rows) return;
  const uint64_t s = seeds[r];
  for (int v = blockIdx.x * blockDim.x + threadIdx.x; v < V; v += gridDim.x * blockDim.x) {
    const int64_t b24 = (int64_t)(mix64(s ^ ((uint64_t)(v + 1) * K1)) >> 40);
    float x = (float)(b24 - (1 << 23)) * 0x1p-21f;
    if (target) {
      const int64_t p21 = (int64_t)(mix64(s ^ ((uint64_t)(v + 1) * K2)) >> 43);
      x = x + (float)(p21 - (1 << 20)) * 0x1p-21f;
    }
    out[(size_t)r * ld + v] = x;
  }
}

struct Toy {
  int B, V, max_len;
  std::vector<uint64_t> h[2];  // [B][max_len + 1]
  std::vector<int> len[2];     // cached positions per sequence
  int errors = 0;
  uint64_t* d_seeds = nullptr;
};

uint64_t& H(Toy* t, int m, int b, int p) { return t->h[m][(size_t)b * (t->max_len + 1) + p]; }

// Appends tokens[b*n + j] at positions pos[b] + j of model m's cache and
// returns the row seeds, or -1 after counting a cache error.
int advance(Toy* t, int m, const int32_t* tok, const int32_t* pos, int B, int n,
            std::vector<uint64_t>& seeds) {
  seeds.assign((size_t)B * n, 0);
  for (int b = 0; b < B; b++) {
    if (pos[b] != t->len[m][b] || pos[b] + n > t->max_len) {
      t->errors++;
      return -1;
    }
    for (int j = 0; j < n; j++) {
      const int p = pos[b] + j;
      H(t, m, b, p + 1) = mix64(H(t, m, b, p) ^ ((uint64_t)(uint32_t)(tok[(size_t)b * n + j] + 1) * K1));
      seeds[(size_t)b * n + j] = H(t, m, b, p + 1);
    }
    t->len[m][b] = pos[b] + n;
  }
  return 0;
}

int forward(Toy* t, int m, const int32_t* d_tokens, const int32_t* pos, int B, int n,
            float* d_logits, long ld, void* stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  std::vector<int32_t> tok((size_t)B * n);
  if (hipMemcpyAsync(tok.data(), d_tokens, tok.size() * sizeof(int32_t), hipMemcpyDeviceToHost,
                     st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess)
    return -1;
  std::vector<uint64_t> seeds;
  if (advance(t, m, tok.data(), pos, B, n, seeds) != 0) return -1;
  if (hipMemcpy(t->d_seeds, seeds.data(), seeds.size() * sizeof(uint64_t),
                hipMemcpyHostToDevice) != hipSuccess)
    return -1;
  // rows: sequence b, token j at d_logits + (b * n + j) * ld for the target;
  // the draft's single token per sequence at d_logits + b * ld
  hipLaunchKernelGGL(k_toy_logits, dim3((t->V + 255) / 256, B * n), dim3(256), 0, st, t->d_seeds,
                     B * n, t->V, d_logits, ld, m);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

extern "C" {

// Caches of both models hold positions < len[b] - 1 of tokens [B, max_len].
void* toy_create(int B, int V, int max_len, uint64_t seed, const int32_t* tokens,
                 const int32_t* len) {
  Toy* t = new Toy();
  t->B = B;
  t->V = V;
  t->max_len = max_len;
  for (int m = 0; m < 2; m++) {
    t->h[m].assign((size_t)B * (max_len + 1), 0);
    t->len[m].assign(B, 0);
    for (int b = 0; b < B; b++) {
      H(t, m, b, 0) = seed ^ (uint64_t)b;
      const int32_t* row = tokens + (size_t)b * max_len;
      for (int p = 0; p + 1 < len[b]; p++)
        H(t, m, b, p + 1) = mix64(H(t, m, b, p) ^ ((uint64_t)(uint32_t)(row[p] + 1) * K1));
      t->len[m][b] = len[b] - 1;
    }
  }
  if (hipMalloc(&t->d_seeds, (size_t)B * 65 * sizeof(uint64_t)) != hipSuccess) {
    delete t;
    return nullptr;
  }
  return t;
}

void toy_destroy(void* ctx) {
  Toy* t = static_cast<Toy*>(ctx);
  if (!t) return;
  (void)hipFree(t->d_seeds);
  delete t;
}

int toy_errors(void* ctx) { return static_cast<Toy*>(ctx)->errors; }

int toy_draft_step(void* ctx, const int32_t* d_tokens, const int32_t* pos, int B, float* d_logits,
                   long ld, void* stream) {
  return forward(static_cast<Toy*>(ctx), 0, d_tokens, pos, B, 1, d_logits, ld, stream);
}

int toy_target_forward(void* ctx, const int32_t* d_tokens, const int32_t* pos, int B, int n,
                       float* d_logits, long ld, void* stream) {
  if (n > 65) return -1;
  return forward(static_cast<Toy*>(ctx), 1, d_tokens, pos, B, n, d_logits, ld, stream);
}

int toy_kv_rollback(void* ctx, int model, const int32_t* pos, int B) {
  Toy* t = static_cast<Toy*>(ctx);
  if (model < 0 || model > 1) return -1;
  for (int b = 0; b < B; b++) {
    if (pos[b] > t->len[model][b] || pos[b] < 0) {
      t->errors++;
      return -1;
    }
    t->len[model][b] = pos[b];
  }
  return 0;
}

}  // extern "C"
