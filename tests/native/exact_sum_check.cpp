// Host check of the integer-state emulation of sequential fp32 sums
// (project-zero_amd/csrc/pz_exact.h): every step of pz_acc_add must equal the
// plain fp32 addition s = s + v bit for bit.  Built and run by
// tests/test_exact_sum.py with g++ -ffp-contract=off (SSE fp32 arithmetic).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "pz_exact.h"

static uint64_t rs = 0x12345678abcdefULL;
static uint64_t rnd() {
  rs ^= rs >> 12; rs ^= rs << 25; rs ^= rs >> 27;
  return rs * 0x2545F4914F6CDD1DULL;
}
static double unif() { return (double)(rnd() >> 11) * (1.0 / 9007199254740992.0); }
static float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static long fails = 0, steps = 0;

// Runs one sequence from s = 0; returns false at the first mismatch.
static bool run(const float* v, int n, const char* what) {
  float s = 0.0f;
  PzAcc a = pz_acc_of(0.0f);
  for (int i = 0; i < n; i++) {
    s = s + v[i];
    a = pz_acc_add(a, v[i]);
    steps++;
    if (fbits(pz_acc_value(a)) != fbits(s)) {
      std::printf("MISMATCH %s at %d: v=%a want %a got %a\n", what, i, v[i], s,
                  pz_acc_value(a));
      fails++;
      return false;
    }
  }
  return true;
}

int main() {
  const int N = 200000;
  float* v = (float*)std::malloc(sizeof(float) * N);
  // 1. softmax-like terms: expf(N(0, sigma) - max) over a long row
  for (int rep = 0; rep < 6; rep++) {
    double sigma = 1.0 + rep;
    for (int i = 0; i < N; i++) {
      double u1 = 1.0 - unif(), u2 = unif();
      double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
      v[i] = std::exp((float)(sigma * z) - (float)(5.0 * sigma));
    }
    run(v, N, "softmax-like");
  }
  // 2. descending sorted probabilities (top-p cumulative order)
  for (int i = 0; i < N; i++) v[i] = (float)(0.3 / (1.0 + i) / 12.0);
  run(v, N, "sorted-desc");
  // 3. grid ties: terms that are exactly half a grid step of the running sum
  for (int rep = 0; rep < 20; rep++) {
    float s = 1.0f + (float)unif();
    int n = 0;
    v[n++] = s;
    for (int i = 0; i < 5000; i++) {
      float cur = 0.0f;
      for (int j = 0; j < n; j++) cur = cur + v[j];
      int e;
      std::frexp(cur, &e);
      float half = std::ldexp(1.0f, e - 25);  // half an ulp of cur
      uint64_t r = rnd() % 4;
      v[n++] = r == 0 ? half : (r == 1 ? 3 * half : (r == 2 ? half * 0.5f : half * (float)(rnd() % 64)));
      if (n >= 400) break;
    }
    run(v, n, "ties");
  }
  // 4. subnormal terms and sums, crossing into the normal range
  for (int rep = 0; rep < 20; rep++) {
    for (int i = 0; i < 20000; i++) v[i] = bitsf((uint32_t)(rnd() % 0x400000u) + (rep & 1 ? 0u : 0x800000u * (rnd() % 3)));
    run(v, 20000, "subnormal");
  }
  // 5. zeros, exact powers of two, huge dynamic range
  for (int rep = 0; rep < 50; rep++) {
    for (int i = 0; i < 5000; i++) {
      uint64_t r = rnd() % 5;
      if (r == 0) v[i] = 0.0f;
      else if (r == 1) v[i] = std::ldexp(1.0f, (int)(rnd() % 60) - 40);
      else if (r == 2) v[i] = bitsf((uint32_t)(rnd() % 0x7f000000u));
      else v[i] = (float)unif() * std::ldexp(1.0f, (int)(rnd() % 30) - 20);
    }
    run(v, 5000, "mixed");
  }
  // 6. every pair (s, v) of a grid of edge values
  const uint32_t edges[] = {0u, 1u, 2u, 3u, 0x7fffffu, 0x800000u, 0x800001u, 0xffffffu,
                            0x1000000u, 0x3f000000u, 0x3f7fffffu, 0x3f800000u, 0x3f800001u,
                            0x33800000u, 0x33800001u, 0x337fffffu, 0x34000000u, 0x4b000000u,
                            0x4b7fffffu, 0x4b800000u, 0x7effffffu, 0x3fffffffu, 0x40000000u};
  const int ne = sizeof(edges) / sizeof(edges[0]);
  for (int i = 0; i < ne; i++)
    for (int j = 0; j < ne; j++)
      for (int d = -3; d <= 3; d++) {
        uint32_t sb = edges[i] + (uint32_t)d, vb = edges[j];
        if ((int)edges[i] + d < 0 || (sb >> 23) >= 0xfe) continue;
        float s = bitsf(sb), w = bitsf(vb);
        float want = s + w;
        if (!std::isfinite(want)) continue;
        float got = pz_acc_value(pz_acc_add(pz_acc_of(s), w));
        steps++;
        if (fbits(got) != fbits(want)) {
          std::printf("MISMATCH pair s=%a v=%a want %a got %a\n", s, w, want, got);
          fails++;
        }
      }
  std::printf("exact_sum_check: %ld steps, %ld mismatches\n", steps, fails);
  return fails ? 1 : 0;
}
