// pz_topk.hip -- batched top-k sampling, optionally chained with top-p.
//
// Reference semantics (src/sampling/top_k.c:8-73):
//   * selection: the k largest values above -1e30, ties to the lower id,
//     sorted by (value desc, id asc); unfilled slots are (-1e30, -1);
//   * softmax over the k values: e = expf(v - v0), a sequential fp32 sum,
//     p = e / sum (a true division);
//   * draw: first slot with r < cdf (sequential), fallback slot 0.
// Chain (0 < top_p < 1): cut-off, truncated mass and draw of
// src/sampling/top_p.c:79-105 over those k sorted probabilities.
//
// Design (one workgroup per row, BLOCK threads):
//   1. LDS histogram of the order keys of a sample tile -> a lower bound tau
//      on the k-th largest key (the sample's k-th largest lies in a bin whose
//      lower edge is <= the row's k-th largest).
//   2. One streaming pass over the row (128-bit loads; penalties and
//      temperature applied on the fly) appends every (key, id) >= tau to an
//      LDS candidate buffer with one atomic per wave.  If the buffer
//      overflows, the k-th largest (key, id) of the buffer is a tighter lower
//      bound and the row is rescanned (from L2 / Infinity Cache).
//   3. Bitonic sort of the candidates in LDS by (key desc, id asc).
//   4. Wave 0 evaluates the k-slot softmax, cut-off and draw with the exact
//      sequential fp32 sums of the reference (lane-ordered scans).
#include "pz_device.h"
#include "pz_launch.h"
#include "pz_seq.h"
#include "pz_sort.h"

namespace {

constexpr int TOPK_BLOCK = 1024;
constexpr int TOPK_CAP = 4096;      // candidate buffer entries (8 B each)
constexpr int HBINS = 2048;         // 11-bit key digit

struct TopkShared {
  uint32_t hist[HBINS];
  int count;
  int over;
  uint32_t tau_key;
  uint32_t tau_nid;  // composite mode: accept (key, ~id) >= (tau_key, tau_nid)
  int composite;
};

__device__ __forceinline__ uint64_t comp_of(uint32_t key, int id) {
  return ((uint64_t)key << 32) | (uint32_t)(0xffffffffu - (uint32_t)id);
}

__device__ __forceinline__ bool tk_pass(const TopkShared& S, uint32_t key, int id) {
  if (!S.composite) return key >= S.tau_key;
  const uint32_t nid = 0xffffffffu - (uint32_t)id;
  return key > S.tau_key || (key == S.tau_key && nid >= S.tau_nid);
}

// Wave-aggregated append of up to one candidate per lane.
__device__ __forceinline__ void tk_append(TopkShared& S, uint64_t* buf, bool want,
                                          uint64_t comp) {
  const uint64_t ball = __ballot(want);
  if (ball == 0) return;
  const int lane = threadIdx.x & (PZ_WAVE - 1);
  const int n = __popcll(ball);
  const int before = __popcll(ball & ((1ull << lane) - 1ull));
  int base = 0;
  const int leader = __ffsll((long long)ball) - 1;
  if (lane == leader) base = atomicAdd(&S.count, n);
  base = __shfl(base, leader, PZ_WAVE);
  if (want) {
    const int slot = base + before;
    if (slot < TOPK_CAP) buf[slot] = comp;
    else S.over = 1;
  }
}

template <int BLOCK, bool VEC>
__device__ void tk_stream(TopkShared& S, uint64_t* buf, const float* x, int V,
                          const PzPenalty& P, const pz_row_params_dev& prm) {
  const int tid = threadIdx.x;
  if (VEC) {
    const pz_f4* x4 = reinterpret_cast<const pz_f4*>(x);
    const int n4 = V >> 2;
    constexpr int U = 4;
    for (int base = 0; base < n4; base += BLOCK * U) {
      pz_f4 v[U];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int i4 = base + u * BLOCK + tid;
        if (i4 < n4) v[u] = x4[i4];
      }
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int i4 = base + u * BLOCK + tid;
        const bool in = i4 < n4;
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const int i = (i4 << 2) + c;
          bool want = false;
          uint64_t comp = 0;
          if (in) {
            const float y = pz_transform(P, prm, v[u][c], i);
            if (y > -1e30f) {
              const uint32_t key = pz_key(y);
              want = tk_pass(S, key, i);
              comp = comp_of(key, i);
            }
          }
          tk_append(S, buf, want, comp);
        }
      }
    }
    // tail (V not a multiple of 4): at most 3 elements
    const int i = (n4 << 2) + tid;
    bool want = false;
    uint64_t comp = 0;
    if (i < V) {
      const float y = pz_transform(P, prm, x[i], i);
      if (y > -1e30f) {
        const uint32_t key = pz_key(y);
        want = tk_pass(S, key, i);
        comp = comp_of(key, i);
      }
    }
    tk_append(S, buf, want, comp);
  } else {
    for (int base = 0; base < V; base += BLOCK) {
      const int i = base + tid;
      bool want = false;
      uint64_t comp = 0;
      if (i < V) {
        const float y = pz_transform(P, prm, x[i], i);
        if (y > -1e30f) {
          const uint32_t key = pz_key(y);
          want = tk_pass(S, key, i);
          comp = comp_of(key, i);
        }
      }
      tk_append(S, buf, want, comp);
    }
  }
}

template <int BLOCK, bool VEC>
__global__ __launch_bounds__(BLOCK) void k_topk(
    const float* __restrict__ logits, long ld, int V, const int32_t* __restrict__ rows,
    const pz_row_params_dev* __restrict__ params, int n_params,
    const int32_t* __restrict__ hist, int H, int hcap, size_t pen_bytes,
    const float* __restrict__ u, int32_t* __restrict__ ids_out, float* __restrict__ p_out) {
  extern __shared__ __align__(16) char lds[];
  __shared__ TopkShared S;
  const int row = pz_row_of(rows, blockIdx.x);
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const float* x = logits + (long)row * ld;
  const int tid = threadIdx.x;
  const int lane = tid & (PZ_WAVE - 1);
  uint64_t* buf = reinterpret_cast<uint64_t*>(lds + pen_bytes);

  PzPenalty P;
  pz_penalty_build<BLOCK>(P, lds, V, hcap, hist ? hist + (long)row * H : nullptr, H, prm);
  const int k = prm.top_k;

  // ---- 1. sample tile -> lower bound on the k-th key
  for (int j = tid; j < HBINS; j += BLOCK) S.hist[j] = 0;
  if (tid == 0) { S.count = 0; S.over = 0; S.composite = 0; S.tau_nid = 0; }
  __syncthreads();
  const int ns = V < BLOCK * 4 ? V : BLOCK * 4;
  for (int i = tid; i < ns; i += BLOCK) {
    const float y = pz_transform(P, prm, x[i], i);
    if (y > -1e30f) atomicAdd(&S.hist[pz_key(y) >> 21], 1u);
  }
  __syncthreads();
  if (tid < PZ_WAVE) {
    // lane l owns bins [32*l, 32*l+32); suffix counts from the top bin down
    uint32_t own = 0;
    for (int j = 0; j < 32; j++) own += S.hist[32 * lane + j];
    uint32_t above = 0;  // count in lanes > l
    for (int l = PZ_WAVE - 1; l >= 0; l--) {
      const uint32_t o = __shfl(own, l, PZ_WAVE);
      if (l > lane) above += o;
    }
    const uint32_t total = __shfl(above + own, 0, PZ_WAVE);
    uint32_t tau = 0;
    if (total >= (uint32_t)k) {
      // lane whose range holds the k-th largest: above < k <= above + own
      const bool mine = above < (uint32_t)k && above + own >= (uint32_t)k;
      const uint64_t b = __ballot(mine);
      const int l = __ffsll((long long)b) - 1;
      if (lane == l) {
        uint32_t acc = above;
        int bin = 32 * lane + 31;
        for (; bin >= 32 * lane; bin--) {
          acc += S.hist[bin];
          if (acc >= (uint32_t)k) break;
        }
        S.tau_key = (uint32_t)bin << 21;
      }
    } else if (lane == 0) {
      S.tau_key = tau;  // fewer than k valid in the sample: keep every valid value
    }
  }
  __syncthreads();

  // ---- 2. stream the row, rescanning with a tighter bound on overflow
  for (;;) {
    tk_stream<BLOCK, VEC>(S, buf, x, V, P, prm);
    __syncthreads();
    if (!S.over) break;
    // the buffer holds TOPK_CAP >= k candidates of the row: its k-th largest
    // (key, id) bounds the row's k-th largest from below
    pz_bitonic_desc<BLOCK>(buf, TOPK_CAP);
    if (tid == 0) {
      const uint64_t c = buf[k - 1];
      S.tau_key = (uint32_t)(c >> 32);
      S.tau_nid = (uint32_t)c;
      S.composite = 1;
      S.count = 0;
      S.over = 0;
    }
    __syncthreads();
  }

  // ---- 3. sort the candidates
  const int n = S.count;
  int N = 1;
  while (N < n) N <<= 1;
  for (int i = n + tid; i < N; i += BLOCK) buf[i] = 0;  // sentinel below any key
  __syncthreads();
  pz_bitonic_desc<BLOCK>(buf, N);

  // ---- 4. softmax over k slots, cut-off and draw (wave 0).  Lane l owns
  // slots l, l+64, ...: every LDS word of pv is written and read by the same
  // lane, so no cross-lane LDS ordering is needed.
  if (tid < PZ_WAVE) {
    float* pv = reinterpret_cast<float*>(S.hist);  // k <= 1024 probabilities
    const float v0 = n > 0 ? pz_unkey((uint32_t)(buf[0] >> 32)) : -1e30f;
    // e_i = expf(v_i - v0), then the sequential sum
    float sum = 0.0f;
    for (int c0 = 0; c0 < k; c0 += PZ_WAVE) {
      const int i = c0 + lane;
      float e = 0.0f;
      if (i < k) {
        const float v = i < n ? pz_unkey((uint32_t)(buf[i] >> 32)) : -1e30f;
        e = pz_expf(v - v0);
        pv[i] = e;
      }
      sum = pz_seq_sum_lanes(sum, e, k - c0);
    }
    for (int i = lane; i < k; i += PZ_WAVE) pv[i] = pv[i] / sum;
    const float uu = u[row];
    const bool chain = prm.top_p > 0.0f && prm.top_p < 1.0f;
    int cutoff = k;
    float r = uu;
    if (chain) {
      // cumulative (top_p.c:80-88): first slot with cum >= top_p
      float cum = 0.0f;
      int found = -1;
      for (int c0 = 0; c0 < k && found < 0; c0 += PZ_WAVE) {
        const int i = c0 + lane;
        const float p = i < k ? pv[i] : 0.0f;
        const float cs = pz_seq_scan_lanes(cum, p, k - c0);
        const uint64_t hit = __ballot(i < k && cs >= prm.top_p);
        if (hit) {
          const int l = __ffsll((long long)hit) - 1;
          found = c0 + l;
          cum = __shfl(cs, l, PZ_WAVE);
        } else {
          cum = __shfl(cs, PZ_WAVE - 1, PZ_WAVE);
        }
      }
      float trunc_sum = cum;  // sequential sum of the same slots (top_p.c:91-93)
      if (found >= 0) cutoff = found + 1;
      r = uu * trunc_sum;
    }
    // draw: first slot < cutoff with r < cdf, else slot 0
    float cdf = 0.0f;
    int pick = -1;
    float p_pick = 0.0f;
    for (int c0 = 0; c0 < cutoff && pick < 0; c0 += PZ_WAVE) {
      const int i = c0 + lane;
      const float p = i < cutoff ? pv[i] : 0.0f;
      if (c0 == 0) p_pick = __shfl(p, 0, PZ_WAVE);  // fallback slot 0
      const float cs = pz_seq_scan_lanes(cdf, p, cutoff - c0);
      const uint64_t hit = __ballot(i < cutoff && r < cs);
      if (hit) {
        const int l = __ffsll((long long)hit) - 1;
        pick = c0 + l;
        p_pick = __shfl(p, l, PZ_WAVE);
      } else {
        cdf = __shfl(cs, PZ_WAVE - 1, PZ_WAVE);
      }
    }
    if (pick < 0) pick = 0;
    if (lane == 0) {
      const int id = pick < n ? (int)(0xffffffffu - (uint32_t)buf[pick]) : -1;
      ids_out[row] = id;
      if (p_out) p_out[row] = p_pick;
    }
  }
}

}  // namespace

template <bool VEC>
static int launch_topk_t(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  const size_t pen = L.pen_any ? (pz_penalty_lds_bytes(L.V, L.hcap) + 15) & ~(size_t)15 : 0;
  const size_t lds = pen + (size_t)TOPK_CAP * 8;
  if ((int)(lds + sizeof(TopkShared)) > L.max_lds) return -2;
  auto kern = k_topk<TOPK_BLOCK, VEC>;
  if (lds > 65536 &&
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)lds) != hipSuccess)
    return -1;
  hipLaunchKernelGGL(kern, dim3(n_rows), dim3(TOPK_BLOCK), lds, L.stream, L.logits, L.ld, L.V,
                     d_rows, L.params, L.n_params, L.hist, L.H, L.hcap, pen, L.u, L.ids,
                     L.p_out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

int pz_launch_topk(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  if (n_rows <= 0) return 0;
  const bool vec = (L.ld % 4 == 0) && (((uintptr_t)L.logits & 15) == 0);
  return vec ? launch_topk_t<true>(L, n_rows, d_rows) : launch_topk_t<false>(L, n_rows, d_rows);
}
