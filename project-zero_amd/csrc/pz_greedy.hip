// pz_greedy.hip -- batched greedy sampling: virtual penalties + argmax.
//
// Reference semantics: sample_argmax (src/sampling/argmax.c:3-13): the first
// maximum wins (strict '>' scan from x[0]), so ties go to the lowest id and a
// NaN at x[0] returns 0.  Penalties (repetition / presence / frequency) are
// applied on the fly from an LDS bitmap of the row's history; the row in HBM
// is read exactly once with 128-bit non-temporal loads and never written.
//
// Layout: one workgroup per row, BLOCK threads, each thread walks float4
// groups tid, tid+BLOCK, ... in ascending id order, U loads in flight.
#include "pz_device.h"
#include "pz_launch.h"

namespace {

template <int BLOCK, int U, bool VEC>
__global__ __launch_bounds__(BLOCK) void k_greedy(
    const float* __restrict__ logits, long ld, int V,
    const int32_t* __restrict__ rows, const pz_row_params_dev* __restrict__ params,
    int n_params, const int32_t* __restrict__ hist, int H, int hcap,
    int32_t* __restrict__ ids_out, float* __restrict__ p_out) {
  extern __shared__ __align__(16) char lds[];
  __shared__ float red_v[BLOCK / PZ_WAVE];
  __shared__ int red_i[BLOCK / PZ_WAVE];

  const int row = pz_row_of(rows, blockIdx.x);
  const pz_row_params_dev& prm = pz_params_of(params, n_params, row);
  const float* x = logits + (long)row * ld;

  PzPenalty P;
  pz_penalty_build<BLOCK>(P, lds, V, hcap, hist ? hist + (long)row * H : nullptr, H, prm);

  // top-p rows above the reference's vocabulary guard take argmax of the
  // tempered row (top_p.c:33-34, after apply_temperature)
  const bool temper = prm.mode == PZ_MODE_TOPP;
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  const int tid = threadIdx.x;

  if (VEC) {
    const pz_f4* x4 = reinterpret_cast<const pz_f4*>(x);
    const int n4 = V >> 2;
    for (int base = 0; base < n4; base += BLOCK * U) {
      // unconditional loads (clamped to the row's last float4) keep all U
      // in flight; out-of-range groups are skipped below
      pz_f4 v[U];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int i4 = base + u * BLOCK + tid;
        v[u] = __builtin_nontemporal_load(&x4[i4 < n4 ? i4 : n4 - 1]);
      }
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int i4 = base + u * BLOCK + tid;
        if (i4 < n4) {
          const int i = i4 << 2;
          float e0 = v[u].x, e1 = v[u].y, e2 = v[u].z, e3 = v[u].w;
          if (P.active) {
            const uint32_t nib = pz_pen_nibble(P, i);
            if (nib) {
              if (nib & 1u) e0 = pz_penalize(P, e0, i);
              if (nib & 2u) e1 = pz_penalize(P, e1, i + 1);
              if (nib & 4u) e2 = pz_penalize(P, e2, i + 2);
              if (nib & 8u) e3 = pz_penalize(P, e3, i + 3);
            }
          }
          if (temper) {
            e0 = pz_temper(e0, prm);
            e1 = pz_temper(e1, prm);
            e2 = pz_temper(e2, prm);
            e3 = pz_temper(e3, prm);
          }
          if (e0 > bv) { bv = e0; bi = i; }
          if (e1 > bv) { bv = e1; bi = i + 1; }
          if (e2 > bv) { bv = e2; bi = i + 2; }
          if (e3 > bv) { bv = e3; bi = i + 3; }
        }
      }
    }
    for (int i = (n4 << 2) + tid; i < V; i += BLOCK) {
      float e = x[i];
      if (P.active && pz_pen_member(P, i)) e = pz_penalize(P, e, i);
      if (temper) e = pz_temper(e, prm);
      if (e > bv) { bv = e; bi = i; }
    }
  } else {
    for (int i = tid; i < V; i += BLOCK) {
      float e = x[i];
      if (P.active && pz_pen_member(P, i)) e = pz_penalize(P, e, i);
      if (temper) e = pz_temper(e, prm);
      if (e > bv) { bv = e; bi = i; }
    }
  }

  pz_block_argmax<BLOCK>(bv, bi, red_v, red_i);
  if (tid == 0) {
    float x0 = x[0];
    if (P.active && pz_pen_member(P, 0)) x0 = pz_penalize(P, x0, 0);
    if (temper) x0 = pz_temper(x0, prm);
    // argmax.c:4-5 starts from x[0]: a NaN there is never replaced; and if
    // nothing beats -inf the scan also ends on index 0.
    if (x0 != x0 || bi == 0x7fffffff) bi = 0;
    ids_out[row] = bi;
    if (p_out) p_out[row] = 1.0f;
  }
}

}  // namespace

constexpr int GREEDY_BLOCK = 256;
constexpr int GREEDY_U = 8;

int pz_launch_greedy(const pz_launch& L, int n_rows, const int32_t* d_rows) {
  if (n_rows <= 0) return 0;
  const size_t lds = L.pen_any ? pz_penalty_lds_bytes(L.V, L.hcap) : 0;
  const bool vec = (L.ld % 4 == 0) && (((uintptr_t)L.logits & 15) == 0);
  dim3 grid(n_rows), block(GREEDY_BLOCK);
  if (vec)
    hipLaunchKernelGGL((k_greedy<GREEDY_BLOCK, GREEDY_U, true>), grid, block, lds, L.stream,
                       L.logits, L.ld, L.V, d_rows, L.params, L.n_params, L.hist, L.H,
                       L.hcap, L.ids, L.p_out);
  else
    hipLaunchKernelGGL((k_greedy<GREEDY_BLOCK, GREEDY_U, false>), grid, block, lds, L.stream,
                       L.logits, L.ld, L.V, d_rows, L.params, L.n_params, L.hist, L.H,
                       L.hcap, L.ids, L.p_out);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

size_t pz_greedy_lds_bytes(int V, int hcap) { return pz_penalty_lds_bytes(V, hcap); }
