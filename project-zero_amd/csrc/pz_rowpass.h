// pz_rowpass.h -- streaming passes of one 1024-thread workgroup over one
// logits row, shared by the kernels whose normaliser is a full-row sequential
// fp32 sum (top-p, plain categorical, speculative verification).
//
// Layout: the row is walked in tiles of 4096 elements, one 128-bit load per
// thread per tile; thread t of a tile holds elements 4t..4t+3.  A segment is
// one wave's 256-element slice of a tile (segment k = tile*16 + wave), the
// unit at which the exact-sum walk (pz_exact.h) keeps integer records.
#pragma once
#include "pz_device.h"
#include "pz_exact.h"

constexpr int PZ_RB = 1024;           // threads per row workgroup
constexpr int PZ_TILE = PZ_RB * 4;    // elements per tile
constexpr int PZ_SEG = 256;           // elements per segment
constexpr int PZ_SEGS_PER_TILE = PZ_RB / 64;

__host__ __device__ inline int pz_tiles(int V) { return (V + PZ_TILE - 1) / PZ_TILE; }
__host__ __device__ inline int pz_nseg(int V) { return pz_tiles(V) * PZ_SEGS_PER_TILE; }

// First element of this thread's 4 in tile t, and of this lane's 4 in segment k.
__device__ __forceinline__ int pz_tile_e0(int t) { return t * PZ_TILE + 4 * (int)threadIdx.x; }
__device__ __forceinline__ int pz_seg_e0(int k) {
  return (k >> 4) * PZ_TILE + (k & 15) * PZ_SEG + 4 * ((int)threadIdx.x & 63);
}

// Raw logits of elements e0..e0+3 (e0 a multiple of 4); entries at or past V
// read as 0.  Returns how many are < V.
template <bool VEC, bool NT>
__device__ __forceinline__ int pz_load4(const float* __restrict__ x, int V, int e0, float (&r)[4]) {
  if (VEC && e0 + 3 < V) {
    const pz_f4* p = reinterpret_cast<const pz_f4*>(x + e0);
    const pz_f4 v = NT ? __builtin_nontemporal_load(p) : *p;
    r[0] = v.x;
    r[1] = v.y;
    r[2] = v.z;
    r[3] = v.w;
    return 4;
  }
  int n = 0;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    r[c] = 0.0f;
    if (e0 + c < V) {
      r[c] = x[e0 + c];
      n++;
    }
  }
  return n;
}

// One row as the sampling chain sees it: y_i = temperature(penalties(x_i)).
template <bool VEC>
struct PzRow {
  const float* x;
  int V;
  PzPenalty P;
  const pz_row_params_dev* prm;

  __device__ __forceinline__ int get(int e0, float (&y)[4]) const {
    const int n = pz_load4<VEC, false>(x, V, e0, y);
#pragma unroll
    for (int c = 0; c < 4; c++)
      if (c < n) y[c] = pz_transform(P, *prm, y[c], e0 + c);
    return n;
  }
};

// A plain row scaled by temperature only (speculative verification).
template <bool VEC>
struct PzTempRow {
  const float* x;
  int V;
  const pz_row_params_dev* prm;

  __device__ __forceinline__ int get(int e0, float (&y)[4]) const {
    const int n = pz_load4<VEC, false>(x, V, e0, y);
#pragma unroll
    for (int c = 0; c < 4; c++)
      if (c < n) y[c] = pz_temper(y[c], *prm);
    return n;
  }
};

struct PzPass1Shared {
  float red[PZ_RB / 64];
  int any_nan;
  float y0;
};

// Pass 1 (the one compulsory HBM read of the row): the row maximum (NaN
// ignored, as the reference's strict '>' scans do), whether any y is NaN,
// y[0], and per segment k an estimate seg_m[k] = max, seg_s[k] =
// sum exp(y - seg_m[k]) (hardware exp: estimates only, used to predict the
// binade of the running sum).  Returns the maximum in every thread.
template <int U, class Row>
__device__ __forceinline__ float pz_pass1(const Row& row, int ntiles, float* seg_m, float* seg_s,
                          PzPass1Shared& S) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  if (tid == 0) S.any_nan = 0;
  float tmax = -__builtin_inff();
  bool nan = false;
  for (int t0 = 0; t0 < ntiles; t0 += U) {
    float r[U][4];
    int nv[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      nv[u] = 0;
      if (t0 + u < ntiles) nv[u] = row.get(pz_tile_e0(t0 + u), r[u]);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int t = t0 + u;
      if (t >= ntiles) continue;
      float lm = -__builtin_inff();
#pragma unroll
      for (int c = 0; c < 4; c++) {
        if (c >= nv[u]) continue;
        const float y = r[u][c];
        if (y != y) nan = true;
        else lm = fmaxf(lm, y);
      }
      if (t == 0 && tid == 0) S.y0 = r[u][0];
      tmax = fmaxf(tmax, lm);
      const float sm = pz_wave_max(lm);
      float s = 0.0f;
      if (sm > -__builtin_inff() && sm < __builtin_inff()) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const float y = r[u][c];
          if (c < nv[u] && y > -__builtin_inff()) s += __expf(y - sm);
        }
      }
      s = pz_wave_sum(s);
      if (lane == 0) {
        seg_m[t * PZ_SEGS_PER_TILE + w] = sm;
        seg_s[t * PZ_SEGS_PER_TILE + w] = s;
      }
    }
  }
  tmax = pz_wave_max(tmax);
  if (__ballot(nan) && lane == 0) S.any_nan = 1;
  if (lane == 0) S.red[w] = tmax;
  __syncthreads();
  float M = S.red[0];
#pragma unroll
  for (int i = 1; i < PZ_RB / 64; i++) M = fmaxf(M, S.red[i]);
  return M;
}

// Sentinel grid of a segment that has no record (the walk regenerates it).
constexpr uint32_t PZ_NO_RECORD = 0xffffffffu;

// One wave: grid exponent of the estimated running sum at the start of each
// segment, where segment k adds about scale * seg_s[k] * exp(seg_m[k] - M).
// Segments whose estimated start exceeds `limit` get PZ_NO_RECORD.  Writes
// seg_gf[k]; returns the last segment at or below the limit (-1 if none).
__device__ __forceinline__ int pz_predict_grids(const float* seg_m, const float* seg_s,
                                                int nseg, float M, float scale,
                                                uint32_t* seg_gf,
                                                float limit = __builtin_inff()) {
  const int lane = threadIdx.x & 63;
  float carry = 0.0f;
  int kmax = -1;
  for (int k0 = 0; k0 < nseg; k0 += 64) {
    const int k = k0 + lane;
    float a = 0.0f;
    if (k < nseg) {
      const float m = seg_m[k];
      if (m > -__builtin_inff()) a = seg_s[k] * __expf(m - M) * scale;
    }
    const float incl = pz_wave_scan_f32(a);
    const float start = carry + (incl - a);
    const bool in = k < nseg && start <= limit;
    if (k < nseg) seg_gf[k] = in ? pz_grid_of(start) : PZ_NO_RECORD;
    const uint64_t ball = __ballot(in);
    if (ball) kmax = k0 + 63 - (int)__builtin_clzll(ball);
    carry += pz_readlane_f32(incl, 63);
  }
  return kmax;
}

struct PzDrawShared {
  float sum;
  int kmax;
  int hit;
};

// Exact term of element i of a row: e = expf(y - M) for y >= thr (0
// otherwise), times inv when as_p.
template <class Row>
struct PzTermRegen {
  Row R;
  float M, thr, inv;
  bool as_p;
  __device__ __forceinline__ void operator()(int k, float (&v)[4]) const {
    float yy[4];
    const int n = R.get(pz_seg_e0(k), yy);
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float e = (c < n && yy[c] >= thr) ? pz_expf(yy[c] - M) : 0.0f;
      v[c] = as_p ? e * inv : e;
    }
  }
};

// Records pass over tiles [0, tmax]: the exact terms of every segment whose
// seg_gf holds a predicted grid are recorded at that grid.
template <int U2, class Row>
__device__ __forceinline__ void pz_record_terms(const PzTermRegen<Row>& G, int tmax,
                                                uint32_t* seg_d, uint32_t* seg_gf) {
  const int w = threadIdx.x >> 6;
  for (int t0 = 0; t0 <= tmax; t0 += U2) {
    float y[U2][4];
    int nv[U2];
#pragma unroll
    for (int uu = 0; uu < U2; uu++) {
      nv[uu] = 0;
      if (t0 + uu <= tmax) nv[uu] = G.R.get(pz_tile_e0(t0 + uu), y[uu]);
    }
#pragma unroll
    for (int uu = 0; uu < U2; uu++) {
      const int t = t0 + uu;
      if (t > tmax) continue;
      const int k = t * PZ_SEGS_PER_TILE + w;
      const uint32_t g = seg_gf[k];
      if (g == PZ_NO_RECORD) continue;
      float v[4];
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float e = (c < nv[uu] && y[uu][c] >= G.thr) ? pz_expf(y[uu][c] - G.M) : 0.0f;
        v[c] = G.as_p ? e * G.inv : e;
      }
      pz_segment_record(v, g, true, seg_d, seg_gf, k);
    }
  }
}

// The reference's softmax normaliser (softmax.c:12-16; top_p.c:57-65 with
// thr = max - 20): exact sequential fp32 sum of expf(y - M) over y >= thr in
// ascending id.  seg_m/seg_s hold the row's pass-1 estimates.  Called by
// every thread; returns the sum in every thread.
template <int U2, class Row>
__device__ __forceinline__ float pz_exact_normaliser(const Row& R, int ntiles, float M, float thr,
                                                     const float* seg_m, const float* seg_s,
                                                     uint32_t* seg_d, uint32_t* seg_gf,
                                                     PzDrawShared& S) {
  const int nseg = ntiles * PZ_SEGS_PER_TILE;
  if (threadIdx.x < 64) pz_predict_grids(seg_m, seg_s, nseg, M, 1.0f, seg_gf);
  __syncthreads();
  PzTermRegen<Row> G{R, M, thr, 0.0f, false};
  pz_record_terms<U2>(G, ntiles - 1, seg_d, seg_gf);
  __syncthreads();
  if (threadIdx.x < 64) {
    PzAcc st;
    st.n = 0;
    st.g = 1;
    pz_wave_walk(st, seg_d, seg_gf, nseg, 0.0f, PZ_STOP_NONE, G);
    if (threadIdx.x == 0) S.sum = pz_acc_value(st);
  }
  __syncthreads();
  return S.sum;
}

// The reference's categorical draw (generate.c:162-168): cdf += p_i with
// p_i = expf(y_i - M) * inv in ascending id, the first i with r < cdf.
// Records are made only for the segments the estimated CDF can reach.
// Called by every thread; returns the index or -1 (no hit) in every thread.
template <int U2, class Row>
__device__ __forceinline__ int pz_exact_cdf_draw(const Row& R, int V, int ntiles, float M,
                                                 float inv, float r, const float* seg_m,
                                                 const float* seg_s, uint32_t* seg_d,
                                                 uint32_t* seg_gf, PzDrawShared& S) {
  const int nseg = ntiles * PZ_SEGS_PER_TILE;
  if (threadIdx.x < 64) {
    const int kmax = pz_predict_grids(seg_m, seg_s, nseg, M, inv, seg_gf, r + 0.01f);
    if (threadIdx.x == 0) S.kmax = kmax;
  }
  __syncthreads();
  const int kmax = S.kmax;
  PzTermRegen<Row> G{R, M, -__builtin_inff(), inv, true};
  pz_record_terms<U2>(G, kmax < 0 ? -1 : kmax / PZ_SEGS_PER_TILE, seg_d, seg_gf);
  __syncthreads();
  if (threadIdx.x < 64) {
    PzAcc st;
    st.n = 0;
    st.g = 1;
    int hit = pz_wave_walk(st, seg_d, seg_gf, nseg, r, PZ_STOP_GT, G);
    if (hit >= V) hit = -1;  // padding terms are 0 and never raise the CDF
    if (threadIdx.x == 0) S.hit = hit;
  }
  __syncthreads();
  return S.hit;
}
