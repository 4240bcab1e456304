// pz_attn.hip -- the reference softmax over attention scores: many short
// rows, one per (sequence, head), each over its valid context.
//
// The call sites (src/transformer/attention.c:210, mla_attention.c:282,
// qwen35_attention.c:156, qwen3moe_attention.c:136) all run
// tn_softmax(att, valid_ctx) per head: softmax.c:4-23, i.e. the maximum by
// strict '>' from x[0], e = expf(x - max), a sequential fp32 sum in index
// order, x *= 1/sum.  Rows of up to 4096 scores take one wave each (four rows
// per 256-thread workgroup): the row sits in the wave's registers, 4
// consecutive scores per lane per 256-score segment, so the maximum, the
// exponentials, the exact sum and the write need no LDS beyond the exp
// table.  The sum is the exact sequential one (pz_exact.h): the first
// segment by serial fp32 adds, every later one through the integer state --
// a segment with at most one binade exit and no tie in one step
// (pz_sp_fast), else one ballot per event over the segment's increment
// prefix, each taken with one exact add (pz_sp_events).  Longer rows use
// the one-workgroup-per-row softmax (pz_softmax.hip).
#include <hip/hip_runtime.h>

#include "../../include/pz_sampler.h"
#include "pz_device.h"
#include "pz_exact.h"
#include "pz_sampler_impl.h"
#include "pz_split.h"

namespace {

constexpr int ATTN_WAVES = 4;               // rows per workgroup
constexpr int ATTN_WAVE_MAX = 16 * 256;     // longest row of the wave kernel

// One 256-term segment added to the running sum st (the whole wave, lane l
// holding terms 4l .. 4l+3): serial fp32 adds from a zero sum, else the
// events of the increment prefixes at the state's binade and the next.  Out
// of line so the unrolled segment loop holds one copy.
__device__ __noinline__ PzAcc attn_seg_sum(PzAcc st, float a, float b, float c, float d) {
  const float v[4] = {a, b, c, d};
  if (st.n == 0u && st.g == 1u) {
    pz_sp_serial<PZ_STOP_NONE>(st, v, 0, 0.0f);
  } else {
    uint32_t P[4], Q[4], fP, fQ;
    const uint32_t g0 = st.g;
    pz_sp_prefix4(v, g0, P, fP);
    pz_sp_prefix4(v, g0 + 1u, Q, fQ);
    if (!pz_sp_fast<PZ_STOP_NONE>(st, v, P, fP, Q, fQ, 0.0f))
      pz_sp_events<PZ_STOP_NONE>(st, v, g0, P, fP, g0 + 1u, Q, fQ, 0.0f);
  }
  pz_sp_uni(st);
  return st;
}

// Row of NSEG segments (256 scores each, lane l: scores 256s + 4l .. +3).
template <int NSEG, bool VEC_IN, bool VEC_OUT>
__global__ __launch_bounds__(64 * ATTN_WAVES) void k_attn_wave(const float* in, long ld_in,
                                                              float* out, long ld_out,
                                                              int n_rows, int n,
                                                              const int32_t* lens) {
  __shared__ uint64_t etab[32];
  pz_etab_fill((pz_lds_u64*)etab);
  __syncthreads();
  const pz_lds_u64* et = (const pz_lds_u64*)etab;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * ATTN_WAVES + (threadIdx.x >> 6);
  if (row >= n_rows) return;  // whole waves
  int len = lens ? lens[row] : n;
  len = len < n ? len : n;
  if (len <= 0) return;  // softmax.c with size 0 writes nothing
  const float* x = in + (size_t)row * ld_in;
  float v[NSEG][4];
  bool nan_seen = false;
  float m = -__builtin_inff();
#pragma unroll
  for (int s = 0; s < NSEG; s++) {
    const int i0 = s * 256 + 4 * lane;
    if (VEC_IN && i0 + 3 < len) {
      const pz_f4 q = *reinterpret_cast<const pz_f4*>(x + i0);
      v[s][0] = q.x;
      v[s][1] = q.y;
      v[s][2] = q.z;
      v[s][3] = q.w;
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++) v[s][c] = i0 + c < len ? x[i0 + c] : -__builtin_inff();
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
      nan_seen |= v[s][c] != v[s][c];
      m = fmaxf(m, v[s][c]);
    }
  }
  // softmax.c:6-9: a NaN anywhere makes the sum NaN (a NaN x[0] is the
  // maximum itself, a later one a NaN term), and so does an infinite
  // maximum (inf - inf, or -inf - -inf); every output is then NaN
  const bool any_nan = __ballot(nan_seen) != 0ull;
  const float M = pz_wave_max(m);
  float* o = out + (size_t)row * ld_out;
  if (any_nan || !(M > -__builtin_inff() && M < __builtin_inff())) {
    for (int i = lane; i < len; i += 64) o[i] = __builtin_nanf("");
    return;
  }
  // terms e = expf(x - M) (glibc's expf, bit for bit); 0 past the row
#pragma unroll
  for (int s = 0; s < NSEG; s++)
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int i = s * 256 + 4 * lane + c;
      v[s][c] = i < len ? pz_expf_tab(v[s][c] - M, et) : 0.0f;
    }
  // the sequential fp32 sum (softmax.c:12-16)
  PzAcc st;
  st.n = 0;
  st.g = 1;
  const int nseg = (len + 255) >> 8;
#pragma unroll
  for (int s = 0; s < NSEG; s++)
    if (s < nseg) st = attn_seg_sum(st, v[s][0], v[s][1], v[s][2], v[s][3]);
  const float inv = 1.0f / pz_acc_value(st);  // softmax.c:19
#pragma unroll
  for (int s = 0; s < NSEG; s++) {
    const int i0 = s * 256 + 4 * lane;
    if (VEC_OUT && i0 + 3 < len) {
      pz_f4 q;
      q.x = v[s][0] * inv;
      q.y = v[s][1] * inv;
      q.z = v[s][2] * inv;
      q.w = v[s][3] * inv;
      *reinterpret_cast<pz_f4*>(o + i0) = q;
    } else {
#pragma unroll
      for (int c = 0; c < 4; c++)
        if (i0 + c < len) o[i0 + c] = v[s][c] * inv;
    }
  }
}

template <int NSEG>
int launch_wave(pz_sampler* s, const float* d_in, long ld_in, float* d_out, long ld_out,
                int n_rows, int n, const int32_t* d_len) {
  const bool vi = (ld_in % 4 == 0) && (((uintptr_t)d_in & 15) == 0);
  const bool vo = (ld_out % 4 == 0) && (((uintptr_t)d_out & 15) == 0);
  auto k = vi ? (vo ? k_attn_wave<NSEG, true, true> : k_attn_wave<NSEG, true, false>)
              : (vo ? k_attn_wave<NSEG, false, true> : k_attn_wave<NSEG, false, false>);
  const int blocks = (n_rows + ATTN_WAVES - 1) / ATTN_WAVES;
  hipLaunchKernelGGL(k, dim3(blocks), dim3(64 * ATTN_WAVES), 0, s->stream, d_in, ld_in, d_out,
                     ld_out, n_rows, n, d_len);
  PZ_HIP(s, hipGetLastError());
  return PZ_OK;
}

}  // namespace

extern "C" int pz_attn_softmax(pz_sampler* s, const float* d_in, long ld_in, float* d_out,
                               long ld_out, int n_rows, int n, const int32_t* d_len) {
  if (!s) return PZ_EINVAL;
  if (!d_in || !d_out || n_rows < 0 || n < 0 || ld_in < n || ld_out < n)
    return fail(s, PZ_EINVAL, "bad attention softmax shape");
  if (n_rows == 0 || n == 0) return PZ_OK;
  PZ_HIP(s, hipSetDevice(s->device));
  if (n > ATTN_WAVE_MAX) {
    PzTemp one;  // scores are softmaxed as they are: x * 1.0f == x
    one.t = 1.0f;
    one.inv = 1.0f;
    one.div = 0;
    return pz_launch_softmax_rows(s, d_in, ld_in, d_out, ld_out, n_rows, n, one, d_len);
  }
  const int nseg = (n + 255) / 256;
  if (nseg <= 1) return launch_wave<1>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len);
  if (nseg <= 2) return launch_wave<2>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len);
  if (nseg <= 4) return launch_wave<4>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len);
  if (nseg <= 8) return launch_wave<8>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len);
  return launch_wave<16>(s, d_in, ld_in, d_out, ld_out, n_rows, n, d_len);
}
