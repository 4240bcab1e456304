// pz_noalloc.hip -- pz_sample_batch_noalloc: the batched sampler without a
// sampler object and without any allocation, for callers that cannot call
// hipMalloc (code under HIP graph capture, serving loops that forbid it).
//
// The device memory the kernels need beyond inputs and outputs -- the row
// parameters, the mode-grouped row list, the top-p fallback's queue counters
// and sort slots, and the workspace of the row-split passes -- lives in one
// file-scope device array, `scratch`, sized for PZ_NOALLOC_MAX_BATCH rows of
// up to PZ_NOALLOC_MAX_VOCAB ids.  Each device holds its own copy for the
// life of the process.  Host code never uses the array's name as an address:
// the device address comes from hipGetSymbolAddress, once per device.
//
// Parameters reach the device as kernel arguments of a staging kernel, by
// value, so a call enqueues kernels only: no host staging buffer, no copy
// command.  Every call on one device shares that device's array; calls that
// overlap on one device race.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string.h>

#include "../../include/pz_sampler.h"
#include "pz_launch.h"
#include "pz_params.h"
#include "pz_sampler_impl.h"

namespace {

constexpr int kFbSlots = 3;       // top-p fallback sort slots (rows sorted at once)
constexpr int kMaxDevices = 64;
constexpr size_t kScratchBytes = (size_t)24 << 20;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct NoallocLayout {
  pz_row_params_dev* params;  // [PZ_NOALLOC_MAX_BATCH]
  int32_t* rows;              // [PZ_NOALLOC_MAX_BATCH] mode-grouped row list
  pz_scratch sc;
  PzSplitWs ws;
};

size_t up256(size_t v) { return (v + 255) & ~(size_t)255; }

// Carves the array at base (a device address); returns the bytes used.
size_t carve(char* base, NoallocLayout* out) {
  size_t off = 0;
  const size_t o_par = off;
  off = up256(off + PZ_NOALLOC_MAX_BATCH * sizeof(pz_row_params_dev));
  const size_t o_rows = off;
  off = up256(off + PZ_NOALLOC_MAX_BATCH * sizeof(int32_t));
  const size_t o_sc = off;
  off = up256(off + pz_scratch_layout(PZ_NOALLOC_MAX_BATCH, PZ_NOALLOC_MAX_VOCAB, kFbSlots,
                                      nullptr, nullptr));
  const size_t o_ws = off;
  off = up256(off + pz_split_ws_layout(PZ_NOALLOC_MAX_BATCH, PZ_NOALLOC_MAX_VOCAB,
                                       PZ_TOPP_CAPG, nullptr, nullptr));
  if (base && out) {
    out->params = reinterpret_cast<pz_row_params_dev*>(base + o_par);
    out->rows = reinterpret_cast<int32_t*>(base + o_rows);
    pz_scratch_layout(PZ_NOALLOC_MAX_BATCH, PZ_NOALLOC_MAX_VOCAB, kFbSlots, base + o_sc,
                      &out->sc);
    pz_split_ws_layout(PZ_NOALLOC_MAX_BATCH, PZ_NOALLOC_MAX_VOCAB, PZ_TOPP_CAPG, base + o_ws,
                       &out->ws);
  }
  return off;
}

struct DeviceState {
  bool ready = false;
  int max_lds = 0;
  int n_cu = 0;
  NoallocLayout lay{};
};

DeviceState g_dev[kMaxDevices];
std::mutex g_mu;

// Set-up on the first call on a device (that device current): the array's
// device address, the LDS limit, and the carved layout.
int device_setup(int device, const DeviceState** out) {
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceState& d = g_dev[device];
  if (!d.ready) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return PZ_EDEVICE;
    if (carve(nullptr, nullptr) > kScratchBytes) return PZ_ENOTSUP;
    if (hipDeviceGetAttribute(&d.max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device) !=
            hipSuccess ||
        hipDeviceGetAttribute(&d.n_cu, hipDeviceAttributeMultiprocessorCount, device) !=
            hipSuccess)
      return PZ_EDEVICE;
    carve(static_cast<char*>(ptr), &d.lay);
    d.ready = true;
  }
  *out = &d;
  return PZ_OK;
}

// One staging launch: up to kStageWords words copied to dst[first..], and
// with zero_counters the fallback's queue counters, the rows' arrival
// counters and the rows' meeting words cleared (they must read zero when a
// launch starts; the kernels re-zero them when they end, but a call
// interrupted before then would leave them set, and the array's first use
// must not depend on its initial contents).
constexpr int kStageWords = 480;
struct StageChunk {
  uint32_t first;
  uint32_t n;
  uint32_t zero_counters;
  uint32_t pad_;
  uint32_t w[kStageWords];
};

__global__ void k_noalloc_stage(StageChunk c, uint32_t* dst, int32_t* counters,
                                uint32_t* arrive, uint64_t* meet, uint32_t n_meet) {
  for (uint32_t i = threadIdx.x; i < c.n; i += blockDim.x) dst[c.first + i] = c.w[i];
  if (c.zero_counters) {
    if (threadIdx.x < PZ_COUNTERS) counters[threadIdx.x] = 0;
    for (uint32_t i = threadIdx.x; i < PZ_NOALLOC_MAX_BATCH; i += blockDim.x) arrive[i] = 0u;
    for (uint32_t i = threadIdx.x; i < n_meet; i += blockDim.x) meet[i] = 0ull;
  }
}

// Copies `words` words from host src to device dst through staging launches.
int stage(const uint32_t* src, uint32_t words, uint32_t* dst, int32_t* counters,
          const PzSplitWs& ws, bool zero, hipStream_t st) {
  const uint32_t n_meet = (uint32_t)(PZ_NOALLOC_MAX_BATCH * 2 * ws.smax);
  StageChunk c;
  c.pad_ = 0;
  uint32_t first = 0;
  do {
    const uint32_t n = words - first < (uint32_t)kStageWords ? words - first : kStageWords;
    c.first = first;
    c.n = n;
    c.zero_counters = zero ? 1u : 0u;
    memcpy(c.w, src + first, n * sizeof(uint32_t));
    hipLaunchKernelGGL(k_noalloc_stage, dim3(1), dim3(256), 0, st, c, dst, counters, ws.arrive,
                       ws.meet, n_meet);
    if (hipGetLastError() != hipSuccess) return PZ_EDEVICE;
    zero = false;
    first += n;
  } while (first < words);
  return PZ_OK;
}

}  // namespace

extern "C" int pz_sample_batch_noalloc(int device, void* stream, int temp_mode,
                                       const float* d_logits, int B, int V, long ld,
                                       const pz_row_params* params, int n_params,
                                       const int32_t* d_hist, int H, const float* d_u,
                                       int32_t* d_ids_out, float* d_p_out) {
  if (device < 0 || device >= kMaxDevices) return PZ_EINVAL;
  if (temp_mode != PZ_TEMP_MUL_RECIP && temp_mode != PZ_TEMP_DIV) return PZ_EINVAL;
  if (!d_logits || !params || !d_ids_out || B < 0 || V <= 0 || ld < V) return PZ_EINVAL;
  if (n_params != 1 && n_params != B) return PZ_EINVAL;
  if (H < 0 || (H > 0 && !d_hist)) return PZ_EINVAL;
  if (B > PZ_NOALLOC_MAX_BATCH || V > PZ_NOALLOC_MAX_VOCAB || H > PZ_NOALLOC_MAX_HIST)
    return PZ_ERANGE;
  if (B == 0) return PZ_OK;
  // the caller's current device is restored on every return
  struct DeviceGuard {
    int prev = -1;
    ~DeviceGuard() {
      if (prev >= 0) (void)hipSetDevice(prev);
    }
  } guard;
  if (hipGetDevice(&guard.prev) != hipSuccess) guard.prev = -1;
  if (hipSetDevice(device) != hipSuccess) return PZ_EDEVICE;
  const DeviceState* ds = nullptr;
  const int rc0 = device_setup(device, &ds);
  if (rc0 != PZ_OK) return rc0;

  // the staged image: parameters in kernel form, then the grouped row list
  struct {
    pz_row_params_dev res[PZ_NOALLOC_MAX_BATCH];
    int32_t rows[PZ_NOALLOC_MAX_BATCH];
  } img;
  static_assert(sizeof(pz_row_params_dev) % 4 == 0, "parameters are staged as words");
  bool pen_any = false, counts_any = false;
  for (int i = 0; i < n_params; i++) {
    img.res[i] = pz_resolve_row(params[i], V, temp_mode);
    if (H > 0 && pz_penalty_active(params[i])) {
      pen_any = true;
      counts_any |= pz_needs_counts(params[i]);
    }
  }
  int count[PZ_MODE_COUNT], offset[PZ_MODE_COUNT], modes_present = 0;
  pz_group_rows(img.res, B, n_params, count, offset, &modes_present);
  if (!d_u) {
    for (int b = 0; b < B; b++)
      if (img.res[n_params == 1 ? 0 : b].mode != PZ_MODE_GREEDY) return PZ_EINVAL;
  }
  const NoallocLayout& lay = ds->lay;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint32_t pwords = (uint32_t)(n_params * sizeof(pz_row_params_dev) / 4);
  int rc = stage(reinterpret_cast<const uint32_t*>(img.res), pwords,
                 reinterpret_cast<uint32_t*>(lay.params), lay.sc.counters, lay.ws, true, st);
  if (rc == PZ_OK && modes_present > 1) {
    pz_fill_rows(img.res, B, n_params, offset, img.rows);
    rc = stage(reinterpret_cast<const uint32_t*>(img.rows), (uint32_t)B,
               reinterpret_cast<uint32_t*>(lay.rows), lay.sc.counters, lay.ws, false, st);
  }
  if (rc != PZ_OK) return rc;

  pz_launch L;
  L.logits = d_logits;
  L.ld = ld;
  L.V = V;
  L.params = lay.params;
  L.n_params = n_params;
  L.hist = H > 0 ? d_hist : nullptr;
  L.H = H;
  L.pen_any = pen_any;
  L.temp_div = temp_mode == PZ_TEMP_DIV;
  L.hcap = pz_hash_capacity(counts_any, H);
  L.u = d_u;
  L.ids = d_ids_out;
  L.p_out = d_p_out;
  L.sc = lay.sc;
  L.ws = lay.ws;
  L.kmax = pz_max_top_k(img.res, B, n_params);
  L.max_lds = ds->max_lds;
  L.n_cu = ds->n_cu;
  L.stream = st;
  int m = -1;
  rc = pz_launch_modes(L, count, offset, modes_present, lay.rows, &m);
  if (rc == -2) return PZ_ENOTSUP;
  return rc == 0 ? PZ_OK : PZ_EDEVICE;
}
