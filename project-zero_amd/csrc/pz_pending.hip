// pz_pending.hip -- modes whose kernels are not built yet report PZ_ENOTSUP.
#include "pz_launch.h"
#include "../../include/pz_sampler.h"

extern "C" int pz_spec_verify(pz_sampler*, const float*, const float*, int, int, int, long, int,
                              float, const int32_t*, const float*, const float*, int32_t*,
                              int32_t*) {
  return PZ_ENOTSUP;
}
