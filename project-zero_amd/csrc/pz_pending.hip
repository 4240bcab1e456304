// pz_pending.hip -- modes whose kernels are not built yet report PZ_ENOTSUP.
#include "pz_launch.h"
#include "../../include/pz_sampler.h"

int pz_launch_categorical(const pz_launch&, int, const int32_t*) { return -2; }
extern "C" int pz_spec_verify(pz_sampler*, const float*, const float*, int, int, int, long, int,
                              float, const int32_t*, const float*, const float*, int32_t*,
                              int32_t*) {
  return PZ_ENOTSUP;
}
