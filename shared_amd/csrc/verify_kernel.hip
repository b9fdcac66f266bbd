// verify_kernel.hip - speculative accept/resample (placeholder until the
// rejection-sampling kernels land; fails loudly).
#include <hip/hip_runtime.h>

#include "shared_amd_sampler.h"

extern "C" int sas_verify(sas_sampler *s, const sas_verify_rows *v, void *stream) {
  (void)s;
  (void)v;
  (void)stream;
  return SAS_ERR_INVALID;
}
