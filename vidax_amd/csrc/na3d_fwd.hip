// 3D neighbourhood attention forward for gfx950 (placeholder until the
// MFMA kernel lands: reports "not supported" through the C ABI).
#include <hip/hip_runtime.h>

#include "vx_kernels.h"

namespace vx {

int launch_na3d_fwd(const Na3dArgs& a, void* stream) {
  (void)a;
  (void)stream;
  return (int)hipErrorNotSupported;
}

}  // namespace vx
