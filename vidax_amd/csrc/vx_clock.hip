// Clock stamps for measurement: each workgroup of a small grid records where
// it ran (its XCD and its hardware id: shader engine, CU, SIMD, wave slot),
// the shader clock counter and the real-time counter. The shader counter is
// read per CU, so two stamps launched on a stream around a run of kernels
// are paired by CU: the shader cycles that passed over the real time that
// passed is the clock the chip held under that load (it moves with board
// power by +-10 %). Not part of the attention path; the attention kernels do
// not use it.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vx_kernels.h"

namespace vx {
namespace {

// hwreg(id, offset 0, size) operands of s_getreg
constexpr int kXccIdReg = 20 | (0 << 6) | ((4 - 1) << 11);  // HW_REG_XCC_ID: the XCD
constexpr int kHwIdReg = 4 | (0 << 6) | ((32 - 1) << 11);   // HW_REG_HW_ID

__global__ __launch_bounds__(64) void clock_stamp_kernel(unsigned long long* out) {
  const uint32_t xcc = __builtin_amdgcn_s_getreg(kXccIdReg);
  const uint32_t hw = __builtin_amdgcn_s_getreg(kHwIdReg);
  const uint64_t cycles = __builtin_amdgcn_s_memtime();
  const uint64_t real = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    unsigned long long* p = out + 4 * blockIdx.x;
    p[0] = xcc;
    p[1] = hw;
    p[2] = cycles;
    p[3] = real;
  }
}

}  // namespace

int launch_clock_stamp(uint64_t* out, int n_groups, void* stream, int* wall_clock_khz) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  e = hipDeviceGetAttribute(wall_clock_khz, hipDeviceAttributeWallClockRate, dev);
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(clock_stamp_kernel, dim3(n_groups), dim3(64), 0, (hipStream_t)stream,
                     (unsigned long long*)out);
  return (int)hipGetLastError();
}

}  // namespace vx
