// Measurement support: the shader clock, read on the device on the caller's stream.
//
// Kernel durations depend on the shader clock the part sustains under load, which differs by a few
// percent from box to box and drifts with temperature and power.  A reading taken right before
// and one right after a timed region bracket the clock that region ran at.  Each reading is made
// inside one wave: the shader-cycle counter (s_memtime) and the 100 MHz real-time counter
// (s_memrealtime) are read, the wave spins until the real-time counter has advanced by
// `spin_ticks`, and both are read again; the clock of that CU is the ratio of the two advances.
// (s_memtime is a per-CU count of the CU's own clocks: it does not advance while the CU is
// clock-gated, and two CUs' counts are unrelated, so a reading never mixes two work-groups.)
// Each work-group records its XCD's id, so the readings can be grouped per XCD.
#include "fa2_common.h"

namespace mi_fa2 {

constexpr int kStampWords = 5;

__global__ __launch_bounds__(64) void clock_stamp_kernel(uint64_t* out, uint32_t spin_ticks) {
  if (threadIdx.x != 0) return;
  uint32_t xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  const uint64_t c0 = __builtin_amdgcn_s_memtime();
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  uint64_t t1 = t0;
  // The real-time counter always advances; the iteration bound only caps the wait should it not.
  for (int i = 0; i < (1 << 22) && t1 - t0 < spin_ticks; ++i) t1 = __builtin_amdgcn_s_memrealtime();
  const uint64_t c1 = __builtin_amdgcn_s_memtime();
  uint64_t* o = out + kStampWords * (uint64_t)blockIdx.x;
  o[0] = c0;
  o[1] = t0;
  o[2] = c1;
  o[3] = t1;
  o[4] = xcc & 0xfu;
}

hipError_t launch_clock_stamp(uint64_t* out, int n_groups, int spin_ticks, hipStream_t stream) {
  hipLaunchKernelGGL(clock_stamp_kernel, dim3(n_groups), dim3(64), 0, stream, out,
                     (uint32_t)spin_ticks);
  return hipGetLastError();
}

}  // namespace mi_fa2
