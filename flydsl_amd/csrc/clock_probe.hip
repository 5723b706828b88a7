// Measurement aid for bench.py (not part of the GEMM ABI): the shader clock while other work
// runs.  One wave reads the core-clock counter (s_memtime) and the constant 100 MHz counter
// (s_memrealtime) before and after spinning until the latter has advanced `ticks`; launched on
// a side stream next to a GEMM, it reports the clock the GEMM runs at.  The spin is bounded by
// an iteration cap as well, so the kernel always ends.
#include <hip/hip_runtime.h>
#include <stdint.h>

__global__ void __launch_bounds__(64) clock_probe_kernel(unsigned long long* out, unsigned long long ticks) {
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  const unsigned long long c0 = __builtin_amdgcn_s_memtime();
  unsigned long long r1 = r0;
  for (int i = 0; i < (1 << 26) && r1 - r0 < ticks; ++i) r1 = __builtin_amdgcn_s_memrealtime();
  const unsigned long long c1 = __builtin_amdgcn_s_memtime();
  if (threadIdx.x == 0) {
    out[0] = c1 - c0;
    out[1] = r1 - r0;
    out[2] = r0;
    out[3] = r1;
  }
}

// out: four device uint64 (core cycles, 100 MHz ticks elapsed, then the 100 MHz counter at the
// start and at the end); ticks: the spin, in 10 ns units.
extern "C" int flygemm_clock_probe(unsigned long long* out, long long ticks, void* stream) {
  if (!out || ticks <= 0 || ticks > 100000000) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(clock_probe_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, out, (unsigned long long)ticks);
  return (int)hipGetLastError();
}
