// lds_poison.hip -- test support for the GPU tests (not part of the product):
// fills the whole LDS of every compute unit with a NaN bit pattern.
//
// LDS keeps the contents of the previous workgroup that ran on a compute
// unit.  A kernel launched right after this one on the same stream that reads
// an LDS location before writing it therefore reads the pattern (NaN as bf16
// pairs and as fp32, a negative int32), which turns its output NaN or moves a
// selected position, so the parity checks see the read-before-write.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kLdsBytes = 160 * 1024;  // the LDS of one gfx950 compute unit
constexpr int kThreads = 1024;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void lds_poison_kernel(uint32_t pattern) {
  __shared__ u32x4 lds[kLdsBytes / 16];
  const u32x4 v = {pattern, pattern, pattern, pattern};
  // ds_write_b128 as asm: stores to LDS that nothing reads would otherwise
  // be dropped by the compiler
  for (int i = threadIdx.x; i < kLdsBytes / 16; i += kThreads) {
    const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) u32x4 *)(lds + i);
    asm volatile("ds_write_b128 %0, %1" ::"v"(a), "v"(v) : "memory");
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

}  // namespace

extern "C" {

// Launches `workgroups` workgroups that each take the whole LDS of a compute
// unit (one at a time per unit) and fill it with `pattern`.  Returns the HIP
// status of the launch.
int lds_poison_fill(uint32_t pattern, int workgroups, void *stream) {
  hipLaunchKernelGGL(lds_poison_kernel, dim3(workgroups), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), pattern);
  return (int)hipGetLastError();
}

}  // extern "C"
