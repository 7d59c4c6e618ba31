// On-box ceilings for bench.py's roofline fractions (not part of the product ABI; built
// into libdeltaattn_diag.so): the bf16 MFMA issue rate of this GPU at the clock it holds
// under a pure MFMA load.
//
// diag_mfma_loop: every wave runs `iters` rounds of 32 v_mfma_f32_32x32x16_bf16 over
// four independent accumulators (a dependency distance of four MFMAs, more than the
// instruction's latency), two waves per SIMD, and writes one float per lane at the end
// so the work is live.  FLOPs = grid * 8 waves * iters * 32 * 32768.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                  0, 0, 0);
}

__global__ __launch_bounds__(512) void mfma_loop_kernel(int iters, float* __restrict__ sink) {
  const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  // small bf16 operands (exponent field 0x3c..) so the accumulators stay finite
  const u32x4 a = {0x3c003c00u + lane, 0x3c013c01u, 0x3c023c02u, 0x3c033c03u + wid};
  const u32x4 b = {0x3c043c04u, 0x3c053c05u + lane, 0x3c063c06u, 0x3c073c07u};
  f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      c0 = mfma(a, b, c0);
      c1 = mfma(b, a, c1);
      c2 = mfma(a, a, c2);
      c3 = mfma(b, b, c3);
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
  sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace

// Launches the loop on `grid` workgroups of 512 threads; sink holds grid * 512 floats.
// Returns 0, or the HIP error code of the launch.
extern "C" int diag_mfma_loop(float* sink, int iters, int grid, void* stream) {
  if (!sink || iters <= 0 || grid <= 0) return -1;
  hipLaunchKernelGGL(mfma_loop_kernel, dim3((unsigned)grid), dim3(512), 0, (hipStream_t)stream, iters, sink);
  return (int)hipGetLastError();
}
