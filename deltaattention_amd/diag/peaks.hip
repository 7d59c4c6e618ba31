// On-box ceilings for bench.py's roofline fractions (not part of the product ABI; built
// into libdeltaattn_diag.so): the bf16 MFMA issue rate of this GPU, with constant operands
// and with random ones, and the shader clock it holds meanwhile.
//
// diag_mfma_loop: every wave runs `iters` rounds of 32 v_mfma_f32_32x32x16_bf16 over four
// independent accumulators (a dependency distance of four MFMAs, more than the
// instruction's latency) and eight operand registers combined in 16 (A, B) pairs, two
// waves per SIMD, and writes one float per lane at the end so the work is live.
// FLOPs = grid * 8 waves * iters * 32 * 32768.
//
// The operands decide the clock: the chip's power limit lowers the shader clock as the
// multiplier arrays switch more.  With `operands` null every lane multiplies the same few
// constants (little switching: the clock stays near its maximum); otherwise each lane
// loads eight random 16-byte operands from `operands` (kDiagOperandU32x4 entries of
// 16 bytes), which is what attention's data does to the arrays.
//
// clocks (optional, grid * 4 entries): per workgroup, s_memtime (shader clock cycles) and
// s_memrealtime (100 MHz) at the start and at the end of wave 0.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kOperandSets = 64;  // workgroup i reads set i % 64

__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                  0, 0, 0);
}

__global__ __launch_bounds__(512) void mfma_loop_kernel(int iters, const u32x4* __restrict__ src,
                                                        float* __restrict__ sink,
                                                        unsigned long long* __restrict__ clocks) {
  const uint32_t lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  u32x4 a0, a1, a2, a3, b0, b1, b2, b3;
  if (src) {
    const u32x4* p = src + ((size_t)(blockIdx.x % kOperandSets) * 512 + threadIdx.x) * 8;
    a0 = p[0], a1 = p[1], a2 = p[2], a3 = p[3], b0 = p[4], b1 = p[5], b2 = p[6], b3 = p[7];
  } else {
    // small bf16 operands (exponent field 0x3c..) so the accumulators stay finite
    a0 = a1 = a2 = a3 = u32x4{0x3c003c00u + lane, 0x3c013c01u, 0x3c023c02u, 0x3c033c03u + wid};
    b0 = b1 = b2 = b3 = u32x4{0x3c043c04u, 0x3c053c05u + lane, 0x3c063c06u, 0x3c073c07u};
  }
  f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      c0 = mfma(a0, b0, c0), c1 = mfma(a1, b1, c1), c2 = mfma(a2, b2, c2), c3 = mfma(a3, b3, c3);
      c0 = mfma(a1, b2, c0), c1 = mfma(a2, b3, c1), c2 = mfma(a3, b0, c2), c3 = mfma(a0, b1, c3);
      c0 = mfma(a2, b0, c0), c1 = mfma(a3, b1, c1), c2 = mfma(a0, b2, c2), c3 = mfma(a1, b3, c3);
      c0 = mfma(a3, b2, c0), c1 = mfma(a0, b3, c1), c2 = mfma(a1, b0, c2), c3 = mfma(a2, b1, c3);
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
  sink[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
  const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (clocks && threadIdx.x == 0) {
    unsigned long long* c = clocks + (size_t)blockIdx.x * 4;
    c[0] = t0, c[1] = t1, c[2] = r0, c[3] = r1;
  }
}

}  // namespace

// Entries of 16 bytes that a non-null `operands` must hold.
extern "C" int64_t diag_mfma_operand_count(void) { return (int64_t)kOperandSets * 512 * 8; }

// Launches the loop on `grid` workgroups of 512 threads; sink holds grid * 512 floats,
// operands null or diag_mfma_operand_count() entries of 16 bytes, clocks null or grid * 4
// entries.  Returns 0, -1 for a bad argument, or the HIP error code of the launch.
extern "C" int diag_mfma_loop(float* sink, const void* operands, unsigned long long* clocks, int iters, int grid,
                              void* stream) {
  if (!sink || iters <= 0 || grid <= 0) return -1;
  hipLaunchKernelGGL(mfma_loop_kernel, dim3((unsigned)grid), dim3(512), 0, (hipStream_t)stream, iters,
                     (const u32x4*)operands, sink, clocks);
  return (int)hipGetLastError();
}
