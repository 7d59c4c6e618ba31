// Shared device/host helpers of the gfx950 DeltaAttention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/deltaattn.h"

namespace da {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ------------------------------------------------------------------------------------
// error state (host)
// ------------------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

#define DA_REQUIRE(cond, ...)                                   \
  do {                                                          \
    if (!(cond)) return ::da::set_error(DA_ERR_INVALID, __VA_ARGS__); \
  } while (0)

// ------------------------------------------------------------------------------------
// bf16 helpers (device)
// ------------------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round two fp32 values to bf16 (nearest even) and pack them (a in the low half).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// The two 16-bit element formats (DA_BF16, DA_F16): unpacking a pair held in 32 bits
// (low half first), rounding to the format (nearest even) and packing, and the
// v_mfma_f32_32x32x16 of the format on 8-element operands held as 4 x 32 bits.
template <int DT>
struct E16;
template <>
struct E16<DA_BF16> {
  static __device__ __forceinline__ float lo(uint32_t w) { return bf16_lo(w); }
  static __device__ __forceinline__ float hi(uint32_t w) { return bf16_hi(w); }
  static __device__ __forceinline__ float one(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
  static __device__ __forceinline__ uint16_t bits(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
  static __device__ __forceinline__ uint32_t pack(float a, float b) { return pack_bf16x2(a, b); }
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                    c, 0, 0, 0);
  }
};
template <>
struct E16<DA_F16> {
  static __device__ __forceinline__ float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  static __device__ __forceinline__ float hi(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }
  static __device__ __forceinline__ float one(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
  static __device__ __forceinline__ uint16_t bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    f16x2 v;
    v[0] = (_Float16)a;
    v[1] = (_Float16)b;
    return __builtin_bit_cast(uint32_t, v);
  }
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                   c, 0, 0, 0);
  }
};

// ------------------------------------------------------------------------------------
// batch layouts (device): a fixed-length batch puts sequence b at b * stride_b; a packed
// ragged batch (cu_seqlens, the varlen entry points) puts it at tokens cu[b] ..
// cu[b + 1] - 1, i.e. at cu[b] * stride_n.  Offsets and lengths read from cu are
// clamped into [0, total] and to max_len, so malformed cu_seqlens cannot address memory
// outside the tensors.
// ------------------------------------------------------------------------------------
struct SeqMap {
  const int32_t* cu;  // null: fixed-length batch
  int total;          // tokens in the packed batch (varlen) / unused
  int max_len;        // the longest sequence (varlen) / the fixed length
  __device__ __forceinline__ int start(int b) const {
    if (!cu) return 0;
    const int s = cu[b];
    return s < 0 ? 0 : (s > total ? total : s);
  }
  __device__ __forceinline__ int len(int b) const {
    if (!cu) return max_len;
    const int s = start(b);
    int e = cu[b + 1];
    e = e < s ? s : (e > total ? total : e);
    return e - s > max_len ? max_len : e - s;
  }
  // element offset of row 0 of sequence b in a tensor with strides (s_b, s_n)
  __device__ __forceinline__ int64_t base(int b, int64_t s_b, int64_t s_n) const {
    return cu ? (int64_t)start(b) * s_n : (int64_t)b * s_b;
  }
};

// ------------------------------------------------------------------------------------
// wave-level data movement (device)
// ------------------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// DPP controls: quad_perm [1,0,3,2] = lane^1, [2,3,0,1] = lane^2,
// row_half_mirror = lane ^ 7 within 8, row_mirror = lane ^ 15 within 16.
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

// Exchange with lane ^ 32 (the other half of the wave).
__device__ __forceinline__ float swap_halves(float v) {
  return __shfl_xor(v, 32, 64);
}

__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Workgroup barrier that orders LDS accesses only: unlike __syncthreads() it does not
// wait for outstanding global loads, so prefetches stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Fixed-order fp32 sum over a wave where lane l holds the pair sum of head-dimension
// slots 2l and 2l+1 (level 1 of a perfect pairwise tree over 128 slots): DPP lane^1,
// lane^2, 8-lane mirror and 16-lane mirror give levels 2-5, then (r0 + r1) + (r2 + r3)
// over the four 16-lane row sums.  The result is wave-uniform.
__device__ __forceinline__ float wave_tree_sum(float t) {
#pragma clang fp contract(off)
  t = t + dpp_f32<kDppXor1>(t);
  t = t + dpp_f32<kDppXor2>(t);
  t = t + dpp_f32<kDppHalfMirror>(t);
  t = t + dpp_f32<kDppMirror>(t);
  const float r0 = readlane_f32(t, 0);
  const float r1 = readlane_f32(t, 16);
  const float r2 = readlane_f32(t, 32);
  const float r3 = readlane_f32(t, 48);
  return (r0 + r1) + (r2 + r3);
}

// The same tree, with the sum in every lane: after the four DPP levels every 16-lane
// row holds its row sum; v_permlane16_swap pairs rows 0/1 and 2/3, v_permlane32_swap
// the two halves, so every lane computes (r0 + r1) + (r2 + r3) (additions commute
// bit-exactly).  No scalar round trip.
__device__ __forceinline__ float wave_tree_sum_all(float t) {
#pragma clang fp contract(off)
  t = t + dpp_f32<kDppXor1>(t);
  t = t + dpp_f32<kDppXor2>(t);
  t = t + dpp_f32<kDppHalfMirror>(t);
  t = t + dpp_f32<kDppMirror>(t);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(t), __float_as_uint(t), false, false);
  const float u = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(u), __float_as_uint(u), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// Correctly rounded fp32 square root (round to nearest even), as the CPU restatement's
// sqrtf.  HIP's __fsqrt_rn is the hardware approximation unless OCML's rounded
// operations are enabled, and differs from it in the last place often enough to flip a
// cosine decision that sits at the threshold (one row in a million keys of 64 heads).
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }

// x0*y0 + x1*y1 with both products rounded (no fused multiply-add).
__device__ __forceinline__ float pair_dot(float x0, float x1, float y0, float y1) {
#pragma clang fp contract(off)
  const float p0 = x0 * y0;
  const float p1 = x1 * y1;
  return p0 + p1;
}

}  // namespace da
