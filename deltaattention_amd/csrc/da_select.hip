// Delta-mode anchor selection on gfx950.
//
// Replaces chunked_eval_kernel (tritonModules.py:7-69) and its launch
// (modeling_llama.py:634-653).  One wave64 walks one chunk of one KV head
// sequentially: the first row is an anchor; every later row is compared with the
// current anchor and becomes the anchor when it is far enough (Euclidean
// ||k - a||^2 > tau^2, or cosine < tau).
//
// Lane l holds head-dimension elements 2l and 2l+1 (one 4-byte load per lane, a
// coalesced 256-byte row per wave for D = 128).  The distance is fp32 and reduced
// by a fixed perfect pairwise tree over 128 slots: the per-lane pair sum is level 1,
// DPP lane^1, lane^2, 8-lane mirror and 16-lane mirror give levels 2-5 (every lane
// of a 16-lane row then holds the row sum), and the four row sums are combined as
// (r0 + r1) + (r2 + r3).  No multiply-add is fused, so the result is bit-identical
// to the CPU restatement of the same tree.
//
// Rows are prefetched 32 at a time one batch ahead, since loads never depend on
// the decisions.  Keep decisions collect in a 64-bit scalar mask and are stored as
// int32 (the reference's keep-mask format) 64 rows at a time.
#include "da_common.hpp"

namespace da {

__device__ __forceinline__ void store_keep_bits(int32_t* keep_row, int64_t base, int64_t end,
                                                uint64_t bits, int lane) {
  const int64_t r = base + lane;
  if (r < end) keep_row[r] = (int32_t)((bits >> lane) & 1ull);
}

constexpr int kSelBatch = 32;

template <bool COS>
__global__ __launch_bounds__(256) void select_kernel(
    const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_h, int64_t sk_n, int H, int64_t N,
    int D, int64_t cs, int64_t nc, int64_t total_chunks, float thr, int32_t* __restrict__ keep,
    int32_t* __restrict__ chunk_counts) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= total_chunks) return;
  const int64_t bh = w / nc;
  const int64_t c = w - bh * nc;
  const int64_t b = bh / H, h = bh - (bh / H) * H;
  const int64_t s = c * cs;
  if (s >= N) {  // tritonModules.py:34-35 (count stays 0, modeling_llama.py:637)
    if (lane == 0) chunk_counts[w] = 0;
    return;
  }
  const int64_t e = (s + cs < N) ? s + cs : N;
  const uint16_t* base = k + b * sk_b + h * sk_h + 2 * lane;
  const bool active = 2 * lane < D;
  int32_t* keep_row = keep + bh * N;

  const uint32_t a_bits = active ? *(const uint32_t*)(base + s * sk_n) : 0u;
  float a0 = bf16_lo(a_bits), a1 = bf16_hi(a_bits);
  const float eps = 1e-8f;
  float a_norm = 0.0f;
  if (COS) a_norm = __fsqrt_rn(wave_tree_sum(pair_dot(a0, a1, a0, a1)) + eps);

  int count = 1;
  uint64_t bits = 1ull;  // row s is an anchor (tritonModules.py:41)
  int64_t wbase = s;

  uint32_t cur[kSelBatch], nxt[kSelBatch];
#pragma unroll
  for (int j = 0; j < kSelBatch; ++j) {
    const int64_t r = s + 1 + j;
    cur[j] = (active && r < e) ? *(const uint32_t*)(base + r * sk_n) : 0u;
  }
  for (int64_t i0 = s + 1; i0 < e; i0 += kSelBatch) {
    const int64_t n0 = i0 + kSelBatch;
#pragma unroll
    for (int j = 0; j < kSelBatch; ++j) {
      const int64_t r = n0 + j;
      nxt[j] = (active && r < e) ? *(const uint32_t*)(base + r * sk_n) : 0u;
    }
#pragma unroll
    for (int j = 0; j < kSelBatch; ++j) {
      const int64_t i = i0 + j;
      if (i < e) {
        const float x0 = bf16_lo(cur[j]), x1 = bf16_hi(cur[j]);
        bool kp;
        float x_norm = 0.0f;
        if (COS) {  // tritonModules.py:48-54
          const float dot = wave_tree_sum(pair_dot(x0, x1, a0, a1));
          x_norm = __fsqrt_rn(wave_tree_sum(pair_dot(x0, x1, x0, x1)) + eps);
          const float sim = __fdiv_rn(dot, x_norm * a_norm);
          kp = sim < thr;
        } else {  // tritonModules.py:55-58
          const float d0 = x0 - a0, d1 = x1 - a1;
          kp = wave_tree_sum(pair_dot(d0, d1, d0, d1)) > thr;
        }
        if (kp) {  // tritonModules.py:60-63
          a0 = x0;
          a1 = x1;
          if (COS) a_norm = x_norm;
          ++count;
        }
        const int64_t off = i - wbase;
        if (off == 64) {
          store_keep_bits(keep_row, wbase, e, bits, lane);
          wbase += 64;
          bits = 0ull;
        }
        bits |= (uint64_t)kp << (i - wbase);
      }
    }
#pragma unroll
    for (int j = 0; j < kSelBatch; ++j) cur[j] = nxt[j];
  }
  store_keep_bits(keep_row, wbase, e, bits, lane);
  if (lane == 0) chunk_counts[w] = count;  // tritonModules.py:68-69
}

}  // namespace da

using namespace da;

extern "C" int da_select(const void* k, int dtype, int64_t B, int64_t Hkv, int64_t N, int64_t D,
                         int64_t sk_b, int64_t sk_h, int64_t sk_n, float threshold, int use_cosine,
                         int64_t chunk_size, int64_t num_chunks, int32_t* keep,
                         int32_t* chunk_counts, void* stream) {
  DA_REQUIRE(k && keep && chunk_counts, "da_select: null pointer");
  if (dtype != DA_BF16) return set_error(DA_ERR_UNSUPPORTED, "da_select: only bf16 keys are supported");
  DA_REQUIRE(B > 0 && Hkv > 0 && N > 0 && D > 0, "da_select: empty shape");
  if (D > 128 || (D & 1)) return set_error(DA_ERR_UNSUPPORTED, "da_select: head_dim must be even and <= 128 (got %lld)", (long long)D);
  DA_REQUIRE(chunk_size > 0 && num_chunks > 0, "da_select: chunk_size and num_chunks must be positive");
  DA_REQUIRE(N < (1ll << 31), "da_select: sequence too long");
  DA_REQUIRE(((sk_b | sk_h | sk_n) & 1) == 0 && ((uintptr_t)k & 3) == 0,
             "da_select: key rows must be 4-byte aligned (even strides)");
  const int64_t total = B * Hkv * num_chunks;
  const int64_t blocks = (total + 3) / 4;
  DA_REQUIRE(blocks < (1ll << 31), "da_select: too many chunks");
  hipStream_t st = (hipStream_t)stream;
  if (use_cosine)
    hipLaunchKernelGGL(select_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const uint16_t*)k, sk_b, sk_h, sk_n, (int)Hkv, N, (int)D, chunk_size,
                       num_chunks, total, threshold, keep, chunk_counts);
  else
    hipLaunchKernelGGL(select_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, st,
                       (const uint16_t*)k, sk_b, sk_h, sk_n, (int)Hkv, N, (int)D, chunk_size,
                       num_chunks, total, threshold, keep, chunk_counts);
  return check_launch("da_select");
}
