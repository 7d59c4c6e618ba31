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
// With A16 (DA_SELECT_ARITH16) the Euclidean distance rounds every difference, square
// and tree addition to the keys' 16-bit type, as the reference's Triton code evaluates
// curr - ref, diff * diff and tl.sum on 16-bit tensors (tritonModules.py:55-58); only
// the reduction order stays the fixed tree.  The cosine test is fp32 either way (the
// reference upcasts it, :48-54).
//
// Rows are prefetched 32 at a time one batch ahead, since loads never depend on
// the decisions.  The distance reaches every lane through v_permlane16/32_swap (no
// scalar round trip), the anchor update is a select, and a batch's decisions collect
// in a 32-bit mask stored as int32 (the reference's keep-mask format).
//
// From 2048 chunks on (two per SIMD), select_pair_kernel walks two chunks per wave,
// one per 32-lane half with four slots per lane, over the same tree (bit-identical);
// below that, one wave per chunk keeps every chunk on a SIMD of its own.
#include <algorithm>

#include "da_common.hpp"

namespace da {

constexpr int kSelBatch = 32;
constexpr int64_t kSelPairMinChunks = 2048;

// x rounded to the 16-bit type DT (nearest even) and widened back to fp32.  For bf16
// one v_cvt_pk_bf16_f32 with x in the high half and 0 in the low half leaves exactly
// that fp32 value in the register (the widening is free); fp16 converts there and back.
template <int DT>
__device__ __forceinline__ float round16(float x) {
  if constexpr (DT == DA_BF16) {
    // as asm: written in C the compiler swaps the halves back and adds a v_perm_b32
    float r;
    asm("v_cvt_pk_bf16_f32 %0, 0, %1" : "=v"(r) : "v"(x));
    return r;
  } else
    return E16<DT>::one(E16<DT>::bits(x));
}

// wave_tree_sum_all with every addition rounded to DT: the same pairing (DPP lane^1,
// lane^2, 8-lane and 16-lane mirror, then (r0 + r1) + (r2 + r3)).
template <int DT>
__device__ __forceinline__ float wave_tree_sum_all_r16(float t) {
#pragma clang fp contract(off)
  t = round16<DT>(t + dpp_f32<kDppXor1>(t));
  t = round16<DT>(t + dpp_f32<kDppXor2>(t));
  t = round16<DT>(t + dpp_f32<kDppHalfMirror>(t));
  t = round16<DT>(t + dpp_f32<kDppMirror>(t));
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(t), __float_as_uint(t), false, false);
  const float u = round16<DT>(__uint_as_float(r[0]) + __uint_as_float(r[1]));
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(u), __float_as_uint(u), false, false);
  return round16<DT>(__uint_as_float(q[0]) + __uint_as_float(q[1]));
}

// A lane's two key elements (2l, 2l + 1) of one row: one 4-byte word of a 16-bit type,
// or two fp32 values (8 bytes; fp32 keys are compared in fp32, the reference's
// arithmetic on fp32 tensors).
template <int DT>
struct SelKey {
  using Elem = uint16_t;
  using Row = uint32_t;
  static __device__ __forceinline__ float lo(Row w) { return E16<DT>::lo(w); }
  static __device__ __forceinline__ float hi(Row w) { return E16<DT>::hi(w); }
};
template <>
struct SelKey<DA_F32> {
  using Elem = float;
  using Row = u32x2;
  static __device__ __forceinline__ float lo(Row w) { return __uint_as_float(w[0]); }
  static __device__ __forceinline__ float hi(Row w) { return __uint_as_float(w[1]); }
};

// One key of the walk: the decision and the anchor update without a branch (the
// decision is the same in every lane).
template <bool COS, bool A16, int DT>
__device__ __forceinline__ bool select_step(float x0, float x1, float& a0, float& a1, float& a_norm,
                                            float thr) {
#pragma clang fp contract(off)
  const float eps = 1e-8f;
  bool kp;
  float x_norm = 0.0f;
  if constexpr (COS) {  // tritonModules.py:48-54
    const float dot = wave_tree_sum_all(pair_dot(x0, x1, a0, a1));
    x_norm = sqrt_rn(wave_tree_sum_all(pair_dot(x0, x1, x0, x1)) + eps);
    const float sim = __fdiv_rn(dot, x_norm * a_norm);
    kp = sim < thr;
  } else if constexpr (A16) {  // tritonModules.py:55-58 in the keys' 16-bit arithmetic
    const float d0 = round16<DT>(x0 - a0), d1 = round16<DT>(x1 - a1);
    const float p0 = round16<DT>(d0 * d0), p1 = round16<DT>(d1 * d1);
    kp = wave_tree_sum_all_r16<DT>(round16<DT>(p0 + p1)) > thr;
  } else {  // tritonModules.py:55-58
    const float d0 = x0 - a0, d1 = x1 - a1;
    kp = wave_tree_sum_all(pair_dot(d0, d1, d0, d1)) > thr;
  }
  a0 = kp ? x0 : a0;  // tritonModules.py:60-63
  a1 = kp ? x1 : a1;
  if (COS) a_norm = kp ? x_norm : a_norm;
  return kp;
}

// Keys: a fixed-length batch [B, H, N, D] with the caller's chunk size cs, or (seq.cu set)
// a ragged batch of [T, H, D] tensors where sequence b is chunked by the reference's rule
// on its own length: min(cs, N_b) rows per chunk, or ceil(N_b / divide_to) when
// divide_to > 0 (modeling_llama.py:602-610).  keep is [B, H, N] for a fixed batch and
// [H, T] (row h * keep_sh + token) for a ragged one; chunk_counts is [B, H, nc].
template <bool COS, bool A16, int DT>
__global__ __launch_bounds__(256) void select_kernel(
    const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_h, int64_t sk_n, int H, int64_t N,
    int D, int64_t cs, int64_t nc, int64_t total_chunks, float thr, int32_t* __restrict__ keep,
    int32_t* __restrict__ chunk_counts, SeqMap seq, int64_t keep_sh, int divide_to) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= total_chunks) return;
  const int64_t bh = w / nc;
  const int64_t c = w - bh * nc;
  const int64_t b = bh / H, h = bh - (bh / H) * H;
  const int64_t Nb = seq.cu ? seq.len((int)b) : N;
  int64_t csb = cs;
  if (seq.cu) csb = divide_to > 0 ? (Nb + divide_to - 1) / divide_to : (cs < Nb ? cs : Nb);
  if (Nb <= 0 || c * csb >= Nb) {  // tritonModules.py:34-35 (count stays 0, modeling_llama.py:637)
    if (lane == 0) chunk_counts[w] = 0;
    return;
  }
  // rows are 32-bit from here on (N < 2^31)
  const int s = (int)(c * csb);
  const int e = (int)((c * csb + csb < Nb) ? c * csb + csb : Nb);
  using KT = SelKey<DT>;
  using Row = typename KT::Row;
  const typename KT::Elem* base =
      (const typename KT::Elem*)(const void*)k + seq.base((int)b, sk_b, sk_n) + h * sk_h + 2 * lane;
  const bool active = 2 * lane < D;
  int32_t* keep_row = keep + (seq.cu ? h * keep_sh + seq.start((int)b) : bh * N);
  auto row_bits = [&](int r) -> Row {
    return (active && r < e) ? *(const Row*)(base + (int64_t)r * sk_n) : Row{};
  };

  const Row a_bits = row_bits(s);
  float a0 = KT::lo(a_bits), a1 = KT::hi(a_bits);
  float a_norm = 0.0f;
  if (COS) a_norm = sqrt_rn(wave_tree_sum_all(pair_dot(a0, a1, a0, a1)) + 1e-8f);
  if (lane == 0) keep_row[s] = 1;  // row s is an anchor (tritonModules.py:41)
  int count = 1;

  // Rows s + 1 .. e - 1 in batches of 32, each loaded one batch ahead (the loads never
  // depend on the decisions); a batch's 32 decisions are stored by lanes 0..31.
  Row cur[kSelBatch], nxt[kSelBatch];
#pragma unroll
  for (int j = 0; j < kSelBatch; ++j) cur[j] = row_bits(s + 1 + j);
  for (int i0 = s + 1; i0 < e; i0 += kSelBatch) {
#pragma unroll
    for (int j = 0; j < kSelBatch; ++j) nxt[j] = row_bits(i0 + kSelBatch + j);
    uint32_t bb = 0;
    if (i0 + kSelBatch <= e) {
#pragma unroll
      for (int j = 0; j < kSelBatch; ++j)
        bb |= (uint32_t)select_step<COS, A16, DT>(KT::lo(cur[j]), KT::hi(cur[j]), a0, a1, a_norm, thr) << j;
    } else {
#pragma unroll
      for (int j = 0; j < kSelBatch; ++j)
        if (i0 + j < e)
          bb |= (uint32_t)select_step<COS, A16, DT>(KT::lo(cur[j]), KT::hi(cur[j]), a0, a1, a_norm, thr) << j;
    }
    count += __builtin_popcount(bb);  // tritonModules.py:68
    if (lane < kSelBatch && i0 + lane < e) keep_row[i0 + lane] = (int32_t)((bb >> lane) & 1u);
#pragma unroll
    for (int j = 0; j < kSelBatch; ++j) cur[j] = nxt[j];
  }
  if (lane == 0) chunk_counts[w] = count;  // tritonModules.py:68-69
}

// ---- two chunks per wave, one per 32-lane half ----
// Lane q of a half holds head-dimension slots 4q .. 4q+3 of a row (one 8-byte load), so
// a wave walks two chunks at once.  The tree keeps its pairing: levels 1-2 add slots
// inside the lane, lane^1, lane^2, the 8-lane and the 16-lane mirror give levels 3-6, and
// v_permlane16_swap pairs the two 16-lane rows of each half for level 7 -- the blocks
// that the one-chunk-per-wave tree pairs at each level, so the sums are bit-identical.
template <bool R16, int DT>
__device__ __forceinline__ float half_tree_sum(float p0, float p1, float p2, float p3) {
#pragma clang fp contract(off)
  auto r = [](float v) { return R16 ? round16<DT>(v) : v; };
  float t = r(r(p0 + p1) + r(p2 + p3));
  t = r(t + dpp_f32<kDppXor1>(t));
  t = r(t + dpp_f32<kDppXor2>(t));
  t = r(t + dpp_f32<kDppHalfMirror>(t));
  t = r(t + dpp_f32<kDppMirror>(t));
  const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(t), __float_as_uint(t), false, false);
  return r(__uint_as_float(sw[0]) + __uint_as_float(sw[1]));
}

// select_step for the row a 32-lane half holds (x: four slots); rows with `valid` false
// are never kept.
template <bool COS, bool A16, int DT>
__device__ __forceinline__ bool half_step(const uint2 xb, float (&a)[4], float& a_norm, float thr, bool valid) {
#pragma clang fp contract(off)
  const float x[4] = {E16<DT>::lo(xb.x), E16<DT>::hi(xb.x), E16<DT>::lo(xb.y), E16<DT>::hi(xb.y)};
  bool kp;
  float x_norm = 0.0f;
  if (COS) {  // tritonModules.py:48-54
    const float dot = half_tree_sum<false, DT>(x[0] * a[0], x[1] * a[1], x[2] * a[2], x[3] * a[3]);
    x_norm = sqrt_rn(half_tree_sum<false, DT>(x[0] * x[0], x[1] * x[1], x[2] * x[2], x[3] * x[3]) + 1e-8f);
    kp = __fdiv_rn(dot, x_norm * a_norm) < thr;
  } else if (A16) {  // tritonModules.py:55-58 in the keys' 16-bit arithmetic
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float d = round16<DT>(x[i] - a[i]);
      p[i] = round16<DT>(d * d);
    }
    kp = half_tree_sum<true, DT>(p[0], p[1], p[2], p[3]) > thr;
  } else {  // tritonModules.py:55-58
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float d = x[i] - a[i];
      p[i] = d * d;
    }
    kp = half_tree_sum<false, DT>(p[0], p[1], p[2], p[3]) > thr;
  }
  kp = kp && valid;
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = kp ? x[i] : a[i];  // tritonModules.py:60-63
  if (COS) a_norm = kp ? x_norm : a_norm;
  return kp;
}

// The chunks as select_kernel walks them, two per wave (chunk 2 w + half).  Needs D a
// multiple of 4 and 8-byte aligned rows.
template <bool COS, bool A16, int DT>
__global__ __launch_bounds__(256) void select_pair_kernel(
    const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_h, int64_t sk_n, int H, int64_t N,
    int D, int64_t cs, int64_t nc, int64_t total_chunks, float thr, int32_t* __restrict__ keep,
    int32_t* __restrict__ chunk_counts, SeqMap seq, int64_t keep_sh, int divide_to) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int q = lane & 31;
  const int64_t w = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 2 + (lane >> 5);
  // rows [s, e) of this half's chunk; none for a chunk past the grid or the sequence
  int s = 0, e = 0;
  int32_t* keep_row = keep;
  const uint16_t* base = k;
  if (w < total_chunks) {
    const int64_t bh = w / nc;
    const int64_t c = w - bh * nc;
    const int64_t b = bh / H, h = bh - (bh / H) * H;
    const int64_t Nb = seq.cu ? seq.len((int)b) : N;
    int64_t csb = cs;
    if (seq.cu) csb = divide_to > 0 ? (Nb + divide_to - 1) / divide_to : (cs < Nb ? cs : Nb);
    if (Nb > 0 && c * csb < Nb) {
      s = (int)(c * csb);
      e = (int)((c * csb + csb < Nb) ? c * csb + csb : Nb);
      base = k + seq.base((int)b, sk_b, sk_n) + h * sk_h + 4 * q;
      keep_row = keep + (seq.cu ? h * keep_sh + seq.start((int)b) : bh * N);
    } else if (q == 0) {
      chunk_counts[w] = 0;  // tritonModules.py:34-35 (count stays 0, modeling_llama.py:637)
    }
  }
  const bool active = 4 * q < D;
  auto row_bits = [&](int r) -> uint2 {
    return (active && r < e) ? *(const uint2*)(base + (int64_t)r * sk_n) : uint2{0u, 0u};
  };
  const uint2 ab = row_bits(s);
  float a[4] = {E16<DT>::lo(ab.x), E16<DT>::hi(ab.x), E16<DT>::lo(ab.y), E16<DT>::hi(ab.y)};
  float a_norm = 0.0f;
  if (COS)
    a_norm = sqrt_rn(half_tree_sum<false, DT>(a[0] * a[0], a[1] * a[1], a[2] * a[2], a[3] * a[3]) + 1e-8f);
  if (q == 0 && e > s) keep_row[s] = 1;  // row s is an anchor (tritonModules.py:41)
  int count = 1;
  // batches of both halves (wave-uniform): the longer of the two walks
  const int nbh = e > s ? (e - s - 1 + kSelBatch - 1) / kSelBatch : 0;
  const int nb = max(__builtin_amdgcn_readlane(nbh, 0), __builtin_amdgcn_readlane(nbh, 32));
  uint2 cur[kSelBatch], nxt[kSelBatch];
#pragma unroll
  for (int j = 0; j < kSelBatch; ++j) cur[j] = row_bits(s + 1 + j);
  for (int bi = 0; bi < nb; ++bi) {
    const int i0 = s + 1 + bi * kSelBatch;
#pragma unroll
    for (int j = 0; j < kSelBatch; ++j) nxt[j] = row_bits(i0 + kSelBatch + j);
    uint32_t bb = 0;
#pragma unroll
    for (int j = 0; j < kSelBatch; ++j)
      bb |= (uint32_t)half_step<COS, A16, DT>(cur[j], a, a_norm, thr, i0 + j < e) << j;
    count += __builtin_popcount(bb);  // tritonModules.py:68
    if (i0 + q < e) keep_row[i0 + q] = (int32_t)((bb >> q) & 1u);
#pragma unroll
    for (int j = 0; j < kSelBatch; ++j) cur[j] = nxt[j];
  }
  if (q == 0 && e > s) chunk_counts[w] = count;  // tritonModules.py:68-69
}

static int launch_select(const void* k, int dtype, int64_t B, int64_t Hkv, int64_t N, int64_t D, int64_t sk_b,
                         int64_t sk_h, int64_t sk_n, float threshold, bool use_cosine, bool a16, int64_t chunk_size,
                         int64_t num_chunks, int32_t* keep, int32_t* chunk_counts, SeqMap seq, int64_t keep_sh,
                         int divide_to, hipStream_t st, const char* who) {
  DA_REQUIRE(((sk_b | sk_h | sk_n) & 1) == 0 && ((uintptr_t)k & (dtype == DA_F32 ? 7 : 3)) == 0,
             "%s: key rows must be %d-byte aligned (even strides)", who, dtype == DA_F32 ? 8 : 4);
  const int64_t total = B * Hkv * num_chunks;
  const int64_t blocks = (total + 3) / 4;
  DA_REQUIRE(blocks < (1ll << 31), "%s: too many chunks", who);
  if (dtype == DA_F32) {
    // fp32 keys: one wave per chunk, each lane two fp32 elements; the 16-bit definition
    // does not apply (the keys' own arithmetic is fp32)
    if (use_cosine)
      hipLaunchKernelGGL((select_kernel<true, false, DA_F32>), dim3((unsigned)blocks), dim3(256), 0, st,
                         (const uint16_t*)k, sk_b, sk_h, sk_n, (int)Hkv, N, (int)D, chunk_size, num_chunks, total,
                         threshold, keep, chunk_counts, seq, keep_sh, divide_to);
    else
      hipLaunchKernelGGL((select_kernel<false, false, DA_F32>), dim3((unsigned)blocks), dim3(256), 0, st,
                         (const uint16_t*)k, sk_b, sk_h, sk_n, (int)Hkv, N, (int)D, chunk_size, num_chunks, total,
                         threshold, keep, chunk_counts, seq, keep_sh, divide_to);
    return check_launch(who);
  }
  // From two chunks per SIMD on (256 CUs x 4 SIMDs), one wave per pair of chunks walks
  // both in one instruction stream and leaves the SIMDs one wave each: 79 against 85 us
  // at 131072 keys x 8 heads.  Fewer chunks keep one wave per chunk (the pair layout
  // would leave SIMDs idle).
  if (total >= kSelPairMinChunks && (D & 3) == 0 && ((sk_b | sk_h | sk_n) & 3) == 0 && ((uintptr_t)k & 7) == 0) {
    const int64_t pblocks = (total + 7) / 8;
#define DA_SELPAIR_LAUNCH(COS, A16, DT)                                                                      \
  hipLaunchKernelGGL((select_pair_kernel<COS, A16, DT>), dim3((unsigned)pblocks), dim3(256), 0, st,           \
                     (const uint16_t*)k, sk_b, sk_h, sk_n, (int)Hkv, N, (int)D, chunk_size, num_chunks, total, \
                     threshold, keep, chunk_counts, seq, keep_sh, divide_to)
    if (dtype == DA_F16) {
      if (use_cosine) DA_SELPAIR_LAUNCH(true, false, DA_F16);
      else if (a16) DA_SELPAIR_LAUNCH(false, true, DA_F16);
      else DA_SELPAIR_LAUNCH(false, false, DA_F16);
    } else {
      if (use_cosine) DA_SELPAIR_LAUNCH(true, false, DA_BF16);
      else if (a16) DA_SELPAIR_LAUNCH(false, true, DA_BF16);
      else DA_SELPAIR_LAUNCH(false, false, DA_BF16);
    }
#undef DA_SELPAIR_LAUNCH
    return check_launch(who);
  }
#define DA_SELECT_LAUNCH(COS, A16, DT)                                                                       \
  hipLaunchKernelGGL((select_kernel<COS, A16, DT>), dim3((unsigned)blocks), dim3(256), 0, st, (const uint16_t*)k, \
                     sk_b, sk_h, sk_n, (int)Hkv, N, (int)D, chunk_size, num_chunks, total, threshold, keep,  \
                     chunk_counts, seq, keep_sh, divide_to)
  if (dtype == DA_F16) {
    if (use_cosine) DA_SELECT_LAUNCH(true, false, DA_F16);
    else if (a16) DA_SELECT_LAUNCH(false, true, DA_F16);
    else DA_SELECT_LAUNCH(false, false, DA_F16);
  } else {
    if (use_cosine) DA_SELECT_LAUNCH(true, false, DA_BF16);
    else if (a16) DA_SELECT_LAUNCH(false, true, DA_BF16);
    else DA_SELECT_LAUNCH(false, false, DA_BF16);
  }
#undef DA_SELECT_LAUNCH
  return check_launch(who);
}

}  // namespace da

using namespace da;

extern "C" int da_select(const void* k, int dtype, int64_t B, int64_t Hkv, int64_t N, int64_t D,
                         int64_t sk_b, int64_t sk_h, int64_t sk_n, float threshold, int flags,
                         int64_t chunk_size, int64_t num_chunks, int32_t* keep,
                         int32_t* chunk_counts, void* stream) {
  DA_REQUIRE(k && keep && chunk_counts, "da_select: null pointer");
  DA_REQUIRE((flags & ~(DA_SELECT_COSINE | DA_SELECT_ARITH16)) == 0, "da_select: unknown flags 0x%x", flags);
  const bool use_cosine = flags & DA_SELECT_COSINE;
  const bool a16 = !use_cosine && (flags & DA_SELECT_ARITH16);
  if (dtype != DA_BF16 && dtype != DA_F16 && dtype != DA_F32)
    return set_error(DA_ERR_UNSUPPORTED, "da_select: keys must be bf16, fp16 or fp32");
  DA_REQUIRE(B > 0 && Hkv > 0 && N > 0 && D > 0, "da_select: empty shape");
  if (D > 128 || (D & 1)) return set_error(DA_ERR_UNSUPPORTED, "da_select: head_dim must be even and <= 128 (got %lld)", (long long)D);
  DA_REQUIRE(chunk_size > 0 && num_chunks > 0, "da_select: chunk_size and num_chunks must be positive");
  DA_REQUIRE(N < (1ll << 31), "da_select: sequence too long");
  return launch_select(k, dtype, B, Hkv, N, D, sk_b, sk_h, sk_n, threshold, use_cosine, a16, chunk_size,
                       num_chunks, keep, chunk_counts, SeqMap{nullptr, 0, (int)N}, N, 0, (hipStream_t)stream,
                       "da_select");
}

extern "C" int da_select_varlen(const void* k, int dtype, int64_t B, int64_t Hkv, int64_t T, int64_t D,
                                int64_t sk_t, int64_t sk_h, const int32_t* cu_seqlens, int64_t max_seqlen,
                                float threshold, int flags, int64_t chunk_size, int64_t divide_to,
                                int32_t* keep, int32_t* chunk_counts, int64_t max_chunks, void* stream) {
  const char* who = "da_select_varlen";
  DA_REQUIRE(k && keep && chunk_counts && cu_seqlens, "%s: null pointer", who);
  DA_REQUIRE((flags & ~(DA_SELECT_COSINE | DA_SELECT_ARITH16)) == 0, "%s: unknown flags 0x%x", who, flags);
  const bool use_cosine = flags & DA_SELECT_COSINE;
  const bool a16 = !use_cosine && (flags & DA_SELECT_ARITH16);
  if (dtype != DA_BF16 && dtype != DA_F16 && dtype != DA_F32)
    return set_error(DA_ERR_UNSUPPORTED, "%s: keys must be bf16, fp16 or fp32", who);
  DA_REQUIRE(B > 0 && Hkv > 0 && T > 0 && D > 0, "%s: empty shape", who);
  if (D > 128 || (D & 1)) return set_error(DA_ERR_UNSUPPORTED, "%s: head_dim must be even and <= 128 (got %lld)", who, (long long)D);
  DA_REQUIRE(T < (1ll << 31) && max_seqlen > 0 && max_seqlen <= T, "%s: need 0 < max_seqlen <= total tokens < 2^31", who);
  DA_REQUIRE(divide_to >= 0, "%s: divide_to must be >= 0", who);
  // the chunking rule of modeling_llama.py:602-610, per sequence
  const int64_t cs = chunk_size > 0 ? chunk_size : 0;
  const int div = chunk_size > 0 ? 0 : (divide_to > 0 ? (int)divide_to : 1);
  const int64_t need = chunk_size > 0 ? std::max<int64_t>(1, (max_seqlen + chunk_size - 1) / chunk_size) : div;
  DA_REQUIRE(max_chunks >= need, "%s: max_chunks must be at least %lld", who, (long long)need);
  return launch_select(k, dtype, B, Hkv, max_seqlen, D, 0, sk_h, sk_t, threshold, use_cosine, a16, cs, max_chunks,
                       keep, chunk_counts, SeqMap{cu_seqlens, (int)T, (int)max_seqlen}, T, div,
                       (hipStream_t)stream, who);
}
