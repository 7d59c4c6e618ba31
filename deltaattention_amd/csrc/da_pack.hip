// Index + pack + counts on gfx950, fused and free of host synchronisation.
//
// Replaces index_map = cumsum(keep) - 1 and P = max count with its .item()
// (modeling_llama.py:655-656), parallel_scatter_pack_kv_kernel
// (tritonModules.py:72-132, launch modeling_llama.py:658-680) and the run-length
// scatter_add_ (modeling_llama.py:682-685).
//
// pack_scan_kernel (one 1024-thread workgroup per (batch, kv head)): the keep mask is
// read in 64-row groups, 32 groups per wave at once; a ballot gives each group's
// anchor count and first anchor.  A
// block-wide exclusive scan gives every group's first packed index and a suffix
// minimum gives the first anchor after each group, which ends the run of the
// group's last anchor.  The head's anchor count c goes to anchor_counts.
//
// pack_scatter_kernel (one wave per 64-row group): rank = popcount of the lower
// keep bits, packed index = group offset + rank, timestamp = row, count = next
// anchor - row (the number of rows index_map sends to this anchor).  The wave
// copies the anchor rows of K and V (one coalesced row per step) and every
// workgroup zero-fills its share of the padding rows [c, P) of its head, so the
// packed tensors equal the reference's zero-initialised ones.  P = max_g c_g is
// computed on the device and written to num_packed.
//
// Both kernels also take a ragged batch (SeqMap with cu_seqlens): sequence b is then
// packed exactly as a B = 1 batch of its own length -- its own anchors, counts and
// P_b = max over its heads, written to num_packed[b] -- into rows [0, P_b) of its
// slice of the token-major outputs.
#include "da_common.hpp"

namespace da {

constexpr int kMaxGroups = 8192;  // N <= 524288

__device__ __forceinline__ int wave_incl_scan_add(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

__device__ __forceinline__ int wave_incl_scan_min(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d, 64);
    if (lane >= d) v = min(v, o);
  }
  return v;
}

__device__ __forceinline__ int wave_reduce_max(int v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = max(v, __shfl_xor(v, d, 64));
  return v;
}

constexpr int kScanThreads = 1024;
constexpr int kScanWaves = kScanThreads / 64;
constexpr int kScanUnroll = 32;  // groups per wave per pass: that many loads in flight

// keep: [B, H, N] (fixed batch) or [H, T] with row h * keep_sh (ragged batch); the
// workspace rows hold ngroups_cap groups per (batch, head).
__global__ __launch_bounds__(kScanThreads) void pack_scan_kernel(const int32_t* __restrict__ keep,
                                                                 int64_t N_fixed, int ngroups_cap,
                                                                 int H, SeqMap seq, int64_t keep_sh,
                                                                 int32_t* __restrict__ ws_off,
                                                                 int32_t* __restrict__ ws_next,
                                                                 int32_t* __restrict__ anchor_counts) {
  __shared__ int32_t s_info[kMaxGroups];  // count | first << 8
  __shared__ int32_t s_wave[kScanWaves];
  __shared__ int32_t s_suffix[kScanThreads];
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t bh = blockIdx.x;
  const int b = (int)(bh / H), h = (int)(bh - (bh / H) * H);
  const int64_t N = seq.cu ? seq.len(b) : N_fixed;
  const int ngroups = (int)((N + 63) / 64);
  const int32_t* krow = seq.cu ? keep + (int64_t)h * keep_sh + seq.start(b) : keep + bh * N_fixed;

  // wave w takes groups 32w .. 32w + 31 of every 32 * kScanWaves.  Rows past the end
  // are clamped to row N - 1 and masked afterwards, so the 32 loads issue without
  // branches (a guarded load is waited for before the next one is issued).
  for (int gb = wid * kScanUnroll; gb < ngroups; gb += kScanWaves * kScanUnroll) {
    int kv[kScanUnroll];
#pragma unroll
    for (int j = 0; j < kScanUnroll; ++j) {
      const int64_t r = (int64_t)(gb + j) * 64 + lane;
      kv[j] = krow[r < N ? r : N - 1];
    }
#pragma unroll
    for (int j = 0; j < kScanUnroll; ++j) {
      const int64_t r = (int64_t)(gb + j) * 64 + lane;
      const uint64_t bits = __ballot(r < N && kv[j] != 0);
      if (lane == 0 && gb + j < ngroups) {
        const int cnt = __popcll(bits);
        const int first = bits ? __builtin_ctzll(bits) : 64;
        s_info[gb + j] = cnt | (first << 8);
      }
    }
  }
  __syncthreads();

  // Each thread owns a contiguous slice of groups.
  const int per = (ngroups + kScanThreads - 1) / kScanThreads;
  const int g0 = min(tid * per, ngroups), g1 = min(g0 + per, ngroups);
  int sum = 0;
  int first_pos = (int)N;  // first anchor inside the slice (N if none)
  for (int g = g1 - 1; g >= g0; --g) {
    const int info = s_info[g];
    sum += info & 0xff;
    if (info & 0xff) first_pos = g * 64 + (info >> 8);
  }
  // exclusive prefix sum of the slice sums
  int incl = wave_incl_scan_add(sum, lane);
  if (lane == 63) s_wave[wid] = incl;
  __syncthreads();
  int wave_prefix = 0, total = 0;
  for (int w2 = 0; w2 < kScanWaves; ++w2) {
    if (w2 < wid) wave_prefix += s_wave[w2];
    total += s_wave[w2];
  }
  int run = wave_prefix + incl - sum;
  __syncthreads();
  // suffix minimum of first_pos over later slices: scan the reversed sequence
  s_suffix[tid] = first_pos;
  __syncthreads();
  const int rv = s_suffix[kScanThreads - 1 - tid];
  int rincl = wave_incl_scan_min(rv, lane);
  if (lane == 63) s_wave[wid] = rincl;
  __syncthreads();
  int rpre = (int)N;
  for (int w2 = 0; w2 < wid; ++w2) rpre = min(rpre, s_wave[w2]);
  rincl = min(rincl, rpre);  // min over original slices [kScanThreads - 1 - tid, end)
  __syncthreads();
  s_suffix[kScanThreads - 1 - tid] = rincl;
  __syncthreads();
  int nxt = (tid < kScanThreads - 1) ? s_suffix[tid + 1] : (int)N;

  int32_t* off_row = ws_off + bh * ngroups_cap;
  int32_t* next_row = ws_next + bh * ngroups_cap;
  for (int g = g0; g < g1; ++g) {
    off_row[g] = run;
    run += s_info[g] & 0xff;
  }
  for (int g = g1 - 1; g >= g0; --g) {
    next_row[g] = nxt;
    const int info = s_info[g];
    if (info & 0xff) nxt = g * 64 + (info >> 8);
  }
  if (tid == 0) anchor_counts[bh] = total;
}

// Packed outputs: K-hat / V-hat row j of (b, h) at kp + base(b) + h * sp_h + j * sp_n, its
// timestamp and count at ts / cnt + base_c(b) + h * sc_h + j.  A fixed batch uses
// contiguous [B, H, capacity, D] / [B, H, capacity] tensors; a ragged batch token-major
// [T, H, D] / head-major [H, T] ones, with capacity N_b for sequence b.
struct PackOut {
  uint16_t* kp;
  uint16_t* vp;
  int32_t* ts;
  int32_t* cnt;
  int64_t sp_b, sp_h, sp_n;
  int64_t sc_b, sc_h;
  int64_t capacity;  // fixed batch
};

// VEC: K, V and the packed rows are 16-byte aligned with D a multiple of 8, and each
// anchor row moves as 16-byte chunks, four rows per load instruction.  D counts 16-bit
// words (rows of fp32 elements are moved as twice as many words): up to 256, a row in
// one or two passes of 16 chunks (VEC) or 64 words.
template <bool VEC>
__global__ __launch_bounds__(256) void pack_scatter_kernel(
    const int32_t* __restrict__ keep, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, int64_t sk_b, int64_t sk_h, int64_t sk_n, int64_t sv_b,
    int64_t sv_h, int64_t sv_n, int Hkv, int64_t N_fixed, int D, int ngroups_cap, int BH,
    SeqMap seq, int64_t keep_sh, PackOut po, const int32_t* __restrict__ ws_off,
    const int32_t* __restrict__ ws_next, const int32_t* __restrict__ anchor_counts,
    int32_t* __restrict__ num_packed) {
  __shared__ int s_rows[VEC ? 4 : 1][64];  // a wave's anchor rows in packed order
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / Hkv, h = bh - (bh / Hkv) * Hkv;
  const int g = blockIdx.x * 4 + wid;
  const int64_t N = seq.cu ? seq.len((int)b) : N_fixed;
  const int ngroups = (int)((N + 63) / 64);
  const int64_t capacity = seq.cu ? N : po.capacity;

  // P: over every (batch, head) of a fixed batch (modeling_llama.py:656), over the heads
  // of this sequence for a ragged one
  int P = 0;
  if (seq.cu) {
    for (int i = lane; i < Hkv; i += 64) P = max(P, anchor_counts[b * Hkv + i]);
  } else {
    for (int i = lane; i < BH; i += 64) P = max(P, anchor_counts[i]);
  }
  P = wave_reduce_max(P);
  const int c = anchor_counts[bh];
  if (blockIdx.x == 0 && tid == 0) {
    if (seq.cu && h == 0) num_packed[b] = P;
    else if (!seq.cu && bh == 0) *num_packed = P;
  }

  const int64_t kp_row0 = seq.base((int)b, po.sp_b, po.sp_n) + h * po.sp_h;  // packed row 0 of this head
  const int64_t c_row0 = seq.base((int)b, po.sc_b, 1) + h * po.sc_h;
  const int32_t* krow = seq.cu ? keep + h * keep_sh + seq.start((int)b) : keep + bh * N_fixed;
  const int nw = D >> 1;               // 4-byte words per row
  if (g < ngroups) {
    const int64_t r = (int64_t)g * 64 + lane;
    const bool is_anchor = r < N && krow[r] != 0;
    const uint64_t bits = __ballot(is_anchor);
    const int off = ws_off[bh * ngroups_cap + g];
    if (is_anchor) {
      const int rank = __popcll(bits & ((1ull << lane) - 1ull));
      const uint64_t higher = (lane == 63) ? 0ull : (bits >> (lane + 1)) << (lane + 1);
      const int next = higher ? g * 64 + __builtin_ctzll(higher) : ws_next[bh * ngroups_cap + g];
      const int64_t dst = off + rank;
      if (dst < capacity) {
        po.ts[c_row0 + dst] = (int32_t)r;                // tritonModules.py:131-132
        po.cnt[c_row0 + dst] = (int32_t)(next - r);      // modeling_llama.py:683-685
      }
      if (VEC) s_rows[wid][rank] = lane;
    }
    if (VEC) {
      // sixteen anchor rows per step: lane (sub, c) moves 16-byte chunk c of row sub + 4i
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
      const int na = __popcll(bits);
      const int sub = lane >> 4;
      for (int c0 = 0; c0 < (D >> 3); c0 += 16)
      for (int j0 = 0; j0 < na; j0 += 16) {
        const int cq = c0 + (lane & 15);
        const bool actq = cq < (D >> 3);
        const uint16_t* kbase = k + seq.base((int)b, sk_b, sk_n) + h * sk_h + 8 * cq;
        const uint16_t* vbase = v + seq.base((int)b, sv_b, sv_n) + h * sv_h + 8 * cq;
        uint4 kw[4], vw[4];
        int64_t dj[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = j0 + 4 * i + sub;
          const bool ok = actq && j < na;
          const int64_t src = (int64_t)g * 64 + (ok ? s_rows[wid][j] : 0);
          dj[i] = ok ? off + j : -1;
          kw[i] = ok ? *(const uint4*)(kbase + src * sk_n) : uint4{0u, 0u, 0u, 0u};
          vw[i] = ok ? *(const uint4*)(vbase + src * sv_n) : uint4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (dj[i] >= 0 && dj[i] < capacity) {
            *(uint4*)(po.kp + kp_row0 + dj[i] * po.sp_n + 8 * cq) = kw[i];
            *(uint4*)(po.vp + kp_row0 + dj[i] * po.sp_n + 8 * cq) = vw[i];
          }
        }
      }
    }
    // Copy the anchor rows, sixteen rows per step so that their loads are in flight
    // together (a 64-row group holds about 64 / r anchors).
    constexpr int kRows = 16;
    for (int w0 = 0; w0 < (VEC ? 0 : nw); w0 += 64) {
    const int wl = w0 + lane;
    const uint16_t* kbase = k + seq.base((int)b, sk_b, sk_n) + h * sk_h + 2 * wl;
    const uint16_t* vbase = v + seq.base((int)b, sv_b, sv_n) + h * sv_h + 2 * wl;
    const bool act = wl < nw;
    uint64_t rem = bits;
    int64_t dst = off;
    while (rem) {
      int rows[kRows];
      int nr = 0;
#pragma unroll
      for (int j = 0; j < kRows; ++j) {
        rows[j] = rem ? (int)__builtin_ctzll(rem) : -1;
        if (rem) {
          rem &= rem - 1ull;
          ++nr;
        }
      }
      uint32_t kw[kRows], vw[kRows];
#pragma unroll
      for (int j = 0; j < kRows; ++j) {
        const int64_t src = (int64_t)g * 64 + rows[j];
        kw[j] = (act && j < nr) ? *(const uint32_t*)(kbase + src * sk_n) : 0u;
        vw[j] = (act && j < nr) ? *(const uint32_t*)(vbase + src * sv_n) : 0u;
      }
#pragma unroll
      for (int j = 0; j < kRows; ++j) {
        const int64_t d = dst + j;
        if (act && j < nr && d < capacity) {
          *(uint32_t*)(po.kp + kp_row0 + d * po.sp_n + 2 * wl) = kw[j];
          *(uint32_t*)(po.vp + kp_row0 + d * po.sp_n + 2 * wl) = vw[j];
        }
      }
      dst += nr;
    }
    }
  }

  // Zero padding rows [c, min(P, capacity)) of this head, 256 rows per workgroup; most
  // workgroups have none and skip the loop.
  const int64_t pad_end = (P < capacity) ? P : capacity;
  const int64_t r0 = (int64_t)c + (int64_t)blockIdx.x * 256;
  if (r0 < pad_end) {
    const int nrows = pad_end - r0 < 256 ? (int)(pad_end - r0) : 256;
    for (int i = tid; i < nrows * nw; i += 256) {
      const int rr = i / nw;
      const int wd = i - rr * nw;
      const int64_t row = r0 + rr;
      *(uint32_t*)(po.kp + kp_row0 + row * po.sp_n + 2 * wd) = 0u;
      *(uint32_t*)(po.vp + kp_row0 + row * po.sp_n + 2 * wd) = 0u;
      if (wd == 0) {
        po.ts[c_row0 + row] = 0;
        po.cnt[c_row0 + row] = 0;
      }
    }
  }
}

}  // namespace da

using namespace da;

extern "C" int64_t da_pack_workspace_size(int64_t B, int64_t Hkv, int64_t N) {
  const int64_t ngroups = (N + 63) / 64;
  return 2 * B * Hkv * ngroups * (int64_t)sizeof(int32_t);
}

// Launch of the two kernels for a fixed batch (seq.cu null) or a ragged one.
static int launch_pack(const char* who, const int32_t* keep, const void* k, const void* v, int64_t B, int64_t Hkv,
                       int64_t N_fixed, int64_t D, int64_t sk_b, int64_t sk_h, int64_t sk_n, int64_t sv_b,
                       int64_t sv_h, int64_t sv_n, int64_t ngroups, SeqMap seq, int64_t keep_sh, PackOut po,
                       int32_t* anchor_counts, int32_t* num_packed, void* workspace, hipStream_t st) {
  int32_t* ws_off = (int32_t*)workspace;
  int32_t* ws_next = ws_off + B * Hkv * ngroups;
  hipLaunchKernelGGL(pack_scan_kernel, dim3((unsigned)(B * Hkv)), dim3(kScanThreads), 0, st, keep, N_fixed,
                     (int)ngroups, (int)Hkv, seq, keep_sh, ws_off, ws_next, anchor_counts);
  if (int rc = check_launch(who)) return rc;
  const bool vec = (D & 7) == 0 && ((sk_b | sk_h | sk_n | sv_b | sv_h | sv_n | po.sp_b | po.sp_h | po.sp_n) & 7) == 0 &&
                   (((uintptr_t)k | (uintptr_t)v | (uintptr_t)po.kp | (uintptr_t)po.vp) & 15) == 0;
  const dim3 grid((unsigned)((ngroups + 3) / 4), (unsigned)(B * Hkv));
  if (vec)
    hipLaunchKernelGGL(pack_scatter_kernel<true>, grid, dim3(256), 0, st, keep, (const uint16_t*)k,
                       (const uint16_t*)v, sk_b, sk_h, sk_n, sv_b, sv_h, sv_n, (int)Hkv, N_fixed, (int)D,
                       (int)ngroups, (int)(B * Hkv), seq, keep_sh, po, ws_off, ws_next, anchor_counts, num_packed);
  else
    hipLaunchKernelGGL(pack_scatter_kernel<false>, grid, dim3(256), 0, st, keep, (const uint16_t*)k,
                       (const uint16_t*)v, sk_b, sk_h, sk_n, sv_b, sv_h, sv_n, (int)Hkv, N_fixed, (int)D,
                       (int)ngroups, (int)(B * Hkv), seq, keep_sh, po, ws_off, ws_next, anchor_counts, num_packed);
  return check_launch(who);
}

extern "C" int da_pack(const int32_t* keep, const void* k, const void* v, int dtype, int64_t B,
                       int64_t Hkv, int64_t N, int64_t D, int64_t sk_b, int64_t sk_h, int64_t sk_n,
                       int64_t sv_b, int64_t sv_h, int64_t sv_n, int64_t capacity, void* k_packed,
                       void* v_packed, int32_t* timestamps, int32_t* counts,
                       int32_t* anchor_counts, int32_t* num_packed, void* workspace,
                       int64_t workspace_bytes, void* stream) {
  DA_REQUIRE(keep && k && v && k_packed && v_packed && timestamps && counts && anchor_counts &&
                 num_packed,
             "da_pack: null pointer");
  if (dtype != DA_BF16 && dtype != DA_F16 && dtype != DA_F32)
    return set_error(DA_ERR_UNSUPPORTED, "da_pack: K and V must be bf16, fp16 or fp32");
  DA_REQUIRE(B > 0 && Hkv > 0 && N > 0 && D > 0 && capacity > 0, "da_pack: empty shape");
  if (D > 128 || (D & 1)) return set_error(DA_ERR_UNSUPPORTED, "da_pack: head_dim must be even and <= 128");
  if (dtype == DA_F32) {  // the rows move as 16-bit words: twice as many, at twice the strides
    D *= 2;
    sk_b *= 2, sk_h *= 2, sk_n *= 2, sv_b *= 2, sv_h *= 2, sv_n *= 2;
  }
  const int64_t ngroups = (N + 63) / 64;
  if (ngroups > kMaxGroups) return set_error(DA_ERR_UNSUPPORTED, "da_pack: sequence longer than %d", kMaxGroups * 64);
  DA_REQUIRE(B * Hkv < 65536, "da_pack: too many heads");
  DA_REQUIRE(((sk_b | sk_h | sk_n | sv_b | sv_h | sv_n) & 1) == 0 && ((uintptr_t)k & 3) == 0 &&
                 ((uintptr_t)v & 3) == 0 && ((uintptr_t)k_packed & 3) == 0 &&
                 ((uintptr_t)v_packed & 3) == 0,
             "da_pack: rows must be 4-byte aligned");
  if (!workspace || workspace_bytes < da_pack_workspace_size(B, Hkv, N))
    return set_error(DA_ERR_WORKSPACE, "da_pack: workspace of %lld bytes required",
                     (long long)da_pack_workspace_size(B, Hkv, N));
  PackOut po = {(uint16_t*)k_packed, (uint16_t*)v_packed, timestamps, counts,
                Hkv * capacity * D, capacity * D, D, Hkv * capacity, capacity, capacity};
  return launch_pack("da_pack", keep, k, v, B, Hkv, N, D, sk_b, sk_h, sk_n, sv_b, sv_h, sv_n, ngroups,
                     SeqMap{nullptr, 0, (int)N}, N, po, anchor_counts, num_packed, workspace, (hipStream_t)stream);
}

extern "C" int64_t da_pack_varlen_workspace_size(int64_t B, int64_t Hkv, int64_t max_seqlen) {
  return da_pack_workspace_size(B, Hkv, max_seqlen);
}

extern "C" int da_pack_varlen(const int32_t* keep, const void* k, const void* v, int dtype, int64_t B,
                              int64_t Hkv, int64_t T, int64_t D, int64_t sk_t, int64_t sk_h, int64_t sv_t,
                              int64_t sv_h, const int32_t* cu_seqlens, int64_t max_seqlen, void* k_packed,
                              void* v_packed, int32_t* timestamps, int32_t* counts, int32_t* anchor_counts,
                              int32_t* num_packed, void* workspace, int64_t workspace_bytes, void* stream) {
  const char* who = "da_pack_varlen";
  DA_REQUIRE(keep && k && v && k_packed && v_packed && timestamps && counts && anchor_counts && num_packed &&
                 cu_seqlens,
             "%s: null pointer", who);
  if (dtype != DA_BF16 && dtype != DA_F16 && dtype != DA_F32)
    return set_error(DA_ERR_UNSUPPORTED, "%s: K and V must be bf16, fp16 or fp32", who);
  DA_REQUIRE(B > 0 && Hkv > 0 && T > 0 && D > 0, "%s: empty shape", who);
  if (D > 128 || (D & 1)) return set_error(DA_ERR_UNSUPPORTED, "%s: head_dim must be even and <= 128", who);
  if (dtype == DA_F32) {  // the rows move as 16-bit words: twice as many, at twice the strides
    D *= 2;
    sk_t *= 2, sk_h *= 2, sv_t *= 2, sv_h *= 2;
  }
  DA_REQUIRE(T < (1ll << 31) && max_seqlen > 0 && max_seqlen <= T, "%s: need 0 < max_seqlen <= total tokens < 2^31", who);
  const int64_t ngroups = (max_seqlen + 63) / 64;
  if (ngroups > kMaxGroups) return set_error(DA_ERR_UNSUPPORTED, "%s: sequence longer than %d", who, kMaxGroups * 64);
  DA_REQUIRE(B * Hkv < 65536, "%s: too many heads", who);
  DA_REQUIRE(((sk_t | sk_h | sv_t | sv_h) & 1) == 0 && ((uintptr_t)k & 3) == 0 && ((uintptr_t)v & 3) == 0 &&
                 ((uintptr_t)k_packed & 3) == 0 && ((uintptr_t)v_packed & 3) == 0,
             "%s: rows must be 4-byte aligned", who);
  if (!workspace || workspace_bytes < da_pack_varlen_workspace_size(B, Hkv, max_seqlen))
    return set_error(DA_ERR_WORKSPACE, "%s: workspace of %lld bytes required", who,
                     (long long)da_pack_varlen_workspace_size(B, Hkv, max_seqlen));
  // outputs: K-hat / V-hat token-major [T, Hkv, D], timestamps / counts head-major [Hkv, T]
  PackOut po = {(uint16_t*)k_packed, (uint16_t*)v_packed, timestamps, counts, 0, D, Hkv * D, 0, T, 0};
  return launch_pack(who, keep, k, v, B, Hkv, max_seqlen, D, 0, sk_h, sk_t, 0, sv_h, sv_t, ngroups,
                     SeqMap{cu_seqlens, (int)T, (int)max_seqlen}, T, po, anchor_counts, num_packed, workspace,
                     (hipStream_t)stream);
}
