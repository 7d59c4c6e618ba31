// Delta decoding on gfx950: the compressed-cache update and q_len = 1 attention.
//
// decode_update_kernel replaces fused_hybrid_decode_update_kernel
// (deltaDecoding.py:9-104).  One wave per (batch, kv head): when the exact ring is
// full, the token in slot exact_len % W is evicted and either merged into the last
// packed anchor (count + 1) when it is close enough -- Euclidean dist^2 <= tau^2 or
// cosine >= tau, computed with the same fixed pairwise fp32 tree as the selection --
// or appended as a new anchor (count 1, timestamp total - W).  The new token then
// takes the ring slot.
//
// decode_attn_kernel + decode_combine_kernel replace fused_hybrid_decode_kernel
// (deltaDecoding.py:236-362).  The key list of a kv head is its packed anchors
// [0, length) followed by the ring slots [0, exact_len).  Packed scores get
// + log(count) (so a count-c anchor weighs like c equal keys, and padding with count 0
// gets no weight); ring scores are unmasked.  The list is cut into slices of 64 keys;
// one wave scores a slice for all query heads of the group (the key and value rows
// are read once per group), keeps the slice's max / sum / P.V partials, and the
// combine kernel merges the slices exactly (rescaling by exp(m_s - M)).  As in the
// reference, P is rounded to the cache's 16-bit type before the P.V product while the
// row sum stays fp32.  The cache is bf16 or fp16 (the E16 element type), or fp32
// (decode_attn_f32_kernel: p stays fp32, as the reference's p.to(v.dtype) leaves it).
#include <mutex>

#include "da_common.hpp"

namespace da {

struct DecodeUpdateArgs {
  const uint16_t* new_k;
  const uint16_t* new_v;
  int64_t sn_b, sn_h;
  uint16_t* kx;
  uint16_t* vx;
  int64_t sx_b, sx_h, sx_s;
  uint16_t* kp;
  uint16_t* vp;
  int64_t sp_b, sp_h, sp_s;
  int32_t* counts;
  int32_t* ts;
  int64_t sc_b, sc_h;
  int32_t* lengths;
  int64_t capacity;
  int64_t exact_len, total_len, window;
  int B, H, D;
  float thr;
};

// A lane's two elements (dims 2l and 2l + 1) of a cache row: one 32-bit word of a 16-bit
// type, or two fp32 values (8 bytes).
template <int DT>
struct DecPair {
  using Elem = uint16_t;
  using Word = uint32_t;
  static __device__ __forceinline__ float lo(Word w) { return E16<DT>::lo(w); }
  static __device__ __forceinline__ float hi(Word w) { return E16<DT>::hi(w); }
};
template <>
struct DecPair<DA_F32> {
  using Elem = float;
  using Word = u32x2;
  static __device__ __forceinline__ float lo(Word w) { return __uint_as_float(w[0]); }
  static __device__ __forceinline__ float hi(Word w) { return __uint_as_float(w[1]); }
};

// The update's test (deltaDecoding.py:61-77): does the evicted token (this lane's pair
// ek, dims 2l and 2l + 1) merge into the last packed anchor (pair lk)?  Euclidean
// dist^2 <= thr or cosine >= thr, with the selection's fixed fp32 tree; the same result
// in every lane.
template <bool COS, int DT>
__device__ __forceinline__ bool evict_merges(typename DecPair<DT>::Word ek, typename DecPair<DT>::Word lk,
                                             float thr) {
#pragma clang fp contract(off)
  using PT = DecPair<DT>;
  const float e0 = PT::lo(ek), e1 = PT::hi(ek), l0 = PT::lo(lk), l1 = PT::hi(lk);
  if (COS) {
    const float eps = 1e-8f;
    const float dot = wave_tree_sum(pair_dot(e0, e1, l0, l1));
    const float ne = sqrt_rn(wave_tree_sum(pair_dot(e0, e1, e0, e1)) + eps);
    const float nl = sqrt_rn(wave_tree_sum(pair_dot(l0, l1, l0, l1)) + eps);
    return __fdiv_rn(dot, ne * nl) >= thr;
  }
  const float d0 = e0 - l0, d1 = e1 - l1;
  return wave_tree_sum(pair_dot(d0, d1, d0, d1)) <= thr;
}

template <bool COS, int DT>
__global__ __launch_bounds__(256) void decode_update_kernel(DecodeUpdateArgs a) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (w >= a.B * a.H) return;
  const int b = w / a.H, h = w - (w / a.H) * a.H;
  using E = typename DecPair<DT>::Elem;
  using Word = typename DecPair<DT>::Word;
  const bool act = 2 * lane < a.D;
  const int64_t widx = a.exact_len % a.window;                       // :35
  E* ring_k = (E*)(void*)a.kx + b * a.sx_b + h * a.sx_h + 2 * lane;
  E* ring_v = (E*)(void*)a.vx + b * a.sx_b + h * a.sx_h + 2 * lane;
  E* pk = (E*)(void*)a.kp + b * a.sp_b + h * a.sp_h + 2 * lane;
  E* pv = (E*)(void*)a.vp + b * a.sp_b + h * a.sp_h + 2 * lane;
  int32_t* cnt = a.counts + b * a.sc_b + h * a.sc_h;
  int32_t* tsr = a.ts + b * a.sc_b + h * a.sc_h;
  if (a.exact_len >= a.window) {                                     // :54
    const Word ek = act ? *(const Word*)(ring_k + widx * a.sx_s) : Word{};
    const Word ev = act ? *(const Word*)(ring_v + widx * a.sx_s) : Word{};
    const int plen = a.lengths[w];
    bool merge = false;
    if (plen > 0) {                                                  // :61-77
      const Word lk = act ? *(const Word*)(pk + (int64_t)(plen - 1) * a.sp_s) : Word{};
      merge = evict_merges<COS, DT>(ek, lk, a.thr);
    }
    if (merge) {                                                     // :78-82
      if (lane == 0) cnt[plen - 1] += 1;
    } else if (plen < a.capacity) {                                  // :83-96
      if (act) {
        *(Word*)(pk + (int64_t)plen * a.sp_s) = ek;
        *(Word*)(pv + (int64_t)plen * a.sp_s) = ev;
      }
      if (lane == 0) {
        cnt[plen] = 1;
        tsr[plen] = (int32_t)(a.total_len - a.window);
        a.lengths[w] = plen + 1;
      }
    }
  }
  // insert the new token into the ring (:101-104)
  if (act) {
    const Word nk = *(const Word*)((const E*)(const void*)a.new_k + b * a.sn_b + h * a.sn_h + 2 * lane);
    const Word nv = *(const Word*)((const E*)(const void*)a.new_v + b * a.sn_b + h * a.sn_h + 2 * lane);
    *(Word*)(ring_k + widx * a.sx_s) = nk;
    *(Word*)(ring_v + widx * a.sx_s) = nv;
  }
}

constexpr int kDecSlice = 64;
constexpr int kDecMaxG = 8;     // query heads one wave scores (a larger group is split)
constexpr int kDecMaxGroup = 64;
constexpr int kDecD = 128;      // the largest head dimension; partials keep this stride

struct DecodeAttnArgs {
  const uint16_t* q;
  int64_t sq_b, sq_h;
  const uint16_t* kp;
  const uint16_t* vp;
  int64_t sp_b, sp_h, sp_s;
  const int32_t* counts;
  int64_t sc_b, sc_h;
  const int32_t* lengths;
  int64_t capacity;
  const uint16_t* kx;
  const uint16_t* vx;
  int64_t sx_b, sx_h, sx_s;
  int exact_len;
  float scale;
  uint16_t* out;
  int64_t so_b, so_h;
  float* part;      // [B*Hkv][nslice][G][kDecD + 2]: max, sum, P.V partial
  int nslice;
  int B, Hq, Hkv, G;
  int D;            // head dimension: a multiple of 8, at most kDecD
  // da_decode_step's fused update only: the new token, its ring slot widx, whether the
  // ring was full (evict: the token in slot widx leaves it), the update's test, the
  // timestamp base, the writable cache arrays, and per (batch, kv head) two ints in the
  // workspace: the update's decision (0 drop, 1 merge, 2 append) and the key list length
  const uint16_t* new_k;
  const uint16_t* new_v;
  int64_t sn_b, sn_h;
  int widx, evict, cosine;
  float thr;
  int64_t total_len, window;
  int32_t* ts;
  int32_t* fused;
};

__device__ __forceinline__ float wave_max_all(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, d, 64));
  return v;
}
__device__ __forceinline__ float wave_sum_all(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

// One wave per (batch, kv head, 64-key slice, sub-group of at most G query heads of
// the KV head's group: blockIdx.z picks heads G z .. G z + G - 1; where the last
// sub-group runs past the group, its extra slots repeat the group's last head and store
// the same values to the same place).  After the length of the list, lane t's whole key row and the sub-group's
// query rows are loaded together; the slice's 64 value rows are issued as soon as the
// scores are done and arrive during the softmax.  Lane t scores key j0 + t for every
// query head of the sub-group (q broadcast from LDS); the slice max and sum are wave
// reductions; for P.V lane l owns dims 2l and 2l + 1.  Outputs past the head dimension
// are not stored.  FULL (D = 128) loads each key row at immediate offsets from one base;
// the clamped chunk addresses of the general form cost 12% of the attention's time at
// D = 128 (22.5 against 20.0 us per call after the config-1 prefill).
// Small slices keep many waves in flight per CU: the kernel is latency-bound at decode
// sizes, and holding K and V rows at once would halve the waves per SIMD.
//
// FUSED (da_decode_step): the token's cache update enters this launch instead of running
// before it.  The list is the packed anchors [0, plen) (as before the update), the ring
// slots [0, exact_len) with slot widx holding the new token (read from new_k / new_v),
// and, when the ring was full, one extra key jx = plen + exact_len: the evicted token,
// still in slot widx.  Its row never depends on the update's decision; the weights do.
// A merge gives the last anchor count + 1, as the update would, and the extra key weight
// zero; an append gives the extra key count 1, which is the update's new anchor at
// another place in the list; a drop (no room) gives it zero.  So merges and drops score
// exactly the list the update leaves, and an append adds the same terms in another
// order.  The waves whose slice holds key plen - 1 or key jx evaluate the update's test
// (its two rows loaded with the key rows, the test after the scores), and the wave
// holding jx records the decision.  The cache itself is written by the combine kernel,
// after every read of this launch.
template <int G, int DT, bool FULL, bool FUSED>
__global__ __launch_bounds__(64) void decode_attn_kernel(DecodeAttnArgs a) {
  __shared__ float s_q[G][kDecD];
  __shared__ float s_p[G][kDecSlice];
  const int lane = threadIdx.x;
  const int bg = blockIdx.x, slice = blockIdx.y;
  const int hh0 = blockIdx.z * G;  // first query head of the sub-group
  auto head = [&](int hh) { return min(hh0 + hh, a.G - 1); };
  const int D = FULL ? kDecD : a.D;
  // Loads stay unconditional: key chunks past the head dimension repeat its last chunk
  // and meet zero query elements, value lanes past it read its last pair and their
  // partials are never stored
  const int dlast8 = D / 8 - 1;
  const int vdim = FULL ? 2 * lane : min(2 * lane, D - 2);
  const int b = bg / a.Hkv, g = bg - (bg / a.Hkv) * a.Hkv;
  int plen = a.lengths[bg];
  plen = plen < 0 ? 0 : (plen > a.capacity ? (int)a.capacity : plen);
  const int jx = plen + a.exact_len;                   // the extra key's index (FUSED)
  const int total = jx + (FUSED && a.evict ? 1 : 0);
  const int j0 = slice * kDecSlice;
  if (FUSED && slice == 0 && blockIdx.z == 0 && lane == 0) a.fused[2 * bg + 1] = total;
  if (j0 >= total) return;  // the combine kernel skips slices past the end
  const uint16_t* const pk_row0 = a.kp + b * a.sp_b + g * a.sp_h;
  const uint16_t* const pv_row0 = a.vp + b * a.sp_b + g * a.sp_h;
  const uint16_t* const xk_row0 = a.kx + b * a.sx_b + g * a.sx_h;
  const uint16_t* const xv_row0 = a.vx + b * a.sx_b + g * a.sx_h;
  // FUSED: the waves whose slice holds the last anchor or the extra key need the update's
  // decision; the two rows it compares are loaded first, the test waits for the scores
  const bool holds_last = FUSED && plen > 0 && plen - 1 >= j0 && plen - 1 < j0 + kDecSlice;
  const bool holds_extra = FUSED && jx < j0 + kDecSlice;  // jx >= j0: slice j0 is not past the end
  const bool need_dec = FUSED && a.evict && (holds_last || holds_extra);
  uint32_t ek = 0u, lk = 0u;
  if (need_dec && 2 * lane < D) {
    ek = *(const uint32_t*)(xk_row0 + (int64_t)a.widx * a.sx_s + 2 * lane);
    if (plen > 0) lk = *(const uint32_t*)(pk_row0 + (int64_t)(plen - 1) * a.sp_s + 2 * lane);
  }
  // the key / value row of list index jj (FUSED: the new token in ring slot widx, and the
  // extra key jx, the evicted token, still in that slot)
  auto key_row = [&](int jj, const uint16_t* p0, const uint16_t* x0, const uint16_t* nw) -> const uint16_t* {
    if (jj < plen) return p0 + (int64_t)jj * a.sp_s;
    const int r = FUSED && jj >= jx ? a.widx : jj - plen;
    if (FUSED && r == a.widx && jj < jx) return nw + b * a.sn_b + g * a.sn_h;
    return x0 + (int64_t)r * a.sx_s;
  };

  // This lane's key row and count and the group's query rows (G * D / 64 elements per
  // lane) go out together, before the first wait.
  const int j = j0 + lane;
  const bool valid = j < total;
  u32x4 kw[kDecD / 8];
  int cnt = 1;
  if (valid) {
    const uint16_t* krow = key_row(j, pk_row0, xk_row0, a.new_k);
#pragma unroll
    for (int c8 = 0; c8 < kDecD / 8; ++c8) kw[c8] = *(const u32x4*)(krow + 8 * (FULL ? c8 : min(c8, dlast8)));
    if (j < plen) cnt = a.counts[b * a.sc_b + g * a.sc_h + j];
  }
  constexpr int kQPerLane = G * kDecD / 64;
  uint16_t qh[kQPerLane];
#pragma unroll
  for (int it = 0; it < kQPerLane; ++it) {
    const int i = lane + 64 * it, hh = i / kDecD, d = i - hh * kDecD;
    qh[it] = FULL || d < D ? a.q[b * a.sq_b + (int64_t)(g * a.G + head(hh)) * a.sq_h + d] : (uint16_t)0;
  }
#pragma unroll
  for (int it = 0; it < kQPerLane; ++it) {
    const int i = lane + 64 * it, hh = i / kDecD, d = i - hh * kDecD;
    s_q[hh][d] = E16<DT>::one(qh[it]);
  }
  __syncthreads();

  // ---- scores: lane t scores key j0 + t for every query head of the group ----
  float sc[G];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) sc[hh] = -INFINITY;
  // q . k for the group's heads (this lane's key row)
  auto dot_group = [&](float (&acc)[G]) {
#pragma unroll
    for (int hh = 0; hh < G; ++hh) acc[hh] = 0.0f;
#pragma unroll
    for (int c8 = 0; c8 < kDecD / 8; ++c8) {
      const u32x4 w = kw[c8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float k0 = E16<DT>::lo(w[e]), k1 = E16<DT>::hi(w[e]);
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
          acc[hh] = __builtin_fmaf(s_q[hh][8 * c8 + 2 * e], k0, acc[hh]);
          acc[hh] = __builtin_fmaf(s_q[hh][8 * c8 + 2 * e + 1], k1, acc[hh]);
        }
      }
    }
  };
  // log(count) bias; log(0) = -inf: padding anchors get no weight (:309-311); ring keys
  // weigh one
  auto bias_of = [&](int c) {
    return j >= plen && (!FUSED || j < jx) ? 0.0f : (c <= 0 ? -INFINITY : __logf((float)c));
  };
  if constexpr (!FUSED) {
    if (valid) {
      const float bias = bias_of(cnt);
      float acc[G];
      dot_group(acc);
#pragma unroll
      for (int hh = 0; hh < G; ++hh) sc[hh] = acc[hh] * a.scale + bias;
    }
  } else {
    float acc[G];
    if (valid) dot_group(acc);
    // the update's decision (deltaDecoding.py:61-96): a merge weighs the last anchor with
    // count + 1, an append gives the evicted token (key jx) weight one, a drop (no room)
    // weight zero; the extra key of a merge or drop carries no weight.  Every lane runs
    // the test (wave reductions).
    if (need_dec) {
      const bool merge = plen > 0 && (a.cosine ? evict_merges<true, DT>(ek, lk, a.thr)
                                               : evict_merges<false, DT>(ek, lk, a.thr));
      const int dec = merge ? 1 : (plen < a.capacity ? 2 : 0);
      if (holds_extra && blockIdx.z == 0 && lane == 0) a.fused[2 * bg] = dec;
      if (j == plen - 1 && dec == 1) cnt += 1;
      if (j == jx) cnt = dec == 2 ? 1 : 0;
    }
    if (valid) {
      const float bias = bias_of(cnt);
#pragma unroll
      for (int hh = 0; hh < G; ++hh) sc[hh] = acc[hh] * a.scale + bias;
    }
  }

  // ---- the slice's 64 value rows (rows past the end load nothing and carry p = 0),
  // in flight during the softmax ----
  // A slice of packed anchors only (most of them) reads its rows at one stride from one
  // base.  In the others, lane t finds the source of row j0 + t (clamped to the list's
  // last key: every pointer is a real row) and row u's loads take lane u's pointer; rows
  // past the end carry p = 0.
  uint32_t vw[kDecSlice];
  if (j0 + kDecSlice <= plen) {
    const uint16_t* vrow = pv_row0 + (int64_t)j0 * a.sp_s + vdim;
#pragma unroll
    for (int u = 0; u < kDecSlice; ++u) vw[u] = *(const uint32_t*)(vrow + (int64_t)u * a.sp_s);
  } else {
    const uint64_t mine = (uint64_t)key_row(min(j, total - 1), pv_row0, xv_row0, a.new_v);
    const uint32_t lo = (uint32_t)mine, hi = (uint32_t)(mine >> 32);
    const uint32_t voff = 2u * (uint32_t)vdim;  // bytes; unsigned, for scalar base + vector offset
#pragma unroll
    for (int u = 0; u < kDecSlice; ++u) {
      const uint64_t row = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, u) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane(lo, u);
      vw[u] = *(const __attribute__((address_space(1))) uint32_t*)(row + voff);  // a global load
      // in groups of 16 rows: the addresses are not all formed ahead of the loads
      if ((u & 15) == 15) __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- per-head slice max and sum; weights rounded to the cache's type, to LDS ----
  float* part = a.part + ((int64_t)bg * a.nslice + slice) * a.G * (kDecD + 2);
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    if (hh < G) {
      const float m = wave_max_all(sc[hh]);
      const float p = (sc[hh] == -INFINITY) ? 0.0f : __expf(sc[hh] - m);
      const float l = wave_sum_all(p);
      s_p[hh][lane] = E16<DT>::one(E16<DT>::bits(p));  // p rounded to the cache's type
      if (lane == 0) {
        part[head(hh) * (kDecD + 2)] = m;
        part[head(hh) * (kDecD + 2) + 1] = l;
      }
    }
  }
  __syncthreads();

  // ---- P.V: lane l owns dims 2l, 2l+1 ----
  float av[G][2];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) av[hh][0] = av[hh][1] = 0.0f;
#pragma unroll
  for (int u = 0; u < kDecSlice; ++u) {
    const float v0 = E16<DT>::lo(vw[u]), v1 = E16<DT>::hi(vw[u]);
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
      av[hh][0] = __builtin_fmaf(s_p[hh][u], v0, av[hh][0]);
      av[hh][1] = __builtin_fmaf(s_p[hh][u], v1, av[hh][1]);
    }
  }
#pragma unroll
  for (int hh = 0; hh < G; ++hh)
    {
      part[head(hh) * (kDecD + 2) + 2 + 2 * lane] = av[hh][0];
      part[head(hh) * (kDecD + 2) + 3 + 2 * lane] = av[hh][1];
    }
}

// fp32 caches: the reference's kernels load the cache's own type and compute in fp32, and
// P.V takes p in the cache's type (deltaDecoding.py:319), here fp32 itself, unrounded.
// Slices, partials and the combine are decode_attn_kernel's.  A key row is D fp32 values
// (twice the bytes of a 16-bit row), so lane t reads its row eight 16-byte chunks at a
// time and the slice's value rows go in four batches of 16 (8 bytes per lane each), which
// keeps the wave's registers near the 16-bit kernel's.  Value rows: lane t finds the
// source of row j0 + t (clamped to the list's last key) and row u's loads take lane u's
// pointer, as in the 16-bit kernel's mixed slices.
template <int G>
__global__ __launch_bounds__(64) void decode_attn_f32_kernel(DecodeAttnArgs a) {
  __shared__ float s_q[G][kDecD];
  __shared__ float s_p[G][kDecSlice];
  const int lane = threadIdx.x;
  const int bg = blockIdx.x, slice = blockIdx.y;
  const int hh0 = blockIdx.z * G;
  auto head = [&](int hh) { return min(hh0 + hh, a.G - 1); };
  const int D = a.D;
  const int b = bg / a.Hkv, g = bg - (bg / a.Hkv) * a.Hkv;
  int plen = a.lengths[bg];
  plen = plen < 0 ? 0 : (plen > a.capacity ? (int)a.capacity : plen);
  const int total = plen + a.exact_len;
  const int j0 = slice * kDecSlice;
  if (j0 >= total) return;  // the combine kernel skips slices past the end
  const float* const pk_row0 = (const float*)(const void*)a.kp + b * a.sp_b + g * a.sp_h;
  const float* const pv_row0 = (const float*)(const void*)a.vp + b * a.sp_b + g * a.sp_h;
  const float* const xk_row0 = (const float*)(const void*)a.kx + b * a.sx_b + g * a.sx_h;
  const float* const xv_row0 = (const float*)(const void*)a.vx + b * a.sx_b + g * a.sx_h;
  auto row_of = [&](int jj, const float* p0, const float* x0) -> const float* {
    return jj < plen ? p0 + (int64_t)jj * a.sp_s : x0 + (int64_t)(jj - plen) * a.sx_s;
  };

  const float* const q = (const float*)(const void*)a.q;
  constexpr int kQPerLane = G * kDecD / 64;
#pragma unroll
  for (int it = 0; it < kQPerLane; ++it) {
    const int i = lane + 64 * it, hh = i / kDecD, d = i - hh * kDecD;
    s_q[hh][d] = d < D ? q[b * a.sq_b + (int64_t)(g * a.G + head(hh)) * a.sq_h + d] : 0.0f;
  }
  __syncthreads();

  // ---- scores: lane t scores key j0 + t for every query head of the sub-group ----
  const int j = j0 + lane;
  const bool valid = j < total;
  float sc[G];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) sc[hh] = -INFINITY;
  if (valid) {
    const float* krow = row_of(j, pk_row0, xk_row0);
    const int cnt = j < plen ? a.counts[b * a.sc_b + g * a.sc_h + j] : 1;
    float acc[G];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) acc[hh] = 0.0f;
#pragma unroll
    for (int c0 = 0; c0 < kDecD / 4; c0 += 8) {
      if (4 * c0 < D) {  // D is a multiple of 8: a chunk of four is all in or all out
        f32x4 kk[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
          kk[u] = 4 * (c0 + u) < D ? *(const f32x4*)(krow + 4 * (c0 + u)) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int hh = 0; hh < G; ++hh) acc[hh] = __builtin_fmaf(s_q[hh][4 * (c0 + u) + e], kk[u][e], acc[hh]);
      }
    }
    // log(count) bias; log(0) = -inf: padding anchors get no weight (:309-311)
    const float bias = j >= plen ? 0.0f : (cnt <= 0 ? -INFINITY : __logf((float)cnt));
#pragma unroll
    for (int hh = 0; hh < G; ++hh) sc[hh] = acc[hh] * a.scale + bias;
  }

  // ---- per-head slice max and sum; p (fp32) to LDS ----
  float* part = a.part + ((int64_t)bg * a.nslice + slice) * a.G * (kDecD + 2);
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    const float m = wave_max_all(sc[hh]);
    const float p = (sc[hh] == -INFINITY) ? 0.0f : __expf(sc[hh] - m);
    const float l = wave_sum_all(p);
    s_p[hh][lane] = p;
    if (lane == 0) {
      part[head(hh) * (kDecD + 2)] = m;
      part[head(hh) * (kDecD + 2) + 1] = l;
    }
  }
  __syncthreads();

  // ---- P.V: lane l owns dims 2l, 2l+1 (lanes past the head dimension read its last
  // pair; their partials are never stored by the combine) ----
  const int vdim = min(2 * lane, D - 2);
  const uint64_t mine = (uint64_t)row_of(min(j, total - 1), pv_row0, xv_row0);
  const uint32_t lo = (uint32_t)mine, hi = (uint32_t)(mine >> 32);
  const uint32_t voff = 4u * (uint32_t)vdim;  // bytes
  float av[G][2];
#pragma unroll
  for (int hh = 0; hh < G; ++hh) av[hh][0] = av[hh][1] = 0.0f;
#pragma unroll
  for (int u0 = 0; u0 < kDecSlice; u0 += 16) {
    f32x2 vv[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const uint64_t row = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(hi, u0 + u) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane(lo, u0 + u);
      vv[u] = *(const __attribute__((address_space(1))) f32x2*)(row + voff);  // a global load
    }
#pragma unroll
    for (int u = 0; u < 16; ++u)
#pragma unroll
      for (int hh = 0; hh < G; ++hh) {
        av[hh][0] = __builtin_fmaf(s_p[hh][u0 + u], vv[u][0], av[hh][0]);
        av[hh][1] = __builtin_fmaf(s_p[hh][u0 + u], vv[u][1], av[hh][1]);
      }
    __builtin_amdgcn_sched_barrier(0);  // one batch of rows in flight at a time
  }
#pragma unroll
  for (int hh = 0; hh < G; ++hh) {
    part[head(hh) * (kDecD + 2) + 2 + 2 * lane] = av[hh][0];
    part[head(hh) * (kDecD + 2) + 3 + 2 * lane] = av[hh][1];
  }
}

// Merge of the slices of one query head, split over kCombParts workgroups of
// kCombDims dims each.  Thread (dim d, phase q) adds dim d of the P.V partials of the
// slices s = q (mod kCombPhases), kCombUnroll slices at a time with all of their loads in
// flight; the first batch (256 slices) goes out together with the slice maxima and sums,
// which each thread folds into a running (max, sum) before one workgroup reduction.
// The phases are added in LDS.
constexpr int kDecMaxSlices = 16384;
constexpr int kCombParts = 4, kCombDims = kDecD / kCombParts, kCombPhases = 256 / kCombDims;
constexpr int kCombUnroll = 32;
//
// FUSED (da_decode_step): the list length comes from the attention launch (the update
// below may change the packed length), and after the merge the workgroup of the
// group's first query head and first dim part writes the token's cache update
// (deltaDecoding.py:54-104) with the attention's decision: a merge adds one to the last
// anchor's count, an append copies the evicted token out of its ring slot into packed
// row plen (count 1, timestamp total - W, length plen + 1), and then the new token takes
// the ring slot.  Every read of the attention launch is done by then (stream order).
template <int DT, bool FUSED>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeAttnArgs a) {
  __shared__ float s_f[kDecMaxSlices];
  __shared__ float s_red[8];
  __shared__ float s_acc[kCombPhases][kCombDims];
  const int bhq = blockIdx.x;
  const int b = bhq / a.Hq, hq = bhq - (bhq / a.Hq) * a.Hq;
  const int g = hq / a.G, hh = hq - g * a.G;
  const int bg = b * a.Hkv + g;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  // FUSED: the writer's reads (the update's decision, the evicted token, the new token,
  // the last anchor's count) go out with the first loads; its writes come at the end
  const bool writer = FUSED && hh == 0 && blockIdx.y == 0 && tid < 64;
  const bool wact = writer && 2 * tid < a.D;
  uint16_t* const ring_k = const_cast<uint16_t*>(a.kx) + b * a.sx_b + g * a.sx_h + (int64_t)a.widx * a.sx_s + 2 * tid;
  uint16_t* const ring_v = const_cast<uint16_t*>(a.vx) + b * a.sx_b + g * a.sx_h + (int64_t)a.widx * a.sx_s + 2 * tid;
  int32_t* const cnt = const_cast<int32_t*>(a.counts) + b * a.sc_b + g * a.sc_h;
  uint32_t ek = 0u, ev = 0u, nk = 0u, nv = 0u;
  int dec = 0;
  if (wact) {
    ek = *(const uint32_t*)ring_k;
    ev = *(const uint32_t*)ring_v;
    nk = *(const uint32_t*)(a.new_k + b * a.sn_b + g * a.sn_h + 2 * tid);
    nv = *(const uint32_t*)(a.new_v + b * a.sn_b + g * a.sn_h + 2 * tid);
  }
  if (writer && a.evict) dec = a.fused[2 * bg];
  int plen = a.lengths[bg];
  plen = plen < 0 ? 0 : (plen > a.capacity ? (int)a.capacity : plen);
  const int c_last = writer && tid == 0 && a.evict && plen > 0 ? cnt[plen - 1] : 0;
  int total = FUSED ? a.fused[2 * bg + 1] : plen + a.exact_len;
  total = total < 0 ? 0 : (total > a.nslice * kDecSlice ? a.nslice * kDecSlice : total);
  const int ns = (total + kDecSlice - 1) / kDecSlice;
  const float* base = a.part + (int64_t)bg * a.nslice * a.G * (kDecD + 2) + hh * (kDecD + 2);
  // 32-bit offsets within one (batch, KV head): nslice * G * (kDecD + 2) stays below
  // 2^31 under the launch's limits (16384 slices, groups of at most 64: 1.4e8)
  const int sstride = a.G * (kDecD + 2);
  // the first batch of P.V partials goes out first: it does not depend on the maxima.
  // Slice indexes past the last are clamped to a slice that exists and masked when
  // added, so the loads issue without branches.
  const int dl = tid & (kCombDims - 1), q = tid / kCombDims;
  const int d = blockIdx.y * kCombDims + dl;
  const int last = ns > 0 ? ns - 1 : 0;
  const float* pv = base + 2 + d;
  float x[kCombUnroll];
#pragma unroll
  for (int u = 0; u < kCombUnroll; ++u)
    x[u] = pv[__builtin_elementwise_min(q + kCombPhases * u, last) * sstride];
  // slice maxima and sums: a running (max, sum) per thread, then over the workgroup
  float m = -INFINITY, l = 0.0f;
  for (int s2 = tid; s2 < ns; s2 += 256) {
    const float ms = base[s2 * sstride], ls = base[s2 * sstride + 1];
    s_f[s2] = ms;
    if (ms == -INFINITY) continue;
    if (ms > m) {
      l = m == -INFINITY ? 0.0f : l * __expf(m - ms);
      m = ms;
    }
    l += ls * __expf(ms - m);
  }
  auto merge = [](float& m1, float& l1, float m2, float l2) {
    const float mm = __builtin_fmaxf(m1, m2);
    if (mm == -INFINITY) return;
    l1 = (m1 == -INFINITY ? 0.0f : l1 * __expf(m1 - mm)) + (m2 == -INFINITY ? 0.0f : l2 * __expf(m2 - mm));
    m1 = mm;
  };
#pragma unroll
  for (int dd = 32; dd >= 1; dd >>= 1) merge(m, l, __shfl_xor(m, dd, 64), __shfl_xor(l, dd, 64));
  if (lane == 0) {
    s_red[wid] = m;
    s_red[4 + wid] = l;
  }
  __syncthreads();
  float M = s_red[0], L = s_red[4];
#pragma unroll
  for (int w2 = 1; w2 < 4; ++w2) merge(M, L, s_red[w2], s_red[4 + w2]);
  // P.V partials of dim d over the slices of this phase
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kCombUnroll; ++u) {
    const int s2 = q + kCombPhases * u;
    const float ms = s2 < ns ? s_f[s2] : -INFINITY;
    acc += ms == -INFINITY ? 0.0f : x[u] * __expf(ms - M);
  }
  for (int s0 = q + kCombPhases * kCombUnroll; s0 < ns; s0 += kCombPhases * kCombUnroll) {
#pragma unroll
    for (int u = 0; u < kCombUnroll; ++u)
      x[u] = pv[__builtin_elementwise_min(s0 + kCombPhases * u, last) * sstride];
#pragma unroll
    for (int u = 0; u < kCombUnroll; ++u) {
      const int s2 = s0 + kCombPhases * u;
      const float ms = s2 < ns ? s_f[s2] : -INFINITY;
      acc += ms == -INFINITY ? 0.0f : x[u] * __expf(ms - M);
    }
  }
  s_acc[q][dl] = acc;
  __syncthreads();
  if (q == 0 && d < a.D) {
    float o = acc;
#pragma unroll
    for (int p = 1; p < kCombPhases; ++p) o += s_acc[p][dl];
    if constexpr (DT == DA_F32)
      ((float*)(void*)a.out)[b * a.so_b + hq * a.so_h + d] = o / L;
    else
      a.out[b * a.so_b + hq * a.so_h + d] = E16<DT>::bits(o / L);
  }
  if constexpr (FUSED) {
    if (writer) {
      if (a.evict) {
        if (dec == 1) {  // :78-82
          if (tid == 0) cnt[plen - 1] = c_last + 1;
        } else if (dec == 2) {  // :83-96
          if (wact) {
            uint16_t* const pk = const_cast<uint16_t*>(a.kp) + b * a.sp_b + g * a.sp_h + (int64_t)plen * a.sp_s + 2 * tid;
            uint16_t* const pv = const_cast<uint16_t*>(a.vp) + b * a.sp_b + g * a.sp_h + (int64_t)plen * a.sp_s + 2 * tid;
            *(uint32_t*)pk = ek;
            *(uint32_t*)pv = ev;
          }
          if (tid == 0) {
            cnt[plen] = 1;
            a.ts[b * a.sc_b + g * a.sc_h + plen] = (int32_t)(a.total_len - a.window);
            const_cast<int32_t*>(a.lengths)[bg] = plen + 1;
          }
        }
      }
      // the new token into the ring (:101-104), in place of the evicted one
      if (wact) {
        *(uint32_t*)ring_k = nk;
        *(uint32_t*)ring_v = nv;
      }
    }
  }
}

}  // namespace da

using namespace da;

// Checks and launch of the cache update, shared by da_decode_update and da_decode_step.
static int decode_update_impl(const void* new_k, const void* new_v, int dtype, int64_t B, int64_t Hkv, int64_t D,
                              int64_t sn_b, int64_t sn_h, void* k_exact, void* v_exact, int64_t sx_b,
                              int64_t sx_h, int64_t sx_s, void* k_packed, void* v_packed, int64_t sp_b,
                              int64_t sp_h, int64_t sp_s, int32_t* counts, int32_t* timestamps, int64_t sc_b,
                              int64_t sc_h, int32_t* lengths, int64_t capacity, int64_t exact_seq_len,
                              int64_t total_seq_len, int64_t window, float threshold, int use_cosine,
                              void* stream, const char* who) {
  DA_REQUIRE(new_k && new_v && k_exact && v_exact && k_packed && v_packed && counts && timestamps && lengths,
             "%s: null pointer", who);
  if (dtype != DA_BF16 && dtype != DA_F16 && dtype != DA_F32)
    return set_error(DA_ERR_UNSUPPORTED, "%s: the cache must be bf16, fp16 or fp32", who);
  DA_REQUIRE(B > 0 && Hkv > 0 && window > 0 && capacity > 0, "%s: empty shape", who);
  if (D > 128 || (D & 1)) return set_error(DA_ERR_UNSUPPORTED, "%s: head_dim must be even and <= 128", who);
  DA_REQUIRE(exact_seq_len >= 0 && total_seq_len >= 0, "%s: negative lengths", who);
  // a lane moves an element pair: 4 bytes (16-bit) or 8 bytes (fp32) at once
  const uintptr_t pair_align = dtype == DA_F32 ? 7 : 3;
  DA_REQUIRE(((sn_b | sn_h | sx_b | sx_h | sx_s | sp_b | sp_h | sp_s) & 1) == 0 &&
                 (((uintptr_t)new_k | (uintptr_t)new_v | (uintptr_t)k_exact | (uintptr_t)v_exact |
                   (uintptr_t)k_packed | (uintptr_t)v_packed) & pair_align) == 0,
             "%s: rows must be %d-byte aligned (even strides)", who, dtype == DA_F32 ? 8 : 4);
  DecodeUpdateArgs a = {};
  a.new_k = (const uint16_t*)new_k; a.new_v = (const uint16_t*)new_v; a.sn_b = sn_b; a.sn_h = sn_h;
  a.kx = (uint16_t*)k_exact; a.vx = (uint16_t*)v_exact; a.sx_b = sx_b; a.sx_h = sx_h; a.sx_s = sx_s;
  a.kp = (uint16_t*)k_packed; a.vp = (uint16_t*)v_packed; a.sp_b = sp_b; a.sp_h = sp_h; a.sp_s = sp_s;
  a.counts = counts; a.ts = timestamps; a.sc_b = sc_b; a.sc_h = sc_h; a.lengths = lengths;
  a.capacity = capacity; a.exact_len = exact_seq_len; a.total_len = total_seq_len; a.window = window;
  a.B = (int)B; a.H = (int)Hkv; a.D = (int)D; a.thr = threshold;
  const unsigned blocks = (unsigned)((B * Hkv + 3) / 4);
  hipStream_t st = (hipStream_t)stream;
  if (dtype == DA_F32) {
    if (use_cosine) hipLaunchKernelGGL((decode_update_kernel<true, DA_F32>), dim3(blocks), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((decode_update_kernel<false, DA_F32>), dim3(blocks), dim3(256), 0, st, a);
  } else if (dtype == DA_F16) {
    if (use_cosine) hipLaunchKernelGGL((decode_update_kernel<true, DA_F16>), dim3(blocks), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((decode_update_kernel<false, DA_F16>), dim3(blocks), dim3(256), 0, st, a);
  } else {
    if (use_cosine) hipLaunchKernelGGL((decode_update_kernel<true, DA_BF16>), dim3(blocks), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((decode_update_kernel<false, DA_BF16>), dim3(blocks), dim3(256), 0, st, a);
  }
  return check_launch(who);
}

extern "C" int da_decode_update(const void* new_k, const void* new_v, int dtype, int64_t B,
                                int64_t Hkv, int64_t D, int64_t sn_b, int64_t sn_h, void* k_exact,
                                void* v_exact, int64_t sx_b, int64_t sx_h, int64_t sx_s,
                                void* k_packed, void* v_packed, int64_t sp_b, int64_t sp_h,
                                int64_t sp_s, int32_t* counts, int32_t* timestamps, int64_t sc_b,
                                int64_t sc_h, int32_t* lengths, int64_t capacity,
                                int64_t exact_seq_len, int64_t total_seq_len, int64_t window,
                                float threshold, int use_cosine, void* stream) {
  return decode_update_impl(new_k, new_v, dtype, B, Hkv, D, sn_b, sn_h, k_exact, v_exact, sx_b, sx_h, sx_s,
                            k_packed, v_packed, sp_b, sp_h, sp_s, counts, timestamps, sc_b, sc_h, lengths,
                            capacity, exact_seq_len, total_seq_len, window, threshold, use_cosine, stream,
                            "da_decode_update");
}

template <int DT, bool FULL, bool FUSED>
static int launch_decode_g(DecodeAttnArgs& a, int64_t n_heads, hipStream_t st) {
  // a group above kDecMaxG query heads is split into ceil(G / kDecMaxG) sub-groups of
  // equal size (the last one smaller when G does not divide), one wave each
  const int nsub = (a.G + kDecMaxG - 1) / kDecMaxG;
  const int gw = (a.G + nsub - 1) / nsub;
  const dim3 agrid((unsigned)(a.B * a.Hkv), (unsigned)a.nslice, (unsigned)nsub);
  switch (gw) {
    case 1: hipLaunchKernelGGL((decode_attn_kernel<1, DT, FULL, FUSED>), agrid, dim3(64), 0, st, a); break;
    case 2: hipLaunchKernelGGL((decode_attn_kernel<2, DT, FULL, FUSED>), agrid, dim3(64), 0, st, a); break;
    case 3: hipLaunchKernelGGL((decode_attn_kernel<3, DT, FULL, FUSED>), agrid, dim3(64), 0, st, a); break;
    case 4: hipLaunchKernelGGL((decode_attn_kernel<4, DT, FULL, FUSED>), agrid, dim3(64), 0, st, a); break;
    case 5: hipLaunchKernelGGL((decode_attn_kernel<5, DT, FULL, FUSED>), agrid, dim3(64), 0, st, a); break;
    case 6: hipLaunchKernelGGL((decode_attn_kernel<6, DT, FULL, FUSED>), agrid, dim3(64), 0, st, a); break;
    case 7: hipLaunchKernelGGL((decode_attn_kernel<7, DT, FULL, FUSED>), agrid, dim3(64), 0, st, a); break;
    default: hipLaunchKernelGGL((decode_attn_kernel<8, DT, FULL, FUSED>), agrid, dim3(64), 0, st, a); break;
  }
  if (int rc = check_launch("da_decode_attention")) return rc;
  hipLaunchKernelGGL((decode_combine_kernel<DT, FUSED>), dim3((unsigned)n_heads, kCombParts), dim3(256), 0, st, a);
  return check_launch("da_decode_attention(combine)");
}
static int launch_decode_f32(DecodeAttnArgs& a, int64_t n_heads, hipStream_t st) {
  const int nsub = (a.G + kDecMaxG - 1) / kDecMaxG;
  const int gw = (a.G + nsub - 1) / nsub;
  const dim3 agrid((unsigned)(a.B * a.Hkv), (unsigned)a.nslice, (unsigned)nsub);
  switch (gw) {
    case 1: hipLaunchKernelGGL((decode_attn_f32_kernel<1>), agrid, dim3(64), 0, st, a); break;
    case 2: hipLaunchKernelGGL((decode_attn_f32_kernel<2>), agrid, dim3(64), 0, st, a); break;
    case 3: hipLaunchKernelGGL((decode_attn_f32_kernel<3>), agrid, dim3(64), 0, st, a); break;
    case 4: hipLaunchKernelGGL((decode_attn_f32_kernel<4>), agrid, dim3(64), 0, st, a); break;
    case 5: hipLaunchKernelGGL((decode_attn_f32_kernel<5>), agrid, dim3(64), 0, st, a); break;
    case 6: hipLaunchKernelGGL((decode_attn_f32_kernel<6>), agrid, dim3(64), 0, st, a); break;
    case 7: hipLaunchKernelGGL((decode_attn_f32_kernel<7>), agrid, dim3(64), 0, st, a); break;
    default: hipLaunchKernelGGL((decode_attn_f32_kernel<8>), agrid, dim3(64), 0, st, a); break;
  }
  if (int rc = check_launch("da_decode_attention")) return rc;
  hipLaunchKernelGGL((decode_combine_kernel<DA_F32, false>), dim3((unsigned)n_heads, kCombParts), dim3(256), 0, st,
                     a);
  return check_launch("da_decode_attention(combine)");
}
template <int DT, bool FUSED>
static int launch_decode(DecodeAttnArgs& a, int64_t n_heads, hipStream_t st) {
  return a.D == kDecD ? launch_decode_g<DT, true, FUSED>(a, n_heads, st)
                      : launch_decode_g<DT, false, FUSED>(a, n_heads, st);
}

// Slices of a key list of up to capacity + window keys, plus the extra key of
// da_decode_step's fused update.
static int64_t decode_slices(int64_t capacity, int64_t window) {
  return (capacity + window + 1 + kDecSlice - 1) / kDecSlice;
}

// The slice partials, then (da_decode_step) two ints per (batch, query head).
extern "C" int64_t da_decode_workspace_size(int64_t B, int64_t Hq, int64_t capacity, int64_t window) {
  return B * Hq * decode_slices(capacity, window) * (kDecD + 2) * (int64_t)sizeof(float) +
         2 * B * Hq * (int64_t)sizeof(int32_t);
}

// Validation and launch shared by da_decode_attention and da_decode_attention_noalloc:
// `part` is the slice-partials buffer (caller workspace or the static scratch).
static int decode_attention_impl(const void* q, int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                 int64_t sq_b, int64_t sq_h, const void* k_packed, const void* v_packed,
                                 int64_t sp_b, int64_t sp_h, int64_t sp_s, const int32_t* counts,
                                 int64_t sc_b, int64_t sc_h, const int32_t* lengths, int64_t capacity,
                                 const void* k_exact, const void* v_exact, int64_t sx_b, int64_t sx_h,
                                 int64_t sx_s, int64_t window, int64_t exact_len, float scale, void* out,
                                 int64_t so_b, int64_t so_h, float* part, hipStream_t st) {
  DecodeAttnArgs a = {};
  a.q = (const uint16_t*)q; a.sq_b = sq_b; a.sq_h = sq_h;
  a.kp = (const uint16_t*)k_packed; a.vp = (const uint16_t*)v_packed; a.sp_b = sp_b; a.sp_h = sp_h; a.sp_s = sp_s;
  a.counts = counts; a.sc_b = sc_b; a.sc_h = sc_h; a.lengths = lengths; a.capacity = capacity;
  a.kx = (const uint16_t*)k_exact; a.vx = (const uint16_t*)v_exact; a.sx_b = sx_b; a.sx_h = sx_h; a.sx_s = sx_s;
  a.exact_len = (int)exact_len; a.scale = scale; a.out = (uint16_t*)out; a.so_b = so_b; a.so_h = so_h;
  a.part = part;
  a.nslice = (int)((capacity + window + kDecSlice - 1) / kDecSlice);
  a.B = (int)B; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.G = (int)(Hq / Hkv); a.D = (int)D;
  if (dtype == DA_F32) return launch_decode_f32(a, B * Hq, st);
  return dtype == DA_F16 ? launch_decode<DA_F16, false>(a, B * Hq, st) : launch_decode<DA_BF16, false>(a, B * Hq, st);
}

// Argument checks common to both decode attention entry points.
static int decode_attention_check(const void* q, int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                  const void* k_packed, const void* v_packed, int64_t sp_b, int64_t sp_h,
                                  int64_t sp_s, const int32_t* counts, const int32_t* lengths,
                                  int64_t capacity, const void* k_exact, const void* v_exact, int64_t sx_b,
                                  int64_t sx_h, int64_t sx_s, int64_t window, int64_t exact_len, void* out,
                                  const char* who) {
  DA_REQUIRE(q && k_packed && v_packed && counts && lengths && k_exact && v_exact && out,
             "%s: null pointer", who);
  if (dtype != DA_BF16 && dtype != DA_F16 && dtype != DA_F32)
    return set_error(DA_ERR_UNSUPPORTED, "%s: the cache must be bf16, fp16 or fp32", who);
  if (D <= 0 || D > kDecD || (D & 7))
    return set_error(DA_ERR_UNSUPPORTED, "%s: head_dim must be a multiple of 8 in [8, %d]", who, kDecD);
  DA_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0, "%s: bad head counts", who);
  if (Hq / Hkv > kDecMaxGroup) return set_error(DA_ERR_UNSUPPORTED, "%s: GQA group above %d", who, kDecMaxGroup);
  DA_REQUIRE(window > 0 && exact_len >= 0 && exact_len <= window && capacity > 0, "%s: bad cache lengths", who);
  // key rows are read 16 bytes at a time, value rows 4 bytes per lane
  DA_REQUIRE(((sp_b | sp_h | sp_s | sx_b | sx_h | sx_s) & 7) == 0 && (((uintptr_t)k_packed | (uintptr_t)k_exact) & 15) == 0,
             "%s: key rows must be 16-byte aligned", who);
  DA_REQUIRE((((uintptr_t)v_packed | (uintptr_t)v_exact) & (dtype == DA_F32 ? 7 : 3)) == 0,
             "%s: value rows must be %d-byte aligned", who, dtype == DA_F32 ? 8 : 4);
  if (decode_slices(capacity, window) > kDecMaxSlices)
    return set_error(DA_ERR_UNSUPPORTED, "%s: cache longer than %d keys", who, kDecMaxSlices * kDecSlice - 1);
  return DA_OK;
}

extern "C" int da_decode_attention(const void* q, int dtype, int64_t B, int64_t Hq, int64_t Hkv,
                                   int64_t D, int64_t sq_b, int64_t sq_h, const void* k_packed,
                                   const void* v_packed, int64_t sp_b, int64_t sp_h, int64_t sp_s,
                                   const int32_t* counts, int64_t sc_b, int64_t sc_h,
                                   const int32_t* lengths, int64_t capacity, const void* k_exact,
                                   const void* v_exact, int64_t sx_b, int64_t sx_h, int64_t sx_s,
                                   int64_t window, int64_t exact_len, float scale, void* out,
                                   int64_t so_b, int64_t so_h, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
  const char* who = "da_decode_attention";
  if (int rc = decode_attention_check(q, dtype, B, Hq, Hkv, D, k_packed, v_packed, sp_b, sp_h, sp_s, counts,
                                      lengths, capacity, k_exact, v_exact, sx_b, sx_h, sx_s, window, exact_len,
                                      out, who))
    return rc;
  const int64_t need = da_decode_workspace_size(B, Hq, capacity, window);
  if (!workspace || workspace_bytes < need)
    return set_error(DA_ERR_WORKSPACE, "%s: workspace of %lld bytes required", who, (long long)need);
  return decode_attention_impl(q, dtype, B, Hq, Hkv, D, sq_b, sq_h, k_packed, v_packed, sp_b, sp_h, sp_s, counts,
                               sc_b, sc_h, lengths, capacity, k_exact, v_exact, sx_b, sx_h, sx_s, window,
                               exact_len, scale, out, so_b, so_h, (float*)workspace, (hipStream_t)stream);
}

// One token of da_decode_step as two launches: the attention with the update folded into
// its key list, and the combine that then writes the cache (decode_attn_kernel and
// decode_combine_kernel, FUSED).  Needs the new token's rows 16-byte aligned, as the
// attention reads key rows; the caller falls back to update + attention otherwise.
static int decode_step_fused(const DaDecodeStep* s, int64_t exact_len, hipStream_t st) {
  DecodeAttnArgs a = {};
  a.q = (const uint16_t*)s->q; a.sq_b = s->sq_b; a.sq_h = s->sq_h;
  a.kp = (const uint16_t*)s->k_packed; a.vp = (const uint16_t*)s->v_packed;
  a.sp_b = s->sp_b; a.sp_h = s->sp_h; a.sp_s = s->sp_s;
  a.counts = s->counts; a.sc_b = s->sc_b; a.sc_h = s->sc_h; a.lengths = s->lengths; a.capacity = s->capacity;
  a.kx = (const uint16_t*)s->k_exact; a.vx = (const uint16_t*)s->v_exact;
  a.sx_b = s->sx_b; a.sx_h = s->sx_h; a.sx_s = s->sx_s;
  a.exact_len = (int)exact_len; a.scale = s->scale; a.out = (uint16_t*)s->out; a.so_b = s->so_b; a.so_h = s->so_h;
  a.part = (float*)s->workspace;
  a.nslice = (int)decode_slices(s->capacity, s->window);
  a.B = (int)s->B; a.Hq = (int)s->Hq; a.Hkv = (int)s->Hkv; a.G = (int)(s->Hq / s->Hkv); a.D = (int)s->D;
  a.new_k = (const uint16_t*)s->new_k; a.new_v = (const uint16_t*)s->new_v; a.sn_b = s->sn_b; a.sn_h = s->sn_h;
  a.widx = (int)(s->exact_seq_len % s->window);
  a.evict = s->exact_seq_len >= s->window ? 1 : 0;
  a.cosine = s->use_cosine ? 1 : 0;
  a.thr = s->threshold;
  a.total_len = s->total_seq_len; a.window = s->window;
  a.ts = s->timestamps;
  a.fused = (int32_t*)((float*)s->workspace + s->B * s->Hq * a.nslice * (int64_t)(kDecD + 2));
  return s->dtype == DA_F16 ? launch_decode<DA_F16, true>(a, s->B * s->Hq, st)
                            : launch_decode<DA_BF16, true>(a, s->B * s->Hq, st);
}

// One decode token in one call: the cache update, then the attention over the updated
// cache (its ring holds min(exact_seq_len + 1, window) tokens).
extern "C" int da_decode_step(const DaDecodeStep* s, void* stream) {
  const char* who = "da_decode_step";
  DA_REQUIRE(s, "%s: null argument block", who);
  const int64_t exact_len = s->exact_seq_len + 1 < s->window ? s->exact_seq_len + 1 : s->window;
  if (int rc = decode_attention_check(s->q, s->dtype, s->B, s->Hq, s->Hkv, s->D, s->k_packed, s->v_packed, s->sp_b,
                                      s->sp_h, s->sp_s, s->counts, s->lengths, s->capacity, s->k_exact,
                                      s->v_exact, s->sx_b, s->sx_h, s->sx_s, s->window, exact_len, s->out, who))
    return rc;
  const int64_t need = da_decode_workspace_size(s->B, s->Hq, s->capacity, s->window);
  if (!s->workspace || s->workspace_bytes < need)
    return set_error(DA_ERR_WORKSPACE, "%s: workspace of %lld bytes required", who, (long long)need);
  DA_REQUIRE(s->new_k && s->new_v && s->timestamps, "%s: null pointer", who);
  DA_REQUIRE(s->exact_seq_len >= 0 && s->total_seq_len >= 0, "%s: negative lengths", who);
  // the fused path reads the new token's key row like the cache's: 16-byte aligned rows
  if (s->dtype != DA_F32 && ((s->sn_b | s->sn_h) & 7) == 0 &&
      (((uintptr_t)s->new_k | (uintptr_t)s->new_v) & 15) == 0)
    return decode_step_fused(s, exact_len, (hipStream_t)stream);
  if (int rc = decode_update_impl(s->new_k, s->new_v, s->dtype, s->B, s->Hkv, s->D, s->sn_b, s->sn_h, s->k_exact,
                                  s->v_exact, s->sx_b, s->sx_h, s->sx_s, s->k_packed, s->v_packed, s->sp_b,
                                  s->sp_h, s->sp_s, s->counts, s->timestamps, s->sc_b, s->sc_h, s->lengths,
                                  s->capacity, s->exact_seq_len, s->total_seq_len, s->window, s->threshold,
                                  s->use_cosine, stream, who))
    return rc;
  return decode_attention_impl(s->q, s->dtype, s->B, s->Hq, s->Hkv, s->D, s->sq_b, s->sq_h, s->k_packed, s->v_packed,
                               s->sp_b, s->sp_h, s->sp_s, s->counts, s->sc_b, s->sc_h, s->lengths, s->capacity,
                               s->k_exact, s->v_exact, s->sx_b, s->sx_h, s->sx_s, s->window, exact_len, s->scale,
                               s->out, s->so_b, s->so_h, (float*)s->workspace, (hipStream_t)stream);
}

// ------------------------------------------------------------------------------------
// Decode attention without any allocation: the slice partials live in `scratch`, a
// file-scope device array (one copy per GPU, held until the process ends).  Host code
// never passes the array's name to a kernel: on each device the first call looks up
// the array's device address with hipGetSymbolAddress (with that device current) and
// keeps it per device; kernels receive that address.  Every call on one GPU shares its
// copy, so calls that overlap on one GPU (different streams, no ordering) race.
// ------------------------------------------------------------------------------------
static __device__ __align__(256) float scratch[DA_DECODE_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device (looked up once per device).
static int scratch_for_current_device(void** ptr, hipStream_t stream, const char* who) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(DA_ERR_HIP, "%s: hipGetDevice: %s", who, hipGetErrorString(e));
  if (stream) {
    // the scratch array is per device: a stream of another device would get this
    // device's copy, so the stream's device must be the current one
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return set_error(DA_ERR_HIP, "%s: hipStreamGetDevice: %s", who, hipGetErrorString(e));
    if ((int)sdev != dev)
      return set_error(DA_ERR_INVALID, "%s: the stream belongs to device %d but device %d is current", who,
                       (int)sdev, dev);
  }
  if (dev < 0 || dev >= kMaxScratchDevices)
    return set_error(DA_ERR_UNSUPPORTED, "%s: device index %d above %d", who, dev, kMaxScratchDevices - 1);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(DA_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev,
                       hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return DA_OK;
}

extern "C" int da_decode_attention_noalloc(const void* q, int dtype, int64_t B, int64_t Hq, int64_t Hkv,
                                           int64_t D, int64_t sq_b, int64_t sq_h, const void* k_packed,
                                           const void* v_packed, int64_t sp_b, int64_t sp_h, int64_t sp_s,
                                           const int32_t* counts, int64_t sc_b, int64_t sc_h,
                                           const int32_t* lengths, int64_t capacity, const void* k_exact,
                                           const void* v_exact, int64_t sx_b, int64_t sx_h, int64_t sx_s,
                                           int64_t window, int64_t exact_len, float scale, void* out,
                                           int64_t so_b, int64_t so_h, void* stream) {
  const char* who = "da_decode_attention_noalloc";
  if (int rc = decode_attention_check(q, dtype, B, Hq, Hkv, D, k_packed, v_packed, sp_b, sp_h, sp_s, counts,
                                      lengths, capacity, k_exact, v_exact, sx_b, sx_h, sx_s, window, exact_len,
                                      out, who))
    return rc;
  const int64_t need = da_decode_workspace_size(B, Hq, capacity, window);
  if (need > (int64_t)DA_DECODE_SCRATCH_BYTES)
    return set_error(DA_ERR_UNSUPPORTED,
                     "%s: needs %lld bytes of scratch, above the static maximum of %lld "
                     "(B * Hq * (ceil((capacity + window + 1) / 64) * 520 + 8) bytes); use da_decode_attention",
                     who, (long long)need, (long long)DA_DECODE_SCRATCH_BYTES);
  void* part = nullptr;
  if (int rc = scratch_for_current_device(&part, (hipStream_t)stream, who)) return rc;
  return decode_attention_impl(q, dtype, B, Hq, Hkv, D, sq_b, sq_h, k_packed, v_packed, sp_b, sp_h, sp_s, counts,
                               sc_b, sc_h, lengths, capacity, k_exact, v_exact, sx_b, sx_h, sx_s, window,
                               exact_len, scale, out, so_b, so_h, (float*)part, (hipStream_t)stream);
}
