// Causal GQA flash prefill on gfx950: the dense control and the two-phase
// compressed (delta) prefill share one kernel.
//
// Replaces _attn_fwd_flat (flashAttention.py:5-91) and
// hybrid_compressed_flash_kernel / _sanity / pure_phase1_flash_kernel
// (deltaFlashAttention.py:9-357) with their wrappers (modeling_llama.py:306-451).
//
// Work decomposition.  A workgroup is 4 waves; each wave owns 32 query rows of one
// query head.  The 4 waves always read the same KV head: with a GQA group of 4 they
// are the 4 query heads of the group on the same 32 rows, so every K/V tile staged
// in LDS serves 4 heads (repeat_kv is never materialised).  With smaller groups the
// waves split 64 or 128 rows instead.  The rows of a workgroup lie inside one
// logical 128-row query block of the reference, so the whole workgroup follows the
// reference's schedule for that block.
//
// Logical schedule (deltaFlashAttention.py:58-113).  Phase 1 takes packed blocks of
// 128 anchors while their maximum timestamp is < start_m - W; Phase 2 covers dense
// keys from ((last + 1) / 128) * 128 to the diagonal.  The prefix of safe packed
// blocks is counted over the per-head prefix maxima of the block maxima
// (hybrid_schedule_kernel), which reproduces the reference's stop-at-first-unsafe-block
// loop for any timestamps, including its zero-padding behaviour (fully padded blocks
// have maximum 0).
//
// MFMA formulation.  Scores are computed transposed, S^T = K Q^T, with
// v_mfma_f32_32x32x16_bf16 (the _f16 form for fp16 tensors; the kernels are templated on
// the 16-bit type, and P is rounded to it as the reference rounds p to V's type): K
// (32 keys x 16 dims) comes from LDS as the A operand,
// Q^T stays in registers as the B operand for the whole key loop.  In the S^T
// accumulator a lane holds one query and 16 keys, so the row max and row sum of the
// online softmax are mostly in-lane (one exchange with lane ^ 32 per tile).  The
// output is accumulated transposed too, O^T += V^T P^T: the 16-bit probabilities are
// already in the B-operand layout, and V^T comes from an LDS tile that the loader
// transposes while staging it.
//
// Pipeline.  Tiles of 64 keys (K: 16 KiB, V^T: 16 KiB, counts and timestamps:
// 512 B) are double-buffered in LDS; the global loads of tile t+1 are issued before
// tile t is computed and written to the other buffer afterwards, with one barrier
// per tile.  Two workgroups fit per CU (66.5 KiB LDS each).
//
// Softmax numerics.  exp2 with the softmax scale folded in: p = 2^(s*c - m*c) with
// c = scale * log2(e) -- the same values as exp(s*scale - m*scale).  In Phase 1
// p is multiplied by the anchor count in fp32 and then rounded to bf16 for the
// P.V product while l accumulates the fp32 weights (deltaFlashAttention.py:86-98).
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <utility>

#include "da_common.hpp"

namespace da {

constexpr int kD = 128;
constexpr int kTileN = 64;
constexpr int kKBytes = kTileN * kD * 2;
constexpr int kVBytes = kD * kTileN * 2;
constexpr int kStageBytes = kKBytes + kVBytes + kTileN * 4 + kTileN * 4;
constexpr int kBlock = 128;  // logical block of the reference schedule

enum Variant : int { kHybrid = 0, kSanity = 1, kPure = 2, kDense = 3 };

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* kp;
  const uint16_t* vp;
  const int32_t* ts;
  const void* cnt;
  uint16_t* out;
  int64_t sq_b, sq_h, sq_n;
  int64_t sk_b, sk_h, sk_n;
  int64_t sv_b, sv_h, sv_n;
  int64_t skp_b, skp_h, skp_n;
  int64_t svp_b, svp_h, svp_n;
  int64_t so_b, so_h, so_n;
  int64_t sts_b, sts_h;
  int64_t scnt_b, scnt_h;
  int B, Hq, Hkv, G, Nq, Nk;
  SeqMap seq;  // ragged batch (varlen): every sequence has Nq = Nk = seq.len(b)
  int D;  // head dimension: a multiple of 8, at most 128 (dims D..127 are zero-filled)
  int P_host;
  const int32_t* P_dev;  // P on the device ([B], one per sequence, for a ragged batch)
  int window;
  float scale_log2;  // softmax scale * log2(e)
  int no_count;
  int cnt_is_float;
  int causal;
  const int32_t* sched;  // [B*Hkv][2][nblk_cap]: block maxima, prefix maxima
  int nblk_cap;
  // prepared by the schedule kernel for the ping-pong kernel, [B*Hkv][wcap] each:
  const float* wts;    // key bias log2(w_i) / scale_log2 of packed row i (-inf where w_i = 0)
  const int32_t* tsw;  // timestamp of packed row i, INT_MAX where the weight is 0
  const float* zeros;  // 64 zero biases (the exact tiles)
  int wcap;            // nblk_cap * 128
  int hpw;          // query heads per workgroup (4, 2 or 1)
  int rows_per_wg;  // 32 * (4 / hpw)
  int n_row_groups;
  int units;        // B * Hkv * (G / hpw)
  int* queue;       // 8 work-queue counters (persistent attn_w64_kernel grid) or null
};

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// LDS byte offsets inside a stage.
__device__ __forceinline__ int k_lds_off(int row, int chunk) {
  return row * (kD * 2) + ((chunk ^ (row & 15)) << 4);
}
// V^T rows (one per head dimension) hold the 64 keys of the tile permuted so that
// the 8 keys one lane feeds to a P.V MFMA -- keys 16u + 4h + {0..3} and
// 16u + 8 + 4h + {0..3} -- form 16-byte chunk 2u + h.  A group of 4 consecutive keys
// 4kg..4kg+3 is the 8-byte half (kg >> 1) & 1 of chunk 2 (kg >> 2) + (kg & 1).
// Chunks are XOR-swizzled with (d & 7) ^ ((d >> 3) & 1) so that 8 (or 16) consecutive
// rows read at one chunk index hit distinct banks.
__device__ __forceinline__ int vt_swz(int d) { return (d & 7) ^ ((d >> 3) & 1); }
__device__ __forceinline__ int vt_lds_chunk(int d, int chunk) {
  return kKBytes + d * (kTileN * 2) + ((chunk ^ vt_swz(d)) << 4);
}
__device__ __forceinline__ int vt_lds_group(int d, int kg) {
  return vt_lds_chunk(d, 2 * (kg >> 2) + (kg & 1)) + (((kg >> 1) & 1) << 3);
}
constexpr int kCntOff = kKBytes + kVBytes;
constexpr int kTsOff = kCntOff + kTileN * 4;

struct TileRegs {
  u32x4 k[4];
  u32x4 v[4];
  float cnt;
  int ts;
};

// Global -> registers for one 64-key tile.  For K, thread tid loads 16-byte chunk
// (tid % 16) of keys 4 * (tid / 16) + j, j = 0..3 (a wave writes whole 256-byte K
// rows).  For V the roles swap -- chunk tid / 16 of keys 4 * (tid % 16) + j -- so that
// after the in-register transpose the 16 lanes of one chunk write one complete
// 128-byte V^T row, which keeps the LDS stores free of bank conflicts.
__device__ __forceinline__ void load_tile(TileRegs& r, const uint16_t* kbase, const uint16_t* vbase,
                                          int64_t sk_n, int64_t sv_n, int key0, int limit, int D,
                                          int tid, bool with_meta, const int32_t* tsrow,
                                          const void* cntrow, int cnt_is_float, int no_count,
                                          int meta_limit, int ts_oob) {
  const int chunk = tid & 15, kg = tid >> 4;    // K mapping
  const int vchunk = tid >> 4, vkg = tid & 15;  // V mapping
  // 8-dim chunks at or beyond the head dimension are zero (BLOCK_D padding of the reference)
  const bool kin = chunk * 8 < D, vin = vchunk * 8 < D;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int key = key0 + kg * 4 + j;
    r.k[j] = (kin && key < limit) ? *(const u32x4*)(kbase + (int64_t)key * sk_n + chunk * 8)
                                  : u32x4{0, 0, 0, 0};
    const int vkey = key0 + vkg * 4 + j;
    r.v[j] = (vin && vkey < limit) ? *(const u32x4*)(vbase + (int64_t)vkey * sv_n + vchunk * 8)
                                   : u32x4{0, 0, 0, 0};
  }
  if (with_meta && tid < kTileN) {
    const int key = key0 + tid;
    if (key < meta_limit) {
      if (no_count)
        r.cnt = 1.0f;
      else if (cnt_is_float)
        r.cnt = ((const float*)cntrow)[key];
      else
        r.cnt = (float)((const int32_t*)cntrow)[key];
      r.ts = tsrow ? tsrow[key] : 0;
    } else {
      r.cnt = 0.0f;
      r.ts = ts_oob;
    }
  }
}

__device__ __forceinline__ void store_tile(const TileRegs& r, char* stage, int tid, bool with_meta) {
  const int chunk = tid & 15, kg = tid >> 4;
  const int vchunk = tid >> 4, vkg = tid & 15;
#pragma unroll
  for (int j = 0; j < 4; ++j) *(u32x4*)(stage + k_lds_off(kg * 4 + j, chunk)) = r.k[j];
  // transpose 4 keys x 8 dims into 8 rows (dims) of 4 keys
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t a = r.v[0][w], b = r.v[1][w], c = r.v[2][w], d = r.v[3][w];
    const int d0 = vchunk * 8 + 2 * w;
    // v_perm_b32 picks bytes of {S0 = high word, S1 = low word}: 0x05040100 gives
    // (lo16(a), lo16(b)), 0x07060302 gives (hi16(a), hi16(b)).
    u32x2 lo, hi;
    lo[0] = __builtin_amdgcn_perm(b, a, 0x05040100u);
    lo[1] = __builtin_amdgcn_perm(d, c, 0x05040100u);
    hi[0] = __builtin_amdgcn_perm(b, a, 0x07060302u);
    hi[1] = __builtin_amdgcn_perm(d, c, 0x07060302u);
    *(u32x2*)(stage + vt_lds_group(d0, vkg)) = lo;
    *(u32x2*)(stage + vt_lds_group(d0 + 1, vkg)) = hi;
  }
  if (with_meta && tid < kTileN) {
    ((float*)(stage + kCntOff))[tid] = r.cnt;
    ((int*)(stage + kTsOff))[tid] = r.ts;
  }
}

// Phase-1 extent of a query block (deltaFlashAttention.py:58-80): n_safe = the number of
// packed blocks whose prefix maximum timestamp is below thr -- the prefix maxima do not
// decrease, so these are exactly the blocks before the first unsafe one -- and last = the
// maximum timestamp of the last of them (-1 if none).  A ballot per 64 blocks counts
// them; the entries of 256 blocks are loaded together, so the usual case is one round
// trip to memory.  Needs all 64 lanes of the wave.
__device__ __forceinline__ void safe_prefix(const int32_t* __restrict__ bmax, const int32_t* __restrict__ pmax,
                                            int nblk, int thr, int& n_safe, int& last, int lane) {
  int n = 0, prev_last = -1;
  last = -1;
  for (int base = 0; base < nblk; base += 256) {
    int pv[4], bv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = base + 64 * j + lane;
      pv[j] = i < nblk ? pmax[i] : INT_MAX;
      bv[j] = i < nblk ? bmax[i] : -1;
    }
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) cnt += __popcll(__ballot(pv[j] < thr));
    n += cnt;
    if (cnt > 0) {
      const int k = cnt - 1;  // the last safe block is entry k of this chunk
      const int j = k >> 6;
      const int v = j == 0 ? bv[0] : j == 1 ? bv[1] : j == 2 ? bv[2] : bv[3];
      last = __builtin_amdgcn_readlane(v, k & 63);
    } else {
      last = prev_last;
    }
    if (cnt < 256) break;
    prev_last = last;
  }
  n_safe = n;
}

template <int VARIANT, int DT>
__device__ __forceinline__ void attn_body(const AttnArgs& a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  const int hl = lane >> 5;   // which half of the wave
  const int ql = lane & 31;   // query column of this lane

  // ---- workgroup -> (unit, row group): XCD-aware, longest rows first ----
  const int wg = blockIdx.x;
  int unit, rg;
  if ((a.units & 7) == 0) {
    // workgroup i runs on XCD i mod 8; each XCD takes whole units (a KV head of one
    // sequence) and runs them one after another, every unit's row groups longest first,
    // so the 32 CUs of an XCD share one unit's K/V in their L2
    const int xcd = wg & 7, idx = wg >> 3, upx = a.units >> 3;
    unit = xcd * upx + idx / a.n_row_groups;
    rg = a.n_row_groups - 1 - idx % a.n_row_groups;
  } else {
    unit = wg % a.units;
    rg = a.n_row_groups - 1 - wg / a.units;
  }
  // units are KV-head major, so that the XCD mapping above gives each XCD whole KV
  // heads of every sequence (balanced when the sequences of a batch differ in length)
  const int hunits = a.G / a.hpw;
  const int gb = unit / hunits;  // g * B + b
  const int hu = unit - gb * hunits;
  const int g = gb / a.B, b = gb - (gb / a.B) * a.B;
  const int bg = b * a.Hkv + g;
  const int h = g * a.G + hu * a.hpw + (wid % a.hpw);
  const int R0 = rg * a.rows_per_wg;
  const int Nq = a.seq.cu ? a.seq.len(b) : a.Nq;
  const int Nk = a.seq.cu ? a.seq.len(b) : a.Nk;
  if (R0 >= Nq) return;  // a row group past the end of a shorter sequence (whole workgroup)
  const int r0w = R0 + (wid / a.hpw) * 32;  // first row of this wave
  const int wg_end = R0 + a.rows_per_wg;    // one past the last row of the workgroup
  const int start_m = (R0 / kBlock) * kBlock;

  // ---- schedule ----
  int P = a.P_host;
  if (a.P_dev) P = min(a.seq.cu ? a.P_dev[b] : *a.P_dev, a.P_host);
  if (a.seq.cu) P = min(P, Nk);  // a sequence's packed rows lie inside its own tokens
  int n1 = 0, ds = 0;
  int kend = a.causal ? min(Nk, wg_end) : Nk;
  if (VARIANT == kHybrid || VARIANT == kSanity) {
    const int nblk = (P + kBlock - 1) / kBlock;
    const int32_t* bmax = a.sched + (int64_t)bg * 2 * a.nblk_cap;
    const int32_t* pmax = bmax + a.nblk_cap;
    int n_safe, last;
    safe_prefix(bmax, pmax, nblk, start_m - a.window, n_safe, last, lane);
    ds = max(0, ((last + 1) / kBlock) * kBlock);
    if (VARIANT == kHybrid) n1 = n_safe * (kBlock / kTileN);
    kend = min(Nk, wg_end);
  } else if (VARIANT == kPure) {
    n1 = (P + kTileN - 1) / kTileN;
    kend = 0;
  }
  const int n2 = kend > ds ? (kend - ds + kTileN - 1) / kTileN : 0;
  const int ntiles = n1 + n2;

  const uint16_t* kp_base = a.kp + a.seq.base(b, a.skp_b, a.skp_n) + (int64_t)g * a.skp_h;
  const uint16_t* vp_base = a.vp + a.seq.base(b, a.svp_b, a.svp_n) + (int64_t)g * a.svp_h;
  const uint16_t* k_base = a.k + a.seq.base(b, a.sk_b, a.sk_n) + (int64_t)g * a.sk_h;
  const uint16_t* v_base = a.v + a.seq.base(b, a.sv_b, a.sv_n) + (int64_t)g * a.sv_h;
  const int32_t* ts_row = a.ts ? a.ts + a.seq.base(b, a.sts_b, 1) + (int64_t)g * a.sts_h : nullptr;
  const char* cnt_row = a.cnt ? (const char*)a.cnt + (a.seq.base(b, a.scnt_b, 1) + (int64_t)g * a.scnt_h) * 4 : nullptr;
  const bool meta = (VARIANT == kHybrid || VARIANT == kPure);

  // ---- Q^T in registers (B operand): lane (ql, hl) holds dims 16t + 8hl .. +7 ----
  u32x4 qreg[kD / 16];
  {
    const int row = r0w + ql;
    const uint16_t* qrow = a.q + a.seq.base(b, a.sq_b, a.sq_n) + (int64_t)h * a.sq_h + (int64_t)row * a.sq_n;
#pragma unroll
    for (int t = 0; t < kD / 16; ++t)
      qreg[t] = (row < Nq && 16 * t + 8 * hl < a.D) ? *(const u32x4*)(qrow + 16 * t + 8 * hl)
                                                       : u32x4{0, 0, 0, 0};
  }

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f32x16{};
  float m_i = -INFINITY, l_i = 0.0f;
  const float c = a.scale_log2;

  TileRegs regs;
  auto tile_src = [&](int t, const uint16_t*& kb, const uint16_t*& vb, int64_t& skn, int64_t& svn,
                      int& key0, int& limit, bool& ph1) {
    ph1 = t < n1;
    if (ph1) {
      kb = kp_base; vb = vp_base; skn = a.skp_n; svn = a.svp_n; key0 = t * kTileN; limit = P;
    } else {
      kb = k_base; vb = v_base; skn = a.sk_n; svn = a.sv_n; key0 = ds + (t - n1) * kTileN; limit = Nk;
    }
  };

  if (ntiles > 0) {
    const uint16_t *kb, *vb; int64_t skn, svn; int key0, limit; bool ph1;
    tile_src(0, kb, vb, skn, svn, key0, limit, ph1);
    load_tile(regs, kb, vb, skn, svn, key0, limit, a.D, tid, meta && ph1, ts_row, cnt_row,
              a.cnt_is_float, a.no_count, P, Nk + 1);
    store_tile(regs, smem, tid, meta && ph1);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    char* stage = smem + (t & 1) * kStageBytes;
    const bool has_next = t + 1 < ntiles;
    bool next_ph1 = false;
    if (has_next) {
      const uint16_t *kb, *vb; int64_t skn, svn; int key0, limit;
      tile_src(t + 1, kb, vb, skn, svn, key0, limit, next_ph1);
      load_tile(regs, kb, vb, skn, svn, key0, limit, a.D, tid, meta && next_ph1, ts_row, cnt_row,
                a.cnt_is_float, a.no_count, P, Nk + 1);
    }

    const bool ph1 = t < n1;
    const int key0 = ph1 ? t * kTileN : ds + (t - n1) * kTileN;
    // wave-uniform skip of tiles entirely above this wave's rows (causal)
    const bool skip = !ph1 && a.causal && key0 > r0w + 31;
    if (!skip) {
      // ---- S^T = K Q^T for two 32-key blocks ----
      // the two key blocks alternate so that consecutive MFMAs do not depend on each other
      f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
      for (int tt = 0; tt < kD / 16; ++tt) {
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2) {
          const u32x4 w = *(const u32x4*)(stage + k_lds_off(kb2 * 32 + ql, 2 * tt + hl));
          s[kb2] = E16<DT>::mfma(w, qreg[tt], s[kb2]);
        }
      }
      // ---- masks ----
      const int row = r0w + ql;
      if (VARIANT == kPure) {
        const float* cl = (const float*)(stage + kCntOff);
        const int* tl = (const int*)(stage + kTsOff);
#pragma unroll
        for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kl = kb2 * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
            const bool ok = cl[kl] > 0.0f && tl[kl] <= row;  // deltaFlashAttention.py:321-330
            if (!ok) s[kb2][r] = -INFINITY;
          }
      } else if (!ph1) {
        const bool need = (a.causal && key0 + kTileN - 1 > r0w) || key0 + kTileN > Nk;
        if (need) {
#pragma unroll
          for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = key0 + kb2 * 32 + 8 * (r >> 2) + 4 * hl + (r & 3);
              const bool ok = key < Nk && (!a.causal || key <= row);
              if (!ok) s[kb2][r] = -INFINITY;
            }
        }
      }
      // ---- online softmax ----
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = __builtin_fmaxf(mx, __builtin_fmaxf(s[0][r], s[1][r]));
      mx = fmaxf(mx, swap_halves(mx));
      const float m_new = fmaxf(m_i, mx);
      const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
      const float alpha = exp2_fast((m_i - m_use) * c);
      const float neg = -m_use * c;
      // P^T as four B operands (16 keys each): operand u = 2 * kb2 + (r4 >> 1) holds
      // S^T registers 8 * (r4 >> 1) .. +7 of block kb2.
      u32x4 pw[4];
      float psum = 0.0f;
      const bool weighted = (VARIANT == kPure) || (VARIANT == kHybrid && ph1);
      const float* cl = (const float*)(stage + kCntOff);
#pragma unroll
      for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          f32x4 w4 = f32x4{1.0f, 1.0f, 1.0f, 1.0f};
          if (weighted) w4 = *(const f32x4*)(cl + kb2 * 32 + 8 * r4 + 4 * hl);
          float p[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            p[e] = exp2_fast(__builtin_fmaf(s[kb2][4 * r4 + e], c, neg));
            if (weighted) p[e] *= w4[e];
          }
          psum += (p[0] + p[1]) + (p[2] + p[3]);
          pw[2 * kb2 + (r4 >> 1)][(r4 & 1) * 2 + 0] = E16<DT>::pack(p[0], p[1]);
          pw[2 * kb2 + (r4 >> 1)][(r4 & 1) * 2 + 1] = E16<DT>::pack(p[2], p[3]);
        }
      }
      l_i = l_i * alpha + psum;
      m_i = m_new;
      if (__ballot(alpha != 1.0f)) {
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[db][r] *= alpha;
      }
      // ---- O^T += V^T P^T ----
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const int d = db * 32 + ql;
          const u32x4 vw = *(const u32x4*)(stage + vt_lds_chunk(d, 2 * u + hl));
          o[db] = E16<DT>::mfma(vw, pw[u], o[db]);
        }
      }
    }
    if (has_next) store_tile(regs, smem + ((t + 1) & 1) * kStageBytes, tid, meta && next_ph1);
    __syncthreads();
  }

  // ---- finalize: out = acc / l ----
  const float l_tot = l_i + swap_halves(l_i);
  float inv;
  if (VARIANT == kPure)
    inv = l_tot > 0.0f ? 1.0f / l_tot : 1.0f;  // deltaFlashAttention.py:353-354
  else
    inv = 1.0f / l_tot;
  const int row = r0w + ql;
  if (row < Nq) {
    uint16_t* orow = a.out + a.seq.base(b, a.so_b, a.so_n) + (int64_t)h * a.so_h + (int64_t)row * a.so_n;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x2 w;
        w[0] = E16<DT>::pack(o[db][4 * j + 0] * inv, o[db][4 * j + 1] * inv);
        w[1] = E16<DT>::pack(o[db][4 * j + 2] * inv, o[db][4 * j + 3] * inv);
        if (db * 32 + 8 * j + 4 * hl < a.D) *(u32x2*)(orow + db * 32 + 8 * j + 4 * hl) = w;
      }
  }
}

// Per-head kernel entry points.  Dense, hybrid and sanity fit two waves per SIMD
// (<= 256 registers).  The pure-Phase-1 body needs more: capped at 256 it spills, and that
// build gave wrong pure-Phase-1 outputs on every row while the same source without the
// cap (no spills) matches the oracle, so it runs at one wave per SIMD.
template <int VARIANT, int DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_kernel(AttnArgs a) {
  attn_body<VARIANT, DT>(a);
}
template <int DT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2)))
void attn_kernel_pure(AttnArgs a) {
  attn_body<kPure, DT>(a);
}

// min(max(x, 0), hi) for a wave-uniform x, kept in scalar registers (the compiler would
// otherwise form a clamp that only exists as a vector instruction, v_med3).
__device__ __forceinline__ int clamp0_uniform(int x, int hi) {
  x = __builtin_amdgcn_readfirstlane(x < hi ? x : hi);
  asm volatile("" : "+s"(x));
  return x > 0 ? x : 0;
}

// Third dword of a raw buffer resource on gfx9 (32-bit data format, no swizzle).
constexpr int kBufferDword3 = 0x00020000;

// A wave-uniform pointer moved into scalar registers.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const void*)(((uint64_t)hi << 32) | lo);
}

// Workgroup barrier after the wave's own LDS reads and writes are done, leaving
// loads to LDS (buffer_load ... lds) in flight.  A fence for LDS would wait for those
// too (vmcnt(0)): the loads issued in this window are only read after the next
// barrier, and their wait is explicit.  The asm is a compiler memory barrier.
__device__ __forceinline__ void barrier_keep_loads() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

// LDS byte address of a pointer into the kernel's LDS.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}
// ds_read_b64_tr_b16 at addr + OFF: in each group of 16 lanes, lane i receives element
// i % 4 of the 8 bytes read by lanes 4e + i / 4, e = 0..3 (a 4 x 4 transpose of 16-bit
// elements per group of four lanes).  Issued as asm: the caller waits with lgkm_wait.
template <int OFF>
__device__ __forceinline__ i16x4 ds_read_tr16(uint32_t addr) {
  i16x4 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}
// s_waitcnt lgkmcnt(N) that the uses of a and b cannot move above.
template <int N>
__device__ __forceinline__ void lgkm_wait(i16x4& a, i16x4& b) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}
// ds_read_b128 issued as asm (waited for with lgkm_wait), so that the reads stay ahead
// of the MFMAs that use them.
__device__ __forceinline__ u32x4 ds_read_b128_asm(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
template <int N>
__device__ __forceinline__ void lgkm_wait(u32x4& a, u32x4& b) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}
// An unspecified value that costs no instruction: for a register array on a path where
// it is dead, so that it is not live around the loop.
template <typename T>
__device__ __forceinline__ void undefined(T& x) {
  asm volatile("" : "=v"(x));
}
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
// f(integral_constant<int, i>) for i = 0 .. N-1, in order
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Max / sum of x over lanes l and l ^ 32, without LDS (v_permlane32_swap); the order
// of the returned pair does not matter for either.
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// s_waitcnt immediate (gfx9 encoding) that waits for vmcnt <= n only.
constexpr int vmcnt_only(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// The 64-row kernel updates its running maximum lazily: only when a tile's maximum
// exceeds it by more than 2^8 in probability (8 in log2 units) are O and l rescaled.
constexpr float kLazyLog2 = 8.0f;
// The 64-row kernel computes p against the current maximum before it looks at the
// tile's maximum, and needs the latter only where a lane's sum of its 16 p exceeds
// 16 * 2^8: below that bound every p is at most 2^8 * 16, and a rescale is not needed
// (p stays far from fp32's range and keeps bf16's relative precision).
constexpr float kLazySum = 16.0f * 256.0f;

// ====================================================================================
// Ping-pong kernel for GQA groups that are a multiple of 4 (the Llama-3 hot path).
//
// A workgroup is 8 waves, two per SIMD, and covers one logical 128-row query block of
// the reference's schedule for 4 query heads of one GQA group, so all 8 waves read the
// same K/V tiles.  Waves 0-3 (group A) own rows R0..R0+63 and waves 4-7 (group B) rows
// R0+64..R0+127, each wave one query head, as two 32-row column blocks.  Tiles are 32
// keys; every tile boundary falls on the reference's logical 128-key grid.
//
// In every section one group runs its matrix work (P.V of the previous tile, then Q.K
// of the current one: 32 MFMAs at raised issue priority) while the other group runs its
// softmax (VALU); group B runs one section behind group A, so the two waves sharing a
// SIMD have complementary work and the MFMA pipe and the VALU co-execute.  Two sections
// form a window; the workgroup synchronises once per window.  Every K fragment and every
// V^T fragment read from LDS feeds two MFMAs, one per column block.
//
// K and V tiles go straight from memory to LDS (buffer_load ... lds), three stages each,
// issued two windows (K) and one window (V) ahead of their use; V is kept row-major and
// read as V^T with ds_read_b64_tr_b16.  No tile passes through registers.  Q of column
// block 0 stays in registers; Q of column block 1 sits in LDS, lane-private (each lane
// reads back only what it wrote), which keeps the wave within 256 registers.
// ====================================================================================
constexpr int kWTK = 32;                         // keys per tile
constexpr int kWKBytes = kWTK * kD * 2;          // 8 KiB
constexpr int kWVBytes = kWTK * kD * 2;          // 8 KiB
constexpr int kWMetaSlot = 64 * 8;               // weights[64] fp32, timestamps[64] int32
constexpr int kWCnt = 0, kWTs = 64 * 4;          // offsets inside a meta slot
constexpr int kWQBytes = 32 * kD * 2;          // Q of one 32-row column block, per wave
// the persistent grid's item broadcast (two ints) after the Q regions
constexpr int kWItemSlot = 3 * kWKBytes + 3 * kWVBytes + 4 * kWMetaSlot + 8 * kWQBytes;
constexpr int kWLds = kWItemSlot + 16;  // item: queue, index, queues found empty
// K stages and Q blocks start at multiples of 256 bytes (the kernel has no static LDS, so
// its dynamic LDS starts at address 0): the K / Q fragment addresses are formed by XOR.
static_assert(kWKBytes % 256 == 0 && (3 * kWKBytes + 3 * kWVBytes + 4 * kWMetaSlot) % 256 == 0 &&
              kWQBytes % 256 == 0, "K stages and Q blocks must be 256-byte aligned");

// Masks of one 32-key x 32-row score block (S^T register r holds key 8 (r / 4) + 4 hl +
// r % 4 of the tile for the lane's row).
__device__ __forceinline__ void mask_dense32(f32x16& s, int key0, int row, int hl, int Nk, bool causal) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int key = key0 + 8 * (r >> 2) + 4 * hl + (r & 3);
    const bool ok = key < Nk && (!causal || key <= row);
    if (!ok) s[r] = -INFINITY;
  }
}
__device__ __forceinline__ void mask_pure32(f32x16& s, const int* tl, int row, int hl) {
#pragma unroll
  for (int r4 = 0; r4 < 4; ++r4) {
    const int4 t4 = *(const int4*)(tl + 8 * r4 + 4 * hl);
    if (!(t4.x <= row)) s[4 * r4 + 0] = -INFINITY;
    if (!(t4.y <= row)) s[4 * r4 + 1] = -INFINITY;
    if (!(t4.z <= row)) s[4 * r4 + 2] = -INFINITY;
    if (!(t4.w <= row)) s[4 * r4 + 3] = -INFINITY;
  }
}

// Units of work queue q (one queue per XCD): the contiguous range [ulo, uhi) of the
// units, in the order of the static grid below.
__device__ __forceinline__ void queue_units(int q, int units, int& ulo, int& uhi) {
  ulo = (q * units) >> 3;
  uhi = ((q + 1) * units) >> 3;
}

// One (unit, row group) of attn_w64_kernel: 4 query heads of one (batch, KV head) over
// the logical 128-row query block rg.  Ends with every LDS read of the window loop done
// (its last barrier) and every load landed; the finalize uses only the wave's own Q
// region, so the next item may start staging at once.
template <int VARIANT, int DT>
__device__ __forceinline__ void attn_w64_item(const AttnArgs& a, const int unit, const int rg) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  char* const kst0 = smem;
  char* const vst0 = smem + 3 * kWKBytes;
  char* const meta0 = smem + 3 * kWKBytes + 3 * kWVBytes;
  // opaque per item: what derives from the thread index is formed here, not hoisted out
  // of the persistent grid's item loop into registers held across items
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave
  // Q of column block 1, lane-private: each lane reads back only the 16-byte chunks it
  // wrote (the K fragment layout), so the 32 registers it would take stay free
  char* const qs = meta0 + 4 * kWMetaSlot + wid * kWQBytes;
  const int grp = wid >> 2, hw = wid & 3;
  const int hl = lane >> 5, ql = lane & 31;
  const int hunits = a.G >> 2;
  const int gb = unit / hunits;  // g * B + b
  const int hu = unit - gb * hunits;
  const int g = gb / a.B, b = gb - (gb / a.B) * a.B;
  const int bg = b * a.Hkv + g;
  const int h = g * a.G + hu * 4 + hw;
  const int R0 = rg * 128;
  const int Nq = a.seq.cu ? a.seq.len(b) : a.Nq;
  const int Nk = a.seq.cu ? a.seq.len(b) : a.Nk;
  if (R0 >= Nq) return;  // a row group past the end of a shorter sequence (whole workgroup)
  const int r0w = R0 + grp * 64;  // first row of this wave; column block cb holds r0w + 32 cb + ql
  const int wg_end = R0 + 128;
  const int start_m = R0;

  // ---- schedule of the logical 128-row block R0 ----
  int P = a.P_host;
  if (a.P_dev) P = min(a.seq.cu ? a.P_dev[b] : *a.P_dev, a.P_host);
  if (a.seq.cu) P = min(P, Nk);
  int n1 = 0, ds = 0;
  int kend = a.causal ? min(Nk, wg_end) : Nk;
  if (VARIANT == kHybrid || VARIANT == kSanity) {
    const int nblk = (P + kBlock - 1) / kBlock;
    const int32_t* bmax = a.sched + (int64_t)bg * 2 * a.nblk_cap;
    const int32_t* pmax = bmax + a.nblk_cap;
    int n_safe, last;
    safe_prefix(bmax, pmax, nblk, start_m - a.window, n_safe, last, lane);
    ds = max(0, ((last + 1) / kBlock) * kBlock);
    if (VARIANT == kHybrid) n1 = n_safe * (kBlock / kWTK);
    kend = min(Nk, wg_end);
  } else if (VARIANT == kPure) {
    n1 = (P + kWTK - 1) / kWTK;
    kend = 0;
  }
  const int n2 = kend > ds ? (kend - ds + kWTK - 1) / kWTK : 0;
  const int T = n1 + n2;

  const uint16_t* kp_base = a.kp + a.seq.base(b, a.skp_b, a.skp_n) + (int64_t)g * a.skp_h;
  const uint16_t* vp_base = a.vp + a.seq.base(b, a.svp_b, a.svp_n) + (int64_t)g * a.svp_h;
  const uint16_t* k_base = a.k + a.seq.base(b, a.sk_b, a.sk_n) + (int64_t)g * a.sk_h;
  const uint16_t* v_base = a.v + a.seq.base(b, a.sv_b, a.sv_n) + (int64_t)g * a.sv_h;
  const float* w_row = a.wts ? a.wts + (int64_t)bg * a.wcap : nullptr;
  const int32_t* tsw_row = a.tsw ? a.tsw + (int64_t)bg * a.wcap : nullptr;
  constexpr bool kPureV = VARIANT == kPure;
  constexpr bool kWeights = VARIANT == kHybrid || VARIANT == kPure;

  auto key0_of = [&](int t) { return t < n1 ? t * kWTK : ds + (t - n1) * kWTK; };
  // causal: a Phase-2 tile whose first key is past the wave's last row (r0w + 63) is
  // skipped; tiles n1 + (r0w + 63 - ds) / 32 + 1 onwards are
  int t_skip = INT_MAX;
  if (a.causal) {
    const int d = r0w + 63 - ds;
    t_skip = __builtin_amdgcn_readfirstlane(d < 0 ? n1 : n1 + d / kWTK + 1);
  }
  auto skipped = [&](int t) { return t >= t_skip; };

  // ---- staging: loads straight into LDS, three stages each for K and V and a ring of
  // four slots for the tiles' weights.  Wave w loads rows 4w .. 4w + 3 of both tiles:
  // lane l writes 16 bytes at 1 KiB w + 16 l, i.e. row 4w + l / 16 at position l % 16,
  // so it fetches the source chunk that the swizzled layout keeps there.  The buffer
  // resource covers exactly the tile's valid keys: rows past the end, and 8-dim chunks
  // at or beyond the head dimension, arrive as zeros.  Each wave issues the same loads
  // in every window, so the s_waitcnt vmcnt(n) at the end of a window, n = the loads of
  // this window, waits exactly for those of the window before. ----
  const int wid_s = __builtin_amdgcn_readfirstlane(wid);
  const char* kb1 = (const char*)uniform_ptr(kp_base);
  const char* kb2 = (const char*)uniform_ptr(k_base);
  const char* vb1 = (const char*)uniform_ptr(vp_base);
  const char* vb2 = (const char*)uniform_ptr(v_base);
  const int skpb = __builtin_amdgcn_readfirstlane((int)(2 * a.skp_n));
  const int skb = __builtin_amdgcn_readfirstlane((int)(2 * a.sk_n));
  const int svpb = __builtin_amdgcn_readfirstlane((int)(2 * a.svp_n));
  const int svb = __builtin_amdgcn_readfirstlane((int)(2 * a.sv_n));
  auto dma_rows = [&](bool isK, int t_raw, unsigned st) {
    const int t = min(t_raw, T - 1);
    const bool ph1 = t < n1;
    const int key0 = key0_of(t);
    const int limit = ph1 ? P : Nk;
    const int snb = isK ? (ph1 ? skpb : skb) : (ph1 ? svpb : svb);
    const char* src = isK ? (ph1 ? kb1 : kb2) : (ph1 ? vb1 : vb2);
    const void* base = uniform_ptr(src + (int64_t)key0 * snb);
    const int range = clamp0_uniform(limit - key0, kWTK) * snb;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(base), (short)0, range, kBufferDword3);
    char* dst = isK ? kst0 + st : vst0 + st;
    const int rowt = wid_s * 4 + (lane >> 4);
    const int pos = lane & 15;
    const int chunk = pos ^ (isK ? (rowt & 15) : 4 * (rowt & 3));
    // rowt < 32 and snb < 2^24 (the host limits sequence strides to 2^23 elements), so the
    // unsigned 24-bit multiply is exact (a signed one would read snb >= 2^23 as negative);
    // a chunk at or past the head dimension reads past the range (zeros), without a branch
    const int off = (int)__umul24((unsigned)rowt, (unsigned)snb) + chunk * 16 + (chunk * 8 < a.D ? 0 : range);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(dst + wid_s * 1024), 16,
                                             off, 0, 0, 0);
  };
  // key biases (and timestamps) of the tile's 32 keys, into slot t % 4 of their ring
  // (lanes 32-63 read past the range: zeros); a packed tile reads the prepared biases,
  // an exact tile zeros; S^T starts at them
  auto meta_of = [&](int t) { return meta0 + (t & 3) * kWMetaSlot; };
  auto dma_meta = [&](int t_raw) {
    if (!kWeights) return;
    const int t = min(t_raw, T - 1);
    const bool ph1 = t < n1;
    const int key0 = ph1 ? t * kWTK : 0;
    const int nrows = ph1 ? clamp0_uniform(a.wcap - key0, kWTK) : kWTK;
    char* dst = meta_of(t_raw);
    // the lane's offset, formed here from an opaque lane index rather than held
    int mlane = lane;
    asm volatile("" : "+v"(mlane));
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(uniform_ptr(ph1 ? w_row + key0 : a.zeros)), (short)0,
        nrows * 4, kBufferDword3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, (__attribute__((address_space(3))) void*)(dst + kWCnt), 4,
                                             mlane * 4, 0, 0, 0);
    if (kPureV) {
      const __amdgpu_buffer_rsrc_t rt = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<void*>(uniform_ptr(tsw_row + key0)), (short)0, nrows * 4, kBufferDword3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, (__attribute__((address_space(3))) void*)(dst + kWTs), 4,
                                               mlane * 4, 0, 0, 0);
    }
  };
  auto dma_issue = [&](int tk, int tv, unsigned kst, unsigned vst) {
    dma_rows(true, tk, kst);
    dma_rows(false, tv, vst);
    if (wid_s == 0) dma_meta(tk);
  };

  // ---- per-lane LDS offsets (stage-relative).  K: rows of 256 bytes, 16-byte chunk c
  // of row r at position c ^ (r & 15); the lane reads chunk 2 j + hl of row ql.  V^T:
  // fragments of 16 keys x 32 head dims (db) read with ds_read_b64_tr_b16 from rows
  // whose chunks sit at c ^ 4 (r & 3).  Both are recomputed in each matrix section
  // (made opaque there) rather than held in registers ----
  int k_lane = ql * 256 + (((hl ^ ql) & 1) << 4) + ((ql & 14) << 4);
  int v_lane = (4 * ((lane >> 4) >> 1) + ((lane & 15) >> 2)) * 256 +
               ((2 * ((lane >> 4) & 1) + ((lane & 3) >> 1)) << 4) + 8 * (lane & 1) + 64 * ((lane & 15) >> 2);

  f32x16 o[2][4];
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int i = 0; i < 4; ++i) o[cb][i] = f32x16{};
  f32x16 s[2];
  u32x4 pw[2][2];
  // mc: the running maximum times c, the reference point of p = 2^(s c - mc).  Until a
  // lane has seen a finite score it is -FLT_MAX: every finite score then gives p = +inf
  // (the exact rule takes over), a masked one p = 0, and s c - mc is never NaN
  float mc[2] = {-__FLT_MAX__, -__FLT_MAX__}, l_i[2] = {0.0f, 0.0f};
  const float c = a.scale_log2;

  unsigned stA = 0, stB = kWKBytes, stC = 2 * kWKBytes;
  if (T > 0) {
    dma_rows(true, 0, stA);
    if (wid_s == 0) dma_meta(0);
    dma_issue(1, 0, stB, stA);
  }
  // ---- Q^T of both column blocks in registers, loaded while the first tiles are in
  // flight; rows past Nq load row Nq - 1 and dims past D dims 0..7, zeroed after ----
  u32x4 qreg[kD / 16];
  {
    // both column blocks requested before either is used: one round trip, not two
    u32x4 w[2][kD / 16];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int row = r0w + 32 * cb + ql;
      const uint16_t* qrow = a.q + a.seq.base(b, a.sq_b, a.sq_n) + (int64_t)h * a.sq_h + (int64_t)min(row, Nq - 1) * a.sq_n;
#pragma unroll
      for (int t = 0; t < kD / 16; ++t) {
        const int d0 = 16 * t + 8 * hl;
        w[cb][t] = *(const u32x4*)(qrow + (d0 < a.D ? d0 : 0));
      }
    }
    // redefined so that the loop does not see Q as an outstanding load (the S = K Q^T
    // blocks would otherwise wait for every memory load, the staging loads included)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int row = r0w + 32 * cb + ql;
#pragma unroll
      for (int t = 0; t < kD / 16; ++t) {
        asm volatile("" : "+v"(w[cb][t]));
        const u32x4 qv = (row < Nq && 16 * t + 8 * hl < a.D) ? w[cb][t] : u32x4{0, 0, 0, 0};
        if (cb == 0)
          qreg[t] = qv;
        else
          *(u32x4*)(qs + ql * 256 + (((2 * t + hl) ^ (ql & 15)) << 4)) = qv;
      }
    }
  }
  if (T > 0) {
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    lds_barrier();
  }

  constexpr int kWAhead = 3;    // V^T fragments read ahead of their MFMAs
  constexpr int kWQKAhead = 2;  // (K, Q) fragment pairs read ahead of their MFMAs
  const int nwin = T > 0 ? T + 1 : 0;
  // One window = two sections.  Group 0 runs matrix(w), softmax(w); group 1 runs
  // softmax(w - 1), matrix(w).  Each group has a loop of its own with the section kinds
  // fixed at compile time, so that only P (group 0) or only S (group 1) is live across
  // the loop's back edge.
  auto section = [&](const int sec, auto GRP, auto ODD) {
    constexpr int grp_c = decltype(GRP)::value;
    constexpr bool odd = decltype(ODD)::value;
    const int tl = sec >> 1;
    const int sw = sec - grp_c;
    // each wave issues its window's tile loads in its matrix section, after MFMA pair 6
    bool issued = odd != (grp_c != 0);
    auto issue_once = [&]() {
      if (!issued) {
        dma_issue(tl + 2, tl + 1, stC, stB);
        issued = true;
      }
    };
    if (sw >= 0) {
      const int t = sw >> 1;
      if constexpr (((odd ? 1 : 0) + grp_c) % 2 == 0) {
        // ---- matrix section: O^T += V^T P^T for tile t-1, then S^T = K Q^T for tile t,
        // each LDS fragment feeding both column blocks ----
        __builtin_amdgcn_s_setprio(1);
        const bool do_pv = t >= 1 && !skipped(t - 1);
        const bool do_qk = t < T && !skipped(t);
        // One stream of LDS operand reads for the section: the V^T fragments of the P.V
        // block, then (hybrid, pure) the keys' biases, then the (K, Q) fragment pairs of
        // the S^T block, each read a few MFMA pairs ahead of its use, across the border
        // between the blocks.  The stream's order is fixed at compile time, so every wait
        // is an exact lgkmcnt.
        auto block = [&](auto PVC, auto QKC) {
          constexpr bool PV = decltype(PVC)::value, QK = decltype(QKC)::value;
          constexpr bool BIAS = QK && kWeights;
          constexpr int NPV = PV ? 8 : 0, NQK = QK ? kD / 16 : 0;
          constexpr int EBIAS = NPV;                   // stream index of the bias reads
          constexpr int EQK = NPV + (BIAS ? 1 : 0);    // stream index of (K, Q) pair 0
          constexpr int E = EQK + NQK;                 // stream length
          constexpr int NM = NPV + NQK;                // MFMA pairs
          // stream element of MFMA pair i; elements issued before pair i's wait
          constexpr auto el = [](int i) { return i < NPV ? i : EQK + (i - NPV); };
          constexpr auto size = [](int e) { return (BIAS && e == EBIAS) ? 4 : 2; };
          constexpr auto issued = [el](int i) {
            int n = 0;
            for (int k = 0; k <= i; ++k) {
              const int a = el(k) + 1 + (k < NPV ? kWAhead - 1 : kWQKAhead - 1);
              n = a > n ? a : n;
            }
            return n < E ? n : E;
          };
          constexpr auto pending = [el, size, issued](int i) {
            int c = 0;
            for (int e = el(i) + 1; e < issued(i); ++e) c += size(e);
            return c;
          };
          uint32_t va[4] = {0, 0, 0, 0};
          if constexpr (PV) {
            const uint32_t vb = lds_addr(vst0) + stC;
            // opaque: otherwise the offsets are hoisted out of the loop into registers
            asm volatile("" : "+v"(v_lane));
            const uint32_t vl = vb + v_lane;
#pragma unroll
            for (int db = 0; db < 4; ++db) va[db] = vl ^ (64u * db);
          }
          uint32_t kla = 0, qla = 0, bla = 0;
          if constexpr (QK) {
            asm volatile("" : "+v"(k_lane));
            kla = lds_addr(kst0) + stA + k_lane;
            qla = lds_addr(qs) + k_lane;
            bla = lds_addr(meta_of(t) + kWCnt) + 16 * hl;
          }
          i16x4 vlo[8], vhi[8];
          u32x4 kw[kD / 16], qw[kD / 16], bw[4];
          auto read = [&](auto EC) {
            constexpr int e = decltype(EC)::value;
            if constexpr (e < NPV) {
              vlo[e] = ds_read_tr16<(e >> 2) * 4096>(va[e & 3]);
              vhi[e] = ds_read_tr16<(e >> 2) * 4096 + 2048>(va[e & 3]);
            } else if constexpr (BIAS && e == EBIAS) {
#pragma unroll
              for (int r = 0; r < 4; ++r) bw[r] = ds_read_b128_asm(bla + 32 * r);
            } else {
              constexpr int j = e - EQK;
              kw[j] = ds_read_b128_asm(kla ^ (32u * j));
              qw[j] = ds_read_b128_asm(qla ^ (32u * j));
            }
          };
          static_for<issued(0)>(read);
          static_for<NM>([&](auto I) {
            constexpr int i = decltype(I)::value;
            // the tile loads' scalar address work goes out between MFMA pairs 6 and 7,
            // where it fills the matrix pipe's issue gaps (before pair 0 it delayed the
            // first MFMA by about a hundred instructions)
            if constexpr (i == 6) issue_once();
            if constexpr (i < NPV) {
              lgkm_wait<pending(i)>(vlo[i], vhi[i]);
              const u32x4 vw = __builtin_bit_cast(u32x4, __builtin_shufflevector(vlo[i], vhi[i], 0, 1, 2, 3, 4, 5, 6, 7));
              o[0][i & 3] = E16<DT>::mfma(vw, pw[0][i >> 2], o[0][i & 3]);
              o[1][i & 3] = E16<DT>::mfma(vw, pw[1][i >> 2], o[1][i & 3]);
            } else {
              constexpr int j = i - NPV;
              lgkm_wait<pending(i)>(kw[j], qw[j]);
              if constexpr (j == 0) {
                // S^T starts at the keys' biases (read before pair 0, so complete now),
                // or at zero (the MFMA's inline constant)
                if constexpr (BIAS) {
                  asm volatile("" : "+v"(bw[0]), "+v"(bw[1]), "+v"(bw[2]), "+v"(bw[3]));
                  const f32x4 b0 = __builtin_bit_cast(f32x4, bw[0]), b1 = __builtin_bit_cast(f32x4, bw[1]);
                  const f32x4 b2 = __builtin_bit_cast(f32x4, bw[2]), b3 = __builtin_bit_cast(f32x4, bw[3]);
                  const f32x16 c0 = __builtin_shufflevector(__builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7),
                                                            __builtin_shufflevector(b2, b3, 0, 1, 2, 3, 4, 5, 6, 7),
                                                            0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
                  s[0] = E16<DT>::mfma(kw[0], qreg[0], c0);
                  s[1] = E16<DT>::mfma(kw[0], qw[0], c0);
                } else {
                  s[0] = E16<DT>::mfma(kw[0], qreg[0], f32x16{});
                  s[1] = E16<DT>::mfma(kw[0], qw[0], f32x16{});
                }
              } else {
                s[0] = E16<DT>::mfma(kw[j], qreg[j], s[0]);
                s[1] = E16<DT>::mfma(kw[j], qw[j], s[1]);
              }
            }
            static_for<issued(i + 1 < NM ? i + 1 : i) - issued(i)>([&](auto K) {
              read(std::integral_constant<int, issued(i) + decltype(K)::value>{});
            });
          });
        };
        using BT = std::integral_constant<bool, true>;
        using BF = std::integral_constant<bool, false>;
        // The S^T block always runs: where tile t is past the end or skipped, it reads a
        // stage and a bias slot that hold other data (in bounds) and the softmax ignores
        // the result.  A third instantiation without it costs more registers than the
        // few blocks it saves.
        if (do_pv)
          block(BT{}, BT{});
        else
          block(BF{}, BT{});
        issue_once();
        if (!do_qk) {
          // not read before the next QK block defines it
          undefined(s[0]);
          undefined(s[1]);
        }
        __builtin_amdgcn_s_setprio(0);
      } else if (!(t < T && !skipped(t))) {
        // not read before the next softmax defines it
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
          for (int j = 0; j < 2; ++j) undefined(pw[cb][j]);
      } else {
        // ---- softmax section for tile t: the two column blocks one after the other, one
        // check each ----
        const char* ms = meta_of(t);
        const int key0 = key0_of(t);
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          const int row = r0w + 32 * cb + ql;
          if (kPureV) {
            mask_pure32(s[cb], (const int*)(ms + kWTs), row, hl);
          } else if (t >= n1) {
            if ((a.causal && key0 + kWTK - 1 > r0w + 32 * cb) || key0 + kWTK > Nk)
              mask_dense32(s[cb], key0, row, hl, Nk, a.causal);
          }
        }
        // p against the current maximum first; only where a lane's sum of its 16 p
        // exceeds kLazySum (some p above 2^8, a score above the maximum by 8 / c; +inf
        // while the lane has no maximum yet) is the tile's maximum taken and the column
        // block redone with the lazy-rescale rule.  P in the 16-bit type for the P.V
        // MFMAs; the row sum adds the fp32 p, as deltaFlashAttention.py:86-98
        auto exps = [&](const int cb, const float neg) {
          float psa, psb;
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            float p[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) p[e] = exp2_fast(__builtin_fmaf(s[cb][4 * r4 + e], c, neg));
            pw[cb][r4 >> 1][(r4 & 1) * 2 + 0] = E16<DT>::pack(p[0], p[1]);
            pw[cb][r4 >> 1][(r4 & 1) * 2 + 1] = E16<DT>::pack(p[2], p[3]);
            psa = r4 == 0 ? p[0] + p[1] : psa + (p[0] + p[1]);
            psb = r4 == 0 ? p[2] + p[3] : psb + (p[2] + p[3]);
          }
          return psa + psb;
        };
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          float ps = exps(cb, -mc[cb]);
          // the bound also catches an infinite sum
          if (__builtin_amdgcn_ballot_w64(ps > kLazySum)) {
            float m = -INFINITY;
#pragma unroll
            for (int r = 0; r < 16; r += 2) m = __builtin_fmaxf(m, __builtin_fmaxf(s[cb][r], s[cb][r + 1]));
            const float mxc = halves_max(m) * c;
            // alpha = 1 exactly where a lane keeps its maximum (also where it has none yet)
            const bool upd = mxc > mc[cb] + kLazyLog2;
            const float m_new = upd ? mxc : mc[cb];
            const float alpha = upd ? exp2_fast(mc[cb] - m_new) : 1.0f;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
              for (int r = 0; r < 16; ++r) o[cb][db][r] *= alpha;
            l_i[cb] *= alpha;
            mc[cb] = m_new;
            ps = exps(cb, -m_new);
          }
          l_i[cb] += ps;
        }
      }
    }
    issue_once();
    if (odd) {
      // the loads of window tl - 1 are done when at most this window's are pending
      if (wid_s == 0)
        __builtin_amdgcn_s_waitcnt(vmcnt_only(2 + (kWeights ? 1 : 0) + (kPureV ? 1 : 0)));
      else
        __builtin_amdgcn_s_waitcnt(vmcnt_only(2));
      barrier_keep_loads();
    }
  };
  using False = std::integral_constant<bool, false>;
  using True = std::integral_constant<bool, true>;
  auto rotate_stages = [&]() {
    const unsigned t0 = stA;
    stA = stB;
    stB = stC;
    stC = t0;
  };
  if (grp == 0) {
    for (int w = 0; w < nwin; ++w) {
      section(2 * w, std::integral_constant<int, 0>{}, False{});
      section(2 * w + 1, std::integral_constant<int, 0>{}, True{});
      rotate_stages();
    }
  } else {
    for (int w = 0; w < nwin; ++w) {
      section(2 * w, std::integral_constant<int, 1>{}, False{});
      section(2 * w + 1, std::integral_constant<int, 1>{}, True{});
      rotate_stages();
    }
  }
  __builtin_amdgcn_s_waitcnt(vmcnt_only(0));  // no load may land in LDS after the exit

  // ---- finalize: each column block goes through the wave's own Q region of LDS (its
  // last Q.K is done), 16-byte chunk c of row r at position c ^ (r & 15), and leaves as
  // whole rows, four per store instruction, instead of 16 bytes of 32 rows ----
  uint16_t* const obase = a.out + a.seq.base(b, a.so_b, a.so_n) + (int64_t)h * a.so_h;
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const float l_tot = halves_sum(l_i[cb]);
    float inv;
    if (VARIANT == kPure)
      inv = l_tot > 0.0f ? 1.0f / l_tot : 1.0f;  // deltaFlashAttention.py:353-354
    else
      inv = 1.0f / l_tot;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x2 w;
        w[0] = E16<DT>::pack(o[cb][db][4 * j + 0] * inv, o[cb][db][4 * j + 1] * inv);
        w[1] = E16<DT>::pack(o[cb][db][4 * j + 2] * inv, o[cb][db][4 * j + 3] * inv);
        // dims db * 32 + 8 j + 4 hl .. + 3 of row ql: half hl of chunk 4 db + j
        *(u32x2*)(qs + ql * 256 + (((4 * db + j) ^ (ql & 15)) << 4) + 8 * hl) = w;
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    const int cq = lane & 15;
    u32x4 rw[8];
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int r = 4 * it + (lane >> 4);
      rw[it] = *(const u32x4*)(qs + r * 256 + ((cq ^ (r & 15)) << 4));
    }
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int row = r0w + 32 * cb + 4 * it + (lane >> 4);
      if (row < Nq && cq * 8 < a.D) *(u32x4*)(obase + (int64_t)row * a.so_n + cq * 8) = rw[it];
    }
    // the reads of this block are done before the next block overwrites the region
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
  }
}

// Work distribution.  Static (a.queue null, the dense control): workgroup i runs on XCD
// i mod 8 and takes one item; when the units split evenly over the 8 XCDs, each XCD gets
// a contiguous range of units and walks their row groups longest first, so a unit's K/V
// stay in one XCD's L2.  Persistent (a.queue set, the hybrid, sanity and pure Phase 1
// variants, whose schedule kernel zeroes the 8 counters just before): one workgroup per
// CU loops over items.  Queue q holds the units of XCD q's static share in the same
// order (unit by unit, longest row group first) and a.queue[q] counts the items taken;
// a workgroup takes from the queue of the XCD it runs on and, once that is empty, from
// the others, so the XCDs, whose clocks differ by several per cent, finish together,
// and no dispatch gap lies between two items on a CU.  Every counter only grows, so each
// workgroup's loop ends after at most 8 empty takes; workgroups never wait on each other.
template <int VARIANT, int DT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_w64_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  int* const slot = (int*)(smem + kWItemSlot);
  const int tid = threadIdx.x;
  const int n_rg = a.n_row_groups;
  const bool persistent = a.queue != nullptr;
  unsigned xcc = 0;
  if (persistent) {
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    if (tid == 0) slot[2] = 0;  // queues found empty so far, from this XCD's own
  }
  for (int first = 1;; first = 0) {
    int unit, rg;
    if (!persistent) {
      if (!first) break;
      const int wg = blockIdx.x;
      if ((a.units & 7) == 0) {
        const int xcd = wg & 7, idx = wg >> 3, upx = a.units >> 3;
        unit = xcd * upx + idx / n_rg;
        rg = n_rg - 1 - idx % n_rg;
      } else {
        unit = wg % a.units;
        rg = n_rg - 1 - wg / a.units;
      }
    } else {
      if (tid == 0) {
        int q = 0, k = -1, qi = slot[2];
        while (qi < 8) {
          q = (int)((xcc + qi) & 7);
          int ulo, uhi;
          queue_units(q, a.units, ulo, uhi);
          const int taken = atomicAdd(a.queue + q, 1);
          if (taken < (uhi - ulo) * n_rg) {
            k = taken;
            break;
          }
          ++qi;
        }
        slot[0] = q;
        slot[1] = k;
        slot[2] = qi;
      }
      lds_barrier();
      const int q = __builtin_amdgcn_readfirstlane(slot[0]);
      const int k = __builtin_amdgcn_readfirstlane(slot[1]);
      lds_barrier();  // the slot is read before thread 0 writes it again
      if (k < 0) break;
      int ulo, uhi;
      queue_units(q, a.units, ulo, uhi);
      const int j = k / n_rg;
      unit = ulo + j;
      rg = n_rg - 1 - (k - j * n_rg);
    }
#if defined(__HIP_DEVICE_COMPILE__)
    // the argument block read through the kernel-argument segment's address, made
    // opaque per item: its fields are loaded inside each item instead of being held in
    // scalar registers across the loop (the block is the kernel's only argument, at
    // offset 0)
    const __attribute__((address_space(4))) AttnArgs* ap =
        (const __attribute__((address_space(4))) AttnArgs*)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    const AttnArgs ai = *ap;
    attn_w64_item<VARIANT, DT>(ai, unit, rg);
#else
    attn_w64_item<VARIANT, DT>(a, unit, rg);
#endif
  }
}

// Per (batch, kv head): maxima of packed blocks of 128 timestamps (lanes at or
// beyond P read seq_len_k + 1, deltaFlashAttention.py:70) and their prefix maxima.
// Blocks with blockIdx.y = 0 do that; those with blockIdx.y = 1 + c (when wts is set)
// write, for packed rows [1024 c, 1024 c + 1024), the key bias log2(w) / scale_log2 of
// the row's weight w (the count, 1 with no_count, 0 at and beyond P:
// modeling_llama.py:321-324 and the masked loads of deltaFlashAttention.py:84-90; -inf
// for w = 0), so that exp2(scale_log2 (q.k + bias) - m) = w exp2(scale_log2 q.k - m);
// with tsw set the timestamps with INT_MAX where the weight is 0; block (0, 1) writes
// 64 zero biases.
struct SchedPrep {
  const void* cnt;
  int64_t scnt_b, scnt_h;
  int cnt_is_float, no_count;
  float scale_log2;
  float* wts;
  int32_t* tsw;
  float* zeros;
  int wcap;
};
constexpr int kSchedThreads = 1024;
constexpr int kSchedWaves = kSchedThreads / 64;
__global__ __launch_bounds__(kSchedThreads) void hybrid_schedule_kernel(const int32_t* __restrict__ ts,
                                                              int64_t sts_b, int64_t sts_h,
                                                              int Hkv, int P_host,
                                                              const int32_t* P_dev, int Nk,
                                                              SeqMap seq, int nblk_cap,
                                                              int32_t* __restrict__ sched,
                                                              SchedPrep prep, int* __restrict__ queue) {
  __shared__ int32_t s_bmax[4096];
  __shared__ int32_t s_wave[kSchedWaves];
  const int tid = threadIdx.x, lane = tid & 63;
  // the attention kernel's work-queue counters start at zero
  if (queue && blockIdx.x == 0 && blockIdx.y == 0 && tid < 8) queue[tid] = 0;
  const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  const int bg = blockIdx.x;
  const int b = bg / Hkv, g = bg - (bg / Hkv) * Hkv;
  int P = P_host;
  if (P_dev) P = min(seq.cu ? P_dev[b] : *P_dev, P_host);
  if (seq.cu) {
    Nk = seq.len(b);
    P = min(P, Nk);  // a sequence's packed rows lie inside its own tokens
  }
  const int nblk = (P + kBlock - 1) / kBlock;
  const int32_t* row = ts + seq.base(b, sts_b, 1) + (int64_t)g * sts_h;
  if (blockIdx.y > 0) {
    const int32_t* crow = (const int32_t*)prep.cnt + seq.base(b, prep.scnt_b, 1) + (int64_t)g * prep.scnt_h;
    float* wrow = prep.wts + (int64_t)bg * prep.wcap;
    int32_t* trow = prep.tsw ? prep.tsw + (int64_t)bg * prep.wcap : nullptr;
    if (bg == 0 && blockIdx.y == 1 && tid < kTileN) prep.zeros[tid] = 0.0f;
    // the attention kernels read rows below nblk * 128 only
    const int i = (blockIdx.y - 1) * kSchedThreads + tid;
    if ((blockIdx.y - 1) * kSchedThreads >= nblk * kBlock || i >= prep.wcap) return;
    float w = 0.0f;
    int tv = INT_MAX;
    if (i < P) {
      const int32_t raw = crow[i];
      w = prep.no_count ? 1.0f : (prep.cnt_is_float ? __int_as_float(raw) : (float)raw);
      if (trow && w > 0.0f) tv = row[i];
    }
    wrow[i] = w > 0.0f ? log2f(w) / prep.scale_log2 : -INFINITY;
    if (trow) trow[i] = tv;
    return;
  }
  // wave w takes blocks 8w .. 8w + 7 of every 8 kSchedWaves, their loads in flight together:
  // rows at or beyond P are clamped to row P - 1 and masked after the load (a guarded
  // load is waited for before the next one is issued); nblk > 0 implies P > 0
  for (int jb0 = wid * 8; jb0 < nblk; jb0 += 8 * kSchedWaves) {
    int m[8];
    int r0[8], r1[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i0 = (jb0 + u) * kBlock + lane, i1 = i0 + 64;
      r0[u] = row[min(i0, P - 1)];
      r1[u] = row[min(i1, P - 1)];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i0 = (jb0 + u) * kBlock + lane, i1 = i0 + 64;
      m[u] = max(i0 < P ? r0[u] : Nk + 1, i1 < P ? r1[u] : Nk + 1);
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) m[u] = max(m[u], __shfl_xor(m[u], d, 64));
      if (lane == 0 && jb0 + u < nblk) s_bmax[jb0 + u] = m[u];
    }
  }
  __syncthreads();
  const int per = (nblk + kSchedThreads - 1) / kSchedThreads;
  const int j0 = min(tid * per, nblk), j1 = min(j0 + per, nblk);
  int mloc = INT_MIN;
  for (int j = j0; j < j1; ++j) mloc = max(mloc, s_bmax[j]);
  int incl = mloc;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(incl, d, 64);
    if (lane >= d) incl = max(incl, o);
  }
  if (lane == 63) s_wave[wid] = incl;
  __syncthreads();
  int pre = INT_MIN;
  for (int w2 = 0; w2 < wid; ++w2) pre = max(pre, s_wave[w2]);
  int excl = __shfl_up(incl, 1, 64);  // maximum over earlier lanes of this wave
  if (lane == 0) excl = INT_MIN;
  int run = max(pre, excl);
  int32_t* bm = sched + (int64_t)bg * 2 * nblk_cap;
  int32_t* pm = bm + nblk_cap;
  for (int j = j0; j < j1; ++j) {
    run = max(run, s_bmax[j]);
    bm[j] = s_bmax[j];
    pm[j] = run;
  }
}

// ====================================================================================
// fp32 tensors.  The reference's kernels take fp32 Q, K, V as they take 16-bit ones
// (dtype-agnostic loads, deltaFlashAttention.py:41-42, 80; flashAttention.py:94-130), and
// p.to(v.dtype) then leaves p in fp32 (:98, :137).  attn_f32_kernel computes the same
// attention in fp32 throughout: one workgroup of 256 threads per (batch, query head,
// 64 query rows), LDS tiles of 64 keys, fp32 FMAs on the VALU (the MFMA path is 16-bit),
// an exact running maximum (rescaled at every new maximum) and P.V on the fp32 p.  The
// logical 128-row schedule, the key biases log2(w)/c and the variants come from the same
// schedule pre-pass as the 16-bit kernels.  Thread (ti, tj) holds scores of rows
// 4 ti .. 4 ti + 3 and keys tj + 16 jj, and output dims 4 tj + 64 gg of the same rows.
// ====================================================================================
constexpr int kFRows = 64, kFKeys = 64;
constexpr int kFStride = kD + 4;        // row stride (floats) of the Q, K and V tiles
constexpr int kFPStride = kFKeys + 4;   // row stride of the P tile
constexpr int kFLds = (kFRows * kFStride + 2 * kFKeys * kFStride + kFRows * kFPStride + 2 * kFKeys) * 4;

template <int VARIANT>
__global__ __launch_bounds__(256) void attn_f32_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) float fsm[];
  float* const sQ = fsm;
  float* const sK = sQ + kFRows * kFStride;
  float* const sV = sK + kFKeys * kFStride;
  float* const sP = sV + kFKeys * kFStride;
  float* const sB = sP + kFRows * kFPStride;  // the tile's key biases (units of the score)
  int* const sT = (int*)(sB + kFKeys);        // the tile's timestamps (pure Phase 1)
  const int tid = threadIdx.x;
  const int ti = tid >> 4, tj = tid & 15;
  const int nrb = (a.Nq + kFRows - 1) / kFRows;
  const int rb = (int)(blockIdx.x % (unsigned)nrb);
  const int bh = (int)(blockIdx.x / (unsigned)nrb);
  const int h = bh % a.Hq, b = bh / a.Hq;
  const int g = h / a.G;
  const int bg = b * a.Hkv + g;
  const int Nq = a.seq.cu ? a.seq.len(b) : a.Nq;
  const int Nk = a.seq.cu ? a.seq.len(b) : a.Nk;
  const int R0 = rb * kFRows;
  if (R0 >= Nq) return;  // a row block past the end of a shorter sequence (whole workgroup)
  const int D = a.D;
  const float c = a.scale_log2;

  // ---- schedule of the logical 128-row block holding these rows (every wave computes
  // the same values).  Phase 1: packed keys [0, n1); Phase 2: keys [ds, kend), causal.
  // Keys past the block's own last row are all masked, so Phase 2 ends there. ----
  const int start_m = (R0 / kBlock) * kBlock;
  int P = a.P_host;
  if (a.P_dev) P = min(a.seq.cu ? a.P_dev[b] : *a.P_dev, a.P_host);
  if (a.seq.cu) P = min(P, Nk);
  int n1 = 0, ds = 0;
  int kend = a.causal ? min(Nk, R0 + kFRows) : Nk;
  if (VARIANT == kHybrid || VARIANT == kSanity) {
    const int nblk = (P + kBlock - 1) / kBlock;
    const int32_t* bmax = a.sched + (int64_t)bg * 2 * a.nblk_cap;
    int n_safe, last;
    safe_prefix(bmax, bmax + a.nblk_cap, nblk, start_m - a.window, n_safe, last, tid & 63);
    ds = max(0, ((last + 1) / kBlock) * kBlock);
    if (VARIANT == kHybrid) n1 = min(n_safe * kBlock, a.wcap);
  } else if (VARIANT == kPure) {
    n1 = P;
    kend = 0;
  }
  const int t1 = (n1 + kFKeys - 1) / kFKeys;
  const int t2 = kend > ds ? (kend - ds + kFKeys - 1) / kFKeys : 0;

  const float* qg = (const float*)a.q + a.seq.base(b, a.sq_b, a.sq_n) + (int64_t)h * a.sq_h;
  const float* kg = (const float*)a.k + a.seq.base(b, a.sk_b, a.sk_n) + (int64_t)g * a.sk_h;
  const float* vg = (const float*)a.v + a.seq.base(b, a.sv_b, a.sv_n) + (int64_t)g * a.sv_h;
  const float* kpg = (const float*)a.kp + a.seq.base(b, a.skp_b, a.skp_n) + (int64_t)g * a.skp_h;
  const float* vpg = (const float*)a.vp + a.seq.base(b, a.svp_b, a.svp_n) + (int64_t)g * a.svp_h;
  const float* wrow = a.wts ? a.wts + (int64_t)bg * a.wcap : nullptr;
  const int32_t* tsrow = a.tsw ? a.tsw + (int64_t)bg * a.wcap : nullptr;

  // ---- Q of the 64 rows (rows past Nq and dims past D are zero) ----
  for (int i = tid; i < kFRows * (kD / 4); i += 256) {
    const int r = i / (kD / 4), d = 4 * (i % (kD / 4));
    float4 x = {0.0f, 0.0f, 0.0f, 0.0f};
    if (R0 + r < Nq && d < D) x = *(const float4*)(qg + (int64_t)(R0 + r) * a.sq_n + d);
    *(float4*)(sQ + r * kFStride + d) = x;
  }

  float o[4][2][4];
  float m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.0f;
#pragma unroll
    for (int gg = 0; gg < 2; ++gg)
#pragma unroll
      for (int e = 0; e < 4; ++e) o[i][gg][e] = 0.0f;
  }

  for (int t = 0; t < t1 + t2; ++t) {
    const bool ph1 = t < t1;
    const int key0 = ph1 ? t * kFKeys : ds + (t - t1) * kFKeys;
    if (!ph1 && a.causal && key0 > R0 + kFRows - 1) break;  // every later tile is masked
    const int kvalid = ph1 ? n1 : kend;  // keys [key0, kvalid) of this tile are real
    const int klimit = ph1 ? P : Nk;     // rows of the source tensor that exist
    const float* ksrc = ph1 ? kpg : kg;
    const float* vsrc = ph1 ? vpg : vg;
    const int64_t skn = ph1 ? a.skp_n : a.sk_n, svn = ph1 ? a.svp_n : a.sv_n;
    __syncthreads();  // the previous tile's K, V, P and biases are read
    for (int i = tid; i < kFKeys * (kD / 4); i += 256) {
      const int r = i / (kD / 4), d = 4 * (i % (kD / 4));
      const int key = key0 + r;
      float4 kx = {0.0f, 0.0f, 0.0f, 0.0f}, vx = kx;
      if (key < kvalid && key < klimit && d < D) {
        kx = *(const float4*)(ksrc + (int64_t)key * skn + d);
        vx = *(const float4*)(vsrc + (int64_t)key * svn + d);
      }
      *(float4*)(sK + r * kFStride + d) = kx;
      *(float4*)(sV + r * kFStride + d) = vx;
    }
    if (tid < kFKeys) {
      const int key = key0 + tid;
      float bias = key < kvalid ? 0.0f : -INFINITY;
      int ts = 0;
      if (ph1 && (VARIANT == kHybrid || VARIANT == kPure) && key < kvalid) bias = wrow[key];
      if (ph1 && VARIANT == kPure && key < kvalid) ts = tsrow[key];
      sB[tid] = bias;
      sT[tid] = ts;
    }
    __syncthreads();

    // ---- scores of rows 4 ti + i and keys tj + 16 jj ----
    float sc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) sc[i][jj] = 0.0f;
    for (int d = 0; d < D; d += 4) {
      float4 qv[4], kv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) qv[i] = *(const float4*)(sQ + (4 * ti + i) * kFStride + d);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) kv[jj] = *(const float4*)(sK + (tj + 16 * jj) * kFStride + d);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          sc[i][jj] = __builtin_fmaf(qv[i].x, kv[jj].x, sc[i][jj]);
          sc[i][jj] = __builtin_fmaf(qv[i].y, kv[jj].y, sc[i][jj]);
          sc[i][jj] = __builtin_fmaf(qv[i].z, kv[jj].z, sc[i][jj]);
          sc[i][jj] = __builtin_fmaf(qv[i].w, kv[jj].w, sc[i][jj]);
        }
    }
    // ---- masks, online softmax (exact maximum), p to LDS ----
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = R0 + 4 * ti + i;
      float mt = -INFINITY;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int kl = tj + 16 * jj;
        bool ok = sB[kl] != -INFINITY;
        if (!ph1 && a.causal) ok = ok && key0 + kl <= row;                 // deltaFlashAttention.py:126-130
        if (VARIANT == kPure) ok = ok && sT[kl] <= row;                    // :338-341
        sc[i][jj] = ok ? (sc[i][jj] + sB[kl]) * c : -INFINITY;
        mt = __builtin_fmaxf(mt, sc[i][jj]);
      }
#pragma unroll
      for (int x = 1; x < 16; x <<= 1) mt = __builtin_fmaxf(mt, __shfl_xor(mt, x, 64));
      const float mn = __builtin_fmaxf(m[i], mt);
      const float alpha = mn == -INFINITY ? 1.0f : exp2f(m[i] - mn);
      float ps = 0.0f;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float pv = mn == -INFINITY ? 0.0f : exp2f(sc[i][jj] - mn);
        ps += pv;
        sP[(4 * ti + i) * kFPStride + tj + 16 * jj] = pv;
      }
#pragma unroll
      for (int x = 1; x < 16; x <<= 1) ps += __shfl_xor(ps, x, 64);
      l[i] = l[i] * alpha + ps;
      m[i] = mn;
#pragma unroll
      for (int gg = 0; gg < 2; ++gg)
#pragma unroll
        for (int e = 0; e < 4; ++e) o[i][gg][e] *= alpha;
    }
    __syncthreads();
    // ---- O += P V on dims 4 tj + 64 gg ----
    for (int j = 0; j < kFKeys; ++j) {
      float pj[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pj[i] = sP[(4 * ti + i) * kFPStride + j];
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        const float4 vv = *(const float4*)(sV + j * kFStride + 4 * tj + 64 * gg);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o[i][gg][0] = __builtin_fmaf(pj[i], vv.x, o[i][gg][0]);
          o[i][gg][1] = __builtin_fmaf(pj[i], vv.y, o[i][gg][1]);
          o[i][gg][2] = __builtin_fmaf(pj[i], vv.z, o[i][gg][2]);
          o[i][gg][3] = __builtin_fmaf(pj[i], vv.w, o[i][gg][3]);
        }
      }
    }
  }

  // ---- normalise and store rows < Nq, dims < D ----
  float* og = (float*)a.out + a.seq.base(b, a.so_b, a.so_n) + (int64_t)h * a.so_h;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = R0 + 4 * ti + i;
    if (row >= Nq) continue;
    // a row without any key (pure Phase 1) stays zero, deltaFlashAttention.py:353-354
    const float inv = l[i] > 0.0f ? 1.0f / l[i] : 0.0f;
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      const int d = 4 * tj + 64 * gg;
      if (d < D)
        *(float4*)(og + (int64_t)row * a.so_n + d) =
            float4{o[i][gg][0] * inv, o[i][gg][1] * inv, o[i][gg][2] * inv, o[i][gg][3] * inv};
    }
  }
}

template <int V, int DT>
static const void* attn_kernel_fn() {
  if constexpr (V == kPure) return reinterpret_cast<const void*>(&attn_kernel_pure<DT>);
  else return reinterpret_cast<const void*>(&attn_kernel<V, DT>);
}

template <int V, int DT>
static int allow_lds(size_t bytes) {
  static int done = 0;
  if (!done) {
    hipError_t e = hipFuncSetAttribute(attn_kernel_fn<V, DT>(),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e != hipSuccess) return set_error(DA_ERR_HIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    done = 1;
  }
  return DA_OK;
}

// Compute units of the current device (cached per device).
static int cu_count() {
  static int n[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!n[dev]) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    n[dev] = v;
  }
  return n[dev];
}

template <int V, int DT>
static int allow_lds_w64(size_t bytes) {
  static int done = 0;
  if (!done) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_w64_kernel<V, DT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e != hipSuccess) return set_error(DA_ERR_HIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    done = 1;
  }
  return DA_OK;
}

template <int V, int DT>
static int launch_attn_t(AttnArgs& a, hipStream_t st) {
  if (a.hpw == 4) {
    a.rows_per_wg = 128;
    a.n_row_groups = (a.Nq + 127) / 128;
    const size_t lds = kWLds;
    const int64_t items = (int64_t)a.n_row_groups * a.units;
    // persistent: one workgroup per CU (the LDS of one fills a CU) takes items until the
    // queues are empty; static: one workgroup per item
    const unsigned grid = (unsigned)(a.queue ? std::min<int64_t>(items, cu_count()) : items);
    if (int rc = allow_lds_w64<V, DT>(lds)) return rc;
    hipLaunchKernelGGL((attn_w64_kernel<V, DT>), dim3(grid), dim3(512), lds, st, a);
    return check_launch("attention kernel (ping-pong)");
  }
  const size_t lds = 2 * kStageBytes;
  const unsigned grid = (unsigned)((int64_t)a.n_row_groups * a.units);
  if (int rc = allow_lds<V, DT>(lds)) return rc;
  if constexpr (V == kPure)
    hipLaunchKernelGGL((attn_kernel_pure<DT>), dim3(grid), dim3(256), lds, st, a);
  else
    hipLaunchKernelGGL((attn_kernel<V, DT>), dim3(grid), dim3(256), lds, st, a);
  return check_launch("attention kernel");
}

template <int DT>
static int launch_attn_dt(int variant, AttnArgs& a, hipStream_t st) {
  switch (variant) {
    case kHybrid: return launch_attn_t<kHybrid, DT>(a, st);
    case kSanity: return launch_attn_t<kSanity, DT>(a, st);
    case kPure: return launch_attn_t<kPure, DT>(a, st);
    default: return launch_attn_t<kDense, DT>(a, st);
  }
}

template <int V>
static int launch_attn_f32_t(const AttnArgs& a, hipStream_t st) {
  static int done = 0;
  if (!done) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_f32_kernel<V>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, kFLds);
    if (e != hipSuccess) return set_error(DA_ERR_HIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    done = 1;
  }
  const int64_t grid = (int64_t)a.B * a.Hq * ((a.Nq + kFRows - 1) / kFRows);
  if (grid >= (1ll << 31)) return set_error(DA_ERR_INVALID, "attention (fp32): grid too large");
  hipLaunchKernelGGL((attn_f32_kernel<V>), dim3((unsigned)grid), dim3(256), kFLds, st, a);
  return check_launch("attention kernel (fp32)");
}

static int launch_attn(int variant, int dtype, AttnArgs& a, hipStream_t st) {
  if (dtype == DA_F32) {
    switch (variant) {
      case kHybrid: return launch_attn_f32_t<kHybrid>(a, st);
      case kSanity: return launch_attn_f32_t<kSanity>(a, st);
      case kPure: return launch_attn_f32_t<kPure>(a, st);
      default: return launch_attn_f32_t<kDense>(a, st);
    }
  }
  return dtype == DA_F16 ? launch_attn_dt<DA_F16>(variant, a, st) : launch_attn_dt<DA_BF16>(variant, a, st);
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

static int fill_common(AttnArgs& a, const void* q, const void* k, const void* v, void* out,
                       int64_t B, int64_t Hq, int64_t Hkv, int64_t Nq, int64_t Nk, int64_t D,
                       const int64_t* st, float scale, const char* who) {
  DA_REQUIRE(q && k && v && out && st, "%s: null pointer", who);
  DA_REQUIRE(B > 0 && Hq > 0 && Hkv > 0 && Nq > 0 && Nk > 0, "%s: empty shape", who);
  if (D <= 0 || D > kD || (D & 7))
    return set_error(DA_ERR_UNSUPPORTED, "%s: head_dim must be a multiple of 8 in [8, 128] (got %lld)", who,
                     (long long)D);
  DA_REQUIRE(Hq % Hkv == 0, "%s: Hq (%lld) must be a multiple of Hkv (%lld)", who, (long long)Hq, (long long)Hkv);
  DA_REQUIRE(Nq < (1ll << 30) && Nk < (1ll << 30), "%s: sequence too long", who);
  DA_REQUIRE(scale > 0.0f, "%s: scale must be positive", who);
  for (int i = 0; i < 18; ++i)
    DA_REQUIRE((st[i] & 7) == 0, "%s: strides must be multiples of 8 elements (stride %d = %lld)", who, i, (long long)st[i]);
  DA_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out), "%s: tensors must be 16-byte aligned", who);
  for (int i : {DA_STRIDE_K + 2, DA_STRIDE_V + 2})
    DA_REQUIRE(st[i] >= D && st[i] < (1ll << 23),
               "%s: key/value sequence strides must be in [head_dim, 2^23) (stride %d = %lld)", who, i, (long long)st[i]);
  a.q = (const uint16_t*)q; a.k = (const uint16_t*)k; a.v = (const uint16_t*)v; a.out = (uint16_t*)out;
  a.sq_b = st[DA_STRIDE_Q]; a.sq_h = st[DA_STRIDE_Q + 1]; a.sq_n = st[DA_STRIDE_Q + 2];
  a.sk_b = st[DA_STRIDE_K]; a.sk_h = st[DA_STRIDE_K + 1]; a.sk_n = st[DA_STRIDE_K + 2];
  a.sv_b = st[DA_STRIDE_V]; a.sv_h = st[DA_STRIDE_V + 1]; a.sv_n = st[DA_STRIDE_V + 2];
  a.so_b = st[DA_STRIDE_OUT]; a.so_h = st[DA_STRIDE_OUT + 1]; a.so_n = st[DA_STRIDE_OUT + 2];
  a.B = (int)B; a.Hq = (int)Hq; a.Hkv = (int)Hkv; a.G = (int)(Hq / Hkv);
  a.Nq = (int)Nq; a.Nk = (int)Nk;
  a.D = (int)D;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.hpw = (a.G % 4 == 0) ? 4 : (a.G % 2 == 0 ? 2 : 1);
  a.rows_per_wg = 32 * (4 / a.hpw);
  a.n_row_groups = (int)((Nq + a.rows_per_wg - 1) / a.rows_per_wg);
  a.units = (int)(B * Hkv * (a.G / a.hpw));
  DA_REQUIRE((int64_t)a.n_row_groups * a.units < (1ll << 31), "%s: grid too large", who);
  return DA_OK;
}

}  // namespace da

using namespace da;

// Workspace of da_hybrid_prefill: the schedule ([B*Hkv][2][nblk] int32), then, each at
// a 256-byte boundary, the key biases ([B*Hkv][wcap] fp32), the timestamps of the pure
// Phase-1 variant ([B*Hkv][wcap] int32), 64 zeros and the attention kernel's 8
// work-queue counters; nblk = ceil(num_packed / 128) (at least 1), wcap = 128 nblk.
struct HybridWs {
  int nblk, wcap;
  int64_t w_off, ts_off, zeros_off, queue_off, total;
};
static int64_t round256(int64_t x) { return (x + 255) & ~(int64_t)255; }
static HybridWs hybrid_ws(int64_t B, int64_t Hkv, int64_t num_packed) {
  HybridWs w;
  const int64_t nblk = std::max<int64_t>(1, (num_packed + kBlock - 1) / kBlock);
  w.nblk = (int)nblk;
  w.wcap = (int)(nblk * kBlock);
  w.w_off = round256(B * Hkv * 2 * nblk * (int64_t)sizeof(int32_t));
  w.ts_off = w.w_off + round256(B * Hkv * w.wcap * (int64_t)sizeof(float));
  w.zeros_off = w.ts_off + round256(B * Hkv * w.wcap * (int64_t)sizeof(int32_t));
  w.queue_off = w.zeros_off + 256;
  w.total = w.queue_off + 256;
  return w;
}

extern "C" int64_t da_hybrid_workspace_size(int64_t B, int64_t Hkv, int64_t num_packed) {
  return hybrid_ws(B, Hkv, num_packed).total;
}

// Everything of da_hybrid_prefill / da_hybrid_prefill_varlen after the shapes are known:
// validation of the packed tensors and workspace, the schedule pre-pass, the launch.
// P_bound is the host upper bound of P (num_packed, or the longest sequence of a ragged
// batch), which sizes the workspace.
static int hybrid_impl(const char* who, AttnArgs& a, const void* k_packed, const void* v_packed,
                       const int32_t* timestamps, const void* counts, int counts_dtype, int dtype,
                       int64_t B, int64_t Hkv, int64_t Nk, const int64_t* strides, int64_t P_bound,
                       const int32_t* num_packed_dev, int64_t window, int variant, int no_count,
                       void* workspace, int64_t workspace_bytes, hipStream_t st) {
  DA_REQUIRE(variant == DA_VARIANT_HYBRID || variant == DA_VARIANT_SANITY ||
                 variant == DA_VARIANT_PURE_PHASE1,
             "%s: unknown variant %d", who, variant);
  DA_REQUIRE(k_packed && v_packed && timestamps && counts, "%s: null packed tensor", who);
  DA_REQUIRE(counts_dtype == DA_I32 || counts_dtype == DA_F32, "%s: counts must be int32 or fp32", who);
  DA_REQUIRE(P_bound > 0 && P_bound <= 4096 * kBlock, "%s: num_packed must be in [1, %d]", who, 4096 * kBlock);
  DA_REQUIRE(window >= 0 && window < (1ll << 30), "%s: window must be >= 0", who);
  DA_REQUIRE(aligned16(k_packed) && aligned16(v_packed), "%s: packed tensors must be 16-byte aligned", who);
  for (int i : {DA_STRIDE_KP + 2, DA_STRIDE_VP + 2})
    DA_REQUIRE(strides[i] >= a.D && strides[i] < (1ll << 23),
               "%s: packed sequence strides must be in [head_dim, 2^23) (stride %d = %lld)", who, i,
               (long long)strides[i]);
  DA_REQUIRE(strides[DA_STRIDE_TS + 2] == 1 && strides[DA_STRIDE_CNT + 2] == 1,
             "%s: timestamps and counts must be contiguous along the packed axis", who);
  const int64_t need = da_hybrid_workspace_size(B, Hkv, P_bound);
  if (!workspace || workspace_bytes < need)
    return set_error(DA_ERR_WORKSPACE, "%s: workspace of %lld bytes required", who, (long long)need);
  a.kp = (const uint16_t*)k_packed; a.vp = (const uint16_t*)v_packed;
  a.ts = timestamps; a.cnt = counts;
  a.skp_b = strides[DA_STRIDE_KP]; a.skp_h = strides[DA_STRIDE_KP + 1]; a.skp_n = strides[DA_STRIDE_KP + 2];
  a.svp_b = strides[DA_STRIDE_VP]; a.svp_h = strides[DA_STRIDE_VP + 1]; a.svp_n = strides[DA_STRIDE_VP + 2];
  a.sts_b = strides[DA_STRIDE_TS]; a.sts_h = strides[DA_STRIDE_TS + 1];
  a.scnt_b = strides[DA_STRIDE_CNT]; a.scnt_h = strides[DA_STRIDE_CNT + 1];
  a.P_host = (int)P_bound;
  a.P_dev = num_packed_dev;
  a.window = (int)window;
  a.no_count = no_count ? 1 : 0;
  a.cnt_is_float = counts_dtype == DA_F32;
  a.causal = 1;
  const HybridWs wl = hybrid_ws(B, Hkv, P_bound);
  char* ws = (char*)workspace;
  a.nblk_cap = wl.nblk;
  a.sched = (const int32_t*)ws;
  a.wcap = wl.wcap;
  a.wts = (const float*)(ws + wl.w_off);
  a.tsw = (const int32_t*)(ws + wl.ts_off);
  a.zeros = (const float*)(ws + wl.zeros_off);
  SchedPrep prep = {};
  if (variant != DA_VARIANT_SANITY) {
    prep.cnt = counts;
    prep.scnt_b = a.scnt_b;
    prep.scnt_h = a.scnt_h;
    prep.cnt_is_float = a.cnt_is_float;
    prep.no_count = a.no_count;
    prep.scale_log2 = a.scale_log2;
    prep.wts = (float*)(ws + wl.w_off);
    prep.tsw = variant == DA_VARIANT_PURE_PHASE1 ? (int32_t*)(ws + wl.ts_off) : nullptr;
    prep.zeros = (float*)(ws + wl.zeros_off);
    prep.wcap = wl.wcap;
  }
  const unsigned prep_chunks = prep.wts ? (unsigned)((wl.wcap + kSchedThreads - 1) / kSchedThreads) : 0u;
  // the grouped kernel's persistent grid takes its items from 8 counters in the workspace
  a.queue = a.hpw == 4 && dtype != DA_F32 ? (int*)(ws + wl.queue_off) : nullptr;
  hipLaunchKernelGGL(hybrid_schedule_kernel, dim3((unsigned)(B * Hkv), 1 + prep_chunks), dim3(kSchedThreads), 0, st,
                     timestamps, a.sts_b, a.sts_h, (int)Hkv, (int)P_bound, num_packed_dev, (int)Nk, a.seq,
                     a.nblk_cap, (int32_t*)ws, prep, a.queue);
  if (int rc = check_launch("hybrid prefill (schedule)")) return rc;
  const int kv = variant == DA_VARIANT_HYBRID ? kHybrid : (variant == DA_VARIANT_SANITY ? kSanity : kPure);
  return launch_attn(kv, dtype, a, st);
}

extern "C" int da_hybrid_prefill(const void* q, const void* k, const void* v, const void* k_packed,
                                 const void* v_packed, const int32_t* timestamps,
                                 const void* counts, int counts_dtype, void* out, int dtype,
                                 int64_t B, int64_t Hq, int64_t Hkv, int64_t Nq, int64_t Nk,
                                 int64_t D, const int64_t* strides, int64_t num_packed,
                                 const int32_t* num_packed_dev, int64_t window, float scale,
                                 int variant, int no_count, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  const char* who = "da_hybrid_prefill";
  if (dtype != DA_BF16 && dtype != DA_F16 && dtype != DA_F32)
    return set_error(DA_ERR_UNSUPPORTED, "%s: tensors must be bf16, fp16 or fp32", who);
  AttnArgs a = {};
  if (int rc = fill_common(a, q, k, v, out, B, Hq, Hkv, Nq, Nk, D, strides, scale, who)) return rc;
  a.seq = SeqMap{nullptr, 0, (int)Nq};
  return hybrid_impl(who, a, k_packed, v_packed, timestamps, counts, counts_dtype, dtype, B, Hkv, Nk, strides,
                     num_packed, num_packed_dev, window, variant, no_count, workspace, workspace_bytes,
                     (hipStream_t)stream);
}

extern "C" int da_dense_prefill(const void* q, const void* k, const void* v, void* out, int dtype,
                                int64_t B, int64_t Hq, int64_t Hkv, int64_t Nq, int64_t Nk,
                                int64_t D, const int64_t* strides, int causal, float scale,
                                void* stream) {
  if (dtype != DA_BF16 && dtype != DA_F16 && dtype != DA_F32)
    return set_error(DA_ERR_UNSUPPORTED, "da_dense_prefill: tensors must be bf16, fp16 or fp32");
  AttnArgs a = {};
  int rc = fill_common(a, q, k, v, out, B, Hq, Hkv, Nq, Nk, D, strides, scale, "da_dense_prefill");
  if (rc) return rc;
  a.seq = SeqMap{nullptr, 0, (int)Nq};
  a.kp = a.k; a.vp = a.v;
  a.causal = causal ? 1 : 0;
  a.P_host = 0;
  return launch_attn(kDense, dtype, a, (hipStream_t)stream);
}

// ---- ragged (varlen) batches: sequence b is tokens cu_seqlens[b] .. cu_seqlens[b+1]-1 of
// [T, H, D] tensors; every sequence is exactly a B = 1 prefill of its own length ----
static int varlen_common(const char* who, AttnArgs& a, const void* q, const void* k, const void* v, void* out,
                         int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D,
                         const int64_t* strides, const int32_t* cu_seqlens, int64_t max_seqlen, float scale) {
  if (dtype != DA_BF16 && dtype != DA_F16 && dtype != DA_F32)
    return set_error(DA_ERR_UNSUPPORTED, "%s: tensors must be bf16, fp16 or fp32", who);
  DA_REQUIRE(cu_seqlens, "%s: null cu_seqlens", who);
  DA_REQUIRE(T > 0 && max_seqlen > 0 && max_seqlen <= T, "%s: need 0 < max_seqlen <= total tokens", who);
  DA_REQUIRE(T < (1ll << 31), "%s: too many tokens", who);
  if (int rc = fill_common(a, q, k, v, out, B, Hq, Hkv, max_seqlen, max_seqlen, D, strides, scale, who)) return rc;
  a.seq = SeqMap{cu_seqlens, (int)T, (int)max_seqlen};
  return DA_OK;
}

extern "C" int64_t da_hybrid_varlen_workspace_size(int64_t B, int64_t Hkv, int64_t max_seqlen) {
  return da_hybrid_workspace_size(B, Hkv, max_seqlen);
}

extern "C" int da_hybrid_prefill_varlen(const void* q, const void* k, const void* v, const void* k_packed,
                                        const void* v_packed, const int32_t* timestamps, const void* counts,
                                        int counts_dtype, void* out, int dtype, int64_t B, int64_t Hq,
                                        int64_t Hkv, int64_t T, int64_t D, const int64_t* strides,
                                        const int32_t* cu_seqlens, int64_t max_seqlen,
                                        const int32_t* num_packed, int64_t window, float scale, int variant,
                                        int no_count, void* workspace, int64_t workspace_bytes, void* stream) {
  const char* who = "da_hybrid_prefill_varlen";
  AttnArgs a = {};
  if (int rc = varlen_common(who, a, q, k, v, out, dtype, B, Hq, Hkv, T, D, strides, cu_seqlens, max_seqlen, scale))
    return rc;
  DA_REQUIRE(num_packed, "%s: null num_packed", who);
  return hybrid_impl(who, a, k_packed, v_packed, timestamps, counts, counts_dtype, dtype, B, Hkv, max_seqlen,
                     strides, max_seqlen, num_packed, window, variant, no_count, workspace, workspace_bytes,
                     (hipStream_t)stream);
}

extern "C" int da_dense_prefill_varlen(const void* q, const void* k, const void* v, void* out, int dtype,
                                       int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D,
                                       const int64_t* strides, const int32_t* cu_seqlens, int64_t max_seqlen,
                                       int causal, float scale, void* stream) {
  AttnArgs a = {};
  if (int rc = varlen_common("da_dense_prefill_varlen", a, q, k, v, out, dtype, B, Hq, Hkv, T, D, strides,
                             cu_seqlens, max_seqlen, scale))
    return rc;
  a.kp = a.k; a.vp = a.v;
  a.causal = causal ? 1 : 0;
  a.P_host = 0;
  return launch_attn(kDense, dtype, a, (hipStream_t)stream);
}
