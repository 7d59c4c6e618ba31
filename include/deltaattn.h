/*
 * deltaattn.h -- C ABI of the MI355X (gfx950) DeltaAttention prefill path.
 *
 * Every entry point takes raw device pointers, int64 element strides for the
 * (batch, head, sequence) dimensions (the head dimension must be contiguous),
 * sizes, and a hipStream_t passed as void*.  Nothing allocates device memory:
 * scratch space comes in through a caller-provided workspace whose size the
 * matching *_workspace_size function returns.  Calls enqueue work on the given
 * stream and return without synchronising.  The library is reentrant; the only
 * per-thread state is the text of the last error, and the only device state is the
 * static scratch array of da_decode_attention_noalloc.
 *
 * Return value: DA_OK (0) or a negative DA_ERR_* code; da_last_error() then
 * holds a message.
 *
 * The reference (Emruur/DeltaAttention) is Python + Triton with no FFI; each
 * entry point names the reference kernel/launch it replaces.
 */
#ifndef DELTAATTN_H
#define DELTAATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DA_OK 0
#define DA_ERR_INVALID (-1)     /* bad argument (shape, stride, null pointer) */
#define DA_ERR_UNSUPPORTED (-2) /* valid but not implemented (dtype, head_dim) */
#define DA_ERR_HIP (-3)         /* HIP runtime error while launching */
#define DA_ERR_WORKSPACE (-4)   /* workspace missing or too small */

/* element types */
#define DA_BF16 1
#define DA_F16 2
#define DA_I32 3
#define DA_F32 4

/* attention variants (deltaFlashAttention.py kernels) */
#define DA_VARIANT_HYBRID 0      /* hybrid_compressed_flash_kernel, :9-146 */
#define DA_VARIANT_SANITY 1      /* hybrid_compressed_flash_kernel_sanity, :149-259 */
#define DA_VARIANT_PURE_PHASE1 2 /* pure_phase1_flash_kernel, :262-357 */

/* Text of the last error on the calling thread ("" when none). */
const char* da_last_error(void);

/* ABI version of this library. */
int da_version(void);

/*
 * Delta-mode anchor selection.  Replaces chunked_eval_kernel
 * (tritonModules.py:7-69) and its launch (modeling_llama.py:634-653).
 *
 * k: [B, Hkv, N, D] bf16, fp16 or fp32 (dtype DA_BF16 / DA_F16 / DA_F32), strides
 * (sk_b, sk_h, sk_n), D even and <= 128; fp32 rows 8-byte aligned.
 * threshold: tau^2 for Euclidean, tau for cosine (modeling_llama.py:641-642).
 * flags: DA_SELECT_COSINE selects the cosine test (keep iff cos < tau, else Euclidean
 *   keep iff dist^2 > tau^2); DA_SELECT_ARITH16 evaluates the Euclidean distance in the
 *   keys' 16-bit arithmetic (every difference, square and tree addition rounded to
 *   bf16 / fp16, as the reference's Triton code does on 16-bit keys,
 *   tritonModules.py:55-58); without it, and always for fp32 keys, the distance is fp32.
 * chunk_size / num_chunks: from the chunking rule of modeling_llama.py:602-610.
 * keep: [B, Hkv, N] int32 contiguous, 1 for anchors and 0 otherwise (rows of
 *   chunks that start at or beyond N are not written).
 * chunk_counts: [B, Hkv, num_chunks] int32 contiguous (0 for empty chunks).
 * The squared distance (or cosine) is reduced over a fixed pairwise tree, so the
 * result is deterministic and bit-identical to the CPU oracle.
 */
#define DA_SELECT_COSINE 1
#define DA_SELECT_ARITH16 2
int da_select(const void* k, int dtype, int64_t B, int64_t Hkv, int64_t N, int64_t D,
              int64_t sk_b, int64_t sk_h, int64_t sk_n, float threshold, int flags,
              int64_t chunk_size, int64_t num_chunks, int32_t* keep, int32_t* chunk_counts,
              void* stream);

/*
 * Index + pack + counts.  Replaces index_map / P (modeling_llama.py:655-656),
 * parallel_scatter_pack_kv_kernel (tritonModules.py:72-132, launch
 * modeling_llama.py:658-680) and the count scatter_add_ (:682-685), fused, with
 * P kept on the device (no host synchronisation).
 *
 * keep: [B, Hkv, N] int32 contiguous; keep[..., 0] must be 1 (every mode of the
 *   reference guarantees it, modeling_llama.py:623/630 and tritonModules.py:41).
 * k, v: [B, Hkv, N, D] bf16, fp16 or fp32 (dtype) with strides (s*_b, s*_h, s*_n); the
 *   packed rows are copies of theirs, in the same type.
 * capacity: rows allocated per head in the packed outputs; must be >= P
 *   (N always suffices).
 * k_packed, v_packed: [B, Hkv, capacity, D] contiguous; rows [0, c) receive the
 *   anchor rows, rows [c, P) are zero-filled (the reference's zero padding).
 * timestamps, counts: [B, Hkv, capacity] int32 contiguous: anchor position and run
 *   length; padding rows get 0.
 * anchor_counts: [B, Hkv] int32 (c per head); num_packed: [1] int32 (P).
 * workspace: da_pack_workspace_size() bytes of device memory.
 */
int64_t da_pack_workspace_size(int64_t B, int64_t Hkv, int64_t N);
int da_pack(const int32_t* keep, const void* k, const void* v, int dtype, int64_t B,
            int64_t Hkv, int64_t N, int64_t D, int64_t sk_b, int64_t sk_h, int64_t sk_n,
            int64_t sv_b, int64_t sv_h, int64_t sv_n, int64_t capacity, void* k_packed,
            void* v_packed, int32_t* timestamps, int32_t* counts, int32_t* anchor_counts,
            int32_t* num_packed, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Two-phase compressed flash prefill with GQA.  Replaces
 * hybrid_compressed_flash_kernel / _sanity / pure_phase1_flash_kernel
 * (deltaFlashAttention.py:9-357) and their wrappers (modeling_llama.py:306-451)
 * including the repeat_kv expansion (:701-708): query head h reads KV head
 * h / (Hq / Hkv) directly.
 *
 * q, out: [B, Hq, Nq, D]; k, v: [B, Hkv, Nk, D]; k_packed, v_packed: [B, Hkv, >=P, D], all
 * of one type (dtype DA_BF16, DA_F16 or DA_F32; P is rounded to it before P.V, as
 * deltaFlashAttention.py:98, 137 round p to V's type: fp32 tensors run an fp32 kernel
 * with p in fp32); timestamps: [B, Hkv, >=P] int32;
 * counts: [B, Hkv, >=P] int32 or fp32 (counts_dtype DA_I32 / DA_F32).
 * num_packed: P (rows of the packed tensors that are read); if num_packed_dev
 *   is non-null the device value is used instead (it must be <= num_packed).
 * window: dense window W >= 0 (modeling_llama.py:716); scale > 0 (:289).
 * no_count: every count, padding included, is 1 (modeling_llama.py:323-324).
 * Logical schedule: 128-row query blocks x 128-anchor packed blocks exactly as
 * the reference (Phase 1 stops at the first packed block whose maximum
 * timestamp is >= start_m - W; Phase 2 starts at ((last+1)/128)*128).
 * D: a multiple of 8 in [8, 128] (the kernels zero-fill dims D..127, as the reference's
 * BLOCK_D = next_pow2(D) masked loads do, deltaFlashAttention.py:39-42); Hq % Hkv == 0.
 * workspace: da_hybrid_workspace_size() bytes (the schedule, the key biases and the
 *   attention grid's work-queue counters, all written by the call on its stream): calls
 *   in stream order may share one workspace, concurrent calls may not.
 */
int64_t da_hybrid_workspace_size(int64_t B, int64_t Hkv, int64_t num_packed);
int da_hybrid_prefill(const void* q, const void* k, const void* v, const void* k_packed,
                      const void* v_packed, const int32_t* timestamps, const void* counts,
                      int counts_dtype, void* out, int dtype, int64_t B, int64_t Hq,
                      int64_t Hkv, int64_t Nq, int64_t Nk, int64_t D, const int64_t* strides,
                      int64_t num_packed, const int32_t* num_packed_dev, int64_t window,
                      float scale, int variant, int no_count, void* workspace,
                      int64_t workspace_bytes, void* stream);

/*
 * Dense flash prefill (the uncompressed control).  Replaces _attn_fwd_flat and
 * triton_flash_attention (flashAttention.py:5-130) with GQA handled by head
 * indexing instead of repeat_kv.
 * q, out: [B, Hq, Nq, D]; k, v: [B, Hkv, Nk, D]; causal: mask j > i.  D as for
 * da_hybrid_prefill (flashAttention.py:25-32 pads it the same way).
 */
int da_dense_prefill(const void* q, const void* k, const void* v, void* out, int dtype,
                     int64_t B, int64_t Hq, int64_t Hkv, int64_t Nq, int64_t Nk, int64_t D,
                     const int64_t* strides, int causal, float scale, void* stream);

/*
 * Ragged (varlen) batches.  The reference has no varlen API; its semantics for a batch of
 * sequences of different lengths is "each sequence is a B = 1 prefill" (modeling_llama.py:
 * 602-685 per sequence: own chunking, anchors, P and schedule), which these entry points
 * compute in one launch per stage over the whole batch.  Sequence b is tokens
 * cu_seqlens[b] .. cu_seqlens[b + 1] - 1 (cu_seqlens: device int32 [B + 1], non-decreasing
 * from 0 to T; lengths at most max_seqlen).  Offsets and lengths read from cu_seqlens are
 * clamped into [0, T] and to max_seqlen on the device.  Token-major tensors are [T, H, D]
 * with strides (token, head) and a contiguous head dimension.
 *
 * da_select_varlen: keys k [T, Hkv, D]; keep [Hkv, T] int32 contiguous (position
 * cu_seqlens[b] + i of row g for token i of sequence b); chunk_counts [B, Hkv, max_chunks]
 * int32 contiguous, 0 for chunks past a sequence's end.  Chunking per sequence: chunk_size
 * > 0 gives min(chunk_size, N_b) rows per chunk, else ceil(N_b / divide_to) (divide_to 0
 * meaning 1); max_chunks must be at least ceil(max_seqlen / chunk_size) (chunk_size > 0)
 * or max(1, divide_to).  threshold and flags as for da_select.
 */
int da_select_varlen(const void* k, int dtype, int64_t B, int64_t Hkv, int64_t T, int64_t D,
                     int64_t sk_t, int64_t sk_h, const int32_t* cu_seqlens, int64_t max_seqlen,
                     float threshold, int flags, int64_t chunk_size, int64_t divide_to,
                     int32_t* keep, int32_t* chunk_counts, int64_t max_chunks, void* stream);

/*
 * da_pack_varlen: keep [Hkv, T] (as da_select_varlen writes it, keep of token 0 of every
 * sequence must be 1); k, v [T, Hkv, D].  Outputs: k_packed, v_packed [T, Hkv, D]
 * contiguous, packed row j of (b, g) at token cu_seqlens[b] + j; timestamps, counts
 * [Hkv, T] int32 contiguous, likewise (timestamps are positions inside the sequence);
 * rows [c_bg, P_b) zero-filled.  anchor_counts [B, Hkv]; num_packed [B] int32 receives
 * P_b = max over the sequence's heads.  workspace: da_pack_varlen_workspace_size bytes.
 */
int64_t da_pack_varlen_workspace_size(int64_t B, int64_t Hkv, int64_t max_seqlen);
int da_pack_varlen(const int32_t* keep, const void* k, const void* v, int dtype, int64_t B,
                   int64_t Hkv, int64_t T, int64_t D, int64_t sk_t, int64_t sk_h, int64_t sv_t,
                   int64_t sv_h, const int32_t* cu_seqlens, int64_t max_seqlen, void* k_packed,
                   void* v_packed, int32_t* timestamps, int32_t* counts, int32_t* anchor_counts,
                   int32_t* num_packed, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * da_hybrid_prefill_varlen / da_dense_prefill_varlen: q, out [T, Hq, D]; k, v [T, Hkv, D];
 * k_packed, v_packed, timestamps, counts as da_pack_varlen writes them (any token and head
 * strides); num_packed: device [B] (P_b).  strides: the 24-entry array of
 * da_hybrid_prefill with the batch entries ignored and the sequence entries holding the
 * token strides.  Each sequence gets exactly the schedule and result of a B = 1
 * da_hybrid_prefill / da_dense_prefill of its own length.
 */
int64_t da_hybrid_varlen_workspace_size(int64_t B, int64_t Hkv, int64_t max_seqlen);
int da_hybrid_prefill_varlen(const void* q, const void* k, const void* v, const void* k_packed,
                             const void* v_packed, const int32_t* timestamps, const void* counts,
                             int counts_dtype, void* out, int dtype, int64_t B, int64_t Hq,
                             int64_t Hkv, int64_t T, int64_t D, const int64_t* strides,
                             const int32_t* cu_seqlens, int64_t max_seqlen,
                             const int32_t* num_packed, int64_t window, float scale, int variant,
                             int no_count, void* workspace, int64_t workspace_bytes, void* stream);
int da_dense_prefill_varlen(const void* q, const void* k, const void* v, void* out, int dtype,
                            int64_t B, int64_t Hq, int64_t Hkv, int64_t T, int64_t D,
                            const int64_t* strides, const int32_t* cu_seqlens, int64_t max_seqlen,
                            int causal, float scale, void* stream);

/*
 * Decode step of the compressed cache.  Replaces fused_hybrid_decode_update_kernel
 * (deltaDecoding.py:9-104) as launched by HybridCompressedCache.update (:181-211).
 *
 * new_k, new_v: [B, Hkv, 1, D] bf16, fp16 or fp32 like the cache (strides sn_b, sn_h;
 *   even strides, rows 4-byte aligned for 16-bit caches and 8-byte aligned for fp32).
 * k_exact, v_exact: ring [B, Hkv, W, D] (strides sx_*); k_packed, v_packed:
 *   [B, Hkv, capacity, D] (strides sp_*); counts, timestamps: [B, Hkv, capacity]
 *   int32 (strides sc_b, sc_h, packed axis contiguous); lengths: [B * Hkv] int32.
 * exact_seq_len, total_seq_len: the cache's host trackers before this token.
 * threshold: tau^2 (Euclidean, merge iff dist^2 <= tau^2) or tau (cosine, merge iff
 *   cos >= tau).  When the ring is full the evicted token merges into the last packed
 *   anchor or is appended (count 1, timestamp total - W); the new token then takes
 *   ring slot exact_seq_len % W.  The caller keeps capacity > length (the reference's
 *   host tracker, :185-187).
 */
int da_decode_update(const void* new_k, const void* new_v, int dtype, int64_t B, int64_t Hkv,
                     int64_t D, int64_t sn_b, int64_t sn_h, void* k_exact, void* v_exact,
                     int64_t sx_b, int64_t sx_h, int64_t sx_s, void* k_packed, void* v_packed,
                     int64_t sp_b, int64_t sp_h, int64_t sp_s, int32_t* counts,
                     int32_t* timestamps, int64_t sc_b, int64_t sc_h, int32_t* lengths,
                     int64_t capacity, int64_t exact_seq_len, int64_t total_seq_len,
                     int64_t window, float threshold, int use_cosine, void* stream);

/*
 * q_len = 1 attention over the compressed cache.  Replaces fused_hybrid_decode_kernel
 * (deltaDecoding.py:236-362) and its wrapper (modeling_llama.py:453-518).
 *
 * q: [B, Hq, D] bf16, fp16 or fp32 like the cache (strides sq_b, sq_h); query head h reads kv
 * head h / (Hq / Hkv).
 * Scores over the packed anchors [0, lengths[b*Hkv + g]) get + log(count); then the
 * ring slots [0, exact_len) (exact_len = min(exact_seq_len, W)).  out: [B, Hq, D]
 * (strides so_b, so_h).  D: a multiple of 8 up to 128 (the reference's BLOCK_D masking,
 * deltaDecoding.py:255-268); Hq / Hkv <= 64 (groups above 8 are scored in sub-groups).
 */
int64_t da_decode_workspace_size(int64_t B, int64_t Hq, int64_t capacity, int64_t window);
int da_decode_attention(const void* q, int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                        int64_t sq_b, int64_t sq_h, const void* k_packed, const void* v_packed,
                        int64_t sp_b, int64_t sp_h, int64_t sp_s, const int32_t* counts,
                        int64_t sc_b, int64_t sc_h, const int32_t* lengths, int64_t capacity,
                        const void* k_exact, const void* v_exact, int64_t sx_b, int64_t sx_h,
                        int64_t sx_s, int64_t window, int64_t exact_len, float scale, void* out,
                        int64_t so_b, int64_t so_h, void* workspace, int64_t workspace_bytes,
                        void* stream);

/*
 * One decode token in one call: da_decode_update, then da_decode_attention over the
 * updated cache (exact_len = min(exact_seq_len + 1, window)).  No counterpart in the
 * reference, which runs the two kernels from its cache object and attention wrapper
 * (deltaDecoding.py:181-233, modeling_llama.py:453-518): it is for callers whose host
 * path per token matters (token-by-token decode, one call per layer instead of two,
 * with every argument in one block the caller fills once per layer and updates per
 * token).  Fields mean what the same-named arguments of the two entries above mean;
 * the checks are theirs.
 *
 * Two launches instead of three: the attention scores the cache as it was plus the new
 * token in its ring slot and, when the ring was full, the evicted token as one more key
 * whose weight follows the update's decision (a merge gives the last anchor count + 1,
 * an append gives the evicted token count 1, a drop gives it 0); the launch that merges
 * the slices then writes the update into the cache.  The cache afterwards is
 * bit-identical to the two calls'.  The output is bit-identical for every KV head whose
 * token merged, was dropped or evicted nothing; where it appended, the new anchor is
 * scored at the end of the key list instead of after the packed anchors, so the output
 * equals the two calls' up to fp32 summation order.  New-token rows that are not 16-byte
 * aligned (sn_b, sn_h multiples of 8 elements, new_k / new_v 16-byte aligned) run the
 * update and attention kernels in sequence instead, bit-identical to the two calls; so do
 * fp32 caches.
 */
typedef struct DaDecodeStep {
  /* this token */
  const void* new_k;   /* [B, Hkv, 1, D] */
  const void* new_v;
  int64_t sn_b, sn_h;
  const void* q;       /* [B, Hq, D] */
  int64_t sq_b, sq_h;
  void* out;           /* [B, Hq, D] */
  int64_t so_b, so_h;
  /* one layer of the cache */
  void* k_exact;       /* [B, Hkv, W, D] */
  void* v_exact;
  int64_t sx_b, sx_h, sx_s;
  void* k_packed;      /* [B, Hkv, capacity, D] */
  void* v_packed;
  int64_t sp_b, sp_h, sp_s;
  int32_t* counts;     /* [B, Hkv, capacity] */
  int32_t* timestamps;
  int64_t sc_b, sc_h;
  int32_t* lengths;    /* [B * Hkv] */
  int64_t capacity;
  int64_t exact_seq_len, total_seq_len, window;  /* host trackers before this token */
  float threshold;
  int32_t use_cosine;
  float scale;
  int32_t dtype;
  int64_t B, Hq, Hkv, D;
  void* workspace;     /* da_decode_workspace_size(B, Hq, capacity, window) bytes */
  int64_t workspace_bytes;
} DaDecodeStep;
int da_decode_step(const DaDecodeStep* step, void* stream);

/*
 * da_decode_attention without a workspace and without any allocation.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc).  Arguments and
 * results are those of da_decode_attention minus the workspace; the slice partials
 * live in a static device array of DA_DECODE_SCRATCH_BYTES per GPU (held until the
 * process ends), so da_decode_workspace_size(B, Hq, capacity, window) must not exceed
 * DA_DECODE_SCRATCH_BYTES (DA_ERR_UNSUPPORTED otherwise; e.g. B = 1, Hq = 32 allows
 * capacity + window up to 129023 keys).  The stream must belong to the current device
 * (checked: DA_ERR_INVALID otherwise; the null stream is the current device's).
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (on
 * streams not ordered with each other) race.
 */
#define DA_DECODE_SCRATCH_BYTES (32ll << 20)
int da_decode_attention_noalloc(const void* q, int dtype, int64_t B, int64_t Hq, int64_t Hkv,
                                int64_t D, int64_t sq_b, int64_t sq_h, const void* k_packed,
                                const void* v_packed, int64_t sp_b, int64_t sp_h, int64_t sp_s,
                                const int32_t* counts, int64_t sc_b, int64_t sc_h,
                                const int32_t* lengths, int64_t capacity, const void* k_exact,
                                const void* v_exact, int64_t sx_b, int64_t sx_h, int64_t sx_s,
                                int64_t window, int64_t exact_len, float scale, void* out,
                                int64_t so_b, int64_t so_h, void* stream);

/*
 * strides for da_hybrid_prefill / da_dense_prefill: int64[3 * 8] element strides
 * (batch, head, sequence) of, in order: q, k, v, k_packed, v_packed, out,
 * timestamps (sequence stride must be 1), counts (sequence stride must be 1).
 * The sequence strides of k, v, k_packed and v_packed must lie in [D, 2^23): key and
 * value rows may not overlap.  da_dense_prefill reads the q, k, v and out triples only.
 */
#define DA_STRIDE_Q 0
#define DA_STRIDE_K 3
#define DA_STRIDE_V 6
#define DA_STRIDE_KP 9
#define DA_STRIDE_VP 12
#define DA_STRIDE_OUT 15
#define DA_STRIDE_TS 18
#define DA_STRIDE_CNT 21
#define DA_NUM_STRIDES 24

#ifdef __cplusplus
}
#endif

#endif /* DELTAATTN_H */
