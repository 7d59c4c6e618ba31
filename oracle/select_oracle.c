/*
 * CPU restatement of the delta-mode anchor selection -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this
 * library, as the checker or the timed CPU baseline; the product never links it.
 *
 * Restates chunked_eval_kernel (tritonModules.py:7-69) with the launch arithmetic of
 * modeling_llama.py:634-653.  The distance is fp32 arithmetic on the key values
 * reduced by a perfect pairwise tree over the head dimension zero-padded to 128
 * slots (t[j] = t[2j] + t[2j+1], level by level), the build's fixed reduction
 * order; oracle/delta_oracle.py restates the same definition in numpy and the HIP
 * kernel computes the same tree.  Build with -ffp-contract=off so that no
 * multiply-add is fused.
 *
 * With arith16 = 1 (bf16) or 2 (fp16) the Euclidean distance rounds every elementwise
 * difference, square and tree addition to the keys' 16-bit type, as the reference's
 * Triton code does when it evaluates curr - ref, diff * diff and tl.sum on 16-bit
 * tensors (tritonModules.py:55-58); only the reduction order stays the build's tree.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* round-to-nearest-even to bf16, returned as float (inf and NaN pass through) */
static float bf16r(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) return x;
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  memcpy(&x, &u, 4);
  return x;
}

/* round-to-nearest-even to IEEE binary16, returned as float */
static float f16r(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  const uint32_t sign = u & 0x80000000u;
  uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return x;                 /* inf, NaN */
  if (a >= 0x477ff000u) {                         /* >= 65520 rounds to infinity */
    u = sign | 0x7f800000u;
    memcpy(&x, &u, 4);
    return x;
  }
  if (a < 0x38800000u) {                          /* below 2^-14: quantum 2^-24 */
    const float q = nearbyintf(fabsf(x) * 16777216.0f) / 16777216.0f;
    return sign ? -q : q;
  }
  a = (a + 0xfffu + ((a >> 13) & 1u)) & ~0x1fffu; /* keep 10 mantissa bits */
  u = sign | a;
  memcpy(&x, &u, 4);
  return x;
}

static float round16(float x, int arith16) {
  return arith16 == 1 ? bf16r(x) : (arith16 == 2 ? f16r(x) : x);
}

static int tree_width(int d) {
  int w = 128;
  while (w < d) w *= 2;
  return w;
}

/* pairwise tree sum of t[0..w), destroys t; every addition rounded per arith16 */
static float tree_reduce(float* t, int w, int arith16) {
  while (w > 1) {
    for (int j = 0; j < w / 2; ++j) t[j] = round16(t[2 * j] + t[2 * j + 1], arith16);
    w /= 2;
  }
  return t[0];
}

static float sq_dist(const float* x, const float* a, int d, int w, float* t, int arith16) {
  for (int j = 0; j < w; ++j) {
    if (j < d) {
      float df = round16(x[j] - a[j], arith16);
      t[j] = round16(df * df, arith16);
    } else {
      t[j] = 0.0f;
    }
  }
  return tree_reduce(t, w, arith16);
}

static float dotp(const float* x, const float* a, int d, int w, float* t) {
  for (int j = 0; j < w; ++j) t[j] = (j < d) ? x[j] * a[j] : 0.0f;
  return tree_reduce(t, w, 0);
}

/*
 * k: float32 [B, H, N, D] contiguous.  thr: tau^2 (Euclidean) or tau (cosine) as fp32.
 * keep: int32 [B, H, N] (written for every row of every non-empty chunk; rows of
 * empty chunks are left untouched, as in the reference), counts: int32 [B, H, nc].
 * arith16: 0 fp32 distance, 1 / 2 Euclidean distance in bf16 / fp16 arithmetic (the
 * cosine test is always fp32: the reference upcasts it, tritonModules.py:48-54).
 * Returns 0, or -1 for an unsupported head_dim or arith16.
 */
int oracle_select_delta(const float* k, int64_t B, int64_t H, int64_t N, int64_t D,
                        float thr, int64_t cs, int64_t nc, int use_cos, int arith16,
                        int32_t* keep, int32_t* counts) {
  if (D <= 0 || D > 1024 || arith16 < 0 || arith16 > 2) return -1;
  int w = tree_width((int)D);
  float t[1024];
  const float eps = 1e-8f;
  for (int64_t bh = 0; bh < B * H; ++bh) {
    const float* kh = k + bh * N * D;
    int32_t* kp = keep + bh * N;
    for (int64_t c = 0; c < nc; ++c) {
      int64_t s = c * cs;
      if (s >= N) continue;                      /* tritonModules.py:34-35 */
      int64_t e = s + cs < N ? s + cs : N;       /* :32 */
      const float* a = kh + s * D;
      kp[s] = 1;                                 /* :41 */
      int32_t cnt = 1;
      float a_norm = 0.0f;
      if (use_cos) a_norm = sqrtf(dotp(a, a, (int)D, w, t) + eps);
      for (int64_t i = s + 1; i < e; ++i) {      /* :44 */
        const float* x = kh + i * D;
        int kp_i;
        if (use_cos) {                           /* :48-54 */
          float dot = dotp(x, a, (int)D, w, t);
          float nx = sqrtf(dotp(x, x, (int)D, w, t) + eps);
          float prod = nx * a_norm;
          float sim = dot / prod;
          kp_i = sim < thr;
        } else {                                 /* :55-58 */
          kp_i = sq_dist(x, a, (int)D, w, t, arith16) > thr;
        }
        if (kp_i) {                              /* :60-63 */
          kp[i] = 1;
          a = x;
          if (use_cos) a_norm = sqrtf(dotp(a, a, (int)D, w, t) + eps);
          ++cnt;
        } else {
          kp[i] = 0;                             /* :64-65 */
        }
      }
      counts[bh * nc + c] = cnt;                 /* :68-69 */
    }
  }
  return 0;
}
