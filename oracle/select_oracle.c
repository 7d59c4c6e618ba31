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
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static int tree_width(int d) {
  int w = 128;
  while (w < d) w *= 2;
  return w;
}

/* pairwise tree sum of t[0..w), destroys t */
static float tree_reduce(float* t, int w) {
  while (w > 1) {
    for (int j = 0; j < w / 2; ++j) t[j] = t[2 * j] + t[2 * j + 1];
    w /= 2;
  }
  return t[0];
}

static float sq_dist(const float* x, const float* a, int d, int w, float* t) {
  for (int j = 0; j < w; ++j) {
    if (j < d) {
      float df = x[j] - a[j];
      t[j] = df * df;
    } else {
      t[j] = 0.0f;
    }
  }
  return tree_reduce(t, w);
}

static float dotp(const float* x, const float* a, int d, int w, float* t) {
  for (int j = 0; j < w; ++j) t[j] = (j < d) ? x[j] * a[j] : 0.0f;
  return tree_reduce(t, w);
}

/*
 * k: float32 [B, H, N, D] contiguous.  thr: tau^2 (Euclidean) or tau (cosine) as fp32.
 * keep: int32 [B, H, N] (written for every row of every non-empty chunk; rows of
 * empty chunks are left untouched, as in the reference), counts: int32 [B, H, nc].
 * Returns 0, or -1 for an unsupported head_dim.
 */
int oracle_select_delta(const float* k, int64_t B, int64_t H, int64_t N, int64_t D,
                        float thr, int64_t cs, int64_t nc, int use_cos,
                        int32_t* keep, int32_t* counts) {
  if (D <= 0 || D > 1024) return -1;
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
          kp_i = sq_dist(x, a, (int)D, w, t) > thr;
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
