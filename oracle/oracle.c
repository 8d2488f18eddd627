/*
 * CPU oracle for the paged-attention path of nano-vllm-java.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain C, the reference's fp32 algorithm so
 * that the HIP path can be checked against it.  Only the tests, the smoke check and the CPU
 * baseline leg of the benchmark load it; the product library never links or calls it.
 *
 * Reference files restated here (paths relative to
 * nano-vllm-java/src/main/java/com/igormaznitsa/nanollvm/):
 *   layers/Attention.java:131-137   pagedSlots            -> paged_slots()
 *   layers/Attention.java:152-171   forward dispatch      -> orc_attention_forward()
 *   layers/Attention.java:176-216   attendFromCache/gather -> shared-KV branch
 *   layers/Attention.java:221-240   storeKvCache          -> orc_store_kv()
 *   layers/Attention.java:245-299   prefillDense / prefillWithCache / decode
 *   layers/Attention.java:308-326   attendRange (job split, sequential below cost 256)
 *   layers/Attention.java:328-396   attendJobs (tile-64 online softmax)  -> attend_jobs()
 *   layers/Attention.java:401-410   kvHeadBase
 *   layers/Norms.java:183-204       RotaryEmbedding table and inv-freq -> orc_rope_*()
 *   layers/Norms.java:275-346       RotaryEmbedding.forward/rotateTokens/apply
 *   tensor/scalar/ScalarFloatKernels.java:27-42,164-182   dot/scale/axpy (kernels mode 0)
 *   tensor/vector/VectorFloatKernels.java:57-87,285-317   dot/scale/axpy (kernels mode LANE)
 *   tensor/MatmulRuntime.java:194-225                     parallelRanges (threads > 1)
 *   tensor/Ops.java:444-500         rmsNorm (weightless / weight / onePlusWeight) -> orc_rms_norm()
 *   tensor/Ops.java:84-124, tensor/MatmulRuntime.java:234-255,396-432   Ops.linear (sequential
 *                                   runtime) -> orc_linear()
 *   tensor/scalar/ScalarFloatKernels.java:82-140          gemv / gemvPanel8 (kernels mode 0)
 *   tensor/vector/VectorFloatKernels.java:158-250         gemv / gemvPanel8 (kernels mode LANE)
 *   tensor/scalar/ScalarFloatKernels.java:45-80           sumSquares/scaleAdd/scaleAddOnePlus
 *   tensor/vector/VectorFloatKernels.java:90-156          sumSquares/scaleAdd/scaleAddOnePlus
 *
 * Build with -ffp-contract=off: every float operation below is a separately rounded IEEE op,
 * as in Java, and an explicit fmaf() stands wherever Java calls FloatVector.fma.
 *
 * Parity pinning of each function is listed in the header of oracle.py.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_OK 0
#define ORC_E_ARG -1
#define ORC_E_ROPE_POS -2
#define ORC_E_SHARED_KV -3
#define ORC_E_NO_ARENA -4

#define KEY_TILE 64

/* Planted mistakes, used only by the tests that show the pinning checks catch them. */
#define MUT_NONE 0
#define MUT_DROP_SCALE 1     /* score = dot(q,k) without the scale */
#define MUT_KVH_MODULO 2     /* kvh = h % Hkv instead of h / rep */
#define MUT_CAUSAL_OFF1 3    /* causal end one key too far */
#define MUT_WINDOW_OFF1 4    /* sliding window one key too wide */
#define MUT_NO_RESCALE 5     /* acc not multiplied by alpha between tiles */
#define MUT_ROPE_SIGN 6      /* rotate-half with the sign of the sin term flipped */
#define MUT_NORM_NO_EPS 7    /* rmsNorm without eps under the root */
#define MUT_NORM_DIV_N1 8    /* mean of squares divided by n - 1 */
#define MUT_NORM_PAIRWISE 9  /* sumSquares summed as a pairwise tree, not in the scalar order */
#define MUT_NORM_NO_ONE 10   /* onePlusWeight ignored (w instead of 1 + w) */
#define MUT_LIN_TRANSPOSE 11 /* weight read as [in, out] instead of [out, in] */
#define MUT_LIN_NO_BIAS 12   /* bias dropped */

typedef struct {
  int num_heads;
  int head_dim;
  float scale;
  int num_kv_heads;
  int sliding_window;
  int write_kv;
} orc_attn;

typedef struct {
  int is_prefill;
  const int32_t *cu_q;         /* [num_seqs+1] prefill only */
  const int32_t *cu_k;         /* [num_seqs+1] prefill only */
  int num_seqs;                /* prefill: sequences; decode: rows */
  const int32_t *slot_mapping; /* may be NULL */
  int num_slots;
  const int32_t *context_lens; /* [num_seqs] decode only */
  const int32_t *block_tables; /* [num_seqs, bt_stride] or NULL */
  int bt_stride;
} orc_ctx;

/* ---------------------------------------------------------------- float kernels (a15) */

/* ScalarFloatKernels.dot: 4-wide unrolled non-fused sum, ScalarFloatKernels.java:27-42. */
static float dot_scalar(const float *a, const float *b, int n) {
  float sum = 0.0f;
  int i = 0;
  for (; i + 4 <= n; i += 4) {
    float t = a[i] * b[i];
    t = t + a[i + 1] * b[i + 1];
    t = t + a[i + 2] * b[i + 2];
    t = t + a[i + 3] * b[i + 3];
    sum = sum + t;
  }
  for (; i < n; i++) sum = sum + a[i] * b[i];
  return sum;
}

/* VectorFloatKernels.dot with LANE lanes: four FMA accumulators, (acc0+acc1)+(acc2+acc3),
 * lane reduction, scalar tail (VectorFloatKernels.java:57-87).  The Vector API leaves the
 * order of reduceLanes unspecified; a pairwise tree is used here. */
static inline float dot_vector(const float *a, const float *b, int n, int lane) {
  float acc[4][16];
  memset(acc, 0, sizeof(acc));
  int upper = n - n % lane;
  int span = lane * 4;
  int ubound = upper - upper % span;
  int i = 0;
  for (; i < ubound; i += span)
    for (int r = 0; r < 4; r++)
      for (int j = 0; j < lane; j++)
        acc[r][j] = fmaf(a[i + r * lane + j], b[i + r * lane + j], acc[r][j]);
  for (; i < upper; i += lane)
    for (int j = 0; j < lane; j++) acc[0][j] = fmaf(a[i + j], b[i + j], acc[0][j]);
  float red[16];
  for (int j = 0; j < lane; j++) red[j] = (acc[0][j] + acc[1][j]) + (acc[2][j] + acc[3][j]);
  for (int w = lane / 2; w >= 1; w /= 2)
    for (int j = 0; j < w; j++) red[j] = red[j] + red[j + w];
  float sum = red[0];
  for (; i < n; i++) sum = sum + a[i] * b[i];
  return sum;
}

/* The lane counts of AVX2 and AVX-512 hosts as constants, so the compiler can vectorize the
 * lane loops (the arithmetic and its order are those of dot_vector). */
static float dot(const float *a, const float *b, int n, int mode) {
  if (mode == 0) return dot_scalar(a, b, n);
  if (mode == 16) return dot_vector(a, b, n, 16);
  if (mode == 8) return dot_vector(a, b, n, 8);
  return dot_vector(a, b, n, mode);
}

/* axpy: dst += alpha*src.  Scalar: separate mul and add; vector: FMA body, scalar tail. */
static void axpy(float *dst, float alpha, const float *src, int n, int mode) {
  int i = 0;
  if (mode != 0) {
    int upper = n - n % mode;
    for (; i < upper; i++) dst[i] = fmaf(src[i], alpha, dst[i]);
  }
  for (; i < n; i++) dst[i] = dst[i] + alpha * src[i];
}

static void scale_vec(const float *src, float f, float *dst, int n) {
  for (int i = 0; i < n; i++) dst[i] = src[i] * f;
}

/* ---------------------------------------------------------------- RoPE (a3, a4) */

/* Math.round(float): floor(x + 1/2) evaluated exactly; NaN -> 0; saturates to int range. */
int orc_java_round_f32(float x) {
  if (isnan(x)) return 0;
  float f = floorf(x);
  float frac = x - f; /* exact: both operands share the binade */
  double r = (double)f + (frac >= 0.5f ? 1.0 : 0.0);
  if (r >= 2147483647.0) return 2147483647;
  if (r <= -2147483648.0) return (-2147483647 - 1);
  return (int)r;
}

/* RotaryEmbedding.defaultInvFreq, Norms.java:194-204. */
int orc_rope_inv_freq(int head_size, int rotary_dim, float base, float *inv_freq) {
  if (rotary_dim != head_size || head_size <= 0 || head_size % 2) return ORC_E_ARG;
  int half = rotary_dim / 2;
  for (int i = 0; i < half; i++)
    inv_freq[i] = (float)(1.0 / pow((double)base, (2.0 * i) / rotary_dim));
  return ORC_OK;
}

/* RotaryEmbedding(headSize, maxPos, invFreq), Norms.java:177-191.  pos*invFreq[i] is a float
 * product (int promoted to float) widened to double for cos/sin. */
void orc_rope_table(int head_size, int max_pos, const float *inv_freq, float *table) {
  int half = head_size / 2;
  for (int pos = 0; pos < max_pos; pos++)
    for (int i = 0; i < half; i++) {
      float prod = (float)pos * inv_freq[i];
      double freq = (double)prod;
      table[(size_t)pos * head_size + i] = (float)cos(freq);
      table[(size_t)pos * head_size + half + i] = (float)sin(freq);
    }
}

/* RotaryEmbedding.forward -> rotateTokens -> apply, Norms.java:275-346.  Returns
 * ORC_E_ROPE_POS (Java: IllegalArgumentException) for a rounded position outside
 * [0, max_pos) and leaves the outputs of earlier tokens written, as Java does. */
int orc_rope_forward(const float *table, int max_pos, int head_size, const float *positions,
                     const float *q, const float *k, float *q_out, float *k_out, int tokens,
                     int hq, int hk, int mutation) {
  int half = head_size / 2;
  for (int t = 0; t < tokens; t++) {
    int pos = orc_java_round_f32(positions[t]);
    if (pos < 0 || pos >= max_pos) return ORC_E_ROPE_POS;
    const float *cs = table + (size_t)pos * head_size;
    for (int pass = 0; pass < 2; pass++) {
      int heads = pass == 0 ? hq : hk;
      const float *in = pass == 0 ? q : k;
      float *out = pass == 0 ? q_out : k_out;
      for (int h = 0; h < heads; h++) {
        size_t base = ((size_t)t * heads + h) * head_size;
        for (int i = 0; i < half; i++) {
          float x1 = in[base + i], x2 = in[base + half + i];
          float c = cs[i], s = cs[half + i];
          float a = x1 * c, b = x2 * s;
          float e = x2 * c, f = x1 * s;
          out[base + i] = mutation == MUT_ROPE_SIGN ? a + b : a - b;
          out[base + half + i] = e + f;
        }
      }
    }
  }
  return ORC_OK;
}

/* ---------------------------------------------------------------- RMSNorm (q/k/v head norms) */

/* ScalarFloatKernels.sumSquares, ScalarFloatKernels.java:55-70: groups of four summed left to
 * right, ((v0*v0 + v1*v1) + v2*v2) + v3*v3, each group added to the running sum in order, then
 * the tail element by element. */
static float sum_squares_scalar(const float *a, int n) {
  float sum = 0.0f;
  int i = 0;
  for (; i + 4 <= n; i += 4) {
    float t = a[i] * a[i];
    t = t + a[i + 1] * a[i + 1];
    t = t + a[i + 2] * a[i + 2];
    t = t + a[i + 3] * a[i + 3];
    sum = sum + t;
  }
  for (; i < n; i++) sum = sum + a[i] * a[i];
  return sum;
}

/* VectorFloatKernels.sumSquares with LANE lanes, VectorFloatKernels.java:90-119: four FMA
 * accumulators over spans of 4*LANE, leftover whole vectors into acc0, (acc0+acc1)+(acc2+acc3),
 * reduceLanes (order unspecified by the JDK: a pairwise tree here), then the scalar tail. */
static float sum_squares_vector(const float *a, int n, int lane) {
  float acc[4][16];
  memset(acc, 0, sizeof(acc));
  int upper = n - n % lane;
  int span = lane * 4;
  int ubound = upper - upper % span;
  int i = 0;
  for (; i < ubound; i += span)
    for (int r = 0; r < 4; r++)
      for (int j = 0; j < lane; j++) {
        float v = a[i + r * lane + j];
        acc[r][j] = fmaf(v, v, acc[r][j]);
      }
  for (; i < upper; i += lane)
    for (int j = 0; j < lane; j++) acc[0][j] = fmaf(a[i + j], a[i + j], acc[0][j]);
  float red[16];
  for (int j = 0; j < lane; j++) red[j] = (acc[0][j] + acc[1][j]) + (acc[2][j] + acc[3][j]);
  for (int w = lane / 2; w >= 1; w /= 2)
    for (int j = 0; j < w; j++) red[j] = red[j] + red[j + w];
  float sum = red[0];
  for (; i < n; i++) sum = sum + a[i] * a[i];
  return sum;
}

/* Planted order mistake: squares summed as a pairwise tree. */
static float sum_squares_pairwise(const float *a, int n) {
  float buf[4096];
  int m = n < 4096 ? n : 4096;
  for (int i = 0; i < m; i++) buf[i] = a[i] * a[i];
  while (m > 1) {
    int h = (m + 1) / 2;
    for (int i = 0; i + h < m; i++) buf[i] = buf[i] + buf[i + h];
    m = h;
  }
  return n > 0 ? buf[0] : 0.0f;
}

/* VectorMath.sumSquares with the chosen backend (mode 0 scalar, else Vector API lanes). */
float orc_sum_squares(const float *a, int n, int mode, int mutation) {
  if (mutation == MUT_NORM_PAIRWISE) return sum_squares_pairwise(a, n);
  return mode == 0 ? sum_squares_scalar(a, n) : sum_squares_vector(a, n, mode);
}

/* Ops.rmsNorm(x, eps) and Ops.rmsNorm(x, weight, eps, onePlusWeight), Ops.java:444-500, over
 * rows of `width` floats: var = sumSquares / width (float division), inv =
 * (float)(1.0 / Math.sqrt(var + eps)) with var + eps a float sum widened to double, then
 * out = x * inv (weightless, VectorMath.scale), x * inv * w (scaleAdd) or x * inv * (1 + w)
 * (scaleAddOnePlus), each product separately rounded, left to right. */
void orc_rms_norm(const float *x, int rows, int width, const float *weight, float eps,
                  int one_plus, int mode, int mutation, float *out) {
  for (int r = 0; r < rows; r++) {
    const float *xr = x + (size_t)r * width;
    float *o = out + (size_t)r * width;
    float sum = orc_sum_squares(xr, width, mode, mutation);
    float var = sum / (float)(mutation == MUT_NORM_DIV_N1 ? width - 1 : width);
    float ve = mutation == MUT_NORM_NO_EPS ? var : var + eps;
    float inv = (float)(1.0 / sqrt((double)ve));
    for (int i = 0; i < width; i++) {
      float y = xr[i] * inv;
      if (weight) {
        float w = one_plus && mutation != MUT_NORM_NO_ONE ? 1.0f + weight[i] : weight[i];
        y = y * w;
      }
      o[i] = y;
    }
  }
}

/* ---------------------------------------------------------------- linear (o_proj) */

/* gemv over outputs [0, out) of one row: panels of 8 outputs, then the tail one by one
 * (ScalarFloatKernels.gemv / gemvPanel8, ScalarFloatKernels.java:82-140: a_j = bias,
 * a_j += x_i * w_ji in i order; tail: bias + dot; VectorFloatKernels.java:158-250: per-output
 * FMA lane accumulators, reduceLanes, scalar tail, then + bias; tail: bias + dot). */
static void gemv(const float *x, const float *w, const float *bias, float *y, int in, int out,
                 int mode, int mutation) {
  const float *b = mutation == MUT_LIN_NO_BIAS ? NULL : bias;
  float wt[64];
  int o = 0;
  for (; o + 8 <= out; o += 8) {
    if (mode == 0) {
      float a[8];
      for (int j = 0; j < 8; j++) a[j] = b ? b[o + j] : 0.0f;
      for (int i = 0; i < in; i++) {
        float xv = x[i];
        for (int j = 0; j < 8; j++) {
          float wv = mutation == MUT_LIN_TRANSPOSE ? w[(size_t)i * out + o + j]
                                                   : w[(size_t)(o + j) * in + i];
          a[j] = a[j] + xv * wv;
        }
      }
      for (int j = 0; j < 8; j++) y[o + j] = a[j];
    } else {
      int lane = mode, upper = in - in % lane;
      for (int j = 0; j < 8; j++) {
        const float *wr = w + (size_t)(o + j) * in;
        float acc[16];
        memset(acc, 0, sizeof(acc));
        int i = 0;
        for (; i < upper; i += lane)
          for (int l = 0; l < lane; l++) acc[l] = fmaf(x[i + l], wr[i + l], acc[l]);
        for (int l = 0; l < lane; l++) wt[l] = acc[l];
        for (int half = lane / 2; half >= 1; half /= 2)
          for (int l = 0; l < half; l++) wt[l] = wt[l] + wt[l + half];
        float s = wt[0];
        for (; i < in; i++) s = s + x[i] * wr[i];
        if (b) s = s + b[o + j];
        y[o + j] = s;
      }
    }
  }
  for (; o < out; o++) {
    float sum = b ? b[o] : 0.0f;
    const float *wr = w + (size_t)o * in;
    if (mutation == MUT_LIN_TRANSPOSE) {
      float d = 0.0f;
      for (int i = 0; i < in; i++) d = d + x[i] * w[(size_t)i * out + o];
      y[o] = sum + d;
    } else {
      y[o] = sum + dot(x, wr, in, mode);
    }
  }
}

/* Ops.linear(x, weight[out, in], bias) on the sequential runtime: y = x W^T + bias, one gemv per
 * row (MatmulRuntime.linear -> linearRange / linearDecode1 -> gemv over [0, out)). */
void orc_linear(const float *x, const float *w, const float *bias, float *y, int rows, int in,
                int out, int mode, int mutation) {
  for (int r = 0; r < rows; r++)
    gemv(x + (size_t)r * in, w, bias, y + (size_t)r * out, in, out, mode, mutation);
}

/* ---------------------------------------------------------------- store (a2) */

/* storeKvCache, Attention.java:221-240: negative slots are skipped. */
void orc_store_kv(const float *key, const float *value, const int32_t *slots, int n, int row,
                  float *k_cache, float *v_cache) {
  for (int i = 0; i < n; i++) {
    int slot = slots[i];
    if (slot < 0) continue;
    memcpy(k_cache + (size_t)slot * row, key + (size_t)i * row, sizeof(float) * row);
    memcpy(v_cache + (size_t)slot * row, value + (size_t)i * row, sizeof(float) * row);
  }
}

/* ---------------------------------------------------------------- attend (a8) */

typedef struct {
  const orc_attn *a;
  const float *q, *k, *v;
  float *out;
  int q_start, q_len, k_index_base, k_len, causal;
  const int32_t *slots; /* NULL: dense keys from k_index_base */
  int mode, mutation;
} job_args;

static size_t kv_head_base(const job_args *j, int kj, int kvh) {
  int64_t token = j->slots ? j->slots[kj] : (int64_t)j->k_index_base + kj;
  return (size_t)((token * j->a->num_kv_heads + kvh) * (int64_t)j->a->head_dim);
}

/* attendJobs, Attention.java:328-396. */
static void attend_jobs(const job_args *j, int job_start, int job_end) {
  const orc_attn *a = j->a;
  int d = a->head_dim;
  int rep = a->num_heads / a->num_kv_heads;
  float *acc = (float *)malloc(sizeof(float) * d);
  float tile[KEY_TILE];
  for (int job = job_start; job < job_end; job++) {
    int h = job / j->q_len;
    int qi = job % j->q_len;
    int q_pos = j->q_start + qi;
    int end = j->causal ? (j->k_len - j->q_len + qi + 1) : j->k_len;
    if (j->mutation == MUT_CAUSAL_OFF1 && j->causal && end < j->k_len) end += 1;
    int start = 0;
    if (a->sliding_window > 0) {
      int abs_q = j->causal ? (j->k_len - j->q_len + qi) : (j->k_len - 1);
      int w = a->sliding_window + (j->mutation == MUT_WINDOW_OFF1 ? 1 : 0);
      start = abs_q - w + 1;
      if (start < 0) start = 0;
    }
    int kvh = j->mutation == MUT_KVH_MODULO ? h % a->num_kv_heads : h / rep;
    const float *qrow = j->q + ((size_t)q_pos * a->num_heads + h) * d;
    float *orow = j->out + ((size_t)q_pos * a->num_heads + h) * d;
    memset(acc, 0, sizeof(float) * d);
    float m = -INFINITY;
    float l = 0.0f;
    for (int k0 = start; k0 < end; k0 += KEY_TILE) {
      int k1 = end < k0 + KEY_TILE ? end : k0 + KEY_TILE;
      float tmax = -INFINITY;
      for (int kj = k0; kj < k1; kj++) {
        float s = dot(qrow, j->k + kv_head_base(j, kj, kvh), d, j->mode);
        if (j->mutation != MUT_DROP_SCALE) s = s * a->scale;
        tile[kj - k0] = s;
        if (s > tmax) tmax = s;
      }
      float m_new = m > tmax ? m : tmax;
      float alpha = m == -INFINITY ? 0.0f : (float)exp((double)(m - m_new));
      float l_new = l * alpha;
      if (j->mutation != MUT_NO_RESCALE) scale_vec(acc, alpha, acc, d);
      for (int kj = k0; kj < k1; kj++) {
        float w = (float)exp((double)(tile[kj - k0] - m_new));
        l_new = l_new + w;
        axpy(acc, w, j->v + kv_head_base(j, kj, kvh), d, j->mode);
      }
      m = m_new;
      l = l_new;
    }
    float inv = l == 0.0f ? 0.0f : 1.0f / l;
    scale_vec(acc, inv, orow, d);
  }
  free(acc);
}

typedef struct {
  const job_args *j;
  int start, end;
} range_arg;

static void *range_thread(void *p) {
  range_arg *r = (range_arg *)p;
  attend_jobs(r->j, r->start, r->end);
  return NULL;
}

/* attendRange + MatmulRuntime.parallelRanges: head-major jobs split into ceil(work/workers)
 * contiguous ranges; sequential below cost 256 or with one thread. */
static void attend_range(const job_args *j, int threads) {
  int work = j->q_len * j->a->num_heads;
  int kl = j->k_len > 1 ? j->k_len : 1;
  long cost = (long)work * kl;
  if (cost < 256 || threads <= 1 || work <= 1) {
    attend_jobs(j, 0, work);
    return;
  }
  int workers = threads < work ? threads : work;
  int chunk = (work + workers - 1) / workers;
  pthread_t tid[256];
  range_arg args[256];
  int n = 0;
  for (int w = 0; w < workers && w < 256; w++) {
    int s = w * chunk;
    int e = s + chunk < work ? s + chunk : work;
    if (s >= e) break;
    args[n].j = j;
    args[n].start = s;
    args[n].end = e;
    pthread_create(&tid[n], NULL, range_thread, &args[n]);
    n++;
  }
  for (int i = 0; i < n; i++) pthread_join(tid[i], NULL);
}

static void paged_slots(const int32_t *table, int k_len, int block_size, int32_t *slots) {
  for (int t = 0; t < k_len; t++) slots[t] = table[t / block_size] * block_size + t % block_size;
}

/* Attention.forward, Attention.java:152-171, with the branches it dispatches to.
 * k_cache/v_cache: [num_blocks, block_size, Hkv, d] of this layer, or NULL for a layer whose
 * arena tensor is the numel-1 dummy.  has_arena == 0 reproduces the missing-arena NPE. */
int orc_attention_forward(const orc_attn *a, const orc_ctx *c, int has_arena, float *k_cache,
                          float *v_cache, int block_size, const float *q, const float *k,
                          const float *v, int num_tokens, float *out, int threads, int mode,
                          int mutation) {
  if (!has_arena) return ORC_E_NO_ARENA;
  if (a->num_kv_heads <= 0 || a->num_heads % a->num_kv_heads) return ORC_E_ARG;
  int d = a->head_dim;
  int row = a->num_kv_heads * d;
  int allocated = k_cache != NULL && v_cache != NULL;
  memset(out, 0, sizeof(float) * (size_t)num_tokens * a->num_heads * d);
  if (a->write_kv && allocated && c->slot_mapping != NULL && c->num_slots == num_tokens)
    orc_store_kv(k, v, c->slot_mapping, num_tokens, row, k_cache, v_cache);

  job_args j;
  memset(&j, 0, sizeof(j));
  j.a = a;
  j.q = q;
  j.out = out;
  j.mode = mode;
  j.mutation = mutation;

  float *gk = NULL, *gv = NULL;
  int prefill_cache = c->is_prefill && c->block_tables != NULL;
  int prefill_dense = c->is_prefill && c->block_tables == NULL;
  if (!a->write_kv && prefill_dense) {
    /* attendFromCache -> gatherKvCache, Attention.java:176-216. */
    if (c->slot_mapping == NULL || c->num_slots != num_tokens) return ORC_E_SHARED_KV;
    gk = (float *)calloc((size_t)num_tokens * row, sizeof(float));
    gv = (float *)calloc((size_t)num_tokens * row, sizeof(float));
    for (int i = 0; i < num_tokens; i++) {
      int slot = c->slot_mapping[i];
      if (slot < 0) continue;
      memcpy(gk + (size_t)i * row, k_cache + (size_t)slot * row, sizeof(float) * row);
      memcpy(gv + (size_t)i * row, v_cache + (size_t)slot * row, sizeof(float) * row);
    }
    k = gk;
    v = gv;
  }

  if (prefill_dense) {
    j.k = k;
    j.v = v;
    for (int b = 0; b < c->num_seqs; b++) {
      j.q_start = c->cu_q[b];
      j.q_len = c->cu_q[b + 1] - c->cu_q[b];
      j.k_index_base = c->cu_k[b];
      j.k_len = c->cu_k[b + 1] - c->cu_k[b];
      j.causal = 1;
      j.slots = NULL;
      attend_range(&j, threads);
    }
  } else {
    j.k = k_cache;
    j.v = v_cache;
    int rows = prefill_cache ? c->num_seqs : num_tokens; /* decode: bs = q.size(0) */
    for (int b = 0; b < rows; b++) {
      int k_len = prefill_cache ? c->cu_k[b + 1] - c->cu_k[b] : c->context_lens[b];
      int32_t *slots = (int32_t *)malloc(sizeof(int32_t) * (k_len > 0 ? k_len : 1));
      paged_slots(c->block_tables + (size_t)b * c->bt_stride, k_len, block_size, slots);
      j.q_start = prefill_cache ? c->cu_q[b] : b;
      j.q_len = prefill_cache ? c->cu_q[b + 1] - c->cu_q[b] : 1;
      j.k_index_base = 0;
      j.k_len = k_len;
      j.causal = prefill_cache;
      j.slots = slots;
      attend_range(&j, threads);
      free(slots);
    }
  }
  free(gk);
  free(gv);
  return ORC_OK;
}
