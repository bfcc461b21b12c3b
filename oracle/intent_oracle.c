/*
 * intent_oracle.c — CPU restatement of the reference semantics of the hot-path operators.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker of the hip provider and
 * the CPU baseline that bench.py reports; the product (intent_amd) never loads it.
 *
 * Each function restates one reference definition (paths relative to
 * /root/reference/python/intent/examples/kernels/) under the numerics contract of
 * /root/reference/doc/dsl/types-numerics-and-effects.en.md:
 *   - reductions ("reduce") accumulate in f32 in the order of a vectorised reduction;
 *   - ordered loops (`for nz in range(...)`) are strict left folds, here without
 *     fused multiply-add (the file is built with -ffp-contract=off);
 *   - casts to f16/bf16 round to nearest even (section 5.2, :105-112);
 *   - approximate exp2/fdiv with flush_to_zero (section 5.1, :93-103) are computed
 *     accurately and then flushed at their boundaries, which is inside the contract.
 * CPU worker teams use the reference's static contiguous row-range split
 * (python/intent/runtime/mojo/task_dispatch.c:28-75) and run in IEEE mode with
 * FTZ/DAZ cleared (python/intent/runtime/mojo/fp_environment.c:3-8).
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <xmmintrin.h>

#define ORACLE_F32 0
#define ORACLE_F16 1
#define ORACLE_BF16 2

/* ------------------------------------------------------------------ IEEE environment */
static uint32_t enter_ieee(void) {
  uint32_t previous = _mm_getcsr();
  _mm_setcsr(previous & ~(UINT32_C(0x8040) | UINT32_C(0x6000)));
  return previous;
}
static void leave_ieee(uint32_t previous) { _mm_setcsr(previous); }

/* Rank `rank` of `size` gets rows [begin, end): the first count % size ranks get one extra. */
static void row_range(int64_t count, int rank, int size, int64_t *begin, int64_t *end) {
  int64_t chunk = count / size, extra = count % size;
  *begin = rank * chunk + (rank < extra ? rank : extra);
  *end = *begin + chunk + (rank < extra);
}

static int team_size(int workers, int64_t count) {
  if (workers < 1) workers = 1;
  if (count < workers) workers = count > 0 ? (int)count : 1;
  return workers;
}

/* ------------------------------------------------------------------ 16-bit formats */
static inline uint32_t f32_bits(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  return u;
}
static inline float bits_f32(uint32_t u) {
  float v;
  memcpy(&v, &u, 4);
  return v;
}

float oracle_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exponent = (h >> 10) & 0x1fu;
  uint32_t mantissa = h & 0x3ffu;
  if (exponent == 0x1fu) return bits_f32(sign | 0x7f800000u | (mantissa << 13));
  if (exponent == 0) {
    /* zero or subnormal: mantissa * 2^-24, exact in f32 */
    float magnitude = (float)mantissa * 5.9604644775390625e-8f;
    return sign ? -magnitude : magnitude;
  }
  return bits_f32(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

/* Round-to-nearest-even f32 -> f16; finite overflow gives infinity, NaN stays NaN. */
uint16_t oracle_float_to_half(float v) {
  uint32_t u = f32_bits(v);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t magnitude = u & 0x7fffffffu;
  if (magnitude > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((magnitude >> 13) & 0x1ffu));
  if (magnitude >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520: rounds to inf */
  if (magnitude < 0x38800000u) {
    /* result is subnormal or zero in f16: value / 2^-24 rounded to an integer, RNE */
    float scaled = bits_f32(magnitude) * 16777216.0f; /* exact: power-of-two scale */
    float rounded = nearbyintf(scaled);               /* default rounding mode: nearest even */
    return (uint16_t)(sign | (uint16_t)rounded);
  }
  uint32_t exponent = (magnitude >> 23) - 112u;
  uint32_t mantissa = magnitude & 0x7fffffu;
  uint32_t result = (exponent << 10) | (mantissa >> 13);
  uint32_t rest = mantissa & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (result & 1u))) result += 1u; /* carry may reach inf: correct */
  return (uint16_t)(sign | result);
}

float oracle_bf16_to_float(uint16_t h) { return bits_f32((uint32_t)h << 16); }

uint16_t oracle_float_to_bf16(float v) {
  uint32_t u = f32_bits(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

void oracle_halves_to_floats(const uint16_t *in, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_half_to_float(in[i]);
}
void oracle_floats_to_halves(const float *in, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_float_to_half(in[i]);
}
void oracle_floats_to_bf16(const float *in, uint16_t *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_float_to_bf16(in[i]);
}

static inline float load_elem(const void *base, int dtype, int64_t index) {
  switch (dtype) {
    case ORACLE_F16: return oracle_half_to_float(((const uint16_t *)base)[index]);
    case ORACLE_BF16: return oracle_bf16_to_float(((const uint16_t *)base)[index]);
    default: return ((const float *)base)[index];
  }
}
static inline void store_elem(void *base, int dtype, int64_t index, float v) {
  switch (dtype) {
    case ORACLE_F16: ((uint16_t *)base)[index] = oracle_float_to_half(v); break;
    case ORACLE_BF16: ((uint16_t *)base)[index] = oracle_float_to_bf16(v); break;
    default: ((float *)base)[index] = v;
  }
}

/* Sum in the order of a vectorised CPU reduction, which is how the reference CPU backend
 * evaluates `I.reduce.sum` (vector accumulators, then a horizontal reduce_add:
 * lib/Target/Mojo/Serialization/Serializer.cpp:558-592): four 16-lane f32 accumulators
 * (64 partial sums; accumulator j takes elements j, j+64, j+128, ... in order), added
 * pairwise at the end. A reduce may be re-associated
 * (doc/dsl/types-numerics-and-effects.en.md:154-160); a strictly sequential f32 sum would
 * drop every term below half an ulp of the running total. */
static float lane_sum(const float *v, int64_t n) {
  float lanes[64];
  for (int j = 0; j < 64; ++j) lanes[j] = 0.0f;
  for (int64_t i = 0; i < n; ++i) lanes[i & 63] += v[i];
  for (int width = 32; width >= 1; width >>= 1)
    for (int j = 0; j < width; ++j) lanes[j] += lanes[j + width];
  return lanes[0];
}

/* ------------------------------------------------------------------ softmax forward
 * normalization/softmax.py:12-66. max = maximum_num fold with identity -inf (fmaxf returns
 * the non-NaN operand); e = exp(x - max); s = sum(e).
 * f32 (stable_softmax, :23-36):        y = e * (1.0f / s)
 * f16/bf16 (stable_softmax_f16 :39-51, chunked_softmax_bf16 :54-66): y = cast(e / s). */
static void softmax_fwd_rows(int dtype, const void *x, void *y, int64_t cols, int64_t xs, int64_t ys,
                             int64_t begin, int64_t end, float *scratch) {
  for (int64_t r = begin; r < end; ++r) {
    float m = -INFINITY;
    for (int64_t c = 0; c < cols; ++c) m = fmaxf(m, load_elem(x, dtype, r * xs + c));
    for (int64_t c = 0; c < cols; ++c) scratch[c] = expf(load_elem(x, dtype, r * xs + c) - m);
    const float s = lane_sum(scratch, cols);
    if (dtype == ORACLE_F32) {
      const float inv = 1.0f / s;
      for (int64_t c = 0; c < cols; ++c) store_elem(y, dtype, r * ys + c, scratch[c] * inv);
    } else {
      for (int64_t c = 0; c < cols; ++c) store_elem(y, dtype, r * ys + c, scratch[c] / s);
    }
  }
}

int oracle_softmax_fwd(int dtype, const void *x, void *y, int64_t rows, int64_t cols, int64_t xs, int64_t ys,
                       int workers) {
  if (rows <= 0 || cols <= 0) return 0;
  const uint32_t csr = enter_ieee();
  const int size = team_size(workers, rows);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(rows, omp_get_thread_num(), size, &begin, &end);
    float *scratch = (float *)malloc(sizeof(float) * (size_t)cols);
    softmax_fwd_rows(dtype, x, y, cols, xs, ys, begin, end, scratch);
    free(scratch);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

/* ------------------------------------------------------------------ softmax backward
 * backward/softmax.py:9-25: proj = sum(p * dy); dx = p * (dy - proj). The f16 variant casts
 * p and dy to f32, reduces in f32 and casts dx to f16. */
int oracle_softmax_bwd(int dtype, const void *p, const void *dy, void *dx, int64_t rows, int64_t cols, int64_t ps,
                       int64_t dys, int64_t dxs, int workers) {
  if (rows <= 0 || cols <= 0) return 0;
  const uint32_t csr = enter_ieee();
  const int size = team_size(workers, rows);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(rows, omp_get_thread_num(), size, &begin, &end);
    float *scratch = (float *)malloc(sizeof(float) * (size_t)cols);
    for (int64_t r = begin; r < end; ++r) {
      for (int64_t c = 0; c < cols; ++c) scratch[c] = load_elem(p, dtype, r * ps + c) * load_elem(dy, dtype, r * dys + c);
      const float proj = lane_sum(scratch, cols);
      for (int64_t c = 0; c < cols; ++c) {
        const float pc = load_elem(p, dtype, r * ps + c);
        store_elem(dx, dtype, r * dxs + c, pc * (load_elem(dy, dtype, r * dys + c) - proj));
      }
    }
    free(scratch);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

/* ------------------------------------------------------------------ 16-bit GEMM
 * contraction/gemm.py:54-92: accumulator = matmul(a, b, acc_dtype=f32); for `gemm` (f16,
 * :54-73) with ACTIVATION == RELU, accumulator = maximum(accumulator, 0.0) (NaN propagates,
 * types-numerics-and-effects.en.md:117; maximum(-0, +0) = +0); c = cast(accumulator) to the
 * operand type, nearest even. bf16_gemm (:76-92) is dtype bf16 without activation.
 * Each c[i][j] is accumulated in f32 over k in increasing order (a row of accumulators per i,
 * so the inner loop over j vectorises without changing any element's order). */
static inline float relu_maximum(float v) { return v != v ? v : (v > 0.0f ? v : 0.0f); }

int oracle_gemm16(int dtype, int activation, const uint16_t *a, const uint16_t *b, uint16_t *c, int64_t m,
                  int64_t n, int64_t k, int64_t lda, int64_t ldb, int64_t ldc, int workers) {
  if (m <= 0 || n <= 0) return 0;
  if (dtype != 1 && dtype != 2) return 1;
  const uint32_t csr = enter_ieee();
  const int size = team_size(workers, m);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(m, omp_get_thread_num(), size, &begin, &end);
    float *acc = (float *)malloc(sizeof(float) * (size_t)n);
    float *brow = (float *)malloc(sizeof(float) * (size_t)n);
    for (int64_t i = begin; i < end; ++i) {
      for (int64_t j = 0; j < n; ++j) acc[j] = 0.0f;
      for (int64_t kk = 0; kk < k; ++kk) {
        const float av = load_elem(a, dtype, i * lda + kk);
        const uint16_t *src = b + kk * ldb;
        if (dtype == ORACLE_BF16)
          for (int64_t j = 0; j < n; ++j) brow[j] = bits_f32((uint32_t)src[j] << 16);
        else
          for (int64_t j = 0; j < n; ++j) brow[j] = oracle_half_to_float(src[j]);
        for (int64_t j = 0; j < n; ++j) acc[j] = acc[j] + av * brow[j];
      }
      for (int64_t j = 0; j < n; ++j) store_elem(c, dtype, i * ldc + j, activation ? relu_maximum(acc[j]) : acc[j]);
    }
    free(acc);
    free(brow);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

int oracle_gemm_bf16(const uint16_t *a, const uint16_t *b, uint16_t *c, int64_t m, int64_t n, int64_t k,
                     int64_t lda, int64_t ldb, int64_t ldc, int workers) {
  return oracle_gemm16(2, 0, a, b, c, m, n, k, lda, ldb, ldc, workers);
}

/* ------------------------------------------------------------------ f32 GEMM
 * contraction/gemm.py:15-38: gemm_f32, c = matmul(a, b, acc_dtype=f32); linear_f32,
 * output = matmul(x, weight, transpose_rhs=True, acc_dtype=f32) with weight [N,K]
 * (transpose_b = 1). f32 products and sums over k in increasing order, no fused multiply-add. */
int oracle_gemm_f32(const float *a, const float *b, float *c, int64_t m, int64_t n, int64_t k, int64_t lda,
                    int64_t ldb, int64_t ldc, int transpose_b, int workers) {
  if (m <= 0 || n <= 0) return 0;
  const uint32_t csr = enter_ieee();
  const int size = team_size(workers, m);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(m, omp_get_thread_num(), size, &begin, &end);
    float *acc = (float *)malloc(sizeof(float) * (size_t)n);
    float *brow = (float *)malloc(sizeof(float) * (size_t)n);
    for (int64_t i = begin; i < end; ++i) {
      if (transpose_b) {
        /* weight rows are k-contiguous: one dot product per output, k ascending */
        for (int64_t j = 0; j < n; ++j) {
          const float *w = b + j * ldb;
          float dot = 0.0f;
          for (int64_t kk = 0; kk < k; ++kk) dot = dot + a[i * lda + kk] * w[kk];
          c[i * ldc + j] = dot;
        }
        continue;
      }
      for (int64_t j = 0; j < n; ++j) acc[j] = 0.0f;
      for (int64_t kk = 0; kk < k; ++kk) {
        const float av = a[i * lda + kk];
        const float *src = b + kk * ldb;
        for (int64_t j = 0; j < n; ++j) acc[j] = acc[j] + av * src[j];
      }
      for (int64_t j = 0; j < n; ++j) c[i * ldc + j] = acc[j];
    }
    free(acc);
    free(brow);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

/* ------------------------------------------------------------------ attention forward
 * streaming/attention.py:428-553 as a region fold over key chunks of `chunk` keys:
 * summarize_attention_chunk_f16 (:152-191) / summarize_attention_chunk_bf16 (:193-237, with
 * active = True), merge_attention_summaries (:82-114), normalize_attention_summary (:417-425);
 * scores in the exp2 domain; exp2/fdiv are the approximate flush-to-zero operations (accurate
 * values, subnormals flushed). dtype 1 = f16 (flash_attention_fwd :428-466,
 * flash_gqa_attention_fwd :469-507), 2 = bf16 (flash_attention_bf16_fwd :510-553): the element
 * type of q, k, v, o and of the weights P before P @ V. Query head h reads key/value head
 * h / head_group (key_head = query_head // HEAD_GROUP). */
static inline float ftz(float v) { return fabsf(v) < 1.17549435e-38f ? copysignf(0.0f, v) : v; }
static inline float exp2_approx_ftz(float v) { return ftz(exp2f(ftz(v))); }
static inline float rcp_approx_ftz(float v) { return ftz(1.0f / ftz(v)); }

int oracle_attention_fwd(int dtype, const uint16_t *q, const uint16_t *k, const uint16_t *v, uint16_t *o,
                         int64_t batch, int64_t heads, int64_t head_group, int64_t sq, int64_t sk, int64_t d,
                         int64_t dv, const int64_t *strides, float scale, int causal, int64_t chunk, int workers) {
  if (batch <= 0 || heads <= 0 || sq <= 0) return 0;
  if ((dtype != 1 && dtype != 2) || head_group < 1 || heads % head_group) return 1;
  if (chunk <= 0) chunk = 64;
  const uint32_t csr = enter_ieee();
  const float log2e = 1.4426950408889634f;
  const float factor = scale * log2e;
  const int64_t count = batch * heads * sq;
  const int size = team_size(workers, count);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(count, omp_get_thread_num(), size, &begin, &end);
    float *scores = (float *)malloc(sizeof(float) * (size_t)chunk);
    float *qrow = (float *)malloc(sizeof(float) * (size_t)d);
    float *acc = (float *)malloc(sizeof(float) * (size_t)dv);
    float *cacc = (float *)malloc(sizeof(float) * (size_t)dv);
    for (int64_t item = begin; item < end; ++item) {
      const int64_t bi = item / (heads * sq), hi = (item / sq) % heads, qi = item % sq;
      const uint16_t *qp = q + bi * strides[0] + hi * strides[1] + qi * strides[2];
      const int64_t kh = hi / head_group;
      for (int64_t t = 0; t < d; ++t) qrow[t] = load_elem(qp, dtype, t * strides[3]);
      int valid = 0;
      float maximum = 0.0f, denominator = 0.0f;
      for (int64_t t = 0; t < dv; ++t) acc[t] = 0.0f;
      for (int64_t k0 = 0; k0 < sk; k0 += chunk) {
        const int64_t k1 = k0 + chunk < sk ? k0 + chunk : sk;
        /* summarize this chunk */
        int cvalid = 0;
        float cmax = -INFINITY;
        for (int64_t j = k0; j < k1; ++j) {
          const uint16_t *kp = k + bi * strides[4] + kh * strides[5] + j * strides[6];
          float dot = 0.0f;
          for (int64_t t = 0; t < d; ++t) dot = dot + qrow[t] * load_elem(kp, dtype, t * strides[7]);
          const int ok = !causal || qi >= j;
          scores[j - k0] = ok ? dot * factor : -INFINITY;
          if (ok) {
            cvalid = 1;
            cmax = fmaxf(cmax, scores[j - k0]);
          }
        }
        if (!cvalid) cmax = 0.0f;
        float cden = 0.0f;
        for (int64_t t = 0; t < dv; ++t) cacc[t] = 0.0f;
        for (int64_t j = k0; j < k1; ++j) {
          const int ok = !causal || qi >= j;
          const float weight = ok ? exp2_approx_ftz(scores[j - k0] - cmax) : 0.0f;
          cden += weight;
          const float w16 = dtype == 2 ? oracle_bf16_to_float(oracle_float_to_bf16(weight))
                                       : oracle_half_to_float(oracle_float_to_half(weight));
          const uint16_t *vp = v + bi * strides[8] + kh * strides[9] + j * strides[10];
          for (int64_t t = 0; t < dv; ++t) cacc[t] = cacc[t] + w16 * load_elem(vp, dtype, t * strides[11]);
        }
        if (!cvalid)
          for (int64_t t = 0; t < dv; ++t) cacc[t] = 0.0f;
        /* merge (running, chunk) */
        float merged = valid ? maximum : cmax;
        if (cvalid) merged = fmaxf(merged, cmax);
        const float left = valid ? exp2_approx_ftz((valid ? maximum : merged) - merged) : 0.0f;
        const float right = cvalid ? exp2_approx_ftz((cvalid ? cmax : merged) - merged) : 0.0f;
        denominator = left * denominator + right * cden;
        for (int64_t t = 0; t < dv; ++t) acc[t] = left * acc[t] + right * cacc[t];
        maximum = merged;
        valid = valid || cvalid;
      }
      uint16_t *op = o + bi * strides[12] + hi * strides[13] + qi * strides[14];
      const float reciprocal = rcp_approx_ftz(valid ? denominator : 1.0f);
      for (int64_t t = 0; t < dv; ++t) store_elem(op, dtype, t * strides[15], valid ? acc[t] * reciprocal : 0.0f);
    }
    free(scores);
    free(qrow);
    free(acc);
    free(cacc);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

/* flash_attention_bias_fwd (streaming/attention.py:800-836) with summarize_biased_attention_chunk
 * (:327-365): f16 q, k, v, o; bias [B,H,K] f32 (bias_strides: batch, head, key). Every key is
 * valid; a chunk's scores are (dot * scale + bias[j]) * log2(e) and its maximum is the NaN-ignoring
 * maximum, so a chunk whose scores are all -inf gives NaN weights, as the reference's does. */
int oracle_attention_bias_fwd(const uint16_t *q, const uint16_t *k, const uint16_t *v, const float *bias, uint16_t *o,
                              int64_t batch, int64_t heads, int64_t sq, int64_t sk, int64_t d, int64_t dv,
                              const int64_t *strides, const int64_t *bias_strides, float scale, int64_t chunk,
                              int workers) {
  if (batch <= 0 || heads <= 0 || sq <= 0) return 0;
  if (chunk <= 0) chunk = 64;
  const uint32_t csr = enter_ieee();
  const float log2e = 1.4426950408889634f;
  const int64_t count = batch * heads * sq;
  const int size = team_size(workers, count);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(count, omp_get_thread_num(), size, &begin, &end);
    float *scores = (float *)malloc(sizeof(float) * (size_t)chunk);
    float *qrow = (float *)malloc(sizeof(float) * (size_t)d);
    float *acc = (float *)malloc(sizeof(float) * (size_t)dv);
    float *cacc = (float *)malloc(sizeof(float) * (size_t)dv);
    for (int64_t item = begin; item < end; ++item) {
      const int64_t bi = item / (heads * sq), hi = (item / sq) % heads, qi = item % sq;
      const uint16_t *qp = q + bi * strides[0] + hi * strides[1] + qi * strides[2];
      const float *bp = bias + bi * bias_strides[0] + hi * bias_strides[1];
      for (int64_t t = 0; t < d; ++t) qrow[t] = load_elem(qp, 1, t * strides[3]);
      int valid = 0;
      float maximum = 0.0f, denominator = 0.0f;
      for (int64_t t = 0; t < dv; ++t) acc[t] = 0.0f;
      for (int64_t k0 = 0; k0 < sk; k0 += chunk) {
        const int64_t k1 = k0 + chunk < sk ? k0 + chunk : sk;
        float cmax = -INFINITY;
        for (int64_t j = k0; j < k1; ++j) {
          const uint16_t *kp = k + bi * strides[4] + hi * strides[5] + j * strides[6];
          float dot = 0.0f;
          for (int64_t t = 0; t < d; ++t) dot = dot + qrow[t] * load_elem(kp, 1, t * strides[7]);
          scores[j - k0] = (dot * scale + bp[j * bias_strides[2]]) * log2e;
          cmax = fmaxf(cmax, scores[j - k0]);   /* maximum_num: a NaN score is ignored */
        }
        float cden = 0.0f;
        for (int64_t t = 0; t < dv; ++t) cacc[t] = 0.0f;
        for (int64_t j = k0; j < k1; ++j) {
          const float weight = exp2_approx_ftz(scores[j - k0] - cmax);
          cden += weight;
          const float w16 = oracle_half_to_float(oracle_float_to_half(weight));
          const uint16_t *vp = v + bi * strides[8] + hi * strides[9] + j * strides[10];
          for (int64_t t = 0; t < dv; ++t) cacc[t] = cacc[t] + w16 * load_elem(vp, 1, t * strides[11]);
        }
        /* merge (running, chunk); every chunk is valid */
        const float merged = valid ? fmaxf(maximum, cmax) : cmax;
        const float left = valid ? exp2_approx_ftz(maximum - merged) : 0.0f;
        const float right = exp2_approx_ftz(cmax - merged);
        denominator = left * denominator + right * cden;
        for (int64_t t = 0; t < dv; ++t) acc[t] = left * acc[t] + right * cacc[t];
        maximum = merged;
        valid = 1;
      }
      uint16_t *op = o + bi * strides[12] + hi * strides[13] + qi * strides[14];
      const float reciprocal = rcp_approx_ftz(valid ? denominator : 1.0f);
      for (int64_t t = 0; t < dv; ++t) store_elem(op, 1, t * strides[15], valid ? acc[t] * reciprocal : 0.0f);
    }
    free(scores);
    free(qrow);
    free(acc);
    free(cacc);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

/* mla_prefill (streaming/attention.py:756-798) with summarize_mla_chunk (:368-415): f16 q [B,H,Q,D],
 * qpe [B,H,Q,P], k [B,HK,K,D], kpe [B,1,K,P], v [B,HK,K,D] (contiguous); output [B,H,Q,D]. Scores
 * are (q . k + qpe . kpe) * scale * log2e, each product summed in f32 on its own and then added;
 * key j is valid for query i iff i >= j; the chunk fold is the attention forward's. */
int oracle_mla_prefill(const uint16_t *q, const uint16_t *qpe, const uint16_t *k, const uint16_t *kpe,
                       const uint16_t *v, uint16_t *o, int64_t batch, int64_t heads, int64_t kv_heads, int64_t sq,
                       int64_t sk, int64_t d, int64_t p, float scale, int64_t chunk, int workers) {
  if (batch <= 0 || heads <= 0 || sq <= 0) return 0;
  if (kv_heads < 1 || heads % kv_heads) return 1;
  if (chunk <= 0) chunk = 64;
  const uint32_t csr = enter_ieee();
  const float factor = scale * 1.4426950408889634f;
  const int64_t group = heads / kv_heads, count = batch * heads * sq;
  const int size = team_size(workers, count);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(count, omp_get_thread_num(), size, &begin, &end);
    float *scores = (float *)malloc(sizeof(float) * (size_t)chunk);
    float *qrow = (float *)malloc(sizeof(float) * (size_t)(d + p));
    float *acc = (float *)malloc(sizeof(float) * (size_t)d), *cacc = (float *)malloc(sizeof(float) * (size_t)d);
    for (int64_t item = begin; item < end; ++item) {
      const int64_t b = item / (heads * sq), h = (item / sq) % heads, qi = item % sq, kh = h / group;
      for (int64_t t = 0; t < d; ++t) qrow[t] = oracle_half_to_float(q[((b * heads + h) * sq + qi) * d + t]);
      for (int64_t t = 0; t < p; ++t) qrow[d + t] = oracle_half_to_float(qpe[((b * heads + h) * sq + qi) * p + t]);
      int valid = 0;
      float maximum = 0.0f, denominator = 0.0f;
      for (int64_t t = 0; t < d; ++t) acc[t] = 0.0f;
      for (int64_t k0 = 0; k0 < sk; k0 += chunk) {
        const int64_t k1 = k0 + chunk < sk ? k0 + chunk : sk;
        int cvalid = 0;
        float cmax = -INFINITY;
        for (int64_t j = k0; j < k1; ++j) {
          const uint16_t *kp = k + ((b * kv_heads + kh) * sk + j) * d, *pp = kpe + (b * sk + j) * p;
          float content = 0.0f, position = 0.0f;
          for (int64_t t = 0; t < d; ++t) content = content + qrow[t] * oracle_half_to_float(kp[t]);
          for (int64_t t = 0; t < p; ++t) position = position + qrow[d + t] * oracle_half_to_float(pp[t]);
          const int ok = qi >= j;
          scores[j - k0] = ok ? (content + position) * factor : -INFINITY;
          if (ok) {
            cvalid = 1;
            cmax = fmaxf(cmax, scores[j - k0]);
          }
        }
        if (!cvalid) cmax = 0.0f;
        float cden = 0.0f;
        for (int64_t t = 0; t < d; ++t) cacc[t] = 0.0f;
        for (int64_t j = k0; j < k1; ++j) {
          const float weight = qi >= j ? exp2_approx_ftz(scores[j - k0] - cmax) : 0.0f;
          cden += weight;
          const float w16 = oracle_half_to_float(oracle_float_to_half(weight));
          const uint16_t *vp = v + ((b * kv_heads + kh) * sk + j) * d;
          for (int64_t t = 0; t < d; ++t) cacc[t] = cacc[t] + w16 * oracle_half_to_float(vp[t]);
        }
        if (!cvalid)
          for (int64_t t = 0; t < d; ++t) cacc[t] = 0.0f;
        float merged = valid ? maximum : cmax;
        if (cvalid) merged = fmaxf(merged, cmax);
        const float left = valid ? exp2_approx_ftz(maximum - merged) : 0.0f;
        const float right = cvalid ? exp2_approx_ftz(cmax - merged) : 0.0f;
        denominator = left * denominator + right * cden;
        for (int64_t t = 0; t < d; ++t) acc[t] = left * acc[t] + right * cacc[t];
        maximum = merged;
        valid = valid || cvalid;
      }
      uint16_t *op = o + ((b * heads + h) * sq + qi) * d;
      const float reciprocal = rcp_approx_ftz(valid ? denominator : 1.0f);
      for (int64_t t = 0; t < d; ++t) op[t] = oracle_float_to_half(valid ? acc[t] * reciprocal : 0.0f);
    }
    free(scores);
    free(qrow);
    free(acc);
    free(cacc);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

int oracle_attention_fwd_f16(const uint16_t *q, const uint16_t *k, const uint16_t *v, uint16_t *o, int64_t batch,
                             int64_t heads, int64_t sq, int64_t sk, int64_t d, int64_t dv, const int64_t *strides,
                             float scale, int causal, int64_t chunk, int workers) {
  return oracle_attention_fwd(1, q, k, v, o, batch, heads, 1, sq, sk, d, dv, strides, scale, causal, chunk, workers);
}

/* ------------------------------------------------------------------ attention backward
 * backward/attention.py (f16 storage, f32 arithmetic):
 *   attention_backward_delta (:17-34): delta[b,h,q] = sum_d f32(o) * f32(do) (a reduce);
 *   attention_backward_dq (:171-211) with summarize_query_gradients (:140-163): per query,
 *     p = exp2_approx_ftz(s * (scale * log2e) - lse * log2e), s = q . k (f32); causal validity
 *     q >= k; dp = do . v; ds = p * (dp - delta); dq = sum over valid keys of f16(ds) * k;
 *     grad_q = f16(dq * scale);
 *   attention_backward_dkdv (:87-137) with summarize_key_value_gradients (:47-79): per key of
 *     key head hk, over the HEAD_GROUP query heads hk * G + g and their queries in order:
 *     dv = sum f16(p) * do, dk = sum f16(ds) * q over valid pairs; grad_k = f16(dk * scale),
 *     grad_v = f16(dv).
 * Excluded (causally invalid) pairs contribute nothing (masked_gradient_product, :37-44). The
 * key axis of dq and the query axis of dk/dv are region folds whose chunks are combined by
 * addition (:82-84, :166-168); each chunk of `chunk` positions is summed, then added. lse is
 * the natural logarithm of the forward's softmax denominator (programs/attention_backward.py:25).
 * Strides are in elements: delta: o[4], do[4], delta[3]; dq: q, k, v, do (4 each), lse[3],
 * delta[3], dq[4]; dkdv: the same inputs, then dk[4], dv[4]. */
int oracle_attention_bwd_delta(const uint16_t *o, const uint16_t *dout, float *delta, int64_t batch, int64_t heads,
                               int64_t sq, int64_t d, const int64_t *st, int workers) {
  if (batch <= 0 || heads <= 0 || sq <= 0) return 0;
  const uint32_t csr = enter_ieee();
  const int64_t count = batch * heads * sq;
  const int size = team_size(workers, count);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(count, omp_get_thread_num(), size, &begin, &end);
    float *prod = (float *)malloc(sizeof(float) * (size_t)(d > 0 ? d : 1));
    for (int64_t item = begin; item < end; ++item) {
      const int64_t bi = item / (heads * sq), hi = (item / sq) % heads, qi = item % sq;
      const uint16_t *op = o + bi * st[0] + hi * st[1] + qi * st[2];
      const uint16_t *gp = dout + bi * st[4] + hi * st[5] + qi * st[6];
      for (int64_t t = 0; t < d; ++t) prod[t] = oracle_half_to_float(op[t * st[3]]) * oracle_half_to_float(gp[t * st[7]]);
      delta[bi * st[8] + hi * st[9] + qi * st[10]] = lane_sum(prod, d);
    }
    free(prod);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

static float dot_f16(const uint16_t *a, int64_t as, const uint16_t *b, int64_t bs, int64_t d) {
  float acc = 0.0f;
  for (int64_t t = 0; t < d; ++t) acc = acc + oracle_half_to_float(a[t * as]) * oracle_half_to_float(b[t * bs]);
  return acc;
}

int oracle_attention_bwd_dq(const uint16_t *q, const uint16_t *k, const uint16_t *v, const uint16_t *dout,
                            const float *lse, const float *delta, uint16_t *dq, int64_t batch, int64_t heads,
                            int64_t head_group, int64_t sq, int64_t sk, int64_t d, const int64_t *st, float scale,
                            int causal, int64_t chunk, int workers) {
  if (batch <= 0 || heads <= 0 || sq <= 0) return 0;
  if (head_group < 1 || heads % head_group) return 1;
  if (chunk <= 0) chunk = 64;
  const uint32_t csr = enter_ieee();
  const float log2e = 1.4426950408889634f;
  const float factor = scale * log2e;
  const int64_t count = batch * heads * sq;
  const int size = team_size(workers, count);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(count, omp_get_thread_num(), size, &begin, &end);
    float *acc = (float *)malloc(sizeof(float) * (size_t)d);
    float *part = (float *)malloc(sizeof(float) * (size_t)d);
    for (int64_t item = begin; item < end; ++item) {
      const int64_t bi = item / (heads * sq), hi = (item / sq) % heads, qi = item % sq, kh = hi / head_group;
      const uint16_t *qp = q + bi * st[0] + hi * st[1] + qi * st[2];
      const uint16_t *gp = dout + bi * st[12] + hi * st[13] + qi * st[14];
      const float l = lse[bi * st[16] + hi * st[17] + qi * st[18]];
      const float dl = delta[bi * st[19] + hi * st[20] + qi * st[21]];
      for (int64_t t = 0; t < d; ++t) acc[t] = 0.0f;
      for (int64_t k0 = 0; k0 < sk; k0 += chunk) {
        const int64_t k1 = k0 + chunk < sk ? k0 + chunk : sk;
        for (int64_t t = 0; t < d; ++t) part[t] = 0.0f;
        for (int64_t j = k0; j < k1; ++j) {
          if (causal && qi < j) continue;                        /* excluded pair */
          const uint16_t *kp = k + bi * st[4] + kh * st[5] + j * st[6];
          const uint16_t *vp = v + bi * st[8] + kh * st[9] + j * st[10];
          const float s = dot_f16(qp, st[3], kp, st[7], d);
          const float p = exp2_approx_ftz(s * factor - l * log2e);
          const float dp = dot_f16(gp, st[15], vp, st[11], d);
          const float ds16 = oracle_half_to_float(oracle_float_to_half(p * (dp - dl)));
          for (int64_t t = 0; t < d; ++t) part[t] = part[t] + ds16 * oracle_half_to_float(kp[t * st[7]]);
        }
        for (int64_t t = 0; t < d; ++t) acc[t] = acc[t] + part[t];
      }
      uint16_t *out = dq + bi * st[22] + hi * st[23] + qi * st[24];
      for (int64_t t = 0; t < d; ++t) out[t * st[25]] = oracle_float_to_half(acc[t] * scale);
    }
    free(acc);
    free(part);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

int oracle_attention_bwd_dkdv(const uint16_t *q, const uint16_t *k, const uint16_t *v, const uint16_t *dout,
                              const float *lse, const float *delta, uint16_t *dk, uint16_t *dv, int64_t batch,
                              int64_t heads, int64_t head_group, int64_t sq, int64_t sk, int64_t d, const int64_t *st,
                              float scale, int causal, int64_t chunk, int workers) {
  if (batch <= 0 || heads <= 0 || sk <= 0) return 0;
  if (head_group < 1 || heads % head_group) return 1;
  if (chunk <= 0) chunk = 64;
  const uint32_t csr = enter_ieee();
  const float log2e = 1.4426950408889634f;
  const float factor = scale * log2e;
  const int64_t kv_heads = heads / head_group;
  const int64_t count = batch * kv_heads * sk;
  const int64_t members = head_group * sq;                      /* the region-fold axis */
  const int size = team_size(workers, count);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(count, omp_get_thread_num(), size, &begin, &end);
    float *ak = (float *)malloc(sizeof(float) * (size_t)d), *av = (float *)malloc(sizeof(float) * (size_t)d);
    float *pk = (float *)malloc(sizeof(float) * (size_t)d), *pv = (float *)malloc(sizeof(float) * (size_t)d);
    for (int64_t item = begin; item < end; ++item) {
      const int64_t bi = item / (kv_heads * sk), kh = (item / sk) % kv_heads, kj = item % sk;
      const uint16_t *kp = k + bi * st[4] + kh * st[5] + kj * st[6];
      const uint16_t *vp = v + bi * st[8] + kh * st[9] + kj * st[10];
      for (int64_t t = 0; t < d; ++t) ak[t] = av[t] = 0.0f;
      for (int64_t m0 = 0; m0 < members; m0 += chunk) {
        const int64_t m1 = m0 + chunk < members ? m0 + chunk : members;
        for (int64_t t = 0; t < d; ++t) pk[t] = pv[t] = 0.0f;
        for (int64_t member = m0; member < m1; ++member) {
          const int64_t hi = kh * head_group + member / sq, qi = member % sq;
          if (causal && kj > qi) continue;                       /* excluded pair */
          const uint16_t *qp = q + bi * st[0] + hi * st[1] + qi * st[2];
          const uint16_t *gp = dout + bi * st[12] + hi * st[13] + qi * st[14];
          const float l = lse[bi * st[16] + hi * st[17] + qi * st[18]];
          const float dl = delta[bi * st[19] + hi * st[20] + qi * st[21]];
          const float s = dot_f16(kp, st[7], qp, st[3], d);
          const float p = exp2_approx_ftz(s * factor - l * log2e);
          const float p16 = oracle_half_to_float(oracle_float_to_half(p));
          for (int64_t t = 0; t < d; ++t) pv[t] = pv[t] + p16 * oracle_half_to_float(gp[t * st[15]]);
          const float dp = dot_f16(vp, st[11], gp, st[15], d);
          const float ds16 = oracle_half_to_float(oracle_float_to_half(p * (dp - dl)));
          for (int64_t t = 0; t < d; ++t) pk[t] = pk[t] + ds16 * oracle_half_to_float(qp[t * st[3]]);
        }
        for (int64_t t = 0; t < d; ++t) {
          ak[t] = ak[t] + pk[t];
          av[t] = av[t] + pv[t];
        }
      }
      uint16_t *ko = dk + bi * st[22] + kh * st[23] + kj * st[24];
      uint16_t *vo = dv + bi * st[26] + kh * st[27] + kj * st[28];
      for (int64_t t = 0; t < d; ++t) {
        ko[t * st[25]] = oracle_float_to_half(ak[t] * scale);
        vo[t * st[29]] = oracle_float_to_half(av[t]);
      }
    }
    free(ak);
    free(av);
    free(pk);
    free(pv);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

/* ------------------------------------------------------------------ paged decode (split-K)
 * streaming/paged_attention.py:77-165 (paged_gqa_decode_partials) with
 * summarize_masked_attention_chunk (streaming/attention.py:250-285) and
 * merge_attention_summaries (:82-114); contiguous layouts: q [B,HQ,D], key_cache [P,PS,HK,D],
 * value_cache [P,PS,HK,DV], partial_lse [B,HQ,SPLITS], partial_output [B,HQ,SPLITS,DV].
 * Job j = batch * SPLITS + split covers page positions [split_offsets[j], split_offsets[j+1]);
 * token t of the job: position first + t / PS, offset t % PS, physical page page_indices[position],
 * logical token (position - page_offsets[batch]) * PAGE_SIZE + offset, active below the sequence
 * length. Chunks of `chunk` tokens are summarized (exp2 domain, P rounded to f16) and merged.
 * partial_lse = maximum + logf(denominator) * log2e, partial_output = accumulator * (1 / den);
 * an empty job gives -inf and zeros. */
int oracle_paged_decode_partials(const uint16_t *q, const uint16_t *kc, const uint16_t *vc, const int32_t *page_offsets,
                                 const int32_t *page_indices, const int32_t *lengths, const int32_t *split_offsets,
                                 float *partial_lse, float *partial_out, int64_t batch, int64_t heads, int64_t d,
                                 int64_t ps, int64_t kv_heads, int64_t dv, int64_t page_size, int64_t head_group,
                                 int64_t splits, float scale, int64_t chunk, int workers) {
  if (batch <= 0 || heads <= 0 || splits <= 0) return 0;
  if (head_group < 1 || heads != kv_heads * head_group) return 1;
  if (chunk <= 0) chunk = 64;
  const uint32_t csr = enter_ieee();
  const float log2e = 1.4426950408889634f;
  const float factor = scale * log2e;
  const int64_t count = batch * splits * heads;
  const int size = team_size(workers, count);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(count, omp_get_thread_num(), size, &begin, &end);
    float *acc = (float *)malloc(sizeof(float) * (size_t)dv), *cacc = (float *)malloc(sizeof(float) * (size_t)dv);
    float *scores = (float *)malloc(sizeof(float) * (size_t)chunk);
    for (int64_t item = begin; item < end; ++item) {
      const int64_t job = item / heads, h = item % heads, b = job / splits, split = job % splits;
      const int64_t kh = h / head_group;
      const int64_t first = split_offsets[job], pages = split_offsets[job + 1] - split_offsets[job];
      const int64_t tokens = pages * ps, length = lengths[b], page_begin = page_offsets[b];
      const uint16_t *qp = q + (b * heads + h) * d;
      int valid = 0;
      float maximum = 0.0f, denominator = 0.0f;
      for (int64_t t = 0; t < dv; ++t) acc[t] = 0.0f;
      for (int64_t t0 = 0; t0 < tokens; t0 += chunk) {
        const int64_t t1 = t0 + chunk < tokens ? t0 + chunk : tokens;
        int cvalid = 0;
        float cmax = -INFINITY;
        for (int64_t t = t0; t < t1; ++t) {
          const int64_t position = first + t / ps, offset = t % ps;
          const int64_t logical = (position - page_begin) * page_size + offset;
          const int active = logical < length;
          const uint16_t *kp = kc + ((page_indices[position] * ps + offset) * kv_heads + kh) * d;
          float dot = 0.0f;
          for (int64_t c = 0; c < d; ++c) dot = dot + oracle_half_to_float(qp[c]) * oracle_half_to_float(kp[c]);
          scores[t - t0] = active ? dot * factor : -INFINITY;
          if (active) {
            cvalid = 1;
            cmax = fmaxf(cmax, scores[t - t0]);
          }
        }
        if (!cvalid) cmax = 0.0f;
        float cden = 0.0f;
        for (int64_t c = 0; c < dv; ++c) cacc[c] = 0.0f;
        for (int64_t t = t0; t < t1; ++t) {
          const int64_t position = first + t / ps, offset = t % ps;
          const int active = (position - page_begin) * page_size + offset < length;
          const float weight = active ? exp2_approx_ftz(scores[t - t0] - cmax) : 0.0f;
          cden += weight;
          const float w16 = oracle_half_to_float(oracle_float_to_half(weight));
          const uint16_t *vp = vc + ((page_indices[position] * ps + offset) * kv_heads + kh) * dv;
          for (int64_t c = 0; c < dv; ++c) cacc[c] = cacc[c] + w16 * oracle_half_to_float(vp[c]);
        }
        float merged = valid ? maximum : cmax;
        if (cvalid) merged = fmaxf(merged, cmax);
        const float left = valid ? exp2_approx_ftz(maximum - merged) : 0.0f;
        const float right = cvalid ? exp2_approx_ftz(cmax - merged) : 0.0f;
        denominator = left * denominator + right * cden;
        for (int64_t c = 0; c < dv; ++c) acc[c] = left * acc[c] + right * cacc[c];
        maximum = merged;
        valid = valid || cvalid;
      }
      const float safe = valid ? denominator : 1.0f;
      const float inverse = 1.0f / safe;
      partial_lse[(b * heads + h) * splits + split] = valid ? maximum + logf(safe) * log2e : -INFINITY;
      float *op = partial_out + ((b * heads + h) * splits + split) * dv;
      for (int64_t c = 0; c < dv; ++c) op[c] = valid ? acc[c] * inverse : 0.0f;
    }
    free(acc);
    free(cacc);
    free(scores);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

/* ------------------------------------------------------------------ decode variants
 * The fold of one query over a list of keys, chunk by chunk, as the attention definitions write it
 * (summarize_attention_chunk_f16 / _bf16 and summarize_masked_attention_chunk,
 * streaming/attention.py:152-285, merged by merge_attention_summaries :82-114): scores
 * dot * scale * log2e over active keys, the chunk maximum by maximum_num (0 for a chunk with no
 * active key), weights exp2(s - chunk max) rounded to the storage type before P @ V, chunks merged
 * with exp2 factors. krows[j] / vrows[j] are key j's rows (unit inner stride); active may be null
 * (every key active). chunk_max, when not null, receives each chunk's maximum. */
typedef struct {
  int valid;
  float maximum, denominator;
} fold_state;

static fold_state fold_keys(int dtype, const float *qrow, int64_t d, int64_t dv, const uint16_t *const *krows,
                            const uint16_t *const *vrows, const unsigned char *active, int64_t n, float factor,
                            int64_t chunk, float *scores, float *cacc, float *acc, float *chunk_max) {
  fold_state st = {0, 0.0f, 0.0f};
  for (int64_t t = 0; t < dv; ++t) acc[t] = 0.0f;
  for (int64_t k0 = 0; k0 < n; k0 += chunk) {
    const int64_t k1 = k0 + chunk < n ? k0 + chunk : n;
    int cvalid = 0;
    float cmax = -INFINITY;
    for (int64_t j = k0; j < k1; ++j) {
      const int on = active == NULL || active[j];
      float dot = 0.0f;
      if (on)
        for (int64_t t = 0; t < d; ++t) dot = dot + qrow[t] * load_elem(krows[j], dtype, t);
      scores[j - k0] = on ? dot * factor : -INFINITY;
      if (on) {
        cvalid = 1;
        cmax = fmaxf(cmax, scores[j - k0]);
      }
    }
    if (!cvalid) cmax = 0.0f;
    if (chunk_max != NULL) chunk_max[k0 / chunk] = cmax;
    float cden = 0.0f;
    for (int64_t t = 0; t < dv; ++t) cacc[t] = 0.0f;
    for (int64_t j = k0; j < k1; ++j) {
      if (active != NULL && !active[j]) continue;
      const float weight = exp2_approx_ftz(scores[j - k0] - cmax);
      cden += weight;
      const float rounded = dtype == ORACLE_BF16 ? oracle_bf16_to_float(oracle_float_to_bf16(weight))
                                                 : oracle_half_to_float(oracle_float_to_half(weight));
      for (int64_t t = 0; t < dv; ++t) cacc[t] = cacc[t] + rounded * load_elem(vrows[j], dtype, t);
    }
    float merged = st.valid ? st.maximum : cmax;
    if (cvalid) merged = fmaxf(merged, cmax);
    const float left = st.valid ? exp2_approx_ftz(st.maximum - merged) : 0.0f;
    const float right = cvalid ? exp2_approx_ftz(cmax - merged) : 0.0f;
    st.denominator = left * st.denominator + right * cden;
    for (int64_t t = 0; t < dv; ++t) acc[t] = left * acc[t] + right * cacc[t];
    st.maximum = merged;
    st.valid = st.valid || cvalid;
  }
  return st;
}

/* grouped_flash_decode_partials (streaming/attention.py:556-627): bf16 q [B,HQ,1,D], k [B,HK,K,D],
 * v [B,HK,K,DV] (contiguous); part p of (b, key head) covers key slots p * split .. + split, active
 * below K. partial_lse [B,HQ,P] = max + logf(den) * log2e (-inf for an empty part),
 * partial_output bf16 [B,HQ,P,DV] = acc * rcp(den) (0 for an empty part). */
int oracle_grouped_decode_partials(const uint16_t *q, const uint16_t *k, const uint16_t *v, float *partial_lse,
                                   uint16_t *partial_out, int64_t batch, int64_t heads, int64_t kv_heads,
                                   int64_t keys, int64_t d, int64_t dv, int64_t parts, int64_t split, float scale,
                                   int64_t chunk, int workers) {
  if (batch <= 0 || heads <= 0 || parts <= 0) return 0;
  if (kv_heads < 1 || heads % kv_heads || split < 1) return 1;
  if (chunk <= 0) chunk = 64;
  const uint32_t csr = enter_ieee();
  const float log2e = 1.4426950408889634f;
  const int64_t group = heads / kv_heads, count = batch * heads * parts;
  const int size = team_size(workers, count);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(count, omp_get_thread_num(), size, &begin, &end);
    const uint16_t **krows = (const uint16_t **)malloc(sizeof(void *) * (size_t)split);
    const uint16_t **vrows = (const uint16_t **)malloc(sizeof(void *) * (size_t)split);
    float *qrow = (float *)malloc(sizeof(float) * (size_t)d), *scores = (float *)malloc(sizeof(float) * (size_t)chunk);
    float *acc = (float *)malloc(sizeof(float) * (size_t)dv), *cacc = (float *)malloc(sizeof(float) * (size_t)dv);
    for (int64_t item = begin; item < end; ++item) {
      const int64_t b = item / (heads * parts), h = (item / parts) % heads, part = item % parts, kh = h / group;
      for (int64_t t = 0; t < d; ++t) qrow[t] = oracle_bf16_to_float(q[(b * heads + h) * d + t]);
      const int64_t first = part * split;
      const int64_t n = first >= keys ? 0 : (keys - first < split ? keys - first : split);
      for (int64_t j = 0; j < n; ++j) {
        krows[j] = k + ((b * kv_heads + kh) * keys + first + j) * d;
        vrows[j] = v + ((b * kv_heads + kh) * keys + first + j) * dv;
      }
      const fold_state st = fold_keys(ORACLE_BF16, qrow, d, dv, krows, vrows, NULL, n, scale * log2e, chunk, scores,
                                      cacc, acc, NULL);
      const float safe = st.valid ? st.denominator : 1.0f;
      partial_lse[(b * heads + h) * parts + part] = st.valid ? st.maximum + logf(safe) * log2e : -INFINITY;
      const float inverse = rcp_approx_ftz(safe);
      uint16_t *op = partial_out + ((b * heads + h) * parts + part) * dv;
      for (int64_t t = 0; t < dv; ++t) op[t] = oracle_float_to_bf16(st.valid ? acc[t] * inverse : 0.0f);
    }
    free(krows);
    free(vrows);
    free(qrow);
    free(scores);
    free(acc);
    free(cacc);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

/* continuous_gqa_decode (streaming/attention.py:629-670): f16 q [B,HQ,D], k [B,K,HK,D],
 * v [B,K,HK,DV], valid_mask u8 [B,K,HK] (contiguous); output f16 [B,HQ,DV] = acc * rcp(den), 0 for a
 * query with no admitted key. */
int oracle_continuous_gqa_decode(const uint16_t *q, const uint16_t *k, const uint16_t *v, const uint8_t *mask,
                                 uint16_t *out, int64_t batch, int64_t heads, int64_t kv_heads, int64_t keys,
                                 int64_t d, int64_t dv, float scale, int64_t chunk, int workers) {
  if (batch <= 0 || heads <= 0) return 0;
  if (kv_heads < 1 || heads % kv_heads) return 1;
  if (chunk <= 0) chunk = 64;
  const uint32_t csr = enter_ieee();
  const float log2e = 1.4426950408889634f;
  const int64_t group = heads / kv_heads, count = batch * heads;
  const int size = team_size(workers, count);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(count, omp_get_thread_num(), size, &begin, &end);
    const size_t n = keys > 0 ? (size_t)keys : 1;
    const uint16_t **krows = (const uint16_t **)malloc(sizeof(void *) * n);
    const uint16_t **vrows = (const uint16_t **)malloc(sizeof(void *) * n);
    unsigned char *active = (unsigned char *)malloc(n);
    float *qrow = (float *)malloc(sizeof(float) * (size_t)d), *scores = (float *)malloc(sizeof(float) * (size_t)chunk);
    float *acc = (float *)malloc(sizeof(float) * (size_t)dv), *cacc = (float *)malloc(sizeof(float) * (size_t)dv);
    for (int64_t item = begin; item < end; ++item) {
      const int64_t b = item / heads, h = item % heads, kh = h / group;
      for (int64_t t = 0; t < d; ++t) qrow[t] = oracle_half_to_float(q[(b * heads + h) * d + t]);
      for (int64_t j = 0; j < keys; ++j) {
        krows[j] = k + ((b * keys + j) * kv_heads + kh) * d;
        vrows[j] = v + ((b * keys + j) * kv_heads + kh) * dv;
        active[j] = mask[(b * keys + j) * kv_heads + kh] != 0;
      }
      const fold_state st = fold_keys(ORACLE_F16, qrow, d, dv, krows, vrows, active, keys, scale * log2e, chunk,
                                      scores, cacc, acc, NULL);
      const float inverse = rcp_approx_ftz(st.valid ? st.denominator : 1.0f);
      for (int64_t t = 0; t < dv; ++t)
        out[(b * heads + h) * dv + t] = oracle_float_to_half(st.valid ? acc[t] * inverse : 0.0f);
    }
    free(krows);
    free(vrows);
    free(active);
    free(qrow);
    free(scores);
    free(acc);
    free(cacc);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

/* varlen_gqa_decode_with_sink_logits (streaming/attention.py:672-754): f16 q [B,HQ,D], k [U,HK,D],
 * v [U,HK,DV] (contiguous), cu [B+1], sink f32 [HQ]. Sequence b's keys are rows cu[b] .. cu[b+1]; the
 * first 64 * max_blocks of them are folded in 64-key blocks. With M the merged maximum and
 * inverse = rcp(den + sink[h]) (rcp(1) for an empty sequence): output = acc * inverse (0 when
 * empty), block_logits [B,HQ,max_blocks] = exp2(block max - M) * inverse below ceil(length / 64),
 * else 0. */
int oracle_varlen_decode_sink(const uint16_t *q, const uint16_t *k, const uint16_t *v, const int32_t *cu,
                              const float *sink, uint16_t *out, float *block_logits, int64_t sequences,
                              int64_t heads, int64_t kv_heads, int64_t d, int64_t dv, int64_t max_blocks,
                              float scale, int workers) {
  if (sequences <= 0 || heads <= 0) return 0;
  if (kv_heads < 1 || heads % kv_heads) return 1;
  const uint32_t csr = enter_ieee();
  const float log2e = 1.4426950408889634f;
  const int64_t group = heads / kv_heads, count = sequences * heads, cap = 64 * max_blocks;
  const int size = team_size(workers, count);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(count, omp_get_thread_num(), size, &begin, &end);
    const size_t n = cap > 0 ? (size_t)cap : 1;
    const uint16_t **krows = (const uint16_t **)malloc(sizeof(void *) * n);
    const uint16_t **vrows = (const uint16_t **)malloc(sizeof(void *) * n);
    float *maxima = (float *)malloc(sizeof(float) * (max_blocks > 0 ? (size_t)max_blocks : 1));
    float *qrow = (float *)malloc(sizeof(float) * (size_t)d), *scores = (float *)malloc(sizeof(float) * 64);
    float *acc = (float *)malloc(sizeof(float) * (size_t)dv), *cacc = (float *)malloc(sizeof(float) * (size_t)dv);
    for (int64_t item = begin; item < end; ++item) {
      const int64_t b = item / heads, h = item % heads, kh = h / group;
      const int64_t length = (int64_t)cu[b + 1] - cu[b], blocks = (length + 63) / 64;
      const int64_t taken = length < cap ? length : cap;
      for (int64_t t = 0; t < d; ++t) qrow[t] = oracle_half_to_float(q[(b * heads + h) * d + t]);
      for (int64_t j = 0; j < taken; ++j) {
        krows[j] = k + ((cu[b] + j) * kv_heads + kh) * d;
        vrows[j] = v + ((cu[b] + j) * kv_heads + kh) * dv;
      }
      const fold_state st = fold_keys(ORACLE_F16, qrow, d, dv, krows, vrows, NULL, taken, scale * log2e, 64, scores,
                                      cacc, acc, maxima);
      const float inverse = rcp_approx_ftz(st.valid ? st.denominator + sink[h] : 1.0f);
      for (int64_t t = 0; t < dv; ++t)
        out[(b * heads + h) * dv + t] = oracle_float_to_half(st.valid ? acc[t] * inverse : 0.0f);
      for (int64_t j = 0; j < max_blocks; ++j)
        block_logits[(b * heads + h) * max_blocks + j] =
            j < blocks ? exp2_approx_ftz(maxima[j] - st.maximum) * inverse : 0.0f;
    }
    free(krows);
    free(vrows);
    free(maxima);
    free(qrow);
    free(scores);
    free(acc);
    free(cacc);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

/* streaming/splitk_reduce.py:129-155 (splitk_attention_f32_to_f16_reduce): per (b, h),
 * m = maximum_num over splits of lse (identity -inf), w_s = expf(lse_s - m) (a natural exponential,
 * as the definition writes it), out = f16((sum_s w_s * partial_s) * rcp_approx(sum_s w_s)). All
 * splits empty (-inf) gives NaN, as the definition does. Contiguous [B,H,S,D], [B,H,S], [B,H,D]. */
int oracle_splitk_reduce_f32_to_f16(const float *partial, const float *lse, uint16_t *out, int64_t batch,
                                    int64_t heads, int64_t splits, int64_t d, int workers) {
  if (batch <= 0 || heads <= 0) return 0;
  const uint32_t csr = enter_ieee();
  const int64_t count = batch * heads;
  const int size = team_size(workers, count);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(count, omp_get_thread_num(), size, &begin, &end);
    float *num = (float *)malloc(sizeof(float) * (size_t)(d > 0 ? d : 1));
    for (int64_t row = begin; row < end; ++row) {
      const float *l = lse + row * splits;
      float m = -INFINITY;
      for (int64_t s = 0; s < splits; ++s) m = fmaxf(m, l[s]);
      float den = 0.0f;
      for (int64_t c = 0; c < d; ++c) num[c] = 0.0f;
      for (int64_t s = 0; s < splits; ++s) {
        const float w = expf(l[s] - m);
        den = den + w;
        const float *p = partial + (row * splits + s) * d;
        for (int64_t c = 0; c < d; ++c) num[c] = num[c] + w * p[c];
      }
      const float r = rcp_approx_ftz(den);
      for (int64_t c = 0; c < d; ++c) out[row * d + c] = oracle_float_to_half(num[c] * r);
    }
    free(num);
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

/* ------------------------------------------------------------------ CSR SpMM
 * sparse/csr_spmm.py:11-33: per row r and feature f, acc = 0.0f; for nz in [off[r], off[r+1]) in
 * order: acc = acc + values[nz] * dense[col[nz], f] (product rounded, then added); out[r, f] = acc.
 * dense [cols, features] with row stride ldd, out [rows, features] with row stride ldo. */
int oracle_csr_spmm_f32(const int32_t *off, const int32_t *col, const float *val, const float *dense, float *out,
                        int64_t rows, int64_t features, int64_t ldd, int64_t ldo, int workers) {
  if (rows <= 0 || features <= 0) return 0;
  const uint32_t csr = enter_ieee();
  const int size = team_size(workers, rows);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(rows, omp_get_thread_num(), size, &begin, &end);
    for (int64_t r = begin; r < end; ++r) {
      float *o = out + r * ldo;
      for (int64_t f = 0; f < features; ++f) o[f] = 0.0f;
      for (int64_t nz = off[r]; nz < off[r + 1]; ++nz) {
        const float v = val[nz];
        const float *d = dense + (int64_t)col[nz] * ldd;
        for (int64_t f = 0; f < features; ++f) {
          const float product = v * d[f];
          o[f] = o[f] + product;
        }
      }
    }
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}

/* ------------------------------------------------------------------ CSR SpMV
 * sparse/csr_spmv.py:11-29: acc = 0.0f; for nz in [off[r], off[r+1]) in order:
 * acc = acc + values[nz] * vector[col[nz]] (product rounded, then added); y[r] = acc. */
int oracle_csr_spmv_f32(const int32_t *off, const int32_t *col, const float *val, const float *x, float *y,
                        int64_t rows, int workers) {
  if (rows <= 0) return 0;
  const uint32_t csr = enter_ieee();
  const int size = team_size(workers, rows);
#pragma omp parallel num_threads(size)
  {
    const uint32_t inner = enter_ieee();
    int64_t begin, end;
    row_range(rows, omp_get_thread_num(), size, &begin, &end);
    for (int64_t r = begin; r < end; ++r) {
      float acc = 0.0f;
      for (int64_t nz = off[r]; nz < off[r + 1]; ++nz) {
        const float product = val[nz] * x[col[nz]];
        acc = acc + product;
      }
      y[r] = acc;
    }
    leave_ieee(inner);
  }
  leave_ieee(csr);
  return 0;
}
