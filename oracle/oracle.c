/*
 * CPU oracle for the quantized-weights matmul. TEST INFRASTRUCTURE ONLY:
 * loaded by tests/, the smoke check and the benchmark's CPU-baseline leg,
 * never by the product library. See oracle.h for what pins each function.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; the AVX2 restatements
 * carry their own target attribute, as the reference's do).
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------- */
/* Scalars                                                                  */
/* ---------------------------------------------------------------------- */

/* IEEE binary16 -> binary32 by bit manipulation.
 * Follows adapters/llama/gguf.c:601-630: signed zero, subnormals
 * renormalised by shifting the mantissa until the implicit bit appears,
 * inf/NaN keep the payload shifted left by 13. */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
  uint32_t f = (uint32_t)h & 0x3FFu;
  uint32_t bits;
  float out;
  if (e == 0u && f == 0u) {
    bits = sign;
  } else if (e == 0u) {
    /* subnormal: value = f * 2^-24; normalise */
    uint32_t ex = 113u; /* 127 - 15 + 1 */
    while ((f & 0x400u) == 0u) {
      f <<= 1;
      ex -= 1u;
    }
    bits = sign | (ex << 23) | ((f & 0x3FFu) << 13);
  } else if (e == 0x1Fu) {
    bits = sign | 0x7F800000u | (f << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (f << 13);
  }
  memcpy(&out, &bits, sizeof out);
  return out;
}

/* Bulk form writing raw bit patterns (a float return value would be
 * widened to double by some callers, which quiets signalling NaNs). */
void orc_f16_to_f32_bits(const uint16_t *h, uint32_t *out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) {
    const float f = orc_f16_to_f32(h[i]);
    memcpy(&out[i], &f, sizeof f);
  }
}

static float le_half(const uint8_t *p) {
  return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

/* Round-to-nearest-even binary32 -> binary16 (for the textbook encoders
 * below; the reference has no f32->f16 encoder). */
static uint16_t f32_to_f16_rne(float v) {
  uint32_t x;
  memcpy(&x, &v, sizeof x);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) { /* inf / nan */
    return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
  }
  if (ax >= 0x477FF000u) { /* rounds to >= 65520 -> inf */
    return (uint16_t)(sign | 0x7C00u);
  }
  if (ax < 0x38800000u) { /* below the smallest normal half: subnormal */
    /* value in units of 2^-24, rounded to nearest even */
    float a;
    memcpy(&a, &ax, sizeof a);
    float scaled = a * 16777216.0f; /* exact: power of two */
    float r = nearbyintf(scaled);   /* default rounding mode: RNE */
    return (uint16_t)(sign | (uint16_t)r);
  }
  uint32_t e = (ax >> 23) - 112u;
  uint32_t mant = ax & 0x7FFFFFu;
  uint32_t h = (e << 10) | (mant >> 13);
  uint32_t rest = mant & 0x1FFFu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) {
    h += 1u; /* carries into the exponent correctly */
  }
  return (uint16_t)(sign | h);
}

/* 6-bit (scale, min) pair j of a Q4_K super-block's 12 packed bytes.
 * Follows adapters/llama/gguf.c:639-648. */
void orc_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn) {
  if (j >= 4) {
    *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
    *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  } else {
    *sc = (uint8_t)(q[j] & 0x3F);
    *mn = (uint8_t)(q[j + 4] & 0x3F);
  }
}

/* Bytes of `numel` elements; 0 when numel is not a whole number of
 * blocks or the type is not one of the four on this path.
 * Follows adapters/llama/gguf.c:562-597 (Q4_0 :571, Q8_0 :578,
 * Q4_K :586, Q6_K :590). */
uint64_t orc_type_bytes(uint32_t type, uint64_t numel) {
  switch (type) {
  case ORC_Q4_0:
    return (numel % 32u) ? 0u : numel / 32u * 18u;
  case ORC_Q8_0:
    return (numel % 32u) ? 0u : numel / 32u * 34u;
  case ORC_Q4_K:
    return (numel % 256u) ? 0u : numel / 256u * 144u;
  case ORC_Q6_K:
    return (numel % 256u) ? 0u : numel / 256u * 210u;
  default:
    return 0u;
  }
}

/* ---------------------------------------------------------------------- */
/* Block dequantization                                                     */
/* ---------------------------------------------------------------------- */

/* Q4_0, adapters/llama/gguf.c:680-694: 18-byte block = f16 d + 16 bytes;
 * byte j holds element j (low nibble) and element j+16 (high nibble),
 * both offset by 8; value = (float)(nibble-8) * d. */
static void dq_q4_0(const uint8_t *blk, float *out) {
  const float d = le_half(blk);
  for (int j = 0; j < 16; ++j) {
    const uint8_t b = blk[2 + j];
    out[j] = (float)((int)(b & 0x0F) - 8) * d;
    out[j + 16] = (float)((int)(b >> 4) - 8) * d;
  }
}

/* Q8_0, adapters/llama/gguf.c:750-761: f16 d + 32 int8; value = q * d. */
static void dq_q8_0(const uint8_t *blk, float *out) {
  const float d = le_half(blk);
  for (int j = 0; j < 32; ++j) {
    out[j] = (float)(int8_t)blk[2 + j] * d;
  }
}

/* Q4_K, adapters/llama/gguf.c:852-882: 144-byte super-block = f16 d,
 * f16 dmin, 12 bytes of packed 6-bit (scale, min), 128 bytes of codes.
 * Chunk c (64 elements) uses bytes q[32c .. 32c+32): low nibbles are
 * elements 64c+l with pair 2c, high nibbles are 64c+32+l with pair 2c+1.
 * The reference forms d1 = d*sc and m1 = dmin*m first, then d1*q - m1. */
static void dq_q4_k(const uint8_t *blk, float *out) {
  const float d = le_half(blk);
  const float dmin = le_half(blk + 2);
  const uint8_t *scales = blk + 4;
  const uint8_t *q = blk + 16;
  for (int c = 0; c < 4; ++c) {
    uint8_t s0, m0, s1, m1;
    orc_scale_min_k4(2 * c, scales, &s0, &m0);
    orc_scale_min_k4(2 * c + 1, scales, &s1, &m1);
    const float dlo = d * (float)s0, mlo = dmin * (float)m0;
    const float dhi = d * (float)s1, mhi = dmin * (float)m1;
    for (int l = 0; l < 32; ++l) {
      out[64 * c + l] = dlo * (float)(q[32 * c + l] & 0x0F) - mlo;
    }
    for (int l = 0; l < 32; ++l) {
      out[64 * c + 32 + l] = dhi * (float)(q[32 * c + l] >> 4) - mhi;
    }
  }
}

/* Q6_K, adapters/llama/gguf.c:920-947: 210-byte super-block = ql[128],
 * qh[64], int8 scales[16], f16 d. Two halves of 128 elements; in half h,
 * for l < 32 the four 6-bit codes are
 *   e = l      : ql[l] low nibble,    qh[l] bits 0-1, scale sc[l/16 + 0]
 *   e = l + 32 : ql[l+32] low nibble, qh[l] bits 2-3, scale sc[l/16 + 2]
 *   e = l + 64 : ql[l] high nibble,   qh[l] bits 4-5, scale sc[l/16 + 4]
 *   e = l + 96 : ql[l+32] high nibble,qh[l] bits 6-7, scale sc[l/16 + 6]
 * with ql/qh/sc advanced by 64/32/8 per half; value = d * sc * (code-32),
 * evaluated left to right. */
static void dq_q6_k(const uint8_t *blk, float *out) {
  const float d = le_half(blk + 208);
  for (int h = 0; h < 2; ++h) {
    const uint8_t *ql = blk + 64 * h;
    const uint8_t *qh = blk + 128 + 32 * h;
    const int8_t *sc = (const int8_t *)(blk + 192 + 8 * h);
    float *o = out + 128 * h;
    for (int l = 0; l < 32; ++l) {
      const int s = l / 16;
      const int c0 = (int)((ql[l] & 0x0F) | (((qh[l] >> 0) & 3) << 4)) - 32;
      const int c1 = (int)((ql[l + 32] & 0x0F) | (((qh[l] >> 2) & 3) << 4)) - 32;
      const int c2 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
      const int c3 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
      o[l] = d * (float)sc[s + 0] * (float)c0;
      o[l + 32] = d * (float)sc[s + 2] * (float)c1;
      o[l + 64] = d * (float)sc[s + 4] * (float)c2;
      o[l + 96] = d * (float)sc[s + 6] * (float)c3;
    }
  }
}

/* Dequantize `numel` elements of contiguous blocks.
 * Follows the Q4_0/Q8_0/Q4_K/Q6_K cases of adapters/llama/gguf.c:650-967;
 * other types return UNSUPPORTED (gguf.c:964-966). */
int32_t orc_dequant(uint32_t type, const uint8_t *src, float *dst,
                    uint64_t numel) {
  if (src == NULL || dst == NULL) {
    return ORC_ERR_INVALID_ARG;
  }
  if (orc_type_bytes(type, numel) == 0u) {
    return ORC_ERR_UNSUPPORTED;
  }
  switch (type) {
  case ORC_Q4_0:
    for (uint64_t b = 0; b < numel / 32u; ++b) dq_q4_0(src + 18u * b, dst + 32u * b);
    break;
  case ORC_Q8_0:
    for (uint64_t b = 0; b < numel / 32u; ++b) dq_q8_0(src + 34u * b, dst + 32u * b);
    break;
  case ORC_Q4_K:
    for (uint64_t b = 0; b < numel / 256u; ++b) dq_q4_k(src + 144u * b, dst + 256u * b);
    break;
  case ORC_Q6_K:
    for (uint64_t b = 0; b < numel / 256u; ++b) dq_q6_k(src + 210u * b, dst + 256u * b);
    break;
  default:
    return ORC_ERR_UNSUPPORTED;
  }
  return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* Matmuls                                                                  */
/* ---------------------------------------------------------------------- */

/* c[i][j] = sum_{l<k} a[i][l] * b[l][j], one f32 accumulator per output,
 * l ascending, no contraction (built with -ffp-contract=off).
 * Follows cpu/reference/ref_ops.c:427-444 including its argument checks. */
int32_t orc_gemm_seq_f32(uint64_t m, uint64_t n, uint64_t k, const float *a,
                         const float *b, float *c) {
  if (m == 0u || n == 0u || k == 0u || a == NULL || b == NULL || c == NULL) {
    return ORC_ERR_INVALID_ARG;
  }
  for (uint64_t i = 0; i < m; ++i) {
    for (uint64_t j = 0; j < n; ++j) {
      float acc = 0.0f;
      for (uint64_t l = 0; l < k; ++l) {
        acc += a[i * k + l] * b[l * n + j];
      }
      c[i * n + j] = acc;
    }
  }
  return ORC_OK;
}

static int32_t dequant_matrix(uint32_t type, uint64_t n, uint64_t k,
                              const uint8_t *blocks, float **out) {
  const uint64_t row_bytes = orc_type_bytes(type, k);
  if (row_bytes == 0u) {
    return ORC_ERR_UNSUPPORTED;
  }
  float *w = (float *)malloc((size_t)(n * k) * sizeof(float));
  if (w == NULL) {
    return ORC_ERR_NOMEM;
  }
  for (uint64_t r = 0; r < n; ++r) {
    int32_t st = orc_dequant(type, blocks + r * row_bytes, w + r * k, k);
    if (st != ORC_OK) {
      free(w);
      return st;
    }
  }
  *out = w;
  return ORC_OK;
}

/* The reference's CPU operator for one projection, as a composition:
 * dequantize the native [N][K] blocks (adapters/llama/gguf.c:969-1012),
 * transpose to [K][N] (adapters/llama/llama.c:196-209, used at :433),
 * then pai_ref_gemm_f32 (cpu/reference/ref_ops.c:427-444) with a = x[M][K].
 * The transpose is folded into the index: b[l][j] == W[j][l]. */
int32_t orc_qgemm_seq_f32(uint32_t type, uint64_t n, uint64_t k,
                          const uint8_t *blocks, uint64_t m, const float *x,
                          float *y) {
  if (m == 0u || n == 0u || k == 0u || blocks == NULL || x == NULL || y == NULL) {
    return ORC_ERR_INVALID_ARG;
  }
  float *w = NULL;
  int32_t st = dequant_matrix(type, n, k, blocks, &w);
  if (st != ORC_OK) {
    return st;
  }
  for (uint64_t i = 0; i < m; ++i) {
    for (uint64_t j = 0; j < n; ++j) {
      float acc = 0.0f;
      for (uint64_t l = 0; l < k; ++l) {
        acc += x[i * k + l] * w[j * k + l];
      }
      y[i * n + j] = acc;
    }
  }
  free(w);
  return ORC_OK;
}

/* Same composition with an f64 accumulator (the tolerance anchor). */
int32_t orc_qgemm_f64(uint32_t type, uint64_t n, uint64_t k,
                      const uint8_t *blocks, uint64_t m, const float *x,
                      double *y) {
  if (m == 0u || n == 0u || k == 0u || blocks == NULL || x == NULL || y == NULL) {
    return ORC_ERR_INVALID_ARG;
  }
  float *w = NULL;
  int32_t st = dequant_matrix(type, n, k, blocks, &w);
  if (st != ORC_OK) {
    return st;
  }
  for (uint64_t i = 0; i < m; ++i) {
    for (uint64_t j = 0; j < n; ++j) {
      double acc = 0.0;
      for (uint64_t l = 0; l < k; ++l) {
        acc += (double)x[i * k + l] * (double)w[j * k + l];
      }
      y[i * n + j] = acc;
    }
  }
  free(w);
  return ORC_OK;
}

/* h[i] = silu(g[i]) * u[i]: pai_ref_silu_f32 (cpu/reference/ref_ops.c:
 * 219-228, g / (1 + expf(-g)) with the C library's expf) followed by
 * pai_ref_vecmul_f32 (ref_ops.c:124-133), the SILU and MUL ops of the
 * reference's FFN (adapters/llama/llama.c:774-784). */
int32_t orc_silu_mul_f32(const float *g, const float *u, float *h, uint64_t n) {
  if ((g == NULL || u == NULL || h == NULL) && n != 0u) {
    return ORC_ERR_INVALID_ARG;
  }
  for (uint64_t i = 0; i < n; ++i) {
    const float s = g[i] / (1.0f + expf(-g[i]));
    h[i] = s * u[i];
  }
  return ORC_OK;
}

/* |a-b| <= max(abs_tol, |b|*rel_tol) per element; first failing index.
 * Follows cpu/reference/ref_ops.c:518-541. */
int32_t orc_compare_f32(const float *a, const float *b, uint64_t n,
                        float abs_tol, float rel_tol, uint64_t *first_bad) {
  if (first_bad != NULL) {
    *first_bad = UINT64_MAX;
  }
  if ((a == NULL || b == NULL) && n != 0u) {
    return ORC_ERR_INVALID_ARG;
  }
  for (uint64_t i = 0; i < n; ++i) {
    const float diff = fabsf(a[i] - b[i]);
    const float rel = fabsf(b[i]) * rel_tol;
    if (diff > (abs_tol > rel ? abs_tol : rel)) {
      if (first_bad != NULL) {
        *first_bad = i;
      }
      return ORC_ERR_MISMATCH;
    }
  }
  return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* AVX2+FMA restatements (the CPU baseline)                                 */
/* ---------------------------------------------------------------------- */

#define ORC_AVX2 __attribute__((target("avx2,fma")))

/* Horizontal sum of 8 lanes: high half onto low half, then the [1,0,3,2]
 * and [2,3,0,1] shuffles. Follows cpu/optimized/opt_ops.c:89-99. */
ORC_AVX2 static inline float hsum8(__m256 v) {
  __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
  s = _mm_add_ps(s, _mm_shuffle_ps(s, s, 0x4E));
  s = _mm_add_ps(s, _mm_shuffle_ps(s, s, 0xB1));
  return _mm_cvtss_f32(s);
}

/* y[i] = A[i][:] . x, A row-major [m][k]: one 8-wide FMA accumulator per
 * row, horizontal sum, then a scalar tail.
 * Follows cpu/optimized/opt_ops.c:527-550. */
ORC_AVX2 int32_t orc_opt_gemv_avx2(uint64_t m, uint64_t k, const float *a,
                                   const float *x, float *y) {
  if (m == 0u || k == 0u || a == NULL || x == NULL || y == NULL) {
    return ORC_ERR_INVALID_ARG;
  }
  for (uint64_t i = 0; i < m; ++i) {
    const float *row = a + i * k;
    __m256 acc = _mm256_setzero_ps();
    uint64_t l = 0;
    for (; l + 8u <= k; l += 8u) {
      acc = _mm256_fmadd_ps(_mm256_loadu_ps(row + l), _mm256_loadu_ps(x + l), acc);
    }
    float s = hsum8(acc);
    for (; l < k; ++l) {
      s += row[l] * x[l];
    }
    y[i] = s;
  }
  return ORC_OK;
}

typedef struct {
  uint64_t r0, r1, k;
  const float *a, *x;
  float *y;
} gemv_part_t;

static void *gemv_part(void *arg) {
  gemv_part_t *p = (gemv_part_t *)arg;
  if (p->r1 > p->r0) {
    orc_opt_gemv_avx2(p->r1 - p->r0, p->k, p->a + p->r0 * p->k, p->x, p->y + p->r0);
  }
  return NULL;
}

/* Harness-parallel wrapper: contiguous row ranges of the single-thread
 * kernel above on `threads` pthreads (the reference itself is serial). */
int32_t orc_opt_gemv_avx2_mt(uint64_t m, uint64_t k, const float *a,
                             const float *x, float *y, int threads) {
  if (threads <= 1) {
    return orc_opt_gemv_avx2(m, k, a, x, y);
  }
  if (m == 0u || k == 0u || a == NULL || x == NULL || y == NULL) {
    return ORC_ERR_INVALID_ARG;
  }
  if (threads > 256) {
    threads = 256;
  }
  pthread_t tid[256];
  gemv_part_t part[256];
  for (int t = 0; t < threads; ++t) {
    part[t].r0 = m * (uint64_t)t / (uint64_t)threads;
    part[t].r1 = m * (uint64_t)(t + 1) / (uint64_t)threads;
    part[t].k = k;
    part[t].a = a;
    part[t].x = x;
    part[t].y = y;
    if (pthread_create(&tid[t], NULL, gemv_part, &part[t]) != 0) {
      gemv_part(&part[t]);
      tid[t] = 0;
    }
  }
  for (int t = 0; t < threads; ++t) {
    if (tid[t] != 0) {
      pthread_join(tid[t], NULL);
    }
  }
  return ORC_OK;
}

/* c = a[m][k] * b[k][n]: 8 output columns per FMA accumulator, scalar
 * tail columns. Follows cpu/optimized/opt_ops.c:497-525. */
ORC_AVX2 int32_t orc_opt_gemm_avx2(uint64_t m, uint64_t n, uint64_t k,
                                   const float *a, const float *b, float *c) {
  if (m == 0u || n == 0u || k == 0u || a == NULL || b == NULL || c == NULL) {
    return ORC_ERR_INVALID_ARG;
  }
  for (uint64_t i = 0; i < m; ++i) {
    const float *ar = a + i * k;
    float *cr = c + i * n;
    uint64_t j = 0;
    for (; j + 8u <= n; j += 8u) {
      __m256 acc = _mm256_setzero_ps();
      for (uint64_t l = 0; l < k; ++l) {
        acc = _mm256_fmadd_ps(_mm256_set1_ps(ar[l]), _mm256_loadu_ps(b + l * n + j), acc);
      }
      _mm256_storeu_ps(cr + j, acc);
    }
    for (; j < n; ++j) {
      float s = 0.0f;
      for (uint64_t l = 0; l < k; ++l) {
        s += ar[l] * b[l * n + j];
      }
      cr[j] = s;
    }
  }
  return ORC_OK;
}

/* W8 GEMM: int8 w_q[k][n] with f32 scales per (group of k-rows, column);
 * group_size 0 or > k means one group. 8-column tiles, per-group scale
 * vector, fmadd(a[t], cvt(w)*scale, acc).
 * Follows cpu/optimized/opt_ops.c:552-592. */
ORC_AVX2 int32_t orc_opt_gemm_w8_avx2(uint64_t m, uint64_t n, uint64_t k,
                                      const float *a, const int8_t *w_q,
                                      const float *b_scales,
                                      uint64_t group_size, float *c) {
  if (m == 0u || n == 0u || k == 0u || a == NULL || w_q == NULL ||
      b_scales == NULL || c == NULL) {
    return ORC_ERR_INVALID_ARG;
  }
  const uint64_t gs = (group_size == 0u || group_size > k) ? k : group_size;
  for (uint64_t i = 0; i < m; ++i) {
    const float *ar = a + i * k;
    float *cr = c + i * n;
    uint64_t j = 0;
    for (; j + 8u <= n; j += 8u) {
      __m256 acc = _mm256_setzero_ps();
      for (uint64_t g0 = 0; g0 < k; g0 += gs) {
        const uint64_t g1 = g0 + gs < k ? g0 + gs : k;
        const __m256 sv = _mm256_loadu_ps(b_scales + (g0 / gs) * n + j);
        for (uint64_t t = g0; t < g1; ++t) {
          const __m128i w8 = _mm_loadl_epi64((const __m128i *)(const void *)(w_q + t * n + j));
          const __m256 wf = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(w8));
          acc = _mm256_fmadd_ps(_mm256_set1_ps(ar[t]), _mm256_mul_ps(wf, sv), acc);
        }
      }
      _mm256_storeu_ps(cr + j, acc);
    }
    for (; j < n; ++j) {
      float s = 0.0f;
      for (uint64_t t = 0; t < k; ++t) {
        s += ar[t] * (float)w_q[t * n + j] * b_scales[(t / gs) * n + j];
      }
      cr[j] = s;
    }
  }
  return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* v0 per-group schemes (models/quantize.c) and the GEMMs over them       */
/* (cpu/reference/ref_ops.c:446-499)                                      */
/* ---------------------------------------------------------------------- */

/* models/quantize.c:6-26: 4 or 8 bits, signed only; group size 0 means
 * one group over all n elements. */
int32_t orc_quant_group_size(const orc_quant_scheme_t *s, uint64_t n, uint64_t *out_gs) {
  if (s == NULL) return ORC_ERR_INVALID_ARG;
  if (s->bit_width != 8u && s->bit_width != 4u) return ORC_ERR_UNSUPPORTED;
  if (!s->is_signed) return ORC_ERR_UNSUPPORTED;
  const uint64_t gs = s->group_size == 0u ? n : (uint64_t)s->group_size;
  if (gs == 0u) return ORC_ERR_INVALID_ARG;
  *out_gs = gs;
  return ORC_OK;
}

/* models/quantize.c:34-49 */
uint64_t orc_quant_num_groups(uint64_t n, const orc_quant_scheme_t *s) {
  uint64_t gs;
  if (s == NULL || n == 0u || orc_quant_group_size(s, n, &gs) != ORC_OK) return 0u;
  return n / gs + (n % gs != 0u ? 1u : 0u);
}

/* models/quantize.c:51-60 (no scheme validation there either) */
uint64_t orc_quant_value_bytes(uint64_t n, const orc_quant_scheme_t *s) {
  if (s == NULL || n == 0u) return 0u;
  return s->bit_width == 4u ? (n + 1u) / 2u : n;
}

/* models/quantize.c:74-141: per group, scale = max|x| / qmax (127 or 7),
 * q = lrintf(x / scale) clamped to [-qmax, qmax] (0 for a zero group);
 * 4-bit codes go two per byte, element 2i in the low nibble. */
int32_t orc_quantize_v0_f32(const float *src, uint64_t n, const orc_quant_scheme_t *s,
                            int8_t *out_q, float *out_scales, uint64_t *out_groups) {
  if (src == NULL || out_q == NULL || out_scales == NULL) return ORC_ERR_INVALID_ARG;
  uint64_t gs;
  const int32_t st = orc_quant_group_size(s, n, &gs);
  if (st != ORC_OK) return st;
  const int32_t qmax = s->bit_width == 8u ? 127 : 7;
  memset(out_q, 0, (size_t)orc_quant_value_bytes(n, s));
  uint64_t g = 0;
  for (uint64_t t = 0; t < n; ++g, t += gs) {
    const uint64_t t1 = t + gs < n ? t + gs : n;
    float max_abs = 0.0f;
    for (uint64_t i = t; i < t1; ++i) {
      const float av = fabsf(src[i]);
      if (av > max_abs) max_abs = av;
    }
    const float scale = max_abs > 0.0f ? max_abs / (float)qmax : 0.0f;
    out_scales[g] = scale;
    for (uint64_t i = t; i < t1; ++i) {
      int32_t q = 0;
      if (scale > 0.0f) {
        q = (int32_t)lrintf(src[i] / scale);
        q = q > qmax ? qmax : (q < -qmax ? -qmax : q);
      }
      if (s->bit_width == 4u) {
        uint8_t *byte = (uint8_t *)out_q + i / 2u;
        const uint8_t nib = (uint8_t)(q & 0x0F);
        *byte = (i & 1u) == 0u ? (uint8_t)((*byte & 0xF0u) | nib) : (uint8_t)((*byte & 0x0Fu) | (nib << 4));
      } else {
        out_q[i] = (int8_t)q;
      }
    }
  }
  if (out_groups != NULL) *out_groups = g;
  return ORC_OK;
}

/* The signed 4-bit value of element `flat` of a nibble array (low nibble
 * for even indices; ref_ops.c:487-490, quantize.c:167-171). */
static inline int32_t nibble_at(const int8_t *q4, uint64_t flat) {
  const uint8_t byte = (uint8_t)q4[flat / 2u];
  const int32_t nib = (flat & 1u) == 0u ? (byte & 0x0F) : (byte >> 4);
  return (nib & 0x08) ? nib - 16 : nib;
}

/* models/quantize.c:143-181: out[i] = scale * (float)q */
int32_t orc_dequantize_v0_f32(const int8_t *q, const float *scales, uint64_t n,
                              const orc_quant_scheme_t *s, float *out) {
  if (q == NULL || scales == NULL || out == NULL) return ORC_ERR_INVALID_ARG;
  uint64_t gs;
  const int32_t st = orc_quant_group_size(s, n, &gs);
  if (st != ORC_OK) return st;
  uint64_t g = 0;
  for (uint64_t t = 0; t < n; ++g, t += gs) {
    const uint64_t t1 = t + gs < n ? t + gs : n;
    const float scale = scales[g];
    for (uint64_t i = t; i < t1; ++i)
      out[i] = scale * (float)(s->bit_width == 4u ? nibble_at(q, i) : (int32_t)q[i]);
  }
  return ORC_OK;
}

/* cpu/reference/ref_ops.c:446-468 (bits 8) and :470-499 (bits 4):
 * c[i][j] = sum over t ascending of (a[i][t] * q(t, j)) * scale[t/gs][j],
 * q(t, j) at flat index t*n+j; group size 0 or > k means one group. */
int32_t orc_gemm_wq_seq_f32(uint32_t bits, uint64_t m, uint64_t n, uint64_t k, const float *a,
                            const int8_t *w_q, const float *b_scales, uint64_t group_size,
                            float *c) {
  if (m == 0u || n == 0u || k == 0u || a == NULL || w_q == NULL || b_scales == NULL || c == NULL)
    return ORC_ERR_INVALID_ARG;
  if (bits != 8u && bits != 4u) return ORC_ERR_UNSUPPORTED;
  const uint64_t gs = (group_size == 0u || group_size > k) ? k : group_size;
  for (uint64_t i = 0; i < m; ++i) {
    for (uint64_t j = 0; j < n; ++j) {
      float sum = 0.0f;
      for (uint64_t t = 0; t < k; ++t) {
        const uint64_t flat = t * n + j;
        const int32_t qv = bits == 4u ? nibble_at(w_q, flat) : (int32_t)w_q[flat];
        sum += a[i * k + t] * (float)qv * b_scales[(t / gs) * n + j];
      }
      c[i * n + j] = sum;
    }
  }
  return ORC_OK;
}

/* The same sums in f64 (each term a[i][t] * q * scale exact in f64). */
int32_t orc_gemm_wq_f64(uint32_t bits, uint64_t m, uint64_t n, uint64_t k, const float *a,
                        const int8_t *w_q, const float *b_scales, uint64_t group_size,
                        double *c) {
  if (m == 0u || n == 0u || k == 0u || a == NULL || w_q == NULL || b_scales == NULL || c == NULL)
    return ORC_ERR_INVALID_ARG;
  if (bits != 8u && bits != 4u) return ORC_ERR_UNSUPPORTED;
  const uint64_t gs = (group_size == 0u || group_size > k) ? k : group_size;
  for (uint64_t i = 0; i < m; ++i) {
    for (uint64_t j = 0; j < n; ++j) {
      double sum = 0.0;
      for (uint64_t t = 0; t < k; ++t) {
        const uint64_t flat = t * n + j;
        const int32_t qv = bits == 4u ? nibble_at(w_q, flat) : (int32_t)w_q[flat];
        sum += (double)a[i * k + t] * (double)qv * (double)b_scales[(t / gs) * n + j];
      }
      c[i * n + j] = sum;
    }
  }
  return ORC_OK;
}

/* ---------------------------------------------------------------------- */
/* Textbook encoders (llama.cpp ggml-quants.c reference quantizers)         */
/* ---------------------------------------------------------------------- */

/* Q8_0: d = max|x|/127, q = round(x/d) (round half away from zero), d
 * stored as f16. Published llama.cpp quantize_row_q8_0_ref algorithm. */
void orc_q8_0_encode_ref(const float *x, uint8_t *out, uint64_t numel) {
  for (uint64_t b = 0; b < numel / 32u; ++b) {
    const float *v = x + 32u * b;
    uint8_t *o = out + 34u * b;
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) {
      amax = fmaxf(amax, fabsf(v[j]));
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = f32_to_f16_rne(d);
    o[0] = (uint8_t)(dh & 0xFF);
    o[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < 32; ++j) {
      o[2 + j] = (uint8_t)(int8_t)roundf(v[j] * id);
    }
  }
}

/* Q4_0: the signed value of largest magnitude m gives d = m / -8;
 * code = min(15, (int8)(x/d + 8.5)). Published llama.cpp
 * quantize_row_q4_0_ref algorithm. */
void orc_q4_0_encode_ref(const float *x, uint8_t *out, uint64_t numel) {
  for (uint64_t b = 0; b < numel / 32u; ++b) {
    const float *v = x + 32u * b;
    uint8_t *o = out + 18u * b;
    float amax = 0.0f, mx = 0.0f;
    for (int j = 0; j < 32; ++j) {
      if (fabsf(v[j]) > amax) {
        amax = fabsf(v[j]);
        mx = v[j];
      }
    }
    const float d = mx / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = f32_to_f16_rne(d);
    o[0] = (uint8_t)(dh & 0xFF);
    o[1] = (uint8_t)(dh >> 8);
    for (int j = 0; j < 16; ++j) {
      int c0 = (int)(int8_t)(v[j] * id + 8.5f);
      int c1 = (int)(int8_t)(v[j + 16] * id + 8.5f);
      c0 = c0 < 15 ? c0 : 15;
      c1 = c1 < 15 ? c1 : 15;
      o[2 + j] = (uint8_t)(c0 | (c1 << 4));
    }
  }
}

/* ---------------------------------------------------------------------- */
/* Decode step of the LLaMA graph                                           */
/* ---------------------------------------------------------------------- */

uint16_t orc_f32_to_f16(float v) { return f32_to_f16_rne(v); }

/* c = a * gamma * rms, rms = 1 / sqrtf((float)(sum a^2 / n) + eps), the
 * sum sequential in double; eps == 0 means 1e-5.
 * Follows cpu/reference/ref_ops.c:196-218. */
int32_t orc_rmsnorm_gamma_f32(const float *a, float *c, uint64_t n, const float *gamma,
                              float eps) {
  if (n == 0u || a == NULL || c == NULL || gamma == NULL) {
    return ORC_ERR_INVALID_ARG;
  }
  if (eps == 0.0f) {
    eps = 1e-5f;
  }
  double acc = 0.0;
  for (uint64_t i = 0; i < n; ++i) {
    acc += (double)a[i] * (double)a[i];
  }
  const float rms = 1.0f / sqrtf((float)(acc / (double)n) + eps);
  for (uint64_t i = 0; i < n; ++i) {
    c[i] = a[i] * gamma[i] * rms;
  }
  return ORC_OK;
}

/* Rotary embedding of `rows` rows of hd floats, position-major
 * (row = p * heads + h): pairs (i, i + r2) of position p's row rotated by
 * cos_t/sin_t[p * r2 + i]; columns from 2 r2 on are copied.
 * Follows cpu/reference/ref_ops.c:231-256. */
int32_t orc_rope_f32(const float *x, uint64_t rows, uint64_t hd, uint64_t seq, uint64_t heads,
                     const float *cos_t, const float *sin_t, uint64_t r2, float *out) {
  if (rows == 0u || hd == 0u || seq == 0u || heads == 0u || r2 == 0u || 2u * r2 > hd ||
      rows % heads != 0u || x == NULL || out == NULL || cos_t == NULL || sin_t == NULL) {
    return ORC_ERR_INVALID_ARG;
  }
  for (uint64_t row = 0; row < rows; ++row) {
    const uint64_t p = row / heads;
    const float *xr = x + row * hd;
    float *o = out + row * hd;
    for (uint64_t i = 0; i < r2; ++i) {
      const float c = cos_t[p * r2 + i], s = sin_t[p * r2 + i];
      const float x0 = xr[i], x1 = xr[i + r2];
      o[i] = x0 * c - x1 * s;
      o[i + r2] = x0 * s + x1 * c;
    }
    for (uint64_t i = 2u * r2; i < hd; ++i) {
      o[i] = xr[i];
    }
  }
  return ORC_OK;
}

/* The adapter's RoPE tables for positions 0..ctx-1:
 * freq_i = powf(theta, -(float)(2 i) / (float)n_rot),
 * cos_t[p][i] = cosf((float)p * freq_i), sin_t[p][i] = sinf(...).
 * Follows adapters/llama/llama.c:855-861. */
void orc_rope_tables_llama(uint32_t ctx, uint32_t r2, uint32_t n_rot, float theta, float *cos_t,
                           float *sin_t) {
  for (uint32_t p = 0; p < ctx; ++p) {
    for (uint32_t i = 0; i < r2; ++i) {
      const float freq = powf(theta, -(float)(2u * i) / (float)n_rot);
      cos_t[(uint64_t)p * r2 + i] = cosf((float)p * freq);
      sin_t[(uint64_t)p * r2 + i] = sinf((float)p * freq);
    }
  }
}

/* One (query, head) row of causal attention over keys/values 0..p, each
 * key/value row given by a pointer function of its position. */
static void attention_row(const float *qp, uint64_t p, uint64_t hd, float inv_scale,
                          const float *kbase, const float *vbase, uint64_t stride, float *scores,
                          float *op) {
  for (uint64_t i = 0; i <= p; ++i) {
    const float *kp = kbase + i * stride;
    float dot = 0.0f;
    for (uint64_t d = 0; d < hd; ++d) {
      dot += qp[d] * kp[d];
    }
    scores[i] = dot * inv_scale;
  }
  float maxv = scores[0];
  for (uint64_t i = 1; i <= p; ++i) {
    if (scores[i] > maxv) {
      maxv = scores[i];
    }
  }
  float sum = 0.0f;
  for (uint64_t i = 0; i <= p; ++i) {
    const float e = expf(scores[i] - maxv);
    scores[i] = e;
    sum += e;
  }
  for (uint64_t i = 0; i <= p; ++i) {
    scores[i] /= sum;
  }
  for (uint64_t d = 0; d < hd; ++d) {
    float acc = 0.0f;
    for (uint64_t i = 0; i <= p; ++i) {
      acc += scores[i] * vbase[i * stride + d];
    }
    op[d] = acc;
  }
}

/* Causal multi-head attention, position-major buffers: q, out [seq][h][hd],
 * k, v [seq][hk][hd]; head hh reads KV head (hh * hk) / h.
 * Follows cpu/reference/ref_ops.c:287-350. */
int32_t orc_attention_f32(uint64_t h, uint64_t hk, uint64_t seq, uint64_t hd, const float *q,
                          const float *k, const float *v, float *out) {
  if (h == 0u || hk == 0u || seq == 0u || hd == 0u || h % hk != 0u || q == NULL || k == NULL ||
      v == NULL || out == NULL) {
    return ORC_ERR_INVALID_ARG;
  }
  float *scores = (float *)malloc((size_t)seq * sizeof(float));
  if (scores == NULL) {
    return ORC_ERR_NOMEM;
  }
  const float inv_scale = 1.0f / sqrtf((float)hd);
  for (uint64_t p = 0; p < seq; ++p) {
    for (uint64_t hh = 0; hh < h; ++hh) {
      const uint64_t kvh = (hh * hk) / h;
      attention_row(q + (p * h + hh) * hd, p, hd, inv_scale, k + kvh * hd, v + kvh * hd, hk * hd,
                    scores, out + (p * h + hh) * hd);
    }
  }
  free(scores);
  return ORC_OK;
}

/* The last row (position len - 1) of orc_attention_f32, with keys and
 * values read from caches laid out [hk][ctx][hd]. q, out: [h][hd]. */
int32_t orc_attention_last_f32(uint64_t h, uint64_t hk, uint64_t ctx, uint64_t len, uint64_t hd,
                               const float *q, const float *k_cache, const float *v_cache,
                               float *out) {
  if (h == 0u || hk == 0u || len == 0u || len > ctx || hd == 0u || h % hk != 0u || q == NULL ||
      k_cache == NULL || v_cache == NULL || out == NULL) {
    return ORC_ERR_INVALID_ARG;
  }
  float *scores = (float *)malloc((size_t)len * sizeof(float));
  if (scores == NULL) {
    return ORC_ERR_NOMEM;
  }
  const float inv_scale = 1.0f / sqrtf((float)hd);
  for (uint64_t hh = 0; hh < h; ++hh) {
    const uint64_t kvh = (hh * hk) / h;
    attention_row(q + hh * hd, len - 1u, hd, inv_scale, k_cache + kvh * ctx * hd,
                  v_cache + kvh * ctx * hd, hd, scores, out + hh * hd);
  }
  free(scores);
  return ORC_OK;
}

/* Greedy pick: best = x[0], then i replaces it when x[i] > best.
 * Follows models/sampler.c:146-155. */
uint32_t orc_argmax_first(const float *x, uint64_t n) {
  float best = x[0];
  uint32_t chosen = 0;
  for (uint64_t i = 1; i < n; ++i) {
    if (x[i] > best) {
      best = x[i];
      chosen = (uint32_t)i;
    }
  }
  return chosen;
}

/* y[j] = sum_l x[l] * w[j][l], sequential f32: pai_ref_gemm_f32
 * (cpu/reference/ref_ops.c:427-444) on the transposed weight
 * (adapters/llama/llama.c:196-209) for one row of activations. */
static void gemv_seq(const float *w, uint64_t n, uint64_t k, const float *x, float *y) {
  for (uint64_t j = 0; j < n; ++j) {
    float acc = 0.0f;
    for (uint64_t l = 0; l < k; ++l) {
      acc += x[l] * w[j * k + l];
    }
    y[j] = acc;
  }
}

/* One decode position of the adapter's graph (adapters/llama/llama.c:
 * 499-800, the last row of a sequence-mode run, models/model.c:453-507),
 * with the keys and values of earlier positions read from m's caches and
 * this position's appended to them (rounded to fp16 when m->kv_f16). */
int32_t orc_llama_step(const orc_llama_t *m, uint32_t token, uint32_t pos, float *logits,
                       uint32_t *next) {
  if (m == NULL || logits == NULL || next == NULL || token >= m->vocab || pos >= m->ctx ||
      m->n_head == 0u || m->n_head_kv == 0u || m->n_embd % m->n_head != 0u) {
    return ORC_ERR_INVALID_ARG;
  }
  const uint64_t E = m->n_embd, F = m->n_ff, H = m->n_head, HK = m->n_head_kv;
  const uint64_t hd = E / H, kvd = HK * hd;
  uint32_t n_rot = m->n_rot;
  if (n_rot == 0u || n_rot > hd || (n_rot & 1u) != 0u) {
    n_rot = (uint32_t)hd; /* adapters/llama/llama.c:372-375 */
  }
  const uint32_t r2 = n_rot / 2u;
  const float theta = m->rope_theta != 0.0f ? m->rope_theta : 10000.0f;
  const uint64_t nf = 5u * E + 3u * E + 2u * kvd + 3u * F + 2u * r2;
  float *buf = (float *)malloc(nf * sizeof(float));
  float *cs = (float *)malloc((size_t)(pos + 1u) * r2 * 2u * sizeof(float));
  if (buf == NULL || cs == NULL) {
    free(buf);
    free(cs);
    return ORC_ERR_NOMEM;
  }
  float *x = buf, *xn = x + E, *o = xn + E, *t = o + E, *a = t + E, *q = a + E, *qr = q + E;
  float *kr = qr + E, *k = kr + E, *v = k + kvd, *g = v + kvd, *u = g + F, *hh = u + F;
  float *cos_t = cs, *sin_t = cs + (size_t)(pos + 1u) * r2;
  orc_rope_tables_llama(pos + 1u, r2, n_rot, theta, cos_t, sin_t);
  /* the rope ops of this position read the tables at row pos */
  const float *cp = cos_t + (size_t)pos * r2, *sp = sin_t + (size_t)pos * r2;

  memcpy(x, m->token_embd + (size_t)token * E, E * sizeof(float)); /* one-hot GEMM */
  for (uint32_t l = 0; l < m->n_layer; ++l) {
    const float *const *w = m->w + (size_t)l * 7u;
    orc_rmsnorm_gamma_f32(x, xn, E, m->attn_norm + (size_t)l * E, m->norm_eps);
    gemv_seq(w[0], E, E, xn, q);
    gemv_seq(w[1], kvd, E, xn, k);
    gemv_seq(w[2], kvd, E, xn, v);
    orc_rope_f32(q, H, hd, 1u, H, cp, sp, r2, qr);
    orc_rope_f32(k, HK, hd, 1u, HK, cp, sp, r2, kr);
    float *kc = m->k_cache + (size_t)l * HK * m->ctx * hd;
    float *vc = m->v_cache + (size_t)l * HK * m->ctx * hd;
    for (uint64_t h = 0; h < HK; ++h) {
      for (uint64_t d = 0; d < hd; ++d) {
        float kv = kr[h * hd + d], vv = v[h * hd + d];
        if (m->kv_f16) {
          kv = orc_f16_to_f32(f32_to_f16_rne(kv));
          vv = orc_f16_to_f32(f32_to_f16_rne(vv));
        }
        kc[(h * m->ctx + pos) * hd + d] = kv;
        vc[(h * m->ctx + pos) * hd + d] = vv;
      }
    }
    orc_attention_last_f32(H, HK, m->ctx, pos + 1u, hd, qr, kc, vc, a);
    gemv_seq(w[3], E, E, a, o);
    for (uint64_t i = 0; i < E; ++i) {
      x[i] = x[i] + o[i]; /* pai_ref_vecadd_f32 */
    }
    orc_rmsnorm_gamma_f32(x, xn, E, m->ffn_norm + (size_t)l * E, m->norm_eps);
    gemv_seq(w[4], F, E, xn, g);
    gemv_seq(w[5], F, E, xn, u);
    orc_silu_mul_f32(g, u, hh, F);
    gemv_seq(w[6], E, F, hh, t);
    for (uint64_t i = 0; i < E; ++i) {
      x[i] = x[i] + t[i];
    }
  }
  orc_rmsnorm_gamma_f32(x, xn, E, m->output_norm, m->norm_eps);
  gemv_seq(m->output, m->vocab, E, xn, logits);
  *next = orc_argmax_first(logits, m->vocab);
  free(buf);
  free(cs);
  return ORC_OK;
}
