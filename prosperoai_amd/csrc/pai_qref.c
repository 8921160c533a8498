/*
 * CPU twin of the quantized matmul (host C11): the operator the qgemm_*
 * registry descriptors carry as their CPU reference implementation, with
 * PAI_OP_CAP_CPU_REF. The reference's executor and plan checks require
 * that capability of every op they run (scheduler/scheduler.c:720-756);
 * the GPU entry points of this library never call this code.
 *
 * It computes what the reference computes for a GGUF weight today: the
 * blocks dequantized to f32 (adapters/llama/gguf.c:601-947, the same
 * operations in the same order), then pai_ref_gemm_f32's sequential f32
 * sum (cpu/reference/ref_ops.c:427-444) over the transposed weights, so
 * its results equal that composition bit for bit. The dequantization runs
 * one block at a time into a stack buffer and the sums accumulate in y, so
 * nothing is allocated. Built without floating-point contraction.
 *
 * The twins of the v0 GEMMs (pai_ref_gemm_w8_f32 / _w4_f32,
 * cpu/reference/ref_ops.c:446-499) follow at the end.
 */
#include <stdint.h>
#include <string.h>

#include "pai_hip.h"

/* IEEE binary16 -> binary32, exact; a NaN keeps its payload (the
 * reference's bit construction, gguf.c:601-630). */
static float half_bits_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, f = h & 0x3FFu;
  uint32_t bits;
  if (e == 0u) {
    /* zero or subnormal: f * 2^-24 is exact in binary32 */
    const float mag = (float)f * 5.9604644775390625e-08f;
    memcpy(&bits, &mag, 4);
    bits |= sign;
  } else if (e == 31u) {
    bits = sign | 0x7F800000u | (f << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (f << 13);
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

static float half_at(const uint8_t *p) {
  return half_bits_to_float((uint16_t)(p[0] | (p[1] << 8)));
}

/* 6-bit scale and min of sub-block j of a Q4_K super-block from its 12
 * packed bytes (the format's bit fields, gguf.c:639-648). */
static void k4_scale_min(int j, const uint8_t *p, float d, float dmin, float *d1, float *m1) {
  uint32_t s, m;
  if (j < 4) {
    s = p[j] & 63u;
    m = p[j + 4] & 63u;
  } else {
    s = (p[j + 4] & 0x0Fu) | ((uint32_t)(p[j - 4] >> 6) << 4);
    m = (uint32_t)(p[j + 4] >> 4) | ((uint32_t)(p[j] >> 6) << 4);
  }
  *d1 = d * (float)s;
  *m1 = dmin * (float)m;
}

/* One block of `type` as f32 values in element order. */
static void block_values(uint32_t type, const uint8_t *b, float *o) {
  switch (type) {
  case PAI_QTYPE_Q4_0: { /* f16 d, 16 bytes of nibbles: low = 0..15, high = 16..31 */
    const float d = half_at(b);
    for (int j = 0; j < 16; ++j) {
      o[j] = (float)((int)(b[2 + j] & 0x0Fu) - 8) * d;
      o[j + 16] = (float)((int)(b[2 + j] >> 4) - 8) * d;
    }
    break;
  }
  case PAI_QTYPE_Q8_0: { /* f16 d, 32 int8 codes */
    const float d = half_at(b);
    for (int j = 0; j < 32; ++j) o[j] = (float)(int8_t)b[2 + j] * d;
    break;
  }
  case PAI_QTYPE_Q4_K: { /* f16 d, f16 dmin, 12 scale bytes, 128 bytes of nibbles */
    const float d = half_at(b), dmin = half_at(b + 2);
    for (int c = 0; c < 4; ++c) {
      const uint8_t *q = b + 16 + 32 * c;
      float d1, m1, d2, m2;
      k4_scale_min(2 * c, b + 4, d, dmin, &d1, &m1);
      k4_scale_min(2 * c + 1, b + 4, d, dmin, &d2, &m2);
      for (int l = 0; l < 32; ++l) o[64 * c + l] = d1 * (float)(q[l] & 0x0Fu) - m1;
      for (int l = 0; l < 32; ++l) o[64 * c + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
    }
    break;
  }
  case PAI_QTYPE_Q6_K: { /* 128 low-nibble bytes, 64 high-bit bytes, 16 int8 scales, f16 d */
    const float d = half_at(b + 208);
    for (int h = 0; h < 2; ++h) {
      const uint8_t *ql = b + 64 * h, *qh = b + 128 + 32 * h;
      const int8_t *sc = (const int8_t *)(b + 192 + 8 * h);
      float *oh = o + 128 * h;
      for (int l = 0; l < 32; ++l) {
        const int g = l / 16;
        const int q1 = (int)((ql[l] & 0x0Fu) | ((qh[l] & 3u) << 4)) - 32;
        const int q2 = (int)((ql[l + 32] & 0x0Fu) | (((qh[l] >> 2) & 3u) << 4)) - 32;
        const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3u) << 4)) - 32;
        const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3u) << 4)) - 32;
        oh[l] = d * (float)sc[g] * (float)q1;
        oh[l + 32] = d * (float)sc[g + 2] * (float)q2;
        oh[l + 64] = d * (float)sc[g + 4] * (float)q3;
        oh[l + 96] = d * (float)sc[g + 6] * (float)q4;
      }
    }
    break;
  }
  default:
    break;
  }
}

static uint32_t block_elems(uint32_t type) {
  return type == PAI_QTYPE_Q4_0 || type == PAI_QTYPE_Q8_0   ? 32u
         : type == PAI_QTYPE_Q4_K || type == PAI_QTYPE_Q6_K ? 256u
                                                            : 0u;
}

pai_status_t pai_qgemm_ref_f32(uint32_t type, uint64_t m, uint64_t n, uint64_t k, const float *x,
                               const void *blocks, float *y) {
  if (x == NULL || blocks == NULL || y == NULL || m == 0u || n == 0u || k == 0u)
    return PAI_ERR_INVALID_ARG;
  const uint32_t qk = block_elems(type);
  if (qk == 0u || k % qk != 0u) return PAI_ERR_UNSUPPORTED;
  const uint64_t bb = pai_qtype_bytes(type, qk), nb = k / qk;
  const uint8_t *w = (const uint8_t *)blocks;
  float vals[256];
  for (uint64_t j = 0; j < n; ++j) {
    for (uint64_t i = 0; i < m; ++i) y[i * n + j] = 0.0f;
    for (uint64_t b = 0; b < nb; ++b) {
      block_values(type, w + (j * nb + b) * bb, vals);
      /* y[i][j] = sum over l of x[i][l] * W[j][l], l ascending: the
       * reference's running sum, kept in y */
      for (uint64_t i = 0; i < m; ++i) {
        const float *xi = x + i * k + b * qk;
        float s = y[i * n + j];
        for (uint32_t l = 0; l < qk; ++l) s += xi[l] * vals[l];
        y[i * n + j] = s;
      }
    }
  }
  return PAI_OK;
}

/* Code (t, j) of a [K][N] operand: int8, or the sign-extended nibble at
 * flat index t*n+j (low nibble for even indices). */
static int32_t wq_code(uint32_t bits, const int8_t *w, uint64_t flat) {
  if (bits == 8u) return w[flat];
  const uint8_t byte = (uint8_t)w[flat / 2u];
  const int32_t nib = (flat & 1u) == 0u ? (byte & 0x0F) : (byte >> 4);
  return (nib & 0x08) ? nib - 16 : nib;
}

/* c[i][j] = sum over t ascending of (a[i][t] * q(t, j)) * scale, the
 * reference's order and roundings. */
static pai_status_t gemm_wq_ref(uint32_t bits, uint64_t m, uint64_t n, uint64_t k, const float *a,
                                const int8_t *w, const float *b_scales, uint64_t group_size,
                                float *c) {
  if (m == 0u || n == 0u || k == 0u || a == NULL || w == NULL || b_scales == NULL || c == NULL)
    return PAI_ERR_INVALID_ARG;
  const uint64_t gs = (group_size == 0u || group_size > k) ? k : group_size;
  for (uint64_t i = 0; i < m; ++i) {
    for (uint64_t j = 0; j < n; ++j) {
      float sum = 0.0f;
      for (uint64_t t = 0; t < k; ++t)
        sum += a[i * k + t] * (float)wq_code(bits, w, t * n + j) * b_scales[(t / gs) * n + j];
      c[i * n + j] = sum;
    }
  }
  return PAI_OK;
}

pai_status_t pai_gemm_w8_ref_f32(uint64_t m, uint64_t n, uint64_t k, const float *a,
                                 const int8_t *w_q, const float *b_scales, uint64_t group_size,
                                 float *c) {
  return gemm_wq_ref(8u, m, n, k, a, w_q, b_scales, group_size, c);
}

pai_status_t pai_gemm_w4_ref_f32(uint64_t m, uint64_t n, uint64_t k, const float *a,
                                 const int8_t *w_q4, const float *b_scales, uint64_t group_size,
                                 float *c) {
  return gemm_wq_ref(4u, m, n, k, a, w_q4, b_scales, group_size, c);
}
