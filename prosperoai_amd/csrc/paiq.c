/*
 * GGUF block encoders (Q8_0, Q4_0, Q4_K, Q6_K), f16 conversions and the
 * seeded normal generator. Host C11, no GPU calls. See include/paiq.h.
 *
 * Block layouts are the ones pai_gguf_dequant reads
 * (adapters/llama/gguf.c:680-694 Q4_0, :750-761 Q8_0, :852-882 Q4_K,
 * :920-947 Q6_K); the encoders write exactly those bytes.
 */
#define _GNU_SOURCE
#include "paiq.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

/* ---------------------------------------------------------------------- */
/* f16                                                                      */
/* ---------------------------------------------------------------------- */

uint16_t paiq_f32_to_f16(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t mag = u & 0x7FFFFFFFu;
  if (mag > 0x7F800000u) {
    return (uint16_t)(sign | 0x7E00u); /* quiet NaN */
  }
  if (mag >= 0x477FF000u) {
    return (uint16_t)(sign | 0x7C00u); /* overflow (and inf) */
  }
  if (mag < 0x33000001u) {
    return sign; /* |v| <= 2^-25 rounds to zero (ties to even = 0) */
  }
  int32_t exp = (int32_t)(mag >> 23) - 127;
  uint32_t sig = (mag & 0x7FFFFFu) | 0x800000u; /* 24-bit significand */
  uint32_t shift;                               /* bits to drop */
  uint32_t base;
  if (exp < -14) {
    /* subnormal half: units of 2^-24 */
    shift = (uint32_t)(13 + (-14 - exp));
    base = 0u;
  } else {
    shift = 13u;
    base = (uint32_t)(exp + 15) << 10;
    sig &= 0x7FFFFFu;
  }
  uint32_t keep = sig >> shift;
  const uint32_t rem = sig & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1u);
  if (rem > half || (rem == half && (keep & 1u))) {
    keep += 1u;
  }
  /* For normals a mantissa carry bumps the exponent through the add;
   * for subnormals keep == 1024 is exactly the smallest normal. */
  return (uint16_t)(sign | (base + keep));
}

float paiq_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  const uint32_t man = h & 0x3FFu;
  uint32_t u;
  if (exp == 0u) {
    /* zero or subnormal: man * 2^-24, exact in f32 */
    const float f = (float)man * 5.9604644775390625e-08f;
    memcpy(&u, &f, 4);
    u |= sign;
  } else if (exp == 31u) {
    u = sign | 0x7F800000u | (man << 13);
  } else {
    u = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float out;
  memcpy(&out, &u, 4);
  return out;
}

static void put_f16(uint8_t *p, float v) {
  const uint16_t h = paiq_f32_to_f16(v);
  p[0] = (uint8_t)(h & 0xFFu);
  p[1] = (uint8_t)(h >> 8);
}

static float rt_f16(float v) { return paiq_f16_to_f32(paiq_f32_to_f16(v)); }

static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* ---------------------------------------------------------------------- */
/* Per-block encoders                                                       */
/* ---------------------------------------------------------------------- */

/* Q8_0: d = max|x| / 127; code = round(x / d) (half away from zero). */
static void enc_q8_0(const float *x, uint8_t *o) {
  float amax = 0.0f;
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
  const float d = amax / 127.0f;
  const float inv = d != 0.0f ? 1.0f / d : 0.0f;
  put_f16(o, d);
  for (int j = 0; j < 32; ++j) o[2 + j] = (uint8_t)(int8_t)roundf(x[j] * inv);
}

/* Q4_0: the signed extreme m maps to code 0 (d = m / -8);
 * code = min(15, trunc(x / d + 8.5)). */
static void enc_q4_0(const float *x, uint8_t *o) {
  float amax = 0.0f, ext = 0.0f;
  for (int j = 0; j < 32; ++j) {
    if (fabsf(x[j]) > amax) {
      amax = fabsf(x[j]);
      ext = x[j];
    }
  }
  const float d = ext / -8.0f;
  const float inv = d != 0.0f ? 1.0f / d : 0.0f;
  put_f16(o, d);
  for (int j = 0; j < 16; ++j) {
    const int lo = clampi((int)(int8_t)(x[j] * inv + 8.5f), 0, 15);
    const int hi = clampi((int)(int8_t)(x[j + 16] * inv + 8.5f), 0, 15);
    o[2 + j] = (uint8_t)(lo | (hi << 4));
  }
}

/* Q4_K: eight 32-element sub-blocks, value = d*sc_j*q - dmin*m_j with
 * q in [0,15], sc_j, m_j 6-bit. Each sub-block's range [lo, hi] (lo
 * clipped to <= 0) gives step (hi-lo)/15 and offset -lo; the steps and
 * offsets are quantized against d = max step / 63 and dmin = max offset
 * / 63 (both stored f16), then the codes are refit to the stored scales. */
static void enc_q4_k(const float *x, uint8_t *o) {
  float step[8], off[8];
  float smax = 0.0f, omax = 0.0f;
  for (int j = 0; j < 8; ++j) {
    float lo = 0.0f, hi = -INFINITY;
    for (int l = 0; l < 32; ++l) {
      lo = fminf(lo, x[32 * j + l]);
      hi = fmaxf(hi, x[32 * j + l]);
    }
    if (hi < lo) hi = lo;
    step[j] = (hi - lo) / 15.0f;
    off[j] = -lo;
    smax = fmaxf(smax, step[j]);
    omax = fmaxf(omax, off[j]);
  }
  const float d = rt_f16(smax / 63.0f);
  const float dmin = rt_f16(omax / 63.0f);
  put_f16(o, smax / 63.0f);
  put_f16(o + 2, omax / 63.0f);
  uint8_t sc[8], mn[8];
  for (int j = 0; j < 8; ++j) {
    sc[j] = (uint8_t)(d > 0.0f ? clampi((int)lrintf(step[j] / d), 0, 63) : 0);
    mn[j] = (uint8_t)(dmin > 0.0f ? clampi((int)lrintf(off[j] / dmin), 0, 63) : 0);
  }
  /* 12-byte packing, the inverse of the 6-bit unpack in
   * adapters/llama/gguf.c:639-648. */
  uint8_t *s = o + 4;
  for (int j = 0; j < 4; ++j) {
    s[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
    s[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
    s[j + 8] = (uint8_t)((sc[j + 4] & 0x0F) | ((mn[j + 4] & 0x0F) << 4));
  }
  uint8_t code[256];
  for (int j = 0; j < 8; ++j) {
    const float st = d * (float)sc[j];
    const float mo = dmin * (float)mn[j];
    for (int l = 0; l < 32; ++l) {
      code[32 * j + l] =
          (uint8_t)(st > 0.0f ? clampi((int)lrintf((x[32 * j + l] + mo) / st), 0, 15) : 0);
    }
  }
  /* byte 32c+l: element 64c+l in the low nibble, 64c+32+l in the high */
  for (int c = 0; c < 4; ++c) {
    for (int l = 0; l < 32; ++l) {
      o[16 + 32 * c + l] = (uint8_t)(code[64 * c + l] | (code[64 * c + 32 + l] << 4));
    }
  }
}

/* Q6_K: sixteen 16-element sub-blocks, value = d*sc_j*(q-32), q in
 * [0,63], sc_j int8. Each sub-block's signed extreme e gives scale
 * e / -32; the scales are quantized against d = max|scale| / 127 (f16),
 * then the codes are refit to the stored scales. */
static void enc_q6_k(const float *x, uint8_t *o) {
  float scl[16];
  float amax_s = 0.0f;
  for (int j = 0; j < 16; ++j) {
    float amax = 0.0f, ext = 0.0f;
    for (int l = 0; l < 16; ++l) {
      if (fabsf(x[16 * j + l]) > amax) {
        amax = fabsf(x[16 * j + l]);
        ext = x[16 * j + l];
      }
    }
    scl[j] = ext / -32.0f;
    amax_s = fmaxf(amax_s, fabsf(scl[j]));
  }
  const float d = rt_f16(amax_s / 127.0f);
  int8_t sc[16];
  for (int j = 0; j < 16; ++j) {
    sc[j] = (int8_t)(d > 0.0f ? clampi((int)lrintf(scl[j] / d), -127, 127) : 0);
  }
  uint8_t code[256];
  for (int j = 0; j < 16; ++j) {
    const float st = d * (float)sc[j];
    for (int l = 0; l < 16; ++l) {
      const int q = st != 0.0f ? clampi((int)lrintf(x[16 * j + l] / st), -32, 31) : 0;
      code[16 * j + l] = (uint8_t)(q + 32);
    }
  }
  /* ql[128] | qh[64] | sc[16] | d, per adapters/llama/gguf.c:920-947 */
  uint8_t *ql = o, *qh = o + 128;
  memset(o, 0, 192);
  for (int h = 0; h < 2; ++h) {
    for (int l = 0; l < 32; ++l) {
      const uint8_t c0 = code[128 * h + l], c1 = code[128 * h + 32 + l];
      const uint8_t c2 = code[128 * h + 64 + l], c3 = code[128 * h + 96 + l];
      ql[64 * h + l] = (uint8_t)((c0 & 0x0F) | ((c2 & 0x0F) << 4));
      ql[64 * h + 32 + l] = (uint8_t)((c1 & 0x0F) | ((c3 & 0x0F) << 4));
      qh[32 * h + l] = (uint8_t)((c0 >> 4) | ((c1 >> 4) << 2) | ((c2 >> 4) << 4) | ((c3 >> 4) << 6));
    }
  }
  memcpy(o + 192, sc, 16);
  put_f16(o + 208, amax_s / 127.0f);
}

/* ---------------------------------------------------------------------- */
/* Row-parallel driver                                                      */
/* ---------------------------------------------------------------------- */

typedef struct {
  uint32_t type;
  const float *src;
  uint8_t *dst;
  uint64_t k, row_bytes, r0, r1;
} enc_job_t;

static void *enc_rows(void *arg) {
  const enc_job_t *j = (const enc_job_t *)arg;
  const uint64_t qk = (j->type == PAI_QTYPE_Q4_K || j->type == PAI_QTYPE_Q6_K) ? 256u : 32u;
  const uint64_t bb = pai_qtype_bytes(j->type, qk);
  for (uint64_t r = j->r0; r < j->r1; ++r) {
    const float *x = j->src + r * j->k;
    uint8_t *o = j->dst + r * j->row_bytes;
    for (uint64_t b = 0; b < j->k / qk; ++b) {
      switch (j->type) {
      case PAI_QTYPE_Q8_0: enc_q8_0(x + qk * b, o + bb * b); break;
      case PAI_QTYPE_Q4_0: enc_q4_0(x + qk * b, o + bb * b); break;
      case PAI_QTYPE_Q4_K: enc_q4_k(x + qk * b, o + bb * b); break;
      case PAI_QTYPE_Q6_K: enc_q6_k(x + qk * b, o + bb * b); break;
      default: break;
      }
    }
  }
  return NULL;
}

static int host_threads(int threads) {
  if (threads > 0) return threads > 64 ? 64 : threads;
  long n = sysconf(_SC_NPROCESSORS_ONLN);
  if (n < 1) n = 1;
  return n > 16 ? 16 : (int)n;
}

pai_status_t paiq_quantize(uint32_t type, const float *src, uint64_t rows,
                           uint64_t k, void *out, uint64_t out_bytes,
                           int threads) {
  if (src == NULL || out == NULL || rows == 0u || k == 0u) {
    return PAI_ERR_INVALID_ARG;
  }
  const uint64_t row_bytes = pai_qtype_bytes(type, k);
  if (row_bytes == 0u) {
    return PAI_ERR_UNSUPPORTED;
  }
  if (out_bytes != rows * row_bytes) {
    return PAI_ERR_MISMATCH;
  }
  int nt = host_threads(threads);
  if ((uint64_t)nt > rows) nt = (int)rows;
  pthread_t tid[64];
  enc_job_t job[64];
  int started[64];
  for (int t = 0; t < nt; ++t) {
    job[t] = (enc_job_t){type, src, (uint8_t *)out, k, row_bytes,
                         rows * (uint64_t)t / (uint64_t)nt,
                         rows * (uint64_t)(t + 1) / (uint64_t)nt};
    started[t] = (nt > 1) && pthread_create(&tid[t], NULL, enc_rows, &job[t]) == 0;
    if (!started[t]) enc_rows(&job[t]);
  }
  for (int t = 0; t < nt; ++t) {
    if (started[t]) pthread_join(tid[t], NULL);
  }
  return PAI_OK;
}

/* ---------------------------------------------------------------------- */
/* Seeded N(mean, std^2)                                                    */
/* ---------------------------------------------------------------------- */

/* Output i of a splitmix64 stream seeded with `seed` (counter form:
 * state_i = seed + (i+1) * golden gamma), so ranges can be generated in
 * parallel and still equal the sequential stream. */
static uint64_t splitmix_at(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1u) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

typedef struct {
  uint64_t seed, p0, p1, n;
  float mean, std;
  float *out;
} rng_job_t;

static void *rng_pairs(void *arg) {
  const rng_job_t *j = (const rng_job_t *)arg;
  const double two_pi = 6.283185307179586476925286766559;
  for (uint64_t p = j->p0; p < j->p1; ++p) {
    /* uniforms in (0, 1]: never log(0) */
    const double u1 = (double)((splitmix_at(j->seed, 2u * p) >> 11) + 1u) * 0x1.0p-53;
    const double u2 = (double)((splitmix_at(j->seed, 2u * p + 1u) >> 11) + 1u) * 0x1.0p-53;
    const double r = sqrt(-2.0 * log(u1));
    const double z0 = r * cos(two_pi * u2), z1 = r * sin(two_pi * u2);
    j->out[2u * p] = (float)((double)j->mean + (double)j->std * z0);
    if (2u * p + 1u < j->n) {
      j->out[2u * p + 1u] = (float)((double)j->mean + (double)j->std * z1);
    }
  }
  return NULL;
}

void paiq_normal_f32(uint64_t seed, float mean, float std, float *out, uint64_t n) {
  if (out == NULL || n == 0u) return;
  const uint64_t pairs = (n + 1u) / 2u;
  int nt = pairs < (1u << 16) ? 1 : host_threads(0);
  pthread_t tid[64];
  rng_job_t job[64];
  int started[64];
  for (int t = 0; t < nt; ++t) {
    job[t] = (rng_job_t){seed, pairs * (uint64_t)t / (uint64_t)nt,
                         pairs * (uint64_t)(t + 1) / (uint64_t)nt, n, mean, std, out};
    started[t] = (nt > 1) && pthread_create(&tid[t], NULL, rng_pairs, &job[t]) == 0;
    if (!started[t]) rng_pairs(&job[t]);
  }
  for (int t = 0; t < nt; ++t) {
    if (started[t]) pthread_join(tid[t], NULL);
  }
}
