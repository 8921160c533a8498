/*
 * Host side of the v0 per-group formats (C11): argument checks with the
 * reference's error codes (cpu/reference/ref_ops.c:446-499,
 * models/quantize.c:6-181), and the launches of qv0.hip. No CPU fallback:
 * without a gfx950 device every entry point returns PAI_ERR_INIT.
 */
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <string.h>

#include "pai_hip.h"
#include "paik.h"

pai_status_t pai__map_hip(int e, const char *what);
pai_status_t pai__ready(void);
pai_status_t pai__fail(pai_status_t st, const char *fmt, ...);

#define V0_MAX_DIM 0x7FFFFFFFull
#define V0_TOKENS_PER_LAUNCH 65535u

static uint64_t v0_groups(uint64_t n, uint64_t gs) { return n / gs + (n % gs != 0u ? 1u : 0u); }

static int aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1u)) == 0u; }

pai_status_t pai_hip_gemm_wq_f32_async(uint32_t bits, uint64_t m, uint64_t n, uint64_t k,
                                       const float *a, const void *w_q, const float *b_scales,
                                       uint64_t group_size, float *c, void *workspace,
                                       uint64_t workspace_bytes, void *stream) {
  if (m == 0u || n == 0u || k == 0u || a == NULL || w_q == NULL || b_scales == NULL || c == NULL)
    return pai__fail(PAI_ERR_INVALID_ARG, "NULL argument or zero dimension");
  if (bits != 8u && bits != 4u) return pai__fail(PAI_ERR_UNSUPPORTED, "bits must be 8 or 4");
  if (m > V0_MAX_DIM || n > V0_MAX_DIM || k > V0_MAX_DIM)
    return pai__fail(PAI_ERR_UNSUPPORTED, "dimension above 2^31 - 1");
  if (!aligned(a, 4u) || !aligned(b_scales, 4u) || !aligned(c, 4u))
    return pai__fail(PAI_ERR_INVALID_ARG, "a, b_scales and c must be 4-byte aligned");
  pai_status_t st = pai__ready();
  if (st != PAI_OK) return st;
  const uint64_t gs = (group_size == 0u || group_size > k) ? k : group_size;
  paik_v0_gemm_t p;
  memset(&p, 0, sizeof p);
  p.wq = w_q;
  p.scales = b_scales;
  p.workspace = workspace;
  p.workspace_bytes = workspace != NULL ? workspace_bytes : 0u;
  p.bits = bits;
  p.n = (uint32_t)n;
  p.k = (uint32_t)k;
  p.gs = (uint32_t)gs;
  p.strip_ok = n % 16u == 0u && (gs == k || gs % 16u == 0u) && aligned(w_q, 16u) &&
               aligned(b_scales, 16u);
  p.sequential = paik_tune.v0_sequential != 0;
  for (uint64_t t0 = 0; t0 < m; t0 += V0_TOKENS_PER_LAUNCH) {
    p.m = (uint32_t)(m - t0 < V0_TOKENS_PER_LAUNCH ? m - t0 : V0_TOKENS_PER_LAUNCH);
    p.a = a + t0 * k;
    p.c = c + t0 * n;
    const int e = paik_v0_gemm(&p, stream);
    if (e != 0) return pai__map_hip(e, "v0 gemm launch");
  }
  return PAI_OK;
}

/* The host-pointer forms copy every operand to one device allocation. */
static pai_status_t gemm_host(uint32_t bits, uint64_t m, uint64_t n, uint64_t k, const float *a,
                              const int8_t *w_q, const float *b_scales, uint64_t group_size,
                              float *c) {
  if (m == 0u || n == 0u || k == 0u || a == NULL || w_q == NULL || b_scales == NULL || c == NULL)
    return pai__fail(PAI_ERR_INVALID_ARG, "NULL argument or zero dimension");
  if (m > V0_MAX_DIM || n > V0_MAX_DIM || k > V0_MAX_DIM)
    return pai__fail(PAI_ERR_UNSUPPORTED, "dimension above 2^31 - 1");
  pai_status_t st = pai__ready();
  if (st != PAI_OK) return st;
  const uint64_t gs = (group_size == 0u || group_size > k) ? k : group_size;
  const uint64_t ab = m * k * 4u, wb = bits == 8u ? k * n : (k * n + 1u) / 2u;
  const uint64_t sb = v0_groups(k, gs) * n * 4u, cb = m * n * 4u;
#define UP(v) (((v) + 255u) & ~(uint64_t)255u)
  const uint64_t oa = 0, ow = UP(ab), os = ow + UP(wb), oc = os + UP(sb), ows = oc + UP(cb);
  const uint64_t total = ows + PAI_HIP_WQ_WORKSPACE_BYTES;
#undef UP
  uint8_t *d = NULL;
  hipError_t e = hipMalloc((void **)&d, total);
  if (e != hipSuccess) return pai__map_hip((int)e, "hipMalloc(v0 gemm operands)");
  e = hipMemcpy(d + oa, a, ab, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(d + ow, w_q, wb, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(d + os, b_scales, sb, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    st = pai_hip_gemm_wq_f32_async(bits, m, n, k, (const float *)(d + oa), d + ow,
                                   (const float *)(d + os), group_size, (float *)(d + oc),
                                   d + ows, PAI_HIP_WQ_WORKSPACE_BYTES, NULL);
    if (st == PAI_OK) {
      e = hipMemcpy(c, d + oc, cb, hipMemcpyDeviceToHost);
      if (e != hipSuccess) st = pai__map_hip((int)e, "hipMemcpy(c)");
    }
  } else {
    st = pai__map_hip((int)e, "hipMemcpy(v0 gemm operands)");
  }
  (void)hipFree(d);
  return st;
}

pai_status_t pai_hip_gemm_w8_f32(uint64_t m, uint64_t n, uint64_t k, const float *a,
                                 const int8_t *w_q, const float *b_scales, uint64_t group_size,
                                 float *c) {
  return gemm_host(8u, m, n, k, a, w_q, b_scales, group_size, c);
}

pai_status_t pai_hip_gemm_w4_f32(uint64_t m, uint64_t n, uint64_t k, const float *a,
                                 const int8_t *w_q4, const float *b_scales, uint64_t group_size,
                                 float *c) {
  return gemm_host(4u, m, n, k, a, w_q4, b_scales, group_size, c);
}

/* models/quantize.c:6-26: INVALID_ARG for a NULL scheme or a zero group
 * size (n == 0 with one group), UNSUPPORTED for other bit widths or an
 * unsigned scheme. */
static pai_status_t scheme_group(const pai_hip_quant_scheme_t *s, uint64_t n, uint64_t *gs) {
  if (s == NULL) return pai__fail(PAI_ERR_INVALID_ARG, "NULL scheme");
  if (s->bit_width != 8u && s->bit_width != 4u)
    return pai__fail(PAI_ERR_UNSUPPORTED, "bit_width must be 8 or 4");
  if (!s->is_signed) return pai__fail(PAI_ERR_UNSUPPORTED, "v0 schemes are signed");
  *gs = s->group_size == 0u ? n : (uint64_t)s->group_size;
  if (*gs == 0u) return pai__fail(PAI_ERR_INVALID_ARG, "zero group size");
  return PAI_OK;
}

pai_status_t pai_hip_quantize_f32_async(const float *src, uint64_t n,
                                        const pai_hip_quant_scheme_t *scheme, int8_t *out_q,
                                        float *out_scales, uint64_t *out_num_groups,
                                        void *stream) {
  if (src == NULL || out_q == NULL || out_scales == NULL)
    return pai__fail(PAI_ERR_INVALID_ARG, "NULL argument");
  uint64_t gs;
  pai_status_t st = scheme_group(scheme, n, &gs);
  if (st != PAI_OK) return st;
  if (n > V0_MAX_DIM) return pai__fail(PAI_ERR_UNSUPPORTED, "n above 2^31 - 1");
  if (!aligned(out_q, 16u) || !aligned(src, 4u) || !aligned(out_scales, 4u))
    return pai__fail(PAI_ERR_INVALID_ARG, "out_q must be 16-byte aligned, src and scales 4");
  if (gs > n) gs = n > 0u ? n : gs; /* a group past the end holds the n elements */
  if (out_num_groups != NULL) *out_num_groups = n > 0u ? v0_groups(n, gs) : 0u;
  if (n == 0u) return PAI_OK;
  st = pai__ready();
  if (st != PAI_OK) return st;
  const int e = paik_v0_quantize(src, (uint32_t)n, scheme->bit_width, (uint32_t)gs, out_q,
                                 out_scales, stream);
  return e == 0 ? PAI_OK : pai__map_hip(e, "v0 quantize launch");
}

pai_status_t pai_hip_dequantize_f32_async(const int8_t *q, const float *scales, uint64_t n,
                                          const pai_hip_quant_scheme_t *scheme, float *out,
                                          void *stream) {
  if (q == NULL || scales == NULL || out == NULL)
    return pai__fail(PAI_ERR_INVALID_ARG, "NULL argument");
  uint64_t gs;
  pai_status_t st = scheme_group(scheme, n, &gs);
  if (st != PAI_OK) return st;
  if (n > V0_MAX_DIM) return pai__fail(PAI_ERR_UNSUPPORTED, "n above 2^31 - 1");
  if (!aligned(out, 16u) || !aligned(scales, 4u))
    return pai__fail(PAI_ERR_INVALID_ARG, "out must be 16-byte aligned, scales 4");
  if (n == 0u) return PAI_OK;
  if (gs > n) gs = n;
  st = pai__ready();
  if (st != PAI_OK) return st;
  const int e = paik_v0_dequantize(q, scales, (uint32_t)n, scheme->bit_width, (uint32_t)gs, out,
                                   stream);
  return e == 0 ? PAI_OK : pai__map_hip(e, "v0 dequantize launch");
}

pai_status_t pai_hip_quantize_f32(const float *src, uint64_t n,
                                  const pai_hip_quant_scheme_t *scheme, int8_t *out_q,
                                  float *out_scales, uint64_t *out_num_groups) {
  if (src == NULL || out_q == NULL || out_scales == NULL)
    return pai__fail(PAI_ERR_INVALID_ARG, "NULL argument");
  uint64_t gs;
  pai_status_t st = scheme_group(scheme, n, &gs);
  if (st != PAI_OK) return st;
  if (n > V0_MAX_DIM) return pai__fail(PAI_ERR_UNSUPPORTED, "n above 2^31 - 1");
  if (gs > n) gs = n > 0u ? n : gs;
  const uint64_t groups = n > 0u ? v0_groups(n, gs) : 0u;
  if (out_num_groups != NULL) *out_num_groups = groups;
  if (n == 0u) return PAI_OK;
  st = pai__ready();
  if (st != PAI_OK) return st;
  const uint64_t qb = scheme->bit_width == 8u ? n : (n + 1u) / 2u;
  const uint64_t xb = (n * 4u + 255u) & ~(uint64_t)255u, qbb = (qb + 255u) & ~(uint64_t)255u;
  uint8_t *d = NULL;
  hipError_t e = hipMalloc((void **)&d, xb + qbb + groups * 4u);
  if (e != hipSuccess) return pai__map_hip((int)e, "hipMalloc(v0 quantize)");
  e = hipMemcpy(d, src, n * 4u, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    st = pai_hip_quantize_f32_async((const float *)d, n, scheme, (int8_t *)(d + xb),
                                    (float *)(d + xb + qbb), NULL, NULL);
    if (st == PAI_OK) {
      e = hipMemcpy(out_q, d + xb, qb, hipMemcpyDeviceToHost);
      if (e == hipSuccess) e = hipMemcpy(out_scales, d + xb + qbb, groups * 4u,
                                         hipMemcpyDeviceToHost);
      if (e != hipSuccess) st = pai__map_hip((int)e, "hipMemcpy(v0 codes)");
    }
  } else {
    st = pai__map_hip((int)e, "hipMemcpy(v0 src)");
  }
  (void)hipFree(d);
  return st;
}

pai_status_t pai_hip_dequantize_f32(const int8_t *q, const float *scales, uint64_t n,
                                    const pai_hip_quant_scheme_t *scheme, float *out) {
  if (q == NULL || scales == NULL || out == NULL)
    return pai__fail(PAI_ERR_INVALID_ARG, "NULL argument");
  uint64_t gs;
  pai_status_t st = scheme_group(scheme, n, &gs);
  if (st != PAI_OK) return st;
  if (n > V0_MAX_DIM) return pai__fail(PAI_ERR_UNSUPPORTED, "n above 2^31 - 1");
  if (n == 0u) return PAI_OK;
  if (gs > n) gs = n;
  st = pai__ready();
  if (st != PAI_OK) return st;
  const uint64_t groups = v0_groups(n, gs);
  const uint64_t qb = scheme->bit_width == 8u ? n : (n + 1u) / 2u;
  const uint64_t ob = (n * 4u + 255u) & ~(uint64_t)255u, qbb = (qb + 255u) & ~(uint64_t)255u;
  uint8_t *d = NULL;
  hipError_t e = hipMalloc((void **)&d, ob + qbb + groups * 4u);
  if (e != hipSuccess) return pai__map_hip((int)e, "hipMalloc(v0 dequantize)");
  e = hipMemcpy(d + ob, q, qb, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(d + ob + qbb, scales, groups * 4u, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    st = pai_hip_dequantize_f32_async((const int8_t *)(d + ob), (const float *)(d + ob + qbb), n,
                                      scheme, (float *)d, NULL);
    if (st == PAI_OK) {
      e = hipMemcpy(out, d, n * 4u, hipMemcpyDeviceToHost);
      if (e != hipSuccess) st = pai__map_hip((int)e, "hipMemcpy(v0 out)");
    }
  } else {
    st = pai__map_hip((int)e, "hipMemcpy(v0 codes)");
  }
  (void)hipFree(d);
  return st;
}
