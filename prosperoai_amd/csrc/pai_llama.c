/*
 * pai_llama host layer (C11): the decode-step operators and the
 * device-resident model of include/pai_llama.h. Every launch goes to the
 * gfx950 kernels of qdecode.hip and the packed projections of pai_hip.c;
 * nothing here computes on the CPU except the RoPE tables, which the
 * reference also builds on the host (adapters/llama/llama.c:855-861).
 */
#define _GNU_SOURCE
#include "pai_llama.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "paik.h"

/* shared with pai_hip.c; not exported */
pai_status_t pai__fail(pai_status_t st, const char *fmt, ...);
const paik_qview_t *pai__qmat_view(const pai_qmat_t *w);
pai_status_t pai__map_hip(int e, const char *what);
pai_status_t pai__ready(void);
#define fail pai__fail

#define LAUNCH(call, what)                                                     \
  do {                                                                         \
    const int e_ = (call);                                                     \
    if (e_ != 0) return pai__map_hip(e_, what);                                \
  } while (0)
#define HIP_TRY(call, what) LAUNCH((int)(call), what)
#define TRY(call)                                                              \
  do {                                                                         \
    const pai_status_t st_ = (call);                                           \
    if (st_ != PAI_OK) return st_;                                             \
  } while (0)

static uint64_t align256(uint64_t v) { return (v + 255u) & ~(uint64_t)255u; }

/* ---------------------------------------------------------------------- */
/* Operators                                                                */
/* ---------------------------------------------------------------------- */

pai_status_t pai_rmsnorm_f32_async(float *x, const float *delta, const float *gamma, float *xn,
                                   uint64_t n, float eps, void *stream) {
  if (x == NULL || gamma == NULL || xn == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (n == 0u) return fail(PAI_ERR_INVALID_ARG, "n == 0");
  if (n > paik_norm_max())
    return fail(PAI_ERR_UNSUPPORTED, "n=%llu above %u", (unsigned long long)n, paik_norm_max());
  TRY(pai__ready());
  if (eps == 0.0f) eps = 1e-5f; /* cpu/reference/ref_ops.c:203-205 */
  LAUNCH(paik_add_rmsnorm(x, delta, gamma, xn, (uint32_t)n, eps, stream), "rmsnorm launch");
  return PAI_OK;
}

/* The one-token projections of the decode step with their neighbours
 * fused in (paik_gemv_one): the RMSNorm before a projection, the residual
 * ADD after one. */
#define PAI_FUSED_MAX 4u
#define PAI_FUSED_NORM_MAX 3u /* matrices per fused-RMSNorm launch */

static pai_status_t check_one(const pai_qmat_t *const *ws, uint32_t count, const float *x,
                              float *const *ys, const paik_qview_t **vs) {
  if (ws == NULL || ys == NULL || x == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (count == 0u || count > PAI_FUSED_MAX)
    return fail(PAI_ERR_INVALID_ARG, "count=%u, expected 1..%u", count, PAI_FUSED_MAX);
  for (uint32_t i = 0; i < count; ++i) {
    if (ws[i] == NULL || ys[i] == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
    vs[i] = pai__qmat_view(ws[i]);
    if (vs[i]->type != vs[0]->type || vs[i]->k != vs[0]->k)
      return fail(PAI_ERR_MISMATCH, "matrix %u differs from matrix 0 in type or K", i);
    if (((uintptr_t)ys[i] & 3u) != 0u) return fail(PAI_ERR_INVALID_ARG, "y must be 4-byte aligned");
  }
  if (((uintptr_t)x & 15u) != 0u) return fail(PAI_ERR_INVALID_ARG, "x must be 16-byte aligned");
  return pai__ready();
}

static pai_status_t check_gamma(const float *gamma, uint32_t type, uint32_t k) {
  if (gamma == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (((uintptr_t)gamma & 15u) != 0u)
    return fail(PAI_ERR_INVALID_ARG, "gamma must be 16-byte aligned");
  if (k > paik_gemv_norm_max_k(type))
    return fail(PAI_ERR_UNSUPPORTED, "K=%u above %u for the fused RMSNorm", k,
                paik_gemv_norm_max_k(type));
  return PAI_OK;
}

pai_status_t pai_qgemv_rmsnorm_f32_async(const pai_qmat_t *const *ws, uint32_t count,
                                         const float *x, const float *gamma, float eps,
                                         float *const *ys, void *stream) {
  const paik_qview_t *vs[PAI_FUSED_MAX];
  if (count > PAI_FUSED_NORM_MAX)
    return fail(PAI_ERR_INVALID_ARG, "count=%u, expected 1..%u", count, PAI_FUSED_NORM_MAX);
  TRY(check_one(ws, count, x, ys, vs));
  TRY(check_gamma(gamma, vs[0]->type, vs[0]->k));
  if (eps == 0.0f) eps = 1e-5f; /* cpu/reference/ref_ops.c:203-205 */
  LAUNCH(paik_gemv_one(vs, ys, count, 0, x, gamma, eps, 0, stream), "kernel launch");
  return PAI_OK;
}

pai_status_t pai_qgemv_rmsnorm_gate_up_async(const pai_qmat_t *w_gate, const pai_qmat_t *w_up,
                                             const float *x, const float *gamma, float eps,
                                             float *h, void *stream) {
  const pai_qmat_t *ws[2] = {w_gate, w_up};
  float *ys[2] = {h, h};
  const paik_qview_t *vs[PAI_FUSED_MAX];
  TRY(check_one(ws, 2u, x, ys, vs));
  if (vs[0]->n != vs[1]->n) return fail(PAI_ERR_MISMATCH, "gate and up differ in shape");
  TRY(check_gamma(gamma, vs[0]->type, vs[0]->k));
  if (eps == 0.0f) eps = 1e-5f;
  LAUNCH(paik_gemv_one(vs, ys, 2u, 1, x, gamma, eps, 0, stream), "kernel launch");
  return PAI_OK;
}

pai_status_t pai_qgemv_add_f32_async(const pai_qmat_t *w, const float *x, float *y,
                                     void *stream) {
  const paik_qview_t *vs[PAI_FUSED_MAX];
  TRY(check_one(&w, 1u, x, &y, vs));
  LAUNCH(paik_gemv_one(vs, &y, 1u, 0, x, NULL, 0.0f, 1, stream), "kernel launch");
  return PAI_OK;
}

pai_status_t pai_rope_kv_append_async(const float *q, const float *k, const float *v,
                                      float *q_out, void *k_cache, void *v_cache,
                                      const float *cos_t, const float *sin_t, uint32_t hq,
                                      uint32_t hk, uint32_t hd, uint32_t r2, uint32_t ctx,
                                      uint32_t pos, void *stream) {
  if (q == NULL || k == NULL || v == NULL || q_out == NULL || k_cache == NULL ||
      v_cache == NULL || cos_t == NULL || sin_t == NULL)
    return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (hq == 0u || hk == 0u || hd == 0u || r2 == 0u || ctx == 0u)
    return fail(PAI_ERR_INVALID_ARG, "zero size");
  if (hd > 256u || 2u * r2 > hd)
    return fail(PAI_ERR_UNSUPPORTED, "hd=%u r2=%u: need hd <= 256 and 2 r2 <= hd", hd, r2);
  if (pos >= ctx) return fail(PAI_ERR_INVALID_ARG, "pos=%u outside the cache (ctx=%u)", pos, ctx);
  TRY(pai__ready());
  LAUNCH(paik_rope_append(q, k, v, q_out, k_cache, v_cache, cos_t, sin_t, hq, hk, hd, r2, ctx, pos,
                          stream),
         "rope launch");
  return PAI_OK;
}

uint64_t pai_attention_workspace_bytes(uint32_t hq, uint32_t hd, uint32_t len) {
  return (uint64_t)hq * paik_attn_chunks(len) * ((uint64_t)hd + 2u) * sizeof(float);
}

static pai_status_t check_attention(const float *q, const void *k_cache, const void *v_cache,
                                    const float *out, const void *workspace, uint32_t hq,
                                    uint32_t hk, uint32_t hd, uint32_t ctx, uint32_t len) {
  if (q == NULL || k_cache == NULL || v_cache == NULL || out == NULL || workspace == NULL)
    return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (hq == 0u || hk == 0u || hd == 0u || ctx == 0u || len == 0u)
    return fail(PAI_ERR_INVALID_ARG, "zero size");
  if (hq % hk != 0u) return fail(PAI_ERR_INVALID_ARG, "hq=%u not a multiple of hk=%u", hq, hk);
  if (hq / hk > 8u) return fail(PAI_ERR_UNSUPPORTED, "hq / hk = %u above 8", hq / hk);
  if (hd != 64u && hd != 128u && hd != 256u)
    return fail(PAI_ERR_UNSUPPORTED, "head size %u (64, 128 or 256)", hd);
  if (len > ctx) return fail(PAI_ERR_INVALID_ARG, "len=%u above ctx=%u", len, ctx);
  if (len > paik_attn_max_len())
    return fail(PAI_ERR_UNSUPPORTED, "len=%u above %u", len, paik_attn_max_len());
  if (((uintptr_t)q & 15u) != 0u || ((uintptr_t)k_cache & 15u) != 0u ||
      ((uintptr_t)v_cache & 15u) != 0u || ((uintptr_t)workspace & 255u) != 0u)
    return fail(PAI_ERR_INVALID_ARG,
                "q and the caches must be 16-byte aligned, the workspace 256-byte aligned");
  return pai__ready();
}

pai_status_t pai_attention_decode_async(const float *q, const void *k_cache, const void *v_cache,
                                        float *out, void *workspace, uint32_t hq, uint32_t hk,
                                        uint32_t hd, uint32_t ctx, uint32_t len, void *stream) {
  TRY(check_attention(q, k_cache, v_cache, out, workspace, hq, hk, hd, ctx, len));
  LAUNCH(paik_attn_decode(q, NULL, NULL, NULL, NULL, 0u, (void *)k_cache, (void *)v_cache,
                          (float *)workspace, out, hq, hk, hd, ctx,
                          len, stream),
         "attention launch");
  return PAI_OK;
}

pai_status_t pai_attention_decode_rope_async(const float *q, const float *k, const float *v,
                                             const float *cos_t, const float *sin_t, uint32_t r2,
                                             void *k_cache, void *v_cache, float *out,
                                             void *workspace, uint32_t hq, uint32_t hk,
                                             uint32_t hd, uint32_t ctx, uint32_t pos,
                                             void *stream) {
  if (k == NULL || v == NULL || cos_t == NULL || sin_t == NULL)
    return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (pos >= ctx) return fail(PAI_ERR_INVALID_ARG, "pos=%u outside the cache (ctx=%u)", pos, ctx);
  if (r2 == 0u || 2u * r2 > hd)
    return fail(PAI_ERR_UNSUPPORTED, "r2=%u: need 1 <= r2 and 2 r2 <= hd=%u", r2, hd);
  TRY(check_attention(q, k_cache, v_cache, out, workspace, hq, hk, hd, ctx, pos + 1u));
  LAUNCH(paik_attn_decode(q, k, v, cos_t, sin_t, r2, k_cache, v_cache,
                          (float *)workspace, out, hq, hk, hd, ctx,
                          pos + 1u, stream),
         "attention launch");
  return PAI_OK;
}

uint64_t pai_argmax_workspace_bytes(void) {
  return (uint64_t)paik_argmax_parts() * (sizeof(float) + sizeof(uint32_t));
}

pai_status_t pai_argmax_f32_async(const float *x, uint64_t n, uint32_t *out, void *workspace,
                                  void *stream) {
  if (x == NULL || out == NULL || workspace == NULL)
    return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (n == 0u) return fail(PAI_ERR_INVALID_ARG, "n == 0");
  if (n > 0xFFFFFFFFull) return fail(PAI_ERR_UNSUPPORTED, "n above 2^32 - 1");
  TRY(pai__ready());
  float *pv = (float *)workspace;
  uint32_t *pi = (uint32_t *)(pv + paik_argmax_parts());
  LAUNCH(paik_argmax(x, (uint32_t)n, pv, pi, out, stream), "argmax launch");
  return PAI_OK;
}

/* ---------------------------------------------------------------------- */
/* Model                                                                    */
/* ---------------------------------------------------------------------- */

enum { W_Q, W_K, W_V, W_O, W_GATE, W_UP, W_DOWN, W_PER_LAYER };

struct pai_llama {
  pai_llama_config_t c;
  uint32_t hd, r2, kv_dim;
  const pai_qmat_t **w; /* [n_layer][W_PER_LAYER] */
  uint8_t *fuse_qkv;    /* q, k, v share type and K: one launch */
  uint8_t *layer_ok;
  const pai_qmat_t *embd, *out;
  int out_ok;
  /* one device allocation: norms | rope tables | step buffers */
  void *dev;
  float *norms; /* attn_norm[L], ffn_norm[L], output_norm: (2 L + 1) * n_embd */
  float *cos_t, *sin_t;
  float *x, *xn, *q, *k, *v, *a, *o, *h, *d, *logits;
  void *attn_ws, *arg_ws;
  uint32_t *tok; /* [0] token in, [1] next out (synchronous form) */
  void *kv;      /* fp16 [n_layer][2][n_head_kv][ctx][hd] */
  uint64_t kv_layer_bytes;
};

static pai_status_t check_config(const pai_llama_config_t *c, uint32_t *hd) {
  if (c->n_layer == 0u || c->n_embd == 0u || c->n_head == 0u || c->n_head_kv == 0u ||
      c->n_ff == 0u || c->vocab == 0u || c->ctx == 0u)
    return fail(PAI_ERR_INVALID_ARG, "zero size in the model configuration");
  if (c->n_embd % c->n_head != 0u || c->n_head % c->n_head_kv != 0u)
    return fail(PAI_ERR_INVALID_ARG, "n_embd, n_head and n_head_kv do not divide");
  if (c->n_head / c->n_head_kv > 8u)
    return fail(PAI_ERR_UNSUPPORTED, "n_head / n_head_kv = %u above 8", c->n_head / c->n_head_kv);
  *hd = c->n_embd / c->n_head;
  if (*hd != 64u && *hd != 128u && *hd != 256u)
    return fail(PAI_ERR_UNSUPPORTED, "head size %u (64, 128 or 256)", *hd);
  if (c->ctx > paik_attn_max_len())
    return fail(PAI_ERR_UNSUPPORTED, "ctx=%u above %u", c->ctx, paik_attn_max_len());
  if (c->n_embd > paik_norm_max() || c->n_ff > 0x40000000u)
    return fail(PAI_ERR_UNSUPPORTED, "n_embd=%u above %u", c->n_embd, paik_norm_max());
  return PAI_OK;
}

void pai_llama_free(pai_llama_t *m) {
  if (m == NULL) return;
  if (m->dev != NULL) (void)hipFree(m->dev);
  if (m->kv != NULL) (void)hipFree(m->kv);
  free(m->w);
  free(m->fuse_qkv);
  free(m->layer_ok);
  free(m);
}

pai_status_t pai_llama_create(pai_llama_t **out, const pai_llama_config_t *cfg) {
  if (out == NULL || cfg == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  *out = NULL;
  uint32_t hd = 0;
  TRY(check_config(cfg, &hd));
  TRY(pai__ready());
  pai_llama_t *m = (pai_llama_t *)calloc(1, sizeof *m);
  if (m == NULL) return fail(PAI_ERR_NOMEM, "model handle");
  m->c = *cfg;
  m->hd = hd;
  uint32_t n_rot = cfg->n_rot;
  if (n_rot == 0u || n_rot > hd || (n_rot & 1u) != 0u) n_rot = hd;
  m->c.n_rot = n_rot;
  m->r2 = n_rot / 2u;
  if (m->c.rope_theta == 0.0f) m->c.rope_theta = 10000.0f;
  if (m->c.norm_eps == 0.0f) m->c.norm_eps = 1e-5f;
  m->kv_dim = cfg->n_head_kv * hd;
  const uint32_t L = cfg->n_layer;
  m->w = (const pai_qmat_t **)calloc((size_t)L * W_PER_LAYER, sizeof *m->w);
  m->fuse_qkv = (uint8_t *)calloc(L, 1);
  m->layer_ok = (uint8_t *)calloc(L, 1);
  if (m->w == NULL || m->fuse_qkv == NULL || m->layer_ok == NULL) {
    pai_llama_free(m);
    return fail(PAI_ERR_NOMEM, "model tables");
  }

  /* device buffers */
  const uint64_t E = cfg->n_embd, QD = (uint64_t)cfg->n_head * hd, KV = m->kv_dim;
  const uint64_t sizes[] = {
      (2u * (uint64_t)L + 1u) * E * 4u,                          /* norms */
      (uint64_t)cfg->ctx * m->r2 * 4u,                           /* cos */
      (uint64_t)cfg->ctx * m->r2 * 4u,                           /* sin */
      E * 4u, E * 4u, QD * 4u, KV * 4u, KV * 4u,                 /* x xn q k v */
      QD * 4u, E * 4u, (uint64_t)cfg->n_ff * 4u, E * 4u,         /* a o h d */
      (uint64_t)cfg->vocab * 4u,                                 /* logits */
      pai_attention_workspace_bytes(cfg->n_head, hd, cfg->ctx),  /* attention */
      pai_argmax_workspace_bytes(),                              /* argmax */
      2u * sizeof(uint32_t),                                     /* tokens */
  };
  enum { NBUF = sizeof sizes / sizeof sizes[0] };
  uint64_t offs[NBUF], total = 0;
  for (int i = 0; i < NBUF; ++i) {
    offs[i] = total;
    total += align256(sizes[i]);
  }
  hipError_t e = hipMalloc(&m->dev, total);
  if (e != hipSuccess) {
    m->dev = NULL;
    pai_llama_free(m);
    return pai__map_hip((int)e, "hipMalloc(model buffers)");
  }
  char *b = (char *)m->dev;
  void *p[NBUF];
  for (int i = 0; i < NBUF; ++i) p[i] = b + offs[i];
  m->norms = (float *)p[0];
  m->cos_t = (float *)p[1];
  m->sin_t = (float *)p[2];
  m->x = (float *)p[3];
  m->xn = (float *)p[4];
  m->q = (float *)p[5];
  m->k = (float *)p[6];
  m->v = (float *)p[7];
  m->a = (float *)p[8];
  m->o = (float *)p[9];
  m->h = (float *)p[10];
  m->d = (float *)p[11];
  m->logits = (float *)p[12];
  m->attn_ws = p[13];
  m->arg_ws = p[14];
  m->tok = (uint32_t *)p[15];

  /* KV cache */
  m->kv_layer_bytes = 2u * (uint64_t)cfg->n_head_kv * cfg->ctx * hd * 2u;
  e = hipMalloc(&m->kv, m->kv_layer_bytes * L);
  if (e == hipSuccess) e = hipMemset(m->kv, 0, m->kv_layer_bytes * L);
  if (e == hipSuccess) e = hipMemset(m->dev, 0, total);
  if (e != hipSuccess) {
    pai_llama_free(m);
    return pai__map_hip((int)e, "KV cache");
  }

  /* RoPE tables, as adapters/llama/llama.c:855-861 */
  const uint64_t nt = (uint64_t)cfg->ctx * m->r2;
  float *tab = (float *)malloc(2u * nt * sizeof(float));
  if (tab == NULL) {
    pai_llama_free(m);
    return fail(PAI_ERR_NOMEM, "RoPE tables");
  }
  for (uint32_t pp = 0; pp < cfg->ctx; ++pp) {
    for (uint32_t i = 0; i < m->r2; ++i) {
      const float freq = powf(m->c.rope_theta, -(float)(2u * i) / (float)n_rot);
      tab[(uint64_t)pp * m->r2 + i] = cosf((float)pp * freq);
      tab[nt + (uint64_t)pp * m->r2 + i] = sinf((float)pp * freq);
    }
  }
  e = hipMemcpy(m->cos_t, tab, nt * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(m->sin_t, tab + nt, nt * sizeof(float), hipMemcpyHostToDevice);
  free(tab);
  if (e != hipSuccess) {
    pai_llama_free(m);
    return pai__map_hip((int)e, "RoPE tables");
  }
  *out = m;
  return PAI_OK;
}

static pai_status_t check_w(const pai_qmat_t *w, uint64_t n, uint64_t k, const char *name) {
  if (w == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL %s", name);
  uint32_t t;
  uint64_t wn, wk;
  TRY(pai_qmat_shape(w, &t, &wn, &wk));
  if (wn != n || wk != k)
    return fail(PAI_ERR_MISMATCH, "%s is %llux%llu, expected %llux%llu", name,
                (unsigned long long)wn, (unsigned long long)wk, (unsigned long long)n,
                (unsigned long long)k);
  return PAI_OK;
}

static uint32_t qtype(const pai_qmat_t *w) {
  uint32_t t = 0;
  uint64_t n, k;
  (void)pai_qmat_shape(w, &t, &n, &k);
  return t;
}

pai_status_t pai_llama_set_layer(pai_llama_t *m, uint32_t layer, const pai_qmat_t *wq,
                                 const pai_qmat_t *wk, const pai_qmat_t *wv,
                                 const pai_qmat_t *wo, const pai_qmat_t *w_gate,
                                 const pai_qmat_t *w_up, const pai_qmat_t *w_down,
                                 const float *attn_norm, const float *ffn_norm) {
  if (m == NULL || attn_norm == NULL || ffn_norm == NULL)
    return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (layer >= m->c.n_layer)
    return fail(PAI_ERR_INVALID_ARG, "layer %u of %u", layer, m->c.n_layer);
  const uint64_t E = m->c.n_embd, F = m->c.n_ff, KV = m->kv_dim;
  TRY(check_w(wq, E, E, "attn_q"));
  TRY(check_w(wk, KV, E, "attn_k"));
  TRY(check_w(wv, KV, E, "attn_v"));
  TRY(check_w(wo, E, E, "attn_output"));
  TRY(check_w(w_gate, F, E, "ffn_gate"));
  TRY(check_w(w_up, F, E, "ffn_up"));
  TRY(check_w(w_down, E, F, "ffn_down"));
  if (qtype(w_gate) != qtype(w_up))
    return fail(PAI_ERR_MISMATCH, "ffn_gate and ffn_up differ in type");
  const pai_qmat_t *ws[W_PER_LAYER] = {wq, wk, wv, wo, w_gate, w_up, w_down};
  memcpy(m->w + (size_t)layer * W_PER_LAYER, ws, sizeof ws);
  m->fuse_qkv[layer] = qtype(wq) == qtype(wk) && qtype(wq) == qtype(wv);
  HIP_TRY(hipMemcpy(m->norms + (size_t)layer * E, attn_norm, E * 4u, hipMemcpyHostToDevice),
          "attn_norm upload");
  HIP_TRY(hipMemcpy(m->norms + ((size_t)m->c.n_layer + layer) * E, ffn_norm, E * 4u,
                    hipMemcpyHostToDevice),
          "ffn_norm upload");
  m->layer_ok[layer] = 1u;
  return PAI_OK;
}

pai_status_t pai_llama_set_output(pai_llama_t *m, const pai_qmat_t *token_embd,
                                  const pai_qmat_t *output, const float *output_norm) {
  if (m == NULL || output_norm == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  TRY(check_w(token_embd, m->c.vocab, m->c.n_embd, "token_embd"));
  TRY(check_w(output, m->c.vocab, m->c.n_embd, "output"));
  m->embd = token_embd;
  m->out = output;
  HIP_TRY(hipMemcpy(m->norms + 2u * (size_t)m->c.n_layer * m->c.n_embd, output_norm,
                    (size_t)m->c.n_embd * 4u, hipMemcpyHostToDevice),
          "output_norm upload");
  m->out_ok = 1;
  return PAI_OK;
}

static uint16_t *cache_of(const pai_llama_t *m, uint32_t layer, int which) {
  return (uint16_t *)((char *)m->kv + m->kv_layer_bytes * layer +
                      (which ? m->kv_layer_bytes / 2u : 0u));
}

pai_status_t pai_llama_kv_cache(const pai_llama_t *m, uint32_t layer, void **k_cache,
                                void **v_cache) {
  if (m == NULL || k_cache == NULL || v_cache == NULL)
    return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (layer >= m->c.n_layer) return fail(PAI_ERR_INVALID_ARG, "layer %u", layer);
  *k_cache = cache_of(m, layer, 0);
  *v_cache = cache_of(m, layer, 1);
  return PAI_OK;
}

pai_status_t pai_llama_kv_write(pai_llama_t *m, uint32_t layer, uint32_t pos0, uint32_t npos,
                                const uint16_t *k, const uint16_t *v) {
  if (m == NULL || k == NULL || v == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (layer >= m->c.n_layer) return fail(PAI_ERR_INVALID_ARG, "layer %u", layer);
  if (npos == 0u) return fail(PAI_ERR_INVALID_ARG, "npos == 0");
  if ((uint64_t)pos0 + npos > m->c.ctx)
    return fail(PAI_ERR_INVALID_ARG, "positions %u..%u outside the cache", pos0, pos0 + npos);
  const size_t row = (size_t)m->hd * 2u, spitch = (size_t)m->kv_dim * 2u;
  for (int which = 0; which < 2; ++which) {
    const uint16_t *src = which ? v : k;
    uint16_t *dst = cache_of(m, layer, which);
    for (uint32_t h = 0; h < m->c.n_head_kv; ++h)
      HIP_TRY(hipMemcpy2D(dst + ((size_t)h * m->c.ctx + pos0) * m->hd, row, src + (size_t)h * m->hd,
                          spitch, row, npos, hipMemcpyHostToDevice),
              "KV upload");
  }
  return PAI_OK;
}

const float *pai_llama_logits(const pai_llama_t *m) { return m == NULL ? NULL : m->logits; }

pai_status_t pai_llama_decode_async(pai_llama_t *m, const uint32_t *token_dev, uint32_t pos,
                                    uint32_t *next_dev, void *stream) {
  if (m == NULL || token_dev == NULL || next_dev == NULL)
    return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  if (pos >= m->c.ctx) return fail(PAI_ERR_INVALID_ARG, "pos=%u outside ctx=%u", pos, m->c.ctx);
  if (!m->out_ok) return fail(PAI_ERR_INVALID_ARG, "output weights not set");
  for (uint32_t l = 0; l < m->c.n_layer; ++l)
    if (!m->layer_ok[l]) return fail(PAI_ERR_INVALID_ARG, "layer %u not set", l);
  TRY(pai__ready());
  const pai_llama_config_t *c = &m->c;
  const uint32_t E = c->n_embd, hq = c->n_head, hk = c->n_head_kv, hd = m->hd;
  const float eps = c->norm_eps;

  /* one-hot embedding row (adapters/llama/llama.c:511-520) */
  LAUNCH(paik_dequant_row(pai__qmat_view(m->embd), token_dev, m->x, stream), "embedding launch");
  /* The residual x is updated in place by the o and down projections
   * (x += W a), and each RMSNorm runs inside the projection that consumes
   * it, so a layer is five launches. */
  for (uint32_t l = 0; l < c->n_layer; ++l) {
    const pai_qmat_t *const *w = m->w + (size_t)l * W_PER_LAYER;
    const float *attn_norm = m->norms + (size_t)l * E;
    const float *ffn_norm = m->norms + ((size_t)c->n_layer + l) * E;
    /* q, k, v = rmsnorm(x, attn_norm) W^T */
    if (m->fuse_qkv[l]) {
      float *ys[3] = {m->q, m->k, m->v};
      TRY(pai_qgemv_rmsnorm_f32_async(w + W_Q, 3, m->x, attn_norm, eps, ys, stream));
    } else {
      for (int i = 0; i < 3; ++i) {
        float *y = i == 0 ? m->q : i == 1 ? m->k : m->v;
        TRY(pai_qgemv_rmsnorm_f32_async(w + W_Q + i, 1, m->x, attn_norm, eps, &y, stream));
      }
    }
    uint16_t *kc = cache_of(m, l, 0), *vc = cache_of(m, l, 1);
    /* RoPE, cache append and attention */
    TRY(pai_attention_decode_rope_async(m->q, m->k, m->v, m->cos_t + (size_t)pos * m->r2,
                                        m->sin_t + (size_t)pos * m->r2, m->r2, kc, vc, m->a,
                                        m->attn_ws, hq, hk, hd, c->ctx, pos, stream));
    /* x += a W_o^T */
    TRY(pai_qgemv_add_f32_async(w[W_O], m->a, m->x, stream));
    /* h = silu(xn W_gate^T) * (xn W_up^T), xn = rmsnorm(x, ffn_norm) */
    TRY(pai_qgemv_rmsnorm_gate_up_async(w[W_GATE], w[W_UP], m->x, ffn_norm, eps, m->h, stream));
    /* x += h W_down^T */
    TRY(pai_qgemv_add_f32_async(w[W_DOWN], m->h, m->x, stream));
  }
  {
    float *y = m->logits;
    TRY(pai_qgemv_rmsnorm_f32_async(&m->out, 1, m->x, m->norms + 2u * (size_t)c->n_layer * E, eps,
                                    &y, stream));
  }
  TRY(pai_argmax_f32_async(m->logits, c->vocab, next_dev, m->arg_ws, stream));
  return PAI_OK;
}

pai_status_t pai_llama_decode(pai_llama_t *m, uint32_t token, uint32_t pos, uint32_t *next,
                              float *logits) {
  if (m == NULL || next == NULL) return fail(PAI_ERR_INVALID_ARG, "NULL argument");
  TRY(pai__ready());
  HIP_TRY(hipMemcpy(m->tok, &token, sizeof token, hipMemcpyHostToDevice), "token upload");
  TRY(pai_llama_decode_async(m, m->tok, pos, m->tok + 1, NULL));
  HIP_TRY(hipMemcpy(next, m->tok + 1, sizeof *next, hipMemcpyDeviceToHost), "token download");
  if (logits != NULL)
    HIP_TRY(hipMemcpy(logits, m->logits, (size_t)m->c.vocab * 4u, hipMemcpyDeviceToHost),
            "logits download");
  return PAI_OK;
}
