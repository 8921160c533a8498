/*
 * pai_llama — the LLaMA decode step on one MI355X around the quantized
 * projections of pai_hip.h: RMSNorm, RoPE, an fp16 KV cache, grouped-query
 * attention and the greedy argmax on the GPU.
 *
 * The reference runs generation in sequence mode: every new token
 * re-executes the whole graph over all positions (models/model.c:453-507)
 * and samples the last position's logits. This header is its decode-mode
 * counterpart: the keys and values of earlier positions stay in an fp16
 * cache, and one step computes only the new position, which equals the
 * last row of the reference's sequence-mode graph (adapters/llama/llama.c:
 * 1-11, :499-800) with the cached keys and values rounded to fp16.
 *
 * Conventions of pai_hip.h: pai_status_t returns, PAI_ERR_INVALID_ARG for
 * NULL pointers or zero sizes, no call aborts. The *_async operator calls
 * take device pointers and a hipStream_t (NULL = the default stream) and
 * return once the kernels are enqueued.
 */
#ifndef PAI_LLAMA_H
#define PAI_LLAMA_H

#include <stdint.h>

#include "pai_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Operators ---------------------------------------------------------- */

/* If delta is not NULL, x[i] += delta[i] (in place); then
 *   xn[i] = x[i] * gamma[i] * rms,  rms = 1 / sqrtf((float)(sum x^2 / n) + eps)
 * with the sum of squares in double and eps = 0 meaning 1e-5.
 * Replaces pai_ref_rmsnorm_gamma_f32 (cpu/reference/ref_ops.c:196-218) for
 * one row, fused with the residual ADD that precedes every norm of the
 * model (adapters/llama/llama.c:746-757, :786-797). n <= 16384.
 * Products round as in the reference; the double sum is taken in another
 * order, so rms agrees to the last bit except in rare ties. */
pai_status_t pai_rmsnorm_f32_async(float *x, const float *delta, const float *gamma,
                                   float *xn, uint64_t n, float eps, void *stream);

/* One-token projections with the decode step's neighbouring operators
 * fused in, each one launch of the packed GEMV (device pointers, matrices
 * of pai_qmat_upload). They produce what the reference's op sequence
 * produces: RMSNORM then GEMM (adapters/llama/llama.c:674-693, :756-769,
 * :884-891), GEMM then ADD (:742-749, :788-795).
 *
 * ys[i] = rmsnorm(x, gamma, eps) W_i^T for count (1..3) matrices of one
 * format and K (q, k, v; the output head). Each workgroup computes the
 * RMS of the whole row itself (sum of squares in double, as
 * pai_rmsnorm_f32_async) while it forms x * gamma, and scales each finished
 * dot product by rms; no normalised copy of x is written. Scaling the sums
 * rather than each element moves one rounding: rel-L2 <= 1e-5 against the
 * reference's RMSNORM then GEMM. K <= 16384 (8192 for Q8_0: one column slice); x and gamma 16-byte aligned,
 * eps = 0 meaning 1e-5. */
pai_status_t pai_qgemv_rmsnorm_f32_async(const pai_qmat_t *const *ws, uint32_t count,
                                         const float *x, const float *gamma, float eps,
                                         float *const *ys, void *stream);

/* h = silu(xn W_gate^T) * (xn W_up^T) with xn = rmsnorm(x, gamma, eps):
 * the feed-forward block's norm, gate, up and SiLU-multiply
 * (adapters/llama/llama.c:756-781) in one launch. Limits as above. */
pai_status_t pai_qgemv_rmsnorm_gate_up_async(const pai_qmat_t *w_gate, const pai_qmat_t *w_up,
                                             const float *x, const float *gamma, float eps,
                                             float *h, void *stream);

/* y += x W^T for one token: the residual ADD after the attention output
 * and down projections. Each y[j] receives one f32 add of the finished
 * dot product (x + delta rounds once, as the reference's ADD). */
pai_status_t pai_qgemv_add_f32_async(const pai_qmat_t *w, const float *x, float *y,
                                     void *stream);

/* RoPE of one position followed by the KV-cache append. q holds hq heads
 * and k, v hold hk heads of hd floats; each head's pairs (i, i + r2),
 * i < r2, are rotated by the tables cos_t[i], sin_t[i] of position pos:
 *   out[i] = x[i] c - x[i+r2] s,  out[i+r2] = x[i] s + x[i+r2] c
 * (pai_ref_rope_f32, cpu/reference/ref_ops.c:231-256, bit for bit). The
 * rotated q goes to q_out; the rotated k and v (not rotated) are rounded to
 * fp16 (nearest even) and stored at position pos of k_cache and v_cache,
 * each laid out [hk][ctx][hd]. hd <= 256, 2 r2 <= hd, pos < ctx. */
pai_status_t pai_rope_kv_append_async(const float *q, const float *k, const float *v,
                                      float *q_out, void *k_cache, void *v_cache,
                                      const float *cos_t, const float *sin_t, uint32_t hq,
                                      uint32_t hk, uint32_t hd, uint32_t r2, uint32_t ctx,
                                      uint32_t pos, void *stream);

/* Bytes of the workspace the attention calls need for hq heads of
 * dimension hd over len positions: the per-chunk partial results, which
 * every call writes before it reads them (no initialisation needed). The
 * workspace is 256-byte aligned; calls sharing one must not overlap. */
uint64_t pai_attention_workspace_bytes(uint32_t hq, uint32_t hd, uint32_t len);

/* Attention of one query position over cache positions 0..len-1:
 *   out[h] = softmax((q[h] . k[p]) / sqrtf(hd))_p · v[p],
 * head h reading KV head h / (hq / hk). The last row of
 * pai_ref_attention_f32 (cpu/reference/ref_ops.c:287-340) with keys and
 * values taken from the fp16 caches ([hk][ctx][hd]). hd in {64, 128, 256},
 * hq / hk <= 8, 1 <= len <= min(ctx, 32768). Two launches: the context
 * is split in chunks of 64 positions (one workgroup per KV head and chunk),
 * then one workgroup per query head combines its chunks. The dot products and
 * sums run in another order (and with FMA) than the reference's: rel-L2
 * <= 1e-5 against its formula where scores are O(1); for large scores,
 * where the reference's own f32 evaluation errs by as much, within twice
 * its error against a float64 evaluation. */
pai_status_t pai_attention_decode_async(const float *q, const void *k_cache,
                                        const void *v_cache, float *out, void *workspace,
                                        uint32_t hq, uint32_t hk, uint32_t hd, uint32_t ctx,
                                        uint32_t len, void *stream);

/* The decode step's attention block in the same two launches: RoPE of q and k at
 * position pos (as pai_rope_kv_append_async, bit for bit), the append of
 * the rotated k and of v at pos (fp16), and pai_attention_decode_async over
 * positions 0..pos. q: [hq][hd] and k, v: [hk][hd] as the projections
 * produce them (not rotated); cos_t, sin_t: the r2 table entries of
 * position pos. Replaces the reference's ROPE(q), ROPE(k), ATTENTION ops
 * of one layer (adapters/llama/llama.c:713-733) for the last position. */
pai_status_t pai_attention_decode_rope_async(const float *q, const float *k, const float *v,
                                             const float *cos_t, const float *sin_t, uint32_t r2,
                                             void *k_cache, void *v_cache, float *out,
                                             void *workspace, uint32_t hq, uint32_t hk,
                                             uint32_t hd, uint32_t ctx, uint32_t pos,
                                             void *stream);

/* Bytes of the workspace pai_argmax_f32_async needs. */
uint64_t pai_argmax_workspace_bytes(void);

/* *out = the first index of the largest of x[0..n), as the greedy branch
 * of pai_sampler_sample_logits (models/sampler.c:146-155): a NaN never
 * replaces the running best, so a NaN at index 0 gives 0. out is a device
 * uint32_t. */
pai_status_t pai_argmax_f32_async(const float *x, uint64_t n, uint32_t *out, void *workspace,
                                  void *stream);

/* ---- Model -------------------------------------------------------------- */

typedef struct pai_llama pai_llama_t;

typedef struct pai_llama_config {
  uint32_t n_layer;   /* blocks */
  uint32_t n_embd;    /* hidden size (<= 16384) */
  uint32_t n_head;    /* query heads */
  uint32_t n_head_kv; /* key/value heads: divides n_head, n_head / n_head_kv <= 8 */
  uint32_t n_ff;      /* feed-forward size */
  uint32_t vocab;     /* logits */
  uint32_t ctx;       /* cache positions (<= 32768) */
  uint32_t n_rot;     /* rotated dimensions per head; 0, odd or above the head
                         size means the head size (adapters/llama/llama.c:372-375) */
  float rope_theta;   /* RoPE base; 0 = 10000 (llama.c:349-352) */
  float norm_eps;     /* RMSNorm epsilon; 0 = 1e-5 (the reference always
                         passes 0: scheduler/scheduler.c:444-480) */
} pai_llama_config_t;

/* Allocates the fp16 KV cache (n_layer * 2 * n_head_kv * ctx * hd * 2
 * bytes, zeroed), the RoPE tables and the step's buffers on the current
 * device. The tables are the reference's (adapters/llama/llama.c:855-861):
 *   freq_i = powf(theta, -(float)(2 i) / (float)n_rot),
 *   cos_t[p][i] = cosf((float)p * freq_i), sin_t[p][i] = sinf(...).
 * Head size hd = n_embd / n_head must be 64, 128 or 256. */
pai_status_t pai_llama_create(pai_llama_t **out, const pai_llama_config_t *cfg);
void pai_llama_free(pai_llama_t *m);

/* Layer weights: the seven projections as packed matrices (borrowed; they
 * must outlive the model), W[N][K] with
 *   wq [n_embd][n_embd], wk, wv [n_head_kv*hd][n_embd], wo [n_embd][n_embd],
 *   w_gate, w_up [n_ff][n_embd], w_down [n_embd][n_ff],
 * and the norm weights (n_embd floats each, host memory, copied). The
 * reference's tensors blk.L.{attn_q,attn_k,attn_v,attn_output,ffn_gate,
 * ffn_up,ffn_down,attn_norm,ffn_norm}.weight (adapters/llama/llama.c:
 * 378-398). PAI_ERR_MISMATCH on a wrong shape. */
pai_status_t pai_llama_set_layer(pai_llama_t *m, uint32_t layer, const pai_qmat_t *wq,
                                 const pai_qmat_t *wk, const pai_qmat_t *wv,
                                 const pai_qmat_t *wo, const pai_qmat_t *w_gate,
                                 const pai_qmat_t *w_up, const pai_qmat_t *w_down,
                                 const float *attn_norm, const float *ffn_norm);

/* token_embd [vocab][n_embd], output [vocab][n_embd] (borrowed) and
 * output_norm (n_embd floats, host, copied). */
pai_status_t pai_llama_set_output(pai_llama_t *m, const pai_qmat_t *token_embd,
                                  const pai_qmat_t *output, const float *output_norm);

/* Writes cache positions [pos0, pos0 + npos) of one layer from host fp16
 * bit patterns laid out [npos][n_head_kv][hd] (position-major, as the
 * reference's k and v values). Synchronous. */
pai_status_t pai_llama_kv_write(pai_llama_t *m, uint32_t layer, uint32_t pos0, uint32_t npos,
                                const uint16_t *k, const uint16_t *v);

/* One greedy decode step: token at position pos, the cache holding
 * positions 0..pos-1. Stores the step's keys and values at pos, leaves the
 * logits in the model (pai_llama_logits) and writes the argmax to *next.
 * logits (host, vocab floats) may be NULL. Synchronous.
 * The step is the embedding row, then per layer: RMSNorm + q/k/v in one
 * launch (pai_qgemv_rmsnorm_f32_async), RoPE + cache append + attention in
 * two (pai_attention_decode_rope_async), the o projection added into the
 * residual (pai_qgemv_add_f32_async), RMSNorm + gate/up + SiLU-mul in one
 * (pai_qgemv_rmsnorm_gate_up_async) and down added into the residual; then
 * the output norm + head in one launch and the two-launch argmax. */
pai_status_t pai_llama_decode(pai_llama_t *m, uint32_t token, uint32_t pos, uint32_t *next,
                              float *logits);

/* The same, enqueued on `stream`: the token is read from device memory
 * (token_dev, e.g. the previous step's next_dev) and the argmax is written
 * to device memory next_dev, so consecutive steps need no host round trip.
 * A token id >= vocab reads the last embedding row. Steps on one model
 * must not overlap (they share its buffers). */
pai_status_t pai_llama_decode_async(pai_llama_t *m, const uint32_t *token_dev, uint32_t pos,
                                    uint32_t *next_dev, void *stream);

/* Device pointer to the last step's logits (vocab floats). */
const float *pai_llama_logits(const pai_llama_t *m);

/* Device pointers to one layer's caches ([n_head_kv][ctx][hd] fp16). */
pai_status_t pai_llama_kv_cache(const pai_llama_t *m, uint32_t layer, void **k_cache,
                                void **v_cache);

#ifdef __cplusplus
}
#endif

#endif /* PAI_LLAMA_H */
