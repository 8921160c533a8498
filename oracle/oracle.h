/*
 * CPU oracle for the quantized-weights matmul (test infrastructure only).
 *
 * This library is the checker, never the product: only the test suite,
 * the smoke check and the benchmark's CPU-baseline leg load it. It
 * restates, function by function, the reference's block dequantization
 * (adapters/llama/gguf.c), its scalar f32 GEMM (cpu/reference/ref_ops.c)
 * and its AVX2+FMA kernels (cpu/optimized/opt_ops.c). Each function cites
 * the reference lines it follows.
 *
 * Parity pins (what checks each function independently of its own text):
 *   orc_f16_to_f32        exhaustive 65536-pattern check against
 *                         numpy float16->float32, plus the reference's
 *                         literals (tests/test_gguf.c:270-276).
 *   orc_scale_min_k4      brute force against a bit-level closed form
 *                         (6-bit fields of a 96-bit little-endian word).
 *   orc_dequant           the reference's hand vectors
 *                         (tests/test_gguf.c:284-298, 317-332, 451-491,
 *                         519-538), invariants (zero block, linearity in
 *                         d, dmin=0 reduction, one-hot codes), and the
 *                         reference's own gguf.c built into oracle/_ref.
 *   orc_gemm_seq_f32      brute-force f64 sums on tiny shapes, one-hot
 *                         activations, and the reference's ref_ops.c
 *                         built into oracle/_ref (bit-exact).
 *   orc_qgemm_seq_f32     composition of the two above; one-hot x returns
 *                         a dequantized column exactly.
 *   orc_qgemm_f64         closed-form sums on tiny shapes.
 *   orc_silu_mul_f32      the reference's pai_ref_silu_f32 and
 *                         pai_ref_vecmul_f32 built into oracle/_ref
 *                         (bit-exact), and silu's closed-form points
 *                         (silu(0) = 0, silu(x) -> x, silu(-x) -> -0).
 *   orc_opt_gemv_avx2 /   the reference's opt_ops.c built into oracle/_ref
 *   orc_opt_gemm_w8_avx2  (bit-exact), and tolerance vs the f64 oracle.
 *   orc_rmsnorm_gamma_f32 the reference's ref_ops.c built into oracle/_ref
 *   orc_rope_f32          (bit-exact), plus closed forms: a constant row
 *   orc_attention_f32     normalises to gamma / sqrt(1 + eps/c^2); RoPE at
 *                         position 0 is the identity and preserves pair
 *                         norms; attention over one position returns v,
 *                         over equal keys the mean of v.
 *   orc_attention_last_f32 equals the last row of orc_attention_f32 on
 *                         the same keys and values (bit-exact).
 *   orc_rope_tables_llama f64 closed form cos(p theta^(-2i/n_rot)).
 *   orc_argmax_first      numpy's first-occurrence argmax on NaN-free rows,
 *                         and hand cases for ties and NaNs.
 *   orc_f32_to_f16        numpy float32 -> float16 (round to nearest even)
 *                         on special values and random bit patterns.
 *   orc_llama_step        composition of the above with the sequential
 *                         GEMM; with kv_f16 = 0 and a prompt run token by
 *                         token it equals the reference's sequence-mode
 *                         graph restated with orc_attention_f32 over all
 *                         positions (last row, bit-exact).
 *   orc_quant_* /         the reference's models/quantize.c built into
 *   orc_quantize_v0_f32 / oracle/_ref (bit-exact on random data, every
 *   orc_dequantize_v0_f32 group size kind, odd lengths), the reference's
 *                         own cases (tests/test_quantize.c:37-117), and
 *                         closed forms: the largest |x| of a group maps to
 *                         +-qmax, the round trip is within half a step,
 *                         zero groups give scale 0.
 *   orc_gemm_wq_seq_f32   the reference's ref_ops.c built into oracle/_ref
 *                         (bit-exact), one-hot activations returning a
 *                         dequantized row exactly, and orc_gemm_wq_f64.
 *   orc_gemm_wq_f64       brute-force sums of exact terms on tiny shapes.
 *   orc_q8_0_encode_ref / textbook llama.cpp encoders used to pin the
 *   orc_q4_0_encode_ref   product encoders; the reference has no encoder.
 *                         Parity unpinned: they are checked only by the
 *                         round-trip bound (half a step plus the f16
 *                         rounding of the scale), the code ranges, and
 *                         hand cases whose codes follow from the
 *                         definition (a block's largest |x| maps to the
 *                         extreme code).
 */
#ifndef PAI_ORACLE_H
#define PAI_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids, as in adapters/llama/gguf.h:34-51. */
#define ORC_Q4_0 2u
#define ORC_Q8_0 8u
#define ORC_Q4_K 12u
#define ORC_Q6_K 14u

/* Status codes, as in sdk/include/pai/error.h:13-23. */
#define ORC_OK 0
#define ORC_ERR_INVALID_ARG -1
#define ORC_ERR_NOMEM -2
#define ORC_ERR_UNSUPPORTED -3
#define ORC_ERR_MISMATCH -6

float orc_f16_to_f32(uint16_t h);
void orc_f16_to_f32_bits(const uint16_t *h, uint32_t *out, uint64_t n);
void orc_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn);
uint64_t orc_type_bytes(uint32_t type, uint64_t numel);
int32_t orc_dequant(uint32_t type, const uint8_t *src, float *dst,
                    uint64_t numel);

int32_t orc_gemm_seq_f32(uint64_t m, uint64_t n, uint64_t k, const float *a,
                         const float *b, float *c);
int32_t orc_qgemm_seq_f32(uint32_t type, uint64_t n, uint64_t k,
                          const uint8_t *blocks, uint64_t m, const float *x,
                          float *y);
int32_t orc_qgemm_f64(uint32_t type, uint64_t n, uint64_t k,
                      const uint8_t *blocks, uint64_t m, const float *x,
                      double *y);
int32_t orc_silu_mul_f32(const float *g, const float *u, float *h, uint64_t n);
int32_t orc_compare_f32(const float *a, const float *b, uint64_t n,
                        float abs_tol, float rel_tol, uint64_t *first_bad);

int32_t orc_opt_gemv_avx2(uint64_t m, uint64_t k, const float *a,
                          const float *x, float *y);
int32_t orc_opt_gemv_avx2_mt(uint64_t m, uint64_t k, const float *a,
                             const float *x, float *y, int threads);
int32_t orc_opt_gemm_avx2(uint64_t m, uint64_t n, uint64_t k, const float *a,
                          const float *b, float *c);
/* v0 per-group scheme (models/quantize.h:36-40). */
typedef struct orc_quant_scheme {
  uint8_t bit_width;
  uint8_t is_signed;
  uint16_t group_size;
} orc_quant_scheme_t;
int32_t orc_quant_group_size(const orc_quant_scheme_t *s, uint64_t n, uint64_t *out_gs);
uint64_t orc_quant_num_groups(uint64_t n, const orc_quant_scheme_t *s);
uint64_t orc_quant_value_bytes(uint64_t n, const orc_quant_scheme_t *s);
int32_t orc_quantize_v0_f32(const float *src, uint64_t n, const orc_quant_scheme_t *s,
                            int8_t *out_q, float *out_scales, uint64_t *out_groups);
int32_t orc_dequantize_v0_f32(const int8_t *q, const float *scales, uint64_t n,
                              const orc_quant_scheme_t *s, float *out);
int32_t orc_gemm_wq_seq_f32(uint32_t bits, uint64_t m, uint64_t n, uint64_t k, const float *a,
                            const int8_t *w_q, const float *b_scales, uint64_t group_size,
                            float *c);
int32_t orc_gemm_wq_f64(uint32_t bits, uint64_t m, uint64_t n, uint64_t k, const float *a,
                        const int8_t *w_q, const float *b_scales, uint64_t group_size,
                        double *c);
int32_t orc_opt_gemm_w8_avx2(uint64_t m, uint64_t n, uint64_t k,
                             const float *a, const int8_t *w_q,
                             const float *b_scales, uint64_t group_size,
                             float *c);

void orc_q8_0_encode_ref(const float *x, uint8_t *out, uint64_t numel);
void orc_q4_0_encode_ref(const float *x, uint8_t *out, uint64_t numel);

/* Decode step of the LLaMA graph (adapters/llama/llama.c). */
uint16_t orc_f32_to_f16(float v);
int32_t orc_rmsnorm_gamma_f32(const float *a, float *c, uint64_t n, const float *gamma,
                              float eps);
int32_t orc_rope_f32(const float *x, uint64_t rows, uint64_t hd, uint64_t seq, uint64_t heads,
                     const float *cos_t, const float *sin_t, uint64_t r2, float *out);
void orc_rope_tables_llama(uint32_t ctx, uint32_t r2, uint32_t n_rot, float theta, float *cos_t,
                           float *sin_t);
int32_t orc_attention_f32(uint64_t h, uint64_t hk, uint64_t seq, uint64_t hd, const float *q,
                          const float *k, const float *v, float *out);
int32_t orc_attention_last_f32(uint64_t h, uint64_t hk, uint64_t ctx, uint64_t len, uint64_t hd,
                               const float *q, const float *k_cache, const float *v_cache,
                               float *out);
uint32_t orc_argmax_first(const float *x, uint64_t n);

/* A model for orc_llama_step: dequantized weights W[N][K] (row-major f32)
 * and f32 caches [n_layer][n_head_kv][ctx][hd], all owned by the caller. */
typedef struct orc_llama {
  uint32_t n_layer, n_embd, n_head, n_head_kv, n_ff, vocab, ctx, n_rot;
  float rope_theta, norm_eps;
  const float *const *w; /* [n_layer * 7]: q, k, v, o, gate, up, down */
  const float *attn_norm, *ffn_norm; /* [n_layer][n_embd] */
  const float *token_embd, *output;  /* [vocab][n_embd] */
  const float *output_norm;          /* [n_embd] */
  float *k_cache, *v_cache;
  int32_t kv_f16; /* round appended keys and values to fp16 */
} orc_llama_t;
int32_t orc_llama_step(const orc_llama_t *m, uint32_t token, uint32_t pos, float *logits,
                       uint32_t *next);

#ifdef __cplusplus
}
#endif

#endif /* PAI_ORACLE_H */
