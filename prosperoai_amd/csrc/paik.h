/*
 * Internal interface between the C host layer (pai_hip.c) and the HIP
 * kernels (*.hip). Plain C so both sides include it.
 *
 * Device layout of a packed matrix W[N][K] ("planes", one allocation).
 * The native GGUF block bytes are regrouped by "chunk" (32 consecutive
 * columns of a row) so that one lane of a wavefront fetches a chunk's
 * codes with one 16-byte load (two for Q8_0) plus its block's scales.
 * Codes are stored as the nibble words described in qdev.h (word j holds
 * columns 8j..8j+7; byte m = column 8j+m low, 8j+m+4 high), as signed
 * 4-bit fields where the format allows:
 *
 *   Q8_0: q    [N][K]       chunk c at 32c: 16 B of low nibbles (l - 8),
 *                           then 16 B of signed high nibbles h
 *         d    [N][K/32]    f16 block scales
 *   Q4_0: q    [N][K/2]     chunk c at 16c: codes n - 8
 *         d    [N][K/32]    f16 block scales
 *   Q4_K: q    [N][K/2]     chunk c (sub-block c%8 of super-block c/8) at
 *                           16c: codes n - 8
 *         meta [N][K/256]   16-byte heads, native (f16 d, f16 dmin, 12
 *                           bytes of packed 6-bit scales and mins)
 *   Q6_K: q    [N][K/2]     chunk c at 16c: low 4 code bits minus 8
 *         aux  [N][K/4]     chunk c at 8c: the 2 high code bits, two words
 *         meta [N][K/256][16] int8 sub-block scales, native
 *         d    [N][K/256]   f16 super-block scales
 *
 * Total bytes equal N * type_bytes(K): the re-layout moves bytes, it does
 * not add any.
 */
#ifndef PAIK_H
#define PAIK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct paik_qview {
  const uint8_t *q;    /* code plane, row stride q_stride bytes           */
  const uint8_t *aux;  /* Q6_K high-bit plane, row stride k/4 bytes       */
  const uint8_t *meta; /* Q4_K heads / Q6_K scales, 16 bytes per block    */
  const uint16_t *d;   /* f16 block scales, nb per row                    */
  uint32_t type;       /* ggml type id                                    */
  uint32_t n, k;       /* rows, columns (elements per row)                */
  uint32_t nb;         /* blocks per row (k/32 or k/256)                  */
  uint32_t q_stride;   /* bytes per row of the code plane                 */
  uint32_t pad_;
} paik_qview_t;

/* Launch-shape overrides for measurements, set only through
 * pai_hip_set_tuning (never from the environment). Zero everywhere is the
 * shipped dispatch; each field is read where the corresponding choice is
 * made. Defined in pai_hip.c. */
typedef struct paik_tune {
  int32_t gemm_splits;        /* MFMA GEMM K parts (1..64; 0: planned)           */
  int32_t gemm_no_x16;        /* 1: MFMA path without the 16-bit workspace        */
  int32_t gemm_atomic_splits; /* 1: multi-matrix split parts added with atomics   */
  int32_t gemv_wgs;           /* GEMV workgroups (1..65535; 0: planned)           */
  int32_t gemv_rows;          /* GEMV rows per group (1, 2, 4; 0: planned)        */
  int32_t gemv_nw;            /* one-token GEMV waves per workgroup (8, 16; 0)    */
  int32_t gemv_no_mx;         /* 1: 2..8-token calls stay on the integer-dot GEMV */
  int32_t mfma_min_m;         /* tokens from which calls take the MFMA GEMM (0: 8) */
  int32_t gemm_tile;          /* 16-bit GEMM tile: 1 = 32 tokens, 2 = 128, 3 = 256 (0: by M) */
  int32_t v0_sequential;      /* 1: v0 GEMMs on the one-thread-per-output kernel */
} paik_tune_t;
extern paik_tune_t paik_tune;

/* Plane offsets of a matrix inside one device allocation (256-byte
 * aligned planes). Returns the total bytes to allocate, 0 on bad input. */
uint64_t paik_plan_layout(uint32_t type, uint64_t n, uint64_t k,
                          uint64_t *off_q, uint64_t *off_aux,
                          uint64_t *off_meta, uint64_t *off_d);

/* The per-device scratch array of the no-allocation entry point
 * (qscratch.hip): its size, and its device address on the current device
 * (hipError_t as int; call with that device current). */
#define PAIK_SCRATCH_BYTES (16u << 20)
int paik_scratch_address(void **ptr);

/* Launchers (HIP side). All return hipError_t as int; 0 on success. The
 * stream is a hipStream_t. Shapes are validated by the caller. */
int paik_repack(const paik_qview_t *v, const uint8_t *native, void *stream);
int paik_dequant(const paik_qview_t *v, float *out, void *stream);
int paik_gemv(const paik_qview_t *v, uint32_t m, const float *x, float *y,
              void *stream);
/* y_i = x * W_i^T for count (1..4) matrices of one format and column
 * count, in one launch per group of up to 4 tokens. */
int paik_gemv_multi(const paik_qview_t *const *vs, float *const *ys,
                    uint32_t count, uint32_t m, const float *x, void *stream);
/* h = silu(x W_gate^T) * (x W_up^T) in one launch per token group
 * (gate and up of one type and shape; K up to paik_gemv_pair_max_k()). */
int paik_gemv_silu_mul(const paik_qview_t *gate, const paik_qview_t *up,
                       uint32_t m, const float *x, float *h, void *stream);
uint32_t paik_gemv_pair_max_k(void);
/* One token on the integer-dot kernel with the decode step's fusions, in
 * one launch: y_i = x' W_i^T for count (1..4; 1..3 with gamma) matrices of one format and K,
 * where x' = rmsnorm(x, gamma, eps) when gamma is set (one RMS per
 * workgroup; K up to paik_gemv_norm_max_k(type)) and x' = x otherwise; accum
 * set adds the products to y (each output has one writer per launch);
 * pair set takes vs = {gate, up} (count 2, no accum) and writes
 * ys[0] = silu(x' W_gate^T) * (x' W_up^T). x and gamma 16-byte aligned. */
uint32_t paik_gemv_norm_max_k(uint32_t type);
int paik_gemv_one(const paik_qview_t *const *vs, float *const *ys, uint32_t count, int pair,
                  const float *x, const float *gamma, float eps, int accum, void *stream);
/* Batched GEMV on the i8 matrix cores (qgemv_mx.hip): y_i = x W_i^T for
 * count (1..4) matrices of one format and K, or h = silu(x Wg^T) * (x Wu^T),
 * for m tokens in launches of paik_gemv_mx_tokens(k, m) tokens (1, 2, 4
 * or 8; 0 when K is not taken: K must be a multiple of 128). */
uint32_t paik_gemv_mx_tokens(uint32_t k, uint32_t m);
int paik_gemv_mx(const paik_qview_t *const *vs, float *const *ys,
                 uint32_t count, uint32_t m, const float *x, void *stream);
int paik_gemv_mx_silu_mul(const paik_qview_t *gate, const paik_qview_t *up,
                          uint32_t m, const float *x, float *h, void *stream);

/* v0 per-group formats (qv0.hip). */
typedef struct paik_v0_gemm {
  const float *a;          /* [m][k] f32                                     */
  const void *wq;          /* [k][n] int8 codes, or nibbles over t*n+j        */
  const float *scales;     /* [ceil(k/gs)][n]                                */
  float *c;                /* [m][n]                                         */
  void *workspace;         /* split-K parts (may be NULL: no split)           */
  uint64_t workspace_bytes;
  uint32_t bits, m, n, k;  /* m <= 65535 per launch                          */
  uint32_t gs;             /* group rows, 1..k                               */
  int strip_ok;            /* n % 16 == 0, gs % 16 == 0 or gs == k, wq and
                              scales 16-byte aligned: the strip kernel runs   */
  int sequential;          /* the one-thread-per-output kernel regardless     */
} paik_v0_gemm_t;
int paik_v0_gemm(const paik_v0_gemm_t *p, void *stream);
/* n < 2^31; q 16-byte aligned; scales hold ceil(n/gs) floats */
int paik_v0_quantize(const float *x, uint32_t n, uint32_t bits, uint32_t gs, int8_t *q,
                     float *scales, void *stream);
/* out 16-byte aligned */
int paik_v0_dequantize(const int8_t *q, const float *scales, uint32_t n, uint32_t bits,
                       uint32_t gs, float *out, void *stream);

/* Decode-step kernels (qdecode.hip). kc/vc are fp16 caches [hk][ctx][hd]. */
uint32_t paik_norm_max(void);
int paik_add_rmsnorm(float *x, const float *delta, const float *gamma, float *xn,
                     uint32_t n, float eps, void *stream);
int paik_rope_append(const float *q, const float *k, const float *v, float *qo,
                     void *kc, void *vc, const float *cos_t, const float *sin_t,
                     uint32_t hq, uint32_t hk, uint32_t hd, uint32_t r2,
                     uint32_t ctx, uint32_t pos, void *stream);
/* Attention over cache positions [0, len). With knew/vnew set, RoPE of q
 * and knew (tables of position len - 1) and the append of knew, vnew at
 * position len - 1 happen in the same launch. part holds
 * hq * paik_attn_chunks(len) * (hd + 2) floats (the per-chunk partials,
 * combined by a second launch). len <= paik_attn_max_len(). */
uint32_t paik_attn_chunks(uint32_t len);
uint32_t paik_attn_max_len(void);
int paik_attn_decode(const float *q, const float *knew, const float *vnew,
                     const float *cos_t, const float *sin_t, uint32_t r2, void *kc,
                     void *vc, float *part, float *o, uint32_t hq,
                     uint32_t hk, uint32_t hd, uint32_t ctx, uint32_t len, void *stream);
/* pv, pi hold paik_argmax_parts() entries */
uint32_t paik_argmax_parts(void);
int paik_argmax(const float *x, uint32_t n, float *pv, uint32_t *pi, uint32_t *out,
                void *stream);
/* out[0..k) = row *row of the matrix (device index, clamped to n - 1) */
int paik_dequant_row(const paik_qview_t *v, const uint32_t *row, float *out,
                     void *stream);
/* x16 (may be NULL): device workspace of x16_bytes for a 16-bit copy of
 * the activations; with it the activations move into LDS by DMA.
 * gate (may be NULL, may equal y): y = silu(gate) * (x W^T) elementwise,
 * gate being [m][n]; such launches are not split over K. */
int paik_gemm_mfma(const paik_qview_t *v, uint32_t m, const float *x,
                   float *y, const float *gate, int bf16, void *x16,
                   uint64_t x16_bytes, void *stream);
/* The same for count (1..4) matrices of one format and K sharing x, in one
 * launch on the 16-bit path (y_i = x W_i^T; gate only with count 1). A
 * launch split over K with part_bytes >= paik_gemm_part_bytes() stores each
 * part in `part` and sums them in a fixed order (a second launch);
 * otherwise it zero-fills y and adds the parts with atomics. silu_pair:
 * vs = {gate, up} of one shape, and the second launch writes
 * ys[0] = silu(x W_gate^T) * (x W_up^T) (needs the parts: a split launch, a
 * large enough part workspace and the 16-bit path for all m tokens).
 * x == NULL: x16 already holds the 16-bit copy of all m tokens (written by
 * an earlier call with the same x and bf16 flag); no conversion runs. */
int paik_gemm_mfma_multi(const paik_qview_t *const *vs, float *const *ys, uint32_t count,
                         uint32_t m, const float *x, const float *gate, int bf16, void *x16,
                         uint64_t x16_bytes, void *part, uint64_t part_bytes, int silu_pair,
                         void *stream);
/* Workspace bytes the split parts of such a launch need (0: no split). */
uint64_t paik_gemm_part_bytes(const paik_qview_t *const *vs, uint32_t count, uint32_t m);
/* K parts a 16-bit-path launch of m tokens (no gate) splits into. */
uint32_t paik_gemm_x16_splits(const paik_qview_t *v, uint32_t m);


#ifdef __cplusplus
}
#endif

#endif /* PAIK_H */
