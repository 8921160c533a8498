/*
 * Internal interface between the C host layer (pai_hip.c) and the HIP
 * kernels (*.hip). Plain C so both sides include it.
 *
 * Device layout of a packed matrix W[N][K] ("planes", one allocation).
 * The bytes are the native GGUF block bytes, regrouped so that each lane
 * of a wavefront can fetch its 32-element "chunk" of a row with one
 * 16-byte load of codes plus a small scale fetch:
 *
 *   Q8_0: q  = int8 codes      [N][K]      (block b at bytes 32b..32b+31)
 *         d  = f16 scales      [N][K/32]
 *   Q4_0: q  = nibble bytes    [N][K/2]    (block b at bytes 16b..16b+15)
 *         d  = f16 scales      [N][K/32]
 *   Q4_K: q  = nibble bytes    [N][K/2]    (super-block b at 128b, native)
 *         meta = 16-byte heads [N][K/256]  (f16 d, f16 dmin, 12 scale bytes)
 *   Q6_K: q  = ql bytes        [N][K/2]    (super-block b at 128b; within
 *              each 64-byte half, 16-byte chunk t holds ql[8t..8t+7] then
 *              ql[32+8t..32+8t+7])
 *         aux = qh bytes       [N][K/4]    (native)
 *         meta = int8 scales   [N][K/256][16] (native)
 *         d  = f16 scales      [N][K/256]
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

/* Plane offsets of a matrix inside one device allocation (256-byte
 * aligned planes). Returns the total bytes to allocate, 0 on bad input. */
uint64_t paik_plan_layout(uint32_t type, uint64_t n, uint64_t k,
                          uint64_t *off_q, uint64_t *off_aux,
                          uint64_t *off_meta, uint64_t *off_d);

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
int paik_gemm_mfma(const paik_qview_t *v, uint32_t m, const float *x,
                   float *y, int bf16, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PAIK_H */
