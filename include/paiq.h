/*
 * paiq — host-side GGUF block encoders and the seeded input generator.
 *
 * The reference can read GGUF blocks (adapters/llama/gguf.c) but has no
 * encoder for them: its only quantizer is the v0 per-group scheme
 * (models/quantize.c:74-143). These functions produce Q8_0, Q4_0, Q4_K and
 * Q6_K blocks in the native GGUF layout from f32 rows, so that synthetic
 * weights can be built without a model file. They are part of
 * libpai_hip.so but make no GPU call.
 *
 * Encoders: Q8_0 and Q4_0 follow the published llama.cpp reference
 * quantizers (round-to-nearest scale from the block's extreme value).
 * Q4_K and Q6_K are this library's own: per sub-block range fit, then
 * 6-bit / int8 scale quantization and a refit of the codes to the stored
 * scales. Their outputs are valid blocks whose dequantization is within
 * the bounds the test suite states; they are not bit-identical to
 * llama.cpp's iterative K-quant search.
 */
#ifndef PAIQ_H
#define PAIQ_H

#include <stdint.h>

#include "pai_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Encode `rows` rows of `k` f32 values into native GGUF blocks (row after
 * row; row r starts at out + r * pai_qtype_bytes(type, k)). UNSUPPORTED
 * for other types or k not a whole number of blocks. Multithreaded over
 * rows (threads <= 0 picks the host's core count). */
pai_status_t paiq_quantize(uint32_t type, const float *src, uint64_t rows,
                           uint64_t k, void *out, uint64_t out_bytes,
                           int threads);

/* IEEE binary32 -> binary16, round to nearest even (inf/NaN preserved). */
uint16_t paiq_f32_to_f16(float v);
/* IEEE binary16 -> binary32, exact. */
float paiq_f16_to_f32(uint16_t h);

/* n samples of N(mean, std^2): splitmix64 stream seeded with `seed`, two
 * uniforms per Box-Muller pair (computed in double, stored as float). The
 * same seed gives the same values on every x86-64 host. */
void paiq_normal_f32(uint64_t seed, float mean, float std, float *out,
                     uint64_t n);

#ifdef __cplusplus
}
#endif

#endif /* PAIQ_H */
