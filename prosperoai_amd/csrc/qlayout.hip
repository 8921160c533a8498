/*
 * Upload re-layout (native GGUF blocks -> device planes) and the exact
 * dequantization kernel.
 *
 * Dequantization must be bit-identical to adapters/llama/gguf.c:650-967,
 * so this translation unit forbids FMA contraction: every product the
 * formats form is exact in f32 (f16 scale significand 11 bits, 6-bit
 * K-scales / int8 Q6_K scales, <= 6-bit codes: <= 24 significant bits),
 * and the single rounding of Q4_K's "d1*q - m1" then matches.
 */
#pragma clang fp contract(off)

#include "qdev.h"

namespace paik {

/* One thread per native block: copy its bytes into the planes. */
template <uint32_t T>
__global__ void __launch_bounds__(256) k_repack(paik_qview_t v, const uint8_t *__restrict__ src,
                                                uint32_t block_bytes) {
  const size_t blk = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)v.n * v.nb;
  if (blk >= total) return;
  const size_t row = blk / v.nb;
  const uint32_t b = (uint32_t)(blk % v.nb);
  const uint8_t *s = src + blk * block_bytes;
  uint8_t *q = const_cast<uint8_t *>(v.q) + row * v.q_stride;
  if constexpr (T == 8u) { /* Q8_0: d | qs[32] */
    const_cast<uint16_t *>(v.d)[blk] = (uint16_t)(s[0] | (s[1] << 8));
    for (int i = 0; i < 32; ++i) q[32u * b + i] = s[2 + i];
  } else if constexpr (T == 2u) { /* Q4_0: d | qs[16] */
    const_cast<uint16_t *>(v.d)[blk] = (uint16_t)(s[0] | (s[1] << 8));
    for (int i = 0; i < 16; ++i) q[16u * b + i] = s[2 + i];
  } else if constexpr (T == 12u) { /* Q4_K: head[16] | qs[128] */
    uint8_t *m = const_cast<uint8_t *>(v.meta) + blk * 16u;
    for (int i = 0; i < 16; ++i) m[i] = s[i];
    for (int i = 0; i < 128; ++i) q[128u * b + i] = s[16 + i];
  } else { /* Q6_K: ql[128] | qh[64] | sc[16] | d */
    for (int h = 0; h < 2; ++h) {
      for (int t = 0; t < 4; ++t) {
        uint8_t *o = q + 128u * b + 64u * h + 16u * t;
        for (int i = 0; i < 8; ++i) {
          o[i] = s[64 * h + 8 * t + i];
          o[8 + i] = s[64 * h + 32 + 8 * t + i];
        }
      }
    }
    uint8_t *a = const_cast<uint8_t *>(v.aux) + row * (v.k >> 2) + 64u * b;
    for (int i = 0; i < 64; ++i) a[i] = s[128 + i];
    uint8_t *m = const_cast<uint8_t *>(v.meta) + blk * 16u;
    for (int i = 0; i < 16; ++i) m[i] = s[192 + i];
    const_cast<uint16_t *>(v.d)[blk] = (uint16_t)(s[208] | (s[209] << 8));
  }
}

/* One thread per chunk: 32 exact values written at their native columns. */
template <class F>
__global__ void __launch_bounds__(256) k_dequant(paik_qview_t v, float *__restrict__ out) {
  const size_t job = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t chunks = v.k >> 5;
  if (job >= (size_t)v.n * chunks) return;
  const uint32_t row = (uint32_t)(job / chunks), c = (uint32_t)(job % chunks);
  float o[32];
  F::dequant(F::load(v, row, c), c, o);
  float *dst = out + (size_t)row * v.k;
#pragma unroll
  for (int i = 0; i < 32; i += 4) {
    const uint32_t e = F::elem(c, i); /* runs are >= 8 long and 8-aligned */
    *reinterpret_cast<float4 *>(dst + e) = make_float4(o[i], o[i + 1], o[i + 2], o[i + 3]);
  }
}

} // namespace paik

using namespace paik;

extern "C" int paik_repack(const paik_qview_t *v, const uint8_t *native, void *stream) {
  const size_t blocks = (size_t)v->n * v->nb;
  const dim3 grid((unsigned)((blocks + 255) / 256)), block(256);
  hipStream_t s = (hipStream_t)stream;
  switch (v->type) {
  case 8u: k_repack<8u><<<grid, block, 0, s>>>(*v, native, 34u); break;
  case 2u: k_repack<2u><<<grid, block, 0, s>>>(*v, native, 18u); break;
  case 12u: k_repack<12u><<<grid, block, 0, s>>>(*v, native, 144u); break;
  case 14u: k_repack<14u><<<grid, block, 0, s>>>(*v, native, 210u); break;
  default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}

extern "C" int paik_dequant(const paik_qview_t *v, float *out, void *stream) {
  const size_t jobs = (size_t)v->n * (v->k >> 5);
  const dim3 grid((unsigned)((jobs + 255) / 256)), block(256);
  hipStream_t s = (hipStream_t)stream;
  switch (v->type) {
  case 8u: k_dequant<Q8_0><<<grid, block, 0, s>>>(*v, out); break;
  case 2u: k_dequant<Q4_0><<<grid, block, 0, s>>>(*v, out); break;
  case 12u: k_dequant<Q4_K><<<grid, block, 0, s>>>(*v, out); break;
  case 14u: k_dequant<Q6_K><<<grid, block, 0, s>>>(*v, out); break;
  default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}
