/*
 * Upload re-layout (native GGUF blocks -> device planes) and the exact
 * dequantization kernel.
 *
 * Dequantization must be bit-identical to adapters/llama/gguf.c:650-967,
 * so this translation unit forbids FMA contraction. Every product the
 * formats form is exact in f32 (f16 scale significand 11 bits, 6-bit
 * K-scales / int8 Q6_K scales, <= 6-bit codes: <= 24 significant bits), and
 * the single rounding of Q4_K's "d1*q - m1" then matches.
 */
#pragma clang fp contract(off)

#include "qdev.h"

namespace paik {

/* 16 bytes of nibble words from 32 per-column 4-bit fields f[0..31]:
 * byte m of word j = f[8j+m] | f[8j+m+4] << 4. */
__device__ void put_nibbles(uint8_t *dst, const uint8_t f[32]) {
  for (int j = 0; j < 4; ++j)
    for (int m = 0; m < 4; ++m)
      dst[4 * j + m] = (uint8_t)((f[8 * j + m] & 0x0Fu) | ((f[8 * j + m + 4] & 0x0Fu) << 4));
}

/* One thread per chunk (32 columns of a row): gather its codes from the
 * native block into the nibble words of qdev.h; the first chunk of a block
 * also copies the block's scales. */
template <uint32_t T>
__global__ void __launch_bounds__(256) k_repack(paik_qview_t v, const uint8_t *__restrict__ src) {
  const size_t job = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t nc = v.k >> 5;
  if (job >= (size_t)v.n * nc) return;
  const size_t row = job / nc;
  const uint32_t c = (uint32_t)(job % nc);
  uint8_t *q = const_cast<uint8_t *>(v.q) + row * v.q_stride;
  uint8_t f[32];
  if constexpr (T == 8u) { /* Q8_0 block: d | qs[32]; chunk = block */
    const uint8_t *s = src + (row * v.nb + c) * 34u;
    const_cast<uint16_t *>(v.d)[row * v.nb + c] = (uint16_t)(s[0] | (s[1] << 8));
    for (int k = 0; k < 32; ++k) f[k] = (uint8_t)((s[2 + k] & 0x0Fu) ^ 8u);
    put_nibbles(q + 32u * c, f);
    for (int k = 0; k < 32; ++k) f[k] = (uint8_t)(s[2 + k] >> 4);
    put_nibbles(q + 32u * c + 16u, f);
  } else if constexpr (T == 2u) { /* Q4_0 block: d | qs[16]; chunk = block */
    const uint8_t *s = src + (row * v.nb + c) * 18u;
    const_cast<uint16_t *>(v.d)[row * v.nb + c] = (uint16_t)(s[0] | (s[1] << 8));
    for (int k = 0; k < 16; ++k) {
      f[k] = (uint8_t)((s[2 + k] & 0x0Fu) ^ 8u);
      f[16 + k] = (uint8_t)((s[2 + k] >> 4) ^ 8u);
    }
    put_nibbles(q + 16u * c, f);
  } else if constexpr (T == 12u) { /* Q4_K block: head[16] | qs[128] */
    const uint32_t b = c >> 3, j = c & 7u, p = j >> 1;
    const uint8_t *s = src + (row * v.nb + b) * 144u;
    const uint8_t *qs = s + 16 + 32u * p;
    /* sub-block 2p: low nibbles of qs[32p + l]; 2p+1: high nibbles */
    for (int l = 0; l < 32; ++l)
      f[l] = (uint8_t)(((j & 1u) ? (qs[l] >> 4) : (qs[l] & 0x0Fu)) ^ 8u);
    put_nibbles(q + 16u * c, f);
    if (j == 0u) {
      uint8_t *m = const_cast<uint8_t *>(v.meta) + (row * v.nb + b) * 16u;
      for (int i = 0; i < 16; ++i) m[i] = s[i];
    }
  } else { /* Q6_K block: ql[128] | qh[64] | sc[16] | d */
    const uint32_t b = c >> 3, j = c & 7u, h = j >> 2, g = j & 3u;
    const uint8_t *s = src + (row * v.nb + b) * 210u;
    const uint8_t *ql = s + 64u * h + ((g & 1u) ? 32u : 0u);
    const uint8_t *qh = s + 128u + 32u * h;
    uint8_t hi2[32];
    for (int l = 0; l < 32; ++l) {
      f[l] = (uint8_t)(((g & 2u) ? (ql[l] >> 4) : (ql[l] & 0x0Fu)) ^ 8u);
      hi2[l] = (uint8_t)((qh[l] >> (2u * g)) & 3u);
    }
    put_nibbles(q + 16u * c, f);
    uint8_t *e = const_cast<uint8_t *>(v.aux) + row * (v.k >> 2) + 8u * c;
    for (int t = 0; t < 2; ++t) {
      uint32_t w = 0;
      for (int i = 0; i < 8; ++i)
        w |= ((uint32_t)hi2[16 * t + i] << nib_off(i)) |
             ((uint32_t)hi2[16 * t + 8 + i] << (nib_off(i) + 2));
      for (int by = 0; by < 4; ++by) e[4 * t + by] = (uint8_t)(w >> (8 * by));
    }
    if (j == 0u) {
      uint8_t *m = const_cast<uint8_t *>(v.meta) + (row * v.nb + b) * 16u;
      for (int i = 0; i < 16; ++i) m[i] = s[192 + i];
      const_cast<uint16_t *>(v.d)[row * v.nb + b] = (uint16_t)(s[208] | (s[209] << 8));
    }
  }
}

/* One thread per chunk: 32 exact values written at columns 32c..32c+31. */
template <class F>
__global__ void __launch_bounds__(256) k_dequant(paik_qview_t v, float *__restrict__ out) {
  const size_t job = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t nc = v.k >> 5;
  if (job >= (size_t)v.n * nc) return;
  const uint32_t row = (uint32_t)(job / nc), c = (uint32_t)(job % nc);
  float o[32];
  F::dequant(F::load(v, row, c), c, o);
  float4 *dst = reinterpret_cast<float4 *>(out + (size_t)row * v.k + 32u * c);
#pragma unroll
  for (int i = 0; i < 8; ++i) dst[i] = make_float4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
}

} // namespace paik

using namespace paik;

extern "C" int paik_repack(const paik_qview_t *v, const uint8_t *native, void *stream) {
  const size_t jobs = (size_t)v->n * (v->k >> 5);
  const dim3 grid((unsigned)((jobs + 255) / 256)), block(256);
  hipStream_t s = (hipStream_t)stream;
  switch (v->type) {
  case 8u: k_repack<8u><<<grid, block, 0, s>>>(*v, native); break;
  case 2u: k_repack<2u><<<grid, block, 0, s>>>(*v, native); break;
  case 12u: k_repack<12u><<<grid, block, 0, s>>>(*v, native); break;
  case 14u: k_repack<14u><<<grid, block, 0, s>>>(*v, native); break;
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
