/*
 * Device-side block formats for gfx950.
 *
 * Every kernel works on "chunks": the 32 consecutive columns 32c..32c+31 of
 * one row (K/32 chunks per row). The upload re-layout (qlayout.hip) stores
 * the codes of a chunk contiguously, so one lane fetches a chunk with one
 * 16-byte load of 4-bit codes (two for Q8_0's int8 codes; Q6_K adds an
 * 8-byte load of its 2-bit high parts) plus the scales of its block.
 *
 * 4-bit code byte order inside a chunk (Q4_0, Q4_K, Q6_K low bits):
 *   byte i (0..15): low nibble = column i, high nibble = column 16 + i.
 * This is the native Q4_0 order; Q4_K and Q6_K are regrouped into it.
 *
 * Per format, F provides:
 *   Raw                 the bytes of one chunk, as loaded
 *   load(v, row, c)     fetch chunk c of a row from the device planes
 *   kNG                 slot groups sharing one scale: group g covers
 *                       columns 16g..16g+15 (kNG = 2) or all 32 (kNG = 1)
 *   kHiScale            columns 16..31 carry codes times 1/kHiScale
 *   decode(w, c, q, a, b)
 *                       q[i] = code of column i as f32 (times 1/kHiScale for
 *                       i >= 16), and the chunk's dot product with x is
 *                         sum_g a[g] * sum_{i in g} q[i] x'[i]  -  b[g] * sum_{i in g} x[i]
 *                       with x'[i] = x[i] for i < 16, kHiScale * x[i] above
 *   dequant(w, c, o)    o[i] = the reference's f32 value of column i,
 *                       bit-exact (same operations, same order)
 */
#ifndef PAI_QDEV_H
#define PAI_QDEV_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "paik.h"

namespace paik {

__device__ __forceinline__ float h2f(uint32_t bits) {
  // v_cvt_f32_f16 is exact for zeros, subnormals, normals and infinities;
  // a NaN stays a NaN (its payload is quieted, unlike a bit copy).
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }

__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
  return *reinterpret_cast<const uint4 *>(p);
}
__device__ __forceinline__ uint2 ld8(const uint8_t *p) {
  return *reinterpret_cast<const uint2 *>(p);
}
__device__ __forceinline__ uint32_t ld2(const uint8_t *p) {
  return *reinterpret_cast<const uint16_t *>(p);
}

__device__ __forceinline__ uint32_t word4(const uint4 &q, int j) {
  return j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
}

/* Hides the known bits of v from the optimizer. Without it, LLVM folds
 * "mask then take byte b" into a bit-field extract followed by
 * v_cvt_f32_ubyte0 (two instructions per code); with it, each code
 * converts in one v_cvt_f32_ubyte{0,1,2,3}. */
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  __asm__("" : "+v"(v));
  return v;
}

/* q[4j+b] = low nibble of byte b of word j (column 4j+b); q[16+4j+b] =
 * 16 * high nibble (column 16+4j+b). */
__device__ __forceinline__ void nibbles_f32(const uint4 &qw, float q[32]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = word4(qw, j);
    const uint32_t lo = opaque(w & 0x0F0F0F0Fu), hi = opaque(w & 0xF0F0F0F0u);
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      q[4 * j + b] = (float)byte_of(lo, b);
      q[16 + 4 * j + b] = (float)byte_of(hi, b);
    }
  }
}

/* ---------------------------------------------------------------- Q8_0 */
/* adapters/llama/gguf.c:750-761: value = (float)int8 * d. */
struct Q8_0 {
  static constexpr uint32_t kType = 8, kNG = 1;
  static constexpr float kHiScale = 1.0f;
  struct Raw {
    uint4 q0, q1;
    uint32_t d;
  };
  __device__ static Raw load(const paik_qview_t &v, uint32_t row, uint32_t c) {
    const uint8_t *p = v.q + (size_t)row * v.q_stride + 32u * c;
    Raw w;
    w.q0 = ld16(p);
    w.q1 = ld16(p + 16);
    w.d = v.d[(size_t)row * v.nb + c];
    return w;
  }
  __device__ static uint32_t word(const Raw &w, int i) {
    return i < 4 ? word4(w.q0, i) : word4(w.q1, i - 4);
  }
  /* q = code + 128 (the bytes with their sign bit flipped, read as
   * unsigned), so the offset is b = 128 * d. */
  __device__ static void decode(const Raw &w, uint32_t, float q[32], float a[kNG], float b[kNG]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t x = opaque(word(w, j) ^ 0x80808080u);
#pragma unroll
      for (int i = 0; i < 4; ++i) q[4 * j + i] = (float)byte_of(x, i);
    }
    a[0] = h2f(w.d);
    b[0] = 128.0f * a[0];
  }
  __device__ static void dequant(const Raw &w, uint32_t, float o[32]) {
    const float d = h2f(w.d);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t x = word(w, j);
#pragma unroll
      for (int i = 0; i < 4; ++i) o[4 * j + i] = (float)(int32_t)(int8_t)byte_of(x, i) * d;
    }
  }
};

/* ---------------------------------------------------------------- Q4_0 */
/* adapters/llama/gguf.c:680-694: byte j -> element j (low nibble) and
 * element j+16 (high nibble), value = (float)(nibble - 8) * d. The chunk is
 * the native block's 16 code bytes, unchanged. */
struct Q4_0 {
  static constexpr uint32_t kType = 2, kNG = 1;
  static constexpr float kHiScale = 0.0625f;
  struct Raw {
    uint4 q;
    uint32_t d;
  };
  __device__ static Raw load(const paik_qview_t &v, uint32_t row, uint32_t c) {
    Raw w;
    w.q = ld16(v.q + (size_t)row * v.q_stride + 16u * c);
    w.d = v.d[(size_t)row * v.nb + c];
    return w;
  }
  __device__ static void decode(const Raw &w, uint32_t, float q[32], float a[kNG], float b[kNG]) {
    nibbles_f32(w.q, q);
    const float d = h2f(w.d);
    a[0] = d;
    b[0] = 8.0f * d;
  }
  __device__ static void dequant(const Raw &w, uint32_t, float o[32]) {
    const float d = h2f(w.d);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t x = word4(w.q, j);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t by = byte_of(x, i);
        o[4 * j + i] = (float)((int32_t)(by & 0x0Fu) - 8) * d;
        o[16 + 4 * j + i] = (float)((int32_t)(by >> 4) - 8) * d;
      }
    }
  }
};

/* ---------------------------------------------------------------- Q4_K */
/* 6-bit (scale, min) pair j from the 12 packed bytes s0|s1|s2 (little
 * endian words). adapters/llama/gguf.c:639-648. */
__device__ __forceinline__ void scale_min_k4(uint32_t j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             uint32_t &sc, uint32_t &mn) {
  if (j < 4u) {
    sc = byte_of(s0, (int)j) & 63u;
    mn = byte_of(s1, (int)j) & 63u;
  } else {
    const int i = (int)j - 4;
    sc = (byte_of(s2, i) & 0x0Fu) | ((byte_of(s0, i) >> 6) << 4);
    mn = (byte_of(s2, i) >> 4) | ((byte_of(s1, i) >> 6) << 4);
  }
}

/* adapters/llama/gguf.c:852-882. Chunk c is sub-block j = c % 8 of
 * super-block c / 8 (columns 32j..32j+31 of it), which the reference
 * dequantizes as d1 * q - m1 with d1 = d * sc_j, m1 = dmin * m_j. Its 32
 * nibbles are stored in the 4-bit chunk order. */
struct Q4_K {
  static constexpr uint32_t kType = 12, kNG = 1;
  static constexpr float kHiScale = 0.0625f;
  struct Raw {
    uint4 q;
    uint4 m; /* d | dmin<<16, scales[0..3], scales[4..7], scales[8..11] */
  };
  __device__ static Raw load(const paik_qview_t &v, uint32_t row, uint32_t c) {
    Raw w;
    w.q = ld16(v.q + (size_t)row * v.q_stride + 16u * c);
    w.m = ld16(v.meta + ((size_t)row * v.nb + (c >> 3)) * 16u);
    return w;
  }
  __device__ static void scales(const Raw &w, uint32_t c, float &d1, float &m1) {
    uint32_t s, mn;
    scale_min_k4(c & 7u, w.m.y, w.m.z, w.m.w, s, mn);
    d1 = h2f(w.m.x) * (float)s;
    m1 = h2f(w.m.x >> 16) * (float)mn;
  }
  __device__ static void decode(const Raw &w, uint32_t c, float q[32], float a[kNG], float b[kNG]) {
    nibbles_f32(w.q, q);
    scales(w, c, a[0], b[0]);
  }
  __device__ static void dequant(const Raw &w, uint32_t c, float o[32]) {
    float d1, m1;
    scales(w, c, d1, m1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t x = word4(w.q, j);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t by = byte_of(x, i);
        o[4 * j + i] = d1 * (float)(by & 0x0Fu) - m1;
        o[16 + 4 * j + i] = d1 * (float)(by >> 4) - m1;
      }
    }
  }
};

/* ---------------------------------------------------------------- Q6_K */
/* adapters/llama/gguf.c:920-947. Chunk c = 4h + g of a super-block covers
 * its columns 128h + 32g + l (l < 32), with scale sc[8h + 2g + l/16], i.e.
 * sc[2(c%8)] for columns 0..15 of the chunk and sc[2(c%8)+1] for 16..31,
 * and 6-bit code q = low4 | high2 << 4; value = d * sc * (q - 32), left to
 * right. Storage: the low 4 bits in the 4-bit chunk order; the high 2 bits
 * as two words e0 (columns 0..15) and e1 (16..31), column 16t + 4k + b at
 * bits 2k..2k+1 of byte b of e_t. */
struct Q6_K {
  static constexpr uint32_t kType = 14, kNG = 2;
  static constexpr float kHiScale = 1.0f;
  struct Raw {
    uint4 ql;
    uint2 qh;
    uint32_t sc; /* int8 scales of columns 0..15 | 16..31 << 8 */
    uint32_t d;
  };
  __device__ static Raw load(const paik_qview_t &v, uint32_t row, uint32_t c) {
    const size_t blk = (size_t)row * v.nb + (c >> 3);
    Raw w;
    w.ql = ld16(v.q + (size_t)row * v.q_stride + 16u * c);
    w.qh = ld8(v.aux + (size_t)row * (v.k >> 2) + 8u * c);
    w.sc = ld2(v.meta + blk * 16u + 2u * (c & 7u));
    w.d = v.d[blk];
    return w;
  }
  /* 6-bit codes of word j: columns 4j+b (hi = 0) or 16+4j+b (hi = 1). */
  __device__ static uint32_t codes(const Raw &w, int j, int hi) {
    const uint32_t x = word4(w.ql, j);
    const uint32_t lo4 = hi ? (x >> 4) & 0x0F0F0F0Fu : x & 0x0F0F0F0Fu;
    const uint32_t e = hi ? w.qh.y : w.qh.x;
    return opaque(lo4 | (((e >> (2 * j)) & 0x03030303u) << 4));
  }
  __device__ static float scale(const Raw &w, int g) {
    return (float)(int32_t)(int8_t)byte_of(w.sc, g);
  }
  __device__ static void decode(const Raw &w, uint32_t, float q[32], float a[kNG], float b[kNG]) {
#pragma unroll
    for (int g = 0; g < 2; ++g) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t cw = codes(w, j, g);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[16 * g + 4 * j + i] = (float)byte_of(cw, i);
      }
    }
    const float d = h2f(w.d);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      a[g] = d * scale(w, g);
      b[g] = 32.0f * a[g];
    }
  }
  __device__ static void dequant(const Raw &w, uint32_t, float o[32]) {
    const float d = h2f(w.d);
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const float s = scale(w, g);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t cw = codes(w, j, g);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          o[16 * g + 4 * j + i] = d * s * (float)((int32_t)byte_of(cw, i) - 32);
      }
    }
  }
};

} // namespace paik

#endif /* PAI_QDEV_H */
