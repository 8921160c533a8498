/*
 * Device-side block formats for gfx950.
 *
 * Every kernel works on "chunks": 32 consecutive codes of one row as seen
 * by one lane (chunk c covers a fixed set of 32 columns; K/32 chunks per
 * row). A chunk is fetched with one 16-byte code load (two for Q8_0) plus
 * its block's scales, decoded in registers, and either dequantized exactly
 * (the reference's f32 formula and operation order) or reduced against
 * activations.
 *
 * Per format, F provides:
 *   Raw                 the bytes of one chunk, as loaded
 *   load(v, row, c)     fetch chunk c of a row from the device planes
 *   elem(c, i)          column of slot i (0..31) of chunk c
 *   kRun                slots come in runs of kRun consecutive columns
 *   kNG                 slot groups sharing one scale (32/kNG slots each)
 *   decode(w, c, q, a, b)
 *                       q[i] = code of slot i as f32 (possibly scaled by a
 *                       power of two), and for group g the chunk's dot
 *                       product with x is  sum_g a[g]*sum(q*x) - b[g]*sum(x)
 *   dequant(w, c, o)    o[i] = the reference's f32 value of slot i, bit-exact
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

/* ---------------------------------------------------------------- Q8_0 */
/* adapters/llama/gguf.c:750-761: value = (float)int8 * d. */
struct Q8_0 {
  static constexpr uint32_t kType = 8, kRun = 32, kNG = 1;
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
  __device__ static uint32_t elem(uint32_t c, int i) { return 32u * c + (uint32_t)i; }
  __device__ static uint32_t word(const Raw &w, int i) {
    const uint32_t ws[8] = {w.q0.x, w.q0.y, w.q0.z, w.q0.w, w.q1.x, w.q1.y, w.q1.z, w.q1.w};
    return ws[i];
  }
  __device__ static void decode(const Raw &w, uint32_t, float q[32], float a[kNG], float b[kNG]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t x = word(w, j);
#pragma unroll
      for (int i = 0; i < 4; ++i) q[4 * j + i] = (float)(int32_t)(int8_t)byte_of(x, i);
    }
    a[0] = h2f(w.d);
    b[0] = 0.0f;
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
 * element j+16 (high nibble), value = (float)(nibble - 8) * d. */
struct Q4_0 {
  static constexpr uint32_t kType = 2, kRun = 32, kNG = 2;
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
  __device__ static uint32_t elem(uint32_t c, int i) { return 32u * c + (uint32_t)i; }
  __device__ static void decode(const Raw &w, uint32_t, float q[32], float a[kNG], float b[kNG]) {
    const uint32_t ws[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = ws[j] & 0x0F0F0F0Fu, hi = ws[j] & 0xF0F0F0F0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        q[4 * j + i] = (float)byte_of(lo, i);
        q[16 + 4 * j + i] = (float)byte_of(hi, i); /* 16 * code */
      }
    }
    const float d = h2f(w.d);
    a[0] = d;
    a[1] = d * 0.0625f;
    b[0] = b[1] = 8.0f * d;
  }
  __device__ static void dequant(const Raw &w, uint32_t, float o[32]) {
    const float d = h2f(w.d);
    const uint32_t ws[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t by = byte_of(ws[j], i);
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

/* adapters/llama/gguf.c:852-882. Chunk c = (super-block b = c/8,
 * pair p = (c%8)/2, half hh = c%2) holds code bytes q[32p+16hh .. +16):
 * low nibbles are columns 256b+64p+16hh+i (scale pair 2p), high nibbles
 * are those +32 (pair 2p+1). Value = (d*sc)*q - (dmin*m). */
struct Q4_K {
  static constexpr uint32_t kType = 12, kRun = 16, kNG = 2;
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
  __device__ static uint32_t elem(uint32_t c, int i) {
    const uint32_t r = c & 7u;
    return 256u * (c >> 3) + 64u * (r >> 1) + 16u * (r & 1u) + (uint32_t)(i & 15) +
           (i >= 16 ? 32u : 0u);
  }
  __device__ static void scales(const Raw &w, uint32_t c, float &d1, float &m1, float &d2,
                                float &m2) {
    const uint32_t p = (c & 7u) >> 1;
    uint32_t s0, n0, s1, n1;
    scale_min_k4(2u * p, w.m.y, w.m.z, w.m.w, s0, n0);
    scale_min_k4(2u * p + 1u, w.m.y, w.m.z, w.m.w, s1, n1);
    const float d = h2f(w.m.x), dmin = h2f(w.m.x >> 16);
    d1 = d * (float)s0;
    m1 = dmin * (float)n0;
    d2 = d * (float)s1;
    m2 = dmin * (float)n1;
  }
  __device__ static void decode(const Raw &w, uint32_t c, float q[32], float a[kNG], float b[kNG]) {
    const uint32_t ws[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = ws[j] & 0x0F0F0F0Fu, hi = ws[j] & 0xF0F0F0F0u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        q[4 * j + i] = (float)byte_of(lo, i);
        q[16 + 4 * j + i] = (float)byte_of(hi, i); /* 16 * code */
      }
    }
    float d1, m1, d2, m2;
    scales(w, c, d1, m1, d2, m2);
    a[0] = d1;
    b[0] = m1;
    a[1] = d2 * 0.0625f;
    b[1] = m2;
  }
  __device__ static void dequant(const Raw &w, uint32_t c, float o[32]) {
    float d1, m1, d2, m2;
    scales(w, c, d1, m1, d2, m2);
    const uint32_t ws[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t by = byte_of(ws[j], i);
        o[4 * j + i] = d1 * (float)(by & 0x0Fu) - m1;
        o[16 + 4 * j + i] = d2 * (float)(by >> 4) - m2;
      }
    }
  }
};

/* ---------------------------------------------------------------- Q6_K */
/* adapters/llama/gguf.c:920-947. Chunk c = (super-block b = c/8,
 * half h = (c%8)/4, t = c%4) covers l = 8t..8t+7 of half h; slot 8g+i is
 * column 256b+128h+32g+8t+i with scale sc[8h + t/2 + 2g] and code
 *   g=0: ql[l] low | qh[l] bits 0-1      g=1: ql[l+32] low | bits 2-3
 *   g=2: ql[l] high | qh[l] bits 4-5     g=3: ql[l+32] high | bits 6-7
 * Value = d * sc * (code - 32), left to right. */
struct Q6_K {
  static constexpr uint32_t kType = 14, kRun = 8, kNG = 4;
  struct Raw {
    uint4 ql; /* ql[l] for the 8 l's, then ql[l+32] */
    uint2 qh;
    uint2 sc; /* scales[8h .. 8h+7] */
    uint32_t d;
  };
  __device__ static Raw load(const paik_qview_t &v, uint32_t row, uint32_t c) {
    const uint32_t b = c >> 3, r = c & 7u;
    Raw w;
    w.ql = ld16(v.q + (size_t)row * v.q_stride + 16u * c);
    w.qh = ld8(v.aux + (size_t)row * (v.k >> 2) + 64u * b + 8u * r);
    w.sc = ld8(v.meta + ((size_t)row * v.nb + b) * 16u + 8u * (r >> 2));
    w.d = v.d[(size_t)row * v.nb + b];
    return w;
  }
  __device__ static uint32_t elem(uint32_t c, int i) {
    const uint32_t r = c & 7u;
    return 256u * (c >> 3) + 128u * (r >> 2) + 32u * (uint32_t)(i >> 3) + 8u * (r & 3u) +
           (uint32_t)(i & 7);
  }
  /* codes of group g for the four l's of word j (0: l=8t..8t+3, 1: +4..+7) */
  __device__ static uint32_t codes(const Raw &w, int g, int j) {
    const uint32_t a = j ? w.ql.y : w.ql.x;
    const uint32_t cc = j ? w.ql.w : w.ql.z;
    const uint32_t e = j ? w.qh.y : w.qh.x;
    switch (g) {
    case 0: return (a & 0x0F0F0F0Fu) | ((e & 0x03030303u) << 4);
    case 1: return (cc & 0x0F0F0F0Fu) | ((e & 0x0C0C0C0Cu) << 2);
    case 2: return ((a >> 4) & 0x0F0F0F0Fu) | (e & 0x30303030u);
    default: return ((cc >> 4) & 0x0F0F0F0Fu) | ((e >> 2) & 0x30303030u);
    }
  }
  __device__ static int32_t scale(const Raw &w, uint32_t c, int g) {
    const uint32_t t2 = (c & 3u) >> 1; /* t/2 */
    const uint32_t word = g < 2 ? w.sc.x : w.sc.y;
    return (int32_t)(int8_t)byte_of(word, (int)(t2 + 2u * (uint32_t)(g & 1)));
  }
  __device__ static void decode(const Raw &w, uint32_t c, float q[32], float a[kNG], float b[kNG]) {
    const float d = h2f(w.d);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t cw = codes(w, g, j);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[8 * g + 4 * j + i] = (float)byte_of(cw, i);
      }
      const float ds = d * (float)scale(w, c, g);
      a[g] = ds;
      b[g] = 32.0f * ds;
    }
  }
  __device__ static void dequant(const Raw &w, uint32_t c, float o[32]) {
    const float d = h2f(w.d);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const float s = (float)scale(w, c, g);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t cw = codes(w, g, j);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          o[8 * g + 4 * j + i] = d * s * (float)((int32_t)byte_of(cw, i) - 32);
        }
      }
    }
  }
};

} // namespace paik

#endif /* PAI_QDEV_H */
