/*
 * Device-side block formats for gfx950.
 *
 * Every kernel works on "chunks": the 32 consecutive columns 32c..32c+31 of
 * one row (K/32 chunks per row). The upload re-layout (qlayout.hip) stores
 * the codes of a chunk contiguously, so one lane fetches a chunk with one
 * 16-byte load of 4-bit codes (two for Q8_0; Q6_K adds an 8-byte load of
 * its 2-bit high parts) plus the scales of its block.
 *
 * Nibble words. 16 bytes of 4-bit fields hold a chunk as four 32-bit words;
 * word j carries columns 8j..8j+7: byte m (0..3) of the word holds column
 * 8j+m in its low nibble and column 8j+m+4 in its high nibble. (The digit
 * planes of the activations are built by byte gathers in this order.)
 * Fields are signed 4-bit integers wherever the format allows, so
 * v_dot8_i32_i4 can consume them as stored:
 *   Q4_0, Q4_K  s = n - 8 (the code n with its top bit flipped)
 *   Q8_0        low word group:  s = l - 8 for the low nibble l of the code,
 *               high word group: h, the code's (signed) high nibble, so
 *               code = 16 h + s + 8
 *   Q6_K        low 4 bits as s = l - 8; the high 2 bits h2 (0..3) in a
 *               separate 8-byte group: word e_t (t = 0, 1) keeps column
 *               16t + i (i < 8) at bits o..o+1 and column 16t + 8 + i at
 *               bits o+2..o+3, o being column i's nibble offset in a nibble
 *               word, so e_t & 0x33333333 and (e_t >> 2) & 0x33333333 are
 *               nibble words; q = 16 h2 + s + 8
 *
 * Per format, F provides:
 *   Raw                 the bytes of one chunk, as loaded
 *   load(v, row, c)     fetch chunk c of a row from the device planes
 *   bload(r, row, cb, l) the same for chunk cb + l through plane buffer
 *                       resources (row and cb wave-uniform, l the lane)
 *   dequant(w, c, o)    o[i] = the reference's f32 value of column i,
 *                       bit-exact (same operations, same order)
 *   dot(w, c, x)        the chunk's dot product with an activation chunk
 *                       given as digit planes (XChunk below)
 */
#ifndef PAI_QDEV_H
#define PAI_QDEV_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "paik.h"

namespace paik {

__device__ __forceinline__ float h2f(uint16_t bits) {
  // v_cvt_f32_f16 is exact for zeros, subnormals, normals and infinities;
  // a NaN stays a NaN (its payload is quieted, unlike a bit copy).
  return (float)__builtin_bit_cast(_Float16, bits);
}
/* f16 in the low / high half of a 32-bit word */
__device__ __forceinline__ float h2f_lo(uint32_t w) { return h2f((uint16_t)w); }
__device__ __forceinline__ float h2f_hi(uint32_t w) { return h2f((uint16_t)(w >> 16)); }

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }

__device__ __forceinline__ uint4 ld16(const uint8_t *p) {
  return *reinterpret_cast<const uint4 *>(p);
}
__device__ __forceinline__ uint2 ld8(const uint8_t *p) {
  return *reinterpret_cast<const uint2 *>(p);
}
__device__ __forceinline__ uint16_t ld2(const uint8_t *p) {
  return *reinterpret_cast<const uint16_t *>(p);
}

__device__ __forceinline__ uint32_t word4(const uint4 &q, int j) {
  return j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
}

/* ------------------------------------------------------------------------
 * Buffer-resource view of a packed matrix for the streaming kernels: one
 * 128-bit resource per plane (base, byte size; reads past the size return
 * zero), so a load is "plane resource + wave-uniform byte offset (SGPR) +
 * lane offset (VGPR)" with no per-lane 64-bit address arithmetic.
 * ---------------------------------------------------------------------- */
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

/* silu(g) * u in the reference's order of operations: g / (1 + e^-g)
 * (cpu/reference/ref_ops.c:219-228), then the product
 * (pai_ref_vecmul_f32, the MUL op at scheduler/scheduler.c:404-410).
 * expf is the device library's; the division is IEEE. */
__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

struct QRes {
  __amdgpu_buffer_rsrc_t q, aux, meta, d;
  uint32_t q_stride, nb, k4;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t plane_rsrc(const void *p, uint32_t bytes) {
  /* 0x00020000: the gfx9 data-format word of a raw byte buffer */
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes,
                                           0x00020000);
}

__device__ __forceinline__ QRes make_qres(const paik_qview_t &v) {
  QRes r;
  r.q = plane_rsrc(v.q, v.n * v.q_stride);
  r.aux = plane_rsrc(v.aux, v.n * (v.k >> 2));
  r.meta = plane_rsrc(v.meta, v.n * v.nb * 16u);
  r.d = plane_rsrc(v.d, v.n * v.nb * 2u);
  r.q_stride = v.q_stride;
  r.nb = v.nb;
  r.k4 = v.k >> 2;
  return r;
}

/* Cache policy of a buffer load: 0 normal; kNT non-temporal (the gfx950
 * `nt` bit), for weights a launch streams once. The decode GEMVs load
 * their weights this way so that the stream does not evict the
 * activations from L2: measured on the Q4_0 / Q4_K decode steps, +6%
 * (3150 -> 3340 and 2810 -> 2975 GB/s), bit-identical results. The
 * prefill GEMM keeps the normal policy: its token tiles re-read weights.
 * So does Q8_0, whose two loads per chunk each read half of a line. */
constexpr int kNT = 2;

template <int CP = 0>
__device__ __forceinline__ uint4 bl16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, CP);
  return make_uint4(x.x, x.y, x.z, x.w);
}
template <int CP = 0>
__device__ __forceinline__ uint2 bl8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, CP);
  return make_uint2(x.x, x.y);
}
/* kept 16-bit: a zero-extension would be an early use of the load */
template <int CP = 0>
__device__ __forceinline__ uint16_t bl2(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, CP);
}

/* Bit offset of column i (0..7) in a nibble word. */
__host__ __device__ constexpr int nib_off(int i) { return 8 * (i & 3) + 4 * (i >> 2); }
/* Signed 4-bit field of column i of a nibble word. */
__device__ __forceinline__ int32_t snib(uint32_t w, int i) {
  return (int32_t)(w << (28 - nib_off(i))) >> 28;
}
/* Unsigned 4-bit field of column i. */
__device__ __forceinline__ uint32_t unib(uint32_t w, int i) { return (w >> nib_off(i)) & 0xFu; }

/* ------------------------------------------------------------------------
 * Activation digit planes.
 *
 * An activation chunk x[0..31] is represented exactly enough for an f32
 * result by 24-bit fixed point relative to the chunk's largest magnitude:
 * with 2^(E-1) <= max|x| < 2^E, xq[k] = rint(x[k] * 2^(22-E)), |xq| <= 2^22,
 * and x[k] ~= xq[k] * xs with xs = 2^(E-22) (error <= 2^-23 max|x|). xq is
 * written in six signed base-16 digits, xq = sum_i 16^i D_i with D_i in
 * [-8, 7] (the nibbles of (xq + 0x888888) with their top bit flipped), and
 * plane X[i] holds digit i of the 32 columns as four nibble words. Then for
 * signed 4-bit codes s, sum_k s[k] xq[k] = sum_i 16^i sum_j dot8(s_j, X[i][j]).
 * sx0 / sx1 are the sums of xq * xs over columns 0..15 / 16..31.
 * A chunk holding an infinity or NaN gets xs = NaN, so every output that
 * touches it is NaN.
 * ---------------------------------------------------------------------- */
struct XChunk {
  uint32_t X[6][4];
  float xs, sx0, sx1;
};

__device__ __forceinline__ int32_t dot8(uint32_t a, uint32_t b, int32_t c) {
  return __builtin_amdgcn_sdot8((int)a, (int)b, c, false);
}
/* dot8 into a fresh accumulator: the three-operand form with an inline
 * zero (the compiler otherwise zeroes a register for v_dot8c first). */
__device__ __forceinline__ int32_t dot8z(uint32_t a, uint32_t b) {
  int32_t r;
  __asm__("v_dot8_i32_i4 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

/* sum_i 16^i A[i] for i < NA (6 or 7), as f32. Each A[i] is at most 2^12
 * in magnitude, so the integer steps cannot overflow. */
template <int NA>
__device__ __forceinline__ float combine(const int32_t A[NA]) {
  const int32_t lo = A[0] + (A[1] << 4) + (A[2] << 8) + (A[3] << 12);
  int32_t hi = A[4] + (A[5] << 4);
  if constexpr (NA > 6) hi += A[6] << 8;
  return fmaf((float)hi, 65536.0f, (float)lo);
}

/* A[i] += dot8(s_j, X[i][j]) for the words j in [J0, J1); with HI the words
 * are high digits worth 16x and land in A[i + 1]. */
template <bool HI, int J0, int J1>
__device__ __forceinline__ void dots(const uint32_t *s, const XChunk &x, int32_t *A) {
  constexpr int o = HI ? 1 : 0;
#pragma unroll
  for (int j = J0; j < J1; ++j)
#pragma unroll
    for (int i = 0; i < 6; ++i) A[i + o] = dot8(s[j], x.X[i][j], A[i + o]);
}
/* Same, starting the six chains A[0..5] from zero (A[6] untouched). */
template <int J0, int J1>
__device__ __forceinline__ void dots0(const uint32_t *s, const XChunk &x, int32_t *A) {
#pragma unroll
  for (int i = 0; i < 6; ++i) A[i] = dot8z(s[J0], x.X[i][J0]);
#pragma unroll
  for (int j = J0 + 1; j < J1; ++j)
#pragma unroll
    for (int i = 0; i < 6; ++i) A[i] = dot8(s[j], x.X[i][j], A[i]);
}

/* ---------------------------------------------------------------- Q8_0 */
/* adapters/llama/gguf.c:750-761: value = (float)int8 * d. */
struct Q8_0 {
  static constexpr uint32_t kType = 8;
  struct Raw {
    uint4 lo, hi; /* low-nibble words (l - 8), high-nibble words (h) */
    uint16_t d;
  };
  __device__ static Raw load(const paik_qview_t &v, uint32_t row, uint32_t c) {
    const uint8_t *p = v.q + (size_t)row * v.q_stride + 32u * c;
    Raw w;
    w.lo = ld16(p);
    w.hi = ld16(p + 16);
    w.d = v.d[(size_t)row * v.nb + c];
    return w;
  }
  /* chunk cb + lane of a row; row and cb wave-uniform. Normal cache
   * policy, unlike the other formats: each of the two loads uses half of
   * every 128-byte line it touches, and the other half must still be in L2
   * when the second load asks for it. Non-temporal loads here measured
   * 9.88 against 7.79 us for 4096 x 4096 (1805 vs 2292 GB/s), same results. */
  __device__ static Raw bload(const QRes &r, uint32_t row, uint32_t cb, uint32_t lane) {
    Raw w;
    const uint32_t so = row * r.q_stride + 32u * cb;
    w.lo = bl16(r.q, 32u * lane, so);
    w.hi = bl16(r.q, 32u * lane + 16u, so);
    w.d = bl2(r.d, 2u * lane, (row * r.nb + cb) * 2u);
    return w;
  }
  __device__ static int32_t code(const Raw &w, int col) {
    const int j = col >> 3, i = col & 7;
    return 16 * snib(word4(w.hi, j), i) + snib(word4(w.lo, j), i) + 8;
  }
  __device__ static void dequant(const Raw &w, uint32_t, float o[32]) {
    const float d = h2f(w.d);
#pragma unroll
    for (int k = 0; k < 32; ++k) o[k] = (float)code(w, k) * d;
  }
  /* code = 16 h + s + 8: sum code*x = [16 sum h xq + sum s xq] xs + 8 sum x */
  __device__ static float dot(const Raw &w, uint32_t, const XChunk &x) {
    const uint32_t s[4] = {w.lo.x, w.lo.y, w.lo.z, w.lo.w};
    const uint32_t h[4] = {w.hi.x, w.hi.y, w.hi.z, w.hi.w};
    int32_t A[7];
    dots0<0, 4>(s, x, A);
    A[6] = 0;
    dots<true, 0, 4>(h, x, A);
    return h2f(w.d) * fmaf(combine<7>(A), x.xs, 8.0f * (x.sx0 + x.sx1));
  }
};

/* ---------------------------------------------------------------- Q4_0 */
/* adapters/llama/gguf.c:680-694: value = (float)(n - 8) * d, n the 4-bit
 * code. Stored as s = n - 8. */
struct Q4_0 {
  static constexpr uint32_t kType = 2;
  struct Raw {
    uint4 q;
    uint16_t d;
  };
  __device__ static Raw load(const paik_qview_t &v, uint32_t row, uint32_t c) {
    Raw w;
    w.q = ld16(v.q + (size_t)row * v.q_stride + 16u * c);
    w.d = v.d[(size_t)row * v.nb + c];
    return w;
  }
  __device__ static Raw bload(const QRes &r, uint32_t row, uint32_t cb, uint32_t lane) {
    Raw w;
    w.q = bl16<kNT>(r.q, 16u * lane, row * r.q_stride + 16u * cb);
    w.d = bl2<kNT>(r.d, 2u * lane, (row * r.nb + cb) * 2u);
    return w;
  }
  __device__ static void dequant(const Raw &w, uint32_t, float o[32]) {
    const float d = h2f(w.d);
#pragma unroll
    for (int k = 0; k < 32; ++k) o[k] = (float)snib(word4(w.q, k >> 3), k & 7) * d;
  }
  __device__ static float dot(const Raw &w, uint32_t, const XChunk &x) {
    const uint32_t s[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
    int32_t A[6];
    dots0<0, 4>(s, x, A);
    return (h2f(w.d) * x.xs) * combine<6>(A);
  }
};

/* ---------------------------------------------------------------- Q4_K */
/* 6-bit (scale, min) pair j from the 12 packed bytes s0|s1|s2 (little
 * endian words). adapters/llama/gguf.c:639-648. */
__device__ __forceinline__ void scale_min_k4(uint32_t j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             uint32_t &sc, uint32_t &mn) {
  /* both cases computed and selected (j differs between lanes) */
  const int i = (int)(j & 3u);
  const uint32_t b0 = byte_of(s0, i), b1 = byte_of(s1, i), b2 = byte_of(s2, i);
  const bool lo = j < 4u;
  sc = lo ? (b0 & 63u) : ((b2 & 0x0Fu) | ((b0 >> 6) << 4));
  mn = lo ? (b1 & 63u) : ((b2 >> 4) | ((b1 >> 6) << 4));
}

/* adapters/llama/gguf.c:852-882. Chunk c is sub-block j = c % 8 of
 * super-block c / 8 (columns 32j..32j+31 of it), which the reference
 * dequantizes as d1 * n - m1 with d1 = d * sc_j, m1 = dmin * m_j. Codes are
 * stored as s = n - 8. */
struct Q4_K {
  static constexpr uint32_t kType = 12;
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
  /* cb is a multiple of 8, so chunk cb + lane is in super-block
   * cb/8 + lane/8 */
  __device__ static Raw bload(const QRes &r, uint32_t row, uint32_t cb, uint32_t lane) {
    Raw w;
    w.q = bl16<kNT>(r.q, 16u * lane, row * r.q_stride + 16u * cb);
    w.m = bl16<kNT>(r.meta, 16u * (lane >> 3), (row * r.nb + (cb >> 3)) * 16u);
    return w;
  }
  /* the same for sub-block j = 4 HI + i, with HI known at compile time */
  template <int HI>
  __device__ static void scales_half(const Raw &w, uint32_t i, float &d1, float &m1) {
    const uint32_t b0 = byte_of(w.m.y, (int)i), b1 = byte_of(w.m.z, (int)i);
    uint32_t s, mn;
    if constexpr (HI) {
      const uint32_t b2 = byte_of(w.m.w, (int)i);
      s = (b2 & 0x0Fu) | ((b0 >> 6) << 4);
      mn = (b2 >> 4) | ((b1 >> 6) << 4);
    } else {
      s = b0 & 63u;
      mn = b1 & 63u;
    }
    d1 = h2f_lo(w.m.x) * (float)s;
    m1 = h2f_hi(w.m.x) * (float)mn;
  }
  __device__ static void scales(const Raw &w, uint32_t c, float &d1, float &m1) {
    uint32_t s, mn;
    scale_min_k4(c & 7u, w.m.y, w.m.z, w.m.w, s, mn);
    d1 = h2f_lo(w.m.x) * (float)s;
    m1 = h2f_hi(w.m.x) * (float)mn;
  }
  __device__ static void dequant(const Raw &w, uint32_t c, float o[32]) {
    float d1, m1;
    scales(w, c, d1, m1);
#pragma unroll
    for (int k = 0; k < 32; ++k) o[k] = d1 * (float)(unib(word4(w.q, k >> 3), k & 7) ^ 8u) - m1;
  }
  /* sum (d1 n - m1) x = d1 (sum s xq) xs + (8 d1 - m1) sum x */
  __device__ static float dot(const Raw &w, uint32_t c, const XChunk &x) {
    const uint32_t s[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
    int32_t A[6];
    dots0<0, 4>(s, x, A);
    float d1, m1;
    scales(w, c, d1, m1);
    return fmaf(d1 * x.xs, combine<6>(A), fmaf(8.0f, d1, -m1) * (x.sx0 + x.sx1));
  }
  /* The scale/min unpack of sub-block j for a lane whose j is fixed (the
   * GEMV: chunk cb + lane with cb a multiple of 8, so j = lane % 8): one
   * byte permute gathers byte i = j % 4 of the min/scale word and of the
   * high-bits word into bytes 0 and 1, and a bit-field insert with a
   * per-lane mask takes the 6-bit field (j < 4) or its low 4 bits plus
   * the 2 high bits (j >= 4). Equal to scale_min_k4 for every j. */
  struct Lane {
    uint32_t sel, mask, msh;
  };
  __device__ static Lane lane_ctx(uint32_t j) {
    const uint32_t i = j & 3u;
    const bool lo = j < 4u;
    Lane l;
    /* perm(hi = scale or min word, lo = high-bits word): byte 0 <- the
     * field's low byte (j < 4: byte i of the scale/min word; else byte i
     * of the high-bits word), byte 1 <- byte i of the scale/min word */
    l.sel = (lo ? (4u + i) : i) | ((4u + i) << 8) | 0x0C0C0000u;
    l.mask = lo ? 0x3Fu : 0x0Fu;
    l.msh = lo ? 0u : 4u;
    return l;
  }
  __device__ static void scales_lane(const Raw &w, const Lane &l, float &d1, float &m1) {
    const uint32_t ps = __builtin_amdgcn_perm(w.m.y, w.m.w, l.sel);
    const uint32_t pm = __builtin_amdgcn_perm(w.m.z, w.m.w, l.sel);
    const uint32_t s = ((ps & l.mask) | ((ps >> 10) & ~l.mask)) & 63u;
    const uint32_t mn = (((pm >> l.msh) & l.mask) | ((pm >> 10) & ~l.mask)) & 63u;
    d1 = h2f_lo(w.m.x) * (float)s;
    m1 = h2f_hi(w.m.x) * (float)mn;
  }
  __device__ static float dot_lane(const Raw &w, const Lane &l, const XChunk &x) {
    const uint32_t s[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
    int32_t A[6];
    dots0<0, 4>(s, x, A);
    float d1, m1;
    scales_lane(w, l, d1, m1);
    return fmaf(d1 * x.xs, combine<6>(A), fmaf(8.0f, d1, -m1) * (x.sx0 + x.sx1));
  }
};

/* ---------------------------------------------------------------- Q6_K */
/* adapters/llama/gguf.c:920-947. Chunk c = 4h + g of a super-block covers
 * its columns 128h + 32g + l (l < 32), with scale sc[8h + 2g + l/16], i.e.
 * sc[2(c%8)] for columns 0..15 of the chunk and sc[2(c%8)+1] for 16..31,
 * and 6-bit code q = low4 | high2 << 4; value = d * sc * (q - 32), left to
 * right. */
struct Q6_K {
  static constexpr uint32_t kType = 14;
  struct Raw {
    uint4 ql;    /* s = low4 - 8, nibble words */
    uint2 qh;    /* e0, e1 (see the top of this file) */
    uint16_t sc; /* int8 scales of columns 0..15 | 16..31 << 8 */
    uint16_t d;
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
  __device__ static Raw bload(const QRes &r, uint32_t row, uint32_t cb, uint32_t lane) {
    const uint32_t blk = row * r.nb + (cb >> 3);
    Raw w;
    w.ql = bl16<kNT>(r.q, 16u * lane, row * r.q_stride + 16u * cb);
    w.qh = bl8<kNT>(r.aux, 8u * lane, row * r.k4 + 8u * cb);
    w.sc = bl2<kNT>(r.meta, 16u * (lane >> 3) + 2u * (lane & 7u), blk * 16u);
    w.d = bl2<kNT>(r.d, 2u * (lane >> 3), blk * 2u);
    return w;
  }
  /* high-2-bit nibble words: word j covers columns 8j..8j+7 */
  __device__ static void highs(const Raw &w, uint32_t h[4]) {
    h[0] = w.qh.x & 0x33333333u;
    h[1] = (w.qh.x >> 2) & 0x33333333u;
    h[2] = w.qh.y & 0x33333333u;
    h[3] = (w.qh.y >> 2) & 0x33333333u;
  }
  __device__ static float scale(const Raw &w, int g) {
    return (float)(int32_t)(int8_t)(g ? (w.sc >> 8) : w.sc);
  }
  __device__ static void dequant(const Raw &w, uint32_t, float o[32]) {
    const float d = h2f(w.d);
    uint32_t h[4];
    highs(w, h);
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      const int j = k >> 3, i = k & 7;
      const int32_t q = (int32_t)((unib(word4(w.ql, j), i) ^ 8u) | (unib(h[j], i) << 4));
      o[k] = d * scale(w, k >> 4) * (float)(q - 32);
    }
  }
  /* q - 32 = 16 h2 + s - 24: per half g,
   * sum (q - 32) x = [16 sum h2 xq + sum s xq] xs - 24 sum x */
  __device__ static float dot(const Raw &w, uint32_t, const XChunk &x) {
    const uint32_t s[4] = {w.ql.x, w.ql.y, w.ql.z, w.ql.w};
    uint32_t h[4];
    highs(w, h);
    int32_t A0[7], A1[7];
    dots0<0, 2>(s, x, A0);
    A0[6] = 0;
    dots<true, 0, 2>(h, x, A0);
    dots0<2, 4>(s, x, A1);
    A1[6] = 0;
    dots<true, 2, 4>(h, x, A1);
    const float d = h2f(w.d);
    const float t0 = fmaf(combine<7>(A0), x.xs, -24.0f * x.sx0);
    const float t1 = fmaf(combine<7>(A1), x.xs, -24.0f * x.sx1);
    return fmaf(d * scale(w, 0), t0, (d * scale(w, 1)) * t1);
  }
};

} // namespace paik

#endif /* PAI_QDEV_H */
