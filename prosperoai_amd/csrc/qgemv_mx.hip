/*
 * Batched decode GEMV (a few tokens) with the integer dot products on the
 * matrix cores: v_mfma_i32_16x16x64_i8.
 *
 * y[t][r] = sum_k x[t][k] * W[r][k] for up to MT = 8 tokens per launch,
 * f32 in and out, for up to 4 matrices that share x (q/k/v), or for a
 * gate/up pair with h = silu(x Wg^T) * (x Wu^T).
 *
 * Exact integer products. The activations of a chunk (32 columns) of one
 * token become a 24-bit fixed-point image xq = rint(x * 2^(22-E))
 * (2^(E-1) <= max|x| < 2^E) written as three signed base-256 digits,
 * xq = D0 + 256 D1 + 65536 D2 (the bytes of (xq + 0x808080) with their top
 * bit flipped). Weight codes are small integers (Q4_0/Q4_K as 16 (n - 8),
 * Q6_K as q, Q8_0 as the int8 code). One MFMA forms, exactly, the dot
 * product of a 16-column half chunk of weight codes with each digit plane
 * of one token; the f32 work per chunk, row and token is one combine of the
 * three plane sums and one or two scale steps. The weight operands are
 * built once per step and shared by all tokens of the launch, which is
 * what makes this kernel pay as the token count grows.
 *
 * Operands of one MFMA (16 output rows x 16 rows of A, k = 64 in four sets
 * of 16 bytes, lane l holding B column l%16 / A row l%16 for k-set l/16):
 *   B  lane (r, g) = (l%16, l/16): 16 codes of weight row r, chunk 4s + g.
 *      The lane loads the whole 16-byte chunk (32 codes); the first MFMA of
 *      a step takes columns 0..15, the second 16..31.
 *   A  row 4g + p (p < 3) holds digit plane p of chunk 4s + g of the token
 *      in k-set g and zeros elsewhere, i.e. lanes 20g + p carry plane bytes
 *      and all other lanes read a zero block.
 *   C  lane (r, g) receives rows 4g..4g+3 of column r: the three plane sums
 *      of its own row and chunk. The accumulator keeps running; a step's
 *      sums are the differences across its MFMAs (exact in int32: a step
 *      adds at most 2^19 per plane and a wave makes at most a few hundred
 *      steps).
 *
 * Work. Rows are taken 16 at a time ("items"; for a gate/up pair an item
 * is 8 gate rows and the same 8 up rows). A workgroup of 16 waves (8 from
 * 4 tokens on) owns a contiguous range of items and every wave takes a
 * fixed share of the columns of each of them, so the activation planes are built once per
 * workgroup in LDS and the weight stream is spread over all waves even
 * when there are fewer items than waves. Each wave keeps a ring of steps
 * of loads in flight across items. At the end of an item a wave sums its
 * four lanes per row (two cross-row shuffles) into one of two LDS slots;
 * after a barrier the first threads add the wave partials of each
 * output in wave order and store it. Every wave passes exactly one barrier
 * per item (waves without steps too), and every summation order is fixed
 * by the launch shape, so results are deterministic.
 *
 * K is a multiple of 128 (whole steps). Rows past a matrix's end re-read
 * its last row and are not stored; tokens past the launch's count have
 * zero planes and are not stored. A chunk of x holding an infinity or NaN
 * makes its scale NaN, so every output of that token it touches is NaN.
 */
#include <string.h>

#include <type_traits>

#include "qdev.h"

namespace paik {
namespace mx {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr uint32_t kPlaneBytes = 96; /* three 32-byte digit planes per chunk-token */
constexpr uint32_t kMaxMats = 4;
constexpr uint32_t kMaxChunkTok = 1024; /* chunk-tokens the plane builder covers */

/* Waves per workgroup: 16 up to 2 tokens; 8 from 4 tokens on, where the
 * planes take most of the LDS (one workgroup per CU either way) and the
 * per-token accumulators need the 256 registers of two waves per SIMD. */
template <int MT>
constexpr int waves() { return MT <= 2 ? 16 : 8; }
/* plane-builder passes: 1024 chunk-tokens, four threads each */
template <int NW>
constexpr int xit() { return (int)(4u * kMaxChunkTok / (64u * (uint32_t)NW)); }
/* Steps of loads in flight per wave: 2 up to 2 tokens (16-wave
 * workgroups), else 4. Deeper rings queue more of the matrix than HBM
 * returns in a round trip and delay every request behind them. Measured
 * on the Q4_K decode step (q/k/v + o + gate/up + down, us): 2 tokens 58.8
 * with the earlier 6-step ring, 48.9 with 2, 51.5 with 3; 4 tokens 79.1,
 * 73.1, 72.9, and 71.9 with 4; 8 tokens 80.5, 81.8, 78.5, 78.2. */
template <class F, int MT>
constexpr int ring() { return MT <= 2 ? 2 : 4; }

/* LDS layout: planes [MT][nch][3][32] | zero [32] | scales [MT][nch]
 * float4 {xs * f, sx0, sx1, sx0 + sx1} | partials [2][waves][MT][rows per item]. */
__host__ __device__ constexpr uint32_t lds_zero(uint32_t nct) { return nct * kPlaneBytes; }
__host__ __device__ constexpr uint32_t lds_scales(uint32_t nct) { return lds_zero(nct) + 32u; }
__host__ __device__ constexpr uint32_t lds_red(uint32_t nct) { return lds_scales(nct) + 16u * nct; }
__host__ __device__ constexpr uint32_t lds_bytes(uint32_t nct, uint32_t mt, uint32_t nw,
                                                  uint32_t ri) {
  return lds_red(nct) + 2u * nw * mt * ri * 4u;
}

typedef int v16i __attribute__((ext_vector_type(16)));

/* One token's three plane sums over the first (a) and the second (b) MFMA
 * of a step, exact integers. */
struct Sums {
  int32_t a0, a1, a2, b0, b1, b2;
};
/* D0 + 256 D1 + 65536 D2 of three plane sums, as f32 */
__device__ __forceinline__ float combine3(int32_t p0, int32_t p1, int32_t p2) {
  return fmaf((float)p2, 65536.0f, (float)(p0 + (p1 << 8)));
}
__device__ __forceinline__ float comb_all(const Sums &s) {
  return combine3(s.a0 + s.b0, s.a1 + s.b1, s.a2 + s.b2);
}

constexpr uint32_t kHi = 0xF0F0F0F0u, kLo = 0x0F0F0F0Fu;

/* ------------------------------------------------------------------------
 * Formats. Each provides the lane-constant offsets of its planes (lane:
 * row r, chunk slot g) and the loads of a step whose first chunk is cb
 * (load), the weight operands of a step (bops), the scale factors of the
 * lane's chunk c (ws) and one token's scale step (apply) from its exact
 * plane sums over the step's two MFMAs and its chunk scale record
 * sc = {xs * kXsScale, sx0, sx1, sx}.
 * ---------------------------------------------------------------------- */
struct Offs {
  uint32_t q, aux, meta, d;
};
struct BOps {
  v4i b1, b2;
};

/* 16 s for the nibble fields of a word (s in the high nibble of a byte) */
__device__ __forceinline__ BOps nib16(const uint4 &q) {
  return {{(int)((q.x << 4) & kHi), (int)(q.x & kHi), (int)((q.y << 4) & kHi), (int)(q.y & kHi)},
          {(int)((q.z << 4) & kHi), (int)(q.z & kHi), (int)((q.w << 4) & kHi), (int)(q.w & kHi)}};
}

/* Q4_0, adapters/llama/gguf.c:680-694: value = (n - 8) d; stored s = n - 8.
 * B bytes are 16 s, hence xs / 16. */
struct Q40 {
  static constexpr float kXsScale = 0.0625f;
  struct Raw {
    uint4 q;
    uint16_t d;
  };
  struct WS {
    float d;
  };
  __device__ static Offs lane(const QRes &R, uint32_t r, uint32_t g) {
    return {r * R.q_stride + 16u * g, 0u, 0u, 2u * (r * R.nb + g)};
  }
  __device__ static Raw load(const QRes &R, const Offs &o, uint32_t row0, uint32_t cb) {
    Raw w;
    w.q = bl16(R.q, o.q, row0 * R.q_stride + 16u * cb);
    w.d = bl2(R.d, o.d, 2u * (row0 * R.nb + cb));
    return w;
  }
  __device__ static BOps bops(const Raw &w) { return nib16(w.q); }
  __device__ static WS ws(const Raw &w, uint32_t) { return {h2f(w.d)}; }
  __device__ static float apply(const WS &f, const Sums &s, const float4 &sc) {
    return (f.d * sc.x) * comb_all(s);
  }
};

/* Q4_K, adapters/llama/gguf.c:852-882: value = d1 n - m1 with d1 = d sc_j,
 * m1 = dmin m_j for sub-block j = c % 8; stored s = n - 8, B bytes 16 s.
 * sum (d1 n - m1) x = d1 xs (sum 16 s xq) / 16 + (8 d1 - m1) sum x. */
struct Q4K {
  static constexpr float kXsScale = 0.0625f;
  struct Raw {
    uint4 q, m;
  };
  struct WS {
    float d1, b;
  };
  __device__ static Offs lane(const QRes &R, uint32_t r, uint32_t g) {
    return {r * R.q_stride + 16u * g, 0u, 16u * r * R.nb, 0u};
  }
  __device__ static Raw load(const QRes &R, const Offs &o, uint32_t row0, uint32_t cb) {
    Raw w;
    w.q = bl16(R.q, o.q, row0 * R.q_stride + 16u * cb);
    w.m = bl16(R.meta, o.meta, 16u * (row0 * R.nb + (cb >> 3)));
    return w;
  }
  __device__ static BOps bops(const Raw &w) { return nib16(w.q); }
  __device__ static WS ws(const Raw &w, uint32_t c) {
    uint32_t s6, m6;
    scale_min_k4(c & 7u, w.m.y, w.m.z, w.m.w, s6, m6);
    const float d1 = h2f_lo(w.m.x) * (float)s6;
    const float m1 = h2f_hi(w.m.x) * (float)m6;
    return {d1, fmaf(8.0f, d1, -m1)};
  }
  __device__ static float apply(const WS &f, const Sums &s, const float4 &sc) {
    return fmaf(f.d1 * sc.x, comb_all(s), f.b * sc.w);
  }
};

/* Q6_K, adapters/llama/gguf.c:920-947: value = d sc (q - 32) with a scale
 * per 16 columns; B bytes are the 6-bit codes q, so each half chunk is
 * d sc (xs sum q xq - 32 sum x). */
struct Q6K {
  static constexpr float kXsScale = 1.0f;
  struct Raw {
    uint4 ql;
    uint2 qh;
    uint16_t sc, d;
  };
  struct WS {
    float f0, f1;
  };
  __device__ static Offs lane(const QRes &R, uint32_t r, uint32_t g) {
    return {r * R.q_stride + 16u * g, r * R.k4 + 8u * g, 16u * r * R.nb + 2u * g, 2u * r * R.nb};
  }
  __device__ static Raw load(const QRes &R, const Offs &o, uint32_t row0, uint32_t cb) {
    Raw w;
    const uint32_t blk = row0 * R.nb + (cb >> 3);
    w.ql = bl16(R.q, o.q, row0 * R.q_stride + 16u * cb);
    w.qh = bl8(R.aux, o.aux, row0 * R.k4 + 8u * cb);
    w.sc = bl2(R.meta, o.meta, 16u * blk + 2u * (cb & 7u));
    w.d = bl2(R.d, o.d, 2u * blk);
    return w;
  }
  /* codes of columns 8j..8j+3 (lo) and 8j+4..8j+7 (hi) from the low-bit
   * nibble word and the high-bit nibble word of word j */
  __device__ static int code_lo(uint32_t ql, uint32_t h) {
    return (int)(((ql ^ 0x88888888u) & kLo) | ((h << 4) & 0x30303030u));
  }
  __device__ static int code_hi(uint32_t ql, uint32_t h) {
    return (int)((((ql ^ 0x88888888u) >> 4) & kLo) | (h & 0x30303030u));
  }
  __device__ static BOps bops(const Raw &w) {
    const uint32_t h0 = w.qh.x & 0x33333333u, h1 = (w.qh.x >> 2) & 0x33333333u;
    const uint32_t h2 = w.qh.y & 0x33333333u, h3 = (w.qh.y >> 2) & 0x33333333u;
    return {{code_lo(w.ql.x, h0), code_hi(w.ql.x, h0), code_lo(w.ql.y, h1), code_hi(w.ql.y, h1)},
            {code_lo(w.ql.z, h2), code_hi(w.ql.z, h2), code_lo(w.ql.w, h3), code_hi(w.ql.w, h3)}};
  }
  __device__ static WS ws(const Raw &w, uint32_t) {
    const float d = h2f(w.d);
    return {d * (float)(int32_t)(int8_t)(w.sc & 0xFFu), d * (float)(int32_t)(int8_t)(w.sc >> 8)};
  }
  __device__ static float apply(const WS &f, const Sums &s, const float4 &sc) {
    const float t0 = fmaf(combine3(s.a0, s.a1, s.a2), sc.x, -32.0f * sc.y);
    const float t1 = fmaf(combine3(s.b0, s.b1, s.b2), sc.x, -32.0f * sc.z);
    return fmaf(f.f0, t0, f.f1 * t1);
  }
};

/* Q8_0, adapters/llama/gguf.c:750-761: value = code d. The int8 code is
 * rebuilt from its stored nibbles: low nibble l = field ^ 8, high nibble h
 * (signed), code = 16 h + l. */
struct Q80 {
  static constexpr float kXsScale = 1.0f;
  struct Raw {
    uint4 lo, hi;
    uint16_t d;
  };
  struct WS {
    float d;
  };
  __device__ static Offs lane(const QRes &R, uint32_t r, uint32_t g) {
    return {r * R.q_stride + 32u * g, 0u, 0u, 2u * (r * R.nb + g)};
  }
  __device__ static Raw load(const QRes &R, const Offs &o, uint32_t row0, uint32_t cb) {
    Raw w;
    const uint32_t so = row0 * R.q_stride + 32u * cb;
    w.lo = bl16(R.q, o.q, so);
    w.hi = bl16(R.q, o.q + 16u, so);
    w.d = bl2(R.d, o.d, 2u * (row0 * R.nb + cb));
    return w;
  }
  __device__ static int code_lo(uint32_t l, uint32_t h) {
    return (int)(((l ^ 0x88888888u) & kLo) | ((h << 4) & kHi));
  }
  __device__ static int code_hi(uint32_t l, uint32_t h) {
    return (int)((((l ^ 0x88888888u) >> 4) & kLo) | (h & kHi));
  }
  __device__ static BOps bops(const Raw &w) {
    return {{code_lo(w.lo.x, w.hi.x), code_hi(w.lo.x, w.hi.x), code_lo(w.lo.y, w.hi.y),
             code_hi(w.lo.y, w.hi.y)},
            {code_lo(w.lo.z, w.hi.z), code_hi(w.lo.z, w.hi.z), code_lo(w.lo.w, w.hi.w),
             code_hi(w.lo.w, w.hi.w)}};
  }
  __device__ static WS ws(const Raw &w, uint32_t) { return {h2f(w.d)}; }
  __device__ static float apply(const WS &f, const Sums &s, const float4 &sc) {
    return (f.d * sc.x) * comb_all(s);
  }
};

/* ------------------------------------------------------------------------
 * Activation planes of nct = MT * nch4 chunk-tokens into LDS: four threads
 * per chunk-token, eight columns each. Loads first (issued before the
 * weight ring), then the conversion.
 * ---------------------------------------------------------------------- */
template <int XI>
__device__ __forceinline__ void x_load(const float *__restrict__ x, uint32_t k, uint32_t ntok,
                                       uint32_t nch, uint32_t nch4, uint32_t nct,
                                       float4 (&va)[XI], float4 (&vb)[XI]) {
#pragma unroll
  for (int it = 0; it < XI; ++it) {
    const uint32_t idx = threadIdx.x + (uint32_t)it * blockDim.x;
    const uint32_t ct = idx >> 2, t = ct / nch4, c = ct % nch4;
    /* idle threads load nothing (a shared clamped address would make the
     * L2 serve one line to every idle thread of every workgroup in turn) */
    const bool ok = ct < nct && t < ntok && c < nch;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
    if (ok) {
      const float4 *src = reinterpret_cast<const float4 *>(x + (size_t)t * k + 32u * c + 8u * (idx & 3u));
      a = src[0];
      b = src[1];
    }
    va[it] = a;
    vb[it] = b;
  }
}

template <int L>
__device__ __forceinline__ float dppf(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), L, 0xF, 0xF, false));
}
template <int L>
__device__ __forceinline__ int dppi(int v) {
  return __builtin_amdgcn_update_dpp(0, v, L, 0xF, 0xF, false);
}
constexpr int kQuadXor1 = 0xB1, kQuadXor2 = 0x4E;

template <int XI>
__device__ __forceinline__ void x_planes(uint32_t nct, float xs_scale, const float4 (&va)[XI],
                                         const float4 (&vb)[XI], uint8_t *lds) {
#pragma unroll
  for (int it = 0; it < XI; ++it) {
    const uint32_t idx = threadIdx.x + (uint32_t)it * blockDim.x;
    if (idx < 4u * nct) { /* whole quads are in or out together */
      const uint32_t ct = idx >> 2, j = idx & 3u;
      const float v[8] = {va[it].x, va[it].y, va[it].z, va[it].w,
                          vb[it].x, vb[it].y, vb[it].z, vb[it].w};
      float m = 0.0f, sa = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        m = fmaxf(m, fabsf(v[i])); /* fmaxf drops NaNs ... */
        sa += fabsf(v[i]);         /* ... which this sum keeps */
      }
      m = fmaxf(m, dppf<kQuadXor1>(m));
      m = fmaxf(m, dppf<kQuadXor2>(m));
      int bad = !(m <= 3.402823466e38f) || sa != sa;
      bad |= dppi<kQuadXor1>(bad);
      bad |= dppi<kQuadXor2>(bad);
      const int e = m > 0.0f ? __builtin_amdgcn_frexp_expf(m) : 0;
      const int sh = bad ? 0 : 22 - e;
      uint32_t u[8];
      int sq = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int q = bad ? 0 : (int)rintf(__builtin_amdgcn_ldexpf(v[i], sh));
        sq += q;
        u[i] = ((uint32_t)q + 0x808080u) ^ 0x808080u; /* bytes 0..2: signed digits */
      }
      /* plane p word = byte p of four consecutive columns */
      const uint32_t a01 = __builtin_amdgcn_perm(u[1], u[0], 0x05010400u);
      const uint32_t b01 = __builtin_amdgcn_perm(u[1], u[0], 0x0C0C0602u);
      const uint32_t a23 = __builtin_amdgcn_perm(u[3], u[2], 0x05010400u);
      const uint32_t b23 = __builtin_amdgcn_perm(u[3], u[2], 0x0C0C0602u);
      const uint32_t a45 = __builtin_amdgcn_perm(u[5], u[4], 0x05010400u);
      const uint32_t b45 = __builtin_amdgcn_perm(u[5], u[4], 0x0C0C0602u);
      const uint32_t a67 = __builtin_amdgcn_perm(u[7], u[6], 0x05010400u);
      const uint32_t b67 = __builtin_amdgcn_perm(u[7], u[6], 0x0C0C0602u);
      uint2 *pl = reinterpret_cast<uint2 *>(lds + ct * kPlaneBytes + 8u * j);
      pl[0] = make_uint2(__builtin_amdgcn_perm(a23, a01, 0x05040100u),
                         __builtin_amdgcn_perm(a67, a45, 0x05040100u));
      pl[4] = make_uint2(__builtin_amdgcn_perm(a23, a01, 0x07060302u),
                         __builtin_amdgcn_perm(a67, a45, 0x07060302u));
      pl[8] = make_uint2(__builtin_amdgcn_perm(b23, b01, 0x05040100u),
                         __builtin_amdgcn_perm(b67, b45, 0x05040100u));
      sq += dppi<kQuadXor1>(sq); /* threads 0+1: columns 0..15; 2+3: 16..31 */
      const float xs = bad ? __builtin_nanf("") : __builtin_amdgcn_ldexpf(1.0f, e - 22);
      const float sx = (float)sq * xs;
      const float sx_other = dppf<kQuadXor2>(sx);
      if (j == 0u) {
        float4 *rec = reinterpret_cast<float4 *>(lds + lds_scales(nct)) + ct;
        *rec = make_float4(xs * xs_scale, sx, sx_other, sx + sx_other);
      }
    }
  }
}

/* ------------------------------------------------------------------------
 * Tile shapes.
 *   T16  v_mfma_i32_16x16x64_i8: items of 16 rows and steps of 4 chunks;
 *        lane (r, g) = (l%16, l/16) loads chunk 4s + g of row r. One token
 *        per pair of MFMAs: A row 4g + p holds plane p of the token's chunk
 *        4s + g in k-set g (lanes 20g + p), and C lane (r, g) receives the
 *        plane sums of its chunk in elements 0..2.
 *   T32  v_mfma_i32_32x32x32_i8: items of 32 rows and steps of 2 chunks;
 *        lane (r, g) = (l%32, l/32). Four tokens per pair of MFMAs: A row
 *        8q + 4g + p holds plane p of token q's chunk 2s + g in k-set g
 *        (lanes 8q + 36g + p), and C lane (r, g) receives token q's plane
 *        sums of its chunk in elements 4q..4q+2. One A operand serves four
 *        tokens, which cuts the activation reads from LDS fourfold.
 * ---------------------------------------------------------------------- */
struct T16 {
  static constexpr uint32_t RI = 16, CPS = 4, TPM = 1;
  typedef v4i C;
  __device__ static C mfma(v4i a, v4i b, C c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  }
  __device__ static uint32_t row(uint32_t l) { return l & 15u; }
  __device__ static uint32_t slot(uint32_t l) { return l >> 4; }
  __device__ static bool a_lane(uint32_t l, uint32_t &q, uint32_t &g, uint32_t &p) {
    q = 0u;
    g = l / 20u;
    p = l % 20u;
    return p < 3u;
  }
  /* the chunk slots of a row: lanes r, r + 16, r + 32, r + 48 */
  __device__ static float slot_sum(float v) {
    v += __shfl_xor(v, 16, 64);
    return v + __shfl_xor(v, 32, 64);
  }
};
struct T32 {
  static constexpr uint32_t RI = 32, CPS = 2, TPM = 4;
  typedef v16i C;
  __device__ static C mfma(v4i a, v4i b, C c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
  __device__ static uint32_t row(uint32_t l) { return l & 31u; }
  __device__ static uint32_t slot(uint32_t l) { return l >> 5; }
  __device__ static bool a_lane(uint32_t l, uint32_t &q, uint32_t &g, uint32_t &p) {
    g = l >= 36u ? 1u : 0u;
    const uint32_t rem = l - 36u * g;
    q = rem >> 3;
    p = rem & 7u;
    return p < 3u && q < 4u;
  }
  /* the chunk slots of a row: lanes r, r + 32 */
  __device__ static float slot_sum(float v) { return v + __shfl_xor(v, 32, 64); }
};

/* the tile shape of a launch of MT tokens */
template <int MT>
using TileOf = typename std::conditional<(MT >= 4), T32, T16>::type;

struct Args {
  paik_qview_t v[kMaxMats];
  float *y[kMaxMats];
  uint32_t item_end[kMaxMats]; /* cumulative items per matrix */
  uint32_t count;
  uint32_t items; /* total items */
};

template <class F, bool PAIR, int MT>
__global__ void __launch_bounds__(64 * waves<MT>()) k_gemv_mx(Args a, const float *__restrict__ x,
                                                              uint32_t ntok) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  using T = TileOf<MT>;
  constexpr int R = ring<F, MT>();
  constexpr int NW = waves<MT>(), XI = xit<NW>();
  constexpr uint32_t RI = T::RI, HALF = RI / 2u;
  constexpr int NG = MT / (int)T::TPM; /* token groups, one accumulator each */
  static_assert(MT % (int)T::TPM == 0, "whole token groups");
  const uint32_t k = a.v[0].k, nch = k >> 5;
  const uint32_t nsteps = nch / T::CPS, nct = (uint32_t)MT * nch;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const uint32_t r = T::row(lane), g = T::slot(lane);

  /* the workgroup's items and this wave's steps of each */
  const uint32_t i_beg = (uint32_t)((uint64_t)blockIdx.x * a.items / gridDim.x);
  const uint32_t i_end = (uint32_t)((uint64_t)(blockIdx.x + 1u) * a.items / gridDim.x);
  const uint32_t ni = i_end - i_beg;
  const uint32_t s_beg = wave * nsteps / NW, s_end = (wave + 1u) * nsteps / NW;
  const uint32_t spw = s_end - s_beg;
  const uint32_t nunits = ni * spw;

  /* Load cursor: the item and step of the next load, with the buffer
   * resources of the item's matrix (or of gate and up) and the lane
   * offsets. Lanes of an item's rows past the matrix end read its last row
   * (a paired item's lanes r and r + RI/2 read row r % (RI/2) of gate and
   * up), so every load stays inside the planes. Past the wave's last unit
   * the cursor repeats the last item's steps (s_beg < nsteps for every
   * wave), so every wave issues the same loads. */
  struct Cur {
    uint32_t it, s;
    QRes r0, r1;
    uint32_t row0;
    Offs o;
  } L;
  const uint32_t rl = PAIR ? (r & (HALF - 1u)) : r;
  const Offs off_full = F::lane(make_qres(a.v[0]), rl, g); /* strides agree across matrices */
  auto item_of = [&](uint32_t it, uint32_t &mi, uint32_t &row0) {
    if constexpr (PAIR) {
      mi = 0u;
      row0 = HALF * it;
    } else {
      uint32_t base = 0u;
      mi = 0u;
#pragma unroll
      for (uint32_t i = 1; i < kMaxMats; ++i)
        if (i < a.count && it >= a.item_end[i - 1]) {
          mi = i;
          base = a.item_end[i - 1];
        }
      row0 = RI * (it - base);
    }
  };
  auto enter = [&](uint32_t it) {
    uint32_t mi;
    item_of(it, mi, L.row0);
    L.it = it;
    L.r0 = make_qres(a.v[mi]);
    if constexpr (PAIR) L.r1 = make_qres(a.v[1]);
    const uint32_t n = a.v[mi].n;
    const uint32_t rows = PAIR ? HALF : RI;
    L.o = L.row0 + rows <= n ? off_full : F::lane(L.r0, min(rl, n - 1u - L.row0), g);
  };
  auto load_next = [&]() -> typename F::Raw {
    typename F::Raw w;
    const uint32_t cb = T::CPS * L.s;
    if constexpr (PAIR) {
      /* lanes of gate rows and of up rows load under complementary masks
       * into the same registers */
      if (r < HALF) w = F::load(L.r0, L.o, L.row0, cb);
      else w = F::load(L.r1, L.o, L.row0, cb);
    } else {
      w = F::load(L.r0, L.o, L.row0, cb);
    }
    if (++L.s >= s_end) {
      L.s = s_beg;
      if (L.it + 1u < i_end) enter(L.it + 1u);
    }
    return w;
  };

  /* activation loads, the first R steps of weights, then the planes; from
   * 4 tokens on the planes come first, so the activation registers are
   * free before the ring fills */
  constexpr bool kEarlyRing = MT <= 2;
  typename F::Raw buf[R];
  L.s = s_beg;
  enter(i_beg);
  {
    float4 xa[XI], xb[XI];
    x_load(x, k, ntok, nch, nch, nct, xa, xb);
    if constexpr (kEarlyRing) {
#pragma unroll
      for (int p = 0; p < R; ++p) buf[p] = load_next();
    }
    if (threadIdx.x < 8u) reinterpret_cast<uint32_t *>(lds + lds_zero(nct))[threadIdx.x] = 0u;
    x_planes(nct, F::kXsScale, xa, xb, lds);
  }
  if constexpr (!kEarlyRing) {
#pragma unroll
    for (int p = 0; p < R; ++p) buf[p] = load_next();
  }
  __syncthreads();

  /* A operand addresses: a carrying lane reads plane p of chunk
   * CPS s + ga of token TPM gi + q; the others read the zero block */
  uint32_t aq, ag, ap;
  const bool a_live = T::a_lane(lane, aq, ag, ap);
  const uint32_t a_base = a_live ? (aq * nch + ag) * kPlaneBytes + 32u * ap : lds_zero(nct);
  const uint32_t a_step = a_live ? T::CPS * kPlaneBytes : 0u;
  const uint32_t a_grp = a_live ? T::TPM * nch * kPlaneBytes : 0u;
  const float4 *scales = reinterpret_cast<const float4 *>(lds + lds_scales(nct));
  float *red = reinterpret_cast<float *>(lds + lds_red(nct));

  /* item end: the wave's partial sums of its rows into LDS slot it & 1, a
   * barrier, then threads 0 .. RI MT - 1 add the NW wave partials of one
   * (token, row) each and store the output */
  auto finish_item = [&](uint32_t it, const float (&acc)[MT]) {
    float *slot = red + (it & 1u) * (uint32_t)(NW * MT) * RI;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const float v = T::slot_sum(acc[t]);
      if (lane < RI) slot[(wave * MT + (uint32_t)t) * RI + lane] = v;
    }
    __syncthreads();
    const uint32_t th = threadIdx.x;
    if (th < RI * MT) {
      const uint32_t tt = th / RI, rr = th % RI;
      float sum = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) sum += slot[((uint32_t)w * MT + tt) * RI + rr];
      uint32_t mi, row0;
      item_of(it, mi, row0);
      if constexpr (PAIR) {
        const float up = __shfl_down(sum, HALF, RI); /* row rr + RI/2 of the item: the up sum */
        const uint32_t n = a.v[0].n, row = row0 + rr;
        if (rr < HALF && row < n && tt < ntok) a.y[0][(size_t)tt * n + row] = silu_mul(sum, up);
      } else {
        float *y = a.y[0];
#pragma unroll
        for (uint32_t i = 1; i < kMaxMats; ++i)
          if (mi == i) y = a.y[i];
        const uint32_t n = a.v[mi].n, row = row0 + rr;
        if (row < n && tt < ntok) y[(size_t)tt * n + row] = sum;
      }
    }
  };

  typename T::C c[NG];
  float acc[MT];
#pragma unroll
  for (int q = 0; q < NG; ++q) c[q] = typename T::C{};
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
  uint32_t ci = i_beg, cs = s_beg; /* compute cursor */
  auto compute = [&](const typename F::Raw &w) {
    const uint32_t cb = T::CPS * cs;
    const BOps b = F::bops(w);
    const typename F::WS f = F::ws(w, cb + g);
    const uint8_t *ap_ = lds + a_base + a_step * cs;
#pragma unroll
    for (int q = 0; q < NG; ++q) {
      const v4i a1 = *reinterpret_cast<const v4i *>(ap_ + a_grp * (uint32_t)q);
      const v4i a2 = *reinterpret_cast<const v4i *>(ap_ + a_grp * (uint32_t)q + 16u);
      const typename T::C c0 = c[q];
      const typename T::C c1 = T::mfma(a1, b.b1, c0);
      c[q] = T::mfma(a2, b.b2, c1);
#pragma unroll
      for (int e = 0; e < (int)T::TPM; ++e) {
        const int t = q * (int)T::TPM + e;
        const Sums sm = {c1[4 * e] - c0[4 * e],     c1[4 * e + 1] - c0[4 * e + 1],
                         c1[4 * e + 2] - c0[4 * e + 2], c[q][4 * e] - c1[4 * e],
                         c[q][4 * e + 1] - c1[4 * e + 1], c[q][4 * e + 2] - c1[4 * e + 2]};
        const float4 sc = scales[(uint32_t)t * nch + cb + g];
        acc[t] += F::apply(f, sm, sc);
      }
    }
    if (++cs == s_end) {
      finish_item(ci, acc);
#pragma unroll
      for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
      cs = s_beg;
      ++ci;
    }
  };
  /* Rounds of R steps: every round but the last refills each buffer right
   * after its step, the last only computes. Every load is unconditional,
   * so the compiler's wait before a step counts exactly the R - 1 steps
   * requested after it. */
  const uint32_t rounds = (nunits + (uint32_t)R - 1u) / (uint32_t)R;
  uint32_t u0 = 0;
  for (uint32_t rd = 1; rd < rounds; ++rd, u0 += (uint32_t)R) {
#pragma unroll
    for (int p = 0; p < R; ++p) {
      compute(buf[p]);
      buf[p] = load_next();
    }
  }
  if (rounds > 0u) {
#pragma unroll
    for (int p = 0; p < R; ++p)
      if (u0 + (uint32_t)p < nunits) compute(buf[p]);
  }
  if (spw == 0u) /* more waves than steps: zero partials, the same barriers */
    for (uint32_t i = i_beg; i < i_end; ++i) finish_item(i, acc);
}

template <class F, bool PAIR, int MT>
static hipError_t launch(const Args &a, const float *x, uint32_t ntok, hipStream_t s) {
  const uint32_t nch = a.v[0].k >> 5;
  const uint32_t grid = a.items < 256u ? a.items : 256u;
  constexpr int NW = waves<MT>();
  const size_t lds = lds_bytes((uint32_t)MT * nch, (uint32_t)MT, (uint32_t)NW, TileOf<MT>::RI);
  k_gemv_mx<F, PAIR, MT><<<dim3(grid), dim3(64u * NW), lds, s>>>(a, x, ntok);
  return hipGetLastError();
}

template <class F, bool PAIR>
static hipError_t launch_mt(const Args &a, const float *x, uint32_t mt, uint32_t ntok,
                            hipStream_t s) {
  switch (mt) {
  case 1u: return launch<F, PAIR, 1>(a, x, ntok, s);
  case 2u: return launch<F, PAIR, 2>(a, x, ntok, s);
  case 4u: return launch<F, PAIR, 4>(a, x, ntok, s);
  default: return launch<F, PAIR, 8>(a, x, ntok, s);
  }
}

template <bool PAIR>
static hipError_t dispatch(const Args &a, const float *x, uint32_t mt, uint32_t ntok,
                           hipStream_t s) {
  switch (a.v[0].type) {
  case 2u: return launch_mt<Q40, PAIR>(a, x, mt, ntok, s);
  case 8u: return launch_mt<Q80, PAIR>(a, x, mt, ntok, s);
  case 12u: return launch_mt<Q4K, PAIR>(a, x, mt, ntok, s);
  case 14u: return launch_mt<Q6K, PAIR>(a, x, mt, ntok, s);
  default: return hipErrorInvalidValue;
  }
}

/* LDS bytes a workgroup may allocate on the current device (read once) */
static size_t lds_max() {
  static size_t v = 0;
  if (v == 0) {
    int dev = 0, b = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&b, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      b = 65536;
    v = (size_t)b;
  }
  return v;
}

/* Tokens per launch for K and a call of m tokens: the smallest of 1, 2, 4,
 * 8 that covers m, halved until the planes fit the plane builder (1024
 * chunk-tokens) and the device's LDS; 0 when K is not a multiple of 128 or
 * even one token does not fit. */
static uint32_t tokens_for(uint32_t k, uint32_t m) {
  if ((k & 127u) != 0u || k == 0u) return 0u;
  const uint32_t nch = k >> 5;
  uint32_t mt = 1u;
  while (mt < m && mt < 8u) mt <<= 1;
  for (; mt >= 1u; mt >>= 1) {
    const uint32_t nw = mt <= 2u ? 16u : 8u, ri = mt >= 4u ? 32u : 16u;
    if (mt * nch <= kMaxChunkTok && lds_bytes(mt * nch, mt, nw, ri) <= lds_max()) return mt;
  }
  return 0u;
}

} // namespace mx
} // namespace paik

using namespace paik;

extern "C" uint32_t paik_gemv_mx_tokens(uint32_t k, uint32_t m) { return mx::tokens_for(k, m); }

extern "C" int paik_gemv_mx(const paik_qview_t *const *vs, float *const *ys, uint32_t count,
                            uint32_t m, const float *x, void *stream) {
  const uint32_t mt = mx::tokens_for(vs[0]->k, m);
  if (count == 0u || count > mx::kMaxMats || mt == 0u || m == 0u) return (int)hipErrorInvalidValue;
  const uint32_t ri = mt >= 4u ? 32u : 16u;
  mx::Args a;
  memset(&a, 0, sizeof a);
  a.count = count;
  uint32_t items = 0;
  for (uint32_t i = 0; i < count; ++i) {
    a.v[i] = *vs[i];
    items += (vs[i]->n + ri - 1u) / ri;
    a.item_end[i] = items;
  }
  a.items = items;
  for (uint32_t t0 = 0; t0 < m; t0 += mt) {
    for (uint32_t i = 0; i < count; ++i) a.y[i] = ys[i] + (size_t)t0 * vs[i]->n;
    const uint32_t nt = m - t0 < mt ? m - t0 : mt;
    const hipError_t e = mx::dispatch<false>(a, x + (size_t)t0 * vs[0]->k, mt, nt,
                                             (hipStream_t)stream);
    if (e != hipSuccess) return (int)e;
  }
  return 0;
}

extern "C" int paik_gemv_mx_silu_mul(const paik_qview_t *gate, const paik_qview_t *up, uint32_t m,
                                     const float *x, float *h, void *stream) {
  const uint32_t mt = mx::tokens_for(gate->k, m);
  if (mt == 0u || m == 0u) return (int)hipErrorInvalidValue;
  const uint32_t half = mt >= 4u ? 16u : 8u;
  mx::Args a;
  memset(&a, 0, sizeof a);
  a.count = 2;
  a.v[0] = *gate;
  a.v[1] = *up;
  a.items = (gate->n + half - 1u) / half;
  a.item_end[0] = a.items;
  for (uint32_t t0 = 0; t0 < m; t0 += mt) {
    a.y[0] = h + (size_t)t0 * gate->n;
    const uint32_t nt = m - t0 < mt ? m - t0 : mt;
    const hipError_t e = mx::dispatch<true>(a, x + (size_t)t0 * gate->k, mt, nt,
                                            (hipStream_t)stream);
    if (e != hipSuccess) return (int)e;
  }
  return 0;
}
