/*
 * Batched / prefill GEMM over packed blocks on MFMA (gfx950).
 *
 * y[M][N] = x[M][K] · Wᵀ with v_mfma_f32_32x32x16_{f16,bf16} and f32
 * accumulation: weights dequantized to fp16 (or bf16), activations
 * rounded once to the same type. Operand layout of the 32x32x16 form:
 * lane l supplies row l%32 of A and column l%32 of B, each with 8 K values
 * (k-set l/32).
 *
 * k_gemm_x16 / k_gemm (weights dequantized in registers). A workgroup owns
 * RWG weight rows x TT tokens (256 x 32, 256 x 128 on 8 waves; 128 x 256
 * on 4 waves); each wave owns RWG/NW rows as 32-row fragments and all TT
 * tokens, so no weight value is shared between waves and the weights never
 * pass through LDS: a lane fetches whole chunks into registers and turns
 * them into MFMA operands. A step covers 128 columns (four chunks per
 * row). Because every operand is already scaled, the two k-sets of one
 * MFMA need not come from the same chunk: lane (r, g) (r = l%32, g = l/32)
 * loads chunks 4s + 2u + g of row r (u = 0, 1), and MFMA (u, w) takes
 * nibble word w of that chunk (its columns 8w..8w+7) as the k-set, so one
 * 16-byte load feeds four MFMAs. Activations come from the 16-bit copy
 * k_cvt_x made (k_gemm_x16: staged into LDS by buffer_load ... lds DMA) or
 * from f32 x rounded through registers (k_gemm, without a workspace).
 *
 * k_gemm_lds (weights dequantized once per workgroup into LDS). A
 * workgroup owns 128 weight rows x 256 tokens on 8 waves; per 64-column
 * stage each thread dequantizes 16 columns of one row into the 16 KiB
 * weight tile (double-buffered) while the 32 KiB activation tile of a
 * later stage arrives by DMA (4 buffers), and every wave reads both MFMA
 * operands from LDS. Its weight loads are asm with waits written against
 * the registers they fill, with exact counts (the compiler cannot count
 * the asm DMA, and would otherwise wait for everything).
 *
 * Dequantization to 16 bits costs about two VALU operations per weight:
 * the 4-bit (or 6- and 8-bit) codes are gathered into bytes, v_perm_b32
 * turns byte pairs into the fp16 values 1024 + q, and v_fma_mix computes
 * (1024 + q) * s + b in f32 precision with one rounding to fp16, where
 * s, b fold the block scale, the code offset and (Q4_K) the block minimum:
 * value = s * q' + b equals the reference's f32 value to within one f32
 * rounding of b, far below the fp16 rounding that follows.
 *
 * Shapes with few tiles split K across workgroups: single-matrix launches
 * add their partial tiles into y (zeroed first) with f32 atomics, so with
 * more than two parts the last bits depend on the order of the adds;
 * multi-matrix launches store the parts in a workspace and sum them in a
 * fixed order (k_split_reduce).
 *
 * Workgroups are numbered so that the ones resident on one XCD (hardware
 * places workgroup i on XCD i % 8) take consecutive tiles of one token
 * tile: their activations are shared through that XCD's L2.
 */
#include <string.h>

#include <type_traits>

#include "qdev.h"

namespace paik {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 b8_t __attribute__((ext_vector_type(8)));
typedef float f16x_t __attribute__((ext_vector_type(16)));

constexpr int kKStep = 128;          /* columns per step */
constexpr int kXPitch = kKStep + 8;  /* LDS row pitch of the activation tile (16-bit units) */
constexpr int kXcds = 8;

template <bool BF>
__device__ __forceinline__ f16x_t mfma(const uint4 &a, const uint4 &b, f16x_t c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(b8_t, a),
                                                   __builtin_bit_cast(b8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8_t, a),
                                                  __builtin_bit_cast(h8_t, b), c, 0, 0, 0);
}

/* Two bytes of `bytes` (selector picks them) as the fp16 values 1024 + b. */
__device__ __forceinline__ uint32_t magic2(uint32_t bytes, uint32_t sel) {
  return __builtin_amdgcn_perm(0x64646464u, bytes, sel);
}
constexpr uint32_t kSel01 = 0x04010400u, kSel23 = 0x04030402u;

/* (1024 + q) * s + b for the two fp16 halves of m, as two 16-bit results
 * (fp16: the compiler emits v_fma_mixlo/hi_f16, f32 arithmetic with one
 * rounding to fp16; bf16: f32 FMA then a packed round-to-nearest-even
 * conversion). Written in plain C++ rather than asm so that the compiler
 * sees every register write (MFMA source hazards). */
template <bool BF>
__device__ __forceinline__ uint32_t scale2(uint32_t m, float s, float b) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  const h2_t h = __builtin_bit_cast(h2_t, m);
  const float lo = __builtin_fmaf((float)h[0], s, b), hi = __builtin_fmaf((float)h[1], s, b);
  if constexpr (BF) {
    typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
    const b2_t p = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, p);
  } else {
    const h2_t p = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, p);
  }
}

/* Operand of one nibble word: lo holds columns 0..3 (byte m = column m),
 * hi columns 4..7, as unsigned byte codes q; value = s * (1024 + q) + b. */
template <bool BF>
__device__ __forceinline__ uint4 word_op(uint32_t lo, uint32_t hi, float s, float b) {
  uint4 o;
  o.x = scale2<BF>(magic2(lo, kSel01), s, b);
  o.y = scale2<BF>(magic2(lo, kSel23), s, b);
  o.z = scale2<BF>(magic2(hi, kSel01), s, b);
  o.w = scale2<BF>(magic2(hi, kSel23), s, b);
  return o;
}

__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) {
  return (a & mask) | (b & ~mask);
}

/* Operands of a chunk, per format: scale<P>(w, c, ok) computes the f32
 * factors once per chunk (`ok` false gives zeros, for a chunk past the end
 * of the row; P = c / 4 % 2, the parity of the step, which fixes the half
 * of a Q4_K super-block the chunk lies in); word(w, j, sc) returns the
 * operand of nibble word j. */
template <class F, bool BF>
struct Ops;

template <bool BF>
struct Ops<Q4_0, BF> {
  struct Sc { float s, b; };
  template <int P>
  __device__ static Sc scale(const Q4_0::Raw &w, uint32_t, bool ok) {
    const float d = ok ? h2f(w.d) : 0.0f;
    return {d, -1032.0f * d}; /* d (n - 8), n = q */
  }
  __device__ static uint4 word(const Q4_0::Raw &w, int j, const Sc &sc) {
    const uint32_t u = word4(w.q, j) ^ 0x88888888u; /* stored n - 8 -> n */
    return word_op<BF>(u & 0x0F0F0F0Fu, (u >> 4) & 0x0F0F0F0Fu, sc.s, sc.b);
  }
};

template <bool BF>
struct Ops<Q4_K, BF> {
  struct Sc { float s, b; };
  template <int P>
  __device__ static Sc scale(const Q4_K::Raw &w, uint32_t c, bool ok) {
    float d1, m1;
    Q4_K::scales_half<P>(w, c & 3u, d1, m1);
    if (!ok) d1 = m1 = 0.0f;
    return {d1, -fmaf(1024.0f, d1, m1)}; /* d1 n - m1 */
  }
  __device__ static uint4 word(const Q4_K::Raw &w, int j, const Sc &sc) {
    const uint32_t u = word4(w.q, j) ^ 0x88888888u;
    return word_op<BF>(u & 0x0F0F0F0Fu, (u >> 4) & 0x0F0F0F0Fu, sc.s, sc.b);
  }
};

template <bool BF>
struct Ops<Q8_0, BF> {
  struct Sc { float s, b; };
  template <int P>
  __device__ static Sc scale(const Q8_0::Raw &w, uint32_t, bool ok) {
    const float d = ok ? h2f(w.d) : 0.0f;
    return {d, -1152.0f * d};
  }
  /* byte = l | (h + 8) << 4 = code + 128 */
  __device__ static uint4 word(const Q8_0::Raw &w, int j, const Sc &sc) {
    const uint32_t l = word4(w.lo, j) ^ 0x88888888u, h = word4(w.hi, j) ^ 0x88888888u;
    return word_op<BF>(bfi(0xF0F0F0F0u, h << 4, l), bfi(0xF0F0F0F0u, h, l >> 4), sc.s, sc.b);
  }
};

template <bool BF>
struct Ops<Q6_K, BF> {
  struct Sc { float s0, b0, s1, b1; }; /* columns 0..15, 16..31 */
  template <int P>
  __device__ static Sc scale(const Q6_K::Raw &w, uint32_t, bool ok) {
    const float d = ok ? h2f(w.d) : 0.0f;
    const float s0 = d * Q6_K::scale(w, 0), s1 = d * Q6_K::scale(w, 1);
    return {s0, -1056.0f * s0, s1, -1056.0f * s1}; /* d sc (q - 32) */
  }
  /* byte = l | h2 << 4 = q (0..63) */
  __device__ static uint4 word(const Q6_K::Raw &w, int j, const Sc &sc) {
    const uint32_t e = j < 2 ? w.qh.x : w.qh.y;
    const uint32_t h = ((j & 1) ? (e >> 2) : e) & 0x33333333u;
    const uint32_t l = word4(w.ql, j) ^ 0x88888888u;
    return word_op<BF>(bfi(0xF0F0F0F0u, h << 4, l), bfi(0xF0F0F0F0u, h, l >> 4),
                       j < 2 ? sc.s0 : sc.s1, j < 2 ? sc.b0 : sc.b1);
  }
};

__device__ __forceinline__ uint32_t cvt2(float a, float b, bool bf) {
  if (bf) {
    typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
    const b2_t p = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, p);
  }
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  const h2_t p = {(_Float16)a, (_Float16)b};
  return __builtin_bit_cast(uint32_t, p);
}

/* Chunk c of a row through the plane buffer resources, with per-lane row
 * and chunk (every lane of the GEMM has its own row). */
template <class F>
struct GLoad;
template <>
struct GLoad<Q4_0> {
  static constexpr int kLoads = 2; /* vector memory instructions per chunk */
  __device__ static Q4_0::Raw get(const QRes &r, uint32_t row, uint32_t c) {
    Q4_0::Raw w;
    w.q = bl16(r.q, row * r.q_stride + 16u * c, 0);
    w.d = bl2(r.d, (row * r.nb + c) * 2u, 0);
    return w;
  }
};
template <>
struct GLoad<Q8_0> {
  static constexpr int kLoads = 3;
  __device__ static Q8_0::Raw get(const QRes &r, uint32_t row, uint32_t c) {
    Q8_0::Raw w;
    const uint32_t o = row * r.q_stride + 32u * c;
    w.lo = bl16(r.q, o, 0);
    w.hi = bl16(r.q, o + 16u, 0);
    w.d = bl2(r.d, (row * r.nb + c) * 2u, 0);
    return w;
  }
};
template <>
struct GLoad<Q4_K> {
  static constexpr int kLoads = 2;
  __device__ static Q4_K::Raw get(const QRes &r, uint32_t row, uint32_t c) {
    Q4_K::Raw w;
    w.q = bl16(r.q, row * r.q_stride + 16u * c, 0);
    w.m = bl16(r.meta, (row * r.nb + (c >> 3)) * 16u, 0);
    return w;
  }
};
template <>
struct GLoad<Q6_K> {
  static constexpr int kLoads = 4;
  __device__ static Q6_K::Raw get(const QRes &r, uint32_t row, uint32_t c) {
    const uint32_t blk = row * r.nb + (c >> 3);
    Q6_K::Raw w;
    w.ql = bl16(r.q, row * r.q_stride + 16u * c, 0);
    w.qh = bl8(r.aux, row * r.k4 + 8u * c, 0);
    w.sc = bl2(r.meta, blk * 16u + 2u * (c & 7u), 0);
    w.d = bl2(r.d, blk * 2u, 0);
    return w;
  }
};

constexpr int kGemmMats = 4; /* matrices of one multi-matrix launch */
struct GemmArgs {
  paik_qview_t v;
  const float *x;
  const uint16_t *x16; /* activations already rounded to 16 bits (k_gemm_x16) */
  float *y;
  /* when set: y = silu(gate) * (x W^T), gate[M][N] the gate projection's
   * output (may be y itself; each element is read before it is written by
   * the same thread), and the launch is not split over K */
  const float *gate;
  uint32_t m;
  uint32_t tiles_n, tiles_m, splits; /* grid: tiles_n * tiles_m * splits (padded to kXcds) */
  uint32_t per_xcd;                  /* workgroups per XCD */
  uint32_t x_bytes;                  /* m * k * 4 (< 2^31) */
  uint32_t steps_per_split;
  /* k_gemm_x16 multi-matrix launches: matrices 0..count-1 (same format and
   * K, matrix 0 being v / y) own row tiles [tile_end[i-1], tile_end[i]) */
  uint32_t count;
  uint32_t tile_end[kGemmMats];
  paik_qview_t mv[kGemmMats];
  float *my[kGemmMats];
  /* split launches with a workspace: part p of matrix i's output goes to
   * part + splits * m * (rows of matrices 0..i-1) + p * m * n_i, and a
   * reduce launch sums the parts in order (no zero fill, no atomics) */
  float *part;
};

/* Tile shapes: TT tokens x RWG weight rows, NW waves of RWG/NW rows; XB
 * activation half-tiles held in registers (2: each half requested a full
 * step ahead; 1: the second half only half a step ahead, for tiles whose
 * halves are large; 4: a ring of four tiles, each requested two steps
 * ahead, for the small tiles of 32 tokens). */
template <class F, bool BF, int TT, int NW, int RWG, int XB>
__global__ void __launch_bounds__(64 * NW, 1) k_gemm(GemmArgs a) {
  constexpr int NT = 64 * NW;         /* threads */
  constexpr int RF = RWG / (32 * NW); /* 32-row fragments per wave */
  constexpr int RW = 32 * RF;             /* rows per wave */
  constexpr int JT = TT / 32;             /* 32-token fragments */
  constexpr int XI = TT * 32 / NT;        /* float4 of activations per thread per step */
  constexpr int XH = XI / 2;              /* ... per half step */
  static_assert(RF >= 1 && XH >= 1, "tile shape");
  /* activation double buffer; after the main loop, the output transpose
   * (NW waves x 32 tokens x (RW + 4) floats) */
  constexpr int kTP = RW + 4;
  constexpr int kTBytes = NW * 32 * kTP * 4;
  constexpr int kXsHalves = 4 * TT * kXPitch >= kTBytes ? TT * kXPitch : kTBytes / 4;
  __shared__ __attribute__((aligned(16))) uint16_t Xs[2][kXsHalves];

  /* tile of this workgroup: XCD-major numbering (see the top of the file) */
  const uint32_t logical = (blockIdx.x % kXcds) * a.per_xcd + blockIdx.x / kXcds;
  const uint32_t ntile = a.tiles_n * a.tiles_m;
  if (logical >= ntile * a.splits) return;
  const uint32_t split = logical / ntile, tile = logical % ntile;
  const uint32_t tn = tile % a.tiles_n, tm = tile / a.tiles_n;
  /* the matrix owning row tile tn (multi-matrix launches, as k_gemm_x16) */
  paik_qview_t v = a.v;
  float *ybase = a.y;
  uint32_t tl = tn, rows_before = 0, cum = 0;
#pragma unroll
  for (int i = 1; i < kGemmMats; ++i) {
    cum += a.mv[i - 1].n;
    if ((uint32_t)i < a.count && tn >= a.tile_end[i - 1]) {
      v = a.mv[i];
      ybase = a.my[i];
      tl = tn - a.tile_end[i - 1];
      rows_before = cum;
    }
  }
  const uint32_t n0 = tl * (uint32_t)RWG, m0 = tm * (uint32_t)TT;
  const uint32_t nchunks = v.k >> 5;
  const uint32_t s0 = split * a.steps_per_split; /* < number of steps */
  const uint32_t s1 = s0 + a.steps_per_split;     /* multiple of 4, may pass the row end */

  const int tid = (int)threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, g = lane >> 5;

  /* this lane's weight rows (one per 32-row fragment), clamped for loads */
  uint32_t rows[RF];
#pragma unroll
  for (int i = 0; i < RF; ++i)
    rows[i] = min(n0 + (uint32_t)(RW * wave + 32 * i + r), v.n - 1u);

  const QRes res = make_qres(v);
  typedef typename F::Raw Raw;
  /* chunk 4s + 2u + g of each of the lane's rows, u = 0, 1 */
  auto load_w = [&](uint32_t s, Raw (&dst)[2 * RF]) {
#pragma unroll
    for (int i = 0; i < RF; ++i)
#pragma unroll
      for (int u = 0; u < 2; ++u)
        dst[2 * i + u] = GLoad<F>::get(res, rows[i], min(4u * s + 2u * u + (uint32_t)g, nchunks - 1u));
  };
  /* Activation tile of a step (TT tokens x 128 columns): item tid + NT e
   * is the float4 at token item / 32, columns 4 (item % 32) .. +3, so 32
   * lanes read one token's 512 contiguous bytes. Tokens past m and
   * columns past k read as zero (offsets beyond the buffer resource). The
   * tile moves in two halves (items e < XH and e >= XH) so that only half
   * of it is held in registers at a time. */
  const __amdgpu_buffer_rsrc_t xres = plane_rsrc(a.x, a.x_bytes);
  const uint32_t xcol = 4u * ((uint32_t)tid & 31u), xt = (uint32_t)tid >> 5;
  uint32_t xoff[XI];
#pragma unroll
  for (int e = 0; e < XI; ++e) {
    const uint32_t tok = m0 + xt + (uint32_t)(NT / 32) * (uint32_t)e;
    xoff[e] = tok < a.m ? (tok * v.k + xcol) * 4u : 0x80000000u;
  }
  auto load_x = [&](uint32_t s, int h, float4 (&xr)[XH]) {
    const bool cok = kKStep * s + xcol < v.k;
#pragma unroll
    for (int e = 0; e < XH; ++e) {
      const uint32_t off = cok ? xoff[h * XH + e] : 0x80000000u;
      const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(xres, (int)off, (int)(512u * s), 0);
      /* element access by index: a bit cast of an ext-vector member (q.y)
       * is compiled as a cast of the vector's first element */
      xr[e] = make_float4(__uint_as_float(q[0]), __uint_as_float(q[1]), __uint_as_float(q[2]),
                          __uint_as_float(q[3]));
    }
  };
  auto store_x = [&](int buf, int h, const float4 (&xr)[XH]) {
#pragma unroll
    for (int e = 0; e < XH; ++e) {
      const uint32_t t = xt + (uint32_t)(NT / 32) * (uint32_t)(h * XH + e);
      uint2 p;
      p.x = cvt2(xr[e].x, xr[e].y, BF);
      p.y = cvt2(xr[e].z, xr[e].w, BF);
      *reinterpret_cast<uint2 *>(&Xs[buf][t * kXPitch + xcol]) = p;
    }
  };

  using Op = Ops<F, BF>;
  f16x_t acc[RF][JT];
#pragma unroll
  for (int i = 0; i < RF; ++i)
#pragma unroll
    for (int j = 0; j < JT; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  /* Step s: the raw chunks of step s (wc, requested two steps earlier)
   * are turned into operands just before their MFMAs, and those of step
   * s+2 are requested into wn; the activations of step s+1 (two register
   * halves, each requested a step earlier) move into the other LDS buffer,
   * each half followed by the request of the same half of step s+2.
   * XB = 4 holds the activations of steps s+1 and s+2 in a ring of four
   * register tiles (step t in slot t % 4) and requests those of step s+3:
   * vector memory results count down in issue order, so with one step of
   * activations in flight the wait for them at step s also waited for the
   * weights of step s+1, and the weights had about one step of lead
   * (32 tokens, q/k/v, o, gate/up, down: 94.2 -> 90.8 us per step). */
  float4 xr0[XH], xr1[XB == 2 ? XH : 1];
  float4 (&xrh)[XH] = *reinterpret_cast<float4 (*)[XH]>(XB == 2 ? &xr1[0] : &xr0[0]);
  float4 xq[XB == 4 ? 4 : 1][2][XH];
  auto step = [&](auto kk, uint32_t s, const Raw (&wc)[2 * RF], Raw (&wn)[2 * RF]) {
    constexpr int KK = decltype(kk)::value;    /* (s - s0) % 4 */
    constexpr int P = KK & 1; /* s % 2 (s0 % 4 == 0) */
    constexpr int cur = P;
    load_w(s + 2u, wn);
    typename Op::Sc sc[2 * RF];
#pragma unroll
    for (int q = 0; q < 2 * RF; ++q) {
      const uint32_t c = 4u * s + 2u * (uint32_t)(q & 1) + (uint32_t)g;
      sc[q] = Op::template scale<P>(wc[q], c, c < nchunks);
    }
    /* eight sub-steps k = 4u + w (chunk pair u, nibble word w): the
     * activation operands of sub-step k+1 are read from LDS before the
     * MFMAs of sub-step k, and its weight operands are dequantized after
     * them, so both overlap the matrix work */
    auto opsB = [&](int k, uint4 (&b)[JT]) {
#pragma unroll
      for (int j = 0; j < JT; ++j)
        b[j] = *reinterpret_cast<const uint4 *>(
            &Xs[cur][(32 * j + r) * kXPitch + 32 * (2 * (k >> 2) + g) + 8 * (k & 3)]);
    };
    auto opsA = [&](int k, uint4 (&A)[RF]) {
#pragma unroll
      for (int i = 0; i < RF; ++i) A[i] = Op::word(wc[2 * i + (k >> 2)], k & 3, sc[2 * i + (k >> 2)]);
    };
    uint4 Ac[RF], bc[JT];
    opsB(0, bc);
    opsA(0, Ac);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      uint4 An[RF], bn[JT];
      if (k < 7) opsB(k + 1, bn);
#pragma unroll
      for (int j = 0; j < JT; ++j)
#pragma unroll
        for (int i = 0; i < RF; ++i) acc[i][j] = mfma<BF>(Ac[i], bc[j], acc[i][j]);
      if (k < 7) opsA(k + 1, An);
      if (k == 3 && XB == 4) {
        store_x(cur ^ 1, 0, xq[(KK + 1) & 3][0]);
        load_x(s + 3u, 0, xq[(KK + 3) & 3][0]);
      } else if (k == 3) {
        store_x(cur ^ 1, 0, xr0);
        if constexpr (XB == 2) load_x(s + 2u, 0, xr0);
        else load_x(s + 1u, 1, xr0);
      }
      if (k < 7) {
#pragma unroll
        for (int i = 0; i < RF; ++i) Ac[i] = An[i];
#pragma unroll
        for (int j = 0; j < JT; ++j) bc[j] = bn[j];
      }
    }
    if constexpr (XB == 4) {
      store_x(cur ^ 1, 1, xq[(KK + 1) & 3][1]);
      load_x(s + 3u, 1, xq[(KK + 3) & 3][1]);
    } else {
      store_x(cur ^ 1, 1, xrh);
      if constexpr (XB == 2) load_x(s + 2u, 1, xrh);
      else load_x(s + 2u, 0, xrh);
    }
    __syncthreads();
  };

  /* The step range [s0, s1) has a length divisible by 4; steps at or past
   * the end of the row have zero operands (scale 0, activations read as
   * 0). The loads issued in the last steps are not used. */
  Raw w0[2 * RF], w1[2 * RF], w2[2 * RF], w3[2 * RF];
  load_w(s0, w0);
  load_w(s0 + 1u, w1);
  if constexpr (XB == 4) {
    load_x(s0, 0, xq[0][0]);
    load_x(s0, 1, xq[0][1]);
    store_x(0, 0, xq[0][0]);
    store_x(0, 1, xq[0][1]);
#pragma unroll
    for (int t = 1; t <= 2; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h) load_x(s0 + (uint32_t)t, h, xq[t][h]);
  } else {
    load_x(s0, 0, xr0);
    store_x(0, 0, xr0);
    load_x(s0, 1, xrh);
    store_x(0, 1, xrh);
    load_x(s0 + 1u, 0, xr0);
    if constexpr (XB == 2) load_x(s0 + 1u, 1, xrh);
  }
  __syncthreads();
  /* four steps per iteration: the four raw-chunk buffers rotate without
   * register copies, and the body has no branch, so each load is waited
   * for only where its data is used */
  for (uint32_t s = s0; s < s1; s += 4u) {
    step(std::integral_constant<int, 0>(), s, w0, w2);
    step(std::integral_constant<int, 1>(), s + 1u, w1, w3);
    step(std::integral_constant<int, 2>(), s + 2u, w2, w0);
    step(std::integral_constant<int, 3>(), s + 3u, w3, w1);
  }

  /* D of v_mfma_f32_32x32x16: lane (r, g) holds rows 8 (e/4) + 4 g + e % 4
   * of the 32-row fragment, token r of the 32-token fragment. Each
   * 32-token fragment is transposed through LDS (the activation buffers
   * are free after the last barrier), so that a lane then owns one row and
   * every store or atomic add of a wave covers RW consecutive outputs of
   * one token. */
  const bool split_k = a.splits > 1u;
  const bool gated = a.gate != nullptr && !split_k;
  float *const pbase = a.part != nullptr ? a.part + (size_t)a.splits * a.m * rows_before +
                                                (size_t)split * a.m * v.n
                                          : nullptr;
  float *Ts = reinterpret_cast<float *>(&Xs[0][0]) + wave * (32 * kTP);
  constexpr int TPI = 64 / RW; /* tokens per read-out instruction */
  const uint32_t orow = n0 + (uint32_t)(RW * wave + (lane % RW));
#pragma unroll
  for (int j = 0; j < JT; ++j) {
#pragma unroll
    for (int i = 0; i < RF; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float4 *>(&Ts[r * kTP + 32 * i + 8 * q + 4 * g]) =
            make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                        acc[i][j][4 * q + 3]);
    /* With the silu epilogue, the fragment's gate values are requested
     * together (clamped addresses) before its stores: one round trip per
     * fragment instead of one per store (the gate may be the output itself;
     * every element is read before this thread writes it). */
    constexpr int NQ = 32 / TPI;
    float gv[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) gv[q] = 0.0f;
    if (gated) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const uint32_t tok = min(m0 + (uint32_t)(32 * j + q * TPI + lane / RW), a.m - 1u);
        gv[q] = a.gate[(size_t)tok * v.n + min(orow, v.n - 1u)];
      }
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int tt = q * TPI + lane / RW;
      const float val = Ts[tt * kTP + lane % RW];
      const uint32_t tok = m0 + (uint32_t)(32 * j + tt);
      if (tok < a.m && orow < v.n) {
        const size_t at = (size_t)tok * v.n + orow;
        if (pbase != nullptr) pbase[at] = val;
        else if (split_k) unsafeAtomicAdd(ybase + at, val);
        else if (gated) ybase[at] = silu_mul(gv[q], val);
        else ybase[at] = val;
      }
    }
  }
}

/* s_waitcnt on the vector memory counter only (gfx9 encoding: vmcnt bits
 * 3:0 and 15:14; expcnt and lgkmcnt at their maximum, i.e. not waited). */
template <int N>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

/* x[m][k] f32 -> 16-bit copy (fp16 or bf16, round to nearest even), four
 * values per thread. */
/* (templates only so that every per-format unit may hold a copy) */
template <int = 0>
__global__ void __launch_bounds__(256) k_cvt_x(const float4 *__restrict__ x,
                                               uint2 *__restrict__ out, size_t n4, int bf) {
  const size_t stride = (size_t)gridDim.x * 256u;
  for (size_t i = (size_t)blockIdx.x * 256u + threadIdx.x; i < n4; i += stride) {
    const float4 f = x[i];
    uint2 p;
    p.x = cvt2(f.x, f.y, bf != 0);
    p.y = cvt2(f.z, f.w, bf != 0);
    out[i] = p;
  }
}

/* The same GEMM with the activations taken from their 16-bit copy and moved
 * from memory straight into LDS (buffer_load ... lds), so they use neither
 * registers nor VALU work. A tile row (token) of a step is 128 columns =
 * 256 bytes = 16 segments of 16 bytes; segment q of token t sits at position
 * q ^ (t % 16) of the row, which spreads the operand reads of 16 lanes (16
 * consecutive tokens, same segment) over all LDS banks. One DMA instruction
 * fills 4 token rows (1 KiB, lane l: token 4i + l/16, position l % 16). */
template <class F, bool BF, int TT, int NW, int RWG>
__global__ void __launch_bounds__(64 * NW, 1) k_gemm_x16(GemmArgs a) {
  constexpr int NT = 64 * NW;
  constexpr int RF = RWG / (32 * NW);
  constexpr int RW = 32 * RF;
  constexpr int JT = TT / 32;
  constexpr int XQ = TT / (4 * NW); /* DMA instructions per wave per step */
  constexpr int kTileBytes = TT * 256;
  constexpr int kTP = RW + 4;
  constexpr int kTBytes = NW * 32 * kTP * 4;
  constexpr int kLdsBytes = 2 * kTileBytes >= kTBytes ? 2 * kTileBytes : kTBytes;
  static_assert(RF >= 1 && XQ >= 1 && NT <= 512, "tile shape");
  __shared__ __attribute__((aligned(16))) uint8_t Xb[kLdsBytes];

  const uint32_t logical = (blockIdx.x % kXcds) * a.per_xcd + blockIdx.x / kXcds;
  const uint32_t ntile = a.tiles_n * a.tiles_m;
  if (logical >= ntile * a.splits) return;
  const uint32_t split = logical / ntile, tile = logical % ntile;
  const uint32_t tn = tile % a.tiles_n, tm = tile / a.tiles_n;
  /* the matrix owning row tile tn (workgroup-uniform) */
  paik_qview_t v = a.v;
  float *ybase = a.y;
  uint32_t tl = tn, rows_before = 0, cum = 0; /* rows of the matrices ahead of this one */
#pragma unroll
  for (int i = 1; i < kGemmMats; ++i) {
    cum += a.mv[i - 1].n;
    if ((uint32_t)i < a.count && tn >= a.tile_end[i - 1]) {
      v = a.mv[i];
      ybase = a.my[i];
      tl = tn - a.tile_end[i - 1];
      rows_before = cum;
    }
  }
  const uint32_t n0 = tl * (uint32_t)RWG, m0 = tm * (uint32_t)TT;
  const uint32_t nchunks = v.k >> 5;
  const uint32_t s0 = split * a.steps_per_split;
  const uint32_t s1 = s0 + a.steps_per_split;

  const int tid = (int)threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, g = lane >> 5;

  uint32_t rows[RF];
#pragma unroll
  for (int i = 0; i < RF; ++i)
    rows[i] = min(n0 + (uint32_t)(RW * wave + 32 * i + r), v.n - 1u);
  const QRes res = make_qres(v);
  typedef typename F::Raw Raw;
  constexpr int kWLoads = 2 * RF * GLoad<F>::kLoads; /* vector loads issued by load_w */
  auto load_w = [&](uint32_t s, Raw (&dst)[2 * RF]) {
#pragma unroll
    for (int i = 0; i < RF; ++i)
#pragma unroll
      for (int u = 0; u < 2; ++u)
        dst[2 * i + u] = GLoad<F>::get(res, rows[i], min(4u * s + 2u * u + (uint32_t)g, nchunks - 1u));
  };

  /* this lane's DMA items: instruction q moves token rows 4 (wave + NW q)
   * .. +3; the lane fills position p = lane % 16 of row t with segment
   * p ^ (t % 16) */
  const __amdgpu_buffer_rsrc_t xres = plane_rsrc(a.x16, a.x_bytes);
  uint32_t doff[XQ], dcol[XQ];
#pragma unroll
  for (int q = 0; q < XQ; ++q) {
    const uint32_t t = 4u * (uint32_t)(wave + NW * q) + ((uint32_t)lane >> 4);
    const uint32_t seg = ((uint32_t)lane & 15u) ^ (t & 15u);
    const uint32_t tok = m0 + t;
    dcol[q] = 8u * seg;
    doff[q] = tok < a.m ? (tok * v.k + 8u * seg) * 2u : 0x80000000u;
  }
  /* Written as asm rather than the buffer-load-to-LDS builtin: the compiler
   * cannot tell which LDS buffer a DMA writes and would wait for every
   * outstanding load before each LDS read; here the waits are explicit
   * (wait_vmem and the barrier at the end of a step). M0 (the LDS base of
   * the DMA) is saved and restored around the load. */
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)Xb;
  auto dma_x = [&](uint32_t s, int buf) {
#pragma unroll
    for (int q = 0; q < XQ; ++q) {
      /* columns past k read as zero (offset beyond the resource) */
      const uint32_t off = kKStep * s + dcol[q] < v.k ? doff[q] : 0x80000000u;
      const uint32_t dst = (uint32_t)__builtin_amdgcn_readfirstlane(
          (int)(lds0 + (uint32_t)(buf * kTileBytes + 4 * (wave + NW * q) * 256)));
      const uint32_t soff = (uint32_t)__builtin_amdgcn_readfirstlane((int)(256u * s));
      uint32_t saved;
      __asm__ volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %1\n\t"
          "s_nop 4\n\t"
          "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(saved)
          : "s"(dst), "v"(off), "s"(xres), "s"(soff)
          : "memory");
    }
  };

  using Op = Ops<F, BF>;
  f16x_t acc[RF][JT];
#pragma unroll
  for (int i = 0; i < RF; ++i)
#pragma unroll
    for (int j = 0; j < JT; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  /* Step s: the MFMAs run on the chunks of step s (wc) and the activation
   * tile of step s; after its second sub-step the activations of step s+1
   * are requested into the other LDS buffer and the raw chunks of step s+2
   * into wn; at the end, the wait leaves only the chunk loads outstanding
   * (so the DMA of step s+1 has landed) and the barrier publishes it. */
  auto step = [&](auto kk, uint32_t s, const Raw (&wc)[2 * RF], Raw (&wn)[2 * RF]) {
    constexpr int P = decltype(kk)::value & 1;
    const uint8_t *Xc = Xb + P * kTileBytes;
    typename Op::Sc sc[2 * RF];
#pragma unroll
    for (int q = 0; q < 2 * RF; ++q) {
      const uint32_t c = 4u * s + 2u * (uint32_t)(q & 1) + (uint32_t)g;
      sc[q] = Op::template scale<P>(wc[q], c, c < nchunks);
    }
    auto opsB = [&](int k, uint4 (&b)[JT]) {
      const int pos = (4 * (2 * (k >> 2) + g) + (k & 3)) ^ (r & 15);
#pragma unroll
      for (int j = 0; j < JT; ++j)
        b[j] = *reinterpret_cast<const uint4 *>(Xc + (32 * j + r) * 256 + pos * 16);
    };
    auto opsA = [&](int k, uint4 (&A)[RF]) {
#pragma unroll
      for (int i = 0; i < RF; ++i) A[i] = Op::word(wc[2 * i + (k >> 2)], k & 3, sc[2 * i + (k >> 2)]);
    };
    uint4 Ac[RF], bc[JT];
    opsB(0, bc);
    opsA(0, Ac);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      uint4 An[RF], bn[JT];
      if (k < 7) opsB(k + 1, bn);
#pragma unroll
      for (int j = 0; j < JT; ++j)
#pragma unroll
        for (int i = 0; i < RF; ++i) acc[i][j] = mfma<BF>(Ac[i], bc[j], acc[i][j]);
#ifndef PAI_GEMM_NO_SCHED
      if (k < 7) {
        /* order: the next sub-step's LDS reads, then each MFMA followed by
         * a few VALU operations (its dequantization work) */
        __builtin_amdgcn_sched_group_barrier(0x100, JT, 0);
#pragma unroll
        for (int q = 0; q < RF * JT; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
        }
      }
#endif
      if (k == 1) {
        /* issued after the first waits on this step's chunks, so those
         * waits do not cover them */
        dma_x(s + 1u, P ^ 1);
        load_w(s + 2u, wn);
      }
      if (k < 7) {
        opsA(k + 1, An);
#pragma unroll
        for (int i = 0; i < RF; ++i) Ac[i] = An[i];
#pragma unroll
        for (int j = 0; j < JT; ++j) bc[j] = bn[j];
      }
    }
    wait_vmem<kWLoads>();
    __syncthreads();
  };

  Raw w0[2 * RF], w1[2 * RF], w2[2 * RF], w3[2 * RF];
  dma_x(s0, 0);
  load_w(s0, w0);
  load_w(s0 + 1u, w1);
  wait_vmem<2 * kWLoads>();
  __syncthreads();
  for (uint32_t s = s0; s < s1; s += 4u) {
    step(std::integral_constant<int, 0>(), s, w0, w2);
    step(std::integral_constant<int, 1>(), s + 1u, w1, w3);
    step(std::integral_constant<int, 2>(), s + 2u, w2, w0);
    step(std::integral_constant<int, 3>(), s + 3u, w3, w1);
  }
  wait_vmem<0>(); /* the last steps' requests land before the LDS is reused */
  __syncthreads();

  const bool split_k = a.splits > 1u;
  const bool gated = a.gate != nullptr && !split_k;
  float *const pbase = a.part != nullptr ? a.part + (size_t)a.splits * a.m * rows_before +
                                                (size_t)split * a.m * v.n
                                          : nullptr;
  float *Ts = reinterpret_cast<float *>(Xb) + wave * (32 * kTP);
  constexpr int TPI = 64 / RW;
  const uint32_t orow = n0 + (uint32_t)(RW * wave + (lane % RW));
#pragma unroll
  for (int j = 0; j < JT; ++j) {
#pragma unroll
    for (int i = 0; i < RF; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<float4 *>(&Ts[r * kTP + 32 * i + 8 * q + 4 * g]) =
            make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                        acc[i][j][4 * q + 3]);
    /* With the silu epilogue, the fragment's gate values are requested
     * together (clamped addresses) before its stores: one round trip per
     * fragment instead of one per store (the gate may be the output itself;
     * every element is read before this thread writes it). */
    constexpr int NQ = 32 / TPI;
    float gv[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) gv[q] = 0.0f;
    if (gated) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const uint32_t tok = min(m0 + (uint32_t)(32 * j + q * TPI + lane / RW), a.m - 1u);
        gv[q] = a.gate[(size_t)tok * v.n + min(orow, v.n - 1u)];
      }
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int tt = q * TPI + lane / RW;
      const float val = Ts[tt * kTP + lane % RW];
      const uint32_t tok = m0 + (uint32_t)(32 * j + tt);
      if (tok < a.m && orow < v.n) {
        const size_t at = (size_t)tok * v.n + orow;
        if (pbase != nullptr) pbase[at] = val;
        else if (split_k) unsafeAtomicAdd(ybase + at, val);
        else if (gated) ybase[at] = silu_mul(gv[q], val);
        else ybase[at] = val;
      }
    }
  }
}

/* y[0 .. count) = 0 (a kernel, so that the call can be captured into a
 * graph). */
template <int = 0>
__global__ void __launch_bounds__(256) k_zero(float4 *__restrict__ y, size_t n4, float *tail,
                                              uint32_t ntail) {
  const size_t i = (size_t)blockIdx.x * 256u + threadIdx.x;
  if (i < n4) y[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (i < ntail) tail[i] = 0.0f;
}

static hipError_t zero_fill(float *y, size_t count, hipStream_t s) {
  const size_t head = ((16u - ((uintptr_t)y & 15u)) & 15u) / 4u; /* floats before 16-B alignment */
  const size_t pre = head < count ? head : count;
  const size_t n4 = (count - pre) / 4u, rest = count - pre - 4u * n4;
  /* the unaligned head and the tail: at most 6 floats, done by one thread each */
  if (pre) k_zero<><<<1, 256, 0, s>>>(nullptr, 0, y, (uint32_t)pre);
  if (rest) k_zero<><<<1, 256, 0, s>>>(nullptr, 0, y + pre + 4u * n4, (uint32_t)rest);
  if (n4) {
    const size_t blocks = (n4 + 255u) / 256u;
    k_zero<><<<dim3((unsigned)blocks), 256, 0, s>>>(reinterpret_cast<float4 *>(y + pre), n4,
                                                   nullptr, 0);
  }
  return hipGetLastError();
}

/* Grid of a launch: tiles of RWG rows x TT tokens; K split while the grid
 * would leave most of the 256 CUs idle (at least 8 steps per split, or 4
 * where there are more than two splits anyway), the step count per split a
 * multiple of 4. */
static void plan_grid(GemmArgs &a, uint32_t rwg, uint32_t tt) {
  if (a.count <= 1u) a.tiles_n = (a.v.n + rwg - 1u) / rwg; /* else set by the caller */
  a.tiles_m = (a.m + tt - 1u) / tt;
  const uint32_t tiles = a.tiles_n * a.tiles_m;
  const uint32_t nsteps = ((a.v.k >> 5) + 3u) >> 2;
  uint32_t splits = 1;
  while (tiles * splits * 2u <= 256u && nsteps / (splits * 2u) >= 8u) splits *= 2u;
  /* Sums of more than two parts already depend on the order of the atomic
   * adds; there the parts may be as short as 4 steps, which fills more of
   * the chip (one or two parts stay exact and repeatable). */
  if (splits > 2u)
    while (tiles * splits * 2u <= 256u && nsteps / (splits * 2u) >= 4u) splits *= 2u;
  if (paik_tune.gemm_splits >= 1 && paik_tune.gemm_splits <= 64)
    splits = (uint32_t)paik_tune.gemm_splits;
  if (a.gate != nullptr) splits = 1u; /* the epilogue needs whole sums */
  a.steps_per_split = (nsteps + splits - 1u) / splits;
  a.steps_per_split = (a.steps_per_split + 3u) & ~3u; /* the loop runs steps in fours */
  a.splits = (nsteps + a.steps_per_split - 1u) / a.steps_per_split;
  a.per_xcd = (tiles * a.splits + kXcds - 1u) / kXcds;
}

/* The split parts summed in part order (0, 1, ...): y_i[e] = sum_p
 * part[base_i + p * len_i + e], base_i = splits * (len_0 + ... + len_{i-1}),
 * len_i = m * n_i; e runs over all matrices' outputs back to back. */
struct ReduceArgs {
  const float *part;
  float *y[kGemmMats];
  size_t end[kGemmMats]; /* cumulative output lengths */
  uint32_t count, splits;
  uint32_t silu; /* gate/up pair: y[0][e] = silu(sum of matrix 0) * (sum of matrix 1) */
};
template <int = 0>
__global__ void __launch_bounds__(256) k_split_reduce(ReduceArgs r) {
  if (r.silu != 0u) { /* two matrices of equal length, one output */
    const size_t len = r.end[0];
    for (size_t e = (size_t)blockIdx.x * 256u + threadIdx.x; e < len; e += (size_t)gridDim.x * 256u) {
      const float *g = r.part + e, *u = r.part + (size_t)r.splits * len + e;
      float sg = g[0], su = u[0];
      for (uint32_t p = 1; p < r.splits; ++p) {
        sg += g[(size_t)p * len];
        su += u[(size_t)p * len];
      }
      r.y[0][e] = silu_mul(sg, su);
    }
    return;
  }
  const size_t total = r.end[r.count - 1];
  for (size_t e = (size_t)blockIdx.x * 256u + threadIdx.x; e < total; e += (size_t)gridDim.x * 256u) {
    uint32_t i = 0;
    size_t start = 0;
#pragma unroll
    for (int j = 1; j < kGemmMats; ++j)
      if ((uint32_t)j < r.count && e >= r.end[j - 1]) {
        i = (uint32_t)j;
        start = r.end[j - 1];
      }
    const size_t len = r.end[i] - start, off = e - start;
    const float *src = r.part + (size_t)r.splits * start + off;
    float acc = src[0];
    for (uint32_t p = 1; p < r.splits; ++p) acc += src[(size_t)p * len];
    float *yi = r.y[0];
#pragma unroll
    for (int j = 1; j < kGemmMats; ++j)
      if ((uint32_t)j == i) yi = r.y[j];
    yi[off] = acc;
  }
}

static hipError_t launch_reduce(float *part, float *const *ys, const uint32_t *ns, uint32_t count,
                                uint32_t m, uint32_t splits, hipStream_t s, bool silu = false) {
  ReduceArgs r;
  memset(&r, 0, sizeof r);
  r.part = part;
  r.silu = silu ? 1u : 0u;
  size_t cum = 0;
  for (uint32_t i = 0; i < count; ++i) {
    r.y[i] = ys[i];
    cum += (size_t)m * ns[i];
    r.end[i] = cum;
  }
  r.count = count;
  r.splits = splits;
  const size_t blocks = (cum + 255u) / 256u;
  k_split_reduce<><<<dim3((unsigned)(blocks < 4096u ? blocks : 4096u)), 256, 0, s>>>(r);
  return hipGetLastError();
}

/* Several matrices sharing x in one register-staged launch (as launch_x16
 * without the 16-bit copy): split parts go to the workspace and one reduce
 * launch sums them in order (silu_pair: forms silu(gate) * up). */
template <class F, int TT, int NW, int RWG, int XB>
static hipError_t launch_tt_multi(const paik_qview_t *const *vs, float *const *ys, uint32_t count,
                                  uint32_t m, const float *x, bool bf16, float *part,
                                  size_t part_bytes, bool silu_pair, hipStream_t s) {
  GemmArgs a;
  memset(&a, 0, sizeof a);
  a.v = *vs[0];
  a.x = x;
  a.y = ys[0];
  a.m = m;
  a.count = count;
  uint32_t tiles = 0;
  size_t rows = 0;
  uint32_t ns[kGemmMats];
  for (uint32_t i = 0; i < count; ++i) {
    a.mv[i] = *vs[i];
    a.my[i] = ys[i];
    tiles += (vs[i]->n + (uint32_t)RWG - 1u) / (uint32_t)RWG;
    a.tile_end[i] = tiles;
    ns[i] = vs[i]->n;
    rows += vs[i]->n;
  }
  a.tiles_n = tiles;
  plan_grid(a, RWG, TT);
  a.x_bytes = (uint32_t)((size_t)m * a.v.k * 4u);
  const bool parts = a.splits > 1u && part != nullptr &&
                     (size_t)a.splits * m * rows * 4u <= part_bytes;
  if (silu_pair && !parts) return hipErrorInvalidValue;
  if (parts) {
    a.part = part;
  } else if (a.splits > 1u) {
    for (uint32_t i = 0; i < count; ++i) {
      const hipError_t e = zero_fill(ys[i], (size_t)m * vs[i]->n, s);
      if (e != hipSuccess) return e;
    }
  }
  const dim3 grid(a.per_xcd * kXcds), block(64 * NW);
  if (bf16) k_gemm<F, true, TT, NW, RWG, XB><<<grid, block, 0, s>>>(a);
  else k_gemm<F, false, TT, NW, RWG, XB><<<grid, block, 0, s>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !parts) return e;
  return launch_reduce(part, ys, ns, count, m, a.splits, s, silu_pair);
}

template <class F, int TT, int NW, int RWG, int XB>
static hipError_t launch_tt(const paik_qview_t &v, uint32_t m, const float *x, float *y,
                            const float *gate, bool bf16, float *part, size_t part_bytes,
                            hipStream_t s) {
  GemmArgs a;
  memset(&a, 0, sizeof a);
  a.v = v;
  a.x = x;
  a.y = y;
  a.gate = gate;
  a.m = m;
  plan_grid(a, RWG, TT);
  a.x_bytes = (uint32_t)((size_t)m * v.k * 4u);
  const bool parts = a.splits > 1u && part != nullptr &&
                     (size_t)a.splits * m * v.n * 4u <= part_bytes;
  if (parts) {
    a.part = part;
  } else if (a.splits > 1u) {
    const hipError_t e = zero_fill(y, (size_t)m * v.n, s);
    if (e != hipSuccess) return e;
  }
  const dim3 grid(a.per_xcd * kXcds), block(64 * NW);
  if (bf16) k_gemm<F, true, TT, NW, RWG, XB><<<grid, block, 0, s>>>(a);
  else k_gemm<F, false, TT, NW, RWG, XB><<<grid, block, 0, s>>>(a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !parts) return e;
  const uint32_t n = v.n;
  return launch_reduce(part, &y, &n, 1u, m, a.splits, s);
}


/* ======================================================================
 * Prefill GEMM with the weights shared through LDS (k_gemm_lds, 256 tokens
 * and more per call).
 *
 * Workgroup: 8 waves (two per SIMD), 128 weight rows x 256 tokens. Each
 * 64-column stage, every thread dequantizes 16 weights (one row, one
 * quarter of the stage) once into the 16-bit weight tile, and the
 * activation tile (256 tokens x 64 columns of the 16-bit copy) moves into
 * LDS by DMA. Wave (wr, wt) = (wave % 2, wave / 2) then multiplies tokens
 * 64 wt .. 64 wt + 63 by rows 64 wr .. 64 wr + 63: 2 x 2 fragments of
 * v_mfma_f32_32x32x16 with the activations as A (32 tokens x 16 columns)
 * and the weights as B (16 columns x 32 rows), both read from LDS. A lane's
 * accumulator then holds one weight row for 16 tokens, so each store
 * instruction writes 2 x 128 contiguous bytes of y and no transpose is
 * needed.
 *
 * Why this shape: on gfx950 an MFMA loop that reads one 1 KiB LDS operand
 * per 32x32x16 MFMA reaches 0.82 of the matrix peak with two waves per
 * SIMD and 0.53-0.59 with one (probe), and dequantizing each weight once
 * per 256 tokens keeps the dequantization near 1.5 VALU operations per
 * MFMA. LDS: the weight tile double-buffered (2 x 16 KiB), the activation
 * tile in four buffers (4 x 32 KiB), 160 KiB in all; with the buffer
 * index of every stage known at compile time (the loop runs stages in
 * fours), each operand read is one instruction with an immediate offset.
 *
 * Pipeline per stage s: DMA of activations s+2, weight loads of stage s+4
 * (a ring of 4 register slots), the 16 MFMAs of stage s, dequantization of
 * stage s+1 into the other weight tile, then one barrier. The waits count
 * loads exactly (every wave issues the same sequence).
 * ==================================================================== */
namespace lg {
constexpr int BM = 128;                  /* weight rows per workgroup */
constexpr int BN = 256;                  /* tokens per workgroup */
constexpr int KS = 64;                   /* columns per stage */
constexpr int NW = 8;                    /* waves */
constexpr int NT = 64 * NW;
constexpr int kWTile = BM * KS * 2;      /* 16 KiB */
constexpr int kXTile = BN * KS * 2;      /* 32 KiB */
constexpr int kXDma = kXTile / 1024 / NW; /* DMA instructions per wave per stage */
constexpr int kRing = 4;                 /* weight-load stages in flight */
constexpr int kXBufs = 4;                /* activation tiles (stage s in buffer s % 4) */
constexpr int kLds = 2 * kWTile + kXBufs * kXTile;
static_assert(kLds <= 160 * 1024, "LDS");
} // namespace lg

/* Byte offset of 16-byte segment `seg` (columns 8 seg .. 8 seg + 7 of the
 * stage) of tile row `row`. Two rows share a 256-byte line, whose 16 slots
 * are permuted per line: the 16 rows a quarter-wave reads (one segment)
 * land in 16 distinct slots, i.e. on every LDS bank once, and any 8
 * consecutive rows in distinct slots modulo 128 bytes. */
__device__ __forceinline__ uint32_t lg_off(uint32_t row, uint32_t seg) {
  const uint32_t line = row >> 1;
  return line * 256u + (((((seg ^ line) & 7u) << 1) | (row & 1u)) << 4);
}

/* Weight loads of k_gemm_lds, written as asm so that the compiler's wait
 * insertion, which cannot count the activation DMA (also asm), leaves them
 * alone: the kernel waits for them itself (qq_wait), with exact counts. */
__device__ __forceinline__ u32x2 ql8(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  u32x2 v;
  __asm__ volatile("buffer_load_dwordx2 %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(r));
  return v;
}
__device__ __forceinline__ u32x4 ql16(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  u32x4 v;
  __asm__ volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(r));
  return v;
}
__device__ __forceinline__ uint32_t ql4(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  uint32_t v;
  __asm__ volatile("buffer_load_dword %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(r));
  return v;
}
__device__ __forceinline__ uint32_t ql2(__amdgpu_buffer_rsrc_t r, uint32_t voff) {
  uint32_t v;
  __asm__ volatile("buffer_load_ushort %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(r));
  return v;
}

/* 16 columns of one row (nibble words 2h and 2h+1 of chunk c): the raw
 * bytes as loaded (kLoads requests), a wait for them that also orders
 * their uses after it (wait<N>: vmcnt N, the registers as operands), and
 * their 16-bit values as two 8-column segments (value = s (1024 + q) + b
 * as in Ops; zeros when !ok). */
template <class F>
struct QQ;
template <>
struct QQ<Q4_0> {
  static constexpr int kLoads = 2;
  struct Raw { u32x2 q; uint32_t d; };
  __device__ static Raw get(const QRes &r, uint32_t row, uint32_t c, uint32_t h) {
    Raw w;
    w.q = ql8(r.q, row * r.q_stride + 16u * c + 8u * h);
    w.d = ql2(r.d, (row * r.nb + c) * 2u);
    return w;
  }
  template <int N>
  __device__ static void wait(Raw &w) {
    __asm__ volatile("s_waitcnt vmcnt(%2)" : "+v"(w.q), "+v"(w.d) : "i"(N));
  }
  template <bool BF, int HI>
  __device__ static void vals(const Raw &w, uint32_t, uint32_t, bool ok, uint4 &o0, uint4 &o1) {
    const float d = ok ? h2f((uint16_t)w.d) : 0.0f, b = -1032.0f * d;
    const uint32_t u0 = w.q[0] ^ 0x88888888u, u1 = w.q[1] ^ 0x88888888u;
    o0 = word_op<BF>(u0 & 0x0F0F0F0Fu, (u0 >> 4) & 0x0F0F0F0Fu, d, b);
    o1 = word_op<BF>(u1 & 0x0F0F0F0Fu, (u1 >> 4) & 0x0F0F0F0Fu, d, b);
  }
};
template <>
struct QQ<Q8_0> {
  static constexpr int kLoads = 3;
  struct Raw { u32x2 lo, hi; uint32_t d; };
  __device__ static Raw get(const QRes &r, uint32_t row, uint32_t c, uint32_t h) {
    const uint32_t o = row * r.q_stride + 32u * c + 8u * h;
    Raw w;
    w.lo = ql8(r.q, o);
    w.hi = ql8(r.q, o + 16u);
    w.d = ql2(r.d, (row * r.nb + c) * 2u);
    return w;
  }
  template <int N>
  __device__ static void wait(Raw &w) {
    __asm__ volatile("s_waitcnt vmcnt(%3)" : "+v"(w.lo), "+v"(w.hi), "+v"(w.d) : "i"(N));
  }
  template <bool BF>
  __device__ static uint4 word(uint32_t lo, uint32_t hi, float d, float b) {
    const uint32_t l = lo ^ 0x88888888u, h = hi ^ 0x88888888u; /* byte = code + 128 */
    return word_op<BF>(bfi(0xF0F0F0F0u, h << 4, l), bfi(0xF0F0F0F0u, h, l >> 4), d, b);
  }
  template <bool BF, int HI>
  __device__ static void vals(const Raw &w, uint32_t, uint32_t, bool ok, uint4 &o0, uint4 &o1) {
    const float d = ok ? h2f((uint16_t)w.d) : 0.0f, b = -1152.0f * d;
    o0 = word<BF>(w.lo[0], w.hi[0], d, b);
    o1 = word<BF>(w.lo[1], w.hi[1], d, b);
  }
};
template <>
struct QQ<Q4_K> {
  static constexpr int kLoads = 2;
  struct Raw { u32x2 q; u32x4 m; };
  __device__ static Raw get(const QRes &r, uint32_t row, uint32_t c, uint32_t h) {
    Raw w;
    w.q = ql8(r.q, row * r.q_stride + 16u * c + 8u * h);
    w.m = ql16(r.meta, (row * r.nb + (c >> 3)) * 16u);
    return w;
  }
  template <int N>
  __device__ static void wait(Raw &w) {
    __asm__ volatile("s_waitcnt vmcnt(%2)" : "+v"(w.q), "+v"(w.m) : "i"(N));
  }
  /* HI: the chunk lies in sub-blocks 4..7 of its super-block */
  template <bool BF, int HI>
  __device__ static void vals(const Raw &w, uint32_t c, uint32_t, bool ok, uint4 &o0, uint4 &o1) {
    const int i = (int)(c & 3u);
    const uint32_t b0 = byte_of(w.m[1], i), b1 = byte_of(w.m[2], i);
    uint32_t sc, mn;
    if constexpr (HI != 0) {
      const uint32_t b2 = byte_of(w.m[3], i);
      sc = (b2 & 0x0Fu) | ((b0 >> 6) << 4);
      mn = (b2 >> 4) | ((b1 >> 6) << 4);
    } else {
      sc = b0 & 63u;
      mn = b1 & 63u;
    }
    float d1 = h2f_lo(w.m[0]) * (float)sc, m1 = h2f_hi(w.m[0]) * (float)mn;
    if (!ok) d1 = m1 = 0.0f;
    const float b = -fmaf(1024.0f, d1, m1); /* d1 n - m1 */
    const uint32_t u0 = w.q[0] ^ 0x88888888u, u1 = w.q[1] ^ 0x88888888u;
    o0 = word_op<BF>(u0 & 0x0F0F0F0Fu, (u0 >> 4) & 0x0F0F0F0Fu, d1, b);
    o1 = word_op<BF>(u1 & 0x0F0F0F0Fu, (u1 >> 4) & 0x0F0F0F0Fu, d1, b);
  }
};
template <>
struct QQ<Q6_K> {
  static constexpr int kLoads = 4;
  struct Raw { u32x2 ql; uint32_t qh, sc, d; };
  __device__ static Raw get(const QRes &r, uint32_t row, uint32_t c, uint32_t h) {
    const uint32_t blk = row * r.nb + (c >> 3);
    Raw w;
    w.ql = ql8(r.q, row * r.q_stride + 16u * c + 8u * h);
    w.qh = ql4(r.aux, row * r.k4 + 8u * c + 4u * h);
    w.sc = ql2(r.meta, blk * 16u + 2u * (c & 7u)); /* both halves' scales */
    w.d = ql2(r.d, blk * 2u);
    return w;
  }
  template <int N>
  __device__ static void wait(Raw &w) {
    __asm__ volatile("s_waitcnt vmcnt(%4)"
                     : "+v"(w.ql), "+v"(w.qh), "+v"(w.sc), "+v"(w.d)
                     : "i"(N));
  }
  /* byte = l | h2 << 4 = q (0..63); value = d sc (q - 32) */
  template <bool BF, int HI>
  __device__ static void vals(const Raw &w, uint32_t, uint32_t h, bool ok, uint4 &o0, uint4 &o1) {
    const float d = ok ? h2f((uint16_t)w.d) : 0.0f;
    const float s = d * (float)(int32_t)(int8_t)(h ? (w.sc >> 8) : w.sc), b = -1056.0f * s;
    const uint32_t h0 = w.qh & 0x33333333u, h1 = (w.qh >> 2) & 0x33333333u;
    const uint32_t l0 = w.ql[0] ^ 0x88888888u, l1 = w.ql[1] ^ 0x88888888u;
    o0 = word_op<BF>(bfi(0xF0F0F0F0u, h0 << 4, l0), bfi(0xF0F0F0F0u, h0, l0 >> 4), s, b);
    o1 = word_op<BF>(bfi(0xF0F0F0F0u, h1 << 4, l1), bfi(0xF0F0F0F0u, h1, l1 >> 4), s, b);
  }
};

template <class F, bool BF>
__global__ void __launch_bounds__(lg::NT, 1) k_gemm_lds(GemmArgs a) {
  using namespace lg;
  __shared__ __attribute__((aligned(16))) uint8_t L[kLds];

  const uint32_t logical = (blockIdx.x % kXcds) * a.per_xcd + blockIdx.x / kXcds;
  const uint32_t ntile = a.tiles_n * a.tiles_m;
  if (logical >= ntile * a.splits) return;
  const uint32_t split = logical / ntile, tile = logical % ntile;
  const uint32_t tn = tile % a.tiles_n, tm = tile / a.tiles_n;
  paik_qview_t v = a.v;
  float *ybase = a.y;
  uint32_t tl = tn, rows_before = 0, cum = 0;
#pragma unroll
  for (int i = 1; i < kGemmMats; ++i) {
    cum += a.mv[i - 1].n;
    if ((uint32_t)i < a.count && tn >= a.tile_end[i - 1]) {
      v = a.mv[i];
      ybase = a.my[i];
      tl = tn - a.tile_end[i - 1];
      rows_before = cum;
    }
  }
  const uint32_t n0 = tl * (uint32_t)BM, m0 = tm * (uint32_t)BN;
  const uint32_t nchunks = v.k >> 5;
  const uint32_t s0 = split * a.steps_per_split; /* multiple of 4 */
  const uint32_t s1 = s0 + a.steps_per_split;

  const int tid = (int)threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t wr = (uint32_t)wave & 1u, wt = (uint32_t)wave >> 1;

  /* dequantization role: row drow of the tile, columns 16 dq .. 16 dq + 15
   * of each stage (nibble words 2 (dq % 2), +1 of chunk 2 s + dq / 2). A
   * quarter-wave writes one segment of 16 consecutive rows, which the tile
   * layout spreads over every LDS bank. */
  const uint32_t drow = 16u * (uint32_t)wave + ((uint32_t)lane & 15u);
  const uint32_t dq = (uint32_t)lane >> 4, dh = dq & 1u;
  const uint32_t grow = min(n0 + drow, v.n - 1u);
  const QRes res = make_qres(v);
  using Q = QQ<F>;
  typedef typename Q::Raw Raw;
  constexpr int kW = Q::kLoads;
  auto load_w = [&](uint32_t s, Raw &dst) {
    dst = Q::get(res, grow, min(2u * s + (dq >> 1), nchunks - 1u), dh);
  };
  const uint32_t woff0 = lg_off(drow, 2u * dq), woff1 = lg_off(drow, 2u * dq + 1u);
  auto deq = [&](auto uu, uint32_t s, Raw &w) {
    constexpr int U = decltype(uu)::value; /* s % 4 */
    const uint32_t c = 2u * s + (dq >> 1);
    uint4 o0, o1;
    Q::template vals<BF, (U >= 2)>(w, c, dh, c < nchunks, o0, o1);
    uint8_t *Wt = L + (U & 1) * kWTile;
    *reinterpret_cast<uint4 *>(Wt + woff0) = o0;
    *reinterpret_cast<uint4 *>(Wt + woff1) = o1;
  };

  /* DMA items: instruction u of this wave fills lines 4 (kXDma wave + u) ..
   * +3 of the activation tile; the lane writes slot lane % 16 of its line,
   * i.e. token row 2 line + slot % 2, segment (slot / 2) ^ line */
  const __amdgpu_buffer_rsrc_t xres = plane_rsrc(a.x16, a.x_bytes);
  uint32_t doff[kXDma], dcol[kXDma];
#pragma unroll
  for (int u = 0; u < kXDma; ++u) {
    const uint32_t line = 4u * (uint32_t)(kXDma * wave + u) + ((uint32_t)lane >> 4);
    const uint32_t slot = (uint32_t)lane & 15u;
    const uint32_t row = 2u * line + (slot & 1u), seg = ((slot >> 1) ^ line) & 7u;
    const uint32_t tok = m0 + row;
    dcol[u] = 8u * seg;
    doff[u] = tok < a.m ? (tok * v.k + 8u * seg) * 2u : 0x80000000u;
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)L;
  auto dma_one = [&](uint32_t s, uint32_t buf, int u, uint32_t off) {
    const uint32_t dst = (uint32_t)__builtin_amdgcn_readfirstlane((int)(
        lds0 + 2u * kWTile + buf * (uint32_t)kXTile + (uint32_t)(kXDma * wave + u) * 1024u));
    const uint32_t soff = (uint32_t)__builtin_amdgcn_readfirstlane((int)(2u * KS * s));
    uint32_t saved;
    __asm__ volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 4\n\t"
        "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(dst), "v"(off), "s"(xres), "s"(soff)
        : "memory");
  };
  auto dma_x = [&](uint32_t s, uint32_t buf) {
    /* a stage inside K needs no per-lane column check (uniform branch) */
    if ((uint32_t)KS * (s + 1u) <= v.k) {
#pragma unroll
      for (int u = 0; u < kXDma; ++u) dma_one(s, buf, u, doff[u]);
    } else {
#pragma unroll
      for (int u = 0; u < kXDma; ++u)
        dma_one(s, buf, u, (uint32_t)KS * s + dcol[u] < v.k ? doff[u] : 0x80000000u);
    }
  };

  /* operand offsets: fragment rows (A: tokens 64 wt + 32 i + lane % 32; B:
   * rows 64 wr + 32 j + lane % 32), segment 2 sub + lane / 32 */
  const uint32_t kset = (uint32_t)lane >> 5;
  uint32_t aoff[2][4], boff[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      aoff[i][u] = lg_off(64u * wt + 32u * (uint32_t)i + ((uint32_t)lane & 31u), 2u * (uint32_t)u + kset);
      boff[i][u] = lg_off(64u * wr + 32u * (uint32_t)i + ((uint32_t)lane & 31u), 2u * (uint32_t)u + kset);
    }
  f16x_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  /* Issue order per stage: DMA (kXDma), then weight loads (kW). Waits:
   * weights of stage s+1 before their dequantization (all but the last
   * 3 kW + 2 kXDma requests), activations of stage s+1 before the barrier
   * (all but the last 2 kW + kXDma). The prologue issues X(s0), W(s0..s0+2),
   * X(s0+1), W(s0+3), for which the same counts hold. */
  Raw ring[kRing];
  dma_x(s0, 0u);
  load_w(s0, ring[0]);
  load_w(s0 + 1u, ring[1]);
  load_w(s0 + 2u, ring[2]);
  dma_x(s0 + 1u, 1u);
  load_w(s0 + 3u, ring[3]);
  Q::template wait<3 * kW + kXDma>(ring[0]);
  deq(std::integral_constant<int, 0>(), s0, ring[0]);
  __syncthreads();

  auto body = [&](auto uu, uint32_t s) {
    constexpr int U = decltype(uu)::value; /* s % 4 (s0 % 4 == 0) */
    dma_x(s + 2u, (uint32_t)((U + 2) & 3));
    load_w(s + 4u, ring[U]);
    const uint8_t *Xt = L + 2 * kWTile + U * kXTile;
    const uint8_t *Wt = L + (U & 1) * kWTile;
    /* operands of sub-step u + 1 are read before the MFMAs of sub-step u */
    uint4 Ac[2], Bc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      Ac[i] = *reinterpret_cast<const uint4 *>(Xt + aoff[i][0]);
      Bc[i] = *reinterpret_cast<const uint4 *>(Wt + boff[i][0]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      uint4 An[2], Bn[2];
      if (u < 3) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          An[i] = *reinterpret_cast<const uint4 *>(Xt + aoff[i][u + 1]);
          Bn[i] = *reinterpret_cast<const uint4 *>(Wt + boff[i][u + 1]);
        }
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma<BF>(Ac[i], Bc[j], acc[i][j]);
      if (u == 1) {
        Q::template wait<3 * kW + 2 * kXDma>(ring[(U + 1) & 3]);
        deq(std::integral_constant<int, (U + 1) & 3>(), s + 1u, ring[(U + 1) & 3]);
      }
      if (u < 3) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          Ac[i] = An[i];
          Bc[i] = Bn[i];
        }
      }
    }
    wait_vmem<2 * kW + kXDma>();
    __syncthreads();
  };
  for (uint32_t s = s0; s < s1; s += 4u) {
    body(std::integral_constant<int, 0>(), s);
    body(std::integral_constant<int, 1>(), s + 1u);
    body(std::integral_constant<int, 2>(), s + 2u);
    body(std::integral_constant<int, 3>(), s + 3u);
  }
  /* The last iteration's ring loads are never used: wait for them with
   * their registers bound, so none is reused while a load may still write
   * it, and no DMA lands in LDS after the workgroup ends. */
#pragma unroll
  for (int i = 0; i < kRing; ++i) Q::template wait<0>(ring[i]);

  /* lane (r, g) holds row 64 wr + 32 j + r for tokens 8 (e / 4) + 4 g + e % 4
   * of fragment i */
  const bool split_k = a.splits > 1u;
  const bool gated = a.gate != nullptr && !split_k;
  float *const pbase = a.part != nullptr ? a.part + (size_t)a.splits * a.m * rows_before +
                                                (size_t)split * a.m * v.n
                                          : nullptr;
  const uint32_t r = (uint32_t)lane & 31u, g = (uint32_t)lane >> 5;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t row = n0 + 64u * wr + 32u * (uint32_t)j + r;
      const uint32_t t0 = m0 + 64u * wt + 32u * (uint32_t)i + 4u * g;
      float gv[16];
      if (gated) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const uint32_t tok = min(t0 + 8u * (uint32_t)(e >> 2) + (uint32_t)(e & 3), a.m - 1u);
          gv[e] = a.gate[(size_t)tok * v.n + min(row, v.n - 1u)];
        }
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t tok = t0 + 8u * (uint32_t)(e >> 2) + (uint32_t)(e & 3);
        if (tok < a.m && row < v.n) {
          const size_t at = (size_t)tok * v.n + row;
          const float val = acc[i][j][e];
          if (pbase != nullptr) pbase[at] = val;
          else if (split_k) unsafeAtomicAdd(ybase + at, val);
          else if (gated) ybase[at] = silu_mul(gv[e], val);
          else ybase[at] = val;
        }
      }
    }
}

/* Grid of a k_gemm_lds launch: 128-row x 256-token tiles; K split while
 * the tiles leave most CUs idle, each part at least 16 stages (1024
 * columns), the stage count per part a multiple of 4. */
static void plan_lds(GemmArgs &a) {
  if (a.count <= 1u) a.tiles_n = (a.v.n + lg::BM - 1u) / lg::BM;
  a.tiles_m = (a.m + lg::BN - 1u) / lg::BN;
  const uint32_t tiles = a.tiles_n * a.tiles_m;
  const uint32_t nst = ((a.v.k + lg::KS - 1u) / lg::KS + 3u) & ~3u;
  uint32_t splits = 1;
  while (tiles * splits * 2u <= 256u && nst / (splits * 2u) >= 16u) splits *= 2u;
  if (paik_tune.gemm_splits >= 1 && paik_tune.gemm_splits <= 64)
    splits = (uint32_t)paik_tune.gemm_splits;
  if (a.gate != nullptr) splits = 1u;
  a.steps_per_split = ((nst + splits - 1u) / splits + 3u) & ~3u;
  a.splits = (nst + a.steps_per_split - 1u) / a.steps_per_split;
  a.per_xcd = (tiles * a.splits + kXcds - 1u) / kXcds;
}

/* TT = 0: the LDS-shared prefill kernel (k_gemm_lds); otherwise k_gemm_x16
 * with that tile. */
template <class F, int TT, int NW, int RWG>
static hipError_t launch_x16(const paik_qview_t *const *vs, float *const *ys, uint32_t count,
                             uint32_t m, const float *x, uint16_t *x16, const float *gate,
                             bool bf16, float *part, size_t part_bytes, bool silu_pair,
                             hipStream_t s) {
  constexpr uint32_t kRows = TT == 0 ? (uint32_t)lg::BM : (uint32_t)RWG;
  const paik_qview_t &v = *vs[0];
  hipError_t e = hipSuccess;
  if (x != nullptr) { /* x == nullptr: x16 already holds these tokens */
    const size_t n4 = (size_t)m * v.k / 4u;
    const size_t blocks = (n4 + 255u) / 256u;
    k_cvt_x<><<<dim3((unsigned)(blocks < 2048u ? blocks : 2048u)), 256, 0, s>>>(
        reinterpret_cast<const float4 *>(x), reinterpret_cast<uint2 *>(x16), n4, bf16 ? 1 : 0);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  GemmArgs a;
  memset(&a, 0, sizeof a);
  a.v = v;
  a.x16 = x16;
  a.y = ys[0];
  a.gate = gate;
  a.m = m;
  a.count = count;
  uint32_t tiles = 0;
  for (uint32_t i = 0; i < count; ++i) {
    a.mv[i] = *vs[i];
    a.my[i] = ys[i];
    tiles += (vs[i]->n + kRows - 1u) / kRows;
    a.tile_end[i] = tiles;
  }
  a.tiles_n = tiles;
  if constexpr (TT == 0) plan_lds(a);
  else plan_grid(a, RWG, TT);
  a.x_bytes = (uint32_t)((size_t)m * v.k * 2u);
  size_t rows = 0;
  uint32_t ns[kGemmMats];
  for (uint32_t i = 0; i < count; ++i) {
    ns[i] = vs[i]->n;
    rows += vs[i]->n;
  }
  const bool parts = a.splits > 1u && part != nullptr &&
                     (size_t)a.splits * m * rows * 4u <= part_bytes;
  if (silu_pair && !parts) return hipErrorInvalidValue; /* the caller checks first */
  if (parts) {
    a.part = part;
  } else if (a.splits > 1u) {
    for (uint32_t i = 0; i < count; ++i) {
      e = zero_fill(ys[i], (size_t)m * vs[i]->n, s);
      if (e != hipSuccess) return e;
    }
  }
  const dim3 grid(a.per_xcd * kXcds);
  if constexpr (TT == 0) {
    if (bf16) k_gemm_lds<F, true><<<grid, dim3(lg::NT), 0, s>>>(a);
    else k_gemm_lds<F, false><<<grid, dim3(lg::NT), 0, s>>>(a);
  } else {
    if (bf16) k_gemm_x16<F, true, TT, NW, RWG><<<grid, dim3(64 * NW), 0, s>>>(a);
    else k_gemm_x16<F, false, TT, NW, RWG><<<grid, dim3(64 * NW), 0, s>>>(a);
  }
  e = hipGetLastError();
  if (e != hipSuccess || !parts) return e;
  return launch_reduce(part, ys, ns, count, m, a.splits, s, silu_pair);
}

/* The 16-bit kernel a block of mt tokens of format `type` runs on:
 *   1  k_gemm_x16, 32-token x 256-row tiles (up to 32 tokens)
 *   2  k_gemm_x16, 128-token x 256-row tiles on 8 waves
 *   3  k_gemm_x16, 256-token x 128-row tiles on 4 waves (measurement only)
 *   4  k_gemm_lds (Q6_K from 256 tokens)
 * Measured at 512 tokens (gate 14336 x 4096 / down 4096 x 14336): Q4_K
 * 81 / -, Q4_0 82, Q8_0 96 us on tiles 2; Q6_K down 118.9 us on 4 against
 * 126.6 on 2 and 121.1 on 3; from 1024 tokens the order holds. The
 * gemm_tile tuning field overrides the choice. */
static int pick_kind(uint32_t type, uint32_t mt) {
  const int t = paik_tune.gemm_tile;
  if (t >= 1 && t <= 4) return t;
  if (mt <= 32u) return 1;
  if (mt < 256u || type != 14u) return 2;
  return 4;
}

template <class F>
static hipError_t launch_gemm(const paik_qview_t *const *vs, float *const *ys, uint32_t count,
                              uint32_t m, const float *x, const float *gate, bool bf16,
                              uint16_t *x16, size_t x16_bytes, float *part, size_t part_bytes,
                              bool silu_pair, hipStream_t s) {
  const paik_qview_t &v = *vs[0];
  /* token blocks whose activations span less than 2^31 bytes (32-bit
   * buffer offsets) and, on the 16-bit path, fit the workspace */
  const size_t row_bytes = (size_t)v.k * 4u;
  uint32_t blk = (uint32_t)((0x7FFFFFFFu / row_bytes) & ~255u);
  if (blk == 0u) return hipErrorInvalidValue; /* k > 2M columns */
  const bool use16 = x16 != nullptr && x16_bytes >= (size_t)v.k * 2u * 256u;
  if (use16) {
    const uint32_t fit = (uint32_t)((x16_bytes / ((size_t)v.k * 2u)) & ~(size_t)255u);
    if (fit < blk) blk = fit;
  }
  /* x == nullptr: the 16-bit workspace already holds all m tokens */
  if (x == nullptr && (!use16 || m > blk)) return hipErrorInvalidValue;
  for (uint32_t t0 = 0; t0 < m; t0 += blk) {
    const uint32_t mt = m - t0 < blk ? m - t0 : blk;
    const float *xt = x != nullptr ? x + (size_t)t0 * v.k : nullptr;
    float *yt[kGemmMats];
    for (uint32_t i = 0; i < count; ++i) yt[i] = ys[i] + (size_t)t0 * vs[i]->n;
    const float *gt = gate != nullptr ? gate + (size_t)t0 * v.n : nullptr;
    /* The 16-bit path takes all matrices in one launch (kernel by
     * pick_kind); the register-staged path one per matrix. */
    hipError_t e = hipSuccess;
    if (use16) {
      const int kind = pick_kind(F::kType, mt);
      e = kind == 1   ? launch_x16<F, 32, 8, 256>(vs, yt, count, mt, xt, x16, gt, bf16, part,
                                                  part_bytes, silu_pair, s)
          : kind == 2 ? launch_x16<F, 128, 8, 256>(vs, yt, count, mt, xt, x16, gt, bf16, part,
                                                   part_bytes, silu_pair, s)
          : kind == 3 ? launch_x16<F, 256, 4, 128>(vs, yt, count, mt, xt, x16, gt, bf16, part,
                                                   part_bytes, silu_pair, s)
                      : launch_x16<F, 0, 8, 0>(vs, yt, count, mt, xt, x16, gt, bf16, part,
                                               part_bytes, silu_pair, s);
    } else if ((count > 1u || silu_pair) && mt <= 32u && gt == nullptr) {
      /* up to 32 tokens: the matrices share one register-staged launch */
      e = launch_tt_multi<F, 32, 8, 256, 4>(vs, yt, count, mt, xt, bf16, part, part_bytes,
                                            silu_pair, s);
    } else {
      if (silu_pair) return hipErrorInvalidValue; /* the pair form needs the 16-bit path */
      for (uint32_t i = 0; i < count && e == hipSuccess; ++i)
        e = mt <= 32u    ? launch_tt<F, 32, 8, 256, 4>(*vs[i], mt, xt, yt[i], gt, bf16, part,
                                                       part_bytes, s)
            : mt < 256u ? launch_tt<F, 128, 8, 256, 2>(*vs[i], mt, xt, yt[i], gt, bf16, part,
                                                       part_bytes, s)
                        : launch_tt<F, 256, 4, 128, 1>(*vs[i], mt, xt, yt[i], gt, bf16, part,
                                                       part_bytes, s);
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

} // namespace paik

using namespace paik;

/* One translation unit per block format (PAI_GEMM_FMT = Q4_0, Q8_0, Q4_K or
 * Q6_K, entry point PAI_GEMM_ENTRY), so the four formats' GEMM kernels
 * compile in parallel; the unit without PAI_GEMM_FMT holds the dispatcher. */
#define PAI_GEMM_ARGS                                                                         \
  const paik_qview_t *const *vs, float *const *ys, uint32_t count, uint32_t m, const float *x, \
      const float *gate, int bf16, void *x16, uint64_t x16_bytes, void *part,                  \
      uint64_t part_bytes, int silu_pair, void *stream
#ifdef PAI_GEMM_FMT
extern "C" int PAI_GEMM_ENTRY(PAI_GEMM_ARGS) {
  return (int)launch_gemm<PAI_GEMM_FMT>(vs, ys, count, m, x, gate, bf16 != 0,
                                        static_cast<uint16_t *>(x16), (size_t)x16_bytes,
                                        static_cast<float *>(part), (size_t)part_bytes,
                                        silu_pair != 0, (hipStream_t)stream);
}
#else
extern "C" int paik_gemm_mfma_q4_0(PAI_GEMM_ARGS);
extern "C" int paik_gemm_mfma_q8_0(PAI_GEMM_ARGS);
extern "C" int paik_gemm_mfma_q4_k(PAI_GEMM_ARGS);
extern "C" int paik_gemm_mfma_q6_k(PAI_GEMM_ARGS);
extern "C" int paik_gemm_mfma_multi(PAI_GEMM_ARGS) {
  if (count == 0u || count > (uint32_t)kGemmMats || (gate != nullptr && count != 1u))
    return (int)hipErrorInvalidValue;
  if (silu_pair && (count != 2u || vs[0]->n != vs[1]->n || gate != nullptr))
    return (int)hipErrorInvalidValue;
  for (uint32_t i = 1; i < count; ++i)
    if (vs[i]->type != vs[0]->type || vs[i]->k != vs[0]->k) return (int)hipErrorInvalidValue;
  switch (vs[0]->type) {
  case 8u: return paik_gemm_mfma_q8_0(vs, ys, count, m, x, gate, bf16, x16, x16_bytes, part,
                                   part_bytes, silu_pair, stream);
  case 2u: return paik_gemm_mfma_q4_0(vs, ys, count, m, x, gate, bf16, x16, x16_bytes, part,
                                   part_bytes, silu_pair, stream);
  case 12u: return paik_gemm_mfma_q4_k(vs, ys, count, m, x, gate, bf16, x16, x16_bytes, part,
                                   part_bytes, silu_pair, stream);
  case 14u: return paik_gemm_mfma_q6_k(vs, ys, count, m, x, gate, bf16, x16, x16_bytes, part,
                                   part_bytes, silu_pair, stream);
  default: return (int)hipErrorInvalidValue;
  }
}
extern "C" int paik_gemm_mfma(const paik_qview_t *v, uint32_t m, const float *x, float *y,
                              const float *gate, int bf16, void *x16, uint64_t x16_bytes,
                              void *stream) {
  return paik_gemm_mfma_multi(&v, &y, 1u, m, x, gate, bf16, x16, x16_bytes, nullptr, 0u, 0,
                              stream);
}
extern "C" uint32_t paik_gemm_x16_splits(const paik_qview_t *v, uint32_t m) {
  GemmArgs a;
  memset(&a, 0, sizeof a);
  a.v = *v;
  a.m = m;
  switch (pick_kind(v->type, m)) {
  case 1: plan_grid(a, 256u, 32u); break;
  case 2: plan_grid(a, 256u, 128u); break;
  case 3: plan_grid(a, 128u, 256u); break;
  default: plan_lds(a); break;
  }
  return a.splits;
}
extern "C" uint64_t paik_gemm_part_bytes(const paik_qview_t *const *vs, uint32_t count,
                                         uint32_t m) {
  if (m > 1024u) m = 1024u; /* the largest token block of the 16-bit path */
  GemmArgs a;
  memset(&a, 0, sizeof a);
  a.v = *vs[0];
  a.m = m;
  a.count = count;
  const int kind = pick_kind(vs[0]->type, m);
  const uint32_t tt = kind == 1 ? 32u : kind == 2 ? 128u : 256u;
  const uint32_t rwg = kind == 3 ? 128u : kind == 4 ? (uint32_t)lg::BM : 256u;
  uint64_t rows = 0;
  for (uint32_t i = 0; i < count; ++i) {
    a.tiles_n += (vs[i]->n + rwg - 1u) / rwg;
    rows += vs[i]->n;
  }
  if (kind == 4) plan_lds(a);
  else plan_grid(a, rwg, tt);
  return a.splits > 1u ? (uint64_t)a.splits * m * rows * 4u : 0u;
}
#endif
