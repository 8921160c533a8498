/*
 * Decode GEMV / small-batch GEMM over packed blocks with integer dot
 * products (v_dot8_i32_i4).
 *
 * y[t][r] = sum_k x[t][k] * W[r][k] for up to MT tokens per launch.
 *
 * Streaming design. The grid is about one 16-wave workgroup per CU; each
 * wave owns a contiguous range of rows and walks it block by block, where
 * a block is U rows x one 64-chunk step (lane l takes chunk 64s + l, so
 * one row's loads of a block are one contiguous 1 KiB read). Each lane
 * keeps 4 row-chunk loads in flight (a ring of 4/U blocks, refilled as
 * each block is multiplied): about 8-16 MB requested across the chip at
 * any time, enough to keep HBM busy while the dot products overlap the
 * stream (see kInFlight).
 *
 * Per workgroup:
 *   1. each wave issues the loads of its first 4/U blocks, then all threads
 *      turn the activations of the launch's column slice into digit planes
 *      in LDS (XChunk in qdev.h: six signed 4-bit digit planes of a 24-bit
 *      fixed-point image of x with a per-chunk scale 2^(E-22)). Four
 *      threads build one chunk, one nibble word of every plane each;
 *   2. per block, a lane reads its chunk's planes from LDS once for the U
 *      rows; a row-chunk costs 24 v_dot8 (48 for Q8_0 and Q6_K) and one
 *      scale step;
 *   3. after a row group's last step the wave sums each of its U*MT
 *      per-lane partials across the 64 lanes in registers (DPP row steps,
 *      then two cross-row steps). The summation order is fixed by the
 *      launch shape, so results do not depend on scheduling.
 *
 * Rows longer than one slice (the chunk-tokens whose planes fit the 64 KiB
 * LDS budget: 585, i.e. rows up to 18720 columns at MT = 1, 9344 at MT = 2
 * and 4672 at MT = 4) are covered by successive launches over column
 * slices of a multiple of 64 chunks; all but the first add into y (each
 * output is read and written by one lane, in launch order).
 *
 * The integer sums are exact; the roundings are the 24-bit image of x
 * (<= 2^-23 of the chunk's largest |x|), the per-chunk scale steps and the
 * f32 additions across chunks and lanes.
 */
#include <string.h>

#include "qdev.h"

namespace paik {

constexpr int kWaves = 16;   /* waves per workgroup (one workgroup per CU) */
constexpr int kWavesSmall = 8; /* for one-token launches with under 2 rows per wave at kWaves */
/* Row-chunk loads per lane kept in flight. Deeper rings request more of
 * the matrix at once than HBM can return in a round trip; the queue that
 * builds up delays every request behind it, the activation loads that the
 * dot products wait for included. Measured on the Q4_K decode step
 * (q/k/v, o, gate/up, down): 8 loads (2 blocks at U = 4, 4 at U = 2)
 * 7.5 / 5.8 / 15.8 / 10.2 us, 3050 GB/s; 4 loads 6.3 / 5.0 / 14.3 / 9.7 us,
 * 3340 GB/s; the 8B decode step 1.965 -> 1.836 ms per token. A ring
 * longer than a wave's blocks also re-reads its last block: q/k/v at 2
 * blocks per wave took 7.5 us with 4 ring slots against 6.3 with 2. One
 * slot at U = 2 starves the longer rows (down: 11.9 us). 16-wave
 * workgroups take half of this (see PD). */
constexpr int kInFlight = 4;
constexpr size_t kLdsBudget = 65536; /* bytes of LDS per workgroup */

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dppi(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kQuadXor1 = 0xB1, kQuadXor2 = 0x4E;

/* Sum of v over aligned groups of L lanes (L a power of two <= 64); every
 * lane of a group receives the group's sum. */
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (L >= 2) v += dpp<kQuadXor1>(v);
  if constexpr (L >= 4) v += dpp<kQuadXor2>(v);
  if constexpr (L >= 8) v += dpp<0x141>(v);  /* row_half_mirror: 8-lane halves */
  if constexpr (L >= 16) v += dpp<0x140>(v); /* row_mirror: 16-lane rows */
  if constexpr (L >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (L >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

/* LDS image of one activation chunk. */
struct XSlot {
  uint4 X[6];
};
struct XScale {
  float xs, sx0, sx1, pad;
};

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

/* One quad-thread's share of a chunk: columns 8j..8j+7 (v[0..7]) of one
 * token; writes word j of the six planes and, from threads 0 and 2 of the
 * quad, the chunk's scale and half sums. */
__device__ __forceinline__ void plane_words(const float v[8], uint32_t jw, XSlot *slot,
                                            XScale *f) {
  float m = 0.0f, sa = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    m = fmaxf(m, fabsf(v[i])); /* fmaxf drops NaNs ... */
    sa += fabsf(v[i]);         /* ... which this sum keeps */
  }
  m = fmaxf(m, dpp<kQuadXor1>(m));
  m = fmaxf(m, dpp<kQuadXor2>(m));
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
    u[i] = ((uint32_t)q + 0x888888u) ^ 0x888888u; /* bytes 0..2: digit pairs */
  }
  /* gather byte b of u0..u3 (lo) and u4..u7 (hi) */
  const uint32_t a01 = perm(u[1], u[0], 0x05010400u), b01 = perm(u[1], u[0], 0x0C0C0602u);
  const uint32_t a23 = perm(u[3], u[2], 0x05010400u), b23 = perm(u[3], u[2], 0x0C0C0602u);
  const uint32_t a45 = perm(u[5], u[4], 0x05010400u), b45 = perm(u[5], u[4], 0x0C0C0602u);
  const uint32_t a67 = perm(u[7], u[6], 0x05010400u), b67 = perm(u[7], u[6], 0x0C0C0602u);
  const uint32_t g[3][2] = {{perm(a23, a01, 0x05040100u), perm(a67, a45, 0x05040100u)},
                            {perm(a23, a01, 0x07060302u), perm(a67, a45, 0x07060302u)},
                            {perm(b23, b01, 0x05040100u), perm(b67, b45, 0x05040100u)}};
  uint32_t *dst = reinterpret_cast<uint32_t *>(slot) + jw;
#pragma unroll
  for (int b = 0; b < 3; ++b) {
    /* byte m of a plane word = column m (low nibble) | column m+4 (high) */
    dst[4 * (2 * b)] = (g[b][0] & 0x0F0F0F0Fu) | ((g[b][1] & 0x0F0F0F0Fu) << 4);
    dst[4 * (2 * b + 1)] = ((g[b][0] >> 4) & 0x0F0F0F0Fu) | (g[b][1] & 0xF0F0F0F0u);
  }
  sq += dppi<kQuadXor1>(sq); /* words 0+1: columns 0..15; 2+3: 16..31 */
  const float xs = bad ? __builtin_nanf("") : __builtin_amdgcn_ldexpf(1.0f, e - 22);
  if (jw == 0u) {
    f->xs = xs;
    f->sx0 = (float)sq * xs;
  } else if (jw == 2u) {
    f->sx1 = (float)sq * xs;
  }
}

/* Planes of chunks [cs, cs + nsc) for MT tokens, in two phases so that
 * the activation loads can be issued ahead of the weight loads (vector
 * memory results are consumed in issue order: an activation load issued
 * after the weight ring would wait for all of it). Four consecutive
 * threads share a chunk; a thread takes up to kXIt chunk quarters, which
 * covers up to kXIt * 1024 / 4 = 1024 chunk-tokens (more than the LDS
 * budget holds). */
constexpr int kXIt = 4;
/* The fused-RMSNorm kernels also hold gamma in registers; with 2 passes
 * (1 for Q8_0, whose codes take twice the registers) they fit the plain
 * kernels' register budget without spills. */
template <class F> constexpr int kXItNorm = 2;
template <> constexpr int kXItNorm<Q8_0> = 1;
/* chunk-tokens one pass of the plane builder covers, per workgroup size
 * and passes per thread */
__host__ __device__ constexpr uint32_t max_slice_tok(int nw, int xi = kXIt) {
  return (uint32_t)xi * 64u * (uint32_t)nw / 4u;
}

template <int MT, int XI>
__device__ __forceinline__ void x_load(const float *__restrict__ x, uint32_t k, uint32_t ntok,
                                       uint32_t cs, uint32_t nsc, float4 (&va)[XI],
                                       float4 (&vb)[XI]) {
  const uint32_t total = (uint32_t)MT * nsc * 4u;
#pragma unroll
  for (int it = 0; it < XI; ++it) {
    const uint32_t idx = threadIdx.x + (uint32_t)it * blockDim.x;
    const uint32_t t = idx / (nsc * 4u), r = idx % (nsc * 4u);
    /* Idle threads and tokens >= ntok load nothing (zeros). Given a
     * clamped address instead, every idle thread of every workgroup would
     * request the same line, which the L2 serves one request at a time:
     * that held the activations of a 256-workgroup launch for microseconds. */
    const bool ok = idx < total && t < ntok;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
    if (ok) {
      const float4 *src = reinterpret_cast<const float4 *>(
          x + (size_t)t * k + 32u * (cs + (r >> 2)) + 8u * (r & 3u));
      a = src[0];
      b = src[1];
    }
    va[it] = a;
    vb[it] = b;
  }
}

template <int MT, int XI>
__device__ __forceinline__ void x_planes(uint32_t nsc, const float4 (&va)[XI],
                                         const float4 (&vb)[XI], XSlot *xp, XScale *xf) {
  const uint32_t total = (uint32_t)MT * nsc * 4u;
#pragma unroll
  for (int it = 0; it < XI; ++it) {
    const uint32_t idx = threadIdx.x + (uint32_t)it * blockDim.x;
    if (idx < total) { /* whole quads are in or out together */
      const uint32_t t = idx / (nsc * 4u), r = idx % (nsc * 4u);
      const float v[8] = {va[it].x, va[it].y, va[it].z, va[it].w,
                          vb[it].x, vb[it].y, vb[it].z, vb[it].w};
      plane_words(v, r & 3u, &xp[t * nsc + (r >> 2)], &xf[t * nsc + (r >> 2)]);
    }
  }
}

/* A format's dot product for a lane whose chunk's position in its
 * super-block is fixed for the whole launch (chunk cb + lane, cb a
 * multiple of 8): Q4_K precomputes its scale/min unpack selectors from the
 * lane once; the other formats take the plain dot. */
template <class F>
struct LaneDot {
  struct Ctx {};
  __device__ static Ctx make(uint32_t) { return {}; }
  __device__ static float dot(const typename F::Raw &w, uint32_t c, const Ctx &, const XChunk &x) {
    return F::dot(w, c, x);
  }
};
template <>
struct LaneDot<Q4_K> {
  typedef Q4_K::Lane Ctx;
  __device__ static Ctx make(uint32_t lane) { return Q4_K::lane_ctx(lane & 7u); }
  __device__ static float dot(const Q4_K::Raw &w, uint32_t, const Ctx &l, const XChunk &x) {
    return Q4_K::dot_lane(w, l, x);
  }
};

/* Matrices of one launch: up to kMaxMats weights with the same format and
 * column count, multiplied by the same activations (the q/k/v or gate/up
 * projections of a layer). Waves [wave_end[i-1], wave_end[i]) work on
 * matrix i, so no wave's rows cross a matrix boundary.
 * Paired launches (the PAIR kernels) instead take v[0] = gate and v[1] = up
 * of one row count and write y[0] = silu(x W_gate^T) * (x W_up^T): every
 * wave works on both matrices over the same rows. */
constexpr int kMaxMats = 4;
struct GemvArgs {
  paik_qview_t v[kMaxMats];
  float *y[kMaxMats];
  uint32_t wave_end[kMaxMats];
  uint32_t count;
  float eps; /* NORM kernels: RMSNorm epsilon (in the struct's tail padding) */
};
/* NORM launches take at most kMaxMats - 1 matrices and carry the RMSNorm
 * weights (K floats) in the last output slot, so the argument block keeps
 * its layout (560 bytes with the launch's hidden arguments). Measured on
 * the Q4_0 decode step against this layout (3160 GB/s): 16 bytes more,
 * same instructions otherwise, 3055; a compact 512-byte block (per-matrix
 * planes and row count, shared K), 3070. */
constexpr int kNormGammaSlot = kMaxMats - 1;

/* RMSNorm of a one-token activation row held in registers (the x_load
 * layout, every element of the row loaded once across the workgroup),
 * rms = 1 / sqrtf((float)(sum x^2 / n) + eps) with the sum of squares in
 * double (pai_ref_rmsnorm_gamma_f32, cpu/reference/ref_ops.c:195-216), in
 * two parts so that nothing waits for the reduction before the planes are
 * built: rms_begin turns x into x * gamma and leaves each wave's partial
 * sum of squares (lanes in a fixed order) in red[]; after the barrier that
 * publishes the planes, rms_end adds the waves in a fixed tree and forms
 * rms, which scales every finished dot product. Against the reference's
 * per-element (x * gamma) * rms this moves one rounding, O(2^-24)
 * relative. The double arithmetic sits on every wave's path to its first
 * dot product (q/k/v with the norm: 7.0-7.1 us, 6.0-6.3 in a timing build
 * with rms taken as 1), so it is kept short: a wave adds its lanes within
 * 16-lane rows by DPP and reads the four row sums with readlane (in place
 * of six LDS shuffles), rms_end adds the waves as a tree, and 1/K is formed
 * before the barrier (gate/up with the norm 15.5 -> 15.0 us; the 8B decode
 * step 1.827 -> 1.816 ms per token). Formed after the first row group
 * instead, rms only moved the same chain to the end (q/k/v 7.1 -> 7.5 us). */
template <int CTRL>
__device__ __forceinline__ double dppd(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
  const uint32_t hi =
      (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ double readlane_d(double v, int l) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
template <int XI>
__device__ __forceinline__ void rms_begin(float4 (&va)[XI], float4 (&vb)[XI],
                                          const float4 (&ga)[XI], const float4 (&gb)[XI],
                                          double *red) {
  double acc = 0.0;
#pragma unroll
  for (int it = 0; it < XI; ++it) {
    acc += (double)va[it].x * (double)va[it].x;
    acc += (double)va[it].y * (double)va[it].y;
    acc += (double)va[it].z * (double)va[it].z;
    acc += (double)va[it].w * (double)va[it].w;
    acc += (double)vb[it].x * (double)vb[it].x;
    acc += (double)vb[it].y * (double)vb[it].y;
    acc += (double)vb[it].z * (double)vb[it].z;
    acc += (double)vb[it].w * (double)vb[it].w;
  }
  /* every lane of a 16-lane row ends with the row's sum (each step adds
   * the same two partial sums in every lane) */
  acc += dppd<kQuadXor1>(acc);
  acc += dppd<kQuadXor2>(acc);
  acc += dppd<0x141>(acc); /* row_half_mirror */
  acc += dppd<0x140>(acc); /* row_mirror */
  const double wsum = (readlane_d(acc, 0) + readlane_d(acc, 16)) +
                      (readlane_d(acc, 32) + readlane_d(acc, 48));
  if ((threadIdx.x & 63u) == 0u) red[threadIdx.x >> 6] = wsum;
  auto mul = [](float4 x, float4 g) {
    return make_float4(x.x * g.x, x.y * g.y, x.z * g.z, x.w * g.w);
  };
#pragma unroll
  for (int it = 0; it < XI; ++it) {
    va[it] = mul(va[it], ga[it]);
    vb[it] = mul(vb[it], gb[it]);
  }
}
template <int NW>
__device__ __forceinline__ float rms_end(const double *red, double inv_n, float eps) {
  static_assert((NW & (NW - 1)) == 0, "waves: a power of two");
  double p[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) p[w] = red[w];
#pragma unroll
  for (int h = NW / 2; h >= 1; h /= 2)
#pragma unroll
    for (int w = 0; w < h; ++w) p[w] += p[w + h];
  return 1.0f / sqrtf((float)(p[0] * inv_n) + eps);
}

/* Weight loads of a block are issued for all its lanes and rows with
 * addresses clamped into the matrix (lanes or rows past the end re-read
 * valid data whose contribution is masked with a select), so a block is
 * one straight run of loads; whole blocks past the wave's last one are
 * not issued. Outputs are written without reading y (a load inside the
 * loop would wait for every weight load in flight): accumulating launches
 * add with a non-returning atomic (each output has one writer per launch,
 * and launches on a stream run in order, so the result is the same as a
 * read-add-write). */
template <class F, int U, int MT, bool PAIR, int NW, bool NORM>
__global__ void __launch_bounds__(64 * NW) k_gemv(GemvArgs a, const float *__restrict__ x,
                                                      uint32_t ntok, uint32_t cs, uint32_t nsc,
                                                      int accumulate) {
  static_assert(U * MT <= 16, "at most 16 outputs per row group");
  static_assert(!NORM || MT == 1, "the fused RMSNorm takes one token");
  static_assert(!PAIR || U % 2 == 0, "a paired row group holds gate and up rows");
  /* output rows per row group; in a paired launch slot u of a group holds
   * row u/2 of matrix u%2 */
  constexpr int UR = PAIR ? U / 2 : U;
  extern __shared__ uint4 smem[];
  XSlot *xp = reinterpret_cast<XSlot *>(smem);
  XScale *xf = reinterpret_cast<XScale *>(xp + (size_t)MT * nsc);

  const uint32_t lane = threadIdx.x & 63u;
  /* the wave index is uniform; reading it from lane 0 lets every row and
   * block quantity below live in scalar registers */
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const uint32_t gw = blockIdx.x * (uint32_t)NW + wave;
  /* the matrix this wave works on, and its share of that matrix's rows */
  uint32_t mi = 0, w0 = 0;
  if constexpr (!PAIR) {
#pragma unroll
    for (int i = 1; i < kMaxMats; ++i)
      if ((uint32_t)i < a.count && gw >= a.wave_end[i - 1]) {
        mi = (uint32_t)i;
        w0 = a.wave_end[i - 1];
      }
  }
  paik_qview_t v = a.v[0];
  float *y = a.y[0];
  if constexpr (!PAIR) {
#pragma unroll
    for (int i = 1; i < kMaxMats; ++i)
      if (mi == (uint32_t)i) {
        v = a.v[i];
        y = a.y[i];
      }
  }
  const uint64_t lw = gw - w0, tw = a.wave_end[mi] - w0;
  const uint32_t r_beg = (uint32_t)(lw * v.n / tw), r_end = (uint32_t)((lw + 1u) * v.n / tw);
  const uint32_t steps = (nsc + 63u) >> 6;
  const uint32_t groups = (r_end - r_beg + (uint32_t)UR - 1u) / (uint32_t)UR;
  const uint32_t nblk = groups * steps; /* wave-uniform; 0 for a wave without rows */
  const uint32_t blk_last = nblk > 0u ? nblk - 1u : 0u;
  const uint32_t row_last = r_end > r_beg ? r_end - 1u : min(r_beg, v.n - 1u);

  const QRes res = make_qres(v);
  const QRes res_up = make_qres(a.v[PAIR ? 1 : 0]);
  /* block, row and chunk base are wave-uniform; readfirstlane keeps them
   * in SGPRs (the buffer offset operand) when the compiler would compute
   * them on the vector unit */
  auto rfl = [](uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); };
  auto load_block = [&](uint32_t b, typename F::Raw (&buf)[U]) {
    const uint32_t bb = rfl(min(b, blk_last));
    const uint32_t g = rfl(bb / steps), s = rfl(bb % steps);
    const uint32_t cb = rfl(cs + 64u * s);             /* wave-uniform chunk base */
    const uint32_t ln = min(lane, nsc - 1u - 64u * s); /* cb + ln stays in the slice */
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t row =
          rfl(min(r_beg + g * (uint32_t)UR + (uint32_t)(PAIR ? u / 2 : u), row_last));
      buf[u] = F::bload((PAIR && (u & 1)) ? res_up : res, row, cb, ln);
    }
  };

  /* Activation loads first, then the ring of PD blocks (kInFlight
   * row-chunks per lane); the planes are built while the ring is in
   * flight. */
  constexpr int XI = NORM ? kXItNorm<F> : kXIt;
  float4 xa[XI], xb[XI];
  x_load<MT, XI>(x, v.k, ntok, cs, nsc, xa, xb);
  float4 ga[XI], gb[XI]; /* NORM: gamma in the same layout (one slice covers the row) */
  if constexpr (NORM) x_load<1, XI>(a.y[kNormGammaSlot], v.k, 1u, cs, nsc, ga, gb);
  /* 16-wave workgroups run twice the waves of the 8-wave ones, so each of
   * their lanes keeps half the loads in flight (q/k/v: 6.2 -> 5.9 us) */
  constexpr int kIF = NW == 16 ? kInFlight / 2 : kInFlight;
  constexpr int PD = kIF / U > 0 ? kIF / U : 1;
  typename F::Raw buf[PD][U];
  /* Every load below is unconditional (blocks past the wave's last one
   * re-read that block, an L2 hit), so each wave issues the same sequence
   * and the compiler's wait before block b's dot products counts exactly
   * the PD - 1 blocks requested after it. With loads under conditions it
   * has to assume fewer and waited for nearly the whole ring. */
#pragma unroll
  for (int p = 0; p < PD; ++p) load_block((uint32_t)p, buf[p]);

  __shared__ __attribute__((aligned(16))) double red[NORM ? NW : 1];
  /* 1/K in double, formed while the activations are in flight */
  const double inv_k = NORM ? 1.0 / (double)v.k : 1.0;
  if constexpr (NORM) rms_begin<XI>(xa, xb, ga, gb, red);
  x_planes<MT, XI>(nsc, xa, xb, xp, xf);
  __syncthreads();
  const float rms = NORM ? rms_end<NW>(red, inv_k, a.eps) : 1.0f;

  float acc[U][MT];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[u][t] = 0.0f;
  /* lanes past the slice end (clamped chunks) are masked below */
  const typename LaneDot<F>::Ctx lctx = LaneDot<F>::make(lane);

  auto compute_block = [&](uint32_t b, const typename F::Raw (&buf)[U]) {
    const uint32_t g = b / steps, s = b % steps;
    const uint32_t cl = 64u * s + lane;
    const bool live = cl < nsc;
    const uint32_t clc = min(cl, nsc - 1u);
    const uint32_t row0 = r_beg + g * (uint32_t)UR;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      XChunk xc;
      const XSlot &sl = xp[(uint32_t)t * nsc + clc];
#pragma unroll
      for (int p = 0; p < 6; ++p) {
        const uint4 q = sl.X[p];
        xc.X[p][0] = q.x;
        xc.X[p][1] = q.y;
        xc.X[p][2] = q.z;
        xc.X[p][3] = q.w;
      }
      const XScale f = xf[(uint32_t)t * nsc + clc];
      xc.xs = f.xs;
      xc.sx0 = f.sx0;
      xc.sx1 = f.sx1;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float d = LaneDot<F>::dot(buf[u], cs + clc, lctx, xc);
        /* a bitwise select, not a branch around the dot product */
        const uint32_t keep = (live && row0 + (uint32_t)(PAIR ? u / 2 : u) < r_end) ? ~0u : 0u;
        acc[u][t] += __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, d) & keep);
      }
    }
    if (PAIR && s + 1u == steps) {
      /* paired row group done: lane j = p*MT + t combines row p's gate and
       * up sums for token t (a paired launch covers the whole row) */
#pragma unroll
      for (int p = 0; p < UR; ++p)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          float sg = group_sum<64>(acc[2 * p][t]);
          float su = group_sum<64>(acc[2 * p + 1][t]);
          if constexpr (NORM) {
            sg *= rms;
            su *= rms;
          }
          acc[2 * p][t] = 0.0f;
          acc[2 * p + 1][t] = 0.0f;
          const uint32_t row = row0 + (uint32_t)p;
          if (lane == (uint32_t)(p * MT + t) && row < r_end && (uint32_t)t < ntok)
            y[(size_t)t * v.n + row] = silu_mul(sg, su);
        }
    } else if (s + 1u == steps) {
      /* Row group done: every output's 64 lane partials are summed in
       * registers (DPP within 16-lane rows, then two cross-row steps); lane
       * j then writes output j = u*MT + t. */
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          float sum = group_sum<64>(acc[u][t]);
          if constexpr (NORM) sum *= rms;
          acc[u][t] = 0.0f;
          const uint32_t row = row0 + (uint32_t)u;
          if (lane == (uint32_t)(u * MT + t) && row < r_end && (uint32_t)t < ntok) {
            float *dst = y + (size_t)t * v.n + row;
            if (accumulate) unsafeAtomicAdd(dst, sum);
            else *dst = sum;
          }
        }
    }
  };

  /* Rounds of PD blocks: every round but the last refills each buffer
   * right after its block (the refills of the round before the last may
   * re-read the last block); the last round only computes, so no load is
   * left to return before the wave retires. */
  const uint32_t rounds = (nblk + (uint32_t)PD - 1u) / (uint32_t)PD;
  uint32_t b0 = 0;
  for (uint32_t rd = 1; rd < rounds; ++rd, b0 += (uint32_t)PD) {
#pragma unroll
    for (int p = 0; p < PD; ++p) {
      compute_block(b0 + (uint32_t)p, buf[p]);
      load_block(b0 + (uint32_t)p + (uint32_t)PD, buf[p]);
    }
  }
  if (rounds > 0u) {
#pragma unroll
    for (int p = 0; p < PD; ++p)
      if (b0 + (uint32_t)p < nblk) compute_block(b0 + (uint32_t)p, buf[p]);
  }
}

/* Workgroups: one per CU (256), fewer when that would leave waves with
 * under two rows (a one-row group re-reads the activation planes for a
 * single row). Rows per group U: 4 when waves get four or more rows, else
 * 2 (U*MT <= 8). The gemv_wgs / gemv_rows tuning fields override both. */
static uint32_t pick_grid(uint32_t n, uint32_t count) {
  uint32_t g = (n + 2u * kWaves - 1u) / (2u * kWaves);
  if (g > 256u) g = 256u;
  if (paik_tune.gemv_wgs >= 1 && paik_tune.gemv_wgs <= 65535) g = (uint32_t)paik_tune.gemv_wgs;
  const uint32_t need = (n + kWaves - 1u) / kWaves; /* at least one row per wave */
  if (need < g) g = need;
  const uint32_t least = (count + kWaves - 1u) / kWaves; /* a wave per matrix */
  return g < least ? least : g;
}

template <int MT>
static int pick_rows(uint32_t n, uint32_t grid) {
  const uint32_t rw = (n + grid * kWaves - 1u) / (grid * kWaves);
  int u = (rw >= 4u && 4 * MT <= 8) ? 4 : (2 * MT <= 8 ? 2 : 1);
  const int r = paik_tune.gemv_rows;
  if ((r == 1 || r == 2 || r == 4) && r * MT <= 8) u = r;
  return u;
}

/* Waves per matrix in proportion to its rows (at least one each). */
static void split_waves(GemvArgs &a, uint32_t total_waves) {
  uint64_t rows = 0;
  for (uint32_t i = 0; i < a.count; ++i) rows += a.v[i].n;
  uint32_t given = 0;
  for (uint32_t i = 0; i < a.count; ++i) {
    uint32_t w = (uint32_t)((uint64_t)total_waves * a.v[i].n / rows);
    if (w < 1u) w = 1u;
    const uint32_t left = total_waves - given - (a.count - 1u - i); /* keep one per later matrix */
    if (w > left || i + 1u == a.count) w = left;
    given += w;
    a.wave_end[i] = given;
  }
}

/* Chunks of one column slice: those whose activation planes for MT
 * tokens fit the LDS budget and one pass of the plane builder. */
static uint32_t slice_cap(uint32_t mt, int nw = kWaves, int xi = kXIt) {
  const uint32_t fit = (uint32_t)(kLdsBudget / ((size_t)mt * (sizeof(XSlot) + sizeof(XScale))));
  return min(fit, max_slice_tok(nw, xi) / mt);
}

/* One-token launches of up to 4096 rows (two rows per wave on 256
 * workgroups of 8 waves) run on that grid instead of half as many 16-wave
 * workgroups, so every CU shares the dot-product work, when a row still
 * fits one column slice of the smaller plane builder (the gemv_nw tuning
 * field, 16 or 8, forces either). */
static bool small_wg(uint32_t rows, uint32_t k, int xi = kXIt) {
  const int nw = paik_tune.gemv_nw;
  if ((k >> 5) > slice_cap(1u, kWavesSmall, xi)) return false; /* rows stay one slice */
  if (nw == 16) return false;
  if (nw == 8) return true;
  return rows <= kWavesSmall * 2u * 256u;
}

template <class F, int U, int MT, bool PAIR, int NW = kWaves, bool NORM = false>
static hipError_t launch_u(GemvArgs a, const float *x, uint32_t ntok, uint32_t grid,
                           hipStream_t s, int accum = 0) {
  const uint32_t nchunks = a.v[0].k >> 5;
  const uint32_t cap = slice_cap((uint32_t)MT, NW, NORM ? kXItNorm<F> : kXIt);
  const uint32_t slice = cap >= nchunks ? nchunks : (cap & ~63u);
  /* the silu epilogue and the fused RMSNorm need whole rows */
  if ((PAIR || NORM) && slice != nchunks) return hipErrorInvalidValue;
  if constexpr (PAIR) a.wave_end[0] = grid * (uint32_t)NW;
  else split_waves(a, grid * (uint32_t)NW);
  for (uint32_t cs = 0; cs < nchunks; cs += slice) {
    const uint32_t nsc = min(slice, nchunks - cs);
    const size_t lds = (size_t)MT * nsc * (sizeof(XSlot) + sizeof(XScale));
    k_gemv<F, U, MT, PAIR, NW, NORM><<<dim3(grid), dim3(64u * NW), lds, s>>>(
        a, x, ntok, cs, nsc, (accum != 0 || cs != 0u) ? 1 : 0);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <class F, int MT, bool NORM = false>
static hipError_t launch_gemv(const GemvArgs &a, const float *x, uint32_t ntok, hipStream_t s,
                              int accum = 0) {
  uint32_t rows = 0;
  for (uint32_t i = 0; i < a.count; ++i) rows += a.v[i].n;
  const uint32_t grid = pick_grid(rows, a.count);
  const int u = pick_rows<MT>(rows, grid);
  if constexpr (MT == 1) {
    if (small_wg(rows, a.v[0].k, NORM ? kXItNorm<F> : kXIt)) {
      /* 256 workgroups of kWavesSmall waves, two or more rows per wave */
      const uint32_t g8 = min(256u, (rows + 2u * kWavesSmall - 1u) / (2u * kWavesSmall));
      const uint32_t rw = (rows + g8 * kWavesSmall - 1u) / (g8 * kWavesSmall);
      if (rw >= 4u) return launch_u<F, 4, 1, false, kWavesSmall, NORM>(a, x, ntok, g8, s, accum);
      return launch_u<F, 2, 1, false, kWavesSmall, NORM>(a, x, ntok, g8, s, accum);
    }
    if (u == 4) return launch_u<F, 4, 1, false, kWaves, NORM>(a, x, ntok, grid, s, accum);
    if (u == 2) return launch_u<F, 2, 1, false, kWaves, NORM>(a, x, ntok, grid, s, accum);
    return launch_u<F, 1, 1, false, kWaves, NORM>(a, x, ntok, grid, s, accum);
  } else if constexpr (MT == 2) {
    if (u == 4) return launch_u<F, 4, 2, false>(a, x, ntok, grid, s);
    if (u == 2) return launch_u<F, 2, 2, false>(a, x, ntok, grid, s);
    return launch_u<F, 1, 2, false>(a, x, ntok, grid, s);
  } else {
    if (u == 2) return launch_u<F, 2, MT, false>(a, x, ntok, grid, s);
    return launch_u<F, 1, MT, false>(a, x, ntok, grid, s);
  }
}

/* Paired gate/up launch: grid sized for both matrices' rows; a row group
 * holds 2 rows of each matrix when waves get 2 or more rows (and MT <= 2),
 * else 1. */
template <class F, int MT, bool NORM = false>
static hipError_t launch_pair(const GemvArgs &a, const float *x, uint32_t ntok, hipStream_t s) {
  const uint32_t n = a.v[0].n;
  const uint32_t grid = pick_grid(2u * n, 1u);
  const uint32_t rw = (n + grid * kWaves - 1u) / (grid * kWaves);
  if constexpr (MT <= 2) {
    if (rw >= 2u) return launch_u<F, 4, MT, true, kWaves, NORM>(a, x, ntok, grid, s);
  }
  return launch_u<F, 2, MT, true, kWaves, NORM>(a, x, ntok, grid, s);
}

/* One token through the integer-dot kernel with the decode step's fusions:
 * gamma set, x is RMSNorm-ed on the way in; accum set, the products are
 * added to y; pair set, vs = {gate, up} and ys[0] = silu(gate) * up. */
template <class F>
static hipError_t gemv_one(const paik_qview_t *const *vs, float *const *ys, uint32_t count,
                           int pair, const float *x, const float *gamma, float eps, int accum,
                           hipStream_t s) {
  GemvArgs a;
  memset(&a, 0, sizeof a);
  a.count = count;
  for (uint32_t i = 0; i < count; ++i) {
    a.v[i] = *vs[i];
    a.y[i] = ys[i];
  }
  a.eps = eps;
  if (gamma != nullptr) {
    if (count > (uint32_t)kNormGammaSlot) return hipErrorInvalidValue;
    a.y[kNormGammaSlot] = const_cast<float *>(gamma); /* read only */
  }
  if (pair) {
    if (gamma != nullptr) return launch_pair<F, 1, true>(a, x, 1u, s);
    return launch_pair<F, 1>(a, x, 1u, s);
  }
  if (gamma != nullptr) return launch_gemv<F, 1, true>(a, x, 1u, s, accum);
  return launch_gemv<F, 1>(a, x, 1u, s, accum);
}

/* Calls of two or more tokens run on the matrix-core kernel (qgemv_mx.hip)
 * where it takes K: its weight operands are shared by all tokens of a
 * launch, while this kernel's integer dots are paid per token. One token
 * stays here, where the dots are cheaper than the matrix-core operand
 * layout's scattered loads. The gemv_no_mx tuning field keeps every call
 * here. */
static bool use_mx(uint32_t k, uint32_t m) {
  return paik_tune.gemv_no_mx == 0 && m >= 2u && paik_gemv_mx_tokens(k, m) != 0u;
}

template <class F>
static hipError_t gemv_tokens(const paik_qview_t *const *vs, float *const *ys, uint32_t count,
                              uint32_t m, const float *x, hipStream_t s) {
  if (use_mx(vs[0]->k, m)) return (hipError_t)paik_gemv_mx(vs, ys, count, m, x, s);
  /* groups of up to 4 tokens per launch; each launch re-streams W */
  for (uint32_t t0 = 0; t0 < m; t0 += 4u) {
    const uint32_t nt = m - t0 < 4u ? m - t0 : 4u;
    GemvArgs a;
    memset(&a, 0, sizeof a);
    a.count = count;
    for (uint32_t i = 0; i < count; ++i) {
      a.v[i] = *vs[i];
      a.y[i] = ys[i] + (size_t)t0 * vs[i]->n;
    }
    const float *xt = x + (size_t)t0 * vs[0]->k;
    hipError_t e;
    if (nt == 1u) e = launch_gemv<F, 1>(a, xt, 1u, s);
    else if (nt == 2u) e = launch_gemv<F, 2>(a, xt, 2u, s);
    else e = launch_gemv<F, 4>(a, xt, nt, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

/* h = silu(x W_gate^T) * (x W_up^T), in token groups whose activation
 * planes fit one slice (so every output is finished in one launch). */
template <class F>
static hipError_t gemv_pair_tokens(const paik_qview_t *vg, const paik_qview_t *vu, uint32_t m,
                                   const float *x, float *h, hipStream_t s) {
  if (use_mx(vg->k, m)) return (hipError_t)paik_gemv_mx_silu_mul(vg, vu, m, x, h, s);
  const uint32_t nchunks = vg->k >> 5;
  const uint32_t group = slice_cap(4u) >= nchunks ? 4u : slice_cap(2u) >= nchunks ? 2u : 1u;
  if (slice_cap(group) < nchunks) return hipErrorInvalidValue;
  for (uint32_t t0 = 0; t0 < m; t0 += group) {
    const uint32_t nt = m - t0 < group ? m - t0 : group;
    GemvArgs a;
    memset(&a, 0, sizeof a);
    a.count = 2;
    a.v[0] = *vg;
    a.v[1] = *vu;
    a.y[0] = h + (size_t)t0 * vg->n;
    const float *xt = x + (size_t)t0 * vg->k;
    hipError_t e;
    if (nt == 1u) e = launch_pair<F, 1>(a, xt, 1u, s);
    else if (nt == 2u) e = launch_pair<F, 2>(a, xt, 2u, s);
    else e = launch_pair<F, 4>(a, xt, nt, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

} // namespace paik

using namespace paik;

extern "C" uint32_t paik_gemv_pair_max_k(void) { return slice_cap(1u) * 32u; }
extern "C" uint32_t paik_gemv_norm_max_k(uint32_t type) {
  return slice_cap(1u, kWaves, type == 8u ? kXItNorm<Q8_0> : kXItNorm<Q4_K>) * 32u;
}

extern "C" int paik_gemv_silu_mul(const paik_qview_t *gate, const paik_qview_t *up, uint32_t m,
                                  const float *x, float *h, void *stream) {
  hipStream_t s = (hipStream_t)stream;
  if (gate->type != up->type || gate->n != up->n || gate->k != up->k)
    return (int)hipErrorInvalidValue;
  switch (gate->type) {
  case 8u: return (int)gemv_pair_tokens<Q8_0>(gate, up, m, x, h, s);
  case 2u: return (int)gemv_pair_tokens<Q4_0>(gate, up, m, x, h, s);
  case 12u: return (int)gemv_pair_tokens<Q4_K>(gate, up, m, x, h, s);
  case 14u: return (int)gemv_pair_tokens<Q6_K>(gate, up, m, x, h, s);
  default: return (int)hipErrorInvalidValue;
  }
}

extern "C" int paik_gemv_multi(const paik_qview_t *const *vs, float *const *ys, uint32_t count,
                               uint32_t m, const float *x, void *stream) {
  if (count == 0u || count > (uint32_t)kMaxMats) return (int)hipErrorInvalidValue;
  hipStream_t s = (hipStream_t)stream;
  switch (vs[0]->type) {
  case 8u: return (int)gemv_tokens<Q8_0>(vs, ys, count, m, x, s);
  case 2u: return (int)gemv_tokens<Q4_0>(vs, ys, count, m, x, s);
  case 12u: return (int)gemv_tokens<Q4_K>(vs, ys, count, m, x, s);
  case 14u: return (int)gemv_tokens<Q6_K>(vs, ys, count, m, x, s);
  default: return (int)hipErrorInvalidValue;
  }
}

extern "C" int paik_gemv_one(const paik_qview_t *const *vs, float *const *ys, uint32_t count,
                             int pair, const float *x, const float *gamma, float eps, int accum,
                             void *stream) {
  if (count == 0u || count > (uint32_t)kMaxMats) return (int)hipErrorInvalidValue;
  if (pair && (count != 2u || accum || vs[0]->n != vs[1]->n)) return (int)hipErrorInvalidValue;
  for (uint32_t i = 1; i < count; ++i)
    if (vs[i]->type != vs[0]->type || vs[i]->k != vs[0]->k) return (int)hipErrorInvalidValue;
  hipStream_t s = (hipStream_t)stream;
  switch (vs[0]->type) {
  case 8u: return (int)gemv_one<Q8_0>(vs, ys, count, pair, x, gamma, eps, accum, s);
  case 2u: return (int)gemv_one<Q4_0>(vs, ys, count, pair, x, gamma, eps, accum, s);
  case 12u: return (int)gemv_one<Q4_K>(vs, ys, count, pair, x, gamma, eps, accum, s);
  case 14u: return (int)gemv_one<Q6_K>(vs, ys, count, pair, x, gamma, eps, accum, s);
  default: return (int)hipErrorInvalidValue;
  }
}

extern "C" int paik_gemv(const paik_qview_t *v, uint32_t m, const float *x, float *y,
                         void *stream) {
  return paik_gemv_multi(&v, &y, 1u, m, x, stream);
}
