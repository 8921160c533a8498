/*
 * Batched / prefill GEMM over packed blocks on MFMA (gfx950).
 *
 * y[M][N] = x[M][K] · Wᵀ with W dequantized tile by tile into LDS as fp16
 * (or bf16), x converted to the same type, v_mfma_f32_16x16x32_{f16,bf16}
 * with f32 accumulation.
 *
 * Workgroup tile: 128 weight rows x 128 tokens; K advances 64 columns (two
 * 32-column chunks) per step. 256 threads: in a step every thread fetches
 * one chunk of one weight row and dequantizes it exactly (the reference's
 * f32 values, then one rounding to 16 bits), and converts eight float4 of
 * activations (a load instruction covers four tokens' 256 contiguous
 * bytes); both land in the step's LDS buffer. The loads of step s+1 are issued before the MFMAs of
 * step s, and the two LDS buffers alternate, so the fetch, the dequant and
 * the matrix work of neighbouring steps overlap.
 *
 * Four waves in a 2x2 grid each own a 64x64 output block: per 32-column
 * slice a wave reads four 16-row A fragments and four 16-token B fragments
 * from LDS and issues 16 MFMAs.
 *
 * Operand layout used for v_mfma_f32_16x16x32_*: lane l supplies row
 * (l % 16) of the A tile and column (l % 16) of the B tile, each with the
 * 8 K values [8*(l/16), 8*(l/16)+8) of the 32-wide slice; both operands
 * use the same K assignment, so the product is the full 32-term dot
 * product. Lane l receives D[4*(l/16) + i][l % 16], i = 0..3.
 */
#include "qdev.h"

namespace paik {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 b8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int BN = 128, BM = 128, BK = 64;
constexpr int LDK = BK + 8; /* LDS row pitch in 16-bit elements (bank spread) */

template <bool BF>
__device__ __forceinline__ uint16_t to16(float f) {
  if constexpr (BF) return __builtin_bit_cast(uint16_t, (__bf16)f);
  else return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <bool BF>
__device__ __forceinline__ f4_t mfma(const uint4 &a, const uint4 &b, f4_t c) {
  if constexpr (BF)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8_t, a),
                                                   __builtin_bit_cast(b8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a),
                                                  __builtin_bit_cast(h8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return (uint32_t)lo | ((uint32_t)hi << 16);
}

/* 32 values -> 16-bit, stored as four 16-byte words at dst */
template <bool BF>
__device__ __forceinline__ void put32(uint16_t *dst, const float o[32]) {
#pragma unroll
  for (int i = 0; i < 32; i += 8) {
    uint4 p;
    p.x = pack2(to16<BF>(o[i]), to16<BF>(o[i + 1]));
    p.y = pack2(to16<BF>(o[i + 2]), to16<BF>(o[i + 3]));
    p.z = pack2(to16<BF>(o[i + 4]), to16<BF>(o[i + 5]));
    p.w = pack2(to16<BF>(o[i + 6]), to16<BF>(o[i + 7]));
    *reinterpret_cast<uint4 *>(dst + i) = p;
  }
}

/* What one thread fetches for one K step: one weight chunk (row tid/2,
 * chunk tid%2) and eight float4 of activations (token tid/16 + 16i,
 * columns 4*(tid%16)..+3), so that the 64 lanes of a load instruction read
 * four tokens' 256 contiguous bytes each. */
template <class F>
struct StepRegs {
  typename F::Raw w;
  float4 xv[8];
  bool wv;
};

template <class F, bool BF>
__global__ void __launch_bounds__(256) k_gemm(paik_qview_t v, const float *__restrict__ x,
                                              float *__restrict__ y, uint32_t m) {
  __shared__ __attribute__((aligned(16))) uint16_t Ws[2][BN * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Xs[2][BM * LDK];

  const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const uint32_t n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const uint32_t nchunks = v.k >> 5;
  const uint32_t nsteps = (nchunks + 1u) >> 1;

  /* this thread's share of a step */
  const int rr = tid >> 1, hf = tid & 1; /* weight row, chunk half */
  const int xt = tid >> 4, x4 = tid & 15; /* first token, float4 column */
  const uint32_t wrow = n0 + (uint32_t)rr;

  auto fetch = [&](uint32_t s, StepRegs<F> &r) {
    const uint32_t c = 2u * s + (uint32_t)hf;
    r.wv = wrow < v.n && c < nchunks;
    if (r.wv) r.w = F::load(v, wrow, c);
    const uint32_t col = 64u * s + 4u * (uint32_t)x4;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t tok = m0 + (uint32_t)(xt + 16 * i);
      r.xv[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (tok < m && col < v.k)
        r.xv[i] = *reinterpret_cast<const float4 *>(x + (size_t)tok * v.k + col);
    }
  };
  auto stage = [&](uint32_t s, const StepRegs<F> &r, int buf) {
    const uint32_t c = 2u * s + (uint32_t)hf;
    float o[32];
    if (r.wv) {
      F::dequant(r.w, c, o);
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i) o[i] = 0.0f;
    }
    put32<BF>(&Ws[buf][rr * LDK + 32 * hf], o);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 f = r.xv[i];
      uint2 p;
      p.x = pack2(to16<BF>(f.x), to16<BF>(f.y));
      p.y = pack2(to16<BF>(f.z), to16<BF>(f.w));
      *reinterpret_cast<uint2 *>(&Xs[buf][(xt + 16 * i) * LDK + 4 * x4]) = p;
    }
  };

  f4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  StepRegs<F> r;
  fetch(0u, r);
  stage(0u, r, 0);
  __syncthreads();

  for (uint32_t s = 0; s < nsteps; ++s) {
    const int cur = (int)(s & 1u);
    const bool more = s + 1u < nsteps;
    if (more) fetch(s + 1u, r); /* in flight during this step's MFMAs */
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      const int ko = kk + 8 * (lane >> 4);
      uint4 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = *reinterpret_cast<const uint4 *>(
            &Ws[cur][(wr * 64 + i * 16 + (lane & 15)) * LDK + ko]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = *reinterpret_cast<const uint4 *>(
            &Xs[cur][(wc * 64 + j * 16 + (lane & 15)) * LDK + ko]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma<BF>(a[i], b[j], acc[i][j]);
    }
    if (more) stage(s + 1u, r, cur ^ 1);
    __syncthreads();
  }

  /* D[row][tok]: rows 4*(lane/16)+q, token lane%16 of each 16x16 tile */
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t tok = m0 + (uint32_t)(wc * 64 + j * 16 + (lane & 15));
      const uint32_t rb = n0 + (uint32_t)(wr * 64 + i * 16 + 4 * (lane >> 4));
      if (tok >= m) continue;
      float *dst = y + (size_t)tok * v.n;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (rb + (uint32_t)q < v.n) dst[rb + (uint32_t)q] = acc[i][j][q];
    }
  }
}

template <class F>
static hipError_t launch_gemm(const paik_qview_t &v, uint32_t m, const float *x, float *y,
                              bool bf16, hipStream_t s) {
  const dim3 grid((v.n + BN - 1) / BN, (m + BM - 1) / BM), block(256);
  if (bf16) k_gemm<F, true><<<grid, block, 0, s>>>(v, x, y, m);
  else k_gemm<F, false><<<grid, block, 0, s>>>(v, x, y, m);
  return hipGetLastError();
}

} // namespace paik

using namespace paik;

extern "C" int paik_gemm_mfma(const paik_qview_t *v, uint32_t m, const float *x, float *y,
                              int bf16, void *stream) {
  hipStream_t s = (hipStream_t)stream;
  switch (v->type) {
  case 8u: return (int)launch_gemm<Q8_0>(*v, m, x, y, bf16 != 0, s);
  case 2u: return (int)launch_gemm<Q4_0>(*v, m, x, y, bf16 != 0, s);
  case 12u: return (int)launch_gemm<Q4_K>(*v, m, x, y, bf16 != 0, s);
  case 14u: return (int)launch_gemm<Q6_K>(*v, m, x, y, bf16 != 0, s);
  default: return (int)hipErrorInvalidValue;
  }
}
