/*
 * Batched / prefill GEMM over packed blocks on MFMA (gfx950).
 *
 * y[M][N] = x[M][K] · Wᵀ with W dequantized tile by tile into LDS as fp16
 * (or bf16), x converted to the same type, v_mfma_f32_16x16x32_{f16,bf16}
 * with f32 accumulation.
 *
 * Tile: 64 weight rows x 64 tokens per workgroup, 256-column K steps (one
 * K-quant super-block, eight Q4_0/Q8_0 blocks). Four waves in a 2x2 grid
 * each own a 32x32 output block (2x2 MFMA tiles). A K step is: x tile ->
 * fp16 in LDS, 512 weight chunks dequantized (exact f32 value, then one
 * rounding to fp16) into LDS, barrier, 8 MFMA k-slices, barrier.
 *
 * Operand layout used for v_mfma_f32_16x16x32_*: lane l supplies row
 * (l % 16) of the A tile and column (l % 16) of the B tile, each with the
 * 8 K values [8*(l/16), 8*(l/16)+8) of the 32-wide k-slice; both operands
 * use the same K assignment, so the product is the full 32-term dot
 * product. Lane l receives D[4*(l/16) + i][l % 16], i = 0..3.
 */
#include "qdev.h"

namespace paik {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 b8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int BN = 64, BM = 64, BK = 256, LDK = BK + 8; /* LDK in 16-bit elements */

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

template <class F, bool BF>
__global__ void __launch_bounds__(256) k_gemm(paik_qview_t v, const float *__restrict__ x,
                                              float *__restrict__ y, uint32_t m) {
  __shared__ __attribute__((aligned(16))) uint16_t Ws[BN * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Xs[BM * LDK];

  const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const uint32_t n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const uint32_t nchunks = v.k >> 5;

  f4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  for (uint32_t k0 = 0; k0 < v.k; k0 += BK) {
    /* activations: BM x BK f32 -> 16-bit, 16 float4 per thread */
    for (int i = tid; i < BM * (BK / 4); i += 256) {
      const int tok = i / (BK / 4), kk = (i % (BK / 4)) * 4;
      float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
      if (m0 + (uint32_t)tok < m && k0 + (uint32_t)kk < v.k)
        f = *reinterpret_cast<const float4 *>(x + (size_t)(m0 + tok) * v.k + k0 + kk);
      uint2 p;
      p.x = pack2(to16<BF>(f.x), to16<BF>(f.y));
      p.y = pack2(to16<BF>(f.z), to16<BF>(f.w));
      *reinterpret_cast<uint2 *>(&Xs[tok * LDK + kk]) = p;
    }
    /* weights: BN rows x 8 chunks, exact f32 dequant then one rounding */
    for (int j = tid; j < BN * (BK / 32); j += 256) {
      const int row = j / (BK / 32);
      const uint32_t c = (k0 >> 5) + (uint32_t)(j % (BK / 32));
      float o[32];
      if (n0 + (uint32_t)row < v.n && c < nchunks) {
        F::dequant(F::load(v, n0 + (uint32_t)row, c), c, o);
      } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) o[i] = 0.0f;
      }
#pragma unroll
      for (int i = 0; i < 32; i += 8) {
        const uint32_t e = 32u * c + (uint32_t)i - k0;
        uint4 p;
        p.x = pack2(to16<BF>(o[i]), to16<BF>(o[i + 1]));
        p.y = pack2(to16<BF>(o[i + 2]), to16<BF>(o[i + 3]));
        p.z = pack2(to16<BF>(o[i + 4]), to16<BF>(o[i + 5]));
        p.w = pack2(to16<BF>(o[i + 6]), to16<BF>(o[i + 7]));
        *reinterpret_cast<uint4 *>(&Ws[row * LDK + (int)e]) = p;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      const int ko = kk + 8 * (lane >> 4);
      uint4 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = *reinterpret_cast<const uint4 *>(&Ws[(wr * 32 + i * 16 + (lane & 15)) * LDK + ko]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = *reinterpret_cast<const uint4 *>(&Xs[(wc * 32 + j * 16 + (lane & 15)) * LDK + ko]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma<BF>(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }

  /* D[row][tok]: rows 4*(lane/16)+r, token lane%16 of each 16x16 tile */
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t tok = m0 + (uint32_t)(wc * 32 + j * 16 + (lane & 15));
      const uint32_t rb = n0 + (uint32_t)(wr * 32 + i * 16 + 4 * (lane >> 4));
      if (tok >= m) continue;
      float *dst = y + (size_t)tok * v.n;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (rb + (uint32_t)r < v.n) dst[rb + (uint32_t)r] = acc[i][j][r];
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
