/*
 * The v0 per-group formats on gfx950 (models/quantize.h: signed
 * symmetric, 8 or 4 bits, one f32 scale per group):
 *
 *   GEMMs over W[K][N] as the reference's pai_ref_gemm_w8_f32 / _w4_f32
 *   take it (cpu/reference/ref_ops.c:446-499): int8 codes w[t*n+j], or
 *   nibbles over that flat index (low nibble for even indices, sign-
 *   extended); scales[(t/gs)*n + j], one per (group of gs rows, column).
 *
 *   Quantize / dequantize of a flat array (models/quantize.c:74-181).
 *
 * GEMM (k_v0_gemm). A workgroup owns a strip of 256 columns and a range
 * of 16-row blocks (one part of K); its 16 x 16 threads are 16 column
 * threads of 16 columns each (one 16-byte load of int8 codes or one
 * 8-byte load of nibbles per row) by 16 thread rows, each thread row
 * walking every 16th block of the range. Row t of a strip is 256 (or 128)
 * contiguous bytes, so a wave's load covers 4 rows of whole 64-byte
 * segments. A block never straddles a group (gs is a multiple of 16 or
 * covers K), so each thread loads its 16 scales once per block, and the
 * dequantized weight is fma(s, u, -z s) with u = code + z (z = 128 or 8,
 * u taken from the code byte by v_cvt_f32_ubyte), which is s * q rounded
 * once: the reference's dequantized value. Up to 4 tokens share each
 * weight load. The 16 thread rows are summed in a fixed order (lane
 * shuffles, then the 4 waves through LDS); with K split over workgroups
 * the parts go to a workspace and a second launch adds them in part
 * order, so results repeat bit for bit.
 *
 * Shapes the strip kernel does not take (n not a multiple of 16, gs not a
 * multiple of 16 and below K, unaligned pointers) run on k_v0_gemm_seq:
 * one thread per output, the reference's sum in its order with separately
 * rounded products (bit-identical to it).
 */
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "paik.h"

namespace paik {
namespace v0 {

constexpr int kCols = 16;      /* columns per thread */
constexpr int kColThreads = 16;
constexpr int kStrip = kCols * kColThreads; /* 256 columns per workgroup */
constexpr int kRowThreads = 16;
constexpr int kBlk = 16;       /* rows per block */

struct GemmArgs {
  const float *a;        /* [m][k] */
  const uint8_t *wq;     /* [k][n] codes */
  const float *scales;   /* [groups][n] */
  float *out;            /* c [m][n], or the parts [parts][m][n] */
  uint32_t m, n, k, gs;  /* gs in 1..k */
  uint32_t strips, parts, bpp; /* 16-row blocks per part */
};

/* The 16 weights of one row of a thread's columns, dequantized: s * q
 * with one rounding (fma of s, the biased code u = q + z, and -z s). */
template <int BITS>
__device__ __forceinline__ void decode_row(const uint4 &raw, const float (&s)[kCols],
                                           const float (&o)[kCols], float (&w)[kCols]) {
  if constexpr (BITS == 8) {
    const uint32_t wd[4] = {raw.x ^ 0x80808080u, raw.y ^ 0x80808080u, raw.z ^ 0x80808080u,
                            raw.w ^ 0x80808080u};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int b = 0; b < 4; ++b)
        w[4 * i + b] = __builtin_fmaf(s[4 * i + b], (float)((wd[i] >> (8 * b)) & 0xFFu),
                                      o[4 * i + b]);
  } else {
    /* 8 bytes: byte b of word i holds columns 8i + 2b (low) and 8i + 2b + 1 */
    const uint32_t wd[2] = {raw.x ^ 0x88888888u, raw.y ^ 0x88888888u};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t lo = wd[i] & 0x0F0F0F0Fu, hi = (wd[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int c = 8 * i + 2 * b;
        w[c] = __builtin_fmaf(s[c], (float)((lo >> (8 * b)) & 0xFFu), o[c]);
        w[c + 1] = __builtin_fmaf(s[c + 1], (float)((hi >> (8 * b)) & 0xFFu), o[c + 1]);
      }
    }
  }
}

template <int BITS, int MT>
__global__ void __launch_bounds__(256) k_v0_gemm(GemmArgs g) {
  __shared__ float red[4][MT][kStrip];
  const int tid = (int)threadIdx.x;
  const int ct = tid & 15, tr = tid >> 4;
  const uint32_t strip = blockIdx.x % g.strips, part = blockIdx.x / g.strips;
  const uint32_t m0 = blockIdx.y * (uint32_t)MT;
  const uint32_t c0 = strip * (uint32_t)kStrip + (uint32_t)(ct * kCols);
  const uint32_t nblk = (g.k + kBlk - 1u) / kBlk;
  const uint32_t b0 = part * g.bpp, b1 = min(b0 + g.bpp, nblk);
  constexpr float kBias = BITS == 8 ? -128.0f : -8.0f;

  float acc[MT][kCols];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int c = 0; c < kCols; ++c) acc[t][c] = 0.0f;

  if (c0 < g.n) {
    for (uint32_t b = b0 + (uint32_t)tr; b < b1; b += kRowThreads) {
      const uint32_t t0 = b * kBlk;
      const float4 *sp = (const float4 *)(g.scales + (size_t)(t0 / g.gs) * g.n + c0);
      float s[kCols], o[kCols];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 v = sp[i];
        s[4 * i] = v.x; s[4 * i + 1] = v.y; s[4 * i + 2] = v.z; s[4 * i + 3] = v.w;
      }
#pragma unroll
      for (int c = 0; c < kCols; ++c) o[c] = kBias * s[c];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint4 raw[8];
        float xv[MT][8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const uint32_t t = t0 + (uint32_t)(8 * h + r);
          const bool ok = t < g.k;
          const size_t flat = (size_t)min(t, g.k - 1u) * g.n + c0;
          if constexpr (BITS == 8) {
            raw[r] = *(const uint4 *)(g.wq + flat);
          } else {
            const uint2 v = *(const uint2 *)(g.wq + flat / 2u);
            raw[r] = make_uint4(v.x, v.y, 0u, 0u);
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const uint32_t tok = min(m0 + (uint32_t)mt, g.m - 1u);
            const float xa = g.a[(size_t)tok * g.k + min(t, g.k - 1u)];
            xv[mt][r] = ok && m0 + (uint32_t)mt < g.m ? xa : 0.0f;
          }
        }
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          float w[kCols];
          decode_row<BITS>(raw[r], s, o, w);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int c = 0; c < kCols; ++c) acc[mt][c] = __builtin_fmaf(xv[mt][r], w[c], acc[mt][c]);
        }
      }
    }
  }

  /* thread rows 0..3 of each wave (lanes 16 apart), then the 4 waves */
  const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int c = 0; c < kCols; ++c) {
      float v = acc[mt][c];
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (lane < 16) red[wave][mt][lane * kCols + c] = v;
    }
  __syncthreads();
  const uint32_t col = strip * (uint32_t)kStrip + (uint32_t)tid;
  if (col < g.n) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const uint32_t tok = m0 + (uint32_t)mt;
      if (tok >= g.m) break;
      const float v = ((red[0][mt][tid] + red[1][mt][tid]) + red[2][mt][tid]) + red[3][mt][tid];
      g.out[((size_t)part * g.m + tok) * g.n + col] = v;
    }
  }
}

/* c[e] = sum over p ascending of parts[p][e]. */
__global__ void __launch_bounds__(256) k_v0_reduce(const float *parts, float *c, size_t len,
                                                   uint32_t np) {
  for (size_t e = (size_t)blockIdx.x * 256u + threadIdx.x; e < len;
       e += (size_t)gridDim.x * 256u) {
    float s = parts[e];
    for (uint32_t p = 1; p < np; ++p) s += parts[(size_t)p * len + e];
    c[e] = s;
  }
}

template <int BITS>
__device__ __forceinline__ int32_t code_at(const uint8_t *wq, size_t flat) {
  if constexpr (BITS == 8) {
    return (int32_t)(int8_t)wq[flat];
  } else {
    const uint32_t byte = wq[flat / 2u];
    const int32_t nib = (int32_t)((flat & 1u) == 0u ? (byte & 0x0Fu) : (byte >> 4));
    return (nib & 8) ? nib - 16 : nib;
  }
}

/* One output per thread: sum over t ascending of (a[i][t] * q) * s, each
 * product and sum rounded separately, as the reference evaluates it. */
template <int BITS>
__global__ void __launch_bounds__(256) k_v0_gemm_seq(GemmArgs g) {
  /* device code contracts a * b + c into one fma by default */
#pragma clang fp contract(off)
  const uint32_t j = blockIdx.x * 256u + threadIdx.x, i = blockIdx.y;
  if (j >= g.n) return;
  const float *ar = g.a + (size_t)i * g.k;
  float sum = 0.0f;
  uint32_t grp = 0, in_grp = 0;
  for (uint32_t t = 0; t < g.k; ++t) {
    const float q = (float)code_at<BITS>(g.wq, (size_t)t * g.n + j);
    sum += (ar[t] * q) * g.scales[(size_t)grp * g.n + j];
    if (++in_grp == g.gs) {
      in_grp = 0;
      ++grp;
    }
  }
  g.out[(size_t)i * g.n + j] = sum;
}

/* ---------------------------------------------------------------------- */
/* Quantize / dequantize (models/quantize.c:74-181)                        */
/* ---------------------------------------------------------------------- */

constexpr uint32_t kRun = 16; /* consecutive elements (8-bit) or bytes (4-bit) per thread */

/* max |x| of (group, chunk) items, one wave each (NaN is skipped, as the
 * reference's `av > max_abs` skips it). With one chunk per group the wave
 * writes the scale; otherwise it raises maxbits[group] (the scale array,
 * zero-filled, read as the bits of non-negative floats) and a second
 * launch turns maxima into scales. */
__global__ void __launch_bounds__(256) k_v0_absmax(const float *x, uint32_t n, uint32_t gs,
                                                   uint32_t chunks, uint32_t chunk, uint32_t items,
                                                   float qmax, float *scales) {
  const uint32_t item = blockIdx.x * 4u + (threadIdx.x >> 6), lane = threadIdx.x & 63u;
  if (item >= items) return;
  const uint32_t grp = item / chunks, ch = item % chunks;
  const uint32_t gend = (uint32_t)min((uint64_t)grp * gs + gs, (uint64_t)n);
  const uint32_t begin = grp * gs + ch * chunk;
  const uint32_t end = (uint32_t)min((uint64_t)begin + chunk, (uint64_t)gend);
  float m = 0.0f;
  for (uint32_t i = begin + lane; i < end; i += 64u) {
    const float v = fabsf(x[i]);
    m = v > m ? v : m;
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const float o = __shfl_xor(m, d);
    m = o > m ? o : m;
  }
  if (lane != 0u) return;
  if (chunks == 1u)
    scales[grp] = m > 0.0f ? __fdiv_rn(m, qmax) : 0.0f;
  else
    atomicMax((unsigned int *)scales + grp, __float_as_uint(m));
}

__global__ void __launch_bounds__(256) k_v0_scale_final(float *scales, uint32_t groups, float qmax) {
  const uint32_t g = blockIdx.x * 256u + threadIdx.x;
  if (g >= groups) return;
  const float m = scales[g];
  scales[g] = m > 0.0f ? __fdiv_rn(m, qmax) : 0.0f;
}

__global__ void __launch_bounds__(256) k_v0_fill_zero(uint32_t *p, uint32_t n) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i < n) p[i] = 0u;
}

/* lrintf(x / s) clamped to [-qmax, qmax]; 0 for s = 0. A NaN quotient
 * gives 0, which is what the reference's conversion of lrintf's result to
 * int32 gives for it. */
__device__ __forceinline__ int32_t quant_one(float x, float s, float qmax) {
  if (!(s > 0.0f)) return 0;
  const float r = rintf(__fdiv_rn(x, s));
  if (!(fabsf(r) <= 1.0e9f)) return 0;
  return (int32_t)fminf(fmaxf(r, -qmax), qmax);
}

/* Group of element i when a thread walks a run upward from i0, whose group
 * is g0 = i0 / gs at offset r0 = i0 % gs in it. */
struct GroupWalk {
  uint32_t g, r, gs;
  __device__ GroupWalk(uint32_t i0, uint32_t gs_) : g(i0 / gs_), r(i0 % gs_), gs(gs_) {}
  __device__ void step() {
    if (++r == gs) {
      r = 0u;
      ++g;
    }
  }
};

template <int BITS>
__global__ void __launch_bounds__(256) k_v0_quant(const float *x, uint32_t n, uint32_t gs,
                                                  const float *scales, uint8_t *q, float qmax) {
  const uint64_t run = (uint64_t)blockIdx.x * 256u + threadIdx.x;
  if constexpr (BITS == 8) {
    const uint64_t i0 = run * kRun;
    if (i0 >= n) return;
    GroupWalk w((uint32_t)i0, gs);
    uint8_t out[kRun];
#pragma unroll
    for (uint32_t e = 0; e < kRun; ++e) {
      const uint64_t i = i0 + e;
      out[e] = i < n ? (uint8_t)quant_one(x[i], scales[w.g], qmax) : 0u;
      w.step();
    }
    if (i0 + kRun <= n) {
      uint4 v;
      v.x = out[0] | (out[1] << 8) | (out[2] << 16) | ((uint32_t)out[3] << 24);
      v.y = out[4] | (out[5] << 8) | (out[6] << 16) | ((uint32_t)out[7] << 24);
      v.z = out[8] | (out[9] << 8) | (out[10] << 16) | ((uint32_t)out[11] << 24);
      v.w = out[12] | (out[13] << 8) | (out[14] << 16) | ((uint32_t)out[15] << 24);
      *(uint4 *)(q + i0) = v;
    } else {
      for (uint64_t i = i0; i < n; ++i) q[i] = out[i - i0];
    }
  } else {
    const uint64_t byte0 = run * kRun, nbytes = ((uint64_t)n + 1u) / 2u;
    if (byte0 >= nbytes) return;
    GroupWalk w((uint32_t)(2u * byte0), gs);
    uint8_t out[kRun];
#pragma unroll
    for (uint32_t e = 0; e < kRun; ++e) {
      const uint64_t i = 2u * (byte0 + e);
      const uint32_t lo = i < n ? (uint32_t)quant_one(x[i], scales[w.g], qmax) & 15u : 0u;
      w.step();
      const uint32_t hi = i + 1u < n ? (uint32_t)quant_one(x[i + 1u], scales[w.g], qmax) & 15u : 0u;
      w.step();
      out[e] = (uint8_t)(lo | (hi << 4));
    }
    if (byte0 + kRun <= nbytes) {
      uint4 v;
      v.x = out[0] | (out[1] << 8) | (out[2] << 16) | ((uint32_t)out[3] << 24);
      v.y = out[4] | (out[5] << 8) | (out[6] << 16) | ((uint32_t)out[7] << 24);
      v.z = out[8] | (out[9] << 8) | (out[10] << 16) | ((uint32_t)out[11] << 24);
      v.w = out[12] | (out[13] << 8) | (out[14] << 16) | ((uint32_t)out[15] << 24);
      *(uint4 *)(q + byte0) = v;
    } else {
      for (uint64_t b = byte0; b < nbytes; ++b) q[b] = out[b - byte0];
    }
  }
}

/* out[i] = scale * (float)q, one rounding (models/quantize.c:177). */
template <int BITS>
__global__ void __launch_bounds__(256) k_v0_dequant(const uint8_t *q, const float *scales,
                                                    uint32_t n, uint32_t gs, float *out) {
  const uint64_t i0 = ((uint64_t)blockIdx.x * 256u + threadIdx.x) * kRun;
  if (i0 >= n) return;
  GroupWalk w((uint32_t)i0, gs);
  float v[kRun];
#pragma unroll
  for (uint32_t e = 0; e < kRun; ++e) {
    const uint64_t i = i0 + e;
    v[e] = i < n ? scales[w.g] * (float)code_at<BITS>(q, i) : 0.0f;
    w.step();
  }
  if (i0 + kRun <= n) {
#pragma unroll
    for (uint32_t e = 0; e < kRun; e += 4u)
      *(float4 *)(out + i0 + e) = make_float4(v[e], v[e + 1], v[e + 2], v[e + 3]);
  } else {
    for (uint64_t i = i0; i < n; ++i) out[i] = v[i - i0];
  }
}

/* ---------------------------------------------------------------------- */
/* Launchers                                                                */
/* ---------------------------------------------------------------------- */

static uint32_t cdiv(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1u) / b); }

template <int BITS, int MT>
static hipError_t launch_strips(GemmArgs g, float *c, float *ws, size_t ws_bytes, hipStream_t s) {
  const uint32_t mblocks = cdiv(g.m, MT);
  const uint32_t nblk = cdiv(g.k, kBlk);
  /* split K while fewer than 512 workgroups would run, each part keeping
   * at least one block per thread row, the parts fitting the workspace */
  uint32_t parts = 1;
  while ((uint64_t)g.strips * mblocks * parts * 2u <= 512u && nblk / (parts * 2u) >= kRowThreads &&
         (uint64_t)parts * 2u * g.m * g.n * 4u <= ws_bytes)
    parts *= 2u;
  g.bpp = cdiv(nblk, parts);
  g.parts = cdiv(nblk, g.bpp);
  g.out = g.parts > 1u ? ws : c;
  const dim3 grid(g.strips * g.parts, mblocks);
  hipLaunchKernelGGL((k_v0_gemm<BITS, MT>), grid, dim3(256), 0, s, g);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || g.parts == 1u) return e;
  const size_t len = (size_t)g.m * g.n;
  const uint32_t blocks = (uint32_t)min((size_t)2048u, (len + 255u) / 256u);
  hipLaunchKernelGGL(k_v0_reduce, dim3(blocks), dim3(256), 0, s, (const float *)ws, c, len,
                     g.parts);
  return hipGetLastError();
}

template <int BITS>
static hipError_t gemm(const paik_v0_gemm_t *p, hipStream_t s) {
  GemmArgs g = {};
  g.a = p->a;
  g.wq = (const uint8_t *)p->wq;
  g.scales = p->scales;
  g.m = p->m;
  g.n = p->n;
  g.k = p->k;
  g.gs = p->gs;
  g.strips = cdiv(p->n, kStrip);
  if (!p->strip_ok || p->sequential) {
    g.out = p->c;
    hipLaunchKernelGGL(k_v0_gemm_seq<BITS>, dim3(cdiv(p->n, 256u), p->m), dim3(256), 0, s, g);
    return hipGetLastError();
  }
  float *ws = (float *)p->workspace;
  const size_t wb = p->workspace != nullptr ? p->workspace_bytes : 0u;
  if (p->m == 1u) return launch_strips<BITS, 1>(g, p->c, ws, wb, s);
  if (p->m == 2u) return launch_strips<BITS, 2>(g, p->c, ws, wb, s);
  return launch_strips<BITS, 4>(g, p->c, ws, wb, s);
}

} // namespace v0
} // namespace paik

using namespace paik::v0;

extern "C" int paik_v0_gemm(const paik_v0_gemm_t *p, void *stream) {
  const hipStream_t s = (hipStream_t)stream;
  return (int)(p->bits == 8u ? gemm<8>(p, s) : gemm<4>(p, s));
}

extern "C" int paik_v0_quantize(const float *x, uint32_t n, uint32_t bits, uint32_t gs,
                                int8_t *q, float *scales, void *stream) {
  const hipStream_t s = (hipStream_t)stream;
  const float qmax = bits == 8u ? 127.0f : 7.0f;
  const uint32_t groups = cdiv(n, gs);
  /* chunks of at most 16384 elements: one wave reduces each */
  const uint32_t chunk = gs < 16384u ? gs : 16384u;
  const uint32_t chunks = cdiv(gs, chunk);
  const uint64_t items = (uint64_t)groups * chunks;
  if (items > 0x7FFFFFFFull) return (int)hipErrorInvalidValue;
  if (chunks > 1u) {
    hipLaunchKernelGGL(k_v0_fill_zero, dim3(cdiv(groups, 256u)), dim3(256), 0, s,
                       (uint32_t *)scales, groups);
  }
  hipLaunchKernelGGL(k_v0_absmax, dim3(cdiv(items, 4u)), dim3(256), 0, s, x, n, gs, chunks, chunk,
                     (uint32_t)items, qmax, scales);
  if (chunks > 1u) {
    hipLaunchKernelGGL(k_v0_scale_final, dim3(cdiv(groups, 256u)), dim3(256), 0, s, scales,
                       groups, qmax);
  }
  const uint64_t runs = bits == 8u ? cdiv(n, kRun) : cdiv(((uint64_t)n + 1u) / 2u, kRun);
  if (bits == 8u)
    hipLaunchKernelGGL(k_v0_quant<8>, dim3(cdiv(runs, 256u)), dim3(256), 0, s, x, n, gs,
                       (const float *)scales, (uint8_t *)q, qmax);
  else
    hipLaunchKernelGGL(k_v0_quant<4>, dim3(cdiv(runs, 256u)), dim3(256), 0, s, x, n, gs,
                       (const float *)scales, (uint8_t *)q, qmax);
  return (int)hipGetLastError();
}

extern "C" int paik_v0_dequantize(const int8_t *q, const float *scales, uint32_t n, uint32_t bits,
                                  uint32_t gs, float *out, void *stream) {
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid(cdiv(cdiv(n, kRun), 256u));
  if (bits == 8u)
    hipLaunchKernelGGL(k_v0_dequant<8>, grid, dim3(256), 0, s, (const uint8_t *)q, scales, n, gs,
                       out);
  else
    hipLaunchKernelGGL(k_v0_dequant<4>, grid, dim3(256), 0, s, (const uint8_t *)q, scales, n, gs,
                       out);
  return (int)hipGetLastError();
}
