/*
 * Decode GEMV / small-batch GEMM over packed blocks (f32 arithmetic).
 *
 * y[t][r] = sum_k x[t][k] * W[r][k] for up to MT tokens per launch.
 *
 * Work split (memory-bound path, HBM streaming of the code planes):
 *   - a "segment" is 64 chunks = 2048 columns: lane l of a wavefront owns
 *     chunk 64s+l of every row, so the wave's 64 x 16-byte code loads of a
 *     row are one contiguous 1 KiB (2 KiB for Q8_0) read;
 *   - the lane's 32 activations per token stay in registers for all the
 *     rows the wave visits (no LDS traffic for x);
 *   - a workgroup holds one wave per segment (up to 8; more segments are
 *     looped) and a tile of rows; each wave reduces its per-row partials
 *     across lanes with DPP/permute, and the waves' partials are summed in
 *     a fixed order through LDS, so results do not depend on scheduling.
 * Codes are turned into f32 in registers (v_cvt_f32_ubyte*) and multiplied
 * against x with f32 FMA; per-group scales and the code offsets are applied
 * once per group using precomputed per-lane sums of x.
 */
#include "qdev.h"

namespace paik {

constexpr int kMaxRowsPerWg = 32;
constexpr int kMaxWaves = 8;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <class F, int MT>
__global__ void __launch_bounds__(512) k_gemv(paik_qview_t v, const float *__restrict__ x,
                                              float *__restrict__ y, uint32_t ntok,
                                              uint32_t rows_per_wg) {
  constexpr int NG = (int)F::kNG, GS = 32 / NG, RUN = (int)F::kRun;
  __shared__ float red[kMaxWaves][kMaxRowsPerWg * MT];

  const int lane = (int)(threadIdx.x & 63u), wave = (int)(threadIdx.x >> 6);
  const int nwaves = (int)(blockDim.x >> 6);
  const uint32_t r0 = blockIdx.x * rows_per_wg;
  const int nrows = (int)min(rows_per_wg, v.n - r0);
  const uint32_t nchunks = v.k >> 5;
  const uint32_t nseg = (nchunks + 63u) >> 6;

  for (int i = lane; i < nrows * MT; i += 64) red[wave][i] = 0.0f;

  for (uint32_t s = (uint32_t)wave; s < nseg; s += (uint32_t)nwaves) {
    const uint32_t c = 64u * s + (uint32_t)lane;
    const bool valid = c < nchunks;

    float xs[MT][32];
    float sx[MT][NG];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
#pragma unroll
      for (int r = 0; r < 32; r += RUN) {
        const uint32_t e = valid ? F::elem(c, r) : 0u;
        const float *src = x + (size_t)t * v.k + e;
#pragma unroll
        for (int i = 0; i < RUN; i += 4) {
          float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
          if (valid && (uint32_t)t < ntok) f = *reinterpret_cast<const float4 *>(src + i);
          xs[t][r + i] = f.x;
          xs[t][r + i + 1] = f.y;
          xs[t][r + i + 2] = f.z;
          xs[t][r + i + 3] = f.w;
        }
      }
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < GS; ++i) a += xs[t][g * GS + i];
        sx[t][g] = a;
      }
    }

    constexpr int U = 4; /* rows in flight per wave */
    for (int rr = 0; rr < nrows; rr += U) {
      typename F::Raw w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t row = r0 + (uint32_t)min(rr + u, nrows - 1);
        if (valid) w[u] = F::load(v, row, c);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (rr + u >= nrows) break; /* wave-uniform */
        float part[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) part[t] = 0.0f;
        if (valid) {
          float q[32], a[NG], b[NG];
          F::decode(w[u], c, q, a, b);
#pragma unroll
          for (int t = 0; t < MT; ++t) {
            float p = 0.0f;
#pragma unroll
            for (int g = 0; g < NG; ++g) {
              float acc = 0.0f;
#pragma unroll
              for (int i = 0; i < GS; ++i) acc = fmaf(q[g * GS + i], xs[t][g * GS + i], acc);
              p = fmaf(a[g], acc, p);
              p = fmaf(-b[g], sx[t][g], p);
            }
            part[t] = p;
          }
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const float tot = wave_sum(part[t]);
          if (lane == 0) red[wave][(rr + u) * MT + t] += tot;
        }
      }
    }
  }
  __syncthreads();
  for (int i = (int)threadIdx.x; i < nrows * MT; i += (int)blockDim.x) {
    const int row = i / MT, t = i % MT;
    if ((uint32_t)t >= ntok) continue;
    float acc = 0.0f;
    for (int w = 0; w < nwaves; ++w) acc += red[w][i];
    y[(size_t)t * v.n + r0 + (uint32_t)row] = acc;
  }
}

template <class F, int MT>
static hipError_t launch_gemv(const paik_qview_t &v, const float *x, float *y, uint32_t ntok,
                              hipStream_t s) {
  const uint32_t nchunks = v.k >> 5;
  const uint32_t nseg = (nchunks + 63u) >> 6;
  const uint32_t waves = nseg < (uint32_t)kMaxWaves ? nseg : (uint32_t)kMaxWaves;
  /* Row tile: enough workgroups to cover 256 CUs several times over, and
   * enough rows per wave to amortise its activation load. */
  uint32_t rows = v.n / 1024u;
  if (rows < 4u) rows = 4u;
  if (rows > (uint32_t)kMaxRowsPerWg) rows = (uint32_t)kMaxRowsPerWg;
  if (const char *e = getenv("PAI_GEMV_ROWS")) {
    const int r = atoi(e);
    if (r >= 1 && r <= kMaxRowsPerWg) rows = (uint32_t)r;
  }
  const dim3 grid((v.n + rows - 1u) / rows), block(64u * waves);
  k_gemv<F, MT><<<grid, block, 0, s>>>(v, x, y, ntok, rows);
  return hipGetLastError();
}

template <class F>
static hipError_t gemv_tokens(const paik_qview_t &v, uint32_t m, const float *x, float *y,
                              hipStream_t s) {
  /* groups of up to 4 tokens per launch; each launch re-streams W */
  for (uint32_t t0 = 0; t0 < m; t0 += 4u) {
    const uint32_t nt = m - t0 < 4u ? m - t0 : 4u;
    const float *xt = x + (size_t)t0 * v.k;
    float *yt = y + (size_t)t0 * v.n;
    hipError_t e;
    if (nt == 1u) e = launch_gemv<F, 1>(v, xt, yt, 1u, s);
    else if (nt == 2u) e = launch_gemv<F, 2>(v, xt, yt, 2u, s);
    else e = launch_gemv<F, 4>(v, xt, yt, nt, s);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

} // namespace paik

using namespace paik;

extern "C" int paik_gemv(const paik_qview_t *v, uint32_t m, const float *x, float *y,
                         void *stream) {
  hipStream_t s = (hipStream_t)stream;
  switch (v->type) {
  case 8u: return (int)gemv_tokens<Q8_0>(*v, m, x, y, s);
  case 2u: return (int)gemv_tokens<Q4_0>(*v, m, x, y, s);
  case 12u: return (int)gemv_tokens<Q4_K>(*v, m, x, y, s);
  case 14u: return (int)gemv_tokens<Q6_K>(*v, m, x, y, s);
  default: return (int)hipErrorInvalidValue;
  }
}
