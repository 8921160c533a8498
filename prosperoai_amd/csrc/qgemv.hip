/*
 * Decode GEMV / small-batch GEMM over packed blocks (f32 arithmetic).
 *
 * y[t][r] = sum_k x[t][k] * W[r][k] for up to MT tokens per launch.
 *
 * Work split (memory-bound path, HBM streaming of the code planes):
 *   - a "segment" is 64 chunks = 2048 columns: lane l of a wave owns chunk
 *     64s+l of every row, so the wave's 64 x 16-byte code loads of one row
 *     are one contiguous 1 KiB read (2 KiB for Q8_0);
 *   - a workgroup owns U rows and has one wave per segment (at most 8; a
 *     longer K loops over segments). Each wave issues the loads of all U
 *     rows of its segment before it decodes any, so U x 16 bytes per lane
 *     are in flight; the lane's 32 activations per token stay in registers
 *     for all U rows;
 *   - codes become f32 in registers (v_cvt_f32_ubyte*) and meet x in f32
 *     FMAs; per-group scales and code offsets are applied once per group
 *     from per-lane sums of x;
 *   - the U*MT per-lane partials of a wave are transposed through LDS
 *     (each lane then sums U*MT partials of one output) and finished with
 *     DPP row operations; the waves' sums are added in wave order. The
 *     summation order is fixed by the launch shape, so results do not
 *     depend on scheduling.
 */
#include "qdev.h"

namespace paik {

constexpr int kMaxWaves = 8;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

/* Sum of v over aligned groups of L lanes (L a power of two <= 64); every
 * lane of a group receives the group's sum. */
template <int L>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (L >= 2) v += dpp<0xB1>(v);   /* quad_perm [1,0,3,2]: lane ^ 1 */
  if constexpr (L >= 4) v += dpp<0x4E>(v);   /* quad_perm [2,3,0,1]: lane ^ 2 */
  if constexpr (L >= 8) v += dpp<0x141>(v);  /* row_half_mirror: 8-lane halves */
  if constexpr (L >= 16) v += dpp<0x140>(v); /* row_mirror: 16-lane rows */
  if constexpr (L >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (L >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

template <class F, int U, int MT>
__global__ void __launch_bounds__(512) k_gemv(paik_qview_t v, const float *__restrict__ x,
                                              float *__restrict__ y, uint32_t ntok) {
  constexpr int NG = (int)F::kNG, GS = 32 / NG;
  constexpr int J = U * MT; /* outputs of the workgroup */
  constexpr int L = 64 / J; /* lanes that finish one output */
  static_assert(J >= 1 && J <= 64 && (J & (J - 1)) == 0, "U*MT must be a power of two <= 64");
  __shared__ float tr[kMaxWaves][J * 64];
  __shared__ float part[kMaxWaves][J];

  const int lane = (int)(threadIdx.x & 63u), wave = (int)(threadIdx.x >> 6);
  const int nwaves = (int)(blockDim.x >> 6);
  const uint32_t r0 = blockIdx.x * (uint32_t)U;
  const uint32_t nchunks = v.k >> 5;
  const uint32_t nseg = (nchunks + 63u) >> 6;

  float p[U][MT];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int t = 0; t < MT; ++t) p[u][t] = 0.0f;

  for (uint32_t s = (uint32_t)wave; s < nseg; s += (uint32_t)nwaves) {
    const uint32_t c = 64u * s + (uint32_t)lane;
    if (c < nchunks) {
      typename F::Raw w[U];
#pragma unroll
      for (int u = 0; u < U; ++u) w[u] = F::load(v, min(r0 + (uint32_t)u, v.n - 1u), c);

      float xs[MT][32], sx[MT][NG];
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const float4 *src = reinterpret_cast<const float4 *>(x + (size_t)t * v.k + 32u * c);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float4 f = make_float4(0.f, 0.f, 0.f, 0.f);
          if ((uint32_t)t < ntok) f = src[i];
          xs[t][4 * i] = f.x;
          xs[t][4 * i + 1] = f.y;
          xs[t][4 * i + 2] = f.z;
          xs[t][4 * i + 3] = f.w;
        }
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          float a = 0.0f;
#pragma unroll
          for (int i = 0; i < GS; ++i) a += xs[t][g * GS + i];
          sx[t][g] = a;
        }
        if constexpr (F::kHiScale != 1.0f) {
#pragma unroll
          for (int i = 16; i < 32; ++i) xs[t][i] *= F::kHiScale;
        }
      }

#pragma unroll
      for (int u = 0; u < U; ++u) {
        float q[32], a[NG], b[NG];
        F::decode(w[u], c, q, a, b);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          float acc = p[u][t];
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            float dot = 0.0f;
#pragma unroll
            for (int i = 0; i < GS; ++i) dot = fmaf(q[g * GS + i], xs[t][g * GS + i], dot);
            acc = fmaf(a[g], dot, acc);
            acc = fmaf(-b[g], sx[t][g], acc);
          }
          p[u][t] = acc;
        }
      }
    }
  }

  /* Transpose: output j = u*MT + t, entry (j, lane) at tr[wave][j*64 + lane];
   * lane l then sums entries (j = l / L, lanes (l % L)*J .. +J-1). */
  float *T = tr[wave];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int t = 0; t < MT; ++t) T[(u * MT + t) * 64 + lane] = p[u][t];
  __syncthreads();
  const int j = lane / L, sub = lane % L;
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < J; ++i) sum += T[j * 64 + sub * J + i];
  sum = group_sum<L>(sum);
  if (sub == 0) part[wave][j] = sum;
  __syncthreads();
  if ((int)threadIdx.x < J) {
    const int jj = (int)threadIdx.x, u = jj / MT, t = jj % MT;
    float acc = 0.0f;
    for (int w = 0; w < nwaves; ++w) acc += part[w][jj];
    if (r0 + (uint32_t)u < v.n && (uint32_t)t < ntok) y[(size_t)t * v.n + r0 + (uint32_t)u] = acc;
  }
}

/* Rows per workgroup: the largest U (4, 8 or 16, with U*MT <= 16) whose
 * grid still puts about 8 waves on each of the 256 CUs. */
template <int MT>
static int pick_rows(uint32_t n, uint32_t waves_per_wg) {
  int best = 4;
  for (int u = 8; u <= 16 / MT; u *= 2) {
    const uint64_t waves = (uint64_t)((n + (uint32_t)u - 1u) / (uint32_t)u) * waves_per_wg;
    if (waves >= 2048u) best = u;
  }
  if (const char *e = getenv("PAI_GEMV_ROWS")) {
    const int r = atoi(e);
    if ((r == 4 || r == 8 || r == 16) && r * MT <= 16) best = r;
  }
  return best;
}

template <class F, int U, int MT>
static hipError_t launch_u(const paik_qview_t &v, const float *x, float *y, uint32_t ntok,
                           uint32_t waves, hipStream_t s) {
  const dim3 grid((v.n + U - 1u) / U), block(64u * waves);
  k_gemv<F, U, MT><<<grid, block, 0, s>>>(v, x, y, ntok);
  return hipGetLastError();
}

template <class F, int MT>
static hipError_t launch_gemv(const paik_qview_t &v, const float *x, float *y, uint32_t ntok,
                              hipStream_t s) {
  const uint32_t nseg = ((v.k >> 5) + 63u) >> 6;
  const uint32_t waves = nseg < (uint32_t)kMaxWaves ? nseg : (uint32_t)kMaxWaves;
  const int u = pick_rows<MT>(v.n, waves);
  if constexpr (MT == 1) {
    if (u == 16) return launch_u<F, 16, 1>(v, x, y, ntok, waves, s);
    if (u == 8) return launch_u<F, 8, 1>(v, x, y, ntok, waves, s);
    return launch_u<F, 4, 1>(v, x, y, ntok, waves, s);
  } else if constexpr (MT == 2) {
    if (u == 8) return launch_u<F, 8, 2>(v, x, y, ntok, waves, s);
    return launch_u<F, 4, 2>(v, x, y, ntok, waves, s);
  } else {
    return launch_u<F, 4, MT>(v, x, y, ntok, waves, s);
  }
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
