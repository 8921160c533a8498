/*
 * The non-matmul kernels of one LLaMA decode step: the residual add fused
 * with RMSNorm, RoPE of q and k fused with the fp16 KV-cache append,
 * grouped-query attention of the new token over the cache (split over the
 * context, then combined), the token-embedding row and the greedy argmax.
 * The projections are the packed GEMV kernels (qgemv.hip, qgemv_mx.hip).
 *
 * Each kernel follows one of the reference's operators
 * (cpu/reference/ref_ops.c, models/sampler.c); the KV cache holds fp16
 * keys and values, so attention reads the cached values widened back to
 * f32. No FMA contraction in this unit: RMSNorm's two products, RoPE's
 * products and differences and the row dequantization round like the
 * reference's C (explicit fmaf only where the order is the build's own).
 */
#pragma clang fp contract(off)

#include "qdev.h"

namespace paik {
namespace dec {

constexpr int kNormThreads = 256;
constexpr int kNormVec = 16; /* float4 groups per thread: n <= 16384 */

/* Block-wide sum of a double in a fixed order; every thread gets it. */
__device__ double block_sum(double v, double *sh) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  double t = 0.0;
  for (int w = 0; w < nw; ++w) t += sh[w];
  return t;
}

/* x += delta (when delta is set), then xn = x * gamma * rms with
 * rms = 1 / sqrtf((float)(sum x^2 / n) + eps), the sum taken in double:
 * pai_ref_rmsnorm_gamma_f32 (cpu/reference/ref_ops.c:196-218) after the
 * residual ADD (adapters/llama/llama.c:746-751, :786-791). One workgroup;
 * thread j holds the float4 groups j, j + 256, ... of x, delta and gamma in
 * registers (all loads issued before the reduction). n % 4 == 0. */
__global__ void __launch_bounds__(kNormThreads) k_add_rmsnorm(float *__restrict__ x,
                                                              const float *__restrict__ delta,
                                                              const float *__restrict__ gamma,
                                                              float *__restrict__ xn, uint32_t n,
                                                              float eps) {
  __shared__ double sh[kNormThreads / 64];
  const uint32_t n4 = n >> 2;
  float4 v[kNormVec], g[kNormVec];
#pragma unroll
  for (int j = 0; j < kNormVec; ++j) {
    const uint32_t i = threadIdx.x + (uint32_t)j * kNormThreads;
    v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    g[j] = v[j];
    if (i < n4) {
      v[j] = reinterpret_cast<const float4 *>(x)[i];
      g[j] = reinterpret_cast<const float4 *>(gamma)[i];
    }
  }
  if (delta != nullptr) {
#pragma unroll
    for (int j = 0; j < kNormVec; ++j) {
      const uint32_t i = threadIdx.x + (uint32_t)j * kNormThreads;
      if (i < n4) {
        const float4 d = reinterpret_cast<const float4 *>(delta)[i];
        v[j] = make_float4(v[j].x + d.x, v[j].y + d.y, v[j].z + d.z, v[j].w + d.w);
        reinterpret_cast<float4 *>(x)[i] = v[j];
      }
    }
  }
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < kNormVec; ++j) {
    acc += (double)v[j].x * (double)v[j].x;
    acc += (double)v[j].y * (double)v[j].y;
    acc += (double)v[j].z * (double)v[j].z;
    acc += (double)v[j].w * (double)v[j].w;
  }
  const double tot = block_sum(acc, sh);
  const float rms = 1.0f / sqrtf((float)(tot / (double)n) + eps);
#pragma unroll
  for (int j = 0; j < kNormVec; ++j) {
    const uint32_t i = threadIdx.x + (uint32_t)j * kNormThreads;
    if (i < n4)
      reinterpret_cast<float4 *>(xn)[i] =
          make_float4(v[j].x * g[j].x * rms, v[j].y * g[j].y * rms, v[j].z * g[j].z * rms,
                      v[j].w * g[j].w * rms);
  }
}

/* The same for any n (one element per step), for rows whose length is not
 * a multiple of 4 or whose pointers are not 16-byte aligned. */
__global__ void __launch_bounds__(kNormThreads) k_add_rmsnorm_any(float *__restrict__ x,
                                                                  const float *__restrict__ delta,
                                                                  const float *__restrict__ gamma,
                                                                  float *__restrict__ xn,
                                                                  uint32_t n, float eps) {
  __shared__ double sh[kNormThreads / 64];
  double acc = 0.0;
  for (uint32_t i = threadIdx.x; i < n; i += kNormThreads) {
    float t = x[i];
    if (delta != nullptr) {
      t = t + delta[i];
      x[i] = t;
    }
    acc += (double)t * (double)t;
  }
  const double tot = block_sum(acc, sh);
  const float rms = 1.0f / sqrtf((float)(tot / (double)n) + eps);
  for (uint32_t i = threadIdx.x; i < n; i += kNormThreads) xn[i] = x[i] * gamma[i] * rms;
}

/* RoPE at position pos on the heads of q (hq heads) and k (hk heads) of
 * dimension hd, rotating the pairs (i, i + r2), i < r2, with the f32
 * tables cos_t/sin_t of that position (pai_ref_rope_f32,
 * cpu/reference/ref_ops.c:231-256). The rotated q goes to qo; the rotated
 * k and the v row are rounded to fp16 and stored at position pos of the
 * caches kc/vc ([hk][ctx][hd]). Workgroup h < hq: q head h; otherwise KV
 * head h - hq. One thread per element (hd <= 256). */
__global__ void __launch_bounds__(256) k_rope_append(const float *__restrict__ q,
                                                     const float *__restrict__ k,
                                                     const float *__restrict__ v,
                                                     float *__restrict__ qo,
                                                     _Float16 *__restrict__ kc,
                                                     _Float16 *__restrict__ vc,
                                                     const float *__restrict__ cos_t,
                                                     const float *__restrict__ sin_t,
                                                     uint32_t hq, uint32_t hd, uint32_t r2,
                                                     uint32_t ctx, uint32_t pos) {
  const uint32_t h = blockIdx.x, i = threadIdx.x;
  if (i >= hd) return;
  const bool isq = h < hq;
  const uint32_t kh = isq ? 0u : h - hq;
  const float *src = isq ? q + (size_t)h * hd : k + (size_t)kh * hd;
  float o;
  if (i < r2) {
    o = src[i] * cos_t[i] - src[i + r2] * sin_t[i];
  } else if (i < 2u * r2) {
    o = src[i - r2] * sin_t[i - r2] + src[i] * cos_t[i - r2];
  } else {
    o = src[i];
  }
  if (isq) {
    qo[(size_t)h * hd + i] = o;
  } else {
    const size_t at = ((size_t)kh * ctx + pos) * hd + i;
    kc[at] = (_Float16)o;
    vc[at] = (_Float16)v[(size_t)kh * hd + i];
  }
}

/* Attention of one token over cache positions [0, len):
 * pai_ref_attention_f32 (cpu/reference/ref_ops.c:287-340) for the last
 * position. Head h reads KV head h / G with G = hq / hk (the reference's
 * (h * hk) / hq), scores are (q . k) / sqrtf(hd), softmax subtracts the
 * maximum, and the output is the probability-weighted sum of v.
 *
 * With knew set, the kernel first does the step's RoPE and cache append
 * (k_rope_append's arithmetic): q is rotated on the fly, and the chunk
 * holding position len - 1 rotates knew, rounds it and vnew to fp16,
 * stores them at that position and uses its own copies of them.
 *
 * Split over the context: workgroup (kvh, c) covers positions
 * [64c, 64c + 64) for the G heads of KV head kvh, so each K and V row is
 * read once for all G heads. A wave takes 16 positions; HD/8 lanes share a
 * row (16 bytes of fp16 each: one coalesced 256-byte row read for HD=128).
 * Each wave keeps (max, sum of e^(s-max), sum of e^(s-max) v) per head;
 * the four waves are merged in LDS and the chunk's triple goes to
 * part[(kvh*nch + c)*G + g] = {m, l, o[HD]}. k_attn_merge, the next
 * launch, combines the chunks of each head in chunk order:
 * M = max m_c, o = (sum o_c e^(m_c - M)) / (sum l_c e^(m_c - M)).
 * (A single launch whose last chunk merges needs a device-scope release and
 * acquire per workgroup; across the chip's separate L2 caches that cost
 * about 30 us per call at 264 workgroups, against a few for a launch.) */
constexpr uint32_t kChunk = 64;
constexpr uint32_t kMaxG = 8;
constexpr uint32_t kMaxChunks = 512; /* len <= 32768 */

/* Reductions over aligned groups of L lanes (L <= 16) on DPP: quad swaps,
 * then the 8-lane half-row and 16-lane row mirrors (sum and max are
 * symmetric, so mirrored partners combine like butterflies). */
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int L>
__device__ __forceinline__ float row_sum(float v) {
  static_assert(L <= 16, "DPP covers one 16-lane row");
  if constexpr (L >= 2) v += dpp_f<0xB1>(v);  /* quad: lane ^ 1 */
  if constexpr (L >= 4) v += dpp_f<0x4E>(v);  /* quad: lane ^ 2 */
  if constexpr (L >= 8) v += dpp_f<0x141>(v); /* row_half_mirror */
  if constexpr (L >= 16) v += dpp_f<0x140>(v); /* row_mirror */
  return v;
}
/* Sum over groups of L lanes: DPP within a row, shuffles across rows. */
template <int L>
__device__ __forceinline__ float lane_group_sum(float v) {
  v = row_sum<(L < 16 ? L : 16)>(v);
  if constexpr (L >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (L >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

__device__ __forceinline__ float f16lo(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
}
__device__ __forceinline__ float f16hi(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

/* RoPE's pairing for element i of a head (pai_ref_rope_f32's
 * arithmetic): i < r2 pairs with i + r2 and uses table entry i; r2 <= i <
 * 2 r2 pairs with i - r2 and uses entry i - r2; the rest are not rotated
 * (partner i, entry 0, unused). */
__device__ __forceinline__ void rope_pair(uint32_t i, uint32_t r2, uint32_t &partner,
                                          uint32_t &entry) {
  partner = i < r2 ? i + r2 : (i < 2u * r2 ? i - r2 : i);
  entry = i < r2 ? i : (i < 2u * r2 ? i - r2 : 0u);
}
/* the rotated value from x[i], x[partner], cos and sin of the entry */
__device__ __forceinline__ float rope_val(uint32_t i, uint32_t r2, float xi, float xp, float c,
                                          float s) {
  if (i < r2) return xi * c - xp * s;
  if (i < 2u * r2) return xp * s + xi * c;
  return xi;
}

template <int HD, bool ROPE, int GM>
__global__ void __launch_bounds__(256) k_attn(const float *__restrict__ q,
                                              const float *__restrict__ knew,
                                              const float *__restrict__ vnew,
                                              const float *__restrict__ cos_t,
                                              const float *__restrict__ sin_t, uint32_t r2,
                                              _Float16 *__restrict__ kc, _Float16 *__restrict__ vc,
                                              float *__restrict__ part, uint32_t G,
                                              uint32_t ctx, uint32_t len, uint32_t nch) {
  constexpr int LP = HD / 8;   /* lanes per row */
  constexpr int PPI = 64 / LP; /* rows per wave instruction */
  constexpr int IT = 16 / PPI; /* iterations over a wave's 16 rows */
  constexpr int QPT = (GM * HD + 255) / 256; /* q elements per thread, at most */
  static_assert(GM >= 1 && GM <= (int)kMaxG, "head group");
  __shared__ float qs[GM][HD];
  __shared__ float nk[HD], nv[HD];
  __shared__ float sm[4][GM], sl[4][GM];
  __shared__ float so[4][GM][HD];
  const uint32_t kvh = blockIdx.x / nch, c = blockIdx.x % nch;
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t slot = lane / LP, t = lane % LP;
  const float scale = 1.0f / sqrtf((float)HD);
  _Float16 *kb = kc + (size_t)kvh * ctx * HD;
  _Float16 *vb = vc + (size_t)kvh * ctx * HD;
  const uint32_t base = c * kChunk + wave * 16u;
  const uint32_t pos = len - 1u;

  /* The small loads go first, unconditionally (indices clamped into
   * range), so they return ahead of the K/V stream and nothing waits on a
   * branch: q of the G heads of this KV head (consecutive in q), with
   * RoPE's partner element and table entries, and the step's new k, v. */
  const float *qg = q + (size_t)kvh * G * HD;
  const uint32_t nq = G * (uint32_t)HD;
  float qa[QPT], qb[QPT], qc[QPT], qn[QPT];
#pragma unroll
  for (int j = 0; j < QPT; ++j) {
    const uint32_t e = min(threadIdx.x + 256u * (uint32_t)j, nq - 1u);
    const uint32_t i = e % (uint32_t)HD;
    qa[j] = qg[e];
    if constexpr (ROPE) {
      uint32_t pt, en;
      rope_pair(i, r2, pt, en);
      qb[j] = qg[e - i + pt];
      qc[j] = cos_t[en];
      qn[j] = sin_t[en];
    }
  }
  const uint32_t ni = min(threadIdx.x, (uint32_t)HD - 1u);
  float ka = 0.f, kp = 0.f, kcs = 0.f, ksn = 0.f, va = 0.f;
  if constexpr (ROPE) {
    uint32_t pt, en;
    rope_pair(ni, r2, pt, en);
    ka = knew[(size_t)kvh * HD + ni];
    kp = knew[(size_t)kvh * HD + pt];
    va = vnew[(size_t)kvh * HD + ni];
    kcs = cos_t[en];
    ksn = sin_t[en];
  }

  /* this lane's rows: 8 K and 8 V values each */
  uint4 kw[IT], vw[IT];
  bool ok[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const uint32_t p = base + (uint32_t)(it * PPI) + slot;
    ok[it] = p < len;
    const uint32_t pc = ok[it] ? p : 0u; /* an in-bounds row for idle lanes */
    kw[it] = *reinterpret_cast<const uint4 *>(kb + (size_t)pc * HD + 8u * t);
    vw[it] = *reinterpret_cast<const uint4 *>(vb + (size_t)pc * HD + 8u * t);
  }
  /* q of the G heads (rotated for the append form) into LDS; threads past
   * the end repeat the last element with its own value (no branch, so the
   * loads above stay ahead of the K/V stream) */
#pragma unroll
  for (int j = 0; j < QPT; ++j) {
    const uint32_t e = min(threadIdx.x + 256u * (uint32_t)j, nq - 1u);
    const uint32_t i = e % (uint32_t)HD;
    (&qs[0][0])[e] = ROPE ? rope_val(i, r2, qa[j], qb[j], qc[j], qn[j]) : qa[j];
  }
  /* The new k (rotated) and v in fp16: every workgroup forms them into
   * LDS (threads past HD repeat element HD - 1 with the same value), so
   * their loads stay ahead of the K/V stream; the chunk holding position
   * pos also stores them in the cache and uses these copies. */
  if constexpr (ROPE) {
    const _Float16 kh = (_Float16)rope_val(ni, r2, ka, kp, kcs, ksn);
    const _Float16 vh = (_Float16)va;
    nk[ni] = (float)kh;
    nv[ni] = (float)vh;
    if (pos / kChunk == c && threadIdx.x < (uint32_t)HD) {
      kb[(size_t)pos * HD + ni] = kh;
      vb[(size_t)pos * HD + ni] = vh;
    }
  }
  __syncthreads();

  float kr[IT][8], vr[IT][8];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const uint32_t ka[4] = {kw[it].x, kw[it].y, kw[it].z, kw[it].w};
    const uint32_t va[4] = {vw[it].x, vw[it].y, vw[it].z, vw[it].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      kr[it][2 * e] = f16lo(ka[e]);
      kr[it][2 * e + 1] = f16hi(ka[e]);
      vr[it][2 * e] = f16lo(va[e]);
      vr[it][2 * e + 1] = f16hi(va[e]);
    }
    if (ROPE && base + (uint32_t)(it * PPI) + slot == pos) { /* this step's row */
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        kr[it][e] = nk[8u * t + e];
        vr[it][e] = nv[8u * t + e];
      }
    }
  }

  /* Scores, softmax terms and weighted v of the GM head slots (heads g <
   * G are real): unrolled over the heads, so their reduction chains
   * overlap. A row's dot product is summed over its LP lanes on DPP; the
   * wave's PPI rows combine across rows with shuffles. */
  float s[GM][IT];
#pragma unroll
  for (int g = 0; g < GM; ++g) {
    float qv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) qv[e] = qs[g][8u * t + e];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      float d = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) d = fmaf(qv[e], kr[it][e], d);
      d = lane_group_sum<LP>(d);
      s[g][it] = ok[it] ? d * scale : -INFINITY;
    }
  }
  float m[GM];
#pragma unroll
  for (int g = 0; g < GM; ++g) {
    m[g] = -INFINITY;
#pragma unroll
    for (int it = 0; it < IT; ++it) m[g] = fmaxf(m[g], s[g][it]);
  }
#pragma unroll
  for (int sh = 32; sh >= LP; sh >>= 1)
#pragma unroll
    for (int g = 0; g < GM; ++g) m[g] = fmaxf(m[g], __shfl_xor(m[g], sh, 64));
  float l[GM], acc[GM][8];
#pragma unroll
  for (int g = 0; g < GM; ++g) {
    l[g] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[g][j] = 0.0f;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const float e = ok[it] ? expf(s[g][it] - m[g]) : 0.0f;
      l[g] += e;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] = fmaf(e, vr[it][j], acc[g][j]);
    }
  }
#pragma unroll
  for (int sh = 32; sh >= LP; sh >>= 1)
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      l[g] += __shfl_xor(l[g], sh, 64);
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[g][j] += __shfl_xor(acc[g][j], sh, 64);
    }
  if (slot == 0u) {
#pragma unroll
    for (int g = 0; g < GM; ++g) {
      if ((uint32_t)g < G) {
#pragma unroll
        for (int j = 0; j < 8; ++j) so[wave][g][8u * t + j] = acc[g][j];
        if (t == 0u) {
          sm[wave][g] = m[g];
          sl[wave][g] = l[g];
        }
      }
    }
  }
  __syncthreads();
  /* merge the four waves (a wave with no valid row has m = -inf, l = 0) */
  const uint32_t stride = HD + 2u;
  float *out = part + (size_t)blockIdx.x * G * stride;
  for (uint32_t e = threadIdx.x; e < G * (uint32_t)HD; e += blockDim.x) {
    const uint32_t g = e / HD, d = e % HD;
    float M = -INFINITY;
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sm[w][g]);
    float L = 0.0f, O = 0.0f;
    for (int w = 0; w < 4; ++w) {
      const float f = sm[w][g] == -INFINITY ? 0.0f : expf(sm[w][g] - M);
      L = fmaf(sl[w][g], f, L);
      O = fmaf(so[w][g][d], f, O);
    }
    out[g * stride + 2u + d] = O;
    if (d == 0u) {
      out[g * stride] = M;
      out[g * stride + 1u] = L;
    }
  }

}

/* The chunks' triples of one head combined in chunk order (see k_attn):
 * workgroup h is query head h, thread d output element d. */
template <int HD>
__global__ void __launch_bounds__(HD) k_attn_merge(const float *__restrict__ part,
                                                   float *__restrict__ o, uint32_t G,
                                                   uint32_t nch) {
  constexpr uint32_t stride = HD + 2u;
  constexpr int PER = kMaxChunks / 64; /* chunks per lane of the first wave */
  __shared__ float fsc[kMaxChunks];
  __shared__ float sL;
  const uint32_t h = blockIdx.x, kvh = h / G, g = h % G;
  const size_t cstep = (size_t)G * stride; /* floats from one chunk's triple to the next */
  const float *pk = part + ((size_t)kvh * nch * G + g) * stride;
  /* The first 64 chunks' partial sums for this thread's element are
   * requested before the (m, l) loads, so both return in one round trip. */
  const uint32_t d = threadIdx.x;
  const float *pc = pk + 2u + d;
  constexpr int kPre = 64;
  float ov[kPre];
#pragma unroll
  for (int j = 0; j < kPre; ++j) ov[j] = pc[(size_t)min((uint32_t)j, nch - 1u) * cstep];
  if (threadIdx.x < 64u) {
    /* (m, l) of every chunk: clamped, unconditional loads, masked after */
    const uint32_t lane = threadIdx.x;
    float mv[PER], lv[PER];
    float M = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const uint32_t cc = lane + 64u * (uint32_t)j;
      const size_t at = (size_t)min(cc, nch - 1u) * cstep;
      mv[j] = pk[at];
      lv[j] = pk[at + 1u];
    }
#pragma unroll
    for (int j = 0; j < PER; ++j)
      if (lane + 64u * (uint32_t)j < nch) M = fmaxf(M, mv[j]);
    for (int sh = 32; sh > 0; sh >>= 1) M = fmaxf(M, __shfl_xor(M, sh, 64));
    float L = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const uint32_t cc = lane + 64u * (uint32_t)j;
      if (cc < nch) {
        const float f = expf(mv[j] - M);
        fsc[cc] = f;
        L = fmaf(lv[j], f, L);
      }
    }
    for (int sh = 32; sh > 0; sh >>= 1) L += __shfl_xor(L, sh, 64);
    if (lane == 0u) sL = L;
  }
  __syncthreads();
  /* o: the chunks' partial sums in chunk order */
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < kPre; ++j)
    if ((uint32_t)j < nch) acc = fmaf(ov[j], fsc[j], acc);
  for (uint32_t c0 = kPre; c0 < nch; c0 += 32u) {
    float ow[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) ow[j] = pc[(size_t)min(c0 + (uint32_t)j, nch - 1u) * cstep];
#pragma unroll
    for (int j = 0; j < 32; ++j)
      if (c0 + (uint32_t)j < nch) acc = fmaf(ow[j], fsc[c0 + (uint32_t)j], acc);
  }
  o[(size_t)h * HD + d] = acc / sL;
}

/* Greedy token: the first index of the largest logit, as the reference's
 * scan `if (p[i] > best)` from best = p[0] (models/sampler.c:146-155):
 * NaNs after index 0 never win, and a NaN at index 0 wins outright. Two
 * passes: per-workgroup (value, index) pairs, then one workgroup over
 * them. */
constexpr uint32_t kArgParts = 256;

__device__ void better(float &v, uint32_t &i, float v2, uint32_t i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

__device__ void block_best(float &v, uint32_t &i, float *shv, uint32_t *shi) {
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(v, o, 64);
    const uint32_t i2 = (uint32_t)__shfl_xor((int)i, o, 64);
    better(v, i, v2, i2);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    shv[wave] = v;
    shi[wave] = i;
  }
  __syncthreads();
  if (threadIdx.x == 0)
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) better(v, i, shv[w], shi[w]);
}

__global__ void __launch_bounds__(256) k_argmax_part(const float *__restrict__ x, uint32_t n,
                                                     float *__restrict__ pv,
                                                     uint32_t *__restrict__ pi) {
  __shared__ float shv[4];
  __shared__ uint32_t shi[4];
  float v = -INFINITY;
  uint32_t i = 0xFFFFFFFFu;
  for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < n; j += gridDim.x * blockDim.x)
    better(v, i, x[j], j);
  block_best(v, i, shv, shi);
  if (threadIdx.x == 0) {
    pv[blockIdx.x] = v;
    pi[blockIdx.x] = i;
  }
}

__global__ void __launch_bounds__(256) k_argmax_final(const float *__restrict__ x,
                                                      const float *__restrict__ pv,
                                                      const uint32_t *__restrict__ pi,
                                                      uint32_t *__restrict__ out) {
  __shared__ float shv[4];
  __shared__ uint32_t shi[4];
  float v = -INFINITY;
  uint32_t i = 0xFFFFFFFFu;
  for (uint32_t j = threadIdx.x; j < kArgParts; j += blockDim.x) better(v, i, pv[j], pi[j]);
  block_best(v, i, shv, shi);
  if (threadIdx.x == 0) {
    const float x0 = x[0];
    /* x0 is NaN, or every logit is NaN: the reference keeps index 0 */
    out[0] = (x0 != x0 || i == 0xFFFFFFFFu) ? 0u : i;
  }
}

/* Row `*row` of a packed matrix, dequantized exactly: the token-embedding
 * lookup (the reference multiplies a one-hot row by the dequantized
 * token_embd, adapters/llama/llama.c:511-520, which selects that row
 * exactly). One thread per chunk; a row index past the end reads the last
 * row. */
template <class F>
__global__ void __launch_bounds__(256) k_dequant_row(paik_qview_t v,
                                                     const uint32_t *__restrict__ row_p,
                                                     float *__restrict__ out) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= (v.k >> 5)) return;
  const uint32_t row = min(row_p[0], v.n - 1u);
  float o[32];
  F::dequant(F::load(v, row, c), c, o);
  float4 *dst = reinterpret_cast<float4 *>(out + 32u * c);
#pragma unroll
  for (int i = 0; i < 8; ++i) dst[i] = make_float4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
}

} // namespace dec
} // namespace paik

using namespace paik;
using namespace paik::dec;

extern "C" uint32_t paik_norm_max(void) { return (uint32_t)(4 * kNormVec * kNormThreads); }

extern "C" int paik_add_rmsnorm(float *x, const float *delta, const float *gamma, float *xn,
                                uint32_t n, float eps, void *stream) {
  if (n == 0u || n > paik_norm_max()) return (int)hipErrorInvalidValue;
  const uintptr_t al = (uintptr_t)x | (uintptr_t)delta | (uintptr_t)gamma | (uintptr_t)xn;
  hipStream_t s = (hipStream_t)stream;
  if ((n & 3u) == 0u && (al & 15u) == 0u)
    k_add_rmsnorm<<<1, kNormThreads, 0, s>>>(x, delta, gamma, xn, n, eps);
  else
    k_add_rmsnorm_any<<<1, kNormThreads, 0, s>>>(x, delta, gamma, xn, n, eps);
  return (int)hipGetLastError();
}

extern "C" int paik_rope_append(const float *q, const float *k, const float *v, float *qo,
                                void *kc, void *vc, const float *cos_t, const float *sin_t,
                                uint32_t hq, uint32_t hk, uint32_t hd, uint32_t r2, uint32_t ctx,
                                uint32_t pos, void *stream) {
  if (hd == 0u || hd > 256u || r2 == 0u || 2u * r2 > hd || pos >= ctx)
    return (int)hipErrorInvalidValue;
  k_rope_append<<<hq + hk, 256, 0, (hipStream_t)stream>>>(
      q, k, v, qo, static_cast<_Float16 *>(kc), static_cast<_Float16 *>(vc), cos_t, sin_t, hq, hd,
      r2, ctx, pos);
  return (int)hipGetLastError();
}

extern "C" uint32_t paik_attn_chunks(uint32_t len) { return (len + kChunk - 1u) / kChunk; }
extern "C" uint32_t paik_attn_max_len(void) { return kMaxChunks * kChunk; }

extern "C" int paik_attn_decode(const float *q, const float *knew, const float *vnew,
                                const float *cos_t, const float *sin_t, uint32_t r2, void *kc,
                                void *vc, float *part, float *o, uint32_t hq, uint32_t hk,
                                uint32_t hd, uint32_t ctx, uint32_t len, void *stream) {
  if (hk == 0u || hq % hk != 0u || hq / hk > kMaxG || len == 0u || len > ctx ||
      len > paik_attn_max_len())
    return (int)hipErrorInvalidValue;
  if (knew != nullptr && (r2 == 0u || 2u * r2 > hd)) return (int)hipErrorInvalidValue;
  const uint32_t G = hq / hk, nch = paik_attn_chunks(len);
  hipStream_t s = (hipStream_t)stream;
  _Float16 *k16 = static_cast<_Float16 *>(kc), *v16 = static_cast<_Float16 *>(vc);
  const bool rope = knew != nullptr;
  /* head-group width: G itself for 1, 2, 4 or 8, else the next of those */
  const uint32_t gm = G <= 1u ? 1u : G <= 2u ? 2u : G <= 4u ? 4u : 8u;
#define PAIK_ATTN_G(HD, GMV)                                                                   \
  do {                                                                                         \
    if (rope)                                                                                  \
      k_attn<HD, true, GMV><<<hk * nch, 256, 0, s>>>(q, knew, vnew, cos_t, sin_t, r2, k16, v16, \
                                                     part, G, ctx, len, nch);                  \
    else                                                                                       \
      k_attn<HD, false, GMV><<<hk * nch, 256, 0, s>>>(q, knew, vnew, cos_t, sin_t, r2, k16,     \
                                                      v16, part, G, ctx, len, nch);            \
  } while (0)
#define PAIK_ATTN(HD)                                                                          \
  do {                                                                                         \
    if (gm == 1u) PAIK_ATTN_G(HD, 1);                                                          \
    else if (gm == 2u) PAIK_ATTN_G(HD, 2);                                                     \
    else if (gm == 4u) PAIK_ATTN_G(HD, 4);                                                     \
    else PAIK_ATTN_G(HD, 8);                                                                   \
    k_attn_merge<HD><<<hq, HD, 0, s>>>(part, o, G, nch);                                       \
  } while (0)
  switch (hd) {
  case 64: PAIK_ATTN(64); break;
  case 128: PAIK_ATTN(128); break;
  case 256: PAIK_ATTN(256); break;
  default: return (int)hipErrorInvalidValue;
  }
#undef PAIK_ATTN
#undef PAIK_ATTN_G
  return (int)hipGetLastError();
}

extern "C" uint32_t paik_argmax_parts(void) { return kArgParts; }

extern "C" int paik_argmax(const float *x, uint32_t n, float *pv, uint32_t *pi, uint32_t *out,
                           void *stream) {
  if (n == 0u) return (int)hipErrorInvalidValue;
  hipStream_t s = (hipStream_t)stream;
  k_argmax_part<<<kArgParts, 256, 0, s>>>(x, n, pv, pi);
  k_argmax_final<<<1, 256, 0, s>>>(x, pv, pi, out);
  return (int)hipGetLastError();
}

extern "C" int paik_dequant_row(const paik_qview_t *v, const uint32_t *row, float *out,
                                void *stream) {
  const uint32_t nc = v->k >> 5;
  const dim3 grid((nc + 255u) / 256u), block(256);
  hipStream_t s = (hipStream_t)stream;
  switch (v->type) {
  case 8u: k_dequant_row<Q8_0><<<grid, block, 0, s>>>(*v, row, out); break;
  case 2u: k_dequant_row<Q4_0><<<grid, block, 0, s>>>(*v, row, out); break;
  case 12u: k_dequant_row<Q4_K><<<grid, block, 0, s>>>(*v, row, out); break;
  case 14u: k_dequant_row<Q6_K><<<grid, block, 0, s>>>(*v, row, out); break;
  default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}
