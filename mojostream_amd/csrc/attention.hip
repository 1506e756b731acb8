// Causal GQA attention over the sliding (circular) and full/demo (linear) KV
// caches for decode and row-chunked prefill.
//
// Reference semantics (compute_sliding_attention gemma4_e4b.mojo:259-338,
// compute_full_attention :341-411, gqa_attention_decode main.mojo:445-519):
// row at position p attends keys [max(0,p-W+1), p] (circular window W) or
// [0, p] (linear; E4B full clamps to max_full_seq), score = dot(q,k)/sqrt(hd),
// softmax, sum p*v; query head hq reads kv head hq / (n_heads/n_kv).
//
// Two launches:
//  k_attn_chunks   one block per (sequence, kv head, 16-key chunk, row group):
//                  q (after RoPE) for the kv head's G query heads staged in LDS,
//                  the chunk's V rows prefetched into registers while the
//                  scores are computed, then (max, sum, o[hd]) per (row, head).
//  k_attn_combine  one block per (sequence, row, kv head): merges the chunks
//                  (log-sum-exp rescaling), writes the O-projection input
//                  (fp32 and fp16 hi/lo) and appends the row's K (after RoPE)
//                  and V to the cache.  It runs after every chunk block has
//                  read the cache, so rows that wrap the circular window never
//                  overwrite a key another row still needs.
// Keys of the current rows are read from the fresh projections, older keys
// from the cache.
#include <cmath>

#include "attention.h"

namespace ms {

__device__ inline float qkv_val(const AttnArgs &a, int row, int col) {
  const size_t idx = (size_t)row * a.ld + col;
  float x = a.qkv[idx];
  for (int s = 1; s < a.S; ++s) x = x + a.qkv[(size_t)s * a.split_stride + idx];
  return x;
}

// Element d of a head starting at column c0 of row `row`, rotated by RoPE at
// position pos (apply_rope_inplace, kernels.mojo:579-595; pairs (i, i+rot/2)
// over the first rot dims).
__device__ inline float rope_val(const AttnArgs &a, int row, int c0, int d, int pos) {
  const float x = qkv_val(a, row, c0 + d);
  if (!a.apply_rope || d >= a.rot) return x;
  const int half = a.rot >> 1;
  const int i = d < half ? d : d - half;
  const float cv = a.cos_t[(size_t)pos * half + i];
  const float sv = a.sin_t[(size_t)pos * half + i];
  if (d < half) {
    const float y = qkv_val(a, row, c0 + d + half);
    return x * cv - y * sv;
  }
  const float y = qkv_val(a, row, c0 + d - half);
  return y * sv + x * cv;
}

__device__ inline void key_range(const AttnArgs &a, int p, int *lo, int *hi) {
  if (a.cache_kind == MS_CACHE_CIRCULAR) {
    const int l = p - a.cache_len + 1;
    *lo = l > 0 ? l : 0;
    *hi = p;
  } else {
    *lo = 0;
    int h = p;
    if (a.clamp && h > a.cache_len - 1) h = a.cache_len - 1;
    *hi = h;
  }
}

__device__ inline int cache_slot(const AttnArgs &a, int t) {
  return a.cache_kind == MS_CACHE_CIRCULAR ? t % a.cache_len : t;
}

__device__ inline int row_group(const AttnArgs &a, int *RG) {
  const int G = a.n_heads / a.n_kv;
  const int TR = max(1, min(a.T, kAttnMaxTG / G));
  *RG = (a.T + TR - 1) / TR;
  return TR;
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_chunks(AttnArgs a) {
  extern __shared__ float lds[];
  constexpr int CH = kAttnChunk;
  constexpr int DPT = (HD + 255) / 256;  // P.V dims per thread
  constexpr int NV = HD / 64;            // float4 per thread per key (scores)
  const int G = a.n_heads / a.n_kv;
  int RG;
  const int TR = row_group(a, &RG);
  int bid = blockIdx.x;
  const int rg = bid % RG;
  bid /= RG;
  const int c = bid % a.n_chunks;
  bid /= a.n_chunks;
  const int h = bid % a.n_kv;
  const int b = bid / a.n_kv;
  const int tid = threadIdx.x;

  const int base = a.pos[b];
  int kmin, kmax, dummy;
  key_range(a, base, &kmin, &dummy);
  key_range(a, base + a.T - 1, &dummy, &kmax);
  const int c0 = kmin + c * CH;
  if (c0 > kmax) return;  // beyond the attended span at this position
  const int r0 = rg * TR;
  const int nr = min(TR, a.T - r0);
  const int TG = nr * G;
  const int nk = min(CH, kmax - c0 + 1);

  float *sq = lds;                     // [TG][HD] rotated queries
  float *ss = lds + kAttnLds;          // [TG][CH] scores -> probabilities
  float *sm = ss + kAttnMaxTG * CH;    // [TG]
  float *sl = sm + kAttnMaxTG;         // [TG]
  const float *kcache = a.kc + (size_t)b * a.cache_seq_stride;
  const float *vcache = a.vc + (size_t)b * a.cache_seq_stride;

  // V rows of the chunk -> registers (independent of the scores)
  float vreg[CH][DPT];
#pragma unroll
  for (int k = 0; k < CH; ++k)
#pragma unroll
    for (int j = 0; j < DPT; ++j) {
      const int d = tid + 256 * j;
      const int kp = c0 + k;
      float v = 0.f;
      if (k < nk && d < HD) {
        if (kp >= base)
          v = qkv_val(a, b * a.T + (kp - base), a.q_dim + a.kv_dim + h * HD + d);
        else
          v = vcache[(size_t)cache_slot(a, kp) * a.kv_dim + h * HD + d];
      }
      vreg[k][j] = v;
    }

  // rotated q for rows r0..r0+nr-1, query heads h*G..h*G+G-1
  for (int e = tid; e < TG * HD; e += 256) {
    const int tg = e / HD, d = e % HD;
    const int t = r0 + tg / G, g = tg % G;
    sq[e] = rope_val(a, b * a.T + t, (h * G + g) * HD, d, base + t);
  }
  __syncthreads();

  // scores: thread (key kk, dim group dg of 16)
  const int kk = tid >> 4, dg = tid & 15;
  const int kp = c0 + kk;
  float acc[kAttnMaxTG];
#pragma unroll
  for (int i = 0; i < kAttnMaxTG; ++i) acc[i] = 0.f;
  if (kk < nk) {
    float4 kv[NV];
    if (kp >= base) {
      const int row = b * a.T + (kp - base);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int d = dg * 4 + 64 * i;
        kv[i] = float4{rope_val(a, row, a.q_dim + h * HD, d, kp),
                       rope_val(a, row, a.q_dim + h * HD, d + 1, kp),
                       rope_val(a, row, a.q_dim + h * HD, d + 2, kp),
                       rope_val(a, row, a.q_dim + h * HD, d + 3, kp)};
      }
    } else {
      const float *krow = kcache + (size_t)cache_slot(a, kp) * a.kv_dim + h * HD;
#pragma unroll
      for (int i = 0; i < NV; ++i)
        kv[i] = *reinterpret_cast<const float4 *>(krow + dg * 4 + 64 * i);
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = dg * 4 + 64 * i;
#pragma unroll
      for (int t = 0; t < kAttnMaxTG; ++t)
        if (t < TG) {
          const float4 qq = *reinterpret_cast<const float4 *>(sq + t * HD + d);
          acc[t] += qq.x * kv[i].x + qq.y * kv[i].y + qq.z * kv[i].z + qq.w * kv[i].w;
        }
    }
  }
#pragma unroll
  for (int t = 0; t < kAttnMaxTG; ++t) {
    float v = acc[t];
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 4, 64);
    v += __shfl_xor(v, 8, 64);
    acc[t] = v;
  }
  if (dg == 0) {
    for (int t = 0; t < TG; ++t) {
      const int row_t = r0 + t / G;
      int lo, hi;
      key_range(a, base + row_t, &lo, &hi);
      const bool ok = kk < nk && kp >= lo && kp <= hi;
      ss[t * CH + kk] = ok ? acc[t] * a.scale : -INFINITY;
    }
  }
  __syncthreads();

  if (tid < TG) {
    float m = -INFINITY;
    for (int k = 0; k < CH; ++k) m = fmaxf(m, ss[tid * CH + k]);
    float l = 0.f;
    for (int k = 0; k < CH; ++k) {
      const float s = ss[tid * CH + k];
      const float p = (s == -INFINITY) ? 0.f : expf(s - m);
      ss[tid * CH + k] = p;
      l += p;
    }
    sm[tid] = m;
    sl[tid] = l;
  }
  __syncthreads();

#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int d = tid + 256 * j;
    if (d >= HD) continue;
    for (int t = 0; t < TG; ++t) {
      float o = 0.f;
#pragma unroll
      for (int k = 0; k < CH; ++k) o += ss[t * CH + k] * vreg[k][j];
      const int row_t = r0 + t / G, g = t % G;
      float *pp = a.part + ((((size_t)b * a.n_kv + h) * a.n_chunks + c) * a.T * G +
                            (size_t)row_t * G + g) * (HD + 2);
      pp[d] = o;
      if (d == 0) {
        pp[HD] = sm[t];
        pp[HD + 1] = sl[t];
      }
    }
  }
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_combine(AttnArgs a) {
  extern __shared__ float wsh[];  // [G][n_active] chunk weights
  const int G = a.n_heads / a.n_kv;
  int bid = blockIdx.x;
  const int h = bid % a.n_kv;
  bid /= a.n_kv;
  const int t = bid % a.T;
  const int b = bid / a.T;
  const int tid = threadIdx.x;
  const int base = a.pos[b];
  int kmin, kmax, dummy;
  key_range(a, base, &kmin, &dummy);
  key_range(a, base + a.T - 1, &dummy, &kmax);
  const int n_active = (kmax - kmin) / kAttnChunk + 1;
  const size_t cstride = (size_t)a.T * G * (HD + 2);
  const float *p0 = a.part + (((size_t)b * a.n_kv + h) * a.n_chunks * a.T * G +
                              (size_t)t * G) * (HD + 2);
  if (tid < G) {
    const float *pg = p0 + (size_t)tid * (HD + 2);
    float M = -INFINITY;
    for (int cc = 0; cc < n_active; ++cc) M = fmaxf(M, pg[cc * cstride + HD]);
    float L = 0.f;
    for (int cc = 0; cc < n_active; ++cc) {
      const float m = pg[cc * cstride + HD];
      const float w = (m == -INFINITY) ? 0.f : expf(m - M);
      wsh[tid * n_active + cc] = w;
      L += pg[cc * cstride + HD + 1] * w;
    }
    const float inv = 1.0f / L;
    for (int cc = 0; cc < n_active; ++cc) wsh[tid * n_active + cc] *= inv;
  }
  __syncthreads();
  const int row = b * a.T + t;
  for (int e = tid; e < G * HD; e += 256) {
    const int g = e / HD, d = e % HD;
    const float *pg = p0 + (size_t)g * (HD + 2) + d;
    float o = 0.f;
    for (int cc = 0; cc < n_active; ++cc) o += pg[cc * cstride] * wsh[g * n_active + cc];
    const size_t oi = (size_t)row * a.q_dim + (h * G + g) * HD + d;
    if (a.out) a.out[oi] = o;
    if (a.out_hi) {
      _Float16 hh, ll;
      split_hi_lo(o * a.out_prescale, &hh, &ll);
      a.out_hi[oi] = hh;
      a.out_lo[oi] = ll;
    }
  }
  if (a.write_cache) {
    // write_kv_sliding / write_kv_full (gemma4_e4b.mojo:211-249)
    const int p = base + t;
    if (!(a.cache_kind == MS_CACHE_LINEAR && p >= a.cache_len)) {
      float *kc = a.kc + (size_t)b * a.cache_seq_stride;
      float *vc = a.vc + (size_t)b * a.cache_seq_stride;
      for (int d = tid; d < HD; d += 256) {
        const size_t ci = (size_t)cache_slot(a, p) * a.kv_dim + h * HD + d;
        kc[ci] = rope_val(a, row, a.q_dim + h * HD, d, p);
        vc[ci] = qkv_val(a, row, a.q_dim + a.kv_dim + h * HD + d);
      }
    }
  }
}

int attn_check(const AttnArgs &a) {
  MS_CHECK_ARG(a.n_kv > 0 && a.n_heads % a.n_kv == 0, "attention: n_heads % n_kv != 0");
  const int G = a.n_heads / a.n_kv;
  MS_CHECK_ARG(G <= kAttnMaxTG, "attention: GQA group too large");
  const int TR = std::max(1, std::min(a.T, kAttnMaxTG / G));
  MS_CHECK_ARG(TR * G * a.hd <= kAttnLds, "attention: q staging exceeds LDS budget");
  MS_CHECK_ARG(a.hd == 128 || a.hd == 256 || a.hd == 512,
               "attention: head_dim must be 128, 256 or 512");
  MS_CHECK_ARG(a.rot % 2 == 0 && a.rot <= a.hd, "attention: bad rotary width");
  MS_CHECK_ARG(a.cache_len > 0, "attention: empty cache");
  MS_CHECK_ARG(a.n_chunks <= kAttnMaxChunks, "attention: too many key chunks");
  return MS_OK;
}

int launch_attention(const AttnArgs &a, hipStream_t st) {
  if (int rc = attn_check(a)) return rc;
  const int G = a.n_heads / a.n_kv;
  const int TR = std::max(1, std::min(a.T, kAttnMaxTG / G));
  const int RG = (a.T + TR - 1) / TR;
  const long blocks = (long)a.B * a.n_kv * a.n_chunks * RG;
  const size_t shmem = (size_t)(kAttnLds + kAttnMaxTG * kAttnChunk + 2 * kAttnMaxTG) * 4;
  const long cblocks = (long)a.B * a.T * a.n_kv;
  const size_t cshmem = (size_t)G * a.n_chunks * 4;
#define MS_ATTN(HDV)                                                                      \
  hipLaunchKernelGGL(k_attn_chunks<HDV>, dim3(blocks), dim3(256), shmem, st, a);       \
  hipLaunchKernelGGL(k_attn_combine<HDV>, dim3(cblocks), dim3(256), cshmem, st, a)
  switch (a.hd) {
    case 128: MS_ATTN(128); break;
    case 256: MS_ATTN(256); break;
    default: MS_ATTN(512); break;
  }
#undef MS_ATTN
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

}  // namespace ms
