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
//                  the chunk's K and V rows and q (after RoPE) for the kv
//                  head's G query heads staged in LDS with every load issued
//                  up front, then (max, sum, o[hd]) per (row, head).
//  k_attn_combine  one block per (sequence, row, query head): merges the chunks
//                  (log-sum-exp rescaling), writes the O-projection input
//                  rows (fp32) and appends the row's K (after RoPE)
//                  and V to the cache.  It runs after every chunk block has
//                  read the cache, so rows that wrap the circular window never
//                  overwrite a key another row still needs.
// Keys of the current rows are read from the fresh projections, older keys
// from the cache.
#include <cmath>

#include "attention.h"

namespace ms {

// q|k|v element (row, col) of the fused projection output.
__device__ inline float qkv_val(const AttnArgs &a, int row, int col) {
  return a.qkv[(size_t)row * a.ld + col];
}

// Element d of a head starting at column c0 of row `row`, rotated by RoPE at
// position pos (apply_rope_inplace, kernels.mojo:579-595; pairs (i, i+rot/2)
// over the first rot dims).  Branch-free: the pair element and the table
// entries are loaded for every d (clamped into range) and selected afterwards.
__device__ inline float rope_val(const AttnArgs &a, int row, int c0, int d, int pos) {
  const int half = a.rot >> 1;
  const bool rot = a.apply_rope && d < a.rot;
  const int dd = d < a.rot ? d : 0;
  const int i = dd < half ? dd : dd - half;
  const int pd = dd < half ? dd + half : dd - half;
  const float x = qkv_val(a, row, c0 + d);
  const float y = qkv_val(a, row, c0 + pd);
  const size_t ti = a.apply_rope ? (size_t)pos * half + i : 0;
  const float cv = a.apply_rope ? a.cos_t[ti] : 1.f;
  const float sv = a.apply_rope ? a.sin_t[ti] : 0.f;
  const float r = (dd < half) ? x * cv - y * sv : y * sv + x * cv;
  return rot ? r : x;
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

__device__ inline float block_reduce(float v, float *sh, bool is_max) {
  // 256-thread blocks (a blockDim read would load the dispatch packet)
  constexpr int nw = 4;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float u = __shfl_xor(v, o, 64);
    v = is_max ? fmaxf(v, u) : v + u;
  }
  __syncthreads();
  if (lane == 0) sh[w] = v;
  __syncthreads();
  float t = sh[0];
  for (int i = 1; i < nw; ++i) t = is_max ? fmaxf(t, sh[i]) : t + sh[i];
  return t;
}

template <int HD>
__global__ __launch_bounds__(256) void k_attn_chunks(AttnArgs a) {
  extern __shared__ float lds[];
  constexpr int CH = kAttnChunk;
  constexpr int F4 = CH * HD / 4 / 256;  // float4 of K (and of V) per thread
  constexpr int NV = HD / 64;            // float4 per thread per key (scores)
  constexpr int DPT = (HD + 255) / 256;  // P.V dims per thread
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

  float *sk = lds;                     // [CH][HD] keys of the chunk
  float *sv = sk + CH * HD;            // [CH][HD] values
  float *sq = sv + CH * HD;            // [TG][HD] rotated queries
  float *ss = sq + kAttnLds;           // [TG][CH] scores -> probabilities
  float *sm = ss + kAttnMaxTG * CH;    // [TG]
  float *sl = sm + kAttnMaxTG;         // [TG]
  const float *kcache = a.kc + (size_t)b * a.cache_seq_stride;
  const float *vcache = a.vc + (size_t)b * a.cache_seq_stride;

  // cache rows of the chunk -> LDS, all loads in flight at once
  float4 kr[F4], vr[F4];
#pragma unroll
  for (int j = 0; j < F4; ++j) {
    const int f = tid + 256 * j;            // float4 index in [CH][HD/4]
    const int k = f / (HD / 4), d4 = f % (HD / 4);
    const int kp = c0 + k;
    if (k < nk && kp < base) {
      const size_t off = (size_t)cache_slot(a, kp) * a.kv_dim + h * HD + 4 * d4;
      kr[j] = *reinterpret_cast<const float4 *>(kcache + off);
      vr[j] = *reinterpret_cast<const float4 *>(vcache + off);
    } else {
      kr[j] = float4{0.f, 0.f, 0.f, 0.f};
      vr[j] = float4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // rotated q for rows r0..r0+nr-1, query heads h*G..h*G+G-1
#pragma unroll 4
  for (int e = tid; e < TG * HD; e += 256) {
    const int tg = e / HD, d = e % HD;
    const int t = r0 + tg / G, g = tg % G;
    sq[e] = rope_val(a, b * a.T + t, (h * G + g) * HD, d, base + t);
  }
  // slots of this call's rows are filled below; every other slot (cache rows,
  // and zeros past the chunk end so that 0 * v stays finite) is written here
#pragma unroll
  for (int j = 0; j < F4; ++j) {
    const int f = tid + 256 * j;
    const int k = f / (HD / 4);
    if (!(k < nk && c0 + k >= base)) {
      reinterpret_cast<float4 *>(sk)[f] = kr[j];
      reinterpret_cast<float4 *>(sv)[f] = vr[j];
    }
  }
  // rows of this call that fall in the chunk: fresh K (after RoPE) and V
  const int kin0 = max(c0, base), kin1 = min(c0 + nk, base + a.T);
  for (int e = tid; e < (kin1 - kin0) * HD; e += 256) {
    const int kp = kin0 + e / HD, d = e % HD;
    const int row = b * a.T + (kp - base);
    sk[(kp - c0) * HD + d] = rope_val(a, row, a.q_dim + h * HD, d, kp);
    sv[(kp - c0) * HD + d] = qkv_val(a, row, a.q_dim + a.kv_dim + h * HD + d);
  }
  __syncthreads();

  // scores: thread (key kk, dim group dg of 16)
  const int kk = tid >> 4, dg = tid & 15;
  const int kp = c0 + kk;
  float acc[kAttnMaxTG];
#pragma unroll
  for (int i = 0; i < kAttnMaxTG; ++i) acc[i] = 0.f;
  if (kk < nk) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = dg * 4 + 64 * i;
      const float4 kv = *reinterpret_cast<const float4 *>(sk + kk * HD + d);
#pragma unroll
      for (int t = 0; t < kAttnMaxTG; ++t)
        if (t < TG) {
          const float4 qq = *reinterpret_cast<const float4 *>(sq + t * HD + d);
          acc[t] += qq.x * kv.x + qq.y * kv.y + qq.z * kv.z + qq.w * kv.w;
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
      const float sc = ss[tid * CH + k];
      const float p = (sc == -INFINITY) ? 0.f : expf(sc - m);
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
      for (int k = 0; k < CH; ++k) o += ss[t * CH + k] * sv[k * HD + d];
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

// One block per (sequence, row, query head): chunk weights exp(m_c - M) / L,
// then o[d] = sum_c w_c * o_c[d] with every chunk's load of a 16-chunk group
// in flight together.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_combine(AttnArgs a) {
  extern __shared__ float wsh[];  // [n_active] chunk weights
  __shared__ float sh[16];
  constexpr int DPT = (HD + 255) / 256;
  constexpr int CG = 16;  // chunk loads in flight per dim
  const int G = a.n_heads / a.n_kv;
  int bid = blockIdx.x;
  const int hq = bid % a.n_heads;
  bid /= a.n_heads;
  const int t = bid % a.T;
  const int b = bid / a.T;
  const int h = hq / G, g = hq % G;
  const int tid = threadIdx.x;
  const int base = a.pos[b];
  int kmin, kmax, dummy;
  key_range(a, base, &kmin, &dummy);
  key_range(a, base + a.T - 1, &dummy, &kmax);
  const int n_active = (kmax - kmin) / kAttnChunk + 1;
  const size_t cstride = (size_t)a.T * G * (HD + 2);
  const float *pg = a.part + (((size_t)b * a.n_kv + h) * a.n_chunks * a.T * G +
                              (size_t)t * G + g) * (HD + 2);
  float mloc[2], lloc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int cc = min(tid + 256 * j, n_active - 1);
    mloc[j] = pg[cc * cstride + HD];
    lloc[j] = pg[cc * cstride + HD + 1];
    if (tid + 256 * j >= n_active) {
      mloc[j] = -INFINITY;
      lloc[j] = 0.f;
    }
  }
  const float M = block_reduce(fmaxf(mloc[0], mloc[1]), sh, true);
  float wl[2], part = 0.f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    wl[j] = (mloc[j] == -INFINITY) ? 0.f : expf(mloc[j] - M);
    part += lloc[j] * wl[j];
  }
  const float L = block_reduce(part, sh, false);
  const float inv = 1.0f / L;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int cc = tid + 256 * j;
    if (cc < n_active) wsh[cc] = wl[j] * inv;
  }
  __syncthreads();
  const int row = b * a.T + t;
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int d = tid + 256 * j;
    if (d < HD) {
      float o = 0.f;
      for (int c0 = 0; c0 < n_active; c0 += CG) {
        float v[CG];
#pragma unroll
        for (int u = 0; u < CG; ++u) v[u] = pg[(size_t)min(c0 + u, n_active - 1) * cstride + d];
#pragma unroll
        for (int u = 0; u < CG; ++u)
          if (c0 + u < n_active) o += v[u] * wsh[c0 + u];
      }
      a.out[(size_t)row * a.q_dim + hq * HD + d] = o;
    }
  }
  if (a.write_cache && g == 0) {
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
  MS_CHECK_ARG(a.ld >= a.q_dim + 2 * a.kv_dim, "attention: q|k|v row stride too small");
  return MS_OK;
}

int launch_attention(const AttnArgs &a, hipStream_t st) {
  if (int rc = attn_check(a)) return rc;
  MS_CHECK_ARG(a.qkv && a.part && a.pos && a.out, "attention: missing buffers");
  const int G = a.n_heads / a.n_kv;
  const int TR = std::max(1, std::min(a.T, kAttnMaxTG / G));
  const int RG = (a.T + TR - 1) / TR;
  const long blocks = (long)a.B * a.n_kv * a.n_chunks * RG;
  const size_t shmem =
      (size_t)(2 * kAttnChunk * a.hd + kAttnLds + kAttnMaxTG * kAttnChunk + 2 * kAttnMaxTG) * 4;
  const long cblocks = (long)a.B * a.T * a.n_heads;
  const size_t cshmem = (size_t)a.n_chunks * 4;
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
