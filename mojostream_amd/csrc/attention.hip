// Causal GQA attention over the sliding (circular) and full/demo (linear) KV
// caches for decode and row-chunked prefill.
//
// Reference semantics (compute_sliding_attention gemma4_e4b.mojo:259-338,
// compute_full_attention :341-411, gqa_attention_decode main.mojo:445-519):
// row at position p attends keys [max(0,p-W+1), p] (circular window W) or
// [0, p] (linear; E4B full clamps to max_full_seq), score = dot(q,k)/sqrt(hd),
// softmax, sum p*v; query head hq reads kv head hq / (n_heads/n_kv).
//
// Work split: one block per (sequence, kv head, 32-key chunk, row group).  q
// (after RoPE) for the kv head's G query heads is staged in LDS; each block
// writes a partial (max, sum, o[hd]) per (row, head).  The last block of a
// (sequence, kv head) merges the chunks (the usual log-sum-exp rescaling) and
// then appends the rows' K (after RoPE) and V to the cache, so no block reads
// a slot that is being overwritten even when T rows wrap the circular cache.
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

__global__ __launch_bounds__(256) void k_attention(AttnArgs a) {
  extern __shared__ float lds[];
  const int G = a.n_heads / a.n_kv;
  const int TR = max(1, min(a.T, kAttnMaxTG / G));
  const int RG = (a.T + TR - 1) / TR;
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
  const int r0 = rg * TR;
  const int nr = min(TR, a.T - r0);
  const int TG = nr * G;
  const int c0 = kmin + c * kAttnChunk;
  const int hd = a.hd;
  const int CH = kAttnChunk;

  float *sq = lds;                     // [TG][hd] rotated queries
  float *ss = lds + kAttnLds;          // [TG][CH] scores -> probabilities
  float *sm = ss + kAttnMaxTG * CH;    // [TG] chunk max
  float *sl = sm + kAttnMaxTG;         // [TG] chunk sum

  float *kcache = a.kc + (size_t)b * a.cache_seq_stride;
  float *vcache = a.vc + (size_t)b * a.cache_seq_stride;

  if (c0 <= kmax) {
    // ---- stage rotated q for rows r0..r0+nr-1, heads h*G..h*G+G-1 ----
    for (int e = tid; e < TG * hd; e += blockDim.x) {
      const int tg = e / hd, d = e % hd;
      const int t = r0 + tg / G, g = tg % G;
      const int row = b * a.T + t;
      sq[e] = rope_val(a, row, (h * G + g) * hd, d, base + t);
    }
    __syncthreads();

    // ---- scores: thread (key kk, dim group dg) ----
    const int kk = tid >> 3, dg = tid & 7;
    const int kp = c0 + kk;
    float acc[kAttnMaxTG];
#pragma unroll
    for (int i = 0; i < kAttnMaxTG; ++i) acc[i] = 0.f;
    if (kp <= kmax) {
      if (kp >= base) {
        const int row = b * a.T + (kp - base);
        for (int d = dg; d < hd; d += 8) {
          const float kv = rope_val(a, row, a.q_dim + h * hd, d, kp);
#pragma unroll
          for (int i = 0; i < kAttnMaxTG; ++i)
            if (i < TG) acc[i] += sq[i * hd + d] * kv;
        }
      } else {
        const float *krow = kcache + (size_t)cache_slot(a, kp) * a.kv_dim + h * hd;
        for (int d = dg * 4; d < hd; d += 32) {
          const float4 kv = *reinterpret_cast<const float4 *>(krow + d);
#pragma unroll
          for (int i = 0; i < kAttnMaxTG; ++i)
            if (i < TG) {
              const float *qq = sq + i * hd + d;
              acc[i] += qq[0] * kv.x + qq[1] * kv.y + qq[2] * kv.z + qq[3] * kv.w;
            }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kAttnMaxTG; ++i) {
      float v = acc[i];
      v += __shfl_xor(v, 1, 64);
      v += __shfl_xor(v, 2, 64);
      v += __shfl_xor(v, 4, 64);
      acc[i] = v;
    }
    if (dg == 0) {
      for (int i = 0; i < TG; ++i) {
        const int t = r0 + i / G;
        int lo, hi;
        key_range(a, base + t, &lo, &hi);
        const bool ok = kp <= kmax && kp >= lo && kp <= hi;
        ss[i * CH + kk] = ok ? acc[i] * a.scale : -INFINITY;
      }
    }
    __syncthreads();

    // ---- chunk softmax statistics ----
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

    // ---- o = sum_k p_k v_k ----
    const int nk = min(CH, kmax - c0 + 1);
    for (int d = tid; d < hd; d += blockDim.x) {
      float o[kAttnMaxTG];
#pragma unroll
      for (int i = 0; i < kAttnMaxTG; ++i) o[i] = 0.f;
      for (int k = 0; k < nk; ++k) {
        const int kp2 = c0 + k;
        float v;
        if (kp2 >= base)
          v = qkv_val(a, b * a.T + (kp2 - base), a.q_dim + a.kv_dim + h * hd + d);
        else
          v = vcache[(size_t)cache_slot(a, kp2) * a.kv_dim + h * hd + d];
#pragma unroll
        for (int i = 0; i < kAttnMaxTG; ++i)
          if (i < TG) o[i] += ss[i * CH + k] * v;
      }
      for (int i = 0; i < TG; ++i) {
        const int t = r0 + i / G, g = i % G;
        float *pp = a.part + ((((size_t)b * a.n_kv + h) * a.n_chunks + c) * a.T * G +
                              (size_t)t * G + g) * (hd + 2);
        pp[d] = o[i];
        if (d == 0) {
          pp[hd] = sm[i];
          pp[hd + 1] = sl[i];
        }
      }
    }
  }

  // ---- last block of (b, h): merge chunks, then append K/V rows ----
  __shared__ int is_last;
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned target = (unsigned)(a.n_chunks * RG);
    is_last = (atomicAdd(&a.counters[b * a.n_kv + h], 1u) == target - 1) ? 1 : 0;
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();

  const int n_active = (kmax - kmin) / CH + 1;
  for (int e = tid; e < a.T * G * hd; e += blockDim.x) {
    const int tg = e / hd, d = e % hd;
    const int t = tg / G, g = tg % G;
    const float *p0 = a.part + (((size_t)b * a.n_kv + h) * a.n_chunks * a.T * G +
                                (size_t)t * G + g) * (hd + 2);
    const size_t cstride = (size_t)a.T * G * (hd + 2);
    float M = -INFINITY;
    for (int cc = 0; cc < n_active; ++cc) M = fmaxf(M, p0[cc * cstride + hd]);
    float O = 0.f, L = 0.f;
    for (int cc = 0; cc < n_active; ++cc) {
      const float *pc = p0 + cc * cstride;
      const float m = pc[hd];
      if (m == -INFINITY) continue;
      const float w = expf(m - M);
      O += pc[d] * w;
      L += pc[hd + 1] * w;
    }
    const float y = O / L;
    const size_t oi = (size_t)(b * a.T + t) * a.q_dim + (h * G + g) * hd + d;
    if (a.out) a.out[oi] = y;
    if (a.out_hi) {
      _Float16 hh, ll;
      split_hi_lo(y * a.out_prescale, &hh, &ll);
      a.out_hi[oi] = hh;
      a.out_lo[oi] = ll;
    }
  }
  if (a.write_cache) {
    // write_kv_sliding / write_kv_full (gemma4_e4b.mojo:211-249)
    for (int e = tid; e < a.T * hd; e += blockDim.x) {
      const int t = e / hd, d = e % hd;
      const int p = base + t;
      if (a.cache_kind == MS_CACHE_LINEAR && p >= a.cache_len) continue;
      const int row = b * a.T + t;
      const size_t ci = (size_t)cache_slot(a, p) * a.kv_dim + h * hd + d;
      kcache[ci] = rope_val(a, row, a.q_dim + h * hd, d, p);
      vcache[ci] = qkv_val(a, row, a.q_dim + a.kv_dim + h * hd + d);
    }
  }
  __syncthreads();
  if (tid == 0) atomicExch(&a.counters[b * a.n_kv + h], 0u);
}

int attn_check(const AttnArgs &a) {
  MS_CHECK_ARG(a.n_kv > 0 && a.n_heads % a.n_kv == 0, "attention: n_heads % n_kv != 0");
  const int G = a.n_heads / a.n_kv;
  MS_CHECK_ARG(G <= kAttnMaxTG, "attention: GQA group too large");
  const int TR = std::max(1, std::min(a.T, kAttnMaxTG / G));
  MS_CHECK_ARG(TR * G * a.hd <= kAttnLds, "attention: q staging exceeds LDS budget");
  MS_CHECK_ARG(a.hd % 32 == 0, "attention: head_dim % 32 != 0");
  MS_CHECK_ARG(a.rot % 2 == 0 && a.rot <= a.hd, "attention: bad rotary width");
  MS_CHECK_ARG(a.cache_len > 0, "attention: empty cache");
  return MS_OK;
}

int launch_attention(const AttnArgs &a, hipStream_t st) {
  if (int rc = attn_check(a)) return rc;
  const int G = a.n_heads / a.n_kv;
  const int TR = std::max(1, std::min(a.T, kAttnMaxTG / G));
  const int RG = (a.T + TR - 1) / TR;
  const long blocks = (long)a.B * a.n_kv * a.n_chunks * RG;
  const size_t shmem = (size_t)(kAttnLds + kAttnMaxTG * kAttnChunk + 2 * kAttnMaxTG) * 4;
  hipLaunchKernelGGL(k_attention, dim3(blocks), dim3(256), shmem, st, a);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

}  // namespace ms
