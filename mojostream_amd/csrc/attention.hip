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
//  k_attn_chunks   one block per (16-key chunk, row group, sequence x kv head):
//                  the chunk's cached K and V rows, the rows' fresh K/V and q
//                  (after RoPE) for the kv head's G query heads staged in LDS,
//                  then (max, sum, o[hd]) per (row, head).
//  k_attn_combine  one block per (query head, row, sequence): merges the
//                  chunks (log-sum-exp rescaling), writes the O-projection
//                  input row (fp32) and appends the row's K (after RoPE) and V
//                  to the cache.  It runs after every chunk block has read the
//                  cache, so rows that wrap the circular window never
//                  overwrite a key another row still needs.
// Keys of the current rows come from the fresh projections, older keys from
// the cache.  Every phase issues all of its global loads before the first use
// (one memory round trip per phase after the position load).
#include <cmath>

#include "attention.h"

namespace ms {

template <class T>
__device__ inline T aldg(const void *p) {
  return *(const __attribute__((address_space(1))) T *)p;
}
template <>
__device__ inline float4 aldg<float4>(const void *p) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const f32x4 v = *(const __attribute__((address_space(1))) f32x4 *)p;
  return float4{v.x, v.y, v.z, v.w};
}

// A value that is the same for every lane, loaded per lane (an opaque zero
// offset): the compiler keeps it in a vector register instead of waiting for
// it at once to move it into a scalar register, so the loads issued after it
// go out before it arrives.
template <class T>
__device__ inline T aldg_lane(const T *p) {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return aldg<T>(p + z);
}

// Launch parameters as scalars, read once at kernel entry (an opaque register
// move keeps the compiler from re-reading the argument struct later).
template <class T>
__device__ inline T keep(T v) {
  asm volatile("" : "+s"(v));
  return v;
}

struct AttnP {
  int T, q_dim, kv_dim, n_heads, n_kv, G, rot, half, circular, cache_len, clamp, ld, apply_rope,
      n_chunks, write_cache, grid_chunks;
  float scale;
  const float *qkv, *cos_t, *sin_t, *rope_cur;
  const int32_t *pos;
  float *kc, *vc, *part, *out;
  unsigned *ctr;
  size_t cache_seq_stride;
};

__device__ inline AttnP load_params(const AttnArgs &a) {
  AttnP p;
  p.T = keep(a.T);
  p.q_dim = keep(a.q_dim);
  p.kv_dim = keep(a.kv_dim);
  p.n_heads = keep(a.n_heads);
  p.n_kv = keep(a.n_kv);
  p.G = p.n_heads / p.n_kv;
  p.rot = keep(a.rot);
  p.half = p.rot >> 1;
  p.circular = keep(a.cache_kind) == MS_CACHE_CIRCULAR;
  p.cache_len = keep(a.cache_len);
  p.clamp = keep(a.clamp);
  p.ld = keep(a.ld);
  p.apply_rope = keep(a.apply_rope);
  p.n_chunks = keep(a.n_chunks);
  p.write_cache = keep(a.write_cache);
  p.grid_chunks = keep(a.grid_chunks);
  p.scale = keep(a.scale);
  p.qkv = keep(a.qkv);
  p.rope_cur = keep(a.rope_cur);
  p.cos_t = keep(a.cos_t);
  p.sin_t = keep(a.sin_t);
  p.pos = keep(a.pos);
  p.kc = keep(a.kc);
  p.vc = keep(a.vc);
  p.part = keep(a.part);
  p.out = keep(a.out);
  p.ctr = keep(a.ctr);
  p.cache_seq_stride = keep(a.cache_seq_stride);
  return p;
}

__device__ inline void key_range(const AttnP &p, int pos, int *lo, int *hi) {
  if (p.circular) {
    const int l = pos - p.cache_len + 1;
    *lo = l > 0 ? l : 0;
    *hi = pos;
  } else {
    *lo = 0;
    int h = pos;
    if (p.clamp && h > p.cache_len - 1) h = p.cache_len - 1;
    *hi = h;
  }
}

__device__ inline int cache_slot(const AttnP &p, int t) {
  return p.circular ? t % p.cache_len : t;
}

// Element d of a head (starting at column c0 of qkv row `row`) after RoPE at
// position pos (apply_rope_inplace, kernels.mojo:579-595: pairs (i, i+rot/2)
// over the first rot dims).  Split into a load step and a compute step so the
// loads of many elements are issued together.
struct RopeIn {
  float x, y, c, s;
  bool rot, lo;
};

__device__ inline void rope_load(const AttnP &p, int row, int c0, int d, int pos, RopeIn &r) {
  const bool rot = p.apply_rope && d < p.rot;
  const bool lo = d < p.half;
  const int i = lo ? d : d - p.half;
  const int pd = rot ? (lo ? d + p.half : d - p.half) : d;
  const float *base = p.qkv + (size_t)row * p.ld + c0;
  r.x = aldg<float>(base + d);
  r.y = aldg<float>(base + pd);
  const size_t ti = rot ? (size_t)pos * p.half + i : 0;
  r.c = rot ? aldg<float>(p.cos_t + ti) : 1.f;
  r.s = rot ? aldg<float>(p.sin_t + ti) : 0.f;
  r.rot = rot;
  r.lo = lo;
}

__device__ inline float rope_apply(const RopeIn &r) {
  if (!r.rot) return r.x;
  return r.lo ? r.x * r.c - r.y * r.s : r.y * r.s + r.x * r.c;
}

// 256-thread block reduction (sum or max); every thread gets the result.
__device__ inline float block_reduce(float v, float *sh, bool is_max) {
  constexpr int nw = 4;  // 256 threads: a blockDim read would load the dispatch packet
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
#pragma unroll
  for (int i = 1; i < nw; ++i) t = is_max ? fmaxf(t, sh[i]) : t + sh[i];
  return t;
}

constexpr int kRopeBatch = 8;  // q elements per thread per load batch

// TGM: compile-time bound on the (row, query head) pairs of a block (4 for a
// decode step with 4 query heads per kv head, kAttnMaxTG for prefill row
// groups); rows past the real count hold zero queries, so every LDS read of
// the score loop is unconditional.
template <int HD, int TGM>
__global__ __launch_bounds__(256) void k_attn_chunks(AttnArgs args) {
  extern __shared__ __align__(16) float lds[];
  constexpr int CH = kAttnChunk;
  constexpr int F4 = CH * HD / 4 / 256;  // float4 of K (and of V) per thread
  constexpr int NV = HD / 64;            // float4 per thread per key (scores)
  constexpr int DPT = (HD + 255) / 256;  // P.V dims per thread
  const AttnP p = load_params(args);
  const int tid = threadIdx.x;
  const int c = blockIdx.x, rg = blockIdx.y;
  const int b = (int)blockIdx.z / p.n_kv, h = (int)blockIdx.z % p.n_kv;
  const int G = p.G;
  const int TR = max(1, min(p.T, kAttnMaxTG / G));

  const int base = aldg<int32_t>(p.pos + b);
  int kmin, kmax, dummy;
  key_range(p, base, &kmin, &dummy);
  key_range(p, base + p.T - 1, &dummy, &kmax);
  const int c0 = kmin + c * CH;
  if (c0 > kmax) return;  // beyond the attended span at this position
  const int r0 = rg * TR;
  const int nr = min(TR, p.T - r0);
  const int TG = nr * G;
  const int nk = min(CH, kmax - c0 + 1);

  float *sk = lds;                     // [CH][HD] keys of the chunk
  float *sv = sk + CH * HD;            // [CH][HD] values
  float *sq = sv + CH * HD;            // [TG][HD] rotated queries
  float *ss = sq + kAttnLds;           // [TG][CH] scores -> probabilities
  float *sm = ss + kAttnMaxTG * CH;    // [TG]
  float *sl = sm + kAttnMaxTG;         // [TG]
  const float *kcache = p.kc + (size_t)b * p.cache_seq_stride;
  const float *vcache = p.vc + (size_t)b * p.cache_seq_stride;

  // ---- phase 1: every load of the cached rows and of the first q batch
  float4 kr[F4], vr[F4];
#pragma unroll
  for (int j = 0; j < F4; ++j) {
    const int f = tid + 256 * j;  // float4 index in [CH][HD/4]
    const int k = f / (HD / 4), d4 = f % (HD / 4);
    const int kp = c0 + k;
    kr[j] = float4{0.f, 0.f, 0.f, 0.f};
    vr[j] = float4{0.f, 0.f, 0.f, 0.f};
    if (k < nk && kp < base) {
      const size_t off = (size_t)cache_slot(p, kp) * p.kv_dim + h * HD + 4 * d4;
      kr[j] = aldg<float4>(kcache + off);
      vr[j] = aldg<float4>(vcache + off);
    }
  }
  const int nq = TG * HD;
  RopeIn qi[kRopeBatch];
#pragma unroll
  for (int u = 0; u < kRopeBatch; ++u) {
    const int e = tid + 256 * u;
    if (e < nq) {
      const int tg = e / HD, d = e % HD;
      const int t = r0 + tg / G, g = tg % G;
      rope_load(p, b * p.T + t, (h * G + g) * HD, d, base + t, qi[u]);
    }
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
#pragma unroll
  for (int u = 0; u < kRopeBatch; ++u) {
    const int e = tid + 256 * u;
    if (e < nq) sq[e] = rope_apply(qi[u]);
  }
  for (int e = nq + tid; e < TGM * HD; e += 256) sq[e] = 0.f;
  // remaining q elements (prefill row groups), in batches
  for (int e0 = 256 * kRopeBatch; e0 < nq; e0 += 256 * kRopeBatch) {
#pragma unroll
    for (int u = 0; u < kRopeBatch; ++u) {
      const int e = e0 + tid + 256 * u;
      if (e < nq) {
        const int tg = e / HD, d = e % HD;
        const int t = r0 + tg / G, g = tg % G;
        rope_load(p, b * p.T + t, (h * G + g) * HD, d, base + t, qi[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < kRopeBatch; ++u) {
      const int e = e0 + tid + 256 * u;
      if (e < nq) sq[e] = rope_apply(qi[u]);
    }
  }
  // rows of this call that fall in the chunk: fresh K (after RoPE) and V
  const int kin0 = max(c0, base), kin1 = min(c0 + nk, base + p.T);
  const int nin = (kin1 - kin0) * HD;
  for (int e0 = 0; e0 < nin; e0 += 256 * kRopeBatch) {
    RopeIn ki[kRopeBatch];
    float vv[kRopeBatch];
#pragma unroll
    for (int u = 0; u < kRopeBatch; ++u) {
      const int e = e0 + tid + 256 * u;
      if (e < nin) {
        const int kp = kin0 + e / HD, d = e % HD;
        const int row = b * p.T + (kp - base);
        rope_load(p, row, p.q_dim + h * HD, d, kp, ki[u]);
        vv[u] = aldg<float>(p.qkv + (size_t)row * p.ld + p.q_dim + p.kv_dim + h * HD + d);
      }
    }
#pragma unroll
    for (int u = 0; u < kRopeBatch; ++u) {
      const int e = e0 + tid + 256 * u;
      if (e < nin) {
        const int kp = kin0 + e / HD, d = e % HD;
        sk[(kp - c0) * HD + d] = rope_apply(ki[u]);
        sv[(kp - c0) * HD + d] = vv[u];
      }
    }
  }
  __syncthreads();

  // ---- scores: thread (key kk, dim group dg of 16); keys past the chunk end
  // hold zeros, rows past TG zero queries: no conditional LDS reads
  const int kk = tid >> 4, dg = tid & 15;
  const int kp = c0 + kk;
  float acc[TGM];
#pragma unroll
  for (int i = 0; i < TGM; ++i) acc[i] = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int d = dg * 4 + 64 * i;
    const float4 kv = *reinterpret_cast<const float4 *>(sk + kk * HD + d);
#pragma unroll
    for (int t = 0; t < TGM; ++t) {
      const float4 qq = *reinterpret_cast<const float4 *>(sq + t * HD + d);
      acc[t] += qq.x * kv.x + qq.y * kv.y + qq.z * kv.z + qq.w * kv.w;
    }
  }
#pragma unroll
  for (int t = 0; t < TGM; ++t) {
    float v = acc[t];
    v += __shfl_xor(v, 1, 64);
    v += __shfl_xor(v, 2, 64);
    v += __shfl_xor(v, 4, 64);
    v += __shfl_xor(v, 8, 64);
    acc[t] = v;
  }
  if (dg == 0) {
#pragma unroll
    for (int t = 0; t < TGM; ++t) {
      if (t < TG) {
        const int row_t = r0 + t / G;
        int lo, hi;
        key_range(p, base + row_t, &lo, &hi);
        const bool ok = kk < nk && kp >= lo && kp <= hi;
        ss[t * CH + kk] = ok ? acc[t] * p.scale : -INFINITY;
      }
    }
  }
  __syncthreads();

  if (tid >= TG && tid < TGM) {
#pragma unroll
    for (int k = 0; k < CH; ++k) ss[tid * CH + k] = 0.f;
  }
  if (tid < TG) {
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < CH; ++k) m = fmaxf(m, ss[tid * CH + k]);
    float l = 0.f;
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const float sc = ss[tid * CH + k];
      const float pr = (sc == -INFINITY) ? 0.f : expf(sc - m);
      ss[tid * CH + k] = pr;
      l += pr;
    }
    sm[tid] = m;
    sl[tid] = l;
  }
  __syncthreads();

  // ---- P.V: values of the chunk in registers, probabilities broadcast from LDS
  float *pbase = p.part + (((size_t)b * p.n_kv + h) * p.n_chunks + c) * p.T * G * (HD + 2);
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int d = tid + 256 * j;
    if (d >= HD) continue;
    float vk[CH];
#pragma unroll
    for (int k = 0; k < CH; ++k) vk[k] = sv[k * HD + d];
    float o[TGM];
#pragma unroll
    for (int t = 0; t < TGM; ++t) {
      o[t] = 0.f;
#pragma unroll
      for (int k = 0; k < CH; ++k) o[t] += ss[t * CH + k] * vk[k];
    }
#pragma unroll
    for (int t = 0; t < TGM; ++t) {
      if (t < TG) {
        const int row_t = r0 + t / G, g = t % G;
        float *pp = pbase + ((size_t)row_t * G + g) * (HD + 2);
        pp[d] = o[t];
        if (d == 0) {
          pp[HD] = sm[t];
          pp[HD + 1] = sl[t];
        }
      }
    }
  }
}

// One block per (query head, row, sequence): chunk weights exp(m_c - M) / L,
// then o[d] = sum_c w_c * o_c[d] with the loads of a 16-chunk group in flight
// together.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_combine(AttnArgs args) {
  extern __shared__ float wsh[];  // [n_active] chunk weights
  __shared__ float sh[16];
  constexpr int DPT = (HD + 255) / 256;
  constexpr int CG = HD > 256 ? 16 : 32;  // chunk rows of o loaded in the first batch
  const AttnP p = load_params(args);
  const int tid = threadIdx.x;
  const int hq = blockIdx.x, t = blockIdx.y, b = blockIdx.z;
  const int G = p.G;
  const int h = hq / G, g = hq % G;
  const int base = aldg<int32_t>(p.pos + b);
  int kmin, kmax, dummy;
  key_range(p, base, &kmin, &dummy);
  key_range(p, base + p.T - 1, &dummy, &kmax);
  const int n_active = (kmax - kmin) / kAttnChunk + 1;
  const size_t cstride = (size_t)p.T * G * (HD + 2);
  const float *pg = p.part + (((size_t)b * p.n_kv + h) * p.n_chunks * p.T * G +
                              (size_t)t * G + g) * (HD + 2);
  const int row = b * p.T + t;
  const int pt = base + t;
  const bool do_cache =
      p.write_cache && g == 0 && !(!p.circular && pt >= p.cache_len);

  // every load of this block issued before the reductions: chunk (m, l), the
  // first 16-chunk group of o values, and the row's K/V for the cache append
  float mloc[2], lloc[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int cc = tid + 256 * j;
    mloc[j] = -INFINITY;
    lloc[j] = 0.f;
    if (cc < n_active) {
      mloc[j] = aldg<float>(pg + cc * cstride + HD);
      lloc[j] = aldg<float>(pg + cc * cstride + HD + 1);
    }
  }
  float v0[DPT][CG];
#pragma unroll
  for (int j = 0; j < DPT; ++j)
#pragma unroll
    for (int u = 0; u < CG; ++u) {
      v0[j][u] = 0.f;
      const int d = tid + 256 * j;
      if (d < HD && u < n_active) v0[j][u] = aldg<float>(pg + (size_t)u * cstride + d);
    }
  RopeIn kin[DPT];
  float vin[DPT];
  if (do_cache) {
#pragma unroll
    for (int j = 0; j < DPT; ++j) {
      const int d = tid + 256 * j;
      if (d < HD) {
        rope_load(p, row, p.q_dim + h * HD, d, pt, kin[j]);
        vin[j] = aldg<float>(p.qkv + (size_t)row * p.ld + p.q_dim + p.kv_dim + h * HD + d);
      }
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
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int d = tid + 256 * j;
    if (d < HD) {
      float o = 0.f;
#pragma unroll
      for (int u = 0; u < CG; ++u)
        if (u < n_active) o += v0[j][u] * wsh[u];
      for (int c0 = CG; c0 < n_active; c0 += CG) {
        float v[CG];
#pragma unroll
        for (int u = 0; u < CG; ++u) {
          v[u] = 0.f;
          if (c0 + u < n_active) v[u] = aldg<float>(pg + (size_t)(c0 + u) * cstride + d);
        }
        // (prefill spans past CG chunks only)
#pragma unroll
        for (int u = 0; u < CG; ++u)
          if (c0 + u < n_active) o += v[u] * wsh[c0 + u];
      }
      p.out[(size_t)row * p.q_dim + hq * HD + d] = o;
    }
  }
  if (do_cache) {
    // write_kv_sliding / write_kv_full (gemma4_e4b.mojo:211-249)
    float *kc = p.kc + (size_t)b * p.cache_seq_stride;
    float *vc = p.vc + (size_t)b * p.cache_seq_stride;
    const size_t cbase = (size_t)cache_slot(p, pt) * p.kv_dim + h * HD;
#pragma unroll
    for (int j = 0; j < DPT; ++j) {
      const int d = tid + 256 * j;
      if (d < HD) {
        kc[cbase + d] = rope_apply(kin[j]);
        vc[cbase + d] = vin[j];
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
  MS_CHECK_ARG(a.hd == 64 || a.hd == 128 || a.hd == 256 || a.hd == 512,
               "attention: head_dim must be 64, 128, 256 or 512");
  MS_CHECK_ARG(a.rot % 2 == 0 && a.rot <= a.hd, "attention: bad rotary width");
  MS_CHECK_ARG(a.cache_len > 0, "attention: empty cache");
  MS_CHECK_ARG(a.n_chunks >= 1 && a.n_chunks <= kAttnMaxChunks, "attention: bad key chunk count");
  MS_CHECK_ARG(a.ld >= a.q_dim + 2 * a.kv_dim, "attention: q|k|v row stride too small");
  MS_CHECK_ARG(a.B >= 1 && a.T >= 1, "attention: empty batch");
  return MS_OK;
}

static int launch_attention_decode(const AttnArgs &a, hipStream_t st);

int launch_attention(const AttnArgs &a, hipStream_t st) {
  if (int rc = attn_check(a)) return rc;
  MS_CHECK_ARG(a.qkv && a.part && a.pos && a.out, "attention: missing buffers");
  if (a.T == 1) return launch_attention_decode(a, st);
  const int G = a.n_heads / a.n_kv;
  const int TR = std::max(1, std::min(a.T, kAttnMaxTG / G));
  const int RG = (a.T + TR - 1) / TR;
  const dim3 grid(a.n_chunks, RG, a.B * a.n_kv);
  const int TG = TR * G;
  const size_t shmem =
      (size_t)(2 * kAttnChunk * a.hd + kAttnLds + kAttnMaxTG * kAttnChunk + 2 * kAttnMaxTG) * 4;
  const dim3 cgrid(a.n_heads, a.T, a.B);
  const size_t cshmem = (size_t)a.n_chunks * 4;
#define MS_ATTN(HDV)                                                                      \
  if (TG <= 4)                                                                             \
    hipLaunchKernelGGL((k_attn_chunks<HDV, 4>), grid, dim3(256), shmem, st, a);          \
  else if (TG <= 8)                                                                        \
    hipLaunchKernelGGL((k_attn_chunks<HDV, 8>), grid, dim3(256), shmem, st, a);          \
  else                                                                                     \
    hipLaunchKernelGGL((k_attn_chunks<HDV, kAttnMaxTG>), grid, dim3(256), shmem, st, a); \
  hipLaunchKernelGGL(k_attn_combine<HDV>, cgrid, dim3(256), cshmem, st, a)
  switch (a.hd) {
    case 64: MS_ATTN(64); break;
    case 128: MS_ATTN(128); break;
    case 256: MS_ATTN(256); break;
    default: MS_ATTN(512); break;
  }
#undef MS_ATTN
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}


// ------------------------------------------------------------------------------
// Prefill attention: many rows of one sequence.
//
//  k_rope_rows      q and k of every row after RoPE (qr, kr).
//  k_flash_prefill  one block per (16 rows, kv head), wave g = query head
//                   h*4 + g.  Keys in tiles of 16: K (row pitch HD + 4) and V
//                   transposed (V^T, pitch 20) staged in LDS, the next tile's
//                   loads in registers while the current one computes.
//                   S = Q K^T and O += P V on v_mfma_f32_16x16x4f32 (fp32
//                   products, fp32 sums); online softmax with DPP row
//                   reductions (the 16 keys of a score row sit in one 16-lane
//                   row of the C fragment).  Keys older than the rows come
//                   from the cache, the rows' own keys from kr / qkv.
//  k_cache_append   the rows' k (after RoPE) and v into the cache, after every
//                   block has read it (a circular window must not lose a key
//                   an earlier row still needs).
// The dot product runs over the head dims in the order d = 16u + 4c + r for
// MFMA step 4u + r and k-group c, the same for q and k, so each lane loads its
// q as float4 and reads K with one 16-byte LDS load per four steps.
// ------------------------------------------------------------------------------
typedef float af32x4 __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ inline float adpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
// max / sum over the 16 lanes of each row of the wave (quad permutes, then the
// half-row and row mirrors); every lane of the row gets the result
__device__ inline float row16_max(float v) {
  v = fmaxf(v, adpp<0xB1>(v));
  v = fmaxf(v, adpp<0x4E>(v));
  v = fmaxf(v, adpp<0x141>(v));
  return fmaxf(v, adpp<0x140>(v));
}
__device__ inline float row16_sum(float v) {
  v += adpp<0xB1>(v);
  v += adpp<0x4E>(v);
  v += adpp<0x141>(v);
  return v + adpp<0x140>(v);
}

// The same on float4 units (the rotated half of a head a multiple of 4):
// unit u of a head is four rotation pairs (dims i .. i + 3 and half + i ..,
// both rotated from one float4 of each half and of the tables) or four dims
// past the rotary ones (copied).  Same arithmetic per value as rope_apply.
__global__ __launch_bounds__(256) void k_rope_rows4(AttnArgs args, float *qr, float *kr,
                                                    int hd) {
  const AttnP p = load_params(args);
  const int r = blockIdx.x;
  const int pos = aldg<int32_t>(p.pos) + r;
  const int rot = p.apply_rope ? p.rot : 0, half = rot >> 1;
  const int pq = half >> 2, per = pq + ((hd - rot) >> 2);  // units per head
  const int nh = p.n_heads + p.n_kv;
  const float *row = p.qkv + (size_t)r * p.ld;
  const float *ct = p.cos_t + (size_t)pos * half, *st = p.sin_t + (size_t)pos * half;
  for (int u = threadIdx.x; u < nh * per; u += 256) {
    const int head = u / per, j = u - head * per;
    const bool isq = head < p.n_heads;
    const int hk = isq ? head : head - p.n_heads;
    const float *src = row + (isq ? 0 : p.q_dim) + hk * hd;
    float *dst = isq ? qr + (size_t)r * p.q_dim + hk * hd : kr + (size_t)r * p.kv_dim + hk * hd;
    if (j < pq) {
      const int i = 4 * j;
      const float4 xl = aldg<float4>(src + i), xh = aldg<float4>(src + half + i);
      const float4 c = aldg<float4>(ct + i), sn = aldg<float4>(st + i);
      *reinterpret_cast<float4 *>(dst + i) =
          float4{xl.x * c.x - xh.x * sn.x, xl.y * c.y - xh.y * sn.y, xl.z * c.z - xh.z * sn.z,
                 xl.w * c.w - xh.w * sn.w};
      *reinterpret_cast<float4 *>(dst + half + i) =
          float4{xl.x * sn.x + xh.x * c.x, xl.y * sn.y + xh.y * c.y, xl.z * sn.z + xh.z * c.z,
                 xl.w * sn.w + xh.w * c.w};
    } else {
      const int d = rot + 4 * (j - pq);
      *reinterpret_cast<float4 *>(dst + d) = aldg<float4>(src + d);
    }
  }
}

__global__ __launch_bounds__(256) void k_rope_rows(AttnArgs args, float *qr, float *kr, int hd) {
  const AttnP p = load_params(args);
  const int r = blockIdx.x;
  const int pos = aldg<int32_t>(p.pos) + r;
  const int nq = p.q_dim, nall = p.q_dim + p.kv_dim;
#pragma unroll 4
  for (int e = threadIdx.x; e < nall; e += 256) {
    const bool isq = e < nq;
    const int ee = isq ? e : e - nq;
    const int head = ee / hd, d = ee - head * hd;
    RopeIn ri;
    rope_load(p, r, (isq ? 0 : nq) + head * hd, d, pos, ri);
    const float v = rope_apply(ri);
    if (isq)
      qr[(size_t)r * nq + ee] = v;
    else
      kr[(size_t)r * p.kv_dim + ee] = v;
  }
}

// DS waves per query head, each with 1/DS of the head dims (its q and o in
// registers); their partial scores meet in LDS.
template <int HD, int DS>
constexpr int flash_lds_floats() {
  return 16 * (HD + 4) + HD * 20 + 4 * DS * 16 * 20 + (DS > 1 ? 4 * DS * 256 : 0);
}

template <int HD, int DS>
__global__ __launch_bounds__(256 * DS) void k_flash_prefill(AttnArgs args, const float *qr,
                                                            const float *kr, FlashSplit fs) {
  constexpr int NT = 256 * DS;
  constexpr int HW = HD / DS;             // head dims per wave
  constexpr int NU = HW / 16;             // q float4 per lane; O tiles of 16 dims
  constexpr int KP = HD + 4;              // K row pitch (floats)
  constexpr int VP = 20;                  // V^T row pitch
  constexpr int PP = 20;                  // P row pitch
  constexpr int NF = 16 * HD / 4 / NT;    // float4 of K (and of V) per thread per tile
  extern __shared__ __align__(16) float fl[];
  float *Ks = fl;                     // [16][KP]
  float *VT = Ks + 16 * KP;           // [HD][VP]
  float *Ps = VT + HD * VP;           // [4 DS][16][PP]
  float *Sx = Ps + 4 * DS * 16 * PP;  // [4 DS][256] partial scores (DS > 1)
  const AttnP p = load_params(args);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int li = lane & 15, lk = lane >> 4;
  const int g = wave / DS, hf = wave % DS;
  // block j = (sp * n_rt + n_rt - 1 - rt) * n_kv + h: key split sp of row
  // tile rt and kv head h.  Splits in order, the row tiles with the most keys
  // first, the heads interleaved: the heavy blocks start first and the
  // round-robin of blocks over the XCDs spreads every kind of block.
  const int maxs = keep(fs.maxs), stt = keep(fs.st_tiles), n_rt = keep(fs.n_rt);
  const int j = blockIdx.x;
  const int h = j % p.n_kv, rt = n_rt - 1 - (j / p.n_kv) % n_rt, sp = j / (p.n_kv * n_rt);
  const int hq = h * 4 + g;
  const int d0 = hf * HW;  // first head dim of this wave
  const int r0 = rt * 16;
  const int base = aldg<int32_t>(p.pos);
  const int rlast = min(r0 + 15, p.T - 1);
  int klo, khi, dummy;
  key_range(p, base + r0, &klo, &dummy);
  key_range(p, base + rlast, &dummy, &khi);
  const int kbeg = klo & ~15;
  // the last split takes every remaining tile
  const int nsplit = maxs == 1 ? 1 : min(maxs, ((khi - kbeg) / 16 + stt) / stt);
  if (sp >= nsplit) return;
  const int kfirst = kbeg + sp * stt * 16;
  const int klast = sp == nsplit - 1 ? khi : kbeg + (sp + 1) * stt * 16 - 1;

  // q rows of this wave (A operand, head dims in MFMA order)
  af32x4 q[NU];
  {
    const int row = r0 + li;
    const float *qp = qr + (size_t)row * p.q_dim + hq * HD + d0 + 4 * lk;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      q[u] = af32x4{0.f, 0.f, 0.f, 0.f};
      if (row < p.T) q[u] = aldg<af32x4>(qp + 16 * u);
    }
  }
  // key range of each of this lane's four score rows
  int rlo[4], rhi[4];
  bool rok[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int row = r0 + 4 * lk + e;
    rok[e] = row < p.T;
    key_range(p, base + row, &rlo[e], &rhi[e]);
  }

  // K: a wave's lanes take consecutive dims of one key (whole rows, one
  // float4 LDS store each).  V (VK, head dim 256 and below): lanes take the
  // 16 keys of four dim quads, so the transposed stores of a wave fall in
  // different banks; with a wave over the dims of one key, lane l's V^T rows
  // start 4 l * VP floats apart and each 4-byte store hits a few banks many
  // times over.  At head dim 512 (the key-fastest deal's V addresses would
  // spill registers) thread t takes a 4 x 4 block instead: keys 4 (t / (HD /
  // 4)) .. + 3 of dim quad t % (HD / 4), four coalesced float4 loads, a
  // transpose in registers and four float4 stores to V^T.  The four-key
  // groups of V^T row r sit in slot group ^ ((r >> 4) & 3): the 16 lanes of
  // a store phase (rows 4 d4 + c, 80 bytes apart) then cover 16 distinct
  // bank quads, and a read of dims 16u .. 16u + 15 uses one rotation.
  constexpr bool VK = HD <= 256;
  static_assert(VK || (NF == 4 && NT == 4 * (HD / 4)), "V blocks: 4 keys x 4 dims per thread");
  // (NT is a multiple of 16: with VK, a thread's V key is the same for every f)
  const int vkey = tid % 16;
  af32x4 kreg[NF], vreg[NF];
  auto tile_load = [&](int k0) {
    const int vk = k0 + vkey;
    const float *vrow = nullptr;
    if (VK && vk <= khi)
      vrow = vk < base ? p.vc + (size_t)cache_slot(p, vk) * p.kv_dim + h * HD
                       : p.qkv + (size_t)(vk - base) * p.ld + p.q_dim + p.kv_dim + h * HD;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int idx = tid + NT * f;
      const int key = idx / (HD / 4), d4 = idx % (HD / 4);
      const int k = k0 + key;
      kreg[f] = af32x4{0.f, 0.f, 0.f, 0.f};
      vreg[f] = af32x4{0.f, 0.f, 0.f, 0.f};
      if (k <= khi) {
        if (k < base) {
          const size_t o = (size_t)cache_slot(p, k) * p.kv_dim + h * HD + 4 * d4;
          kreg[f] = aldg<af32x4>(p.kc + o);
        } else {
          const int rr = k - base;
          kreg[f] = aldg<af32x4>(kr + (size_t)rr * p.kv_dim + h * HD + 4 * d4);
        }
      }
      if (VK && vrow) vreg[f] = aldg<af32x4>(vrow + 4 * (idx / 16));
    }
    if constexpr (!VK) {
      // V block: keys k0 + 4 (tid / (HD / 4)) + r, dim quad tid % (HD / 4)
      const int kq = tid / (HD / 4), d4 = tid % (HD / 4);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int k = k0 + 4 * kq + r;
        vreg[r] = af32x4{0.f, 0.f, 0.f, 0.f};
        if (k <= khi)
          vreg[r] = k < base
                        ? aldg<af32x4>(p.vc + (size_t)cache_slot(p, k) * p.kv_dim + h * HD +
                                       4 * d4)
                        : aldg<af32x4>(p.qkv + (size_t)(k - base) * p.ld + p.q_dim +
                                       p.kv_dim + h * HD + 4 * d4);
      }
    }
  };
  auto tile_store = [&]() {
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int idx = tid + NT * f;
      const int key = idx / (HD / 4), d4 = idx % (HD / 4);
      *reinterpret_cast<af32x4 *>(Ks + key * KP + 4 * d4) = kreg[f];
      if constexpr (VK) {
#pragma unroll
        for (int c = 0; c < 4; ++c) VT[(4 * (idx / 16) + c) * VP + vkey] = vreg[f][c];
      }
    }
    if constexpr (!VK) {
      const int kq = tid / (HD / 4), d4 = tid % (HD / 4);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<af32x4 *>(VT + (4 * d4 + c) * VP + 4 * (kq ^ ((d4 >> 2) & 3))) =
            af32x4{vreg[0][c], vreg[1][c], vreg[2][c], vreg[3][c]};
    }
  };

  af32x4 o[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) o[u] = af32x4{0.f, 0.f, 0.f, 0.f};
  float m[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    m[e] = -INFINITY;
    l[e] = 0.f;
  }
  float *Pw = Ps + wave * 16 * PP;

  tile_load(kfirst);
  tile_store();
  __syncthreads();
  for (int k0 = kfirst; k0 <= klast; k0 += 16) {
    const bool more = k0 + 16 <= klast;
    if (more) tile_load(k0 + 16);
    // scores over this wave's dims: row 4lk + e, key k0 + li
    af32x4 sc = af32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const af32x4 kv = *reinterpret_cast<const af32x4 *>(Ks + li * KP + d0 + 16 * u + 4 * lk);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        sc = __builtin_amdgcn_mfma_f32_16x16x4f32(q[u][r], kv[r], sc, 0, 0, 0);
    }
    if constexpr (DS > 1) {
      // sum the partial scores of the head's DS waves, in wave order (every
      // wave of the head gets the same bits)
      *reinterpret_cast<af32x4 *>(Sx + wave * 256 + lane * 4) = sc;
      __syncthreads();
      af32x4 t = *reinterpret_cast<const af32x4 *>(Sx + (g * DS) * 256 + lane * 4);
#pragma unroll
      for (int w2 = 1; w2 < DS; ++w2)
        t += *reinterpret_cast<const af32x4 *>(Sx + (g * DS + w2) * 256 + lane * 4);
      sc = t;
    }
    const int key = k0 + li;
    float pe[4], corr[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool ok = rok[e] && key >= rlo[e] && key <= rhi[e];
      const float x = ok ? sc[e] * p.scale : -INFINITY;
      const float mn = fmaxf(m[e], row16_max(x));
      const float msafe = mn == -INFINITY ? 0.f : mn;
      pe[e] = ok ? expf(x - msafe) : 0.f;
      corr[e] = m[e] == -INFINITY ? 0.f : expf(m[e] - msafe);
      l[e] = l[e] * corr[e] + row16_sum(pe[e]);
      m[e] = mn;
    }
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) o[u][e] *= corr[e];
    // P: C layout [row][key] -> LDS -> A layout (this wave only; LDS accesses
    // of one wave complete in order)
#pragma unroll
    for (int e = 0; e < 4; ++e) Pw[(4 * lk + e) * PP + li] = pe[e];
    __builtin_amdgcn_wave_barrier();
    const af32x4 pa = *reinterpret_cast<const af32x4 *>(Pw + li * PP + 4 * lk);
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      // (head dim 512: the row's key groups are rotated by ((row >> 4) & 3))
      const int vs = VK ? lk : lk ^ (((d0 >> 4) + u) & 3);
      const af32x4 vt =
          *reinterpret_cast<const af32x4 *>(VT + (d0 + 16 * u + li) * VP + 4 * vs);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        o[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[r], vt[r], o[u], 0, 0, 0);
    }
    __syncthreads();  // every wave is done with this tile (and with Sx)
    if (more) tile_store();
    __syncthreads();
  }
  if (nsplit == 1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = r0 + 4 * lk + e;
      if (row >= p.T) continue;
      const float inv = 1.0f / l[e];
      float *op = p.out + (size_t)row * p.q_dim + hq * HD + d0 + li;
#pragma unroll
      for (int u = 0; u < NU; ++u) op[16 * u] = o[u][e] * inv;
    }
  } else {
    // partial of this split: o (unnormalized), max and sum per (row, head)
    float *pb = keep(fs.part) + (size_t)j * 64 * (HD + 2);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int rl = 4 * lk + e;
      float *po = pb + (rl * 4 + g) * HD + d0 + li;
#pragma unroll
      for (int u = 0; u < NU; ++u) po[16 * u] = o[u][e];
      if (li == 0 && hf == 0) {
        float *pm = pb + 64 * HD + (rl * 4 + g) * 2;
        pm[0] = m[e];
        pm[1] = l[e];
      }
    }
  }
}

// Row tiles whose key tiles were split over several blocks: log-sum-exp merge
// of the splits' partials.  One block per (row tile, kv head, query head of
// the group); the splits' weights exp(m_s - M) / L of the 16 rows go through
// LDS, then every thread sums float4 of o over the splits.
constexpr int kFlashMaxSplits = 32;
constexpr int kFlashMaxBlocks = 512;  // blocks of a split launch (two per CU)

template <int HD>
__global__ __launch_bounds__(256) void k_flash_merge(AttnArgs args, FlashSplit fs) {
  __shared__ float wsh[kFlashMaxSplits][16];
  const AttnP p = load_params(args);
  const int maxs = keep(fs.maxs), stt = keep(fs.st_tiles), n_rt = keep(fs.n_rt);
  const int rt = blockIdx.x, h = blockIdx.y >> 2, g = blockIdx.y & 3;
  const int r0 = rt * 16;
  const int base = aldg<int32_t>(p.pos);
  const int rlast = min(r0 + 15, p.T - 1);
  int klo, khi, dummy;
  key_range(p, base + r0, &klo, &dummy);
  key_range(p, base + rlast, &dummy, &khi);
  const int kbeg = klo & ~15;
  const int nsplit = min(maxs, ((khi - kbeg) / 16 + stt) / stt);
  if (nsplit <= 1) return;
  // record of split s: block (s * n_rt + n_rt - 1 - rt) * n_kv + h
  const float *pb = keep(fs.part) + ((size_t)(n_rt - 1 - rt) * p.n_kv + h) * 64 * (HD + 2);
  const size_t sstride = (size_t)n_rt * p.n_kv * 64 * (HD + 2);
  const int tid = threadIdx.x;
  if (tid < 16) {
    const float *pm = pb + 64 * HD + (tid * 4 + g) * 2;
    float M = -INFINITY;
    for (int s2 = 0; s2 < nsplit; ++s2) M = fmaxf(M, pm[s2 * sstride]);
    float L = 0.f;
    for (int s2 = 0; s2 < nsplit; ++s2) {
      const float ms2 = pm[s2 * sstride];
      const float w = ms2 == -INFINITY ? 0.f : expf(ms2 - M);
      wsh[s2][tid] = w;
      L += pm[s2 * sstride + 1] * w;
    }
    // rows past T have no keys (L = 0); they are not stored
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    for (int s2 = 0; s2 < nsplit; ++s2) wsh[s2][tid] *= inv;
  }
  __syncthreads();
  constexpr int N4 = 16 * HD / 4;
#pragma unroll 4
  for (int e = tid; e < N4; e += 256) {
    const int rl = e / (HD / 4), d = 4 * (e % (HD / 4));
    const int row = r0 + rl;
    const float *po = pb + (rl * 4 + g) * HD + d;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s2 = 0; s2 < nsplit; ++s2) {
      const float w = wsh[s2][rl];
      const float4 v = *reinterpret_cast<const float4 *>(po + s2 * sstride);
      acc.x += w * v.x;
      acc.y += w * v.y;
      acc.z += w * v.z;
      acc.w += w * v.w;
    }
    if (row < p.T) {
      float *op = p.out + (size_t)row * p.q_dim + (h * 4 + g) * HD + d;
      op[0] = acc.x;
      op[1] = acc.y;
      op[2] = acc.z;
      op[3] = acc.w;
    }
  }
}

// Split plan of a prefill launch.  Row tile rt (rows at positions
// plan_pos + 16 rt ...) attends to about min(plan_pos / 16 + rt + 2, bound)
// key tiles, bound = cache_len / 16 + 2.  Splits of st tiles, st = the launch's
// tiles / 256 CUs (at least 8), so that the blocks make about one round of
// the chip; no split unless the longest row tile is a third longer than st.
// At most kFlashMaxBlocks blocks and kFlashMaxSplits splits per row tile (the
// last split of a row tile takes every tile left).
static FlashSplit flash_split_plan(const AttnArgs &a) {
  FlashSplit fs{};
  fs.n_rt = (a.T + 15) / 16;
  fs.maxs = 1;
  fs.st_tiles = 1 << 30;
  const long bound = (a.cache_len + 15) / 16 + 1;
  const long p0 = std::max(0, a.plan_pos);
  auto tiles = [&](long rt) { return std::min((p0 + rt * 16 + 15) / 16 + 1, bound); };
  long tot = 0;
  for (long rt = 0; rt < fs.n_rt; ++rt) tot += tiles(rt);
  tot *= a.n_kv;
  const long maxw = tiles(fs.n_rt - 1);
  long st = std::max(8L, (tot + 255) / 256);
  if (st * 4 > maxw * 3) return fs;
  long maxs = std::min<long>((maxw + st - 1) / st, kFlashMaxSplits);
  maxs = std::min<long>(maxs, kFlashMaxBlocks / ((long)fs.n_rt * a.n_kv));
  if (maxs <= 1) return fs;
  st = std::max(st, (maxw + maxs - 1) / maxs);
  fs.maxs = (int)maxs;
  fs.st_tiles = (int)st;
  return fs;
}

size_t flash_part_floats(const AttnArgs &a) {
  const FlashSplit fs = flash_split_plan(a);
  if (fs.maxs <= 1) return 0;
  return (size_t)a.n_kv * fs.n_rt * fs.maxs * 64 * (a.hd + 2);
}

size_t flash_part_floats_max(int hd) { return (size_t)kFlashMaxBlocks * 64 * (hd + 2); }

// write_kv_sliding / write_kv_full (gemma4_e4b.mojo:211-249) for the rows
__global__ __launch_bounds__(256) void k_cache_append(AttnArgs args, const float *kr) {
  const AttnP p = load_params(args);
  const int r = blockIdx.x;
  // a circular cache keeps the last cache_len rows; older rows of the call
  // would share their slots with later ones
  if (p.circular && r < p.T - p.cache_len) return;
  const int pt = aldg<int32_t>(p.pos) + r;
  if (!p.circular && pt >= p.cache_len) return;  // linear cache full: dropped
  const size_t cb = (size_t)cache_slot(p, pt) * p.kv_dim;
  for (int c = threadIdx.x; c < p.kv_dim; c += 256) {
    p.kc[cb + c] = aldg<float>(kr + (size_t)r * p.kv_dim + c);
    p.vc[cb + c] = aldg<float>(p.qkv + (size_t)r * p.ld + p.q_dim + p.kv_dim + c);
  }
}

bool prefill_flash_ok(const AttnArgs &a) {
  return a.B == 1 && a.n_kv > 0 && a.n_heads == 4 * a.n_kv &&
         (a.hd == 128 || a.hd == 256 || a.hd == 512);
}

int launch_attention_prefill(const AttnArgs &a, float *qr, float *kr, float *fpart,
                             size_t fpart_floats, hipStream_t st) {
  if (int rc = attn_check(a)) return rc;
  MS_CHECK_ARG(prefill_flash_ok(a), "prefill attention: needs B = 1, 4 query heads per kv "
                                    "head and head_dim 128, 256 or 512");
  MS_CHECK_ARG(a.qkv && a.pos && a.out && a.kc && a.vc && qr && kr,
               "prefill attention: missing buffers");
  FlashSplit fs = flash_split_plan(a);
  const size_t need = flash_part_floats(a);
  if (need == 0 || !fpart || fpart_floats < need) fs.maxs = 1;  // no split
  fs.part = fpart;
  if (a.hd % 4 == 0 && (!a.apply_rope || a.rot % 8 == 0) && a.ld % 4 == 0 && a.q_dim % 4 == 0 &&
      a.kv_dim % 4 == 0)
    hipLaunchKernelGGL(k_rope_rows4, dim3(a.T), dim3(256), 0, st, a, qr, kr, a.hd);
  else
    hipLaunchKernelGGL(k_rope_rows, dim3(a.T), dim3(256), 0, st, a, qr, kr, a.hd);
  const dim3 grid(fs.maxs * fs.n_rt * a.n_kv);
#define MS_FLASH(HDV, DSV)                                                                \
  hipLaunchKernelGGL((k_flash_prefill<HDV, DSV>), grid, dim3(256 * DSV),                   \
                     (flash_lds_floats<HDV, DSV>() * 4), st, a, (const float *)qr,         \
                     (const float *)kr, fs);                                               \
  if (fs.maxs > 1)                                                                         \
  hipLaunchKernelGGL(k_flash_merge<HDV>, dim3(fs.n_rt, a.n_kv * 4), dim3(256), 0, st, a, fs)
  switch (a.hd) {
    case 128: MS_FLASH(128, 1); break;
    case 256: MS_FLASH(256, 2); break;
    default: MS_FLASH(512, 2); break;
  }
#undef MS_FLASH
  if (a.write_cache)
    hipLaunchKernelGGL(k_cache_append, dim3(a.T), dim3(256), 0, st, a, (const float *)kr);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

// ------------------------------------------------------------------------------
// Decode attention: one row per sequence (T == 1), one launch.
//
//  k_attn_decode  one block per (16-slot chunk of the cache, sequence x kv
//                 head).  Chunk c covers cache slots 16c..16c+15 at every
//                 position: slot j of a circular cache holds position
//                 base - ((base - j) mod W), slot j of a linear cache position
//                 j.  Softmax does not depend on the order of the keys, so the
//                 slot order serves, and a circular cache's rows are loaded
//                 before the position arrives.  The slot of the current
//                 position takes the row's fresh k (after RoPE) and v; the
//                 block holding it also appends them to the cache, which is
//                 safe because no other block reads that slot and the row it
//                 replaces has left the window.  Each block writes (max, sum,
//                 o[hd]) per query head with agent-coherent stores and counts
//                 itself done; the last block of a (sequence, kv head) merges
//                 the chunks and resets the counter for the next launch.
// ------------------------------------------------------------------------------
__device__ inline void st_agent(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float lane_of(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ inline float wave64_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_of(v, 0), lane_of(v, 16)), fmaxf(lane_of(v, 32), lane_of(v, 48)));
}
__device__ inline float wave64_sum(float v) {
  v = row16_sum(v);
  return (lane_of(v, 0) + lane_of(v, 16)) + (lane_of(v, 32) + lane_of(v, 48));
}

// Partner dim of d under RoPE and the rotation of x (partner y) at position
// pos; the same arithmetic as rope_apply.
__device__ inline int rope_partner(const AttnP &p, int d) {
  const bool rot = p.apply_rope && d < p.rot;
  return rot ? (d < p.half ? d + p.half : d - p.half) : d;
}
__device__ inline void rope_cs(const AttnP &p, int d, int pos, float &c, float &s) {
  const bool rot = p.apply_rope && d < p.rot;
  const int i = d < p.half ? d : d - p.half;
  const size_t ti = rot ? (size_t)pos * p.half + i : 0;
  c = rot ? aldg<float>(p.cos_t + ti) : 1.f;
  s = rot ? aldg<float>(p.sin_t + ti) : 0.f;
}
// rope_cs from the factors prepared for the row's position ([2][rot / 2])
__device__ inline void rope_cur_cs(const AttnP &p, int d, float &c, float &s) {
  const bool rot = p.apply_rope && d < p.rot;
  const int i = d < p.half ? d : d - p.half;
  c = rot ? aldg<float>(p.rope_cur + i) : 1.f;
  s = rot ? aldg<float>(p.rope_cur + p.half + i) : 0.f;
}
__device__ inline float rope_mix(const AttnP &p, int d, float x, float y, float c, float s) {
  if (!(p.apply_rope && d < p.rot)) return x;
  return d < p.half ? x * c - y * s : y * s + x * c;
}

constexpr int kSc1 = 16;  // buffer cache policy: sc1 (agent-coherent)

// Merge units (float4 of one head) per thread: a power of two, so that a
// thread's units share one head (HD / 4 is a multiple of it).
constexpr int dec_units_per_thread(int HD, int TGM) {
  const int n = (TGM * HD / 4 + 255) / 256;
  return n <= 1 ? 1 : (n <= 2 ? 2 : (n <= 4 ? 4 : 8));
}
// Chunks per merge batch: 128 registers of o partials in flight per thread.
constexpr int dec_merge_batch(int upt) { return 32 / upt < 4 ? 4 : 32 / upt; }

template <int HD, int TGM>
__global__ __launch_bounds__(256) void k_attn_decode(AttnArgs args) {
  // 16-byte aligned: the float4 LDS accesses below (a static variable placed
  // first would otherwise shift the dynamic region by its size)
  extern __shared__ __align__(16) float lds[];
  __shared__ int s_last;
  constexpr int CH = kAttnChunk;
  constexpr int F4 = CH * HD / 4 / 256;  // float4 of K (and of V) per thread
  constexpr int NV = HD / 64;            // float4 per thread per key (scores)
  constexpr int DPT = (HD + 255) / 256;  // head dims per thread
  const AttnP p = load_params(args);
  const int tid = threadIdx.x;
  const int c = blockIdx.x;
  const int b = (int)blockIdx.y / p.n_kv, h = (int)blockIdx.y % p.n_kv;
  const int G = p.G;
  const int L = p.cache_len;
  const int nq = G * HD;

  float *sk = lds;              // [CH][HD] keys of the chunk
  float *sv = sk + CH * HD;     // [CH][HD] values
  float *sq = sv + CH * HD;     // [TGM][HD] rotated queries
  float *ss = sq + TGM * HD;    // [TGM][CH] scores -> probabilities
  float *sm = ss + TGM * CH;    // [TGM]
  float *sl = sm + TGM;         // [TGM]
  float *wsh = sl + TGM;        // [n_chunks][G] merge weights (last block)
  const size_t cbase = (size_t)b * p.cache_seq_stride;
  const float *qrow = p.qkv + (size_t)b * p.ld;

  // ---- loads that do not depend on the position: the position itself, the
  // chunk's cached rows, the raw q of the first batch, the fresh k and v.  The
  // host launches only the chunks its bound on the position can reach, so
  // the rows are loaded before the position arrives (slots past it are
  // zeroed below).
  const int base = aldg<int32_t>(p.pos + b);
  float4 kr[F4], vr[F4];
#pragma unroll
  for (int j = 0; j < F4; ++j) {
    kr[j] = float4{0.f, 0.f, 0.f, 0.f};
    vr[j] = float4{0.f, 0.f, 0.f, 0.f};
    const int f = tid + 256 * j;
    const int slot = c * CH + f / (HD / 4), d4 = f % (HD / 4);
    if (slot < L) {
      const size_t off = cbase + (size_t)slot * p.kv_dim + h * HD + 4 * d4;
      kr[j] = aldg<float4>(p.kc + off);
      vr[j] = aldg<float4>(p.vc + off);
    }
  }
  float qx[kRopeBatch], qy[kRopeBatch];
#pragma unroll
  for (int u = 0; u < kRopeBatch; ++u) {
    const int e = tid + 256 * u;
    qx[u] = qy[u] = 0.f;
    if (e < nq) {
      const int g = e / HD, d = e % HD;
      const float *qh = qrow + (h * G + g) * HD;
      qx[u] = aldg<float>(qh + d);
      qy[u] = aldg<float>(qh + rope_partner(p, d));
    }
  }
  float kx[DPT], ky[DPT], vx[DPT];
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int d = tid + 256 * j;
    kx[j] = ky[j] = vx[j] = 0.f;
    if (d < HD) {
      const float *kh = qrow + p.q_dim + h * HD;
      kx[j] = aldg<float>(kh + d);
      ky[j] = aldg<float>(kh + rope_partner(p, d));
      vx[j] = aldg<float>(qrow + p.q_dim + p.kv_dim + h * HD + d);
    }
  }

  // ---- the position: attended slots [0, nslots), the slot of this row
  int lo, hi;
  key_range(p, base, &lo, &hi);
  const int nslots = p.circular ? min(L, base + 1) : min(hi + 1, L);
  // (clamped to the launched chunks, so the counter stays consistent)
  const int n_active = min((nslots + CH - 1) / CH, p.grid_chunks);
  if (c >= n_active) return;
  const int fslot = p.circular ? base % L : base;
  const bool fresh_here = fslot < nslots && fslot / CH == c;
  float qc[kRopeBatch], qs[kRopeBatch];
#pragma unroll
  for (int u = 0; u < kRopeBatch; ++u) {
    const int e = tid + 256 * u;
    qc[u] = 1.f;
    qs[u] = 0.f;
    if (e < nq) rope_cs(p, e % HD, base, qc[u], qs[u]);
  }
  float kc_[DPT], ks_[DPT];
#pragma unroll
  for (int j = 0; j < DPT; ++j) {
    const int d = tid + 256 * j;
    kc_[j] = 1.f;
    ks_[j] = 0.f;
    if (fresh_here && d < HD) rope_cs(p, d, base, kc_[j], ks_[j]);
  }

  // cached rows (zeros for slots past the attended ones, so 0 * v stays
  // finite); the fresh slot is filled below
#pragma unroll
  for (int j = 0; j < F4; ++j) {
    const int f = tid + 256 * j;
    const int slot = c * CH + f / (HD / 4);
    if (slot >= nslots) {
      kr[j] = float4{0.f, 0.f, 0.f, 0.f};
      vr[j] = float4{0.f, 0.f, 0.f, 0.f};
    }
    if (!(fresh_here && slot == fslot)) {
      reinterpret_cast<float4 *>(sk)[f] = kr[j];
      reinterpret_cast<float4 *>(sv)[f] = vr[j];
    }
  }
#pragma unroll
  for (int u = 0; u < kRopeBatch; ++u) {
    const int e = tid + 256 * u;
    if (e < nq) sq[e] = rope_mix(p, e % HD, qx[u], qy[u], qc[u], qs[u]);
  }
  // q elements past the first batch (more than 2048 per kv head)
  for (int e = 256 * kRopeBatch + tid; e < nq; e += 256) {
    const int g = e / HD, d = e % HD;
    const float *qh = qrow + (h * G + g) * HD;
    float cc, sn;
    rope_cs(p, d, base, cc, sn);
    sq[e] = rope_mix(p, d, aldg<float>(qh + d), aldg<float>(qh + rope_partner(p, d)), cc, sn);
  }
  for (int e = nq + tid; e < TGM * HD; e += 256) sq[e] = 0.f;
  if (fresh_here) {
    // write_kv_sliding / write_kv_full (gemma4_e4b.mojo:211-249)
    const int kf = fslot - c * CH;
    const size_t off = cbase + (size_t)fslot * p.kv_dim + h * HD;
#pragma unroll
    for (int j = 0; j < DPT; ++j) {
      const int d = tid + 256 * j;
      if (d < HD) {
        const float kv = rope_mix(p, d, kx[j], ky[j], kc_[j], ks_[j]);
        sk[kf * HD + d] = kv;
        sv[kf * HD + d] = vx[j];
        if (p.write_cache) {
          p.kc[off + d] = kv;
          p.vc[off + d] = vx[j];
        }
      }
    }
  }
  __syncthreads();

  // ---- scores: thread (key kk, dim group dg of 16 lanes), row sums by DPP
  const int kk = tid >> 4, dg = tid & 15;
  float acc[TGM];
#pragma unroll
  for (int i = 0; i < TGM; ++i) acc[i] = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int d = dg * 4 + 64 * i;
    const float4 kv = *reinterpret_cast<const float4 *>(sk + kk * HD + d);
#pragma unroll
    for (int t = 0; t < TGM; ++t) {
      const float4 qq = *reinterpret_cast<const float4 *>(sq + t * HD + d);
      acc[t] += qq.x * kv.x + qq.y * kv.y + qq.z * kv.z + qq.w * kv.w;
    }
  }
#pragma unroll
  for (int t = 0; t < TGM; ++t) acc[t] = row16_sum(acc[t]);
  if (dg == 0) {
    const bool ok = c * CH + kk < nslots;
#pragma unroll
    for (int t = 0; t < TGM; ++t)
      if (t < G) ss[t * CH + kk] = ok ? acc[t] * p.scale : -INFINITY;
  }
  __syncthreads();
  // softmax of the chunk: query head t on a 16-lane row, lane = key
  for (int t = tid >> 4; t < G; t += 16) {
    const int k = tid & 15;
    const float sc = ss[t * CH + k];
    const float m = row16_max(sc);
    const float pr = (sc == -INFINITY) ? 0.f : expf(sc - m);
    const float l = row16_sum(pr);
    ss[t * CH + k] = pr;
    if (k == 0) {
      sm[t] = m;
      sl[t] = l;
    }
  }
  __syncthreads();

  // ---- P.V of the chunk on float4 units (head t, dims 4u..4u+3).  Partials:
  // o [n_chunks][G][HD] then (max, sum) [n_chunks][G][2] per (sequence, kv
  // head), written with agent-coherent (sc1) stores
  constexpr int H4 = HD / 4;
  const int nu = G * H4;
  const size_t bh_stride = ((size_t)p.n_chunks * G * (HD + 2) + 3) & ~(size_t)3;
  float *po = p.part + (size_t)(b * p.n_kv + h) * bh_stride;
  float *pml = po + (size_t)p.n_chunks * G * HD;
  const __amdgpu_buffer_rsrc_t rs_o =
      __builtin_amdgcn_make_buffer_rsrc(po, 0, p.n_chunks * G * HD * 4, 0x00020000);
  float *orow = p.out + (size_t)b * p.q_dim + h * G * HD;
  const float4 *sv4 = reinterpret_cast<const float4 *>(sv);
  for (int u = tid; u < nu; u += 256) {
    const int t = u / H4, d4 = u % H4;
    af32x4 o = af32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < CH; ++k) {
      const float pk = ss[t * CH + k];
      const float4 v = sv4[k * H4 + d4];
      o.x += pk * v.x;
      o.y += pk * v.y;
      o.z += pk * v.z;
      o.w += pk * v.w;
    }
    if (n_active == 1) {
      // the only chunk: weight 1 / sum, as in the merge
      const float w = 1.0f / sl[t];
      *reinterpret_cast<float4 *>(orow + 4 * u) = float4{o.x * w, o.y * w, o.z * w, o.w * w};
    } else {
      __builtin_amdgcn_raw_buffer_store_b128(o, rs_o, ((c * G + t) * HD + 4 * d4) * 4, 0,
                                             kSc1);
    }
  }
  if (n_active == 1) return;
  if (tid < G) {
    st_agent(pml + (c * G + tid) * 2, sm[tid]);
    st_agent(pml + (c * G + tid) * 2 + 1, sl[tid]);
  }

  // ---- count this block done; the last one merges.  The block's partial
  // stores complete (device-scope stores, waited for), the barrier orders
  // every thread's stores before thread 0's increment, and the increment is
  // an agent-scope release + acquire: a block that sees the count reach
  // n_active reads the other blocks' partials after their releases: the
  // acquire invalidates this CU's stale cache lines, and the barrier after it
  // orders every thread's loads after the acquire, so ordinary loads see the
  // partials (device-scope loads were no faster).
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
  __syncthreads();
  if (tid == 0) {
    unsigned *ctr = p.ctr + b * p.n_kv + h;
    const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    const int last = old + 1 == (unsigned)n_active;
    if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;

  // The merge.  Each thread owns UPT float4 units (head t, dims 4d4..) and
  // issues the loads of its o partials for the first CB chunks before the
  // (max, sum) pairs are read (buffer loads), so both arrive
  // in one memory round trip.  Wave w turns the pairs of heads w, w+4, .. into
  // chunk weights e^(m_c - M) / sum_c e^(m_c - M) l_c (lanes over chunks),
  // shared through LDS; then o = sum_c w_c o_c.  Chunks past the first CB (long
  // linear caches) follow in further batches.
  // NUG unit groups of 256 * UPT units: more than one only at head dim 512
  // with more than 16 query heads per kv head (the first group's loads go out
  // before the weights, later groups' after them).
  constexpr int UPT = dec_units_per_thread(HD, TGM);
  constexpr int CB = dec_merge_batch(UPT);
  constexpr int NUG = (TGM * HD / 4 + 256 * UPT - 1) / (256 * UPT);
  int u0 = tid * UPT;
  int t0 = u0 / H4, d40 = u0 % H4;
  af32x4 ov[CB][UPT];
  auto load_o = [&](int c0) {
#pragma unroll
    for (int j = 0; j < CB; ++j) {
      // (block-uniform condition: chunks past the last are not loaded and
      // get weight 0)
      const int cc = c0 + j;
#pragma unroll
      for (int k = 0; k < UPT; ++k)
        ov[j][k] = cc < n_active ? __builtin_amdgcn_raw_buffer_load_b128(
                                       rs_o, ((cc * G + t0) * HD + 4 * (d40 + k)) * 4, 0, 0)
                                 : af32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  if (u0 < nu) load_o(0);
  const __amdgpu_buffer_rsrc_t rs_ml =
      __builtin_amdgcn_make_buffer_rsrc(pml, 0, p.n_chunks * G * 2 * 4, 0x00020000);
  const int wave = tid >> 6, lane = tid & 63;
  constexpr int MPL = kAttnMaxChunks / 64;  // chunks per lane
  for (int g = wave; g < G; g += 4) {
    float mc[MPL], lc[MPL];
#pragma unroll
    for (int i = 0; i < MPL; ++i) {
      const int cc = lane + 64 * i;
      mc[i] = -INFINITY;
      lc[i] = 0.f;
      if (cc < n_active) {
        const float2 v = __builtin_bit_cast(
            float2, __builtin_amdgcn_raw_buffer_load_b64(rs_ml, (cc * G + g) * 8, 0, 0));
        mc[i] = v.x;
        lc[i] = v.y;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < MPL; ++i) mx = fmaxf(mx, mc[i]);
    const float M = wave64_max(mx);
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < MPL; ++i) {
      mc[i] = (mc[i] == -INFINITY) ? 0.f : expf(mc[i] - M);
      part += lc[i] * mc[i];
    }
    const float inv = 1.0f / wave64_sum(part);
#pragma unroll
    for (int i = 0; i < MPL; ++i) {
      const int cc = lane + 64 * i;
      if (cc < n_active) wsh[cc * G + g] = mc[i] * inv;
    }
  }
  __syncthreads();
#pragma unroll
  for (int ug = 0; ug < NUG; ++ug) {
    if (ug > 0) {
      u0 = (tid + 256 * ug) * UPT;
      t0 = u0 / H4;
      d40 = u0 % H4;
    }
    if (u0 >= nu) return;
    float4 oacc[UPT];
#pragma unroll
    for (int k = 0; k < UPT; ++k) oacc[k] = float4{0.f, 0.f, 0.f, 0.f};
    for (int c0 = 0; c0 < n_active; c0 += CB) {
      if (c0 > 0 || ug > 0) load_o(c0);
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        const float w = c0 + j < n_active ? wsh[(c0 + j) * G + t0] : 0.f;
#pragma unroll
        for (int k = 0; k < UPT; ++k) {
          oacc[k].x += w * ov[j][k].x;
          oacc[k].y += w * ov[j][k].y;
          oacc[k].z += w * ov[j][k].z;
          oacc[k].w += w * ov[j][k].w;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < UPT; ++k)
      if (u0 + k < nu) *reinterpret_cast<float4 *>(orow + 4 * (u0 + k)) = oacc[k];
  }
}

// ------------------------------------------------------------------------------
// k_attn_part: the decode attention of one row per sequence without the merge.
// Block (c, b x h), 1024 threads: cache slots 32c..32c+31 of sequence b, kv
// head h, for its G <= 4 query heads.  The chunk's cached rows, q, the fresh
// k, v and the RoPE factors prepared for the position are loaded before the
// position arrives (branch-free range-checked loads; the host launches only
// the chunks below its bound on the position); rows past the attended ones
// are zeroed and the slot of the current position takes the fresh row (and
// appends it to the cache).  Thread t holds dims of key t / 32 (32 lanes per
// key, coalesced 16-byte pieces): the scores are its partial dots summed over
// the key's lanes, then the chunk's softmax numerators (max and sum over its
// keys), and o = sum_k e^(s_k - m) v_k over groups of keys (V through LDS),
// stored with (m, l) per query head.  The consumer (the O projection) merges
// the chunks, so no block waits for another.  Sixteen waves keep every SIMD
// busy and every dependent step short.
// ------------------------------------------------------------------------------
template <int HD, int GQ, bool MRG>
__global__ __launch_bounds__(1024) void k_attn_part(AttnArgs args) {
  extern __shared__ __align__(16) float lds[];
  __shared__ int s_last;
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  constexpr int CH = kDecPartChunk;
  static_assert(CH == 32, "32 keys per chunk: one key per 32 lanes");
  constexpr int NT = 1024;
  constexpr int H4 = HD / 4;
  constexpr int NF = HD / 128;                  // float4 of a key row per thread
  constexpr int QPT = (GQ * HD + NT - 1) / NT;   // q elements per thread (staging)
  constexpr int NU = GQ * H4;                   // P.V float4 units (head, dims)
  constexpr int NKG = NT / NU;                  // key groups of the P.V sums
  constexpr int KPG = CH / NKG;                 // keys per group
  static_assert(NF >= 1 && NKG >= 1 && CH % NKG == 0, "head dim 256 or 512");
  constexpr uint32_t kOut = 0x80000000u;
  const AttnP p = load_params(args);
  const int tid = threadIdx.x;
  const int c = blockIdx.x;
  const int G = p.G;
  // blockIdx.y = (b n_kv + h) NS + s: query heads s GQ .. s GQ + GQ - 1 of
  // kv head h (the G heads of a kv head split over NS blocks)
  const int NS = G > GQ ? G / GQ : 1;
  const int s = (int)blockIdx.y % NS, bh = (int)blockIdx.y / NS;
  const int b = bh / p.n_kv, h = bh % p.n_kv;
  const int g0 = s * GQ;                 // first query head of the block
  const int Gl = min(GQ, G - g0);        // its query heads
  const int L = p.cache_len;
  const int nq = Gl * HD;
  const int key = tid >> 5, j = tid & 31;

  float *sv = lds;               // [CH][HD] values
  float *sq = sv + CH * HD;      // [GQ][HD] rotated queries
  float *sf = sq + GQ * HD;      // [HD] fresh key, rotated
  float *ss = sf + HD;           // [GQ][CH] scores -> numerators
  float *sm = ss + GQ * CH;      // [GQ]
  float *sl = sm + 4;            // [GQ]
  float4 *so = reinterpret_cast<float4 *>(sl + 4);  // [NKG][NU] partial o
  const size_t cbase = (size_t)b * p.cache_seq_stride;
  const float *qrow = p.qkv + (size_t)b * p.ld;

  // ---- loads that do not depend on the position
  const int base = aldg_lane<int32_t>(p.pos + b);
  const uint32_t cbytes = (uint32_t)L * (uint32_t)p.kv_dim * 4u;
  const __amdgpu_buffer_rsrc_t rk =
      __builtin_amdgcn_make_buffer_rsrc(p.kc + cbase, 0, cbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv =
      __builtin_amdgcn_make_buffer_rsrc(p.vc + cbase, 0, cbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(qrow), 0, (uint32_t)p.ld * 4u, 0x00020000);
  const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(p.rope_cur), 0, (uint32_t)p.rot * 4u, 0x00020000);
  const int slot = c * CH + key;
  float4 kr[NF], vr[NF];
#pragma unroll
  for (int i = 0; i < NF; ++i) {
    const uint32_t off =
        slot < L ? ((uint32_t)slot * (uint32_t)p.kv_dim + (uint32_t)(h * HD + 4 * (i * 32 + j))) * 4u
                 : kOut;
    const f32x4 kv = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
    const f32x4 vv = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
    kr[i] = float4{kv.x, kv.y, kv.z, kv.w};
    vr[i] = float4{vv.x, vv.y, vv.z, vv.w};
  }
  auto ld1 = [&](const __amdgpu_buffer_rsrc_t &r, bool on, int idx) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(r, on ? (uint32_t)idx * 4u : kOut, 0, 0));
  };
  // q element e = tid + NT u: head e / HD, dim e % HD; its RoPE partner and
  // factors
  float qx[QPT], qy[QPT], qc[QPT], qs[QPT];
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int e = tid + NT * u;
    const int g = e / HD, d = e % HD;
    const int q0 = (h * G + g0 + g) * HD;
    const bool on = e < nq;
    qx[u] = ld1(rq, on, q0 + d);
    qy[u] = ld1(rq, on, q0 + rope_partner(p, d));
    if constexpr (!MRG) {
      const bool rot = p.apply_rope && d < p.rot;
      const int ri = d < p.half ? d : d - p.half;
      const float cv = ld1(rr, rot, ri);
      qs[u] = ld1(rr, rot, p.half + ri);
      qc[u] = rot ? cv : 1.f;
    }
  }
  // fresh k, v: dim tid (threads below HD)
  const int df = tid < HD ? tid : 0;
  const int k0 = p.q_dim + h * HD;
  const float kx = ld1(rq, tid < HD, k0 + df);
  const float ky = ld1(rq, tid < HD, k0 + rope_partner(p, df));
  const float vx = ld1(rq, tid < HD, p.q_dim + p.kv_dim + h * HD + df);
  float kc_ = 1.f, ks_ = 0.f;
  if constexpr (!MRG) {
    const bool krot = p.apply_rope && df < p.rot;
    const int kri = df < p.half ? df : df - p.half;
    const float kcv = ld1(rr, krot, kri);
    ks_ = ld1(rr, krot, p.half + kri);
    kc_ = krot ? kcv : 1.f;
  }
  // every load above goes out here, before the position arrives (the
  // compiler would otherwise sink the fresh row's loads past the position
  // test into the block that uses them, one memory round trip later)
  asm volatile("" ::: "memory");

  // ---- the position: attended slots [0, nslots), the slot of this row
  int lo, hi;
  key_range(p, base, &lo, &hi);
  const int nslots = p.circular ? min(L, base + 1) : min(hi + 1, L);
  const int n_active = min((nslots + CH - 1) / CH, p.grid_chunks);
  if (c >= n_active) return;
  const int fslot = p.circular ? base % L : base;
  const bool fresh_here = fslot < nslots && fslot / CH == c;
  const int kf = fslot - c * CH;  // key of the fresh row in this chunk
  const bool own_fresh = fresh_here && key == kf;
  if constexpr (MRG) {
    // the RoPE factors of this sequence's position, from the tables
#pragma unroll
    for (int u = 0; u < QPT; ++u) rope_cs(p, (tid + NT * u) % HD, base, qc[u], qs[u]);
    if (fresh_here) rope_cs(p, df, base, kc_, ks_);
  }
  if (slot >= nslots) {
#pragma unroll
    for (int i = 0; i < NF; ++i) {
      kr[i] = float4{0.f, 0.f, 0.f, 0.f};
      vr[i] = float4{0.f, 0.f, 0.f, 0.f};
    }
  }
  if (!own_fresh) {
#pragma unroll
    for (int i = 0; i < NF; ++i)
      *reinterpret_cast<float4 *>(sv + key * HD + 4 * (i * 32 + j)) = vr[i];
  }
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int e = tid + NT * u;
    if (e < GQ * HD) sq[e] = e < nq ? rope_mix(p, e % HD, qx[u], qy[u], qc[u], qs[u]) : 0.f;
  }
  if (fresh_here && tid < HD) {
    // write_kv_sliding / write_kv_full (gemma4_e4b.mojo:211-249)
    const float kv = rope_mix(p, tid, kx, ky, kc_, ks_);
    sf[tid] = kv;
    sv[kf * HD + tid] = vx;
    if (p.write_cache && s == 0) {
      const size_t off = cbase + (size_t)fslot * p.kv_dim + h * HD + tid;
      p.kc[off] = kv;
      p.vc[off] = vx;
    }
  }
  __syncthreads();

  // ---- scores: the thread's dims of its key against the G queries, summed
  // over the key's 32 lanes
  if (own_fresh) {
#pragma unroll
    for (int i = 0; i < NF; ++i) kr[i] = *reinterpret_cast<const float4 *>(sf + 4 * (i * 32 + j));
  }
  float acc[GQ];
#pragma unroll
  for (int t = 0; t < GQ; ++t) {
    acc[t] = 0.f;
#pragma unroll
    for (int i = 0; i < NF; ++i) {
      const float4 qq = *reinterpret_cast<const float4 *>(sq + t * HD + 4 * (i * 32 + j));
      acc[t] += qq.x * kr[i].x + qq.y * kr[i].y + qq.z * kr[i].z + qq.w * kr[i].w;
    }
    acc[t] = row16_sum(acc[t]);
    acc[t] += __shfl_xor(acc[t], 16, 64);
  }
  if (j == 0) {
    const bool ok = slot < nslots;
#pragma unroll
    for (int t = 0; t < GQ; ++t)
      if (t < Gl) ss[t * CH + key] = ok ? acc[t] * p.scale : -INFINITY;
  }
  __syncthreads();
  // numerators of the chunk: query head t on CH lanes, lane = key; max and
  // sum over the chunk's keys (a row of 16 by DPP, two rows by one exchange)
  if (tid < CH * GQ) {
    const int t = tid / CH, k = tid % CH;
    const float sc = t < Gl ? ss[t * CH + k] : -INFINITY;
    float m = row16_max(sc);
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    const float pr = (sc == -INFINITY) ? 0.f : expf(sc - m);
    float l = row16_sum(pr);
    l += __shfl_xor(l, 16, 64);
    if (t < Gl) {
      ss[t * CH + k] = pr;
      if (k == 0) {
        sm[t] = m;
        sl[t] = l;
      }
    }
  }
  __syncthreads();

  // ---- P.V: unit u = (head t, dims 4d4..4d4+3) over key group kq
  const int u = tid % NU, kq = tid / NU;
  const int t = u / H4, d4 = u % H4;
  {
    const float4 *sv4 = reinterpret_cast<const float4 *>(sv);
    float4 o = float4{0.f, 0.f, 0.f, 0.f};
    if (t < Gl) {
#pragma unroll
      for (int k = kq * KPG; k < kq * KPG + KPG; ++k) {
        const float pk = ss[t * CH + k];
        const float4 v = sv4[k * H4 + d4];
        o.x += pk * v.x;
        o.y += pk * v.y;
        o.z += pk * v.z;
        o.w += pk * v.w;
      }
    }
    so[kq * NU + u] = o;
  }
  __syncthreads();
  const int nhq = p.n_heads;
  float *po = p.part + (size_t)b * kDecPartMaxChunks * nhq * (HD + 2);
  float *pml = po + (size_t)kDecPartMaxChunks * nhq * HD;
  f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
  if (tid < NU && t < Gl) {
#pragma unroll
    for (int g = 0; g < NKG; ++g) {
      const float4 w = so[g * NU + u];
      o += f32x4{w.x, w.y, w.z, w.w};
    }
  }
  if constexpr (!MRG) {
    if (tid < NU && t < Gl)
      *reinterpret_cast<float4 *>(po + ((size_t)c * nhq + h * G + g0 + t) * HD + 4 * d4) =
          float4{o.x, o.y, o.z, o.w};
    if (tid < Gl)
      *reinterpret_cast<float2 *>(pml + ((size_t)c * nhq + h * G + g0 + tid) * 2) =
          float2{sm[tid], sl[tid]};
    return;
  } else {
    // MRG: the chunks merged here, into out [B][q_dim]
    float *orow = p.out + (size_t)b * p.q_dim + (h * G + g0) * HD;
    if (n_active == 1) {
      // the only chunk: o / l, as the merge would form it
      if (tid < NU && t < Gl) {
        const float w = 1.0f / sl[t];
        *reinterpret_cast<float4 *>(orow + t * HD + 4 * d4) =
            float4{o.x * w, o.y * w, o.z * w, o.w * w};
      }
      return;
    }
    const __amdgpu_buffer_rsrc_t rs_o = __builtin_amdgcn_make_buffer_rsrc(
        po, 0, (uint32_t)(kDecPartMaxChunks * nhq * HD * 4), 0x00020000);
    if (tid < NU && t < Gl)
      __builtin_amdgcn_raw_buffer_store_b128(
          o, rs_o, ((c * nhq + h * G + g0 + t) * HD + 4 * d4) * 4, 0, kSc1);
    if (tid < Gl) {
      st_agent(pml + (c * nhq + h * G + g0 + tid) * 2, sm[tid]);
      st_agent(pml + (c * nhq + h * G + g0 + tid) * 2 + 1, sl[tid]);
    }
    // count this block done; the last block of (sequence, kv head, head pair)
    // merges (k_attn_decode's protocol: device-scope partial stores waited
    // for, a barrier, an agent-scope release + acquire increment; the last
    // block reads the partials after the others' releases and resets the
    // counter for the next launch)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      unsigned *ctr = p.ctr + ((size_t)b * p.n_kv + h) * NS + s;
      const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
      const int last = old + 1 == (unsigned)n_active;
      if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    // log-sum-exp over the chunks: thread (unit u, chunk group kq) sums
    // w_c o_c over chunks kq, kq + NKG, ..; its first batch of o partials is
    // loaded before the weights are formed.  Wave t < Gl turns query head t's
    // (m, l) pairs into w_c = e^(m_c - M) (one chunk per lane) and 1 / sum_c
    // l_c w_c.  The group sums meet through LDS.
    constexpr int MB = 4;  // chunks per thread per load batch
    const __amdgpu_buffer_rsrc_t rs_ml = __builtin_amdgcn_make_buffer_rsrc(
        pml, 0, (uint32_t)(kDecPartMaxChunks * nhq * 2 * 4), 0x00020000);
    const uint32_t ou = ((h * G + g0 + (t < Gl ? t : 0)) * HD + 4 * d4) * 4;
    f32x4 ov[MB];
    auto load_o = [&](int c0) {
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        const int cc = c0 + NKG * i;
        ov[i] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       rs_o, cc < n_active ? (uint32_t)cc * nhq * HD * 4 + ou : kOut, 0, 0));
      }
    };
    load_o(kq);
    float *wsh = sq;   // [kDecPartMaxChunks][GQ] chunk weights (queries no longer read)
    float *sinv = sm;  // [GQ] 1 / l
    const int wave = tid >> 6, lane = tid & 63;
    static_assert(kDecPartMaxChunks == 64, "one chunk per lane");
    if (wave < Gl) {
      const bool on = lane < n_active;
      const f32x2 ml = __builtin_bit_cast(
          f32x2, __builtin_amdgcn_raw_buffer_load_b64(
                     rs_ml, on ? (uint32_t)(lane * nhq + h * G + g0 + wave) * 8 : kOut, 0, 0));
      const float M = wave64_max(on ? ml.x : -INFINITY);
      const float w = on ? expf(ml.x - M) : 0.f;
      const float l = wave64_sum(on ? ml.y * w : 0.f);
      wsh[lane * GQ + wave] = w;
      if (lane == 0) sinv[wave] = 1.0f / l;
    }
    __syncthreads();
    f32x4 oa = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int c0 = kq; c0 < n_active; c0 += NKG * MB) {
      if (c0 != kq) load_o(c0);
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        const int cc = c0 + NKG * i;
        const float w = cc < n_active && t < Gl ? wsh[cc * GQ + t] : 0.f;
        oa += w * ov[i];
      }
    }
    so[kq * NU + u] = float4{oa.x, oa.y, oa.z, oa.w};
    __syncthreads();
    if (tid < NU && t < Gl) {
      f32x4 r = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < NKG; ++q) {
        const float4 w = so[q * NU + u];
        r += f32x4{w.x, w.y, w.z, w.w};
      }
      const float inv = sinv[t];
      *reinterpret_cast<float4 *>(orow + t * HD + 4 * d4) =
          float4{r.x * inv, r.y * inv, r.z * inv, r.w * inv};
    }
  }
}

// ------------------------------------------------------------------------------
// k_attn_rows: T = 2..4 rows of one sequence at positions base .. base + T - 1
// on a linear cache (a harness step of a few rows), the decode chunk scheme
// per row.  Block (c, (t n_kv + h) NS + s), 1024 threads: cache slots
// 32c..32c+31 for row t and query heads s GQ .. s GQ + GQ - 1 of kv head h.
// Slots base .. base + t are this call's rows 0 .. t: their keys and values
// come from the q|k|v rows (rotated here), never from the cache, which the
// block of row t' writes at slot base + t' (head split 0 only), so no block
// reads a slot another block writes.  Slots past base + t are masked.  The
// chunk's (o, m, l) per query head go to the row's partials (region t), which
// k_attn_rows_merge combines.
// ------------------------------------------------------------------------------
constexpr int kRowsMax = 4;

template <int HD, int GQ>
__global__ __launch_bounds__(1024) void k_attn_rows(AttnArgs args) {
  extern __shared__ __align__(16) float lds[];
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  constexpr int CH = kDecPartChunk;
  static_assert(CH == 32, "32 keys per chunk: one key per 32 lanes");
  constexpr int NT = 1024;
  constexpr int H4 = HD / 4;
  constexpr int NF = HD / 128;                        // float4 of a key row per thread
  constexpr int QPT = (GQ * HD + NT - 1) / NT;         // q elements per thread
  constexpr int FPT = (kRowsMax * HD + NT - 1) / NT;   // fresh row elements per thread
  constexpr int NU = GQ * H4;
  constexpr int NKG = NT / NU;
  constexpr int KPG = CH / NKG;
  static_assert(NF >= 1 && NKG >= 1 && CH % NKG == 0, "head dim 128, 256 or 512");
  constexpr uint32_t kOut = 0x80000000u;
  const AttnP p = load_params(args);
  const int tid = threadIdx.x;
  const int c = blockIdx.x;
  const int G = p.G, T = p.T;
  const int NS = G > GQ ? G / GQ : 1;
  const int s = (int)blockIdx.y % NS, r = (int)blockIdx.y / NS;
  const int h = r % p.n_kv, t = r / p.n_kv;
  const int g0 = s * GQ, Gl = min(GQ, G - g0);
  const int L = p.cache_len;
  const int nq = Gl * HD;
  const int key = tid >> 5, j = tid & 31;

  float *sv = lds;                      // [CH][HD] values
  float *sq = sv + CH * HD;             // [GQ][HD] rotated queries
  float *sf = sq + GQ * HD;             // [kRowsMax][HD] this call's keys, rotated
  float *ss = sf + kRowsMax * HD;       // [GQ][CH] scores -> numerators
  float *sm = ss + GQ * CH;             // [GQ]
  float *sl = sm + 4;                   // [GQ]
  float4 *so = reinterpret_cast<float4 *>(sl + 4);  // [NKG][NU] partial o

  // ---- loads that do not depend on the position (branch-free, range-checked)
  const int base = aldg_lane<int32_t>(p.pos);
  const uint32_t cbytes = (uint32_t)L * (uint32_t)p.kv_dim * 4u;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(p.kc, 0, cbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(p.vc, 0, cbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(p.qkv), 0, (uint32_t)(T * p.ld) * 4u, 0x00020000);
  const int slot = c * CH + key;
  float4 kr[NF], vr[NF];
#pragma unroll
  for (int i = 0; i < NF; ++i) {
    const uint32_t off =
        slot < L ? ((uint32_t)slot * (uint32_t)p.kv_dim + (uint32_t)(h * HD + 4 * (i * 32 + j))) * 4u
                 : kOut;
    const f32x4 kv = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0));
    const f32x4 vv = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0));
    kr[i] = float4{kv.x, kv.y, kv.z, kv.w};
    vr[i] = float4{vv.x, vv.y, vv.z, vv.w};
  }
  auto ld1 = [&](const __amdgpu_buffer_rsrc_t &rs, bool on, int idx) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(rs, on ? (uint32_t)idx * 4u : kOut, 0, 0));
  };
  float qx[QPT], qy[QPT];
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int e = tid + NT * u;
    const int g = e / HD, d = e % HD;
    const int q0 = t * p.ld + (h * G + g0 + g) * HD;
    qx[u] = ld1(rq, e < nq, q0 + d);
    qy[u] = ld1(rq, e < nq, q0 + rope_partner(p, d));
  }
  // this call's keys and values: element e = (row e / HD, dim e % HD)
  float kx[FPT], ky[FPT], vx[FPT];
#pragma unroll
  for (int u = 0; u < FPT; ++u) {
    const int e = tid + NT * u;
    const int tf = e / HD, d = e % HD;
    const bool on = tf < T;
    const int k0 = tf * p.ld + p.q_dim + h * HD;
    kx[u] = ld1(rq, on, k0 + d);
    ky[u] = ld1(rq, on, k0 + rope_partner(p, d));
    vx[u] = ld1(rq, on, tf * p.ld + p.q_dim + p.kv_dim + h * HD + d);
  }
  asm volatile("" ::: "memory");

  // ---- the position: row t attends slots [0, base + t]
  const int pos_t = base + t;
  const int nslots = min(pos_t + 1, L);
  const int n_active = min((nslots + CH - 1) / CH, p.grid_chunks);
  if (c >= n_active) return;
  // RoPE factors of row t (queries) and of this call's rows (keys)
  float qc[QPT], qs[QPT];
#pragma unroll
  for (int u = 0; u < QPT; ++u) rope_cs(p, (tid + NT * u) % HD, pos_t, qc[u], qs[u]);
  const bool own_fresh = slot >= base && slot < nslots;
  if (slot >= nslots) {
#pragma unroll
    for (int i = 0; i < NF; ++i) {
      kr[i] = float4{0.f, 0.f, 0.f, 0.f};
      vr[i] = float4{0.f, 0.f, 0.f, 0.f};
    }
  }
  if (!own_fresh) {
#pragma unroll
    for (int i = 0; i < NF; ++i)
      *reinterpret_cast<float4 *>(sv + key * HD + 4 * (i * 32 + j)) = vr[i];
  }
#pragma unroll
  for (int u = 0; u < QPT; ++u) {
    const int e = tid + NT * u;
    if (e < GQ * HD) sq[e] = e < nq ? rope_mix(p, e % HD, qx[u], qy[u], qc[u], qs[u]) : 0.f;
  }
#pragma unroll
  for (int u = 0; u < FPT; ++u) {
    const int e = tid + NT * u;
    const int tf = e / HD, d = e % HD;
    const int sf_slot = base + tf;  // rows 0 .. t of this call in this chunk
    if (tf <= t && sf_slot >= c * CH && sf_slot < c * CH + CH) {
      float cs, sn;
      rope_cs(p, d, sf_slot, cs, sn);
      // write_kv_full (gemma4_e4b.mojo:211-249)
      const float kv = rope_mix(p, d, kx[u], ky[u], cs, sn);
      sf[tf * HD + d] = kv;
      sv[(sf_slot - c * CH) * HD + d] = vx[u];
      if (p.write_cache && tf == t && s == 0) {
        const size_t off = (size_t)sf_slot * p.kv_dim + h * HD + d;
        p.kc[off] = kv;
        p.vc[off] = vx[u];
      }
    }
  }
  __syncthreads();

  // ---- scores, numerators, P.V (as k_attn_part)
  if (own_fresh) {
#pragma unroll
    for (int i = 0; i < NF; ++i)
      kr[i] = *reinterpret_cast<const float4 *>(sf + (slot - base) * HD + 4 * (i * 32 + j));
  }
  float acc[GQ];
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
    acc[g] = 0.f;
#pragma unroll
    for (int i = 0; i < NF; ++i) {
      const float4 qq = *reinterpret_cast<const float4 *>(sq + g * HD + 4 * (i * 32 + j));
      acc[g] += qq.x * kr[i].x + qq.y * kr[i].y + qq.z * kr[i].z + qq.w * kr[i].w;
    }
    acc[g] = row16_sum(acc[g]);
    acc[g] += __shfl_xor(acc[g], 16, 64);
  }
  if (j == 0) {
    const bool ok = slot < nslots;
#pragma unroll
    for (int g = 0; g < GQ; ++g)
      if (g < Gl) ss[g * CH + key] = ok ? acc[g] * p.scale : -INFINITY;
  }
  __syncthreads();
  if (tid < CH * GQ) {
    const int g = tid / CH, k = tid % CH;
    const float sc = g < Gl ? ss[g * CH + k] : -INFINITY;
    float m = row16_max(sc);
    m = fmaxf(m, __shfl_xor(m, 16, 64));
    const float pr = (sc == -INFINITY) ? 0.f : expf(sc - m);
    float l = row16_sum(pr);
    l += __shfl_xor(l, 16, 64);
    if (g < Gl) {
      ss[g * CH + k] = pr;
      if (k == 0) {
        sm[g] = m;
        sl[g] = l;
      }
    }
  }
  __syncthreads();
  const int u = tid % NU, kq = tid / NU;
  const int g = u / H4, d4 = u % H4;
  {
    const float4 *sv4 = reinterpret_cast<const float4 *>(sv);
    float4 o = float4{0.f, 0.f, 0.f, 0.f};
    if (g < Gl) {
#pragma unroll
      for (int k = kq * KPG; k < kq * KPG + KPG; ++k) {
        const float pk = ss[g * CH + k];
        const float4 v = sv4[k * H4 + d4];
        o.x += pk * v.x;
        o.y += pk * v.y;
        o.z += pk * v.z;
        o.w += pk * v.w;
      }
    }
    so[kq * NU + u] = o;
  }
  __syncthreads();
  const int nhq = p.n_heads;
  float *po = p.part + (size_t)t * kDecPartMaxChunks * nhq * (HD + 2);
  float *pml = po + (size_t)kDecPartMaxChunks * nhq * HD;
  if (tid < NU && g < Gl) {
    float4 o = so[u];
#pragma unroll
    for (int q = 1; q < NKG; ++q) {
      const float4 w = so[q * NU + u];
      o.x += w.x;
      o.y += w.y;
      o.z += w.z;
      o.w += w.w;
    }
    *reinterpret_cast<float4 *>(po + ((size_t)c * nhq + h * G + g0 + g) * HD + 4 * d4) = o;
  }
  if (tid < Gl)
    *reinterpret_cast<float2 *>(pml + ((size_t)c * nhq + h * G + g0 + tid) * 2) =
        float2{sm[tid], sl[tid]};
}

// The chunks of k_attn_rows merged per (query head, row) (log-sum-exp over
// the chunks the row attends): out [T][q_dim].  One block per (query head,
// row), max(64, HD / 4) threads, a float4 of dims each.  Every load goes out
// at entry: the position, lane c's (m, l) of chunk c, and the o partials of
// the first kMergeBatch chunks (range-checked buffer loads: chunks past the
// launched ones read zeros without a memory access).  The weights
// w_c = e^(m_c - M) and l = sum_c l_c w_c come from wave reductions; chunks
// past the row's last attended one are dropped by selects, so a stale
// partial never enters the sum.
constexpr int kMergeBatch = 8;
template <int HD>
__global__ __launch_bounds__(128) void k_attn_rows_merge(AttnArgs args) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  constexpr int H4 = HD / 4;
  const int hq = blockIdx.x, t = blockIdx.y, d4 = threadIdx.x, lane = threadIdx.x & 63;
  const int nhq = keep(args.n_heads), gc = keep(args.grid_chunks);
  const int cache_len = keep(args.cache_len), q_dim = keep(args.q_dim);
  const float *po = args.part + (size_t)t * kDecPartMaxChunks * nhq * (HD + 2);
  const float *pml = po + (size_t)kDecPartMaxChunks * nhq * HD;
  const int base = aldg_lane<int32_t>(args.pos);
  const __amdgpu_buffer_rsrc_t rml = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(pml), 0, gc * nhq * 8, 0x00020000);
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(po), 0, gc * nhq * HD * 4, 0x00020000);
  const f32x2 ml = __builtin_bit_cast(
      f32x2, __builtin_amdgcn_raw_buffer_load_b64(rml, (lane * nhq + hq) * 8, 0, 0));
  const int od = d4 < H4 ? 16 * d4 : 0;  // idle lanes re-read dims 0..3
  f32x4 v[kMergeBatch];
#pragma unroll
  for (int u = 0; u < kMergeBatch; ++u)
    v[u] = __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, (u * nhq + hq) * HD * 4 + od, 0, 0));
  const int nslots = min(base + t + 1, cache_len);
  const int n_act = min((nslots + kDecPartChunk - 1) / kDecPartChunk, gc);
  const bool on = lane < n_act;
  const float M = wave64_max(on ? ml.x : -INFINITY);
  const float w = on ? expf(ml.x - M) : 0.f;
  const float l = wave64_sum(on ? ml.y * w : 0.f);
  f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < kMergeBatch; ++u) {
    const float wu = lane_of(w, u);
    const f32x4 a = o + wu * v[u];
    o = u < n_act ? a : o;
  }
  for (int c0 = kMergeBatch; c0 < n_act; c0 += kMergeBatch) {
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u)
      v[u] = __builtin_bit_cast(
          f32x4, __builtin_amdgcn_raw_buffer_load_b128(ro, ((c0 + u) * nhq + hq) * HD * 4 + od,
                                                        0, 0));
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const float wu = lane_of(w, c0 + u);
      const f32x4 a = o + wu * v[u];
      o = c0 + u < n_act ? a : o;
    }
  }
  if (d4 < H4) {
    const float inv = 1.0f / l;
    *reinterpret_cast<float4 *>(args.out + (size_t)t * q_dim + hq * HD + 4 * d4) =
        float4{o.x * inv, o.y * inv, o.z * inv, o.w * inv};
  }
}

bool attn_rows_ok(const AttnArgs &a) {
  const int G = a.n_kv > 0 ? a.n_heads / a.n_kv : 0;
  return a.B == 1 && a.T >= 2 && a.T <= kRowsMax && G >= 1 && G <= 4 && G != 3 &&
         a.n_heads % a.n_kv == 0 && (a.hd == 128 || a.hd == 256 || a.hd == 512) &&
         a.rot % 2 == 0 && a.rot <= a.hd && a.cache_kind != MS_CACHE_CIRCULAR &&
         a.ld >= a.q_dim + 2 * a.kv_dim && a.pos_bound > 0 && a.pos_bound <= a.cache_len &&
         dec_part_chunks(a) <= kDecPartMaxChunks;
}

int launch_attention_rows(const AttnArgs &a, hipStream_t st) {
  MS_CHECK_ARG(attn_rows_ok(a), "attention rows: unsupported shape");
  MS_CHECK_ARG(a.qkv && a.part && a.pos && a.kc && a.vc && a.out && a.cos_t && a.sin_t,
               "attention rows: missing buffers");
  AttnArgs a2 = a;
  a2.grid_chunks = dec_part_chunks(a);
  constexpr int GQ = 2;
  const int G = a.n_heads / a.n_kv;
  const int ns = G > GQ ? G / GQ : 1;
  const dim3 grid(a2.grid_chunks, a.T * a.n_kv * ns);
  constexpr int CH = kDecPartChunk;
  const size_t shmem =
      (size_t)(CH * a.hd + GQ * a.hd + kRowsMax * a.hd + GQ * CH + 8) * 4 + 16384;
  if (a.hd == 128) hipLaunchKernelGGL((k_attn_rows<128, GQ>), grid, dim3(1024), shmem, st, a2);
  else if (a.hd == 256) hipLaunchKernelGGL((k_attn_rows<256, GQ>), grid, dim3(1024), shmem, st, a2);
  else hipLaunchKernelGGL((k_attn_rows<512, GQ>), grid, dim3(1024), shmem, st, a2);
  MS_HIP_TRY(hipGetLastError());
  const dim3 mgrid(a.n_heads, a.T);
  const int mthreads = a.hd / 4 < 64 ? 64 : a.hd / 4;
  if (a.hd == 128) hipLaunchKernelGGL(k_attn_rows_merge<128>, mgrid, dim3(mthreads), 0, st, a2);
  else if (a.hd == 256) hipLaunchKernelGGL(k_attn_rows_merge<256>, mgrid, dim3(mthreads), 0, st, a2);
  else hipLaunchKernelGGL(k_attn_rows_merge<512>, mgrid, dim3(mthreads), 0, st, a2);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

int dec_part_chunks(const AttnArgs &a) {
  const int reach = a.pos_bound > 0 ? std::min(a.pos_bound, a.cache_len) : a.cache_len;
  return std::max(1, (reach + kDecPartChunk - 1) / kDecPartChunk);
}

bool dec_part_ok(const AttnArgs &a) {
  const int G = a.n_kv > 0 ? a.n_heads / a.n_kv : 0;
  return a.T == 1 && G >= 1 && G <= 4 && G != 3 && a.n_heads % a.n_kv == 0 &&
         (a.hd == 256 || a.hd == 512) && a.rot % 2 == 0 && a.rot <= a.hd &&
         a.ld >= a.q_dim + 2 * a.kv_dim && dec_part_chunks(a) <= kDecPartMaxChunks;
}

// cos, sin rows of the tables at the position of sequence 0 (rope_table_host's
// angles, kernels.mojo:563-577), copied to a.rope_cur
__global__ __launch_bounds__(256) void k_rope_cur(AttnArgs args) {
  const int half = args.rot >> 1;
  const int pos = aldg<int32_t>(args.pos);
  float *o = const_cast<float *>(args.rope_cur);
  for (int i = threadIdx.x; i < half; i += 256) {
    o[i] = aldg<float>(args.cos_t + (size_t)pos * half + i);
    o[half + i] = aldg<float>(args.sin_t + (size_t)pos * half + i);
  }
}

int launch_rope_cur(const AttnArgs &a, hipStream_t st) {
  MS_CHECK_ARG(a.rope_cur && a.pos && a.cos_t && a.sin_t && a.rot >= 0,
               "rope factors: missing buffers");
  hipLaunchKernelGGL(k_rope_cur, dim3(1), dim3(256), 0, st, a);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

int launch_attention_partials(const AttnArgs &a, hipStream_t st, bool merge) {
  MS_CHECK_ARG(dec_part_ok(a), "attention partials: unsupported shape");
  MS_CHECK_ARG(a.qkv && a.part && a.pos && a.kc && a.vc &&
                   (merge ? a.ctr && a.out && a.cos_t && a.sin_t : a.rope_cur != nullptr),
               "attention partials: missing buffers");
  AttnArgs a2 = a;
  a2.grid_chunks = dec_part_chunks(a);
  // two query heads per block: the G heads of a kv head over G / 2 blocks
  constexpr int GQ = 2;
  const int G = a.n_heads / a.n_kv;
  const int ns = G > GQ ? G / GQ : 1;
  const dim3 grid(a2.grid_chunks, a.B * a.n_kv * ns);
  constexpr int CH = kDecPartChunk;
  // sv, sq, sf, ss, sm / sl (4 + 4 floats), so (16 KB at every head dim)
  const size_t shmem = (size_t)(CH * a.hd + GQ * a.hd + a.hd + GQ * CH + 8) * 4 + 16384;
  if (merge && G == 4) {
    // the merging kernel on all four query heads of a kv head per block (half
    // the blocks, each K/V row loaded once): batch 4 2,429 -> 2,436 tok/s
    constexpr int GQ4 = 4;
    const dim3 grid4(a2.grid_chunks, a.B * a.n_kv);
    const size_t shmem4 = (size_t)(CH * a.hd + GQ4 * a.hd + a.hd + GQ4 * CH + 8) * 4 + 16384;
    if (a.hd == 256) hipLaunchKernelGGL((k_attn_part<256, GQ4, true>), grid4, dim3(1024), shmem4, st, a2);
    else hipLaunchKernelGGL((k_attn_part<512, GQ4, true>), grid4, dim3(1024), shmem4, st, a2);
  } else if (merge) {
    if (a.hd == 256) hipLaunchKernelGGL((k_attn_part<256, GQ, true>), grid, dim3(1024), shmem, st, a2);
    else hipLaunchKernelGGL((k_attn_part<512, GQ, true>), grid, dim3(1024), shmem, st, a2);
  } else {
    if (a.hd == 256) hipLaunchKernelGGL((k_attn_part<256, GQ, false>), grid, dim3(1024), shmem, st, a2);
    else hipLaunchKernelGGL((k_attn_part<512, GQ, false>), grid, dim3(1024), shmem, st, a2);
  }
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

static size_t attn_decode_lds(const AttnArgs &a, int tgm) {
  const int G = a.n_heads / a.n_kv;
  return (size_t)(2 * kAttnChunk * a.hd + tgm * a.hd + tgm * kAttnChunk + 2 * tgm +
                  a.n_chunks * G) * 4;
}

static int launch_attention_decode(const AttnArgs &a, hipStream_t st) {
  MS_CHECK_ARG(a.ctr, "attention: decode needs the chunk counters");
  const int G = a.n_heads / a.n_kv;
  const int tgm = G <= 4 ? 4 : (G <= 8 ? 8 : kAttnMaxTG);
  AttnArgs a2 = a;
  const int reach = a.pos_bound > 0 ? std::min(a.pos_bound, a.cache_len) : a.cache_len;
  a2.grid_chunks = std::max(1, std::min(a.n_chunks, (reach + kAttnChunk - 1) / kAttnChunk));
  const dim3 grid(a2.grid_chunks, a.B * a.n_kv);
  const size_t shmem = attn_decode_lds(a, tgm);
#define MS_DEC(HDV)                                                                        \
  if (tgm == 4)                                                                            \
    hipLaunchKernelGGL((k_attn_decode<HDV, 4>), grid, dim3(256), shmem, st, a2);          \
  else if (tgm == 8)                                                                       \
    hipLaunchKernelGGL((k_attn_decode<HDV, 8>), grid, dim3(256), shmem, st, a2);          \
  else                                                                                     \
    hipLaunchKernelGGL((k_attn_decode<HDV, kAttnMaxTG>), grid, dim3(256), shmem, st, a2)
  switch (a.hd) {
    case 64: MS_DEC(64); break;
    case 128: MS_DEC(128); break;
    case 256: MS_DEC(256); break;
    default: MS_DEC(512); break;
  }
#undef MS_DEC
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

}  // namespace ms
