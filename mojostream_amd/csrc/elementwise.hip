// RMSNorm, PLE scale, SwiGLU, RoPE, embedding gather and the kernel-level
// attention / LM-head entry points.
#include <cmath>
#include <vector>

#include "attention.h"
#include "q4.h"
#include "rope.h"

namespace ms {

// rmsnorm_inplace / rmsnorm_weighted_inplace (kernels.mojo:474-489, :598-613):
// one block per row.
__global__ void k_rmsnorm(float *x, const float *gamma, int cols) {
  __shared__ float sh[16];
  float *rp = x + (size_t)blockIdx.x * cols;
  float ss = 0.f;
  for (int i = threadIdx.x; i < cols; i += kBlock) ss += rp[i] * rp[i];
  // block reduction
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = ss;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < (kBlock >> 6); ++w) t += sh[w];
  const float inv = 1.0f / sqrtf(t / (float)cols + 1e-6f);
  for (int i = threadIdx.x; i < cols; i += kBlock)
    rp[i] = gamma ? rp[i] * inv * gamma[i] : rp[i] * inv;
}

__global__ void k_scale(float *x, size_t n, float s) {
  const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) x[i] = x[i] * s;
}

// swiglu_inplace (kernels.mojo:519-532): up = up * gate * sigmoid(gate)
__global__ void k_swiglu(const float *gate, float *up, size_t n) {
  const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= n) return;
  const float g = gate[i];
  up[i] = up[i] * g * (1.0f / (1.0f + expf(-g)));
}

// apply_rope_inplace (kernels.mojo:579-595) with host-built tables
// cs/sn [rows][rot/2] (row r at position base_pos + r).
__global__ void k_rope(float *x, int rows, int row_stride, int n_heads, int head_stride,
                       int rot, const float *cs, const float *sn) {
  const int half = rot / 2;
  const long total = (long)rows * n_heads * half;
  const long i = (long)blockIdx.x * kBlock + threadIdx.x;
  if (i >= total) return;
  const int r = (int)(i / ((long)n_heads * half));
  const int hh = (int)((i / half) % n_heads);
  const int k = (int)(i % half);
  float *hp = x + (size_t)r * row_stride + (size_t)hh * head_stride;
  const float c = cs[(size_t)r * half + k], s = sn[(size_t)r * half + k];
  const float xi = hp[k], xih = hp[k + half];
  hp[k] = xi * c - xih * s;
  hp[k + half] = xi * s + xih * c;
}

// get_token_embedding Q4 branch (lm_head.mojo:186-195) from the panel layout.
__global__ void k_embed(const uint8_t *w, int D, int vocab, float scale,
                        const int32_t *tokens, int n, float *out) {
  const int i = blockIdx.x * kBlock + threadIdx.x;
  if (i >= n * D) return;
  const int r = i / D, k = i % D;
  const int tok = tokens[r];
  size_t byte;
  int hi;
  panel_locate(D, k, tok, &byte, &hi);
  const uint8_t b = w[byte];
  const int nib = hi ? (b >> 4) : (b & 15);
  out[i] = (float)(nib - 8) * scale;
}

int launch_embed(const uint8_t *w, int D, int vocab, float scale, const int32_t *tokens,
                 int n, float *out, hipStream_t st) {
  hipLaunchKernelGGL(k_embed, dim3(cdiv((long)n * D, kBlock)), dim3(kBlock), 0, st, w, D,
                     vocab, scale, tokens, n, out);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

// Host-side RoPE tables: the reference's fp32 formula (kernels.mojo:563-577):
// inv_freq_i = exp(-(2i)/rot * ln(theta)), angle = pos * inv_freq_i.
void rope_table_host(int rot, float theta, int pos0, int n_pos, std::vector<float> &cs,
                     std::vector<float> &sn) {
  const int half = rot / 2;
  cs.resize((size_t)n_pos * half);
  sn.resize((size_t)n_pos * half);
  const float ln_base = logf(theta);
  for (int p = 0; p < n_pos; ++p) {
    const float pos_f = (float)(pos0 + p);
    for (int i = 0; i < half; ++i) {
      const float inv_freq = expf(-(float)(2 * i) / (float)rot * ln_base);
      const float th = pos_f * inv_freq;
      cs[(size_t)p * half + i] = cosf(th);
      sn[(size_t)p * half + i] = sinf(th);
    }
  }
}

}  // namespace ms

using namespace ms;

extern "C" int ms_rmsnorm(float *d_x, int rows, int cols) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(rows > 0 && cols > 0, "rmsnorm: bad shape");
  hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(kBlock), 0, ctx().stream, d_x,
                     (const float *)nullptr, cols);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

extern "C" int ms_rmsnorm_weighted(float *d_x, const float *d_gamma, int rows, int cols) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(rows > 0 && cols > 0, "rmsnorm_weighted: bad shape");
  hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(kBlock), 0, ctx().stream, d_x, d_gamma,
                     cols);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

extern "C" int ms_ple_scale(float *d_x, size_t n, float s) {
  if (int rc = require_init()) return rc;
  if (!n) return MS_OK;
  hipLaunchKernelGGL(k_scale, dim3(cdiv((long)n, kBlock)), dim3(kBlock), 0, ctx().stream, d_x,
                     n, s);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

extern "C" int ms_swiglu(const float *d_gate, float *d_up, size_t n) {
  if (int rc = require_init()) return rc;
  if (!n) return MS_OK;
  hipLaunchKernelGGL(k_swiglu, dim3(cdiv((long)n, kBlock)), dim3(kBlock), 0, ctx().stream,
                     d_gate, d_up, n);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

extern "C" int ms_rope(float *d_x, int rows, int row_stride, int n_heads, int head_stride,
                       int rot_dim, float theta, int base_pos) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(rows > 0 && n_heads > 0 && rot_dim > 0 && rot_dim % 2 == 0 &&
                   rot_dim <= head_stride && base_pos >= 0,
               "rope: bad arguments");
  std::vector<float> cs, sn;
  rope_table_host(rot_dim, theta, base_pos, rows, cs, sn);
  void *buf = nullptr;
  const size_t nb = cs.size() * sizeof(float);
  if (int rc = scratch(2 * nb, &buf)) return rc;
  float *dcs = static_cast<float *>(buf), *dsn = dcs + cs.size();
  MS_HIP_TRY(hipMemcpyAsync(dcs, cs.data(), nb, hipMemcpyHostToDevice, ctx().stream));
  MS_HIP_TRY(hipMemcpyAsync(dsn, sn.data(), nb, hipMemcpyHostToDevice, ctx().stream));
  const long total = (long)rows * n_heads * (rot_dim / 2);
  hipLaunchKernelGGL(k_rope, dim3(cdiv(total, kBlock)), dim3(kBlock), 0, ctx().stream, d_x, rows,
                     row_stride, n_heads, head_stride, rot_dim, dcs, dsn);
  MS_HIP_TRY(hipGetLastError());
  MS_HIP_TRY(hipStreamSynchronize(ctx().stream));  // scratch may be reused
  return MS_OK;
}

extern "C" int ms_attention(const ms_layer_desc *L, const float *d_q, const float *d_knew,
                            const float *d_vnew, float *d_kcache, float *d_vcache, int T,
                            int base, float *d_out) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(L && T >= 1 && base >= 0, "attention: bad arguments");
  if (L->cache_kind == MS_CACHE_LINEAR && !L->clamp_reads)
    MS_CHECK_ARG(base + T <= L->cache_len,
                 "attention: positions exceed the linear cache (reference reads out of "
                 "bounds here, main.mojo:463,476-477)");
  hipStream_t st = ctx().stream;
  const int ld = L->q_dim + 2 * L->kv_dim;
  AttnArgs a{};
  a.B = 1;
  a.T = T;
  a.q_dim = L->q_dim;
  a.kv_dim = L->kv_dim;
  a.hd = L->head_dim;
  a.n_heads = L->n_heads;
  a.n_kv = L->n_kv_heads;
  a.rot = L->rot_dim;
  a.cache_kind = L->cache_kind;
  a.cache_len = L->cache_len;
  a.clamp = L->clamp_reads;
  a.scale = 1.0f / sqrtf((float)L->head_dim);
  a.ld = ld;
  a.apply_rope = 0;
  const int span = (L->cache_kind == MS_CACHE_CIRCULAR) ? L->cache_len + T - 1
                                                        : (base + T);
  a.n_chunks = cdiv(span, kAttnChunk);
  a.write_cache = 1;
  a.kc = d_kcache;
  a.vc = d_vcache;
  a.cache_seq_stride = 0;
  a.out = d_out;
  a.plan_pos = base;
  a.pos_bound = base + T;
  if (int rc = attn_check(a)) return rc;
  const int G = a.n_heads / a.n_kv;
  // many rows: the flash-attention prefill path (needs no chunk partials, but
  // buffers for the rows' q and k)
  const bool flash = T > kGemvMaxM && prefill_flash_ok(a);
  const size_t qkv_f = (size_t)T * ld;
  const size_t fsplit_f = flash ? flash_part_floats(a) : 0;
  const size_t part_f = flash ? (size_t)T * (L->q_dim + L->kv_dim) + fsplit_f
                              : attn_part_floats(1, a.n_kv, a.n_chunks, T, G, a.hd);
  const size_t need = (qkv_f + part_f) * 4 + 64 + (size_t)a.n_kv * 4;
  void *buf = nullptr;
  if (int rc = scratch(need, &buf)) return rc;
  float *qkv = static_cast<float *>(buf);
  float *part = qkv + qkv_f;
  int32_t *dpos = reinterpret_cast<int32_t *>(part + part_f);
  unsigned *ctr = reinterpret_cast<unsigned *>(dpos + 16);
  MS_HIP_TRY(hipMemsetAsync(ctr, 0, (size_t)a.n_kv * 4, st));
  MS_HIP_TRY(hipMemcpy2DAsync(qkv, ld * 4, d_q, L->q_dim * 4, L->q_dim * 4, T,
                              hipMemcpyDeviceToDevice, st));
  MS_HIP_TRY(hipMemcpy2DAsync(qkv + L->q_dim, ld * 4, d_knew, L->kv_dim * 4,
                              L->kv_dim * 4, T, hipMemcpyDeviceToDevice, st));
  MS_HIP_TRY(hipMemcpy2DAsync(qkv + L->q_dim + L->kv_dim, ld * 4, d_vnew, L->kv_dim * 4,
                              L->kv_dim * 4, T, hipMemcpyDeviceToDevice, st));
  MS_HIP_TRY(hipMemcpyAsync(dpos, &base, sizeof(int32_t), hipMemcpyHostToDevice, st));
  a.qkv = qkv;
  a.part = part;
  a.pos = dpos;
  a.ctr = ctr;
  if (flash) {
    float *fsplit = part + (size_t)T * (L->q_dim + L->kv_dim);
    if (int rc = launch_attention_prefill(a, part, part + (size_t)T * L->q_dim,
                                          fsplit_f ? fsplit : nullptr, fsplit_f, st))
      return rc;
  } else if (int rc = launch_attention(a, st)) {
    return rc;
  }
  MS_HIP_TRY(hipStreamSynchronize(st));
  return MS_OK;
}

extern "C" int ms_embed_q4(const uint8_t *d_packed, int D, int vocab, float scale,
                           const int32_t *d_tokens, int n, float *d_out) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(D % 128 == 0 && vocab % 16 == 0 && n >= 0, "embed: bad shape");
  if (!n) return MS_OK;
  return launch_embed(d_packed, D, vocab, scale, d_tokens, n, d_out, ctx().stream);
}

extern "C" int ms_lm_head_argmax(const float *d_x, int M, int D, const uint8_t *d_packed,
                                 int vocab, float scale, float *d_logits, int32_t *d_ids) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(M >= 1 && M <= kGemvMaxM, "lm_head: 1 <= M <= 16");
  MS_CHECK_ARG(D % 128 == 0 && D <= kQuantMaxK && vocab % 64 == 0,
               "lm_head: D % 128 (D <= 16384), vocab % 64");
  hipStream_t st = ctx().stream;
  const int P = 4;
  const long blocks = vocab / 16 / P;
  const size_t qb = (quant_rows_bytes(M, D) + 255) & ~(size_t)255;
  const size_t need = qb + (size_t)blocks * M * 8 + 64;
  void *buf = nullptr;
  if (int rc = scratch(need, &buf)) return rc;
  const QuantRows q = quant_rows_view(buf, M, D);
  float *bv = reinterpret_cast<float *>(static_cast<uint8_t *>(buf) + qb);
  int32_t *bi = reinterpret_cast<int32_t *>(bv + blocks * M);
  RowSrc r{};
  r.x = d_x;
  r.ld = D;
  r.pre_scale = 1.f;
  if (int rc = launch_quant_rows(r, M, D, q, st)) return rc;
  GemvArgs a{};
  a.epi = EPI_ARGMAX;
  a.asrc = AS_QUANT;
  a.K = D;
  a.M = M;
  a.q = q;
  a.seg[0] = GemvSeg{d_packed, scale, vocab, 0};
  a.nseg = 1;
  a.P = P;
  a.waves = 4;
  a.out = d_logits;
  a.ldo = vocab;
  a.arg_val = bv;
  a.arg_idx = bi;
  if (int rc = launch_gemv(a, st)) return rc;
  ArgmaxFin f{};
  f.arg_val = bv;
  f.arg_idx = bi;
  f.n_blocks = (int)blocks;
  f.M = M;
  f.ids_out = d_ids;
  if (int rc = launch_argmax_fin(f, st)) return rc;
  MS_HIP_TRY(hipStreamSynchronize(st));
  return MS_OK;
}
