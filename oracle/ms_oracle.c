/*
 * ms_oracle.c -- CPU restatement of MojoStream's Gemma-4 layer loop.
 *
 * TEST INFRASTRUCTURE ONLY (parity reference + timed CPU baseline); see
 * ms_oracle.h for the pinning of each function.  Built by oracle/Makefile with
 * -ffp-contract=off so every a*b+c in the reference text is a rounded multiply
 * followed by a rounded add, independent of the host's FMA support.
 */
#include "ms_oracle.h"

#include <assert.h>
#include <pthread.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* The reference's SIMD shapes on its AVX2 target (kernels.mojo:13-21). */
#define SIMD_W 8
#define NR (2 * SIMD_W)
#define MR 4
#define BK 128

typedef float v8f __attribute__((vector_size(32)));

/* Mojo SIMD.reduce_add: halve the vector and add, recursively. */
static float reduce_add8(const float l[8]) {
  float b0 = l[0] + l[4], b1 = l[1] + l[5], b2 = l[2] + l[6], b3 = l[3] + l[7];
  float c0 = b0 + b2, c1 = b1 + b3;
  return c0 + c1;
}

/* ---- a1: dequant (kernels.mojo:66-69, :100-108; gen_reference.py:62-66) ---- */
void or_dequant_q4(const uint8_t *wq, int K, int N, float scale, float *out) {
  const int pc = N / 2;
  for (int k = 0; k < K; ++k)
    for (int j = 0; j < pc; ++j) {
      const uint8_t b = wq[(size_t)k * pc + j];
      const int lo = (int)(b & 0x0F) - 8;
      const int hi = (int)((b >> 4) & 0x0F) - 8;
      out[(size_t)k * N + 2 * j] = (float)lo * scale;
      out[(size_t)k * N + 2 * j + 1] = (float)hi * scale;
    }
}

/* ---- a3: matmul_q4_bpack_raw (kernels.mojo:201-267) ----
 * For each k-tile of BK rows and each NR-column tile the weights are
 * dequantized once into b_buf (:232-236); then MR rows at a time accumulate
 * acc = acc + a*B sequentially over the tile (:243-253) and C += acc (:255-262).
 * SIMD lanes are columns, so each C element sees the same scalar order on any
 * SIMD width. */
static void bpack_block(float *C, const float *A, const uint8_t *wq, int m0,
                        int m1, int K, int N, int n0, int n1, float scale) {
  const int pc = N / 2;
  float b_buf[BK * NR] __attribute__((aligned(32)));
  for (int kt = 0; kt < K; kt += BK) {
    const int bk = (K - kt < BK) ? K - kt : BK;
    for (int nt = n0; nt < n1; nt += NR) {
      const int nw = (n1 - nt < NR) ? n1 - nt : NR; /* reference: N % NR == 0 */
      for (int kl = 0; kl < bk; ++kl) {
        const uint8_t *row = wq + (size_t)(kt + kl) * pc + nt / 2;
        float *bp = b_buf + kl * NR;
        for (int j = 0; j < NR / 2; ++j) {
          if (2 * j >= nw) { bp[2 * j] = bp[2 * j + 1] = 0.f; continue; }
          const uint8_t b = row[j];
          bp[2 * j] = (float)((int)(b & 0x0F) - 8) * scale;
          bp[2 * j + 1] = (float)((int)((b >> 4) & 0x0F) - 8) * scale;
        }
      }
      for (int m = m0; m < m1; m += MR) {
        const int mr = (m1 - m < MR) ? m1 - m : MR;
        v8f acc[MR][2];
        memset(acc, 0, sizeof(acc));
        for (int kl = 0; kl < bk; ++kl) {
          v8f B0, B1;
          memcpy(&B0, b_buf + kl * NR, 32);
          memcpy(&B1, b_buf + kl * NR + SIMD_W, 32);
          for (int r = 0; r < mr; ++r) {
            const float a = A[(size_t)(m + r) * K + kt + kl];
            const v8f av = {a, a, a, a, a, a, a, a};
            acc[r][0] = acc[r][0] + av * B0;
            acc[r][1] = acc[r][1] + av * B1;
          }
        }
        for (int r = 0; r < mr; ++r) {
          float *c = C + (size_t)(m + r) * N + nt;
          float t[NR];
          memcpy(t, &acc[r][0], 32);
          memcpy(t + SIMD_W, &acc[r][1], 32);
          for (int j = 0; j < nw; ++j) c[j] = c[j] + t[j];
        }
      }
    }
  }
}

/* Optional column split over threads for the oracle (not the reference's
 * threading, which splits rows): every C element keeps its summation order,
 * so results are bit-identical for any thread count. */
static int g_threads = 1;
void or_set_threads(int n) { g_threads = n < 1 ? 1 : (n > 64 ? 64 : n); }

typedef struct {
  float *C; const float *A; const uint8_t *wq;
  int M, K, N, n0, n1;
  float scale;
} mm_job;

static void *mm_worker(void *p) {
  mm_job *j = (mm_job *)p;
  bpack_block(j->C, j->A, j->wq, 0, j->M, j->K, j->N, j->n0, j->n1, j->scale);
  return NULL;
}

void or_matmul_q4(float *C, const float *A, const uint8_t *wq, int M, int K,
                  int N, float scale) {
  /* parallelize over BM=64-row blocks (kernels.mojo:212,266): decode shapes
   * (M <= 64) are one work item, i.e. single-threaded, as here by default. */
  int nt = g_threads;
  if (nt > 1 && N >= nt * NR) {
    pthread_t th[64];
    mm_job jobs[64];
    const int tiles = (N + NR - 1) / NR;
    for (int t = 0; t < nt; ++t) {
      const int t0 = (int)((long)tiles * t / nt), t1 = (int)((long)tiles * (t + 1) / nt);
      jobs[t] = (mm_job){C, A, wq, M, K, N, t0 * NR, t1 * NR < N ? t1 * NR : N, scale};
      pthread_create(&th[t], NULL, mm_worker, &jobs[t]);
    }
    for (int t = 0; t < nt; ++t) pthread_join(th[t], NULL);
    return;
  }
  bpack_block(C, A, wq, 0, M, K, N, 0, N, scale);
}

void or_matmul_q4_f64(double *C, const float *A, const uint8_t *wq, int M,
                      int K, int N, float scale) {
  const int pc = N / 2;
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      double s = 0.0;
      for (int k = 0; k < K; ++k) {
        const uint8_t b = wq[(size_t)k * pc + n / 2];
        const int nib = (n & 1) ? ((b >> 4) & 0x0F) : (b & 0x0F);
        s += (double)A[(size_t)m * K + k] * (double)(nib - 8);
      }
      C[(size_t)m * N + n] = s * (double)scale;
    }
}

/* ---- a5 / a13: rmsnorm (kernels.mojo:474-489, :598-613) ---- */
static float row_rms_inv(const float *rp, int n) {
  float lanes[SIMD_W] = {0};
  for (int i = 0; i < n; ++i) lanes[i % SIMD_W] = lanes[i % SIMD_W] + rp[i] * rp[i];
  const float ss = reduce_add8(lanes);
  return 1.0f / sqrtf(ss / (float)n + 1e-6f);
}

void or_rmsnorm(float *x, int rows, int cols) {
  for (int r = 0; r < rows; ++r) {
    float *rp = x + (size_t)r * cols;
    const float inv = row_rms_inv(rp, cols);
    for (int i = 0; i < cols; ++i) rp[i] = rp[i] * inv;
  }
}

void or_rmsnorm_weighted(float *x, const float *gamma, int rows, int cols) {
  for (int r = 0; r < rows; ++r) {
    float *rp = x + (size_t)r * cols;
    const float inv = row_rms_inv(rp, cols);
    for (int i = 0; i < cols; ++i)
      rp[i] = rp[i] * inv * (gamma ? gamma[i] : 1.0f);
  }
}

/* ---- a6: ple_scale_inplace (kernels.mojo:506-516) ---- */
void or_ple_scale(float *x, int n, float s) {
  for (int i = 0; i < n; ++i) x[i] = x[i] * s;
}

/* ---- a8: swiglu_inplace (kernels.mojo:519-532) ---- */
void or_swiglu(const float *gate, float *up, int n) {
  const int body = n - n % SIMD_W;
  int i = 0;
  for (; i < body; ++i) {
    /* SIMD body (:522-527): sig = 1/(1+exp(-g)); up = u*g*sig */
    const float g = gate[i];
    const float sig = 1.0f / (1.0f + expf(-g));
    up[i] = up[i] * g * sig;
  }
  for (; i < n; ++i) {
    const float g = gate[i];
    up[i] = up[i] * g / (1.0f + expf(-g)); /* scalar tail (:528-532) */
  }
}

/* ---- a7: RoPE (kernels.mojo:553-595) ---- */
void or_rope_table(int rot_dim, int pos, float theta, float *cs, float *sn) {
  const int half = rot_dim / 2;
  const float ln_base = logf(theta);
  const float pos_f = (float)pos;
  for (int i = 0; i < half; ++i) {
    const float inv_freq = expf(-(float)(2 * i) / (float)rot_dim * ln_base);
    const float th = pos_f * inv_freq;
    cs[i] = cosf(th);
    sn[i] = sinf(th);
  }
}

void or_rope(float *x, int n_heads, int head_stride, int rot_dim, int pos,
             float theta) {
  const int half = rot_dim / 2;
  float *cs = (float *)malloc(sizeof(float) * half);
  float *sn = (float *)malloc(sizeof(float) * half);
  or_rope_table(rot_dim, pos, theta, cs, sn);
  for (int h = 0; h < n_heads; ++h) {
    float *hp = x + (size_t)h * head_stride;
    for (int i = 0; i < half; ++i) {
      const float xi = hp[i], xih = hp[i + half];
      hp[i] = xi * cs[i] - xih * sn[i];
      hp[i + half] = xi * sn[i] + xih * cs[i];
    }
  }
  free(cs);
  free(sn);
}

/* ---- a9: KV write (gemma4_e4b.mojo:211-249; main.mojo:584-592) ---- */
static int cache_slot(const or_layer *L, int t) {
  return L->cache_kind == OR_CACHE_CIRCULAR ? t % L->cache_len : t;
}

void or_kv_write(const or_layer *L, const float *knew, const float *vnew,
                 int T, int base) {
  for (int r = 0; r < T; ++r) {
    const int t = base + r;
    if (L->cache_kind == OR_CACHE_LINEAR && t >= L->cache_len) continue;
    const int s = cache_slot(L, t);
    memcpy(L->kc + (size_t)s * L->kv_dim, knew + (size_t)r * L->kv_dim,
           sizeof(float) * L->kv_dim);
    memcpy(L->vc + (size_t)s * L->kv_dim, vnew + (size_t)r * L->kv_dim,
           sizeof(float) * L->kv_dim);
  }
}

/* ---- a10/a11: attention ----
 * Rows are independent given the cache and the fresh K/V, so the oracle may
 * split them over threads (or_set_threads); each row's arithmetic is the same
 * for any split. */
typedef struct {
  const or_layer *L;
  const float *q, *knew, *vnew;
  int r0, r1, base, mode;
  float *out;
} attn_job;

static void attention_rows(const or_layer *L, const float *q, const float *knew,
                           const float *vnew, int r0, int r1, int base, int mode,
                           float *out) {
  const int hd = L->head_dim, kvd = L->kv_dim, qd = L->q_dim;
  const int ratio = L->n_heads / L->n_kv_heads;
  const float scale = 1.0f / sqrtf((float)hd);
  int max_keys = base + r1;
  float *sp = (float *)malloc(sizeof(float) * (size_t)(max_keys > 0 ? max_keys : 1));
  for (int r = r0; r < r1; ++r) {
    const int p = base + r;
    int k0, k1; /* attended absolute positions [k0, k1) */
    if (L->cache_kind == OR_CACHE_CIRCULAR) {
      const int seq_len = p + 1;
      k0 = seq_len - L->cache_len;
      if (k0 < 0) k0 = 0;
      k1 = seq_len;
    } else {
      k0 = 0;
      k1 = p + 1;
      if (L->clamp_reads && k1 > L->cache_len) k1 = L->cache_len;
      assert(k1 <= L->cache_len || mode == OR_MODE_CAUSAL);
    }
    for (int hq = 0; hq < L->n_heads; ++hq) {
      const int hkv = hq / ratio;
      const float *qh = q + (size_t)r * qd + (size_t)hq * hd;
      int n = 0;
      for (int t = k0; t < k1; ++t, ++n) {
        const float *kh;
        if (mode == OR_MODE_CAUSAL && t >= base)
          kh = knew + (size_t)(t - base) * kvd + (size_t)hkv * hd;
        else
          kh = L->kc + (size_t)cache_slot(L, t) * kvd + (size_t)hkv * hd;
        /* SIMD_W-lane partial sums (lane l takes dims j + l), then reduce_add */
        v8f lanes = {0, 0, 0, 0, 0, 0, 0, 0};
        int j = 0;
        for (; j + SIMD_W <= hd; j += SIMD_W) {
          v8f qv, kv;
          memcpy(&qv, qh + j, sizeof qv);
          memcpy(&kv, kh + j, sizeof kv);
          lanes = lanes + qv * kv;
        }
        float l8[SIMD_W];
        memcpy(l8, &lanes, sizeof l8);
        float s = reduce_add8(l8) * scale;
        for (; j < hd; ++j) s = s + qh[j] * kh[j] * scale;
        sp[n] = s;
      }
      float mx = sp[0];
      for (int i = 1; i < n; ++i)
        if (sp[i] > mx) mx = sp[i];
      float sum = 0.f;
      for (int i = 0; i < n; ++i) {
        const float e = expf(sp[i] - mx);
        sp[i] = e;
        sum = sum + e;
      }
      const float inv = 1.0f / sum;
      for (int i = 0; i < n; ++i) sp[i] = sp[i] * inv;
      float *oh = out + (size_t)r * qd + (size_t)hq * hd;
      for (int j = 0; j < hd; ++j) oh[j] = 0.f;
      n = 0;
      for (int t = k0; t < k1; ++t, ++n) {
        const float *vh;
        if (mode == OR_MODE_CAUSAL && t >= base)
          vh = vnew + (size_t)(t - base) * kvd + (size_t)hkv * hd;
        else
          vh = L->vc + (size_t)cache_slot(L, t) * kvd + (size_t)hkv * hd;
        const float pr = sp[n];
        for (int j = 0; j < hd; ++j) oh[j] = oh[j] + pr * vh[j];
      }
    }
  }
  free(sp);
}

static void *attn_worker(void *p) {
  attn_job *j = (attn_job *)p;
  attention_rows(j->L, j->q, j->knew, j->vnew, j->r0, j->r1, j->base, j->mode, j->out);
  return NULL;
}

void or_attention(const or_layer *L, const float *q, const float *knew,
                  const float *vnew, int T, int base, int mode, float *out) {
  int nt = g_threads < T ? g_threads : T;
  if (nt > 1 && T >= 8) {
    pthread_t th[64];
    attn_job jobs[64];
    /* causal rows attend to more keys the later they are: cut the rows into
     * ranges of about equal key counts */
    double total = 0;
    for (int r = 0; r < T; ++r) {
      const int p = base + r + 1;
      total += (L->cache_kind == OR_CACHE_CIRCULAR && p > L->cache_len) ? L->cache_len : p;
    }
    int r = 0;
    double acc = 0;
    for (int t = 0; t < nt; ++t) {
      const int r0 = r;
      const double goal = total * (t + 1) / nt;
      while (r < T && (acc < goal || t == nt - 1)) {
        const int p = base + r + 1;
        acc += (L->cache_kind == OR_CACHE_CIRCULAR && p > L->cache_len) ? L->cache_len : p;
        ++r;
      }
      jobs[t] = (attn_job){L, q, knew, vnew, r0, r, base, mode, out};
      pthread_create(&th[t], NULL, attn_worker, &jobs[t]);
    }
    for (int t = 0; t < nt; ++t) pthread_join(th[t], NULL);
    return;
  }
  attention_rows(L, q, knew, vnew, 0, T, base, mode, out);
}

/* ---- a12: one layer (gemma4_e4b.mojo:459-540; main.mojo:538-613) ---- */
void or_layer_forward(const or_layer *L, int D, int F, float *x, int T,
                      int base, int mode) {
  const int qd = L->q_dim, kvd = L->kv_dim, hd = L->head_dim;
  float *q = (float *)calloc((size_t)T * qd, sizeof(float));
  float *k = (float *)calloc((size_t)T * kvd, sizeof(float));
  float *v = (float *)calloc((size_t)T * kvd, sizeof(float));
  float *att = (float *)calloc((size_t)T * qd, sizeof(float));
  float *proj = (float *)calloc((size_t)T * D, sizeof(float));
  float *gate = (float *)calloc((size_t)T * F, sizeof(float));
  float *up = (float *)calloc((size_t)T * F, sizeof(float));
  float *ffn = (float *)calloc((size_t)T * D, sizeof(float));

  /* 1. PLE + pre-norm (:474-475) */
  or_ple_scale(x, T * D, L->ple);
  or_rmsnorm(x, T, D);
  /* 2. Q/K/V into zeroed buffers (:480-486) */
  or_matmul_q4(q, x, L->w[0], T, D, qd, L->scale[0]);
  or_matmul_q4(k, x, L->w[1], T, D, kvd, L->scale[1]);
  or_matmul_q4(v, x, L->w[2], T, D, kvd, L->scale[2]);
  /* 3. RoPE at position base+row (:489-505; main.mojo:579-581) */
  for (int r = 0; r < T; ++r) {
    or_rope(q + (size_t)r * qd, L->n_heads, hd, L->rot_dim, base + r, L->theta);
    or_rope(k + (size_t)r * kvd, L->n_kv_heads, hd, L->rot_dim, base + r,
            L->theta);
  }
  /* 4-5. KV write + attention (:508-515) */
  if (mode == OR_MODE_WRITE_FIRST) {
    or_kv_write(L, k, v, T, base);
    or_attention(L, q, k, v, T, base, mode, att);
  } else {
    or_attention(L, q, k, v, T, base, mode, att);
    or_kv_write(L, k, v, T, base);
  }
  /* 6. O projection + residual on the normalized stream (:519-522) */
  or_matmul_q4(proj, att, L->w[3], T, qd, D, L->scale[3]);
  for (int j = 0; j < T * D; ++j) x[j] = x[j] + proj[j];
  /* 7. post-attention norm (:525) */
  or_rmsnorm(x, T, D);
  /* 8. SwiGLU FFN + residual (:528-538) */
  or_matmul_q4(gate, x, L->w[4], T, D, F, L->scale[4]);
  or_matmul_q4(up, x, L->w[5], T, D, F, L->scale[5]);
  or_swiglu(gate, up, T * F);
  or_matmul_q4(ffn, up, L->w[6], T, F, D, L->scale[6]);
  for (int j = 0; j < T * D; ++j) x[j] = x[j] + ffn[j];

  free(q); free(k); free(v); free(att); free(proj); free(gate); free(up);
  free(ffn);
}

/* ---- a13: LM head, greedy, embedding (lm_head.mojo) ---- */
void or_lm_head(const float *x, int M, int D, const uint8_t *wlm, int vocab,
                float scale, float *logits) {
  memset(logits, 0, sizeof(float) * (size_t)M * vocab);
  or_matmul_q4(logits, x, wlm, M, D, vocab, scale);
}

int or_argmax(const float *v, int n) {
  int best = 0;
  float bv = v[0];
  for (int j = 1; j < n; ++j)
    if (v[j] > bv) { bv = v[j]; best = j; }
  return best;
}

/* lm_head.mojo:247-248: lcg = (seed * 6364136223846793005 +
 * 1442695040888963407) & 0x7FFFFFFF in wrapping 64-bit arithmetic (the low 31
 * bits do not depend on signedness), target = Float32(lcg) / Float32(2^31 - 1). */
float or_sample_target(uint64_t seed) {
  const uint64_t lcg = (seed * 6364136223846793005ull + 1442695040888963407ull) & 0x7FFFFFFFull;
  return (float)lcg / (float)0x7FFFFFFF;
}

/* temperature_sampling, lm_head.mojo:198-254 */
int or_sample(float *logits, int n, float temperature, const int32_t *generated,
              int n_generated, float penalty, uint64_t seed) {
  if (penalty > 1.0f) {                       /* :211-220 */
    for (int i = 0; i < n_generated; ++i) {
      const int tid = generated[i];
      if (tid >= 0 && tid < n) {
        const float v = logits[tid];
        logits[tid] = v > 0.0f ? v / penalty : v * penalty;
      }
    }
  }
  if (temperature <= 0.01f) return or_argmax(logits, n);  /* :222-228 */
  const float inv_t = 1.0f / temperature;     /* :230-233 */
  float max_v = logits[0];
  for (int j = 1; j < n; ++j)
    if (logits[j] > max_v) max_v = logits[j];
  float sum_e = 0.0f;                         /* :235-239 */
  for (int j = 0; j < n; ++j) {
    const float e = expf((logits[j] - max_v) * inv_t);
    logits[j] = e;
    sum_e += e;
  }
  const float inv_s = 1.0f / sum_e;           /* :240-242 */
  for (int j = 0; j < n; ++j) logits[j] = logits[j] * inv_s;
  const float target = or_sample_target(seed);  /* :246-248 */
  float cdf = 0.0f;                           /* :250-254 */
  for (int j = 0; j < n; ++j) {
    cdf += logits[j];
    if (cdf >= target) return j;
  }
  return n - 1;
}

/* matmul_fp32_raw, kernels.mojo:616-671 (BK = 128, NR = 16, :636-668) */
void or_matmul_f32(float *C, const float *A, const float *B, int M, int K, int N) {
  for (int kt = 0; kt < K; kt += 128) {
    const int k1 = kt + 128 < K ? kt + 128 : K;
    for (int nt = 0; nt + 16 <= N; nt += 16)
      for (int m = 0; m < M; ++m)
        for (int j = 0; j < 16; ++j) {
          float acc = 0.0f;
          for (int k = kt; k < k1; ++k) acc = acc + A[(size_t)m * K + k] * B[(size_t)k * N + nt + j];
          C[(size_t)m * N + nt + j] = C[(size_t)m * N + nt + j] + acc;
        }
  }
}

void or_embed(const uint8_t *wlm, int D, int vocab, float scale, int token,
              float *out) {
  const int pc = vocab / 2, bc = token / 2, hi = token & 1;
  for (int r = 0; r < D; ++r) {
    const uint8_t b = wlm[(size_t)r * pc + bc];
    const int nib = hi ? ((b >> 4) & 0x0F) : (b & 0x0F);
    out[r] = (float)(nib - 8) * scale;
  }
}

int or_decode_token(const or_layer *layers, int n_layers, int D, int F,
                    const uint8_t *wlm, int vocab, float lm_scale,
                    const float *gamma, int token, int pos, float *hidden_out) {
  float *x = (float *)malloc(sizeof(float) * D);
  float *logits = (float *)malloc(sizeof(float) * (size_t)vocab);
  or_embed(wlm, D, vocab, lm_scale, token, x);
  for (int l = 0; l < n_layers; ++l) {
    or_layer_forward(&layers[l], D, F, x, 1, pos, OR_MODE_CAUSAL);
    if (hidden_out) memcpy(hidden_out + (size_t)l * D, x, sizeof(float) * D);
  }
  or_rmsnorm_weighted(x, gamma, 1, D);
  or_lm_head(x, 1, D, wlm, vocab, lm_scale, logits);
  const int id = or_argmax(logits, vocab);
  free(x);
  free(logits);
  return id;
}

/* scripts/convert.py:296-323 on the transposed (n_in, n_out) matrix
 * (convert.py:503-506): block scales over the flat array, in double as Python
 * computes them (:310-314), their maximum (:316), then float32 division by the
 * float32 scale, round half to even, clip to [-8, 7], +8, and even columns in
 * the low nibble (:318-323). */
void or_q4_quantize(const float *w_hf, int n_out, int n_in, int block_size, uint8_t *packed,
                    float *scale) {
  const size_t total = (size_t)n_out * n_in;
  double gs = 0.0;
  int any = 0;
  for (size_t b0 = 0; b0 < total; b0 += (size_t)block_size) {
    const size_t b1 = b0 + (size_t)block_size < total ? b0 + (size_t)block_size : total;
    float m = 0.0f;
    for (size_t i = b0; i < b1; ++i) {
      const size_t k = i / (size_t)n_out, o = i % (size_t)n_out;
      const float a = fabsf(w_hf[o * (size_t)n_in + k]);
      if (a > m) m = a;
    }
    const double bs = (double)m > 1e-8 ? (double)m / 7.0 : 1e-8;
    if (!any || bs > gs) gs = bs;
    any = 1;
  }
  if (!any) gs = 1e-8;
  const float s = (float)gs;
  const size_t half = (size_t)n_out / 2;
  for (int k = 0; k < n_in; ++k)
    for (size_t j = 0; j < half; ++j) {
      uint8_t byte = 0;
      for (int h = 0; h < 2; ++h) {
        const float x = w_hf[(2 * j + h) * (size_t)n_in + k];
        float q = nearbyintf(x / s);
        if (q < -8.0f) q = -8.0f;
        if (q > 7.0f) q = 7.0f;
        byte |= (uint8_t)(((int)q + 8) & 0x0F) << (4 * h);
      }
      packed[(size_t)k * half + j] = byte;
    }
  *scale = s;
}
