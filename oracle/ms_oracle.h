/*
 * ms_oracle.h -- CPU restatement of MojoStream's Gemma-4 per-token layer loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity reference for the HIP
 * path and the timed CPU baseline in bench.py.  It is never linked into,
 * loaded by or called from the product library (libms_gpu.so); only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Every function follows a reference function step by step (file:line given
 * per function, paths relative to the MojoStream repository).  Arithmetic is
 * plain IEEE fp32 in the reference's operation order; the matmul keeps the
 * reference's B-pack blocking (MR=4, NR=16, BK=128) so that its timing is the
 * reference CPU algorithm's timing.
 *
 * Pinning (how each function is checked independently of its own formula):
 *   or_dequant_q4          exhaustive over all 256 byte values x scales against
 *                          the closed form, and round-tripped through a
 *                          quantizer (tests/test_oracle.py).
 *   or_matmul_q4           against or_matmul_q4_f64 (f64 brute force on the
 *                          exact integer weights), identity/one-hot inputs,
 *                          and linearity in A and in the scale.
 *   or_rmsnorm(_weighted)  unit-RMS output invariant, scale invariance,
 *                          f64 closed form.
 *   or_rope                pos=0 identity, pair-norm preservation, composition
 *                          R(p1)R(p2)=R(p1+p2) to rounding, f64 closed form.
 *   or_swiglu              sigmoid special values, f64 closed form.
 *   or_attention           one key returns V, uniform scores return mean(V),
 *                          brute-force f64 softmax on tiny shapes, window and
 *                          GQA index maps against explicit enumeration.
 *   or_layer_forward       against an independently written numpy f64 layer
 *                          (tests/golden/layer_ref.py): demo, sliding-window
 *                          wrap, partial RoPE + clamped full cache, GQA 4:1
 *                          and 5:1, T=1..4 rows.
 *   or_lm_head / argmax    ties resolve to the lowest index; logits against
 *                          or_matmul_q4_f64.
 *   or_matmul_f32          against an f64 product; the columns of a partial
 *                          last 16-column tile stay untouched; C += A . B.
 *   or_sample              penalty cases with closed forms (positive divided,
 *                          negative multiplied, repeats applied per
 *                          occurrence, out-of-range ids ignored); greedy
 *                          branch equals or_argmax; sampled frequencies over
 *                          many seeds against the f64 softmax (chi-square);
 *                          LCG targets uniform on [0, 1].
 *   or_q4_quantize         weights on the exact grid q * 2^-e come back as q
 *                          with scale 2^-e; random weights round-trip through
 *                          or_dequant_q4 within half a scale step, with scale
 *                          float(max|w| / 7); the tiny-block rule (scale 1e-8)
 *                          with and without a tiny block; the transposed
 *                          packing order checked against or_dequant_q4.
 */
#ifndef MS_ORACLE_H
#define MS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* KV cache addressing kinds (reference: main.mojo:257-301 linear KVCache,
 * gemma4_e4b.mojo:83-116 HybridKVCache sliding=circular, full=linear). */
enum { OR_CACHE_LINEAR = 0, OR_CACHE_CIRCULAR = 1 };

/* Attention/KV ordering modes.
 * OR_MODE_CAUSAL   : every row attends exactly its causal (windowed) key set;
 *                    keys of rows in the same call come from the fresh K/V
 *                    rows, the cache is written after attention.  Equal to
 *                    the reference whenever no circular-slot collision occurs.
 * OR_MODE_WRITE_FIRST: the reference's literal order -- write all T rows into
 *                    the cache, then attend reading the cache
 *                    (gemma4_e4b.mojo:507-515, main.mojo:583-595).  Used to
 *                    show where the two differ (circular wrap with T>1). */
enum { OR_MODE_CAUSAL = 0, OR_MODE_WRITE_FIRST = 1 };

typedef struct {
  int q_dim, kv_dim, head_dim, n_heads, n_kv_heads;
  int rot_dim;        /* rotated dims per head (== head_dim, or 128 for E4B full) */
  float theta;        /* RoPE base */
  int cache_kind;     /* OR_CACHE_* */
  int cache_len;      /* linear: max positions; circular: window */
  int clamp_reads;    /* linear only: clamp attended keys to cache_len (E4B full,
                         gemma4_e4b.mojo:362-363); 0 = demo semantics */
  const uint8_t *w[7];/* Q K V O Gate Up Down, row-major [K][N/2] Q4 */
  float scale[7];
  float ple;
  float *kc, *vc;     /* this layer's cache for one sequence: [cache_len][kv_dim] */
} or_layer;

/* a1: Q4 dequant, kernels.mojo:66-69 (layout) and :100-108 (dequant_vec). */
void or_dequant_q4(const uint8_t *wq, int K, int N, float scale, float *out);

/* a3: C += A . deq(W), matmul_q4_bpack_raw, kernels.mojo:201-267.
 * A [M][K] fp32, W [K][N/2] Q4, C [M][N].  Any M (the reference needs M%4==0;
 * rows beyond a multiple of 4 follow the same per-element order). */
void or_matmul_q4(float *C, const float *A, const uint8_t *wq, int M, int K,
                  int N, float scale);

/* Test-only column split of or_matmul_q4 over n threads (default 1, the
 * reference's decode threading).  Bit-identical results for any n. */
void or_set_threads(int n);

/* f64 brute force of the same product (pin for or_matmul_q4 and the GPU). */
void or_matmul_q4_f64(double *C, const float *A, const uint8_t *wq, int M,
                      int K, int N, float scale);

/* a5: rmsnorm_inplace, kernels.mojo:474-489 (no gamma). */
void or_rmsnorm(float *x, int rows, int cols);
/* a13: rmsnorm_weighted_inplace, kernels.mojo:598-613. */
void or_rmsnorm_weighted(float *x, const float *gamma, int rows, int cols);
/* a6: ple_scale_inplace, kernels.mojo:506-516. */
void or_ple_scale(float *x, int n, float s);
/* a8: swiglu_inplace, kernels.mojo:519-532 (result in up). */
void or_swiglu(const float *gate, float *up, int n);
/* a7: RoPE cos/sin for one position, kernels.mojo:562-577.  cs/sn [rot/2]. */
void or_rope_table(int rot_dim, int pos, float theta, float *cs, float *sn);
/* a7: apply_rope_inplace over n_heads heads of stride head_stride, rotating the
 * first rot_dim dims of each head, kernels.mojo:579-595 with the partial use at
 * gemma4_e4b.mojo:489-505. */
void or_rope(float *x, int n_heads, int head_stride, int rot_dim, int pos,
             float theta);

/* a10/a11: attention for T rows of one sequence at positions base..base+T-1.
 * q [T][q_dim] (after RoPE); knew/vnew [T][kv_dim] (after RoPE for K) are the
 * rows' own keys; the cache holds older positions.  out [T][q_dim].
 * Follows compute_sliding_attention (gemma4_e4b.mojo:259-338),
 * compute_full_attention (:341-411) and gqa_attention_decode
 * (main.mojo:445-519): dot in 8-lane partial sums, x scale, 3-pass softmax,
 * sum p*v sequential in key order. */
void or_attention(const or_layer *L, const float *q, const float *knew,
                  const float *vnew, int T, int base, int mode, float *out);

/* Cache write of T rows (write_kv_sliding/full, gemma4_e4b.mojo:211-249;
 * main.mojo:584-592). Linear caches drop positions >= cache_len. */
void or_kv_write(const or_layer *L, const float *knew, const float *vnew,
                 int T, int base);

/* a12: one layer, x [T][D] in place (e4b_forward_layer gemma4_e4b.mojo:459-540;
 * gemma4_forward_layer main.mojo:538-613).  Scratch is allocated inside. */
void or_layer_forward(const or_layer *L, int D, int F, float *x, int T,
                      int base, int mode);

/* a13: logits [M][vocab] = x . deq(W_lm) (project_lm_head lm_head.mojo:146-168,
 * zeroed C then matmul_q4_bpack_raw). */
void or_lm_head(const float *x, int M, int D, const uint8_t *wlm, int vocab,
                float scale, float *logits);
/* greedy branch of temperature_sampling, lm_head.mojo:224-230. */
int or_argmax(const float *v, int n);
/* temperature_sampling (lm_head.mojo:198-254) with the seed as an argument
 * where the reference reads the clock (:246).  In list order, each
 * occurrence of an id of `generated` below n divides a positive logit by
 * `penalty` or multiplies a non-positive one (:211-220, when penalty > 1).
 * Temperature <= 0.01: first index of the maximum (:222-228).  Otherwise the
 * logits become exp((v - max) / T) / sum in place (:230-243), one LCG step
 * of the seed gives the target (:246-248), and the first index whose running
 * fp32 sum reaches it is returned, else n - 1 (:250-254).  Modifies logits in
 * place like the reference. */
int or_sample(float *logits, int n, float temperature, const int32_t *generated,
              int n_generated, float penalty, uint64_t seed);
/* The LCG target of one seed (lm_head.mojo:247-248). */
float or_sample_target(uint64_t seed);
/* matmul_fp32_raw (kernels.mojo:616-671): C += A . B, B fp32 row-major [K][N];
 * per 128 rows of K, per whole 16-column tile (:640; a partial last tile is
 * left untouched), per row: the products of the tile's rows added in k order,
 * then added to C. */
void or_matmul_f32(float *C, const float *A, const float *B, int M, int K, int N);
/* quantize_q4_blockwise (scripts/convert.py:296-323) after the converter's
 * transpose (convert.py:503-506): w_hf [n_out][n_in] fp32 in, packed
 * [n_in][n_out/2] and the global scale out. */
void or_q4_quantize(const float *w_hf, int n_out, int n_in, int block_size, uint8_t *packed,
                    float *scale);
/* get_token_embedding Q4 branch, lm_head.mojo:186-195. */
void or_embed(const uint8_t *wlm, int D, int vocab, float scale, int token,
              float *out);

/* Whole-model token step for one sequence (used by the CPU baseline and the
 * greedy-ID tests): x = embed(token) -> n_layers x or_layer_forward ->
 * final weighted rmsnorm -> logits -> argmax.  Returns the greedy ID.
 * hidden_out [n_layers][D] (optional) receives each layer's output row. */
int or_decode_token(const or_layer *layers, int n_layers, int D, int F,
                    const uint8_t *wlm, int vocab, float lm_scale,
                    const float *gamma, int token, int pos, float *hidden_out);

#ifdef __cplusplus
}
#endif
#endif
