// Q4 GEMV/GEMM interfaces shared between translation units.
#pragma once
#include "common.h"

namespace ms {

// One output segment of a fused GEMV launch (e.g. Q, K, V of one layer).
struct GemvSeg {
  const uint8_t *w;  // panel-layout weights [K][n_cols]
  float scale;       // per-tensor Q4 scale
  int n_cols;        // multiple of 16
  int out_col0;      // first output column of this segment
};

enum GemvEpilogue {
  EPI_STORE = 0,       // out[s][m][col] = value (s = K split)
  EPI_ACCUMULATE = 1,  // out[m][col] += value (S must be 1)
  EPI_SWIGLU = 2,      // seg0 = gate, seg1 = up, same panel per block:
                       // up*gate*sigmoid(gate) -> f16 hi/lo (times act_scale)
                       // and optionally fp32 into out
  EPI_ARGMAX = 3,      // LM head: logits (optional) + per-block argmax
  EPI_RESID = 4,       // S=1, P=1: x = resid + value -> out [M][ldo] and the
                       // block's sum of squares per row -> ss_out[m][block]
};

// Optional GEMV prologue: every block rebuilds the activation rows it needs
// in LDS.  x = base + sum_{s<n_parts} parts[s]; y = rmsnorm(x * pre_scale)
// (* gamma); the block keeps fp16 hi/lo of y for its K range.  Block 0 also
// stores x (the previous layer's output) and y (the residual base).
struct PrepArgs {
  int on;
  // Reduced-row mode (xsum set): x = xsum[m][k] was summed by a producer,
  // which also left n_ss partial sums of (x*pre_scale)^2 per row in ss.
  const float *xsum;    // [M][K] or null
  const float *ss;      // [M][n_ss]
  int n_ss;
  // Direct mode: x = base + sum of split partials.
  const float *base;    // [M][K] or null
  const float *parts;   // [n_parts][M][K] or null
  int n_parts;
  size_t part_stride;   // floats between split slices
  float pre_scale;      // PLE of this layer (1 for the post-attention norm)
  const float *gamma;   // final-norm weights or null
  float *xn_out;        // block 0: y [M][K] or null
  float *hid_out;       // block 0: x [M][K] or null
  float *hid_out2;      // block 0: second copy of x or null
};

struct GemvArgs {
  int epi;                        // GemvEpilogue
  int K, M;
  const _Float16 *a_hi, *a_lo;  // activations [M][lda] (hi/lo fp16 split), unless prep.on
  int lda;
  float out_mul;                 // undoes the activation pre-scale
  GemvSeg seg[3];
  int nseg;
  int P;                          // panels per block (EPI_SWIGLU: 2)
  int S;                          // K splits
  int waves;                      // waves per block (4 or 8)
  float *out;                     // EPI_STORE: [S][M][ldo]
  int ldo;
  size_t split_stride;
  // EPI_SWIGLU
  _Float16 *sw_hi, *sw_lo;        // [M][ldo_sw]
  int ldo_sw;
  float sw_prescale;
  // EPI_ARGMAX: per-block maximum and its first index, per row
  float *arg_val;                 // [blocks][M]
  int32_t *arg_idx;               // [blocks][M]
  // EPI_RESID
  const float *resid;             // [M][ldo]
  float *ss_out;                  // [M][n_blocks]
  PrepArgs prep;
};

// Final argmax over the LM head's per-block maxima (greedy branch of
// temperature_sampling, lm_head.mojo:224-230) and decode-state update.
struct ArgmaxFin {
  const float *arg_val;
  const int32_t *arg_idx;
  int n_blocks, M;
  int32_t *ids_out;     // [M] or null
  int32_t *tok_state;   // [M] or null: next input token
  int32_t *pos_state;   // [M] or null: incremented
  int32_t *ids_hist;    // [cap][M] or null
  int32_t *step;        // step counter (with ids_hist)
};

int launch_gemv(const GemvArgs &a, hipStream_t st);
// fp32 rows -> hi/lo fp16 (times prescale)
int launch_split(const float *x, int M, int K, int ldx, float prescale,
                 _Float16 *hi, _Float16 *lo, int ldo, hipStream_t st);
int launch_sum_parts(float *out, const float *parts, int S, size_t n, hipStream_t st);
int pack_device(uint8_t *dst, const uint8_t *src, int K, int N, hipStream_t st);
int launch_argmax_fin(const ArgmaxFin &f, hipStream_t st);
// Standalone row preparation (same math as the GEMV prologue) writing the
// fp16 hi/lo split to global memory: used where the consumer is not a GEMV.
int launch_prep_rows(const PrepArgs &p, int M, int K, _Float16 *hi, _Float16 *lo,
                     hipStream_t st);
// Residual sum of a row: xsum = base + sum parts (also into hid_out/hid_out2)
// and per-256-column partial sums of (xsum*pre_scale)^2 -> ss [M][ceil(K/256)].
int launch_rowsum(const PrepArgs &p, int M, int K, float *xsum, float *ss, hipStream_t st);

}  // namespace ms
