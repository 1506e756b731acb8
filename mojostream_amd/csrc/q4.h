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
};

// Row finalisation run by the last block of a GEMV (or by a prep kernel).
// x = (base ? base : 0) + sum_{s<n_parts} parts[s]; hidden_out <- x;
// x *= pre_scale; x = x / rms(x) * (gamma ? gamma : 1);
// xn_out <- x (fp32); a_hi/a_lo <- split(x * a_prescale).
struct FinArgs {
  int M, D;
  const float *base;    // [M][D] or null
  const float *parts;   // [n_parts][M][D] or null
  int n_parts;
  size_t part_stride;   // floats between split slices
  float *hidden_out;    // [M][D] or null (x before scaling/normalisation)
  float pre_scale;      // PLE of the next layer, or 1
  int normalize;        // 0: skip the rmsnorm (plain residual output)
  const float *gamma;   // final norm weights or null
  float *xn_out;        // [M][D] or null
  _Float16 *a_hi, *a_lo;  // [M][D] or null
  float a_prescale;     // power of two
};

// Arguments of the fused attention-block finalisation (see attention.hip).
struct AttnArgs;

struct GemvArgs {
  int epi;                        // GemvEpilogue
  int K, M;
  const _Float16 *a_hi, *a_lo;  // activations [M][lda] (hi/lo fp16 split)
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
  // EPI_ARGMAX
  float *arg_val;                 // [blocks][M]
  int32_t *arg_idx;               // [blocks][M]
  int32_t *ids_out;               // [M] final ids (last block)
  int32_t *tok_state;             // optional: next-token state [M]
  int32_t *pos_state;             // optional: positions [M], incremented
  int32_t *ids_hist;              // optional: history [step][M]
  const int32_t *step_ptr;        // optional: step counter for ids_hist
  // last-block finalisation
  unsigned *counter;              // null: none
  int fin_kind;                   // 0 none, 1 rows (FinArgs)
  FinArgs fin;
};

int launch_gemv(const GemvArgs &a, hipStream_t st);
// fp32 rows -> hi/lo fp16 (times prescale)
int launch_split(const float *x, int M, int K, int ldx, float prescale,
                 _Float16 *hi, _Float16 *lo, int ldo, hipStream_t st);
int launch_fin_rows(const FinArgs &f, hipStream_t st);
int launch_sum_parts(float *out, const float *parts, int S, size_t n, hipStream_t st);
int pack_device(uint8_t *dst, const uint8_t *src, int K, int N, hipStream_t st);

__device__ void fin_rows_block(const FinArgs &f);

}  // namespace ms
