// Q4 GEMV interfaces shared between translation units.
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
  EPI_STORE = 0,       // out[m][col] = value
  EPI_ACCUMULATE = 1,  // out[m][col] += value
  EPI_SWIGLU = 2,      // seg0 = gate, seg1 = up, same panel per block:
                       // sw_out[m][col] = up*gate*sigmoid(gate)
  EPI_ARGMAX = 3,      // LM head: logits (optional) + per-block argmax
  EPI_RESID = 4,       // out[m][col] = resid[m][col] + value (and out2)
};

// Activation rows enter the MFMA as four signed int8 limbs of a per-row
// fixed-point value X = rint(y * 2^s), |X| < 2^30:  y * 2^s = sum_l limb_l 2^(8l).
// The weights enter as signed bytes n - 8 (n the nibble), so each limb's
// integer dot product sum_k limb_l(k) (n_k - 8) is exact in int32; the limbs
// are combined in int64 and scaled by 2^-s and the tensor scale once per output.
enum GemvASource {
  AS_ROWS = 0,   // prologue: every block quantizes the fp32 rows into LDS
  AS_QUANT = 1,  // limbs prepared in global memory by launch_quant_rows
  AS_ATTN = 2,   // one row: the attention chunks of k_attn_part, merged per
                 // query head by the wave that owns the head's K range
  AS_WAVES = 3,  // one to four rows: each wave quantizes its own contiguous
                 // K slice of every row with its own shift per row (no
                 // block-wide prologue); a row's RMSNorm factor is applied in
                 // the epilogue
  AS_WSTREAM = 4,  // AS_WAVES with the same slices, shifts and limbs, but each
                   // wave quantizes one 128-value super-tile of its rows at a
                   // time into a wave-private LDS buffer just before that
                   // tile's MFMAs (rows whose limbs would not fit in LDS)
};

// AS_ATTN: the chunk partials of one decode row (layout in attention.h:
// o [kDecPartMaxChunks][n_heads][hd], then (m, l)).  Wave w of the block owns
// head w, K = n_heads * hd with hd / 128 super-tiles per wave; it merges the
// head's chunks, quantizes the head with its own shift and multiplies its
// super-tiles, and the epilogue scales each wave's sums by its shift.
struct AttnSrc {
  const float *part;
  const int32_t *pos;   // position of the row
  int hd, n_heads;
  int circular, cache_len, clamp;
  int chunks;           // chunks the attention launch covered
};

// What the one-row Q|K|V projection prepares for the decode attention
// (k_attn_part) of the same layer: block 0 writes the RoPE factors of the
// row's position to rope_cur, so that the attention loads them at entry
// instead of after the position.  rope_cur == null: nothing.
struct AttnPrep {
  const int32_t *pos;          // position of the row
  const float *cos_t, *sin_t;  // [rope_rows][half]
  int half, rope_rows;
  float *rope_cur;             // [2][half]: cos, sin at the position
};

// fp32 rows and the transform applied before quantization:
// y = x * pre_scale; if norm: y *= 1/sqrt(mean(y^2) + 1e-6); if gamma: y *= gamma.
struct RowSrc {
  const float *x;      // [M][ld]
  int ld;
  float pre_scale;
  int norm;
  const float *gamma;  // or null
  float *y_out;        // y [M][K] (written once: block 0 or the quant kernel) or null
  float *x_out;        // copy of x [M][K] (same writer) or null
};

// Quantized rows in global memory: limb l of row m at
// limbs[(4m + l) * K + limb position of k] (MFMA fragment order per 128-row
// super-tile), shift[m] = s.  The GEMM's operand (launch_quant_rows3) has
// three limbs in planes: limb l of row m at limbs[(l * plane_rows + m) * K +
// limb position of k].
struct QuantRows {
  int8_t *limbs;
  int32_t *shift;
  int64_t *xsum;  // sum over the row of X (launch_quant_rows); the GEMM feeds
                  // unsigned nibbles n and subtracts 8 * xsum
  int plane_rows; // three-limb planes: rows per plane (0: four limbs per row)
};

struct GemvArgs {
  int epi;        // GemvEpilogue
  int asrc;       // GemvASource
  int K, M;
  RowSrc rows;    // AS_ROWS, AS_WAVES (no gamma, no x_out)
  QuantRows q;    // AS_QUANT
  AttnSrc at;     // AS_ATTN
  AttnPrep pf;    // AS_WAVES, one row, store epilogue: the decode attention's inputs
  GemvSeg seg[3];
  int nseg;
  int P;          // panels per block (EPI_SWIGLU: 2, gate and up)
  int waves;      // waves per block
  float *out;     // [M][ldo]
  int ldo;
  float *sw_out;  // EPI_SWIGLU: [M][ldo_sw]
  int ldo_sw;
  float *arg_val;    // EPI_ARGMAX: [blocks][M]
  int32_t *arg_idx;  // EPI_ARGMAX: [blocks][M]
  const float *resid;  // EPI_RESID: [M][ldo]
  float *out2;         // EPI_RESID: optional second copy [M][ldo]
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
  const int32_t *ids_in;  // [M] or null: ids already chosen (no reduction)
  int32_t *draws;         // or null: incremented once per launch (sampler draw counter)
};

// Prefill GEMM (gemm.hip): the rows of `a` are quantized for
// gemm_row_pad(M) rows (rows past M are read but never stored).
struct GemmArgs {
  int epi;        // EPI_STORE, EPI_ACCUMULATE, EPI_RESID or EPI_SWIGLU (gate, up)
  int M, K;
  QuantRows a;
  GemvSeg seg[3];
  int nseg;
  float *out;     // [M][ldo]
  int ldo;
  const float *resid;  // EPI_RESID: [M][ldo]
  float *out2;         // EPI_RESID: optional copy
  float *sw_out;       // EPI_SWIGLU: [M][ldo_sw]
  int ldo_sw;
  // K split over ksplit block groups (> 1: one segment, store or accumulate):
  // each group stores its exact partial sums, int64 [ksplit][M][N], and a
  // combine kernel adds them and scales (the same value as without the split)
  int ksplit;
  int64_t *kpart;
};

constexpr int kGemvMaxM = 16;
// AS_WAVES: at most this many rows, and K = waves * tpw * 128 (tpw super-tiles
// per wave; E4B: 5 on 4 waves for K = 2560 and on 16 for 10240; the demo
// model: 2 for K = 1024 on 4 waves and 4096 on 16)
constexpr int kWaveRowsMax = 4;
constexpr int kQuantMaxK = 16384;  // longest row a 1024-thread block quantizes

int launch_gemv(const GemvArgs &a, hipStream_t st);
// (epilogue, panels, waves, K) of a GemvArgs that an AS_WAVES launch takes:
// store with 4 waves (tpw 2, 5) or 8 (tpw 1, 2, 4), accumulate with 8, SwiGLU
// with 4 (tpw 2, 5), residual with 16 (tpw 2, 5) or 8 (tpw 1, 2, 4)
bool wave_shape_ok(const GemvArgs &a);
// LDS bytes a GEMV launch needs.
size_t gemv_lds_need(const GemvArgs &a);
// Quantize M rows of length K (one block per row) into q.
int launch_quant_rows(const RowSrc &r, int M, int K, const QuantRows &q, hipStream_t st);
// Device bytes of a QuantRows buffer for M rows of length K (limbs, shifts,
// row sums).
size_t quant_rows_bytes(int M, int K);
// Carve a QuantRows view out of one buffer of quant_rows_bytes(M, K).
QuantRows quant_rows_view(void *buf, int M, int K);
// The GEMM's operand: M rows (of Mp = gemm_row_pad(M) in the planes) as 22-bit
// fixed point (max |y| 2^s < 2^22) in three int8 limbs, limb planes of Mp
// rows.  The view fits in a buffer of quant_rows_bytes(Mp, K).
QuantRows quant_rows3_view(void *buf, int Mp, int K);
int launch_quant_rows3(const RowSrc &r, int M, int K, const QuantRows &q, hipStream_t st);
int pack_device(uint8_t *dst, const uint8_t *src, int K, int N, hipStream_t st);
int launch_argmax_fin(const ArgmaxFin &f, hipStream_t st);
int launch_gemm(const GemmArgs &g, hipStream_t st);
// K parts for C = A deq(W) with M rows, one segment: > 1 where the 32-row
// GEMM would leave most CUs idle (a few row and column tiles, long K)
int gemm_ksplit(int M, int K, int N);
// Rows a GEMM reads from its quantized operand (M rounded up to the row tile).
int gemm_row_pad(int M);

}  // namespace ms
