// Q4 GEMM for prefill rows (M > 16) on v_mfma_i32_16x16x64_i8.
//
// The A operand: activation rows quantized by launch_quant_rows3 to 22-bit
// fixed point, X = rint(y 2^s) with max |y| 2^s < 2^22 (s per row), in three
// balanced int8 limbs stored as limb planes (plane l: limb l of every row, in
// the MFMA fragment order of the GEMV's limb rows inside each 128-row
// super-tile of K).  An A tile is 16 rows of one limb plane, so the D fragment
// of limb l gives lane j + 16r the limb-l sums of rows 4r .. 4r + 3 at column
// j, and the three limbs of an output meet in one lane.  (The GEMV's four
// limbs, 31-bit fixed point, would cost a third more MFMAs here, where the
// MFMAs set the time; 22 bits keep every row within 2^-23 of its maximum,
// the rounding of an fp32 product.)  The weights enter as the unsigned
// nibbles n straight from the panel layout (a mask per dword), and the zero
// point comes back per row: sum_k X_k (n_k - 8) = sum_k X_k n_k - 8 * xsum,
// with xsum = sum_k X_k from the quantization.  Each limb's dot product is
// exact in int32; the three limbs of an output combine exactly
// (limb_combine3), minus 8 * xsum, and are scaled by 2^-s and the tensor
// scale.  launch_gemm picks the 32-row kernel (k_gemm) or the big tile
// (k_gemm_big, described further down) per launch.
//
// k_gemm tiling: a block computes kBM = 32 activation rows (96 limb rows, 6 MFMA A
// tiles) by 4 kWB panels (8 panels, 128 columns).  Wave (wa, wb) owns rows
// 16wa..16wa+15 (one A tile per limb) and panels 4wb..4wb+3: 12 accumulators
// and 24 MFMAs per 128-row step of K.  Both operands of a step (A 96 limb rows
// x 128 bytes, B one 1 KiB super-tile of each panel) go from global memory
// straight into LDS (global_load_lds: each wave instruction fills 1 KiB), in
// a ring of three steps; loads run two steps ahead of the MFMAs, which a
// step's MFMA time alone does not cover.  A limb rows are stored without
// padding, chunk c of row r at chunk position c ^ a_swz(r), so the rows one
// fragment read touches fall in different bank groups.
//
// EPI_SWIGLU: the first half of the wave columns computes gate panels, the
// second half the up panels of the same columns; the gate values pass through
// LDS and the up waves write up * gate * sigmoid(gate) (swiglu_inplace,
// kernels.mojo:519-532).
#include <algorithm>

#include "devutil.h"
#include "q4.h"

namespace ms {
namespace {

constexpr int kBM = 32;                  // activation rows per block
constexpr int kWB = 2;                   // wave columns: 4 panels each
constexpr int kNT = 128 * kWB;           // threads (2 wave rows x kWB wave columns)
constexpr int kLimbs = 3;                // limb planes of the A operand
constexpr int kAstage = kLimbs * kBM * 128;  // one K step of A: 96 limb rows x 128 bytes
constexpr int kBstage = 8 * 1024;        // one super-tile of each of the 8 panels
constexpr int kStage = kAstage + kBstage;
constexpr int kStages = 3;               // K steps resident in LDS
constexpr int kGemmLds = kStages * kStage;  // 60 KiB
constexpr int kLoads = 5;                // direct loads per thread per K step

typedef __attribute__((address_space(3))) void lds_void;

// LDS position of 16-byte chunk c of A limb row r: c ^ a_swz(r).  The rows
// one A fragment read touches are r0 + 0..15; a 16-byte read goes in phases
// of 8 lanes over 32 banks of 4 bytes (128 bytes per phase), so rows
// r .. r + 7 must take 8 different chunk positions (r & 7), and rows r and
// r + 8 of a 16-lane phase a different one again (the bit r >> 3).
__device__ inline int a_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// Panel pi of the GEMM's 1-3 weight segments (concatenated): its weights,
// scale, first output column and whether it exists.  The candidates come in
// as values: a lambda capturing them would keep them in private memory and
// turn the block-uniform selects into an indexed scratch load.
__device__ inline void seg_panel(int pi, int K, const uint8_t *w0, const uint8_t *w1,
                                 const uint8_t *w2, float s0, float s1, float s2, int n0,
                                 int n1, int n2, int c0, int c1, int c2, const uint8_t **w,
                                 float *sc, int *col, bool *ok) {
  const int si = pi < n0 ? 0 : (pi < n0 + n1 ? 1 : 2);
  const int loc = pi - (si == 0 ? 0 : (si == 1 ? n0 : n0 + n1));
  *ok = pi < n0 + n1 + n2;
  const uint8_t *base = si == 0 ? w0 : (si == 1 ? w1 : w2);
  *w = *ok ? base + (size_t)loc * K * 8 : w0;
  *sc = si == 0 ? s0 : (si == 1 ? s1 : s2);
  *col = (si == 0 ? c0 : (si == 1 ? c1 : c2)) + loc * 16;
}
typedef const __attribute__((address_space(1))) void gbl_void;

// Exact limb combine of one output, minus the zero-point term z: each limb's
// int32 dot product is below 2^25 in magnitude (K <= 16384, |limb| <= 128,
// nibble <= 15), so d0 + 2^8 d1 + 2^16 d2 - z is an integer below 2^43,
// formed exactly in double by FMAs.
__device__ inline double limb_combine3(int d0, int d1, int d2, double z) {
  return __builtin_fma((double)d2, 65536.0, __builtin_fma((double)d1, 256.0, (double)d0)) - z;
}

template <int EPI>
__global__ __launch_bounds__(kNT) void k_gemm(GemmArgs g) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int M = launder(g.M), K = launder(g.K);
  const int8_t *limbs = launder(g.a.limbs);
  const int32_t *shift = launder(g.a.shift);
  const int64_t *xsum = launder(g.a.xsum);
  const uint8_t *sw0 = launder(g.seg[0].w), *sw1 = launder(g.seg[1].w),
                *sw2 = launder(g.seg[2].w);
  const float ss0 = launder(g.seg[0].scale), ss1 = launder(g.seg[1].scale),
              ss2 = launder(g.seg[2].scale);
  const int nseg = launder(g.nseg);
  const int sn0 = launder(g.seg[0].n_cols) >> 4;
  const int sn1 = nseg > 1 ? launder(g.seg[1].n_cols) >> 4 : 0;
  const int sn2 = nseg > 2 ? launder(g.seg[2].n_cols) >> 4 : 0;
  const int sc0 = launder(g.seg[0].out_col0), sc1 = launder(g.seg[1].out_col0),
            sc2 = launder(g.seg[2].out_col0);
  float *out = launder(g.out);
  const int ldo = launder(g.ldo);
  const float *resid = EPI == EPI_RESID ? launder(g.resid) : nullptr;
  float *out2 = EPI == EPI_RESID ? launder(g.out2) : nullptr;
  float *sw_out = EPI == EPI_SWIGLU ? launder(g.sw_out) : nullptr;
  const int ldo_sw = EPI == EPI_SWIGLU ? launder(g.ldo_sw) : 0;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int wa = wave & 1, wb = wave >> 1;
  // EPI_SWIGLU: wave columns [0, kWB/2) hold gate panels, the rest the up
  // panels of the same columns
  const int half = wb / (kWB / 2), sub = wb % (kWB / 2);
  const int r0 = blockIdx.y * kBM;
  const int KG = K >> 7;

  // panel slot sl of the block's 8 -> weights, scale, first column, valid
  // (block-uniform selects).  EPI_SWIGLU: slots 0-3 gate, 4-7 up panels of
  // the same 4 column groups.
  auto slot = [&](int sl, const uint8_t **w, float *sc, int *cl, bool *ok) {
    if constexpr (EPI == EPI_SWIGLU) {
      const int hf = sl >> 2, cp = blockIdx.x * 4 + (sl & 3);
      *ok = cp < sn0;
      *w = (hf == 0 ? sw0 : sw1) + (size_t)(*ok ? cp : 0) * K * 8;
      *sc = hf == 0 ? ss0 : ss1;
      *cl = cp * 16;
    } else {
      seg_panel(blockIdx.x * 8 + sl, K, sw0, sw1, sw2, ss0, ss1, ss2, sn0, sn1, sn2, sc0, sc1,
                sc2, w, sc, cl, ok);
    }
  };
  // the panels this wave computes: slots 4 wb .. 4 wb + 3
  float wsc[4];
  int col[4];
  bool pv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint8_t *w;
    slot(4 * wb + j, &w, &wsc[j], &col[j], &pv[j]);
  }
  // the panels this wave loads: slots 2 wave, 2 wave + 1 (an invalid slot
  // loads a valid panel, so every wave issues the same number of loads)
  const uint8_t *lw[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    float sc;
    int cl;
    bool ok;
    slot(2 * wave + j, &lw[j], &sc, &cl, &ok);
  }

  // A: a stage holds limb rows 32l + m (limb l of block row m); this wave
  // fills LDS blocks 3 wave + i (stage rows 8q .. 8q + 7); lane l writes row
  // 8q + l / 8 at chunk position l % 8, which holds chunk (l % 8) ^
  // a_swz(row) of the row, so the rows one fragment read touches fall in
  // different bank groups
  const int pr = launder(g.a.plane_rows);
  const int8_t *asrc[kLimbs];
#pragma unroll
  for (int i = 0; i < kLimbs; ++i) {
    const int row = 8 * (kLimbs * wave + i) + (lane >> 3);
    const int c = (lane & 7) ^ a_swz(row);
    asrc[i] = limbs + ((size_t)(row >> 5) * pr + r0 + (row & 31)) * K + c * 16;
  }
  // K step G into stage stg: global memory straight into LDS
  auto issue = [&](int G, int stg) {
    uint8_t *sa = lds + stg * kStage;
#pragma unroll
    for (int i = 0; i < kLimbs; ++i)
      __builtin_amdgcn_global_load_lds((gbl_void *)(asrc[i] + (size_t)G * 128),
                                       (lds_void *)(sa + (kLimbs * wave + i) * 1024), 16, 0, 0);
#pragma unroll
    for (int j = 0; j < 2; ++j)
      __builtin_amdgcn_global_load_lds((gbl_void *)(lw[j] + (size_t)G * 1024 + lane * 16),
                                       (lds_void *)(sa + kAstage + (2 * wave + j) * 1024), 16,
                                       0, 0);
  };

  // acc[l][j]: limb l of block rows 16 wa .. 16 wa + 15, panel 4 wb + j
  v4i acc[kLimbs][4];
#pragma unroll
  for (int a = 0; a < kLimbs; ++a)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[a][j] = v4i{0, 0, 0, 0};

  const int li = lane & 15, lg = lane >> 4;
  const int swz = a_swz(li);  // a_swz(row) for every row this lane reads
  auto compute = [&](int stg) {
    const uint8_t *sa = lds + stg * kStage;
    u32x4 braw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      braw[j] = *reinterpret_cast<const u32x4 *>(sa + kAstage + (4 * wb + j) * 1024 + lane * 16);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v4i bf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t d0 = braw[j][2 * h], d1 = braw[j][2 * h + 1];
        bf[j] = v4i{(int)(d0 & 0x0F0F0F0Fu), (int)((d0 >> 4) & 0x0F0F0F0Fu),
                    (int)(d1 & 0x0F0F0F0Fu), (int)((d1 >> 4) & 0x0F0F0F0Fu)};
      }
      const int pos = (2 * lg + h) ^ swz;
#pragma unroll
      for (int a = 0; a < kLimbs; ++a) {
        const v4i af = *reinterpret_cast<const v4i *>(sa + (32 * a + 16 * wa + li) * 128 +
                                                      pos * 16);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[a][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf[j], acc[a][j], 0, 0, 0);
      }
    }
  };

  // the epilogue's row shifts and sums, loaded before the K loop: lane
  // j + 16 rr holds rows 16 wa + 4 rr + i of column j (rows past M: shift
  // 0, sum 0; their outputs are not stored)
  int32_t rsh[4];
  double rz[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = r0 + 16 * wa + 4 * (lane >> 4) + i;
    rsh[i] = row < M ? ldg<int32_t>(shift + row) : 0;
    rz[i] = row < M ? (double)(8 * ldg<long long>(xsum + row)) : 0.0;
  }

  // K steps of this block: all of them, or part blockIdx.z of ksplit
  const int ks = launder(g.ksplit) > 1 ? launder(g.ksplit) : 1;
  const int G0 = (int)((long)KG * blockIdx.z / ks), NG = (int)((long)KG * (blockIdx.z + 1) / ks) - G0;

  // Ring of kStages K steps: step i + 2 is issued into the stage step i - 1
  // used, once every wave has passed the barrier after computing it.  The
  // barrier is a bare s_barrier: this wave's own loads of step i are waited
  // for explicitly, and those of step i + 1 stay in flight (a __syncthreads
  // would wait for them too).
  issue(G0, 0);
  if (NG > 1) issue(G0 + 1, 1);
  for (int i = 0; i < NG; ++i) {
    if (i + 1 < NG)
      __builtin_amdgcn_s_waitcnt(0x0F70 | kLoads);  // vmcnt(6)
    else
      __builtin_amdgcn_s_waitcnt(0x0F70);           // vmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (i + 2 < NG) issue(G0 + i + 2, (i + 2) % kStages);
    compute(i % kStages);
  }

  // ---- epilogue: lane (column jc, row rr of each A tile)
  const int jc = lane & 15, rr = lane >> 4;
  if constexpr (EPI == EPI_STORE || EPI == EPI_ACCUMULATE) {
    if (ks > 1) {
      // this part's exact sums d0 + 2^8 d1 + 2^16 d2 (k_gemm_kcombine)
      int64_t *kp = launder(g.kpart) + (size_t)blockIdx.z * M * ldo;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = r0 + 16 * wa + 4 * rr + i;
        if (row >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (!pv[j]) continue;
          kp[(size_t)row * ldo + col[j] + jc] = (int64_t)acc[0][j][i] +
                                                ((int64_t)acc[1][j][i] << 8) +
                                                ((int64_t)acc[2][j][i] << 16);
        }
      }
      return;
    }
  }
  float v[4][4];  // [row i][panel j]
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float sc = ldexpf(1.0f, -rsh[i]);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      v[i][j] = (float)(limb_combine3(acc[0][j][i], acc[1][j][i], acc[2][j][i], rz[i]) *
                        (double)sc * (double)wsc[j]);
  }
  if constexpr (EPI == EPI_SWIGLU) {
    // gate values of wave (wa, sub) -> LDS -> up wave (wa, sub)
    __syncthreads();  // every wave is done reading the operand stages
    float *xg = reinterpret_cast<float *>(lds);
    const int xo = (wa * (kWB / 2) + sub) * 16;
    if (half == 0) {
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int j = 0; j < 4; ++j) xg[(xo + a * 4 + j) * 64 + lane] = v[a][j];
    }
    __syncthreads();
    if (half == 1) {
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const int row = r0 + 16 * wa + 4 * rr + a;
        if (row >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (!pv[j]) continue;
          const float gt = xg[(xo + a * 4 + j) * 64 + lane], up = v[a][j];
          sw_out[(size_t)row * ldo_sw + col[j] + jc] = up * gt * (1.0f / (1.0f + expf(-gt)));
        }
      }
    }
  } else {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int row = r0 + 16 * wa + 4 * rr + a;
      if (row >= M) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (!pv[j]) continue;
        const size_t oi = (size_t)row * ldo + col[j] + jc;
        if constexpr (EPI == EPI_STORE) {
          out[oi] = v[a][j];
        } else if constexpr (EPI == EPI_ACCUMULATE) {
          out[oi] += v[a][j];
        } else {
          const float x = resid[oi] + v[a][j];
          out[oi] = x;
          if (out2) out2[oi] = x;
        }
      }
    }
  }
}

// ------------------------------------------------------------------------------
// Big-tile variant for GEMMs with many blocks.  A block computes kGBM = 32
// activation rows (96 limb rows) by kGPan = 16 panel slots (SwiGLU: the gate
// and the up panels of 8 column groups).  Four waves; wave (wr, wc) owns rows
// 16wr..16wr+15 (one A tile per limb) and 8 panel slots: 24 accumulators.
// Both operands of a K step (A 12 KiB, B 16 KiB) go from global memory
// straight into LDS (global_load_lds_dwordx4: each wave instruction fills
// 1 KiB, lane l the 16 bytes at l * 16), in a ring of two steps: 56 KiB, so
// two blocks share a CU and one block's barriers, pipeline start and epilogue
// overlap the other's MFMAs (with one 8-wave block per CU, the per-step
// barrier and the epilogue left the MFMA units idle for a third of the time).
// A limb rows are stored without padding, the 16-byte chunk c of row r at
// chunk position c ^ a_swz(r): the rows one A fragment read touches then fall
// in different bank groups.
//
// EPI_SWIGLU: wave column wc holds the gate panels of column groups
// CGW wc .. CGW wc + CGW - 1 (slots j < CGW, CGW = PS / 4) and the up panels
// of the same groups (j >= CGW), so each output's gate and up values meet in
// one lane.
//
// PS = 16 panel slots per block, 20 (wave tile 3 A tiles x 10 panels) or 10
// (3 x 5) for launches whose 16-slot tiles leave a last round of blocks
// mostly empty: O and Down at 2048 rows (N = 160 panels) make 512
// twenty-slot tiles, one full round at two blocks per CU, against 640
// sixteen-slot ones (1.25 rounds).  The 20-slot tile also reads each A step
// for 20 panels instead of 16 or 10.  For SwiGLU a block of PS slots holds
// the gate and up panels of PS / 2 column groups, PS / 4 per wave column.
// ------------------------------------------------------------------------------
constexpr int kGBM = 32;                     // activation rows per block
constexpr int kGPan = 16;                    // panel slots per block (wide tile)
constexpr int kGPanNarrow = 10;              // panel slots per block (narrow tile)
constexpr int kGPanWide = 20;                // panel slots per block (20-slot tile)
constexpr int kGStageA = kLimbs * kGBM * 128;  // 96 limb rows x 128 bytes
constexpr int kGStages = 2;
constexpr int kGNT = 256;                    // threads per block
// one super-tile per panel slot after the A step; two stages
constexpr int gemm_big_stage(int ps) { return kGStageA + ps * 1024; }
constexpr int gemm_big_lds(int ps) { return kGStages * gemm_big_stage(ps); }

template <int EPI, int PS>
__global__ __launch_bounds__(kGNT, 2) void k_gemm_big(GemmArgs g) {
  static_assert(PS == kGPan || PS == kGPanWide || (PS == kGPanNarrow && EPI != EPI_SWIGLU),
                "panel slots");
  constexpr int PW = PS / 2;                 // panel slots per wave
  constexpr int CG = PS / 2;                 // SwiGLU: column groups per block
  constexpr int CGW = CG / 2;                // SwiGLU: column groups per wave column
  constexpr int kGStage = gemm_big_stage(PS);
  extern __shared__ __align__(16) uint8_t lds[];
  const int M = launder(g.M), K = launder(g.K);
  const int8_t *limbs = launder(g.a.limbs);
  const int32_t *shift = launder(g.a.shift);
  const int64_t *xsum = launder(g.a.xsum);
  const uint8_t *sw0 = launder(g.seg[0].w), *sw1 = launder(g.seg[1].w),
                *sw2 = launder(g.seg[2].w);
  const float ss0 = launder(g.seg[0].scale), ss1 = launder(g.seg[1].scale),
              ss2 = launder(g.seg[2].scale);
  const int nseg = launder(g.nseg);
  const int sn0 = launder(g.seg[0].n_cols) >> 4;
  const int sn1 = nseg > 1 ? launder(g.seg[1].n_cols) >> 4 : 0;
  const int sn2 = nseg > 2 ? launder(g.seg[2].n_cols) >> 4 : 0;
  const int sc0 = launder(g.seg[0].out_col0), sc1 = launder(g.seg[1].out_col0),
            sc2 = launder(g.seg[2].out_col0);
  float *out = launder(g.out);
  const int ldo = launder(g.ldo);
  const float *resid = EPI == EPI_RESID ? launder(g.resid) : nullptr;
  float *out2 = EPI == EPI_RESID ? launder(g.out2) : nullptr;
  float *sw_out = EPI == EPI_SWIGLU ? launder(g.sw_out) : nullptr;
  const int ldo_sw = EPI == EPI_SWIGLU ? launder(g.ldo_sw) : 0;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int wr = wave & 1, wc = wave >> 1;
  const int r0 = blockIdx.y * kGBM;
  const int KG = K >> 7;

  // panel slot -> weights, scale, first column, valid (block-uniform selects)
  auto slot = [=](int sl, const uint8_t **w, float *sc, int *col, bool *ok) {
    if constexpr (EPI == EPI_SWIGLU) {
      const int half = sl / CG, cp = blockIdx.x * CG + sl % CG;
      *ok = cp < sn0;
      *w = (half == 0 ? sw0 : sw1) + (size_t)(*ok ? cp : 0) * K * 8;
      *sc = half == 0 ? ss0 : ss1;
      *col = cp * 16;
    } else {
      seg_panel(blockIdx.x * PS + sl, K, sw0, sw1, sw2, ss0, ss1, ss2, sn0, sn1, sn2, sc0, sc1,
                sc2, w, sc, col, ok);
    }
  };
  // the panel slot of this wave's accumulator column j
  auto wslot = [&](int j) {
    if constexpr (EPI == EPI_SWIGLU) return j < CGW ? CGW * wc + j : CG + CGW * wc + (j - CGW);
    else return PW * wc + j;
  };
  // this wave loads panel slots wave, wave + 4, .. (an invalid slot loads a
  // valid panel)
  constexpr int kBL = (PS + 3) / 4;  // B loads per wave per step (the most)
  const uint8_t *lw[kBL];
#pragma unroll
  for (int j = 0; j < kBL; ++j) {
    float sc;
    int col;
    bool ok;
    slot(wave + 4 * j < PS ? wave + 4 * j : wave, &lw[j], &sc, &col, &ok);
  }
  // A: a stage holds limb rows 32l + m (limb l of block row m); this wave
  // fills LDS blocks 3 wave + i (stage rows 8q .. 8q + 7); lane l writes row
  // 8q + l / 8 at chunk position l % 8, which holds chunk (l % 8) ^
  // a_swz(row) of the row
  const int pr = launder(g.a.plane_rows);
  const int8_t *asrc[kLimbs];
#pragma unroll
  for (int i = 0; i < kLimbs; ++i) {
    const int row = 8 * (kLimbs * wave + i) + (lane >> 3);
    const int c = (lane & 7) ^ a_swz(row);
    asrc[i] = limbs + ((size_t)(row >> 5) * pr + r0 + (row & 31)) * K + c * 16;
  }
  auto issue = [&](int G, int stg) {
    uint8_t *sa = lds + stg * kGStage;
#pragma unroll
    for (int i = 0; i < kLimbs; ++i)
      __builtin_amdgcn_global_load_lds((gbl_void *)(asrc[i] + (size_t)G * 128),
                                       (lds_void *)(sa + (kLimbs * wave + i) * 1024), 16, 0, 0);
#pragma unroll
    for (int j = 0; j < kBL; ++j)
      if (wave + 4 * j < PS)
        __builtin_amdgcn_global_load_lds((gbl_void *)(lw[j] + (size_t)G * 1024 + lane * 16),
                                         (lds_void *)(sa + kGStageA + (wave + 4 * j) * 1024), 16,
                                         0, 0);
  };

  // acc[l][j]: limb l of block rows 16 wr .. 16 wr + 15, panel slot wslot(j)
  v4i acc[kLimbs][PW];
#pragma unroll
  for (int a = 0; a < kLimbs; ++a)
#pragma unroll
    for (int j = 0; j < PW; ++j) acc[a][j] = v4i{0, 0, 0, 0};

  const int li = lane & 15, lg = lane >> 4;
  const int swz = a_swz(li);  // a_swz(row) for every row this lane reads
  auto compute = [&](int stg) {
    const uint8_t *sa = lds + stg * kGStage;
    const uint8_t *sb = sa + kGStageA + lane * 16;
    u32x4 braw[PW];
#pragma unroll
    for (int j = 0; j < PW; ++j) braw[j] = *reinterpret_cast<const u32x4 *>(sb + wslot(j) * 1024);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v4i bf[PW];
#pragma unroll
      for (int j = 0; j < PW; ++j) {
        const uint32_t d0 = braw[j][2 * h], d1 = braw[j][2 * h + 1];
        bf[j] = v4i{(int)(d0 & 0x0F0F0F0Fu), (int)((d0 >> 4) & 0x0F0F0F0Fu),
                    (int)(d1 & 0x0F0F0F0Fu), (int)((d1 >> 4) & 0x0F0F0F0Fu)};
      }
      const int pos = (2 * lg + h) ^ swz;
#pragma unroll
      for (int a = 0; a < kLimbs; ++a) {
        const v4i af = *reinterpret_cast<const v4i *>(sa + (32 * a + 16 * wr + li) * 128 +
                                                      pos * 16);
#pragma unroll
        for (int j = 0; j < PW; ++j)
          acc[a][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf[j], acc[a][j], 0, 0, 0);
      }
    }
  };

  // Ring of two K steps: step G + 1 is issued into the stage step G - 1 used,
  // once every wave has passed the barrier after computing it.  The barrier
  // is a bare s_barrier after this wave's own loads of step G have landed.
  issue(0, 0);
  for (int G = 0; G < KG; ++G) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (G + 1 < KG) issue(G + 1, (G + 1) & 1);
    compute(G & 1);
  }

  // ---- epilogue: lane (column jc, row rr of each A tile)
  const int jc = lane & 15, rr = lane >> 4;
  // lane j + 16 rr holds rows 16 wr + 4 rr + i of column j
  double rsc[4], rz[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = r0 + 16 * wr + 4 * (lane >> 4) + i;
    rsc[i] = row < M ? (double)ldexpf(1.0f, -ldg<int32_t>(shift + row)) : 0.0;
    rz[i] = row < M ? (double)(8 * ldg<long long>(xsum + row)) : 0.0;
  }
  float wsc[PW];
  int col[PW];
  bool pv[PW];
#pragma unroll
  for (int j = 0; j < PW; ++j) {
    const uint8_t *w;
    slot(wslot(j), &w, &wsc[j], &col[j], &pv[j]);
  }
  auto value = [&](int i, int j) {
    return (float)(limb_combine3(acc[0][j][i], acc[1][j][i], acc[2][j][i], rz[i]) * rsc[i] *
                   (double)wsc[j]);
  };
  if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int row = r0 + 16 * wr + 4 * rr + a;
      if (row >= M) continue;
#pragma unroll
      for (int j = 0; j < CGW; ++j) {
        if (!pv[j]) continue;
        const float gt = value(a, j), up = value(a, j + CGW);
        sw_out[(size_t)row * ldo_sw + col[j] + jc] = up * gt * (1.0f / (1.0f + expf(-gt)));
      }
    }
  } else {
#pragma unroll
    for (int a = 0; a < 4; ++a) {
      const int row = r0 + 16 * wr + 4 * rr + a;
      if (row >= M) continue;
#pragma unroll
      for (int j = 0; j < PW; ++j) {
        if (!pv[j]) continue;
        const size_t oi = (size_t)row * ldo + col[j] + jc;
        const float x = value(a, j);
        if constexpr (EPI == EPI_STORE) {
          out[oi] = x;
        } else if constexpr (EPI == EPI_ACCUMULATE) {
          out[oi] += x;
        } else {
          const float y = resid[oi] + x;
          out[oi] = y;
          if (out2) out2[oi] = y;
        }
      }
    }
  }
}

}  // namespace

// Rows of the quantized operand a GEMM reads: the big tile's row block.
int gemm_row_pad(int M) { return (M + kGBM - 1) / kGBM * kGBM; }

namespace {

// The kernel for a GEMM, from a model of its time in wide-tile K steps: a
// launch of B blocks runs ceil(B / slots) rounds (two blocks per CU); a K step
// of the 10-slot tile costs 0.85 of a 16-slot one (5/8 of the MFMAs, but more
// LDS reads and barriers per MFMA), and the 32-row, 8-panel kernel's 0.8: the
// factors that reproduce the measured choices (at 2048 rows O and Down run
// 146 us with 16 slots, 126 us with 10; at 512 rows the 32-row kernel's 49 us
// beat the 10-slot tile's 52).  (A split of K over several blocks, their
// exact partials meeting through a counter or in a second launch, was
// slower: see the notes on the measured variants.)
constexpr double kNarrowStepCost = 0.85;
// the 20-slot tile's K step: 1.25 times the MFMAs of a 16-slot one, less the
// A reads it saves (each A step serves 20 panels).  At 2048 rows O and Down
// make 512 twenty-slot tiles, one round (TTFT at 2048 tokens 32.9 -> 32.4
// ms), and Gate|Up 4096 tiles, 8 rounds against 10 (31.9 -> 31.4 ms; 512
// tokens 10.5 -> 10.3 ms)
constexpr double kWideStepCost = 1.2;
constexpr double kSmallStepCost = 0.8;

// 0: the 32-row kernel; else the big tile's panel slots (16, 20 or 10)
int gemm_pick(const GemmArgs &g, int np) {
  const bool swiglu = g.epi == EPI_SWIGLU;
  const long slots = 2L * (ctx().n_cu > 0 ? ctx().n_cu : 256);
  auto rounds = [&](long blocks) { return (double)((blocks + slots - 1) / slots); };
  const long rows = gemm_row_pad(g.M) / kGBM;
  const long wide = (long)(swiglu ? (np / 2 + 7) / 8 : (np + kGPan - 1) / kGPan) * rows;
  const long narrow = (long)((np + kGPanNarrow - 1) / kGPanNarrow) * rows;
  const long small = (long)(swiglu ? (np / 2 + 2 * kWB - 1) / (2 * kWB)
                                   : (np + 4 * kWB - 1) / (4 * kWB)) *
                     ((g.M + kBM - 1) / kBM);
  const long wide20 =
      (long)(swiglu ? (np / 2 + kGPanWide / 2 - 1) / (kGPanWide / 2)
                    : (np + kGPanWide - 1) / kGPanWide) * rows;
  int pick = kGPan;
  double cost = rounds(wide);
  if (rounds(wide20) * kWideStepCost < cost) {
    pick = kGPanWide;
    cost = rounds(wide20) * kWideStepCost;
  }
  if (!swiglu && rounds(narrow) * kNarrowStepCost < cost) {
    pick = kGPanNarrow;
    cost = rounds(narrow) * kNarrowStepCost;
  }
  if (rounds(small) * kSmallStepCost < cost) pick = 0;
  return pick;
}

template <int PS>
void launch_big(const GemmArgs &g, int np, hipStream_t st) {
  const int gxb = g.epi == EPI_SWIGLU ? (np / 2 + PS / 2 - 1) / (PS / 2) : (np + PS - 1) / PS;
  const dim3 grid(gxb, gemm_row_pad(g.M) / kGBM);
  const size_t lds = gemm_big_lds(PS);
  switch (g.epi) {
    case EPI_STORE: hipLaunchKernelGGL((k_gemm_big<EPI_STORE, PS>), grid, dim3(kGNT), lds, st, g); break;
    case EPI_ACCUMULATE:
      hipLaunchKernelGGL((k_gemm_big<EPI_ACCUMULATE, PS>), grid, dim3(kGNT), lds, st, g);
      break;
    case EPI_RESID: hipLaunchKernelGGL((k_gemm_big<EPI_RESID, PS>), grid, dim3(kGNT), lds, st, g); break;
    default:
      if constexpr (PS == kGPan || PS == kGPanWide)
        hipLaunchKernelGGL((k_gemm_big<EPI_SWIGLU, PS>), grid, dim3(kGNT), lds, st, g);
      break;
  }
}

}  // namespace

// The K parts of a split GEMM added and scaled: row `blockIdx.y`, 256
// columns per block.  The int64 sum is the exact integer the unsplit kernel
// forms with limb_combine, so every output equals the unsplit one.
template <int EPI>
__global__ __launch_bounds__(256) void k_gemm_kcombine(GemmArgs g) {
  const int M = g.M, N = g.ldo, ks = g.ksplit;
  const int row = blockIdx.y, c = blockIdx.x * 256 + threadIdx.x;
  if (c >= N) return;
  long long t = 0;
  for (int z = 0; z < ks; ++z) t += ldg<long long>(g.kpart + ((size_t)z * M + row) * N + c);
  const double z8 = (double)(8 * ldg<long long>(g.a.xsum + row));
  const float sc = ldexpf(1.0f, -ldg<int32_t>(g.a.shift + row));
  const float v = (float)(((double)t - z8) * (double)sc * (double)g.seg[0].scale);
  float *o = g.out + (size_t)row * N + c;
  if constexpr (EPI == EPI_STORE) *o = v;
  else *o += v;
}

int gemm_ksplit(int M, int K, int N) {
  if (M <= kGemvMaxM || K % 128 != 0 || N % 16 != 0) return 1;
  GemmArgs g{};
  g.epi = EPI_STORE;
  g.M = M;
  g.K = K;
  g.nseg = 1;
  const int np = N / 16;
  if (gemm_pick(g, np) != 0) return 1;
  const long blocks = (long)((np + 4 * kWB - 1) / (4 * kWB)) * ((M + kBM - 1) / kBM);
  const long cus = ctx().n_cu > 0 ? ctx().n_cu : 256;
  long ks = cus / blocks;
  ks = std::min<long>(ks, std::min(8, K / 128 / 8));  // at least 8 K steps a part
  return ks > 1 ? (int)ks : 1;
}

int launch_gemm(const GemmArgs &g, hipStream_t st) {
  MS_CHECK_ARG(g.M >= 1 && g.K >= 128 && g.K % 128 == 0 && g.K <= kQuantMaxK,
               "GEMM: K must be a multiple of 128 in [128, 16384]");
  MS_CHECK_ARG(g.a.limbs && g.a.shift && g.a.xsum, "GEMM: quantized rows missing");
  MS_CHECK_ARG(g.nseg >= 1 && g.nseg <= 3, "GEMM: 1..3 weight segments");
  for (int i = 0; i < g.nseg; ++i)
    MS_CHECK_ARG(g.seg[i].w && g.seg[i].n_cols > 0 && g.seg[i].n_cols % 16 == 0,
                 "GEMM: segment columns must be a positive multiple of 16");
  if (g.epi == EPI_STORE || g.epi == EPI_ACCUMULATE || g.epi == EPI_RESID) {
    MS_CHECK_ARG(g.out && g.ldo > 0, "GEMM: output missing");
    MS_CHECK_ARG(g.epi != EPI_RESID || g.resid, "GEMM: residual missing");
  } else if (g.epi == EPI_SWIGLU) {
    MS_CHECK_ARG(g.nseg == 2 && g.seg[0].n_cols == g.seg[1].n_cols && g.sw_out,
                 "GEMM: SwiGLU needs gate and up of equal width and an output");
  } else {
    return fail(MS_E_INVALID, "GEMM: unsupported epilogue");
  }
  int np = 0;
  for (int i = 0; i < g.nseg; ++i) np += g.seg[i].n_cols / 16;
  const bool swiglu = g.epi == EPI_SWIGLU;
  if (g.ksplit > 1) {
    MS_CHECK_ARG((g.epi == EPI_STORE || g.epi == EPI_ACCUMULATE) && g.nseg == 1 && g.kpart &&
                     g.ldo == g.seg[0].n_cols && g.ksplit <= g.K / 128,
                 "GEMM: K split needs one segment, store or accumulate, ldo = N");
    const dim3 grid((np + 4 * kWB - 1) / (4 * kWB), (g.M + kBM - 1) / kBM, g.ksplit);
    const dim3 cgrid((g.ldo + 255) / 256, g.M);
    if (g.epi == EPI_STORE) {
      hipLaunchKernelGGL(k_gemm<EPI_STORE>, grid, dim3(kNT), kGemmLds, st, g);
      hipLaunchKernelGGL(k_gemm_kcombine<EPI_STORE>, cgrid, dim3(256), 0, st, g);
    } else {
      hipLaunchKernelGGL(k_gemm<EPI_ACCUMULATE>, grid, dim3(kNT), kGemmLds, st, g);
      hipLaunchKernelGGL(k_gemm_kcombine<EPI_ACCUMULATE>, cgrid, dim3(256), 0, st, g);
    }
    MS_HIP_TRY(hipGetLastError());
    return MS_OK;
  }
  const int pick = gemm_pick(g, np);
  if (pick == kGPan) {
    launch_big<kGPan>(g, np, st);
  } else if (pick == kGPanWide) {
    launch_big<kGPanWide>(g, np, st);
  } else if (pick == kGPanNarrow) {
    launch_big<kGPanNarrow>(g, np, st);
  } else {
    const dim3 blk(kNT);
    const int gy = (g.M + kBM - 1) / kBM;
    const dim3 grid(swiglu ? (np / 2 + 2 * kWB - 1) / (2 * kWB) : (np + 4 * kWB - 1) / (4 * kWB),
                    gy);
#define MS_GS(E) hipLaunchKernelGGL(k_gemm<E>, grid, blk, kGemmLds, st, g)
    switch (g.epi) {
      case EPI_STORE: MS_GS(EPI_STORE); break;
      case EPI_ACCUMULATE: MS_GS(EPI_ACCUMULATE); break;
      case EPI_RESID: MS_GS(EPI_RESID); break;
      default: MS_GS(EPI_SWIGLU); break;
    }
#undef MS_GS
  }
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

}  // namespace ms
