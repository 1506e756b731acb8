// Q4 weight kernels for gfx950: panel repack, bit-exact dequant, and the
// MFMA GEMV used for decode (M <= 16 rows) with fused epilogues.
//
// Reference: matmul_q4_bpack_raw (kernels.mojo:201-267) computes
// C += A . deq(W) with w = (nibble-8)*scale.  Here the weights go into
// v_mfma_i32_16x16x64_i8 as signed bytes n-8 (a few bit operations per eight
// weights), each activation row as four int8 limbs of a 31-bit fixed-point
// value with a per-row power-of-two scale, so the dot product sum X*(n-8) is
// exact integer arithmetic; it is scaled by 2^-s and the tensor scale once per
// output.  For M <= 4 the 4M limb rows share one MFMA, so one MFMA covers
// 1024 weights.  Prefill rows (M > 16) go through the GEMM in gemm.hip, which
// uses the same operands and therefore gives the same values.
#include "attention.h"
#include "devutil.h"
#include "q4.h"

#include <cmath>
#include <vector>

namespace ms {

// ------------------------------------------------------------------------------
// packing
// ------------------------------------------------------------------------------
__global__ void k_pack(uint32_t *__restrict__ dst, const uint8_t *__restrict__ src,
                       int K, int N) {
  const size_t total = (size_t)K * N / 8;
  const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= total) return;
  const size_t per_panel = (size_t)K * 2;  // dwords per panel
  const int nb = (int)(i / per_panel);
  const int r = (int)(i % per_panel);
  const int G = r / 256, lane = (r % 256) / 4, t = r % 4;
  const int j = lane % 16, g = lane / 16;
  const int n = nb * 16 + j;
  const size_t pc = (size_t)N / 2;
  uint32_t d = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = 128 * G + 32 * g + 8 * t + e;
    const uint8_t b = src[(size_t)k * pc + (n >> 1)];
    const uint32_t nib = (n & 1) ? (uint32_t)(b >> 4) : (uint32_t)(b & 15);
    const int q = (e >> 1) + 4 * (e & 1);
    d |= nib << (4 * q);
  }
  dst[i] = d;
}

static int check_q4_shape(int K, int N) {
  MS_CHECK_ARG(K > 0 && N > 0, "Q4: K and N must be positive");
  MS_CHECK_ARG(K % kSuperK == 0, "Q4 panel layout needs K % 128 == 0");
  MS_CHECK_ARG(N % kPanelCols == 0, "Q4 panel layout needs N % 16 == 0");
  return MS_OK;
}

__global__ void k_dequant_rowmajor(float *__restrict__ out,
                                   const uint8_t *__restrict__ w, size_t nbytes,
                                   float scale) {
  const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= nbytes) return;
  const uint8_t b = w[i];
  // (nibble - 8) * scale: one exact int->fp32 conversion and one rounded
  // multiply, the same two operations as dequant_vec (kernels.mojo:100-108).
  out[2 * i] = (float)((int)(b & 15) - 8) * scale;
  out[2 * i + 1] = (float)((int)(b >> 4) - 8) * scale;
}

__global__ void k_dequant_packed(float *__restrict__ out,
                                 const uint32_t *__restrict__ w, int K, int N,
                                 float scale) {
  const size_t total = (size_t)K * N / 8;
  const size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= total) return;
  const size_t per_panel = (size_t)K * 2;
  const int nb = (int)(i / per_panel);
  const int r = (int)(i % per_panel);
  const int G = r / 256, lane = (r % 256) / 4, t = r % 4;
  const int j = lane % 16, g = lane / 16;
  const int n = nb * 16 + j;
  const uint32_t d = w[i];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = 128 * G + 32 * g + 8 * t + e;
    const int q = (e >> 1) + 4 * (e & 1);
    const int nib = (int)((d >> (4 * q)) & 15u);
    out[(size_t)k * N + n] = (float)(nib - 8) * scale;
  }
}

// ------------------------------------------------------------------------------
// helpers
// ------------------------------------------------------------------------------

// Wave reductions: DPP moves inside each 16-lane row (quad permutes, then
// the half-row and row mirrors leave the row total in every lane of the row),
// then readlane of the four row totals.  The result is wave-uniform.  No LDS
// round trips (a shuffle through ds_bpermute costs an LDS access and a wait
// per step).
template <int CTRL>
__device__ inline float dpp_f(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ inline float lane_f(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}
__device__ inline float row_sum16(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  return v;
}
__device__ inline float row_max16(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  return fmaxf(v, dpp_f<0x140>(v));
}
__device__ inline float wave_sum(float v) {
  v = row_sum16(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}
__device__ inline float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}

// Block reductions over NT threads; every thread returns the result.
// sh: >= 32 entries.  The block size is a template constant: reading blockDim
// loads it from the dispatch packet, and waiting for that load would also wait
// for every weight load already in flight.
template <int NT>
__device__ inline float block_sum(float v, float *sh) {
  constexpr int nw = NT / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) sh[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += sh[i];
  return t;
}
template <int NT>
__device__ inline float block_max(float v, float *sh) {
  constexpr int nw = NT / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) sh[w] = v;
  __syncthreads();
  float t = sh[0];
  for (int i = 1; i < nw; ++i) t = fmaxf(t, sh[i]);
  return t;
}

// ------------------------------------------------------------------------------
// Row quantization.
//
// Element order of the limb rows (MFMA fragment order): inside a 128-row
// super-tile, lane group g of the B operand holds rows 32g..32g+31 of its
// column, dword t = rows 8t..8t+7 with row e in nibble (e>>1) + 4(e&1).  The
// B fragment of MFMA h (two per super-tile) is the four dwords
// [d & 0x0F0F0F0F, (d >> 4) & 0x0F0F0F0F] of dwords t = 2h and 2h+1 (each byte
// then mapped to the signed value n - 8), so byte b
// of the low/high word holds rows e = {0,4,1,5} / {2,6,3,7}.  The A limbs are
// stored in that same order: an 8-row group t of lane group g lands at byte
// 128G + 32g + 16(t>>1) + 8(t&1), low word then high word.
// ------------------------------------------------------------------------------
__device__ inline int limb_pos8(int k) {
  return (k >> 7) * 128 + ((k >> 5) & 3) * 32 + ((k >> 4) & 1) * 16 + ((k >> 3) & 1) * 8;
}

// Rows of the 4x4 byte matrix with rows a, b, c, d: word l holds byte l of
// a, b, c, d (in that byte order).  v_perm_b32 picks bytes of {s0, s1} (s1 the
// low word): two rounds of four permutes.
__device__ inline void byte_transpose4(uint32_t a, uint32_t b, uint32_t c, uint32_t d,
                                       uint32_t (&r)[4]) {
  const uint32_t ab_lo = __builtin_amdgcn_perm(b, a, 0x05010400u);  // a0 b0 a1 b1
  const uint32_t ab_hi = __builtin_amdgcn_perm(b, a, 0x07030602u);  // a2 b2 a3 b3
  const uint32_t cd_lo = __builtin_amdgcn_perm(d, c, 0x05010400u);
  const uint32_t cd_hi = __builtin_amdgcn_perm(d, c, 0x07030602u);
  r[0] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x05040100u);  // a0 b0 c0 d0
  r[1] = __builtin_amdgcn_perm(cd_lo, ab_lo, 0x07060302u);
  r[2] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x05040100u);
  r[3] = __builtin_amdgcn_perm(cd_hi, ab_hi, 0x07060302u);
}

// X = rint(v * mul) for eight consecutive rows; limb l of the group as its
// low/high words.
//
// For |X| < 2^30 the bytes of E = (X + 0x80808080) ^ 0x80808080 are the four
// balanced limbs of X: X + 0x80808080 = sum_l u_l 2^(8l) with bytes u_l, so
// X = sum_l (u_l - 128) 2^(8l), and u_l - 128 as a signed byte is u_l ^ 0x80.
// The low word of limb l takes byte l of rows {0,4,1,5}, the high word rows
// {2,6,3,7}.
// *xs (XS): the sum of the eight X values.
template <bool XS = false>
__device__ inline void quant8(const float (&v)[8], float mul, uint32_t (&lo)[4],
                              uint32_t (&hi)[4], long long *xs = nullptr) {
  uint32_t E[8];
  long long sum = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int x = (int)rintf(v[e] * mul);
    if (XS) sum += x;
    E[e] = ((uint32_t)x + 0x80808080u) ^ 0x80808080u;
  }
  if (XS) *xs += sum;
  byte_transpose4(E[0], E[4], E[1], E[5], lo);
  byte_transpose4(E[2], E[6], E[3], E[7], hi);
}

// Per-row shift s with max|y| * 2^s < 2^30 (four limbs; 2^22 with three).
template <int LIMBS = 4>
__device__ inline int row_shift(float amax) {
  if (!(amax > 0.f)) return 0;
  int ex;
  (void)frexpf(amax, &ex);  // amax < 2^ex
  return (LIMBS == 4 ? 30 : 22) - ex;
}

// One row through NT threads, NG 8-row groups per thread (K <= 8 * NG * NT).
template <int NT, int NG, bool GAM>
struct RowRegs {
  float v[NG][8];
  float g[GAM ? NG : 1][8];
};

// Issue the loads of row m.  Threads past the end of the row load nothing (a
// clamped duplicate address would send every idle thread of every block to
// the same cache line).
template <int NT, int NG, bool GAM>
__device__ inline void row_load(const RowSrc &r, int K, int m, RowRegs<NT, NG, GAM> &R) {
  const int nq = K >> 3;
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    const int q = (int)threadIdx.x + gi * NT;
#pragma unroll
    for (int e = 0; e < 8; ++e) R.v[gi][e] = 0.f;
    if (GAM) {
#pragma unroll
      for (int e = 0; e < 8; ++e) R.g[gi][e] = 0.f;
    }
    if (q < nq) {
      const float *p = r.x + (size_t)m * r.ld + 8 * q;
      const float4 a = ldg<float4>(p), b = ldg<float4>(p + 4);
      R.v[gi][0] = a.x; R.v[gi][1] = a.y; R.v[gi][2] = a.z; R.v[gi][3] = a.w;
      R.v[gi][4] = b.x; R.v[gi][5] = b.y; R.v[gi][6] = b.z; R.v[gi][7] = b.w;
      if (GAM) {
        const float4 c = ldg<float4>(r.gamma + 8 * q), d = ldg<float4>(r.gamma + 8 * q + 4);
        R.g[gi][0] = c.x; R.g[gi][1] = c.y; R.g[gi][2] = c.z; R.g[gi][3] = c.w;
        R.g[gi][4] = d.x; R.g[gi][5] = d.y; R.g[gi][6] = d.z; R.g[gi][7] = d.w;
      }
    }
  }
}

// Sum of squares and maximum |value| over the block in one reduction pass.
// sh: >= 2 * 16 floats.  fresh (block-uniform): sh has not been used yet in
// this block, so no barrier is needed before writing it.
template <int NT>
__device__ inline void block_sum_max(float &ss, float &mx, float *sh, bool fresh = false) {
  constexpr int nw = NT / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  ss = wave_sum(ss);
  mx = wave_max(mx);
  if (!fresh) __syncthreads();
  if (lane == 0) {
    sh[w] = ss;
    sh[16 + w] = mx;
  }
  __syncthreads();
  float t = 0.f, u = 0.f;
#pragma unroll
  for (int i = 0; i < nw; ++i) {
    t += sh[i];
    u = fmaxf(u, sh[16 + i]);
  }
  ss = t;
  mx = u;
}

// Transform (x * pre_scale, rmsnorm, gamma: rmsnorm_inplace kernels.mojo:474-489,
// ple_scale_inplace :506-516, rmsnorm_weighted_inplace :598-613), optional
// fp32 stores by `writer`, quantization and limb stores: limb l of row m goes
// to dst + (4m + l) * ld_dst + limb position (LIMBS 3: dst + (l * planes + m)
// * ld_dst).  Returns the row shift s.
// XS: also the row's sum of X, exact (integer partial sums below 2^53 add
// exactly in double), into *xsum_out for every thread.
template <int NT, int NG, bool GAM, bool XS = false, int LIMBS = 4>
__device__ inline void row_finish(const RowSrc &r, int K, int m, bool writer,
                                  RowRegs<NT, NG, GAM> &R, int8_t *dst, size_t ld_dst,
                                  float *sh, int *s_out, double *xsum_out = nullptr,
                                  bool sh_fresh = false, int planes = 0) {
  const int nq = K >> 3;
  float y[NG][8];
  float ss = 0.f, mx = 0.f;
#pragma unroll
  for (int gi = 0; gi < NG; ++gi)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      y[gi][e] = R.v[gi][e] * r.pre_scale;
      ss += y[gi][e] * y[gi][e];
      mx = fmaxf(mx, fabsf(y[gi][e]));
    }
  // one reduction for the norm and the maximum (max|y * inv| = max|y| * inv)
  block_sum_max<NT>(ss, mx, sh, sh_fresh);
  float inv = 1.f;
  if (r.norm) {
    inv = 1.0f / sqrtf(ss / (float)K + 1e-6f);
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
#pragma unroll
      for (int e = 0; e < 8; ++e) y[gi][e] = y[gi][e] * inv;
  }
  float amax = mx * inv;
  if (GAM) {
    float gm = 0.f;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        y[gi][e] = y[gi][e] * R.g[gi][e];
        gm = fmaxf(gm, fabsf(y[gi][e]));
      }
    float dummy = 0.f;
    block_sum_max<NT>(dummy, gm, sh);
    amax = gm;
  } else {
    // mx * inv can round below the largest |y * inv|; one ulp of headroom
    amax = amax * (1.0f + 1.0f / 4194304.0f);
  }
  const int s = row_shift<LIMBS>(amax);
  const float mul = ldexpf(1.0f, s);
  long long xs = 0;
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    const int q = (int)threadIdx.x + gi * NT;
    if (q >= nq) continue;
    if (writer) {
      const size_t o = (size_t)m * K + 8 * q;
      if (r.y_out) {
        *reinterpret_cast<float4 *>(r.y_out + o) = float4{y[gi][0], y[gi][1], y[gi][2], y[gi][3]};
        *reinterpret_cast<float4 *>(r.y_out + o + 4) = float4{y[gi][4], y[gi][5], y[gi][6], y[gi][7]};
      }
      if (r.x_out) {
        *reinterpret_cast<float4 *>(r.x_out + o) =
            float4{R.v[gi][0], R.v[gi][1], R.v[gi][2], R.v[gi][3]};
        *reinterpret_cast<float4 *>(r.x_out + o + 4) =
            float4{R.v[gi][4], R.v[gi][5], R.v[gi][6], R.v[gi][7]};
      }
    }
    uint32_t lo[4], hi[4];
    quant8<XS>(y[gi], mul, lo, hi, &xs);
    const int pos = limb_pos8(8 * q);
#pragma unroll
    for (int l = 0; l < LIMBS; ++l) {
      const size_t row = LIMBS == 4 ? (size_t)(4 * m + l) : (size_t)l * planes + m;
      *reinterpret_cast<uint2 *>(dst + row * ld_dst + pos) = uint2{lo[l], hi[l]};
    }
  }
  *s_out = s;
  if constexpr (XS) {
    double v = (double)xs;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    __syncthreads();
    double *shd = reinterpret_cast<double *>(sh);
    if ((threadIdx.x & 63) == 0) shd[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) t += shd[i];
    *xsum_out = t;
  }
}

// One row per block of NT threads, NG groups of 8 values per thread
// (K <= 8 NG NT).  LIMBS 3: the GEMM's planes.
template <bool GAM, int NT, int LIMBS = 4, int NG = 2>
__global__ __launch_bounds__(NT) void k_quant_rows(RowSrc r, int K, QuantRows q) {
  __shared__ __align__(8) float sh[32];  // also 16 doubles (row sum)
  RowRegs<NT, NG, GAM> R;
  const int m = blockIdx.x;
  row_load<NT, NG, GAM>(r, K, m, R);
  int s;
  double xs;
  row_finish<NT, NG, GAM, true, LIMBS>(r, K, m, true, R, q.limbs, K, sh, &s, &xs, true,
                                       q.plane_rows);
  if (threadIdx.x == 0) {
    q.shift[m] = s;
    q.xsum[m] = (int64_t)xs;
  }
}

size_t quant_rows_bytes(int M, int K) {
  return (size_t)4 * M * K + 64 + (size_t)M * 4 + 64 + (size_t)M * 8;
}

QuantRows quant_rows_view(void *buf, int M, int K) {
  QuantRows q{};
  uint8_t *b = static_cast<uint8_t *>(buf);
  q.limbs = reinterpret_cast<int8_t *>(b);
  const size_t o1 = ((size_t)4 * M * K + 63) & ~(size_t)63;
  q.shift = reinterpret_cast<int32_t *>(b + o1);
  const size_t o2 = (o1 + (size_t)M * 4 + 63) & ~(size_t)63;
  q.xsum = reinterpret_cast<int64_t *>(b + o2);
  return q;
}

QuantRows quant_rows3_view(void *buf, int Mp, int K) {
  QuantRows q = quant_rows_view(buf, Mp, K);  // limbs first; three planes fit in four
  q.plane_rows = Mp;
  return q;
}

int launch_quant_rows3(const RowSrc &r, int M, int K, const QuantRows &q, hipStream_t st) {
  MS_CHECK_ARG(M >= 1 && K >= 8 && K % 8 == 0 && K <= kQuantMaxK,
               "quant: row length must be a multiple of 8 in [8, 16384]");
  MS_CHECK_ARG(r.x && r.ld >= K && q.limbs && q.shift && q.xsum && q.plane_rows >= M,
               "quant: missing buffers");
  if (K <= 16 * 256 && M >= 64) {
    if (r.gamma)
      hipLaunchKernelGGL((k_quant_rows<true, 256, 3>), dim3(M), dim3(256), 0, st, r, K, q);
    else
      hipLaunchKernelGGL((k_quant_rows<false, 256, 3>), dim3(M), dim3(256), 0, st, r, K, q);
  } else if (K <= 40 * 256 && M >= 64 && !r.gamma && !r.norm) {
    // long rows without a norm (the Down input, K = 10240): 256 threads of
    // five groups, so that more rows of a prompt chunk are resident at once
    // (1024-thread blocks fit two per CU: 2048 rows took four rounds).  Only
    // the maximum and the exact sum of X are reduced, so the limbs, shift
    // and sum equal those of the 1024-thread kernel.
    hipLaunchKernelGGL((k_quant_rows<false, 256, 3, 5>), dim3(M), dim3(256), 0, st, r, K, q);
  } else if (r.gamma) {
    hipLaunchKernelGGL((k_quant_rows<true, 1024, 3>), dim3(M), dim3(1024), 0, st, r, K, q);
  } else {
    hipLaunchKernelGGL((k_quant_rows<false, 1024, 3>), dim3(M), dim3(1024), 0, st, r, K, q);
  }
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

int launch_quant_rows(const RowSrc &r, int M, int K, const QuantRows &q, hipStream_t st) {
  MS_CHECK_ARG(M >= 1 && K >= 8 && K % 8 == 0 && K <= kQuantMaxK,
               "quant: row length must be a multiple of 8 in [8, 16384]");
  MS_CHECK_ARG(r.x && r.ld >= K && q.limbs && q.shift && q.xsum, "quant: missing buffers");
  // many rows of up to 4096 values on 256 threads: more rows per CU, shorter
  // reductions (a few decode rows keep the 1024 threads per row)
  if (K <= 16 * 256 && M >= 64) {
    if (r.gamma)
      hipLaunchKernelGGL((k_quant_rows<true, 256>), dim3(M), dim3(256), 0, st, r, K, q);
    else
      hipLaunchKernelGGL((k_quant_rows<false, 256>), dim3(M), dim3(256), 0, st, r, K, q);
  } else if (r.gamma) {
    hipLaunchKernelGGL((k_quant_rows<true, 1024>), dim3(M), dim3(1024), 0, st, r, K, q);
  } else {
    hipLaunchKernelGGL((k_quant_rows<false, 1024>), dim3(M), dim3(1024), 0, st, r, K, q);
  }
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

// ------------------------------------------------------------------------------
// MFMA GEMV: v_mfma_i32_16x16x64_i8 with the activation limbs as A (rows
// 4m + l) and the weight nibbles as B (16 columns of one panel).
// ------------------------------------------------------------------------------

// Resolve panel slot p of panel group pg with selects only (no loop over the
// argument struct: every launch parameter is read in one batch at kernel
// entry).  Segment fields arrive as separate scalars.  Slots past the last
// segment get segment 0's first panel (a valid address, so every load stays
// a global load) and valid = false; their results are dropped.
template <int EPI>
__device__ inline void gemv_slot(const uint8_t *w0, const uint8_t *w1, const uint8_t *w2,
                                 float s0, float s1, float s2, int n0, int n1, int n2, int c0,
                                 int c1, int c2, int K, int P, int pg, int p,
                                 const uint8_t **w, float *scale, int *col, bool *valid) {
  if constexpr (EPI == EPI_SWIGLU) {
    // paired mode: slot p comes from segment p (gate, up), same panel pg
    *w = (p == 0 ? w0 : w1) + (size_t)pg * K * 8;
    *scale = p == 0 ? s0 : s1;
    *col = pg * 16;
    *valid = true;
  } else {
    const int panel = pg * P + p;
    const int si = panel < n0 ? 0 : (panel < n0 + n1 ? 1 : 2);
    const int loc = panel - (si == 0 ? 0 : (si == 1 ? n0 : n0 + n1));
    const bool ok = panel < n0 + n1 + n2;
    const uint8_t *base = si == 0 ? w0 : (si == 1 ? w1 : w2);
    const float sc = si == 0 ? s0 : (si == 1 ? s1 : s2);
    const int cc = si == 0 ? c0 : (si == 1 ? c1 : c2);
    *w = ok ? base + (size_t)loc * K * 8 : w0;
    *scale = ok ? sc : 0.f;
    *col = ok ? cc + loc * 16 : 0;
    *valid = ok;
  }
}

// D fragment index of output row i, column j (v_mfma_*_16x16x* layout:
// lane j + 16*(i/4), element i%4).
__device__ inline int dfrag(int i, int j) { return (j + 16 * (i >> 2)) * 4 + (i & 3); }

// Super-tiles each wave keeps in flight per batch: A fragments of a global-A
// GEMV live in registers next to the weights, so it holds fewer.  Ten per
// wave lets the decode shapes (E4B gate|up: 5 per panel at W = 4) finish
// in one batch.
template <int C, int P, int AS, int W>
constexpr int gemv_batch() {
  // one to four rows from global limbs in 16 waves (the Down projection at
  // batch 2-4): five super-tiles per wave take K <= 10240 in one batch
  if (AS == AS_QUANT && C == 1 && P == 1 && W == 16) return 5;
  // four panels per block from global limbs (the LM head): two super-tiles per
  // batch (one: 0.2% slower per decode step, three to five: no faster)
  if (AS == AS_QUANT && C == 1 && P == 4 && W == 4) return 2;
  constexpr int u = (AS == AS_QUANT ? 4 / C : 10 / C) / P;
  return u < 1 ? 1 : u;
}

// LDS layout: int partial sums [W][P][C][256], output values [P][M][16],
// shifts, then (AS_ROWS, AS_ATTN, AS_WAVES) limb rows [4M][K + 16] (16-byte
// aligned).
__host__ __device__ inline size_t gemv_lds_red(int W, int P, int C) {
  return (size_t)W * P * C * 256 * 4;
}
// shifts: one per row, or per (row, wave) with AS_WAVES (4 rows x 16 waves)
constexpr int kRowShiftSlots = 64;
__host__ __device__ inline size_t gemv_lds_fixed(int W, int P, int C, int M) {
  return gemv_lds_red(W, P, C) + (size_t)P * M * 16 * 4 + (size_t)kRowShiftSlots * 4;
}
__host__ __device__ inline int gemv_ldl(int K) { return K + 16; }

// 8-row groups per thread in the row prologue: K <= 8 * rows_ng(W) * 64 * W.
__host__ __device__ constexpr int rows_ng(int W) { return (void)W, 2; }

// Row prologue for two to four rows in a block of W = 4 or 8 waves: row r
// belongs to waves r*G .. r*G + G - 1 (G = W / 4), so the rows are normalized
// and quantized side by side instead of one after another.  The values are
// dealt as in the one-row prologue of the same block (thread t = 64 vw + lane
// of "virtual wave" vw holds groups t + 64 W gi): each real wave plays W / G
// virtual waves, keeps a partial sum of squares per virtual wave, reduces each
// with the same lane butterfly and adds them in virtual-wave order, so every
// row's statistics, and therefore its limbs, are bit-identical to the one-row
// prologue's.  Returns after the limb stores (no barrier after them).
// kw: issue the first weight loads once the rows have arrived.
template <int W, class KW>
__device__ inline void rows_to_waves(const RowSrc &rs, int K, int M, int8_t *limbs, int ldl,
                                     int32_t *row_s, float *sh, KW kw) {
  constexpr int NT = 64 * W;
  constexpr int G = W / 4;       // real waves per row
  constexpr int VPR = W / G;     // virtual waves per real wave (4)
  constexpr int NG = rows_ng(W);
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int r = wave / G, j = wave % G;
  const bool on = r < M;
  const int nq = K >> 3;
  float v[VPR][NG][8];
#pragma unroll
  for (int k = 0; k < VPR; ++k)
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      const int q = 64 * (j + G * k) + lane + NT * gi;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[k][gi][e] = 0.f;
      if (on && q < nq) {
        const float *p = rs.x + (size_t)r * rs.ld + 8 * q;
        const float4 a = ldg<float4>(p), b = ldg<float4>(p + 4);
        v[k][gi][0] = a.x; v[k][gi][1] = a.y; v[k][gi][2] = a.z; v[k][gi][3] = a.w;
        v[k][gi][4] = b.x; v[k][gi][5] = b.y; v[k][gi][6] = b.z; v[k][gi][7] = b.w;
      }
    }
  asm volatile("" ::"v"(v[0][0][0]), "v"(v[VPR - 1][NG - 1][7]) : "memory");
  kw();
  // statistics per virtual wave, in the one-row prologue's order
  float ss[VPR], mx[VPR];
#pragma unroll
  for (int k = 0; k < VPR; ++k) {
    ss[k] = 0.f;
    mx[k] = 0.f;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = v[k][gi][e] * rs.pre_scale;
        ss[k] += y * y;
        mx[k] = fmaxf(mx[k], fabsf(y));
      }
    ss[k] = wave_sum(ss[k]);
    mx[k] = wave_max(mx[k]);
  }
  float SS = 0.f, MX = 0.f;
  if constexpr (G == 1) {
#pragma unroll
    for (int k = 0; k < VPR; ++k) {
      SS += ss[k];
      MX = fmaxf(MX, mx[k]);
    }
  } else {
    // the row's G waves meet in LDS: sh[(2 r) * W + vw] sums, [(2 r + 1) * W + vw] maxima
    if (lane == 0) {
#pragma unroll
      for (int k = 0; k < VPR; ++k) {
        sh[(2 * r) * W + j + G * k] = ss[k];
        sh[(2 * r + 1) * W + j + G * k] = mx[k];
      }
    }
    __syncthreads();
#pragma unroll
    for (int vw = 0; vw < W; ++vw) {
      SS += sh[(2 * r) * W + vw];
      MX = fmaxf(MX, sh[(2 * r + 1) * W + vw]);
    }
  }
  if (!on) return;
  // row_emit's transform, quantization and stores for this thread's values
  float inv = 1.f;
  if (rs.norm) inv = 1.0f / sqrtf(SS / (float)K + 1e-6f);
  const float amax = MX * inv * (1.0f + 1.0f / 4194304.0f);
  const int s = row_shift(amax);
  const float mul = ldexpf(1.0f, s);
  const bool writer = blockIdx.x == 0;
#pragma unroll
  for (int k = 0; k < VPR; ++k)
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      const int q = 64 * (j + G * k) + lane + NT * gi;
      if (q >= nq) continue;
      float y[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        y[e] = v[k][gi][e] * rs.pre_scale;
        if (rs.norm) y[e] = y[e] * inv;
      }
      if (writer) {
        const size_t o = (size_t)r * K + 8 * q;
        if (rs.y_out) {
          *reinterpret_cast<float4 *>(rs.y_out + o) = float4{y[0], y[1], y[2], y[3]};
          *reinterpret_cast<float4 *>(rs.y_out + o + 4) = float4{y[4], y[5], y[6], y[7]};
        }
        if (rs.x_out) {
          *reinterpret_cast<float4 *>(rs.x_out + o) =
              float4{v[k][gi][0], v[k][gi][1], v[k][gi][2], v[k][gi][3]};
          *reinterpret_cast<float4 *>(rs.x_out + o + 4) =
              float4{v[k][gi][4], v[k][gi][5], v[k][gi][6], v[k][gi][7]};
        }
      }
      uint32_t lo[4], hi[4];
      quant8<false>(y, mul, lo, hi);
      const int pos = limb_pos8(8 * q);
#pragma unroll
      for (int l = 0; l < 4; ++l)
        *reinterpret_cast<uint2 *>(limbs + (size_t)(4 * r + l) * ldl + pos) = uint2{lo[l], hi[l]};
    }
  if (j == 0 && lane == 0) row_s[r] = s;
}

// AS_ATTN instantiations carry the head dim and the load batch in the RP
// template slot: RP = (hd / 128) * 100 + NJ.
__host__ __device__ constexpr int attn_hd(int rp) { return rp / 100 * 128; }
__host__ __device__ constexpr int attn_nj(int rp) { return rp % 100; }

// AS_ATTN prologue of wave `wave` (head h = wave) in a block of W waves:
// merge the head's attention chunks (k_attn_part), quantize the merged head
// with its own shift and store its four limb rows into the block's limb rows
// (the head's K range only; the wave reads nothing else, so no block barrier).
//
// Loads.  Each lane loads 8 dims of a chunk's o partial per load pair, so one
// pair of 16-byte loads covers CPI = 512 / HD chunks (HD / 8 lanes each); NJ
// pairs cover a batch of NJ * CPI chunks.  Every lane of every load reads
// data (a wave load instruction costs the CU's address unit the same time
// whatever lanes read), and loads of chunks past the launched ones read past
// the buffer range: zeros, no memory access.  The position, the (m, l) pairs
// (lane = chunk), the o partials and then the wave's weights (kw) are issued
// in that order and without branches, so the compiler can count them and the
// merge waits for the partials only.
//
// Merge (k_attn_decode's): w_c = e^(m_c - M) / sum_c e^(m_c - M) l_c and
// o = sum_c w_c o_c, each lane summing its chunks in order, then the CPI lane
// groups added.  Chunks past the position take no part (a select, so a stale
// partial never enters the sum).
template <int W, int HD, int NJ, class KW>
__device__ inline void attn_merge_quant(const AttnSrc &at_, int8_t *limbs, int ldl,
                                        int32_t *row_s, int wave, int lane, KW kw) {
  constexpr int LPC = HD / 8;    // lanes per chunk
  constexpr int CPI = 64 / LPC;  // chunks per load pair
  constexpr int CPB = NJ * CPI;  // chunks per batch
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const float *po = launder(at_.part);
  const int32_t *ppos = launder(at_.pos);
  const int nhq = launder(at_.n_heads);
  const int circular = launder(at_.circular), L = launder(at_.cache_len);
  const int clamp = launder(at_.clamp), nch = launder(at_.chunks);
  const float *pml = po + (size_t)kDecPartMaxChunks * nhq * HD;
  const int h = wave;
  const int q8 = lane % LPC, csub = lane / LPC;
  const int base = ldg<int32_t>(ppos);
  const __amdgpu_buffer_rsrc_t rs_ml = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(pml), 0, nch * nhq * 2 * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs_o = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(po), 0, nch * nhq * HD * 4, 0x00020000);
  const f32x2 ml = __builtin_bit_cast(
      f32x2, __builtin_amdgcn_raw_buffer_load_b64(rs_ml, (lane * nhq + h) * 8, 0, 0));
  const uint32_t qoff = (uint32_t)(h * HD + 8 * q8) * 4u;
  f32x4 ov[NJ][2];
  auto load_o = [&](int c0) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t off = (uint32_t)((c0 + j * CPI + csub) * nhq * HD) * 4u + qoff;
      ov[j][0] = __builtin_amdgcn_raw_buffer_load_b128(rs_o, off, 0, 0);
      ov[j][1] = __builtin_amdgcn_raw_buffer_load_b128(rs_o, off + 16, 0, 0);
    }
  };
  // the scheduler would otherwise hold the partials back until the (m, l)
  // pairs arrive, one more memory round trip
  __builtin_amdgcn_sched_barrier(0);
  load_o(0);
  __builtin_amdgcn_sched_barrier(0);
  kw();
  __builtin_amdgcn_sched_barrier(0);
  // attended slots and chunks (as k_attn_part computes them)
  int hi = base;
  if (!circular && clamp && hi > L - 1) hi = L - 1;
  const int nslots = circular ? min(L, base + 1) : min(hi + 1, L);
  const int n_active = min((nslots + kDecPartChunk - 1) / kDecPartChunk, nch);
  const float mc = lane < n_active ? ml.x : -INFINITY;
  const float M = wave_max(mc);
  const float e = lane < n_active ? expf(mc - M) : 0.f;
  const float inv = 1.0f / wave_sum((lane < n_active ? ml.y : 0.f) * e);
  const float wl = e * inv;
  float o[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) o[k] = 0.f;
  for (int c0 = 0; c0 < n_active; c0 += CPB) {
    if (c0 > 0) load_o(c0);
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int c = c0 + j * CPI + csub;
      const float w = __shfl(wl, c & 63, 64);
      const bool on = c < n_active;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        o[k] = on ? o[k] + w * ov[j][0][k] : o[k];
        o[4 + k] = on ? o[4 + k] + w * ov[j][1][k] : o[4 + k];
      }
    }
  }
  // the lane groups holding the same dims (lanes q8 + LPC s)
#pragma unroll
  for (int x = LPC; x < 64; x <<= 1)
#pragma unroll
    for (int k = 0; k < 8; ++k) o[k] += __shfl_xor(o[k], x, 64);
  float mx = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) mx = fmaxf(mx, fabsf(o[k]));
  const int s = row_shift(wave_max(mx));
  if (lane < LPC) {
    uint32_t lo[4], hi4[4];
    quant8<false>(o, ldexpf(1.0f, s), lo, hi4);
    const int pos8 = limb_pos8(h * HD + 8 * lane);
#pragma unroll
    for (int l = 0; l < 4; ++l)
      *reinterpret_cast<uint2 *>(limbs + (size_t)l * ldl + pos8) = uint2{lo[l], hi4[l]};
  }
  if (lane == 0) row_s[h] = s;
  // this wave's limb stores before its own operand reads
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// AS_WAVES instantiations carry the row bound and the super-tiles per wave in
// the RP template slot: RP = 10 * rows + tiles (+ 100 with AttnPrep).
__host__ __device__ constexpr int waves_rows(int rp) { return (rp / 10) % 10; }
__host__ __device__ constexpr int waves_tpw(int rp) { return rp % 10; }
// + 100: one row, store epilogue, preparing the decode attention (AttnPrep)
__host__ __device__ constexpr bool waves_pf(int rp) { return rp >= 100; }
// 64-lane slots of 8-value groups that hold a wave's slice of one row
__host__ __device__ constexpr int waves_nsl(int rp) { return (waves_tpw(rp) * 16 + 63) / 64; }

// AS_WAVES prologue of wave `wave` in a block of W waves: the wave's slice of
// each row, K values [128 TPW wave, 128 TPW (wave + 1)), as 8-value groups
// (lane l: groups l, l + 64, ..).  y = x * pre_scale; the wave's own maximum
// |y| of row m sets its shift row_s[m W + wave], its sum of y^2 goes to
// ssw[m W + wave] for the epilogue's RMSNorm factor.  A row's arithmetic
// does not depend on the other rows, so a row gives the same limbs, shifts
// and sums in a launch of any row count.  The limbs go to the block's limb
// rows in the wave's K range only, which the wave alone reads, so no block
// barrier.  The rows' loads are waited for before the first weights go out
// (kw): they would otherwise queue behind the weights.  yv keeps y for the
// epilogue (the normalized rows, block 0).
template <int TPW, int MR, int W, class KW>
__device__ inline void wave_rows_quant(const RowSrc &rs, int M, int8_t *limbs, int ldl,
                                       int32_t *row_s, float *ssw,
                                       float (&yv)[MR][(TPW * 16 + 63) / 64][8], int wave,
                                       int lane, KW kw) {
  constexpr int NG8 = TPW * 16;
  constexpr int NSL = (NG8 + 63) / 64;
  const int k0 = wave * TPW * 128;
#pragma unroll
  for (int m = 0; m < MR; ++m)
#pragma unroll
    for (int r = 0; r < NSL; ++r) {
      const int gq = lane + 64 * r;
#pragma unroll
      for (int e = 0; e < 8; ++e) yv[m][r][e] = 0.f;
      if ((MR == 1 || m < M) && gq < NG8) {
        const float *p = rs.x + (size_t)m * rs.ld + k0 + 8 * gq;
        const float4 a = ldg<float4>(p), b = ldg<float4>(p + 4);
        yv[m][r][0] = a.x; yv[m][r][1] = a.y; yv[m][r][2] = a.z; yv[m][r][3] = a.w;
        yv[m][r][4] = b.x; yv[m][r][5] = b.y; yv[m][r][6] = b.z; yv[m][r][7] = b.w;
      }
    }
#pragma unroll
  for (int m = 0; m < MR; ++m)
    asm volatile("" ::"v"(yv[m][0][0]), "v"(yv[m][NSL - 1][7]) : "memory");
  kw();
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    if (MR > 1 && m >= M) break;
    float mx = 0.f, ss = 0.f;
#pragma unroll
    for (int r = 0; r < NSL; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = yv[m][r][e] * rs.pre_scale;
        yv[m][r][e] = y;
        ss += y * y;
        mx = fmaxf(mx, fabsf(y));
      }
    mx = wave_max(mx);
    ss = wave_sum(ss);
    const int s = row_shift(mx);
    const float mul = ldexpf(1.0f, s);
#pragma unroll
    for (int r = 0; r < NSL; ++r) {
      const int gq = lane + 64 * r;
      if (gq < NG8) {
        uint32_t lo[4], hi[4];
        quant8<false>(yv[m][r], mul, lo, hi);
        const int pos = limb_pos8(k0 + 8 * gq);
#pragma unroll
        for (int l = 0; l < 4; ++l)
          *reinterpret_cast<uint2 *>(limbs + (size_t)(4 * m + l) * ldl + pos) =
              uint2{lo[l], hi[l]};
      }
    }
    if (lane == 0) {
      row_s[m * W + wave] = s;
      ssw[m * W + wave] = ss;
    }
  }
  // this wave's limb stores before its own operand reads
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// DPP move of a double (its two words), inside rows of 16 lanes.
template <int CTRL>
__device__ inline double dpp_d(double x) {
  const unsigned long long b = __builtin_bit_cast(unsigned long long, x);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

// Sum over aligned groups of W consecutive lanes (W = 4, 8 or 16; every lane
// of the group gets it): quad permutes, then the half-row and row mirrors.
template <int W>
__device__ inline double lanes_sum_d(double v) {
  static_assert(W == 4 || W == 8 || W == 16, "groups of 4, 8 or 16 lanes");
  v += dpp_d<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_d<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (W >= 8) v += dpp_d<0x141>(v);   // row_half_mirror
  if constexpr (W == 16) v += dpp_d<0x140>(v);  // row_mirror
  return v;
}

// AS_WSTREAM: wave-private limb buffer, one super-tile of 4 MR limb rows
// (128 bytes each, 16 bytes of padding against bank conflicts).
constexpr int kWsLd = 144;

// AS_WSTREAM prologue of wave `wave` in a block of W waves (MR = 4 rows): the
// wave's slice of each row, K values [128 TPW wave, 128 TPW (wave + 1)) as in
// AS_WAVES, dealt so that lane l holds row l / 16, the 8-value group l % 16
// of every super-tile u (values 128 u + 8 (l % 16) ..).  A row's values then
// sit in one 16-lane DPP row: its maximum |y| and sum of y^2 are row16
// reductions, and every lane quantizes one group per super-tile.  Rows past
// M read zeros (range-checked loads).  The same maximum over the same values
// as wave_rows_quant, so the same shift, limbs and integer sums (the sum of
// squares, used by norm rows only, adds in another order).  Returns the
// lane's row shift; ys keeps y for the per-tile quantization.
template <int TPW, int W, class KW>
__device__ inline int wave_stream_load(const RowSrc &rs, int M, int32_t *row_s, float *ssw,
                                       float (&ys)[TPW][8], int wave, int lane, KW kw) {
  const int m = lane >> 4, j = lane & 15;
  const int k0 = wave * TPW * 128;
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(rs.x), 0, (uint32_t)(M * rs.ld * 4), 0x00020000);
  const uint32_t base = (uint32_t)((m * rs.ld + k0 + 8 * j) * 4);
  typedef float f32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const f32x4 a = __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, base + u * 512, 0, 0));
    const f32x4 b = __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, base + u * 512 + 16, 0, 0));
    ys[u][0] = a.x; ys[u][1] = a.y; ys[u][2] = a.z; ys[u][3] = a.w;
    ys[u][4] = b.x; ys[u][5] = b.y; ys[u][6] = b.z; ys[u][7] = b.w;
  }
  asm volatile("" ::"v"(ys[0][0]), "v"(ys[TPW - 1][7]) : "memory");
  kw();
  float mx = 0.f, ss = 0.f;
#pragma unroll
  for (int u = 0; u < TPW; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float y = ys[u][e] * rs.pre_scale;
      ys[u][e] = y;
      ss += y * y;
      mx = fmaxf(mx, fabsf(y));
    }
  mx = row_max16(mx);
  ss = row_sum16(ss);
  const int s = row_shift(mx);
  if (j == 0) {
    row_s[m * W + wave] = s;
    ssw[m * W + wave] = ss;
  }
  return s;
}

// C: 16-row MFMA groups (4 limb rows per activation row: M <= 4C).
// P: panels per block.  AS: GemvASource.  W: waves per block.  EPI: epilogue.
// RP: activation rows whose loads the AS_ROWS prologue issues at once
// (AS_ATTN: head dim and load batch, attn_hd / attn_nj; AS_WAVES: row bound
// and super-tiles per wave, waves_rows / waves_tpw).
//
// Block pg = P panels of 16 columns over the whole K.  Wave w owns super-tiles
// w, w+W, ...; each batch issues U of them (P panels each) before any is
// consumed, and the first batch is issued before the prologue so that the
// weight stream overlaps the activation quantization.
template <int C, int P, int AS, int W, int EPI, int RP>
__global__ __launch_bounds__(64 * W, W == 4 ? 3 : 1) void k_gemv(GemvArgs a) {
  extern __shared__ __align__(16) uint8_t lds[];
  // reduction scratch (AS_WAVES: a sum of squares per (row, wave))
  __shared__ float sh[W > 4 ? 64 : 32];
  constexpr int NT = 64 * W;
  // AS_ATTN: the head's super-tiles, one batch
  // (AS_WAVES: the wave's RP super-tiles, one batch)
  constexpr bool WS = AS == AS_WSTREAM;
  constexpr int U = AS == AS_ATTN    ? attn_hd(RP) / 128
                    : (AS == AS_WAVES || WS) ? waves_tpw(RP)
                                     : gemv_batch<C, P, AS, W>();
  // rows a WAVE_K epilogue finishes (AS_ATTN: one)
  constexpr int MR = (AS == AS_WAVES || WS) ? waves_rows(RP) : 1;
  constexpr int NSL = AS == AS_WAVES ? waves_nsl(RP) : 1;
  constexpr bool WAVE_K = AS == AS_ATTN || AS == AS_WAVES || WS;  // contiguous K per wave
  static_assert(!WS || MR == 4, "streamed slices: four rows (lane l holds row l / 16)");
  // wave-uniform in a scalar register: tile predicates below are then scalar
  // branches, and loads behind them need no merge (and no wait) at the join
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  // Every launch parameter the kernel uses is read here, in one batch: uses
  // further down would otherwise become dependent argument loads.
  const int K = launder(a.K), M = launder(a.M);
  const int nseg = launder(a.nseg);
  const uint8_t *sw0 = launder(a.seg[0].w), *sw1 = launder(a.seg[1].w),
                *sw2 = launder(a.seg[2].w);
  const float ss0 = launder(a.seg[0].scale), ss1 = launder(a.seg[1].scale),
              ss2 = launder(a.seg[2].scale);
  const int sn0 = launder(a.seg[0].n_cols) >> 4;
  const int sn1 = nseg > 1 ? launder(a.seg[1].n_cols) >> 4 : 0;
  const int sn2 = nseg > 2 ? launder(a.seg[2].n_cols) >> 4 : 0;
  const int sc0 = launder(a.seg[0].out_col0), sc1 = launder(a.seg[1].out_col0),
            sc2 = launder(a.seg[2].out_col0);
  const int ldo = launder(a.ldo);
  float *out = launder(a.out);
  const float *resid = (EPI == EPI_RESID) ? launder(a.resid) : nullptr;
  float *out2 = (EPI == EPI_RESID) ? launder(a.out2) : nullptr;
  float *sw_out = (EPI == EPI_SWIGLU) ? launder(a.sw_out) : nullptr;
  const int ldo_sw = (EPI == EPI_SWIGLU) ? launder(a.ldo_sw) : 0;
  float *arg_val = (EPI == EPI_ARGMAX) ? launder(a.arg_val) : nullptr;
  int32_t *arg_idx = (EPI == EPI_ARGMAX) ? launder(a.arg_idx) : nullptr;
  // the decode attention's RoPE factors (one-row Q|K|V projection)
  constexpr bool PF = AS == AS_WAVES && waves_pf(RP);
  static_assert(!PF || (EPI == EPI_STORE && P == 1 && MR == 1), "AttnPrep: one row, store");
  AttnPrep pf{};
  int pf_base = 0;
  if constexpr (PF) {
    pf.cos_t = launder(a.pf.cos_t);
    pf.sin_t = launder(a.pf.sin_t);
    pf.half = launder(a.pf.half);
    pf.rope_rows = launder(a.pf.rope_rows);
    pf.rope_cur = launder(a.pf.rope_cur);
    // first load of the kernel: it has arrived when the weights have gone
    // out.  Loaded per lane (an opaque zero offset), so that no wait for it
    // is placed here to move it into a scalar register.
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    pf_base = ldg<int32_t>(launder(a.pf.pos) + z);
  }
  RowSrc rs{};
  QuantRows qr{};
  if (AS == AS_ROWS || AS == AS_WAVES || WS) {
    rs.x = launder(a.rows.x);
    rs.ld = launder(a.rows.ld);
    rs.pre_scale = launder(a.rows.pre_scale);
    rs.norm = launder(a.rows.norm);
    rs.y_out = launder(a.rows.y_out);
    rs.x_out = launder(a.rows.x_out);
  } else if (AS == AS_QUANT) {
    qr.limbs = launder(a.q.limbs);
    qr.shift = launder(a.q.shift);
  }

  const int KG = K / kSuperK;
  const int pg = blockIdx.x;
  // AS_ATTN: wave w owns the super-tiles of head w, contiguous; otherwise
  // super-tiles are dealt to the waves round-robin
  const int tpw = WAVE_K ? U : 0;  // = K / (128 W), checked by the launcher
  const int nb = WAVE_K ? 1 : ((KG + W - 1) / W + U - 1) / U;  // batches

  const uint8_t *wl[P];
  float wsc[P];
  int col[P];
  bool wv[P];
#pragma unroll
  for (int p = 0; p < P; ++p)
    gemv_slot<EPI>(sw0, sw1, sw2, ss0, ss1, ss2, sn0, sn1, sn2, sc0, sc1, sc2, K, P, pg, p,
                   &wl[p], &wsc[p], &col[p], &wv[p]);

  // WAVE_K, residual epilogue: the thread that finishes output (p, j) loads
  // its residual value now (a memory round trip off the epilogue's path)
  float resid_pre[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) resid_pre[m] = 0.f;
  if constexpr (WAVE_K && EPI == EPI_RESID) {
    const int t = threadIdx.x, w = t % W, p = (t / W) % P, j = t / (W * P);
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if ((MR == 1 || m < M) && t < 16 * P * W && w == 0 && wv[p])
        resid_pre[m] = ldg<float>(resid + (size_t)m * ldo + col[p] + j);
  }
  int32_t *red = reinterpret_cast<int32_t *>(lds);
  float *vals = reinterpret_cast<float *>(lds + gemv_lds_red(W, P, C));
  int32_t *row_s = reinterpret_cast<int32_t *>(lds + gemv_lds_red(W, P, C) + (size_t)P * M * 64);
  int8_t *limbs = reinterpret_cast<int8_t *>(lds + gemv_lds_fixed(W, P, C, M));
  const int ldl = gemv_ldl(K);

  // A operand of this lane: row i of MFMA group c is limb row 16c + i
  const int i = lane & 15, g = lane >> 4;
  bool a_on[C];
#pragma unroll
  for (int c = 0; c < C; ++c) a_on[c] = 16 * c + i < 4 * M;

  uint4 q[U][P];
  float pf_cs[2];  // PF: cos, sin at the position (block 0)
  v4i af[AS == AS_QUANT ? U : 1][C][2];
  float yv[MR][NSL][8];  // AS_WAVES: the wave's y values (for the normalized rows)
  float ys[WS ? U : 1][8];  // AS_WSTREAM: the lane's group of each super-tile
  int ws_s = 0;             // AS_WSTREAM: the lane's row shift
  // Loads of super-tiles u0..u1-1 of batch bt; tiles past the end of K are
  // not loaded (their slots stay zero and are never consumed).
  auto tile = [&](int bt, int u) {
    return WAVE_K ? wave * tpw + u : wave + (bt * U + u) * W;
  };
  auto tile_on = [&](int bt, int u) {
    return WAVE_K ? u < tpw : wave + (bt * U + u) * W < KG;
  };
  auto issue_part = [&](int bt, int u0, int u1) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (u < u0 || u >= u1) continue;
      const int Gu = tile(bt, u);
#pragma unroll
      for (int p = 0; p < P; ++p) {
        q[u][p] = uint4{0u, 0u, 0u, 0u};
        if constexpr (AS == AS_ATTN) {
          // the wave's own super-tiles as one range (no branch: tiles past
          // it read zeros without a memory access), streaming hint (nt)
          const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
              const_cast<uint8_t *>(wl[p]) + (size_t)wave * tpw * 1024, 0, tpw * 1024,
              0x00020000);
          const u32x4 v = __builtin_bit_cast(
              u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, u * 1024 + lane * 16, 0, 2));
          q[u][p] = uint4{v.x, v.y, v.z, v.w};
        } else if (tile_on(bt, u)) {
          const u32x4 v = ldg_nt<u32x4>(wl[p] + (size_t)Gu * 1024 + lane * 16);
          q[u][p] = uint4{v.x, v.y, v.z, v.w};
        }
      }
      if constexpr (AS == AS_QUANT) {
#pragma unroll
        for (int c = 0; c < C; ++c) {
          af[u][c][0] = v4i{0, 0, 0, 0};
          af[u][c][1] = v4i{0, 0, 0, 0};
          if (a_on[c]) {
            const int8_t *ar = qr.limbs + (size_t)(16 * c + i) * K + Gu * 128 + 32 * g;
            af[u][c][0] = ldg<v4i>(ar);
            af[u][c][1] = ldg<v4i>(ar + 16);
          }
        }
      }
    }
  };
  auto issue = [&](int bt) { issue_part(bt, 0, U); };

  // ---- prologue: activation limbs, overlapping the first weight batch
  if constexpr (AS == AS_ROWS) {
    // The row is tiny next to the weights, but its loads queue behind every
    // weight load already in flight on the chip, so the weights go out once
    // the row has arrived and overlap the norm and the quantization.  A wave
    // stalls at issue once the memory pipeline is full, which would hold up
    // its share of the quantization: at most four loads per wave go out
    // before it, the rest after the prologue.
    constexpr int kEarly = (4 / P) < 1 ? 1 : ((4 / P) < U ? (4 / P) : U);
    if constexpr (RP == 4 && C == 1) {
      // two to four rows: side by side, one wave group per row
      rows_to_waves<W>(rs, K, M, limbs, ldl, row_s, sh, [&] { issue_part(0, 0, kEarly); });
    } else {
    // The loads of the first RP rows go out together, before the weights, so
    // that rows 1.. are in registers by the time the previous row is done.
    RowRegs<NT, rows_ng(W), false> R[RP];
#pragma unroll
    for (int m = 0; m < RP; ++m)
      if (m < M) row_load<NT, rows_ng(W), false>(rs, K, m, R[m]);
    asm volatile("" ::"v"(R[0].v[0][0]), "v"(R[0].v[rows_ng(W) - 1][7]) : "memory");
    issue_part(0, 0, kEarly);
    int s;
#pragma unroll
    for (int m = 0; m < RP; ++m) {
      if (m < M) {
        row_finish<NT, rows_ng(W), false>(rs, K, m, blockIdx.x == 0, R[m], limbs, ldl, sh, &s,
                                          nullptr, m == 0);
        if (threadIdx.x == 0) row_s[m] = s;
      }
    }
    for (int m = RP; m < M; ++m) {
      row_load<NT, rows_ng(W), false>(rs, K, m, R[0]);
      row_finish<NT, rows_ng(W), false>(rs, K, m, blockIdx.x == 0, R[0], limbs, ldl, sh, &s);
      if (threadIdx.x == 0) row_s[m] = s;
    }
    }
    __syncthreads();
    if constexpr (kEarly < U) issue_part(0, kEarly, U);
  } else if constexpr (AS == AS_ATTN) {
    attn_merge_quant<W, attn_hd(RP), attn_nj(RP)>(a.at, limbs, ldl, row_s, wave, lane,
                                                   [&] { issue(0); });
  } else if constexpr (WS) {
    constexpr int kEarlyW = (4 / P) < 1 ? 1 : ((4 / P) < U ? (4 / P) : U);
    ws_s = wave_stream_load<U, W>(rs, M, row_s, sh, ys, wave, lane,
                                  [&] { issue_part(0, 0, kEarlyW); });
    if constexpr (kEarlyW < U) issue_part(0, kEarlyW, U);
  } else if constexpr (AS == AS_WAVES) {
    constexpr int kEarlyW = (4 / P) < 1 ? 1 : ((4 / P) < U ? (4 / P) : U);
    wave_rows_quant<U, MR, W>(rs, M, limbs, ldl, row_s, sh, yv, wave, lane,
                              [&] { issue_part(0, 0, kEarlyW); });
    if constexpr (kEarlyW < U) issue_part(0, kEarlyW, U);
    if constexpr (PF) {
      __builtin_amdgcn_sched_barrier(0);
      // block 0: the RoPE factors at the position (range-checked loads: the
      // other threads and blocks read nothing)
      const uint32_t tb = (uint32_t)pf.rope_rows * (uint32_t)pf.half * 4u;
      const __amdgpu_buffer_rsrc_t rc_ =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(pf.cos_t), 0, tb, 0x00020000);
      const __amdgpu_buffer_rsrc_t rs_ =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(pf.sin_t), 0, tb, 0x00020000);
      const bool rl = blockIdx.x == 0 && (int)threadIdx.x < pf.half;
      const uint32_t ro = rl ? ((uint32_t)pf_base * (uint32_t)pf.half + threadIdx.x) * 4u
                             : 0x80000000u;
      pf_cs[0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rc_, ro, 0, 0));
      pf_cs[1] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs_, ro, 0, 0));
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    if ((int)threadIdx.x < M) row_s[threadIdx.x] = ldg<int32_t>(qr.shift + threadIdx.x);
    issue(0);
  }

  // Weights enter the MFMA as unsigned nibbles n (one mask per four bytes);
  // accz collects sum_k limb(k) * (-8) with a constant operand, added to every
  // panel's sums after the K loop (exact: each term stays in int32).
  const v4i kMinus8 = v4i{(int)0xF8F8F8F8u, (int)0xF8F8F8F8u, (int)0xF8F8F8F8u,
                          (int)0xF8F8F8F8u};
  v4i acc[P][C], accz[C];
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[p][c] = v4i{0, 0, 0, 0};
#pragma unroll
  for (int c = 0; c < C; ++c) accz[c] = v4i{0, 0, 0, 0};

  for (int bt = 0; bt < nb; ++bt) {
    if (bt > 0) issue(bt);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int Gu = tile(bt, u);
      if (tile_on(bt, u)) {
        // AS_WSTREAM: this super-tile's limbs, each lane quantizing its group
        // of row lane / 16 into the wave's buffer (read back below)
        int8_t *wb = limbs + (size_t)wave * 4 * MR * kWsLd;
        if constexpr (WS) {
          uint32_t lo[4], hi[4];
          quant8<false>(ys[u], ldexpf(1.0f, ws_s), lo, hi);
          const int pos = limb_pos8(8 * (lane & 15));
#pragma unroll
          for (int l = 0; l < 4; ++l)
            *reinterpret_cast<uint2 *>(wb + (size_t)(4 * (lane >> 4) + l) * kWsLd + pos) =
                uint2{lo[l], hi[l]};
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
        v4i al[C][2];
        if constexpr (AS == AS_ROWS || WAVE_K) {
#pragma unroll
          for (int c = 0; c < C; ++c) {
            al[c][0] = v4i{0, 0, 0, 0};
            al[c][1] = v4i{0, 0, 0, 0};
            if (a_on[c]) {
              const int8_t *ar = WS ? wb + (size_t)(16 * c + i) * kWsLd + 32 * g
                                    : limbs + (size_t)(16 * c + i) * ldl + Gu * 128 + 32 * g;
              al[c][0] = *reinterpret_cast<const v4i *>(ar);
              al[c][1] = *reinterpret_cast<const v4i *>(ar + 16);
            }
          }
        }
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const uint32_t dw[4] = {q[u][p].x, q[u][p].y, q[u][p].z, q[u][p].w};
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const uint32_t d0 = dw[2 * h], d1 = dw[2 * h + 1];
            const v4i b = v4i{nib_u8(d0), nib_u8(d0 >> 4), nib_u8(d1), nib_u8(d1 >> 4)};
#pragma unroll
            for (int c = 0; c < C; ++c) {
              const v4i av = (AS == AS_QUANT) ? af[u][c][h] : al[c][h];
              acc[p][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b, acc[p][c], 0, 0, 0);
            }
          }
        }
        // the zero point: sum_k limb(k) * (-8), once for all panels
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int c = 0; c < C; ++c) {
            const v4i av = (AS == AS_QUANT) ? af[u][c][h] : al[c][h];
            accz[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, kMinus8, accz[c], 0, 0, 0);
          }
      }
    }
  }
  // acc = sum_k limb(k) * n_k + sum_k limb(k) * (-8) = sum_k limb(k) * (n_k - 8)
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int c = 0; c < C; ++c) acc[p][c] += accz[c];

#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int c = 0; c < C; ++c) {
      int32_t *r = red + (((size_t)wave * P + p) * C + c) * 256 + lane * 4;
      *reinterpret_cast<v4i *>(r) = acc[p][c];
    }
  __syncthreads();

  // output (slot p, row m, column j): sum the waves per limb row (exact int32:
  // |limb * (n - 8)| <= 1024 per term, K <= 16384), combine the limbs in
  // int64, scale once.  Each output is finished by the thread that sums it
  // (no second pass through LDS).
  if constexpr (WAVE_K) {
    // One shift per (row, wave): thread t takes column j, panel slot p and
    // wave w (t = (j P + p) W + w), combines that wave's limb sums of a row
    // exactly and scales them by the wave's shift; the W lanes of (j, p) are
    // then added.  Rows one after another, each on its own.
    static_assert(16 * P * W <= NT, "one thread per (column, panel, wave)");
    static_assert(EPI == EPI_STORE || EPI == EPI_ACCUMULATE || EPI == EPI_RESID ||
                      EPI == EPI_SWIGLU,
                  "per-wave shifts: store, accumulate, residual or SwiGLU epilogue");
    static_assert(C == 1, "per-wave shifts: at most four rows");
    const int t = threadIdx.x;
    const int w = t % W, p = (t / W) % P, j = t / (W * P);
    const bool on = t < 16 * P * W;
    float inv[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      if (MR > 1 && m >= M) break;
      double v = 0.0;
      if (on) {
        long long tw = 0;
#pragma unroll
        for (int l = 0; l < 4; ++l)
          tw += (long long)red[((size_t)w * P + p) * 256 + dfrag(4 * m + l, j)] << (8 * l);
        v = (double)tw * (double)ldexpf(1.0f, -row_s[m * W + w]);
      }
      v = lanes_sum_d<W>(v);
      // RMSNorm of the row (rmsnorm_inplace kernels.mojo:474-489) as a factor
      // on the products: y . W = inv (x . W)
      inv[m] = 1.0f;
      if ((AS == AS_WAVES || WS) && rs.norm) {
        float ssum = 0.f;
#pragma unroll
        for (int u = 0; u < W; ++u) ssum += sh[m * W + u];
        inv[m] = 1.0f / sqrtf(ssum / (float)K + 1e-6f);
      }
      if constexpr (EPI == EPI_SWIGLU) {
        // gate (p = 0) and up (p = 1) of column j sit W lanes apart
        const double vu = __shfl_down(v, W, 64);
        if (on && w == 0 && p == 0) {
          const float gt = (float)(v * (double)inv[m] * (double)wsc[0]);
          const float up = (float)(vu * (double)inv[m] * (double)wsc[1]);
          sw_out[(size_t)m * ldo_sw + col[0] + j] = up * gt * (1.0f / (1.0f + expf(-gt)));
        }
      } else {
        if (on && w == 0 && wv[p]) {
          const float val = (float)(v * (double)inv[m] * (double)wsc[p]);
          const size_t oi = (size_t)m * ldo + col[p] + j;
          if constexpr (EPI == EPI_STORE) {
            out[oi] = val;
          } else if constexpr (EPI == EPI_ACCUMULATE) {
            out[oi] += val;
          } else {
            // x = x + proj (gemma4_e4b.mojo:522,538)
            const float x = resid_pre[m] + val;
            out[oi] = x;
            if (out2) out2[oi] = x;
          }
        }
      }
    }
    if constexpr (AS == AS_WAVES) {
      // the normalized rows, y * inv (block 0): the next projections' residual
      if (blockIdx.x == 0 && rs.y_out) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          if (MR > 1 && m >= M) break;
#pragma unroll
          for (int r = 0; r < NSL; ++r) {
            const int gq = lane + 64 * r;
            if (gq < U * 16) {
              float *o = rs.y_out + (size_t)m * K + wave * U * 128 + 8 * gq;
              const float f = inv[m];
              *reinterpret_cast<float4 *>(o) = float4{yv[m][r][0] * f, yv[m][r][1] * f,
                                                      yv[m][r][2] * f, yv[m][r][3] * f};
              *reinterpret_cast<float4 *>(o + 4) = float4{yv[m][r][4] * f, yv[m][r][5] * f,
                                                          yv[m][r][6] * f, yv[m][r][7] * f};
            }
          }
        }
      }
    }
    if constexpr (WS) {
      // the normalized rows (block 0): lane l holds row l / 16's groups
      const int m = lane >> 4, j = lane & 15;
      if (blockIdx.x == 0 && rs.y_out && m < M) {
        float f = inv[0];
#pragma unroll
        for (int mm = 1; mm < MR; ++mm)
          if (mm < M && m == mm) f = inv[mm];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          float *o = rs.y_out + (size_t)m * K + wave * U * 128 + 128 * u + 8 * j;
          *reinterpret_cast<float4 *>(o) =
              float4{ys[u][0] * f, ys[u][1] * f, ys[u][2] * f, ys[u][3] * f};
          *reinterpret_cast<float4 *>(o + 4) =
              float4{ys[u][4] * f, ys[u][5] * f, ys[u][6] * f, ys[u][7] * f};
        }
      }
    }
    if constexpr (PF) {
      if (blockIdx.x == 0 && (int)threadIdx.x < pf.half) {
        pf.rope_cur[threadIdx.x] = pf_cs[0];
        pf.rope_cur[pf.half + threadIdx.x] = pf_cs[1];
      }
    }
    return;
  }
  auto value = [&](int p, int m, int j) {
    const int c = m >> 2, r0 = 4 * (m & 3);
    long long t = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      int d = 0;
      for (int w = 0; w < W; ++w)
        d += red[(((size_t)w * P + p) * C + c) * 256 + dfrag(r0 + l, j)];
      t += (long long)d << (8 * l);
    }
    return (float)((double)t * (double)ldexpf(1.0f, -row_s[m]) * (double)wsc[p]);
  };
  if constexpr (EPI == EPI_STORE || EPI == EPI_ACCUMULATE || EPI == EPI_RESID) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      if (!wv[p]) continue;
      for (int o = threadIdx.x; o < M * 16; o += NT) {
        const int m = o >> 4, j = o & 15;
        const size_t oi = (size_t)m * ldo + col[p] + j;
        const float v = value(p, m, j);
        if constexpr (EPI == EPI_STORE) {
          out[oi] = v;
        } else if constexpr (EPI == EPI_ACCUMULATE) {
          out[oi] += v;
        } else {
          // x = x + proj (gemma4_e4b.mojo:522,538)
          const float x = resid[oi] + v;
          out[oi] = x;
          if (out2) out2[oi] = x;
        }
      }
    }
  } else if constexpr (EPI == EPI_SWIGLU) {
    // slot 0 = gate, slot 1 = up (same columns): swiglu_inplace
    // (kernels.mojo:519-532) fused into the producer.
    for (int o = threadIdx.x; o < M * 16; o += NT) {
      const int m = o >> 4, j = o & 15;
      const float gt = value(0, m, j), up = value(1, m, j);
      const float y = up * gt * (1.0f / (1.0f + expf(-gt)));
      sw_out[(size_t)m * ldo_sw + col[0] + j] = y;
    }
  } else if constexpr (EPI == EPI_ARGMAX) {
#pragma unroll
    for (int p = 0; p < P; ++p)
      for (int o = threadIdx.x; o < M * 16; o += NT) vals[p * M * 16 + o] = value(p, o >> 4, o & 15);
    __syncthreads();
    // logits (optional) and the block's first index of the maximum per row
    if (out) {
#pragma unroll
      for (int p = 0; p < P; ++p)
        for (int o = threadIdx.x; o < M * 16; o += NT) {
          const int m = o >> 4, j = o & 15;
          out[(size_t)m * ldo + col[p] + j] = vals[p * M * 16 + o];
        }
    }
    if ((int)threadIdx.x < M) {
      const int m = threadIdx.x;
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int p = 0; p < P; ++p)
        for (int j = 0; j < 16; ++j) {
          const float v = vals[(p * M + m) * 16 + j];
          const int idx = col[p] + j;
          if (v > bv || (v == bv && idx < bi)) {
            bv = v;
            bi = idx;
          }
        }
      arg_val[(size_t)blockIdx.x * M + m] = bv;
      arg_idx[(size_t)blockIdx.x * M + m] = bi;
    }
  }
}

// Greedy id per row from the per-block maxima; blocks are visited in increasing
// column order and ties keep the lowest index (lm_head.mojo:224-230).
// (value, index) argmax step with the partner lane of DPP control CTRL: the
// larger value, the lower index on ties (the greedy branch's first maximum)
template <int CTRL>
__device__ inline void argmax_dpp(float &v, int &i) {
  const float pv = dpp_f<CTRL>(v);
  const int pi = __builtin_amdgcn_update_dpp(0, i, CTRL, 0xF, 0xF, false);
  if (pv > v || (pv == v && pi < i)) {
    v = pv;
    i = pi;
  }
}

// Final argmax over the head's per-block maxima, one pass for all rows: each
// thread scans its blocks for every row (M <= kFinRows per pass), each wave
// reduces its lanes with DPP row steps and readlane, and thread m combines
// the 16 waves' results of row m from LDS.  Then the state updates.
constexpr int kFinRows = 4;
__global__ __launch_bounds__(1024) void k_argmax_fin(ArgmaxFin f) {
  __shared__ float sv[kFinRows][16];
  __shared__ int si[kFinRows][16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  // ids chosen elsewhere (the sampler): only the state updates below
  const int nb = f.ids_in ? 0 : f.n_blocks;
  for (int m0 = 0; m0 < f.M; m0 += kFinRows) {
    float bv[kFinRows];
    int bi[kFinRows];
#pragma unroll
    for (int r = 0; r < kFinRows; ++r) {
      bv[r] = -INFINITY;
      bi[r] = 0x7fffffff;
    }
    for (int b = threadIdx.x; b < nb; b += 1024)
#pragma unroll
      for (int r = 0; r < kFinRows; ++r) {
        if (m0 + r >= f.M) break;
        const float v = f.arg_val[(size_t)b * f.M + m0 + r];
        const int idx = f.arg_idx[(size_t)b * f.M + m0 + r];
        if (v > bv[r] || (v == bv[r] && idx < bi[r])) {
          bv[r] = v;
          bi[r] = idx;
        }
      }
#pragma unroll
    for (int r = 0; r < kFinRows; ++r) {
      argmax_dpp<0xB1>(bv[r], bi[r]);   // quad_perm [1,0,3,2]
      argmax_dpp<0x4E>(bv[r], bi[r]);   // quad_perm [2,3,0,1]
      argmax_dpp<0x141>(bv[r], bi[r]);  // row_half_mirror
      argmax_dpp<0x140>(bv[r], bi[r]);  // row_mirror
      float v = lane_f(bv[r], 0);
      int i = __builtin_amdgcn_readlane(bi[r], 0);
#pragma unroll
      for (int q = 16; q < 64; q += 16) {
        const float qv = lane_f(bv[r], q);
        const int qi = __builtin_amdgcn_readlane(bi[r], q);
        if (qv > v || (qv == v && qi < i)) {
          v = qv;
          i = qi;
        }
      }
      if (lane == 0) {
        sv[r][w] = v;
        si[r][w] = i;
      }
    }
    __syncthreads();
    const int r = threadIdx.x;
    if (r < kFinRows && m0 + r < f.M) {
      const int m = m0 + r;
      float v = sv[r][0];
      int id = si[r][0];
      for (int q = 1; q < 16; ++q)
        if (sv[r][q] > v || (sv[r][q] == v && si[r][q] < id)) {
          v = sv[r][q];
          id = si[r][q];
        }
      if (f.ids_in) id = f.ids_in[m];
      if (f.ids_out) f.ids_out[m] = id;
      if (f.tok_state) f.tok_state[m] = id;
      if (f.pos_state) f.pos_state[m] += 1;
      if (f.ids_hist) f.ids_hist[(size_t)(*f.step) * f.M + m] = id;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0 && f.ids_hist) *f.step += 1;
  if (threadIdx.x == 0 && f.draws) *f.draws += 1;
}

int launch_argmax_fin(const ArgmaxFin &f, hipStream_t st) {
  hipLaunchKernelGGL(k_argmax_fin, dim3(1), dim3(1024), 0, st, f);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

size_t gemv_lds_need(const GemvArgs &a) {
  const int C = a.M <= 4 ? 1 : 4;
  size_t b = gemv_lds_fixed(a.waves, a.P, C, a.M);
  if (a.asrc == AS_ROWS || a.asrc == AS_ATTN || a.asrc == AS_WAVES)
    b += (size_t)4 * a.M * gemv_ldl(a.K);
  else if (a.asrc == AS_WSTREAM)
    b += (size_t)a.waves * 4 * kWaveRowsMax * kWsLd;
  return b;
}

bool wave_shape_ok(const GemvArgs &a) {
  const int w = a.waves;
  if (w <= 0 || a.K % (w * kSuperK) != 0) return false;
  const int tpw = a.K / (w * kSuperK);
  switch (a.epi) {
    case EPI_STORE:
      return a.P == 1 && ((w == 4 && (tpw == 2 || tpw == 5)) ||
                          (w == 8 && (tpw == 1 || tpw == 2 || tpw == 4)));
    case EPI_ACCUMULATE: return a.P == 1 && w == 8 && (tpw == 1 || tpw == 2 || tpw == 4);
    case EPI_SWIGLU: return a.P == 2 && w == 4 && (tpw == 2 || tpw == 5);
    case EPI_RESID:
      return a.P == 1 && ((w == 16 && (tpw == 2 || tpw == 5)) ||
                          (w == 8 && (tpw == 1 || tpw == 2 || tpw == 4)));
    default: return false;
  }
}

int launch_gemv(const GemvArgs &a, hipStream_t st) {
  MS_CHECK_ARG(a.M >= 1 && a.M <= kGemvMaxM, "GEMV: 1 <= M <= 16");
  MS_CHECK_ARG(a.K >= kSuperK && a.K % kSuperK == 0, "GEMV: K % 128 != 0");
  MS_CHECK_ARG(a.asrc == AS_ROWS || a.asrc == AS_QUANT || a.asrc == AS_ATTN ||
                   a.asrc == AS_WAVES || a.asrc == AS_WSTREAM,
               "GEMV: bad activation source");
  MS_CHECK_ARG(a.nseg >= 1 && a.nseg <= 3, "GEMV: 1 to 3 segments");
  MS_CHECK_ARG(a.epi != EPI_RESID || (a.resid && a.out), "GEMV: residual epilogue needs rows");
  MS_CHECK_ARG(a.epi != EPI_SWIGLU || (a.P == 2 && a.nseg == 2 && a.sw_out),
               "GEMV: SwiGLU epilogue needs P=2, two segments and an output");
  MS_CHECK_ARG(a.epi != EPI_ARGMAX || (a.arg_val && a.arg_idx),
               "GEMV: argmax epilogue needs block-max buffers");
  MS_CHECK_ARG(a.epi == EPI_ARGMAX || a.epi == EPI_SWIGLU || a.out, "GEMV: missing output");
  if (a.asrc == AS_ROWS) {
    MS_CHECK_ARG(a.rows.x && a.rows.ld >= a.K && !a.rows.gamma,
                 "GEMV: row prologue needs rows (no gamma)");
    MS_CHECK_ARG(a.K <= 8 * rows_ng(a.waves) * 64 * a.waves, "GEMV: row prologue: row too long");
  } else if (a.asrc == AS_WAVES) {
    MS_CHECK_ARG(a.M <= kWaveRowsMax && a.rows.x && a.rows.ld >= a.K && !a.rows.gamma &&
                     !a.rows.x_out && wave_shape_ok(a),
                 "GEMV: per-wave rows: at most 4 rows, K = waves * tpw * 128 with tpw 1, 2, "
                 "4 or 5, and store or accumulate (4 or 8 waves), SwiGLU (4 waves) or "
                 "residual (8 or 16 waves)");
  } else if (a.asrc == AS_WSTREAM) {
    MS_CHECK_ARG(a.M <= kWaveRowsMax && a.rows.x && a.rows.ld >= a.K && !a.rows.gamma &&
                     !a.rows.x_out && wave_shape_ok(a) &&
                     !(a.epi == EPI_ACCUMULATE && a.waves != 8),
                 "GEMV: streamed per-wave rows: at most 4 rows, K = waves * tpw * 128: "
                 "store on 4 (tpw 2, 5) or 8 waves (tpw 1, 2, 4), accumulate on 8, SwiGLU "
                 "on 4, residual on 8 (tpw 1, 2, 4) or 16 waves (tpw 2, 5)");
  } else if (a.asrc == AS_ATTN) {
    MS_CHECK_ARG(a.M == 1 && a.P == 1 && a.waves == 8 && a.epi == EPI_RESID,
                 "GEMV: attention source: one row, one panel per block, 8 waves, residual");
    MS_CHECK_ARG(a.at.part && a.at.pos && a.at.n_heads == a.waves &&
                     (a.at.hd == 128 || a.at.hd == 256 || a.at.hd == 512) &&
                     a.K == a.at.n_heads * a.at.hd && a.at.chunks >= 1 &&
                     a.at.chunks <= kDecPartMaxChunks && a.at.cache_len > 0,
                 "GEMV: attention source: one head of 128/256/512 per wave, K = heads * hd");
  } else {
    MS_CHECK_ARG(a.q.limbs && a.q.shift, "GEMV: quantized rows missing");
  }
  long n_panels = 0;
  for (int i = 0; i < a.nseg; ++i) {
    MS_CHECK_ARG(a.seg[i].w && a.seg[i].n_cols > 0 && a.seg[i].n_cols % 16 == 0,
                 "GEMV: segment width % 16 != 0");
    n_panels += a.seg[i].n_cols / 16;
    if (a.epi != EPI_SWIGLU)
      MS_CHECK_ARG((a.seg[i].n_cols / 16) % a.P == 0,
                   "GEMV: panels per block must divide every segment");
  }
  if (a.epi == EPI_SWIGLU)
    MS_CHECK_ARG(a.seg[0].n_cols == a.seg[1].n_cols, "GEMV: gate/up widths differ");
  const long blocks = (a.epi == EPI_SWIGLU) ? a.seg[0].n_cols / 16 : n_panels / a.P;
  const size_t shmem = gemv_lds_need(a);
  MS_CHECK_ARG(shmem <= 160 * 1024 - 1024, "GEMV: LDS budget exceeded");
  const int C = a.M <= 4 ? 1 : 4;
  bool ok = false;
  // Supported (epilogue, panels per block, activation source, waves).
#define MS_GEMV_L(CC, EP, PP, AS, WW, RR) \
  hipLaunchKernelGGL((k_gemv<CC, PP, AS, WW, EP, RR>), dim3(blocks), dim3(64 * WW), shmem, st, a)
#define MS_GEMV(EP, PP, AS, WW)                                                   \
  if (!ok && a.epi == EP && a.P == PP && a.asrc == AS && a.waves == WW) {        \
    constexpr int RP = WW > 8 ? 1 : 4;                                            \
    if (a.M == 1) MS_GEMV_L(1, EP, PP, AS, WW, 1);                                \
    else if (C == 1) MS_GEMV_L(1, EP, PP, AS, WW, RP);                            \
    else MS_GEMV_L(4, EP, PP, AS, WW, RP);                                        \
    ok = true;                                                                    \
  }
  MS_GEMV(EPI_STORE, 1, AS_ROWS, 8)
  MS_GEMV(EPI_STORE, 1, AS_QUANT, 4)
  MS_GEMV(EPI_STORE, 4, AS_QUANT, 4)
  MS_GEMV(EPI_ACCUMULATE, 1, AS_QUANT, 4)
  MS_GEMV(EPI_ACCUMULATE, 4, AS_QUANT, 4)
  MS_GEMV(EPI_RESID, 1, AS_ROWS, 4)
  MS_GEMV(EPI_RESID, 1, AS_ROWS, 8)
  MS_GEMV(EPI_RESID, 1, AS_ROWS, 16)
  MS_GEMV(EPI_RESID, 1, AS_QUANT, 4)
  if (!ok && a.asrc == AS_WAVES) {
    // RP = 10 * row bound + super-tiles per wave; one row has instantiations
    // of its own (fewer registers)
    const int tpw = a.K / (a.waves * kSuperK);
    if (a.pf.rope_cur) {
      // one row preparing the decode attention's RoPE factors (Q|K|V)
      MS_CHECK_ARG(a.M == 1 && a.epi == EPI_STORE && a.P == 1 && a.waves == 4 &&
                       (tpw == 5 || tpw == 2) && a.pf.pos && a.pf.cos_t && a.pf.sin_t &&
                       a.pf.half >= 0 && a.pf.half <= 256 && a.pf.rope_rows >= 1,
                   "GEMV: attention preparation: one row, store, 4 waves, K = 1024 or 2560");
      if (tpw == 5) MS_GEMV_L(1, EPI_STORE, 1, AS_WAVES, 4, 115);
      else MS_GEMV_L(1, EPI_STORE, 1, AS_WAVES, 4, 112);
      ok = true;
    }
#define MS_GEMV_W(EP, PP, WW, T)                                       \
  if (!ok && a.epi == EP && a.waves == WW && tpw == T) {               \
    if (a.M == 1) MS_GEMV_L(1, EP, PP, AS_WAVES, WW, 10 + T);          \
    else MS_GEMV_L(1, EP, PP, AS_WAVES, WW, 10 * kWaveRowsMax + T);     \
    ok = true;                                                         \
  }
    MS_GEMV_W(EPI_STORE, 1, 4, 5)
    MS_GEMV_W(EPI_STORE, 1, 4, 2)
    MS_GEMV_W(EPI_SWIGLU, 2, 4, 5)
    MS_GEMV_W(EPI_SWIGLU, 2, 4, 2)
    MS_GEMV_W(EPI_RESID, 1, 16, 5)
    MS_GEMV_W(EPI_RESID, 1, 16, 2)
    MS_GEMV_W(EPI_RESID, 1, 8, 1)
    MS_GEMV_W(EPI_RESID, 1, 8, 2)
    MS_GEMV_W(EPI_RESID, 1, 8, 4)
    MS_GEMV_W(EPI_STORE, 1, 8, 1)
    MS_GEMV_W(EPI_STORE, 1, 8, 2)
    MS_GEMV_W(EPI_STORE, 1, 8, 4)
    MS_GEMV_W(EPI_ACCUMULATE, 1, 8, 1)
    MS_GEMV_W(EPI_ACCUMULATE, 1, 8, 2)
    MS_GEMV_W(EPI_ACCUMULATE, 1, 8, 4)
#undef MS_GEMV_W
    MS_CHECK_ARG(ok, "GEMV: per-wave rows: no instantiation for this shape");
  }
  if (!ok && a.asrc == AS_WSTREAM) {
    const int tpw = a.K / (a.waves * kSuperK);
#define MS_GEMV_S(EP, PP, WW, T)                                            \
  if (!ok && a.epi == EP && a.waves == WW && tpw == T) {                    \
    MS_GEMV_L(1, EP, PP, AS_WSTREAM, WW, 10 * kWaveRowsMax + T);            \
    ok = true;                                                              \
  }
    MS_GEMV_S(EPI_STORE, 1, 4, 5)
    MS_GEMV_S(EPI_STORE, 1, 4, 2)
    MS_GEMV_S(EPI_STORE, 1, 8, 1)
    MS_GEMV_S(EPI_STORE, 1, 8, 2)
    MS_GEMV_S(EPI_STORE, 1, 8, 4)
    MS_GEMV_S(EPI_ACCUMULATE, 1, 8, 1)
    MS_GEMV_S(EPI_ACCUMULATE, 1, 8, 2)
    MS_GEMV_S(EPI_ACCUMULATE, 1, 8, 4)
    MS_GEMV_S(EPI_SWIGLU, 2, 4, 5)
    MS_GEMV_S(EPI_SWIGLU, 2, 4, 2)
    MS_GEMV_S(EPI_RESID, 1, 16, 5)
    MS_GEMV_S(EPI_RESID, 1, 16, 2)
    MS_GEMV_S(EPI_RESID, 1, 8, 1)
    MS_GEMV_S(EPI_RESID, 1, 8, 2)
    MS_GEMV_S(EPI_RESID, 1, 8, 4)
#undef MS_GEMV_S
    MS_CHECK_ARG(ok, "GEMV: streamed per-wave rows: no instantiation for this shape");
  }
  if (!ok && a.asrc == AS_ATTN) {
    // the row-prologue template slot carries the head dim and the load pairs
    // per batch (a pair covers 512 / hd chunks)
    const int pairs = (a.at.chunks * a.at.hd + 511) / 512;
    if (a.at.hd == 128) MS_GEMV_L(1, EPI_RESID, 1, AS_ATTN, 8, 104);
    else if (a.at.hd == 256 && pairs <= 4) MS_GEMV_L(1, EPI_RESID, 1, AS_ATTN, 8, 204);
    else if (a.at.hd == 256) MS_GEMV_L(1, EPI_RESID, 1, AS_ATTN, 8, 208);
    else if (pairs <= 4) MS_GEMV_L(1, EPI_RESID, 1, AS_ATTN, 8, 404);
    else if (pairs <= 8) MS_GEMV_L(1, EPI_RESID, 1, AS_ATTN, 8, 408);
    else MS_GEMV_L(1, EPI_RESID, 1, AS_ATTN, 8, 416);
    ok = true;
  }
  if (!ok && a.epi == EPI_RESID && a.P == 1 && a.asrc == AS_QUANT && a.waves == 16) {
    MS_CHECK_ARG(a.M <= 4, "GEMV: 16 waves over global limbs take at most 4 rows");
    if (a.M == 1) MS_GEMV_L(1, EPI_RESID, 1, AS_QUANT, 16, 1);
    else MS_GEMV_L(1, EPI_RESID, 1, AS_QUANT, 16, 4);
    ok = true;
  }
  MS_GEMV(EPI_SWIGLU, 2, AS_ROWS, 8)
  MS_GEMV(EPI_SWIGLU, 2, AS_ROWS, 4)
  MS_GEMV(EPI_SWIGLU, 2, AS_QUANT, 4)
  MS_GEMV(EPI_ARGMAX, 4, AS_QUANT, 4)
#undef MS_GEMV
#undef MS_GEMV_L
  MS_CHECK_ARG(ok, "GEMV: unsupported (epilogue, P, waves, activation source) combination");
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

// ------------------------------------------------------------------------------
// kernel-level entry points
// ------------------------------------------------------------------------------
int pack_device(uint8_t *dst, const uint8_t *src, int K, int N, hipStream_t st) {
  int rc = check_q4_shape(K, N);
  if (rc) return rc;
  const size_t total = (size_t)K * N / 8;
  hipLaunchKernelGGL(k_pack, dim3(cdiv((long)total, kBlock)), dim3(kBlock), 0, st,
                     reinterpret_cast<uint32_t *>(dst), src, K, N);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

}  // namespace ms

using namespace ms;

extern "C" size_t ms_q4_packed_bytes(int K, int N) { return (size_t)K * N / 2; }

extern "C" int ms_q4_pack(uint8_t *d_packed, const uint8_t *d_rowmajor, int K, int N) {
  if (int rc = require_init()) return rc;
  return pack_device(d_packed, d_rowmajor, K, N, ctx().stream);
}

extern "C" int ms_host_q4_pack(uint8_t *h_packed, const uint8_t *h_rowmajor, int K,
                               int N) {
  if (int rc = check_q4_shape(K, N)) return rc;
  const size_t pc = (size_t)N / 2;
  uint32_t *dst = reinterpret_cast<uint32_t *>(h_packed);
  const size_t per_panel = (size_t)K * 2;
  for (int nb = 0; nb < N / 16; ++nb)
    for (int G = 0; G < K / 128; ++G)
      for (int lane = 0; lane < 64; ++lane)
        for (int t = 0; t < 4; ++t) {
          const int j = lane % 16, g = lane / 16, n = nb * 16 + j;
          uint32_t d = 0;
          for (int e = 0; e < 8; ++e) {
            const int k = 128 * G + 32 * g + 8 * t + e;
            const uint8_t b = h_rowmajor[(size_t)k * pc + (n >> 1)];
            const uint32_t nib = (n & 1) ? (uint32_t)(b >> 4) : (uint32_t)(b & 15);
            d |= nib << (4 * ((e >> 1) + 4 * (e & 1)));
          }
          dst[(size_t)nb * per_panel + (size_t)G * 256 + lane * 4 + t] = d;
        }
  return MS_OK;
}

extern "C" int ms_dequant_q4(float *d_out, const uint8_t *d_rowmajor, int K, int N,
                             float scale) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(K > 0 && N > 0 && N % 2 == 0, "dequant: bad shape");
  const size_t nbytes = (size_t)K * N / 2;
  hipLaunchKernelGGL(k_dequant_rowmajor, dim3(cdiv((long)nbytes, kBlock)), dim3(kBlock), 0,
                     ctx().stream, d_out, d_rowmajor, nbytes, scale);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

extern "C" int ms_dequant_q4_packed(float *d_out, const uint8_t *d_packed, int K, int N,
                                    float scale) {
  if (int rc = require_init()) return rc;
  if (int rc = check_q4_shape(K, N)) return rc;
  const size_t total = (size_t)K * N / 8;
  hipLaunchKernelGGL(k_dequant_packed, dim3(cdiv((long)total, kBlock)), dim3(kBlock), 0,
                     ctx().stream, d_out, reinterpret_cast<const uint32_t *>(d_packed),
                     K, N, scale);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

// ------------------------------------------------------------------------------
// No-allocation scratch: the quantized activation rows of
// ms_q4_matmul_noalloc live in this file-scope device array (one copy per GPU
// the library runs on, held until the process ends).  Its device address is
// taken once per device by q4_noalloc_init (from ms_init, with that device
// current); host code uses that address, never the array's name.
// ------------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = (size_t)4 << 20;  // 4 MiB
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace ms {

constexpr int kNoAllocMaxDevices = 64;
static void *g_noalloc_ptr[kNoAllocMaxDevices] = {};

int q4_noalloc_init(int device) {
  MS_CHECK_ARG(device >= 0 && device < kNoAllocMaxDevices, "no-alloc scratch: device index");
  if (g_noalloc_ptr[device]) return MS_OK;
  void *p = nullptr;
  MS_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(::scratch)));
  MS_CHECK_ARG(p != nullptr, "no-alloc scratch: no device address");
  g_noalloc_ptr[device] = p;
  return MS_OK;
}

// Scratch bytes a q4 matmul of M rows of length K uses for its quantized rows.
// The K split's partial sums follow the quantized rows, 256-byte aligned.
static size_t q4_matmul_rows_bytes(int M, int K) {
  const size_t b = M > kGemvMaxM ? quant_rows_bytes(gemm_row_pad(M), K)
                                 : quant_rows_bytes(kGemvMaxM, K);
  return (b + 255) & ~(size_t)255;
}
static size_t q4_matmul_scratch_bytes(int M, int K, int N, int ks) {
  return q4_matmul_rows_bytes(M, K) + (ks > 1 ? (size_t)ks * M * N * 8 : 0);
}

// C (+)= A . deq(W) with the quantized rows (and, with ks > 1 K parts, their
// partial sums) in `buf` (q4_matmul_scratch_bytes).
static int q4_matmul_impl(float *d_C, const float *d_A, const uint8_t *d_packed, int M, int K,
                          int N, float scale, int accumulate, void *buf, int ks) {
  hipStream_t st = ctx().stream;
  if (M > kGemvMaxM) {
    // many rows: quantize all of them once, then the MFMA GEMM (its K split
    // over ks block groups when few tiles would leave most CUs idle)
    const int Mp = gemm_row_pad(M);
    GemmArgs g{};
    g.epi = accumulate ? EPI_ACCUMULATE : EPI_STORE;
    g.M = M;
    g.K = K;
    g.a = quant_rows3_view(buf, Mp, K);
    g.ksplit = ks;
    if (ks > 1)
      g.kpart = reinterpret_cast<int64_t *>(static_cast<uint8_t *>(buf) +
                                            q4_matmul_rows_bytes(M, K));
    RowSrc r{};
    r.x = d_A;
    r.ld = K;
    r.pre_scale = 1.f;
    if (int rc = launch_quant_rows3(r, M, K, g.a, st)) return rc;
    g.seg[0] = GemvSeg{d_packed, scale, N, 0};
    g.nseg = 1;
    g.out = d_C;
    g.ldo = N;
    return launch_gemm(g, st);
  }
  if (M <= kWaveRowsMax) {
    // one launch: each wave quantizes its own K slice of the rows (a shift
    // per row and wave), no quantization pass before the GEMV.  Two to four
    // rows stream their slices one super-tile at a time (lane l: row l / 16),
    // with the same limbs and shifts as the one-row kernel, so each row's
    // result equals that row alone (K = N = 1024 at four rows: 5.4 -> 3.7 us;
    // 4096: 6.2 -> 5.7 us)
    GemvArgs a{};
    a.epi = accumulate ? EPI_ACCUMULATE : EPI_STORE;
    a.asrc = M > 1 ? AS_WSTREAM : AS_WAVES;
    a.K = K;
    a.M = M;
    a.rows.x = d_A;
    a.rows.ld = K;
    a.rows.pre_scale = 1.f;
    a.seg[0] = GemvSeg{d_packed, scale, N, 0};
    a.nseg = 1;
    a.P = 1;
    a.out = d_C;
    a.ldo = N;
    for (const int w : {8, 4}) {
      a.waves = w;
      if (wave_shape_ok(a) && gemv_lds_need(a) <= 150 * 1024) return launch_gemv(a, st);
    }
  }
  const int chunk = kGemvMaxM;
  const int P = (N / 16) % 4 == 0 && N >= 4 * 16 * 512 ? 4 : 1;
  const QuantRows q = quant_rows_view(buf, chunk, K);
  for (int m0 = 0; m0 < M; m0 += chunk) {
    const int mm = (M - m0 < chunk) ? M - m0 : chunk;
    RowSrc r{};
    r.x = d_A + (size_t)m0 * K;
    r.ld = K;
    r.pre_scale = 1.f;
    if (int rc = launch_quant_rows(r, mm, K, q, st)) return rc;
    GemvArgs a{};
    a.epi = accumulate ? EPI_ACCUMULATE : EPI_STORE;
    a.asrc = AS_QUANT;
    a.K = K;
    a.M = mm;
    a.q = q;
    a.seg[0] = GemvSeg{d_packed, scale, N, 0};
    a.nseg = 1;
    a.P = P;
    a.waves = 4;
    a.out = d_C + (size_t)m0 * N;
    a.ldo = N;
    if (int rc = launch_gemv(a, st)) return rc;
  }
  return MS_OK;
}

static int q4_matmul_check(int M, int K, int N) {
  if (int rc = check_q4_shape(K, N)) return rc;
  MS_CHECK_ARG(M >= 1, "matmul: M must be >= 1");
  MS_CHECK_ARG(K <= kQuantMaxK, "matmul: K must be <= 16384");
  return MS_OK;
}

}  // namespace ms

extern "C" int ms_q4_matmul(float *d_C, const float *d_A, const uint8_t *d_packed, int M,
                            int K, int N, float scale, int accumulate) {
  using namespace ms;
  if (int rc = require_init()) return rc;
  if (int rc = q4_matmul_check(M, K, N)) return rc;
  const int ks = gemm_ksplit(M, K, N);
  void *buf = nullptr;
  if (int rc = ms::scratch(q4_matmul_scratch_bytes(M, K, N, ks), &buf)) return rc;
  return q4_matmul_impl(d_C, d_A, d_packed, M, K, N, scale, accumulate, buf, ks);
}

extern "C" int ms_bench_q4_matmul(float *d_C, const float *d_A, const uint8_t *d_w0,
                                  size_t w_stride, int n_w, int M, int K, int N, float scale,
                                  int reps, double *avg_us) {
  using namespace ms;
  if (int rc = require_init()) return rc;
  if (int rc = q4_matmul_check(M, K, N)) return rc;
  MS_CHECK_ARG(d_C && d_A && d_w0 && n_w >= 1 && reps >= 1 && avg_us, "bench_q4_matmul: bad args");
  MS_CHECK_ARG(n_w == 1 || w_stride >= (size_t)K * N / 2, "bench_q4_matmul: stride < matrix bytes");
  const int ks = gemm_ksplit(M, K, N);
  void *buf = nullptr;
  if (int rc = ms::scratch(q4_matmul_scratch_bytes(M, K, N, ks), &buf)) return rc;
  hipStream_t st = ctx().stream;
  // one untimed call (code objects, caches of the activations)
  if (int rc = q4_matmul_impl(d_C, d_A, d_w0, M, K, N, scale, 0, buf, ks)) return rc;
  hipEvent_t e0, e1;
  MS_HIP_TRY(hipEventCreate(&e0));
  MS_HIP_TRY(hipEventCreate(&e1));
  MS_HIP_TRY(hipEventRecord(e0, st));
  int rc = MS_OK;
  for (int r = 0; r < reps && rc == MS_OK; ++r)
    rc = q4_matmul_impl(d_C, d_A, d_w0 + (size_t)(r % n_w) * w_stride, M, K, N, scale, 0, buf,
                        ks);
  (void)hipEventRecord(e1, st);
  (void)hipEventSynchronize(e1);
  float ms_ = 0.f;
  (void)hipEventElapsedTime(&ms_, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (rc) return rc;
  *avg_us = (double)ms_ * 1e3 / reps;
  return MS_OK;
}

extern "C" int ms_q4_matmul_noalloc(float *d_C, const float *d_A, const uint8_t *d_packed,
                                    int M, int K, int N, float scale, int accumulate) {
  using namespace ms;
  if (int rc = require_init()) return rc;
  if (int rc = q4_matmul_check(M, K, N)) return rc;
  // the K split only where its partial sums fit too (the result is the same
  // either way)
  int ks = gemm_ksplit(M, K, N);
  if (q4_matmul_scratch_bytes(M, K, N, ks) > kNoAllocScratchBytes) ks = 1;
  const size_t need = q4_matmul_scratch_bytes(M, K, N, ks);
  if (need > kNoAllocScratchBytes)
    return fail(MS_E_INVALID, "q4_matmul_noalloc: " + std::to_string(M) + " rows of " +
                                  std::to_string(K) + " need " + std::to_string(need) +
                                  " bytes of scratch, above its 4 MiB maximum");
  void *buf = g_noalloc_ptr[ctx().device];
  if (!buf) return fail(MS_E_STATE, "q4_matmul_noalloc: scratch address not set up");
  return q4_matmul_impl(d_C, d_A, d_packed, M, K, N, scale, accumulate, buf, ks);
}

