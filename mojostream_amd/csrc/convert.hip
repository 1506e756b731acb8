// Converter quantization on the device: quantize_q4_blockwise
// (scripts/convert.py:296-323) applied to a HuggingFace (out, in) weight, as the
// converter does after its transpose (convert.py:503-518).
//
// The reference transposes to (in, out), splits the flat array into blocks of
// block_size, takes max|w| / 7 per block (1e-8 for a block whose max is not
// above 1e-8) and keeps the largest as the one global scale.  Then
// q = clip(round_half_even(w / scale), -8, 7) + 8, even columns in the low
// nibble.  The largest block scale is max|w| / 7 unless that is below 1e-8 and
// some block is "tiny"; only then does the block structure matter, and only
// then is it examined (k_tiny_blocks).
//
// k_absmax_part / k_absmax_fin   max |w| over the matrix and a non-finite flag.
// k_q4_pack_t   64 (in) x 128 (out) tiles through LDS: coalesced reads along
//               the HF rows, the tile transposed in LDS, 16 packed bytes per
//               thread written along the (in, out) rows.  HBM-bound: the
//               weight once (2 or 4 B per element) plus half a byte written.
#include "common.h"
#include "devutil.h"

#include <hip/hip_fp16.h>

#include <algorithm>
#include <cmath>

namespace ms {
namespace {

constexpr int kTk = 64, kTn = 128;
constexpr int kMaxParts = 1024;

// dtype 0 fp32, 1 bf16, 2 fp16 (SafetensorsReader.load_f32, convert.py:100-110)
__device__ inline float load_w(const void *w, int dtype, size_t i) {
  if (dtype == 0) return static_cast<const float *>(w)[i];
  const uint16_t h = static_cast<const uint16_t *>(w)[i];
  if (dtype == 1) return __uint_as_float((uint32_t)h << 16);
  return __half2float(__ushort_as_half(h));
}

// The 16-byte word v as 4 (fp32) or 8 (bf16, fp16) values.
template <int DT>
__device__ inline void unpack16(const u32x4 v, float *o) {
  const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (DT == 0) {
      o[i] = __uint_as_float(u[i]);
    } else if constexpr (DT == 1) {
      o[2 * i] = __uint_as_float(u[i] << 16);
      o[2 * i + 1] = __uint_as_float(u[i] & 0xFFFF0000u);
    } else {
      o[2 * i] = __half2float(__ushort_as_half((uint16_t)(u[i] & 0xFFFFu)));
      o[2 * i + 1] = __half2float(__ushort_as_half((uint16_t)(u[i] >> 16)));
    }
  }
}

// nvec 16-byte words first (the host passes 0 for an unaligned base), then the
// remaining elements one by one.
template <int DT>
__global__ __launch_bounds__(256) void k_absmax_part(const void *w, size_t n, size_t nvec,
                                                     float *part) {
  constexpr int PER = DT == 0 ? 4 : 8;
  __shared__ float sm[256];
  __shared__ int sb[256];
  const int tid = threadIdx.x;
  float m = 0.f;
  int bad = 0;
  const size_t g = (size_t)blockIdx.x * 256 + tid, stride = (size_t)gridDim.x * 256;
  for (size_t v = g; v < nvec; v += stride) {
    float x[PER];
    unpack16<DT>(ldg_nt<u32x4>(static_cast<const uint8_t *>(w) + 16 * v), x);
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      bad |= !isfinite(x[i]);
      m = fmaxf(m, fabsf(x[i]));
    }
  }
  for (size_t i = nvec * PER + g; i < n; i += stride) {
    const float x = load_w(static_cast<const void *>(w), DT, i);
    bad |= !isfinite(x);
    m = fmaxf(m, fabsf(x));
  }
  sm[tid] = m;
  sb[tid] = bad;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) {
      sm[tid] = fmaxf(sm[tid], sm[tid + s]);
      sb[tid] |= sb[tid + s];
    }
    __syncthreads();
  }
  if (tid == 0) {
    part[2 * blockIdx.x] = sm[0];
    part[2 * blockIdx.x + 1] = (float)sb[0];
  }
}

__global__ __launch_bounds__(256) void k_absmax_fin(float *part, int nb) {
  __shared__ float sm[256], sb[256];
  const int tid = threadIdx.x;
  float m = 0.f, b = 0.f;
  for (int i = tid; i < nb; i += 256) {
    m = fmaxf(m, part[2 * i]);
    b = fmaxf(b, part[2 * i + 1]);
  }
  sm[tid] = m;
  sb[tid] = b;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) {
      sm[tid] = fmaxf(sm[tid], sm[tid + s]);
      sb[tid] = fmaxf(sb[tid], sb[tid + s]);
    }
    __syncthreads();
  }
  if (tid == 0) {
    part[0] = sm[0];
    part[1] = sb[0];
  }
}

// flag = 1 when a block of bs consecutive elements of the (in, out) matrix has
// max |w| <= 1e-8 (convert.py:311-314).  Every writer stores the same value.
__global__ __launch_bounds__(256) void k_tiny_blocks(const void *w, int dtype, int n_out, int n_in,
                                                     int bs, size_t nblocks, int *flag) {
  const size_t b = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= nblocks) return;
  const size_t total = (size_t)n_out * n_in;
  const size_t i0 = b * (size_t)bs, i1 = i0 + (size_t)bs < total ? i0 + (size_t)bs : total;
  float m = 0.f;
  for (size_t i = i0; i < i1; ++i) {
    const size_t k = i / (size_t)n_out, o = i % (size_t)n_out;
    m = fmaxf(m, fabsf(load_w(w, dtype, o * (size_t)n_in + k)));
  }
  if (!((double)m > 1e-8)) flag[0] = 1;
}

__device__ inline uint32_t q4_code(float x, float s) {
  const int q = (int)rintf(__fdiv_rn(x, s));
  return (uint32_t)(min(7, max(-8, q)) + 8);
}

// VEC: rows of the weight read as 16-byte words (n_in a multiple of the word's
// element count, base aligned); else element by element.
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void k_q4_pack_t(const void *w, int n_out, int n_in, float s,
                                                   uint8_t *out) {
  constexpr int PER = DT == 0 ? 4 : 8, ESZ = DT == 0 ? 4 : 2;
  __shared__ float t[kTk][kTn + 1];
  const int tid = threadIdx.x;
  const int k0 = blockIdx.x * kTk, n0 = blockIdx.y * kTn;
  if constexpr (VEC) {
    constexpr int CPR = kTk / PER;  // words per tile row
#pragma unroll
    for (int e = tid; e < kTn * CPR; e += 256) {
      const int r = e / CPR, c = (e % CPR) * PER;
      const int n = n0 + r, k = k0 + c;
      float x[PER];
      if (n < n_out && k < n_in) {
        const uint8_t *src = static_cast<const uint8_t *>(w) + ((size_t)n * n_in + k) * ESZ;
        unpack16<DT>(ldg_nt<u32x4>(src), x);
      } else {
#pragma unroll
        for (int i = 0; i < PER; ++i) x[i] = 0.f;
      }
#pragma unroll
      for (int i = 0; i < PER; ++i) t[c + i][r] = x[i];
    }
  } else {
    for (int e = tid; e < kTk * kTn; e += 256) {
      const int r = e / kTk, c = e % kTk;  // r: out index in the tile, c: in index
      const int n = n0 + r, k = k0 + c;
      t[c][r] = (n < n_out && k < n_in) ? load_w(w, DT, (size_t)n * n_in + k) : 0.f;
    }
  }
  __syncthreads();
  const int c = tid >> 2, j0 = (tid & 3) * 16;  // 16 bytes = 32 out values of row k
  const int k = k0 + c;
  if (k >= n_in) return;
  const size_t half = (size_t)n_out / 2;
  const size_t jb = (size_t)n0 / 2 + j0;
  if (jb >= half) return;
  uint32_t wd[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t v = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int j = j0 + 4 * q + b;
      const uint32_t lo = q4_code(t[c][2 * j], s), hi = q4_code(t[c][2 * j + 1], s);
      v |= (lo | (hi << 4)) << (8 * b);
    }
    wd[q] = v;
  }
  uint8_t *dst = out + (size_t)k * half + jb;
  if (jb + 16 <= half && (half & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
    *reinterpret_cast<uint4 *>(dst) = uint4{wd[0], wd[1], wd[2], wd[3]};
  } else {
    for (int j = 0; j < 16 && jb + j < half; ++j) dst[j] = (uint8_t)(wd[j / 4] >> (8 * (j % 4)));
  }
}

}  // namespace

}  // namespace ms

using namespace ms;

extern "C" int ms_q4_quantize(uint8_t *d_packed, float *h_scale, const void *d_w, int dtype,
                              int n_out, int n_in, int block_size) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(d_packed && h_scale && d_w, "q4_quantize: null argument");
  MS_CHECK_ARG(dtype >= 0 && dtype <= 2, "q4_quantize: dtype 0 (fp32), 1 (bf16) or 2 (fp16)");
  MS_CHECK_ARG(n_out >= 2 && n_out % 2 == 0 && n_in >= 1,
               "q4_quantize: out dimension must be even (two values per byte, convert.py:304)");
  MS_CHECK_ARG(block_size >= 1, "q4_quantize: block_size must be positive");
  MS_CHECK_ARG((long)n_in <= 65535L * kTk && n_out / kTn < 65535, "q4_quantize: matrix too large");
  hipStream_t st = ctx().stream;
  const size_t n = (size_t)n_out * n_in;
  void *buf = nullptr;
  if (int rc = scratch(kMaxParts * 2 * 4 + 64, &buf)) return rc;
  float *part = static_cast<float *>(buf);
  int *flag = reinterpret_cast<int *>(part + kMaxParts * 2);
  const int esz = dtype == 0 ? 4 : 2, per = 16 / esz;
  const bool aligned = (reinterpret_cast<uintptr_t>(d_w) & 15) == 0;
  const size_t nvec = aligned ? n / per : 0;
  const int nb = (int)std::min<size_t>(kMaxParts, std::max<size_t>(1, cdiv((long)n, 256 * 32)));
  if (dtype == 0)
    hipLaunchKernelGGL(k_absmax_part<0>, dim3(nb), dim3(256), 0, st, d_w, n, nvec, part);
  else if (dtype == 1)
    hipLaunchKernelGGL(k_absmax_part<1>, dim3(nb), dim3(256), 0, st, d_w, n, nvec, part);
  else
    hipLaunchKernelGGL(k_absmax_part<2>, dim3(nb), dim3(256), 0, st, d_w, n, nvec, part);
  hipLaunchKernelGGL(k_absmax_fin, dim3(1), dim3(256), 0, st, part, nb);
  MS_HIP_TRY(hipGetLastError());
  float fin[2];
  MS_HIP_TRY(hipMemcpyAsync(fin, part, 8, hipMemcpyDeviceToHost, st));
  MS_HIP_TRY(hipStreamSynchronize(st));
  MS_CHECK_ARG(fin[1] == 0.f, "q4_quantize: the weight holds NaN or infinity");
  // max over the block scales (convert.py:310-316), in double as Python does
  const double g = fin[0];
  double gs;
  if (!(g > 1e-8)) {
    gs = 1e-8;  // every block is tiny
  } else {
    gs = g / 7.0;
    if (gs < 1e-8) {
      const size_t nblocks = (n + block_size - 1) / block_size;
      int tiny = 0;
      MS_HIP_TRY(hipMemcpyAsync(flag, &tiny, 4, hipMemcpyHostToDevice, st));
      hipLaunchKernelGGL(k_tiny_blocks, dim3(cdiv((long)nblocks, 256)), dim3(256), 0, st, d_w,
                         dtype, n_out, n_in, block_size, nblocks, flag);
      MS_HIP_TRY(hipGetLastError());
      MS_HIP_TRY(hipMemcpyAsync(&tiny, flag, 4, hipMemcpyDeviceToHost, st));
      MS_HIP_TRY(hipStreamSynchronize(st));
      if (tiny) gs = 1e-8;
    }
  }
  const float s = (float)gs;
  const dim3 grid(cdiv((long)n_in, kTk), cdiv((long)n_out, kTn));
  const bool vec = aligned && n_in % per == 0;
#define MS_PACK(DT, V) \
  hipLaunchKernelGGL((k_q4_pack_t<DT, V>), grid, dim3(256), 0, st, d_w, n_out, n_in, s, d_packed)
  if (dtype == 0) {
    if (vec) MS_PACK(0, true); else MS_PACK(0, false);
  } else if (dtype == 1) {
    if (vec) MS_PACK(1, true); else MS_PACK(1, false);
  } else {
    if (vec) MS_PACK(2, true); else MS_PACK(2, false);
  }
#undef MS_PACK
  MS_HIP_TRY(hipGetLastError());
  MS_HIP_TRY(hipStreamSynchronize(st));
  *h_scale = s;
  return MS_OK;
}
