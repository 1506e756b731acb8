// FP32 LM head (LMHead version 2, lm_head.mojo:61-116): the projection
// matmul_fp32_raw (kernels.mojo:616-671) and the column embedding
// (get_token_embedding, lm_head.mojo:179-185).
//
// k_mm_f32   C[M][N] (+)= A[M][K] . B[K][N] for M <= 16, B fp32 row-major.
//            B is streamed once: a block owns 1024 columns (a float4 per
//            thread) of one K split; the rows of A for its K range are staged
//            in LDS.  Each split writes its partial sums, and k_mm_f32_sum adds
//            the splits in split order, so the result does not depend on
//            scheduling.  HBM-bound: 4 K N bytes of B per launch.
// k_embed_f32  out[t][r] = B[r][token_t]: one column of [D][vocab].
#include "common.h"
#include "head_f32.h"

#include <algorithm>

namespace ms {
namespace {

constexpr int kMmCols = 1024;   // columns per block (256 threads x float4)
constexpr int kMmKChunk = 256;  // K rows of A staged per pass

template <int MR>
__global__ __launch_bounds__(256) void k_mm_f32(const float *__restrict__ A,
                                                const float *__restrict__ B, float *part, int M,
                                                int K, int N, int kps) {
  __shared__ float as[MR][kMmKChunk];
  const int tid = threadIdx.x;
  const int c = blockIdx.x * kMmCols + 4 * tid;
  const int ks = blockIdx.y;
  const int k0 = ks * kps, k1 = min(K, k0 + kps);
  float4 acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = float4{0.f, 0.f, 0.f, 0.f};
  for (int kb = k0; kb < k1; kb += kMmKChunk) {
    const int nk = min(kMmKChunk, k1 - kb);
    __syncthreads();
    for (int e = tid; e < MR * kMmKChunk; e += 256) {
      const int m = e / kMmKChunk, k = e % kMmKChunk;
      as[m][k] = (m < M && k < nk) ? A[(size_t)m * K + kb + k] : 0.f;
    }
    __syncthreads();
    if (c < N) {
#pragma unroll 8
      for (int k = 0; k < nk; ++k) {
        typedef float f32x4 __attribute__((ext_vector_type(4)));
        const f32x4 b = __builtin_nontemporal_load(
            reinterpret_cast<const f32x4 *>(B + (size_t)(kb + k) * N + c));
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const float a = as[m][k];
          acc[m].x += a * b.x;
          acc[m].y += a * b.y;
          acc[m].z += a * b.z;
          acc[m].w += a * b.w;
        }
      }
    }
  }
  if (c < N) {
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < M) *reinterpret_cast<float4 *>(part + ((size_t)ks * M + m) * N + c) = acc[m];
  }
}

__global__ __launch_bounds__(256) void k_mm_f32_sum(const float *part, float *C, int M, int N,
                                                    int ks, int accumulate) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)M * N) return;
  float s = 0.f;
  for (int k = 0; k < ks; ++k) s += part[(size_t)k * M * N + i];
  C[i] = accumulate ? C[i] + s : s;
}

__global__ __launch_bounds__(256) void k_embed_f32(const float *__restrict__ B, int D, int vocab,
                                                   const int32_t *tokens, float *out) {
  const int t = blockIdx.x;
  const int tok = tokens[t];
  for (int r = threadIdx.x; r < D; r += 256) out[(size_t)t * D + r] = B[(size_t)r * vocab + tok];
}

}  // namespace

int mm_f32_splits(int N) {
  // about four blocks per CU: the column tiles times the K splits
  const int tiles = (N + kMmCols - 1) / kMmCols;
  return std::max(1, std::min(16, 1024 / std::max(1, tiles)));
}

size_t mm_f32_part_floats(int M, int N) { return (size_t)mm_f32_splits(N) * M * N; }

int launch_mm_f32(const float *A, const float *B, float *C, int M, int K, int N, int accumulate,
                  float *part, hipStream_t st) {
  MS_CHECK_ARG(A && B && C && part && M >= 1 && M <= 16 && K >= 1 && N >= 16 && N % 16 == 0,
               "matmul_f32: 1 <= M <= 16, N a positive multiple of 16");
  const int ks = std::min(mm_f32_splits(N), K);
  const int kps = (K + ks - 1) / ks;
  const dim3 grid((N + kMmCols - 1) / kMmCols, ks);
  if (M <= 1)
    hipLaunchKernelGGL(k_mm_f32<1>, grid, dim3(256), 0, st, A, B, part, M, K, N, kps);
  else if (M <= 4)
    hipLaunchKernelGGL(k_mm_f32<4>, grid, dim3(256), 0, st, A, B, part, M, K, N, kps);
  else
    hipLaunchKernelGGL(k_mm_f32<16>, grid, dim3(256), 0, st, A, B, part, M, K, N, kps);
  hipLaunchKernelGGL(k_mm_f32_sum, dim3(cdiv((long)M * N, 256)), dim3(256), 0, st, part, C, M,
                     N, ks, accumulate);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

int launch_embed_f32(const float *B, int D, int vocab, const int32_t *tokens, int n, float *out,
                     hipStream_t st) {
  hipLaunchKernelGGL(k_embed_f32, dim3(n), dim3(256), 0, st, B, D, vocab, tokens, out);
  MS_HIP_TRY(hipGetLastError());
  return MS_OK;
}

}  // namespace ms

using namespace ms;

extern "C" int ms_matmul_f32(float *d_c, const float *d_a, const float *d_b, int M, int K, int N,
                             int accumulate) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(M >= 1 && M <= 16 && K >= 1 && N >= 16 && N % 16 == 0,
               "matmul_f32: 1 <= M <= 16, N a positive multiple of 16 (the reference computes "
               "whole 16-column tiles only, kernels.mojo:640)");
  hipStream_t st = ctx().stream;
  void *buf = nullptr;
  if (int rc = scratch(mm_f32_part_floats(M, N) * 4, &buf)) return rc;
  if (int rc = launch_mm_f32(d_a, d_b, d_c, M, K, N, accumulate, static_cast<float *>(buf), st))
    return rc;
  MS_HIP_TRY(hipStreamSynchronize(st));
  return MS_OK;
}
