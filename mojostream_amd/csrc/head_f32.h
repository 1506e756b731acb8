// FP32 LM head (LMHead version 2): projection and column embedding.
#pragma once
#include "common.h"

namespace ms {

// Partial-sum floats launch_mm_f32 needs for M rows and N columns.
size_t mm_f32_part_floats(int M, int N);
// C (+)= A . B, A [M][K], B [K][N] fp32 row-major, M <= 16, N % 16 == 0.
int launch_mm_f32(const float *A, const float *B, float *C, int M, int K, int N, int accumulate,
                  float *part, hipStream_t st);
// out[t][:] = column tokens[t] of B [D][vocab].
int launch_embed_f32(const float *B, int D, int vocab, const int32_t *tokens, int n, float *out,
                     hipStream_t st);

}  // namespace ms
