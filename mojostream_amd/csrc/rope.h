#pragma once
#include <vector>

#include "common.h"

namespace ms {
// cos/sin of the reference's fp32 RoPE angles for positions pos0..pos0+n_pos-1,
// [n_pos][rot/2] (kernels.mojo:563-577).
void rope_table_host(int rot, float theta, int pos0, int n_pos, std::vector<float> &cs,
                     std::vector<float> &sn);
int launch_embed(const uint8_t *w, int D, int vocab, float scale, const int32_t *tokens,
                 int n, float *out, hipStream_t st);
}  // namespace ms
