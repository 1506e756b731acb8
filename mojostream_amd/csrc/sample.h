// Device token sampling (temperature_sampling, lm_head.mojo:198-254).
#pragma once
#include "common.h"

namespace ms {

constexpr int kSampleMaxHistory = 8192;  // ids of a row's history the penalty sees

struct SampleArgs {
  float *logits;          // [rows][ld]; penalized logits or probabilities on return
  int n, ld;              // vocabulary, row stride
  float temperature;      // <= 0.01: greedy
  float penalty;          // > 1: repetition penalty over the history
  int32_t *hist;          // [rows][hist_ld] token history (prompt + generated)
  int hist_ld;
  int32_t *hist_n;        // [rows] history length (device)
  int hist_cap;           // hist_append: capacity of a row's history
  int hist_append;        // append the sampled id to the history
  uint64_t seed;          // with step: base seed of draw_seed(seed, seq0 + row, *step);
                          // without: the seed of the one draw
  int seq0;               // sequence index of row 0 (with step)
  const int32_t *step;    // device draw counter or null
  int32_t *ids_out;       // [rows] or null
  int32_t *tok_state;     // [rows] or null: next input token
};

// Seed of draw k of sequence seq (model sampling): a splitmix64 hash of the
// triple, so that sequences and consecutive draws get independent LCG inputs.
__host__ __device__ inline uint64_t draw_seed(uint64_t seed, uint64_t seq, uint64_t k) {
  return rand_word(seed, seq + 1, k);
}

int launch_sample(const SampleArgs &a, int rows, hipStream_t st);

}  // namespace ms
