// Decode / chunked-prefill attention interface.
#pragma once
#include "common.h"

namespace ms {

struct AttnArgs {
  int B, T;                 // sequences, rows per sequence
  int q_dim, kv_dim, hd, n_heads, n_kv, rot;
  int cache_kind, cache_len, clamp;
  float scale;              // 1/sqrt(head_dim)
  // q|k|v rows [B*T][ld]: q at column 0, k at q_dim, v at q_dim + kv_dim
  const float *qkv;
  int ld;
  int apply_rope;
  const float *cos_t, *sin_t;  // [positions][rot/2]
  const int32_t *pos;          // base position per sequence [B]
  float *kc, *vc;              // caches [B][cache_len][kv_dim]
  size_t cache_seq_stride;     // floats between sequences
  int n_chunks;                // chunks of kAttnChunk keys per (sequence, kv head)
  float *part;                 // attn_part_floats(B, n_kv, n_chunks, T, G, hd)
  // combine
  float *out;                  // [B*T][q_dim]
  int write_cache;
  // decode (T == 1): per (sequence, kv head) count of finished chunk blocks;
  // zero on entry, left zero on exit
  unsigned *ctr;
  // prefill: first position of the rows as the host expects it; it sizes the
  // key split and nothing else (the kernels read pos)
  int plan_pos;
  // decode: every sequence's position is below pos_bound (0: no bound).  Only
  // the chunks below it are launched, and they load their cached rows before
  // the position arrives.  A position at or past the bound loses its keys
  // beyond the launched chunks: the host must keep the bound.
  int pos_bound;
  int grid_chunks;  // set by the launcher
  // decode partials: cos and sin of the RoPE angles at the row's position,
  // [2][rot / 2] (written before the launch: by the one-row Q|K|V projection
  // or by launch_rope_cur), read at kernel entry instead of the tables
  const float *rope_cur;
};

constexpr int kAttnChunk = 16;
constexpr int kAttnMaxTG = 20;    // T * (n_heads / n_kv) per block
constexpr int kAttnLds = 10240;   // floats of q staging
constexpr int kAttnMaxChunks = 512;

// Floats of AttnArgs::part for B sequences of T rows in n_chunks key chunks.
inline size_t attn_part_floats(int B, int n_kv, int n_chunks, int T, int G, int hd) {
  return (size_t)B * n_kv * ((size_t)n_chunks * T * G * (hd + 2) + 4);
}

// Decode at one row per sequence with the merge left to the consumer: one
// block per (32-key chunk, sequence x kv head) writes the chunk's unnormalized
// o = sum_k e^(s_k - m) v_k and (m, l = sum_k e^(s_k - m)) per query head, and
// the block holding the current slot appends the row's k and v to the cache.
// The O projection merges the chunks (AttnSrc in q4.h).  Per sequence, at
// a.part: o [kDecPartMaxChunks][n_heads][hd], then (m, l)
// [kDecPartMaxChunks][n_heads][2].  Needs G <= 4, head dim 256 or 512 and at
// most kDecPartMaxChunks
// launched chunks (dec_part_ok).
constexpr int kDecPartChunk = 32;
constexpr int kDecPartMaxChunks = 64;
inline size_t dec_part_floats(int B, int n_heads, int hd) {
  return (size_t)B * kDecPartMaxChunks * n_heads * (hd + 2);
}
// Chunks a partials launch covers (the host's position bound, else the cache).
int dec_part_chunks(const AttnArgs &a);
bool dec_part_ok(const AttnArgs &a);
// Counters a model keeps for the decode attention (zero between launches):
// k_attn_decode uses one per (sequence, kv head), the merging partials one per
// (sequence, kv head, pair of query heads).
inline size_t attn_ctr_count(int max_seqs, int n_kv) { return (size_t)max_seqs * n_kv * 2; }
// merge = true: the same blocks, the RoPE factors from the tables at each
// sequence's position, and the last block of each (sequence, kv head, pair of
// query heads) merges the chunks into a.out [B][q_dim] (a.ctr: B * n_kv * 2
// counters, zero between launches).
int launch_attention_partials(const AttnArgs &a, hipStream_t st, bool merge = false);
// Two to four rows of one sequence on a linear cache (attn_rows_ok): the
// chunk scheme of the decode step per row (k_attn_rows), then the chunks
// merged per row and query head into a.out [T][q_dim].  The partials need
// dec_part_floats(T, ...).
bool attn_rows_ok(const AttnArgs &a);
int launch_attention_rows(const AttnArgs &a, hipStream_t st);
// a.rope_cur from the tables at the position of sequence 0 (one block)
int launch_rope_cur(const AttnArgs &a, hipStream_t st);

// T == 1 (decode): one launch; the chunk blocks append the row to the cache and
// the last block of each (sequence, kv head) merges the chunks (needs a.ctr).
// T > 1: scores + chunk softmax + P.V partials, then the merge of the chunks
// with the cache append of the rows (two launches).
int launch_attention(const AttnArgs &a, hipStream_t st);
int attn_check(const AttnArgs &a);

// Prefill attention for one sequence (B = 1) and many rows: RoPE of the rows'
// q and k into qr [T][q_dim] / kr [T][kv_dim], a flash-attention pass on fp32
// MFMA (one block per 16 rows and kv head, one wave per query head), then the
// cache append of the rows.  Needs 4 query heads per kv head and head_dim
// 128, 256 or 512 (prefill_flash_ok); a.part is not used.
bool prefill_flash_ok(const AttnArgs &a);
// Row tiles attending to many keys split their key tiles over several blocks
// (so that the launch fills the CUs), merged by a second launch.  The split
// plan follows T, cache_len, n_kv and a.plan_pos; the splits' partials need
// flash_part_floats(a) floats of fpart (0: no split), never more than
// flash_part_floats_max(hd).  With a smaller or null fpart the launch does not
// split.
struct FlashSplit {
  int st_tiles;  // key tiles per split
  int maxs;      // blocks per row tile (1: no split)
  int n_rt;      // row tiles
  float *part;   // per block: o [16 rows][4 heads][hd], then (max, sum) [16][4][2]
};
size_t flash_part_floats(const AttnArgs &a);
size_t flash_part_floats_max(int hd);
int launch_attention_prefill(const AttnArgs &a, float *qr, float *kr, float *fpart,
                             size_t fpart_floats, hipStream_t st);

}  // namespace ms
