/*
 * ms_gpu.h -- C ABI of the MI355X (gfx950) implementation of MojoStream's
 * Gemma-4 per-token layer loop.
 *
 * Conventions
 *   - Every function returns MS_OK (0) or a negative MS_E* code; the message
 *     of the last failure on the calling thread is ms_last_error().  No C++
 *     exception crosses this boundary.  A caller that mirrors the reference's
 *     fail-fast loaders turns a nonzero code into `raise Error(ms_last_error())`.
 *   - Pointers named d_* are device pointers (ms_malloc); h_* are host
 *     pointers.  The caller owns host memory; the library owns what it
 *     allocates behind opaque handles.
 *   - Work is ordered on the library's stream and asynchronous, except
 *     functions that return host data (they synchronize).
 *   - One host thread per library instance (the reference's callers are
 *     single-threaded; its `workers` argument has no GPU meaning and is not
 *     part of this ABI).
 *   - Q4 weights: the reference layout is row-major [K][N/2] bytes, byte j of
 *     row k holding column 2j in its low nibble and 2j+1 in its high nibble,
 *     w = (nibble - 8) * scale with one fp32 scale per tensor
 *     (kernels.mojo:66-69).  On the device they live repacked in the
 *     "panel" layout produced by ms_q4_pack (same byte count, K%128==0,
 *     N%16==0 required).
 *
 * Reference citations are relative to the MojoStream repository.
 */
#ifndef MS_GPU_H
#define MS_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MS_OK 0
#define MS_E_INVALID (-1)   /* bad argument / shape violation */
#define MS_E_HIP (-2)       /* HIP runtime failure */
#define MS_E_STATE (-3)     /* library not initialised / wrong call order */
#define MS_E_NOMEM (-4)     /* allocation failed */
#define MS_E_IO (-5)        /* file / guard failure (host helpers) */

/* ---- context ------------------------------------------------------------ */
/* No reference counterpart (the reference runs on CPU threads); replaces the
 * implicit set-up before matmul_q4_bpack_raw's first `parallelize`
 * (kernels.mojo:266-267). */
int ms_init(int device);
int ms_shutdown(void);
const char *ms_last_error(void);
int ms_synchronize(void);
/* Device name / CU count / HBM bytes for reports. */
int ms_device_info(char *name, size_t name_len, int *n_cu, size_t *hbm_bytes);

/* ---- memory ------------------------------------------------------------- */
/* Device buffers replace the reference's List-backed Matrix storage
 * (kernels.mojo:34-61) and the weight buffers of Gemma4LayerWeights
 * (main.mojo:305-337). */
int ms_malloc(void **d_ptr, size_t bytes);
int ms_free(void *d_ptr);
int ms_memcpy_h2d(void *d_dst, const void *h_src, size_t bytes);
int ms_memcpy_d2h(void *h_dst, const void *d_src, size_t bytes);
int ms_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes);
int ms_memset(void *d_dst, int value, size_t bytes);
/* Pinned host memory (hipHostMalloc) for the streaming double buffer; replaces
 * the scratch List of StreamingRunner (stream_runner.mojo:388-409). */
int ms_host_alloc(void **h_ptr, size_t bytes);
int ms_host_free(void *h_ptr);

/* ---- seeded synthetic data ---------------------------------------------- */
/* Counter-based generator (splitmix64 of seed, stream, index).  Host and
 * device produce identical bytes.  Replaces the unseeded `rand` fills of
 * Q4Matrix.fill_random / init_random_layer_weights (kernels.mojo:91-92,
 * main.mojo:616-633) and create_fake_model.py's rng.integers(0,256)
 * (create_fake_model.py:94-97). */
int ms_fill_random_u8(uint8_t *d_dst, size_t n, uint64_t seed, uint64_t stream);
void ms_host_fill_random_u8(uint8_t *h_dst, size_t n, uint64_t seed,
                            uint64_t stream);
/* The same bytes, or with balanced != 0 every zero nibble replaced by 8.  No
 * reference counterpart.  Uniform nibbles (the reference's synthetic weights)
 * have mean 7.5 against the zero point 8, so every weight has mean -scale/2;
 * through the layers this common component drives every hidden state to one
 * direction, and the model's greedy output no longer depends on its input.
 * Balanced nibbles (1..15, mean 8) give zero-mean weights and a model whose
 * output does; parity checks use them where token ids must discriminate. */
int ms_fill_random_q4(uint8_t *d_dst, size_t n, uint64_t seed, uint64_t stream,
                      int balanced);
void ms_host_fill_random_q4(uint8_t *h_dst, size_t n, uint64_t seed, uint64_t stream,
                            int balanced);
/* Uniform [lo,hi) float for (seed, stream, index) (scales: U(0.04,0.15),
 * PLE: U(0.8,1.2), create_fake_model.py:95,203). */
float ms_host_uniform(uint64_t seed, uint64_t stream, uint64_t index, float lo,
                      float hi);
/* Standard normal fp32 values (Box-Muller) for activation inputs. */
void ms_host_fill_normal(float *h_dst, size_t n, uint64_t seed, uint64_t stream);

/* ---- Q4 kernels (kernel-level parity entry points) ---------------------- */
/* Bytes of the panel layout (== K*N/2). */
size_t ms_q4_packed_bytes(int K, int N);
/* Repack reference row-major Q4 into the panel layout (device->device).
 * Replaces the byte copy of load_weights_from_ms (harness.mojo:80-122). */
int ms_q4_pack(uint8_t *d_packed, const uint8_t *d_rowmajor, int K, int N);
/* Same repack on the host (streaming mode packs once into pinned memory). */
int ms_host_q4_pack(uint8_t *h_packed, const uint8_t *h_rowmajor, int K, int N);
/* Dequantize to fp32 [K][N]: dequant_vec, kernels.mojo:100-108 (row-major
 * input), and the same from the panel layout (bit-exact check of packing). */
int ms_dequant_q4(float *d_out, const uint8_t *d_rowmajor, int K, int N,
                  float scale);
int ms_dequant_q4_packed(float *d_out, const uint8_t *d_packed, int K, int N,
                         float scale);
/* C (+)= A . deq(W): matmul_q4_bpack_raw, kernels.mojo:201-267 (and
 * matmul_q4_bpack :122-193 on a Q4Matrix).  A fp32 [M][K], W panel layout,
 * C fp32 [M][N].  accumulate=1 keeps the reference's C += semantics,
 * accumulate=0 overwrites.  Each row is quantized to fixed point and the dot
 * products are exact integers: up to four rows with K = 1024, 2048 or 4096 (or
 * 2560 without accumulate) in one launch, 31 bits with a shift per row and
 * slice of 128 to 640 values of K; other calls of up to 16 rows quantize the
 * rows (31 bits, a shift per row), then one GEMV; more rows are quantized to
 * 22 bits (three int8 limbs) for the MFMA GEMM.  Every path is within 1e-5 of
 * the f64 product; K <= 16384. */
int ms_q4_matmul(float *d_C, const float *d_A, const uint8_t *d_packed, int M,
                 int K, int N, float scale, int accumulate);
/* ms_q4_matmul without any allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (serving loops, harnesses
 * that forbid hipMalloc).  Its kernels run on the library's own stream, so a
 * graph the caller captures on another stream does not record them.  The quantized
 * rows live in a 4 MiB static device array of the library (one per GPU,
 * held until the process ends, its address taken at ms_init); a call whose
 * rows need more (M <= 16: K <= 16384 always fits; M > 16: about
 * 4 * round_up(M, 32) * K bytes) fails with MS_E_INVALID.  Same kernels and
 * same results as ms_q4_matmul.  Every call on a GPU shares that array, so
 * calls that overlap on one GPU (from several host threads) race; calls on
 * the library's stream are ordered and do not. */
int ms_q4_matmul_noalloc(float *d_C, const float *d_A, const uint8_t *d_packed, int M,
                         int K, int N, float scale, int accumulate);

/* Device time of ms_q4_matmul (overwriting C): `reps` calls back to back
 * between two HIP events on the library stream, call r reading the weights at
 * d_w0 + (r % n_w) * w_stride (panel layout), so that weights rotated over
 * more memory than the caches hold come from HBM.  *avg_us: microseconds per
 * call.  Measurement support for run_q4_benchmark (benchmark_q4.mojo:121-147),
 * whose CPU timing has no device counterpart. */
int ms_bench_q4_matmul(float *d_C, const float *d_A, const uint8_t *d_w0, size_t w_stride,
                       int n_w, int M, int K, int N, float scale, int reps, double *avg_us);

/* ---- elementwise kernels ------------------------------------------------ */
/* rmsnorm_inplace, kernels.mojo:474-489 */
int ms_rmsnorm(float *d_x, int rows, int cols);
/* rmsnorm_weighted_inplace, kernels.mojo:598-613 (d_gamma may be NULL = 1) */
int ms_rmsnorm_weighted(float *d_x, const float *d_gamma, int rows, int cols);
/* ple_scale_inplace, kernels.mojo:506-516 */
int ms_ple_scale(float *d_x, size_t n, float s);
/* swiglu_inplace, kernels.mojo:519-532 (result in d_up) */
int ms_swiglu(const float *d_gate, float *d_up, size_t n);
/* apply_rope_inplace, kernels.mojo:553-595: `rows` rows of stride row_stride,
 * row r at position base_pos + r; n_heads heads of stride head_stride; the
 * first rot_dim dims of each head rotate (partial use gemma4_e4b.mojo:489-500).
 * cos/sin use the reference's fp32 formula, evaluated on the host. */
int ms_rope(float *d_x, int rows, int row_stride, int n_heads, int head_stride,
            int rot_dim, float theta, int base_pos);

/* ---- attention (kernel level) ------------------------------------------- */
#define MS_CACHE_LINEAR 0   /* KVCache (main.mojo:257-301), full cache (gemma4_e4b.mojo:231-249) */
#define MS_CACHE_CIRCULAR 1 /* sliding cache, slot = pos % window (gemma4_e4b.mojo:211-228) */

typedef struct {
  int q_dim, kv_dim, head_dim, n_heads, n_kv_heads;
  int rot_dim;     /* rotated dims per head */
  float theta;     /* RoPE base */
  int cache_kind;  /* MS_CACHE_* */
  int cache_len;   /* linear: positions; circular: window */
  int clamp_reads; /* linear: attend min(pos+1, cache_len) keys (gemma4_e4b.mojo:362-363) */
} ms_layer_desc;

/* Causal GQA attention of T rows of one sequence at positions
 * base..base+T-1 (compute_sliding_attention gemma4_e4b.mojo:259-338,
 * compute_full_attention :341-411, gqa_attention_decode main.mojo:445-519),
 * followed by the cache write of the T rows (write_kv_*: :211-249).  q/k/v
 * are final (after RoPE for q and k).  Keys of the T rows come from
 * d_knew/d_vnew, older keys from the cache. */
int ms_attention(const ms_layer_desc *desc, const float *d_q,
                 const float *d_knew, const float *d_vnew, float *d_kcache,
                 float *d_vcache, int T, int base, float *d_out);

/* ---- LM head (kernel level) --------------------------------------------- */
/* logits = x . deq(W_lm) (project_lm_head, lm_head.mojo:146-168) and the
 * greedy id per row (temperature_sampling T<=0.01 branch, :224-230: first
 * index of the strict maximum).  d_logits may be NULL. */
int ms_lm_head_argmax(const float *d_x, int M, int D, const uint8_t *d_packed,
                      int vocab, float scale, float *d_logits, int32_t *d_ids);
/* temperature_sampling (lm_head.mojo:198-254) on a logits row in device
 * memory, with `seed` where the reference reads the clock (:246): the
 * repetition penalty over the n_generated ids of d_generated (prompt and
 * generated tokens, as gemma4_e4b_infer.mojo:157-182 passes them; at most
 * 8192), greedy below temperature 0.01, else softmax at `temperature` and one
 * LCG draw.  Like the reference it leaves the penalized logits (greedy) or the
 * probabilities in d_logits.  The id goes to *h_id. */
int ms_sample(float *d_logits, int vocab, float temperature, const int32_t *d_generated,
              int n_generated, float penalty, uint64_t seed, int32_t *h_id);
/* The seed ms_prefill / ms_decode_run give the LCG step (lm_head.mojo:246-248)
 * of draw `draw` of sequence `seq` under ms_model_set_sampling(.., seed): a
 * splitmix64 hash of the three, so that sequences and consecutive draws get
 * independent targets.  No reference counterpart (the reference reads the
 * clock); lets a caller reproduce the model's draws with ms_sample. */
uint64_t ms_sample_seed(uint64_t seed, int seq, uint64_t draw);
/* matmul_fp32_raw (kernels.mojo:616-671): C (+)= A . B with B fp32 row-major
 * [K][N], A [M][K], M <= 16; N a multiple of 16 (the reference computes whole
 * 16-column tiles only, :640).  accumulate = 1 keeps the reference's C +=. */
int ms_matmul_f32(float *d_c, const float *d_a, const float *d_b, int M, int K, int N,
                  int accumulate);
/* quantize_q4_blockwise (scripts/convert.py:296-323) of a HuggingFace weight
 * d_w [n_out][n_in] (dtype 0 fp32, 1 bf16, 2 fp16), transposed as the converter
 * does (convert.py:503-518): d_packed receives the (n_in, n_out) Q4 bytes
 * [n_in][n_out/2], even columns in the low nibble; *h_scale the global scale
 * (the largest block scale over blocks of block_size).  n_out must be even; a
 * weight holding NaN or infinity is refused. */
int ms_q4_quantize(uint8_t *d_packed, float *h_scale, const void *d_w, int dtype, int n_out,
                   int n_in, int block_size);

/* ---- tokenizers (host only, no device use) ----------------------------------
 * Strings are byte strings: the reference builds its text from chr(byte), so
 * each byte is one code point 0..255.  Text outputs take (out, cap) and set *len
 * to the size; when cap is too small the call fails with *len the size needed. */
typedef struct ms_tokenizer ms_tokenizer;
typedef struct ms_token_map ms_token_map;
/* BPETokenizer.load (src/nlp/tokenizer.mojo:56-101): an .msvocab file. */
int ms_tokenizer_load(const char *path, ms_tokenizer **out);
int ms_tokenizer_free(ms_tokenizer *t);
/* BPETokenizer.n_tokens (:165-166): the largest id + 1. */
int ms_tokenizer_vocab_size(const ms_tokenizer *t, int *n);
/* BPETokenizer.encode (:103-150): bytes, then lowest-rank leftmost merges;
 * unknown strings give id 0.  ids = NULL asks only for the count *n. */
int ms_tokenizer_encode(const ms_tokenizer *t, const char *text, int len, int32_t *ids,
                        int cap, int *n);
/* BPETokenizer.decode (:152-163): BOS 1, EOS 2 and PAD 3 skipped. */
int ms_tokenizer_decode(const ms_tokenizer *t, const int32_t *ids, int n, char *out, int cap,
                        int *len);
/* BPETokenizer.token_str (:168-172): "<unk>" out of range. */
int ms_tokenizer_token_str(const ms_tokenizer *t, int id, char *out, int cap, int *len);
/* load_token_map (src/tokenizer/gemma_proto.mojo:59-74): vocab_proto.bin. */
int ms_token_map_load(const char *path, ms_token_map **out);
int ms_token_map_free(ms_token_map *m);
int ms_token_map_size(const ms_token_map *m, int *n);
/* TokenMap.decode (gemma_proto.mojo:27-37): "[?:id]" out of range. */
int ms_token_map_decode(const ms_token_map *m, int id, char *out, int cap, int *len);
/* get_token_embedding Q4 branch (lm_head.mojo:186-195): column `token` of the
 * tied head, dequantized, for each of n tokens -> d_out [n][D]. */
int ms_embed_q4(const uint8_t *d_packed, int D, int vocab, float scale,
                const int32_t *d_tokens, int n, float *d_out);

/* ---- model (layer loop) --------------------------------------------------- */
typedef struct ms_model ms_model;

typedef struct {
  int hidden;      /* D */
  int ffn;         /* F */
  int n_layers;
  int vocab;       /* 0: no LM head (demo model) */
  int max_seqs;    /* independent sequences, each with its own caches */
  int max_rows;    /* rows per sequence per call (T) */
  int max_pos;     /* highest position + 1 the RoPE tables cover */
  int resident;    /* 1: weights resident in HBM; 0: streamed per layer from
                      pinned host memory through two HBM slots */
} ms_model_desc;

/* Creates a model with per-layer shapes (ModelRunner / Gemma4Config /
 * E4BLayerRef shapes: main.mojo:230-253, gemma4_e4b.mojo:125-174) and
 * allocates KV caches (KVCache main.mojo:257-301, HybridKVCache
 * gemma4_e4b.mojo:83-116). */
int ms_model_create(const ms_model_desc *desc, const ms_layer_desc *layers,
                    ms_model **out);
int ms_model_destroy(ms_model *m);
/* Binds one of the 7 matrices (0 Q,1 K,2 V,3 O,4 Gate,5 Up,6 Down -- the
 * .mojostream type tag minus one, mojostream.mojo:21-28) of a layer.
 * `src` is row-major reference Q4, on the device if src_on_device else host.
 * Resident models pack it into HBM; streaming models keep a packed copy in
 * pinned host memory (packed on the device when src is there).
 * Replaces load_weights_from_ms (harness.mojo:80-122) and
 * get_layer_ref (sparse_pin.mojo:295-330). */
int ms_model_set_matrix(ms_model *m, int layer, int mat, const uint8_t *src,
                        int src_on_device, float scale);
int ms_model_set_ple(ms_model *m, int layer, float ple);
/* Streaming models only: pinned[l] != 0 keeps layer l's weights in HBM; the
 * two-slot double buffer then streams only the other layers, alternating
 * slots among them (SparsePinEngine: pinned layers via get_layer_ref, the
 * skipping prefetcher advance/next_non_pinned, sparse_pin.mojo:88-92,268-330).
 * Call before binding the weights of any layer whose flag changes. */
int ms_model_set_pinned(ms_model *m, const uint8_t *pinned);
/* Tied Q4 LM head (LMHead v1, lm_head.mojo:41-116); h_gamma NULL = ones. */
int ms_model_set_lm_head(ms_model *m, const uint8_t *src, int src_on_device,
                         float scale, const float *h_gamma);
/* KVCache.reset (main.mojo:295-297): positions restart at 0. */
int ms_model_reset(ms_model *m);

/* One layer over rows d_x [n_seqs*T][D] in place, sequence s at positions
 * h_base[s]..h_base[s]+T-1 (e4b_forward_layer gemma4_e4b.mojo:459-540,
 * gemma4_forward_layer main.mojo:538-613, gemma4_forward_stream
 * stream_runner.mojo:101-161). */
int ms_layer_forward(ms_model *m, int layer, float *d_x, int n_seqs, int T,
                     const int *h_base);
/* All layers in order (the per-step loops of demo_first_light main.mojo:685-695,
 * run_harness harness.mojo:256-269).  d_hidden (optional) receives every
 * layer's output [n_layers][n_seqs*T][D]. */
int ms_forward(ms_model *m, float *d_x, int n_seqs, int T, const int *h_base,
               float *d_hidden);

/* Greedy decode with the tied head (gemma4_e4b_infer.mojo:163-186 with T=0):
 * ms_decode_begin sets, per sequence, the current token and its position;
 * ms_decode_run performs n_steps steps (embedding -> layers -> final norm ->
 * logits -> argmax -> next token) on the device and returns the generated ids
 * [n_steps][n_seqs].  use_graph=1 replays one captured HIP graph per step. */
int ms_decode_begin(ms_model *m, int n_seqs, const int32_t *h_tokens,
                    const int32_t *h_pos);
int ms_decode_run(ms_model *m, int n_steps, int use_graph, int32_t *h_ids_out);
/* Prompt processing for one sequence (the prompt loop of
 * gemma4_e4b_infer.mojo:114-130 done in row chunks): runs the prompt tokens at
 * positions h_pos0.. and returns the first greedy id (TTFT path). */
int ms_prefill(ms_model *m, int seq, const int32_t *h_tokens, int n_tokens,
               int pos0, int32_t *h_first_id);

/* Shapes the model was created with; `layers` (n_layers entries) may be NULL.
 * No reference counterpart (the reference reads its constants directly). */
int ms_model_get_desc(const ms_model *m, ms_model_desc *desc, ms_layer_desc *layers);
/* Sampling for ms_prefill and ms_decode_run: temperature_sampling
 * (lm_head.mojo:198-254) as gemma4_e4b_infer.mojo:134-182 calls it, in place
 * of the greedy argmax, when temperature > 0.01 or penalty > 1 (else greedy
 * again).  Each sequence's penalty history holds its prompt ids (from
 * ms_prefill) and then every sampled id, at most 8192 ids (ms_prefill and
 * ms_decode_run return MS_E_INVALID rather than drop any); ms_model_reset
 * empties it.  The k-th LM head call that draws (counted from this call or
 * ms_model_reset: the prefill's first token, then every decode step) draws
 * for sequence b with ms_sample_seed(seed, b, k), where the reference reads
 * the clock.  Needs an LM head. */
int ms_model_set_sampling(ms_model *m, float temperature, float penalty, uint64_t seed);
/* BOS embedding row (LMHead.bos_emb, lm_head.mojo:41-58).  When set, the row
 * at position 0 of ms_prefill takes it instead of the embedding of its token
 * (apply_bos_embedding, lm_head.mojo:133-143, used for prompt position 0 by
 * gemma4_e4b_infer.mojo:94,116-117).  h_bos NULL clears it. */
int ms_model_set_bos(ms_model *m, const float *h_bos);

/* Taps for parity checks (the per-layer comparison of validate_layer.mojo
 * :138-154 needs each layer's output; the reference's loops hold them in host
 * memory).  With d_hidden set, every decode step of ms_decode_run writes each
 * layer's output rows to d_hidden [n_layers][n_seqs][hidden], and ms_prefill
 * writes each layer's output for the prompt's last row to d_hidden
 * [n_layers][hidden].  With d_logits set, every LM head call writes its raw
 * logits (before any sampling) to d_logits [rows][vocab] (decode: one row per
 * sequence; prefill: the last prompt row).  Each call overwrites the taps.
 * NULL switches a tap off. */
int ms_model_set_taps(ms_model *m, float *d_hidden, float *d_logits);
/* Launch mode of ms_forward (no reference counterpart; results are the same
 * either way).  on = 1 (the default): a whole-model call of a resident model
 * with at most 16 rows that repeats the previous call's buffers, rows and
 * position bucket is captured as a HIP graph and replayed from then on (the
 * harness loop, harness.mojo:256-269); on = 0: every call launches eagerly. */
int ms_model_set_forward_graphs(ms_model *m, int on);
/* Rows of positions pos0..pos0+n-1 of a layer's KV cache for one sequence
 * (K after RoPE, V), into d_k / d_v [n][kv_dim] (either may be NULL).  A
 * circular cache holds position p in slot p % window (write_kv_sliding
 * gemma4_e4b.mojo:211-228), so n is at most the window and only the last
 * window positions are meaningful.  No reference counterpart (the reference's
 * caches are host Lists its tests read directly). */
int ms_model_read_kv(ms_model *m, int layer, int seq, int pos0, int n, float *d_k, float *d_v);

/* ---- .mojostream weight files (host side) -------------------------------- */
/* MojoStreamMeta (mojostream.mojo:47-69) plus the fields the reference parses
 * but does not keep, and the Engram extension of format tag 2
 * (convert.py:383-398; zeros when absent). */
typedef struct {
  uint32_t version, format_tag, n_layers, hidden, kv_dim, ffn_dim, n_heads,
      n_kv_heads;
  uint64_t n_tensors, dir_offset, data_start;
  uint32_t engram_version, n_kv_shared, sliding_kv_dim, full_kv_dim, ple_dim,
      sliding_window;
  uint64_t file_bytes;
  double load_ms; /* time of the whole-file read */
} ms_file_meta;
/* TensorEntry (mojostream.mojo:73-91) with the flags word. */
typedef struct {
  uint32_t layer_id, mat_type, rows, cols;
  float scale;
  uint32_t flags;
  uint64_t data_offset;
} ms_file_entry;
/* Head size and projection widths of one layer (get_layer_dims,
 * convert.py:195-225). */
typedef struct {
  int is_full, head_dim, q_dim, kv_dim;
} ms_file_layer;
typedef struct ms_file ms_file;

/* MojoStreamFile(path) (mojostream.mojo:101-113): one whole-file read, header
 * and directory parse.  Fails on a missing file, a bad magic (first four
 * bytes "MOJO") or a header/directory that extends past the end. */
int ms_file_open(const char *path, ms_file **out);
int ms_file_close(ms_file *f);
int ms_file_get_meta(const ms_file *f, ms_file_meta *out);
int ms_file_get_entry(const ms_file *f, int index, ms_file_entry *out);
/* Layer-type map used by the guards and loaders: is_full[n_layers] (NULL
 * restores the default: full attention at (layer+1) % 6 == 0 for a hybrid
 * file, is_full_attn gemma4_e4b.mojo:60-63; none otherwise). */
int ms_file_set_layer_types(ms_file *f, const uint8_t *is_full, int n_layers);
int ms_file_layer_info(const ms_file *f, int layer, ms_file_layer *out);
/* tensor_ptr (mojostream.mojo:156-175): host pointer into the file buffer,
 * the tensor's scale and its byte count (0 for PLE entries).  An absent
 * tensor is MS_E_IO (the reference returns the buffer start, scale 0). */
int ms_file_tensor(const ms_file *f, int layer, int mat_type,
                   const uint8_t **h_ptr, float *scale, size_t *bytes);
/* ple_scale (mojostream.mojo:177-182): 1.0 when there is no entry. */
int ms_file_ple_scale(const ms_file *f, int layer, float *out);
/* ShapeGuard (validate_gemma4_shape mojostream.mojo:190-219,
 * _check_shape stream_runner.mojo:280-309), layer-type-aware. */
int ms_file_shape_guard(const ms_file *f);
/* TensorGuard (validate_tensor_entries stream_runner.mojo:313-380): entry
 * order, per-layer shapes, 4096 alignment, file bounds, scale > 0. */
int ms_file_tensor_guard(const ms_file *f);
/* Seeded synthetic .mojostream file (create_fake_model.py:188-281).  Uses
 * n_layers, hidden, kv_dim, ffn_dim, n_heads, n_kv_heads, and the Engram
 * fields when engram_version != 0; is_full may be NULL (default map).  The
 * weights equal those the Python synthetic-model helpers put on the device
 * for the same seed. */
int ms_file_write_synthetic(const char *path, const ms_file_meta *hdr,
                            const uint8_t *is_full, uint64_t seed);
/* compute_dir_checksum (src/tests/validate_real.mojo:78-83): XOR of the
 * 32-bit words at byte 16 of every directory entry (the scale fields). */
int ms_file_dir_checksum(const ms_file *f, uint32_t *out);
/* Structural validation of a converted file, run_validation
 * (src/tests/validate_real.mojo:110-260): magic, architecture fields, Engram
 * extension, n_tensors == n_layers * 8, directory offsets inside the file,
 * non-zero directory checksum, and spot checks of the Q and Gate tensors of
 * layers 0, 20 and 41 (first 64 bytes not all 0x00 nor all 0xFF).  Like the
 * reference it reports rather than fails: MS_OK with the counts, a bit per
 * failed check and the first failure's text. */
#define MS_VALIDATE_MAGIC 0
#define MS_VALIDATE_ARCH 1
#define MS_VALIDATE_ENGRAM 2
#define MS_VALIDATE_TENSORS 3
#define MS_VALIDATE_OFFSETS 4
#define MS_VALIDATE_CHECKSUM 5
#define MS_VALIDATE_SPOT 6 /* bits 6..11: layer 0 Q, Gate; layer 20 Q, Gate; 41 Q, Gate */
typedef struct {
  int passed, n_checks, n_failed;
  uint32_t failed_mask;
  uint32_t dir_checksum;
  uint64_t file_bytes;
  char message[256];
} ms_file_validation;
int ms_file_validate(const ms_file *f, ms_file_validation *out);
/* Runs both guards, checks the model's shapes against the file and binds
 * every matrix and PLE scale (the load loops of run_harness
 * harness.mojo:80-122 and StreamingRunner stream_runner.mojo:188-270). */
int ms_model_load_file(ms_model *m, const ms_file *f);
/* FP32 LM head (LMHead version 2, lm_head.mojo:61-116, projected with
 * matmul_fp32_raw :146-160, embedded by column :179-185): src [hidden][vocab]
 * fp32 row-major, h_gamma the final-norm weights (NULL = ones).  Replaces the
 * Q4 head; vocab must be a multiple of 16. */
int ms_model_set_lm_head_f32(ms_model *m, const float *src, int src_on_device,
                             const float *h_gamma);
/* Seeded synthetic version-2 head file: [vocab][scale 1.0][version 2][BOS]
 * [gamma][weights] (the layout load_lm_head reads, lm_head.mojo:67-104). */
int ms_lm_head_file_write_synthetic_v2(const char *path, int hidden, int vocab, uint64_t seed);
/* LM head file (load_lm_head lm_head.mojo:61-116), version 1 (tied Q4) or,
 * when the file is large enough, version 2 (FP32 + final-norm gamma): sets
 * the head, its final-norm gamma (ones for version 1) and the BOS row. */
int ms_model_load_lm_head_file(ms_model *m, const char *path);
int ms_lm_head_file_write_synthetic(const char *path, int hidden, int vocab,
                                    uint64_t seed);

/* ---- streaming statistics ------------------------------------------------ */
typedef struct {
  double io_ms;        /* host->HBM copy time of the last ms_forward / ms_prefill /
                          ms_decode_run call (summed over its layer passes) */
  double compute_ms;   /* wall time minus wait */
  double wait_ms;      /* time compute waited for a copy (measured with events) */
  double total_ms;
  double bytes;        /* bytes copied host->HBM */
  int layers_streamed; /* layer passes whose weights came through an HBM slot */
  int layers_pinned;   /* layer passes of pinned (resident) layers: the hits of
                          SparsePinEngine's pass statistics, sparse_pin.mojo:136-330 */
} ms_stream_stats;
/* I/O vs compute of the last call (run_streaming_bench stream_runner.mojo:503-546
 * reports the same split analytically).  Zero for a resident model. */
int ms_model_stream_stats(ms_model *m, ms_stream_stats *out);

/* ---- ModelRunner: double-buffered layer files ----------------------------- */
/* ModelRunner (loader.mojo:47-144).  n_layers square N x N Q4 matrices, one
 * per file <base_path>/layer_<i>.bin ([f32 scale][N * N/2 row-major bytes],
 * the "row-major" layer files of create_fake_model.py:126-140), two HBM slots.
 * N % 128 == 0. */
typedef struct ms_runner ms_runner;
typedef struct {
  double load_ms;     /* LayerStats.load_ns: loading the next layer (host file read
                         and repack + host->HBM copy); 0 for the last layer */
  double compute_ms;  /* LayerStats.compute_ns: C += A . deq(W) of this layer */
  double wait_ms;     /* LayerStats.wait_ns: measured idle time of the compute
                         stream before the next layer (the reference models it as
                         max(0, load_next - compute)) */
} ms_layer_stats;
/* ModelRunner.__init__ (loader.mojo:59-76): two slots of N * N/2 bytes. */
int ms_runner_create(const char *base_path, int n_layers, int N, ms_runner **out);
int ms_runner_destroy(ms_runner *r);
/* load_into_slot (loader.mojo:82-94): layer idx into slot 0 or 1, synchronous;
 * *load_ms the wall time.  A missing or short file is MS_E_IO (the reference
 * raises). */
int ms_runner_load_into_slot(ms_runner *r, int slot, int idx, double *load_ms);
/* ModelRunner.active (loader.mojo:52): the slot compute_active reads. */
int ms_runner_set_active(ms_runner *r, int slot);
int ms_runner_active(const ms_runner *r, int *slot);
/* compute_active (loader.mojo:97-106): C [M][N] += A [M][N] . deq(W_active);
 * *compute_ms the device time (events on the library stream). */
int ms_runner_compute_active(ms_runner *r, float *d_C, const float *d_A, int M,
                             double *compute_ms);
/* run_pipeline (loader.mojo:115-144): layer 0 loaded cold into slot 0; then
 * per layer i: C += A . deq(W_i) on the active slot, C zeroed, the slots
 * flipped, while layer i+1 loads into the other slot on the copy stream (a
 * real overlap; the reference times the two in sequence).  stats[n_layers].
 * d_taps (or null): [n_layers][M][N], C of each layer before the zeroing. */
int ms_runner_run_pipeline(ms_runner *r, float *d_C, const float *d_A, int M,
                           ms_layer_stats *stats, float *d_taps);

/* ---- profiling ------------------------------------------------------------ */
/* When enabled, ms_decode_run (eager mode) records HIP events around every
 * launch of each kernel class on the library stream; ms_prof_get returns
 * launch counts and total milliseconds per class. */
#define MS_PROF_CLASSES 8
int ms_prof_enable(int on);
int ms_prof_get(int cls, const char **name, long *launches, double *total_ms,
                double *bytes);
/* Class 1 (attention): the last decode attention launch recorded while
 * profiling (of a circular cache if any, else a linear one) re-launched over
 * every layer of that kind, each on its own cache; bytes are the K/V rows
 * attended at the current position plus the appended row.
 * Kernel duration of one projection class (0 QKV, 2 O, 3 Gate|Up, 4 Down)
 * measured on the device: the last launch of that class recorded while
 * profiling was enabled is re-launched back to back `passes` times over every
 * layer with the same shapes, each launch on that layer's weights (so weights
 * come from HBM as in a decode step), between two HIP events on the library
 * stream.  passes < 0 re-launches it -passes times on its own layer's weights
 * (cache-hot after the first launch).  Outputs average microseconds and bytes of Q4 weights per launch.
 * The re-launches overwrite only per-step scratch rows (recomputed by the next
 * decode step); KV caches and positions are untouched.  No reference
 * counterpart: measurement support. */
int ms_prof_sweep(ms_model *m, int cls, int passes, double *avg_us, double *bytes_per_launch,
                  long *launches);

#ifdef __cplusplus
}
#endif
#endif
