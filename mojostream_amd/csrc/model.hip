// The Gemma-4 per-token layer loop on one MI355X.
//
// Per layer (e4b_forward_layer gemma4_e4b.mojo:459-540; gemma4_forward_layer
// main.mojo:538-613) six launches on one stream, each consumer reading one
// fp32 row array (no split-K partials between kernels):
//   1. QKV GEMV   prologue: xn = rmsnorm(ple * x) in LDS (block 0 stores xn);
//                 Q, K, V fused (3 segments, 3 scales) -> qkv rows
//   2. attention  chunk partials (RoPE, causal GQA over the cache), then one
//                 merge block per query head: O input (fp16 hi/lo), K/V append
//   3. O GEMV     A staged in LDS; epilogue x2 = xn + attn.Wo
//   4. GateUp     prologue: x2n = rmsnorm(x2) (block 0 stores x2n); gate and
//                 up panels of the same columns in one block; epilogue
//                 up*gate*sigmoid(gate) -> Down input (fp16 hi/lo)
//   5. Down GEMV  A staged in LDS; epilogue x_out = x2n + ffn.Wd
// The residual adds to the normalized stream, as in the reference
// (gemma4_e4b.mojo:520-538, gen_reference.py:160-172).
//
// Decode (T=1 per sequence) keeps token ids and positions on the device, so
// one captured HIP graph runs every step unchanged.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <vector>

#include "attention.h"
#include "q4.h"
#include "rope.h"
#include "head_f32.h"
#include "sample.h"

namespace ms {

struct RopeTab {
  int rot = 0;
  float theta = 0.f;
  float *cs = nullptr, *sn = nullptr;
};

struct Layer {
  ms_layer_desc d{};
  uint8_t *w[7] = {};        // device panel-layout weights (resident) or slot pointers
  uint8_t *h_packed[7] = {}; // pinned packed copies (streaming)
  size_t bytes[7] = {};
  size_t off[7] = {};        // offsets inside a streaming slot
  float scale[7] = {};
  int set_mask = 0;
  float ple = 1.f;
  float *kc = nullptr, *vc = nullptr;
  size_t cache_seq_stride = 0;
  int rope = 0;
  int n_chunks = 1;
  int pinned = 0;  // streaming models: weights kept in HBM, never copied per call
};

// profiling classes
enum { PC_QKV, PC_ATTN, PC_O, PC_GATEUP, PC_DOWN, PC_LM, PC_PREP, PC_OTHER };
static const char *kProfNames[MS_PROF_CLASSES] = {"qkv_gemv", "attention", "o_gemv",
                                                  "gateup_gemv", "down_gemv", "lm_head",
                                                  "embed_prep", "other"};
struct Prof {
  bool on = false;
  long launches[MS_PROF_CLASSES] = {};
  double ms[MS_PROF_CLASSES] = {};
  double bytes[MS_PROF_CLASSES] = {};
  std::vector<hipEvent_t> pool;
  struct Rec {
    int cls;
    hipEvent_t a, b;
    double bytes;
  };
  std::vector<Rec> pending;
  size_t used = 0;
  int cur = -1;                                 // class of the open ProfScope
  GemvArgs last[MS_PROF_CLASSES] = {};          // last GEMV launch per class
  int last_layer[MS_PROF_CLASSES] = {};
  bool have[MS_PROF_CLASSES] = {};
  // last decode attention launch per cache kind (0 linear, 1 circular)
  AttnArgs last_attn[2] = {};
  int last_attn_layer[2] = {};
  bool have_attn[2] = {};
  bool attn_part[2] = {};  // that launch left its chunks to the O projection
  int layer = -1;
};
static Prof g_prof;

}  // namespace ms

struct ms_model {
  ms_model_desc d{};
  std::vector<ms::Layer> L;
  std::vector<ms::RopeTab> ropes;
  int qkv_max = 0, q_max = 0, kv_max = 0, hd_max = 0, nkv_max = 0;
  int Mmax = 0;
  // LM head
  uint8_t *lm_w = nullptr;
  // FP32 head (LMHead version 2, lm_head.mojo:61-116): used instead of lm_w
  float *lm_f32 = nullptr;   // [D][vocab]
  float *lm_y = nullptr;     // [max_seqs][D] final-normed rows
  float *lm_part = nullptr;  // projection partial sums
  float lm_scale = 0.f;
  float *gamma = nullptr;
  bool has_lm = false;
  float *bos = nullptr;      // BOS embedding row for prompt position 0, or null
  float *bos_buf = nullptr;  // device storage of that row
  // workspaces
  // rows between kernels: x_in (embeddings), xs (layer output), xn and x2n
  // (normalised attention / FFN inputs, the residual bases), x2 (after O)
  float *x_in = nullptr, *xs = nullptr, *xn = nullptr, *x2 = nullptr, *x2n = nullptr;
  // O-projection input (attention output) and Down input (SwiGLU output)
  float *aO = nullptr, *aF = nullptr;
  // quantized activation rows for projections whose rows do not fit in LDS
  void *quant = nullptr;
  int quant_k = 0;
  float *qkv = nullptr, *attn_part = nullptr;
  float *rope_cur = nullptr;  // one-row decode: RoPE factors at the position [2][256]
  unsigned *attn_ctr = nullptr;  // decode attention counters (attn_ctr_count), kept zero
  // prefill: rows per chunk (0: no prefill workspace), attention rows per
  // launch inside a chunk and their base positions on the device
  int prefill_rows = 0;
  int32_t *ppos = nullptr;
  float *fq = nullptr, *fk = nullptr;  // prefill rows' q and k after RoPE
  float *fpart = nullptr;              // flash attention's key-split partials
  size_t fpart_floats = 0;
  int32_t *pos = nullptr, *tok = nullptr, *ids_hist = nullptr, *step = nullptr;
  int hist_cap = 1024;
  float *arg_val = nullptr;
  int32_t *arg_idx = nullptr;
  int lm_blocks = 0;
  // host mirror of positions
  std::vector<int> h_pos;
  int dec_nseq = 0;
  // graph
  // captured decode steps, one per position bound (see decode_bound)
  std::vector<std::pair<int, hipGraphExec_t>> graphs;
  int g_nseq = 0;
  // ms_forward replays: a call identical to the previous one (same buffers,
  // rows and position bucket) is captured, and replayed from then on
  struct FwdKey {
    const float *x = nullptr, *hidden = nullptr;
    int B = 0, T = 0, bound = 0;
    bool operator==(const FwdKey &o) const {
      return x == o.x && hidden == o.hidden && B == o.B && T == o.T && bound == o.bound;
    }
  };
  std::vector<std::pair<FwdKey, hipGraphExec_t>> fgraphs;
  FwdKey fwd_last{};
  bool forward_graphs = true;
  int32_t *h_pos_pin = nullptr;  // pinned staging of a call's positions
  // sampling (ms_model_set_sampling): temperature_sampling in place of the
  // greedy argmax, over a per-sequence history of prompt and generated ids
  bool sampling = false;
  float samp_temp = 0.f, samp_pen = 1.f;
  uint64_t samp_seed = 0;
  float *logits = nullptr;      // [max_seqs][vocab]
  int32_t *shist = nullptr;     // [max_seqs][kSampleMaxHistory]
  int32_t *shist_n = nullptr;   // [max_seqs]
  int32_t *samp_ids = nullptr;  // [max_seqs]
  int32_t *samp_ctr = nullptr;  // LM head calls that drew since set_sampling / reset
  std::vector<int> h_hist_n;    // host mirror of shist_n (ids in each history)
  // taps (ms_model_set_taps): per-layer output rows and raw logits of every
  // decode step and of a prompt's last row, for parity checks
  float *tap_hidden = nullptr, *tap_logits = nullptr;
  // streaming
  uint8_t *slot[2] = {nullptr, nullptr};
  size_t slot_bytes = 0;
  hipEvent_t ev_free[2] = {}, ev_ready[2] = {};
  std::vector<hipEvent_t> io_ev;  // per-call timing events
  ms_stream_stats stats{};
  std::vector<void *> allocs;
};

namespace ms {

static int dmalloc(ms_model *m, void **p, size_t bytes) {
  if (hipMalloc(p, bytes ? bytes : 16) != hipSuccess)
    return fail(MS_E_NOMEM, "model: out of device memory");
  m->allocs.push_back(*p);
  return MS_OK;
}

// ---- profiling helpers -------------------------------------------------------
static bool capturing(hipStream_t st) {
  hipStreamCaptureStatus s = hipStreamCaptureStatusNone;
  (void)hipStreamIsCapturing(st, &s);
  return s != hipStreamCaptureStatusNone;
}
static hipEvent_t prof_event() {
  if (g_prof.used == g_prof.pool.size()) {
    hipEvent_t e;
    (void)hipEventCreate(&e);
    g_prof.pool.push_back(e);
  }
  return g_prof.pool[g_prof.used++];
}
struct ProfScope {
  int cls;
  double bytes;
  hipStream_t st;
  hipEvent_t b{};
  bool active;
  ProfScope(int c, double by, hipStream_t s) : cls(c), bytes(by), st(s) {
    g_prof.cur = c;
    active = g_prof.on && !capturing(s);
    if (active) {
      hipEvent_t a = prof_event();
      b = prof_event();
      (void)hipEventRecord(a, st);
      g_prof.pending.push_back({cls, a, b, bytes});
    }
  }
  ~ProfScope() {
    if (active) (void)hipEventRecord(b, st);
    g_prof.cur = -1;
  }
};
static void prof_collect() {
  for (auto &r : g_prof.pending) {
    float ms = 0.f;
    (void)hipEventSynchronize(r.b);
    (void)hipEventElapsedTime(&ms, r.a, r.b);
    g_prof.launches[r.cls] += 1;
    g_prof.ms[r.cls] += ms;
    g_prof.bytes[r.cls] += r.bytes;
  }
  g_prof.pending.clear();
  g_prof.used = 0;
}

// ---- per-layer enqueue --------------------------------------------------------
// Prefill processes the prompt in chunks of up to kPrefillRows rows; their
// projections run as GEMMs.  Flash attention takes a whole chunk per launch
// (one block per 16 rows and kv head: long chunks fill the chip); the chunked
// attention path runs kPrefillAttnRows rows per launch (its partial-result
// buffer grows with the rows of a launch).  Workspace grows with the chunk:
// about 170 KB per row at E4B shapes.
constexpr int kPrefillRows = 2048;
constexpr int kPrefillAttnRows = 32;

struct RunCfg {
  int B, T;                 // sequences, rows per sequence
  const float *in_rows;     // first layer input rows [B*T][D]
  float *out_rows;          // layer output of the last layer (or null)
  float *hidden;            // optional [n_layers][B*T][D]
  int first_layer, n_layers;
  int seq0;                 // first sequence (caches / positions offset)
  int plan_pos;             // first row's position as the host knows it (B = 1);
                            // sizes the prefill attention's key split only
  int pos_bound;            // every row's position is below it (decode attention
                            // launches only the key chunks below it)
  float *tap_last;          // optional [n_layers][D]: each layer's last output row
  // one row of one sequence (a batch-1 decode step), where the layer's shapes
  // allow it: the attention leaves its key chunks unmerged and the O
  // projection merges them (k_attn_part + AS_ATTN); Q|K|V, Gate|Up and Down
  // quantize their input row per wave (AS_WAVES)
  bool one_row;
};

// Launch a projection of rows r: quantized in the kernel's prologue with
// `waves` waves per block when the limb rows fit in LDS, else by the quant
// kernel into m->quant first (the GEMV then reads them from global memory).
static int launch_gemv_rec(const GemvArgs &a, hipStream_t st) {
  if (g_prof.on && g_prof.cur >= 0) {
    g_prof.last[g_prof.cur] = a;
    g_prof.last_layer[g_prof.cur] = g_prof.layer;
    g_prof.have[g_prof.cur] = true;
  }
  return launch_gemv(a, st);
}

// One row of one sequence with the row quantized per wave (AS_WAVES) when the
// shapes fit (K = waves * 640), else launch_proj.
static int launch_proj_row(ms_model *m, const RunCfg &rc, GemvArgs a, const RowSrc &r,
                           int waves, int waves_row, hipStream_t st);

constexpr size_t kLdsLimit = 150 * 1024;  // LDS of a GEMV launch with its limb rows

static int launch_proj(ms_model *m, GemvArgs a, const RowSrc &r, int waves, hipStream_t st) {
  if (a.M > kGemvMaxM) {
    // prefill rows: quantize every row once (three limbs), then the MFMA GEMM
    GemmArgs g{};
    g.epi = a.epi;
    g.M = a.M;
    g.K = a.K;
    g.a = quant_rows3_view(m->quant, gemm_row_pad(a.M), a.K);
    for (int i = 0; i < 3; ++i) g.seg[i] = a.seg[i];
    g.nseg = a.nseg;
    g.out = a.out;
    g.ldo = a.ldo;
    g.resid = a.resid;
    g.out2 = a.out2;
    g.sw_out = a.sw_out;
    g.ldo_sw = a.ldo_sw;
    if (int rc = launch_quant_rows3(r, a.M, a.K, g.a, st)) return rc;
    return launch_gemm(g, st);
  }
  a.asrc = AS_ROWS;
  a.rows = r;
  a.waves = waves;
  if (a.M > 1 && a.M <= 4 && waves == 16 && a.K <= 8 * 2 * 64 * 8) {
    // two to four rows: 8 waves, each row its own wave pair with the rows'
    // loads in one batch (a 16-wave block takes the rows one after another;
    // the demo model's Down at four rows: 1.165 -> 1.085 ms per harness step)
    a.waves = 8;
    if (gemv_lds_need(a) <= kLdsLimit) return launch_gemv_rec(a, st);
    a.waves = waves;
  }
  if (a.K <= 8 * 2 * 64 * waves && gemv_lds_need(a) <= kLdsLimit) return launch_gemv_rec(a, st);
  a.asrc = AS_QUANT;
  a.rows = RowSrc{};
  a.q = quant_rows_view(m->quant, a.M, a.K);
  // one to four rows of a long residual projection (Down at batch 2-4): 16
  // waves, every super-tile of a wave in one batch
  a.waves = (a.M <= 4 && a.P == 1 && a.epi == EPI_RESID && waves == 16) ? 16 : 4;
  if (int rc = launch_quant_rows(r, a.M, a.K, a.q, st)) return rc;
  return launch_gemv_rec(a, st);
}

// A batch-1 decode row through the per-wave prologue (AS_WAVES, waves_row
// waves) when the matrix's shape has an instantiation and the row's limbs fit
// the LDS; otherwise launch_proj.  (At two to four rows the per-row prologue
// of launch_proj is faster.)
static int launch_proj_row(ms_model *m, const RunCfg &rc, GemvArgs a, const RowSrc &r,
                           int waves, int waves_row, hipStream_t st) {
  if (rc.one_row && a.M == 1 && !r.gamma && !r.x_out) {
    GemvArgs w = a;
    w.asrc = AS_WAVES;
    w.rows = r;
    w.waves = waves_row;
    if (wave_shape_ok(w) && gemv_lds_need(w) <= kLdsLimit) return launch_gemv_rec(w, st);
  }
  // One to four rows of Q|K|V, O and Down: per-wave slices quantized one
  // super-tile at a time (AS_WSTREAM; the same limbs as the one-row per-wave
  // GEMV).  Measured at batch 4 against the block-wide row prologue (and for
  // Down against a quantization launch plus a GEMV reading limbs from
  // memory): Down 2,048 -> 2,255 tok/s, then Q|K|V and O 2,358; the demo
  // harness step (four rows) 1.07 -> 1.00 ms, and with the demo model's Down
  // (K = 4096) streamed too 0.96 ms.  Gate|Up keeps the block-wide prologue
  // (streamed: 2,305 against 2,352 tok/s; quantized up front per wave: 2,265).
  if (a.M <= kWaveRowsMax && !r.gamma && !r.x_out && a.epi != EPI_SWIGLU) {
    GemvArgs w = a;
    w.asrc = AS_WSTREAM;
    w.rows = r;
    w.waves = waves_row;
    if (wave_shape_ok(w) && gemv_lds_need(w) <= kLdsLimit) return launch_gemv_rec(w, st);
  }
  return launch_proj(m, a, r, waves, st);
}

// Rows entering layer l: the previous layer's output or the call's input rows.
static const float *layer_input(ms_model *m, const RunCfg &rc, int l) {
  return l == rc.first_layer ? rc.in_rows : m->xs;
}

static int enqueue_layer(ms_model *m, int l, const RunCfg &rc, hipStream_t st) {
  Layer &Ly = m->L[l];
  g_prof.layer = l;
  const ms_layer_desc &d = Ly.d;
  const int M = rc.B * rc.T;
  const int D = m->d.hidden, F = m->d.ffn;
  const int ld = d.q_dim + 2 * d.kv_dim;

  AttnArgs attn{};
  attn.B = rc.B;
  attn.T = rc.T;
  attn.q_dim = d.q_dim;
  attn.kv_dim = d.kv_dim;
  attn.hd = d.head_dim;
  attn.n_heads = d.n_heads;
  attn.n_kv = d.n_kv_heads;
  attn.rot = d.rot_dim;
  attn.cache_kind = d.cache_kind;
  attn.cache_len = d.cache_len;
  attn.clamp = d.clamp_reads;
  attn.scale = 1.0f / sqrtf((float)d.head_dim);
  attn.qkv = m->qkv;
  attn.ld = ld;
  attn.apply_rope = 1;
  attn.cos_t = m->ropes[Ly.rope].cs;
  attn.sin_t = m->ropes[Ly.rope].sn;
  attn.pos = m->pos + rc.seq0;
  attn.kc = Ly.kc + (size_t)rc.seq0 * Ly.cache_seq_stride;
  attn.vc = Ly.vc + (size_t)rc.seq0 * Ly.cache_seq_stride;
  attn.cache_seq_stride = Ly.cache_seq_stride;
  attn.n_chunks = Ly.n_chunks;
  attn.part = m->attn_part;
  attn.ctr = m->attn_ctr;
  attn.out = m->aO;
  attn.write_cache = 1;
  attn.plan_pos = rc.plan_pos;
  attn.pos_bound = rc.pos_bound;
  attn.rope_cur = m->rope_cur;
  // one decode row: chunk partials (k_attn_part), merged in the O projection
  const bool use_part = rc.one_row && rc.B == 1 && rc.T == 1 && d.n_heads == 8 &&
                        d.q_dim == 8 * d.head_dim && dec_part_ok(attn);

  // 1. x = rmsnorm(ple * x) in the prologue, fused Q|K|V projection
  //    (gemma4_e4b.mojo:473-487)
  {
    RowSrc r{};
    r.x = layer_input(m, rc, l);
    r.ld = D;
    r.pre_scale = Ly.ple;
    r.norm = 1;
    r.y_out = m->xn;
    GemvArgs a{};
    a.epi = EPI_STORE;
    a.K = D;
    a.M = M;
    a.seg[0] = GemvSeg{Ly.w[0], Ly.scale[0], d.q_dim, 0};
    a.seg[1] = GemvSeg{Ly.w[1], Ly.scale[1], d.kv_dim, d.q_dim};
    a.seg[2] = GemvSeg{Ly.w[2], Ly.scale[2], d.kv_dim, d.q_dim + d.kv_dim};
    a.nseg = 3;
    a.P = 1;
    a.out = m->qkv;
    a.ldo = ld;
    ProfScope ps(PC_QKV, (double)D * ld / 2, st);
    GemvArgs w = a;
    w.asrc = AS_WAVES;
    w.rows = r;
    w.waves = 4;
    const int tpw = D % (4 * kSuperK) == 0 ? D / (4 * kSuperK) : 0;
    if (use_part && (tpw == 2 || tpw == 5) && wave_shape_ok(w) &&
        gemv_lds_need(w) <= kLdsLimit) {
      // one launch also prepares the attention's RoPE factors
      w.pf.pos = attn.pos;
      w.pf.cos_t = attn.cos_t;
      w.pf.sin_t = attn.sin_t;
      w.pf.half = d.rot_dim / 2;
      w.pf.rope_rows = m->d.max_pos;
      w.pf.rope_cur = m->rope_cur;
      if (int rc2 = launch_gemv_rec(w, st)) return rc2;
    } else {
      if (int rc2 = launch_proj_row(m, rc, a, r, 8, 4, st)) return rc2;
      if (use_part)
        if (int rc2 = launch_rope_cur(attn, st)) return rc2;
    }
  }
  // 2. attention (chunks + merge/cache append)
  bool merged_in_o = false;
  {
    AttnArgs a = attn;
    // KV bytes read at the current position are counted by bench.py
    ProfScope ps(PC_ATTN, 0.0, st);
    if (use_part) {
      // chunk partials only; the O projection below merges them
      if (g_prof.on) {
        const int k = d.cache_kind == MS_CACHE_CIRCULAR ? 1 : 0;
        g_prof.last_attn[k] = a;
        g_prof.last_attn_layer[k] = l;
        g_prof.have_attn[k] = true;
        g_prof.attn_part[k] = true;
      }
      if (int rc2 = launch_attention_partials(a, st)) return rc2;
      merged_in_o = true;
    } else if (rc.T == 1 && dec_part_ok(a)) {
      // one row per sequence (a batch decode step, a one-row forward): the
      // same chunk blocks, merged by the last block of each (sequence, kv
      // head, head pair), the RoPE factors from the tables at each position
      if (int rc2 = launch_attention_partials(a, st, true)) return rc2;
    } else if (attn_rows_ok(a)) {
      // two to four rows of one sequence: chunk partials per row, merged
      if (int rc2 = launch_attention_rows(a, st)) return rc2;
    } else if (rc.B == 1 && rc.T > kGemvMaxM && m->fq && prefill_flash_ok(a)) {
      // prefill rows: flash attention on fp32 MFMA
      if (int rc2 = launch_attention_prefill(a, m->fq, m->fk, m->fpart, m->fpart_floats, st))
        return rc2;
    } else if (rc.T <= kPrefillAttnRows || rc.B != 1) {
      if (g_prof.on && rc.T == 1) {
        const int k = d.cache_kind == MS_CACHE_CIRCULAR ? 1 : 0;
        g_prof.last_attn[k] = a;
        g_prof.last_attn_layer[k] = l;
        g_prof.have_attn[k] = true;
        g_prof.attn_part[k] = false;
      }
      if (int rc2 = launch_attention(a, st)) return rc2;
    } else {
      // a prefill chunk: consecutive row groups, each attending to the cache
      // the groups before it have written (base positions in m->ppos)
      for (int s = 0, r0 = 0; r0 < rc.T; ++s, r0 += kPrefillAttnRows) {
        AttnArgs b = a;
        b.T = std::min(kPrefillAttnRows, rc.T - r0);
        b.qkv = m->qkv + (size_t)r0 * ld;
        b.out = m->aO + (size_t)r0 * d.q_dim;
        b.pos = m->ppos + s;
        if (int rc2 = launch_attention(b, st)) return rc2;
      }
    }
  }
  // 3. x2 = x + attn . Wo (residual epilogue)
  {
    RowSrc r{};
    r.x = m->aO;
    r.ld = d.q_dim;
    r.pre_scale = 1.f;
    GemvArgs a{};
    a.epi = EPI_RESID;
    a.K = d.q_dim;
    a.M = M;
    a.seg[0] = GemvSeg{Ly.w[3], Ly.scale[3], D, 0};
    a.nseg = 1;
    a.P = 1;
    a.out = m->x2;
    a.ldo = D;
    a.resid = m->xn;
    ProfScope ps(PC_O, (double)d.q_dim * D / 2, st);
    if (merged_in_o) {
      // the attention chunks merged per head in the O projection's prologue
      a.asrc = AS_ATTN;
      a.waves = 8;
      a.at.part = m->attn_part;
      a.at.pos = m->pos + rc.seq0;
      a.at.hd = d.head_dim;
      a.at.n_heads = d.n_heads;
      a.at.circular = d.cache_kind == MS_CACHE_CIRCULAR;
      a.at.cache_len = d.cache_len;
      a.at.clamp = d.clamp_reads;
      AttnArgs pa{};
      pa.cache_len = d.cache_len;
      pa.pos_bound = rc.pos_bound;
      a.at.chunks = dec_part_chunks(pa);
      if (int rc2 = launch_gemv_rec(a, st)) return rc2;
    } else if (int rc2 = launch_proj_row(m, rc, a, r, 8, 8, st)) {
      return rc2;
    }
  }
  // 4. x2n = rmsnorm(x2) in the prologue, Gate|Up, SwiGLU epilogue
  {
    RowSrc r{};
    r.x = m->x2;
    r.ld = D;
    r.pre_scale = 1.f;
    r.norm = 1;
    r.y_out = m->x2n;
    GemvArgs a{};
    a.epi = EPI_SWIGLU;
    a.K = D;
    a.M = M;
    a.seg[0] = GemvSeg{Ly.w[4], Ly.scale[4], F, 0};
    a.seg[1] = GemvSeg{Ly.w[5], Ly.scale[5], F, 0};
    a.nseg = 2;
    a.P = 2;
    a.sw_out = m->aF;
    a.ldo_sw = F;
    ProfScope ps(PC_GATEUP, (double)D * F, st);
    if (int rc2 = launch_proj_row(m, rc, a, r, 4, 4, st)) return rc2;
  }
  // 5. x_out = x2n + ffn . Wd (residual epilogue): the layer output
  {
    RowSrc r{};
    r.x = m->aF;
    r.ld = F;
    r.pre_scale = 1.f;
    GemvArgs a{};
    a.epi = EPI_RESID;
    a.K = F;
    a.M = M;
    a.seg[0] = GemvSeg{Ly.w[6], Ly.scale[6], D, 0};
    a.nseg = 1;
    a.P = 1;
    a.out = m->xs;
    a.ldo = D;
    a.resid = m->x2n;
    if (rc.hidden) a.out2 = rc.hidden + (size_t)(l - rc.first_layer) * M * D;
    ProfScope ps(PC_DOWN, (double)F * D / 2, st);
    if (int rc2 = launch_proj_row(m, rc, a, r, 16, 16, st)) return rc2;
  }
  return MS_OK;
}

// LM head over rows `row0..row0+M-1` of the last layer's output, then the
// greedy id per row.
// The draw (sampling) or the first maximum (greedy, temperature 0) of the
// logits rows of sequences seq0 .. seq0 + M - 1, then the decode-state update.
static int enqueue_pick(ms_model *m, const RunCfg &rc, int M, ArgmaxFin f, hipStream_t st) {
  SampleArgs s{};
  s.logits = m->logits + (size_t)rc.seq0 * m->d.vocab;
  s.n = m->d.vocab;
  s.ld = m->d.vocab;
  s.temperature = m->sampling ? m->samp_temp : 0.f;
  s.penalty = m->sampling ? m->samp_pen : 1.f;
  if (m->sampling) {
    s.hist = m->shist + (size_t)rc.seq0 * kSampleMaxHistory;
    s.hist_ld = kSampleMaxHistory;
    s.hist_n = m->shist_n + rc.seq0;
    s.hist_cap = kSampleMaxHistory;
    s.hist_append = 1;
    s.seed = m->samp_seed;
    s.seq0 = rc.seq0;
    s.step = m->samp_ctr;
    f.draws = m->samp_ctr;
  }
  s.ids_out = m->samp_ids;
  if (int r2 = launch_sample(s, M, st)) return r2;
  f.ids_in = m->samp_ids;
  return launch_argmax_fin(f, st);
}

// Raw logits of the call's rows into the logits tap (before the sampler
// rewrites them in place).
static int tap_logits(ms_model *m, const RunCfg &rc, int M, hipStream_t st) {
  if (!m->tap_logits) return MS_OK;
  const size_t V = (size_t)m->d.vocab;
  MS_HIP_TRY(hipMemcpyAsync(m->tap_logits, m->logits + (size_t)rc.seq0 * V, (size_t)M * V * 4,
                            hipMemcpyDeviceToDevice, st));
  return MS_OK;
}

// FP32 head: final norm (y rows), matmul_fp32_raw into the logits, then the pick.
static int enqueue_lm_f32(ms_model *m, const RunCfg &rc, RowSrc r, int M, const ArgmaxFin &fin,
                          hipStream_t st) {
  const int D = m->d.hidden, V = m->d.vocab;
  r.y_out = m->lm_y;
  {
    ProfScope ps(PC_LM, (double)D * V * 4, st);
    if (int r2 = launch_quant_rows(r, M, D, quant_rows_view(m->quant, M, D), st)) return r2;
    if (int r2 = launch_mm_f32(m->lm_y, m->lm_f32, m->logits + (size_t)rc.seq0 * V, M, D, V, 0,
                               m->lm_part, st))
      return r2;
  }
  ArgmaxFin f = fin;
  f.M = M;
  ProfScope ps(PC_OTHER, 0.0, st);
  if (int r2 = tap_logits(m, rc, M, st)) return r2;
  return enqueue_pick(m, rc, M, f, st);
}

static int enqueue_lm(ms_model *m, const RunCfg &rc, int row0, int M, const ArgmaxFin &fin,
                      hipStream_t st) {
  const int D = m->d.hidden;
  // final norm with gamma (apply_final_norm lm_head.mojo:119-130,
  // rmsnorm_weighted_inplace kernels.mojo:598-613) fused into the quantization
  RowSrc r{};
  r.x = m->xs + (size_t)row0 * D;
  r.ld = D;
  r.pre_scale = 1.f;
  r.norm = 1;
  r.gamma = m->gamma;
  if (rc.out_rows) r.x_out = rc.out_rows + (size_t)row0 * D;
  if (m->lm_f32) return enqueue_lm_f32(m, rc, r, M, fin, st);
  GemvArgs a{};
  a.epi = EPI_ARGMAX;
  a.asrc = AS_QUANT;
  a.K = D;
  a.M = M;
  a.q = quant_rows_view(m->quant, M, D);
  a.seg[0] = GemvSeg{m->lm_w, m->lm_scale, m->d.vocab, 0};
  a.nseg = 1;
  a.P = 4;
  a.waves = 4;
  a.out = m->sampling ? m->logits + (size_t)rc.seq0 * m->d.vocab : m->tap_logits;
  a.ldo = m->d.vocab;
  a.arg_val = m->arg_val;
  a.arg_idx = m->arg_idx;
  {
    ProfScope ps(PC_LM, (double)D * m->d.vocab / 2, st);
    if (int r2 = launch_quant_rows(r, M, D, a.q, st)) return r2;
    if (int r2 = launch_gemv(a, st)) return r2;
  }
  ArgmaxFin f = fin;
  f.arg_val = m->arg_val;
  f.arg_idx = m->arg_idx;
  f.n_blocks = m->lm_blocks;
  f.M = M;
  ProfScope ps(PC_OTHER, 0.0, st);
  if (m->sampling)
    if (int r2 = tap_logits(m, rc, M, st)) return r2;
  // temperature_sampling (lm_head.mojo:198-254) on the logits rows, the
  // draws appended to the sequences' histories
  if (m->sampling) return enqueue_pick(m, rc, M, f, st);
  return launch_argmax_fin(f, st);
}

// Output rows of the last layer without an LM head.
static int enqueue_output(ms_model *m, const RunCfg &rc, hipStream_t st) {
  if (!rc.out_rows) return MS_OK;
  const size_t n = (size_t)rc.B * rc.T * m->d.hidden;
  MS_HIP_TRY(hipMemcpyAsync(rc.out_rows, m->xs, n * 4, hipMemcpyDeviceToDevice, st));
  return MS_OK;
}

// ---- streaming: two HBM slots filled on the copy stream ----------------------
// Copies layer l's packed weights into slot s once the streamed layer that
// used the slot before has finished; a/b bracket the copies on the copy stream.
static int stream_prefetch(ms_model *m, int l, int s, hipEvent_t a, hipEvent_t b) {
  Layer &Ly = m->L[l];
  MS_HIP_TRY(hipStreamWaitEvent(ctx().copy_stream, m->ev_free[s], 0));
  MS_HIP_TRY(hipEventRecord(a, ctx().copy_stream));
  for (int i = 0; i < 7; ++i)
    MS_HIP_TRY(hipMemcpyAsync(m->slot[s] + Ly.off[i], Ly.h_packed[i], Ly.bytes[i],
                              hipMemcpyHostToDevice, ctx().copy_stream));
  MS_HIP_TRY(hipEventRecord(b, ctx().copy_stream));
  MS_HIP_TRY(hipEventRecord(m->ev_ready[s], ctx().copy_stream));
  return MS_OK;
}

// Copy of layer l's last output row into the prefill tap.
static int tap_last_row(ms_model *m, const RunCfg &rc, int l, hipStream_t st) {
  if (!rc.tap_last) return MS_OK;
  const size_t D = (size_t)m->d.hidden;
  MS_HIP_TRY(hipMemcpyAsync(rc.tap_last + (size_t)(l - rc.first_layer) * D,
                            m->xs + (size_t)(rc.B * rc.T - 1) * D, D * 4,
                            hipMemcpyDeviceToDevice, st));
  return MS_OK;
}

static int run_layers(ms_model *m, const RunCfg &rc, hipStream_t st) {
  const bool streaming = !m->d.resident;
  const int l0 = rc.first_layer, l1 = rc.first_layer + rc.n_layers;
  if (streaming) {
    // timing of this pass ([copy start, copy end] per layer and compute
    // waits), added to the statistics of the API call (reset at its start)
    auto t0 = std::chrono::steady_clock::now();
    std::vector<hipEvent_t> ev;
    auto mk = [&]() {
      hipEvent_t e;
      (void)hipEventCreate(&e);
      ev.push_back(e);
      return e;
    };
    MS_HIP_TRY(hipEventRecord(m->ev_free[0], st));
    MS_HIP_TRY(hipEventRecord(m->ev_free[1], st));
    std::vector<hipEvent_t> cp0, cp1, w0, w1;
    int n_streamed = 0;
    for (int l = l0; l < l1; ++l) {
      if (m->L[l].pinned) {
        // pinned layer (SparsePinEngine.get_layer_ref, sparse_pin.mojo:295-330):
        // weights already in HBM; the copy stream moves on to the next
        // streamed layer while this one computes
        if (int r = enqueue_layer(m, l, rc, st)) return r;
        if (int r = tap_last_row(m, rc, l, st)) return r;
        m->stats.layers_pinned += 1;
        continue;
      }
      const int s = n_streamed++ & 1;
      for (int i = 0; i < 7; ++i) m->stats.bytes += (double)m->L[l].bytes[i];
      m->stats.layers_streamed += 1;
      hipEvent_t a = mk(), b = mk();
      if (int r = stream_prefetch(m, l, s, a, b)) return r;
      cp0.push_back(a);
      cp1.push_back(b);
      hipEvent_t c = mk(), e = mk();
      MS_HIP_TRY(hipEventRecord(c, st));
      MS_HIP_TRY(hipStreamWaitEvent(st, m->ev_ready[s], 0));
      MS_HIP_TRY(hipEventRecord(e, st));
      w0.push_back(c);
      w1.push_back(e);
      for (int i = 0; i < 7; ++i) m->L[l].w[i] = m->slot[s] + m->L[l].off[i];
      if (int r = enqueue_layer(m, l, rc, st)) return r;
      if (int r = tap_last_row(m, rc, l, st)) return r;
      MS_HIP_TRY(hipEventRecord(m->ev_free[s], st));
    }
    MS_HIP_TRY(hipStreamSynchronize(st));
    MS_HIP_TRY(hipStreamSynchronize(ctx().copy_stream));
    double io = 0, wait = 0;
    for (size_t i = 0; i < cp0.size(); ++i) {
      float a = 0, b = 0;
      (void)hipEventElapsedTime(&a, cp0[i], cp1[i]);
      (void)hipEventElapsedTime(&b, w0[i], w1[i]);
      io += a;
      wait += b;
    }
    for (auto e : ev) (void)hipEventDestroy(e);
    const double total =
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0)
            .count();
    m->stats.io_ms += io;
    m->stats.wait_ms += wait;
    m->stats.total_ms += total;
    m->stats.compute_ms += total - wait;
    return MS_OK;
  }
  for (int l = l0; l < l1; ++l) {
    if (int r = enqueue_layer(m, l, rc, st)) return r;
    if (int r = tap_last_row(m, rc, l, st)) return r;
  }
  return MS_OK;
}

static int check_positions(ms_model *m, const int *base, int B, int T, int extra) {
  for (int b = 0; b < B; ++b) {
    MS_CHECK_ARG(base[b] >= 0, "model: negative position");
    MS_CHECK_ARG(base[b] + T + extra <= m->d.max_pos,
                 "model: position beyond max_pos (RoPE tables)");
    for (auto &Ly : m->L)
      if (Ly.d.cache_kind == MS_CACHE_LINEAR && !Ly.d.clamp_reads)
        MS_CHECK_ARG(base[b] + T + extra <= Ly.d.cache_len,
                     "model: positions exceed a linear KV cache (the reference reads "
                     "out of bounds here, main.mojo:463,476-477)");
  }
  return MS_OK;
}

static int check_ready(ms_model *m, bool need_lm) {
  for (size_t l = 0; l < m->L.size(); ++l)
    if (m->L[l].set_mask != 0x7f)
      return fail(MS_E_STATE, "model: layer " + std::to_string(l) + " has unset matrices");
  if (need_lm && !m->has_lm) return fail(MS_E_STATE, "model: LM head not set");
  return MS_OK;
}

}  // namespace ms

using namespace ms;

extern "C" int ms_model_create(const ms_model_desc *desc, const ms_layer_desc *layers,
                               ms_model **out) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(desc && layers && out, "model_create: null argument");
  const ms_model_desc &d = *desc;
  MS_CHECK_ARG(d.hidden > 0 && d.hidden % 128 == 0, "model: hidden % 128 != 0");
  MS_CHECK_ARG(d.ffn > 0 && d.ffn % 128 == 0, "model: ffn % 128 != 0");
  MS_CHECK_ARG(d.n_layers > 0, "model: n_layers <= 0");
  MS_CHECK_ARG(d.max_seqs >= 1 && d.max_rows >= 1 && d.max_seqs * d.max_rows <= 16,
               "model: max_seqs * max_rows must be in [1, 16]");
  MS_CHECK_ARG(d.max_pos >= 1, "model: max_pos < 1");
  MS_CHECK_ARG(d.vocab == 0 || d.vocab % 64 == 0, "model: vocab % 64 != 0");
  auto *m = new ms_model();
  m->d = d;
  m->Mmax = d.max_seqs * d.max_rows;
  m->h_pos.assign(d.max_seqs, 0);
  m->h_hist_n.assign(d.max_seqs, 0);
  // models with an LM head prefill prompts in chunks of up to kPrefillRows
  if (d.vocab > 0) m->prefill_rows = std::max(m->Mmax, std::min(kPrefillRows, d.max_pos));
  const int M = std::max(m->Mmax, m->prefill_rows);  // workspace rows
  const int attn_rows = m->prefill_rows > kGemvMaxM
                            ? std::max(d.max_rows, kPrefillAttnRows) : d.max_rows;
  auto cleanup = [&](int rc) {
    ms_model_destroy(m);
    return rc;
  };
  size_t max_part = 0;
  for (int l = 0; l < d.n_layers; ++l) {
    const ms_layer_desc &ld = layers[l];
    if (!(ld.n_heads > 0 && ld.n_kv_heads > 0 && ld.n_heads % ld.n_kv_heads == 0 &&
          ld.q_dim == ld.n_heads * ld.head_dim && ld.kv_dim == ld.n_kv_heads * ld.head_dim &&
          ld.q_dim % 128 == 0 && ld.kv_dim % 16 == 0 && ld.rot_dim > 0 &&
          ld.rot_dim % 2 == 0 && ld.rot_dim <= ld.head_dim && ld.cache_len > 0 &&
          (ld.cache_kind == MS_CACHE_LINEAR || ld.cache_kind == MS_CACHE_CIRCULAR)))
      return cleanup(fail(MS_E_INVALID, "model: inconsistent layer " + std::to_string(l) +
                                            " (ShapeGuard: q_dim = n_heads*head_dim, "
                                            "kv_dim = n_kv*head_dim, q_dim % 128 == 0)"));
    Layer Ly;
    Ly.d = ld;
    const size_t K[7] = {(size_t)d.hidden, (size_t)d.hidden, (size_t)d.hidden,
                         (size_t)ld.q_dim, (size_t)d.hidden, (size_t)d.hidden,
                         (size_t)d.ffn};
    const size_t N[7] = {(size_t)ld.q_dim, (size_t)ld.kv_dim, (size_t)ld.kv_dim,
                         (size_t)d.hidden, (size_t)d.ffn, (size_t)d.ffn, (size_t)d.hidden};
    size_t off = 0;
    for (int i = 0; i < 7; ++i) {
      Ly.bytes[i] = K[i] * N[i] / 2;
      Ly.off[i] = off;
      off += (Ly.bytes[i] + 4095) & ~(size_t)4095;
    }
    m->slot_bytes = std::max(m->slot_bytes, off);
    // rope table id
    int rid = -1;
    for (size_t r = 0; r < m->ropes.size(); ++r)
      if (m->ropes[r].rot == ld.rot_dim && m->ropes[r].theta == ld.theta) rid = (int)r;
    if (rid < 0) {
      RopeTab t;
      t.rot = ld.rot_dim;
      t.theta = ld.theta;
      m->ropes.push_back(t);
      rid = (int)m->ropes.size() - 1;
    }
    Ly.rope = rid;
    const int ncols_qkv = ld.q_dim + 2 * ld.kv_dim;
    const int span = ld.cache_kind == MS_CACHE_CIRCULAR ? ld.cache_len + attn_rows - 1
                                                        : ld.cache_len + attn_rows;
    Ly.n_chunks = cdiv(span, kAttnChunk);
    const int G = ld.n_heads / ld.n_kv_heads;
    max_part = std::max(max_part, attn_part_floats(d.max_seqs, ld.n_kv_heads, Ly.n_chunks,
                                                   attn_rows, G, ld.head_dim));
    // a batch-1 decode step's chunk partials, merged in the O projection, or
    // those of two to four rows of one sequence
    max_part = std::max(max_part, dec_part_floats(std::min(d.max_rows, 4), ld.n_heads,
                                                  ld.head_dim));
    m->qkv_max = std::max(m->qkv_max, ncols_qkv);
    m->q_max = std::max(m->q_max, ld.q_dim);
    m->quant_k = std::max(m->quant_k, std::max(std::max(d.hidden, d.ffn), ld.q_dim));
    m->kv_max = std::max(m->kv_max, ld.kv_dim);
    m->hd_max = std::max(m->hd_max, ld.head_dim);
    m->nkv_max = std::max(m->nkv_max, ld.n_kv_heads);
    m->L.push_back(Ly);
  }
  int rc;
  const int D = d.hidden, F = d.ffn;
  if ((rc = dmalloc(m, (void **)&m->x_in, (size_t)M * D * 4)) ||
      (rc = dmalloc(m, (void **)&m->xs, (size_t)M * D * 4)) ||
      (rc = dmalloc(m, (void **)&m->xn, (size_t)M * D * 4)) ||
      (rc = dmalloc(m, (void **)&m->x2, (size_t)M * D * 4)) ||
      (rc = dmalloc(m, (void **)&m->x2n, (size_t)M * D * 4)) ||
      (rc = dmalloc(m, (void **)&m->aO, (size_t)M * m->q_max * 4)) ||
      (rc = dmalloc(m, (void **)&m->aF, (size_t)M * F * 4)) ||
      (rc = dmalloc(m, &m->quant, quant_rows_bytes(gemm_row_pad(M), m->quant_k))) ||
      (rc = dmalloc(m, (void **)&m->ppos, (size_t)(M / kPrefillAttnRows + 2) * 4)))
    return cleanup(rc);
  if (m->prefill_rows > kGemvMaxM &&
      ((rc = dmalloc(m, (void **)&m->fq, (size_t)m->prefill_rows * m->q_max * 4)) ||
       (rc = dmalloc(m, (void **)&m->fk, (size_t)m->prefill_rows * m->kv_max * 4))))
    return cleanup(rc);
  if (m->prefill_rows > kGemvMaxM) {
    // key-split partials of any flash launch
    for (auto &Ly : m->L)
      m->fpart_floats = std::max(m->fpart_floats, flash_part_floats_max(Ly.d.head_dim));
    if (m->fpart_floats && (rc = dmalloc(m, (void **)&m->fpart, m->fpart_floats * 4)))
      return cleanup(rc);
  }
  if ((rc = dmalloc(m, (void **)&m->qkv, (size_t)M * m->qkv_max * 4)) ||
      (rc = dmalloc(m, (void **)&m->attn_part, max_part * 4)) ||
      (rc = dmalloc(m, (void **)&m->rope_cur, 512 * 4)) ||
      (rc = dmalloc(m, (void **)&m->attn_ctr, attn_ctr_count(d.max_seqs, m->nkv_max) * 4)) ||

      (rc = dmalloc(m, (void **)&m->pos, 64 * 4)) ||
      (hipHostMalloc((void **)&m->h_pos_pin, 64 * 4, hipHostMallocDefault) != hipSuccess &&
       (rc = fail(MS_E_NOMEM, "model: pinned allocation failed"))) ||
      (rc = dmalloc(m, (void **)&m->tok, 64 * 4)) ||
      (rc = dmalloc(m, (void **)&m->step, 64 * 4)) ||
      (rc = dmalloc(m, (void **)&m->ids_hist, (size_t)m->hist_cap * d.max_seqs * 4)))
    return cleanup(rc);
  if (hipMemset(m->pos, 0, 64 * 4) != hipSuccess || hipMemset(m->step, 0, 64 * 4) != hipSuccess ||
      hipMemset(m->attn_part, 0, max_part * 4) != hipSuccess ||
      hipMemset(m->tok, 0, 64 * 4) != hipSuccess ||
      hipMemset(m->attn_ctr, 0, attn_ctr_count(d.max_seqs, m->nkv_max) * 4) != hipSuccess)
    return cleanup(fail(MS_E_HIP, "model: memset failed"));
  // KV caches (zero-initialised like the reference's resized Lists)
  for (auto &Ly : m->L) {
    const size_t per_seq = (size_t)Ly.d.cache_len * Ly.d.kv_dim;
    Ly.cache_seq_stride = per_seq;
    if ((rc = dmalloc(m, (void **)&Ly.kc, per_seq * d.max_seqs * 4)) ||
        (rc = dmalloc(m, (void **)&Ly.vc, per_seq * d.max_seqs * 4)))
      return cleanup(rc);
    (void)hipMemset(Ly.kc, 0, per_seq * d.max_seqs * 4);
    (void)hipMemset(Ly.vc, 0, per_seq * d.max_seqs * 4);
  }
  // RoPE tables for positions 0..max_pos-1
  for (auto &t : m->ropes) {
    std::vector<float> cs, sn;
    rope_table_host(t.rot, t.theta, 0, d.max_pos, cs, sn);
    if ((rc = dmalloc(m, (void **)&t.cs, cs.size() * 4)) ||
        (rc = dmalloc(m, (void **)&t.sn, sn.size() * 4)))
      return cleanup(rc);
    (void)hipMemcpy(t.cs, cs.data(), cs.size() * 4, hipMemcpyHostToDevice);
    (void)hipMemcpy(t.sn, sn.data(), sn.size() * 4, hipMemcpyHostToDevice);
  }
  if (d.vocab > 0) {
    m->lm_blocks = d.vocab / 64;
    if ((rc = dmalloc(m, (void **)&m->arg_val, (size_t)m->lm_blocks * M * 4)) ||
        (rc = dmalloc(m, (void **)&m->arg_idx, (size_t)m->lm_blocks * M * 4)))
      return cleanup(rc);
  }
  if (!d.resident) {
    for (int s = 0; s < 2; ++s) {
      if ((rc = dmalloc(m, (void **)&m->slot[s], m->slot_bytes))) return cleanup(rc);
      (void)hipEventCreateWithFlags(&m->ev_free[s], hipEventDefault);
      (void)hipEventCreateWithFlags(&m->ev_ready[s], hipEventDefault);
    }
  }
  *out = m;
  return MS_OK;
}

static void drop_graphs(ms_model *m) {
  for (auto &g : m->graphs) (void)hipGraphExecDestroy(g.second);
  m->graphs.clear();
  for (auto &g : m->fgraphs) (void)hipGraphExecDestroy(g.second);
  m->fgraphs.clear();
  m->fwd_last = ms_model::FwdKey{};
}

extern "C" int ms_model_destroy(ms_model *m) {
  if (!m) return MS_OK;
  (void)hipStreamSynchronize(ctx().stream);
  (void)hipStreamSynchronize(ctx().copy_stream);
  drop_graphs(m);
  if (m->h_pos_pin) (void)hipHostFree(m->h_pos_pin);
  for (auto &Ly : m->L)
    for (int i = 0; i < 7; ++i)
      if (Ly.h_packed[i]) (void)hipHostFree(Ly.h_packed[i]);
  for (int s = 0; s < 2; ++s) {
    if (m->ev_free[s]) (void)hipEventDestroy(m->ev_free[s]);
    if (m->ev_ready[s]) (void)hipEventDestroy(m->ev_ready[s]);
  }
  for (void *p : m->allocs) (void)hipFree(p);
  delete m;
  return MS_OK;
}

extern "C" int ms_model_set_matrix(ms_model *m, int layer, int mat, const uint8_t *src,
                                   int src_on_device, float scale) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(m && src, "set_matrix: null argument");
  MS_CHECK_ARG(layer >= 0 && layer < (int)m->L.size(), "set_matrix: bad layer");
  MS_CHECK_ARG(mat >= 0 && mat < 7, "set_matrix: mat must be 0..6");
  MS_CHECK_ARG(scale > 0.f && std::isfinite(scale),
               "set_matrix: scale must be > 0 (TensorGuard, stream_runner.mojo:365-367)");
  Layer &Ly = m->L[layer];
  const int D = m->d.hidden, F = m->d.ffn;
  const int K[7] = {D, D, D, Ly.d.q_dim, D, D, F};
  const int N[7] = {Ly.d.q_dim, Ly.d.kv_dim, Ly.d.kv_dim, D, F, F, D};
  hipStream_t st = ctx().stream;
  if (m->d.resident || Ly.pinned) {
    if (!Ly.w[mat]) {
      int rc = dmalloc(m, (void **)&Ly.w[mat], Ly.bytes[mat]);
      if (rc) return rc;
    }
    const uint8_t *dsrc = src;
    void *tmp = nullptr;
    if (!src_on_device) {
      MS_HIP_TRY(hipMalloc(&tmp, Ly.bytes[mat]));
      MS_HIP_TRY(hipMemcpyAsync(tmp, src, Ly.bytes[mat], hipMemcpyHostToDevice, st));
      dsrc = static_cast<const uint8_t *>(tmp);
    }
    int rc = pack_device(Ly.w[mat], dsrc, K[mat], N[mat], st);
    if (tmp) {
      (void)hipStreamSynchronize(st);
      (void)hipFree(tmp);
    }
    if (rc) return rc;
  } else {
    if (!Ly.h_packed[mat])
      if (hipHostMalloc((void **)&Ly.h_packed[mat], Ly.bytes[mat], hipHostMallocDefault) !=
          hipSuccess)
        return fail(MS_E_NOMEM, "set_matrix: pinned allocation failed");
    if (src_on_device) {
      // pack on the device, then keep the packed bytes in pinned host memory
      void *tmp = nullptr;
      MS_HIP_TRY(hipMalloc(&tmp, Ly.bytes[mat]));
      int rc = pack_device(static_cast<uint8_t *>(tmp), src, K[mat], N[mat], st);
      if (rc == MS_OK &&
          hipMemcpyAsync(Ly.h_packed[mat], tmp, Ly.bytes[mat], hipMemcpyDeviceToHost, st) !=
              hipSuccess)
        rc = fail(MS_E_HIP, "set_matrix: copy of the packed weights to pinned memory failed");
      (void)hipStreamSynchronize(st);
      (void)hipFree(tmp);
      if (rc) return rc;
    } else if (int rc = ms_host_q4_pack(Ly.h_packed[mat], src, K[mat], N[mat])) {
      return rc;
    }
  }
  Ly.scale[mat] = scale;
  Ly.set_mask |= 1 << mat;
  drop_graphs(m);
  return MS_OK;
}

extern "C" int ms_model_set_pinned(ms_model *m, const uint8_t *pinned) {
  MS_CHECK_ARG(m && pinned, "set_pinned: null argument");
  MS_CHECK_ARG(!m->d.resident, "set_pinned: resident models keep every layer in HBM");
  for (size_t l = 0; l < m->L.size(); ++l)
    if ((pinned[l] != 0) != (m->L[l].pinned != 0) && m->L[l].set_mask)
      return fail(MS_E_STATE, "set_pinned: layer " + std::to_string(l) +
                                  " already has weights; pin layers before binding them");
  for (size_t l = 0; l < m->L.size(); ++l) m->L[l].pinned = pinned[l] != 0;
  return MS_OK;
}

extern "C" int ms_model_set_ple(ms_model *m, int layer, float ple) {
  MS_CHECK_ARG(m && layer >= 0 && layer < (int)m->L.size(), "set_ple: bad layer");
  MS_CHECK_ARG(ple > 0.f && std::isfinite(ple), "set_ple: PLE scale must be > 0");
  m->L[layer].ple = ple;
  drop_graphs(m);
  return MS_OK;
}

extern "C" int ms_model_get_desc(const ms_model *m, ms_model_desc *desc, ms_layer_desc *layers) {
  MS_CHECK_ARG(m && desc, "get_desc: null argument");
  *desc = m->d;
  if (layers)
    for (size_t l = 0; l < m->L.size(); ++l) layers[l] = m->L[l].d;
  return MS_OK;
}

extern "C" int ms_model_set_bos(ms_model *m, const float *h_bos) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(m, "set_bos: null model");
  m->bos = nullptr;
  if (!h_bos) return MS_OK;
  if (!m->bos_buf)
    if (int rc = dmalloc(m, (void **)&m->bos_buf, (size_t)m->d.hidden * 4)) return rc;
  MS_HIP_TRY(hipMemcpyAsync(m->bos_buf, h_bos, (size_t)m->d.hidden * 4, hipMemcpyHostToDevice,
                            ctx().stream));
  MS_HIP_TRY(hipStreamSynchronize(ctx().stream));
  m->bos = m->bos_buf;
  return MS_OK;
}

extern "C" int ms_model_set_lm_head(ms_model *m, const uint8_t *src, int src_on_device,
                                    float scale, const float *h_gamma) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(m && src, "set_lm_head: null argument");
  MS_CHECK_ARG(m->d.vocab > 0, "set_lm_head: model created with vocab = 0");
  MS_CHECK_ARG(scale > 0.f, "set_lm_head: scale must be > 0");
  const int D = m->d.hidden, V = m->d.vocab;
  const size_t bytes = (size_t)D * V / 2;
  hipStream_t st = ctx().stream;
  if (!m->lm_w)
    if (int rc = dmalloc(m, (void **)&m->lm_w, bytes)) return rc;
  const uint8_t *dsrc = src;
  void *tmp = nullptr;
  if (!src_on_device) {
    MS_HIP_TRY(hipMalloc(&tmp, bytes));
    MS_HIP_TRY(hipMemcpyAsync(tmp, src, bytes, hipMemcpyHostToDevice, st));
    dsrc = static_cast<const uint8_t *>(tmp);
  }
  int rc = pack_device(m->lm_w, dsrc, D, V, st);
  if (tmp) {
    (void)hipStreamSynchronize(st);
    (void)hipFree(tmp);
  }
  if (rc) return rc;
  if (h_gamma) {
    if (!m->gamma)
      if (int r = dmalloc(m, (void **)&m->gamma, (size_t)D * 4)) return r;
    MS_HIP_TRY(hipMemcpyAsync(m->gamma, h_gamma, (size_t)D * 4, hipMemcpyHostToDevice, st));
    MS_HIP_TRY(hipStreamSynchronize(st));
  }
  m->lm_scale = scale;
  m->has_lm = true;
  drop_graphs(m);
  return MS_OK;
}

// Buffers of the logits-based pick (sampler, FP32 head), once per model.
static int alloc_pick(ms_model *m) {
  const size_t S = (size_t)m->d.max_seqs;
  if (!m->logits)
    if (int rc = dmalloc(m, (void **)&m->logits, S * m->d.vocab * 4)) return rc;
  if (!m->samp_ids)
    if (int rc = dmalloc(m, (void **)&m->samp_ids, S * 4)) return rc;
  return MS_OK;
}

extern "C" int ms_model_set_lm_head_f32(ms_model *m, const float *src, int src_on_device,
                                        const float *h_gamma) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(m && src, "set_lm_head_f32: null argument");
  MS_CHECK_ARG(m->d.vocab > 0 && m->d.vocab % 16 == 0,
               "set_lm_head_f32: model vocab must be a positive multiple of 16");
  const size_t D = (size_t)m->d.hidden, V = (size_t)m->d.vocab, S = (size_t)m->d.max_seqs;
  hipStream_t st = ctx().stream;
  if (!m->lm_f32) {
    if (int rc = dmalloc(m, (void **)&m->lm_f32, D * V * 4)) return rc;
    if (int rc = dmalloc(m, (void **)&m->lm_y, S * D * 4)) return rc;
    if (int rc = dmalloc(m, (void **)&m->lm_part, mm_f32_part_floats((int)S, (int)V) * 4))
      return rc;
  }
  if (int rc = alloc_pick(m)) return rc;
  MS_HIP_TRY(hipMemcpyAsync(m->lm_f32, src, D * V * 4,
                            src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, st));
  if (h_gamma) {
    if (!m->gamma)
      if (int r = dmalloc(m, (void **)&m->gamma, D * 4)) return r;
    MS_HIP_TRY(hipMemcpyAsync(m->gamma, h_gamma, D * 4, hipMemcpyHostToDevice, st));
  }
  MS_HIP_TRY(hipStreamSynchronize(st));
  m->has_lm = true;
  drop_graphs(m);
  return MS_OK;
}

extern "C" int ms_model_reset(ms_model *m) {
  MS_CHECK_ARG(m, "reset: null model");
  std::fill(m->h_pos.begin(), m->h_pos.end(), 0);
  // positions restart at 0; stale cache contents are never read (every read
  // position < the current position has been rewritten since the reset).
  // The decode attention's chunk counters are left zero by every completed
  // launch; clearing them here also recovers from an interrupted one.
  if (int rc = require_init()) return rc;
  MS_HIP_TRY(hipMemset(m->attn_ctr, 0, attn_ctr_count(m->d.max_seqs, m->nkv_max) * 4));
  if (m->shist_n) MS_HIP_TRY(hipMemset(m->shist_n, 0, (size_t)m->d.max_seqs * 4));
  std::fill(m->h_hist_n.begin(), m->h_hist_n.end(), 0);
  if (m->samp_ctr) MS_HIP_TRY(hipMemset(m->samp_ctr, 0, 4));
  return MS_OK;
}

extern "C" int ms_model_set_sampling(ms_model *m, float temperature, float penalty,
                                     uint64_t seed) {
  MS_CHECK_ARG(m, "set_sampling: null model");
  MS_CHECK_ARG(temperature == temperature && penalty == penalty,
               "set_sampling: temperature and penalty must be numbers");
  MS_CHECK_ARG(m->has_lm, "set_sampling: the model has no LM head");
  if (int rc = require_init()) return rc;
  const bool on = temperature > 0.01f || penalty > 1.0f;
  if (on && !m->shist) {
    const size_t S = (size_t)m->d.max_seqs;
    if (int rc = alloc_pick(m)) return rc;
    if (int rc = dmalloc(m, (void **)&m->shist, S * kSampleMaxHistory * 4)) return rc;
    if (int rc = dmalloc(m, (void **)&m->shist_n, S * 4)) return rc;
    if (int rc = dmalloc(m, (void **)&m->samp_ctr, 4)) return rc;
    MS_HIP_TRY(hipMemset(m->shist_n, 0, S * 4));
    std::fill(m->h_hist_n.begin(), m->h_hist_n.end(), 0);
  }
  if (m->samp_ctr) MS_HIP_TRY(hipMemset(m->samp_ctr, 0, 4));
  m->sampling = on;
  m->samp_temp = temperature;
  m->samp_pen = penalty;
  m->samp_seed = seed;
  drop_graphs(m);  // the captured step holds the former choice
  return MS_OK;
}

// A captured step serves every step whose positions lie below its bound: the
// end of the kBoundBucket-position bucket of the step's largest position.
// Its attention launches the key chunks below the bound only and loads them
// before the position arrives; a step's unattended loads stay under one
// bucket of cache rows.
constexpr int kBoundBucket = 64;
constexpr size_t kMaxGraphs = 16;
static int decode_bound(int max_pos) { return (max_pos / kBoundBucket + 1) * kBoundBucket; }

static int forward_impl(ms_model *m, int first, int count, float *d_x, int B, int T,
                        const int *h_base, float *d_hidden) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(m && d_x && h_base, "forward: null argument");
  MS_CHECK_ARG(B >= 1 && B <= m->d.max_seqs && T >= 1 && T <= m->d.max_rows,
               "forward: n_seqs/T exceed the model's max_seqs/max_rows");
  if (int rc = check_ready(m, false)) return rc;
  if (int rc = check_positions(m, h_base, B, T, 0)) return rc;
  hipStream_t st = ctx().stream;
  // positions from pinned staging: the copy needs no host wait (the call ends
  // with one, so the staging is free again by the next call)
  for (int b = 0; b < B; ++b) m->h_pos_pin[b] = h_base[b];
  MS_HIP_TRY(hipMemcpyAsync(m->pos, m->h_pos_pin, sizeof(int32_t) * B, hipMemcpyHostToDevice,
                            st));
  m->stats = ms_stream_stats{};
  RunCfg rc{};
  rc.B = B;
  rc.T = T;
  rc.in_rows = d_x;
  rc.out_rows = d_x;
  rc.hidden = d_hidden;
  rc.first_layer = first;
  rc.n_layers = count;
  rc.plan_pos = h_base[0];
  for (int b = 0; b < B; ++b) rc.pos_bound = std::max(rc.pos_bound, h_base[b] + T);
  // A whole-model call of a resident model with decode-sized rows replays a
  // HIP graph once the same call (buffers, rows, position bucket) has come
  // twice in a row: the harness loop's steps.  The attention's key-chunk
  // bound is baked into a graph, so the key holds the decode graphs'
  // 64-position bucket of the call's largest position and the captured
  // launches cover the whole bucket.
  const bool graphable = m->forward_graphs && m->d.resident && !g_prof.on && first == 0 &&
                         count == (int)m->L.size() && T <= kGemvMaxM;
  ms_model::FwdKey key{};
  if (graphable) {
    key.x = d_x;
    key.hidden = d_hidden;
    key.B = B;
    key.T = T;
    key.bound = decode_bound(rc.pos_bound - 1);
    rc.pos_bound = key.bound;
  }
  hipGraphExec_t ge = nullptr;
  if (graphable)
    for (auto &g : m->fgraphs)
      if (g.first == key) ge = g.second;
  if (!ge && graphable && key == m->fwd_last) {
    if (m->fgraphs.size() >= kMaxGraphs) {
      MS_HIP_TRY(hipStreamSynchronize(st));
      (void)hipGraphExecDestroy(m->fgraphs.front().second);
      m->fgraphs.erase(m->fgraphs.begin());
    }
    hipGraph_t g;
    MS_HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    int r = run_layers(m, rc, st);
    if (r == MS_OK) r = enqueue_output(m, rc, st);
    const hipError_t e = hipStreamEndCapture(st, &g);
    if (r) return r;
    if (e != hipSuccess) return fail(MS_E_HIP, "forward graph capture failed");
    const hipError_t ei = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    MS_HIP_TRY(ei);
    m->fgraphs.emplace_back(key, ge);
  }
  if (ge) {
    MS_HIP_TRY(hipGraphLaunch(ge, st));
  } else {
    if (graphable) m->fwd_last = key;
    if (int r = run_layers(m, rc, st)) return r;
    if (int r = enqueue_output(m, rc, st)) return r;
  }
  MS_HIP_TRY(hipStreamSynchronize(st));
  for (int b = 0; b < B; ++b) m->h_pos[b] = h_base[b] + T;
  return MS_OK;
}

extern "C" int ms_layer_forward(ms_model *m, int layer, float *d_x, int n_seqs, int T,
                                const int *h_base) {
  MS_CHECK_ARG(m && layer >= 0 && layer < (int)m->L.size(), "layer_forward: bad layer");
  return forward_impl(m, layer, 1, d_x, n_seqs, T, h_base, nullptr);
}

extern "C" int ms_forward(ms_model *m, float *d_x, int n_seqs, int T, const int *h_base,
                          float *d_hidden) {
  MS_CHECK_ARG(m, "forward: null model");
  return forward_impl(m, 0, (int)m->L.size(), d_x, n_seqs, T, h_base, d_hidden);
}

// ---- decode --------------------------------------------------------------------
// pos_bound: every sequence's position in this step is below it.
static int enqueue_decode_step(ms_model *m, int B, int pos_bound, hipStream_t st) {
  const int D = m->d.hidden;
  {
    ProfScope ps(PC_PREP, (double)D * B / 2, st);
    const int rc = m->lm_f32
                       ? launch_embed_f32(m->lm_f32, D, m->d.vocab, m->tok, B, m->x_in, st)
                       : launch_embed(m->lm_w, D, m->d.vocab, m->lm_scale, m->tok, B, m->x_in, st);
    if (rc) return rc;
  }
  RunCfg rc{};
  rc.B = B;
  rc.T = 1;
  rc.in_rows = m->x_in;
  rc.first_layer = 0;
  rc.n_layers = (int)m->L.size();
  rc.hidden = m->tap_hidden;
  rc.pos_bound = pos_bound;
  rc.one_row = B == 1;
  if (int r = run_layers(m, rc, st)) return r;
  ArgmaxFin f{};
  f.tok_state = m->tok;
  f.pos_state = m->pos;
  f.ids_hist = m->ids_hist;
  f.step = m->step;
  return enqueue_lm(m, rc, 0, B, f, st);
}



static int decode_graph(ms_model *m, int B, int bound, hipStream_t st, hipGraphExec_t *out) {
  if (m->g_nseq != B) {
    drop_graphs(m);
    m->g_nseq = B;
  }
  for (auto &g : m->graphs)
    if (g.first == bound) {
      *out = g.second;
      return MS_OK;
    }
  // a new bound: capture one step while earlier launches run (capture records
  // work, it runs none); an evicted graph may still be in flight, so the
  // stream drains before it is destroyed
  if (m->graphs.size() >= kMaxGraphs) {
    MS_HIP_TRY(hipStreamSynchronize(st));
    (void)hipGraphExecDestroy(m->graphs.front().second);
    m->graphs.erase(m->graphs.begin());
  }
  hipGraph_t g;
  MS_HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  const int rc = enqueue_decode_step(m, B, bound, st);
  const hipError_t e = hipStreamEndCapture(st, &g);
  if (rc) return rc;
  if (e != hipSuccess) return fail(MS_E_HIP, "decode graph capture failed");
  hipGraphExec_t ge = nullptr;
  const hipError_t ei = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  MS_HIP_TRY(ei);
  m->graphs.emplace_back(bound, ge);
  *out = ge;
  return MS_OK;
}

extern "C" int ms_decode_begin(ms_model *m, int n_seqs, const int32_t *h_tokens,
                               const int32_t *h_pos) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(m && h_tokens && h_pos, "decode_begin: null argument");
  MS_CHECK_ARG(n_seqs >= 1 && n_seqs <= m->d.max_seqs, "decode_begin: bad n_seqs");
  MS_CHECK_ARG(m->d.vocab > 0, "decode_begin: model has no LM head");
  for (int b = 0; b < n_seqs; ++b)
    MS_CHECK_ARG(h_tokens[b] >= 0 && h_tokens[b] < m->d.vocab, "decode_begin: bad token id");
  hipStream_t st = ctx().stream;
  MS_HIP_TRY(hipMemcpyAsync(m->tok, h_tokens, 4 * n_seqs, hipMemcpyHostToDevice, st));
  MS_HIP_TRY(hipMemcpyAsync(m->pos, h_pos, 4 * n_seqs, hipMemcpyHostToDevice, st));
  MS_HIP_TRY(hipStreamSynchronize(st));
  for (int b = 0; b < n_seqs; ++b) m->h_pos[b] = h_pos[b];
  m->dec_nseq = n_seqs;
  return MS_OK;
}

extern "C" int ms_decode_run(ms_model *m, int n_steps, int use_graph, int32_t *h_ids_out) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(m && n_steps >= 0, "decode_run: bad arguments");
  MS_CHECK_ARG(m->dec_nseq >= 1, "decode_run: call ms_decode_begin first");
  if (int rc = check_ready(m, true)) return rc;
  const int B = m->dec_nseq;
  if (int rc = check_positions(m, m->h_pos.data(), B, 1, n_steps - 1)) return rc;
  if (m->sampling)
    for (int b = 0; b < B; ++b)
      MS_CHECK_ARG(m->h_hist_n[b] + n_steps <= kSampleMaxHistory,
                   "decode_run: the repetition-penalty history of a sequence would exceed "
                   "8192 ids (prompt + generated); reset the model first");
  if (!m->d.resident) use_graph = 0;  // streaming runs eagerly (host-side slot logic)
  m->stats = ms_stream_stats{};
  hipStream_t st = ctx().stream;
  int p0 = 0;  // largest position of the first step
  for (int b = 0; b < B; ++b) p0 = std::max(p0, m->h_pos[b]);
  int done = 0;
  while (done < n_steps) {
    const int chunk = std::min(n_steps - done, m->hist_cap);
    MS_HIP_TRY(hipMemsetAsync(m->step, 0, 4, st));
    for (int s = 0; s < chunk; ++s) {
      const int p = p0 + done + s;
      if (use_graph) {
        hipGraphExec_t g = nullptr;
        if (int rc = decode_graph(m, B, decode_bound(p), st, &g)) return rc;
        MS_HIP_TRY(hipGraphLaunch(g, st));
      } else if (int rc = enqueue_decode_step(m, B, p + 1, st)) {
        return rc;
      }
    }
    if (h_ids_out)
      MS_HIP_TRY(hipMemcpyAsync(h_ids_out + (size_t)done * B, m->ids_hist,
                                (size_t)chunk * B * 4, hipMemcpyDeviceToHost, st));
    MS_HIP_TRY(hipStreamSynchronize(st));
    done += chunk;
  }
  if (g_prof.on) prof_collect();
  for (int b = 0; b < B; ++b) {
    m->h_pos[b] += n_steps;
    if (m->sampling) m->h_hist_n[b] += n_steps;
  }
  return MS_OK;
}

extern "C" int ms_prefill(ms_model *m, int seq, const int32_t *h_tokens, int n_tokens,
                          int pos0, int32_t *h_first_id) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(m && h_tokens && n_tokens >= 1, "prefill: bad arguments");
  MS_CHECK_ARG(seq >= 0 && seq < m->d.max_seqs, "prefill: bad sequence index");
  MS_CHECK_ARG(m->d.vocab > 0, "prefill: model has no LM head");
  if (int rc = check_ready(m, true)) return rc;
  for (int i = 0; i < n_tokens; ++i)
    MS_CHECK_ARG(h_tokens[i] >= 0 && h_tokens[i] < m->d.vocab, "prefill: token id out of range");
  // the prompt ids open the sequence's penalty history
  // (gemma4_e4b_infer.mojo:134-139,157-161); the history holds at most
  // kSampleMaxHistory ids (prompt, the first draw, then one per step)
  if (m->sampling)
    MS_CHECK_ARG(n_tokens + 1 <= kSampleMaxHistory,
                 "prefill: with sampling on, the prompt and the first draw must fit the "
                 "8192-id repetition-penalty history");
  hipStream_t st = ctx().stream;
  const int D = m->d.hidden;
  // rows per chunk: the prefill workspace (projections as GEMMs)
  const int T = std::max(m->d.max_rows, m->prefill_rows);
  int32_t *dtok = nullptr;
  MS_HIP_TRY(hipMallocAsync((void **)&dtok, (size_t)n_tokens * 4, st));
  MS_HIP_TRY(hipMemcpyAsync(dtok, h_tokens, (size_t)n_tokens * 4, hipMemcpyHostToDevice, st));
  if (m->sampling) {
    const int nh = n_tokens;
    MS_HIP_TRY(hipMemcpyAsync(m->shist + (size_t)seq * kSampleMaxHistory, dtok, (size_t)nh * 4,
                              hipMemcpyDeviceToDevice, st));
    MS_HIP_TRY(hipMemcpyAsync(m->shist_n + seq, &nh, 4, hipMemcpyHostToDevice, st));
    MS_HIP_TRY(hipStreamSynchronize(st));  // nh is a local
  }
  m->stats = ms_stream_stats{};
  int rcode = MS_OK;
  std::vector<int32_t> sub;
  for (int c0 = 0; c0 < n_tokens && rcode == MS_OK; c0 += T) {
    const int t = std::min(T, n_tokens - c0);
    const int base = pos0 + c0;
    if ((rcode = check_positions(m, &base, 1, t, 0))) break;
    MS_HIP_TRY(hipMemcpyAsync(m->pos + seq, &base, 4, hipMemcpyHostToDevice, st));
    // base position of each attention row group of the chunk
    sub.clear();
    for (int r0 = 0; r0 < t; r0 += kPrefillAttnRows) sub.push_back(base + r0);
    MS_HIP_TRY(hipMemcpyAsync(m->ppos, sub.data(), sub.size() * 4, hipMemcpyHostToDevice, st));
    MS_HIP_TRY(hipStreamSynchronize(st));  // `sub` is reused by the next chunk
    if ((rcode = m->lm_f32 ? launch_embed_f32(m->lm_f32, D, m->d.vocab, dtok + c0, t, m->x_in, st)
                           : launch_embed(m->lm_w, D, m->d.vocab, m->lm_scale, dtok + c0, t,
                                          m->x_in, st)))
      break;
    if (m->bos && base == 0)
      MS_HIP_TRY(hipMemcpyAsync(m->x_in, m->bos, (size_t)D * 4, hipMemcpyDeviceToDevice, st));
    RunCfg rc{};
    rc.B = 1;
    rc.T = t;
    rc.in_rows = m->x_in;
    rc.seq0 = seq;
    rc.first_layer = 0;
    rc.n_layers = (int)m->L.size();
    rc.plan_pos = base;
    rc.pos_bound = base + t;
    if (c0 + t >= n_tokens) rc.tap_last = m->tap_hidden;
    if ((rcode = run_layers(m, rc, st))) break;
    if (c0 + t >= n_tokens) {
      // LM head on the last prompt row only
      ArgmaxFin f{};
      f.ids_out = m->tok + seq;
      if ((rcode = enqueue_lm(m, rc, t - 1, 1, f, st))) break;
    }
  }
  (void)hipFreeAsync(dtok, st);
  if (rcode) return rcode;
  int32_t id = 0;
  MS_HIP_TRY(hipMemcpyAsync(&id, m->tok + seq, 4, hipMemcpyDeviceToHost, st));
  MS_HIP_TRY(hipStreamSynchronize(st));
  if (h_first_id) *h_first_id = id;
  m->h_pos[seq] = pos0 + n_tokens;
  if (m->sampling) m->h_hist_n[seq] = n_tokens + 1;
  return MS_OK;
}

extern "C" int ms_model_set_forward_graphs(ms_model *m, int on) {
  MS_CHECK_ARG(m, "set_forward_graphs: null model");
  m->forward_graphs = on != 0;
  drop_graphs(m);
  return MS_OK;
}

extern "C" int ms_model_set_taps(ms_model *m, float *d_hidden, float *d_logits) {
  MS_CHECK_ARG(m, "set_taps: null model");
  MS_CHECK_ARG(!d_logits || m->d.vocab > 0, "set_taps: logits need an LM head");
  m->tap_hidden = d_hidden;
  m->tap_logits = d_logits;
  drop_graphs(m);  // the captured step holds the former targets
  return MS_OK;
}

extern "C" int ms_model_read_kv(ms_model *m, int layer, int seq, int pos0, int n, float *d_k,
                                float *d_v) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(m && layer >= 0 && layer < (int)m->L.size(), "read_kv: bad layer");
  MS_CHECK_ARG(seq >= 0 && seq < m->d.max_seqs, "read_kv: bad sequence");
  MS_CHECK_ARG(pos0 >= 0 && n >= 0 && (d_k || d_v), "read_kv: bad range");
  const Layer &Ly = m->L[layer];
  const int L = Ly.d.cache_len;
  const bool circ = Ly.d.cache_kind == MS_CACHE_CIRCULAR;
  MS_CHECK_ARG(circ ? n <= L : pos0 + n <= L, "read_kv: positions outside the cache");
  const size_t row = (size_t)Ly.d.kv_dim * 4;
  hipStream_t st = ctx().stream;
  const float *kb = Ly.kc + (size_t)seq * Ly.cache_seq_stride;
  const float *vb = Ly.vc + (size_t)seq * Ly.cache_seq_stride;
  // slot of position p: p % window (circular, write_kv_sliding) or p (linear)
  for (int i = 0; i < n;) {
    const int slot = circ ? (pos0 + i) % L : pos0 + i;
    const int run = std::min(n - i, L - slot);  // rows contiguous in the cache
    if (d_k)
      MS_HIP_TRY(hipMemcpyAsync(d_k + (size_t)i * Ly.d.kv_dim, kb + (size_t)slot * Ly.d.kv_dim,
                                (size_t)run * row, hipMemcpyDeviceToDevice, st));
    if (d_v)
      MS_HIP_TRY(hipMemcpyAsync(d_v + (size_t)i * Ly.d.kv_dim, vb + (size_t)slot * Ly.d.kv_dim,
                                (size_t)run * row, hipMemcpyDeviceToDevice, st));
    i += run;
  }
  MS_HIP_TRY(hipStreamSynchronize(st));
  return MS_OK;
}

extern "C" int ms_model_stream_stats(ms_model *m, ms_stream_stats *out) {
  MS_CHECK_ARG(m && out, "stream_stats: null argument");
  *out = m->stats;
  return MS_OK;
}

extern "C" int ms_prof_enable(int on) {
  g_prof.on = on != 0;
  for (int i = 0; i < MS_PROF_CLASSES; ++i) {
    g_prof.launches[i] = 0;
    g_prof.ms[i] = 0;
    g_prof.bytes[i] = 0;
  }
  return MS_OK;
}

extern "C" int ms_prof_get(int cls, const char **name, long *launches, double *total_ms,
                           double *bytes) {
  MS_CHECK_ARG(cls >= 0 && cls < MS_PROF_CLASSES, "prof_get: bad class");
  if (g_prof.on && !g_prof.pending.empty()) prof_collect();
  if (name) *name = kProfNames[cls];
  if (launches) *launches = g_prof.launches[cls];
  if (total_ms) *total_ms = g_prof.ms[cls];
  if (bytes) *bytes = g_prof.bytes[cls];
  return MS_OK;
}

// Decode attention re-launched back to back over every layer of the recorded
// launch's cache kind (circular if one was recorded, else linear) and head
// size, each on its own layer's cache of the recorded sequences.  The
// launches attend the recorded fresh row without appending it (write_cache
// 0), so the caches are left as they were.  Bytes: the K and V rows of every
// attended key (the fresh one read from the projection rows).
static int attn_sweep(ms_model *m, int passes, double *avg_us, double *bytes_per_launch,
                      long *launches) {
  const int k = g_prof.have_attn[1] ? 1 : 0;
  MS_CHECK_ARG(g_prof.have_attn[k], "prof_sweep: no decode attention recorded while profiling");
  MS_CHECK_ARG(m->d.resident, "prof_sweep: resident models only");
  const AttnArgs base = g_prof.last_attn[k];
  std::vector<int> layers;
  for (int l = 0; l < (int)m->L.size(); ++l)
    if ((m->L[l].d.cache_kind == MS_CACHE_CIRCULAR) == (k == 1) &&
        m->L[l].d.head_dim == m->L[g_prof.last_attn_layer[k]].d.head_dim)
      layers.push_back(l);
  if (passes < 0) layers.assign(-passes, g_prof.last_attn_layer[k]);
  if (passes < 0) passes = 1;
  const Layer &Lr = m->L[g_prof.last_attn_layer[k]];
  const size_t seq0 = (size_t)(base.kc - Lr.kc) / Lr.cache_seq_stride;
  hipStream_t st = ctx().stream;
  std::vector<int32_t> pos(base.B);
  MS_HIP_TRY(hipMemcpyAsync(pos.data(), base.pos, 4 * base.B, hipMemcpyDeviceToHost, st));
  MS_HIP_TRY(hipStreamSynchronize(st));
  hipEvent_t e0, e1;
  MS_HIP_TRY(hipEventCreate(&e0));
  MS_HIP_TRY(hipEventCreate(&e1));
  double bytes = 0;
  long n = 0;
  int rc = MS_OK;
  if (g_prof.attn_part[k]) {
    // the RoPE factors of the swept layers (one table for the kind)
    AttnArgs a = base;
    a.cos_t = m->ropes[Lr.rope].cs;
    a.sin_t = m->ropes[Lr.rope].sn;
    if ((rc = launch_rope_cur(a, st))) return rc;
  }
  MS_HIP_TRY(hipEventRecord(e0, st));
  for (int p = 0; p < passes && rc == MS_OK; ++p)
    for (int l : layers) {
      const Layer &Ly = m->L[l];
      AttnArgs a = base;
      a.kc = Ly.kc + seq0 * Ly.cache_seq_stride;
      a.vc = Ly.vc + seq0 * Ly.cache_seq_stride;
      a.cos_t = m->ropes[Ly.rope].cs;
      a.sin_t = m->ropes[Ly.rope].sn;
      a.n_chunks = Ly.n_chunks;
      a.cache_len = Ly.d.cache_len;
      a.clamp = Ly.d.clamp_reads;
      a.write_cache = 0;
      if ((rc = g_prof.attn_part[k] ? launch_attention_partials(a, st)
                                     : launch_attention(a, st)))
        break;
      for (int b = 0; b < a.B; ++b) {
        const int keys = std::min(pos[b] + 1, Ly.d.cache_len);
        bytes += 2.0 * keys * Ly.d.kv_dim * 4;
      }
      ++n;
    }
  (void)hipEventRecord(e1, st);
  (void)hipEventSynchronize(e1);
  float ms = 0.f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (rc) return rc;
  *avg_us = n ? (double)ms * 1e3 / n : 0.0;
  if (bytes_per_launch) *bytes_per_launch = n ? bytes / n : 0.0;
  if (launches) *launches = n;
  return MS_OK;
}

extern "C" int ms_prof_sweep(ms_model *m, int cls, int passes, double *avg_us,
                             double *bytes_per_launch, long *launches) {
  if (int rc = require_init()) return rc;
  MS_CHECK_ARG(m && avg_us && passes != 0, "prof_sweep: bad arguments");
  MS_CHECK_ARG(cls == PC_QKV || cls == PC_ATTN || cls == PC_O || cls == PC_GATEUP ||
                   cls == PC_DOWN,
               "prof_sweep: class must be a layer projection or attention");
  if (cls == PC_ATTN) return attn_sweep(m, passes, avg_us, bytes_per_launch, launches);
  MS_CHECK_ARG(g_prof.have[cls], "prof_sweep: no launch of this class recorded while profiling");
  MS_CHECK_ARG(m->d.resident, "prof_sweep: resident models only");
  const GemvArgs base = g_prof.last[cls];
  const ms_layer_desc &d0 = m->L[g_prof.last_layer[cls]].d;
  // matrices of each class: Q|K|V (0,1,2), O (3), Gate|Up (4,5), Down (6)
  std::vector<int> layers;
  for (int l = 0; l < (int)m->L.size(); ++l) {
    const ms_layer_desc &d = m->L[l].d;
    // Gate|Up and Down shapes are the same in every layer
    const bool same = (cls == PC_GATEUP || cls == PC_DOWN) ||
                      (d.q_dim == d0.q_dim && d.kv_dim == d0.kv_dim);
    if (same) layers.push_back(l);
  }
  // passes < 0: the recorded layer only, -passes times (its weights stay in
  // the caches after the first launch: the cache-hot duration)
  if (passes < 0) layers.assign(-passes, g_prof.last_layer[cls]);
  if (passes < 0) passes = 1;
  hipStream_t st = ctx().stream;
  hipEvent_t e0, e1;
  MS_HIP_TRY(hipEventCreate(&e0));
  MS_HIP_TRY(hipEventCreate(&e1));
  double bytes = 0;
  long n = 0;
  int rc = MS_OK;
  MS_HIP_TRY(hipEventRecord(e0, st));
  for (int p = 0; p < passes && rc == MS_OK; ++p)
    for (int l : layers) {
      Layer &Ly = m->L[l];
      GemvArgs a = base;
      if (cls == PC_QKV) {
        for (int i = 0; i < 3; ++i) a.seg[i].w = Ly.w[i], a.seg[i].scale = Ly.scale[i];
      } else if (cls == PC_O) {
        a.seg[0].w = Ly.w[3], a.seg[0].scale = Ly.scale[3];
      } else if (cls == PC_GATEUP) {
        a.seg[0].w = Ly.w[4], a.seg[0].scale = Ly.scale[4];
        a.seg[1].w = Ly.w[5], a.seg[1].scale = Ly.scale[5];
      } else {
        a.seg[0].w = Ly.w[6], a.seg[0].scale = Ly.scale[6];
      }
      if ((rc = launch_gemv(a, st))) break;
      double b = 0;
      for (int i = 0; i < a.nseg; ++i) b += (double)a.K * a.seg[i].n_cols / 2;
      bytes += b;
      ++n;
    }
  (void)hipEventRecord(e1, st);
  (void)hipEventSynchronize(e1);
  float ms = 0.f;
  (void)hipEventElapsedTime(&ms, e0, e1);
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  if (rc) return rc;
  *avg_us = n ? (double)ms * 1e3 / n : 0.0;
  if (bytes_per_launch) *bytes_per_launch = n ? bytes / n : 0.0;
  if (launches) *launches = n;
  return MS_OK;
}
