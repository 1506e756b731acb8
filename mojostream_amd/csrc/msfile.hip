// .mojostream weight files on the host.
//
// Format (little-endian; create_fake_model.py:11-38, convert.py:362-413):
//   header 128 B: "MOJOSTRM", u32 version, u32 format tag, u32 n_layers,
//     hidden, kv_dim, ffn_dim, n_heads, n_kv_heads, u64 n_tensors,
//     u64 dir_offset (=128), u64 data_start; format tag 2 adds the Engram
//     extension at byte 64: "ENGR", u32 version, n_kv_shared, sliding_kv_dim,
//     full_kv_dim, ple_dim, sliding_window.
//   directory n_tensors x 32 B: u32 layer, u32 type (0 PLE, 1..7 = Q K V O
//     Gate Up Down), u32 rows, u32 cols, f32 scale, u32 flags, u64 offset.
//   data: each matrix rows*cols/2 row-major Q4 bytes at a 4096-aligned offset.
//
// The reader keeps the whole file in one host buffer (MojoStreamFile,
// mojostream.mojo:95-219).  Unlike the reference it checks that the header
// and directory lie inside the file before parsing them.
//
// Guards.  The reference has two ShapeGuards (mojostream.mojo:190-219 and
// stream_runner.mojo:280-309) and one TensorGuard (stream_runner.mojo:313-380)
// whose expected shapes assume one head size for every layer, so they reject
// E4B files (sliding layers hd 256, full layers hd 512).  The guards here take
// the head size per layer type: a file with the Engram extension and
// full_kv_dim != sliding_kv_dim is hybrid, with full-attention layers at
// (layer+1) % 6 == 0 (is_full_attn, gemma4_e4b.mojo:60-63) unless the caller
// sets another map.
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "common.h"

struct ms_file {
  std::vector<uint8_t> raw;
  ms_file_meta meta{};
  std::vector<ms_file_entry> dir;
  std::vector<uint8_t> is_full;
};

namespace ms {
namespace {

constexpr int kHdr = 128, kDirEntry = 32, kPage = 4096, kPerLayer = 8;
const char *kMatNames[kPerLayer] = {"PLE", "Q", "K", "V", "O", "Gate", "Up", "Down"};

template <class T>
T rd(const uint8_t *p) {
  T v;
  memcpy(&v, p, sizeof(T));
  return v;
}
template <class T>
void wr(uint8_t *p, T v) {
  memcpy(p, &v, sizeof(T));
}

bool hybrid(const ms_file_meta &m) {
  return m.engram_version != 0 && m.full_kv_dim != 0 && m.full_kv_dim != m.sliding_kv_dim;
}

void default_types(ms_file *f) {
  f->is_full.assign(f->meta.n_layers, 0);
  if (hybrid(f->meta))
    for (uint32_t l = 0; l < f->meta.n_layers; ++l) f->is_full[l] = (l + 1) % 6 == 0;
}

// Per-layer head size and projection widths (get_layer_dims, convert.py:195-225).
void layer_dims(const ms_file_meta &m, bool full, ms_file_layer *o) {
  const uint32_t kv = full ? m.full_kv_dim : (m.engram_version ? m.sliding_kv_dim : m.kv_dim);
  o->is_full = full ? 1 : 0;
  o->kv_dim = (int)kv;
  o->head_dim = m.n_kv_heads ? (int)(kv / m.n_kv_heads) : 0;
  o->q_dim = (int)m.n_heads * o->head_dim;
}

void expected(const ms_file_meta &m, const ms_file_layer &ld, int type, uint32_t *r,
              uint32_t *c) {
  const uint32_t D = m.hidden, F = m.ffn_dim, Q = ld.q_dim, KV = ld.kv_dim;
  const uint32_t er[kPerLayer] = {1, D, D, D, Q, D, D, F};
  const uint32_t ec[kPerLayer] = {0, Q, KV, KV, D, F, F, D};
  *r = er[type];
  *c = ec[type];
}

// Synthetic weight streams, shared with the Python synthetic-model helpers:
// matrix stream (layer+1)*16 + (type-1), scale U(0.04,0.15) on stream 0x5CA1E,
// PLE U(0.8,1.2) on stream 0x91E (create_fake_model.py:95,203).
uint64_t matrix_stream(int layer, int type) { return (uint64_t)(layer + 1) * 16 + (type - 1); }
constexpr uint64_t kScaleStream = 0x5CA1E, kPleStream = 0x91E, kLmStream = 0xFFFF,
                   kBosStream = 0xB05, kGammaStream = 0x6A44A;

int io_fail(const std::string &msg) { return fail(MS_E_IO, msg); }

}  // namespace
}  // namespace ms

using namespace ms;

extern "C" int ms_file_open(const char *path, ms_file **out) {
  MS_CHECK_ARG(path && out, "file_open: null argument");
  *out = nullptr;
  auto t0 = std::chrono::steady_clock::now();
  FILE *fp = fopen(path, "rb");
  if (!fp) return io_fail(std::string(".mojostream: cannot open ") + path);
  ms_file *f = new ms_file();
  fseek(fp, 0, SEEK_END);
  long sz = ftell(fp);
  fseek(fp, 0, SEEK_SET);
  if (sz > 0) {
    f->raw.resize((size_t)sz);
    if (fread(f->raw.data(), 1, (size_t)sz, fp) != (size_t)sz) {
      fclose(fp);
      delete f;
      return io_fail(std::string(".mojostream: short read of ") + path);
    }
  }
  fclose(fp);
  auto t1 = std::chrono::steady_clock::now();
  ms_file_meta &m = f->meta;
  m.file_bytes = f->raw.size();
  m.load_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
  const uint8_t *b = f->raw.data();
  if (f->raw.size() < (size_t)kHdr) {
    delete f;
    return io_fail(".mojostream: file shorter than the 128-byte header");
  }
  // Magic: the reference compares the first four bytes with "MOJO".
  if (memcmp(b, "MOJO", 4) != 0) {
    delete f;
    return io_fail(".mojostream: invalid magic (expected 'MOJO...')");
  }
  m.version = rd<uint32_t>(b + 8);
  m.format_tag = rd<uint32_t>(b + 12);
  m.n_layers = rd<uint32_t>(b + 16);
  m.hidden = rd<uint32_t>(b + 20);
  m.kv_dim = rd<uint32_t>(b + 24);
  m.ffn_dim = rd<uint32_t>(b + 28);
  m.n_heads = rd<uint32_t>(b + 32);
  m.n_kv_heads = rd<uint32_t>(b + 36);
  m.n_tensors = rd<uint64_t>(b + 40);
  m.dir_offset = rd<uint64_t>(b + 48);
  m.data_start = rd<uint64_t>(b + 56);
  if (memcmp(b + 64, "ENGR", 4) == 0) {
    m.engram_version = rd<uint32_t>(b + 68);
    m.n_kv_shared = rd<uint32_t>(b + 72);
    m.sliding_kv_dim = rd<uint32_t>(b + 76);
    m.full_kv_dim = rd<uint32_t>(b + 80);
    m.ple_dim = rd<uint32_t>(b + 84);
    m.sliding_window = rd<uint32_t>(b + 88);
    if (m.engram_version == 0) m.engram_version = 1;
  }
  if (m.n_layers > 65536) {
    delete f;
    return io_fail(".mojostream: implausible n_layers=" + std::to_string(m.n_layers));
  }
  // The directory is read at byte 128, as the reference does (it ignores
  // dir_offset); the shape guard checks that dir_offset says the same.
  if (m.n_tensors > (f->raw.size() - kHdr) / kDirEntry) {
    delete f;
    return io_fail(".mojostream: directory of " + std::to_string(m.n_tensors) +
                   " entries extends past the end of the file");
  }
  f->dir.resize(m.n_tensors);
  for (uint64_t i = 0; i < m.n_tensors; ++i) {
    const uint8_t *e = b + kHdr + i * kDirEntry;
    ms_file_entry &d = f->dir[i];
    d.layer_id = rd<uint32_t>(e);
    d.mat_type = rd<uint32_t>(e + 4);
    d.rows = rd<uint32_t>(e + 8);
    d.cols = rd<uint32_t>(e + 12);
    d.scale = rd<float>(e + 16);
    d.flags = rd<uint32_t>(e + 20);
    d.data_offset = rd<uint64_t>(e + 24);
  }
  default_types(f);
  *out = f;
  return MS_OK;
}

extern "C" int ms_file_close(ms_file *f) {
  delete f;
  return MS_OK;
}

extern "C" int ms_file_get_meta(const ms_file *f, ms_file_meta *out) {
  MS_CHECK_ARG(f && out, "file_get_meta: null argument");
  *out = f->meta;
  return MS_OK;
}

extern "C" int ms_file_get_entry(const ms_file *f, int index, ms_file_entry *out) {
  MS_CHECK_ARG(f && out, "file_get_entry: null argument");
  MS_CHECK_ARG(index >= 0 && (size_t)index < f->dir.size(), "file_get_entry: index out of range");
  *out = f->dir[index];
  return MS_OK;
}

extern "C" int ms_file_set_layer_types(ms_file *f, const uint8_t *is_full, int n_layers) {
  MS_CHECK_ARG(f, "file_set_layer_types: null file");
  if (!is_full) {
    default_types(f);
    return MS_OK;
  }
  MS_CHECK_ARG(n_layers == (int)f->meta.n_layers, "file_set_layer_types: need one flag per layer");
  f->is_full.assign(is_full, is_full + n_layers);
  return MS_OK;
}

extern "C" int ms_file_layer_info(const ms_file *f, int layer, ms_file_layer *out) {
  MS_CHECK_ARG(f && out, "file_layer_info: null argument");
  MS_CHECK_ARG(layer >= 0 && layer < (int)f->meta.n_layers, "file_layer_info: layer out of range");
  layer_dims(f->meta, f->is_full[layer] != 0, out);
  return MS_OK;
}

// tensor_ptr (mojostream.mojo:156-175): direct index layer*8 + type, then a
// linear search.  A tensor that is absent is an error here; the reference
// returns the buffer start with scale 0.
extern "C" int ms_file_tensor(const ms_file *f, int layer, int mat_type, const uint8_t **h_ptr,
                              float *scale, size_t *bytes) {
  MS_CHECK_ARG(f && h_ptr && scale, "file_tensor: null argument");
  const ms_file_entry *hit = nullptr;
  const size_t idx = (size_t)layer * kPerLayer + (size_t)mat_type;
  if (layer >= 0 && mat_type >= 0 && idx < f->dir.size() && (int)f->dir[idx].layer_id == layer &&
      (int)f->dir[idx].mat_type == mat_type)
    hit = &f->dir[idx];
  for (size_t i = 0; !hit && i < f->dir.size(); ++i)
    if ((int)f->dir[i].layer_id == layer && (int)f->dir[i].mat_type == mat_type) hit = &f->dir[i];
  if (!hit)
    return io_fail(".mojostream: no tensor for layer " + std::to_string(layer) + " type " +
                   std::to_string(mat_type));
  const size_t nbytes = (size_t)hit->rows * (hit->cols / 2);
  if (mat_type != 0 && (hit->data_offset > f->raw.size() || nbytes > f->raw.size() - hit->data_offset))
    return io_fail(".mojostream: tensor data of layer " + std::to_string(layer) + " type " +
                   std::to_string(mat_type) + " lies outside the file");
  *h_ptr = f->raw.data() + (mat_type ? hit->data_offset : 0);
  *scale = hit->scale;
  if (bytes) *bytes = mat_type ? nbytes : 0;
  return MS_OK;
}

// ple_scale (mojostream.mojo:177-182): the PLE entry's scale, 1.0 when the
// directory has no entry at layer*8.
extern "C" int ms_file_ple_scale(const ms_file *f, int layer, float *out) {
  MS_CHECK_ARG(f && out, "file_ple_scale: null argument");
  const size_t idx = (size_t)layer * kPerLayer;
  *out = (layer >= 0 && idx < f->dir.size()) ? f->dir[idx].scale : 1.0f;
  return MS_OK;
}

// compute_dir_checksum (src/tests/validate_real.mojo:78-83): the XOR of the
// 32-bit words at byte 16 of every directory entry, i.e. of the scale fields'
// bit patterns.
extern "C" int ms_file_dir_checksum(const ms_file *f, uint32_t *out) {
  MS_CHECK_ARG(f && out, "dir_checksum: null argument");
  uint32_t acc = 0;
  const uint8_t *b = f->raw.data();
  for (uint64_t i = 0; i < f->meta.n_tensors; ++i) acc ^= rd<uint32_t>(b + kHdr + i * kDirEntry + 16);
  *out = acc;
  return MS_OK;
}

// run_validation (src/tests/validate_real.mojo:110-260): the structural checks
// of a converted file, counted like the reference (one check each; a spot
// check per tensor).  Like the reference it reports instead of failing: the
// return value is MS_OK unless the arguments are bad.
extern "C" int ms_file_validate(const ms_file *f, ms_file_validation *out) {
  MS_CHECK_ARG(f && out, "file_validate: null argument");
  ms_file_validation &r = *out;
  r = ms_file_validation{};
  const ms_file_meta &m = f->meta;
  const uint8_t *b = f->raw.data();
  r.file_bytes = m.file_bytes;
  auto check = [&](bool ok, int bit, const std::string &msg) {
    r.n_checks += 1;
    if (ok) return;
    r.n_failed += 1;
    r.failed_mask |= 1u << bit;
    if (!r.message[0]) snprintf(r.message, sizeof r.message, "%s", msg.c_str());
  };
  // [2] magic: the first word "MOJO" (:130-135), then the architecture fields
  // (:144-155)
  check(rd<uint32_t>(b) == 0x4F4A4F4Du, MS_VALIDATE_MAGIC, "magic: expected 'MOJO...'");
  const bool arch_ok = m.n_layers > 0 && m.hidden > 0 && m.ffn_dim > 0 && m.n_heads > 0 &&
                       !(m.n_kv_heads > 0 && m.kv_dim % m.n_kv_heads != 0);
  check(arch_ok, MS_VALIDATE_ARCH,
        "architecture fields: n_layers, hidden, ffn_dim, n_heads must be positive and kv_dim a "
        "multiple of n_kv_heads");
  // [3] Engram extension at byte 64 (:158-176)
  check(rd<uint32_t>(b + 64) == 0x52474E45u, MS_VALIDATE_ENGRAM, "Engram magic 'ENGR' missing");
  // [4] n_tensors == n_layers * 8 (:179-190), offsets inside the file (:192-205)
  check(m.n_tensors == (uint64_t)m.n_layers * kPerLayer, MS_VALIDATE_TENSORS,
        "n_tensors=" + std::to_string(m.n_tensors) + " != n_layers*8=" +
            std::to_string((uint64_t)m.n_layers * kPerLayer));
  bool off_ok = true;
  for (const auto &e : f->dir)
    if (e.data_offset > 0 && e.data_offset >= m.file_bytes) off_ok = false;
  check(off_ok, MS_VALIDATE_OFFSETS, "a directory offset lies outside the file");
  // [5] directory checksum, zero counts as a failure (:207-217)
  uint32_t chk = 0;
  ms_file_dir_checksum(f, &chk);
  r.dir_checksum = chk;
  check(chk != 0, MS_VALIDATE_CHECKSUM, "directory checksum is 0 (all scales zero?)");
  // [6] spot checks of Q and Gate in layers 0, 20, 41 (:219-232): the first 64
  // bytes neither all 0x00 nor all 0xFF
  int bit = MS_VALIDATE_SPOT;
  for (uint32_t layer : {0u, 20u, 41u}) {
    if (layer >= m.n_layers && layer != 0) continue;
    for (int type : {1, 5}) {
      const uint8_t *ptr = nullptr;
      float sc = 0.f;
      size_t nb = 0;
      bool ok = ms_file_tensor(f, (int)layer, type, &ptr, &sc, &nb) == MS_OK && nb >= 64;
      if (ok) {
        bool zero = true, ff = true;
        for (int i = 0; i < 64; ++i) {
          zero = zero && ptr[i] == 0;
          ff = ff && ptr[i] == 0xFF;
        }
        ok = !zero && !ff;
      }
      check(ok, bit, "layer " + std::to_string(layer) + (type == 1 ? " Q" : " Gate") +
                         ": first 64 bytes all 0x00 or all 0xFF, or the tensor is missing");
      if (bit < 31) ++bit;
    }
  }
  r.passed = r.n_failed == 0;
  set_error("");
  return MS_OK;
}

// ShapeGuard: the invariants of validate_gemma4_shape (mojostream.mojo:190-219)
// plus the head-size checks per layer type.
extern "C" int ms_file_shape_guard(const ms_file *f) {
  MS_CHECK_ARG(f, "shape_guard: null file");
  const ms_file_meta &m = f->meta;
  auto bad = [](const std::string &s) { return io_fail("[ShapeGuard] " + s); };
  if (m.n_heads == 0) return bad("n_heads = 0");
  if (m.n_kv_heads == 0) return bad("n_kv_heads = 0");
  if (m.hidden % m.n_heads != 0)
    return bad("hidden (" + std::to_string(m.hidden) + ") not divisible by n_heads (" +
               std::to_string(m.n_heads) + ")");
  if (m.n_heads % m.n_kv_heads != 0)
    return bad("n_heads (" + std::to_string(m.n_heads) + ") not divisible by n_kv_heads (" +
               std::to_string(m.n_kv_heads) + ")");
  if (m.kv_dim % m.n_kv_heads != 0)
    return bad("kv_dim=" + std::to_string(m.kv_dim) + " not divisible by n_kv_heads=" +
               std::to_string(m.n_kv_heads));
  if (m.n_layers == 0) return bad("n_layers <= 0");
  if (m.ffn_dim == 0) return bad("ffn_dim <= 0");
  if (m.n_tensors != (uint64_t)m.n_layers * kPerLayer)
    return bad("n_tensors=" + std::to_string(m.n_tensors) + " != n_layers*8=" +
               std::to_string((uint64_t)m.n_layers * kPerLayer));
  if (m.dir_offset != (uint64_t)kHdr)
    return bad("dir_offset=" + std::to_string(m.dir_offset) + " != 128");
  if (m.engram_version) {
    // Hybrid files: the header's kv_dim is the sliding one (convert.py:187-189).
    if (m.sliding_kv_dim != m.kv_dim)
      return bad("sliding_kv_dim=" + std::to_string(m.sliding_kv_dim) + " != kv_dim=" +
                 std::to_string(m.kv_dim));
    if (m.full_kv_dim % m.n_kv_heads != 0)
      return bad("full_kv_dim=" + std::to_string(m.full_kv_dim) +
                 " not divisible by n_kv_heads=" + std::to_string(m.n_kv_heads));
  } else {
    // One head size for all layers: kv_dim = n_kv_heads * hidden / n_heads
    // (stream_runner.mojo:296-300).
    const uint32_t want = m.n_kv_heads * (m.hidden / m.n_heads);
    if (m.kv_dim != want)
      return bad("kv_dim=" + std::to_string(m.kv_dim) + " expected=" + std::to_string(want) +
                 " (n_kv_heads x head_dim)");
  }
  return MS_OK;
}

// TensorGuard: the five criteria of validate_tensor_entries
// (stream_runner.mojo:313-380) with per-layer expected shapes.  Scales must be
// finite and positive (the reference's `scale <= 0` lets NaN through).
extern "C" int ms_file_tensor_guard(const ms_file *f) {
  MS_CHECK_ARG(f, "tensor_guard: null file");
  const ms_file_meta &m = f->meta;
  for (size_t i = 0; i < f->dir.size(); ++i) {
    const ms_file_entry &e = f->dir[i];
    const int el = (int)(i / kPerLayer), et = (int)(i % kPerLayer);
    const std::string loc = "[TensorGuard] Tensor[" + std::to_string(i) + "] Layer " +
                            std::to_string(el) + " " + kMatNames[et] + ": ";
    if ((int)e.layer_id != el)
      return io_fail(loc + "layer_id=" + std::to_string(e.layer_id) + " expected=" + std::to_string(el));
    if ((int)e.mat_type != et)
      return io_fail(loc + "mat_type=" + std::to_string(e.mat_type) + " expected=" + std::to_string(et));
    ms_file_layer ld;
    layer_dims(m, el < (int)f->is_full.size() && f->is_full[el], &ld);
    uint32_t er, ec;
    expected(m, ld, et, &er, &ec);
    if (e.rows != er)
      return io_fail(loc + "rows=" + std::to_string(e.rows) + " expected=" + std::to_string(er));
    if (e.cols != ec)
      return io_fail(loc + "cols=" + std::to_string(e.cols) + " expected=" + std::to_string(ec));
    if (!(e.scale > 0.f) || !std::isfinite(e.scale))
      return io_fail(loc + "scale=" + std::to_string(e.scale) + " is not a positive finite value");
    if (et == 0) continue;
    if (e.data_offset % kPage != 0)
      return io_fail(loc + "offset=" + std::to_string(e.data_offset) + " not 4096-aligned (mod=" +
                     std::to_string(e.data_offset % kPage) + ")");
    const uint64_t nbytes = (uint64_t)e.rows * (e.cols / 2);
    if (e.data_offset + nbytes > m.file_bytes)
      return io_fail(loc + "offset=" + std::to_string(e.data_offset) + " + size=" +
                     std::to_string(nbytes) + " = " + std::to_string(e.data_offset + nbytes) +
                     " > file_size=" + std::to_string(m.file_bytes));
  }
  return MS_OK;
}

// Seeded synthetic model file (the .mojostream generator of
// create_fake_model.py:188-281, with this library's counter-based generator so
// that the same seed gives the same weights as a model filled on the device).
extern "C" int ms_file_write_synthetic(const char *path, const ms_file_meta *hdr,
                                       const uint8_t *is_full, uint64_t seed) {
  MS_CHECK_ARG(path && hdr, "file_write_synthetic: null argument");
  MS_CHECK_ARG(hdr->n_layers > 0 && hdr->hidden > 0 && hdr->ffn_dim > 0 && hdr->n_heads > 0 &&
                   hdr->n_kv_heads > 0 && hdr->kv_dim > 0,
               "file_write_synthetic: every dimension must be positive");
  ms_file_meta m = *hdr;
  m.version = 1;
  if (m.format_tag == 0) m.format_tag = m.engram_version ? 2 : 1;
  if (m.engram_version && m.sliding_kv_dim == 0) m.sliding_kv_dim = m.kv_dim;
  m.n_tensors = (uint64_t)m.n_layers * kPerLayer;
  m.dir_offset = kHdr;
  const uint64_t dir_end = kHdr + m.n_tensors * kDirEntry;
  m.data_start = (dir_end + kPage - 1) / kPage * kPage;
  std::vector<uint8_t> types(m.n_layers, 0);
  for (uint32_t l = 0; l < m.n_layers; ++l)
    types[l] = is_full ? is_full[l] : (hybrid(m) && (l + 1) % 6 == 0);

  std::vector<uint8_t> head((size_t)m.data_start, 0);
  memcpy(head.data(), "MOJOSTRM", 8);
  wr<uint32_t>(&head[8], m.version);
  wr<uint32_t>(&head[12], m.format_tag);
  wr<uint32_t>(&head[16], m.n_layers);
  wr<uint32_t>(&head[20], m.hidden);
  wr<uint32_t>(&head[24], m.kv_dim);
  wr<uint32_t>(&head[28], m.ffn_dim);
  wr<uint32_t>(&head[32], m.n_heads);
  wr<uint32_t>(&head[36], m.n_kv_heads);
  wr<uint64_t>(&head[40], m.n_tensors);
  wr<uint64_t>(&head[48], m.dir_offset);
  wr<uint64_t>(&head[56], m.data_start);
  if (m.engram_version) {
    memcpy(&head[64], "ENGR", 4);
    wr<uint32_t>(&head[68], m.engram_version);
    wr<uint32_t>(&head[72], m.n_kv_shared);
    wr<uint32_t>(&head[76], m.sliding_kv_dim);
    wr<uint32_t>(&head[80], m.full_kv_dim);
    wr<uint32_t>(&head[84], m.ple_dim);
    wr<uint32_t>(&head[88], m.sliding_window);
  }
  uint64_t cur = m.data_start;
  size_t biggest = 0;
  for (uint32_t l = 0; l < m.n_layers; ++l) {
    ms_file_layer ld;
    layer_dims(m, types[l] != 0, &ld);
    for (int t = 0; t < kPerLayer; ++t) {
      uint8_t *e = &head[kHdr + ((size_t)l * kPerLayer + t) * kDirEntry];
      uint32_t r, c;
      expected(m, ld, t, &r, &c);
      wr<uint32_t>(e, l);
      wr<uint32_t>(e + 4, (uint32_t)t);
      wr<uint32_t>(e + 8, r);
      wr<uint32_t>(e + 12, c);
      if (t == 0) {
        wr<float>(e + 16, ms_host_uniform(seed, kPleStream, l, 0.8f, 1.2f));
        continue;
      }
      wr<float>(e + 16, ms_host_uniform(seed, kScaleStream, matrix_stream(l, t), 0.04f, 0.15f));
      wr<uint64_t>(e + 24, cur);
      const size_t nb = (size_t)r * (c / 2);
      biggest = std::max(biggest, nb);
      cur = (cur + nb + kPage - 1) / kPage * kPage;
    }
  }
  FILE *fp = fopen(path, "wb");
  if (!fp) return io_fail(std::string(".mojostream: cannot create ") + path);
  bool ok = fwrite(head.data(), 1, head.size(), fp) == head.size();
  std::vector<uint8_t> buf(biggest + kPage);
  for (uint32_t l = 0; l < m.n_layers && ok; ++l) {
    ms_file_layer ld;
    layer_dims(m, types[l] != 0, &ld);
    for (int t = 1; t < kPerLayer && ok; ++t) {
      uint32_t r, c;
      expected(m, ld, t, &r, &c);
      const size_t nb = (size_t)r * (c / 2);
      const size_t padded = (nb + kPage - 1) / kPage * kPage;
      ms_host_fill_random_u8(buf.data(), nb, seed, matrix_stream(l, t));
      memset(buf.data() + nb, 0, padded - nb);
      ok = fwrite(buf.data(), 1, padded, fp) == padded;
    }
  }
  ok = (fclose(fp) == 0) && ok;
  if (!ok) return io_fail(std::string(".mojostream: write failed for ") + path);
  return MS_OK;
}

// Binds every matrix and PLE scale of the file to a model whose shapes match
// (the load loop of run_harness harness.mojo:80-122 / StreamingRunner init
// stream_runner.mojo:188-270), after both guards pass.
extern "C" int ms_model_load_file(ms_model *model, const ms_file *f) {
  MS_CHECK_ARG(model && f, "model_load_file: null argument");
  if (int rc = ms_file_shape_guard(f)) return rc;
  if (int rc = ms_file_tensor_guard(f)) return rc;
  ms_model_desc d;
  if (int rc = ms_model_get_desc(model, &d, nullptr)) return rc;
  const ms_file_meta &m = f->meta;
  if ((uint32_t)d.hidden != m.hidden || (uint32_t)d.ffn != m.ffn_dim ||
      (uint32_t)d.n_layers != m.n_layers)
    return fail(MS_E_INVALID, "model_load_file: model (hidden " + std::to_string(d.hidden) +
                                  ", ffn " + std::to_string(d.ffn) + ", layers " +
                                  std::to_string(d.n_layers) + ") does not match the file (" +
                                  std::to_string(m.hidden) + ", " + std::to_string(m.ffn_dim) +
                                  ", " + std::to_string(m.n_layers) + ")");
  std::vector<ms_layer_desc> L(d.n_layers);
  if (int rc = ms_model_get_desc(model, &d, L.data())) return rc;
  for (int l = 0; l < d.n_layers; ++l) {
    ms_file_layer ld;
    layer_dims(m, f->is_full[l] != 0, &ld);
    if (L[l].q_dim != ld.q_dim || L[l].kv_dim != ld.kv_dim || L[l].n_heads != (int)m.n_heads ||
        L[l].n_kv_heads != (int)m.n_kv_heads)
      return fail(MS_E_INVALID, "model_load_file: layer " + std::to_string(l) +
                                    " of the model has q_dim " + std::to_string(L[l].q_dim) +
                                    ", kv_dim " + std::to_string(L[l].kv_dim) +
                                    " but the file has " + std::to_string(ld.q_dim) + ", " +
                                    std::to_string(ld.kv_dim));
  }
  for (int l = 0; l < d.n_layers; ++l) {
    for (int t = 1; t < kPerLayer; ++t) {
      const uint8_t *p;
      float s;
      if (int rc = ms_file_tensor(f, l, t, &p, &s, nullptr)) return rc;
      if (int rc = ms_model_set_matrix(model, l, t - 1, p, 0, s)) return rc;
    }
    float ple;
    ms_file_ple_scale(f, l, &ple);
    if (int rc = ms_model_set_ple(model, l, ple)) return rc;
  }
  return MS_OK;
}

// LM head file (load_lm_head, lm_head.mojo:61-116), after u32 vocab and f32 scale:
//   version 1 (tied Q4)  hidden fp32 BOS embedding, hidden*vocab/2 Q4 bytes;
//   version 2 (FP32)     u32 version, BOS, final-norm gamma, [hidden][vocab] fp32.
// A file at least as large as version 2 needs is read as version 2.
extern "C" int ms_model_load_lm_head_file(ms_model *model, const char *path) {
  MS_CHECK_ARG(model && path, "load_lm_head_file: null argument");
  ms_model_desc d;
  if (int rc = ms_model_get_desc(model, &d, nullptr)) return rc;
  MS_CHECK_ARG(d.vocab > 0, "load_lm_head_file: model has no LM head");
  FILE *fp = fopen(path, "rb");
  if (!fp) return io_fail(std::string("lm_head: cannot open ") + path);
  fseek(fp, 0, SEEK_END);
  const long sz = ftell(fp);
  fseek(fp, 0, SEEK_SET);
  std::vector<uint8_t> raw(sz > 0 ? (size_t)sz : 0);
  const bool ok = sz > 0 && fread(raw.data(), 1, raw.size(), fp) == raw.size();
  fclose(fp);
  if (!ok || raw.size() < 8) return io_fail(std::string("lm_head: cannot read ") + path);
  const uint32_t vocab = rd<uint32_t>(raw.data());
  const float scale = rd<float>(raw.data() + 4);
  const size_t D = (size_t)d.hidden;
  if (vocab != (uint32_t)d.vocab)
    return io_fail("lm_head: vocab " + std::to_string(vocab) + " != model vocab " +
                   std::to_string(d.vocab));
  // version 2 when the file holds [version][BOS fp32][gamma fp32][weights fp32]
  // after vocab and scale (the size test of lm_head.mojo:74-76)
  const size_t v2_size = 12 + D * 4 * 2 + D * (size_t)vocab * 4;
  if (raw.size() >= v2_size) {
    const uint8_t *p = raw.data() + 12;
    std::vector<float> bos(D), gamma(D);
    memcpy(bos.data(), p, D * 4);
    memcpy(gamma.data(), p + D * 4, D * 4);
    if (int rc = ms_model_set_lm_head_f32(model, reinterpret_cast<const float *>(p + D * 8), 0,
                                          gamma.data()))
      return rc;
    return ms_model_set_bos(model, bos.data());
  }
  const size_t need = 8 + D * 4 + D * (size_t)vocab / 2;
  if (raw.size() < need)
    return io_fail("lm_head: file has " + std::to_string(raw.size()) + " bytes, version 1 needs " +
                   std::to_string(need));
  std::vector<float> bos(D);
  memcpy(bos.data(), raw.data() + 8, D * 4);
  if (int rc = ms_model_set_lm_head(model, raw.data() + 8 + D * 4, 0, scale, nullptr)) return rc;
  return ms_model_set_bos(model, bos.data());
}

extern "C" int ms_lm_head_file_write_synthetic_v2(const char *path, int hidden, int vocab,
                                                  uint64_t seed) {
  MS_CHECK_ARG(path && hidden > 0 && vocab > 0, "lm_head_file_write_synthetic_v2: bad arguments");
  const size_t D = (size_t)hidden, nw = D * (size_t)vocab;
  std::vector<uint8_t> raw(12 + D * 8 + nw * 4);
  wr<uint32_t>(raw.data(), (uint32_t)vocab);
  wr<float>(raw.data() + 4, 1.0f);
  wr<uint32_t>(raw.data() + 8, 2u);
  float *bos = reinterpret_cast<float *>(raw.data() + 12);
  float *gamma = bos + D, *w = gamma + D;
  ms_host_fill_normal(bos, D, seed, kBosStream);
  ms_host_fill_normal(gamma, D, seed, kGammaStream);
  for (size_t i = 0; i < D; ++i) gamma[i] = 1.0f + 0.1f * gamma[i];
  ms_host_fill_normal(w, nw, seed, kLmStream);
  for (size_t i = 0; i < nw; ++i) w[i] *= 0.05f;
  FILE *fp = fopen(path, "wb");
  if (!fp) return io_fail(std::string("lm_head: cannot create ") + path);
  bool ok = fwrite(raw.data(), 1, raw.size(), fp) == raw.size();
  ok = (fclose(fp) == 0) && ok;
  return ok ? MS_OK : io_fail(std::string("lm_head: write failed for ") + path);
}

extern "C" int ms_lm_head_file_write_synthetic(const char *path, int hidden, int vocab,
                                               uint64_t seed) {
  MS_CHECK_ARG(path && hidden > 0 && vocab > 0 && vocab % 2 == 0,
               "lm_head_file_write_synthetic: bad arguments");
  const size_t D = (size_t)hidden, nb = D * (size_t)vocab / 2;
  std::vector<uint8_t> raw(8 + D * 4 + nb);
  wr<uint32_t>(raw.data(), (uint32_t)vocab);
  wr<float>(raw.data() + 4, ms_host_uniform(seed, kScaleStream, kLmStream, 0.04f, 0.15f));
  ms_host_fill_normal(reinterpret_cast<float *>(raw.data() + 8), D, seed, kBosStream);
  ms_host_fill_random_u8(raw.data() + 8 + D * 4, nb, seed, kLmStream);
  FILE *fp = fopen(path, "wb");
  if (!fp) return io_fail(std::string("lm_head: cannot create ") + path);
  bool ok = fwrite(raw.data(), 1, raw.size(), fp) == raw.size();
  ok = (fclose(fp) == 0) && ok;
  return ok ? MS_OK : io_fail(std::string("lm_head: write failed for ") + path);
}
