// Host-side tokenizers (no device code): the demo BPE tokenizer
// (BPETokenizer, src/nlp/tokenizer.mojo:31-180) and the id -> text map
// (TokenMap, src/tokenizer/gemma_proto.mojo:20-74).
//
// The reference builds its strings from chr(byte): every byte is one code
// point 0..255.  Here tokens are byte strings; a caller that wants the
// reference's text reads each returned byte as that code point (Latin-1).
//
// .msvocab (BPETokenizer.load, :56-101): u32 magic "MSVB", u32 n_tokens,
// u32 n_merges, u32 reserved; n_tokens x {u32 id, u32 len, bytes};
// n_merges x {u32 len, left bytes, u32 len, right bytes}, rank = order.
// vocab_proto.bin (load_token_map, gemma_proto.mojo:59-74): u32 n, then
// n x {u32 len, bytes}.
#include "common.h"

#include <cstdio>
#include <algorithm>
#include <cstring>
#include <exception>
#include <string>
#include <unordered_map>
#include <vector>

struct ms_tokenizer {
  std::vector<std::string> id_to_tok;
  std::unordered_map<std::string, int> tok_to_id;
  std::unordered_map<std::string, int> merge_rank;  // key "left|right"
  int vocab_size = 0;
};

struct ms_token_map {
  std::vector<std::string> text;
};

namespace ms {
namespace {

constexpr uint32_t kVocabMagic = 0x4256534D;  // "MSVB"
constexpr int kBos = 1, kEos = 2, kUnk = 0, kPad = 3;
// Largest token id a vocabulary file may use (64 times Gemma's 262,144 ids);
// the id table holds max id + 1 entries.
constexpr uint32_t kMaxTokenId = (1u << 24) - 1;

bool read_file(const char *path, std::vector<uint8_t> &raw) {
  FILE *fp = fopen(path, "rb");
  if (!fp) return false;
  fseek(fp, 0, SEEK_END);
  const long sz = ftell(fp);
  fseek(fp, 0, SEEK_SET);
  raw.resize(sz > 0 ? (size_t)sz : 0);
  const bool ok = sz >= 0 && fread(raw.data(), 1, raw.size(), fp) == raw.size();
  fclose(fp);
  return ok;
}

// Bounds-checked little-endian reader over a file image.
struct Cursor {
  const std::vector<uint8_t> &b;
  size_t pos = 0;
  bool ok = true;
  uint32_t u32() {
    if (pos + 4 > b.size()) {
      ok = false;
      return 0;
    }
    uint32_t v;
    memcpy(&v, b.data() + pos, 4);
    pos += 4;
    return v;
  }
  std::string bytes(uint32_t n) {
    if (pos + n > b.size()) {
      ok = false;
      return {};
    }
    std::string s(reinterpret_cast<const char *>(b.data() + pos), n);
    pos += n;
    return s;
  }
};

int copy_out(const std::string &s, char *out, int cap, int *len) {
  *len = (int)s.size();
  MS_CHECK_ARG(out || cap == 0, "tokenizer: null output buffer");
  if ((int)s.size() > cap)  // *len holds the size needed
    return fail(MS_E_INVALID, "tokenizer: output buffer too small");
  if (!s.empty()) memcpy(out, s.data(), s.size());
  return MS_OK;
}

}  // namespace
}  // namespace ms

using namespace ms;

extern "C" int ms_tokenizer_load(const char *path, ms_tokenizer **out) {
  MS_CHECK_ARG(path && out, "tokenizer_load: null argument");
  std::vector<uint8_t> raw;
  if (!read_file(path, raw)) return fail(MS_E_IO, std::string("tokenizer: cannot read ") + path);
  Cursor c{raw};
  const uint32_t magic = c.u32(), n_tokens = c.u32(), n_merges = c.u32();
  c.u32();
  if (!c.ok || magic != kVocabMagic) return fail(MS_E_IO, "tokenizer: invalid magic number");
  auto *t = new ms_tokenizer;
  bool bad_id = false;
  try {
    for (uint32_t i = 0; i < n_tokens && c.ok; ++i) {
      const uint32_t id = c.u32(), len = c.u32();
      std::string s = c.bytes(len);
      if (!c.ok) break;
      // ids index a table of id + 1 entries and are returned as int32: a
      // larger id cannot come from a real vocabulary (the reference would try
      // to grow its List to that size)
      if (id > kMaxTokenId) {
        bad_id = true;
        break;
      }
      // _set_token (:45-52): grow with "<unk>", both directions, vocab = max id + 1
      if (t->id_to_tok.size() <= id) t->id_to_tok.resize((size_t)id + 1, "<unk>");
      t->id_to_tok[id] = s;
      t->tok_to_id[s] = (int)id;
      t->vocab_size = std::max(t->vocab_size, (int)id + 1);
    }
    for (uint32_t r = 0; r < n_merges && c.ok && !bad_id; ++r) {
      std::string l = c.bytes(c.u32());
      std::string rr = c.bytes(c.u32());
      if (c.ok) t->merge_rank[l + "|" + rr] = (int)r;
    }
  } catch (const std::exception &e) {  // no C++ exception crosses the ABI
    delete t;
    return fail(MS_E_IO, std::string("tokenizer: cannot hold the vocabulary: ") + e.what());
  }
  if (bad_id) {
    delete t;
    return fail(MS_E_IO, "tokenizer: token id above " + std::to_string(kMaxTokenId));
  }
  if (!c.ok) {
    delete t;
    return fail(MS_E_IO, "tokenizer: file truncated");
  }
  *out = t;
  return MS_OK;
}

extern "C" int ms_tokenizer_free(ms_tokenizer *t) {
  delete t;
  return MS_OK;
}

extern "C" int ms_tokenizer_vocab_size(const ms_tokenizer *t, int *n) {
  MS_CHECK_ARG(t && n, "tokenizer_vocab_size: null argument");
  *n = t->vocab_size;
  return MS_OK;
}

// BPETokenizer.encode (:103-150): one token per byte, then repeatedly merge the
// leftmost adjacent pair of lowest rank until no pair has a rank; unknown
// strings map to id 0.  *n gets the count; ids may be null to ask for it.
extern "C" int ms_tokenizer_encode(const ms_tokenizer *t, const char *text, int len,
                                   int32_t *ids, int cap, int *n) {
  MS_CHECK_ARG(t && n && len >= 0 && (text || len == 0), "tokenizer_encode: bad argument");
  std::vector<std::string> toks;
  toks.reserve(len);
  for (int i = 0; i < len; ++i) toks.emplace_back(1, text[i]);
  for (;;) {
    int best_rank = 999999999, best = -1;
    for (size_t k = 0; k + 1 < toks.size(); ++k) {
      auto it = t->merge_rank.find(toks[k] + "|" + toks[k + 1]);
      if (it != t->merge_rank.end() && it->second < best_rank) {
        best_rank = it->second;
        best = (int)k;
      }
    }
    if (best < 0) break;
    toks[best] += toks[best + 1];
    toks.erase(toks.begin() + best + 1);
  }
  *n = (int)toks.size();
  if (!ids) return MS_OK;
  MS_CHECK_ARG(cap >= (int)toks.size(), "tokenizer_encode: output holds fewer ids than needed");
  for (size_t k = 0; k < toks.size(); ++k) {
    auto it = t->tok_to_id.find(toks[k]);
    ids[k] = it == t->tok_to_id.end() ? kUnk : it->second;
  }
  return MS_OK;
}

// BPETokenizer.decode (:152-163): BOS, EOS and PAD skipped; ids past the table
// skipped; a negative id counts from the end of the table, as List indexing does.
extern "C" int ms_tokenizer_decode(const ms_tokenizer *t, const int32_t *ids, int n, char *out,
                                   int cap, int *len) {
  MS_CHECK_ARG(t && len && n >= 0 && (ids || n == 0), "tokenizer_decode: bad argument");
  std::string s;
  const long sz = (long)t->id_to_tok.size();
  for (int k = 0; k < n; ++k) {
    long id = ids[k];
    if (id == kBos || id == kEos || id == kPad) continue;
    if (id >= sz) continue;
    if (id < 0) id += sz;
    if (id < 0) continue;
    s += t->id_to_tok[(size_t)id];
  }
  return copy_out(s, out, cap, len);
}

// BPETokenizer.token_str (:168-172): "<unk>" at or past the end of the table;
// a negative id counts from the end, as in decode (List indexing).
extern "C" int ms_tokenizer_token_str(const ms_tokenizer *t, int id, char *out, int cap,
                                      int *len) {
  MS_CHECK_ARG(t && len, "tokenizer_token_str: null argument");
  const long sz = (long)t->id_to_tok.size();
  long i = id;
  if (i < 0) i += sz;
  const bool in = i >= 0 && i < sz && id < sz;
  return copy_out(in ? t->id_to_tok[(size_t)i] : std::string("<unk>"), out, cap, len);
}

extern "C" int ms_token_map_load(const char *path, ms_token_map **out) {
  MS_CHECK_ARG(path && out, "token_map_load: null argument");
  std::vector<uint8_t> raw;
  if (!read_file(path, raw)) return fail(MS_E_IO, std::string("token map: cannot read ") + path);
  Cursor c{raw};
  const uint32_t n = c.u32();
  auto *m = new ms_token_map;
  for (uint32_t i = 0; i < n && c.ok; ++i) {
    std::string s = c.bytes(c.u32());
    if (c.ok) m->text.push_back(std::move(s));
  }
  if (!c.ok) {
    delete m;
    return fail(MS_E_IO, "token map: file truncated");
  }
  *out = m;
  return MS_OK;
}

extern "C" int ms_token_map_free(ms_token_map *m) {
  delete m;
  return MS_OK;
}

extern "C" int ms_token_map_size(const ms_token_map *m, int *n) {
  MS_CHECK_ARG(m && n, "token_map_size: null argument");
  *n = (int)m->text.size();
  return MS_OK;
}

// TokenMap.decode (gemma_proto.mojo:27-37): "[?:id]" for an id out of range.
extern "C" int ms_token_map_decode(const ms_token_map *m, int id, char *out, int cap, int *len) {
  MS_CHECK_ARG(m && len, "token_map_decode: null argument");
  if (id < 0 || (size_t)id >= m->text.size())
    return copy_out("[?:" + std::to_string(id) + "]", out, cap, len);
  return copy_out(m->text[(size_t)id], out, cap, len);
}
