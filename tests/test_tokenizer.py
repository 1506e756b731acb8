"""Tokenizers through the C ABI (host only, no GPU): the demo BPE tokenizer
(src/nlp/tokenizer.mojo) and TokenMap (src/tokenizer/gemma_proto.mojo).

- Hand-worked merges pin rank order, the leftmost tie, chained merges and
  unknown strings; the restatement in oracle/tokenizer_ref.py must agree with
  them before it checks the library on random text.
- The reference's round trip "Hallo Mojo" (tokenizer_test.mojo:75).
- File errors: wrong magic, truncation; TokenMap's "[?:id]".
"""
import os
import random
import struct

import pytest

from oracle import tokenizer_ref as ref

SPECIAL = [(0, b"<unk>"), (1, b"<bos>"), (2, b"<eos>"), (3, b"<pad>")]


def write_msvocab(path, tokens, merges, magic=0x4256534D):
    b = struct.pack("<IIII", magic, len(tokens), len(merges), 0)
    for i, t in tokens:
        b += struct.pack("<II", i, len(t)) + t
    for l, r in merges:
        b += struct.pack("<I", len(l)) + l + struct.pack("<I", len(r)) + r
    with open(path, "wb") as f:
        f.write(b)


def byte_vocab(extra):
    toks = list(SPECIAL) + [(4 + c, bytes([c])) for c in range(256)]
    nxt = 260
    for t in extra:
        toks.append((nxt, t))
        nxt += 1
    return toks


@pytest.fixture
def tok(tmp_path):
    from mojostream_amd.tokenizer import BPETokenizer
    merges = [(b"l", b"l"), (b"a", b"ll"), (b"H", b"all"), (b"o", b" "), (b"M", b"o")]
    toks = byte_vocab([b"ll", b"all", b"Hall", b"o ", b"Mo"])
    p = str(tmp_path / "v.msvocab")
    write_msvocab(p, toks, merges)
    t = BPETokenizer(p)
    yield t, toks, merges
    t.close()


def test_hand_worked_merges(tok):
    t, toks, merges = tok
    vocab = {s: i for i, s in toks}
    # "Hallo Mojo": l+l (rank 0) -> a+ll (1) -> H+all (2); then "o "(3) and "Mo"(4)
    want = [vocab[b"Hall"], vocab[b"o "], vocab[b"Mo"], vocab[b"j"], vocab[b"o"]]
    assert t.encode("Hallo Mojo") == want
    assert ref.encode(b"Hallo Mojo", merges, vocab) == want
    assert t.decode(want) == "Hallo Mojo"
    # leftmost of equal rank: "lll" merges the first pair
    assert t.encode("lll") == [vocab[b"ll"], vocab[b"l"]]
    assert ref.encode(b"lll", merges, vocab) == [vocab[b"ll"], vocab[b"l"]]
    assert t.encode("") == []
    assert t.n_tokens() == 265


def test_unknown_specials_and_token_str(tmp_path):
    from mojostream_amd.tokenizer import BPETokenizer
    p = str(tmp_path / "small.msvocab")
    write_msvocab(p, SPECIAL + [(10, b"a"), (11, b"b"), (12, b"ab")], [(b"a", b"b")])
    t = BPETokenizer(p)
    assert t.encode("abc") == [12, 0]            # "c" is not in the vocabulary
    assert t.decode([1, 12, 2, 3, 10, 99, 11]) == "abab"
    assert t.decode([-1]) == "ab"                # a negative id counts from the end
    assert t.token_str(5) == "<unk>" and t.token_str(99) == "<unk>"
    assert t.token_str(12) == "ab"
    # a negative id counts from the end in token_str as in decode
    assert t.token_str(-1) == "ab" and t.token_str(-13) == "<unk>"
    assert t.token_str(-14) == "<unk>"           # before the start of the table
    assert t.n_tokens() == 13
    t.close()


def test_random_text_vs_restatement(tmp_path):
    from mojostream_amd.tokenizer import BPETokenizer
    rng = random.Random(7)
    alpha = b"abcde "
    merges, seen = [], set()
    while len(merges) < 40:
        a = bytes(rng.choice(alpha) for _ in range(rng.randint(1, 2)))
        b = bytes(rng.choice(alpha) for _ in range(rng.randint(1, 2)))
        if (a, b) not in seen:
            seen.add((a, b))
            merges.append((a, b))
    extra = sorted({a + b for a, b in merges} - {bytes([c]) for c in range(256)})
    toks = byte_vocab(extra[:-3])                # a few merged strings stay unknown
    p = str(tmp_path / "r.msvocab")
    write_msvocab(p, toks, merges)
    t = BPETokenizer(p)
    vocab = {s: i for i, s in toks}
    id_to_tok = [b"<unk>"] * (max(i for i, _ in toks) + 1)
    for i, s in toks:
        id_to_tok[i] = s
    for _ in range(200):
        text = bytes(rng.choice(alpha) for _ in range(rng.randint(0, 60)))
        ids = t.encode(text.decode())
        assert ids == ref.encode(text, merges, vocab)
        assert t.decode(ids) == ref.decode(ids, id_to_tok).decode("latin-1")
    t.close()


def test_non_ascii_bytes_round_trip(tok):
    t, _, _ = tok
    s = "Grüße"
    ids = t.encode(s)
    assert len(ids) == len(s.encode("utf-8"))
    # one code point per byte, as chr(byte) builds the reference's string
    assert t.decode(ids) == s.encode("utf-8").decode("latin-1")


def test_file_errors(tmp_path):
    import mojostream_amd as ms
    from mojostream_amd.tokenizer import BPETokenizer, TokenMap
    p = str(tmp_path / "bad.msvocab")
    write_msvocab(p, SPECIAL, [], magic=0x12345678)
    with pytest.raises(ms.MSError, match="invalid magic"):
        BPETokenizer(p)
    write_msvocab(p, SPECIAL, [(b"a", b"b")])
    with open(p, "r+b") as f:
        f.truncate(40)
    with pytest.raises(ms.MSError, match="truncated"):
        BPETokenizer(p)
    with pytest.raises(ms.MSError, match="cannot read"):
        TokenMap(str(tmp_path / "missing.bin"))
    # a corrupt id would size the id table to 2^32 entries: refused
    write_msvocab(p, SPECIAL + [(0xFFFFFFFF, b"x")], [])
    with pytest.raises(ms.MSError, match="token id above"):
        BPETokenizer(p)
    write_msvocab(p, SPECIAL + [((1 << 24) - 1, b"x")], [])  # the largest id accepted
    t = BPETokenizer(p)
    assert t.n_tokens() == 1 << 24 and t.token_str((1 << 24) - 1) == "x"
    t.close()


GOLDEN_VOCAB = os.path.join(os.path.dirname(__file__), "golden", "vocab.msvocab")


def test_reference_vocab_fixture():
    """vocab.msvocab as the reference ships it (scripts/create_vocab.py:28-80:
    4 special tokens, printable ASCII 32..126 under their byte values, 15
    merged tokens with ids 256..270, 15 merges in rank order).  tokenizer_test.mojo
    encodes "Hallo Mojo" and expects the round trip.  By hand: H+a (rank 0),
    Ha+l (1), Hal+l (2), Hall+o (3) give "Hallo"; of the pairs left, M+o (rank
    4) beats " "+M (rank 7), then Mo+j (5) and Moj+o (6) give "Mojo"; no rank
    joins " " with "Mojo".  So the ids are [Hallo 259, " " 32, Mojo 262]."""
    from mojostream_amd.tokenizer import BPETokenizer
    raw = open(GOLDEN_VOCAB, "rb").read()
    assert len(raw) == 1252
    magic, n_tok, n_merge, _ = struct.unpack_from("<IIII", raw, 0)
    assert (magic, n_tok, n_merge) == (0x4256534D, 114, 15)
    t = BPETokenizer(GOLDEN_VOCAB)
    assert t.n_tokens() == 271
    ids = t.encode("Hallo Mojo")
    assert ids == [259, 32, 262]
    assert [t.token_str(i) for i in ids] == ["Hallo", " ", "Mojo"]
    assert t.decode(ids) == "Hallo Mojo"
    assert t.decode([1] + ids + [2]) == "Hallo Mojo"      # BOS / EOS skipped
    for c in range(32, 127):
        assert t.encode(chr(c)) == [c]
    assert t.token_str(100) == "d" and t.token_str(200) == "<unk>"  # gap 127..255
    assert t.token_str(-1) == "oj"                        # id 270, the last one
    assert t.encode("Hello") == [72, 101, 269]            # l+l (rank 11), then ll+o (13)
    assert t.encode("é") == [0, 0]                         # two UTF-8 bytes, both unknown
    # the restatement reads the same file the same way
    vocab, id_to_tok, merges = ref.load(GOLDEN_VOCAB)
    for text in ("Hallo Mojo", " Mojo Hallo", "llo all Mo", "HaHal Hall", ""):
        assert t.encode(text) == ref.encode(text.encode(), merges, vocab)
    t.close()


def test_token_map(tmp_path):
    from mojostream_amd.tokenizer import load_token_map
    words = [b"<pad>", b"<eos>", b"Hallo", b" Welt", b"!"]
    p = str(tmp_path / "vocab_proto.bin")
    with open(p, "wb") as f:
        f.write(struct.pack("<I", len(words)))
        for w in words:
            f.write(struct.pack("<I", len(w)) + w)
    m = load_token_map(p)
    assert m.n_tokens == 5
    assert m.decode(2) == "Hallo"
    assert m.decode_sequence([2, 3, 4]) == "Hallo Welt!"
    assert m.decode(5) == "[?:5]" and m.decode(-3) == "[?:-3]"
    assert m.is_eos(1) and not m.is_eos(2)
    m.close()
