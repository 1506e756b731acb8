"""CPU restatement of the demo BPE tokenizer (src/nlp/tokenizer.mojo:103-163).

TEST INFRASTRUCTURE ONLY: tests/ use it to check the library's tokenizer; the
product never imports it.  Tokens are lists of byte values, as the reference's
chr(byte) strings are.  Pinned by hand-worked merge sequences in
tests/test_tokenizer.py (rank order, leftmost tie, chained merges, unknown
tokens) before it is used on random text.
"""
from typing import Dict, List, Sequence, Tuple


def encode(text: bytes, merges: Sequence[Tuple[bytes, bytes]], vocab: Dict[bytes, int],
           unk: int = 0) -> List[int]:
    """:103-150: bytes, then the lowest-rank pair (leftmost on ties) merged until
    none has a rank; strings missing from the vocabulary give unk."""
    rank = {}
    for r, (a, b) in enumerate(merges):
        rank[a + b"|" + b] = r
    toks = [bytes([c]) for c in text]
    while True:
        best, best_rank = -1, 999_999_999
        for k in range(len(toks) - 1):
            r = rank.get(toks[k] + b"|" + toks[k + 1])
            if r is not None and r < best_rank:
                best, best_rank = k, r
        if best < 0:
            break
        toks[best:best + 2] = [toks[best] + toks[best + 1]]
    return [vocab.get(t, unk) for t in toks]


def decode(ids: Sequence[int], id_to_tok: Sequence[bytes]) -> bytes:
    """:152-163: ids 1, 2, 3 skipped; ids past the table skipped."""
    out = b""
    for i in ids:
        if i in (1, 2, 3) or i >= len(id_to_tok):
            continue
        out += id_to_tok[i]
    return out


def load(path: str):
    """An .msvocab file (BPETokenizer.load :56-101; format of
    scripts/create_vocab.py:7-21): header magic "MSVB", n_tokens, n_merges,
    reserved; n_tokens (id, len, bytes); n_merges (len, left, len, right) in
    rank order.  Returns (vocab bytes -> id, id table with "<unk>" in the gaps,
    merges)."""
    import struct
    raw = open(path, "rb").read()
    magic, n_tok, n_merge, _ = struct.unpack_from("<IIII", raw, 0)
    if magic != 0x4256534D:
        raise ValueError("invalid magic")
    pos = 16
    vocab, table = {}, []
    for _ in range(n_tok):
        i, n = struct.unpack_from("<II", raw, pos)
        pos += 8
        s = raw[pos:pos + n]
        pos += n
        while len(table) <= i:
            table.append(b"<unk>")
        table[i] = s
        vocab[s] = i
    merges = []
    for _ in range(n_merge):
        (n,) = struct.unpack_from("<I", raw, pos)
        left = raw[pos + 4:pos + 4 + n]
        pos += 4 + n
        (n,) = struct.unpack_from("<I", raw, pos)
        right = raw[pos + 4:pos + 4 + n]
        pos += 4 + n
        merges.append((left, right))
    return vocab, table, merges
