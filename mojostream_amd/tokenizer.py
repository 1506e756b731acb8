"""Tokenizers over the C ABI (host only): BPETokenizer (src/nlp/tokenizer.mojo:31-180)
and TokenMap (src/tokenizer/gemma_proto.mojo:20-74).

The reference builds text from chr(byte), one code point per byte; these
wrappers return the same str by reading the library's bytes as Latin-1, and
encode a str by its UTF-8 bytes, as the reference iterates the bytes of its
UTF-8 String.
"""
from __future__ import annotations

import ctypes as C
from typing import List, Sequence

import numpy as np

from . import _lib, check

BOS_ID, EOS_ID, UNK_ID, PAD_ID = 1, 2, 0, 3


def _text(call) -> str:
    """Run a (out, cap, len) call twice: once for the size, once to fill."""
    n = C.c_int()
    rc = call(None, 0, C.byref(n))
    if rc == 0 and n.value == 0:
        return ""
    buf = C.create_string_buffer(max(n.value, 1))
    check(call(buf, n.value, C.byref(n)))
    return buf.raw[:n.value].decode("latin-1")


class BPETokenizer:
    """The demo BPE tokenizer loaded from an .msvocab file."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(_lib.ms_tokenizer_load(path.encode(), C.byref(h)))
        self.h = h.value
        self.bos_id, self.eos_id, self.unk_id, self.pad_id = BOS_ID, EOS_ID, UNK_ID, PAD_ID

    def close(self) -> None:
        if self.h:
            _lib.ms_tokenizer_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def n_tokens(self) -> int:
        n = C.c_int()
        check(_lib.ms_tokenizer_vocab_size(self.h, C.byref(n)))
        return n.value

    def encode(self, text: str) -> List[int]:
        b = text.encode("utf-8")
        n = C.c_int()
        check(_lib.ms_tokenizer_encode(self.h, b, len(b), None, 0, C.byref(n)))
        ids = np.zeros(max(n.value, 1), np.int32)
        check(_lib.ms_tokenizer_encode(self.h, b, len(b), ids.ctypes.data, len(ids), C.byref(n)))
        return [int(x) for x in ids[:n.value]]

    def decode(self, ids: Sequence[int]) -> str:
        a = np.ascontiguousarray(ids, np.int32)
        return _text(lambda o, cap, ln: _lib.ms_tokenizer_decode(self.h, a.ctypes.data, len(a),
                                                                  o, cap, ln))

    def token_str(self, id: int) -> str:
        return _text(lambda o, cap, ln: _lib.ms_tokenizer_token_str(self.h, int(id), o, cap, ln))


class TokenMap:
    """id -> text table loaded from vocab_proto.bin (load_token_map)."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(_lib.ms_token_map_load(path.encode(), C.byref(h)))
        self.h = h.value
        n = C.c_int()
        check(_lib.ms_token_map_size(self.h, C.byref(n)))
        self.n_tokens = n.value

    def close(self) -> None:
        if self.h:
            _lib.ms_token_map_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def decode(self, token_id: int) -> str:
        return _text(lambda o, cap, ln: _lib.ms_token_map_decode(self.h, int(token_id), o, cap,
                                                                 ln))

    def decode_sequence(self, ids: Sequence[int]) -> str:
        return "".join(self.decode(i) for i in ids)

    def is_eos(self, token_id: int) -> bool:
        return token_id == 1


def load_token_map(path: str) -> TokenMap:
    return TokenMap(path)
