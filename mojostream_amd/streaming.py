"""Host mirror of the reference's src/streaming/ over the C ABI.

- MojoStreamFile: the .mojostream reader (mojostream.mojo:95-219) with
  tensor_ptr / ple_scale / validate_gemma4_shape and the TensorGuard of
  StreamingRunner (stream_runner.mojo:313-380), both layer-type-aware so that
  E4B files (sliding hd 256, full hd 512) pass.
- write_synthetic / write_synthetic_lm_head: seeded generators of the file
  format (create_fake_model.py:188-281) and of the version-1 tied LM head.
- load_model: file -> model with weights resident in HBM or streamed from
  pinned host memory (run_harness harness.mojo:80-122, StreamingRunner).
- build_pinned_mask: SparsePinEngine's pinning policy (sparse_pin.mojo:49-85).

Every failure raises MSError with the library's message.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np

from . import (MS_CACHE_CIRCULAR, MS_CACHE_LINEAR, Arch, FileEntry, FileLayer, FileMeta,
               FileValidation, LayerDesc, Model, MSError, check, lib)

MS_PLE, MS_Q, MS_K, MS_V, MS_O, MS_GATE, MS_UP, MS_DOWN = range(8)
TENSORS_PER_LAYER = 8
HDR_BYTES = 128
DIR_E_BYTES = 32
MS_PAGE = 4096
TYPE_NAMES = ("PLE", "Q", "K", "V", "O", "Gate", "Up", "Down")

_lib = lib()


@dataclass
class TensorRef:
    """tensor_ptr result (TensorRef, mojostream.mojo:36-45): host address, scale, bytes."""
    ptr: int
    scale: float
    nbytes: int


class MojoStreamFile:
    """An opened .mojostream file held whole in host memory."""

    def __init__(self, path: str):
        h = C.c_void_p()
        check(_lib.ms_file_open(os.fsencode(path), C.byref(h)))
        self.h = h.value
        self.path = path
        self.meta = FileMeta()
        check(_lib.ms_file_get_meta(self.h, C.byref(self.meta)))

    def close(self) -> None:
        if self.h:
            _lib.ms_file_close(self.h)
            self.h = None

    def __enter__(self) -> "MojoStreamFile":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def entries(self) -> List[FileEntry]:
        out = []
        for i in range(self.meta.n_tensors):
            e = FileEntry()
            check(_lib.ms_file_get_entry(self.h, i, C.byref(e)))
            out.append(e)
        return out

    def tensor_ptr(self, layer: int, mat_type: int) -> TensorRef:
        p = C.c_void_p()
        s = C.c_float()
        n = C.c_size_t()
        check(_lib.ms_file_tensor(self.h, layer, mat_type, C.byref(p), C.byref(s), C.byref(n)))
        return TensorRef(p.value or 0, float(s.value), int(n.value))

    def tensor_array(self, layer: int, mat_type: int) -> np.ndarray:
        """Row-major Q4 bytes [rows][cols/2] of one matrix (a copy)."""
        ref = self.tensor_ptr(layer, mat_type)
        info = self.layer_info(layer)
        D, F = self.meta.hidden, self.meta.ffn_dim
        rows = {MS_Q: D, MS_K: D, MS_V: D, MS_O: info["q_dim"], MS_GATE: D, MS_UP: D,
                MS_DOWN: F}[mat_type]
        buf = (C.c_uint8 * ref.nbytes).from_address(ref.ptr)
        return np.frombuffer(buf, dtype=np.uint8).reshape(rows, -1).copy()

    def ple_scale(self, layer: int) -> float:
        v = C.c_float()
        check(_lib.ms_file_ple_scale(self.h, layer, C.byref(v)))
        return float(v.value)

    def file_size_mb(self) -> float:
        return self.meta.file_bytes / 1e6

    def load_time_ms(self) -> float:
        return self.meta.load_ms

    def validate_gemma4_shape(self) -> None:
        """ShapeGuard."""
        check(_lib.ms_file_shape_guard(self.h))

    def validate_tensor_entries(self) -> None:
        """TensorGuard: order, shapes per layer type, alignment, bounds, scale."""
        check(_lib.ms_file_tensor_guard(self.h))

    def dir_checksum(self) -> int:
        """compute_dir_checksum (src/tests/validate_real.mojo:78-83): XOR of
        the scale fields' 32-bit patterns over the directory."""
        v = C.c_uint32()
        check(_lib.ms_file_dir_checksum(self.h, C.byref(v)))
        return int(v.value)

    def validate(self) -> dict:
        """The structural checks of run_validation (src/tests/validate_real.mojo
        :110-260): counts, the failed checks and the directory checksum."""
        v = FileValidation()
        check(_lib.ms_file_validate(self.h, C.byref(v)))
        names = ["magic", "architecture", "engram", "n_tensors", "offsets", "checksum",
                 "spot L0 Q", "spot L0 Gate", "spot L20 Q", "spot L20 Gate", "spot L41 Q",
                 "spot L41 Gate"]
        return dict(passed=bool(v.passed), n_checks=v.n_checks, n_failed=v.n_failed,
                    failed=[n for i, n in enumerate(names) if v.failed_mask >> i & 1],
                    checksum=int(v.dir_checksum), checksum_hex=f"0x{v.dir_checksum:08X}",
                    file_bytes=int(v.file_bytes), message=v.message.decode(errors="replace"))

    def set_layer_types(self, is_full: Optional[Sequence[bool]]) -> None:
        if is_full is None:
            check(_lib.ms_file_set_layer_types(self.h, None, 0))
            return
        a = np.asarray(is_full, dtype=np.uint8)
        check(_lib.ms_file_set_layer_types(self.h, a.ctypes.data, len(a)))

    def layer_info(self, layer: int) -> dict:
        o = FileLayer()
        check(_lib.ms_file_layer_info(self.h, layer, C.byref(o)))
        return dict(is_full=bool(o.is_full), head_dim=o.head_dim, q_dim=o.q_dim,
                    kv_dim=o.kv_dim)

    def arch(self, max_len: int = 4096, vocab: int = 0) -> Arch:
        """Model shapes for this file.  Hybrid files take the E4B attention
        constants (gemma4_e4b.mojo:33-55): sliding layers RoPE theta 1e4 over
        the whole head and a circular cache of the sliding window; full layers
        theta 1e6 over a quarter of the head and a linear cache of `max_len`
        positions whose reads clamp.  Other files get the demo layer
        (main.mojo:230-301): theta 1e4, whole-head RoPE, linear cache."""
        m = self.meta
        layers = []
        hybrid = m.engram_version != 0 and m.full_kv_dim not in (0, m.sliding_kv_dim)
        for l in range(m.n_layers):
            i = self.layer_info(l)
            hd = i["head_dim"]
            if hybrid and i["is_full"]:
                d = LayerDesc(q_dim=i["q_dim"], kv_dim=i["kv_dim"], head_dim=hd,
                              n_heads=m.n_heads, n_kv_heads=m.n_kv_heads, rot_dim=hd // 4,
                              theta=1e6, cache_kind=MS_CACHE_LINEAR, cache_len=max_len,
                              clamp_reads=1)
            elif hybrid:
                d = LayerDesc(q_dim=i["q_dim"], kv_dim=i["kv_dim"], head_dim=hd,
                              n_heads=m.n_heads, n_kv_heads=m.n_kv_heads, rot_dim=hd,
                              theta=1e4, cache_kind=MS_CACHE_CIRCULAR,
                              cache_len=m.sliding_window or 512, clamp_reads=0)
            else:
                d = LayerDesc(q_dim=i["q_dim"], kv_dim=i["kv_dim"], head_dim=hd,
                              n_heads=m.n_heads, n_kv_heads=m.n_kv_heads, rot_dim=hd,
                              theta=1e4, cache_kind=MS_CACHE_LINEAR, cache_len=max_len,
                              clamp_reads=0)
            layers.append(d)
        return Arch(os.path.basename(self.path), m.hidden, m.ffn_dim, layers, vocab)


def write_synthetic(path: str, n_layers: int, hidden: int, kv_dim: int, ffn: int,
                    n_heads: int, n_kv_heads: int, seed: int = 42,
                    full_kv_dim: int = 0, sliding_window: int = 0, ple_dim: int = 0,
                    is_full: Optional[Sequence[bool]] = None) -> None:
    """Seeded .mojostream file.  full_kv_dim > 0 writes the Engram extension
    (format tag 2) of a hybrid model; the default full-attention layers are
    (layer+1) % 6 == 0."""
    m = FileMeta(n_layers=n_layers, hidden=hidden, kv_dim=kv_dim, ffn_dim=ffn,
                 n_heads=n_heads, n_kv_heads=n_kv_heads)
    if full_kv_dim:
        m.format_tag = 2
        m.engram_version = 1
        m.sliding_kv_dim = kv_dim
        m.full_kv_dim = full_kv_dim
        m.sliding_window = sliding_window
        m.ple_dim = ple_dim
    flags = None
    if is_full is not None:
        flags = np.asarray(is_full, dtype=np.uint8)
    check(_lib.ms_file_write_synthetic(os.fsencode(path), C.byref(m),
                                       None if flags is None else flags.ctypes.data, seed))


def write_synthetic_e4b(path: str, n_layers: int = 42, seed: int = 42) -> None:
    """E4B-shaped file: D 2560, F 10240, 8 q / 2 kv heads, hd 256 / 512."""
    write_synthetic(path, n_layers, 2560, 512, 10240, 8, 2, seed, full_kv_dim=1024,
                    sliding_window=512, ple_dim=256)


def write_synthetic_lm_head(path: str, hidden: int, vocab: int, seed: int = 42) -> None:
    check(_lib.ms_lm_head_file_write_synthetic(os.fsencode(path), hidden, vocab, seed))


def load_model(path: str, lm_head_path: Optional[str] = None, vocab: int = 0,
               max_seqs: int = 1, max_rows: int = 1, max_pos: int = 4096,
               max_len: int = 4096, resident: bool = True,
               pinned: Optional[Sequence[bool]] = None) -> Model:
    """Open, guard and bind a .mojostream file (and optionally its LM head).
    A streaming model (resident=False) may keep the layers flagged in
    `pinned` in HBM (build_pinned_mask gives SparsePinEngine's choice)."""
    with MojoStreamFile(path) as f:
        f.validate_gemma4_shape()
        f.validate_tensor_entries()
        model = Model(f.arch(max_len=max_len, vocab=vocab), max_seqs=max_seqs,
                      max_rows=max_rows, max_pos=max_pos, resident=resident, pinned=pinned)
        try:
            model.load_file(f)
            if lm_head_path:
                model.load_lm_head_file(lm_head_path)
        except Exception:
            model.close()
            raise
    return model


def is_full_attn(layer: int) -> bool:
    """gemma4_e4b.mojo:60-63."""
    return (layer + 1) % 6 == 0


def build_pinned_mask(n_layers: int = 42, n_bridge_front: int = 4, n_bridge_back: int = 2,
                      n_filler: int = 11) -> List[bool]:
    """SparsePinEngine's pinning policy (sparse_pin.mojo:49-85): every
    full-attention layer; the first `n_bridge_front` layers and the last
    `n_bridge_back` sliding layers (0-3 and 39, 40 for E4B); then every second
    remaining sliding layer, up to `n_filler` of them.  The defaults pin 24 of
    42 E4B layers.  The fillers follow the reference's code (4, 7, 9, 12, 14,
    16, 19, 21, 24, 26, 28), not the list in its comment."""
    mask = [is_full_attn(l) for l in range(n_layers)]
    for l in range(min(n_bridge_front, n_layers)):
        mask[l] = True
    back = [l for l in range(n_layers) if not is_full_attn(l)][-n_bridge_back:] \
        if n_bridge_back > 0 else []
    for l in back:
        mask[l] = True
    candidates = [l for l in range(n_layers) if not mask[l] and not is_full_attn(l)]
    for l in candidates[0::2][:n_filler]:
        mask[l] = True
    return mask


def next_non_pinned(from_layer: int, mask: Sequence[bool]) -> int:
    """sparse_pin.mojo:88-92: the next streamed layer after `from_layer`, or -1."""
    for l in range(from_layer + 1, len(mask)):
        if not mask[l]:
            return l
    return -1
