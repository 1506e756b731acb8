"""Python binding of libms_gpu.so (the C ABI in include/ms_gpu.h).

This is the host-side plumbing the tests and bench.py use; the product is the
C ABI and the HIP kernels behind it.  Importing this package does not touch
the GPU.  Every wrapper raises MSError with ms_last_error() on a nonzero
status, mirroring the reference's fail-fast loaders (`raise Error(msg)`,
stream_runner.mojo:210-226).  If libms_gpu.so has not been built the import
fails loudly: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libms_gpu.so")

MS_CACHE_LINEAR = 0
MS_CACHE_CIRCULAR = 1
MAT_NAMES = ("Q", "K", "V", "O", "Gate", "Up", "Down")


class MSError(RuntimeError):
    """Nonzero status from the C ABI; message is ms_last_error()."""


if not os.path.exists(LIB_PATH):
    raise ImportError(
        f"{LIB_PATH} is missing: build the HIP library first "
        "(python -c 'import __graft_entry__ as g; g.build()'). "
        "There is no CPU fallback for the product path.")

_lib = C.CDLL(LIB_PATH)


class LayerDesc(C.Structure):
    _fields_ = [("q_dim", C.c_int), ("kv_dim", C.c_int), ("head_dim", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("rot_dim", C.c_int),
                ("theta", C.c_float), ("cache_kind", C.c_int), ("cache_len", C.c_int),
                ("clamp_reads", C.c_int)]


class ModelDesc(C.Structure):
    _fields_ = [("hidden", C.c_int), ("ffn", C.c_int), ("n_layers", C.c_int),
                ("vocab", C.c_int), ("max_seqs", C.c_int), ("max_rows", C.c_int),
                ("max_pos", C.c_int), ("resident", C.c_int)]


class StreamStats(C.Structure):
    _fields_ = [("io_ms", C.c_double), ("compute_ms", C.c_double),
                ("wait_ms", C.c_double), ("total_ms", C.c_double), ("bytes", C.c_double),
                ("layers_streamed", C.c_int), ("layers_pinned", C.c_int)]


class FileMeta(C.Structure):
    """ms_file_meta: MojoStreamMeta (mojostream.mojo:47-69) + Engram fields."""
    _fields_ = [(n, C.c_uint32) for n in ("version", "format_tag", "n_layers", "hidden",
                                          "kv_dim", "ffn_dim", "n_heads", "n_kv_heads")] + \
               [(n, C.c_uint64) for n in ("n_tensors", "dir_offset", "data_start")] + \
               [(n, C.c_uint32) for n in ("engram_version", "n_kv_shared", "sliding_kv_dim",
                                          "full_kv_dim", "ple_dim", "sliding_window")] + \
               [("file_bytes", C.c_uint64), ("load_ms", C.c_double)]


class FileEntry(C.Structure):
    """ms_file_entry: TensorEntry (mojostream.mojo:73-91)."""
    _fields_ = [("layer_id", C.c_uint32), ("mat_type", C.c_uint32), ("rows", C.c_uint32),
                ("cols", C.c_uint32), ("scale", C.c_float), ("flags", C.c_uint32),
                ("data_offset", C.c_uint64)]


class FileValidation(C.Structure):
    """ms_file_validation: the structural checks of run_validation
    (src/tests/validate_real.mojo:110-260)."""
    _fields_ = [("passed", C.c_int), ("n_checks", C.c_int), ("n_failed", C.c_int),
                ("failed_mask", C.c_uint32), ("dir_checksum", C.c_uint32),
                ("file_bytes", C.c_uint64), ("message", C.c_char * 256)]


class FileLayer(C.Structure):
    _fields_ = [("is_full", C.c_int), ("head_dim", C.c_int), ("q_dim", C.c_int),
                ("kv_dim", C.c_int)]


_P = C.c_void_p
_I = C.c_int
_SZ = C.c_size_t
_F = C.c_float
_U64 = C.c_uint64
_IP = C.POINTER(C.c_int)

_SIGS = {
    "ms_init": [_I], "ms_shutdown": [], "ms_synchronize": [],
    "ms_device_info": [C.c_char_p, _SZ, _IP, C.POINTER(C.c_size_t)],
    "ms_malloc": [C.POINTER(C.c_void_p), _SZ], "ms_free": [_P],
    "ms_memcpy_h2d": [_P, _P, _SZ], "ms_memcpy_d2h": [_P, _P, _SZ],
    "ms_memcpy_d2d": [_P, _P, _SZ], "ms_memset": [_P, _I, _SZ],
    "ms_host_alloc": [C.POINTER(C.c_void_p), _SZ], "ms_host_free": [_P],
    "ms_fill_random_u8": [_P, _SZ, _U64, _U64],
    "ms_fill_random_q4": [_P, _SZ, _U64, _U64, _I],
    "ms_q4_pack": [_P, _P, _I, _I], "ms_host_q4_pack": [_P, _P, _I, _I],
    "ms_dequant_q4": [_P, _P, _I, _I, _F], "ms_dequant_q4_packed": [_P, _P, _I, _I, _F],
    "ms_q4_matmul": [_P, _P, _P, _I, _I, _I, _F, _I],
    "ms_q4_matmul_noalloc": [_P, _P, _P, _I, _I, _I, _F, _I],
    "ms_bench_q4_matmul": [_P, _P, _P, _SZ, _I, _I, _I, _I, _F, _I, C.POINTER(C.c_double)],
    "ms_rmsnorm": [_P, _I, _I], "ms_rmsnorm_weighted": [_P, _P, _I, _I],
    "ms_ple_scale": [_P, _SZ, _F], "ms_swiglu": [_P, _P, _SZ],
    "ms_rope": [_P, _I, _I, _I, _I, _I, _F, _I],
    "ms_attention": [C.POINTER(LayerDesc), _P, _P, _P, _P, _P, _I, _I, _P],
    "ms_lm_head_argmax": [_P, _I, _I, _P, _I, _F, _P, _P],
    "ms_sample": [_P, _I, _F, _P, _I, _F, _U64, _P],
    "ms_embed_q4": [_P, _I, _I, _F, _P, _I, _P],
    "ms_model_create": [C.POINTER(ModelDesc), C.POINTER(LayerDesc), C.POINTER(C.c_void_p)],
    "ms_model_destroy": [_P],
    "ms_model_set_matrix": [_P, _I, _I, _P, _I, _F],
    "ms_model_set_ple": [_P, _I, _F],
    "ms_model_set_lm_head": [_P, _P, _I, _F, _P],
    "ms_model_reset": [_P],
    "ms_layer_forward": [_P, _I, _P, _I, _I, _IP],
    "ms_forward": [_P, _P, _I, _I, _IP, _P],
    "ms_decode_begin": [_P, _I, _P, _P],
    "ms_decode_run": [_P, _I, _I, _P],
    "ms_prefill": [_P, _I, _P, _I, _I, _P],
    "ms_model_stream_stats": [_P, C.POINTER(StreamStats)],
    "ms_model_get_desc": [_P, C.POINTER(ModelDesc), C.POINTER(LayerDesc)],
    "ms_model_set_bos": [_P, _P],
    "ms_model_set_sampling": [_P, _F, _F, _U64],
    "ms_model_set_pinned": [_P, _P],
    "ms_model_set_taps": [_P, _P, _P],
    "ms_model_set_forward_graphs": [_P, _I],
    "ms_model_read_kv": [_P, _I, _I, _I, _I, _P, _P],
    "ms_file_open": [C.c_char_p, C.POINTER(C.c_void_p)], "ms_file_close": [_P],
    "ms_file_get_meta": [_P, C.POINTER(FileMeta)],
    "ms_file_get_entry": [_P, _I, C.POINTER(FileEntry)],
    "ms_file_set_layer_types": [_P, _P, _I],
    "ms_file_layer_info": [_P, _I, C.POINTER(FileLayer)],
    "ms_file_tensor": [_P, _I, _I, C.POINTER(C.c_void_p), C.POINTER(C.c_float),
                       C.POINTER(C.c_size_t)],
    "ms_file_ple_scale": [_P, _I, C.POINTER(C.c_float)],
    "ms_file_shape_guard": [_P], "ms_file_tensor_guard": [_P],
    "ms_file_dir_checksum": [_P, C.POINTER(C.c_uint32)],
    "ms_file_validate": [_P, C.POINTER(FileValidation)],
    "ms_file_write_synthetic": [C.c_char_p, C.POINTER(FileMeta), _P, _U64],
    "ms_model_load_file": [_P, _P],
    "ms_model_load_lm_head_file": [_P, C.c_char_p],
    "ms_lm_head_file_write_synthetic": [C.c_char_p, _I, _I, _U64],
    "ms_lm_head_file_write_synthetic_v2": [C.c_char_p, _I, _I, _U64],
    "ms_matmul_f32": [_P, _P, _P, _I, _I, _I, _I],
    "ms_q4_quantize": [_P, _P, _P, _I, _I, _I, _I],
    "ms_tokenizer_load": [C.c_char_p, _P], "ms_tokenizer_free": [_P],
    "ms_tokenizer_vocab_size": [_P, _P],
    "ms_tokenizer_encode": [_P, C.c_char_p, _I, _P, _I, _P],
    "ms_tokenizer_decode": [_P, _P, _I, _P, _I, _P],
    "ms_tokenizer_token_str": [_P, _I, _P, _I, _P],
    "ms_token_map_load": [C.c_char_p, _P], "ms_token_map_free": [_P],
    "ms_token_map_size": [_P, _P], "ms_token_map_decode": [_P, _I, _P, _I, _P],
    "ms_model_set_lm_head_f32": [_P, _P, _I, _P],
    "ms_runner_create": [C.c_char_p, _I, _I, C.POINTER(C.c_void_p)],
    "ms_runner_destroy": [_P],
    "ms_runner_load_into_slot": [_P, _I, _I, C.POINTER(C.c_double)],
    "ms_runner_set_active": [_P, _I], "ms_runner_active": [_P, _IP],
    "ms_runner_compute_active": [_P, _P, _P, _I, C.POINTER(C.c_double)],
    "ms_runner_run_pipeline": [_P, _P, _P, _I, _P, _P],
    "ms_prof_enable": [_I],
    "ms_prof_sweep": [_P, _I, _I, C.POINTER(C.c_double), C.POINTER(C.c_double),
                      C.POINTER(C.c_long)],
    "ms_prof_get": [_I, C.POINTER(C.c_char_p), C.POINTER(C.c_long),
                    C.POINTER(C.c_double), C.POINTER(C.c_double)],
}
for _name, _args in _SIGS.items():
    _fn = getattr(_lib, _name)
    _fn.argtypes = _args
    _fn.restype = C.c_int
_lib.ms_last_error.restype = C.c_char_p
_lib.ms_last_error.argtypes = []
_lib.ms_q4_packed_bytes.restype = C.c_size_t
_lib.ms_q4_packed_bytes.argtypes = [_I, _I]
_lib.ms_host_fill_random_u8.restype = None
_lib.ms_host_fill_random_u8.argtypes = [_P, _SZ, _U64, _U64]
_lib.ms_host_fill_random_q4.restype = None
_lib.ms_host_fill_random_q4.argtypes = [_P, _SZ, _U64, _U64, _I]
_lib.ms_host_uniform.restype = C.c_float
_lib.ms_host_uniform.argtypes = [_U64, _U64, _U64, _F, _F]
_lib.ms_host_fill_normal.restype = None
_lib.ms_host_fill_normal.argtypes = [_P, _SZ, _U64, _U64]
_lib.ms_sample_seed.restype = _U64
_lib.ms_sample_seed.argtypes = [_U64, _I, _U64]

EXPORTED = sorted(_SIGS) + ["ms_last_error", "ms_q4_packed_bytes", "ms_host_fill_random_u8",
                            "ms_host_fill_random_q4", "ms_host_uniform",
                            "ms_host_fill_normal", "ms_sample_seed"]


def lib():
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise MSError(f"[{rc}] {_lib.ms_last_error().decode(errors='replace')}")


def init(device: int = 0) -> None:
    check(_lib.ms_init(device))


def shutdown() -> None:
    check(_lib.ms_shutdown())


def synchronize() -> None:
    check(_lib.ms_synchronize())


def device_info():
    name = C.create_string_buffer(256)
    ncu = C.c_int()
    hbm = C.c_size_t()
    check(_lib.ms_device_info(name, 256, C.byref(ncu), C.byref(hbm)))
    return name.value.decode(), ncu.value, hbm.value


# ---- host-side seeded data (identical to the device generator) -------------
Q4_DTYPES = {"F32": 0, "BF16": 1, "F16": 2}


def q4_quantize(d_w: "DeviceBuffer", dtype: int, n_out: int, n_in: int,
                block_size: int = 32):
    """quantize_q4_blockwise (scripts/convert.py:296-323) of a device weight
    [n_out][n_in] (HuggingFace layout) after the converter's transpose: returns
    (device buffer of [n_in][n_out/2] Q4 bytes, global scale)."""
    out = DeviceBuffer(n_in * (n_out // 2))
    s = C.c_float()
    check(_lib.ms_q4_quantize(out.ptr, C.byref(s), d_w.ptr, int(dtype), n_out, n_in, block_size))
    return out, float(s.value)


def sample(d_logits: "DeviceBuffer", vocab: int, temperature: float, d_generated,
           n_generated: int, penalty: float, seed: int) -> int:
    """temperature_sampling (lm_head.mojo:198-254) on a device logits row, with
    an explicit seed; the row is modified in place like the reference's."""
    out = C.c_int32()
    gp = d_generated.ptr if d_generated is not None else None
    check(_lib.ms_sample(d_logits.ptr, vocab, float(temperature), gp, n_generated,
                         float(penalty), int(seed) & 0xFFFFFFFFFFFFFFFF, C.byref(out)))
    return int(out.value)


def sample_seed(seed: int, seq: int, draw: int) -> int:
    """Seed the model's sampler gives the LCG step of draw `draw` of sequence
    `seq` (ms_sample_seed)."""
    return int(_lib.ms_sample_seed(int(seed) & 0xFFFFFFFFFFFFFFFF, int(seq), int(draw)))


def host_random_u8(n: int, seed: int, stream: int, balanced: bool = False) -> np.ndarray:
    """Seeded bytes (identical to the device generator); balanced: every zero
    nibble becomes 8 (zero-mean Q4 weights, ms_fill_random_q4)."""
    out = np.empty(n, dtype=np.uint8)
    _lib.ms_host_fill_random_q4(out.ctypes.data, n, seed, stream, 1 if balanced else 0)
    return out


def host_uniform(seed: int, stream: int, index: int, lo: float, hi: float) -> float:
    return float(_lib.ms_host_uniform(seed, stream, index, lo, hi))


def host_normal(n: int, seed: int, stream: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _lib.ms_host_fill_normal(out.ctypes.data, n, seed, stream)
    return out


# ---- device buffers ----------------------------------------------------------
class DeviceBuffer:
    """Owned device allocation (ms_malloc / ms_free)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(_lib.ms_malloc(C.byref(p), max(self.nbytes, 1)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            check(_lib.ms_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes))
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(_lib.ms_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes))

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        if out.nbytes:
            check(_lib.ms_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            check(_lib.ms_free(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            if self.ptr:
                _lib.ms_free(self.ptr)
        except Exception:
            pass


# ---- architecture presets -------------------------------------------------------
def demo_layer(D: int, n_heads: int, n_kv: int, max_len: int, theta: float = 1e4) -> LayerDesc:
    """Demo / 14B layer: hd = D/n_heads, linear KVCache (main.mojo:257-301)."""
    hd = D // n_heads
    return LayerDesc(q_dim=D, kv_dim=n_kv * hd, head_dim=hd, n_heads=n_heads,
                     n_kv_heads=n_kv, rot_dim=hd, theta=theta,
                     cache_kind=MS_CACHE_LINEAR, cache_len=max_len, clamp_reads=0)


def e4b_is_full(layer: int) -> bool:
    """is_full_attn (gemma4_e4b.mojo:60-63): (layer+1) % 6 == 0."""
    return (layer + 1) % 6 == 0


def e4b_layer(layer: int, max_full_seq: int) -> LayerDesc:
    """E4B constants, gemma4_e4b.mojo:33-55."""
    if e4b_is_full(layer):
        return LayerDesc(q_dim=4096, kv_dim=1024, head_dim=512, n_heads=8, n_kv_heads=2,
                         rot_dim=128, theta=1e6, cache_kind=MS_CACHE_LINEAR,
                         cache_len=max_full_seq, clamp_reads=1)
    return LayerDesc(q_dim=2048, kv_dim=512, head_dim=256, n_heads=8, n_kv_heads=2,
                     rot_dim=256, theta=1e4, cache_kind=MS_CACHE_CIRCULAR, cache_len=512,
                     clamp_reads=0)


@dataclass
class Arch:
    name: str
    hidden: int
    ffn: int
    layers: List[LayerDesc]
    vocab: int = 0

    @property
    def n_layers(self) -> int:
        return len(self.layers)

    def matrix_shapes(self, l: int):
        d = self.layers[l]
        D, F = self.hidden, self.ffn
        return [(D, d.q_dim), (D, d.kv_dim), (D, d.kv_dim), (d.q_dim, D), (D, F), (D, F),
                (F, D)]

    def layer_bytes(self, l: int) -> int:
        return sum(k * n // 2 for k, n in self.matrix_shapes(l))

    def weight_bytes(self) -> int:
        return sum(self.layer_bytes(l) for l in range(self.n_layers))


def arch_demo(max_len: int = 512, n_layers: int = 40) -> Arch:
    """Demo model: D=1024, 8q/2kv heads, hd 128, F=4096, theta 1e4."""
    return Arch("demo", 1024, 4096, [demo_layer(1024, 8, 2, max_len) for _ in range(n_layers)])


def arch_e4b(max_full_seq: int = 4096, n_layers: int = 42, vocab: int = 262144) -> Arch:
    """Gemma-4-E4B shapes (gemma4_e4b.mojo:33-55), tied Q4 head."""
    return Arch("e4b", 2560, 10240, [e4b_layer(l, max_full_seq) for l in range(n_layers)],
                vocab)


def arch_14b(max_len: int = 4096, n_layers: int = 48, vocab: int = 262144) -> Arch:
    """14B-class: D=5120, 40q/8kv heads, hd 128, F=13824, theta 1e6, all full
    attention; a tied Q4 head of `vocab` ids (0: none).  The layers hold
    6,606,028,800 bytes of Q4 weights, the head 671,088,640 at vocab 262144:
    7.28 GB in all, the "about 7.5 GB" of the 14B configuration."""
    return Arch("14b", 5120, 13824,
                [demo_layer(5120, 40, 8, max_len, theta=1e6) for _ in range(n_layers)], vocab)


# ---- synthetic model (seeded) ------------------------------------------------------
def matrix_stream(layer: int, mat: int) -> int:
    return (layer + 1) * 16 + mat


LM_STREAM = 0xFFFF


# Standard deviation of a balanced nibble minus the zero point: values 1..15
# with 8 twice, sum (n - 8)^2 / 16 = 280 / 16.
BALANCED_NIBBLE_STD = 17.5 ** 0.5


# Gains of the balanced matrices: Q and K 1.0 (attention scores of unit
# spread), V, O, Gate, Up, Down 0.65.
BALANCED_GAINS = (1.0, 1.0, 0.65, 0.65, 0.65, 0.65, 0.65)


def unit_gain_scale(seed: int, stream: int, K: int, gain: float = 1.0) -> float:
    """Scale of a balanced synthetic matrix with K input rows:
    gain * u / (std * sqrt(K)), u ~ U(0.8, 1.2), so a projection scales the
    RMS of its input by about `gain`.
    - With the reference's scale range on zero-mean weights the activations
      grow to the hundreds, attention softmax turns into a near-argmax over
      ties, and fp32 rounding decides which key wins: the model is chaotic and
      no fp32 implementation tracks another.
    - At gain 1 on every matrix a relative perturbation of 1e-6 still grows to
      3e-4 over 42 layers, and the output follows the context, not the token.
    - At 0.5 the network is near the identity and the tied head returns the
      input token.
    The gains of BALANCED_GAINS keep a 1e-6 perturbation near 2e-6 after 42
    layers while the greedy id depends on the token and its context."""
    u = host_uniform(seed, 0x6A1, stream, 0.8, 1.2)
    return float(np.float32(gain * u / (BALANCED_NIBBLE_STD * float(K) ** 0.5)))


def matrix_scale(seed: int, layer: int, mat: int, K: int = 0, balanced: bool = False) -> float:
    """Per-tensor scale U(0.04, 0.15) (create_fake_model.py:95); balanced
    matrices (K input rows) take unit_gain_scale instead."""
    if balanced:
        return unit_gain_scale(seed, matrix_stream(layer, mat), K, BALANCED_GAINS[mat])
    return host_uniform(seed, 0x5CA1E, matrix_stream(layer, mat), 0.04, 0.15)


def layer_ple(seed: int, layer: int) -> float:
    """PLE U(0.8, 1.2) (create_fake_model.py:203)."""
    return host_uniform(seed, 0x91E, layer, 0.8, 1.2)


def lm_scale(seed: int, D: int = 0, balanced: bool = False) -> float:
    if balanced:
        return unit_gain_scale(seed, LM_STREAM, D)
    return host_uniform(seed, 0x5CA1E, LM_STREAM, 0.04, 0.15)


def host_matrix(seed: int, layer: int, mat: int, K: int, N: int,
                balanced: bool = False) -> np.ndarray:
    """Row-major Q4 bytes [K][N/2] of one synthetic matrix (host copy)."""
    return host_random_u8(K * N // 2, seed, matrix_stream(layer, mat),
                          balanced).reshape(K, N // 2)


def host_lm_head(seed: int, D: int, vocab: int, balanced: bool = False) -> np.ndarray:
    return host_random_u8(D * vocab // 2, seed, LM_STREAM, balanced).reshape(D, vocab // 2)


class Model:
    """Owner of an ms_model handle."""

    def __init__(self, arch: Arch, max_seqs: int = 1, max_rows: int = 1,
                 max_pos: int = 4096, resident: bool = True,
                 pinned: Optional[Sequence[bool]] = None):
        self.arch = arch
        self.max_seqs, self.max_rows, self.max_pos = max_seqs, max_rows, max_pos
        desc = ModelDesc(hidden=arch.hidden, ffn=arch.ffn, n_layers=arch.n_layers,
                         vocab=arch.vocab, max_seqs=max_seqs, max_rows=max_rows,
                         max_pos=max_pos, resident=1 if resident else 0)
        arr = (LayerDesc * arch.n_layers)(*arch.layers)
        h = C.c_void_p()
        check(_lib.ms_model_create(C.byref(desc), arr, C.byref(h)))
        self.h = h.value
        self._pinned: List[int] = []
        if pinned is not None:
            flags = np.asarray(pinned, dtype=np.uint8)
            if flags.size != arch.n_layers:
                self.close()
                raise MSError(f"pinned: need {arch.n_layers} flags, got {flags.size}")
            try:
                check(_lib.ms_model_set_pinned(self.h, flags.ctypes.data))
            except MSError:
                self.close()
                raise

    def close(self) -> None:
        if self.h:
            check(_lib.ms_model_destroy(self.h))
            self.h = None
        for p in self._pinned:
            _lib.ms_host_free(p)
        self._pinned = []

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_matrix(self, layer: int, mat: int, q4: np.ndarray, scale: float) -> None:
        q4 = np.ascontiguousarray(q4, dtype=np.uint8)
        check(_lib.ms_model_set_matrix(self.h, layer, mat, q4.ctypes.data, 0, scale))

    def set_matrix_device(self, layer: int, mat: int, dptr: int, scale: float) -> None:
        check(_lib.ms_model_set_matrix(self.h, layer, mat, dptr, 1, scale))

    def set_ple(self, layer: int, ple: float) -> None:
        check(_lib.ms_model_set_ple(self.h, layer, ple))

    def set_lm_head(self, q4: Optional[np.ndarray], scale: float,
                    gamma: Optional[np.ndarray] = None, dptr: Optional[int] = None) -> None:
        g = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.float32)
        gp = None if g is None else g.ctypes.data
        if dptr is not None:
            check(_lib.ms_model_set_lm_head(self.h, dptr, 1, scale, gp))
        else:
            q4 = np.ascontiguousarray(q4, dtype=np.uint8)
            check(_lib.ms_model_set_lm_head(self.h, q4.ctypes.data, 0, scale, gp))

    def fill_synthetic(self, seed: int, balanced: bool = False) -> None:
        """Seeded random Q4 weights generated on the device (no host copy);
        balanced: zero-mean nibbles (ms_fill_random_q4) and unit-gain scales."""
        arch = self.arch
        biggest = max(max(k * n // 2 for k, n in arch.matrix_shapes(l))
                      for l in range(arch.n_layers))
        if arch.vocab:
            biggest = max(biggest, arch.hidden * arch.vocab // 2)
        tmp = DeviceBuffer(biggest)
        try:
            for l in range(arch.n_layers):
                for i, (K, N) in enumerate(arch.matrix_shapes(l)):
                    check(_lib.ms_fill_random_q4(tmp.ptr, K * N // 2, seed,
                                                 matrix_stream(l, i), int(balanced)))
                    self.set_matrix_device(l, i, tmp.ptr, matrix_scale(seed, l, i, K, balanced))
                self.set_ple(l, layer_ple(seed, l))
            if arch.vocab:
                check(_lib.ms_fill_random_q4(tmp.ptr, arch.hidden * arch.vocab // 2, seed,
                                             LM_STREAM, int(balanced)))
                self.set_lm_head(None, lm_scale(seed, arch.hidden, balanced), dptr=tmp.ptr)
            synchronize()
        finally:
            tmp.free()

    def fill_synthetic_host(self, seed: int, balanced: bool = False) -> None:
        """Same weights passed from host memory (streaming models)."""
        arch = self.arch
        for l in range(arch.n_layers):
            for i, (K, N) in enumerate(arch.matrix_shapes(l)):
                self.set_matrix(l, i, host_matrix(seed, l, i, K, N, balanced),
                                matrix_scale(seed, l, i, K, balanced))
            self.set_ple(l, layer_ple(seed, l))
        if arch.vocab:
            self.set_lm_head(host_lm_head(seed, arch.hidden, arch.vocab, balanced),
                             lm_scale(seed, arch.hidden, balanced))

    def read_kv(self, layer: int, seq: int, pos0: int, n: int):
        """K and V rows of positions pos0..pos0+n-1 of a layer's cache (host
        arrays [n][kv_dim])."""
        kvd = self.arch.layers[layer].kv_dim
        dk, dv = DeviceBuffer(max(n, 1) * kvd * 4), DeviceBuffer(max(n, 1) * kvd * 4)
        check(_lib.ms_model_read_kv(self.h, layer, seq, pos0, n, dk.ptr, dv.ptr))
        return dk.download(np.float32, (n, kvd)), dv.download(np.float32, (n, kvd))

    def set_taps(self, hidden: Optional["DeviceBuffer"], logits: Optional["DeviceBuffer"]) -> None:
        """Per-layer output rows and raw logits of decode steps and of a prompt's
        last row written to these device buffers (ms_model_set_taps)."""
        check(_lib.ms_model_set_taps(self.h, hidden.ptr if hidden else None,
                                     logits.ptr if logits else None))

    def reset(self) -> None:
        check(_lib.ms_model_reset(self.h))

    def set_forward_graphs(self, on: bool) -> None:
        """ms_forward's HIP graph replay of repeated calls (on by default)."""
        check(_lib.ms_model_set_forward_graphs(self.h, 1 if on else 0))

    def set_sampling(self, temperature: float, penalty: float = 1.0, seed: int = 0) -> None:
        """temperature_sampling (lm_head.mojo:198-254) in prefill and decode
        instead of the greedy argmax when temperature > 0.01 or penalty > 1;
        the k-th drawing LM head call (prefill's first token, then each decode
        step) draws for sequence b with sample_seed(seed, b, k)."""
        check(_lib.ms_model_set_sampling(self.h, float(temperature), float(penalty),
                                         int(seed) & 0xFFFFFFFFFFFFFFFF))

    def set_bos(self, bos: Optional[np.ndarray]) -> None:
        """BOS row for prompt position 0 (apply_bos_embedding, lm_head.mojo:133-143)."""
        if bos is None:
            check(_lib.ms_model_set_bos(self.h, None))
            return
        b = np.ascontiguousarray(bos, dtype=np.float32)
        if b.size != self.arch.hidden:
            raise MSError(f"set_bos: need {self.arch.hidden} values, got {b.size}")
        check(_lib.ms_model_set_bos(self.h, b.ctypes.data))

    def load_file(self, f) -> None:
        """Guards + bind every matrix and PLE scale of a MojoStreamFile."""
        check(_lib.ms_model_load_file(self.h, f.h))

    def load_lm_head_file(self, path: str) -> None:
        """Tied Q4 head, version 1 (load_lm_head, lm_head.mojo:61-116)."""
        check(_lib.ms_model_load_lm_head_file(self.h, os.fsencode(path)))

    def get_desc(self):
        d = ModelDesc()
        arr = (LayerDesc * self.arch.n_layers)()
        check(_lib.ms_model_get_desc(self.h, C.byref(d), arr))
        return d, list(arr)

    def layer_forward(self, layer: int, x: np.ndarray, base: Sequence[int], T: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        B = len(base)
        d = DeviceBuffer.from_array(x)
        bb = (C.c_int * B)(*base)
        check(_lib.ms_layer_forward(self.h, layer, d.ptr, B, T, bb))
        return d.download(np.float32, x.shape)

    def forward(self, x: np.ndarray, base: Sequence[int], T: int, hidden: bool = False):
        x = np.ascontiguousarray(x, dtype=np.float32)
        B = len(base)
        d = DeviceBuffer.from_array(x)
        bb = (C.c_int * B)(*base)
        hbuf = DeviceBuffer(self.arch.n_layers * x.nbytes) if hidden else None
        check(_lib.ms_forward(self.h, d.ptr, B, T, bb, hbuf.ptr if hbuf else None))
        out = d.download(np.float32, x.shape)
        if hidden:
            return out, hbuf.download(np.float32, (self.arch.n_layers,) + x.shape)
        return out

    def decode(self, tokens: Sequence[int], pos: Sequence[int], n_steps: int,
               use_graph: bool = True) -> np.ndarray:
        B = len(tokens)
        t = np.asarray(tokens, dtype=np.int32)
        p = np.asarray(pos, dtype=np.int32)
        check(_lib.ms_decode_begin(self.h, B, t.ctypes.data, p.ctypes.data))
        out = np.empty((n_steps, B), dtype=np.int32)
        check(_lib.ms_decode_run(self.h, n_steps, 1 if use_graph else 0, out.ctypes.data))
        return out

    def decode_continue(self, n_steps: int, B: int, use_graph: bool = True) -> np.ndarray:
        out = np.empty((n_steps, B), dtype=np.int32)
        check(_lib.ms_decode_run(self.h, n_steps, 1 if use_graph else 0, out.ctypes.data))
        return out

    def prefill(self, tokens: Sequence[int], pos0: int = 0, seq: int = 0) -> int:
        t = np.asarray(tokens, dtype=np.int32)
        first = C.c_int32()
        check(_lib.ms_prefill(self.h, seq, t.ctypes.data, len(t), pos0, C.byref(first)))
        return int(first.value)

    def stream_stats(self) -> dict:
        s = StreamStats()
        check(_lib.ms_model_stream_stats(self.h, C.byref(s)))
        return dict(io_ms=s.io_ms, compute_ms=s.compute_ms, wait_ms=s.wait_ms,
                    total_ms=s.total_ms, bytes=s.bytes, layers_streamed=s.layers_streamed,
                    layers_pinned=s.layers_pinned)


def prof_enable(on: bool) -> None:
    check(_lib.ms_prof_enable(1 if on else 0))


PROF_CLASSES = {"qkv_gemv": 0, "attention": 1, "o_gemv": 2, "gateup_gemv": 3,
                "down_gemv": 4, "lm_head": 5, "embed_prep": 6, "other": 7}


def prof_sweep(model: "Model", cls: str, passes: int = 1) -> dict:
    """Device-side duration of one projection class: its last profiled launch
    re-run back to back over every layer's weights (ms_prof_sweep)."""
    avg = C.c_double()
    by = C.c_double()
    n = C.c_long()
    check(_lib.ms_prof_sweep(model.h, PROF_CLASSES[cls], passes, C.byref(avg), C.byref(by),
                             C.byref(n)))
    return dict(avg_us=avg.value, bytes_per_launch=by.value, launches=n.value)


def prof_get() -> dict:
    out = {}
    for c in range(8):
        name = C.c_char_p()
        n = C.c_long()
        ms = C.c_double()
        by = C.c_double()
        check(_lib.ms_prof_get(c, C.byref(name), C.byref(n), C.byref(ms), C.byref(by)))
        out[name.value.decode()] = dict(launches=n.value, ms=ms.value, bytes=by.value)
    return out
