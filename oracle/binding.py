"""ctypes binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.  The oracle is the
reference the tests compare against; nothing here is on the measured or shipped path.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
OR_CACHE_LINEAR, OR_CACHE_CIRCULAR = 0, 1
OR_MODE_CAUSAL, OR_MODE_WRITE_FIRST = 0, 1


def _load(name: str) -> C.CDLL:
    path = os.path.join(_HERE, name)
    if not os.path.exists(path):
        raise ImportError(f"{path} missing: run `make -C oracle`")
    return C.CDLL(path)


def cpu_has_avx2() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            flags = f.read()
        return " avx2" in flags and " fma" in flags
    except OSError:
        return False


class OrLayer(C.Structure):
    _fields_ = [("q_dim", C.c_int), ("kv_dim", C.c_int), ("head_dim", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("rot_dim", C.c_int),
                ("theta", C.c_float), ("cache_kind", C.c_int), ("cache_len", C.c_int),
                ("clamp_reads", C.c_int), ("w", C.c_void_p * 7), ("scale", C.c_float * 7),
                ("ple", C.c_float), ("kc", C.c_void_p), ("vc", C.c_void_p)]


_P, _I, _F = C.c_void_p, C.c_int, C.c_float
_SIGS = {
    "or_set_threads": ([_I], None),
    "or_dequant_q4": ([_P, _I, _I, _F, _P], None),
    "or_matmul_q4": ([_P, _P, _P, _I, _I, _I, _F], None),
    "or_matmul_q4_f64": ([_P, _P, _P, _I, _I, _I, _F], None),
    "or_rmsnorm": ([_P, _I, _I], None),
    "or_rmsnorm_weighted": ([_P, _P, _I, _I], None),
    "or_ple_scale": ([_P, _I, _F], None),
    "or_swiglu": ([_P, _P, _I], None),
    "or_rope_table": ([_I, _I, _F, _P, _P], None),
    "or_rope": ([_P, _I, _I, _I, _I, _F], None),
    "or_attention": ([C.POINTER(OrLayer), _P, _P, _P, _I, _I, _I, _P], None),
    "or_kv_write": ([C.POINTER(OrLayer), _P, _P, _I, _I], None),
    "or_layer_forward": ([C.POINTER(OrLayer), _I, _I, _P, _I, _I, _I], None),
    "or_lm_head": ([_P, _I, _I, _P, _I, _F, _P], None),
    "or_argmax": ([_P, _I], C.c_int),
    "or_sample": ([_P, _I, _F, _P, _I, _F, C.c_uint64], C.c_int),
    "or_sample_target": ([C.c_uint64], C.c_float),
    "or_matmul_f32": ([_P, _P, _P, _I, _I, _I], None),
    "or_q4_quantize": ([_P, _I, _I, _I, _P, _P], None),
    "or_embed": ([_P, _I, _I, _F, _I, _P], None),
    "or_decode_token": ([C.POINTER(OrLayer), _I, _I, _I, _P, _I, _F, _P, _I, _I, _P],
                        C.c_int),
}


class Oracle:
    def __init__(self, avx2: bool = False, path: Optional[str] = None):
        """avx2 picks the -mavx2 -mfma build when the host has it; path loads
        another build of ms_oracle.c (e.g. one made with -march=native)."""
        if path is not None:
            self.name = os.path.basename(path)
            self.lib = C.CDLL(path)
        else:
            name = "liboracle_avx2.so" if (avx2 and cpu_has_avx2()) else "liboracle.so"
            self.name = name
            self.lib = _load(name)
        for fn, (args, res) in _SIGS.items():
            f = getattr(self.lib, fn)
            f.argtypes = args
            f.restype = res

    # ---- kernels ------------------------------------------------------------------
    def set_threads(self, n: int) -> None:
        self.lib.or_set_threads(int(n))

    def dequant(self, q4: np.ndarray, K: int, N: int, scale: float) -> np.ndarray:
        q4 = np.ascontiguousarray(q4, dtype=np.uint8)
        out = np.empty((K, N), np.float32)
        self.lib.or_dequant_q4(q4.ctypes.data, K, N, scale, out.ctypes.data)
        return out

    def matmul(self, A: np.ndarray, q4: np.ndarray, N: int, scale: float,
               C0: Optional[np.ndarray] = None) -> np.ndarray:
        A = np.ascontiguousarray(A, dtype=np.float32)
        M, K = A.shape
        out = np.zeros((M, N), np.float32) if C0 is None else np.array(C0, np.float32)
        q4 = np.ascontiguousarray(q4, dtype=np.uint8)
        self.lib.or_matmul_q4(out.ctypes.data, A.ctypes.data, q4.ctypes.data, M, K, N, scale)
        return out

    def matmul_f64(self, A: np.ndarray, q4: np.ndarray, N: int, scale: float) -> np.ndarray:
        A = np.ascontiguousarray(A, dtype=np.float32)
        M, K = A.shape
        out = np.zeros((M, N), np.float64)
        q4 = np.ascontiguousarray(q4, dtype=np.uint8)
        self.lib.or_matmul_q4_f64(out.ctypes.data, A.ctypes.data, q4.ctypes.data, M, K, N,
                                  scale)
        return out

    def rmsnorm(self, x: np.ndarray, gamma: Optional[np.ndarray] = None) -> np.ndarray:
        x = np.array(x, np.float32, copy=True)
        rows, cols = x.reshape(-1, x.shape[-1]).shape
        if gamma is None:
            self.lib.or_rmsnorm(x.ctypes.data, rows, cols)
        else:
            g = np.ascontiguousarray(gamma, np.float32)
            self.lib.or_rmsnorm_weighted(x.ctypes.data, g.ctypes.data, rows, cols)
        return x

    def ple_scale(self, x: np.ndarray, s: float) -> np.ndarray:
        x = np.array(x, np.float32, copy=True)
        self.lib.or_ple_scale(x.ctypes.data, x.size, s)
        return x

    def swiglu(self, gate: np.ndarray, up: np.ndarray) -> np.ndarray:
        g = np.ascontiguousarray(gate, np.float32)
        u = np.array(up, np.float32, copy=True)
        self.lib.or_swiglu(g.ctypes.data, u.ctypes.data, u.size)
        return u

    def rope_table(self, rot: int, pos: int, theta: float):
        cs = np.empty(rot // 2, np.float32)
        sn = np.empty(rot // 2, np.float32)
        self.lib.or_rope_table(rot, pos, theta, cs.ctypes.data, sn.ctypes.data)
        return cs, sn

    def rope(self, x: np.ndarray, n_heads: int, head_stride: int, rot: int, pos: int,
             theta: float) -> np.ndarray:
        x = np.array(x, np.float32, copy=True)
        self.lib.or_rope(x.ctypes.data, n_heads, head_stride, rot, pos, theta)
        return x

    def argmax(self, v: np.ndarray) -> int:
        v = np.ascontiguousarray(v, np.float32)
        return int(self.lib.or_argmax(v.ctypes.data, v.size))

    def sample(self, logits: np.ndarray, temperature: float, generated, penalty: float,
               seed: int):
        """temperature_sampling (lm_head.mojo:198-254) with an explicit seed.
        Returns (id, logits after the call: penalized, or probabilities)."""
        v = np.ascontiguousarray(logits, np.float32).copy()
        g = np.ascontiguousarray(np.asarray(generated, np.int32).reshape(-1))
        gp = g.ctypes.data if g.size else None
        tid = self.lib.or_sample(v.ctypes.data, v.size, temperature, gp, g.size, penalty,
                                 int(seed) & 0xFFFFFFFFFFFFFFFF)
        return int(tid), v

    def matmul_f32(self, A: np.ndarray, B: np.ndarray, C0: Optional[np.ndarray] = None):
        """matmul_fp32_raw (kernels.mojo:616-671): C0 + A . B (C0 zeros if None)."""
        A = np.ascontiguousarray(A, np.float32)
        B = np.ascontiguousarray(B, np.float32)
        M, K = A.shape
        N = B.shape[1]
        out = np.zeros((M, N), np.float32) if C0 is None else np.array(C0, np.float32, copy=True)
        self.lib.or_matmul_f32(out.ctypes.data, A.ctypes.data, B.ctypes.data, M, K, N)
        return out

    def q4_quantize(self, w_hf: np.ndarray, block_size: int = 32):
        """quantize_q4_blockwise of w_hf.T (scripts/convert.py:296-323, 503-506):
        returns (packed [n_in][n_out/2] uint8, scale)."""
        w = np.ascontiguousarray(w_hf, np.float32)
        n_out, n_in = w.shape
        packed = np.empty((n_in, n_out // 2), np.uint8)
        s = np.zeros(1, np.float32)
        self.lib.or_q4_quantize(w.ctypes.data, n_out, n_in, block_size, packed.ctypes.data,
                                s.ctypes.data)
        return packed, float(s[0])

    def sample_target(self, seed: int) -> float:
        return float(self.lib.or_sample_target(int(seed) & 0xFFFFFFFFFFFFFFFF))

    def embed(self, wlm: np.ndarray, D: int, vocab: int, scale: float, token: int) -> np.ndarray:
        w = np.ascontiguousarray(wlm, np.uint8)
        out = np.empty(D, np.float32)
        self.lib.or_embed(w.ctypes.data, D, vocab, scale, token, out.ctypes.data)
        return out

    def lm_head(self, x: np.ndarray, wlm: np.ndarray, vocab: int, scale: float) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        M, D = x.shape
        w = np.ascontiguousarray(wlm, np.uint8)
        out = np.empty((M, vocab), np.float32)
        self.lib.or_lm_head(x.ctypes.data, M, D, w.ctypes.data, vocab, scale, out.ctypes.data)
        return out


class OracleModel:
    """A model for one sequence: per-layer OrLayer structs + caches (host)."""

    def __init__(self, oracle: Oracle, arch, weights: List[List[np.ndarray]],
                 scales: List[List[float]], ples: List[float], lm_w=None, lm_scale=0.0,
                 gamma=None):
        self.o = oracle
        self.arch = arch
        self.D, self.F = arch.hidden, arch.ffn
        self.weights = weights  # keep alive
        self.layers = (OrLayer * arch.n_layers)()
        self.caches = []
        for l, d in enumerate(arch.layers):
            L = self.layers[l]
            for f in ("q_dim", "kv_dim", "head_dim", "n_heads", "n_kv_heads", "rot_dim",
                      "theta", "cache_kind", "cache_len", "clamp_reads"):
                setattr(L, f, getattr(d, f))
            for i in range(7):
                L.w[i] = weights[l][i].ctypes.data
                L.scale[i] = scales[l][i]
            L.ple = ples[l]
            kc = np.zeros((d.cache_len, d.kv_dim), np.float32)
            vc = np.zeros((d.cache_len, d.kv_dim), np.float32)
            self.caches.append((kc, vc))
            L.kc = kc.ctypes.data
            L.vc = vc.ctypes.data
        self.lm_w = None if lm_w is None else np.ascontiguousarray(lm_w, np.uint8)
        self.lm_scale = lm_scale
        self.gamma = None if gamma is None else np.ascontiguousarray(gamma, np.float32)

    def layer_forward(self, l: int, x: np.ndarray, base: int,
                      mode: int = OR_MODE_CAUSAL) -> np.ndarray:
        x = np.array(x, np.float32, copy=True)
        T = x.shape[0]
        self.o.lib.or_layer_forward(C.byref(self.layers[l]), self.D, self.F, x.ctypes.data, T,
                                    base, mode)
        return x

    def forward(self, x: np.ndarray, base: int, hidden: bool = False,
                mode: int = OR_MODE_CAUSAL):
        hs = []
        for l in range(self.arch.n_layers):
            x = self.layer_forward(l, x, base, mode)
            if hidden:
                hs.append(x.copy())
        return (x, np.stack(hs)) if hidden else x

    def decode_token(self, token: int, pos: int, hidden: bool = False):
        hbuf = np.empty((self.arch.n_layers, self.D), np.float32) if hidden else None
        g = None if self.gamma is None else self.gamma.ctypes.data
        tid = self.o.lib.or_decode_token(self.layers, self.arch.n_layers, self.D, self.F,
                                         self.lm_w.ctypes.data, self.arch.vocab,
                                         self.lm_scale, g, token, pos,
                                         None if hbuf is None else hbuf.ctypes.data)
        return (int(tid), hbuf) if hidden else int(tid)

    def logits_for(self, x_final: np.ndarray) -> np.ndarray:
        x = self.o.rmsnorm(x_final.reshape(1, -1), self.gamma)
        return self.o.lm_head(x, self.lm_w, self.arch.vocab, self.lm_scale)[0]

    def logits_rows(self, x_final: np.ndarray) -> np.ndarray:
        """Final norm + LM head of many rows [T][D] -> [T][vocab]
        (apply_final_norm + project_lm_head, lm_head.mojo:119-168)."""
        x = self.o.rmsnorm(np.ascontiguousarray(x_final, np.float32), self.gamma)
        return self.o.lm_head(x, self.lm_w, self.arch.vocab, self.lm_scale)

    def embed_rows(self, tokens: Sequence[int]) -> np.ndarray:
        """Embedding rows of tokens (get_token_embedding, lm_head.mojo:186-195)."""
        return np.stack([self.o.embed(self.lm_w, self.D, self.arch.vocab, self.lm_scale, int(t))
                         for t in tokens])

    def forward_keep(self, x: np.ndarray, base: int, keep: Sequence[int]):
        """All layers over rows x [T][D] at positions base..base+T-1 (one causal
        call per layer); returns the last layer's rows and each layer's output
        for the rows `keep` ([n_layers][len(keep)][D])."""
        keep = list(keep)
        hs = np.empty((self.arch.n_layers, len(keep), self.D), np.float32)
        for l in range(self.arch.n_layers):
            x = self.layer_forward(l, x, base)
            hs[l] = x[keep]
        return x, hs


class HostWeights:
    """Seeded synthetic weights generated once on the host and shared by any
    number of OracleModels (each with its own KV caches)."""

    def __init__(self, arch, seed: int, balanced: bool = False, with_lm: bool = True):
        import mojostream_amd as ms
        self.arch = arch
        self.weights, self.scales, self.ples = [], [], []
        for l in range(arch.n_layers):
            self.weights.append([ms.host_matrix(seed, l, i, K, N, balanced)
                                 for i, (K, N) in enumerate(arch.matrix_shapes(l))])
            self.scales.append([ms.matrix_scale(seed, l, i, K, balanced)
                                for i, (K, N) in enumerate(arch.matrix_shapes(l))])
            self.ples.append(ms.layer_ple(seed, l))
        self.lm = (ms.host_lm_head(seed, arch.hidden, arch.vocab, balanced)
                   if (with_lm and arch.vocab) else None)
        self.lm_scale = ms.lm_scale(seed, arch.hidden, balanced) if self.lm is not None else 0.0

    def model(self, oracle: Oracle) -> OracleModel:
        return OracleModel(oracle, self.arch, self.weights, self.scales, self.ples, self.lm,
                           self.lm_scale)


def synthetic_oracle_model(oracle: Oracle, arch, seed: int, with_lm: bool = True,
                           balanced: bool = False):
    """The same seeded weights the device generator produces (host copies)."""
    return HostWeights(arch, seed, balanced, with_lm).model(oracle)
