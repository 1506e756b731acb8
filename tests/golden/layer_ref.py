"""Independent float64 numpy statement of one Gemma-4 layer and the LM head.

Written separately from oracle/ms_oracle.c (different language, vectorised,
double precision) so that a mistake in either (a dropped term, a wrong index,
a transposed operand) shows up as a disagreement far above fp32 rounding.
Semantics follow e4b_forward_layer (gemma4_e4b.mojo:459-540) and
gemma4_forward_layer (main.mojo:538-613); the residual adds to the normalized
stream as in gen_reference.py:160-172.
"""
from __future__ import annotations

import numpy as np


def deq(q4: np.ndarray, scale: float) -> np.ndarray:
    q4 = np.asarray(q4, np.uint8)
    K, P = q4.shape
    W = np.empty((K, 2 * P), np.float64)
    W[:, 0::2] = (q4 & 15).astype(np.float64) - 8.0
    W[:, 1::2] = (q4 >> 4).astype(np.float64) - 8.0
    return W * float(np.float32(scale))


def rms(x: np.ndarray) -> np.ndarray:
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-6)


def rope(x: np.ndarray, rot: int, pos: int, theta: float) -> np.ndarray:
    """x: [heads, hd]; rotate pairs (i, i+rot/2) of the first rot dims."""
    half = rot // 2
    i = np.arange(half, dtype=np.float64)
    ang = pos * np.exp(-(2.0 * i / rot) * np.log(theta))
    c, s = np.cos(ang), np.sin(ang)
    y = x.copy()
    a, b = x[:, :half], x[:, half:rot]
    y[:, :half] = a * c - b * s
    y[:, half:rot] = a * s + b * c
    return y


class RefLayer:
    def __init__(self, desc, D, F, w_q4, scales, ple):
        self.d = desc
        self.D, self.F = D, F
        self.W = [deq(w, s) for w, s in zip(w_q4, scales)]
        self.ple = float(np.float32(ple))
        self.K = {}  # absolute position -> (k [n_kv, hd], v [n_kv, hd])

    def keys_for(self, p: int):
        d = self.d
        if d.cache_kind == 1:  # circular window
            return range(max(0, p - d.cache_len + 1), p + 1)
        hi = p + 1
        if d.clamp_reads:
            hi = min(hi, d.cache_len)
        return range(0, hi)

    def forward(self, x: np.ndarray, base: int) -> np.ndarray:
        d = self.d
        T = x.shape[0]
        hd, nh, nkv = d.head_dim, d.n_heads, d.n_kv_heads
        x = rms(np.asarray(x, np.float64) * self.ple)
        q = (x @ self.W[0]).reshape(T, nh, hd)
        k = (x @ self.W[1]).reshape(T, nkv, hd)
        v = (x @ self.W[2]).reshape(T, nkv, hd)
        for t in range(T):
            q[t] = rope(q[t], d.rot_dim, base + t, d.theta)
            k[t] = rope(k[t], d.rot_dim, base + t, d.theta)
        for t in range(T):  # causal: rows see their own and earlier keys
            p = base + t
            if not (d.cache_kind == 0 and p >= d.cache_len):
                self.K[p] = (k[t], v[t])
        att = np.zeros((T, nh, hd))
        ratio = nh // nkv
        for t in range(T):
            p = base + t
            ks = list(self.keys_for(p))
            Km = np.stack([self.K[j][0] if j in self.K else np.zeros((nkv, hd)) for j in ks])
            Vm = np.stack([self.K[j][1] if j in self.K else np.zeros((nkv, hd)) for j in ks])
            for h in range(nh):
                hk = h // ratio
                s = Km[:, hk, :] @ q[t, h] / np.sqrt(hd)
                e = np.exp(s - s.max())
                att[t, h] = (e / e.sum()) @ Vm[:, hk, :]
        x = x + att.reshape(T, -1) @ self.W[3]
        x = rms(x)
        g = x @ self.W[4]
        u = x @ self.W[5]
        return x + (u * g / (1.0 + np.exp(-g))) @ self.W[6]


def lm_logits(x: np.ndarray, w_q4: np.ndarray, scale: float, gamma=None) -> np.ndarray:
    x = rms(np.asarray(x, np.float64))
    if gamma is not None:
        x = x * gamma
    return x @ deq(w_q4, scale)
