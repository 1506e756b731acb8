"""ModelRunner (src/streaming/loader.mojo:47-144) over the C ABI: a double
buffer of one square Q4 matrix per layer, loaded from
<base_path>/layer_<i>.bin ([f32 scale][N * N/2 row-major Q4 bytes]) into two
HBM slots, with C += A . deq(W) on the active slot.

The reference times a load and a compute one after the other and derives the
wait analytically; ms_runner_run_pipeline overlaps them (the next layer's file
read, repack and host->HBM copy on the copy stream while the current layer
computes) and reports the compute stream's measured idle time as the wait.
The times come back in nanoseconds, in LayerStats' field names.
"""
from __future__ import annotations

import ctypes as C
import os
import struct
from dataclasses import dataclass
from typing import List, Optional

import numpy as np

from . import DeviceBuffer, _lib, check, host_random_u8, host_uniform


class _LayerStatsC(C.Structure):
    _fields_ = [("load_ms", C.c_double), ("compute_ms", C.c_double), ("wait_ms", C.c_double)]


@dataclass
class LayerStats:
    """LayerStats (loader.mojo:29-42): load of the next layer, compute of this
    one, and the wait between them, in nanoseconds."""
    load_ns: int
    compute_ns: int
    wait_ns: int = 0


def layer_path(base_path: str, idx: int) -> str:
    """ModelRunner._layer_path (loader.mojo:79-80)."""
    return base_path + "/layer_" + str(idx) + ".bin"


def write_layer_files(base_path: str, n_layers: int, N: int, seed: int = 42) -> List[float]:
    """Seeded layer files in the runner's format: per layer a scale
    U(0.04, 0.15) and uniform Q4 bytes (the row-major format of
    create_fake_model.py:126-140; the generator is this package's seeded one).
    Returns the scales."""
    os.makedirs(base_path, exist_ok=True)
    scales = []
    for i in range(n_layers):
        sc = float(np.float32(host_uniform(seed, 0x10AD, i, 0.04, 0.15)))
        data = host_random_u8(N * N // 2, seed, 0x10AD00 + i)
        with open(layer_path(base_path, i), "wb") as f:
            f.write(struct.pack("<f", sc))
            f.write(data.tobytes())
        scales.append(sc)
    return scales


class ModelRunner:
    """ModelRunner(base_path, n_layers, N, workers) (loader.mojo:59-76).
    `workers` is accepted for the reference's signature and has no GPU
    meaning."""

    def __init__(self, base_path: str, n_layers: int, N: int, workers: int = 0):
        self.base_path, self.n_layers, self.N = base_path, n_layers, N
        self.packed_size = N * (N // 2)
        h = C.c_void_p()
        check(_lib.ms_runner_create(os.fsencode(base_path), n_layers, N, C.byref(h)))
        self.h = h.value

    def close(self) -> None:
        if self.h:
            _lib.ms_runner_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def active(self) -> int:
        s = C.c_int()
        check(_lib.ms_runner_active(self.h, C.byref(s)))
        return s.value

    @active.setter
    def active(self, slot: int) -> None:
        check(_lib.ms_runner_set_active(self.h, slot))

    def load_into_slot(self, slot: int, idx: int) -> int:
        """Layer idx into slot (0 or 1); the load time in ns (loader.mojo:82-94)."""
        t = C.c_double()
        check(_lib.ms_runner_load_into_slot(self.h, slot, idx, C.byref(t)))
        return int(t.value * 1e6)

    def compute_active(self, C_: DeviceBuffer, A: DeviceBuffer, M: int) -> int:
        """C [M][N] += A [M][N] . deq(W_active); the device time in ns
        (loader.mojo:97-106)."""
        t = C.c_double()
        check(_lib.ms_runner_compute_active(self.h, C_.ptr, A.ptr, M, C.byref(t)))
        return int(t.value * 1e6)

    def run_pipeline(self, C_: DeviceBuffer, A: DeviceBuffer, M: int,
                     taps: Optional[DeviceBuffer] = None) -> List[LayerStats]:
        """Every layer in turn on the active slot, the next one loading into the
        other slot meanwhile, C zeroed after each layer (loader.mojo:115-144).
        taps (or None): [n_layers][M][N], C of each layer before the zeroing."""
        st = (_LayerStatsC * self.n_layers)()
        check(_lib.ms_runner_run_pipeline(self.h, C_.ptr, A.ptr, M, st,
                                          taps.ptr if taps is not None else None))
        return [LayerStats(int(s.load_ms * 1e6), int(s.compute_ms * 1e6), int(s.wait_ms * 1e6))
                for s in st]
