"""Validation entry points of the reference, over the C ABI.

- tensorguard_report: run_validation of src/tests/validate_real.mojo:110-260,
  the structural checks of a converted file and its directory checksum
  (compute_dir_checksum :78-83).
- run_validation: validate.mojo -> src/tests/validate_layer.mojo:159-233,
  layer 0 of the file on the batch-4 input of a layer0_ref.bin, relative RMSE
  against that file's output (PASS below 1e-4).
- run_real_validation: validate_real.mojo:33-143, the guards, a seeded layer-0
  pass checked for NaN / Inf, and the reference comparison when a
  layer0_ref.bin exists.
- read_ref / write_ref: the REFB file (validate_layer.mojo:89-122; written by
  scripts/gen_reference.py:223-226): "REFB", version 1, hidden, batch, then
  the batch x hidden fp32 input and output.
Like the reference these print PASS / FAIL and return their findings; they
raise only where the reference raises (a bad REFB magic, mismatched hidden
sizes, a file its loader rejects).
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass

import numpy as np

from . import DeviceBuffer, MSError, check, init, lib
from .streaming import MojoStreamFile

REF_MAGIC = 0x42464552   # "REFB"
VAL_BATCH = 4            # validate_layer.mojo:29
PASS_TOL = 1e-4          # validate_layer.mojo:31


@dataclass
class RefData:
    hidden: int
    batch: int
    input: np.ndarray    # [batch][hidden] fp32
    output: np.ndarray   # [batch][hidden] fp32


def read_ref(path: str) -> RefData:
    """load_ref (validate_layer.mojo:89-122)."""
    raw = open(path, "rb").read()
    if len(raw) < 16:
        raise MSError(f"{path}: shorter than the 16-byte REFB header")
    magic, _version, hidden, batch = struct.unpack_from("<IIII", raw, 0)
    if magic != REF_MAGIC:
        raise MSError("layer0_ref.bin: invalid magic number")
    n = batch * hidden
    if len(raw) < 16 + 8 * n:
        raise MSError(f"{path}: truncated ({len(raw)} bytes for {batch} x {hidden} rows)")
    data = np.frombuffer(raw, np.float32, 2 * n, 16)
    return RefData(hidden, batch, data[:n].reshape(batch, hidden).copy(),
                   data[n:].reshape(batch, hidden).copy())


def write_ref(path: str, x_in: np.ndarray, x_out: np.ndarray) -> None:
    """A REFB file as scripts/gen_reference.py:223-226 writes it."""
    x_in = np.ascontiguousarray(x_in, np.float32)
    x_out = np.ascontiguousarray(x_out, np.float32)
    batch, hidden = x_in.shape
    with open(path, "wb") as f:
        f.write(struct.pack("<IIII", REF_MAGIC, 1, hidden, batch))
        f.write(x_in.tobytes())
        f.write(x_out.tobytes())


def has_nan_or_inf(x: np.ndarray) -> bool:
    """has_nan_or_inf (validate_layer.mojo:36-48): NaN, or |v| above 1e30."""
    x = np.asarray(x, np.float32)
    return bool(np.isnan(x).any() or (np.abs(x) > np.float32(1e30)).any())


def check_stability(x: np.ndarray, name: str):
    """check_matrix_stability (:51-66): (stable, max |v|)."""
    if has_nan_or_inf(x):
        print(f"  [UNSTABLE] {name}: NaN or Inf found")
        return False, float("nan")
    mx = float(np.abs(np.asarray(x, np.float32)).max()) if np.size(x) else 0.0
    print(f"  [OK]       {name}: max_abs = {mx}")
    return True, mx


def compute_errors(got: np.ndarray, ref: np.ndarray) -> dict:
    """compute_errors (:138-154): sums in double, square roots in float32,
    rel = abs / (rms_ref + 1e-12)."""
    g = np.asarray(got, np.float32).reshape(-1).astype(np.float64)
    r = np.asarray(ref, np.float32).reshape(-1).astype(np.float64)
    n = g.size
    abs_rmse = float(np.sqrt(np.float32(np.sum((g - r) ** 2) / n)))
    rms_ref = float(np.sqrt(np.float32(np.sum(r * r) / n)))
    return dict(abs_rmse=abs_rmse, rms_ref=rms_ref, rel_rmse=abs_rmse / (rms_ref + 1e-12))


def _layer0(f: MojoStreamFile, x: np.ndarray) -> np.ndarray:
    """Layer 0 of the file over the rows x at positions 0..len(x)-1 (a cache of
    8 positions, as validate_layer.mojo:205 builds KVCache(1, kv_dim, 8))."""
    from . import Model
    model = Model(f.arch(max_len=8), max_seqs=1, max_rows=len(x), max_pos=8)
    try:
        model.load_file(f)
        return model.layer_forward(0, x, [0], T=len(x))
    finally:
        model.close()


def tensorguard_report(ms_path: str) -> dict:
    """run_validation, src/tests/validate_real.mojo:110-260."""
    print("=" * 62)
    print("  MojoStream TensorGuard - real-weight validation")
    print(f"  File: {ms_path}")
    print("=" * 62)
    with MojoStreamFile(ms_path) as f:
        r = f.validate()
        m = f.meta
        print(f"  file size {r['file_bytes'] / 1e6:.1f} MB, read in {f.load_time_ms():.1f} ms")
        print(f"  n_layers={m.n_layers} hidden={m.hidden} kv_dim={m.kv_dim} ffn={m.ffn_dim} "
              f"heads={m.n_heads}/{m.n_kv_heads} n_tensors={m.n_tensors}")
        if m.engram_version:
            print(f"  Engram v{m.engram_version}: kv_shared={m.n_kv_shared} "
                  f"kv_sliding={m.sliding_kv_dim} kv_full={m.full_kv_dim} ple_dim={m.ple_dim} "
                  f"window={m.sliding_window}")
    for name in r["failed"]:
        print(f"  [FAIL] {name}")
    print(f"  Checksum: {r['checksum_hex']}")
    print(f"  Checks:   {r['n_checks'] - r['n_failed']} / {r['n_checks']} passed")
    print("  [PASS] TensorGuard: all checks passed" if r["passed"] else
          f"  [FAIL] TensorGuard: {r['n_failed']} check(s) failed ({r['message']})")
    return r


def run_validation(ms_path: str = "model.mojostream", ref_path: str = "layer0_ref.bin") -> dict:
    """validate.mojo -> validate_layer.run_validation (:159-233)."""
    init(0)
    print("=" * 62)
    print("  MojoStream numerical validation - layer 0")
    print("=" * 62)
    with MojoStreamFile(ms_path) as f:
        f.validate_gemma4_shape()
        m = f.meta
        print(f"  ShapeGuard: OK  D={m.hidden} KV={m.kv_dim} FFN={m.ffn_dim} "
              f"heads={m.n_heads}/{m.n_kv_heads}")
        ref = read_ref(ref_path)
        print(f"  reference: hidden={ref.hidden} batch={ref.batch}")
        if ref.hidden != m.hidden:
            raise MSError("reference and model have different hidden sizes")
        y = _layer0(f, ref.input)
    e = compute_errors(y, ref.output)
    passed = e["rel_rmse"] < PASS_TOL
    print(f"  absolute RMSE {e['abs_rmse']}, RMS(reference) {e['rms_ref']}, "
          f"relative RMSE {e['rel_rmse']} (threshold {PASS_TOL})")
    print(f"  [{'PASS' if passed else 'FAIL'}] Validation layer 0: error {e['rel_rmse']}")
    return dict(passed=passed, **e)


def run_real_validation(ms_path: str = "model_converted.mojostream",
                        ref_path: str = "layer0_ref.bin", seed: int = 1234) -> dict:
    """validate_real.mojo:33-143: guards, a layer-0 pass on a seeded batch-4
    input checked for NaN / Inf, and the REFB comparison when the file
    exists (the reference fills the input with unseeded rand, kernels.mojo:57)."""
    init(0)
    print("=" * 62)
    print(f"  MojoStream real-weight validation: {ms_path}")
    print("=" * 62)
    out = {}
    with MojoStreamFile(ms_path) as f:
        f.validate_gemma4_shape()
        f.validate_tensor_entries()
        print(f"  ShapeGuard: OK   TensorGuard: OK ({f.meta.n_tensors} entries)")
        x = np.random.default_rng(seed).random((VAL_BATCH, f.meta.hidden), np.float32)
        stable, mx = check_stability(_layer0(f, x), "layer-0 output")
        out.update(stable=stable, max_abs=mx)
        if stable and os.path.exists(ref_path):
            ref = read_ref(ref_path)
            if ref.hidden != f.meta.hidden:
                print(f"  reference hidden {ref.hidden} != model hidden {f.meta.hidden}: skipped")
            else:
                e = compute_errors(_layer0(f, ref.input), ref.output)
                out.update(e, ref_passed=e["rel_rmse"] < PASS_TOL)
                print(f"  relative RMSE {e['rel_rmse']} (threshold {PASS_TOL}): "
                      f"[{'PASS' if out['ref_passed'] else 'FAIL'}]")
        elif stable:
            print(f"  no reference output ({ref_path} not found)")
    print(f"  stability: [{'PASS' if out['stable'] else 'FAIL'}]")
    return out
