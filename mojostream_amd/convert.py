"""SafeTensors -> .mojostream converter with the Q4 quantization on the device.

Follows scripts/convert.py: the architecture from config.json (extract_arch,
:150-190), the tensor index over one or several .safetensors files
(build_tensor_index, :228-252), the layer-type-aware layout (get_layer_dims,
:195-225; compute_layout, :326-350), the 128-byte header with the Engram
extension and the directory (write_header_and_dir_placeholder, :362-413), the
PLE scale proxy mean|input_layernorm| (:490-498) and, per matrix, the transpose
and quantize_q4_blockwise (:500-536).

What differs is where the work runs: each weight's raw bytes (BF16, F16 or F32,
read straight from the memory-mapped file) go to HBM once, and ms_q4_quantize
converts, transposes, scales and packs them there.  The packed bytes are
identical to the reference converter's.
"""
from __future__ import annotations

import json
import mmap
import os
import struct
import time
from typing import Dict, Tuple

import numpy as np

from . import DeviceBuffer, Q4_DTYPES, q4_quantize

MAGIC = b"MOJOSTRM"
VERSION = 1
FORMAT_TAG = 2
HEADER_BYTES = 128
DIR_E_BYTES = 32
PAGE_ALIGN = 4096
ENGRAM_MAGIC = b"ENGR"
ENGRAM_VER = 1

MS_PLE, MS_Q, MS_K, MS_V, MS_O, MS_GATE, MS_UP, MS_DOWN = range(8)
MAT_ORDER = [MS_Q, MS_K, MS_V, MS_O, MS_GATE, MS_UP, MS_DOWN]
MAT_NAMES = {MS_Q: "Q", MS_K: "K", MS_V: "V", MS_O: "O", MS_GATE: "Gate", MS_UP: "Up",
             MS_DOWN: "Down"}

# HuggingFace names, (out, in) layout (convert.py:50-69)
HF_SUFFIXES = {
    "self_attn.q_proj.weight": MS_Q, "self_attn.k_proj.weight": MS_K,
    "self_attn.v_proj.weight": MS_V, "self_attn.o_proj.weight": MS_O,
    "mlp.gate_proj.weight": MS_GATE, "mlp.up_proj.weight": MS_UP,
    "mlp.down_proj.weight": MS_DOWN,
}
HF_SUFFIXES_ALT = {
    "self_attn.query_proj.weight": MS_Q, "self_attn.key_proj.weight": MS_K,
    "self_attn.value_proj.weight": MS_V, "self_attn.out_proj.weight": MS_O,
    "attention.q_proj.weight": MS_Q, "attention.k_proj.weight": MS_K,
    "attention.v_proj.weight": MS_V, "attention.o_proj.weight": MS_O,
}


def align_up(n: int, a: int) -> int:
    return (n + a - 1) & ~(a - 1)


class SafetensorsFile:
    """A memory-mapped .safetensors file: 8-byte header length, JSON header,
    then the tensor bytes (the format SafetensorsReader parses, convert.py:80-110)."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        (hlen,) = struct.unpack("<Q", self._mm[:8])
        self.header = json.loads(self._mm[8:8 + hlen])
        self.header.pop("__metadata__", None)
        self.base = 8 + hlen

    def keys(self):
        return self.header.keys()

    def raw(self, name: str) -> Tuple[np.ndarray, str, list]:
        e = self.header[name]
        a, b = e["data_offsets"]
        data = np.frombuffer(self._mm, dtype=np.uint8, count=b - a, offset=self.base + a)
        return data, e["dtype"], list(e["shape"])

    def load_f32(self, name: str) -> np.ndarray:
        """The host conversion of convert.py:100-110 (used for small vectors)."""
        data, dtype, shape = self.raw(name)
        if dtype == "BF16":
            u = data.view("<u2").astype(np.uint32) << 16
            return u.view(np.float32).reshape(shape).copy()
        if dtype == "F32":
            return data.view("<f4").reshape(shape).copy()
        if dtype == "F16":
            return data.view("<f2").astype(np.float32).reshape(shape)
        raise ValueError(f"unknown tensor dtype {dtype} ({name})")

    def close(self) -> None:
        try:
            self._mm.close()
        except BufferError:
            pass  # an array still views the map; it closes when that array goes
        self._f.close()


def load_config(model_dir: str) -> dict:
    path = os.path.join(model_dir, "config.json")
    if not os.path.exists(path):
        raise FileNotFoundError(f"config.json not found in {model_dir}")
    with open(path) as f:
        return json.load(f)


def extract_arch(config: dict) -> dict:
    """Gemma-4 (text_config) or older Gemma fields (convert.py:150-190)."""
    tc = config.get("text_config", config)

    def get(*keys, default=None):
        for k in keys:
            if k in tc:
                return tc[k]
        return default

    hidden = get("hidden_size")
    n_layers = get("num_hidden_layers")
    n_heads = get("num_attention_heads")
    n_kv = get("num_key_value_heads", default=n_heads)
    ffn = get("intermediate_size", "ffn_dim")
    for name, val in (("hidden_size", hidden), ("num_hidden_layers", n_layers),
                      ("num_attention_heads", n_heads), ("intermediate_size", ffn)):
        if val is None:
            raise ValueError(f"field '{name}' missing from config.json")
    hd = get("head_dim")
    if hd is None:
        hd = hidden // n_heads
    ghd = get("global_head_dim", default=hd)
    if ghd is None:
        ghd = hd
    return dict(hidden=hidden, n_layers=n_layers, n_heads=n_heads, n_kv_heads=n_kv,
                head_dim=hd, global_head_dim=ghd, ffn_dim=ffn,
                layer_types=get("layer_types", default=[]),
                num_kv_shared_layers=get("num_kv_shared_layers", default=0),
                kv_dim=n_kv * hd, sliding_kv_dim=n_kv * hd, full_kv_dim=n_kv * ghd,
                ple_dim=get("hidden_size_per_layer_input", default=0),
                sliding_window=get("sliding_window", default=0))


def get_layer_dims(arch: dict, layer: int) -> dict:
    """(in, out) shape of each matrix; full-attention layers use the global
    head size (convert.py:195-225)."""
    D, F = arch["hidden"], arch["ffn_dim"]
    lt = arch["layer_types"]
    ltype = lt[layer] if layer < len(lt) else "sliding_attention"
    hd = arch["global_head_dim"] if ltype == "full_attention" else arch["head_dim"]
    q, kv = arch["n_heads"] * hd, arch["n_kv_heads"] * hd
    dims = {MS_Q: (D, q), MS_K: (D, kv), MS_V: (D, kv), MS_O: (q, D), MS_GATE: (D, F),
            MS_UP: (D, F), MS_DOWN: (F, D)}
    return dict(layer_type=ltype, exp_dims=dims,
                mat_bytes={t: r * c // 2 for t, (r, c) in dims.items()})


def compute_layout(arch: dict) -> dict:
    """Page-aligned offsets of every matrix (convert.py:326-350)."""
    n_t = arch["n_layers"] * 8
    dir_bytes = n_t * DIR_E_BYTES
    cur = data_start = align_up(HEADER_BYTES + dir_bytes, PAGE_ALIGN)
    offsets, dims = {}, {}
    for layer in range(arch["n_layers"]):
        dims[layer] = get_layer_dims(arch, layer)
        for t in MAT_ORDER:
            offsets[(layer, t)] = cur
            cur = align_up(cur + dims[layer]["mat_bytes"][t], PAGE_ALIGN)
    return dict(data_start=data_start, dir_bytes=dir_bytes, layer_dims=dims, offsets=offsets,
                total_size=cur)


def build_tensor_index(model_dir: str) -> Dict[str, SafetensorsFile]:
    """name -> file for a sharded index, one model.safetensors, or every
    .safetensors file of the folder (convert.py:228-252)."""
    files: Dict[str, SafetensorsFile] = {}

    def open_(p):
        if p not in files:
            files[p] = SafetensorsFile(p)
        return files[p]

    idx = os.path.join(model_dir, "model.safetensors.index.json")
    if os.path.exists(idx):
        with open(idx) as f:
            wm = json.load(f)["weight_map"]
        return {n: open_(os.path.join(model_dir, fn)) for n, fn in wm.items()}
    single = os.path.join(model_dir, "model.safetensors")
    paths = [single] if os.path.exists(single) else sorted(
        os.path.join(model_dir, p) for p in os.listdir(model_dir) if p.endswith(".safetensors"))
    if not paths:
        raise FileNotFoundError(f"no .safetensors files in {model_dir}")
    index = {}
    for p in paths:
        sf = open_(p)
        for k in sf.keys():
            index[k] = sf
    return index


def detect_model_prefix(index: dict) -> str:
    for name in index:
        if name.startswith("model.language_model.layers."):
            return "model.language_model.layers."
        if name.startswith("model.layers."):
            return "model.layers."
    raise ValueError("no known tensor prefix in the SafeTensors files")


def resolve_tensor_name(index: dict, layer: int, t: int, prefix: str) -> str:
    full = f"{prefix}{layer}."
    for table in (HF_SUFFIXES, HF_SUFFIXES_ALT):
        for suffix, tt in table.items():
            if tt == t and full + suffix in index:
                return full + suffix
    avail = sorted(k for k in index if k.startswith(full))
    raise KeyError(f"no tensor for layer {layer} type {MAT_NAMES[t]} (prefix {full}); "
                   f"available: {avail[:10]}")


def _header(arch: dict, layout: dict) -> bytes:
    n_layers = arch["n_layers"]
    main = struct.pack("<8sIIIIIIIIQQQ", MAGIC, VERSION, FORMAT_TAG, n_layers, arch["hidden"],
                       arch["kv_dim"], arch["ffn_dim"], arch["n_heads"], arch["n_kv_heads"],
                       n_layers * 8, HEADER_BYTES, layout["data_start"])
    eng = struct.pack("<4sIIIIII", ENGRAM_MAGIC, ENGRAM_VER, arch["num_kv_shared_layers"],
                      arch["sliding_kv_dim"], arch["full_kv_dim"], arch["ple_dim"],
                      arch["sliding_window"])
    return main + eng + b"\0" * (HEADER_BYTES - len(main) - len(eng))


def convert(model_dir: str, out_path: str, block_size: int = 32, verbose: bool = True) -> dict:
    """Convert a HuggingFace SafeTensors folder to a .mojostream file.  Returns
    the architecture, the per-matrix scales and the device quantization time."""
    arch = extract_arch(load_config(model_dir))
    index = build_tensor_index(model_dir)
    prefix = detect_model_prefix(index)
    layout = compute_layout(arch)
    entries = []
    scales = {}
    os.makedirs(os.path.dirname(os.path.abspath(out_path)), exist_ok=True)
    try:
        _write(out_path, arch, layout, index, prefix, block_size, verbose, entries, scales,
               t_dev_acc := [0.0])
    finally:
        for sf in {id(v): v for v in index.values()}.values():
            sf.close()
    return dict(arch=arch, scales=scales, device_s=t_dev_acc[0])


def _write(out_path, arch, layout, index, prefix, block_size, verbose, entries, scales, t_dev):
    n_layers = arch["n_layers"]
    with open(out_path, "w+b") as f:
        f.write(b"\0" * layout["data_start"])
        for layer in range(n_layers):
            ld = layout["layer_dims"][layer]
            ple = 1.0
            pname = f"{prefix}{layer}.input_layernorm.weight"
            if pname in index:
                # PLE proxy: mean |input_layernorm| in float32, at least 0.001 (:490-496)
                ple = max(float(np.mean(np.abs(index[pname].load_f32(pname)))), 0.001)
            entries.append(struct.pack("<IIIIfIQ", layer, MS_PLE, 1, 0, np.float32(ple), 0, 0))
            for t in MAT_ORDER:
                name = resolve_tensor_name(index, layer, t, prefix)
                data, dtype, shape = index[name].raw(name)
                if dtype not in Q4_DTYPES:
                    raise ValueError(f"unknown tensor dtype {dtype} ({name})")
                if len(shape) != 2:
                    raise ValueError(f"{name}: expected a matrix, got shape {shape}")
                n_out, n_in = shape
                if (n_in, n_out) != ld["exp_dims"][t]:
                    raise ValueError(
                        f"Layer {layer} {MAT_NAMES[t]}: shape ({n_in},{n_out}) expected "
                        f"{ld['exp_dims'][t]}; check the architecture config")
                d_w = DeviceBuffer.from_array(data)
                t0 = time.perf_counter()
                d_q, s = q4_quantize(d_w, Q4_DTYPES[dtype], n_out, n_in, block_size)
                t_dev[0] += time.perf_counter() - t0
                d_w.free()
                packed = d_q.download(np.uint8, (n_in * n_out // 2,))
                d_q.free()
                assert f.tell() == layout["offsets"][(layer, t)]
                f.write(packed.tobytes())
                f.write(b"\0" * (align_up(packed.nbytes, PAGE_ALIGN) - packed.nbytes))
                entries.append(struct.pack("<IIIIfIQ", layer, t, n_in, n_out, np.float32(s), 0,
                                           layout["offsets"][(layer, t)]))
                scales[(layer, t)] = s
            if verbose:
                print(f"  layer {layer:3d}/{n_layers} [{ld['layer_type'][:7]}] ple {ple:.4f}",
                      flush=True)
        f.seek(0)
        f.write(_header(arch, layout))
        f.write(b"".join(entries))


def main(argv=None) -> int:
    import argparse
    ap = argparse.ArgumentParser(description="SafeTensors -> .mojostream (Q4 on the device)")
    ap.add_argument("model_dir")
    ap.add_argument("output", nargs="?", default="models/gemma4_e4b_q4.mojostream")
    ap.add_argument("--block-size", type=int, default=32)
    ap.add_argument("--quiet", action="store_true")
    a = ap.parse_args(argv)
    from . import init
    init(0)
    r = convert(a.model_dir, a.output, a.block_size, not a.quiet)
    print(f"wrote {a.output}: {r['arch']['n_layers']} layers, device quantization "
          f"{r['device_s']:.2f} s")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
