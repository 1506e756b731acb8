"""The converter's Q4 quantization on the device, through the C ABI.

- ms_q4_quantize gives the oracle's bytes and scale bit for bit
  (quantize_q4_blockwise after the transpose, scripts/convert.py:296-323,
  503-518) for fp32, bf16 and fp16 weights, ragged shapes, the tiny-block
  rule, and the E4B matrix shapes.
- A HuggingFace-style SafeTensors folder (BF16, two shards with an index, one
  sliding and one full-attention layer) converts to a .mojostream file that the
  ShapeGuard and TensorGuard accept and whose every matrix, scale and PLE scale
  equals the oracle's.
"""
import json
import os
import struct
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"\n[case] {msg}", flush=True)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(x, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def device_quantize(ms, w_raw: np.ndarray, dtype: int, n_out: int, n_in: int, bs: int = 32):
    d_w = ms.DeviceBuffer.from_array(w_raw)
    d_q, s = ms.q4_quantize(d_w, dtype, n_out, n_in, bs)
    out = d_q.download(np.uint8, (n_in, n_out // 2))
    d_w.free()
    d_q.free()
    return out, s


@pytest.mark.parametrize("dt", ["F32", "BF16", "F16"])
@pytest.mark.parametrize("shape", [(2, 1), (34, 5), (130, 65), (256, 100), (1000, 333)])
def test_q4_quantize_vs_oracle(gpu, oracle, dt, shape):
    ms = gpu
    n_out, n_in = shape
    say(f"q4_quantize {dt} n_out={n_out} n_in={n_in}")
    rng = np.random.default_rng(n_out * 7 + n_in)
    w = (0.03 * rng.standard_normal((n_out, n_in))).astype(np.float32)
    if dt == "BF16":
        raw = to_bf16_bits(w)
        w = from_bf16_bits(raw)
    elif dt == "F16":
        raw = w.astype(np.float16)
        w = raw.astype(np.float32)
    else:
        raw = w
    got, s = device_quantize(ms, raw, ms.Q4_DTYPES[dt], n_out, n_in)
    want, s_want = oracle.q4_quantize(w)
    assert s == s_want
    assert np.array_equal(got, want)


def test_q4_quantize_grid_ties_and_tiny_blocks(gpu, oracle):
    ms = gpu
    say("q4_quantize: exact grid with ties, tiny-block rule, all zeros")
    w = np.zeros((4, 1), np.float32)
    w[:, 0] = np.array([2.5, 3.5, -2.5, 7.0]) * 2.0 ** -5
    got, s = device_quantize(ms, w, 0, 4, 1)
    assert s == 2.0 ** -5
    assert list(got[0]) == [(2 + 8) | ((4 + 8) << 4), (-2 + 8) | ((7 + 8) << 4)]
    t = np.zeros((64, 2), np.float32)
    t[5, 0] = 3e-8
    for bs in (32, 7):
        got, s = device_quantize(ms, t, 0, 64, 2, bs)
        want, s_want = oracle.q4_quantize(t, bs)
        assert s == s_want == np.float32(1e-8)
        assert np.array_equal(got, want)
    t[:, :] = 2e-8
    t[5, 0] = 3e-8
    got, s = device_quantize(ms, t, 0, 64, 2)
    want, s_want = oracle.q4_quantize(t)
    assert s == s_want and s < 1e-8
    assert np.array_equal(got, want)
    z = np.zeros((6, 3), np.float32)
    got, s = device_quantize(ms, z, 0, 6, 3)
    assert s == np.float32(1e-8) and np.all(got == 0x88)


def test_q4_quantize_rejects_bad_input(gpu):
    ms = gpu
    say("q4_quantize: NaN / infinity and an odd out dimension are refused")
    w = np.ones((4, 4), np.float32)
    w[2, 3] = np.nan
    with pytest.raises(ms.MSError, match="NaN or infinity"):
        device_quantize(ms, w, 0, 4, 4)
    w[2, 3] = np.inf
    with pytest.raises(ms.MSError, match="NaN or infinity"):
        device_quantize(ms, w, 0, 4, 4)
    d = ms.DeviceBuffer(64)
    with pytest.raises(ms.MSError, match="even"):
        ms.q4_quantize(d, 0, 3, 4)
    with pytest.raises(ms.MSError, match="dtype"):
        ms.q4_quantize(d, 3, 4, 4)
    d.free()


@pytest.mark.parametrize("shape", [(10240, 2560), (2560, 10240), (2048, 2560)])
def test_q4_quantize_e4b_shapes(gpu, oracle, shape):
    """Gate/Up (D -> F), Down (F -> D) and Q of a sliding layer, BF16 as the
    HuggingFace checkpoint stores them."""
    ms = gpu
    n_out, n_in = shape
    say(f"q4_quantize E4B shape BF16 n_out={n_out} n_in={n_in}")
    rng = np.random.default_rng(n_out + n_in)
    w = (0.02 * rng.standard_normal((n_out, n_in))).astype(np.float32)
    raw = to_bf16_bits(w)
    d_w = ms.DeviceBuffer.from_array(raw)
    d_q, s = ms.q4_quantize(d_w, 1, n_out, n_in)     # warm
    d_q.free()
    t0 = time.perf_counter()
    n_rep = 5
    for _ in range(n_rep):
        d_q, s = ms.q4_quantize(d_w, 1, n_out, n_in)
        d_q.free()
    dt = (time.perf_counter() - t0) / n_rep
    d_q, s = ms.q4_quantize(d_w, 1, n_out, n_in)
    got = d_q.download(np.uint8, (n_in, n_out // 2))
    d_q.free()
    d_w.free()
    want, s_want = oracle.q4_quantize(from_bf16_bits(raw))
    assert s == s_want
    assert np.array_equal(got, want)
    nbytes = n_out * n_in * 2.5
    print(f"  call {dt * 1e3:.3f} ms (two passes + scale readback + alloc), "
          f"{nbytes / dt / 1e9:.1f} GB/s algorithmic")


# ---- end to end: SafeTensors folder -> .mojostream ----------------------------------

def write_safetensors(path, tensors):
    """tensors: name -> (dtype string, shape, raw bytes)."""
    header, off, blobs = {}, 0, []
    for name, (dt, shape, b) in tensors.items():
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(b)]}
        off += len(b)
        blobs.append(b)
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"".join(blobs))


def test_convert_safetensors_folder(gpu, oracle, tmp_path):
    ms = gpu
    from mojostream_amd import convert as cv
    from mojostream_amd import streaming as st
    say("convert: 2-layer hybrid BF16 checkpoint in two shards -> .mojostream")
    D, F, H, KV, hd, ghd = 256, 512, 4, 1, 64, 128
    cfg = {"text_config": {"hidden_size": D, "num_hidden_layers": 2, "num_attention_heads": H,
                           "num_key_value_heads": KV, "intermediate_size": F, "head_dim": hd,
                           "global_head_dim": ghd,
                           "layer_types": ["sliding_attention", "full_attention"],
                           "hidden_size_per_layer_input": 64, "sliding_window": 128,
                           "num_kv_shared_layers": 0}}
    src = tmp_path / "hf"
    src.mkdir()
    (src / "config.json").write_text(json.dumps(cfg))
    rng = np.random.default_rng(3)
    pre = "model.language_model.layers."
    shards = [{}, {}]
    ref = {}
    for layer, full in ((0, False), (1, True)):
        h = ghd if full else hd
        shapes = {"self_attn.q_proj.weight": (H * h, D), "self_attn.k_proj.weight": (KV * h, D),
                  "self_attn.v_proj.weight": (KV * h, D), "self_attn.o_proj.weight": (D, H * h),
                  "mlp.gate_proj.weight": (F, D), "mlp.up_proj.weight": (F, D),
                  "mlp.down_proj.weight": (D, F)}
        for suffix, shp in shapes.items():
            w = (0.05 * rng.standard_normal(shp)).astype(np.float32)
            bits = to_bf16_bits(w)
            shards[layer][pre + f"{layer}." + suffix] = ("BF16", shp, bits.tobytes())
            ref[(layer, cv.HF_SUFFIXES[suffix])] = from_bf16_bits(bits).reshape(shp)
        ln = (1.0 + 0.2 * rng.standard_normal(D)).astype(np.float32)
        lb = to_bf16_bits(ln)
        shards[layer][pre + f"{layer}.input_layernorm.weight"] = ("BF16", (D,), lb.tobytes())
        ref[(layer, "ln")] = from_bf16_bits(lb)
    wm = {}
    for i, sh in enumerate(shards):
        fn = f"model-{i + 1:05d}-of-00002.safetensors"
        write_safetensors(str(src / fn), sh)
        wm.update({k: fn for k in sh})
    (src / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    out = str(tmp_path / "out.mojostream")
    r = cv.convert(str(src), out, 32, verbose=False)
    with st.MojoStreamFile(out) as f:
        f.set_layer_types([False, True])
        f.validate_gemma4_shape()
        f.validate_tensor_entries()
        for layer in (0, 1):
            want_ple = max(float(np.mean(np.abs(ref[(layer, "ln")]))), 0.001)
            assert f.ple_scale(layer) == np.float32(want_ple)
            for t in cv.MAT_ORDER:
                want, s_want = oracle.q4_quantize(ref[(layer, t)])
                got = f.tensor_array(layer, t)
                assert f.tensor_ptr(layer, t).scale == s_want == r["scales"][(layer, t)]
                assert np.array_equal(got, want), (layer, t)
    print(f"  device quantization {r['device_s'] * 1e3:.1f} ms for 14 matrices")
    # a shape that disagrees with the config is refused, as the reference does
    cfg["text_config"]["intermediate_size"] = F * 2
    (src / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError, match="check the architecture config"):
        cv.convert(str(src), str(tmp_path / "bad.mojostream"), 32, verbose=False)
