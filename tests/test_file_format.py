"""The .mojostream format on the host: reader, writer, guards, pinning policy.

The C reader is checked against an independent writer written here from the
format description (create_fake_model.py:11-38, 188-281; convert.py:362-413),
and the C writer against an independent struct parser of the same layout.
Negative cases corrupt one field each and expect the guard that the
reference's fail-fast loaders raise for it (mojostream.mojo:190-219,
stream_runner.mojo:280-380).  No GPU is used.
"""
import math
import os
import struct

import numpy as np
import pytest

import mojostream_amd as ms
from mojostream_amd import streaming as st

HDR = "<8sIIIIIIIIQQQ"       # 64-byte main header
ENGR = "<4sIIIIII"           # Engram extension at byte 64
ENTRY = "<IIIIfIQ"           # 32-byte directory entry
PAGE = 4096


def align(n, a=PAGE):
    return (n + a - 1) // a * a


def spec_shapes(D, F, q_dim, kv):
    """(rows, cols) per type 1..7 (get_layer_dims, convert.py:208-224)."""
    return [(D, q_dim), (D, kv), (D, kv), (q_dim, D), (D, F), (D, F), (F, D)]


def write_by_spec(path, n_layers, D, kv, F, nh, nkv, rng, engram=None, full=None):
    """Independent writer of the documented layout; returns what it wrote."""
    n_t = n_layers * 8
    data_start = align(128 + 32 * n_t)
    entries, blobs, cur = [], [], data_start
    for l in range(n_layers):
        lkv = engram["full_kv"] if (full and full[l]) else kv
        hd = lkv // nkv
        entries.append((l, 0, 1, 0, float(rng.uniform(0.8, 1.2)), 0, 0))
        blobs.append(None)
        for t, (r, c) in enumerate(spec_shapes(D, F, nh * hd, lkv), start=1):
            data = rng.integers(0, 256, size=r * c // 2, dtype=np.uint8)
            entries.append((l, t, r, c, float(rng.uniform(0.04, 0.15)), 0, cur))
            blobs.append(data)
            cur = align(cur + data.size)
    with open(path, "wb") as f:
        hdr = struct.pack(HDR, b"MOJOSTRM", 1, 2 if engram else 1, n_layers, D, kv, F, nh, nkv,
                          n_t, 128, data_start)
        if engram:
            hdr += struct.pack(ENGR, b"ENGR", 1, 0, kv, engram["full_kv"], 0,
                               engram.get("window", 512))
        f.write(hdr + b"\0" * (128 - len(hdr)))
        for e in entries:
            f.write(struct.pack(ENTRY, *e))
        f.write(b"\0" * (data_start - f.tell()))
        for e, b in zip(entries, blobs):
            if b is None:
                continue
            assert f.tell() == e[6]
            f.write(b.tobytes())
            f.write(b"\0" * (align(b.size) - b.size))
    return entries, blobs


def patch(path, offset, fmt, *vals):
    with open(path, "r+b") as f:
        f.seek(offset)
        f.write(struct.pack(fmt, *vals))


def entry_off(i, field):
    return 128 + 32 * i + {"layer": 0, "type": 4, "rows": 8, "cols": 12, "scale": 16,
                           "offset": 24}[field]


@pytest.fixture
def demo_file(tmp_path):
    p = str(tmp_path / "demo.mojostream")
    st.write_synthetic(p, 3, 256, 64, 512, 4, 1, seed=11)
    return p


@pytest.fixture
def hybrid_file(tmp_path):
    p = str(tmp_path / "hybrid.mojostream")
    st.write_synthetic(p, 6, 256, 64, 512, 4, 2, seed=11, full_kv_dim=128, sliding_window=32)
    return p


# ---- reader against an independent writer ------------------------------------------
def test_reader_matches_spec_writer(tmp_path):
    rng = np.random.default_rng(42)
    p = str(tmp_path / "spec.mojostream")
    entries, blobs = write_by_spec(p, 2, 256, 64, 384, 4, 1, rng)
    with st.MojoStreamFile(p) as f:
        m = f.meta
        assert (m.version, m.format_tag, m.n_layers, m.hidden, m.kv_dim, m.ffn_dim,
                m.n_heads, m.n_kv_heads) == (1, 1, 2, 256, 64, 384, 4, 1)
        assert m.n_tensors == 16 and m.dir_offset == 128 and m.data_start == 4096
        assert m.engram_version == 0
        assert m.file_bytes == os.path.getsize(p)
        f.validate_gemma4_shape()
        f.validate_tensor_entries()
        got = f.entries
        for e, g in zip(entries, got):
            assert (g.layer_id, g.mat_type, g.rows, g.cols, g.flags, g.data_offset) == \
                (e[0], e[1], e[2], e[3], e[5], e[6])
            assert g.scale == np.float32(e[4])
        for i, (e, b) in enumerate(zip(entries, blobs)):
            if b is None:
                assert f.ple_scale(e[0]) == np.float32(e[4])
                continue
            arr = f.tensor_array(e[0], e[1])
            assert arr.shape == (e[2], e[3] // 2)
            assert np.array_equal(arr.reshape(-1), b)
            assert f.tensor_ptr(e[0], e[1]).scale == np.float32(e[4])


def test_reader_hybrid_engram(tmp_path):
    rng = np.random.default_rng(7)
    p = str(tmp_path / "h.mojostream")
    full = [(l + 1) % 6 == 0 for l in range(6)]
    entries, blobs = write_by_spec(p, 6, 256, 64, 384, 4, 2, rng,
                                   engram={"full_kv": 128, "window": 32}, full=full)
    with st.MojoStreamFile(p) as f:
        m = f.meta
        assert (m.format_tag, m.engram_version, m.sliding_kv_dim, m.full_kv_dim,
                m.sliding_window) == (2, 1, 64, 128, 32)
        f.validate_gemma4_shape()
        f.validate_tensor_entries()
        assert f.layer_info(0) == dict(is_full=False, head_dim=32, q_dim=128, kv_dim=64)
        assert f.layer_info(5) == dict(is_full=True, head_dim=64, q_dim=256, kv_dim=128)
        a = f.arch(max_len=64)
        assert [d.cache_kind for d in a.layers] == [1, 1, 1, 1, 1, 0]
        assert a.layers[5].rot_dim == 16 and a.layers[0].rot_dim == 32
        assert a.layers[0].cache_len == 32
        for e, b in zip(entries, blobs):
            if b is not None:
                assert np.array_equal(f.tensor_array(e[0], e[1]).reshape(-1), b)


# ---- writer against an independent parser -------------------------------------------
def test_writer_layout_and_weights(demo_file):
    raw = open(demo_file, "rb").read()
    h = struct.unpack_from(HDR, raw, 0)
    assert h[0] == b"MOJOSTRM" and h[1:9] == (1, 1, 3, 256, 64, 512, 4, 1)
    n_t, dir_off, data_start = h[9:12]
    assert (n_t, dir_off, data_start) == (24, 128, align(128 + 24 * 32))
    assert raw[64:128] == b"\0" * 64
    cur = data_start
    for i in range(n_t):
        l, t, r, c, s, fl, off = struct.unpack_from(ENTRY, raw, 128 + 32 * i)
        assert (l, t, fl) == (i // 8, i % 8, 0)
        if t == 0:
            assert (r, c, off) == (1, 0, 0)
            assert s == np.float32(ms.layer_ple(11, l))
            assert 0.8 <= s < 1.2
            continue
        K, N = spec_shapes(256, 512, 256, 64)[t - 1]
        assert (r, c, off) == (K, N, cur)
        assert s == np.float32(ms.matrix_scale(11, l, t - 1))
        blob = np.frombuffer(raw, np.uint8, K * N // 2, off)
        # the same bytes the device generator writes for this (seed, layer, matrix)
        assert np.array_equal(blob, ms.host_matrix(11, l, t - 1, K, N).reshape(-1))
        cur = align(cur + K * N // 2)
    assert len(raw) == cur


def test_writer_hybrid_header(hybrid_file):
    raw = open(hybrid_file, "rb").read()
    assert struct.unpack_from(HDR, raw, 0)[2] == 2
    e = struct.unpack_from(ENGR, raw, 64)
    assert e == (b"ENGR", 1, 0, 64, 128, 0, 32)
    # layer 5 is full attention: K is [256][128], Q is [256][256]
    q = struct.unpack_from(ENTRY, raw, 128 + 32 * (5 * 8 + 1))
    k = struct.unpack_from(ENTRY, raw, 128 + 32 * (5 * 8 + 2))
    assert (q[2], q[3], k[2], k[3]) == (256, 256, 256, 128)


def test_tensor_lookup_edges(demo_file):
    with st.MojoStreamFile(demo_file) as f:
        with pytest.raises(ms.MSError, match="no tensor"):
            f.tensor_ptr(3, 1)
        with pytest.raises(ms.MSError, match="no tensor"):
            f.tensor_ptr(0, 9)
        # ple_scale past the directory is 1.0 (mojostream.mojo:180-182)
        assert f.ple_scale(99) == 1.0
        assert f.tensor_ptr(0, 0).nbytes == 0
        assert f.load_time_ms() >= 0 and f.file_size_mb() > 0


# ---- the reference's guards reject E4B files; these do not ---------------------------
def reference_demo_expectations(meta):
    """The fixed shapes of StreamingRunner's TensorGuard (stream_runner.mojo:326-335)."""
    D, KVD, F = meta.hidden, meta.kv_dim, meta.ffn_dim
    return [(1, 0), (D, D), (D, KVD), (D, KVD), (D, D), (D, F), (D, F), (F, D)]


def test_e4b_shaped_file_passes_layer_aware_guards(tmp_path):
    p = str(tmp_path / "e4b2.mojostream")
    # E4B widths at 6 layers (full attention at layer 5)
    st.write_synthetic(p, 6, 2560, 512, 256, 8, 2, seed=3, full_kv_dim=1024,
                       sliding_window=512)
    with st.MojoStreamFile(p) as f:
        f.validate_gemma4_shape()
        f.validate_tensor_entries()
        # the demo-shape expectations of the reference reject this file
        exp = reference_demo_expectations(f.meta)
        mism = [(i, e.rows, e.cols) for i, e in enumerate(f.entries)
                if (e.rows, e.cols) != exp[i % 8]]
        assert mism, "E4B shapes differ from the demo expectations"
        # and the strict head-size rule of stream_runner.mojo:296-300 fails too
        m = f.meta
        assert m.kv_dim != m.n_kv_heads * (m.hidden // m.n_heads)
        assert f.layer_info(5)["q_dim"] == 4096 and f.layer_info(0)["q_dim"] == 2048


# ---- negative cases --------------------------------------------------------------------
@pytest.mark.parametrize("field,fmt,value,match", [
    (32, "<I", 0, r"\[ShapeGuard\] n_heads = 0"),
    (36, "<I", 0, r"\[ShapeGuard\] n_kv_heads = 0"),
    (32, "<I", 3, r"hidden \(256\) not divisible by n_heads \(3\)"),
    (36, "<I", 3, r"n_heads \(4\) not divisible by n_kv_heads \(3\)"),
    (24, "<I", 65, r"kv_dim=65 expected=64"),
    (24, "<I", 128, r"kv_dim=128 expected=64"),
    (16, "<I", 2, r"n_tensors=24 != n_layers\*8=16"),
    (28, "<I", 0, r"ffn_dim <= 0"),
    (48, "<Q", 256, r"dir_offset=256"),
])
def test_shape_guard_rejects(demo_file, field, fmt, value, match):
    patch(demo_file, field, fmt, value)
    with st.MojoStreamFile(demo_file) as f:
        with pytest.raises(ms.MSError, match=match):
            f.validate_gemma4_shape()


def test_shape_guard_hybrid_rules(hybrid_file):
    patch(hybrid_file, 24, "<I", 65)  # kv_dim not a multiple of 2 kv heads
    with st.MojoStreamFile(hybrid_file) as f:
        with pytest.raises(ms.MSError, match="kv_dim=65 not divisible by n_kv_heads=2"):
            f.validate_gemma4_shape()
    patch(hybrid_file, 24, "<I", 64)
    patch(hybrid_file, 76, "<I", 32)  # sliding_kv_dim != kv_dim
    with st.MojoStreamFile(hybrid_file) as f:
        with pytest.raises(ms.MSError, match="sliding_kv_dim=32 != kv_dim=64"):
            f.validate_gemma4_shape()
    patch(hybrid_file, 76, "<I", 64)
    patch(hybrid_file, 80, "<I", 129)
    with st.MojoStreamFile(hybrid_file) as f:
        with pytest.raises(ms.MSError, match="full_kv_dim=129 not divisible"):
            f.validate_gemma4_shape()


@pytest.mark.parametrize("idx,field,fmt,value,match", [
    (9, "layer", "<I", 0, r"Tensor\[9\] Layer 1 Q: layer_id=0 expected=1"),
    (10, "type", "<I", 3, r"Tensor\[10\] Layer 1 K: mat_type=3 expected=2"),
    (12, "rows", "<I", 128, r"Layer 1 O: rows=128 expected=256"),
    (15, "rows", "<I", 256, r"Layer 1 Down: rows=256 expected=512"),
    (13, "cols", "<I", 1024, r"Layer 1 Gate: cols=1024 expected=512"),
    (8, "scale", "<f", 0.0, r"Layer 1 PLE: scale="),
    (11, "scale", "<f", -0.5, r"Layer 1 V: scale="),
    (11, "scale", "<f", math.nan, r"Layer 1 V: scale="),
    (11, "scale", "<f", math.inf, r"Layer 1 V: scale="),
    (14, "offset", "<Q", 4096 + 8, r"Layer 1 Up: offset=4104 not 4096-aligned"),
])
def test_tensor_guard_rejects(demo_file, idx, field, fmt, value, match):
    patch(demo_file, entry_off(idx, field), fmt, value)
    with st.MojoStreamFile(demo_file) as f:
        f.validate_gemma4_shape()
        with pytest.raises(ms.MSError, match=match):
            f.validate_tensor_entries()


def test_tensor_guard_bounds(demo_file):
    size = os.path.getsize(demo_file)
    with open(demo_file, "r+b") as f:
        f.truncate(size - PAGE)  # the last matrix loses its last page
    with st.MojoStreamFile(demo_file) as f:
        with pytest.raises(ms.MSError, match=r"Layer 2 Down: offset=.* > file_size"):
            f.validate_tensor_entries()
        with pytest.raises(ms.MSError, match="outside the file"):
            f.tensor_ptr(2, 7)


def test_tensor_guard_layer_types(hybrid_file):
    # a map that calls layer 0 full attention makes layer 0's K width wrong
    with st.MojoStreamFile(hybrid_file) as f:
        f.set_layer_types([True] + [False] * 4 + [True])
        with pytest.raises(ms.MSError, match=r"Layer 0 Q: cols=128 expected=256"):
            f.validate_tensor_entries()
        f.set_layer_types(None)
        f.validate_tensor_entries()
        with pytest.raises(ms.MSError, match="one flag per layer"):
            f.set_layer_types([False] * 5)


@pytest.mark.parametrize("how,match", [
    ("magic", "invalid magic"),
    ("short", "shorter than the 128-byte header"),
    ("dir", "extends past the end"),
    ("layers", "implausible n_layers"),
    ("missing", "cannot open"),
])
def test_open_rejects(demo_file, how, match):
    path = demo_file
    if how == "magic":
        patch(demo_file, 0, "<4s", b"MOJA")
    elif how == "short":
        with open(demo_file, "r+b") as f:
            f.truncate(100)
    elif how == "dir":
        with open(demo_file, "r+b") as f:
            f.truncate(128 + 32 * 10)
    elif how == "layers":
        patch(demo_file, 16, "<I", 1 << 30)
    else:
        path = demo_file + ".absent"
    with pytest.raises(ms.MSError, match=match):
        st.MojoStreamFile(path)


# ---- LM head file (version 1) ----------------------------------------------------------
def test_lm_head_file_layout(tmp_path):
    p = str(tmp_path / "lm.bin")
    st.write_synthetic_lm_head(p, 256, 1024, seed=5)
    raw = open(p, "rb").read()
    vocab, scale = struct.unpack_from("<If", raw, 0)
    assert vocab == 1024 and scale == np.float32(ms.lm_scale(5))
    assert len(raw) == 8 + 256 * 4 + 256 * 1024 // 2
    w = np.frombuffer(raw, np.uint8, 256 * 512, 8 + 256 * 4)
    assert np.array_equal(w, ms.host_lm_head(5, 256, 1024).reshape(-1))
    bos = np.frombuffer(raw, np.float32, 256, 8)
    assert np.all(np.isfinite(bos)) and 0.5 < bos.std() < 1.5


# ---- SparsePinEngine pinning policy ----------------------------------------------------
def test_pinned_mask_e4b():
    m = st.build_pinned_mask()
    pinned = [l for l, x in enumerate(m) if x]
    assert len(pinned) == 24  # "Total: 24" (sparse_pin.mojo:56)
    assert {5, 11, 17, 23, 29, 35, 41} <= set(pinned)     # full-attention anchors
    assert {0, 1, 2, 3, 39, 40} <= set(pinned)            # latency bridge
    # fillers: every second remaining sliding layer, as the loop at
    # sparse_pin.mojo:74-83 picks them
    assert sorted(set(pinned) - {5, 11, 17, 23, 29, 35, 41, 0, 1, 2, 3, 39, 40}) == \
        [4, 7, 9, 12, 14, 16, 19, 21, 24, 26, 28]
    assert st.next_non_pinned(3, m) == 6
    assert st.next_non_pinned(40, m) == -1
    assert st.next_non_pinned(28, m) == 30
