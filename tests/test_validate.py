"""The reference's validation tools on the CPU: the directory checksum and
structural checks of a converted file (src/tests/validate_real.mojo:78-260),
the REFB file (validate_layer.mojo:89-122) and the error metric (:138-154).
The recorded E4B checksum 0x01B27076 (README.md:26,200) needs the real
weights; here the checksum is checked against an independent XOR of the
scale fields read with struct from files written by tests' own writer."""
import os
import shutil
import struct

import numpy as np
import pytest

from mojostream_amd import MSError
from mojostream_amd import streaming as st
from mojostream_amd import validate as val
from tests.test_file_format import entry_off, patch, write_by_spec


def xor_scales(path):
    raw = open(path, "rb").read()
    n = struct.unpack_from("<Q", raw, 40)[0]
    acc = 0
    for i in range(n):
        acc ^= struct.unpack_from("<I", raw, 128 + 32 * i + 16)[0]
    return acc


@pytest.fixture
def e4b_like(tmp_path):
    """42 layers with the Engram extension (hybrid full layers), small dims."""
    p = str(tmp_path / "e4b_like.mojostream")
    full = [(l + 1) % 6 == 0 for l in range(42)]
    write_by_spec(p, 42, 128, 32, 128, 4, 1, np.random.default_rng(5),
                  engram={"full_kv": 64, "window": 16}, full=full)
    return p


def test_dir_checksum_is_xor_of_scale_bits(e4b_like, tmp_path):
    with st.MojoStreamFile(e4b_like) as f:
        assert f.dir_checksum() == xor_scales(e4b_like) != 0
    # one scale changed by one bit flips the same bit of the checksum
    q = str(tmp_path / "flip.mojostream")
    shutil.copy(e4b_like, q)
    raw = open(q, "rb").read()
    bits = struct.unpack_from("<I", raw, entry_off(9, "scale"))[0]
    patch(q, entry_off(9, "scale"), "<I", bits ^ (1 << 7))
    with st.MojoStreamFile(q) as f:
        assert f.dir_checksum() == xor_scales(e4b_like) ^ (1 << 7)


def test_structural_checks_pass_on_a_good_file(e4b_like):
    with st.MojoStreamFile(e4b_like) as f:
        r = f.validate()
    # magic, architecture, Engram, n_tensors, offsets, checksum, 6 spot checks
    assert r["passed"] and r["n_checks"] == 12 and r["n_failed"] == 0, r
    assert r["checksum_hex"] == f"0x{xor_scales(e4b_like):08X}"
    assert val.tensorguard_report(e4b_like)["passed"]


def test_demo_file_lacks_engram_and_spot_layers(tmp_path):
    p = str(tmp_path / "demo.mojostream")
    st.write_synthetic(p, 3, 256, 64, 512, 4, 1, seed=11)
    with st.MojoStreamFile(p) as f:
        r = f.validate()
    # layers 20 and 41 do not exist: only layer 0 is spot-checked (8 checks)
    assert r["n_checks"] == 8 and r["failed"] == ["engram"], r


@pytest.mark.parametrize("edit,failed", [
    ("engram", ["engram"]),
    # the directory then ends before layer 41, whose spot checks find no tensor
    ("n_tensors", ["n_tensors", "spot L41 Q", "spot L41 Gate"]),
    ("offset", ["offsets"]),
    ("scales", ["checksum"]),
    ("q0_zero", ["spot L0 Q"]),
    ("gate20_ff", ["spot L20 Gate"]),
    ("arch", ["architecture"]),
])
def test_structural_checks_catch(e4b_like, tmp_path, edit, failed):
    q = str(tmp_path / f"{edit}.mojostream")
    shutil.copy(e4b_like, q)
    raw = open(q, "rb").read()
    n = struct.unpack_from("<Q", raw, 40)[0]
    if edit == "engram":
        patch(q, 64, "<4s", b"XXXX")
    elif edit == "n_tensors":
        patch(q, 40, "<Q", n - 8)
    elif edit == "offset":
        patch(q, entry_off(17, "offset"), "<Q", len(raw) + 4096)
    elif edit == "scales":
        for i in range(n):
            patch(q, entry_off(i, "scale"), "<f", 0.0)
    elif edit in ("q0_zero", "gate20_ff"):
        i = 1 if edit == "q0_zero" else 20 * 8 + 5
        off = struct.unpack_from("<Q", raw, entry_off(i, "offset"))[0]
        patch(q, off, "<64s", (b"\0" if edit == "q0_zero" else b"\xff") * 64)
    elif edit == "arch":
        patch(q, 36, "<I", 3)    # kv_dim 32 is not a multiple of n_kv_heads 3
    with st.MojoStreamFile(q) as f:
        r = f.validate()
    assert r["failed"] == failed and not r["passed"] and r["n_failed"] == len(failed), r


def test_refb_round_trip_and_errors(tmp_path):
    p = str(tmp_path / "layer0_ref.bin")
    rng = np.random.default_rng(1234)
    x = (rng.standard_normal((4, 256)) * 0.1).astype(np.float32)
    y = rng.standard_normal((4, 256)).astype(np.float32)
    val.write_ref(p, x, y)
    raw = open(p, "rb").read()
    assert raw[:16] == struct.pack("<IIII", 0x42464552, 1, 256, 4)   # "REFB", v1
    assert len(raw) == 16 + 2 * 4 * 256 * 4
    r = val.read_ref(p)
    assert (r.hidden, r.batch) == (256, 4)
    assert np.array_equal(r.input, x) and np.array_equal(r.output, y)
    patch(p, 0, "<I", 0x12345678)
    with pytest.raises(MSError, match="invalid magic"):
        val.read_ref(p)
    with open(p, "wb") as f:
        f.write(struct.pack("<IIII", 0x42464552, 1, 256, 4) + b"\0" * 100)
    with pytest.raises(MSError, match="truncated"):
        val.read_ref(p)


def test_error_metric_and_stability():
    ref = np.array([3.0, 4.0, 0.0, 0.0], np.float32)        # RMS 2.5
    got = ref + np.array([1.0, -1.0, 1.0, -1.0], np.float32)  # RMSE 1
    e = val.compute_errors(got, ref)
    assert abs(e["abs_rmse"] - 1.0) < 1e-7 and abs(e["rms_ref"] - 2.5) < 1e-7
    assert abs(e["rel_rmse"] - 0.4) < 1e-7
    assert val.compute_errors(ref, ref)["rel_rmse"] == 0.0
    assert not val.has_nan_or_inf(ref)
    assert val.has_nan_or_inf(np.array([1.0, np.nan], np.float32))
    assert val.has_nan_or_inf(np.array([2e30], np.float32))     # "Inf" above 1e30
    assert not val.has_nan_or_inf(np.array([9e29, -9e29], np.float32))
    assert val.check_stability(np.array([-7.0, 2.0], np.float32), "x") == (True, 7.0)
