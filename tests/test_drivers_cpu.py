"""Host-only parts of the drivers: the command line and the percentile rule."""
import struct

import pytest

from mojostream_amd import __main__ as cli
from mojostream_amd import drivers
from mojostream_amd import streaming as st


def test_percentile_rule():
    # harness.mojo:48-53: index int(pct/100*(n-1) + 0.5), clamped to n-1
    ns = [i * 1_000_000 for i in range(1, 101)]     # 1..100 ms
    assert drivers.percentile_ms(ns, 50.0) == 51.0  # idx int(49.5 + 0.5) = 50
    assert drivers.percentile_ms(ns, 95.0) == 95.0  # idx int(94.05 + 0.5) = 94
    assert drivers.percentile_ms(ns, 99.0) == 99.0
    assert drivers.percentile_ms(ns, 100.0) == 100.0
    assert drivers.percentile_ms([7_000_000], 95.0) == 7.0


def test_fake_model_cli(tmp_path):
    out = str(tmp_path / "m.mojostream")
    lm = str(tmp_path / "lm.bin")
    assert cli.main(["fake-model", out, "--layers", "2", "--seed", "5", "--lm-head", lm]) == 0
    with st.MojoStreamFile(out) as f:
        m = f.meta
        # create_fake_model.py demo dims: D 1024, KV 256, FFN 2048, 16 / 4 heads
        assert (m.n_layers, m.hidden, m.kv_dim, m.ffn_dim, m.n_heads, m.n_kv_heads) == \
            (2, 1024, 256, 2048, 16, 4)
        f.validate_gemma4_shape()
        f.validate_tensor_entries()
    assert struct.unpack("<I", open(lm, "rb").read(4))[0] == 32768


def test_fake_model_cli_e4b(tmp_path):
    out = str(tmp_path / "e.mojostream")
    assert cli.main(["fake-model", out, "--e4b", "--layers", "6"]) == 0
    with st.MojoStreamFile(out) as f:
        assert f.layer_info(5)["head_dim"] == 512 and f.layer_info(4)["head_dim"] == 256
        f.validate_tensor_entries()


def test_cli_rejects_unknown_command():
    with pytest.raises(SystemExit):
        cli.main(["nope"])
