"""Models loaded from .mojostream files, through the C ABI, on the GPU.

- A file written with seed s holds the same weights that fill_synthetic(s)
  puts on the device, so a file-loaded model must equal it bit for bit.
- A hybrid (sliding + full attention) file with a version-1 LM head file:
  greedy ids equal the oracle's, with the BOS row at prompt position 0
  (apply_bos_embedding, lm_head.mojo:133-143; gemma4_e4b_infer.mojo:116-117).
- Streaming with pinned layers (SparsePinEngine's skipping prefetcher) equals
  the resident model bit for bit.
"""
import os
import struct

import numpy as np
import pytest

from oracle.binding import Oracle, synthetic_oracle_model

pytestmark = pytest.mark.gpu
SEED = 42


def say(msg):
    print(f"\n[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def fast_oracle():
    o = Oracle(avx2=True)
    o.set_threads(min(16, os.cpu_count() or 1))
    return o


def test_file_model_equals_synthetic(gpu, tmp_path):
    ms = gpu
    from mojostream_amd import streaming as st
    say("demo-shaped file (4 layers, D 1024) vs fill_synthetic, forward T=4")
    p = str(tmp_path / "demo.mojostream")
    st.write_synthetic(p, 4, 1024, 256, 4096, 8, 2, seed=SEED)
    a = st.load_model(p, max_rows=4, max_pos=64, max_len=64)
    b = ms.Model(ms.arch_demo(max_len=64, n_layers=4), max_rows=4, max_pos=64)
    b.fill_synthetic(SEED)
    for step in range(2):
        x = ms.host_normal(4 * 1024, 300 + step, 1).reshape(4, 1024)
        assert np.array_equal(a.forward(x, [4 * step], T=4), b.forward(x, [4 * step], T=4))
    a.close()
    b.close()


def hybrid_files(tmp_path, vocab):
    from mojostream_amd import streaming as st
    p = str(tmp_path / "hybrid.mojostream")
    lm = str(tmp_path / "lm_head.bin")
    st.write_synthetic(p, 6, 512, 256, 1024, 8, 2, seed=SEED, full_kv_dim=512,
                       sliding_window=32)
    st.write_synthetic_lm_head(lm, 512, vocab, seed=SEED)
    return p, lm


def test_hybrid_file_greedy_with_bos(gpu, fast_oracle, tmp_path):
    ms = gpu
    from mojostream_amd import streaming as st
    vocab = 2048
    say("hybrid file 6 layers (hd 128 sliding / 256 full) + LM head file, BOS prefill + greedy")
    p, lm = hybrid_files(tmp_path, vocab)
    m = st.load_model(p, lm_head_path=lm, vocab=vocab, max_rows=8, max_pos=128, max_len=128)
    with st.MojoStreamFile(p) as f:
        arch = f.arch(max_len=128, vocab=vocab)
    om = synthetic_oracle_model(fast_oracle, arch, SEED)
    raw = open(lm, "rb").read()
    bos = np.frombuffer(raw, np.float32, 512, 8).copy()
    prompt = [2, 611, 1500, 7]
    first = m.prefill(prompt, 0)
    rest = m.decode([first], [len(prompt)], 7)
    got = [first] + [int(v) for v in rest[:, 0]]
    # oracle: BOS row at position 0, token embeddings after it
    x = None
    for pos, t in enumerate(prompt):
        row = bos if pos == 0 else fast_oracle.embed(om.lm_w, 512, vocab, om.lm_scale, t)
        x = om.forward(np.asarray(row, np.float32)[None, :], pos)
    ref = [int(np.argmax(om.logits_for(x)))]
    pos = len(prompt)
    for _ in range(7):
        ref.append(om.decode_token(ref[-1], pos))
        pos += 1
    print(f"  gpu {got}\n  ref {ref}")
    assert got == ref
    m.close()


def test_streaming_pinned_equals_resident(gpu, tmp_path):
    ms = gpu
    from mojostream_amd import streaming as st
    say("streaming with pinned layers {0,2,5} vs resident, hybrid file")
    p, _ = hybrid_files(tmp_path, 2048)
    r = st.load_model(p, max_rows=4, max_pos=64, max_len=64)
    pinned = [True, False, True, False, False, True]
    s = st.load_model(p, max_rows=4, max_pos=64, max_len=64, resident=False, pinned=pinned)
    u = st.load_model(p, max_rows=4, max_pos=64, max_len=64, resident=False)
    for step in range(3):
        x = ms.host_normal(4 * 512, 700 + step, 2).reshape(4, 512)
        a = r.forward(x, [4 * step], T=4)
        assert np.array_equal(a, s.forward(x, [4 * step], T=4))
        assert np.array_equal(a, u.forward(x, [4 * step], T=4))
    print(f"  pinned stats {s.stream_stats()}\n  all-streamed stats {u.stream_stats()}")
    for m in (r, s, u):
        m.close()


def test_loader_errors(gpu, tmp_path):
    ms = gpu
    from mojostream_amd import streaming as st
    say("loader errors: shape mismatch, LM head vocab / size, v2 by size, pin after bind")
    p, lm = hybrid_files(tmp_path, 2048)
    with st.MojoStreamFile(p) as f:
        arch = f.arch(max_len=64, vocab=4096)
        wrong = ms.Model(ms.arch_demo(max_len=64, n_layers=6), max_pos=64)
        with pytest.raises(ms.MSError, match="does not match"):
            wrong.load_file(f)
        wrong.close()
        m = ms.Model(arch, max_pos=64)
        m.load_file(f)
        with pytest.raises(ms.MSError, match="vocab 2048 != model vocab 4096"):
            m.load_lm_head_file(lm)
        v2 = str(tmp_path / "v2.bin")
        with open(v2, "wb") as g:
            g.write(struct.pack("<IfI", 4096, 0.0, 2))
            g.write(b"\0" * (512 * 4 * 2 + 512 * 4096 * 4))
        # the version is told by the size alone, as lm_head.mojo:74-76 does
        m.load_lm_head_file(v2)
        short = str(tmp_path / "short.bin")
        with open(short, "wb") as g:
            g.write(struct.pack("<If", 4096, 0.1) + b"\0" * 1000)
        with pytest.raises(ms.MSError, match="version 1 needs"):
            m.load_lm_head_file(short)
        m.close()
        s = ms.Model(arch, max_pos=64, resident=False)
        s.load_file(f)
        flags = np.ones(6, np.uint8)
        with pytest.raises(ms.MSError, match="pin layers before binding"):
            ms.check(ms.lib().ms_model_set_pinned(s.h, flags.ctypes.data))
        s.close()


def test_validate_layer0_against_refb(gpu, tmp_path):
    """validate.mojo (validate_layer.run_validation :159-233) on a synthetic
    demo file: the REFB reference is written as scripts/gen_reference.py
    writes it (layer 0 in float64 numpy on 0.1 * N(0,1) rows of seed 1234),
    here by the independent f64 layer of tests/golden/layer_ref.py.  Passes at
    relative RMSE < 1e-4; a reference output off by 1 % fails."""
    import numpy as np
    from mojostream_amd import streaming as st
    from mojostream_amd import validate as val
    from mojostream_amd.__main__ import main as cli
    from tests.golden.layer_ref import RefLayer
    say("validate: layer 0 of a demo file against a layer0_ref.bin")
    p = str(tmp_path / "model.mojostream")
    ref = str(tmp_path / "layer0_ref.bin")
    st.write_synthetic(p, 2, 512, 128, 1024, 8, 2, seed=21)
    with st.MojoStreamFile(p) as f:
        desc = f.arch(max_len=8).layers[0]
        ws = [f.tensor_array(0, t) for t in range(1, 8)]
        sc = [f.tensor_ptr(0, t).scale for t in range(1, 8)]
        layer = RefLayer(desc, 512, 1024, ws, sc, f.ple_scale(0))
    x = (np.random.default_rng(1234).standard_normal((4, 512)) * 0.1).astype(np.float32)
    val.write_ref(ref, x, layer.forward(x, 0).astype(np.float32))
    r = val.run_validation(p, ref)
    print(f"  rel RMSE {r['rel_rmse']:.2e}")
    assert r["passed"] and r["rel_rmse"] < 1e-5
    assert cli(["validate", p, ref]) == 0
    rr = val.run_real_validation(p, ref)
    assert rr["stable"] and rr["ref_passed"]
    off = val.read_ref(ref)
    val.write_ref(ref, off.input, off.output * np.float32(1.01))
    assert not val.run_validation(p, ref)["passed"]
    assert cli(["validate", p, ref]) == 1
