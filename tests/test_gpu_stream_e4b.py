"""E4B-scale layer streaming with SparsePinEngine's pinning (sparse_pin.mojo:
49-330, the gemma4_e4b_infer.mojo:160-186 loop) against the oracle.

A 42-layer E4B-shape .mojostream file and its version-1 LM head file (vocab
262144) are written with the synthetic generator.  Two streaming models load
them: one keeps the 24 layers build_pinned_mask() picks in HBM and streams the
other 18 through the two HBM slots, one streams all 42.  Both run a BOS +
prompt prefill and greedy decode steps with the taps on:
  - the two runs agree bit for bit (ids, logits, hidden rows): pinning moves
    where the weights come from, not what is computed;
  - the oracle, teacher-forced on the device's ids, gives every step's logits
    and every layer's row at sampled steps within relative RMSE 1e-4
    (validate_layer.mojo:31), and the greedy ids unless its top two are
    within 1e-3;
  - the pinned run streams 18 layers and 826 MB per pass, the reference's
    "I/O per token: 826 MB" (README.md:424-431), the other 42 and 1.97 GB.
"""
import os

import numpy as np
import pytest

from oracle.binding import Oracle, synthetic_oracle_model

pytestmark = pytest.mark.gpu
SEED = 42
PROMPT = 8
STEPS = 8
KEEP = (0, STEPS - 1)


def say(msg):
    print(f"\n[case] {msg}", flush=True)


def rel_rmse(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.sqrt(np.mean((a - b) ** 2)) / (np.sqrt(np.mean(b ** 2)) + 1e-30))


@pytest.fixture(scope="module")
def e4b_files(tmp_path_factory):
    from mojostream_amd import streaming as st
    d = tmp_path_factory.mktemp("e4b")
    p, lm = str(d / "e4b.mojostream"), str(d / "lm_head.bin")
    st.write_synthetic_e4b(p, 42, seed=SEED)
    st.write_synthetic_lm_head(lm, 2560, 262144, seed=SEED)
    yield p, lm
    for f in (p, lm):
        os.remove(f)


def run(ms, path, lm, pinned, prompt):
    from mojostream_amd import streaming as st
    max_pos = PROMPT + STEPS + 8
    m = st.load_model(path, lm_head_path=lm, vocab=262144, max_rows=16, max_pos=max_pos,
                      max_len=max_pos, resident=False, pinned=pinned)
    L, D, V = 42, 2560, 262144
    th, tl = ms.DeviceBuffer(L * D * 4), ms.DeviceBuffer(V * 4)
    m.set_taps(th, tl)
    first = m.prefill(prompt, 0)
    pre_stats = m.stream_stats()
    ids, logits, hid, stats = [], [], {}, []
    for k in range(STEPS):
        out = m.decode([first], [PROMPT], 1) if k == 0 else m.decode_continue(1, 1)
        ids.append(int(out[0, 0]))
        logits.append(tl.download(np.float32, (V,)))
        stats.append(m.stream_stats())
        if k in KEEP:
            hid[k] = th.download(np.float32, (L, D))
    m.close()
    return first, ids, np.stack(logits), hid, stats, pre_stats


def test_e4b_sparse_pinned_streaming_vs_oracle(gpu, e4b_files):
    ms = gpu
    from mojostream_amd import streaming as st
    path, lm = e4b_files
    mask = st.build_pinned_mask()
    assert sum(mask) == 24
    prompt = [int(v % 262144) for v in ms.host_random_u8(4 * PROMPT, 9, 80).view(np.uint32)]
    say("E4B file, 24 of 42 layers pinned (build_pinned_mask), prefill 8 + 8 greedy steps")
    a = run(ms, path, lm, mask, prompt)
    say("E4B file, all 42 layers streamed")
    b = run(ms, path, lm, None, prompt)
    first, ids, logits, hid, stats, pre = a
    assert first == b[0] and ids == b[1]
    assert np.array_equal(logits, b[2])
    assert all(np.array_equal(hid[k], b[3][k]) for k in KEEP)
    arch = ms.arch_e4b(max_full_seq=PROMPT + STEPS + 8)
    sl = sum(arch.layer_bytes(l) for l in range(42) if not mask[l])
    for s_pin, s_all in zip(stats, b[4]):
        assert (s_pin["layers_streamed"], s_pin["layers_pinned"]) == (18, 24)
        assert (s_all["layers_streamed"], s_all["layers_pinned"]) == (42, 0)
        assert s_pin["bytes"] == sl and s_all["bytes"] == arch.weight_bytes()
    assert pre["layers_streamed"] == 18 and pre["bytes"] == sl
    io_p = np.mean([s["io_ms"] for s in stats])
    io_a = np.mean([s["io_ms"] for s in b[4]])
    print(f"  streamed per token: pinned {sl / 1e6:.0f} MB (io {io_p:.1f} ms), "
          f"all {arch.weight_bytes() / 1e6:.0f} MB (io {io_a:.1f} ms)")
    assert round(sl / 1e6) == 826
    # the oracle, teacher-forced on the device's ids (BOS row at position 0)
    o = Oracle(avx2=True)
    o.set_threads(min(16, os.cpu_count() or 1))
    om = synthetic_oracle_model(o, arch, SEED)
    raw = open(lm, "rb").read()
    bos = np.frombuffer(raw, np.float32, 2560, 8).copy()
    x0 = om.embed_rows(prompt)
    x0[0] = bos
    y, _ = om.forward_keep(x0, 0, [PROMPT - 1])
    lg = om.logits_rows(y[PROMPT - 1:PROMPT])[0]
    assert int(np.argmax(lg)) == first or np.sort(lg)[-1] - np.sort(lg)[-2] < 1e-3
    toks = [first] + ids[:-1]
    y, hs = om.forward_keep(om.embed_rows(toks), PROMPT, list(KEEP))
    lg = om.logits_rows(y)
    worst = max(rel_rmse(logits[k], lg[k]) for k in range(STEPS))
    hw = max(rel_rmse(hid[k][l], hs[l, i]) for i, k in enumerate(KEEP) for l in range(42))
    for k in range(STEPS):
        top2 = np.sort(lg[k])[-2:]
        assert ids[k] == int(np.argmax(lg[k])) or top2[1] - top2[0] < 1e-3
    print(f"  logits rel RMSE max {worst:.2e}, hidden rows max {hw:.2e}, ids {[first] + ids}")
    assert worst < 1e-4 and hw < 1e-4
