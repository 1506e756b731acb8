"""The host drivers end to end on the GPU (small files, few steps)."""
import json

import pytest

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"\n[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def g4_file(tmp_path_factory):
    from mojostream_amd import streaming as st
    p = str(tmp_path_factory.mktemp("drv") / "g4.mojostream")
    # first_light / create_fake_model dims at 4 layers: hd 64
    st.write_synthetic(p, 4, 1024, 256, 2048, 16, 4, seed=9)
    return p


def test_harness_json(gpu, g4_file, tmp_path):
    from mojostream_amd import drivers
    say("run_harness: 4-layer demo file, 6 steps of batch 4, bench_result.json")
    out = str(tmp_path / "bench_result.json")
    res = drivers.run_harness(g4_file, steps=6, out_json=out)
    saved = json.load(open(out))
    assert saved == json.loads(json.dumps(res))
    for k in ("format", "source", "model", "file_mb", "load_time_ms", "build_time_ms",
              "ttft_ms", "latency_p50_ms", "latency_p95_ms", "latency_p99_ms",
              "latency_best_ms", "latency_worst_ms", "peak_ram_mb", "io_pressure_pct",
              "n_steps", "batch", "tokens_per_sec_p50", "tokens_per_sec_best"):
        assert k in saved, k
    assert saved["model"] == {"n_layers": 4, "hidden": 1024, "kv_dim": 256, "ffn_dim": 2048}
    assert 0 < saved["latency_best_ms"] <= saved["latency_p50_ms"] <= saved["latency_p95_ms"] \
        <= saved["latency_worst_ms"]
    assert saved["n_steps"] == 6 and saved["batch"] == 4


def test_streaming_bench_and_pinning(gpu, g4_file):
    from mojostream_amd import drivers
    say("run_streaming_bench: all streamed, then layers 0 and 3 pinned")
    a = drivers.run_streaming_bench(g4_file, steps=2)
    b = drivers.run_streaming_bench(g4_file, steps=2, pinned=[True, False, False, True])
    assert a["io_ms"] > 0 and b["io_ms"] > 0 and a["total_ms"] > 0


def test_first_light_and_q4_bench(gpu):
    from mojostream_amd import drivers
    say("demo_first_light (40 layers, hd 64) and run_q4_benchmark")
    r = drivers.demo_first_light(steps=2)
    assert r["tokens_per_sec"] > 0
    q = drivers.run_q4_benchmark(shapes=((4, 1024, 1024), (64, 1024, 1024)), reps=3)
    assert all(x["gflops"] > 0 for x in q)


def test_e4b_infer_files(gpu, tmp_path):
    from mojostream_amd import drivers
    from mojostream_amd import streaming as st
    say("run_e4b_infer on a 6-layer hybrid file + LM head file, resident and streamed")
    p = str(tmp_path / "h.mojostream")
    lm = str(tmp_path / "lm.bin")
    st.write_synthetic(p, 6, 512, 256, 1024, 8, 2, seed=4, full_kv_dim=512, sliding_window=32)
    st.write_synthetic_lm_head(lm, 512, 4096, seed=4)
    prompt = (2, 603, 1012, 575)
    a = drivers.run_e4b_infer(p, lm, prompt=prompt, n_stream=6)
    b = drivers.run_e4b_infer(p, lm, prompt=prompt, n_stream=6, resident=False)
    assert a["ids"] == b["ids"] and len(a["ids"]) == 7
