"""Host drivers: the reference's entry points over the GPU path.

Same names, phases and reported fields as the reference's drivers, with the
per-layer CPU loops replaced by calls into the library:

  demo_first_light     main.mojo:646-704            (pixi task first_light)
  run_harness          harness.mojo:185-328         (bench; writes bench_result.json)
  run_streaming_bench  stream_runner.mojo:460-562   (stream)
  run_q4_benchmark     benchmark_q4.mojo:121-147    (bench_q4)
  run_e4b_infer        gemma4_e4b_infer.mojo:57-210 (e4b-infer; greedy, or
                       temperature + repetition penalty with a seed)

Inputs are seeded (the reference's fill_random is unseeded, so its runs are
not repeatable).  Latencies are wall-clock per step, including the copy of
the step's input rows to the device and of the outputs back, as the
reference's steps include their memory traffic.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import time
from typing import List, Optional, Sequence

import numpy as np

from . import (DeviceBuffer, Model, check, demo_layer, device_info, host_normal,
               host_random_u8, init, lib, Arch)
from . import streaming as st

# TokenMap.is_eos (gemma_proto.mojo:51-52)
EOS_ID = 1

BENCH_STEPS = 100   # harness.mojo:30
BENCH_BATCH = 4     # harness.mojo:31
KV_MAX_SEQ = 512    # harness.mojo:32


def percentile_ms(sorted_ns: Sequence[int], pct: float) -> float:
    """harness.mojo:48-53: index round(pct/100 * (n-1)), clamped."""
    n = len(sorted_ns)
    idx = min(int(pct / 100.0 * (n - 1) + 0.5), n - 1)
    return sorted_ns[idx] / 1e6


def rss_mb() -> float:
    """VmRSS of this process (get_rss_kb, stream_runner.mojo:36-65)."""
    try:
        with open("/proc/self/status") as f:
            for line in f:
                if line.startswith("VmRSS:"):
                    return int(line.split()[1]) / 1024.0
    except OSError:
        pass
    return 0.0


def build_json(path: str, meta, file_mb: float, load_ms: float, build_ms: float,
               ttft_ms: float, p50: float, p95: float, p99: float, best: float,
               worst: float, peak_ram_mb: float, n_steps: int, batch: int, io_pct: float,
               tps_p50: float, tps_best: float, device: str) -> dict:
    """The fields of build_json (harness.mojo:133-180), plus the device name."""
    return {
        "format": "mojostream", "source": path,
        "model": {"n_layers": meta.n_layers, "hidden": meta.hidden, "kv_dim": meta.kv_dim,
                  "ffn_dim": meta.ffn_dim},
        "file_mb": file_mb, "load_time_ms": load_ms, "build_time_ms": build_ms,
        "ttft_ms": ttft_ms, "latency_p50_ms": p50, "latency_p95_ms": p95,
        "latency_p99_ms": p99, "latency_best_ms": best, "latency_worst_ms": worst,
        "peak_ram_mb": peak_ram_mb, "io_pressure_pct": io_pct, "n_steps": n_steps,
        "batch": batch, "tokens_per_sec_p50": tps_p50, "tokens_per_sec_best": tps_best,
        "device": device,
    }


def _banner(title: str) -> None:
    print("=" * 62)
    print(f"  {title}")
    print("=" * 62)


def _device() -> str:
    name, ncu, _ = device_info()
    return f"{name} ({ncu} CUs)"


def demo_first_light(steps: int = 3, batch: int = 4, seed: int = 42) -> dict:
    """Random-weight Gemma-4 demo model (D 1024, KV 256, FFN 2048, 40 layers,
    16 q / 4 kv heads of 64; main.mojo:225-227,652-655): `steps` forward
    passes of `batch` rows; prints the fastest step."""
    init(0)
    D, KV, F, L, NH, NKV = 1024, 256, 2048, 40, 16, 4
    _banner("FIRST LIGHT  -  Gemma-4 forward pass (random weights)")
    arch = Arch("first_light", D, F, [demo_layer(D, NH, NKV, 256) for _ in range(L)])
    print(f"  D={D}  KVD={KV}  FFD={F}  head_dim={D // NH}")
    print(f"  Allocating 40 layers of weights (~{arch.weight_bytes() / 1e6:.1f} MB) ...")
    m = Model(arch, max_seqs=1, max_rows=batch, max_pos=256)
    m.fill_synthetic(seed)
    print(f"  Running {steps * batch} tokens (batch={batch}, {steps} steps) ...")
    best = None
    for step in range(steps):
        x = host_normal(batch * D, seed + step, 1).reshape(batch, D)
        t0 = time.perf_counter_ns()
        m.forward(x, [step * batch], T=batch)
        dt = time.perf_counter_ns() - t0
        best = dt if best is None else min(best, dt)
    m.close()
    ms_ = best / 1e6
    tps = batch / (best / 1e9)
    print(f"  Fastest step (batch={batch}):   {ms_:.3f} ms")
    print(f"  Tokens/s (batch={batch}):       {tps:.1f} t/s")
    print(f"  Tokens/s (single, effective): {tps / batch:.1f} t/s")
    return dict(best_ms=ms_, tokens_per_sec=tps)


def run_harness(path: str, steps: int = BENCH_STEPS, batch: int = BENCH_BATCH,
                out_json: Optional[str] = "bench_result.json", seed: int = 1) -> dict:
    """Benchmark harness: load the file, bind the weights, TTFT (load + build
    + first forward), then `steps` forward steps of `batch` rows with the
    sequence growing; percentiles and bench_result.json."""
    init(0)
    _banner("MojoStream benchmark harness")
    print(f"  File: {path}")
    t_start = time.perf_counter_ns()
    f = st.MojoStreamFile(path)
    load_ms, file_mb = f.load_time_ms(), f.file_size_mb()
    print(f"[1/4] file {file_mb:.1f} MB, I/O {load_ms:.1f} ms "
          f"({file_mb / max(load_ms, 1e-9) * 1e3:.0f} MB/s)")
    m_ = f.meta
    print(f"  model: D={m_.hidden} KV={m_.kv_dim} FFN={m_.ffn_dim} layers={m_.n_layers}")
    max_len = KV_MAX_SEQ if (steps + 1) * batch <= KV_MAX_SEQ else (steps + 1) * batch
    t_b = time.perf_counter_ns()
    f.validate_gemma4_shape()
    f.validate_tensor_entries()
    model = Model(f.arch(max_len=max_len), max_seqs=1, max_rows=batch, max_pos=max_len)
    model.load_file(f)
    check(lib().ms_synchronize())
    build_ms = (time.perf_counter_ns() - t_b) / 1e6
    print(f"[2/4] weights bound in {build_ms:.1f} ms")
    D = m_.hidden
    x = host_normal(batch * D, seed, 0).reshape(batch, D)
    model.forward(x, [0], T=batch)
    ttft_ms = (time.perf_counter_ns() - t_start) / 1e6
    print(f"[3/4] TTFT {ttft_ms:.1f} ms (load + build + first forward)")
    print(f"[4/4] latency over {steps} steps, batch={batch} ...")
    lat: List[int] = []
    pos = batch
    dx = DeviceBuffer(batch * D * 4)   # the step's input rows, uploaded per step
    for s in range(steps):
        # fresh rows before the clock starts, as the reference fills x before
        # its timed layer loop (harness.mojo:256-262)
        x = host_normal(batch * D, seed, 1 + s).reshape(batch, D)
        dx.upload(x)
        base = (C.c_int * 1)(pos)
        t0 = time.perf_counter_ns()
        check(lib().ms_forward(model.h, dx.ptr, 1, batch, base, None))
        lat.append(time.perf_counter_ns() - t0)
        pos += batch
        if s % 20 == 19:
            print(f"  step {s + 1}/{steps}  seq_len={pos}  step={lat[-1] / 1e6:.3f} ms")
    lat.sort()
    p50, p95, p99 = (percentile_ms(lat, q) for q in (50.0, 95.0, 99.0))
    best, worst = lat[0] / 1e6, lat[-1] / 1e6
    # I/O pressure as the reference computes it (harness.mojo:296-300)
    amort = load_ms / steps
    io_pct = amort / (amort + best) * 100.0
    tps_p50, tps_best = batch / (p50 / 1e3), batch / (best / 1e3)
    res = build_json(path, m_, file_mb, load_ms, build_ms, ttft_ms, p50, p95, p99, best,
                     worst, rss_mb(), steps, batch, io_pct, tps_p50, tps_best, _device())
    model.close()
    f.close()
    print(f"  P50 {p50:.3f} ms -> {tps_p50:.1f} t/s | P95 {p95:.3f} | P99 {p99:.3f} | "
          f"best {best:.3f} -> {tps_best:.1f} t/s | worst {worst:.3f}")
    print(json.dumps(res, indent=2))
    if out_json:
        with open(out_json, "w") as fp:
            json.dump(res, fp, indent=2)
        print(f"-> {out_json} written.")
    return res


def run_streaming_bench(path: str, steps: int = 3, batch: int = 4,
                        pinned: Optional[Sequence[bool]] = None, seed: int = 2) -> dict:
    """Streaming mode: weights in pinned host memory, each layer copied into
    one of two HBM slots on a side stream while the previous one computes
    (StreamingRunner); reports total / I/O / compute / wait of the best step."""
    init(0)
    _banner("MojoStream  -  streaming mode (pinned host -> 2 HBM slots)")
    rss0 = rss_mb()
    f = st.MojoStreamFile(path)
    f.validate_gemma4_shape()
    print("  ShapeGuard:         OK")
    f.validate_tensor_entries()
    print(f"  TensorGuard:        OK ({f.meta.n_tensors} entries checked)")
    m_ = f.meta
    print(f"  model: D={m_.hidden} KV={m_.kv_dim} FFN={m_.ffn_dim} layers={m_.n_layers}")
    model = Model(f.arch(max_len=64 if steps * batch <= 64 else steps * batch), max_seqs=1,
                  max_rows=batch, max_pos=max(64, steps * batch), resident=False,
                  pinned=pinned)
    model.load_file(f)
    f.close()
    print(f"  RSS before load {rss0:.0f} MB, after bind {rss_mb():.0f} MB")
    best = None
    for s in range(steps):
        x = host_normal(batch * m_.hidden, seed, s).reshape(batch, m_.hidden)
        model.forward(x, [s * batch], T=batch)
        stt = model.stream_stats()
        print(f"  step {s + 1}: total={stt['total_ms']:.3f} ms  I/O={stt['io_ms']:.3f} ms  "
              f"compute={stt['compute_ms']:.3f} ms  wait={stt['wait_ms']:.3f} ms")
        if best is None or stt["total_ms"] < best["total_ms"]:
            best = stt
    model.close()
    io_pct = best["wait_ms"] / best["total_ms"] * 100.0 if best["total_ms"] > 0 else 0.0
    tps = batch / (best["total_ms"] / 1e3)
    print(f"  best step {best['total_ms']:.3f} ms, I/O wait {best['wait_ms']:.3f} ms "
          f"({io_pct:.1f}%), {tps:.1f} t/s (b={batch}), peak RSS {rss_mb():.0f} MB")
    return dict(best, io_pressure_pct=io_pct, tokens_per_sec=tps)


def run_q4_benchmark(shapes=((4, 1024, 1024), (64, 1024, 1024), (4, 4096, 4096),
                             (1024, 1024, 1024)), reps: int = 20, seed: int = 3) -> list:
    """GFLOPS and weight GB/s of ms_q4_matmul at the reference's shapes
    (benchmark_q4.mojo:128-145).  Best of `reps`, timed on the device
    stream around the call (inputs resident)."""
    init(0)
    _banner("Q4 kernel benchmark (ms_q4_matmul)")
    L = lib()
    out = []
    for M, K, N in shapes:
        a = DeviceBuffer.from_array(host_normal(M * K, seed, 1).reshape(M, K))
        raw = DeviceBuffer.from_array(host_random_u8(K * N // 2, seed, 2))
        w = DeviceBuffer(K * N // 2)
        c = DeviceBuffer(M * N * 4)
        check(L.ms_q4_pack(w.ptr, raw.ptr, K, N))
        check(L.ms_synchronize())
        best = None
        for _ in range(reps):
            t0 = time.perf_counter_ns()
            check(L.ms_q4_matmul(c.ptr, a.ptr, w.ptr, M, K, N, C.c_float(0.1), 0))
            check(L.ms_synchronize())
            dt = time.perf_counter_ns() - t0
            best = dt if best is None else min(best, dt)
        flops = 2.0 * M * K * N
        gf = flops / (best / 1e9) / 1e9
        gbs = (K * N / 2) / (best / 1e9) / 1e9
        print(f"M={M} K={K} N={N}: {best / 1e6:.4f} ms / {gf:.1f} GFLOPS / {gbs:.1f} GB/s "
              f"of Q4 weights")
        out.append(dict(M=M, K=K, N=N, ms=best / 1e6, gflops=gf, weight_gbs=gbs))
        for b in (a, raw, w, c):
            b.free()
    return out


def run_e4b_infer(path: Optional[str] = None, lm_head_path: Optional[str] = None,
                  prompt: Sequence[int] = (2, 603, 5012, 575, 4124, 608), n_stream: int = 32,
                  seed: int = 42, resident: bool = True, temperature: float = 0.7,
                  penalty: float = 1.2, sample_seed: int = 0) -> dict:
    """E4B inference driver: BOS row + prompt (TTFT), then up to `n_stream`
    generated tokens, sampled like the reference's run with its TEMPERATURE 0.7
    and REPETITION_PENALTY 1.2 (gemma4_e4b_infer.mojo:38-39,139,179), with
    `sample_seed` in place of the clock, or greedy (temperature <= 0.01 and
    penalty 1).  Like the reference, generation stops after an EOS id (1,
    TokenMap.is_eos gemma_proto.mojo:51-52; :184-185), which is kept in the
    list.  Without files it builds the seeded E4B-shaped synthetic model
    (vocab 262144)."""
    init(0)
    sampled = temperature > 0.01 or penalty > 1.0
    _banner(f"Gemma-4 E4B inference (T={temperature}, penalty={penalty}, seed={sample_seed})"
            if sampled else "Gemma-4 E4B inference (greedy)")
    t0 = time.perf_counter_ns()
    max_pos = len(prompt) + n_stream + 8
    if path:
        vocab = 0
        if lm_head_path:
            with open(lm_head_path, "rb") as fp:
                vocab = int(np.frombuffer(fp.read(4), np.uint32)[0])
        model = st.load_model(path, lm_head_path, vocab=vocab, max_rows=16, max_pos=max_pos,
                              max_len=max(max_pos, 256), resident=resident)
    else:
        from . import arch_e4b
        model = Model(arch_e4b(max_full_seq=max(max_pos, 256)), max_rows=16, max_pos=max_pos,
                      resident=resident)
        if resident:
            model.fill_synthetic(seed)
        else:
            model.fill_synthetic_host(seed)
    if sampled:
        model.set_sampling(temperature, penalty, sample_seed)
    init_ms = (time.perf_counter_ns() - t0) / 1e6
    t1 = time.perf_counter_ns()
    first = model.prefill(list(prompt), 0)
    ttft_ms = (time.perf_counter_ns() - t1) / 1e6
    print(f"  init {init_ms:.0f} ms | TTFT ({len(prompt)} prompt tokens) {ttft_ms:.2f} ms "
          f"-> token {first}")
    t2 = time.perf_counter_ns()
    gen = [first]
    # one step per call (one graph replay each), so that an EOS ends the run
    for k in range(n_stream):
        ids = (model.decode([gen[-1]], [len(prompt)], 1) if k == 0
               else model.decode_continue(1, 1))
        gen.append(int(ids[0, 0]))
        if gen[-1] == EOS_ID:
            break
    stream_ms = (time.perf_counter_ns() - t2) / 1e6
    model.close()
    avg = stream_ms / max(len(gen) - 1, 1)
    print(f"  generated ids: {gen}")
    print(f"  streaming {len(gen) - 1} tokens: {stream_ms:.1f} ms, {avg:.3f} ms/token, "
          f"{1000.0 / avg:.1f} t/s")
    return dict(init_ms=init_ms, ttft_ms=ttft_ms, ids=gen, ms_per_token=avg)
