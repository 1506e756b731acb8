#!/usr/bin/env python3
"""E4B-shape Q4 decode benchmark on one MI355X.

Workload (Gemma-4-E4B shapes, gemma4_e4b.mojo:33-55): D=2560, 42 layers (35
sliding hd 256 window 512, 7 full hd 512 partial RoPE 128), FFN 10240, vocab
262144 tied Q4 head; seeded random Q4 weights resident in HBM.  A step is one
greedy decode token: embedding -> 42 layers -> final norm -> LM head ->
argmax, with token ids and positions kept on the device (one HIP graph per
step).  Batch 1 (the headline value) runs after a 128-token prompt; batch 4
runs four independent sequences.  TTFT is prompt ids on the host -> first id
on the host for a 512-token prompt.

Prints one JSON line (rank 0, N=1).

Profiling: `--eager` times the decode with eager launches instead of the
graph (rocprofv3 traces those), `--only decode` skips the other sections, and
`--rocpd-summary DB` prints per-kernel averages over the last decode steps of
a rocprofv3 database (the summaries kept with the profiles).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "E4B-shape Q4 decode tokens/s (batch 1/4), TTFT ms; achieved HBM GB/s"
HBM_PEAK_GBPS = 8000.0
# GEMV kernel of the Gate|Up projection (dominant decode kernel by bytes)
GATEUP_KERNEL = "k_gemv<1, 2, 3, 4, 2, 15>"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_bytes_per_token(arch, ctx_len):
    """Algorithmic HBM bytes of one batch-1 decode token: every Q4 weight byte
    once (layers and the tied LM head), plus the K and V rows read by attention
    and the K/V row written."""
    b = arch.weight_bytes() + arch.hidden * arch.vocab // 2
    for d in arch.layers:
        keys = min(ctx_len, d.cache_len)
        b += 2 * keys * d.kv_dim * 4 + 2 * d.kv_dim * 4
    return b


def host_cpu():
    """CPU model name and the cores this process may use."""
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return model, os.cpu_count() or 1, usable


def native_oracle():
    """The oracle compiled with -march=native for this host, in a temporary
    directory (None if the compiler is missing or the build fails)."""
    import subprocess
    import tempfile
    from oracle.binding import Oracle
    out = os.path.join(tempfile.mkdtemp(prefix="oracle_native_"), "liboracle_native.so")
    src = os.path.join(ROOT, "oracle", "ms_oracle.c")
    try:
        subprocess.run(["gcc", "-O3", "-fPIC", "-std=c11", "-ffp-contract=off", "-fno-fast-math",
                        "-march=native", "-shared", "-o", out, src, "-lm", "-lpthread"],
                       check=True, capture_output=True, timeout=120)
        return Oracle(path=out)
    except Exception as e:  # noqa: BLE001 - the variant is optional
        log(f"cpu baseline: no native build ({e})")
        return None


def cpu_baseline(arch, seed, prompt, n_tokens, all_threads):
    """The oracle (C restatement of the reference CPU path with its B-pack
    blocking) timed on the host on a bounded sample of the bench's own
    workload: the 128-token prompt runs untimed (all threads), then n_tokens
    batch-1 decode tokens at positions 128.. are timed.  Headline: the AVX2
    build (-mavx2 -mfma, the reference's target) on 1 thread, as the
    reference's decode runs (one 64-row block, kernels.mojo:212,266).  Also
    reported: the same on a -march=native build, and the AVX2 build split
    over all usable cores (a column split the reference does not have)."""
    import numpy as np
    from oracle.binding import HostWeights, Oracle
    model_name, n_cpu, usable = host_cpu()
    o = Oracle(avx2=True)
    log(f"cpu baseline: host weights, {model_name}, {usable} usable of {n_cpu} cores ({o.name})")
    om = HostWeights(arch, seed).model(o)
    o.set_threads(min(16, usable))
    t0 = time.perf_counter()
    y, _ = om.forward_keep(om.embed_rows(prompt), 0, [len(prompt) - 1])
    first = int(np.argmax(om.logits_rows(y[-1:])[0]))
    log(f"cpu baseline: {len(prompt)}-token prompt (untimed) {time.perf_counter() - t0:.1f}s")
    res = {}
    variants = [("avx2_1_thread", o, 1), ("native_1_thread", native_oracle(), 1),
                (f"avx2_{all_threads}_threads", o, all_threads)]
    for label, orc, threads in variants:
        if orc is None:
            continue
        # every variant decodes the same tokens from the prompt's caches (the
        # rows it writes at 128.. are the same each time)
        om.o = orc
        orc.set_threads(threads)
        tok = first
        t0 = time.perf_counter()
        for k in range(n_tokens):
            tok = om.decode_token(tok, len(prompt) + k)
        dt = time.perf_counter() - t0
        res[label] = n_tokens / dt
        log(f"cpu baseline {label}: {n_tokens / dt:.3f} tok/s")
    o.set_threads(1)
    return {"value": res["avx2_1_thread"], "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{n_tokens} batch-1 greedy decode tokens of the full E4B-shape model at "
                      f"positions {len(prompt)}..{len(prompt) + n_tokens - 1} after the bench's "
                      f"{len(prompt)}-token prompt; oracle AVX2 build, 1 thread",
            "host_cpu": model_name, "nproc": n_cpu, "usable_cores": usable,
            "variants_tokens_per_s": {k: round(v, 4) for k, v in res.items()},
            "variants_note": "native_1_thread: -march=native build, 1 thread; "
                             f"avx2_{all_threads}_threads: the AVX2 build split over "
                             "columns on all usable cores, not the reference's threading"}


def bench_c2(ms, seed=3, rotate_bytes=512 << 20):
    """Isolated Q4 matmul (config 2): C = A . deq(W), A fp32 [M][K] N(0,1),
    W Q4 [K][N] with K = N in {1024, 4096}, M in {1, 4, 64}.  Device time per
    call (ms_bench_q4_matmul), the weights rotated over more than
    rotate_bytes of HBM so that every call reads them from memory
    (run_q4_benchmark, benchmark_q4.mojo:121-147).  Bytes: K*N/2 of weights
    + 4MK + 4MN; FLOPs 2MKN."""
    import ctypes as C
    import numpy as np
    L = ms.lib()
    out = []
    for K in (1024, 4096):
        N = K
        wb = K * N // 2
        n_w = rotate_bytes // wb + 1
        w = ms.DeviceBuffer(n_w * wb)
        ms.check(L.ms_fill_random_u8(w.ptr, n_w * wb, seed, K))  # any bytes are valid panels
        for M in (1, 4, 64):
            a = ms.DeviceBuffer.from_array(ms.host_normal(M * K, seed, M).reshape(M, K))
            c = ms.DeviceBuffer(M * N * 4)
            avg = C.c_double()
            ms.check(L.ms_bench_q4_matmul(c.ptr, a.ptr, w.ptr, wb, n_w, M, K, N, C.c_float(0.1),
                                          2 * n_w, C.byref(avg)))
            t = avg.value * 1e-6
            by = wb + 4 * M * K + 4 * M * N
            out.append({"M": M, "K": K, "N": N, "us": round(avg.value, 3),
                        "gb_per_s": round(by / t / 1e9, 1),
                        "hbm_frac": round(by / t / 1e9 / HBM_PEAK_GBPS, 4),
                        "gflops": round(2.0 * M * K * N / t / 1e9, 1)})
            log(f"c2: M={M} K=N={K}: {avg.value:.2f} us, {by / t / 1e9:.0f} GB/s, "
                f"{2.0 * M * K * N / t / 1e9:.0f} GFLOPS")
            a.free()
            c.free()
        w.free()
    return out


def bench_c1(ms, seed=42, steps=100):
    """Demo decode harness (config 1, bench.mojo -> run_harness harness.mojo:185-328):
    a seeded synthetic demo file (D=1024, 40 layers, 8q/2kv heads, hd 128,
    FFN 4096), 4 rows of one sequence per step, 100 steps, the sequence growing
    by 4 a step; a step is the 40 layers (ms_forward) on rows uploaded before
    the clock starts, as the reference fills x before its timed loop
    (harness.mojo:256-262); repeated steps replay a HIP graph.  P50 / P95 and
    tokens/s as the reference's JSON reports them."""
    import contextlib
    import tempfile
    from mojostream_amd import drivers, streaming as st
    path = os.path.join(tempfile.mkdtemp(prefix="c1_"), "demo.mojostream")
    st.write_synthetic(path, 40, 1024, 256, 4096, 8, 2, seed=seed)
    with contextlib.redirect_stdout(sys.stderr):
        r = drivers.run_harness(path, steps=steps, batch=4, out_json=None)
    os.remove(path)
    keys = ("latency_p50_ms", "latency_p95_ms", "latency_p99_ms", "latency_best_ms",
            "latency_worst_ms", "tokens_per_sec_p50", "tokens_per_sec_best", "ttft_ms")
    res = {k: r[k] for k in keys}
    res["workload"] = "demo model D=1024, 40 layers, batch-4 rows, 100 steps (harness)"
    log(f"c1: {res}")
    return res


def rocpd_summary(db, steps, marker="k_embed", end_marker="k_argmax_fin"):
    """Per-kernel duration statistics over the last `steps` decode steps of a
    rocprofv3 database (a step runs from the embedding kernel to the argmax
    finalization; launches after the last step, such as the sweep, are
    excluded)."""
    import re
    import sqlite3
    c = sqlite3.connect(db)
    cols = [r[1] for r in c.execute("pragma table_info(kernels)")]
    name = "name" if "name" in cols else "kernel_name"
    rows = c.execute(f"select {name}, start, end from kernels order by start").fetchall()
    starts = [i for i, r in enumerate(rows) if marker in r[0]]
    if len(starts) < steps:
        raise SystemExit(f"only {len(starts)} decode steps in {db}")
    last = max(i for i, r in enumerate(rows) if end_marker in r[0])
    seg = rows[starts[-steps]:last + 1]
    agg = {}
    for n, s, e in seg:
        n = re.sub(r"\(.*", "", n).replace("void ", "")
        a = agg.setdefault(n, [0, 0.0, 1e30, 0.0])
        d = (e - s) / 1000.0
        a[0] += 1
        a[1] += d
        a[2] = min(a[2], d)
        a[3] = max(a[3], d)
    wall = (seg[-1][2] - seg[0][1]) / 1000.0 / steps
    busy = sum(v[1] for v in agg.values()) / steps
    out = [f"decode steps: {steps}; wall per step {wall:.1f} us; kernel time per step {busy:.1f} us",
           f"{'kernel':48s} {'calls/step':>10s} {'us/step':>9s} {'avg_us':>8s} {'min_us':>8s} {'max_us':>8s}"]
    for k, v in sorted(agg.items(), key=lambda x: -x[1][1]):
        out.append(f"{k[:48]:48s} {v[0] / steps:10.1f} {v[1] / steps:9.1f} {v[1] / v[0]:8.2f} "
                   f"{v[2]:8.2f} {v[3]:8.2f}")
    return "\n".join(out)


def pmc_summary(fetch_csv, write_csv, kernel, copy_bytes):
    """HBM traffic per dispatch of `kernel` (decode launches: one activation
    row) from two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE; KiB per
    dispatch), each scaled by what the same counter reads for the plain copy of
    copy_bytes in the same run."""
    import csv
    res = {}
    for path, counter in ((fetch_csv, "FETCH_SIZE"), (write_csv, "WRITE_SIZE")):
        rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]
        # the largest copy dispatch of the run is the calibration copy
        copy = [float(r["Counter_Value"]) for r in rows if "copyBuffer" in r["Kernel_Name"]]
        if not copy:
            raise SystemExit(f"no calibration copy in {path}")
        # the copy reads and writes copy_bytes
        factor = copy_bytes / 1024.0 / max(copy)
        # decode launches (one activation row: the smallest grid of the kernel;
        # decode attention's grid follows the position, so all of its launches)
        ks = [r for r in rows if kernel in r["Kernel_Name"]]
        g = min((int(r["Grid_Size"]) for r in ks), default=0)
        vals = [float(r["Counter_Value"]) for r in ks
                if int(r["Grid_Size"]) == g or "attn_decode" in kernel]
        if not vals:
            raise SystemExit(f"no {kernel} dispatches in {path}")
        res[counter] = {"factor": factor, "n": len(vals), "min_kib": min(vals),
                        "median_kib": sorted(vals)[len(vals) // 2],
                        "bytes": sorted(vals)[len(vals) // 2] * 1024.0 * factor}
    res["traffic_bytes"] = res["FETCH_SIZE"]["bytes"] + res["WRITE_SIZE"]["bytes"]
    return res


def traffic_from_profile():
    """Traffic per launch of the dominant kernel as recorded in the committed
    profile summary (measured with rocprofv3 --pmc), or None."""
    path = os.path.join(ROOT, "profiles", "gateup_gemv_e4b_decode_hbm_traffic.txt")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def measure_ttft(ms, prompts, seed, reps=3):
    """TTFT: prompt ids on the host -> first greedy id on the host, one
    E4B-shape model per prompt length.  One untimed prefill of the same prompt
    first (kernel code objects loaded, the same launches), then the median of
    `reps` timed prefills, each from an emptied cache (model reset)."""
    import numpy as np
    ttft = {}
    for P in prompts:
        mt = ms.Model(ms.arch_e4b(max_full_seq=P + 8), max_seqs=1, max_rows=16, max_pos=P + 8)
        mt.fill_synthetic(seed)
        pr = [int(v % 262144) for v in ms.host_random_u8(4 * P, 9, 3).view(np.uint32)]
        mt.prefill(pr, 0)  # untimed
        runs = []
        for _ in range(reps):
            mt.reset()
            ms.synchronize()
            t0 = time.perf_counter()
            mt.prefill(pr, 0)
            runs.append((time.perf_counter() - t0) * 1e3)
        runs.sort()
        ttft[P] = runs[len(runs) // 2]
        log(f"TTFT prompt {P}: {ttft[P]:.1f} ms (median of {reps}; "
            + ", ".join(f"{r:.1f}" for r in runs) + ")")
        mt.close()
    return ttft


def host_link_gbps(ms, nbytes=1 << 30):
    """Pinned host -> HBM copy rate of one large copy (the streaming bound)."""
    import ctypes as C
    h = C.c_void_p()
    ms.check(ms.lib().ms_host_alloc(C.byref(h), nbytes))
    d = ms.DeviceBuffer(nbytes)
    try:
        ms.check(ms.lib().ms_memcpy_h2d(d.ptr, h.value, nbytes))  # warm-up
        best = 1e30
        for _ in range(3):
            t0 = time.perf_counter()
            ms.check(ms.lib().ms_memcpy_h2d(d.ptr, h.value, nbytes))
            best = min(best, time.perf_counter() - t0)
    finally:
        d.free()
        ms.lib().ms_host_free(h.value)
    return nbytes / best / 1e9


def bench_c5(ms, seed, steps, prompt_len):
    """14B-class streaming decode (config 5): 48 layers of 6.6 GB Q4 weights in
    pinned host memory, streamed layer by layer into two HBM slots on the copy
    stream (StreamingRunner semantics, stream_runner.mojo:460-562); tied Q4
    head (vocab 262144) resident.  A seeded prompt of prompt_len ids, then
    `steps` greedy steps; per step the copy time (io), the time compute waited
    for a copy (wait) and the rest (compute), as run_streaming_bench reports
    them (:503-546)."""
    import numpy as np
    arch = ms.arch_14b(max_len=prompt_len + steps + 8)
    m = ms.Model(arch, max_seqs=1, max_rows=4, max_pos=prompt_len + steps + 8, resident=False)
    t0 = time.perf_counter()
    m.fill_synthetic(seed)
    log(f"c5: 14B weights generated into pinned memory in {time.perf_counter() - t0:.1f}s")
    link = host_link_gbps(ms)
    log(f"c5: pinned host -> HBM copy {link:.1f} GB/s")
    prompt = [int(v % arch.vocab) for v in ms.host_random_u8(4 * prompt_len, 9, 50).view(np.uint32)]
    ms.synchronize()
    t0 = time.perf_counter()
    tok = m.prefill(prompt, 0)
    ttft = (time.perf_counter() - t0) * 1e3
    log(f"c5: prefill of {prompt_len} tokens {ttft:.0f} ms")
    io = wait = total = 0.0
    t0 = time.perf_counter()
    for k in range(steps):
        out = (m.decode([tok], [prompt_len], 1, use_graph=False) if k == 0
               else m.decode_continue(1, 1, use_graph=False))
        tok = int(out[0, 0])
        st = m.stream_stats()
        io += st["io_ms"]
        wait += st["wait_ms"]
        total += st["total_ms"]
        if (k + 1) % 32 == 0:
            log(f"c5: step {k + 1}/{steps}: {total / (k + 1):.1f} ms/step, io {io / (k + 1):.1f} ms")
    dt = time.perf_counter() - t0
    layer_bytes = arch.weight_bytes()
    m.close()
    ms_step = dt * 1e3 / steps
    return {"workload": "14B-class streaming decode: D=5120, 48 layers, 40q/8kv heads, hd 128, "
                        "FFN 13824, all full attention; layers streamed from pinned host memory "
                        "through 2 HBM slots; tied Q4 head resident",
            "prompt_tokens": prompt_len, "decode_steps": steps, "context_end": prompt_len + steps,
            "tokens_per_s": round(1e3 / ms_step, 3), "ms_per_token": round(ms_step, 2),
            "io_ms_per_token": round(io / steps, 2), "wait_ms_per_token": round(wait / steps, 2),
            "compute_ms_per_token": round((total - wait) / steps, 2),
            "streamed_bytes_per_token": layer_bytes,
            "stream_gbps": round(layer_bytes / (io / steps * 1e-3) / 1e9, 1),
            "host_link_gbps_measured": round(link, 1),
            "stream_frac_of_link": round(layer_bytes / (io / steps * 1e-3) / 1e9 / link, 3),
            "prefill_ms": round(ttft, 1)}


def bench_sparse_pin(ms, seed, steps=32, prompt_len=32):
    """E4B-scale streaming with SparsePinEngine's pinning (sparse_pin.mojo:
    49-330; the gemma4_e4b_infer.mojo:160-186 loop): a 42-layer E4B-shape
    .mojostream file and its LM head file, loaded twice as streaming models,
    once with the 24 layers of build_pinned_mask() kept in HBM and once with
    none; each runs a seeded prompt and `steps` greedy steps, one call per
    step.  Per token: copy time (io), the time compute waited for a copy,
    bytes streamed, and the hit rate (pinned layer passes / all), the figures
    the reference publishes for its SSD run (README.md:424-431)."""
    import shutil
    import tempfile
    import numpy as np
    from mojostream_amd import streaming as st
    d = tempfile.mkdtemp(prefix="e4b_")
    path, lm = os.path.join(d, "e4b.mojostream"), os.path.join(d, "lm_head.bin")
    t0 = time.perf_counter()
    st.write_synthetic_e4b(path, 42, seed=seed)
    st.write_synthetic_lm_head(lm, 2560, 262144, seed=seed)
    log(f"sparse-pin: E4B file written in {time.perf_counter() - t0:.1f}s")
    prompt = [int(v % 262144) for v in ms.host_random_u8(4 * prompt_len, 9, 81).view(np.uint32)]
    out = {"workload": "E4B-shape .mojostream file (42 layers, 1.97 GB Q4) streamed from pinned "
                       "host memory through 2 HBM slots; tied Q4 head resident",
           "prompt_tokens": prompt_len, "decode_steps": steps,
           "reference_ssd_run": {"ms_per_token": 1843, "io_mb_per_token": 826,
                                 "hit_rate": 0.571}}
    try:
        for name, mask in (("pinned_24", st.build_pinned_mask()), ("streamed_all", None)):
            max_pos = prompt_len + steps + 8
            t0 = time.perf_counter()
            m = st.load_model(path, lm_head_path=lm, vocab=262144, max_rows=16, max_pos=max_pos,
                              max_len=max_pos, resident=False, pinned=mask)
            load_s = time.perf_counter() - t0
            tok = m.prefill(prompt, 0)
            io = wait = total = nbytes = 0.0
            hits = passes = 0
            t0 = time.perf_counter()
            for k in range(steps):
                o = (m.decode([tok], [prompt_len], 1) if k == 0 else m.decode_continue(1, 1))
                tok = int(o[0, 0])
                s = m.stream_stats()
                io += s["io_ms"]
                wait += s["wait_ms"]
                total += s["total_ms"]
                nbytes += s["bytes"]
                hits += s["layers_pinned"]
                passes += s["layers_pinned"] + s["layers_streamed"]
            dt = time.perf_counter() - t0
            m.close()
            r = {"ms_per_token": round(dt * 1e3 / steps, 2),
                 "tokens_per_s": round(steps / dt, 2),
                 "io_ms_per_token": round(io / steps, 2),
                 "wait_ms_per_token": round(wait / steps, 2),
                 "compute_ms_per_token": round((total - wait) / steps, 2),
                 "streamed_mb_per_token": round(nbytes / steps / 1e6, 1),
                 "stream_gbps": round(nbytes / (io * 1e-3) / 1e9, 1) if io > 0 else None,
                 "hit_rate": round(hits / passes, 3),
                 "load_s": round(load_s, 2)}
            log(f"sparse-pin {name}: {r['ms_per_token']} ms/token, io {r['io_ms_per_token']} ms, "
                f"wait {r['wait_ms_per_token']} ms, {r['streamed_mb_per_token']} MB/token, "
                f"hit rate {r['hit_rate']}")
            out[name] = r
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--ttft-prompt", type=int, default=512)
    ap.add_argument("--cpu-tokens", type=int, default=8)
    ap.add_argument("--c2", action=argparse.BooleanOptionalAction, default=True,
                    help="isolated Q4 matmul section (config 2)")
    ap.add_argument("--c1", action=argparse.BooleanOptionalAction, default=True,
                    help="demo decode harness section (config 1)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--eager", action="store_true", help="time the decode with eager launches")
    ap.add_argument("--only", choices=["all", "decode", "ttft", "c5", "sparse-pin"],
                    default="all",
                    help="decode: batch-1 decode only; ttft: prefill (TTFT) only; c5: the 14B "
                         "streaming section only; sparse-pin: the E4B pinning section only")
    ap.add_argument("--prof-tokens", type=int, default=16)
    ap.add_argument("--rocpd-summary", metavar="DB", help="summarize a rocprofv3 database and exit")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="one device-to-device copy of this size (HBM counter calibration)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="HBM traffic of a decode kernel from two --pmc runs and exit")
    ap.add_argument("--pmc-kernel", default=GATEUP_KERNEL,
                    help="kernel name (substring) for --pmc-summary")
    ap.add_argument("--seed", type=int, default=42)
    ap.add_argument("--c5-steps", type=int, default=256,
                    help="decode steps of the 14B streaming section (0: skip it)")
    ap.add_argument("--c5-prompt", type=int, default=3840)
    ap.add_argument("--sparse-pin-steps", type=int, default=32,
                    help="decode steps of the E4B sparse-pinning streaming section (0: skip it)")
    args = ap.parse_args()
    if args.rocpd_summary:
        print(rocpd_summary(args.rocpd_summary, args.steps))
        return
    if args.pmc_summary:
        r = pmc_summary(args.pmc_summary[0], args.pmc_summary[1], args.pmc_kernel,
                        (args.copy_mib or 256) << 20)
        for c in ("FETCH_SIZE", "WRITE_SIZE"):
            v = r[c]
            print(f"{c}: dispatches {v['n']}, median {v['median_kib']:.1f} KiB, min {v['min_kib']:.1f} KiB, "
                  f"copy calibration factor {v['factor']:.4f} -> {v['bytes']:.0f} bytes")
        print(f"traffic_bytes_per_launch: {r['traffic_bytes']:.0f}")
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note only)"}))
        sys.exit(2)

    import numpy as np
    import mojostream_amd as ms

    ms.init(0)
    name, ncu, hbm = ms.device_info()
    log(f"device {name} CUs={ncu}")
    if args.only == "c5":
        print(json.dumps({"c5_streaming_14b": bench_c5(ms, args.seed, args.c5_steps,
                                                         args.c5_prompt), "device": name}))
        return
    if args.only == "sparse-pin":
        print(json.dumps({"e4b_sparse_pin": bench_sparse_pin(ms, args.seed,
                                                             args.sparse_pin_steps),
                          "device": name}))
        return
    if args.only == "ttft":
        ttft = measure_ttft(ms, sorted({args.ttft_prompt, 2048}), args.seed)
        print(json.dumps({"ttft_ms": {str(k): round(v, 2) for k, v in ttft.items()},
                          "device": name}))
        return
    max_pos = max(args.prompt + args.warmup + args.steps + args.prof_tokens + 8,
                  args.ttft_prompt + 8)
    arch = ms.arch_e4b(max_full_seq=max_pos)
    use_graph = not args.eager

    # ---- batch 1 ---------------------------------------------------------------
    m = ms.Model(arch, max_seqs=4, max_rows=4, max_pos=max_pos)
    t0 = time.perf_counter()
    m.fill_synthetic(args.seed)
    log(f"weights generated+packed in {time.perf_counter() - t0:.1f}s")
    prompt = [int(v % arch.vocab) for v in ms.host_random_u8(4 * args.prompt, 9, 1).view(np.uint32)]
    first = m.prefill(prompt, 0)
    pos = len(prompt)
    ids_w = m.decode([first], [pos], args.warmup, use_graph=use_graph)  # warmup (+ graph capture)
    pos += args.warmup
    tok = int(ids_w[-1, 0])
    ms.synchronize()
    t0 = time.perf_counter()
    ids = m.decode([tok], [pos], args.steps, use_graph=use_graph)
    ms.synchronize()
    dt1 = time.perf_counter() - t0
    pos += args.steps
    tps1 = args.steps / dt1
    ms_step = dt1 * 1e3 / args.steps
    log(f"batch 1: {tps1:.1f} tok/s ({ms_step:.3f} ms/token, {'graph' if use_graph else 'eager'})")
    ctx_mid = len(prompt) + args.warmup + args.steps // 2
    bpt = decode_bytes_per_token(arch, ctx_mid)
    step_gbps = bpt / (dt1 / args.steps) / 1e9

    # ---- instrumented pass, then the dominant kernel's duration on the device --
    # The profiled eager pass records the last launch of each projection class;
    # ms_prof_sweep re-launches it back to back over every layer's weights
    # between two HIP events on the launch stream (weights cold, as in a step).
    ms.prof_enable(True)
    m.decode([int(ids[-1, 0])], [pos], args.prof_tokens, use_graph=False)
    pos += args.prof_tokens
    prof = ms.prof_get()
    ms.prof_enable(False)
    eager_ms = sum(v["ms"] for v in prof.values()) / args.prof_tokens
    log(f"per-class (eager + events, {args.prof_tokens} tokens): " + ", ".join(
        f"{k} {v['ms'] / args.prof_tokens:.3f}ms" for k, v in prof.items() if v["launches"]))
    sweeps = {}
    for cls in ("qkv_gemv", "attention", "o_gemv", "gateup_gemv", "down_gemv"):
        sw = ms.prof_sweep(m, cls, passes=2)
        sw["gbps"] = sw["bytes_per_launch"] / (sw["avg_us"] * 1e-6) / 1e9
        sweeps[cls] = {k: round(v, 3) for k, v in sw.items()}
        log(f"sweep {cls}: {sw['avg_us']:.2f} us/launch, {sw['gbps']:.0f} GB/s "
            f"({sw['launches']} launches)")
    gu = sweeps["gateup_gemv"]
    roof = {"bound": "hbm", "kernel": f"{GATEUP_KERNEL} (Gate|Up Q4 GEMV, SwiGLU epilogue)",
            "achieved": gu["bytes_per_launch"] / (gu["avg_us"] * 1e-6) / 1e9,
            "peak": HBM_PEAK_GBPS, "unit": "GB/s", "traffic": traffic_from_profile(),
            "avg_launch_us": gu["avg_us"], "bytes_per_launch": gu["bytes_per_launch"]}
    roof["frac"] = roof["achieved"] / roof["peak"]
    for sw in sweeps.values():
        sw["hbm_frac"] = round(sw["gbps"] / HBM_PEAK_GBPS, 4)

    out = {
        "metric": METRIC, "value": round(tps1, 2), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (seeded random Q4 weights, seeded random prompt ids)",
        "config": {"workload": "E4B-shape Q4 greedy decode, batch 1, weights resident",
                   "hidden": 2560, "layers": 42, "ffn": 10240, "vocab": 262144,
                   "prompt_tokens": args.prompt, "decode_steps": args.steps,
                   "launch": "hip graph per step" if use_graph else "eager",
                   "parallelism": "single GPU"},
        "step_hbm_gbps": round(step_gbps, 1),
        "step_roofline_frac": round(step_gbps / HBM_PEAK_GBPS, 4),
        "bytes_per_token": bpt,
        "eager_ms_per_token": round(eager_ms, 4),
        "roofline": roof,
        "kernel_sweep": sweeps,
        "device": name,
    }

    if args.only == "all":
        # ---- batch 4 ----------------------------------------------------------------
        import ctypes as C
        check = ms.lib()
        firsts, lens = [], []
        for s in range(4):
            p = [int(v % arch.vocab) for v in ms.host_random_u8(4 * args.prompt, 9, 20 + s).view(np.uint32)]
            t = np.asarray(p, np.int32)
            f = C.c_int32()
            ms.check(check.ms_prefill(m.h, s, t.ctypes.data, len(t), 0, C.byref(f)))
            firsts.append(int(f.value))
            lens.append(len(p))
        w4 = m.decode(firsts, lens, args.warmup, use_graph=use_graph)
        ms.synchronize()
        t0 = time.perf_counter()
        m.decode(w4[-1].tolist(), [l + args.warmup for l in lens], args.steps, use_graph=use_graph)
        ms.synchronize()
        dt4 = time.perf_counter() - t0
        tps4 = 4 * args.steps / dt4
        log(f"batch 4: {tps4:.1f} tok/s")
        out["batch4_tokens_per_s"] = round(tps4, 2)
        m.close()

        ttft = measure_ttft(ms, sorted({args.ttft_prompt, 2048}), args.seed)
        out["ttft_ms"] = {str(k): round(v, 2) for k, v in ttft.items()}
        if args.c2:
            out["c2_q4_matmul"] = bench_c2(ms)
        if args.c1:
            out["c1_harness"] = bench_c1(ms)
        if args.c5_steps > 0:
            out["c5_streaming_14b"] = bench_c5(ms, args.seed, args.c5_steps, args.c5_prompt)
        if args.sparse_pin_steps > 0:
            out["e4b_sparse_pin"] = bench_sparse_pin(ms, args.seed, args.sparse_pin_steps)
    else:
        m.close()

    if args.copy_mib:
        # a plain copy of known size: what FETCH_SIZE/WRITE_SIZE read for it
        # scales the counters of the GEMV launches
        nb = args.copy_mib << 20
        src, dst = ms.DeviceBuffer(nb), ms.DeviceBuffer(nb)
        ms.check(ms.lib().ms_memcpy_d2d(dst.ptr, src.ptr, nb))
        ms.synchronize()
        out["copy_calibration_bytes"] = nb
        src.free()
        dst.free()

    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(arch, args.seed, prompt, args.cpu_tokens,
                                           min(16, host_cpu()[2]))
    print(json.dumps(out))


if __name__ == "__main__":
    main()
