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


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_bytes_per_token(arch, ctx_len):
    """Algorithmic HBM bytes of one batch-1 decode token: every Q4 weight byte
    once, plus the K and V rows read by attention and the row written."""
    b = arch.weight_bytes() + arch.hidden * arch.vocab // 2
    for d in arch.layers:
        if d.cache_kind == 1:
            keys = min(ctx_len, d.cache_len)
        else:
            keys = min(ctx_len, d.cache_len)
        b += 2 * keys * d.kv_dim * 4 + 2 * d.kv_dim * 4
    return b


def cpu_baseline(ms, arch, seed, n_tokens):
    """The oracle (C restatement of the reference CPU path, B-pack blocking,
    single thread like the reference's decode, AVX2 build when the host has
    it) timed on a bounded sample: n_tokens decode tokens of the full model."""
    from oracle.binding import Oracle, synthetic_oracle_model
    o = Oracle(avx2=True)
    o.set_threads(1)
    log(f"cpu baseline: building host weights ({o.name})")
    om = synthetic_oracle_model(o, arch, seed)
    tok = 11
    t0 = time.perf_counter()
    for p in range(n_tokens):
        tok = om.decode_token(tok, p)
        log(f"cpu baseline: token {p + 1}/{n_tokens} {time.perf_counter() - t0:.1f}s")
    dt = time.perf_counter() - t0
    return {"value": n_tokens / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{n_tokens} batch-1 decode tokens of the full E4B-shape model "
                      f"(positions 0..{n_tokens - 1}), oracle/{o.name}, 1 thread"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--ttft-prompt", type=int, default=512)
    ap.add_argument("--cpu-tokens", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--seed", type=int, default=42)
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note only)"}))
        sys.exit(2)

    import numpy as np
    import mojostream_amd as ms

    ms.init(0)
    name, ncu, hbm = ms.device_info()
    log(f"device {name} CUs={ncu}")
    max_pos = max(args.prompt + args.warmup + args.steps + 8, args.ttft_prompt + 8)
    arch = ms.arch_e4b(max_full_seq=max_pos)

    # ---- batch 1 ---------------------------------------------------------------
    m = ms.Model(arch, max_seqs=4, max_rows=4, max_pos=max_pos)
    t0 = time.perf_counter()
    m.fill_synthetic(args.seed)
    log(f"weights generated+packed in {time.perf_counter() - t0:.1f}s")
    prompt = [int(v % arch.vocab) for v in ms.host_random_u8(4 * args.prompt, 9, 1).view(np.uint32)]
    first = m.prefill(prompt, 0)
    pos = len(prompt)
    ids_w = m.decode([first], [pos], args.warmup)  # warmup (also captures the graph)
    pos += args.warmup
    tok = int(ids_w[-1, 0])
    ms.synchronize()
    check = ms.lib()
    t0 = time.perf_counter()
    ids = m.decode([tok], [pos], args.steps)
    ms.synchronize()
    dt1 = time.perf_counter() - t0
    tps1 = args.steps / dt1
    ms_step = dt1 * 1e3 / args.steps
    log(f"batch 1: {tps1:.1f} tok/s ({ms_step:.3f} ms/token)")
    ctx_mid = pos + args.steps // 2
    bpt = decode_bytes_per_token(arch, ctx_mid)
    step_gbps = bpt / (dt1 / args.steps) / 1e9

    # ---- instrumented pass: per-kernel-class HIP events (eager launches) -------
    ms.prof_enable(True)
    m.decode([int(ids[-1, 0])], [pos + args.steps], 16, use_graph=False)
    prof = ms.prof_get()
    ms.prof_enable(False)
    gu = prof["gateup_gemv"]
    gu_ms = gu["ms"] / max(gu["launches"], 1)
    gu_bytes = gu["bytes"] / max(gu["launches"], 1)
    roof = {"bound": "hbm", "kernel": "k_gemv<0,2> (Gate+Up Q4 GEMV, SwiGLU epilogue)",
            "achieved": gu_bytes / (gu_ms * 1e-3) / 1e9, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "traffic": None, "avg_launch_us": gu_ms * 1e3,
            "bytes_per_launch": gu_bytes}
    roof["frac"] = roof["achieved"] / roof["peak"]
    eager_ms = sum(v["ms"] for v in prof.values()) / 16
    log("per-class (eager, 16 tokens): " + ", ".join(
        f"{k} {v['ms'] / 16:.3f}ms" for k, v in prof.items() if v["launches"]))

    # ---- batch 4 ------------------------------------------------------------------
    firsts, lens = [], []
    for s in range(4):
        p = [int(v % arch.vocab) for v in ms.host_random_u8(4 * args.prompt, 9, 20 + s).view(np.uint32)]
        import ctypes as C
        t = np.asarray(p, np.int32)
        f = C.c_int32()
        ms.check(check.ms_prefill(m.h, s, t.ctypes.data, len(t), 0, C.byref(f)))
        firsts.append(int(f.value))
        lens.append(len(p))
    w4 = m.decode(firsts, lens, args.warmup)
    ms.synchronize()
    t0 = time.perf_counter()
    m.decode(w4[-1].tolist(), [l + args.warmup for l in lens], args.steps)
    ms.synchronize()
    dt4 = time.perf_counter() - t0
    tps4 = 4 * args.steps / dt4
    log(f"batch 4: {tps4:.1f} tok/s")
    m.close()

    # ---- TTFT (prompt ids on host -> first id on host) --------------------------
    ttft = {}
    for P in sorted({args.ttft_prompt, 2048}):
        if P > max_pos - 8:
            continue
        mt = ms.Model(ms.arch_e4b(max_full_seq=max_pos), max_seqs=1, max_rows=16,
                      max_pos=max_pos)
        mt.fill_synthetic(args.seed)
        pr = [int(v % arch.vocab) for v in ms.host_random_u8(4 * P, 9, 3).view(np.uint32)]
        mt.prefill(pr[:16], 0)  # warm-up of the prefill kernels
        mt.reset()
        ms.synchronize()
        t0 = time.perf_counter()
        mt.prefill(pr, 0)
        ttft[P] = (time.perf_counter() - t0) * 1e3
        log(f"TTFT prompt {P}: {ttft[P]:.1f} ms")
        mt.close()

    out = {
        "metric": METRIC, "value": round(tps1, 2), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (seeded random Q4 weights, seeded random prompt ids)",
        "config": {"workload": "E4B-shape Q4 greedy decode, batch 1, weights resident",
                   "hidden": 2560, "layers": 42, "ffn": 10240, "vocab": 262144,
                   "prompt_tokens": args.prompt, "decode_steps": args.steps,
                   "parallelism": "single GPU"},
        "batch4_tokens_per_s": round(tps4, 2),
        "ttft_ms": {str(k): round(v, 2) for k, v in ttft.items()},
        "step_hbm_gbps": round(step_gbps, 1),
        "step_roofline_frac": round(step_gbps / HBM_PEAK_GBPS, 4),
        "bytes_per_token": bpt,
        "eager_ms_per_token": round(eager_ms, 4),
        "roofline": roof,
        "device": name,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(ms, arch, args.seed, args.cpu_tokens)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
