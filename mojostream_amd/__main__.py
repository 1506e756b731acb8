"""Command line: the reference's pixi tasks (pixi.toml:7-14) over the GPU path.

  python -m mojostream_amd first_light
  python -m mojostream_amd bench      FILE [--steps N] [--json PATH]
  python -m mojostream_amd stream     FILE [--steps N] [--pin-sparse]
  python -m mojostream_amd bench_q4
  python -m mojostream_amd e4b-infer  [FILE LM_HEAD] [--tokens N] [--stream]
  python -m mojostream_amd fake-model OUT [--e4b] [--layers N] [--seed S]
  python -m mojostream_amd validate   [FILE [LAYER0_REF]]     (validate.mojo)
  python -m mojostream_amd validate-real [FILE [LAYER0_REF]]  (validate_real.mojo)
  python -m mojostream_amd tensorguard [FILE]  (src/tests/validate_real.mojo)
"""
import argparse
import sys


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m mojostream_amd")
    sub = ap.add_subparsers(dest="cmd", required=True)
    sub.add_parser("first_light")
    b = sub.add_parser("bench")
    b.add_argument("file")
    b.add_argument("--steps", type=int, default=100)
    b.add_argument("--json", default="bench_result.json")
    s = sub.add_parser("stream")
    s.add_argument("file")
    s.add_argument("--steps", type=int, default=3)
    s.add_argument("--pin-sparse", action="store_true",
                   help="keep SparsePinEngine's choice of layers in HBM")
    sub.add_parser("bench_q4")
    e = sub.add_parser("e4b-infer")
    e.add_argument("file", nargs="?")
    e.add_argument("lm_head", nargs="?")
    e.add_argument("--tokens", type=int, default=32)
    e.add_argument("--stream", action="store_true", help="stream weights from pinned host")
    e.add_argument("--temperature", type=float, default=0.7,
                   help="sampling temperature, the reference's 0.7 (<= 0.01 with "
                        "--penalty 1: greedy)")
    e.add_argument("--penalty", type=float, default=1.2,
                   help="repetition penalty, the reference's 1.2")
    e.add_argument("--sample-seed", type=int, default=0, help="seed of the draws")
    v = sub.add_parser("validate", help="layer 0 against a layer0_ref.bin (REFB)")
    v.add_argument("file", nargs="?", default="model.mojostream")
    v.add_argument("ref", nargs="?", default="layer0_ref.bin")
    vr = sub.add_parser("validate-real", help="guards, NaN/Inf scan, optional REFB compare")
    vr.add_argument("file", nargs="?", default="model_converted.mojostream")
    vr.add_argument("ref", nargs="?", default="layer0_ref.bin")
    tg = sub.add_parser("tensorguard", help="structural checks and directory checksum")
    tg.add_argument("file", nargs="?", default="models/gemma4_e4b_q4.mojostream")
    g = sub.add_parser("fake-model", help="write a seeded synthetic .mojostream file")
    g.add_argument("out")
    g.add_argument("--e4b", action="store_true", help="E4B shapes (default: demo shapes)")
    g.add_argument("--layers", type=int, default=0)
    g.add_argument("--seed", type=int, default=42)
    g.add_argument("--lm-head", default=None, help="also write a version-1 LM head file")
    a = ap.parse_args(argv)

    from . import drivers, streaming
    if a.cmd == "first_light":
        drivers.demo_first_light()
    elif a.cmd == "bench":
        drivers.run_harness(a.file, steps=a.steps, out_json=a.json)
    elif a.cmd == "stream":
        pinned = None
        if a.pin_sparse:
            with streaming.MojoStreamFile(a.file) as f:
                pinned = streaming.build_pinned_mask(f.meta.n_layers)
        drivers.run_streaming_bench(a.file, steps=a.steps, pinned=pinned)
    elif a.cmd == "bench_q4":
        drivers.run_q4_benchmark()
    elif a.cmd == "e4b-infer":
        drivers.run_e4b_infer(a.file, a.lm_head, n_stream=a.tokens, resident=not a.stream,
                              temperature=a.temperature, penalty=a.penalty,
                              sample_seed=a.sample_seed)
    elif a.cmd == "validate":
        from . import validate
        return 0 if validate.run_validation(a.file, a.ref)["passed"] else 1
    elif a.cmd == "validate-real":
        from . import validate
        r = validate.run_real_validation(a.file, a.ref)
        return 0 if r["stable"] and r.get("ref_passed", True) else 1
    elif a.cmd == "tensorguard":
        from . import validate
        return 0 if validate.tensorguard_report(a.file)["passed"] else 1
    elif a.cmd == "fake-model":
        if a.e4b:
            streaming.write_synthetic_e4b(a.out, a.layers or 42, a.seed)
            if a.lm_head:
                streaming.write_synthetic_lm_head(a.lm_head, 2560, 262144, a.seed)
        else:
            # demo shapes of create_fake_model.py:55-60
            streaming.write_synthetic(a.out, a.layers or 40, 1024, 256, 2048, 16, 4, a.seed)
            if a.lm_head:
                streaming.write_synthetic_lm_head(a.lm_head, 1024, 32768, a.seed)
    return 0


if __name__ == "__main__":
    sys.exit(main())
