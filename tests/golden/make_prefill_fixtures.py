#!/usr/bin/env python3
"""Writes the prefill fixtures tests/golden/prefill_e4b_{variant}_{P}.npz.

Workload: the E4B-shape model (42 layers, vocab 262144, tied Q4 head) with the
seeded synthetic weights (seed 42; "plain": uniform nibbles and the reference's
scale range, as the bench model; "balanced": zero nibbles mapped to 8 and
unit-gain scales, mojostream_amd.unit_gain_scale), a prompt of P seeded token ids
(host_random_u8(4P, 9, 3) as uint32 % vocab, the ids bench.py's TTFT run
uses), positions 0..P-1.  The CPU oracle runs the whole prompt causally and
records, for the last prompt row:
  hidden_sub   every layer's output at dims 0, 8, 16, ... ([42][320] fp32)
  logit_idx / logit_val   the 64 largest logits and 4096 seeded other ones
  argmax, margin          the greedy id and its lead over the runner-up
Run from the repository root: python tests/golden/make_prefill_fixtures.py
(takes several minutes on 8 cores).  The tests compare the GPU prefill of the
same workload against these files.
"""
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import mojostream_amd as ms  # noqa: E402  (host generator only, no GPU use)
from oracle.binding import HostWeights, Oracle  # noqa: E402

SEED = 42
HIDDEN_STRIDE = 8
N_TOP, N_RANDOM = 64, 4096


def prompt_ids(P, vocab):
    return [int(v % vocab) for v in ms.host_random_u8(4 * P, 9, 3).view(np.uint32)]


def fixture(o, variant, P):
    arch = ms.arch_e4b(max_full_seq=P + 8)
    t0 = time.time()
    hw = HostWeights(arch, SEED, balanced=(variant == "balanced"))
    om = hw.model(o)
    ids = prompt_ids(P, arch.vocab)
    x = om.embed_rows(ids)
    y, hs = om.forward_keep(x, 0, [P - 1])
    lg = om.logits_rows(y[P - 1:P])[0]
    order = np.argsort(lg, kind="stable")[::-1]
    top = order[:N_TOP]
    rng = np.random.default_rng(12345)
    rest = np.setdiff1d(rng.choice(arch.vocab, N_RANDOM + N_TOP, replace=False), top)[:N_RANDOM]
    idx = np.concatenate([top, np.sort(rest)]).astype(np.int32)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)),
                        f"prefill_e4b_{variant}_{P}.npz")
    np.savez_compressed(path, hidden_sub=hs[:, 0, ::HIDDEN_STRIDE].astype(np.float32),
                        logit_idx=idx, logit_val=lg[idx].astype(np.float32),
                        argmax=np.int32(order[0]), margin=np.float32(lg[order[0]] - lg[order[1]]),
                        prompt_len=np.int32(P), hidden_stride=np.int32(HIDDEN_STRIDE))
    print(f"{path}: argmax {order[0]} margin {lg[order[0]] - lg[order[1]]:.4f} "
          f"({time.time() - t0:.0f} s)", flush=True)


def main():
    o = Oracle(avx2=True)
    o.set_threads(min(16, os.cpu_count() or 1))
    variants = sys.argv[1:] or ["plain", "balanced"]
    for variant in variants:
        for P in (512, 2048):
            fixture(o, variant, P)


if __name__ == "__main__":
    main()
