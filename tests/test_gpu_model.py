"""Layer-loop parity of the HIP path against the CPU oracle through the C ABI.

Bars (validate_layer.mojo:31 and the decode contract): per-layer fp32 hidden
states within relative RMSE 1e-4; greedy token ids identical to the oracle.
"""
import os

import numpy as np
import pytest

from oracle.binding import Oracle, synthetic_oracle_model

pytestmark = pytest.mark.gpu
SEED = 42


def say(msg):
    print(f"\n[case] {msg}", flush=True)


def rel_rmse(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.sqrt(np.mean((a - b) ** 2)) / (np.sqrt(np.mean(b ** 2)) + 1e-30))


@pytest.fixture(scope="module")
def fast_oracle():
    o = Oracle(avx2=True)
    o.set_threads(min(16, os.cpu_count() or 1))
    return o


def build(ms, arch, **kw):
    m = ms.Model(arch, **kw)
    m.fill_synthetic(SEED)
    return m


def prompt_ids(n, vocab, stream):
    import mojostream_amd as ms
    return [int(v % vocab) for v in ms.host_random_u8(4 * n, 9, stream).view(np.uint32)]


# ---- demo model (config: D=1024, 40 layers, 8q/2kv, hd 128, F 4096) -----------------
def test_demo_harness_100_steps(gpu, fast_oracle):
    """The harness workload itself (run_harness, harness.mojo:236-269): the
    40-layer demo model, fresh N(0,1) rows [4][1024] every step at bases 0, 4,
    .., 396, 100 steps, against the threaded oracle: the output rows of every
    step, and every layer's rows at sampled steps including the last (per-layer
    bar of validate_layer.mojo:138-154)."""
    ms = gpu
    arch = ms.arch_demo(max_len=512)
    say("demo 40 layers, batch-4 rows, the harness's 100 steps (bases 0..396)")
    m = build(ms, arch, max_seqs=1, max_rows=4, max_pos=512)
    om = synthetic_oracle_model(fast_oracle, arch, SEED, with_lm=False)
    sampled = {0, 1, 2, 50, 98, 99}
    worst_out = worst_layer = 0.0
    for step in range(100):
        base = 4 * step
        x = ms.host_normal(4 * 1024, 1000 + step, 1).reshape(4, 1024)
        if step in sampled:
            g_out, g_hid = m.forward(x, [base], T=4, hidden=True)
            o_out, o_hid = om.forward(x, base, hidden=True)
            errs = [rel_rmse(g_hid[l], o_hid[l]) for l in range(arch.n_layers)]
            worst_layer = max(worst_layer, max(errs))
            print(f"  step {step} (base {base}): max per-layer rel RMSE {max(errs):.2e} "
                  f"(layer {int(np.argmax(errs))})")
            assert np.array_equal(g_out, g_hid[-1])
        else:
            g_out = m.forward(x, [base], T=4)
            o_out = om.forward(x, base)
        worst_out = max(worst_out, rel_rmse(g_out, o_out))
    print(f"  100 steps: output rows rel RMSE max {worst_out:.2e}, sampled layers max "
          f"{worst_layer:.2e}")
    assert worst_out < 1e-4 and worst_layer < 1e-4
    m.close()


@pytest.mark.parametrize("T", [4, 3, 2])
def test_demo_teacher_forced_layers(gpu, fast_oracle, T):
    """Steps of T rows of one sequence (T = 2..4: the chunk partials per row
    and their merge, k_attn_rows), layer by layer against the oracle, at bases
    0, T and 63 (a step across a 32-key chunk boundary)."""
    ms = gpu
    arch = ms.arch_demo(max_len=512, n_layers=6)
    say(f"demo teacher-forced, 6 layers x 3 steps of {T} rows")
    m = build(ms, arch, max_seqs=1, max_rows=4, max_pos=512)
    om = synthetic_oracle_model(fast_oracle, arch, SEED, with_lm=False)
    for step, base in enumerate((0, T, 63)):
        if step == 2:
            # fill positions 2T .. 62 so that the step at 63 attends written rows
            fill = ms.host_normal((63 - 2 * T) * 1024, 90, 2).reshape(63 - 2 * T, 1024)
            for r0 in range(0, fill.shape[0], 4):
                rows = fill[r0:r0 + 4]
                xr = rows
                for l in range(arch.n_layers):
                    ref = om.layer_forward(l, xr, 2 * T + r0)
                    m.layer_forward(l, xr, [2 * T + r0], T=rows.shape[0])
                    xr = ref
        x = ms.host_normal(T * 1024, 77 + step, 2).reshape(T, 1024)
        for l in range(arch.n_layers):
            ref = om.layer_forward(l, x, base)
            got = m.layer_forward(l, x, [base], T=T)
            e = rel_rmse(got, ref)
            assert e < 1e-4, (step, l, e)
            x = ref  # feed the oracle's output to the next GPU layer
    m.close()


# ---- E4B ---------------------------------------------------------------------------------
def oracle_greedy(om, prompt, n_steps):
    ids = None
    for i, t in enumerate(prompt):
        ids = om.decode_token(t, i)
    out = [ids]
    pos = len(prompt)
    for _ in range(n_steps - 1):
        out.append(om.decode_token(out[-1], pos))
        pos += 1
    return out


def test_e4b_full_per_layer_hidden(gpu, fast_oracle):
    ms = gpu
    arch = ms.arch_e4b(max_full_seq=512)
    say("E4B 42 layers: per-layer hidden states for 3 positions (embedding rows)")
    m = build(ms, arch, max_seqs=1, max_rows=1, max_pos=512)
    om = synthetic_oracle_model(fast_oracle, arch, SEED)
    for pos, tok in enumerate([5, 262143, 100000]):
        x = fast_oracle.embed(om.lm_w, 2560, arch.vocab, om.lm_scale, tok)[None, :]
        g_out, g_hid = m.forward(x, [pos], T=1, hidden=True)
        o_out, o_hid = om.forward(x, pos, hidden=True)
        errs = [rel_rmse(g_hid[l], o_hid[l]) for l in range(42)]
        print(f"  pos {pos}: max per-layer rel RMSE {max(errs):.2e}")
        assert max(errs) < 1e-4
    m.close()


def test_e4b_full_greedy_ids(gpu, fast_oracle):
    ms = gpu
    arch = ms.arch_e4b(max_full_seq=512)
    n_steps = int(os.environ.get("MS_GREEDY_STEPS", "100"))
    say(f"E4B 42 layers + vocab 262144: prefill 6 + greedy {n_steps} steps")
    m = build(ms, arch, max_seqs=1, max_rows=16, max_pos=512)
    om = synthetic_oracle_model(fast_oracle, arch, SEED)
    prompt = prompt_ids(6, arch.vocab, 1)
    first = m.prefill(prompt, 0)
    rest = m.decode([first], [len(prompt)], n_steps - 1)
    gpu_ids = [first] + [int(v) for v in rest[:, 0]]
    ref_ids = oracle_greedy(om, prompt, n_steps)
    print(f"  gpu {gpu_ids[:12]}...\n  ref {ref_ids[:12]}...")
    assert gpu_ids == ref_ids
    m.close()


@pytest.mark.parametrize("n_prompt", [100, 600, 2100])
def test_e4b_prefill_gemm_vs_oracle(gpu, fast_oracle, n_prompt):
    """Prompts longer than 16 rows run their projections as MFMA GEMMs and their
    attention as flash attention over the chunk; 600 rows wrap the 512-slot
    sliding window inside one chunk, 2100 rows also cross the 2048-row chunk.
    Prefill + 7 decode steps must give the oracle's greedy ids."""
    ms = gpu
    max_pos = 2400 if n_prompt > 1000 else 1024
    arch = ms.arch_e4b(max_full_seq=max_pos, n_layers=6, vocab=4096)
    say(f"E4B shapes, 6 layers, vocab 4096: GEMM prefill of {n_prompt} tokens + 7 steps")
    m = build(ms, arch, max_seqs=1, max_rows=4, max_pos=max_pos)
    om = synthetic_oracle_model(fast_oracle, arch, SEED)
    prompt = prompt_ids(n_prompt, arch.vocab, 3)
    first = m.prefill(prompt, 0)
    rest = m.decode([first], [n_prompt], 7)
    got = [first] + [int(v) for v in rest[:, 0]]
    ref = oracle_greedy(om, prompt, 8)
    print(f"  gpu {got}\n  ref {ref}")
    assert got == ref
    m.close()


def test_e4b_small_batch4_vs_single(gpu, fast_oracle):
    ms = gpu
    arch = ms.arch_e4b(max_full_seq=256, n_layers=6, vocab=16384)
    say("E4B 6 layers (1 full), vocab 16384: batch 4 independent sequences")
    m = build(ms, arch, max_seqs=4, max_rows=4, max_pos=256)
    lens = [3, 5, 7, 4]
    prompts = [prompt_ids(n, arch.vocab, 10 + i) for i, n in enumerate(lens)]
    firsts = []
    for s, p in enumerate(prompts):
        from ctypes import byref, c_int32
        t = np.asarray(p, np.int32)
        first = c_int32()
        ms.check(ms.lib().ms_prefill(m.h, s, t.ctypes.data, len(t), 0, byref(first)))
        firsts.append(int(first.value))
    steps = 10
    ids = m.decode(firsts, lens, steps - 1)
    for s, p in enumerate(prompts):
        om = synthetic_oracle_model(fast_oracle, arch, SEED)
        ref = oracle_greedy(om, p, steps)
        got = [firsts[s]] + [int(v) for v in ids[:, s]]
        assert got == ref, (s, got, ref)
    m.close()


def test_step_rows_bit_identical_to_single_rows(gpu):
    """The rows of a decode step are independent: a row of a 2-4 row step,
    whose GEMV prologues normalize and quantize the rows side by side (one wave
    group per row), must equal the same row run alone, bit for bit, in every
    layer's output.  The four sequences' caches are primed with the same 20-token
    prompt, so a row's result depends only on its input and position."""
    ms = gpu
    arch = ms.arch_e4b(max_full_seq=256, n_layers=6, vocab=4096)
    say("E4B 6 layers (1 full): rows of 2-4 row steps against single rows")
    m = build(ms, arch, max_seqs=4, max_rows=4, max_pos=256)
    D, P = arch.hidden, 20
    prompt = prompt_ids(P, arch.vocab, 77)
    for s in range(4):
        m.prefill(prompt, 0, seq=s)
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((4, D)) * rng.uniform(0.1, 10, (4, 1))).astype(np.float32)
    for B in (4, 3, 2):
        out, hid = m.forward(x[:B], [P] * B, T=1, hidden=True)
        for i in range(B):
            o1, h1 = m.forward(x[i:i + 1], [P], T=1, hidden=True)
            assert np.array_equal(h1[:, 0], hid[:, i]), (B, i)
            assert np.array_equal(o1[0], out[i]), (B, i)
    m.close()


def oracle_sampled(om, oracle, prompt, n_steps, temperature, penalty, seed):
    """gemma4_e4b_infer.mojo:134-182 with the oracle: the prompt ids open the
    penalty history, every drawn id joins it, draw k of sequence 0 uses
    sample_seed(seed, 0, k)."""
    import mojostream_amd as ms
    hist = list(prompt)
    h = None
    for i, t in enumerate(prompt):
        _, h = om.decode_token(t, i, hidden=True)
    out = []
    pos = len(prompt)
    for k in range(n_steps):
        if k:
            _, h = om.decode_token(out[-1], pos, hidden=True)
            pos += 1
        tid, _ = oracle.sample(om.logits_for(h[-1]), temperature, hist, penalty,
                               ms.sample_seed(seed, 0, k))
        out.append(tid)
        hist.append(tid)
    return out


def test_e4b_small_sampled_decode_vs_oracle(gpu, fast_oracle):
    """Sampling in prefill and decode (graph and eager) against the oracle's
    temperature_sampling on its own logits; a low temperature keeps every draw
    far from the rounding of the cumulative sums."""
    ms = gpu
    arch = ms.arch_e4b(max_full_seq=256, n_layers=6, vocab=16384)
    say("E4B 6 layers, vocab 16384: sampled decode T=0.05, penalty 1.5")
    om = synthetic_oracle_model(fast_oracle, arch, SEED)
    prompt = prompt_ids(5, arch.vocab, 30)
    steps = 12
    ref = oracle_sampled(om, fast_oracle, prompt, steps, 0.05, 1.5, 1234)
    for graph in (True, False):
        m = build(ms, arch, max_seqs=1, max_rows=8, max_pos=256)
        m.set_sampling(0.05, 1.5, 1234)
        first = m.prefill(prompt, 0)
        ids = m.decode([first], [len(prompt)], steps - 1, use_graph=graph)
        got = [first] + [int(v) for v in ids[:, 0]]
        print(f"  graph={graph}: {got}")
        assert got == ref
        # greedy again after switching sampling off
        m.reset()
        m.set_sampling(0.0, 1.0, 0)
        first = m.prefill(prompt, 0)
        gids = [first] + [int(v) for v in m.decode([first], [len(prompt)], 3)[:, 0]]
        assert gids == oracle_greedy(synthetic_oracle_model(fast_oracle, arch, SEED), prompt, 4)
        m.close()


def test_e4b_small_sampled_decode_two_sequences(gpu, fast_oracle):
    """Two sequences with the same prompt sampled together: each draws with
    its own seeds sample_seed(seed, b, k) and matches the oracle's run for that
    sequence."""
    import ctypes as C
    ms = gpu
    arch = ms.arch_e4b(max_full_seq=256, n_layers=6, vocab=16384)
    say("E4B 6 layers, vocab 16384: two sequences sampled together, T=0.05, penalty 1.5")
    prompt = prompt_ids(5, arch.vocab, 31)
    steps = 10
    m = build(ms, arch, max_seqs=2, max_rows=8, max_pos=256)
    m.set_sampling(0.05, 1.5, 99)
    t = np.asarray(prompt, np.int32)
    firsts = []
    for b in range(2):
        f = C.c_int32()
        ms.check(ms.lib().ms_prefill(m.h, b, t.ctypes.data, len(t), 0, C.byref(f)))
        firsts.append(int(f.value))
    ids = m.decode(firsts, [len(prompt)] * 2, steps - 1)
    m.close()
    for b in range(2):
        got = [firsts[b]] + [int(v) for v in ids[:, b]]
        om = synthetic_oracle_model(fast_oracle, arch, SEED)
        # the draw counter counts LM head calls: both prefills, then the steps
        hist = list(prompt)
        _, h = None, None
        for i, tok in enumerate(prompt):
            _, h = om.decode_token(tok, i, hidden=True)
        ref = []
        for k in range(steps):
            if k:
                _, h = om.decode_token(ref[-1], len(prompt) + k - 1, hidden=True)
            draw = b if k == 0 else k + 1
            tid, _ = fast_oracle.sample(om.logits_for(h[-1]), 0.05, hist, 1.5,
                                        ms.sample_seed(99, b, draw))
            ref.append(tid)
            hist.append(tid)
        print(f"  seq {b}: {got}")
        assert got == ref, (b, got, ref)


def test_e4b_small_fp32_head_file_greedy(gpu, fast_oracle, tmp_path):
    """LM head file version 2 (FP32 weights + final-norm gamma + BOS,
    load_lm_head lm_head.mojo:61-116): column embeddings, the final norm with
    gamma, matmul_fp32_raw logits and the greedy pick, against the oracle's
    layers with the same head."""
    ms = gpu
    arch = ms.arch_e4b(max_full_seq=256, n_layers=6, vocab=16384)
    say("E4B 6 layers, FP32 head file (version 2), greedy")
    path = str(tmp_path / "lm_head_v2.bin")
    ms.check(ms.lib().ms_lm_head_file_write_synthetic_v2(os.fsencode(path), arch.hidden,
                                                          arch.vocab, 77))
    raw = np.fromfile(path, np.uint8)
    D, V = arch.hidden, arch.vocab
    f = raw[12:].view(np.float32)
    bos, gamma, W = f[:D], f[D:2 * D], f[2 * D:].reshape(D, V)
    m = build(ms, arch, max_seqs=1, max_rows=8, max_pos=256)
    m.load_lm_head_file(path)
    prompt = prompt_ids(5, V, 40)
    steps = 6
    first = m.prefill(prompt, 0)
    got = [first] + [int(v) for v in m.decode([first], [len(prompt)], steps - 1)[:, 0]]
    om = synthetic_oracle_model(fast_oracle, arch, SEED, with_lm=False)

    def pick(x_last):
        y = fast_oracle.rmsnorm(x_last.reshape(1, -1), gamma)
        return fast_oracle.argmax(fast_oracle.matmul_f32(y, W)[0])

    x = np.ascontiguousarray(W[:, prompt].T)
    x[0] = bos  # prompt position 0 takes the BOS row
    ref = [pick(om.forward(x, 0)[-1])]
    pos = len(prompt)
    for _ in range(steps - 1):
        ref.append(pick(om.forward(np.ascontiguousarray(W[:, [ref[-1]]].T), pos)[-1]))
        pos += 1
    print(f"  device {got}\n  oracle {ref}")
    assert got == ref
    m.close()


def test_e4b_small_graph_replays_match_eager(gpu, fast_oracle):
    ms = gpu
    arch = ms.arch_e4b(max_full_seq=256, n_layers=6, vocab=16384)
    say("graph replays with eager work in between vs eager decode")
    a = build(ms, arch, max_seqs=1, max_rows=1, max_pos=256)
    b = build(ms, arch, max_seqs=1, max_rows=1, max_pos=256)
    ga = [a.decode([7], [0], 4, use_graph=True)]
    for _ in range(3):
        # unrelated eager kernels between replays
        scratch = ms.DeviceBuffer(4096)
        ms.check(ms.lib().ms_memset(scratch.ptr, 1, 4096))
        ms.synchronize()
        ga.append(a.decode_continue(4, 1, use_graph=True))
    gids = np.concatenate(ga)[:, 0].tolist()
    eids = b.decode([7], [0], 16, use_graph=False)[:, 0].tolist()
    om = synthetic_oracle_model(fast_oracle, arch, SEED)
    ref = [om.decode_token(7, 0)]
    for p in range(1, 16):
        ref.append(om.decode_token(ref[-1], p))
    assert gids == eids == ref
    a.close()
    b.close()


def test_graph_position_bounds_match_eager(gpu):
    """A captured decode step serves positions below its bound (64-position
    buckets) and launches only the attention chunks below it; decoding across
    several buckets in graph mode, in runs of uneven length, gives the same
    ids as eager steps with exact bounds.  Balanced weights and a repetition
    penalty keep the ids input-dependent, so a dropped or extra key shows."""
    ms = gpu
    arch = ms.arch_e4b(max_full_seq=256, n_layers=6, vocab=16384)
    say("graph decode across position-bound buckets vs eager, batch 2")
    ids = {}
    for mode in ("graph", "eager"):
        m = ms.Model(arch, max_seqs=2, max_rows=1, max_pos=256)
        m.fill_synthetic(SEED, balanced=True)
        m.set_sampling(0.0, 1.2)
        g = mode == "graph"
        runs = [m.decode([7, 11], [3, 50], 30, use_graph=g)]
        for n in (41, 7, 60):  # the second sequence reaches position 187
            runs.append(m.decode_continue(n, 2, use_graph=g))
        ids[mode] = np.concatenate(runs)
        m.close()
    print(f"  distinct ids {len(set(ids['graph'][:, 0].tolist()))}, "
          f"{len(set(ids['graph'][:, 1].tolist()))}")
    assert len(set(ids["graph"][:, 1].tolist())) >= 5
    assert np.array_equal(ids["graph"], ids["eager"])


def test_streaming_equals_resident(gpu):
    ms = gpu
    arch = ms.arch_demo(max_len=64, n_layers=8)
    say("streaming (pinned host -> 2 HBM slots) vs resident, demo 8 layers")
    r = build(ms, arch, max_seqs=1, max_rows=4, max_pos=64)
    s = ms.Model(arch, max_seqs=1, max_rows=4, max_pos=64, resident=False)
    s.fill_synthetic_host(SEED)
    for step in range(3):
        x = ms.host_normal(4 * 1024, 500 + step, 3).reshape(4, 1024)
        a = r.forward(x, [4 * step], T=4)
        b = s.forward(x, [4 * step], T=4)
        assert np.array_equal(a, b)
    st = s.stream_stats()
    print(f"  stream stats {st}")
    assert st["io_ms"] > 0 and st["total_ms"] > 0
    r.close()
    s.close()


def test_model_guards(gpu):
    ms = gpu
    arch = ms.arch_demo(max_len=16, n_layers=2)
    say("model guards: positions past a linear cache, bad scale, unset matrices")
    m = ms.Model(arch, max_seqs=1, max_rows=4, max_pos=64)
    x = np.zeros((4, 1024), np.float32)
    with pytest.raises(ms.MSError, match="unset"):
        m.forward(x, [0], T=4)
    m.fill_synthetic(SEED)
    with pytest.raises(ms.MSError, match="linear KV cache"):
        m.forward(x, [14], T=4)
    with pytest.raises(ms.MSError, match="scale"):
        m.set_matrix(0, 0, np.zeros((1024, 512), np.uint8), 0.0)
    m.close()


def test_sampling_history_limit(gpu):
    """The repetition-penalty history holds 8192 ids per sequence (prompt, the
    first draw, one per step): a prompt of 8191 ids fills it exactly, 8192 is
    refused; a decode_run that would cross the limit is refused before it runs,
    one that ends exactly at it runs, and the model's host mirror of the count
    follows (reset empties it)."""
    ms = gpu
    arch = ms.arch_e4b(max_full_seq=64, n_layers=1, vocab=4096)
    say("sampling history limit: 1 sliding layer, vocab 4096, prompts of 8191/8192 ids")
    m = ms.Model(arch, max_seqs=1, max_rows=16, max_pos=8400)
    m.fill_synthetic(SEED)
    m.set_sampling(0.7, 1.2, 3)
    ids = prompt_ids(8192, arch.vocab, 60)
    with pytest.raises(ms.MSError, match="8192"):
        m.prefill(ids, 0)
    first = m.prefill(ids[:8191], 0)                     # 8191 + the first draw
    with pytest.raises(ms.MSError, match="8192"):
        m.decode([first], [8191], 1)
    m.reset()
    first = m.prefill(ids[:8000], 0)                     # 8001 ids
    with pytest.raises(ms.MSError, match="8192"):
        m.decode([first], [8000], 192)                   # would reach 8193
    out = m.decode([first], [8000], 191)                 # ends at 8192 exactly
    assert out.shape == (191, 1) and np.all((out >= 0) & (out < arch.vocab))
    with pytest.raises(ms.MSError, match="8192"):
        m.decode_continue(1, 1)
    m.reset()                                            # history emptied
    first = m.prefill(ids[:100], 0)
    assert m.decode([first], [100], 4).shape == (4, 1)
    m.close()


def test_sampled_draw_seeds_per_sequence(gpu, fast_oracle):
    """Two sequences with the same prompt, sampled: every draw of the model
    equals ms_sample on that step's logits with the seed sample_seed(seed, b, k)
    (k counts the drawing LM head calls), and sequence 1's draws are no copy of
    sequence 0's shifted by one draw (the lag a seed of seed + b + k would
    give).  The tied head of a random model puts a token's own id far ahead
    (at temperature 1 every draw is that id), so the draws run at temperature
    50, where the distribution is broad and the draws tell the seeds apart."""
    import ctypes as C
    ms = gpu
    arch = ms.arch_e4b(max_full_seq=256, n_layers=2, vocab=16384)
    say("sampled draw seeds per sequence: T=50, two sequences, identical prompts")
    m = ms.Model(arch, max_seqs=2, max_rows=8, max_pos=256)
    m.fill_synthetic(SEED, balanced=True)
    TEMP = 50.0
    m.set_sampling(TEMP, 1.0, 77)
    V = arch.vocab
    tl = ms.DeviceBuffer(2 * V * 4)
    m.set_taps(None, tl)
    prompt = np.asarray(prompt_ids(6, V, 70), np.int32)
    firsts, pre_logits = [], []
    for b in range(2):
        f = C.c_int32()
        ms.check(ms.lib().ms_prefill(m.h, b, prompt.ctypes.data, len(prompt), 0, C.byref(f)))
        firsts.append(int(f.value))
        pre_logits.append(tl.download(np.float32, (V,)))
    assert np.array_equal(pre_logits[0], pre_logits[1])   # identical rows
    dummy = ms.DeviceBuffer(64)

    def draw(row, seed):
        d = ms.DeviceBuffer.from_array(np.ascontiguousarray(row))
        return ms.sample(d, V, TEMP, dummy, 0, 1.0, seed)

    for b in range(2):
        assert draw(pre_logits[b], ms.sample_seed(77, b, b)) == firsts[b]
    steps = 24
    ids = np.empty((steps, 2), np.int32)
    for k in range(steps):
        out = m.decode(firsts, [len(prompt)] * 2, 1) if k == 0 else m.decode_continue(1, 2)
        ids[k] = out[0]
        lg = tl.download(np.float32, (2, V))
        for b in range(2):
            assert draw(lg[b], ms.sample_seed(77, b, k + 2)) == ids[k, b], (k, b)
    seq0 = [firsts[0]] + ids[:, 0].tolist()
    seq1 = [firsts[1]] + ids[:, 1].tolist()
    print(f"  seq 0 {seq0[:10]}...\n  seq 1 {seq1[:10]}...")
    assert len(set(seq0)) > steps // 2 and len(set(seq1)) > steps // 2
    assert seq0 != seq1
    assert sum(a == b for a, b in zip(seq1[:-1], seq0[1:])) < steps // 2
    m.close()


def test_forward_graph_replays_equal_eager(gpu):
    """ms_forward replays a captured HIP graph once a call repeats the previous
    one's buffers, rows and position bucket (the harness loop).  The replays
    must equal eager launches bit for bit: four rows a step (the harness), and
    one row a step, both across a 64-position bucket edge (the attention's
    key-chunk bound is part of the graph)."""
    import ctypes as C
    ms = gpu
    arch = ms.arch_demo(max_len=512, n_layers=6)
    say("forward graph replays vs eager: demo 6 layers, T=4 and T=1 steps")
    a = build(ms, arch, max_seqs=1, max_rows=4, max_pos=512)
    b = build(ms, arch, max_seqs=1, max_rows=4, max_pos=512)
    b.set_forward_graphs(False)
    for T, positions in ((4, list(range(40, 100, 4))), (1, list(range(100, 108)) + [120, 127, 128, 129])):
        da, db = ms.DeviceBuffer(T * 1024 * 4), ms.DeviceBuffer(T * 1024 * 4)
        ha, hb = ms.DeviceBuffer(6 * T * 1024 * 4), ms.DeviceBuffer(6 * T * 1024 * 4)
        for s, p in enumerate(positions):
            x = ms.host_normal(T * 1024, 900 + s, T).reshape(T, 1024)
            base = (C.c_int * 1)(p)
            da.upload(x)
            db.upload(x)
            ms.check(ms.lib().ms_forward(a.h, da.ptr, 1, T, base, ha.ptr))
            ms.check(ms.lib().ms_forward(b.h, db.ptr, 1, T, base, hb.ptr))
            assert np.array_equal(da.download(np.float32, (T, 1024)),
                                  db.download(np.float32, (T, 1024))), (T, p)
            assert np.array_equal(ha.download(np.float32, (6, T, 1024)),
                                  hb.download(np.float32, (6, T, 1024))), (T, p)
    a.close()
    b.close()
