"""Pins the CPU oracle against closed forms, f64 brute force, invariants and an
independently written f64 layer (tests/golden/layer_ref.py).  CPU only.

Each check is chosen so that a plausible mistake in the oracle (wrong nibble
order, dropped term, wrong sign or index, transposed operand, wrong window or
GQA mapping) fails it.
"""
import numpy as np
import pytest

from oracle.binding import (OR_CACHE_CIRCULAR, OR_CACHE_LINEAR, OR_MODE_CAUSAL,
                            OR_MODE_WRITE_FIRST, OracleModel)
from tests.golden.layer_ref import RefLayer, deq, lm_logits, rms

RNG = np.random.default_rng(20261201)


def rel_rmse(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.sqrt(np.mean((a - b) ** 2)) / (np.sqrt(np.mean(b ** 2)) + 1e-30))


# ---- a1: dequant ------------------------------------------------------------------
@pytest.mark.parametrize("scale", [0.1, 0.04, 0.15, 1e-8, 3.7, 0.0731])
def test_dequant_exhaustive_bytes(oracle, scale):
    q4 = np.arange(256, dtype=np.uint8).reshape(2, 128)  # every byte value
    out = oracle.dequant(q4, 2, 256, scale)
    b = q4.reshape(-1)
    lo = ((b & 15).astype(np.int32) - 8).astype(np.float32) * np.float32(scale)
    hi = ((b >> 4).astype(np.int32) - 8).astype(np.float32) * np.float32(scale)
    exp = np.empty(512, np.float32)
    exp[0::2], exp[1::2] = lo, hi  # low nibble -> even column (kernels.mojo:66-69)
    assert np.array_equal(out.reshape(-1).view(np.uint32), exp.view(np.uint32))


def test_dequant_roundtrips_quantizer(oracle):
    # quantize as convert.py:296-323 does (round, clip, +8, lo=even col)
    K, N = 64, 96
    s = np.float32(0.05)
    q = RNG.integers(-8, 8, size=(K, N))
    u = (q + 8).astype(np.uint8)
    packed = (u[:, 0::2] & 15) | ((u[:, 1::2] & 15) << 4)
    out = oracle.dequant(packed.astype(np.uint8), K, N, float(s))
    assert np.array_equal(out, q.astype(np.float32) * s)


# ---- a3: matmul ---------------------------------------------------------------------
@pytest.mark.parametrize("M,K,N", [(1, 128, 32), (4, 256, 64), (5, 384, 48), (3, 200, 24),
                                   (8, 1024, 256)])
def test_matmul_vs_f64(oracle, M, K, N):
    A = RNG.standard_normal((M, K)).astype(np.float32)
    q4 = RNG.integers(0, 256, size=(K, N // 2), dtype=np.uint8)
    c = oracle.matmul(A, q4, N, 0.1)
    ref = oracle.matmul_f64(A, q4, N, 0.1)
    indep = A.astype(np.float64) @ deq(q4, 0.1)
    assert rel_rmse(ref, indep) < 1e-12  # the two f64 paths agree
    assert np.max(np.abs(c - ref)) / np.max(np.abs(ref)) < 1e-5


def test_matmul_identity_rows_exact(oracle):
    K, N = 256, 64
    q4 = RNG.integers(0, 256, size=(K, N // 2), dtype=np.uint8)
    A = np.eye(K, dtype=np.float32)[:8]
    c = oracle.matmul(A, q4, N, 0.0731)
    assert np.array_equal(c, oracle.dequant(q4, K, N, 0.0731)[:8])


def test_matmul_accumulates_and_is_linear(oracle):
    M, K, N = 4, 256, 32
    A = RNG.standard_normal((M, K)).astype(np.float32)
    q4 = RNG.integers(0, 256, size=(K, N // 2), dtype=np.uint8)
    c1 = oracle.matmul(A, q4, N, 0.1)
    c2 = oracle.matmul(2 * A, q4, N, 0.1)
    assert np.array_equal(c2, 2 * c1)  # power-of-two scaling is exact
    C0 = RNG.standard_normal((M, N)).astype(np.float32)
    acc = oracle.matmul(A, q4, N, 0.1, C0=C0)
    assert np.allclose(acc, C0 + c1, rtol=1e-6, atol=1e-5)


# ---- a5 / a6 / a8: norms, PLE, SwiGLU ---------------------------------------------------
def test_rmsnorm_properties(oracle):
    x = (RNG.standard_normal((3, 1024)) * 37.0).astype(np.float32)
    y = oracle.rmsnorm(x)
    assert np.allclose(np.sqrt(np.mean(y.astype(np.float64) ** 2, axis=1)), 1.0, atol=1e-6)
    assert rel_rmse(y, rms(x.astype(np.float64))) < 1e-6
    y2 = oracle.rmsnorm(x * np.float32(8.0))  # scale invariance
    assert rel_rmse(y2, y) < 1e-6
    g = RNG.uniform(0.5, 1.5, 1024).astype(np.float32)
    yw = oracle.rmsnorm(x, g)
    assert rel_rmse(yw, y * g) < 1e-6


def test_ple_and_swiglu(oracle):
    x = RNG.standard_normal(64).astype(np.float32)
    assert np.array_equal(oracle.ple_scale(x, 0.5), x * np.float32(0.5))
    g = np.array([0.0, 50.0, -50.0, 1.0, -1.0, 3.0, 0.25, -2.0, 7.0, 0.5], np.float32)
    u = np.array([2.0, 3.0, 4.0, 1.0, 1.0, -2.0, 8.0, 1.5, 1.0, -1.0], np.float32)
    out = oracle.swiglu(g, u)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    exp = u64 * g64 / (1 + np.exp(-g64))
    assert out[0] == 0.0
    assert abs(out[1] - 150.0) < 1e-3 and abs(out[2]) < 1e-15
    assert np.allclose(out, exp, rtol=1e-6, atol=1e-12)


# ---- a7: RoPE ---------------------------------------------------------------------------
def test_rope_identity_at_pos0_and_partial(oracle):
    x = RNG.standard_normal(8 * 512).astype(np.float32)
    y = oracle.rope(x, 8, 512, 512, 0, 1e4)
    assert np.array_equal(y, x)
    # partial: only the first 128 dims of each 512-dim head rotate
    y = oracle.rope(x, 8, 512, 128, 77, 1e6).reshape(8, 512)
    assert np.array_equal(y[:, 128:], x.reshape(8, 512)[:, 128:])
    assert not np.array_equal(y[:, :128], x.reshape(8, 512)[:, :128])


def test_rope_norm_composition_and_closed_form(oracle):
    hd = 128
    x = RNG.standard_normal(hd).astype(np.float32)
    y = oracle.rope(x, 1, hd, hd, 9, 1e4)
    half = hd // 2
    n0 = x[:half].astype(np.float64) ** 2 + x[half:].astype(np.float64) ** 2
    n1 = y[:half].astype(np.float64) ** 2 + y[half:].astype(np.float64) ** 2
    assert np.allclose(n0, n1, rtol=1e-5)
    z = oracle.rope(oracle.rope(x, 1, hd, hd, 5, 1e4), 1, hd, hd, 4, 1e4)
    assert rel_rmse(z, y) < 1e-5  # R(5) R(4) = R(9)
    i = np.arange(half)
    ang = 9 * np.exp(-(2.0 * i / hd) * np.log(1e4))
    x64 = x.astype(np.float64)
    exp = np.concatenate([x64[:half] * np.cos(ang) - x64[half:] * np.sin(ang),
                          x64[:half] * np.sin(ang) + x64[half:] * np.cos(ang)])
    assert rel_rmse(y, exp) < 1e-6


# ---- a10 / a11: attention -------------------------------------------------------------
class _Desc:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def _layer(o, desc, D=128, F=256, seed=0):
    rng = np.random.default_rng(seed)
    shapes = [(D, desc.q_dim), (D, desc.kv_dim), (D, desc.kv_dim), (desc.q_dim, D), (D, F),
              (D, F), (F, D)]
    ws = [rng.integers(0, 256, size=(k, n // 2), dtype=np.uint8) for k, n in shapes]
    sc = [float(np.float32(rng.uniform(0.04, 0.15))) for _ in range(7)]
    ple = float(np.float32(rng.uniform(0.8, 1.2)))

    class A:
        hidden, ffn, vocab = D, F, 0
        layers = [desc]
        n_layers = 1
    om = OracleModel(o, A, [ws], [sc], [ple])
    ref = RefLayer(desc, D, F, ws, sc, ple)
    return om, ref


def test_attention_single_key_returns_v(oracle):
    import ctypes as C
    d = _Desc(q_dim=128, kv_dim=64, head_dim=32, n_heads=4, n_kv_heads=2, rot_dim=32,
              theta=1e4, cache_kind=OR_CACHE_LINEAR, cache_len=8, clamp_reads=0)
    om, _ = _layer(oracle, d)
    q = RNG.standard_normal((1, 128)).astype(np.float32)
    k = RNG.standard_normal((1, 64)).astype(np.float32)
    v = RNG.standard_normal((1, 64)).astype(np.float32)
    out = np.empty((1, 128), np.float32)
    oracle.lib.or_attention(C.byref(om.layers[0]), q.ctypes.data, k.ctypes.data,
                            v.ctypes.data, 1, 0, OR_MODE_CAUSAL, out.ctypes.data)
    # GQA: q heads 0,1 -> kv head 0; 2,3 -> kv head 1 (gemma4_e4b.mojo:289)
    exp = np.concatenate([v[0, :32], v[0, :32], v[0, 32:], v[0, 32:]])
    assert np.array_equal(out[0], exp)


def test_attention_uniform_scores_give_mean(oracle):
    import ctypes as C
    d = _Desc(q_dim=64, kv_dim=32, head_dim=32, n_heads=2, n_kv_heads=1, rot_dim=32,
              theta=1e4, cache_kind=OR_CACHE_LINEAR, cache_len=16, clamp_reads=0)
    om, _ = _layer(oracle, d)
    kc, vc = om.caches[0]
    kc[:] = 0.25
    vc[:] = RNG.standard_normal(vc.shape).astype(np.float32)
    q = RNG.standard_normal((1, 64)).astype(np.float32)
    knew = np.full((1, 32), 0.25, np.float32)
    vnew = RNG.standard_normal((1, 32)).astype(np.float32)
    out = np.empty((1, 64), np.float32)
    oracle.lib.or_attention(C.byref(om.layers[0]), q.ctypes.data, knew.ctypes.data,
                            vnew.ctypes.data, 1, 10, OR_MODE_CAUSAL, out.ctypes.data)
    mean = np.concatenate([vc[:10], vnew]).astype(np.float64).mean(axis=0)
    assert np.allclose(out[0, :32], mean, rtol=1e-5, atol=1e-6)
    assert np.allclose(out[0, 32:], mean, rtol=1e-5, atol=1e-6)


def _run_both(oracle, desc, steps, T, D=128, F=256, mode=OR_MODE_CAUSAL, seed=1):
    om, ref = _layer(oracle, desc, D, F, seed)
    rng = np.random.default_rng(seed + 100)
    worst = 0.0
    base = 0
    for _ in range(steps):
        x = rng.standard_normal((T, D)).astype(np.float32)
        a = om.layer_forward(0, x, base, mode)
        b = ref.forward(x, base)
        worst = max(worst, rel_rmse(a, b))
        base += T
    return worst


@pytest.mark.parametrize("T", [1, 4])
def test_layer_demo_semantics_vs_f64(oracle, T):
    # demo: hd = D/n_heads, linear cache, theta 1e4, GQA 4:1
    d = _Desc(q_dim=128, kv_dim=32, head_dim=16, n_heads=8, n_kv_heads=2, rot_dim=16,
              theta=1e4, cache_kind=OR_CACHE_LINEAR, cache_len=64, clamp_reads=0)
    assert _run_both(oracle, d, 6, T) < 1e-5


@pytest.mark.parametrize("T", [1, 3])
def test_layer_sliding_window_wraps_vs_f64(oracle, T):
    # circular window 8: positions run to 30, so slots wrap several times
    d = _Desc(q_dim=128, kv_dim=64, head_dim=32, n_heads=4, n_kv_heads=2, rot_dim=32,
              theta=1e4, cache_kind=OR_CACHE_CIRCULAR, cache_len=8, clamp_reads=0)
    assert _run_both(oracle, d, 10, T) < 1e-5


def test_layer_full_partial_rope_and_clamp_vs_f64(oracle):
    # E4B full layer shape in miniature: partial rotary (rot < hd), theta 1e6,
    # cache truncated at 12 positions with clamped reads (gemma4_e4b.mojo:242,363)
    d = _Desc(q_dim=256, kv_dim=128, head_dim=64, n_heads=4, n_kv_heads=2, rot_dim=16,
              theta=1e6, cache_kind=OR_CACHE_LINEAR, cache_len=12, clamp_reads=1)
    assert _run_both(oracle, d, 8, 2) < 1e-5


def test_layer_gqa_5to1_vs_f64(oracle):
    d = _Desc(q_dim=160, kv_dim=32, head_dim=16, n_heads=10, n_kv_heads=2, rot_dim=16,
              theta=1e6, cache_kind=OR_CACHE_LINEAR, cache_len=32, clamp_reads=0)
    assert _run_both(oracle, d, 5, 1, D=128) < 1e-5


def test_write_first_order_matches_causal_until_wrap(oracle):
    # The reference writes all rows before attending (gemma4_e4b.mojo:507-515).
    # Without a circular-slot collision both orders give the same result; with
    # T > 1 rows past the window they differ (rows overwrite keys an earlier
    # row still needs), which is why the GPU path uses the causal order.
    d = _Desc(q_dim=128, kv_dim=64, head_dim=32, n_heads=4, n_kv_heads=2, rot_dim=32,
              theta=1e4, cache_kind=OR_CACHE_CIRCULAR, cache_len=8, clamp_reads=0)
    om1, _ = _layer(oracle, d, seed=5)
    om2, _ = _layer(oracle, d, seed=5)
    rng = np.random.default_rng(9)
    diffs = []
    for step in range(6):
        x = rng.standard_normal((2, 128)).astype(np.float32)
        a = om1.layer_forward(0, x, 2 * step, OR_MODE_CAUSAL)
        b = om2.layer_forward(0, x, 2 * step, OR_MODE_WRITE_FIRST)
        diffs.append(float(np.max(np.abs(a - b))))
    assert diffs[0] == 0.0 and diffs[1] == 0.0 and diffs[2] == 0.0  # positions < 7
    assert max(diffs[4:]) > 0.0  # positions 8.. wrap: the orders diverge


# ---- a13: LM head, greedy, embedding -------------------------------------------------------
def test_argmax_first_index_on_ties(oracle):
    v = np.array([1.0, 3.0, -2.0, 3.0, 3.0], np.float32)
    assert oracle.argmax(v) == 1
    assert oracle.argmax(np.array([-1.0, -1.0], np.float32)) == 0


def test_embed_is_dequantized_column(oracle):
    D, V = 64, 96
    w = RNG.integers(0, 256, size=(D, V // 2), dtype=np.uint8)
    W = oracle.dequant(w, D, V, 0.07)
    for tok in (0, 1, 2, 57, 95):
        assert np.array_equal(oracle.embed(w, D, V, 0.07, tok), W[:, tok])


def test_lm_head_vs_f64(oracle):
    D, V = 128, 512
    w = RNG.integers(0, 256, size=(D, V // 2), dtype=np.uint8)
    x = RNG.standard_normal((2, D)).astype(np.float32)
    g = RNG.uniform(0.5, 1.5, D).astype(np.float32)
    xn = oracle.rmsnorm(x, g)
    lg = oracle.lm_head(xn, w, V, 0.09)
    ref = lm_logits(x, w, 0.09, g.astype(np.float64))
    assert rel_rmse(lg, ref) < 1e-5


# ---- sampler (temperature_sampling, lm_head.mojo:198-254) -----------------------------

def test_sample_penalty_closed_forms(oracle):
    """Penalty per occurrence: positive divided, non-positive multiplied, ids
    at or beyond the vocabulary ignored; greedy leaves the penalized logits."""
    v = np.array([2.0, -1.0, 0.0, 4.0, 3.0], np.float32)
    tid, out = oracle.sample(v, 0.0, [3, 3, 1, 2, 9, -1], 2.0, 0)
    np.testing.assert_array_equal(out, np.array([2.0, -2.0, 0.0, 1.0, 3.0], np.float32))
    assert tid == 4
    # penalty 1 (or below) leaves the logits alone
    tid, out = oracle.sample(v, 0.0, [3, 3], 1.0, 0)
    np.testing.assert_array_equal(out, v)
    assert tid == 3


def test_sample_greedy_is_argmax(oracle):
    rng = np.random.default_rng(3)
    for _ in range(20):
        v = rng.standard_normal(257).astype(np.float32)
        v[rng.integers(0, 257)] = v.max()  # a tie: the first index wins
        tid, _ = oracle.sample(v, 0.01, [], 1.0, 11)
        assert tid == oracle.argmax(v) == int(np.argmax(v))


def test_sample_targets_uniform(oracle):
    t = np.array([oracle.sample_target(s) for s in range(20000)])
    assert t.min() >= 0.0 and t.max() <= 1.0
    hist, _ = np.histogram(t, bins=10, range=(0.0, 1.0))
    assert np.all(np.abs(hist - 2000) < 5 * np.sqrt(2000))


def test_sample_frequencies_match_softmax(oracle):
    """Draw counts over many seeds against the f64 softmax at temperature T
    (chi-square, 3 degrees of freedom)."""
    v = np.array([0.5, 1.5, -0.3, 1.0], np.float32)
    T = 0.7
    p = np.exp((v.astype(np.float64) - v.max()) / T)
    p /= p.sum()
    n = 20000
    counts = np.bincount([oracle.sample(v, T, [], 1.0, s)[0] for s in range(n)], minlength=4)
    chi2 = float(np.sum((counts - n * p) ** 2 / (n * p)))
    assert chi2 < 16.3  # p = 0.001 for 3 degrees of freedom
    # the probabilities are left in the logits, summing to one
    _, out = oracle.sample(v, T, [], 1.0, 0)
    np.testing.assert_allclose(out, p, rtol=1e-6)


# ---- FP32 head projection (matmul_fp32_raw, kernels.mojo:616-671) -------------------

def test_matmul_f32_vs_f64_and_tail(oracle):
    rng = np.random.default_rng(5)
    A = rng.standard_normal((4, 300)).astype(np.float32)
    B = rng.standard_normal((300, 40)).astype(np.float32)
    C0 = rng.standard_normal((4, 40)).astype(np.float32)
    out = oracle.matmul_f32(A, B, C0)
    ref = C0.astype(np.float64) + A.astype(np.float64) @ B.astype(np.float64)
    # whole 16-column tiles: C0 + A.B; the partial last tile (columns 32..39) untouched
    np.testing.assert_allclose(out[:, :32], ref[:, :32], rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(out[:, 32:], C0[:, 32:])
    # one-hot rows of A select rows of B exactly
    E = np.zeros((3, 300), np.float32)
    E[0, 7] = E[1, 150] = E[2, 299] = 1.0
    np.testing.assert_array_equal(oracle.matmul_f32(E, B)[:, :32], B[[7, 150, 299], :32])


# ---- converter quantization (quantize_q4_blockwise, scripts/convert.py:296-323) ----

def test_q4_quantize_exact_grid_and_ties(oracle):
    """Weights q * 2^-5 with max |q| = 7 have scale 2^-5 and come back as q,
    transposed, even output columns in the low nibble.  Halves round to even."""
    rng = np.random.default_rng(11)
    n_out, n_in = 34, 5
    q = rng.integers(-7, 8, size=(n_out, n_in))
    q[3, 2] = 7
    w = (q * 2.0 ** -5).astype(np.float32)
    packed, s = oracle.q4_quantize(w)
    assert s == 2.0 ** -5
    qt = q.T + 8
    assert np.array_equal(packed, (qt[:, 0::2] | (qt[:, 1::2] << 4)).astype(np.uint8))
    # ties: 2.5 -> 2, 3.5 -> 4, -2.5 -> -2, -0.5 -> -0
    w2 = np.zeros((4, 1), np.float32)
    w2[:, 0] = np.array([2.5, 3.5, -2.5, 7.0]) * 2.0 ** -5
    p2, s2 = oracle.q4_quantize(w2)
    assert s2 == 2.0 ** -5
    assert list(p2[0]) == [(2 + 8) | ((4 + 8) << 4), (-2 + 8) | ((7 + 8) << 4)]


def test_q4_quantize_round_trip_through_dequant(oracle):
    """Random weights: scale float(max|w| / 7) and the pinned dequant returns
    every transposed weight to within half a scale step."""
    rng = np.random.default_rng(12)
    for n_out, n_in in ((64, 48), (130, 7), (2, 1)):
        w = (0.02 * rng.standard_normal((n_out, n_in))).astype(np.float32)
        packed, s = oracle.q4_quantize(w)
        assert s == np.float32(float(np.abs(w).max()) / 7.0)
        back = oracle.dequant(packed, n_in, n_out, s)
        err = np.abs(back.astype(np.float64) - w.T.astype(np.float64))
        assert err.max() <= 0.5 * s * (1 + 1e-6)
        assert np.all(np.abs(back) <= 8 * s)


def test_q4_quantize_tiny_block_rule(oracle):
    """A block whose max is not above 1e-8 contributes a scale of 1e-8
    (convert.py:311-314); it wins only when max|w| / 7 is below that."""
    w = np.zeros((64, 2), np.float32)
    w[5, 0] = 3e-8                       # column k=0 (first 64 flat values) holds it
    _, s = oracle.q4_quantize(w, 32)
    assert s == np.float32(1e-8)         # blocks of k=1 are all zero
    w[:, :] = 2e-8                        # every block above 1e-8
    w[5, 0] = 3e-8
    _, s = oracle.q4_quantize(w, 32)
    assert s == np.float32(float(np.float32(3e-8)) / 7.0)
    _, s = oracle.q4_quantize(np.zeros((4, 4), np.float32))
    assert s == np.float32(1e-8)


# ---- whole-model token step and the oracle's threading ------------------------------
def _small_model(o, n_layers=3, D=128, F=256, V=512, seed=5):
    """A 3-layer model mixing a circular window (6 slots), a linear cache with
    partial RoPE and GQA 2:1, and its tied Q4 head."""
    rng = np.random.default_rng(seed)
    descs = []
    for l in range(n_layers):
        if l % 2 == 0:
            descs.append(_Desc(q_dim=128, kv_dim=64, head_dim=32, n_heads=4, n_kv_heads=2,
                               rot_dim=32, theta=1e4, cache_kind=OR_CACHE_CIRCULAR,
                               cache_len=6, clamp_reads=0))
        else:
            descs.append(_Desc(q_dim=128, kv_dim=64, head_dim=32, n_heads=4, n_kv_heads=2,
                               rot_dim=8, theta=1e6, cache_kind=OR_CACHE_LINEAR,
                               cache_len=64, clamp_reads=1))
    ws, sc, ples = [], [], []
    for d in descs:
        shapes = [(D, d.q_dim), (D, d.kv_dim), (D, d.kv_dim), (d.q_dim, D), (D, F), (D, F),
                  (F, D)]
        ws.append([rng.integers(0, 256, size=(k, n // 2), dtype=np.uint8) for k, n in shapes])
        sc.append([float(np.float32(rng.uniform(0.04, 0.15))) for _ in range(7)])
        ples.append(float(np.float32(rng.uniform(0.8, 1.2))))
    lm = rng.integers(0, 256, size=(D, V // 2), dtype=np.uint8)
    lm_scale = float(np.float32(0.08))
    gamma = rng.uniform(0.5, 1.5, D).astype(np.float32)

    class A:
        hidden, ffn, vocab = D, F, V
        layers = descs
    A.n_layers = n_layers
    om = OracleModel(o, A, ws, sc, ples, lm, lm_scale, gamma)
    refs = [RefLayer(d, D, F, w, s, p) for d, w, s, p in zip(descs, ws, sc, ples)]
    return om, refs, lm, lm_scale, gamma


def test_decode_token_vs_f64_model(oracle):
    """or_decode_token (embedding column -> layers -> final norm with gamma ->
    logits -> first maximum) against the independent f64 layers and head, over
    10 positions so the 6-slot window wraps."""
    om, refs, lm, lm_scale, gamma = _small_model(oracle)
    D = om.D
    W = deq(lm, lm_scale)
    tok = 7
    for pos in range(10):
        tid, hid = om.decode_token(tok, pos, hidden=True)
        x = W[:, tok][None, :]
        for l, ref in enumerate(refs):
            x = ref.forward(x, pos)
            assert rel_rmse(hid[l], x[0]) < 1e-5, (pos, l)
        lg = lm_logits(x, lm, lm_scale, gamma.astype(np.float64))[0]
        order = np.argsort(lg)[::-1]
        # the f64 argmax, unless the top two are closer than fp32 rounding
        if lg[order[0]] - lg[order[1]] > 1e-4 * np.abs(lg).max():
            assert tid == int(order[0]), (pos, tid, int(order[0]))
        tok = tid


def test_threaded_oracle_is_bit_identical(oracle):
    """The oracle's thread split (columns of a matmul, rows of attention)
    keeps every element's summation order."""
    # one loaded library: the thread count is switched between the two runs
    try:
        outs = []
        for n in (1, 8):
            oracle.set_threads(n)
            om, _, _, _, _ = _small_model(oracle)
            x = np.random.default_rng(3).standard_normal((40, om.D)).astype(np.float32)
            y = om.forward(x[:24], 0)           # 24 rows: wraps the 6-slot window
            z = om.forward(x[24:], 24)
            outs.append((y, z))
        assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    finally:
        oracle.set_threads(1)
