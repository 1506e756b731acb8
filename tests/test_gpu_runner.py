"""ModelRunner (loader.mojo:47-144) through the C ABI: layer files loaded into
two HBM slots, C += A . deq(W) on the active slot against the f64 product of
the oracle (max error relative to max |C| <= 1e-5, the Q4 matmul bar), and
run_pipeline's per-layer products (taps), the zeroed C it leaves, and its
LayerStats."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
SEED = 42


def say(msg):
    print(f"\n[case] {msg}", flush=True)


def rel_max(a, ref):
    return float(np.max(np.abs(np.asarray(a, np.float64) - ref)) / (np.max(np.abs(ref)) + 1e-30))


def read_layer(base, i, N):
    raw = np.fromfile(os.path.join(base, f"layer_{i}.bin"), np.uint8)
    scale = float(raw[:4].view(np.float32)[0])
    return raw[4:].reshape(N, N // 2), scale


@pytest.mark.parametrize("N,L,M", [(1024, 6, 4), (2560, 3, 1)])
def test_model_runner_vs_oracle(gpu, oracle, tmp_path, N, L, M):
    ms = gpu
    from mojostream_amd.loader import ModelRunner, write_layer_files
    say(f"ModelRunner N={N} layers={L} M={M}")
    base = str(tmp_path / "packed")
    scales = write_layer_files(base, L, N, seed=SEED)
    A = ms.host_normal(M * N, 5, N).reshape(M, N)
    C0 = ms.host_normal(M * N, 6, N).reshape(M, N)
    dA, dC = ms.DeviceBuffer.from_array(A), ms.DeviceBuffer.from_array(C0)
    r = ModelRunner(base, L, N)
    # load_into_slot + compute_active: C += A . deq(W) on the chosen slot
    t_load = r.load_into_slot(1, L - 1)
    r.active = 1
    assert r.active == 1
    t_comp = r.compute_active(dC, dA, M)
    q4, sc = read_layer(base, L - 1, N)
    assert abs(sc - scales[L - 1]) == 0.0
    err = rel_max(dC.download(np.float32, (M, N)), C0 + oracle.matmul_f64(A, q4, N, sc))
    print(f"  compute_active: rel err {err:.2e}, load {t_load / 1e6:.2f} ms, "
          f"compute {t_comp / 1e3:.1f} us")
    assert err < 1e-5 and t_load > 0 and t_comp > 0
    # run_pipeline: layer i's product before the zeroing; C accumulates into
    # the caller's C for layer 0 (C += A . W), every later layer starts at 0
    dC.upload(C0)
    taps = ms.DeviceBuffer(L * M * N * 4)
    stats = r.run_pipeline(dC, dA, M, taps)
    got = taps.download(np.float32, (L, M, N))
    worst = 0.0
    for i in range(L):
        q4, sc = read_layer(base, i, N)
        ref = oracle.matmul_f64(A, q4, N, sc) + (C0 if i == 0 else 0.0)
        worst = max(worst, rel_max(got[i], ref))
    print(f"  run_pipeline: worst layer rel err {worst:.2e}")
    for i, s in enumerate(stats):
        print(f"    layer {i}: load {s.load_ns / 1e6:.3f} ms compute {s.compute_ns / 1e3:.1f} us "
              f"wait {s.wait_ns / 1e3:.1f} us")
    assert worst < 1e-5
    assert np.count_nonzero(dC.download(np.float32, (M, N))) == 0   # C.zero() after each layer
    assert len(stats) == L
    assert all(s.compute_ns > 0 and s.wait_ns >= 0 for s in stats)
    assert all(s.load_ns > 0 for s in stats[:-1]) and stats[-1].load_ns == 0
    # the slots flipped once per layer, starting from slot 0
    assert r.active == L % 2
    r.close()


def test_model_runner_errors(gpu, tmp_path):
    ms = gpu
    from mojostream_amd.loader import ModelRunner, write_layer_files
    say("ModelRunner errors: missing file, short file, bad slot, bad N")
    base = str(tmp_path / "p")
    write_layer_files(base, 2, 256, seed=1)
    r = ModelRunner(base, 3, 256)
    with pytest.raises(ms.MSError, match="layer_2.bin"):
        r.load_into_slot(0, 2)
    with open(os.path.join(base, "layer_1.bin"), "r+b") as f:
        f.truncate(1000)
    with pytest.raises(ms.MSError, match="expected"):
        r.load_into_slot(0, 1)
    with pytest.raises(ms.MSError, match="slot"):
        r.load_into_slot(2, 0)
    A = ms.DeviceBuffer.from_array(np.ones((4, 256), np.float32))
    C = ms.DeviceBuffer.from_array(np.zeros((4, 256), np.float32))
    with pytest.raises(ms.MSError, match="layer_1.bin"):   # the truncated one
        r.run_pipeline(C, A, 4)
    r.close()
    with pytest.raises(ms.MSError, match="multiple of 128"):
        ModelRunner(base, 2, 100)
