"""ms_q4_matmul_noalloc (the variant of ms_q4_matmul that allocates nothing:
its quantized rows live in the library's static device scratch array) against
ms_q4_matmul through the C ABI.

The two share every kernel, so the outputs must be bit-identical.  Calls run
back to back with shrinking inputs, so each one reads a scratch array still
holding the previous call's rows: stale contents must not leak into results.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"\n[case] {msg}", flush=True)


def _call(ms, name, C0, A, wpk, K, N, scale, acc):
    M = A.shape[0]
    dC = ms.DeviceBuffer.from_array(C0)
    dA = ms.DeviceBuffer.from_array(A)
    fn = getattr(ms.lib(), name)
    ms.check(fn(dC.ptr, dA.ptr, wpk.ptr, M, K, N, C.c_float(scale), acc))
    ms.synchronize()
    return dC.download(np.float32, (M, N))


# (M, K, N, accumulate): GEMM-path calls (M > 16) then GEMV-path calls, each
# smaller than the one before
CASES = [(64, 4096, 1024, 0), (40, 2048, 512, 1), (16, 4096, 1024, 0), (3, 1024, 512, 1)]


def test_noalloc_equals_matmul(gpu):
    ms = gpu
    weights = {}
    for i, (M, K, N, acc) in enumerate(CASES):
        say(f"no-alloc q4 matmul call {i}: M={M} K={K} N={N} accumulate={acc}")
        if (K, N) not in weights:
            raw = ms.DeviceBuffer.from_array(ms.host_random_u8(K * N // 2, 7, K + N))
            pk = ms.DeviceBuffer(K * N // 2)
            ms.check(ms.lib().ms_q4_pack(pk.ptr, raw.ptr, K, N))
            weights[(K, N)] = pk
        A = ms.host_normal(M * K, 11, i).reshape(M, K)
        C0 = ms.host_normal(M * N, 12, i).reshape(M, N)
        ref = _call(ms, "ms_q4_matmul", C0, A, weights[(K, N)], K, N, 0.07, acc)
        got = _call(ms, "ms_q4_matmul_noalloc", C0, A, weights[(K, N)], K, N, 0.07, acc)
        assert np.all(np.isfinite(ref))
        assert np.array_equal(got, ref), f"call {i}: results differ"


def test_noalloc_rejects_oversize(gpu):
    ms = gpu
    say("no-alloc q4 matmul: rows beyond the 4 MiB scratch are refused")
    dummy = ms.DeviceBuffer(16)
    rc = ms.lib().ms_q4_matmul_noalloc(dummy.ptr, dummy.ptr, dummy.ptr, 2048, 4096, 1024,
                                       C.c_float(0.1), 0)
    assert rc == -1
    assert "4 MiB" in ms.lib().ms_last_error().decode()
