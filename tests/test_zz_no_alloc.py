"""slate_hip_matmul_q4k_noalloc: the Q4_K matmul that allocates nothing (its
operand and split-K partials live in the library's fixed device scratch)
against slate_hip_matmul_q4k on the same inputs, through the C ABI: two
calls in a row (the second smaller, so it runs on what the first left in the
scratch), the small-batch path, and the size limit."""
import numpy as np
import pytest

import slate_amd
from slate_amd.synth import quantize_q4k
from tests.conftest import relerr

pytestmark = pytest.mark.gpu


def noalloc_fn():
    return slate_amd.load_library().slate_hip_matmul_q4k_noalloc


def run_both(hip, f, raw, X, M, K):
    B = X.shape[0]
    W = slate_amd.DeviceBuffer.from_array(raw)
    Xd = slate_amd.DeviceBuffer.from_array(X)
    Y0 = slate_amd.DeviceBuffer(B * M * 4)
    Y1 = slate_amd.DeviceBuffer(B * M * 4)
    slate_amd.check(hip.matmul_q4k(Y0.p, W.p, Xd.p, B, M, K), "matmul_q4k")
    slate_amd.check(f(Y1.p, W.p, Xd.p, B, M, K), "matmul_q4k_noalloc")
    hip.sync()
    return Y0.to_array(np.float32, (B, M)), Y1.to_array(np.float32, (B, M))


def device_free_bytes():
    """Free device memory (hipMemGetInfo), after the backend stream drains."""
    import ctypes
    slate_amd.load_library().slate_hip_sync()
    hip_rt = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip_rt.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_noalloc_matmul_allocates_nothing(hip):
    """Device free memory is the same before and after a noalloc call of the
    largest kind (prompt kernel, 64 rows, ~30 MiB of operand and partials),
    made before any other matmul of this module.  Decisive in a fresh
    process (the module run alone), where the backend's own scratch holds
    nothing the call could have reused."""
    f = noalloc_fn()
    rng = np.random.default_rng(30)
    M, K, B = 28672, 4096, 64
    raw = np.frombuffer(quantize_q4k(rng.normal(0, 0.02, (M, K)).astype(np.float32)), np.uint8).copy()
    X = rng.normal(0, 1, (B, K)).astype(np.float32)
    W = slate_amd.DeviceBuffer.from_array(raw)
    Xd = slate_amd.DeviceBuffer.from_array(X)
    Y = slate_amd.DeviceBuffer(B * M * 4)
    before = device_free_bytes()
    slate_amd.check(f(Y.p, W.p, Xd.p, B, M, K), "matmul_q4k_noalloc")
    after = device_free_bytes()
    assert after == before, (before, after)
    hip.sync()
    want = slate_amd.DeviceBuffer(B * M * 4)
    slate_amd.check(hip.matmul_q4k(want.p, W.p, Xd.p, B, M, K), "matmul_q4k")
    hip.sync()
    assert relerr(Y.to_array(np.float32, (B, M)), want.to_array(np.float32, (B, M))) < 1e-6


def test_noalloc_matmul_matches_the_allocating_entry(hip, orc):
    f = noalloc_fn()
    rng = np.random.default_rng(31)
    # a large call first (prompt kernel, several splits), then a smaller one
    # (decode kernel) that reuses the scratch the first one left behind,
    # then a 3-row call (GEMV path, no scratch)
    cases = [(14336, 4096, 64), (4096, 4096, 16), (4096, 4096, 3)]
    for M, K, B in cases:
        raw = np.frombuffer(quantize_q4k(rng.normal(0, 0.02, (M, K)).astype(np.float32)), np.uint8).copy()
        X = rng.normal(0, 1, (B, K)).astype(np.float32)
        y0, y1 = run_both(hip, f, raw, X, M, K)
        assert relerr(y1, y0) < 1e-6, (M, K, B)
        want = orc.q4k_matmul(raw, X, M, K)
        assert relerr(y1, want) < 1e-5, (M, K, B)


def test_noalloc_matmul_rejects_sizes_beyond_its_scratch(hip):
    f = noalloc_fn()
    M, K, B = 128256, 4096, 64          # split partials alone exceed 32 MiB
    W = slate_amd.DeviceBuffer(M * (K // 256) * 144)
    X = slate_amd.DeviceBuffer(B * K * 4)
    Y = slate_amd.DeviceBuffer(B * M * 4)
    rc = f(Y.p, W.p, X.p, B, M, K)
    assert rc == -1
    err = slate_amd.last_error()
    assert err is not None and "limit" in err
    slate_amd.load_library().slate_hip_clear_error()
