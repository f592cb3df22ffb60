"""Q8_0 kernels against the oracle and slate's golden answers, through the C ABI.

Tolerances:
* dequantised weights and the tiled layout: bit-exact (d * q is one exact
  product; the tiles are the same bytes regrouped);
* Q8_0 matmul: normwise relative 1e-5 against the oracle's
  slate_q8_0_matvec arithmetic (quant.c:64-133), and per element 1e-4
  relative to the float64 dot of the dequantised weights (slate's
  tests/test_q8_dot.c bound); tiled and row layouts bit-identical.
"""
import numpy as np
import pytest

from slate_amd import DeviceBuffer as DB
from slate_amd import check
from slate_amd.synth import quantize_q8_0
from tests.helpers import bits, relerr, same_floats

pytestmark = pytest.mark.gpu


def dev(a):
    return DB.from_array(np.ascontiguousarray(a))


def tame_q8_blocks(rng, nblocks):
    """Random Q8_0 bytes with finite, moderate d (|d| in [2^-8, 2^-1))."""
    b = rng.integers(0, 256, (nblocks, 34), dtype=np.uint8)
    b[:, 1] = (b[:, 1] & 0x83) | 0x1C
    return np.ascontiguousarray(b.reshape(-1))


def test_q8_dequant_bitexact_golden(hip, golden):
    raw = golden["q8_raw"]
    n = raw.size // 34 * 32
    out = DB(n * 4)
    check(hip.lib.slate_hip_dequant_q8_0(out.p, dev(raw).p, n), "dequant_q8_0")
    assert np.array_equal(bits(out.to_array(np.float32, n)), bits(golden["q8_deq"]))


def test_q8_dequant_every_scale(hip, orc):
    """d sweeps all 65536 half bit patterns (zero, subnormal, inf, NaN)."""
    rng = np.random.default_rng(21)
    blocks = rng.integers(0, 256, (65536, 34), dtype=np.uint8)
    blocks[:, 0:2] = np.arange(65536, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    blocks[::5, 2:] = 0x80                       # q = -128
    raw = np.ascontiguousarray(blocks.reshape(-1))
    n = 65536 * 32
    out = DB(n * 4)
    check(hip.lib.slate_hip_dequant_q8_0(out.p, dev(raw).p, n), "dequant_q8_0")
    assert same_floats(out.to_array(np.float32, n), orc.dequant_q8_0(raw, n))


def untile_q8(t, M, K):
    """Inverse of the TILED layout, from its definition: tile ti, group kb is
    4352 bytes = row j's eight f16 d at 16j, then for c < 4 and lane
    l = 16g + j the 16 bytes q[j][64c + 8g : +8], q[j][64c + 32 + 8g : +8]."""
    ngrp = (K + 255) // 256
    tiles = (M + 15) // 16
    t = t.reshape(tiles, ngrp, 4352)
    nb = ngrp * 8
    out = np.zeros((tiles * 16, nb, 34), np.uint8)
    for j in range(16):
        d = t[:, :, 16 * j:16 * j + 16].reshape(tiles, ngrp, 8, 2)
        out[j::16, :, 0:2] = d.reshape(tiles, nb, 2)
        for c in range(4):
            for g in range(4):
                l = 16 * g + j
                u = t[:, :, 256 + 1024 * c + 16 * l:256 + 1024 * c + 16 * l + 16]
                out[j::16, 2 * c::8, 2 + 8 * g:10 + 8 * g] = u[:, :, 0:8]
                out[j::16, 2 * c + 1::8, 2 + 8 * g:10 + 8 * g] = u[:, :, 8:16]
    return out


@pytest.mark.parametrize("M,K", [(16, 256), (37, 512), (5, 96), (40, 800), (4096, 4096)])
def test_q8_tile_layout(hip, M, K):
    rng = np.random.default_rng(M + K)
    raw = tame_q8_blocks(rng, M * K // 32)
    nbytes = hip.lib.slate_hip_q8_0_tiled_bytes(M, K)
    assert nbytes == ((M + 15) // 16) * ((K + 255) // 256) * 4352
    T = DB(nbytes)
    check(hip.lib.slate_hip_q8_0_tile(T.p, dev(raw).p, M, K), "q8_0_tile")
    rows = untile_q8(T.to_array(np.uint8, nbytes), M, K)
    nb = K // 32
    assert np.array_equal(rows[:M, :nb].reshape(-1), raw)
    assert not rows[M:].any() and not rows[:, nb:].any()     # padding is zero blocks


def q8_case(M, K, seed):
    rng = np.random.default_rng(seed)
    W = rng.normal(0, 0.02, (M, K)).astype(np.float32)
    return rng, np.frombuffer(quantize_q8_0(W), np.uint8).copy()


@pytest.mark.parametrize("M,K", [(256, 256), (200, 512), (1, 32), (100, 96), (64, 800), (4096, 4096),
                                 (1024, 14336)])
@pytest.mark.parametrize("B", [1, 3, 16, 17, 64, 70])
def test_matmul_q8_0(hip, orc, M, K, B):
    if M * K > 4096 * 4096 and B > 17:
        pytest.skip("oracle time budget")
    rng, raw = q8_case(M, K, M * 7 + K * 3 + B)
    X = rng.normal(0, 1, (B, K)).astype(np.float32)
    Y = DB(B * M * 4)
    check(hip.lib.slate_hip_matmul_q8_0(Y.p, dev(raw).p, dev(X).p, B, M, K), "matmul_q8_0")
    got = Y.to_array(np.float32, (B, M))
    assert relerr(got, orc.q8_0_matmul(raw, X, M, K)) < 1e-5
    if M * K <= 4096 * 4096:
        deq = orc.dequant_q8_0(raw, M * K).reshape(M, K).astype(np.float64)
        ref = X.astype(np.float64) @ deq.T
        assert np.all(np.abs(got - ref) <= 1e-4 * np.abs(ref) + 1e-5 * np.abs(ref).max())


def test_q8_0_matvec_golden(hip, golden):
    """slate_q8_0_matvec's signature on slate's own output for edge-case
    scales (zero, subnormal, negative, all q = -128 / 127 blocks)."""
    M, K = (int(v) for v in golden["q8_MK"])
    A = dev(golden["q8_mv_raw"])
    for i in range(3):
        y = DB(M * 4)
        hip.lib.slate_hip_q8_0_matvec(y.p, A.p, dev(golden["q8_x"][i]).p, M, K)
        check(0 if hip.lib.slate_hip_last_error() is None else -1, "q8_0_matvec")
        got = y.to_array(np.float32, M)
        want = golden["q8_y"][i]
        assert np.all(np.abs(got - want) <= 1e-5 * np.abs(want).max()), i


def test_matmul_q8_0_activation_scales(hip, orc):
    """Rows spanning tiny to large magnitudes, groups of one row at very
    different scales, and an all-zero row."""
    rng, raw = q8_case(384, 2048, 4)
    M, K = 384, 2048
    X = rng.normal(0, 1, (6, K)).astype(np.float32)
    X[0] *= 1e-6
    X[1] *= 3e3
    X[2] = 0
    X[3, ::7] *= 100.0
    X[5, :256] *= 1e4
    X[5, 256:512] *= 1e-4
    X[5, 1024:1280] = 0
    for B in (6, 40):          # decode and prefill kernels
        Xb = np.zeros((B, K), np.float32)
        Xb[:6] = X
        Y = DB(B * M * 4)
        check(hip.lib.slate_hip_matmul_q8_0(Y.p, dev(raw).p, dev(Xb).p, B, M, K), "matmul_q8_0")
        got = Y.to_array(np.float32, (B, M))
        want = orc.q8_0_matmul(raw, Xb[:6], M, K)
        for r in (0, 1, 3, 4, 5):
            assert relerr(got[r], want[r]) < 1e-5, (B, r)
        assert np.all(got[2] == 0)


@pytest.mark.parametrize("M,K,B", [(256, 256, 1), (200, 512, 16), (4096, 4096, 16), (1024, 14336, 7),
                                   (300, 1024, 40), (4096, 4096, 64), (100, 96, 3)])
def test_matmul_q8_0_tiled(hip, orc, M, K, B):
    """Pre-tiled weights give the row layout's results bit for bit."""
    rng, raw = q8_case(M, K, M * 5 + K + B)
    X = rng.normal(0, 1, (B, K)).astype(np.float32)
    T = DB(hip.lib.slate_hip_q8_0_tiled_bytes(M, K))
    check(hip.lib.slate_hip_q8_0_tile(T.p, dev(raw).p, M, K), "q8_0_tile")
    Yt, Yr = DB(B * M * 4), DB(B * M * 4)
    Xd = dev(X)
    check(hip.lib.slate_hip_matmul_q8_0_tiled(Yt.p, T.p, Xd.p, B, M, K), "matmul_q8_0_tiled")
    check(hip.lib.slate_hip_matmul_q8_0(Yr.p, dev(raw).p, Xd.p, B, M, K), "matmul_q8_0")
    got, row = Yt.to_array(np.float32, (B, M)), Yr.to_array(np.float32, (B, M))
    assert np.array_equal(bits(got), bits(row))
    if M * K <= 4096 * 4096 and B <= 16:
        assert relerr(got, orc.q8_0_matmul(raw, X, M, K)) < 1e-5


@pytest.mark.parametrize("M,K", [(14336, 4096), (4096, 14336)])
def test_matmul_q8_0_c2_shapes(hip, orc, M, K):
    """Q8_0 at the Q4_K op's full sizes: W ~ N(0, 0.02) quantised to Q8_0, X ~
    N(0, 1), B in {1, 4, 16, 64} (decode plan and prompt kernel), row and
    tiled layouts bit-identical, against the oracle's Q8_0 matvec
    (quant.c:64-133) at rel 1e-5."""
    rng, raw = q8_case(M, K, M + 5 * K)
    Wd = dev(raw)
    T = DB(hip.lib.slate_hip_q8_0_tiled_bytes(M, K))
    check(hip.lib.slate_hip_q8_0_tile(T.p, Wd.p, M, K), "q8_0_tile")
    for B in (1, 4, 16, 64):
        X = rng.normal(0, 1, (B, K)).astype(np.float32)
        Xd = dev(X)
        Yr, Yt = DB(B * M * 4), DB(B * M * 4)
        check(hip.lib.slate_hip_matmul_q8_0(Yr.p, Wd.p, Xd.p, B, M, K), "matmul_q8_0")
        check(hip.lib.slate_hip_matmul_q8_0_tiled(Yt.p, T.p, Xd.p, B, M, K), "matmul_q8_0_tiled")
        got, gt = Yr.to_array(np.float32, (B, M)), Yt.to_array(np.float32, (B, M))
        assert np.array_equal(bits(got), bits(gt)), B
        assert relerr(got, orc.q8_0_matmul(raw, X, M, K)) < 1e-5, B


def test_matmul_q8_0_rejects_bad_shapes(hip):
    hip.lib.slate_hip_clear_error()
    Y, A, X = DB(64), DB(64), DB(64)
    assert hip.lib.slate_hip_matmul_q8_0(Y.p, A.p, X.p, 1, 1, 48) == -1     # K % 32 != 0
    assert b"multiple of 32" in hip.lib.slate_hip_last_error()
    hip.lib.slate_hip_clear_error()
    assert hip.lib.slate_hip_matmul_q8_0(Y.p, A.p, X.p, 0, 1, 32) == -1
    hip.lib.slate_hip_clear_error()
    assert hip.lib.slate_hip_dequant_q8_0(Y.p, A.p, 33) == -1
    hip.lib.slate_hip_clear_error()
