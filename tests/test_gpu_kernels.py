"""HIP kernels against the oracle and slate's golden answers, through the C ABI.

Tolerances (from slate's own tests and the parity contract):
* dequantised weights, RoPE rotation of identical inputs, argmax and packing
  indices: bit-exact;
* Q4_K matmul: normwise relative 1e-5 against the oracle's
  slate_q4_k_matvec arithmetic, and per element 1e-4 relative to float64;
* vtable row primitives: slate's test_backend.c Linf bounds (1e-4 matvec /
  linear_batch, 1e-5 rmsnorm / silu / attention, exact add / embed / copy).
"""
import ctypes as C

import numpy as np
import pytest

from oracle.pyoracle import fp
from slate_amd import DeviceBuffer as DB
from slate_amd import check, load_library
from slate_amd.synth import quantize_q4k
from tests.helpers import bits, relerr, same_floats

pytestmark = pytest.mark.gpu


def dev(a):
    return DB.from_array(np.ascontiguousarray(a))


def host(b, dtype, shape):
    return b.to_array(dtype, shape)


def tame_random_blocks(rng, nblocks):
    """Random Q4_K bytes with finite, moderate d/dmin."""
    b = rng.integers(0, 256, (nblocks, 144), dtype=np.uint8)
    b[:, 1] = (b[:, 1] & 0x1F) | 0x10
    b[:, 3] = (b[:, 3] & 0x1F) | 0x10
    return np.ascontiguousarray(b.reshape(-1))


# ------------------------------------------------------------ Q4_K
def test_dequant_bitexact_golden(hip, golden):
    raw = golden["q4k_raw"]
    n = raw.size // 144 * 256
    out = DB(n * 4)
    check(hip.dequant_q4k(out.p, dev(raw).p, n), "dequant")
    got = host(out, np.float32, n)
    assert np.array_equal(bits(got), bits(golden["q4k_deq"]))


def test_dequant_bitexact_random(hip, orc):
    rng = np.random.default_rng(1)
    raw = tame_random_blocks(rng, 4096 * 4)          # 4096 x 1024 weights
    n = 4096 * 1024
    out = DB(n * 4)
    check(hip.dequant_q4k(out.p, dev(raw).p, n), "dequant")
    got = host(out, np.float32, n)
    assert np.array_equal(bits(got), bits(orc.dequant_q4k(raw, n)))
    # every f16 header value: d and dmin sweep all 65536 bit patterns
    blocks = np.zeros((65536, 144), np.uint8)
    blocks[:, 0:2] = np.arange(65536, dtype=np.uint16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:4] = np.arange(65536, dtype=np.uint16)[::-1].copy().view(np.uint8).reshape(-1, 2)
    blocks[:, 4:16] = rng.integers(0, 256, (65536, 12), dtype=np.uint8)
    blocks[:, 16:] = rng.integers(0, 256, (65536, 128), dtype=np.uint8)
    raw = np.ascontiguousarray(blocks.reshape(-1))
    n = 65536 * 256
    out = DB(n * 4)
    check(hip.dequant_q4k(out.p, dev(raw).p, n), "dequant")
    got = host(out, np.float32, n)
    assert same_floats(got, orc.dequant_q4k(raw, n))


@pytest.mark.parametrize("M,K", [(256, 256), (200, 512), (4096, 4096), (1024, 14336)])
# 3, 9 and 16 rows: the one-tile kernel that makes its operand from the f32
# rows; 70, 90 and 100 rows: the prompt kernel's last group of activation
# tiles holds one, two and three of its four tiles
@pytest.mark.parametrize("B", [1, 3, 9, 16, 17, 64, 70, 90, 100])
def test_matmul_q4k(hip, orc, M, K, B):
    if M * K > 4096 * 4096 and B > 17:
        pytest.skip("oracle time budget")
    rng = np.random.default_rng(M * 7 + K * 3 + B)
    W = rng.normal(0, 0.02, (M, K)).astype(np.float32)
    raw = np.frombuffer(quantize_q4k(W), np.uint8).copy()
    X = rng.normal(0, 1, (B, K)).astype(np.float32)
    Y = DB(B * M * 4)
    check(hip.matmul_q4k(Y.p, dev(raw).p, dev(X).p, B, M, K), "matmul_q4k")
    got = host(Y, np.float32, (B, M))
    want = orc.q4k_matmul(raw, X, M, K)
    assert relerr(got, want) < 1e-5
    if M * K <= 4096 * 4096:
        deq = orc.dequant_q4k(raw, M * K).reshape(M, K).astype(np.float64)
        ref = X.astype(np.float64) @ deq.T
        assert np.all(np.abs(got - ref) <= 1e-4 * np.abs(ref) + 1e-5 * np.abs(ref).max())


@pytest.mark.parametrize("M,K", [(4096, 4096), (14336, 4096), (4096, 14336)])
def test_matmul_q4k_c2_shapes(hip, orc, M, K):
    """The Q4_K op at its full sizes: W ~ N(0, 0.02) quantised to Q4_K on the
    device, X ~ N(0, 1), B in {1, 4, 16, 32, 64} (the one-row GEMV, the
    decode kernel with one and two 16-row activation tiles and the prompt
    kernel), in slate's row layout and
    the tiled layout, against the oracle's slate_q4_k_matvec
    (quant.c:306-313) and float64."""
    rng = np.random.default_rng(M + 3 * K)
    nbytes = M * (K // 256) * 144
    Wd = DB(nbytes)
    check(hip.lib.slate_hip_synth_q4k(Wd.p, M, K, M * 31 + K, 0.02), "synth_q4k")
    raw = host(Wd, np.uint8, nbytes)
    T = DB(hip.lib.slate_hip_q4k_tiled_bytes(M, K))
    check(hip.lib.slate_hip_q4k_tile(T.p, Wd.p, M, K), "q4k_tile")
    deq = orc.dequant_q4k(raw, M * K).reshape(M, K).astype(np.float64)
    for B in (1, 4, 16, 32, 64):
        X = rng.normal(0, 1, (B, K)).astype(np.float32)
        Xd = dev(X)
        Yr, Yt = DB(B * M * 4), DB(B * M * 4)
        check(hip.matmul_q4k(Yr.p, Wd.p, Xd.p, B, M, K), "matmul_q4k")
        check(hip.lib.slate_hip_matmul_q4k_tiled(Yt.p, T.p, Xd.p, B, M, K), "matmul_q4k_tiled")
        got, gt = host(Yr, np.float32, (B, M)), host(Yt, np.float32, (B, M))
        want = orc.q4k_matmul(raw, X, M, K)
        ref = X.astype(np.float64) @ deq.T
        # one row: the vector-ALU GEMV on the row layout, the MFMA matvec on
        # the tiled one (each against the oracle); more rows: one kernel, the
        # same bits from either layout
        for y in ((got, gt) if B == 1 else (got,)):
            assert relerr(y, want) < 1e-5, B
            assert np.all(np.abs(y - ref) <= 1e-4 * np.abs(ref) + 1e-5 * np.abs(ref).max()), B
        if B > 1:
            assert np.array_equal(bits(got), bits(gt)), B


@pytest.mark.parametrize("M,K", [(1, 256), (37, 256), (100, 16640), (257, 2304)])
@pytest.mark.parametrize("B", [1, 2, 3, 4])
def test_matmul_q4k_small_batch_edges(hip, orc, M, K, B):
    """Small batches at the edges of the kernels' tilings: one super-block
    (in the one-row GEMV a single wave with 8 busy lanes), row counts that
    leave a partial workgroup, K above 64 super-blocks (two GEMV passes; the
    tiled layout's one-row MFMA matvec stops at 64) and K not a multiple of
    2048; against the oracle, and row and tiled layouts bit for bit from two
    rows on."""
    rng = np.random.default_rng(M * 13 + K + B)
    raw = np.frombuffer(quantize_q4k(rng.normal(0, 0.02, (M, K)).astype(np.float32)), np.uint8).copy()
    X = rng.normal(0, 1, (B, K)).astype(np.float32)
    X[0, :256] *= 1e3
    Xd, Wd = dev(X), dev(raw)
    T = DB(hip.lib.slate_hip_q4k_tiled_bytes(M, K))
    check(hip.lib.slate_hip_q4k_tile(T.p, Wd.p, M, K), "q4k_tile")
    Yr, Yt = DB(B * M * 4), DB(B * M * 4)
    check(hip.matmul_q4k(Yr.p, Wd.p, Xd.p, B, M, K), "matmul_q4k")
    check(hip.lib.slate_hip_matmul_q4k_tiled(Yt.p, T.p, Xd.p, B, M, K), "matmul_q4k_tiled")
    got, gt = host(Yr, np.float32, (B, M)), host(Yt, np.float32, (B, M))
    want = orc.q4k_matmul(raw, X, M, K)
    for r in range(B):
        assert relerr(got[r], want[r]) < 1e-5, r
    if B == 1:   # the tiled layout's MFMA matvec (K up to 64 blocks)
        assert relerr(gt[0], want[0]) < 1e-5
    else:
        assert np.array_equal(bits(got), bits(gt))
    if B == 1:   # the vtable entry (backend.h:63-70) is the same kernel
        y = DB(M * 4)
        hip.matvec_q4k(y.p, Wd.p, Xd.p, M, K)
        hip.sync()
        check(0, "matvec_q4k")
        assert np.array_equal(bits(host(y, np.float32, M)), bits(got[0]))


def test_matmul_q4k_activation_scales(hip, orc):
    """Rows spanning tiny to large magnitudes (the per-row power-of-two scale
    keeps the f16 split accurate) and an all-zero row."""
    rng = np.random.default_rng(4)
    M, K = 512, 2048
    raw = np.frombuffer(quantize_q4k(rng.normal(0, 0.02, (M, K)).astype(np.float32)), np.uint8).copy()
    X = rng.normal(0, 1, (6, K)).astype(np.float32)
    X[0] *= 1e-6
    X[1] *= 3e3
    X[2] = 0
    X[3, ::7] *= 100.0
    X[5, :256] *= 1e4        # blocks of one row at very different scales
    X[5, 256:512] *= 1e-4
    X[5, 1024:1280] = 0
    for B in (4, 6, 20):     # small-batch GEMV, one 16-row tile, several tiles
        Xb = np.zeros((B, K), np.float32)
        n = min(B, 6)
        Xb[:n] = X[:n]
        Y = DB(B * M * 4)
        check(hip.matmul_q4k(Y.p, dev(raw).p, dev(Xb).p, B, M, K), "matmul_q4k")
        got = host(Y, np.float32, (B, M))
        want = orc.q4k_matmul(raw, Xb[:n], M, K)
        for r in (0, 1, 3, 4, 5):
            if r < n:
                assert relerr(got[r], want[r]) < 1e-5, (B, r)
        assert np.all(got[2] == 0)
    # one row at a time, both layouts (the tiled layout's MFMA matvec scales
    # each block of x itself)
    Wd = dev(raw)
    T = DB(hip.lib.slate_hip_q4k_tiled_bytes(M, K))
    check(hip.lib.slate_hip_q4k_tile(T.p, Wd.p, M, K), "q4k_tile")
    for r in range(6):
        Y, Yt = DB(M * 4), DB(M * 4)
        Xr = dev(X[r:r + 1])
        check(hip.matmul_q4k(Y.p, Wd.p, Xr.p, 1, M, K), "matmul_q4k")
        check(hip.lib.slate_hip_matmul_q4k_tiled(Yt.p, T.p, Xr.p, 1, M, K), "matmul_q4k_tiled")
        for got in (host(Y, np.float32, (1, M)), host(Yt, np.float32, (1, M))):
            if r == 2:
                assert np.all(got == 0)
            else:
                assert relerr(got, orc.q4k_matmul(raw, X[r:r + 1], M, K)) < 1e-5, r


def untile_q4k(t, M, K):
    """Inverse of the TILED layout, written from its definition: tile ti,
    block kb is 2304 bytes = 16 headers of 16 bytes, then for lane
    l = 16g + j the 16 bytes qs[32g:32g+16] of row j, then qs[32g+16:32g+32]."""
    nblk = K // 256
    tiles = (M + 15) // 16
    t = t.reshape(tiles, nblk, 2304)
    out = np.zeros((tiles * 16, nblk, 144), np.uint8)
    for j in range(16):
        out[j::16, :, 0:16] = t[:, :, 16 * j:16 * j + 16]
        for g in range(4):
            l = 16 * g + j
            out[j::16, :, 16 + 32 * g:32 + 32 * g] = t[:, :, 256 + 16 * l:272 + 16 * l]
            out[j::16, :, 32 + 32 * g:48 + 32 * g] = t[:, :, 1280 + 16 * l:1296 + 16 * l]
    return out, tiles


@pytest.mark.parametrize("M,K", [(16, 256), (37, 512), (4096, 4096)])
def test_q4k_tile_layout(hip, M, K):
    rng = np.random.default_rng(M + K)
    raw = tame_random_blocks(rng, M * K // 256)
    nbytes = hip.lib.slate_hip_q4k_tiled_bytes(M, K)
    assert nbytes == ((M + 15) // 16) * 16 * (K // 256) * 144
    T = DB(nbytes)
    check(hip.lib.slate_hip_q4k_tile(T.p, dev(raw).p, M, K), "q4k_tile")
    t = host(T, np.uint8, nbytes)
    rows, tiles = untile_q4k(t, M, K)
    assert np.array_equal(rows[:M].reshape(-1), raw)
    assert not rows[M:].any()          # padding rows are zero blocks


@pytest.mark.parametrize("M,K,B", [(256, 256, 1), (200, 512, 16), (4096, 4096, 16), (1024, 14336, 7),
                                   (6144, 4096, 16), (300, 1024, 40), (4096, 4096, 64)])
def test_matmul_q4k_tiled(hip, orc, M, K, B):
    """The tiled layout gives the same results as the row layout, bit for
    bit from two rows on (same kernels and plan, only the weight addressing
    differs); one row runs the MFMA matvec on the tiled layout and the
    vector-ALU GEMV on the row layout, both against the oracle."""
    rng = np.random.default_rng(M * 5 + K + B)
    W = rng.normal(0, 0.02, (M, K)).astype(np.float32)
    raw = np.frombuffer(quantize_q4k(W), np.uint8).copy()
    X = rng.normal(0, 1, (B, K)).astype(np.float32)
    T = DB(hip.lib.slate_hip_q4k_tiled_bytes(M, K))
    check(hip.lib.slate_hip_q4k_tile(T.p, dev(raw).p, M, K), "q4k_tile")
    Yt, Yr = DB(B * M * 4), DB(B * M * 4)
    Xd = dev(X)
    check(hip.lib.slate_hip_matmul_q4k_tiled(Yt.p, T.p, Xd.p, B, M, K), "matmul_q4k_tiled")
    check(hip.matmul_q4k(Yr.p, dev(raw).p, Xd.p, B, M, K), "matmul_q4k")
    got, row = host(Yt, np.float32, (B, M)), host(Yr, np.float32, (B, M))
    if B > 1:
        assert np.array_equal(bits(got), bits(row))
    if B == 1 or (M * K <= 4096 * 4096 and B <= 16):
        want = orc.q4k_matmul(raw, X, M, K)
        assert relerr(got, want) < 1e-5 and relerr(row, want) < 1e-5


def test_matvec_q4k_vtable_golden(hip, golden):
    M, K = golden["q4k_MK"]
    raw = dev(golden["q4k_mv_raw"])
    for i in range(3):
        y = DB(M * 4)
        hip.matvec_q4k(y.p, raw.p, dev(golden["q4k_x"][i]).p, M, K)
        hip.sync()
        check(0, "matvec_q4k")
        assert relerr(host(y, np.float32, M), golden["q4k_y"][i]) < 1e-5


# ------------------------------------------------------------ vtable KATs
def test_vtable_known_answers(hip, golden):
    """slate's tests/test_backend.c, staged through alloc/copy_h2d/copy_d2h."""
    g = golden
    assert hip.name == "hip"
    # memory round trip, odd size
    src = (np.arange(137, dtype=np.float32) * np.float32(0.5) - np.float32(12))
    p = hip.alloc(137 * 4)
    assert p
    dst = np.empty_like(src)
    hip.copy_h2d(p, src.ctypes.data, 137 * 4)
    hip.copy_d2h(dst.ctypes.data, p, 137 * 4)
    hip.release(p)
    assert np.array_equal(dst, src)

    y = DB(7 * 4)
    hip.matvec(y.p, dev(g["kat_matvec_A"]).p, dev(g["kat_matvec_x"]).p, 7, 11)
    assert np.max(np.abs(host(y, np.float32, 7) - g["kat_matvec_y"])) < 1e-4
    Cb = DB(24 * 4)
    hip.linear_batch(Cb.p, dev(g["kat_lb_X"]).p, dev(g["kat_lb_W"]).p, 4, 8, 6)
    assert np.max(np.abs(host(Cb, np.float32, 24) - g["kat_lb_C"])) < 1e-4
    yr = DB(16 * 4)
    hip.rmsnorm_row(yr.p, dev(g["kat_rms_x"]).p, dev(g["kat_rms_w"]).p, 16, 1e-5)
    assert np.max(np.abs(host(yr, np.float32, 16) - g["kat_rms_y"])) < 1e-5
    gb = dev(g["kat_silu_g"])
    hip.silu_mul(gb.p, gb.p, dev(g["kat_silu_u"]).p, 24)          # in place, as llama_infer.c:192
    assert np.max(np.abs(host(gb, np.float32, 24) - g["kat_silu_y"])) < 1e-5
    y0 = np.arange(32, dtype=np.float32) * np.float32(0.1)
    x0 = (np.arange(32) - 16).astype(np.float32) * np.float32(0.2)
    ya = dev(y0)
    hip.add_inplace(ya.p, dev(x0).p, 32)
    assert np.array_equal(host(ya, np.float32, 32), y0 + x0)
    W = np.arange(40, dtype=np.float32)
    ye = DB(8 * 4)
    hip.embed_lookup(ye.p, dev(W).p, 3, 8)
    assert np.array_equal(host(ye, np.float32, 8), W[24:32])
    o = DB(16 * 4)
    sc = DB(5 * 4)
    hip.attention_step(o.p, dev(g["kat_att_q"]).p, dev(g["kat_att_K"]).p, dev(g["kat_att_V"]).p, sc.p, 5, 16)
    assert np.max(np.abs(host(o, np.float32, 16) - g["kat_att_out"])) < 1e-5
    L, D = g["att64_K"].shape
    o = DB(D * 4)
    sc = DB(L * 4)
    hip.attention_step(o.p, dev(g["att64_q"]).p, dev(g["att64_K"]).p, dev(g["att64_V"]).p, sc.p, L, D)
    assert np.max(np.abs(host(o, np.float32, D) - g["att64_out"])) < 1e-5
    for Dn in (37, 4096):
        yy = DB(Dn * 4)
        hip.rmsnorm_row(yy.p, dev(g[f"rms{Dn}_x"]).p, dev(g[f"rms{Dn}_w"]).p, Dn, 1e-5)
        assert np.max(np.abs(host(yy, np.float32, Dn) - g[f"rms{Dn}_y"])) < 1e-5
        ss = DB(Dn * 4)
        hip.silu_mul(ss.p, dev(g[f"silu{Dn}_g"]).p, dev(g[f"rms{Dn}_w"]).p, Dn)
        assert np.max(np.abs(host(ss, np.float32, Dn) - g[f"silu{Dn}_y"])) < 1e-5
    hip.sync()
    check(0, "vtable")


def test_matvec_linear_batch_random(hip, orc):
    rng = np.random.default_rng(8)
    for M, K in ((172, 64), (64, 172), (300, 1000)):
        A = rng.normal(0, 0.5, (M, K)).astype(np.float32)
        x = rng.normal(0, 1, K).astype(np.float32)
        y = DB(M * 4)
        hip.matvec(y.p, dev(A).p, dev(x).p, M, K)
        want = np.empty(M, np.float32)
        orc.lib.orc_matvec(fp(want), fp(A), fp(x), M, K)
        assert np.max(np.abs(host(y, np.float32, M) - want)) < 1e-4
        Bn, N = 5, M
        X = rng.normal(0, 1, (Bn, K)).astype(np.float32)
        W = rng.normal(0, 0.5, (K, N)).astype(np.float32)
        Cd = DB(Bn * N * 4)
        hip.linear_batch(Cd.p, dev(X).p, dev(W).p, Bn, K, N)
        want = np.empty((Bn, N), np.float32)
        orc.lib.orc_linear_batch(fp(want), fp(X), fp(W), Bn, K, N)
        assert np.max(np.abs(host(Cd, np.float32, (Bn, N)) - want)) < 1e-4


@pytest.mark.parametrize("Bn,K,N", [(1, 64, 300), (13, 300, 70), (37, 1000, 129)])
def test_linear_batch_row_blocks(hip, orc, Bn, K, N):
    """linear_batch (backend.h:58-61) with batch counts off the kernel's
    8-row blocks and column counts off its 64-column groups."""
    rng = np.random.default_rng(Bn * 1000 + N)
    X = rng.normal(0, 1, (Bn, K)).astype(np.float32)
    W = rng.normal(0, 0.5, (K, N)).astype(np.float32)
    Cd = DB(Bn * N * 4)
    hip.linear_batch(Cd.p, dev(X).p, dev(W).p, Bn, K, N)
    want = np.empty((Bn, N), np.float32)
    orc.lib.orc_linear_batch(fp(want), fp(X), fp(W), Bn, K, N)
    assert np.max(np.abs(host(Cd, np.float32, (Bn, N)) - want)) < 1e-4
    check(0, "linear_batch")


@pytest.mark.parametrize("L,D", [(1, 16), (7, 80), (1000, 128), (3000, 64), (300, 200), (40, 1100)])
def test_attention_step_long_contexts(hip, L, D):
    """The vtable's single-head attention (backend_cpu.c:117-166) at long
    contexts and head sizes off the wave width, against float64 softmax
    attention: out within 1e-5 absolute (test_backend.c's bound), and the
    scratch holds the normalised probabilities, as the reference leaves it."""
    rng = np.random.default_rng(L + D)
    q = rng.normal(0, 1, D).astype(np.float32)
    K = rng.normal(0, 1, (L, D)).astype(np.float32)
    V = rng.normal(0, 1, (L, D)).astype(np.float32)
    o = DB(D * 4)
    sc = DB(L * 4)
    hip.attention_step(o.p, dev(q).p, dev(K).p, dev(V).p, sc.p, L, D)
    hip.sync()
    check(0, "attention_step")
    s = (K.astype(np.float64) @ q.astype(np.float64)) / np.sqrt(D)
    p = np.exp(s - s.max())
    p /= p.sum()
    assert np.max(np.abs(host(sc, np.float32, L) - p)) < 1e-6
    assert np.max(np.abs(host(o, np.float32, D) - p @ V.astype(np.float64))) < 1e-5


# ------------------------------------------------------------ RoPE
def test_rope_rows_bitexact_golden(hip, golden):
    x, y, pos = golden["rope_x"], golden["rope_y"], golden["rope_pos"]
    xb = dev(x)
    check(hip.rope_rows(xb.p, dev(pos).p, len(pos), 4, 128, 10000.0, 16384), "rope_rows")
    assert np.array_equal(bits(host(xb, np.float32, x.shape)), bits(y))


def test_rope_rows_rejects_out_of_range(hip):
    xb = dev(np.ones((2, 64), np.float32))
    rc = hip.rope_rows(xb.p, dev(np.array([3, 99], np.int32)).p, 2, 1, 64, 10000.0, 50)
    assert rc == -1
    load_library().slate_hip_clear_error()
    # the in-range row was rotated, the other left as it was
    out = host(xb, np.float32, (2, 64))
    assert np.array_equal(out[1], np.ones(64, np.float32))


# ------------------------------------------------------------ argmax / packing
def test_argmax_rows(hip, orc):
    rng = np.random.default_rng(12)
    B, V = 16, 128256
    L = rng.integers(-1000, 1000, (B, V)).astype(np.float32)   # many exact ties
    L[3, :] = 7.0
    L[4, 5] = np.nan
    out = DB(B * 4)
    check(hip.argmax_rows(out.p, dev(L).p, B, V), "argmax")
    got = host(out, np.int32, B)
    want = [orc.lib.orc_argmax(fp(np.ascontiguousarray(L[b])), V) for b in range(B)]
    assert list(got) == want
    L2 = np.full((2, 10), 1.0, np.float32)
    L2[0, 0] = np.nan
    out2 = DB(8)
    check(hip.argmax_rows(out2.p, dev(L2).p, 2, 10), "argmax")
    assert list(host(out2, np.int32, 2)) == [0, 0]
    # rows are reduced in chunks of 4096: a NaN opening a chunk must not hide
    # that chunk's maximum, equal maxima in different chunks keep the first,
    # an all -inf row gives 0, and an odd row length (rows not 16-byte
    # aligned) takes the scalar path
    for V3 in (128256, 8197):
        L3 = rng.integers(-1000, 1000, (5, V3)).astype(np.float32)
        L3[0, 4096] = np.nan
        L3[0, 4100] = 5000.0
        L3[1, 1000] = 3000.0
        L3[1, V3 - 2] = 3000.0
        L3[2, :] = -np.inf
        L3[3, V3 - 1] = 4000.0
        L3[4, 0] = -np.inf
        L3[4, 1:] = np.nan
        out3 = DB(5 * 4)
        check(hip.argmax_rows(out3.p, dev(L3).p, 5, V3), "argmax")
        want3 = [orc.lib.orc_argmax(fp(np.ascontiguousarray(L3[b])), V3) for b in range(5)]
        assert want3[0] == 4100 and want3[1] == 1000 and want3[2] == 0 and want3[3] == V3 - 1 and want3[4] == 0
        assert list(host(out3, np.int32, 5)) == want3


def test_pack_batch_bitexact(orc):
    lib = load_library()
    rng = np.random.default_rng(21)
    for trial in range(30):
        B = int(rng.integers(1, 64))
        slot = rng.permutation(128)[:B].astype(np.int32)
        n_new = np.where(rng.random(B) < 0.6, 1, rng.integers(1, 64, B)).astype(np.int32)
        pos0 = rng.integers(0, 2048, B).astype(np.int32)
        if trial == 7:
            n_new[3 % B] = 0
        if trial == 8:
            pos0[0] = 2300
        stride, max_seq, cap = 75497472, 2304, 4096
        rc, want = orc.pack_batch(slot, pos0, n_new, max_seq, stride)
        T = max(int(n_new.sum()), 1)
        outs = [DB((B + 1) * 4), DB(cap * 4), DB(cap * 4), DB(B * 8), DB(B * 4), DB(16)]
        r = lib.slate_hip_pack_batch(dev(slot).p, dev(pos0).p, dev(n_new).p, B, max_seq, stride, cap,
                                     *[o.p for o in outs])
        check(r, "pack_batch")
        status = host(outs[5], np.int32, 4)[0]
        if rc < 0:
            assert status == rc
            continue
        assert status == 0
        got = dict(tok_off=host(outs[0], np.int32, B + 1), tok2seq=host(outs[1], np.int32, T),
                   tok_pos=host(outs[2], np.int32, T), kv_base=host(outs[3], np.int64, B),
                   last_tok=host(outs[4], np.int32, B))
        for k in want:
            assert np.array_equal(got[k], want[k][:len(got[k])]), k


# ------------------------------------------------------------ attention
@pytest.mark.parametrize("hd,Hq,Hkv,extra", [(128, 32, 8, 0), (16, 4, 2, 0), (64, 8, 8, 0), (128, 64, 8, 0),
                                              (64, 32, 4, 0), (32, 8, 4, 0), (128, 32, 8, 70), (64, 8, 8, 70)])
def test_attention_ragged_vs_oracle(hip, orc, hd, Hq, Hkv, extra):
    """Per-token GQA attention over ragged per-sequence caches, one query per
    token (decode) and several consecutive queries of one sequence (prefill
    chunk), lengths across chunk boundaries.  `extra` adds a 70-token prompt
    chunk (launches of more than 64 query tokens take the phased kernel)."""
    lib = load_library()
    rng = np.random.default_rng(hd + Hq)
    max_seq = 4352
    lens = [1, 2, 255, 256, 257, 1000, 4097, 64]
    nslot = len(lens)
    head_stride = max_seq * hd
    slot_stride = Hkv * head_stride
    Kp = rng.normal(0, 1, nslot * slot_stride).astype(np.float32)
    Vp = rng.normal(0, 1, nslot * slot_stride).astype(np.float32)
    tok2seq, tok_pos = [], []
    for b, L in enumerate(lens):
        tok2seq.append(b)
        tok_pos.append(L - 1)
    tok2seq += [5, 5, 5]               # a prefill chunk: positions 10..12 of sequence 5
    tok_pos += [10, 11, 12]
    tok2seq += [6] * extra             # positions 300.. of sequence 6
    tok_pos += list(range(300, 300 + extra))
    T = len(tok2seq)
    kv_base = (np.arange(nslot, dtype=np.int64)[::-1] * slot_stride).copy()   # slot b -> nslot-1-b
    q = rng.normal(0, 1, (T, Hq * hd)).astype(np.float32)
    out = DB(T * Hq * hd * 4)
    r = lib.slate_hip_attention_ragged(out.p, dev(q).p, dev(Kp).p, dev(Vp).p,
                                       dev(np.array(tok2seq, np.int32)).p, dev(np.array(tok_pos, np.int32)).p,
                                       dev(kv_base).p, T, Hq, Hkv, hd, head_stride, max_seq)
    check(r, "attention_ragged")
    got = host(out, np.float32, (T, Hq * hd))
    Kp = Kp.reshape(nslot, Hkv, max_seq, hd)
    Vp = Vp.reshape(nslot, Hkv, max_seq, hd)
    for t in range(T):
        s = nslot - 1 - tok2seq[t]
        L = tok_pos[t] + 1
        Kc = np.ascontiguousarray(Kp[s, :, :L].transpose(1, 0, 2).reshape(L, Hkv * hd))
        Vc = np.ascontiguousarray(Vp[s, :, :L].transpose(1, 0, 2).reshape(L, Hkv * hd))
        want = np.empty(Hq * hd, np.float32)
        sc = np.empty(L, np.float32)
        orc.lib.orc_attention_multihead(fp(want), fp(np.ascontiguousarray(q[t])), fp(Kc), fp(Vc), fp(sc),
                                        L, Hq, Hkv, hd)
        assert np.max(np.abs(got[t] - want)) < 1e-5, (t, L)


def test_attention_ragged_full_size_lognormal(hip, orc):
    """The ragged-attention configuration end to end: 64 sequences, 32 q / 8
    kv heads, head_dim 128, lengths clip(round(exp(N(ln 1024, 1))), 16,
    16384) with one sequence at 16384 (64 key chunks merged), one query per
    sequence.  Each sequence's query and its new key are rotated at the
    sequence's own position p = L - 1 (rope_rows, llama_infer.c:77-92) and
    the new K/V row is appended at p (llama_infer.c:170-174) before the
    attention over 0..p.  K/V (2 x 4.3 GB) are generated on the device; the
    rotations are checked bit for bit, and the shortest, the longest and four
    random sequences against the oracle on the rows they read."""
    lib = load_library()
    rng = np.random.default_rng(0xC3)
    B, Hq, Hkv, hd, theta = 64, 32, 8, 128, 10000.0
    L = np.clip(np.round(np.exp(rng.normal(np.log(1024.0), 1.0, B))), 16, 16384).astype(np.int64)
    L[int(rng.integers(B))] = 16384
    max_seq = int(L.max())
    head_stride = max_seq * hd
    slot = Hkv * head_stride
    Kp, Vp = DB(B * slot * 4), DB(B * slot * 4)
    check(lib.slate_hip_synth_f32(Kp.p, B * slot, 11, 1.0), "synth K")
    check(lib.slate_hip_synth_f32(Vp.p, B * slot, 12, 1.0), "synth V")
    tok_pos = (L - 1).astype(np.int32)
    pos_d = dev(tok_pos)
    q_raw = rng.normal(0, 1, (B, Hq * hd)).astype(np.float32)
    k_raw = rng.normal(0, 1, (B, Hkv * hd)).astype(np.float32)
    v_new = rng.normal(0, 1, (B, Hkv * hd)).astype(np.float32)
    qd, kd = dev(q_raw), dev(k_raw)
    check(hip.rope_rows(qd.p, pos_d.p, B, Hq, hd, theta, max_seq), "rope q")
    check(hip.rope_rows(kd.p, pos_d.p, B, Hkv, hd, theta, max_seq), "rope k")
    q_rot, k_rot = host(qd, np.float32, (B, Hq * hd)), host(kd, np.float32, (B, Hkv * hd))
    want_q, want_k = q_raw.copy(), k_raw.copy()
    for b in range(B):
        orc.lib.orc_rope_row(fp(want_q[b]), Hq, hd, int(tok_pos[b]), theta)
        orc.lib.orc_rope_row(fp(want_k[b]), Hkv, hd, int(tok_pos[b]), theta)
    assert np.array_equal(bits(q_rot), bits(want_q)) and np.array_equal(bits(k_rot), bits(want_k))
    # append the rotated key and the value at position p of every kv head
    for b in range(B):
        for h in range(Hkv):
            off = (b * slot + h * head_stride + int(tok_pos[b]) * hd) * 4
            lib.slate_hip_copy_h2d(C.c_void_p(Kp.ptr + off), k_rot[b, h * hd:].ctypes.data, hd * 4)
            lib.slate_hip_copy_h2d(C.c_void_p(Vp.ptr + off), v_new[b, h * hd:].ctypes.data, hd * 4)
    out = DB(B * Hq * hd * 4)
    kv_base = np.arange(B, dtype=np.int64) * slot
    check(lib.slate_hip_attention_ragged(out.p, qd.p, Kp.p, Vp.p, dev(np.arange(B, dtype=np.int32)).p,
                                         pos_d.p, dev(kv_base).p, B, Hq, Hkv, hd, head_stride, max_seq),
          "attention_ragged")
    got = host(out, np.float32, (B, Hq * hd))
    picks = {int(np.argmin(L)), int(np.argmax(L))} | {int(i) for i in rng.choice(B, 4, replace=False)}
    for b in sorted(picks):
        n = int(L[b])
        Kc = np.empty((Hkv, n, hd), np.float32)
        Vc = np.empty((Hkv, n, hd), np.float32)
        for h in range(Hkv):
            off = (b * slot + h * head_stride) * 4
            lib.slate_hip_copy_d2h(Kc[h].ctypes.data, C.c_void_p(Kp.ptr + off), n * hd * 4)
            lib.slate_hip_copy_d2h(Vc[h].ctypes.data, C.c_void_p(Vp.ptr + off), n * hd * 4)
        assert np.array_equal(bits(Kc[:, n - 1].reshape(-1)), bits(want_k[b]))
        assert np.array_equal(bits(Vc[:, n - 1].reshape(-1)), bits(v_new[b]))
        Kc = np.ascontiguousarray(Kc.transpose(1, 0, 2).reshape(n, Hkv * hd))
        Vc = np.ascontiguousarray(Vc.transpose(1, 0, 2).reshape(n, Hkv * hd))
        want = np.empty(Hq * hd, np.float32)
        sc = np.empty(n, np.float32)
        orc.lib.orc_attention_multihead(fp(want), fp(np.ascontiguousarray(want_q[b])), fp(Kc), fp(Vc), fp(sc),
                                        n, Hq, Hkv, hd)
        assert np.all(np.isfinite(got[b]))
        assert np.max(np.abs(got[b] - want)) < 1e-5, (b, n)
