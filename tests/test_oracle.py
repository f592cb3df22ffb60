"""The oracle (oracle/oracle.c) pinned against slate's own answers and the
mathematics.  CPU only.

Pins, per oracle function:
* golden.npz        -- outputs of slate's compiled C (tests/golden/make_golden.py)
* live reference    -- oracle/_ref where it is built (bit-for-bit)
* mathematics       -- IEEE half conversion (numpy), float64 brute force,
                       quantise/dequantise round trip, rotation invariants,
                       tie rules, brute-force packing.
"""
import ctypes as C

import numpy as np
import pytest

from oracle.pyoracle import OracleModel, bp, fp, ip
from slate_amd.synth import (dequantize_q4k, dequantize_q8_0, make_llama, pack_scales, quantize_q4k,
                             quantize_q8_0)
from tests.helpers import (N_GEN, N_SEQ, Q4, Q4_PROMPT, Q4_SEED, TINY, TINY_SEED, bits, relerr,
                           tensors_digest, tiny_prompts)


# ---------------------------------------------------------------- f16 / Q4_K
def test_f16_exhaustive_matches_ieee(orc):
    h = np.arange(65536, dtype=np.uint16)
    got = np.empty(h.size, np.float32)
    orc.lib.orc_f16_to_f32_n(fp(got), bp(h), h.size)
    want = h.view(np.float16).astype(np.float32)
    assert np.array_equal(bits(got), bits(want))


def test_scale_min_unpack_inverts_packing(orc):
    rng = np.random.default_rng(3)
    for _ in range(200):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        s = np.ascontiguousarray(pack_scales(sc, mn))
        for j in range(8):
            a, b = np.zeros(1, np.uint8), np.zeros(1, np.uint8)
            orc.lib.orc_q4k_scale_min(bp(s), j, a.ctypes.data_as(orc.lib.orc_q4k_scale_min.argtypes[2]),
                                      b.ctypes.data_as(orc.lib.orc_q4k_scale_min.argtypes[3]))
            assert (a[0], b[0]) == (sc[j], mn[j])


def test_dequant_matches_golden(orc, golden):
    raw = golden["q4k_raw"]
    got = orc.dequant_q4k(raw, raw.size // 144 * 256)
    assert np.array_equal(bits(got), bits(golden["q4k_deq"]))


def test_dequant_numpy_restatement_matches_golden(golden):
    M, K = golden["q4k_MK"]
    got = dequantize_q4k(golden["q4k_raw"], M, K).ravel()
    assert np.array_equal(bits(got), bits(golden["q4k_deq"]))


def test_quantize_dequantize_round_trip(orc):
    """A wrong nibble order or scale packing shows up as a large error."""
    rng = np.random.default_rng(5)
    W = rng.normal(0, 0.02, (8, 1024)).astype(np.float32)
    raw = np.frombuffer(quantize_q4k(W), np.uint8).copy()
    deq = orc.dequant_q4k(raw, W.size).reshape(W.shape)
    x = W.reshape(8, 4, 8, 32)
    step = (x.max(-1) - np.minimum(x.min(-1), 0)) / 15.0
    # error per element <= half a step plus the 6-bit code rounding of scale/min
    tol = np.repeat(step, 32, axis=-1).reshape(W.shape) * 1.6 + 2e-4
    assert np.all(np.abs(deq - W) <= tol)
    assert np.abs(deq - W).mean() < 0.2 * np.abs(W).mean()


def test_q4k_matvec_matches_golden(orc, golden):
    M, K = golden["q4k_MK"]
    Y = orc.q4k_matmul(golden["q4k_mv_raw"], golden["q4k_x"], M, K)
    assert np.array_equal(bits(Y), bits(golden["q4k_y"]))


def test_q4k_matvec_vs_float64(orc):
    """slate's test_gguf_q4k.c:60-90 method: dequant then dot in double."""
    rng = np.random.default_rng(7)
    M, K = 16, 4096
    W = rng.normal(0, 0.02, (M, K)).astype(np.float32)
    raw = np.frombuffer(quantize_q4k(W), np.uint8).copy()
    x = rng.normal(0, 1, (2, K)).astype(np.float32)
    Y = orc.q4k_matmul(raw, x, M, K)
    deq = orc.dequant_q4k(raw, M * K).reshape(M, K).astype(np.float64)
    ref = x.astype(np.float64) @ deq.T
    assert np.max(np.abs(Y - ref) / (np.abs(ref) + 1e-9)) < 1e-4
    assert relerr(Y, ref) < 1e-6


# ---------------------------------------------------------------------- Q8_0
def test_q8_dequant_matches_golden(orc, golden):
    raw = golden["q8_raw"]
    got = orc.dequant_q8_0(raw, raw.size // 34 * 32)
    assert np.array_equal(bits(got), bits(golden["q8_deq"]))
    M, K = golden["q8_MK"]
    assert np.array_equal(bits(dequantize_q8_0(raw, M, K).ravel()), bits(golden["q8_deq"]))


def test_q8_dequant_known_answer(orc):
    """slate's tests/test_quant.c:25-41: d = 0.1, q = i - 16 -> 0.1 * (i - 16)
    within 0.01; and d * q is one exact f32 product (19 significant bits)."""
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.1).tobytes(), np.uint8)
    blk[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    out = orc.dequant_q8_0(blk, 32)
    assert np.all(np.abs(out - 0.1 * (np.arange(32) - 16)) <= 0.01)
    exact = np.float64(np.float16(0.1)) * (np.arange(32) - 16)
    assert np.array_equal(out.astype(np.float64), exact)


def test_q8_matvec_matches_golden(orc, golden):
    M, K = golden["q8_MK"]
    Y = orc.q8_0_matmul(golden["q8_mv_raw"], golden["q8_x"], M, K)
    assert np.array_equal(bits(Y), bits(golden["q8_y"]))


def test_q8_matvec_vs_float64(orc):
    """slate's tests/test_q8_dot.c method (K=256, M=8, uniform values in
    [-1, 1]): the fast dot within rel 1e-4 of the dequantised float64 dot;
    plus a large-K case."""
    rng = np.random.default_rng(11)
    for M, K in ((8, 256), (16, 4096)):
        W = (rng.integers(-1000, 1001, (M, K)) / 1000.0).astype(np.float32)
        raw = np.frombuffer(quantize_q8_0(W), np.uint8).copy()
        x = (rng.integers(-1000, 1001, (2, K)) / 1000.0).astype(np.float32)
        Y = orc.q8_0_matmul(raw, x, M, K)
        deq = orc.dequant_q8_0(raw, M * K).reshape(M, K).astype(np.float64)
        assert np.abs(deq - W).max() <= np.abs(W).max() / 127 * 0.51 + 1e-6   # half a step
        ref = x.astype(np.float64) @ deq.T
        assert np.max(np.abs(Y - ref) / (np.abs(ref) + 1e-6)) < 1e-4
        assert relerr(Y, ref) < 1e-6


def test_q8_dot_lane_order_is_pinned(orc):
    """The eight-lane order is what makes the result bit-exact: a plain
    sequential float sum of the same products differs on some rows."""
    rng = np.random.default_rng(12)
    M, K = 64, 1024
    raw = rng.integers(0, 256, (M * K // 32, 34), dtype=np.uint8)
    raw[:, 1] &= 0x3B
    raw = np.ascontiguousarray(raw.reshape(-1))
    x = rng.normal(0, 1, K).astype(np.float32)
    Y = orc.q8_0_matmul(raw, x, M, K)[0]
    deq = orc.dequant_q8_0(raw, M * K).reshape(M, K)
    seq = np.zeros(M, np.float32)
    for k in range(K):
        seq = (seq + deq[:, k] * x[k]).astype(np.float32)
    assert not np.array_equal(bits(Y), bits(seq))
    ref = deq.astype(np.float64) @ x.astype(np.float64)
    assert relerr(Y, ref) < 1e-5


def test_q8_llama_equals_its_dequantised_f32_model(orc):
    """The corrected dtype dispatch: a model whose linears are Q8_0 gives the
    logits of the same model with those weights dequantised to f32 (the f32
    path sums in another order, so within float rounding)."""
    t = make_llama(Q4, Q4_SEED, quant="q8_0", output_quant="q8_0")
    f = {}
    for name, (a, dt, shp) in t.items():
        f[name] = ((orc.dequant_q8_0(a, shp[0] * shp[1]).reshape(shp), 0, shp) if dt == 16 else (a, dt, shp))
    s8, sf = OracleModel(orc, Q4, t).session(), OracleModel(orc, Q4, f).session()
    rc8, l8 = s8.prefill(Q4_PROMPT)
    rcf, lf = sf.prefill(Q4_PROMPT)
    assert rc8 == rcf == 0
    for k in range(6):
        assert relerr(l8, lf) < 1e-5
        tok = int(np.argmax(lf))
        rc8, l8 = s8.decode(tok)
        rcf, lf = sf.decode(tok)
    assert relerr(l8, lf) < 1e-5


# ------------------------------------------------------------ vtable KATs
def test_backend_known_answers(orc, golden):
    """slate's tests/test_backend.c cases, bit-for-bit against slate's output
    and within its tolerances of the float64 definition."""
    g = golden
    y = np.empty(7, np.float32)
    orc.lib.orc_matvec(fp(y), fp(g["kat_matvec_A"]), fp(g["kat_matvec_x"]), 7, 11)
    assert np.array_equal(bits(y), bits(g["kat_matvec_y"]))
    ref = g["kat_matvec_A"].reshape(7, 11).astype(np.float64) @ g["kat_matvec_x"].astype(np.float64)
    assert np.max(np.abs(y - ref)) < 1e-4

    C = np.empty(24, np.float32)
    orc.lib.orc_linear_batch(fp(C), fp(g["kat_lb_X"]), fp(g["kat_lb_W"]), 4, 8, 6)
    assert np.array_equal(bits(C), bits(g["kat_lb_C"]))
    ref = g["kat_lb_X"].reshape(4, 8).astype(np.float64) @ g["kat_lb_W"].reshape(8, 6).astype(np.float64)
    assert np.max(np.abs(C.reshape(4, 6) - ref)) < 1e-4

    yr = np.empty(16, np.float32)
    orc.lib.orc_rmsnorm_row(fp(yr), fp(g["kat_rms_x"]), fp(g["kat_rms_w"]), 16, 1e-5)
    assert np.array_equal(bits(yr), bits(g["kat_rms_y"]))

    ys = np.empty(24, np.float32)
    orc.lib.orc_silu_mul(fp(ys), fp(g["kat_silu_g"]), fp(g["kat_silu_u"]), 24)
    assert np.array_equal(bits(ys), bits(g["kat_silu_y"]))
    gg = g["kat_silu_g"].astype(np.float64)
    assert np.max(np.abs(ys - gg / (1 + np.exp(-gg)) * g["kat_silu_u"])) < 1e-5

    o = np.empty(16, np.float32)
    sc = np.empty(5, np.float32)
    orc.lib.orc_attention_step(fp(o), fp(g["kat_att_q"]), fp(g["kat_att_K"]), fp(g["kat_att_V"]), fp(sc), 5, 16)
    assert np.array_equal(bits(o), bits(g["kat_att_out"]))


@pytest.mark.parametrize("D", [37, 4096])
def test_rmsnorm_silu_random_match_golden(orc, golden, D):
    g = golden
    y = np.empty(D, np.float32)
    orc.lib.orc_rmsnorm_row(fp(y), fp(g[f"rms{D}_x"]), fp(g[f"rms{D}_w"]), D, 1e-5)
    assert np.array_equal(bits(y), bits(g[f"rms{D}_y"]))
    x = g[f"rms{D}_x"].astype(np.float64)
    ref = x * g[f"rms{D}_w"] / np.sqrt((x * x).mean() + 1e-5)
    assert np.max(np.abs(y - ref)) < 1e-5
    s = np.empty(D, np.float32)
    orc.lib.orc_silu_mul(fp(s), fp(g[f"silu{D}_g"]), fp(g[f"rms{D}_w"]), D)
    assert np.array_equal(bits(s), bits(g[f"silu{D}_y"]))


def test_attention_step_random_matches_golden(orc, golden):
    g = golden
    L, D = g["att64_K"].shape
    o = np.empty(D, np.float32)
    sc = np.empty(L, np.float32)
    orc.lib.orc_attention_step(fp(o), fp(g["att64_q"]), fp(g["att64_K"]), fp(g["att64_V"]), fp(sc), L, D)
    assert np.array_equal(bits(o), bits(g["att64_out"]))
    s = g["att64_K"].astype(np.float64) @ g["att64_q"] / np.sqrt(D)
    p = np.exp(s - s.max())
    p /= p.sum()
    assert np.max(np.abs(o - p @ g["att64_V"])) < 1e-5


# ------------------------------------------------------------ RoPE / GQA
def test_rope_matches_golden(orc, golden):
    x, y, pos = golden["rope_x"], golden["rope_y"], golden["rope_pos"]
    for r, p in enumerate(pos):
        row = np.ascontiguousarray(x[r])
        orc.lib.orc_rope_row(fp(row), 4, 128, int(p), 10000.0)
        assert np.array_equal(bits(row), bits(y[r])), f"position {p}"


def test_rope_invariants(orc):
    """Rotation: pairwise norms preserved, p=0 is the identity, and rotating
    by -p undoes +p (slate's test_rope.c:71-90 check, tol 1e-4)."""
    rng = np.random.default_rng(11)
    x = rng.normal(0, 1, 2 * 64).astype(np.float32)
    r0 = x.copy()
    orc.lib.orc_rope_row(fp(r0), 2, 64, 0, 10000.0)
    assert np.array_equal(r0, x)
    for p in (1, 17, 1000, 8191):
        r = x.copy()
        orc.lib.orc_rope_row(fp(r), 2, 64, p, 10000.0)
        a, b = x.reshape(2, 2, 32), r.reshape(2, 2, 32)
        assert np.allclose(np.hypot(a[:, 0], a[:, 1]), np.hypot(b[:, 0], b[:, 1]), rtol=1e-5)
        # first pair rotates by exactly p radians (inv_freq = 1 for i = 0)
        ang = np.arctan2(b[0, 1, 0], b[0, 0, 0]) - np.arctan2(a[0, 1, 0], a[0, 0, 0])
        assert abs(np.remainder(ang - p + np.pi, 2 * np.pi) - np.pi) < 1e-3
        orc.lib.orc_rope_row(fp(r), 2, 64, -p, 10000.0)
        assert np.max(np.abs(r - x)) < 1e-4


def test_gqa_attention_matches_golden_and_float64(orc, golden):
    L, Hq, Hkv, hd = golden["gqa_dims"]
    o = np.empty(Hq * hd, np.float32)
    sc = np.empty(L, np.float32)
    orc.lib.orc_attention_multihead(fp(o), fp(golden["gqa_q"]), fp(golden["gqa_K"]), fp(golden["gqa_V"]),
                                    fp(sc), L, Hq, Hkv, hd)
    assert np.array_equal(bits(o), bits(golden["gqa_out"]))
    q = golden["gqa_q"].reshape(Hq, hd).astype(np.float64)
    K = golden["gqa_K"].reshape(L, Hkv, hd).astype(np.float64)
    V = golden["gqa_V"].reshape(L, Hkv, hd).astype(np.float64)
    for h in range(Hq):
        kv = h // (Hq // Hkv)
        s = K[:, kv] @ q[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.max(np.abs(o[h * hd:(h + 1) * hd] - p @ V[:, kv])) < 1e-5


# ------------------------------------------------------------ argmax / packing
def test_argmax_ties_and_nan(orc):
    cases = [([1, 3, 3, 2], 1), ([5, 5, 5], 0), ([-1, -1], 0), ([np.nan, 9, 9], 0),
             ([0, np.nan, 2, 2], 2), ([-np.inf, -3], 1)]
    for v, want in cases:
        a = np.array(v, np.float32)
        assert orc.lib.orc_argmax(fp(a), len(a)) == want
    rng = np.random.default_rng(2)
    a = rng.integers(0, 50, 10000).astype(np.float32)
    assert orc.lib.orc_argmax(fp(a), a.size) == int(np.argmax(a))


def pack_brute(slot, pos0, n_new, max_seq, stride):
    toks = []
    for b, (s, p, n) in enumerate(zip(slot, pos0, n_new)):
        if n < 1 or p < 0 or s < 0:
            return -1, None
        if p + n > max_seq:
            return -2, None
        toks += [(b, p + i) for i in range(n)]
    off = np.concatenate([[0], np.cumsum(n_new)]).astype(np.int32)
    return len(toks), dict(tok_off=off, tok2seq=np.array([t[0] for t in toks], np.int32),
                           tok_pos=np.array([t[1] for t in toks], np.int32),
                           kv_base=np.array(slot, np.int64) * stride, last_tok=(off[1:] - 1).astype(np.int32))


def test_pack_batch_brute_force(orc):
    rng = np.random.default_rng(9)
    for trial in range(200):
        B = int(rng.integers(1, 40))
        slot = rng.permutation(64)[:B].astype(np.int32)
        n_new = np.where(rng.random(B) < 0.7, 1, rng.integers(1, 300, B)).astype(np.int32)
        pos0 = rng.integers(0, 2048, B).astype(np.int32)
        if trial % 17 == 0:
            n_new[rng.integers(B)] = 0
        rc, got = orc.pack_batch(slot, pos0, n_new, 2304, 75497472)
        want_rc, want = pack_brute(slot, pos0, n_new, 2304, 75497472)
        assert rc == want_rc
        if rc > 0:
            for k, v in want.items():
                assert np.array_equal(got[k][:len(v)], v), k


# ------------------------------------------------------------ whole model
def test_tiny_llama_matches_golden_streams(orc, golden):
    """Config-1 model (f32, GQA): greedy streams and every step's logits are
    bit-identical to slate's slate_llama_prefill / slate_llama_decode_step."""
    t = make_llama(TINY, TINY_SEED, quant="f32")
    if tensors_digest(t) != str(golden["tiny_digest"]):
        pytest.fail("synthetic weights differ from the ones the fixtures were made with")
    m = OracleModel(orc, TINY, t)
    for s, prompt in enumerate(tiny_prompts()):
        sess = m.session()
        rc, lg = sess.prefill(prompt)
        assert rc == 0
        for k in range(N_GEN):
            assert np.array_equal(bits(lg), bits(golden["tiny_logits"][s, k])), (s, k)
            tok = orc.lib.orc_argmax(fp(lg), TINY.vocab)
            assert tok == golden["tiny_streams"][s, k]
            rc, lg = sess.decode(tok)
            assert rc == 0
        assert sess.position == len(prompt) + N_GEN


def test_q4k_llama_matches_golden(orc, golden):
    t = make_llama(Q4, Q4_SEED, quant="q4k", output_quant="f32")
    if tensors_digest(t) != str(golden["q4_digest"]):
        pytest.fail("synthetic weights differ from the ones the fixtures were made with")
    m = OracleModel(orc, Q4, t)
    sess = m.session()
    rc, lg = sess.prefill(Q4_PROMPT)
    assert rc == 0
    for k in range(8):
        assert np.array_equal(bits(lg), bits(golden["q4_logits"][k]))
        tok = orc.lib.orc_argmax(fp(lg), Q4.vocab)
        assert tok == golden["q4_stream"][k]
        rc, lg = sess.decode(tok)
    assert np.array_equal(bits(lg), bits(golden["q4_logits"][8]))


def test_session_error_codes(orc):
    """llama_infer.c:144-145: cache full -> -2, bad token -> -3."""
    shape = TINY.__class__(**{**TINY.__dict__, "max_seq": 4})
    t = make_llama(shape, 1, quant="f32")
    m = OracleModel(orc, shape, t)
    s = m.session()
    assert s.decode(-1)[0] == -3
    assert s.decode(shape.vocab)[0] == -3
    for i in range(4):
        assert s.decode(i)[0] == 0
    assert s.decode(0)[0] == -2
    assert s.position == 4


# ------------------------------------------------------------ live reference
def test_oracle_bitexact_with_live_reference(orc, ref):
    """Where slate's sources are mounted: random cases of every restated
    function, bit-for-bit against the compiled reference."""
    rng = np.random.default_rng(1234)
    W = rng.normal(0, 0.02, (32, 1024)).astype(np.float32)
    raw = np.frombuffer(quantize_q4k(W), np.uint8).copy()
    a = orc.dequant_q4k(raw, W.size)
    b = np.empty(W.size, np.float32)
    ref.lib.slate_dequant_q4_k(fp(b), bp(raw), W.size)
    assert np.array_equal(bits(a), bits(b))
    x = rng.normal(0, 1, 1024).astype(np.float32)
    y1 = orc.q4k_matmul(raw, x, 32, 1024)[0]
    y2 = np.empty(32, np.float32)
    ref.lib.slate_q4_k_matvec(fp(y2), bp(raw), fp(x), 32, 1024)
    assert np.array_equal(bits(y1), bits(y2))
    for D in (8, 13, 100):
        xx = rng.normal(0, 1, D).astype(np.float32)
        ww = rng.normal(0, 1, D).astype(np.float32)
        o1, o2 = np.empty(D, np.float32), np.empty(D, np.float32)
        orc.lib.orc_rmsnorm_row(fp(o1), fp(xx), fp(ww), D, 1e-6)
        ref.rmsnorm_row(fp(o2), fp(xx), fp(ww), D, 1e-6)
        assert np.array_equal(bits(o1), bits(o2))
        orc.lib.orc_silu_mul(fp(o1), fp(xx), fp(ww), D)
        ref.silu_mul(fp(o2), fp(xx), fp(ww), D)
        assert np.array_equal(bits(o1), bits(o2))
    A = rng.normal(0, 1, (33, 300)).astype(np.float32)
    v = rng.normal(0, 1, 300).astype(np.float32)
    y1, y2 = np.empty(33, np.float32), np.empty(33, np.float32)
    orc.lib.orc_matvec(fp(y1), fp(A), fp(v), 33, 300)
    ref.matvec(fp(y2), fp(A), fp(v), 33, 300)
    assert np.array_equal(bits(y1), bits(y2))
    r1 = rng.normal(0, 1, 8 * 64).astype(np.float32)
    r2 = r1.copy()
    orc.lib.orc_rope_row(fp(r1), 8, 64, 4321, 500000.0)
    ref.lib.ref_rope_inplace_row(fp(r2), 8, 64, 4321, 500000.0)
    assert np.array_equal(bits(r1), bits(r2))
    raw8 = np.frombuffer(quantize_q8_0(W), np.uint8).copy()
    a = orc.dequant_q8_0(raw8, W.size)
    ref.lib.slate_dequant_q8_0(fp(b), bp(raw8), W.size)
    assert np.array_equal(bits(a), bits(b))
    y1 = orc.q8_0_matmul(raw8, x, 32, 1024)[0]
    y2 = np.empty(32, np.float32)
    ref.lib.slate_q8_0_matvec(fp(y2), bp(raw8), fp(x), 32, 1024)
    assert np.array_equal(bits(y1), bits(y2))
    h = np.arange(0, 31744, 7, dtype=np.uint16)      # finite positive halves
    assert all(np.float32(orc.lib.orc_f16_to_f32(int(v))).view(np.uint32) ==
               np.float32(ref.lib.slate_f16_to_f32(int(v))).view(np.uint32) for v in h)


def test_oracle_set_state_continues_a_session(orc):
    """orc_session_set_state: a fresh session loaded with another session's
    K/V and position decodes the following tokens bit for bit as that
    session does (the state is the whole of a session's context); a
    planted mistake (the position one short) changes the logits."""
    t = make_llama(Q4, Q4_SEED, quant="q4k", output_quant="f32")
    m = OracleModel(orc, Q4, t)
    a = m.session()
    rc, _ = a.prefill(Q4_PROMPT)
    assert rc == 0
    K, V = a.kv()
    b, c = m.session(), m.session()
    assert b.set_state(K, V, a.position) == 0 and b.position == a.position
    assert c.set_state(K, V, a.position - 1) == 0
    for tok in (3, 41, 9):
        _, la = a.decode(tok)
        _, lb = b.decode(tok)
        assert np.array_equal(bits(la), bits(lb))
    _, lc = c.decode(3)
    assert not np.array_equal(bits(lc), bits(m.session().prefill(np.append(Q4_PROMPT, 3))[1]))
    assert b.set_state(K, V, Q4.max_seq + 1) == -1


def test_reference_parallel_decode_equals_sequential(orc, ref, tmp_path):
    """ref_decode_sessions_parallel (sessions spread over slate's threadpool)
    gives each session the bits of its own slate_llama_decode_step, and the
    oracle started from the same K/V states gives them too."""
    from oracle.pyoracle import RefLlama
    from slate_amd.synth import write_llama_gguf
    t = make_llama(Q4, Q4_SEED, quant="q4k", output_quant="f32")
    path = str(tmp_path / "q4.gguf")
    write_llama_gguf(path, Q4, t)
    rm = RefLlama(ref, path)
    om = OracleModel(orc, Q4, t)
    try:
        rng = np.random.default_rng(5)
        prompts = [rng.integers(0, Q4.vocab, n).astype(np.int32) for n in (3, 9, 1, 5, 12)]
        par, seq, orcs = [rm.session() for _ in prompts], [rm.session() for _ in prompts], []
        for p, s1, s2 in zip(prompts, par, seq):
            assert s1.prefill(p)[0] == 0 and s2.prefill(p)[0] == 0
            o = om.session()
            assert o.prefill(p)[0] == 0
            orcs.append(o)
        toks = np.array([5, 1, 60, 7, 33], np.int32)
        n = len(prompts)
        out = np.empty((n, Q4.vocab), np.float32)
        rc = np.zeros(n, np.int32)
        arr = (C.c_void_p * n)(*[s.h for s in par])
        ref.lib.ref_decode_sessions_parallel(arr, toks.ctypes.data_as(C.POINTER(C.c_int32)), n, fp(out),
                                             rc.ctypes.data_as(C.POINTER(C.c_int32)))
        assert not rc.any() and ref.lib.ref_pool_threads() >= 1
        for i in range(n):
            want = seq[i].decode(int(toks[i]))[1]
            assert np.array_equal(bits(out[i]), bits(want))
            assert np.array_equal(bits(orcs[i].decode(int(toks[i]))[1]), bits(want))
        for s in par + seq:
            s.free()
    finally:
        rm.close()
