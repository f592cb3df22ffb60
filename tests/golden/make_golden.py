#!/usr/bin/env python3
"""Write tests/golden/golden.npz from slate's own C code.

The outputs come from oracle/_ref/libslate_ref.so (slate's sources compiled
where they lie, by `make -C oracle`), so the fixtures are the reference's
answers, not this project's.  Inputs are either the known-answer patterns of
slate's tests/test_backend.c (reproduced as formulas) or seeded random data.
Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle.pyoracle import Ref, RefLlama, bp, fp  # noqa: E402
from slate_amd.synth import make_llama, write_llama_gguf  # noqa: E402
from tests.helpers import (N_GEN, N_SEQ, Q4, Q4_PROMPT, Q4_SEED, TINY, TINY_SEED,  # noqa: E402
                           tensors_digest, tiny_prompts)

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")

def q4k_edge_blocks(rng, n):
    """Random blocks with edge-case headers (zero, subnormal, max f16) and
    extreme scale/min codes."""
    b = rng.integers(0, 256, (n, 144), dtype=np.uint8)
    heads = [0x0000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0x8001, 0xFBFF, 0x1C00, 0x2E66]
    for i in range(n):
        d = heads[i % len(heads)]
        dm = heads[(i * 3 + 1) % len(heads)]
        b[i, 0:2] = np.frombuffer(np.uint16(d).tobytes(), np.uint8)
        b[i, 2:4] = np.frombuffer(np.uint16(dm).tobytes(), np.uint8)
        if i % 7 == 0:
            b[i, 4:16] = 0xFF                  # every 6-bit code = 63
        if i % 11 == 0:
            b[i, 4:16] = 0x00
        if i % 5 == 0:
            b[i, 16:] = 0xFF if i % 2 else 0x00
    return b


def main():
    ref = Ref()
    rng = np.random.default_rng(20261201)
    g = {}

    # ---- Q4_K: dequant and matvec (quant.c:168-313) -------------------------
    M, K = 6, 2048
    blocks = q4k_edge_blocks(rng, M * K // 256)
    raw = np.ascontiguousarray(blocks.reshape(-1))
    deq = np.empty(M * K, np.float32)
    ref.lib.slate_dequant_q4_k(fp(deq), bp(raw), M * K)
    # tame headers for the matvec so results stay finite
    mv_blocks = blocks.copy()
    mv_blocks[:, 1] &= 0x3B
    mv_blocks[:, 3] &= 0x3B
    mv_raw = np.ascontiguousarray(mv_blocks.reshape(-1))
    X = rng.normal(0, 1, (3, K)).astype(np.float32)
    Y = np.empty((3, M), np.float32)
    for i in range(3):
        y = np.empty(M, np.float32)
        ref.lib.slate_q4_k_matvec(fp(y), bp(mv_raw), fp(np.ascontiguousarray(X[i])), M, K)
        Y[i] = y
    g.update(q4k_raw=raw, q4k_deq=deq, q4k_mv_raw=mv_raw, q4k_x=X, q4k_y=Y, q4k_MK=np.array([M, K]))

    # ---- backend primitives on test_backend.c's input patterns --------------
    i = np.arange(7 * 11)
    A = ((i * 13 + 5) % 17).astype(np.float32) * np.float32(0.05) - np.float32(0.4)
    x = np.arange(11).astype(np.float32) * np.float32(0.1) - np.float32(0.5)
    y = np.empty(7, np.float32)
    ref.matvec(fp(y), fp(A), fp(x), 7, 11)
    g.update(kat_matvec_A=A, kat_matvec_x=x, kat_matvec_y=y)
    Xb = ((np.arange(32) * 7) % 13).astype(np.float32) * np.float32(0.1) - np.float32(0.6)
    Wb = ((np.arange(48) * 5) % 11).astype(np.float32) * np.float32(0.08) - np.float32(0.4)
    Cb = np.empty(24, np.float32)
    ref.linear_batch(fp(Cb), fp(Xb), fp(Wb), 4, 8, 6)
    g.update(kat_lb_X=Xb, kat_lb_W=Wb, kat_lb_C=Cb)
    d = np.arange(16)
    xr = (d - 8).astype(np.float32) * np.float32(0.3)
    wr = np.float32(0.5) + d.astype(np.float32) * np.float32(0.05)
    yr = np.empty(16, np.float32)
    ref.rmsnorm_row(fp(yr), fp(xr), fp(wr), 16, 1e-5)
    g.update(kat_rms_x=xr, kat_rms_w=wr, kat_rms_y=yr)
    h = np.arange(24)
    gg = (h - 12).astype(np.float32) * np.float32(0.4)
    uu = (h + 1).astype(np.float32) * np.float32(0.1)
    ys = np.empty(24, np.float32)
    ref.silu_mul(fp(ys), fp(gg), fp(uu), 24)
    g.update(kat_silu_g=gg, kat_silu_u=uu, kat_silu_y=ys)
    q = (np.arange(16) - 8).astype(np.float32) * np.float32(0.1)
    Ka = ((np.arange(80) * 7) % 13).astype(np.float32) * np.float32(0.05)
    Va = ((np.arange(80) * 5) % 11).astype(np.float32) * np.float32(0.07)
    sc = np.empty(5, np.float32)
    oa = np.empty(16, np.float32)
    ref.attention_step(fp(oa), fp(q), fp(Ka), fp(Va), fp(sc), 5, 16)
    g.update(kat_att_q=q, kat_att_K=Ka, kat_att_V=Va, kat_att_out=oa)
    # larger random cases (D not a multiple of 8 exercises the scalar tails)
    for D in (37, 4096):
        xx = rng.normal(0, 1, D).astype(np.float32)
        ww = rng.normal(1, 0.1, D).astype(np.float32)
        yy = np.empty(D, np.float32)
        ref.rmsnorm_row(fp(yy), fp(xx), fp(ww), D, 1e-5)
        g[f"rms{D}_x"], g[f"rms{D}_w"], g[f"rms{D}_y"] = xx, ww, yy
        g_ = rng.normal(0, 3, D).astype(np.float32)
        s_ = np.empty(D, np.float32)
        ref.silu_mul(fp(s_), fp(g_), fp(ww), D)
        g[f"silu{D}_g"], g[f"silu{D}_y"] = g_, s_
    L, D = 64, 128
    q = rng.normal(0, 1, D).astype(np.float32)
    Kr = rng.normal(0, 1, (L, D)).astype(np.float32)
    Vr = rng.normal(0, 1, (L, D)).astype(np.float32)
    o = np.empty(D, np.float32)
    sc = np.empty(L, np.float32)
    ref.attention_step(fp(o), fp(q), fp(Kr), fp(Vr), fp(sc), L, D)
    g.update(att64_q=q, att64_K=Kr, att64_V=Vr, att64_out=o)

    # ---- RoPE (llama_infer.c:77-92) and GQA attention (:97-129) ------------
    pos = np.array([0, 1, 7, 1000, 2047, 16383], np.int32)
    rx = rng.normal(0, 1, (len(pos), 4 * 128)).astype(np.float32)
    ry = rx.copy()
    for r, p in enumerate(pos):
        row = np.ascontiguousarray(ry[r])
        ref.lib.ref_rope_inplace_row(fp(row), 4, 128, int(p), 10000.0)
        ry[r] = row
    g.update(rope_pos=pos, rope_x=rx, rope_y=ry)
    L, Hq, Hkv, hd = 37, 8, 2, 16
    q = rng.normal(0, 1, Hq * hd).astype(np.float32)
    Kc = rng.normal(0, 1, (L, Hkv * hd)).astype(np.float32)
    Vc = rng.normal(0, 1, (L, Hkv * hd)).astype(np.float32)
    o = np.empty(Hq * hd, np.float32)
    sc = np.empty(L, np.float32)
    ref.lib.ref_attention_multihead(fp(o), fp(q), fp(Kc), fp(Vc), fp(sc), L, Hq, Hkv, hd)
    g.update(gqa_q=q, gqa_K=Kc, gqa_V=Vc, gqa_out=o, gqa_dims=np.array([L, Hq, Hkv, hd]))

    # ---- whole model: tiny f32 LLaMA, continuous batch of 4 sequences -------
    t = make_llama(TINY, TINY_SEED, quant="f32")
    path = "/tmp/slate_amd_golden_tiny.gguf"
    write_llama_gguf(path, TINY, t)
    prompts = tiny_prompts()
    lens = np.array([len(p) for p in prompts])
    m = RefLlama(ref, path)
    streams = np.zeros((N_SEQ, N_GEN), np.int32)
    logits = np.zeros((N_SEQ, N_GEN, TINY.vocab), np.float32)
    for s in range(N_SEQ):
        sess = m.session()
        rc, lg = sess.prefill(prompts[s])
        assert rc == 0
        for k in range(N_GEN):
            logits[s, k] = lg
            tok = int(np.argmax(lg))           # numpy argmax: first maximum, as sampling.c:14-18
            streams[s, k] = tok
            rc, lg = sess.decode(tok)
            assert rc == 0
        sess.free()
    m.close()
    g.update(tiny_digest=np.array(tensors_digest(t)), tiny_prompt_lens=lens.astype(np.int32),
             tiny_prompts=np.concatenate(prompts), tiny_streams=streams, tiny_logits=logits)

    # ---- small Q4_K LLaMA (slate's test_llama_infer_q4k shape, with GQA) ----
    t = make_llama(Q4, Q4_SEED, quant="q4k", output_quant="f32")
    path = "/tmp/slate_amd_golden_q4.gguf"
    write_llama_gguf(path, Q4, t)
    m = RefLlama(ref, path)
    sess = m.session()
    rc, lg = sess.prefill(Q4_PROMPT)
    assert rc == 0
    q4_logits = [lg]
    q4_stream = []
    for k in range(8):
        tok = int(np.argmax(lg))
        q4_stream.append(tok)
        rc, lg = sess.decode(tok)
        q4_logits.append(lg)
    sess.free()
    m.close()
    g.update(q4_digest=np.array(tensors_digest(t)), q4_stream=np.array(q4_stream, np.int32),
             q4_logits=np.stack(q4_logits))

    # ---- Q8_0: dequant, dot and matvec (quant.c:12-25, 64-133) --------------
    # own generator, so the vectors above stay what they were
    rng8 = np.random.default_rng(20261202)
    M8, K8 = 5, 1024
    b8 = rng8.integers(0, 256, (M8 * K8 // 32, 34), dtype=np.uint8)
    heads = [0x0000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x2E66, 0x8001, 0xAE66, 0x1C00, 0x7BFF]
    for i in range(b8.shape[0]):
        b8[i, 0:2] = np.frombuffer(np.uint16(heads[i % len(heads)]).tobytes(), np.uint8)
        if i % 6 == 0:
            b8[i, 2:] = 0x80                   # every q = -128
        if i % 9 == 0:
            b8[i, 2:] = 0x7F
    raw8 = np.ascontiguousarray(b8.reshape(-1))
    deq8 = np.empty(M8 * K8, np.float32)
    ref.lib.slate_dequant_q8_0(fp(deq8), bp(raw8), M8 * K8)
    mv8 = b8.copy()
    mv8[:, 1] &= 0x3B                          # finite results for the matvec
    mv8_raw = np.ascontiguousarray(mv8.reshape(-1))
    X8 = rng8.normal(0, 1, (3, K8)).astype(np.float32)
    Y8 = np.empty((3, M8), np.float32)
    for i in range(3):
        y = np.empty(M8, np.float32)
        ref.lib.slate_q8_0_matvec(fp(y), bp(mv8_raw), fp(np.ascontiguousarray(X8[i])), M8, K8)
        Y8[i] = y
    g.update(q8_raw=raw8, q8_deq=deq8, q8_mv_raw=mv8_raw, q8_x=X8, q8_y=Y8, q8_MK=np.array([M8, K8]))

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT}: {os.path.getsize(OUT)} bytes, {len(g)} arrays")


if __name__ == "__main__":
    main()
