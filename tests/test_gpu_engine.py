"""The device LLaMA engine against slate's answers (golden.npz, produced by
slate_llama_prefill / slate_llama_decode_step) and the oracle.

Parity contract: logits within normwise relative 1e-3 of the reference f32
CPU path; greedy token streams identical except where the reference's top-2
logit gap is below that tolerance (then the rest of that stream is free to
diverge and is not compared).
"""
import numpy as np
import pytest

import slate_amd
from oracle.pyoracle import OracleModel
from slate_amd.synth import LlamaShape, engine_tensors, make_llama
from tests.helpers import (N_GEN, Q4, Q4_PROMPT, Q4_SEED, TINY, TINY_SEED, relerr, tensors_digest,
                           tiny_prompts)

pytestmark = pytest.mark.gpu
TOL = 1e-3


def gap_ok(ref_logits):
    """True when the reference's top-2 gap clears the tolerance."""
    s = np.sort(ref_logits.astype(np.float64))
    return (s[-1] - s[-2]) > TOL * max(np.abs(ref_logits).max(), 1e-30)


def tiny_model(golden):
    t = make_llama(TINY, TINY_SEED, quant="f32")
    assert tensors_digest(t) == str(golden["tiny_digest"])
    return t


def test_tiny_llama_ragged_batch_matches_reference(golden):
    """Config 1: 4 sequences prefilled, then decoded together as one ragged
    batch for 32 steps (every step a batch of 4 different positions)."""
    t = tiny_model(golden)
    m = slate_amd.Llama.from_tensors(TINY, t, max_slots=4, max_tokens=64)
    prompts = tiny_prompts()
    sess = [m.session() for _ in prompts]
    last = []
    for s, p in zip(sess, prompts):
        rc, lg = s.prefill(p)
        assert rc == 0
        last.append(lg)
    alive = [True] * len(sess)
    cur = np.stack(last)
    for k in range(N_GEN):
        ref = golden["tiny_logits"][:, k]
        for i in range(len(sess)):
            if alive[i]:
                assert relerr(cur[i], ref[i]) < TOL, (i, k)
        toks = []
        for i in range(len(sess)):
            tok = int(np.argmax(cur[i]))
            if alive[i]:
                if tok != golden["tiny_streams"][i, k]:
                    assert not gap_ok(ref[i]), f"stream {i} diverged at step {k} with a clear top-2 gap"
                    alive[i] = False
            toks.append(tok)
        rc, cur, nxt = m.step(sess, [1] * len(sess), toks)
        assert rc == 0
        assert list(nxt) == [int(np.argmax(c)) for c in cur]
    assert all(alive), "every stream should match the reference for this workload"
    for s, p in zip(sess, prompts):
        assert s.position == len(p) + N_GEN


def test_q4k_llama_matches_reference(golden):
    t = make_llama(Q4, Q4_SEED, quant="q4k", output_quant="f32")
    assert tensors_digest(t) == str(golden["q4_digest"])
    m = slate_amd.Llama.from_tensors(Q4, t, max_slots=2, max_tokens=32)
    s = m.session()
    rc, lg = s.prefill(Q4_PROMPT)
    assert rc == 0
    for k in range(8):
        assert relerr(lg, golden["q4_logits"][k]) < TOL, k
        tok = int(np.argmax(lg))
        assert tok == golden["q4_stream"][k] or not gap_ok(golden["q4_logits"][k])
        rc, lg = s.decode(int(golden["q4_stream"][k]))
        assert rc == 0
    assert relerr(lg, golden["q4_logits"][8]) < TOL


def test_batched_equals_sequential(golden):
    """slate's test_infer.c:159-212 property for the LLaMA engine: one batched
    step equals separate single-session steps (Linf < 1e-4)."""
    t = tiny_model(golden)
    m = slate_amd.Llama.from_tensors(TINY, t, max_slots=8, max_tokens=64)
    prompts = [np.array(p[:6]) for p in tiny_prompts()]
    nxt = [22, 13, 8, 27]
    seq = []
    for p, tk in zip(prompts, nxt):
        s = m.session()
        s.prefill(p)
        seq.append(s.decode(tk)[1])
        s.free()
    sess = [m.session() for _ in prompts]
    for s, p in zip(sess, prompts):
        s.prefill(p)
    rc, lg, _ = m.step(sess, [1] * 4, nxt)
    assert rc == 0
    assert np.max(np.abs(lg - np.stack(seq))) < 1e-4


def test_mixed_prefill_and_decode_step(orc, golden):
    """One ragged step carrying prompt chunks and single decode tokens at
    once matches the oracle's token-serial processing; KV caches match."""
    t = tiny_model(golden)
    om = OracleModel(orc, TINY, t)
    m = slate_amd.Llama.from_tensors(TINY, t, max_slots=4, max_tokens=64)
    rng = np.random.default_rng(3)
    first = [rng.integers(0, TINY.vocab, n).astype(np.int32) for n in (3, 7, 1, 12)]
    second = [rng.integers(0, TINY.vocab, n).astype(np.int32) for n in (1, 5, 1, 9)]
    sess = [m.session() for _ in first]
    osess = [om.session() for _ in first]
    rc, _, _ = m.step(sess, [len(a) for a in first], np.concatenate(first), want_logits=False)
    assert rc == 0
    rc, lg, nxt = m.step(sess, [len(a) for a in second], np.concatenate(second))
    assert rc == 0
    for i, (o, a, b) in enumerate(zip(osess, first, second)):
        o.prefill(a)
        _, want = o.prefill(b)
        assert relerr(lg[i], want) < TOL
        assert sess[i].position == len(a) + len(b) == o.position
        K, V = sess[i].kv()
        Ko, Vo = o.kv()
        n = o.position
        assert relerr(K[:, :n], Ko[:, :n]) < 1e-4 and relerr(V[:, :n], Vo[:, :n]) < 1e-4


def test_engine_error_codes(golden):
    """llama_infer.c:144-145 codes; a rejected step advances no session."""
    shape = LlamaShape(**{**TINY.__dict__, "max_seq": 8})
    t = make_llama(shape, 5, quant="f32")
    m = slate_amd.Llama.from_tensors(shape, t, max_slots=2, max_tokens=16)
    a, b = m.session(), m.session()
    with pytest.raises(slate_amd.HipError):
        m.session()                                  # both KV slots taken
    slate_amd.load_library().slate_hip_clear_error()
    assert a.decode(shape.vocab)[0] == -3
    assert a.decode(-1)[0] == -3
    assert m.step([a, b], [1, 1], [1, 999])[0] == -3
    assert m.step([a, a], [1, 1], [1, 2])[0] == -1
    assert m.step([a, b], [0, 1], [1])[0] == -1
    assert a.position == 0 and b.position == 0
    assert a.prefill(np.arange(8, dtype=np.int32))[0] == 0
    assert a.decode(1)[0] == -2
    assert m.step([a, b], [1, 1], [1, 2])[0] == -2
    assert a.position == 8 and b.position == 0
    assert m.step([b], [9], np.zeros(9, np.int32))[0] == -2
    assert b.prefill(np.arange(17, dtype=np.int32) % 8)[0] == -2
    a.free()
    c = m.session()
    assert c.position == 0


def test_synthetic_q4k_engine_runs_and_is_batch_invariant():
    """A device-generated Q4_K model (8B layer shapes, 2 layers, small vocab):
    batched greedy decode equals one-at-a-time decode."""
    shape = LlamaShape(n_layers=2, d_model=4096, n_heads=32, n_kv_heads=8, ffn=14336, vocab=4096,
                       max_seq=512)
    m = slate_amd.Llama.synthetic(shape, seed=7, quant=18, max_slots=5, max_tokens=64)
    rng = np.random.default_rng(0)
    prompts = [rng.integers(0, shape.vocab, n).astype(np.int32) for n in (5, 17, 40, 2)]
    sess = [m.session() for _ in prompts]
    rc, lg, nxt = m.step(sess, [len(p) for p in prompts], np.concatenate(prompts))
    assert rc == 0 and np.all(np.isfinite(lg))
    solo = m.session()
    rc, lg1 = solo.prefill(prompts[2])
    assert rc == 0
    assert relerr(lg1, lg[2]) < 1e-5
    toks = list(nxt)
    for _ in range(4):
        rc, lg, nxt = m.step(sess, [1] * 4, toks)
        rc2, l2 = solo.decode(toks[2])
        assert rc == 0 and rc2 == 0
        assert relerr(l2, lg[2]) < 1e-5
        toks = list(nxt)


def test_deferred_rmsnorm_matches_row_rmsnorm(golden, monkeypatch):
    """The all-Q4_K layers apply the RMSNorm row factor after the matmul
    (residual_act + the consumer's row scale); the engine built with the
    whole-row RMSNorm kernel instead gives the same logits to 1e-5 on a
    ragged batch with a prompt chunk."""
    t = make_llama(Q4, Q4_SEED, quant="q4k", output_quant="f32")
    outs = []
    for flag in ("1", "0"):
        monkeypatch.setenv("SLATE_HIP_FUSED_NORM", flag)
        m = slate_amd.Llama.from_tensors(Q4, t, max_slots=3, max_tokens=48)
        ss = [m.session() for _ in range(3)]
        rng = np.random.default_rng(11)
        toks = rng.integers(0, Q4.vocab, 20).astype(np.int32)
        rc, lg1, nx1 = m.step(ss, [9, 6, 5], toks)
        assert rc == 0
        rc, lg2, nx2 = m.step(ss, [1, 1, 7], np.concatenate([nx1[:2], toks[:7]]).astype(np.int32))
        assert rc == 0
        outs.append((lg1, lg2))
        for s in ss:
            s.free()
        m.free()
    for a, b in zip(outs[0], outs[1]):
        assert relerr(a, b) < 1e-5


FUSE = LlamaShape(n_layers=2, d_model=512, n_heads=8, n_kv_heads=4, ffn=768, vocab=300, max_seq=96)


def test_q4k_decode_steps_match_oracle(orc):
    """A 512-wide all-Q4_K model (every tensor 256-aligned, LM head Q4_K):
    a prompt step for three sequences, then ragged decode steps, each
    against the oracle (the CPU reference) replaying the same tokens."""
    t = make_llama(FUSE, 4321, quant="q4k", output_quant="q4k")
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, FUSE.vocab, n).astype(np.int32) for n in (6, 1, 11)]
    m = slate_amd.Llama.from_tensors(FUSE, t, max_slots=4, max_tokens=32)
    sess = [m.session() for _ in prompts]
    rc, lg, nxt = m.step(sess, [len(p) for p in prompts], np.concatenate(prompts))
    assert rc == 0
    steps = [lg]
    toks = np.asarray(nxt, np.int32)
    for _ in range(6):
        rc, lg, nxt = m.step(sess, [1, 1, 1], toks)
        assert rc == 0
        steps.append(lg)
        toks = np.asarray(nxt, np.int32)
    om = OracleModel(orc, FUSE, t)
    for i, p in enumerate(prompts):
        o = om.session()
        rc, want = o.prefill(p)
        assert rc == 0 and relerr(steps[0][i], want) < TOL
        tok = int(np.argmax(steps[0][i]))
        for k in range(1, len(steps)):
            rc, want = o.decode(tok)
            assert rc == 0 and relerr(steps[k][i], want) < TOL, (i, k)
            tok = int(np.argmax(steps[k][i]))


def run_fused_and_separate(shape, prompts, extra):
    """The same tokens through single-token steps (RoPE/append fused into
    decode attention) and through one step of several tokens per sequence
    (separate kernels): final logits and each session's K/V cache."""
    t = make_llama(shape, 4321, quant="q4k", output_quant="q4k")
    out = []
    n_ex = len(extra[0])
    for fused in (True, False):
        m = slate_amd.Llama.from_tensors(shape, t, max_slots=len(prompts), max_tokens=512)
        sess = [m.session() for _ in prompts]
        rc, _, _ = m.step(sess, [len(p) for p in prompts], np.concatenate(prompts), want_logits=False)
        assert rc == 0
        if fused:
            for k in range(n_ex):
                rc, lg, _ = m.step(sess, [1] * len(prompts), np.array([e[k] for e in extra], np.int32))
                assert rc == 0
        else:
            rc, lg, _ = m.step(sess, [n_ex] * len(prompts), np.concatenate(extra))
            assert rc == 0
        assert [s.position for s in sess] == [len(p) + n_ex for p in prompts]
        out.append((np.array(lg), [s.kv() for s in sess]))
    return out


def test_fused_rope_attention_first_token_of_a_session(orc):
    """A fresh session's first token in a step where every sequence adds one
    token: the fused decode attention appends K/V at position 0 and attends
    that key alone; logits of both sequences against the oracle, and the
    following steps too."""
    t = make_llama(FUSE, 4321, quant="q4k", output_quant="q4k")
    om = OracleModel(orc, FUSE, t)
    m = slate_amd.Llama.from_tensors(FUSE, t, max_slots=2, max_tokens=32)
    a, b = m.session(), m.session()
    oa, ob = om.session(), om.session()
    rng = np.random.default_rng(23)
    pa = rng.integers(0, FUSE.vocab, 7).astype(np.int32)
    rc, _, _ = m.step([a], [len(pa)], pa, want_logits=False)
    assert rc == 0
    oa.prefill(pa)
    toks = rng.integers(0, FUSE.vocab, (3, 2)).astype(np.int32)
    for k in range(3):
        rc, lg, _ = m.step([a, b], [1, 1], toks[k])
        assert rc == 0
        _, wa = oa.decode(int(toks[k][0]))
        _, wb = (ob.prefill(toks[k][1:2]) if k == 0 else ob.decode(int(toks[k][1])))
        assert relerr(lg[0], wa) < TOL and relerr(lg[1], wb) < TOL, k
    assert b.position == 3 and a.position == 10


@pytest.mark.parametrize("d_model,n_heads,n_kv_heads", [(512, 4, 4), (512, 8, 1), (256, 8, 8)])
def test_fused_rope_attention_head_groups(orc, d_model, n_heads, n_kv_heads):
    """The fused decode attention at more head groups than the model tests
    reach: G = 1 with head_dim 128, G = 8 with head_dim 64 (G * HD = 512, the
    wave kernel's limit), G = 1 with head_dim 32; a prompt step, then decode
    steps of two sequences, every step against the oracle."""
    shape = LlamaShape(2, d_model, n_heads, n_kv_heads, 512, 300, 320)
    t = make_llama(shape, 4321, quant="q4k", output_quant="q4k")
    rng = np.random.default_rng(24)
    prompts = [rng.integers(0, shape.vocab, n).astype(np.int32) for n in (260, 9)]
    m = slate_amd.Llama.from_tensors(shape, t, max_slots=2, max_tokens=320)
    sess = [m.session() for _ in prompts]
    rc, lg, nxt = m.step(sess, [len(p) for p in prompts], np.concatenate(prompts))
    assert rc == 0
    steps, toks = [lg], np.asarray(nxt, np.int32)
    for _ in range(4):
        rc, lg, nxt = m.step(sess, [1, 1], toks)
        assert rc == 0
        steps.append(lg)
        toks = np.asarray(nxt, np.int32)
    om = OracleModel(orc, shape, t)
    for i, p in enumerate(prompts):
        o = om.session()
        rc, want = o.prefill(p)
        assert rc == 0 and relerr(steps[0][i], want) < TOL
        tok = int(np.argmax(steps[0][i]))
        for k in range(1, len(steps)):
            rc, want = o.decode(tok)
            assert rc == 0 and relerr(steps[k][i], want) < TOL, (i, k)
            tok = int(np.argmax(steps[k][i]))


def test_fused_rope_phased_attention_equals_separate_kernels(switch_env):
    """As below for a head group too wide for the wave kernel (8 query heads of
    128 per kv head, as the 70B shape): the fused path runs in the phased
    kernel, the separate path in the same kernel without the prologue; K/V
    caches bit-identical, logits within 1e-5."""
    switch_env.setenv("SLATE_HIP_ATTN_MFMA", "0")
    shape = LlamaShape(2, 2048, 16, 2, 768, 300, 512)
    rng = np.random.default_rng(22)
    prompts = [rng.integers(0, shape.vocab, n).astype(np.int32) for n in (253, 30)]
    extra = [rng.integers(0, shape.vocab, 4).astype(np.int32) for _ in prompts]
    (la, kva), (lb, kvb) = run_fused_and_separate(shape, prompts, extra)
    assert relerr(la, lb) < 1e-5
    for (Ka, Va), (Kb, Vb), p in zip(kva, kvb, prompts):
        n = len(p) + 4
        assert np.array_equal(Ka[:, :n], Kb[:, :n]) and np.array_equal(Va[:, :n], Vb[:, :n])


def test_fused_rope_attention_equals_separate_kernels(switch_env):
    """Steps in which every sequence adds one token rotate q/k and append K/V
    inside the decode attention kernel; a step adding several tokens of a
    sequence runs RoPE/append and attention as separate kernels.  The same
    tokens fed both ways (four single-token steps, or one step of four tokens
    per sequence), across the 256-key chunk boundary (positions 254-257, the
    last a chunk of one key) and beside a short second sequence, give
    bit-identical K/V caches (layer 1's rows carry layer 0's attention
    output): per token the two paths evaluate the same expressions.  The
    final logits agree within 1e-5: single-token steps also defer the final
    RMSNorm factor to the argmax, the four-token step normalises the rows.
    The four-token step's tokens attend tokenwise (SLATE_HIP_ATTN_MFMA=0), in
    the decode kernel the fused path also runs; the MFMA prompt kernel rounds
    differently and has its own tests."""
    switch_env.setenv("SLATE_HIP_ATTN_MFMA", "0")
    shape = LlamaShape(2, 512, 8, 4, 768, 300, 512)
    rng = np.random.default_rng(21)
    prompts = [rng.integers(0, shape.vocab, n).astype(np.int32) for n in (254, 40)]
    extra = [rng.integers(0, shape.vocab, 4).astype(np.int32) for _ in prompts]
    (la, kva), (lb, kvb) = run_fused_and_separate(shape, prompts, extra)
    assert relerr(la, lb) < 1e-5
    for (Ka, Va), (Kb, Vb), n in zip(kva, kvb, (258, 44)):
        assert np.array_equal(Ka[:, :n], Kb[:, :n]) and np.array_equal(Va[:, :n], Vb[:, :n])


XCD_SHAPE = LlamaShape(n_layers=3, d_model=1024, n_heads=8, n_kv_heads=2, ffn=768, vocab=300, max_seq=1100)
# 8 kv heads: the pair list's own scan fills the per-XCD queues
XCD8_SHAPE = LlamaShape(n_layers=3, d_model=2048, n_heads=16, n_kv_heads=8, ffn=768, vocab=300, max_seq=1100)


@pytest.mark.parametrize("shape,kv_f16", [(XCD_SHAPE, False), (XCD_SHAPE, True), (XCD8_SHAPE, False)],
                         ids=["hkv2", "hkv2_f16", "hkv8"])
def test_decode_attention_merged_in_kernel_equals_merge_kernel(orc, switch_env, shape, kv_f16):
    """Decode steps (one token per sequence) of shapes whose kv head groups
    fill whole 256-wide operand blocks (4 or 2 query heads of 128 per kv
    head; 2 kv heads: the queues' own kernel fills them, 8: the pair list's
    scan does) merge the attention chunks inside the attention kernel, from
    per-XCD work queues, instead of in a separate merge kernel
    (SLATE_HIP_ATTN_XCD=0).  Contexts of 1-1000 keys (up to four 256-key
    chunks per pair, pairs whose last chunk holds one key), six sequences,
    three layers (each layer's arrival counts start from zero again), four
    decode steps: the
    merge evaluates the same expressions in the same order, so logits and
    K/V caches are bit-identical to the merge kernel's; the logits also
    against the oracle (f32 caches)."""
    switch_env.setenv("SLATE_HIP_KV_F16", "1" if kv_f16 else "0")
    t = make_llama(shape, 977, quant="q4k", output_quant="q4k")
    rng = np.random.default_rng(31)
    lens = (1000, 300, 256, 40, 1, 511)
    prompts = [rng.integers(0, shape.vocab, n).astype(np.int32) for n in lens]
    runs = []
    for xcd in ("1", "0"):
        switch_env.setenv("SLATE_HIP_ATTN_XCD", xcd)
        m = slate_amd.Llama.from_tensors(shape, t, max_slots=len(prompts), max_tokens=sum(lens))
        sess = [m.session() for _ in prompts]
        rc, lg, nxt = m.step(sess, list(lens), np.concatenate(prompts))
        assert rc == 0
        steps, feed = [], []
        toks = np.asarray(nxt, np.int32)
        for _ in range(4):
            feed.append(toks)
            rc, lg, nxt = m.step(sess, [1] * len(sess), toks)
            assert rc == 0
            steps.append(np.array(lg))
            toks = np.asarray(nxt, np.int32)
        runs.append((steps, feed, [s.kv() for s in sess]))
        for s in sess:
            s.free()
        m.free()
    (sa, fa, kva), (sb, fb, kvb) = runs
    for k in range(4):
        assert np.array_equal(fa[k], fb[k]) and np.array_equal(sa[k], sb[k]), k
    for (Ka, Va), (Kb, Vb) in zip(kva, kvb):
        assert np.array_equal(Ka, Kb) and np.array_equal(Va, Vb)
    # against the oracle (f32 caches); the f16 caches at the same 1e-3 the
    # f16 tolerance study holds them to (head_dim 128 here: the lane map
    # that loads eight f16 values per lane and row)
    om = OracleModel(orc, shape, t)
    for i, p in enumerate(prompts):
        o = om.session()
        rc, _ = o.prefill(p)
        assert rc == 0
        for k in range(4):
            rc, want = o.decode(int(fa[k][i]))
            assert rc == 0 and relerr(sa[k][i], want) < TOL, (i, k, relerr(sa[k][i], want))


def test_decode_attention_misplaced_workgroup_falls_back_to_merge_kernel(switch_env):
    """The in-kernel merge is sound only while all units of a (token, kv
    head) pair run on one XCD.  Every unit tags its partial with the launch
    and its XCD; the merging unit compares the pair's tags with its own and
    on any difference reports to the host, which runs the step again on the
    merge kernel and keeps the engine there.  SLATE_HIP_ATTN_XCD_TAMPER=1
    makes the merge expect a tag no unit writes, so every launch reports: the
    first decode step is run twice, and logits, next tokens and K/V caches
    are bit-identical to an engine on the merge kernel (SLATE_HIP_ATTN_XCD=0).
    Without the switch the engine keeps the in-kernel merge through every
    step (no merge found a partial from another XCD)."""
    shape = XCD_SHAPE
    t = make_llama(shape, 978, quant="q4k", output_quant="q4k")
    rng = np.random.default_rng(32)
    lens = (700, 257, 33, 1)
    prompts = [rng.integers(0, shape.vocab, n).astype(np.int32) for n in lens]
    runs = []
    for env, merge_before, merge_after in ((("SLATE_HIP_ATTN_XCD_TAMPER", "1"), 1, 0),
                                           (("SLATE_HIP_ATTN_XCD", "0"), 0, 0),
                                           (("SLATE_HIP_ATTN_XCD_TAMPER", "0"), 1, 1)):
        switch_env.setenv(*env)
        m = slate_amd.Llama.from_tensors(shape, t, max_slots=len(prompts), max_tokens=sum(lens))
        switch_env.delenv(env[0])
        assert m.lib.slate_hip_llama_attn_xcd_merge(m.h) == merge_before, env
        sess = [m.session() for _ in prompts]
        rc, lg, nxt = m.step(sess, list(lens), np.concatenate(prompts))
        assert rc == 0
        out = []
        for _ in range(3):
            rc, lg, nxt = m.step(sess, [1] * len(sess), np.asarray(nxt, np.int32))
            assert rc == 0
            out.append((np.array(lg), np.array(nxt)))
        assert m.lib.slate_hip_llama_attn_xcd_merge(m.h) == merge_after, env
        runs.append((out, [s.kv() for s in sess]))
        for s in sess:
            s.free()
        m.free()
    (oa, kva), (ob, kvb), (oc, kvc) = runs
    for (la, na), (lb, nb), (lc, nc) in zip(oa, ob, oc):
        assert np.array_equal(la, lb) and np.array_equal(na, nb)
        assert np.array_equal(lc, lb) and np.array_equal(nc, nb)
    for (Ka, Va), (Kb, Vb) in zip(kva, kvb):
        assert np.array_equal(Ka, Kb) and np.array_equal(Va, Vb)
    assert slate_amd.last_error() is None


@pytest.mark.parametrize("nseq", [64, 65])
def test_decode_attention_in_kernel_merge_at_the_batch_limit(switch_env, nseq):
    """The in-kernel merge takes decode steps of up to 64 sequences (64: the
    largest grid and the fullest queues; 65: the merge kernel takes over):
    ragged contexts of 1-700 keys, 8 kv heads, two decode steps, logits and
    next tokens bit-identical to the merge kernel's (SLATE_HIP_ATTN_XCD=0)."""
    t = make_llama(XCD8_SHAPE, 4242, quant="q4k", output_quant="q4k")
    rng = np.random.default_rng(nseq)
    lens = [int(n) for n in rng.integers(1, 700, nseq)]
    prompts = [rng.integers(0, XCD8_SHAPE.vocab, n).astype(np.int32) for n in lens]
    runs = []
    for xcd in ("1", "0"):
        switch_env.setenv("SLATE_HIP_ATTN_XCD", xcd)
        m = slate_amd.Llama.from_tensors(XCD8_SHAPE, t, max_slots=nseq, max_tokens=sum(lens))
        sess = [m.session() for _ in prompts]
        rc, lg, nxt = m.step(sess, lens, np.concatenate(prompts))
        assert rc == 0
        out = []
        for _ in range(2):
            rc, lg, nxt = m.step(sess, [1] * nseq, np.asarray(nxt, np.int32))
            assert rc == 0
            out.append((np.array(lg), np.array(nxt)))
        for s_ in sess:
            s_.free()
        m.free()
        runs.append(out)
    for (la, na), (lb, nb) in zip(*runs):
        assert np.array_equal(la, lb) and np.array_equal(na, nb)


def test_graph_replayed_decode_steps_match_eager_launches(golden):
    """Decode-only steps replay a captured HIP graph; interleaved with eager
    prompt steps and repeated many times, every replay gives bit-identical
    logits, next tokens and KV to the same steps launched kernel by kernel."""
    t = make_llama(Q4, Q4_SEED, quant="q4k", output_quant="f32")
    rng = np.random.default_rng(21)
    prompts = [rng.integers(0, Q4.vocab, n).astype(np.int32) for n in (4, 9)]
    late = rng.integers(0, Q4.vocab, 7).astype(np.int32)
    runs = []
    for use_graphs in (True, False):
        m = slate_amd.Llama.from_tensors(Q4, t, max_slots=3, max_tokens=32)
        m.graphs(use_graphs)
        ss = [m.session() for _ in prompts]
        out = []
        rc, lg, nxt = m.step(ss, [len(p) for p in prompts], np.concatenate(prompts))
        assert rc == 0
        out.append((lg, nxt))
        toks = np.asarray(nxt, np.int32)
        for _ in range(5):                       # replays of the 2-session graph
            rc, lg, nxt = m.step(ss, [1, 1], toks)
            assert rc == 0
            out.append((lg, nxt))
            toks = np.asarray(nxt, np.int32)
        s3 = m.session()                         # eager prompt step between replays
        rc, lg, nxt = m.step(ss + [s3], [1, 1, len(late)], np.concatenate([toks, late]))
        assert rc == 0
        out.append((lg, nxt))
        toks = np.asarray(nxt, np.int32)
        for _ in range(5):                       # a second graph (3 sessions), replayed
            rc, lg, nxt = m.step(ss + [s3], [1, 1, 1], toks)
            assert rc == 0
            out.append((lg, nxt))
            toks = np.asarray(nxt, np.int32)
        rc, lg, nxt = m.step(ss, [1, 1], toks[:2])   # back to the first graph
        assert rc == 0
        out.append((lg, nxt))
        runs.append((out, [s.kv() for s in ss + [s3]]))
        m.free()
    (a, akv), (b, bkv) = runs
    for (la, na), (lb, nb) in zip(a, b):
        assert np.array_equal(la, lb) and np.array_equal(na, nb)
    for (K1, V1), (K2, V2) in zip(akv, bkv):
        assert np.array_equal(K1, K2) and np.array_equal(V1, V2)


@pytest.mark.parametrize("shape", [LlamaShape(2, 512, 8, 4, 768, 300, 512),
                                   LlamaShape(2, 1024, 8, 2, 768, 300, 512)], ids=["hd64", "hd128"])
def test_f16_kv_cache_tolerance_study(orc, monkeypatch, shape):
    """The opt-in f16 K/V cache against the oracle's f32 reference: Q4_K
    models with head_dim 64 (8 query / 4 KV heads) and 128 (8 / 2: the
    16-byte f16 row loads, eight values per lane), three prompts of 150-280
    tokens (contexts over two 256-key chunks), 24 ragged decode steps; every
    step's logits stay within the parity tolerance (normwise relative 1e-3).
    Layer 0's cached K/V equal the f32 engine's rounded to f16 (layers above
    also carry the f16 attention's own rounding)."""
    t = make_llama(shape, 4321, quant="q4k", output_quant="q4k")
    rng = np.random.default_rng(16)
    prompts = [rng.integers(0, shape.vocab, n).astype(np.int32) for n in (150, 220, 280)]
    engines = {}
    for f16 in (True, False):
        monkeypatch.setenv("SLATE_HIP_KV_F16", "1" if f16 else "0")
        m = slate_amd.Llama.from_tensors(shape, t, max_slots=4, max_tokens=1024)
        assert m.lib.slate_hip_llama_kv_f16(m.h) == (1 if f16 else 0)
        sess = [m.session() for _ in prompts]
        rc, lg, nxt = m.step(sess, [len(p) for p in prompts], np.concatenate(prompts))
        assert rc == 0
        steps = [lg]
        toks = np.asarray(nxt, np.int32)
        for _ in range(24):
            rc, lg, nxt = m.step(sess, [1, 1, 1], toks)
            assert rc == 0
            steps.append(lg)
            toks = np.asarray(nxt, np.int32)
        engines[f16] = (m, sess, steps)
    m16, s16, steps16 = engines[True]
    m32, s32, steps32 = engines[False]
    om = OracleModel(orc, shape, t)
    worst = 0.0
    for i, p in enumerate(prompts):
        o = om.session()
        rc, want = o.prefill(p)
        assert rc == 0
        worst = max(worst, relerr(steps16[0][i], want))
        tok = int(np.argmax(steps16[0][i]))
        for k in range(1, len(steps16)):
            rc, want = o.decode(tok)
            assert rc == 0
            e = relerr(steps16[k][i], want)
            worst = max(worst, e)
            assert e < TOL, (i, k, e)
            tok = int(np.argmax(steps16[k][i]))
    print(f"f16 K/V: worst normwise logits error vs the f32 reference {worst:.2e}")
    for a, b in zip(s16, s32):
        (K16, V16), (K32, V32) = a.kv(), b.kv()
        n = a.position
        for X16, X32 in ((K16, K32), (V16, V32)):
            ref = X32[0, :n].astype(np.float16).astype(np.float32)
            assert np.array_equal(X16[0, :n], ref)
    for m, sess, _ in engines.values():
        for s in sess:
            s.free()
        m.free()


MIXQ = LlamaShape(n_layers=2, d_model=1024, n_heads=8, n_kv_heads=4, ffn=2048, vocab=300, max_seq=160)


def replay_against_oracle(orc, shape, t, m, prompts, n_decode):
    """Prompt step for every sequence, then ragged decode steps; each
    sequence's logits against the oracle replaying the engine's tokens."""
    sess = [m.session() for _ in prompts]
    rc, lg, nxt = m.step(sess, [len(p) for p in prompts], np.concatenate(prompts))
    assert rc == 0
    steps = [lg]
    toks = np.asarray(nxt, np.int32)
    for _ in range(n_decode):
        rc, lg, nxt = m.step(sess, [1] * len(prompts), toks)
        assert rc == 0
        steps.append(lg)
        toks = np.asarray(nxt, np.int32)
    om = OracleModel(orc, shape, t)
    for i, p in enumerate(prompts):
        o = om.session()
        rc, want = o.prefill(p)
        assert rc == 0 and relerr(steps[0][i], want) < TOL
        tok = int(np.argmax(steps[0][i]))
        for k in range(1, len(steps)):
            rc, want = o.decode(tok)
            assert rc == 0 and relerr(steps[k][i], want) < TOL, (i, k)
            tok = int(np.argmax(steps[k][i]))


def test_q8_0_llama_matches_oracle(orc):
    """All linears and the LM head Q8_0 (dtype 16, which the reference's
    dispatch would read as f32): a 68-token prompt step (prefill kernels
    over 8 activation tiles) and ragged decode steps against the oracle's
    corrected dispatch; weights read back in slate's row layout unchanged."""
    t = make_llama(FUSE, 77, quant="q8_0", output_quant="q8_0")
    rng = np.random.default_rng(8)
    prompts = [rng.integers(0, FUSE.vocab, n).astype(np.int32) for n in (40, 25, 3)]
    m = slate_amd.Llama.from_tensors(FUSE, t, max_slots=4, max_tokens=96)
    for name in ("blk.0.attn_q.weight", "blk.1.ffn_down.weight", "output.weight"):
        raw, dt = m.get_tensor(name.rsplit(".", 1)[0])
        assert dt == 16 and np.array_equal(raw, t[name][0])
    replay_against_oracle(orc, FUSE, t, m, prompts, 6)


def test_mixed_dtype_groups_match_oracle(orc):
    """Q4_K, Q8_0 and f32 linears sharing one input: the QKV group mixes
    Q4_K and Q8_0 (the Q8_0 kernel writes the split count the Q4_K launch
    chose), gate/up mix Q8_0 and Q4_K, down is f32, o and the LM head Q8_0."""
    from slate_amd.synth import quantize_q4k, quantize_q8_0
    t = make_llama(MIXQ, 99, quant="f32", output_quant="f32")
    kinds = {"attn_q": "q4k", "attn_k": "q8_0", "attn_v": "q4k", "attn_output": "q8_0",
             "ffn_gate": "q8_0", "ffn_up": "q4k", "ffn_down": "f32"}
    for name in list(t):
        base = name.rsplit(".", 1)[0].split(".")[-1]
        kind = "q8_0" if name == "output.weight" else kinds.get(base)
        a, _, shp = t[name]
        if kind == "q4k":
            t[name] = (np.frombuffer(quantize_q4k(a), np.uint8), 18, shp)
        elif kind == "q8_0":
            t[name] = (np.frombuffer(quantize_q8_0(a), np.uint8), 16, shp)
    rng = np.random.default_rng(9)
    prompts = [rng.integers(0, MIXQ.vocab, n).astype(np.int32) for n in (9, 1, 30)]
    m = slate_amd.Llama.from_tensors(MIXQ, t, max_slots=4, max_tokens=48)
    replay_against_oracle(orc, MIXQ, t, m, prompts, 4)


def requantise(t, kinds, output_kind=None):
    """Convert the f32 linears of a make_llama model per tensor kind
    ("q4k" / "q8_0"; others stay f32)."""
    from slate_amd.synth import quantize_q4k, quantize_q8_0
    for name in list(t):
        base = name.rsplit(".", 1)[0].split(".")[-1]
        kind = output_kind if name == "output.weight" else kinds.get(base)
        a, _, shp = t[name]
        if kind == "q4k":
            t[name] = (np.frombuffer(quantize_q4k(a), np.uint8), 18, shp)
        elif kind == "q8_0":
            t[name] = (np.frombuffer(quantize_q8_0(a), np.uint8), 16, shp)
    return t


UNALIGNED_FFN = LlamaShape(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, ffn=352, vocab=300, max_seq=64)


def test_q4k_gate_up_with_unaligned_ffn_width(orc):
    """Q4_K gate/up (K = d_model = 256) with an FFN width that is not a
    multiple of 256 (352, so down is Q8_0): the SwiGLU falls back to the
    f32 kernel, which takes no deferred RMSNorm factor, so the FFN norm must
    be applied before the gate/up matmul; prompt and decode steps against
    the oracle."""
    t = make_llama(UNALIGNED_FFN, 55, quant="f32", output_quant="f32")
    requantise(t, {"attn_q": "q4k", "attn_k": "q4k", "attn_v": "q4k", "attn_output": "q4k",
                   "ffn_gate": "q4k", "ffn_up": "q4k", "ffn_down": "q8_0"}, "q4k")
    rng = np.random.default_rng(56)
    prompts = [rng.integers(0, UNALIGNED_FFN.vocab, n).astype(np.int32) for n in (7, 19, 2)]
    m = slate_amd.Llama.from_tensors(UNALIGNED_FFN, t, max_slots=3, max_tokens=32)
    replay_against_oracle(orc, UNALIGNED_FFN, t, m, prompts, 4)


# Every non-default setting of the engine's plan and path switches (the
# f16 K/V cache has its own tolerance study above).  Six sequences, so that
# decode steps run the 16-row MFMA decode kernels the Q4_K / Q8_0 plan
# switches steer; a 68-token prompt step for the prompt kernels.
SWITCHES = [("SLATE_HIP_FUSED_NORM", "0", "q4k"), ("SLATE_HIP_ATTN_MFMA", "0", "q4k"),
            ("SLATE_HIP_ATTN_MFMA", "2", "q4k"),
            # the query-block prompt kernel: neither the MFMA nor the tokenwise path
            ("SLATE_HIP_ATTN_MFMA=0,SLATE_HIP_ATTN_TOKENWISE", "0", "q4k"),
            ("SLATE_HIP_ATTN_WAVE", "0", "q4k"), ("SLATE_HIP_ATTN_ROPE", "0", "q4k"),
            ("SLATE_HIP_ATTN_ROPE", "2", "q4k"), ("SLATE_HIP_ATTN_XCD", "0", "q4k"), ("SLATE_HIP_GRAPHS", "1", "q4k"),
            ("SLATE_HIP_Q4K_R", "1", "q4k"), ("SLATE_HIP_Q4K_R", "4", "q4k"), ("SLATE_HIP_Q4K_W", "4", "q4k"),
            ("SLATE_HIP_Q4K_S", "1", "q4k"), ("SLATE_HIP_Q4K_S", "3", "q4k"), ("SLATE_HIP_Q4K_WGS", "64", "q4k"),
            ("SLATE_HIP_Q4K_PF_S", "3", "q4k"), ("SLATE_HIP_Q4K_PF_NT", "2", "q4k"),
            ("SLATE_HIP_Q4K_PF_NT", "4", "q4k"), ("SLATE_HIP_Q4K_DEC32", "0", "q4k"), ("SLATE_HIP_Q4K_EARLY", "1", "q4k"),
            ("SLATE_HIP_Q8_R", "1", "q8_0"), ("SLATE_HIP_Q8_R", "4", "q8_0"),
            ("SLATE_HIP_Q8_S", "2", "q8_0"), ("SLATE_HIP_Q8_WGS", "64", "q8_0")]


def test_decode_steps_of_17_to_32_sequences(orc):
    """Ragged decode steps of 24 sequences (32 padded rows: the Q4_K decode
    kernel with two 16-row activation tiles, as the 70B workload's batches of
    up to 32 run), after a prompt step, against the oracle."""
    t = make_llama(FUSE, 4321, quant="q4k", output_quant="q4k")
    rng = np.random.default_rng(24)
    prompts = [rng.integers(0, FUSE.vocab, n).astype(np.int32) for n in rng.integers(1, 9, 24)]
    m = slate_amd.Llama.from_tensors(FUSE, t, max_slots=24, max_tokens=224)
    replay_against_oracle(orc, FUSE, t, m, prompts, 3)


@pytest.fixture
def switch_env(monkeypatch):
    # the switches are read when an engine is created and stay with it
    yield monkeypatch
    monkeypatch.undo()


@pytest.mark.parametrize("name,value,quant", SWITCHES)
def test_engine_switch_matches_oracle(orc, switch_env, name, value, quant):
    for kv in name.split(",")[:-1]:                # leading NAME=VALUE settings
        switch_env.setenv(*kv.split("="))
    switch_env.setenv(name.split(",")[-1], value)
    t = make_llama(FUSE, 4321, quant=quant, output_quant=quant)
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, FUSE.vocab, n).astype(np.int32) for n in (40, 9, 3, 1, 12, 3)]
    m = slate_amd.Llama.from_tensors(FUSE, t, max_slots=6, max_tokens=96)
    replay_against_oracle(orc, FUSE, t, m, prompts, 4)


def test_70b_layer_shapes_match_oracle(orc):
    """LLaMA-3-70B layer shapes (d 8192, 64 q / 8 kv heads, so 8 q heads per
    kv head, SwiGLU 28672), all Q4_K, two layers and a small vocabulary so
    the CPU reference stays within seconds: a ragged prompt step, then decode
    steps, each against the oracle."""
    shape = LlamaShape(n_layers=2, d_model=8192, n_heads=64, n_kv_heads=8, ffn=28672, vocab=512, max_seq=256)
    m = slate_amd.Llama.synthetic(shape, seed=70, quant=18, max_slots=3, max_tokens=64)
    rng = np.random.default_rng(70)
    prompts = [rng.integers(0, shape.vocab, n).astype(np.int32) for n in (9, 3)]
    sess = [m.session() for _ in prompts]
    rc, lg, nxt = m.step(sess, [len(p) for p in prompts], np.concatenate(prompts))
    assert rc == 0 and np.all(np.isfinite(lg))
    steps = [lg]
    toks = np.asarray(nxt, np.int32)
    for _ in range(2):
        rc, lg, nxt = m.step(sess, [1, 1], toks)
        assert rc == 0
        steps.append(lg)
        toks = np.asarray(nxt, np.int32)
    om = OracleModel(orc, shape, engine_tensors(m, shape))
    for i, p in enumerate(prompts):
        o = om.session()
        rc, want = o.prefill(p)
        assert rc == 0 and relerr(steps[0][i], want) < TOL
        tok = int(np.argmax(steps[0][i]))
        for k in range(1, len(steps)):
            rc, want = o.decode(tok)
            assert rc == 0 and relerr(steps[k][i], want) < TOL, (i, k)
            tok = int(np.argmax(steps[k][i]))
