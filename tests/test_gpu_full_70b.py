"""The LLaMA-3-70B-shaped serving workload's kernels at full size, against
slate's own decode step.

Model: 80 layers, d_model 8192, 64 q / 8 kv heads (head_dim 128), SwiGLU
28672, vocabulary 128256, every linear Q4_K from N(0, 0.02) generated on the
device (~39 GB), embeddings f32, norms 1.  As the serving workload runs it:
32 sequences at contexts of 1536-2048 tokens (prefilled in ragged prompt
steps), then

* a mixed step: 31 decode tokens beside one sequence's second prompt chunk
  of 384 tokens at position ~1.5-2k (415 rows: the prompt GEMM's two-tile
  plan, RoPE + K/V append of prompt rows, the MFMA prompt attention with 8
  q heads per kv head at positions in the thousands);
* a decode step of all 32 (32 rows: the decode GEMM with two activation
  tiles at d 8192, the decode attention on the phased kernel).

Checked against slate_llama_decode_step (llama_infer.c:134-206, compiled
from slate's sources into oracle/_ref; sessions spread over slate's
threadpool) started from the GPU's K/V state at the right position:
* three decode sequences: the logits of both steps (rel 1e-3, greedy tokens
  equal unless the reference's top-2 gap is below that);
* the chunked sequence, token by token at sampled chunk positions q (first
  and last tokens, both sides of the 16-token query blocks and of the
  256-key chunk boundary): the reference decodes chunk token q from the
  state holding the GPU's rows before it and writes the K/V row at q in all
  80 layers, compared with the GPU's (rel 1e-4 per layer); at the chunk's
  last token also the mixed step's logits (1e-3), and then the decode step's;
* two other sequences decoded alone on the GPU: the logits they get in the
  batch (1e-4).
Without oracle/_ref the test is skipped (the oracle would need ~10 minutes
per token at this size).
"""
import os

import numpy as np
import pytest

import slate_amd
from oracle.pyoracle import Ref, RefLlama, ref_available
from slate_amd.synth import LlamaShape, engine_tensors, write_llama_gguf
from tests.helpers import relerr

pytestmark = pytest.mark.gpu
TOL = 1e-3
SHAPE = LlamaShape(n_layers=80, d_model=8192, n_heads=64, n_kv_heads=8, ffn=28672, vocab=128256, max_seq=2560)
NSEQ, CHUNK, MAX_TOKENS = 32, 384, 4096
CHUNKED = 3                                    # the sequence carrying the prompt chunk
CHECKED = (0, 1, 2)                            # decode sequences checked against the reference
SOLO = (17, 31)                                # decode sequences checked alone on the GPU
SAMPLE_Q = (0, 1, 15, 16, 17, 255, 256, 383)   # chunk positions checked against the reference
HOST_THREADS = 16


def gap_ok(ref_logits):
    s = np.sort(ref_logits.astype(np.float64))
    return (s[-1] - s[-2]) > TOL * max(np.abs(ref_logits).max(), 1e-30)


@pytest.fixture(scope="module")
def c5():
    if not ref_available():
        pytest.skip("oracle/_ref not built: the reference is needed at this size")
    m = slate_amd.Llama.synthetic(SHAPE, seed=75, quant=18, max_slots=NSEQ + 1, max_tokens=MAX_TOKENS)
    rng = np.random.default_rng(0xC5)
    prompts = [rng.integers(0, SHAPE.vocab, n).astype(np.int32) for n in rng.integers(1536, 2049, NSEQ)]
    chunk = rng.integers(0, SHAPE.vocab, CHUNK).astype(np.int32)
    sess = [m.session() for _ in range(NSEQ)]
    nxt, todo = [None] * NSEQ, list(range(NSEQ))
    while todo:                                # ragged prompt steps of <= MAX_TOKENS rows
        group, T = [], 0
        for i in todo:
            if T + len(prompts[i]) <= MAX_TOKENS:
                group.append(i)
                T += len(prompts[i])
        todo = [i for i in todo if i not in group]
        rc, _, nx = m.step([sess[i] for i in group], [len(prompts[i]) for i in group],
                           np.concatenate([prompts[i] for i in group]), want_logits=False)
        assert rc == 0, slate_amd.last_error()
        for i, t in zip(group, nx):
            nxt[i] = int(t)
    pos = [s.position for s in sess]
    # the mixed step: decode tokens, and the chunked sequence's next 384 prompt tokens
    n_new = [CHUNK if i == CHUNKED else 1 for i in range(NSEQ)]
    toks = np.concatenate([chunk if i == CHUNKED else [nxt[i]] for i in range(NSEQ)]).astype(np.int32)
    rc, lg1, nx1 = m.step(sess, n_new, toks)
    assert rc == 0 and np.all(np.isfinite(lg1)), slate_amd.last_error()
    rc, lg2, nx2 = m.step(sess, [1] * NSEQ, np.asarray(nx1, np.int32))
    assert rc == 0 and np.all(np.isfinite(lg2)), slate_amd.last_error()
    st = dict(m=m, sess=sess, prompts=prompts, chunk=chunk, pos=pos, nxt=nxt, lg1=lg1, nx1=nx1, lg2=lg2,
              nx2=nx2)
    yield st
    for s in sess:
        s.free()
    m.free()


def test_70b_serving_steps_match_reference(c5):
    os.environ.setdefault("SLATE_NUM_THREADS", str(HOST_THREADS))
    m, sess, pos = c5["m"], c5["sess"], c5["pos"]
    path = "/dev/shm/slate_amd_test_70b.gguf"
    write_llama_gguf(path, SHAPE, engine_tensors(m, SHAPE, lazy=True))   # one tensor in host memory at a time
    ref = Ref()
    rm = RefLlama(ref, path)
    rs = []
    try:
        # decode sequences: from the state before the mixed step
        for i in CHECKED:
            K, V = sess[i].kv()
            r = rm.session()
            assert r.set_state(K, V, pos[i]) == 0
            rs.append(r)
            del K, V
        # the chunked sequence: one session per sampled chunk position q,
        # holding the GPU's rows before p0 + q
        p0 = pos[CHUNKED]
        K, V = sess[CHUNKED].kv()
        for q in SAMPLE_Q:
            r = rm.session()
            assert r.set_state(K, V, p0 + q) == 0
            rs.append(r)
        Kc, Vc = K[:, p0:p0 + CHUNK].copy(), V[:, p0:p0 + CHUNK].copy()
        del K, V
        toks = [c5["nxt"][i] for i in CHECKED] + [int(c5["chunk"][q]) for q in SAMPLE_Q]
        want = decode_parallel(ref, rs, toks)
        for k, i in enumerate(CHECKED):
            w, g = want[k], c5["lg1"][i]
            assert relerr(g, w) < TOL, (i, relerr(g, w))
            assert int(c5["nx1"][i]) == int(np.argmax(w)) or not gap_ok(w), i
        for k, q in enumerate(SAMPLE_Q):
            r = rs[len(CHECKED) + k]
            Kr, Vr = r.kv()
            for li in range(SHAPE.n_layers):
                ek = relerr(Kc[li, q], Kr[li, p0 + q])
                ev = relerr(Vc[li, q], Vr[li, p0 + q])
                assert ek < 1e-4 and ev < 1e-4, (q, li, ek, ev)
            del Kr, Vr
        w, g = want[len(CHECKED) + len(SAMPLE_Q) - 1], c5["lg1"][CHUNKED]
        assert relerr(g, w) < TOL, ("chunk", relerr(g, w))
        assert int(c5["nx1"][CHUNKED]) == int(np.argmax(w)) or not gap_ok(w)
        # the decode step: the checked sequences and the chunked one (from its
        # last chunk position's session)
        last = rs[:len(CHECKED)] + [rs[-1]]
        want = decode_parallel(ref, last, [int(c5["nx1"][i]) for i in CHECKED + (CHUNKED,)])
        for k, i in enumerate(CHECKED + (CHUNKED,)):
            w, g = want[k], c5["lg2"][i]
            assert relerr(g, w) < TOL, (i, relerr(g, w))
            assert int(c5["nx2"][i]) == int(np.argmax(w)) or not gap_ok(w), i
    finally:
        for r in rs:
            r.free()
        rm.close()
        os.unlink(path)


def decode_parallel(ref, rs, toks):
    """One slate_llama_decode_step per session, sessions over slate's pool."""
    n = len(rs)
    out = np.empty((n, SHAPE.vocab), np.float32)
    t = np.ascontiguousarray(toks, np.int32)
    rc = np.zeros(n, np.int32)
    arr = (slate_amd.vp * n)(*[r.h for r in rs])
    ref.lib.ref_decode_sessions_parallel(arr, t.ctypes.data_as(slate_amd.i32p), n,
                                         out.ctypes.data_as(slate_amd.f32p), rc.ctypes.data_as(slate_amd.i32p))
    assert not rc.any(), rc
    return out


def test_70b_serving_steps_are_batch_invariant(c5):
    """A sequence prefilled and decoded alone gets, within 1e-4, the logits it
    got in the 32-sequence steps (a ~2k-token prefill and a 415-row mixed step
    split K differently; the rounding of the two compounds over 80 layers)."""
    m = c5["m"]
    for i in SOLO:
        s = m.session()
        rc, _ = s.prefill(c5["prompts"][i])
        assert rc == 0
        rc, l1 = s.decode(c5["nxt"][i])
        assert rc == 0 and relerr(l1, c5["lg1"][i]) < 1e-4, (i, relerr(l1, c5["lg1"][i]))
        rc, l2 = s.decode(int(c5["nx1"][i]))
        assert rc == 0 and relerr(l2, c5["lg2"][i]) < 1e-4, (i, relerr(l2, c5["lg2"][i]))
        s.free()
