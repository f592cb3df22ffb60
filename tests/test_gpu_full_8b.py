"""The LLaMA-3-8B-shaped model at full size, the headline configuration: 32
layers, d_model 4096, 32 q / 8 kv heads (head_dim 128), SwiGLU 14336,
vocabulary 128256, every linear Q4_K from N(0, 0.02) (generated on the
device), embeddings f32, norms 1.

Sixteen sequences with contexts U[128, 2048] are prefilled on the GPU in
ragged prompt steps, then decoded together for two steps.  Each sequence's
logits of both steps are checked against slate's own decode step
(slate_llama_decode_step, llama_infer.c:134-206) started from the GPU's KV
cache after the prefill -- compiled from slate's sources (oracle/_ref),
sixteen sessions at a time over slate's threadpool -- or, where those are
not built, against the oracle's restatement of it: normwise rel 1e-3, and
greedy tokens equal unless the reference's top-2 gap is below that.  The
reference feeds the GPU's first greedy token into its second step, so the
second step also compares the reference's own K/V append with the GPU's.
A third, mixed step (the decode tokens beside a new sequence's 300-token
prompt, all rows on the prompt kernels) is checked the same way, and the new
sequence's logits against its prompt prefilled alone (1e-4).  Then every
sequence takes a 32-token prompt chunk in one step, against slate's
token-serial prefill of the same tokens from the reference's own state: the
K/V rows written in every layer (1e-4) and the last logits (1e-3).  One sequence
prefilled and decoded alone gets the logits it gets in the batch (within
1e-4), and the whole run repeated in fresh sessions gets the same bits."""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import slate_amd
from oracle.pyoracle import OracleModel, Ref, RefLlama, ref_available
from slate_amd.synth import LlamaShape, engine_tensors, write_llama_gguf
from tests.helpers import relerr

pytestmark = pytest.mark.gpu
TOL = 1e-3
SHAPE = LlamaShape(n_layers=32, d_model=4096, n_heads=32, n_kv_heads=8, ffn=14336, vocab=128256, max_seq=2304)
NSEQ, MAX_TOKENS = 16, 4096
HOST_THREADS = 16            # the GPU box's CPU share per GPU


def gap_ok(ref_logits):
    s = np.sort(ref_logits.astype(np.float64))
    return (s[-1] - s[-2]) > TOL * max(np.abs(ref_logits).max(), 1e-30)


def prefill_ragged(m, sess, prompts):
    """Prompts packed into ragged steps of at most MAX_TOKENS tokens; returns
    each sequence's greedy next token."""
    nxt, todo = [None] * len(sess), list(range(len(sess)))
    while todo:
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
    return nxt


class Reference:
    """Reference sessions started from the GPU sessions' KV caches and
    positions; decode(toks) runs one decode step of all of them."""

    def __init__(self, m, sess):
        self.path = None
        pos = [s.position for s in sess]
        if ref_available():
            os.environ.setdefault("SLATE_NUM_THREADS", str(HOST_THREADS))
            self.ref = Ref()
            self.path = "/dev/shm/slate_amd_test_8b.gguf"
            write_llama_gguf(self.path, SHAPE, engine_tensors(m, SHAPE))
            self.rm = RefLlama(self.ref, self.path)
            self.rs = [self.rm.session() for _ in range(NSEQ)]
        else:
            from oracle.pyoracle import Oracle
            self.om = OracleModel(Oracle(), SHAPE, engine_tensors(m, SHAPE))
            self.rs = [self.om.session() for _ in range(NSEQ)]
        for i in range(NSEQ):
            K, V = sess[i].kv()
            assert self.rs[i].set_state(K, V, pos[i]) == 0
            del K, V

    def decode(self, toks):
        out = np.empty((NSEQ, SHAPE.vocab), np.float32)
        t = np.ascontiguousarray(toks, np.int32)
        if self.path:
            arr = (slate_amd.vp * NSEQ)(*[r.h for r in self.rs])
            rc = np.zeros(NSEQ, np.int32)
            self.ref.lib.ref_decode_sessions_parallel(arr, t.ctypes.data_as(slate_amd.i32p), NSEQ,
                                                      out.ctypes.data_as(slate_amd.f32p),
                                                      rc.ctypes.data_as(slate_amd.i32p))
            assert not rc.any(), rc
            return out

        def run(i):
            rc, out[i] = self.rs[i].decode(int(t[i]))
            assert rc == 0

        with ThreadPoolExecutor(HOST_THREADS) as ex:
            list(ex.map(run, range(NSEQ)))
        return out

    def close(self):
        if self.path:
            for r in self.rs:
                r.free()
            self.rm.close()
            os.unlink(self.path)
            self.path = None


def test_8b_full_size_decode_matches_reference():
    m = slate_amd.Llama.synthetic(SHAPE, seed=2026, quant=18, max_slots=NSEQ + 2, max_tokens=MAX_TOKENS)
    rng = np.random.default_rng(0xC4)
    prompts = [rng.integers(0, SHAPE.vocab, n).astype(np.int32) for n in rng.integers(128, 2049, NSEQ)]
    sess = [m.session() for _ in range(NSEQ)]
    toks0 = prefill_ragged(m, sess, prompts)
    assert [s.position for s in sess] == [len(p) for p in prompts]
    ref = Reference(m, sess)
    try:
        rc, lg1, nx1 = m.step(sess, [1] * NSEQ, np.asarray(toks0, np.int32))
        assert rc == 0 and np.all(np.isfinite(lg1))
        rc, lg2, nx2 = m.step(sess, [1] * NSEQ, nx1)
        assert rc == 0 and np.all(np.isfinite(lg2))
        for k, (lg, nx, toks) in enumerate(((lg1, nx1, toks0), (lg2, nx2, nx1))):
            want = ref.decode(toks)
            for i in range(NSEQ):
                assert relerr(lg[i], want[i]) < TOL, (k, i, relerr(lg[i], want[i]))
                assert int(nx[i]) == int(np.argmax(lg[i]))
                assert int(nx[i]) == int(np.argmax(want[i])) or not gap_ok(want[i]), (k, i)
        # a mixed step, as an arrival makes one: the 16 decode tokens ride with
        # a new sequence's 300-token prompt (every row on the prompt kernels)
        arrival = rng.integers(0, SHAPE.vocab, 300).astype(np.int32)
        new = m.session()
        rc, lg3, nx3 = m.step(sess + [new], [1] * NSEQ + [len(arrival)], np.concatenate([nx2, arrival]))
        assert rc == 0 and np.all(np.isfinite(lg3))
        want = ref.decode(nx2)
        for i in range(NSEQ):
            assert relerr(lg3[i], want[i]) < TOL, (i, relerr(lg3[i], want[i]))
            assert int(nx3[i]) == int(np.argmax(want[i])) or not gap_ok(want[i]), i
        alone = m.session()
        rc, la = alone.prefill(arrival)
        assert rc == 0 and relerr(lg3[NSEQ], la) < 1e-4
        alone.free()
        new.free()
        # prompt chunks at the full shape: a 32-token chunk at every
        # sequence's position (contexts ~130-2050) in one step of 512 rows
        # (the MFMA prompt GEMM, RoPE + K/V append of prompt rows, the MFMA
        # prompt attention) against slate's prefill of the same tokens, 32
        # token-serial decode steps (llama_infer.c:262-272) from the
        # reference's own state: the 32 K/V rows written in every layer
        # (rel 1e-4 per layer) and each sequence's last logits (rel 1e-3)
        chunk = rng.integers(0, SHAPE.vocab, (NSEQ, 32)).astype(np.int32)
        p0 = [s.position for s in sess]
        rc, lg4, nx4 = m.step(sess, [32] * NSEQ, chunk.reshape(-1))
        assert rc == 0 and np.all(np.isfinite(lg4))
        for k in range(32):
            want = ref.decode(chunk[:, k])
        for i in range(NSEQ):
            assert relerr(lg4[i], want[i]) < TOL, (i, relerr(lg4[i], want[i]))
            assert int(nx4[i]) == int(np.argmax(want[i])) or not gap_ok(want[i]), i
            K, V = sess[i].kv()
            Kr, Vr = ref.rs[i].kv()
            rows = slice(p0[i], p0[i] + 32)
            for li in range(SHAPE.n_layers):
                ek, ev = relerr(K[li, rows], Kr[li, rows]), relerr(V[li, rows], Vr[li, rows])
                assert ek < 1e-4 and ev < 1e-4, (i, li, ek, ev)
            del K, V, Kr, Vr
    finally:
        ref.close()
    # batch invariance: the first sequence alone
    solo = m.session()
    rc, _ = solo.prefill(prompts[0])
    assert rc == 0
    for lg, tok in ((lg1, toks0[0]), (lg2, int(nx1[0]))):
        rc, l1 = solo.decode(tok)
        assert rc == 0 and relerr(l1, lg[0]) < 1e-4
    solo.free()
    for s in sess:
        s.free()
    # run to run: the same prompts and steps in fresh sessions give the same
    # bits (every reduction of the path runs in a fixed order; the decode
    # attention's arrival counts only pick which unit merges)
    sess = [m.session() for _ in range(NSEQ)]
    assert prefill_ragged(m, sess, prompts) == toks0
    rc, r1, n1 = m.step(sess, [1] * NSEQ, np.asarray(toks0, np.int32))
    assert rc == 0
    rc, r2, n2 = m.step(sess, [1] * NSEQ, n1)
    assert rc == 0
    assert np.array_equal(r1, lg1) and np.array_equal(r2, lg2) and np.array_equal(n2, nx2)
    for s in sess:
        s.free()
    m.free()
