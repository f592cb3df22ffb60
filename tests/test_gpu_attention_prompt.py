"""Attention of prompt tokens on the MFMA prompt kernel (k_attn_mfma.hip),
through the engine, against the oracle (llama_infer.c:97-129 per token).

Each shape runs a ragged prompt step whose prompt lengths straddle the
kernel's 16-token query blocks and 32-key blocks (1, 2, 15, 16, 17, 33, 70),
then a mixed step where some sessions decode one token and the others take a
second prompt chunk at a nonzero position (chunked prefill: query blocks
whose first key block holds the earlier chunk), then decode steps.  Every
logits row must match the oracle within 1e-3 (normwise relative, the parity
contract of the engine tests), and the same steps on the tokenwise decode
kernel (SLATE_HIP_ATTN_MFMA=0; the MFMA run sets 2, which sends every step
with prompt chunks to the MFMA kernel) within 1e-4: the kernel's f16 hi/lo operands
carry ~22 bits of each value, so the two paths differ by f32 rounding only.
Shapes cover head_dim 64 and 128 with 1, 2, 4 and 8 query heads per KV head.
"""
import numpy as np
import pytest

import slate_amd
from oracle.pyoracle import OracleModel
from slate_amd.synth import LlamaShape, make_llama
from tests.helpers import relerr

pytestmark = pytest.mark.gpu
TOL = 1e-3
PATH_TOL = 1e-4

SHAPES = {
    "hd64_g1": LlamaShape(n_layers=2, d_model=256, n_heads=4, n_kv_heads=4, ffn=512, vocab=300, max_seq=128),
    "hd64_g2": LlamaShape(n_layers=2, d_model=512, n_heads=8, n_kv_heads=4, ffn=512, vocab=300, max_seq=128),
    "hd128_g4": LlamaShape(n_layers=2, d_model=1024, n_heads=8, n_kv_heads=2, ffn=512, vocab=300, max_seq=128),
    "hd128_g8": LlamaShape(n_layers=2, d_model=2048, n_heads=16, n_kv_heads=2, ffn=512, vocab=300, max_seq=128),
}
FIRST = (1, 2, 15, 16, 17, 33, 70)
SECOND = {3: 5, 4: 16, 5: 31, 6: 40}          # session -> second chunk length


@pytest.fixture
def mfma_off(monkeypatch):
    yield monkeypatch
    monkeypatch.undo()
    # switches are read at engine creation: restore the defaults
    slate_amd.Llama.synthetic(LlamaShape(1, 256, 2, 2, 256, 16, 16), seed=1, quant=0, max_slots=1,
                              max_tokens=1).free()


def run_steps(shape, t, feed=None):
    """The three kinds of steps; returns per-step logits and the token feed
    (argmax of this run unless `feed` is given)."""
    m = slate_amd.Llama.from_tensors(shape, t, max_slots=len(FIRST), max_tokens=160)
    rng = np.random.default_rng(shape.d_model + shape.n_heads)
    prompts = [rng.integers(0, shape.vocab, n).astype(np.int32) for n in FIRST]
    chunks = {i: rng.integers(0, shape.vocab, n).astype(np.int32) for i, n in SECOND.items()}
    sess = [m.session() for _ in prompts]
    out, fed = [], []
    rc, lg, nxt = m.step(sess, list(FIRST), np.concatenate(prompts))
    assert rc == 0
    out.append(lg)
    toks = list(nxt) if feed is None else feed[0]
    fed.append(toks)
    n_new = [SECOND.get(i, 1) for i in range(len(sess))]
    flat = np.concatenate([chunks[i] if i in chunks else np.array([toks[i]], np.int32) for i in range(len(sess))])
    rc, lg, nxt = m.step(sess, n_new, flat)
    assert rc == 0
    out.append(lg)
    for k in range(2):
        toks = list(nxt) if feed is None else feed[k + 1]
        fed.append(toks)
        rc, lg, nxt = m.step(sess, [1] * len(sess), np.asarray(toks, np.int32))
        assert rc == 0
        out.append(lg)
    for s in sess:
        s.free()
    m.free()
    return out, fed, prompts, chunks


@pytest.mark.parametrize("name", list(SHAPES))
def test_prompt_attention_matches_oracle_and_tokenwise_path(orc, mfma_off, name):
    shape = SHAPES[name]
    t = make_llama(shape, 77, quant="q4k", output_quant="q4k")
    # every step with prompt chunks on the MFMA kernel (by default the mixed
    # step's choice depends on its prompt and decode work)
    mfma_off.setenv("SLATE_HIP_ATTN_MFMA", "2")
    out, fed, prompts, chunks = run_steps(shape, t)
    om = OracleModel(orc, shape, t)
    for i, p in enumerate(prompts):
        o = om.session()
        rc, want = o.prefill(p)
        assert rc == 0 and relerr(out[0][i], want) < TOL, (name, i, 0)
        if i in chunks:
            rc, want = o.prefill(chunks[i])
        else:
            rc, want = o.decode(int(fed[0][i]))
        assert rc == 0 and relerr(out[1][i], want) < TOL, (name, i, 1)
        for k in range(2):
            rc, want = o.decode(int(fed[k + 1][i]))
            assert rc == 0 and relerr(out[k + 2][i], want) < TOL, (name, i, k + 2)
    mfma_off.setenv("SLATE_HIP_ATTN_MFMA", "0")
    other, _, _, _ = run_steps(shape, t, feed=fed)
    for k, (a, b) in enumerate(zip(out, other)):
        for i in range(len(prompts)):
            assert relerr(a[i], b[i]) < PATH_TOL, (name, k, i, relerr(a[i], b[i]))
    assert slate_amd.last_error() is None
