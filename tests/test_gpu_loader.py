"""slate's loader in front of the HIP engine: a GGUF written by
slate_amd.gguf is opened by slate's own slate_gguf_open + slate_llama_open
(gguf.c:122-224, llama.c:42-140, compiled from slate's sources into
oracle/_ref), and the model's mmap views go to slate_hip_llama_new through
the binding slate_amd/bind/slate_llama_to_hip.c.  The engine's logits
against slate's own decode of the same file (slate_llama_prefill /
slate_llama_decode_step) for an untied Q4_K model and a tied-output model
(no output.weight: llama.c:94-101), and against the oracle's corrected
dispatch for a Q8_0 model (llama_infer.c:43-51 reads dtype 16 as f32).
Tolerance: the parity contract's rel 1e-3, with greedy tokens equal unless
the reference's top-2 gap is below it."""
import ctypes as C
import os

import numpy as np
import pytest

import slate_amd
from oracle.pyoracle import OracleModel, Ref, RefLlama, ref_available
from slate_amd.synth import LlamaShape, make_llama, write_llama_gguf
from tests.helpers import relerr

pytestmark = pytest.mark.gpu
TOL = 1e-3
BIND_SO = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref",
                       "libslate_bind.so")
SHAPE = LlamaShape(n_layers=2, d_model=512, n_heads=8, n_kv_heads=4, ffn=768, vocab=300, max_seq=96)


@pytest.fixture(scope="module")
def bind():
    if not (ref_available() and os.path.exists(BIND_SO)):
        pytest.skip("oracle/_ref (slate's loader and the binding) not built")
    slate_amd.load_library()            # the binding links this same instance
    lib = C.CDLL(BIND_SO)
    lib.slate_llama_to_hip.restype = C.c_void_p
    lib.slate_llama_to_hip.argtypes = [C.c_void_p, C.c_int, C.c_int]
    return lib, Ref()


def gap_ok(ref_logits):
    s = np.sort(ref_logits.astype(np.float64))
    return (s[-1] - s[-2]) > TOL * max(np.abs(ref_logits).max(), 1e-30)


def run_case(bind, tmp_path, tensors, want_fn):
    lib, ref = bind
    path = str(tmp_path / "model.gguf")
    write_llama_gguf(path, SHAPE, tensors)
    rm = RefLlama(ref, path)
    try:
        h = lib.slate_llama_to_hip(rm.m, 3, 64)
        assert h, slate_amd.last_error()
        cfg = slate_amd.LlamaConfig(*[getattr(rm.cfg, f) for f, _ in slate_amd.LlamaConfig._fields_])
        m = slate_amd.Llama(h, cfg)
    finally:
        rm.close()                      # the engine holds its own copies
    rng = np.random.default_rng(77)
    prompts = [rng.integers(0, SHAPE.vocab, n).astype(np.int32) for n in (11, 4, 23)]
    sess = [m.session() for _ in prompts]
    rc, lg, nxt = m.step(sess, [len(p) for p in prompts], np.concatenate(prompts))
    assert rc == 0
    steps, toks = [lg], np.asarray(nxt, np.int32)
    for _ in range(4):
        rc, lg, nxt = m.step(sess, [1] * len(prompts), toks)
        assert rc == 0
        steps.append(lg)
        toks = np.asarray(nxt, np.int32)
    for i, p in enumerate(prompts):
        want = want_fn(path, p, [int(np.argmax(s[i])) for s in steps[:-1]])
        for k, w in enumerate(want):
            assert relerr(steps[k][i], w) < TOL, (i, k)
            assert int(np.argmax(steps[k][i])) == int(np.argmax(w)) or not gap_ok(w), (i, k)
    for s in sess:
        s.free()
    m.free()
    return cfg


def ref_stream(bind):
    """slate's own prefill + decode of the GGUF, replaying the engine's tokens."""
    def want(path, prompt, toks):
        rm = RefLlama(bind[1], path)
        try:
            s = rm.session()
            rc, lg = s.prefill(prompt)
            assert rc == 0
            out = [lg]
            for t in toks:
                rc, lg = s.decode(t)
                assert rc == 0
                out.append(lg)
            s.free()
            return out
        finally:
            rm.close()
    return want


def test_loader_q4k_untied(bind, tmp_path):
    t = make_llama(SHAPE, 601, quant="q4k", output_quant="q4k")
    cfg = run_case(bind, tmp_path, t, ref_stream(bind))
    assert cfg.tied_output == 0


def test_loader_tied_output(bind, tmp_path):
    t = make_llama(SHAPE, 602, quant="q4k", output_quant="f32")
    del t["output.weight"]              # slate_llama_open falls back to token_embd
    cfg = run_case(bind, tmp_path, t, ref_stream(bind))
    assert cfg.tied_output == 1


def test_loader_q8_0(bind, orc, tmp_path):
    t = make_llama(SHAPE, 603, quant="q8_0", output_quant="q8_0")
    om = OracleModel(orc, SHAPE, t)

    def want(path, prompt, toks):
        o = om.session()
        rc, lg = o.prefill(prompt)
        assert rc == 0
        out = [lg]
        for tk in toks:
            rc, lg = o.decode(tk)
            assert rc == 0
            out.append(lg)
        return out
    run_case(bind, tmp_path, t, want)


def test_loader_refuses_quantised_embeddings(bind, tmp_path):
    """The engine reads f32 token embeddings (llama_infer.c:149-150): the
    binding returns NULL for a Q8_0 token_embd instead of reading past it."""
    from slate_amd.synth import quantize_q8_0
    t = make_llama(SHAPE, 604, quant="q4k", output_quant="q4k")
    a, _, shp = t["token_embd.weight"]
    t["token_embd.weight"] = (np.frombuffer(quantize_q8_0(a), np.uint8), 16, shp)
    path = str(tmp_path / "model.gguf")
    write_llama_gguf(path, SHAPE, t)
    rm = RefLlama(bind[1], path)
    try:
        assert not bind[0].slate_llama_to_hip(rm.m, 2, 16)
    finally:
        rm.close()
