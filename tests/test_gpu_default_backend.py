"""slate's unchanged callers of slate_backend_default() on the HIP backend.

oracle/_ref/libslate_default_hip.so is every source file of slate compiled
unchanged, except that slate_backend_default (backend_cpu.c:189-194) is the
chooser of slate_amd/bind/backend_default_hip.c, the text INTEGRATION.md
prints: slate_backend_hip_compat() first, then slate's own order.  Through
it, without passing any backend:

* slate's LLaMA sessions (slate_llama_session_new takes the default,
  llama_infer.c:218) prefill and decode a Q4_K model opened by slate's GGUF
  loader; their matvecs, norms and SwiGLU run on the GPU from mmap'd weights
  and calloc'd buffers.  Logits against the same calls in slate's CPU build
  (oracle/_ref/libslate_ref.so) within the parity contract's rel 1e-3.
* slate's toy engine built by the legacy constructor slate_infer_engine_new
  (NULL backend, engine.c:360-368 -> engine.c:318) against the same engine
  on slate_backend_cpu() from the same library, within 1e-4.
"""
import ctypes as C
import os

import numpy as np
import pytest

import slate_amd
from oracle.pyoracle import RefLlama, Ref, ref_available
from slate_amd.synth import LlamaShape, make_llama, write_llama_gguf
from tests.helpers import relerr

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DEFAULT_SO = os.path.join(ROOT, "oracle", "_ref", "libslate_default_hip.so")
vp, i32p, f32p = C.c_void_p, C.POINTER(C.c_int32), C.POINTER(C.c_float)
SHAPE = LlamaShape(n_layers=2, d_model=512, n_heads=8, n_kv_heads=4, ffn=768, vocab=300, max_seq=64)


@pytest.fixture(scope="module")
def dflt():
    if not (ref_available() and os.path.exists(DEFAULT_SO)):
        pytest.skip("oracle/_ref (slate's sources with the HIP default chooser) not built")
    slate_amd.load_library()             # the chooser links this same instance
    lib = C.CDLL(DEFAULT_SO)
    for name, res, args in (
            ("slate_backend_default", vp, []), ("slate_backend_cpu", vp, []),
            ("slate_gguf_open", vp, [C.c_char_p]), ("slate_gguf_close", None, [vp]),
            ("slate_llama_open", vp, [vp]), ("slate_llama_free", None, [vp]),
            ("slate_llama_session_new", vp, [vp]), ("slate_llama_session_free", None, [vp]),
            ("slate_llama_prefill", C.c_int, [vp, i32p, C.c_int, f32p]),
            ("slate_llama_decode_step", C.c_int, [vp, C.c_int32, f32p]),
            ("slate_arena_create", vp, [C.c_size_t]), ("slate_arena_destroy", None, [vp]),
            ("slate_module_causal_lm_new", vp, [vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                                C.c_uint64]),
            ("slate_infer_engine_new", vp, [vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
            ("slate_infer_engine_new_ex", vp, [vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp]),
            ("slate_infer_engine_free", None, [vp]), ("slate_infer_session_new", vp, [vp]),
            ("slate_infer_session_free", None, [vp]),
            ("slate_infer_prefill", C.c_int, [vp, i32p, C.c_int, f32p]),
            ("slate_infer_decode_step", C.c_int, [vp, C.c_int32, f32p])):
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    return lib


def backend_name(ptr):
    """The name member of a slate_backend_t (its first field, backend.h:42)."""
    return C.cast(ptr, C.POINTER(C.c_char_p))[0].decode()


def test_default_chooser_picks_the_hip_backend(dflt):
    assert backend_name(dflt.slate_backend_default()) == "hip-compat"
    assert backend_name(dflt.slate_backend_cpu()) == "cpu"


def llama_stream(lib, path, prompt, n_dec, toks=None):
    """slate_llama_prefill then n_dec greedy decode steps (tokens given, or
    the run's own argmax), through `lib`'s slate_gguf_open/slate_llama_open."""
    g = lib.slate_gguf_open(path.encode())
    assert g
    m = lib.slate_llama_open(g)
    assert m
    s = lib.slate_llama_session_new(m)
    assert s
    out = []
    lg = np.empty(SHAPE.vocab, np.float32)
    p = np.ascontiguousarray(prompt, np.int32)
    assert lib.slate_llama_prefill(s, p.ctypes.data_as(i32p), len(p), lg.ctypes.data_as(f32p)) == 0
    out.append(lg.copy())
    fed = []
    for k in range(n_dec):
        t = int(np.argmax(out[-1])) if toks is None else toks[k]
        fed.append(t)
        assert lib.slate_llama_decode_step(s, t, lg.ctypes.data_as(f32p)) == 0
        out.append(lg.copy())
    lib.slate_llama_session_free(s)
    lib.slate_llama_free(m)
    lib.slate_gguf_close(g)
    return out, fed


@pytest.mark.parametrize("quant", ["q4k", "f32"])
def test_llama_sessions_run_unchanged_on_the_default(dflt, tmp_path, quant):
    path = str(tmp_path / "model.gguf")
    write_llama_gguf(path, SHAPE, make_llama(SHAPE, 0x5EED, quant=quant, output_quant=quant))
    prompt = np.random.default_rng(5).integers(0, SHAPE.vocab, 13).astype(np.int32)
    ref = Ref()
    cpu, fed = llama_stream(ref.lib, path, prompt, 4)
    gpu, _ = llama_stream(dflt, path, prompt, 4, toks=fed)
    for k, (a, b) in enumerate(zip(gpu, cpu)):
        assert np.all(np.isfinite(a))
        assert relerr(a, b) < 1e-3, (quant, k, relerr(a, b))
    assert slate_amd.last_error() is None


def test_toy_engine_legacy_constructor_runs_on_the_default(dflt):
    vocab, max_seq, d, layers, ffn = 300, 48, 64, 3, 172
    arena = dflt.slate_arena_create(32 << 20)
    model = dflt.slate_module_causal_lm_new(arena, vocab, max_seq, d, layers, ffn, 1e-5, 0xABCD)
    assert model
    engs = [dflt.slate_infer_engine_new(model, layers, d, vocab, ffn, max_seq),          # NULL backend
            dflt.slate_infer_engine_new_ex(model, layers, d, vocab, ffn, max_seq, dflt.slate_backend_cpu())]
    assert all(engs)
    prompt = np.random.default_rng(9).integers(0, vocab, 7).astype(np.int32)
    res = []
    for eng in engs:
        s = dflt.slate_infer_session_new(eng)
        assert s
        out = []
        lg = np.empty(vocab, np.float32)
        assert dflt.slate_infer_prefill(s, prompt.ctypes.data_as(i32p), len(prompt), lg.ctypes.data_as(f32p)) == 0
        out.append(lg.copy())
        toks = [int(np.argmax(lg))] if not res else res[0][1]
        for k in range(3):
            assert dflt.slate_infer_decode_step(s, toks[k], lg.ctypes.data_as(f32p)) == 0
            out.append(lg.copy())
            if len(toks) < 3:
                toks.append(int(np.argmax(lg)))
        dflt.slate_infer_session_free(s)
        res.append((out, toks))
    for k, (a, b) in enumerate(zip(res[0][0], res[1][0])):
        assert np.all(np.isfinite(a))
        assert relerr(a, b) < 1e-4, (k, relerr(a, b))
    assert slate_amd.last_error() is None
    for eng in engs:
        dflt.slate_infer_engine_free(eng)
    dflt.slate_arena_destroy(arena)
