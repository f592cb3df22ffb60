"""slate's own toy inference engine (src/infer/engine.c, compiled unchanged
from slate's sources into oracle/_ref/libslate_full.so) running on the HIP
backend's compatibility vtable, slate_backend_hip_compat(), against the same
engine on slate's CPU backend (slate_backend_cpu, backend_cpu.c:170).

The toy engine memcpy's the new K/V rows into backend-allocated caches and
memsets them (engine.c:276-277, 411-412, 586-591) and passes its module's
weights, which live in ordinary host memory, to the compute entries; the
compat vtable allocates pinned host memory and stages the rest.  The model
is slate_module_causal_lm_new with test_infer.c's shape and a larger one;
prefill, greedy decode steps and a ragged batch step of three sessions at
different positions must give the CPU backend's logits within 1e-4
relative (the f32 sums run in another order)."""
import ctypes as C
import os

import numpy as np
import pytest

import slate_amd
from oracle.pyoracle import ref_available
from tests.helpers import relerr

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FULL_SO = os.path.join(ROOT, "oracle", "_ref", "libslate_full.so")
vp, i32p, f32p = C.c_void_p, C.POINTER(C.c_int32), C.POINTER(C.c_float)


@pytest.fixture(scope="module")
def full():
    if not (ref_available() and os.path.exists(FULL_SO)):
        pytest.skip("oracle/_ref (slate's full sources) not built")
    lib = C.CDLL(FULL_SO)
    for name, res, args in (
            ("slate_arena_create", vp, [C.c_size_t]), ("slate_arena_destroy", None, [vp]),
            ("slate_module_causal_lm_new", vp, [vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                                C.c_uint64]),
            ("slate_backend_cpu", vp, []),
            ("slate_infer_engine_new_ex", vp, [vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, vp]),
            ("slate_infer_engine_free", None, [vp]), ("slate_infer_session_new", vp, [vp]),
            ("slate_infer_session_free", None, [vp]), ("slate_infer_session_position", C.c_int, [vp]),
            ("slate_infer_prefill", C.c_int, [vp, i32p, C.c_int, f32p]),
            ("slate_infer_decode_step", C.c_int, [vp, C.c_int32, f32p]),
            ("slate_infer_batch_new", vp, [vp, C.c_int]), ("slate_infer_batch_free", None, [vp]),
            ("slate_infer_batch_step", C.c_int, [vp, C.POINTER(vp), C.c_int, i32p, f32p])):
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    return lib


@pytest.mark.parametrize("vocab,max_seq,d,layers,ffn", [(32, 16, 16, 2, 32), (300, 48, 64, 3, 172)])
def test_toy_engine_runs_unchanged_on_the_compat_backend(full, vocab, max_seq, d, layers, ffn):
    hip = slate_amd.load_library().slate_backend_hip_compat()
    assert hip, slate_amd.last_error()
    arena = full.slate_arena_create(32 << 20)
    model = full.slate_module_causal_lm_new(arena, vocab, max_seq, d, layers, ffn, 1e-5, 0xABCD)
    assert model
    engs = [full.slate_infer_engine_new_ex(model, layers, d, vocab, ffn, max_seq, b)
            for b in (full.slate_backend_cpu(), C.cast(hip, vp).value)]
    assert all(engs)
    rng = np.random.default_rng(vocab + d)
    prompts = [rng.integers(0, vocab, n).astype(np.int32) for n in (5, 1, 9)]
    res = []
    for eng in engs:
        out, sess = [], []
        for p in prompts:
            s = full.slate_infer_session_new(eng)
            assert s
            lg = np.empty(vocab, np.float32)
            assert full.slate_infer_prefill(s, p.ctypes.data_as(i32p), len(p), lg.ctypes.data_as(f32p)) == 0
            out.append(lg)
            sess.append(s)
        # greedy decode steps of the first session, tokens from the CPU run
        toks = [int(np.argmax(out[0]))] if not res else [int(t) for t in res[0][1]]
        for k in range(4):
            lg = np.empty(vocab, np.float32)
            assert full.slate_infer_decode_step(sess[0], toks[k], lg.ctypes.data_as(f32p)) == 0
            out.append(lg)
            if len(toks) < 4:
                toks.append(int(np.argmax(lg)))
        # one ragged batch step: three sessions at positions 9, 1 and 9
        b = full.slate_infer_batch_new(eng, 4)
        arr = (vp * 3)(*sess)
        bt = np.array([3, 7, 11], np.int32)
        blg = np.empty((3, vocab), np.float32)
        assert full.slate_infer_batch_step(b, arr, 3, bt.ctypes.data_as(i32p), blg.ctypes.data_as(f32p)) == 0
        out.extend(blg)
        assert [full.slate_infer_session_position(s) for s in sess] == [len(prompts[0]) + 5, 2, 10]
        full.slate_infer_batch_free(b)
        for s in sess:
            full.slate_infer_session_free(s)
        res.append((out, toks))
    for i, (a, c) in enumerate(zip(res[1][0], res[0][0])):
        assert np.all(np.isfinite(a))
        assert relerr(a, c) < 1e-4, (i, relerr(a, c))
    assert slate_amd.last_error() is None
    for eng in engs:
        full.slate_infer_engine_free(eng)
    full.slate_arena_destroy(arena)
