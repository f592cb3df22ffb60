"""slate's continuous-batching scheduler over the HIP engine, unchanged: the
scheduler's own source (src/server/scheduler.c, compiled from slate's tree
into oracle/_ref and linked to slate_amd/libslate_hip_infer.so) batches
concurrent slate_scheduler_decode calls into slate_infer_batch_step
(scheduler.c:45-99, :78), which libslate_hip_infer.so runs on the device
LLaMA engine.  Eighteen sessions -- more than the scheduler's max_batch of
16 -- are prefilled concurrently through slate_infer_prefill (as the HTTP
workers do) and then decode greedily from eighteen client threads; every
logits vector is checked against the oracle replaying the same tokens
(rel 1e-3), and the scheduler must actually have batched the requests."""
import ctypes as C
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import slate_amd
from oracle.pyoracle import OracleModel, ref_available
from slate_amd.synth import LlamaShape, make_llama
from tests.helpers import relerr

pytestmark = pytest.mark.gpu
TOL = 1e-3
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCHED_SO = os.path.join(ROOT, "oracle", "_ref", "libslate_sched.so")
INFER_SO = os.path.join(ROOT, "slate_amd", "libslate_hip_infer.so")
SHAPE = LlamaShape(n_layers=2, d_model=512, n_heads=8, n_kv_heads=4, ffn=768, vocab=300, max_seq=96)
vp, i32p, f32p = C.c_void_p, C.POINTER(C.c_int32), C.POINTER(C.c_float)


@pytest.fixture(scope="module")
def libs():
    if not (ref_available() and os.path.exists(SCHED_SO)):
        pytest.skip("oracle/_ref (slate's scheduler) not built")
    slate_amd.load_library()
    inf = C.CDLL(INFER_SO)
    for name, res, args in (("slate_hip_infer_engine_new", vp, [vp]), ("slate_infer_engine_free", None, [vp]),
                            ("slate_infer_engine_vocab", C.c_int, [vp]), ("slate_infer_engine_max_seq", C.c_int, [vp]),
                            ("slate_infer_session_new", vp, [vp]), ("slate_infer_session_free", None, [vp]),
                            ("slate_infer_session_reset", None, [vp]), ("slate_infer_session_position", C.c_int, [vp]),
                            ("slate_infer_prefill", C.c_int, [vp, i32p, C.c_int, f32p]),
                            ("slate_infer_decode_step", C.c_int, [vp, C.c_int32, f32p]),
                            ("slate_infer_batch_new", vp, [vp, C.c_int]), ("slate_infer_batch_free", None, [vp]),
                            ("slate_infer_batch_step", C.c_int, [vp, C.POINTER(vp), C.c_int, i32p, f32p])):
        f = getattr(inf, name)
        f.restype, f.argtypes = res, args
    sch = C.CDLL(SCHED_SO)
    for name, res, args in (("slate_scheduler_new", vp, [vp, C.c_int]), ("slate_scheduler_free", None, [vp]),
                            ("slate_scheduler_decode", C.c_int, [vp, vp, C.c_int32, f32p]),
                            ("slate_scheduler_total_batches", C.c_uint64, [vp]),
                            ("slate_scheduler_avg_batch_size", C.c_double, [vp])):
        f = getattr(sch, name)
        f.restype, f.argtypes = res, args
    return inf, sch


def toks_p(a):
    """Pointer to an int32 array the caller keeps alive."""
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(i32p)


def test_scheduler_drives_the_hip_engine(libs, orc):
    inf, sch = libs
    t = make_llama(SHAPE, 4321, quant="q4k", output_quant="q4k")
    m = slate_amd.Llama.from_tensors(SHAPE, t, max_slots=18, max_tokens=64)
    eng = inf.slate_hip_infer_engine_new(m.h)
    assert eng and inf.slate_infer_engine_vocab(eng) == SHAPE.vocab
    assert inf.slate_infer_engine_max_seq(eng) == SHAPE.max_seq
    n, steps, V = 18, 6, SHAPE.vocab
    rng = np.random.default_rng(18)
    prompts = [rng.integers(0, V, k).astype(np.int32) for k in rng.integers(1, 20, n)]
    sess = [inf.slate_infer_session_new(eng) for _ in range(n)]
    assert all(sess)
    first = np.empty((n, V), np.float32)

    def prefill(i):
        p = prompts[i]
        return inf.slate_infer_prefill(sess[i], toks_p(p), len(p), first[i].ctypes.data_as(f32p))

    with ThreadPoolExecutor(n) as ex:             # concurrent prefills, as the HTTP workers do
        assert list(ex.map(prefill, range(n))) == [0] * n
    sched = sch.slate_scheduler_new(eng, 16)
    assert sched
    out = np.empty((n, steps, V), np.float32)
    fed = np.empty((n, steps), np.int32)

    def client(i):
        tok = int(np.argmax(first[i]))
        for k in range(steps):
            fed[i, k] = tok
            rc = sch.slate_scheduler_decode(sched, sess[i], tok, out[i, k].ctypes.data_as(f32p))
            if rc != 0:
                return rc
            tok = int(np.argmax(out[i, k]))
        return 0

    try:
        with ThreadPoolExecutor(n) as ex:
            assert list(ex.map(client, range(n))) == [0] * n
        batches = sch.slate_scheduler_total_batches(sched)
        assert batches < n * steps and sch.slate_scheduler_avg_batch_size(sched) > 1.0
    finally:
        sch.slate_scheduler_free(sched)
    assert [inf.slate_infer_session_position(s) for s in sess] == [len(p) + steps for p in prompts]
    om = OracleModel(orc, SHAPE, t)
    for i in range(n):
        o = om.session()
        rc, want = o.prefill(prompts[i])
        assert rc == 0 and relerr(first[i], want) < TOL, i
        for k in range(steps):
            rc, want = o.decode(int(fed[i, k]))
            assert rc == 0 and relerr(out[i, k], want) < TOL, (i, k)
    # reset (infer.h:116): the session starts over and recomputes its prompt
    inf.slate_infer_session_reset(sess[0])
    assert inf.slate_infer_session_position(sess[0]) == 0
    again = np.empty(V, np.float32)
    assert inf.slate_infer_prefill(sess[0], toks_p(prompts[0]), len(prompts[0]), again.ctypes.data_as(f32p)) == 0
    assert relerr(again, first[0]) < 1e-5
    # batch_step's argument and token checks (engine.c:549-559)
    b = inf.slate_infer_batch_new(eng, 4)
    arr = (vp * 2)(sess[1], sess[2])
    lg = np.empty((2, V), np.float32)
    good, bad = np.array([1, 2], np.int32), np.array([1, V], np.int32)
    assert inf.slate_infer_batch_step(b, arr, 5, toks_p(good), lg.ctypes.data_as(f32p)) == -1
    assert inf.slate_infer_batch_step(b, arr, 2, toks_p(bad), lg.ctypes.data_as(f32p)) == -3
    assert inf.slate_infer_batch_step(b, arr, 2, toks_p(good), lg.ctypes.data_as(f32p)) == 0
    inf.slate_infer_batch_free(b)
    for s in sess:
        inf.slate_infer_session_free(s)
    inf.slate_infer_engine_free(eng)
    m.free()
