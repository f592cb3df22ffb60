"""ctypes bindings for the CPU checker (test infrastructure).

``Oracle`` wraps ``oracle/liboracle.so`` (the C restatement).  ``Ref`` wraps
``oracle/_ref/libslate_ref.so`` (slate's own sources compiled in place) and is
only available where that file was built.  Only tests/, smoke() and bench.py's
CPU-baseline leg use this module, and only to check or time the CPU path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libslate_ref.so")

f32p = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int32)
i64p = C.POINTER(C.c_int64)
vp = C.c_void_p


def fp(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(f32p)


def ip(a):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(i32p)


def bp(a):
    return C.c_void_p(a.ctypes.data)


class CfgStruct(C.Structure):       # llama.h:53-65 field order
    _fields_ = [("n_layers", C.c_int), ("d_model", C.c_int), ("ffn_hidden", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int),
                ("max_seq", C.c_int), ("vocab", C.c_int), ("theta_base", C.c_float),
                ("rms_eps", C.c_float), ("tied_output", C.c_int)]


class LayerStruct(C.Structure):     # llama.h:69-86 field order
    _fields_ = [(n, vp) for n in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                  "ffn_norm", "ffn_gate", "ffn_up", "ffn_down")] + \
               [(n, C.c_int) for n in ("attn_q_dtype", "attn_k_dtype", "attn_v_dtype",
                                       "attn_output_dtype", "ffn_gate_dtype", "ffn_up_dtype",
                                       "ffn_down_dtype")]


class ModelStruct(C.Structure):
    _fields_ = [("cfg", CfgStruct), ("token_embd", f32p), ("output_norm", f32p),
                ("output", vp), ("output_dtype", C.c_int), ("layers", C.POINTER(LayerStruct))]


class PackOut(C.Structure):
    _fields_ = [("tok_off", i32p), ("tok2seq", i32p), ("tok_pos", i32p),
                ("kv_base", i64p), ("last_tok", i32p)]


def _sig(lib, name, res, *args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = list(args)
    return f


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        _sig(L, "orc_f16_to_f32", C.c_float, C.c_uint16)
        _sig(L, "orc_f16_to_f32_n", None, f32p, C.c_void_p, C.c_int64)
        _sig(L, "orc_q4k_scale_min", None, C.c_void_p, C.c_int, C.POINTER(C.c_uint8), C.POINTER(C.c_uint8))
        _sig(L, "orc_dequant_q4k", None, f32p, vp, C.c_int64)
        _sig(L, "orc_dot_q4k_f32", C.c_float, vp, f32p, C.c_int64)
        _sig(L, "orc_q4k_matvec", None, f32p, vp, f32p, C.c_int, C.c_int)
        _sig(L, "orc_q4k_matmul", None, f32p, vp, f32p, C.c_int, C.c_int, C.c_int)
        _sig(L, "orc_dequant_q8_0", None, f32p, vp, C.c_int64)
        _sig(L, "orc_dot_q8_0_f32", C.c_float, vp, f32p, C.c_int64)
        _sig(L, "orc_q8_0_matmul", None, f32p, vp, f32p, C.c_int, C.c_int, C.c_int)
        _sig(L, "orc_matvec", None, f32p, f32p, f32p, C.c_int, C.c_int)
        _sig(L, "orc_linear_batch", None, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int)
        _sig(L, "orc_rmsnorm_row", None, f32p, f32p, f32p, C.c_int, C.c_float)
        _sig(L, "orc_silu_mul", None, f32p, f32p, f32p, C.c_int)
        _sig(L, "orc_add_inplace", None, f32p, f32p, C.c_int)
        _sig(L, "orc_embed_lookup", None, f32p, f32p, C.c_int, C.c_int)
        _sig(L, "orc_attention_step", None, f32p, f32p, f32p, f32p, f32p, C.c_int, C.c_int)
        _sig(L, "orc_rope_row", None, f32p, C.c_int, C.c_int, C.c_int, C.c_float)
        _sig(L, "orc_attention_multihead", None, f32p, f32p, f32p, f32p, f32p,
             C.c_int, C.c_int, C.c_int, C.c_int)
        _sig(L, "orc_argmax", C.c_int, f32p, C.c_int)
        _sig(L, "orc_pack_batch", C.c_int, i32p, i32p, i32p, C.c_int, C.c_int, C.c_int64,
             C.POINTER(PackOut))
        _sig(L, "orc_session_new", vp, C.POINTER(ModelStruct))
        _sig(L, "orc_session_free", None, vp)
        _sig(L, "orc_session_position", C.c_int, vp)
        _sig(L, "orc_decode_step", C.c_int, vp, C.c_int32, f32p)
        _sig(L, "orc_prefill", C.c_int, vp, i32p, C.c_int, f32p)
        _sig(L, "orc_session_kv", None, vp, f32p, f32p)
        _sig(L, "orc_session_set_state", C.c_int, vp, f32p, f32p, C.c_int)

    # -- numpy conveniences ------------------------------------------------
    def dequant_q4k(self, raw, n):
        raw = np.ascontiguousarray(np.frombuffer(bytes(raw), np.uint8))
        out = np.empty(n, np.float32)
        self.lib.orc_dequant_q4k(fp(out), bp(raw), n)
        return out

    def q4k_matmul(self, raw, X, M, K):
        raw = np.ascontiguousarray(np.frombuffer(bytes(raw), np.uint8)) if not isinstance(raw, np.ndarray) else raw
        X = np.ascontiguousarray(X, np.float32).reshape(-1, K)
        Y = np.empty((X.shape[0], M), np.float32)
        self.lib.orc_q4k_matmul(fp(Y), bp(raw), fp(X), X.shape[0], M, K)
        return Y

    def dequant_q8_0(self, raw, n):
        raw = np.ascontiguousarray(np.frombuffer(bytes(raw), np.uint8))
        out = np.empty(n, np.float32)
        self.lib.orc_dequant_q8_0(fp(out), bp(raw), n)
        return out

    def q8_0_matmul(self, raw, X, M, K):
        raw = np.ascontiguousarray(np.frombuffer(bytes(raw), np.uint8)) if not isinstance(raw, np.ndarray) else raw
        X = np.ascontiguousarray(X, np.float32).reshape(-1, K)
        Y = np.empty((X.shape[0], M), np.float32)
        self.lib.orc_q8_0_matmul(fp(Y), bp(raw), fp(X), X.shape[0], M, K)
        return Y

    def pack_batch(self, slot, pos0, n_new, max_seq, slot_stride):
        slot, pos0, n_new = (np.ascontiguousarray(a, np.int32) for a in (slot, pos0, n_new))
        B = len(slot)
        T = int(max(n_new.sum(), 1))
        bufs = dict(tok_off=np.zeros(B + 1, np.int32), tok2seq=np.zeros(T, np.int32),
                    tok_pos=np.zeros(T, np.int32), kv_base=np.zeros(B, np.int64),
                    last_tok=np.zeros(B, np.int32))
        po = PackOut(ip(bufs["tok_off"]), ip(bufs["tok2seq"]), ip(bufs["tok_pos"]),
                     bufs["kv_base"].ctypes.data_as(i64p), ip(bufs["last_tok"]))
        rc = self.lib.orc_pack_batch(ip(slot), ip(pos0), ip(n_new), B, max_seq, slot_stride, C.byref(po))
        return rc, bufs


class OracleModel:
    """orc_llama_model over host arrays from slate_amd.synth.make_llama."""

    def __init__(self, orc: Oracle, shape, tensors):
        self.orc, self.shape, self._keep = orc, shape, tensors
        s = shape
        cfg = CfgStruct(s.n_layers, s.d_model, s.ffn, s.n_heads, s.n_kv_heads, s.head_dim,
                        s.max_seq, s.vocab, s.theta, s.eps, 0)
        self.layers = (LayerStruct * s.n_layers)()
        for i in range(s.n_layers):
            L = self.layers[i]
            for n in ("attn_norm", "ffn_norm"):
                setattr(L, n, tensors[f"blk.{i}.{n}.weight"][0].ctypes.data)
            for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"):
                a, dt, _ = tensors[f"blk.{i}.{n}.weight"]
                setattr(L, n, a.ctypes.data)
                setattr(L, n + "_dtype", dt)
        out, odt, _ = tensors["output.weight"]
        self.model = ModelStruct(cfg, fp(tensors["token_embd.weight"][0]),
                                 fp(tensors["output_norm.weight"][0]), out.ctypes.data, odt,
                                 self.layers)

    def session(self):
        return OracleSession(self)


class OracleSession:
    def __init__(self, m: OracleModel):
        self.m = m
        self.h = m.orc.lib.orc_session_new(C.byref(m.model))
        if not self.h:
            raise MemoryError("orc_session_new failed")

    def __del__(self):
        if getattr(self, "h", None):
            self.m.orc.lib.orc_session_free(self.h)
            self.h = None

    @property
    def position(self):
        return self.m.orc.lib.orc_session_position(self.h)

    def prefill(self, toks):
        toks = np.ascontiguousarray(toks, np.int32)
        lg = np.empty(self.m.shape.vocab, np.float32)
        rc = self.m.orc.lib.orc_prefill(self.h, ip(toks), len(toks), fp(lg))
        return rc, lg

    def decode(self, tok):
        lg = np.empty(self.m.shape.vocab, np.float32)
        rc = self.m.orc.lib.orc_decode_step(self.h, int(tok), fp(lg))
        return rc, lg

    def set_state(self, K, V, pos):
        return self.m.orc.lib.orc_session_set_state(self.h, fp(np.ascontiguousarray(K, np.float32)),
                                                    fp(np.ascontiguousarray(V, np.float32)), pos)

    def kv(self):
        s = self.m.shape
        n = s.n_layers * s.max_seq * s.kv_dim
        K = np.empty(n, np.float32)
        V = np.empty(n, np.float32)
        self.m.orc.lib.orc_session_kv(self.h, fp(K), fp(V))
        return K.reshape(s.n_layers, s.max_seq, s.kv_dim), V.reshape(s.n_layers, s.max_seq, s.kv_dim)


# ---------------------------------------------------------------------------
class BackendStruct(C.Structure):   # include/slate/backend.h:41-99
    _fields_ = [("name", C.c_char_p), ("alloc", vp), ("release", vp), ("copy_h2d", vp),
                ("copy_d2h", vp), ("matvec", vp), ("linear_batch", vp), ("matvec_q4k", vp),
                ("rmsnorm_row", vp), ("silu_mul", vp), ("add_inplace", vp),
                ("embed_lookup", vp), ("attention_step", vp), ("sync", vp)]


def ref_available():
    return os.path.exists(REF_SO)


class Ref:
    """slate's own C code (built from its sources into oracle/_ref)."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        _sig(L, "slate_f16_to_f32", C.c_float, C.c_uint16)
        _sig(L, "slate_dequant_q4_k", None, f32p, vp, C.c_int64)
        _sig(L, "slate_dot_q4_k_f32", C.c_float, vp, f32p, C.c_int64)
        _sig(L, "slate_q4_k_matvec", None, f32p, vp, f32p, C.c_int, C.c_int)
        _sig(L, "slate_dequant_q8_0", None, f32p, vp, C.c_int64)
        _sig(L, "slate_dot_q8_0_f32", C.c_float, vp, f32p, C.c_int64)
        _sig(L, "slate_q8_0_matvec", None, f32p, vp, f32p, C.c_int, C.c_int)
        _sig(L, "ref_rope_inplace_row", None, f32p, C.c_int, C.c_int, C.c_int, C.c_float)
        _sig(L, "ref_attention_multihead", None, f32p, f32p, f32p, f32p, f32p,
             C.c_int, C.c_int, C.c_int, C.c_int)
        _sig(L, "slate_backend_cpu", C.POINTER(BackendStruct))
        _sig(L, "slate_gguf_open", vp, C.c_char_p)
        _sig(L, "slate_gguf_close", None, vp)
        _sig(L, "slate_llama_open", vp, vp)
        _sig(L, "slate_llama_free", None, vp)
        _sig(L, "slate_llama_config", C.POINTER(CfgStruct), vp)
        _sig(L, "slate_llama_session_new", vp, vp)
        _sig(L, "slate_llama_session_free", None, vp)
        _sig(L, "slate_llama_session_position", C.c_int, vp)
        _sig(L, "slate_llama_prefill", C.c_int, vp, i32p, C.c_int, f32p)
        _sig(L, "slate_llama_decode_step", C.c_int, vp, C.c_int32, f32p)
        _sig(L, "ref_session_set_state", C.c_int, vp, f32p, f32p, C.c_int)
        _sig(L, "ref_session_get_kv", C.c_int, vp, f32p, f32p)
        _sig(L, "ref_decode_sessions_parallel", None, C.POINTER(vp), i32p, C.c_int, f32p, i32p)
        _sig(L, "ref_pool_threads", C.c_int)
        be = L.slate_backend_cpu().contents
        self.cpu = be
        T = C.CFUNCTYPE
        self.matvec = T(None, f32p, f32p, f32p, C.c_int, C.c_int)(be.matvec)
        self.linear_batch = T(None, f32p, f32p, f32p, C.c_int, C.c_int, C.c_int)(be.linear_batch)
        self.rmsnorm_row = T(None, f32p, f32p, f32p, C.c_int, C.c_float)(be.rmsnorm_row)
        self.silu_mul = T(None, f32p, f32p, f32p, C.c_int)(be.silu_mul)
        self.add_inplace = T(None, f32p, f32p, C.c_int)(be.add_inplace)
        self.embed_lookup = T(None, f32p, f32p, C.c_int, C.c_int)(be.embed_lookup)
        self.attention_step = T(None, f32p, f32p, f32p, f32p, f32p, C.c_int, C.c_int)(be.attention_step)


class RefLlama:
    """slate_gguf_open -> slate_llama_open -> sessions, on slate's own code."""

    def __init__(self, ref: Ref, path):
        self.ref = ref
        self.g = ref.lib.slate_gguf_open(path.encode())
        if not self.g:
            raise IOError(f"slate_gguf_open({path}) failed")
        self.m = ref.lib.slate_llama_open(self.g)
        if not self.m:
            raise IOError("slate_llama_open failed")
        self.cfg = ref.lib.slate_llama_config(self.m).contents

    def close(self):
        if self.m:
            self.ref.lib.slate_llama_free(self.m)
            self.m = None
        if self.g:
            self.ref.lib.slate_gguf_close(self.g)
            self.g = None

    def session(self):
        return RefSession(self)


class RefSession:
    def __init__(self, m: RefLlama):
        self.m = m
        self.h = m.ref.lib.slate_llama_session_new(m.m)
        if not self.h:
            raise MemoryError("slate_llama_session_new failed")

    def free(self):
        if self.h:
            self.m.ref.lib.slate_llama_session_free(self.h)
            self.h = None

    __del__ = free

    def prefill(self, toks):
        toks = np.ascontiguousarray(toks, np.int32)
        lg = np.empty(self.m.cfg.vocab, np.float32)
        rc = self.m.ref.lib.slate_llama_prefill(self.h, ip(toks), len(toks), fp(lg))
        return rc, lg

    def decode(self, tok):
        lg = np.empty(self.m.cfg.vocab, np.float32)
        rc = self.m.ref.lib.slate_llama_decode_step(self.h, int(tok), fp(lg))
        return rc, lg

    def set_state(self, K, V, pos):
        return self.m.ref.lib.ref_session_set_state(self.h, fp(K), fp(V), pos)

    def kv(self):
        """The session's K/V caches, [n_layers, max_seq, kv_dim] each."""
        c = self.m.cfg
        shp = (c.n_layers, c.max_seq, c.n_kv_heads * c.head_dim)
        K = np.empty(shp, np.float32)
        V = np.empty(shp, np.float32)
        assert self.m.ref.lib.ref_session_get_kv(self.h, fp(K), fp(V)) == 0
        return K, V
