"""slate_amd -- Python host side of the MI355X HIP backend for slate.

Loads ``slate_amd/libslate_hip.so`` (built from ``slate_amd/csrc`` by
``make -C slate_amd``) and exposes its C ABI (``include/slate_hip.h``):

* ``Backend``    -- the drop-in ``slate_backend_t`` vtable plus extensions,
                    with device buffers for tests and tools;
* ``Llama``      -- the device-resident LLaMA engine (sessions, prefill,
                    decode, ragged continuous-batching step).

There is no CPU fallback: if the shared library is missing or no gfx950
device is present, constructors raise.
"""
from __future__ import annotations

import ctypes as C
import os
import weakref

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libslate_hip.so")

vp = C.c_void_p
f32p = C.POINTER(C.c_float)
i32p = C.POINTER(C.c_int32)
i64p = C.POINTER(C.c_int64)


class BackendStruct(C.Structure):       # include/slate/backend.h:41-99
    _fields_ = [("name", C.c_char_p), ("alloc", vp), ("release", vp), ("copy_h2d", vp),
                ("copy_d2h", vp), ("matvec", vp), ("linear_batch", vp), ("matvec_q4k", vp),
                ("rmsnorm_row", vp), ("silu_mul", vp), ("add_inplace", vp),
                ("embed_lookup", vp), ("attention_step", vp), ("sync", vp)]


class HipBackendStruct(C.Structure):    # slate_hip_backend_t
    _fields_ = [("base", BackendStruct), ("matmul_q4k", vp), ("dequant_q4k", vp),
                ("rmsnorm_rows", vp), ("rope_rows", vp), ("argmax_rows", vp), ("last_error", vp)]


class LlamaConfig(C.Structure):         # slate_hip_llama_config_t == llama.h:53-65
    _fields_ = [("n_layers", C.c_int), ("d_model", C.c_int), ("ffn_hidden", C.c_int),
                ("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("head_dim", C.c_int),
                ("max_seq", C.c_int), ("vocab", C.c_int), ("theta_base", C.c_float),
                ("rms_eps", C.c_float), ("tied_output", C.c_int)]


class LlamaLayer(C.Structure):          # slate_hip_llama_layer_t == llama.h:69-86
    _fields_ = [(n, vp) for n in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                  "ffn_norm", "ffn_gate", "ffn_up", "ffn_down")] + \
               [(n, C.c_int) for n in ("attn_q_dtype", "attn_k_dtype", "attn_v_dtype",
                                       "attn_output_dtype", "ffn_gate_dtype", "ffn_up_dtype",
                                       "ffn_down_dtype")]


# name -> (restype, argtypes) for every exported entry point
SIGNATURES = {
    "slate_backend_hip": (C.POINTER(BackendStruct), []),
    "slate_backend_hip_compat": (C.POINTER(BackendStruct), []),
    "slate_hip_last_error": (C.c_char_p, []),
    "slate_hip_clear_error": (None, []),
    "slate_hip_stream": (vp, []),
    "slate_hip_alloc": (vp, [C.c_size_t]),
    "slate_hip_release": (None, [vp]),
    "slate_hip_copy_h2d": (None, [vp, vp, C.c_size_t]),
    "slate_hip_copy_d2h": (None, [vp, vp, C.c_size_t]),
    "slate_hip_matvec": (None, [vp, vp, vp, C.c_int, C.c_int]),
    "slate_hip_linear_batch": (None, [vp, vp, vp, C.c_int, C.c_int, C.c_int]),
    "slate_hip_matvec_q4k": (None, [vp, vp, vp, C.c_int, C.c_int]),
    "slate_hip_rmsnorm_row": (None, [vp, vp, vp, C.c_int, C.c_float]),
    "slate_hip_silu_mul": (None, [vp, vp, vp, C.c_int]),
    "slate_hip_add_inplace": (None, [vp, vp, C.c_int]),
    "slate_hip_embed_lookup": (None, [vp, vp, C.c_int, C.c_int]),
    "slate_hip_attention_step": (None, [vp, vp, vp, vp, vp, C.c_int, C.c_int]),
    "slate_hip_sync": (None, []),
    "slate_hip_matmul_q4k": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int]),
    "slate_hip_dequant_q4k": (C.c_int, [vp, vp, C.c_int64]),
    "slate_hip_q4k_tiled_bytes": (C.c_int64, [C.c_int, C.c_int]),
    "slate_hip_q4k_tile": (C.c_int, [vp, vp, C.c_int, C.c_int]),
    "slate_hip_matmul_q4k_tiled": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int]),
    "slate_hip_matmul_q4k_noalloc": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int]),
    "slate_hip_q8_0_matvec": (None, [vp, vp, vp, C.c_int, C.c_int]),
    "slate_hip_matmul_q8_0": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int]),
    "slate_hip_dequant_q8_0": (C.c_int, [vp, vp, C.c_int64]),
    "slate_hip_q8_0_tiled_bytes": (C.c_int64, [C.c_int, C.c_int]),
    "slate_hip_q8_0_tile": (C.c_int, [vp, vp, C.c_int, C.c_int]),
    "slate_hip_matmul_q8_0_tiled": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int]),
    "slate_hip_rmsnorm_rows": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_float]),
    "slate_hip_rope_rows": (C.c_int, [vp, vp, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int]),
    "slate_hip_rope_table": (None, [vp, C.c_int, C.c_int, C.c_float]),
    "slate_hip_argmax_rows": (C.c_int, [vp, vp, C.c_int, C.c_int]),
    "slate_hip_pack_batch": (C.c_int, [vp, vp, vp, C.c_int, C.c_int, C.c_int64, C.c_int,
                                       vp, vp, vp, vp, vp, vp]),
    "slate_hip_attention_ragged": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, C.c_int, C.c_int,
                                             C.c_int, C.c_int, C.c_int64, C.c_int]),
    "slate_hip_synth_f32": (C.c_int, [vp, C.c_int64, C.c_uint64, C.c_float]),
    "slate_hip_synth_q4k": (C.c_int, [vp, C.c_int64, C.c_int64, C.c_uint64, C.c_float]),
    "slate_hip_llama_new": (vp, [C.POINTER(LlamaConfig), vp, vp, vp, C.c_int,
                                 C.POINTER(LlamaLayer), C.c_int, C.c_int]),
    "slate_hip_llama_new_synthetic": (vp, [C.POINTER(LlamaConfig), C.c_uint64, C.c_int,
                                           C.c_int, C.c_int]),
    "slate_hip_llama_free": (None, [vp]),
    "slate_hip_llama_get_tensor": (C.c_int64, [vp, C.c_char_p, vp, C.c_int64, C.POINTER(C.c_int)]),
    "slate_hip_llama_session_new": (vp, [vp]),
    "slate_hip_llama_session_free": (None, [vp]),
    "slate_hip_llama_session_position": (C.c_int, [vp]),
    "slate_hip_llama_session_reset": (None, [vp]),
    "slate_hip_llama_config": (C.POINTER(LlamaConfig), [vp]),
    "slate_hip_llama_prefill": (C.c_int, [vp, vp, C.c_int, vp]),
    "slate_hip_llama_decode_step": (C.c_int, [vp, C.c_int32, vp]),
    "slate_hip_llama_step": (C.c_int, [vp, vp, C.c_int, vp, vp, vp, vp]),
    "slate_hip_llama_batch_step": (C.c_int, [vp, vp, C.c_int, vp, vp]),
    "slate_hip_llama_session_kv": (C.c_int, [vp, vp, vp]),
    "slate_hip_llama_profile": (C.c_int, [vp, C.c_int]),
    "slate_hip_llama_graphs": (C.c_int, [vp, C.c_int]),
    "slate_hip_llama_kv_f16": (C.c_int, [vp]),
    "slate_hip_llama_attn_xcd_merge": (C.c_int, [vp]),
    "slate_hip_llama_profile_read": (C.c_int, [vp, C.c_int, C.POINTER(C.c_double),
                                               C.POINTER(C.c_double), C.POINTER(C.c_int64)]),
}

_lib = None


def load_library(path: str = LIB_PATH):
    """Load libslate_hip.so (no device access).  Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `make -C slate_amd` "
                           "(or __graft_entry__.build()); there is no CPU fallback")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _ptr(a):
    return C.c_void_p(a.ctypes.data)


class HipError(RuntimeError):
    pass


def last_error():
    e = load_library().slate_hip_last_error()
    return e.decode() if e else None


def check(rc=0, what="call"):
    """Raise HipError if rc != 0 or a sticky error is pending (and clear it)."""
    lib = load_library()
    err = lib.slate_hip_last_error()
    if rc != 0 or err:
        msg = err.decode() if err else f"rc={rc}"
        lib.slate_hip_clear_error()
        raise HipError(f"{what}: {msg} (rc={rc})")


class DevicePtr(C.c_void_p):
    """A device address that keeps its DeviceBuffer alive while it exists, so
    `f(DeviceBuffer.from_array(a).p)` cannot free the memory before f runs."""


class DeviceBuffer:
    """A device allocation made through the vtable's alloc()."""

    def __init__(self, nbytes: int):
        lib = load_library()
        self.nbytes = int(nbytes)
        self.ptr = lib.slate_hip_alloc(max(self.nbytes, 1))
        if not self.ptr:
            check(-2, f"alloc({nbytes})")

    @classmethod
    def from_array(cls, a: np.ndarray):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            load_library().slate_hip_copy_h2d(b.ptr, _ptr(a), a.nbytes)
        return b

    def to_array(self, dtype, shape):
        out = np.empty(shape, dtype)
        if out.nbytes:
            load_library().slate_hip_copy_d2h(_ptr(out), self.ptr, out.nbytes)
        return out

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        load_library().slate_hip_copy_h2d(self.ptr, _ptr(a), a.nbytes)

    def free(self):
        if getattr(self, "ptr", None):
            load_library().slate_hip_release(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    @property
    def p(self):
        v = DevicePtr(self.ptr)
        v._owner = self
        return v


class Backend:
    """slate_backend_hip(): the vtable (base entries called through their
    function pointers, exactly as slate's engines would)."""

    def __init__(self):
        lib = self.lib = load_library()
        vt = lib.slate_backend_hip()
        if not vt:
            raise HipError(f"slate_backend_hip() returned NULL: {last_error()}")
        self.vt = vt.contents
        self.ext = C.cast(vt, C.POINTER(HipBackendStruct)).contents
        self.name = self.vt.name.decode()
        F = C.CFUNCTYPE
        b = self.vt
        self.alloc = F(vp, C.c_size_t)(b.alloc)
        self.release = F(None, vp)(b.release)
        self.copy_h2d = F(None, vp, vp, C.c_size_t)(b.copy_h2d)
        self.copy_d2h = F(None, vp, vp, C.c_size_t)(b.copy_d2h)
        self.matvec = F(None, vp, vp, vp, C.c_int, C.c_int)(b.matvec)
        self.linear_batch = F(None, vp, vp, vp, C.c_int, C.c_int, C.c_int)(b.linear_batch)
        self.matvec_q4k = F(None, vp, vp, vp, C.c_int, C.c_int)(b.matvec_q4k)
        self.rmsnorm_row = F(None, vp, vp, vp, C.c_int, C.c_float)(b.rmsnorm_row)
        self.silu_mul = F(None, vp, vp, vp, C.c_int)(b.silu_mul)
        self.add_inplace = F(None, vp, vp, C.c_int)(b.add_inplace)
        self.embed_lookup = F(None, vp, vp, C.c_int, C.c_int)(b.embed_lookup)
        self.attention_step = F(None, vp, vp, vp, vp, vp, C.c_int, C.c_int)(b.attention_step)
        self.sync = F(None)(b.sync)
        e = self.ext
        self.matmul_q4k = F(C.c_int, vp, vp, vp, C.c_int, C.c_int, C.c_int)(e.matmul_q4k)
        self.dequant_q4k = F(C.c_int, vp, vp, C.c_int64)(e.dequant_q4k)
        self.rmsnorm_rows = F(C.c_int, vp, vp, vp, C.c_int, C.c_int, C.c_float)(e.rmsnorm_rows)
        self.rope_rows = F(C.c_int, vp, vp, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int)(e.rope_rows)
        self.argmax_rows = F(C.c_int, vp, vp, C.c_int, C.c_int)(e.argmax_rows)

    # conveniences -----------------------------------------------------------
    def buf(self, a):
        return DeviceBuffer.from_array(a)

    def empty(self, nbytes):
        return DeviceBuffer(nbytes)


# ---------------------------------------------------------------------------
class Llama:
    """Device-resident LLaMA engine over the C ABI."""

    def __init__(self, handle, cfg: LlamaConfig):
        self.lib = load_library()
        if not handle:
            raise HipError(f"engine creation failed: {last_error()}")
        self.h = handle
        self.cfg = cfg
        self.vocab = cfg.vocab
        # sessions must be released before the engine that owns their slots
        self._sessions = weakref.WeakSet()

    @staticmethod
    def config(shape):
        return LlamaConfig(shape.n_layers, shape.d_model, shape.ffn, shape.n_heads,
                           shape.n_kv_heads, shape.head_dim, shape.max_seq, shape.vocab,
                           shape.theta, shape.eps, 0)

    @classmethod
    def from_tensors(cls, shape, tensors, max_slots=8, max_tokens=256):
        """Upload a host model (slate_amd.synth.make_llama layout)."""
        lib = load_library()
        cfg = cls.config(shape)
        layers = (LlamaLayer * shape.n_layers)()
        keep = []
        for i in range(shape.n_layers):
            L = layers[i]
            for n in ("attn_norm", "ffn_norm"):
                a = np.ascontiguousarray(tensors[f"blk.{i}.{n}.weight"][0])
                keep.append(a)
                setattr(L, n, a.ctypes.data)
            for n in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"):
                a, dt, _ = tensors[f"blk.{i}.{n}.weight"]
                a = np.ascontiguousarray(a)
                keep.append(a)
                setattr(L, n, a.ctypes.data)
                setattr(L, n + "_dtype", dt)
        te = np.ascontiguousarray(tensors["token_embd.weight"][0], np.float32)
        on = np.ascontiguousarray(tensors["output_norm.weight"][0], np.float32)
        out, odt, _ = tensors["output.weight"]
        out = np.ascontiguousarray(out)
        h = lib.slate_hip_llama_new(C.byref(cfg), _ptr(te), _ptr(on), _ptr(out), odt, layers,
                                    max_slots, max_tokens)
        return cls(h, cfg)

    @classmethod
    def synthetic(cls, shape, seed, quant=18, max_slots=16, max_tokens=256):
        lib = load_library()
        cfg = cls.config(shape)
        h = lib.slate_hip_llama_new_synthetic(C.byref(cfg), seed, quant, max_slots, max_tokens)
        return cls(h, cfg)

    def free(self):
        if getattr(self, "h", None):
            for s in list(self._sessions):
                s.free()
            self.lib.slate_hip_llama_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def get_tensor(self, name):
        dt = C.c_int(0)
        n = self.lib.slate_hip_llama_get_tensor(self.h, name.encode(), None, 0, C.byref(dt))
        if n < 0:
            raise KeyError(name)
        buf = np.empty(n, np.uint8)
        r = self.lib.slate_hip_llama_get_tensor(self.h, name.encode(), _ptr(buf), n, C.byref(dt))
        check(0 if r == n else r, f"get_tensor({name})")
        return buf, dt.value

    def tensor_dtype(self, name):
        """slate dtype of a weight (no copy)."""
        dt = C.c_int(0)
        if self.lib.slate_hip_llama_get_tensor(self.h, name.encode(), None, 0, C.byref(dt)) < 0:
            raise KeyError(name)
        return dt.value

    def session(self):
        return Session(self)

    def profile(self, enable=True, reset=True):
        """Start (reset=True: from zero; False: keep the totals) or stop
        recording kernel-class timings."""
        mode = (1 if reset else 2) if enable else 0
        check(self.lib.slate_hip_llama_profile(self.h, mode), "profile")

    def graphs(self, enable=True):
        """Replay decode-only steps from captured HIP graphs (default off)."""
        check(self.lib.slate_hip_llama_graphs(self.h, 1 if enable else 0), "graphs")

    def profile_read(self):
        """{class: (device ms, algorithmic bytes, launches)}; *_pf classes are
        launches in steps that carry prompt chunks (or matmuls over > 16 rows)."""
        out = {}
        for cls, name in enumerate(("q4k_mm", "attention", "step", "q4k_mm_pf", "attention_pf", "step_pf")):
            ms, by, n = C.c_double(), C.c_double(), C.c_int64()
            self.lib.slate_hip_llama_profile_read(self.h, cls, C.byref(ms), C.byref(by), C.byref(n))
            out[name] = (ms.value, by.value, n.value)
        return out

    def step(self, sessions, n_new, tokens, want_logits=True):
        n = len(sessions)
        arr = (vp * n)(*[s.h for s in sessions])
        nn = np.ascontiguousarray(n_new, np.int32)
        tk = np.ascontiguousarray(tokens, np.int32)
        lg = np.empty((n, self.vocab), np.float32) if want_logits else None
        nx = np.empty(n, np.int32)
        rc = self.lib.slate_hip_llama_step(self.h, arr, n, _ptr(nn), _ptr(tk),
                                           _ptr(lg) if want_logits else None, _ptr(nx))
        return rc, lg, nx


class Session:
    def __init__(self, m: Llama):
        self.m = m
        self.h = m.lib.slate_hip_llama_session_new(m.h)
        if not self.h:
            raise HipError(f"session_new failed: {last_error()}")
        m._sessions.add(self)

    def free(self):
        if getattr(self, "h", None):
            if self.m.h:   # the engine frees its live sessions first
                self.m.lib.slate_hip_llama_session_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    @property
    def position(self):
        return self.m.lib.slate_hip_llama_session_position(self.h)

    def prefill(self, toks):
        toks = np.ascontiguousarray(toks, np.int32)
        lg = np.empty(self.m.vocab, np.float32)
        rc = self.m.lib.slate_hip_llama_prefill(self.h, _ptr(toks), len(toks), _ptr(lg))
        return rc, lg

    def decode(self, tok):
        lg = np.empty(self.m.vocab, np.float32)
        rc = self.m.lib.slate_hip_llama_decode_step(self.h, int(tok), _ptr(lg))
        return rc, lg

    def kv(self):
        c = self.m.cfg
        n = c.n_layers * c.max_seq * c.n_kv_heads * c.head_dim
        K = np.empty(n, np.float32)
        V = np.empty(n, np.float32)
        rc = self.m.lib.slate_hip_llama_session_kv(self.h, _ptr(K), _ptr(V))
        check(rc, "session_kv")
        shp = (c.n_layers, c.max_seq, c.n_kv_heads * c.head_dim)
        return K.reshape(shp), V.reshape(shp)
