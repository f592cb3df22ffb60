"""The C ABI: the shared library loads and exports every entry point that
include/slate_hip.h declares, with the vtable laid out as slate's
slate_backend_t (include/slate/backend.h:41-99).  CPU only: no kernel runs."""
import ctypes as C
import os
import re
import subprocess

import pytest

import slate_amd
from tests.conftest import ROOT

HEADER = os.path.join(ROOT, "include", "slate_hip.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = set(re.findall(r"\b(slate_(?:hip_\w+|backend_hip\w*))\s*\(", src))
    # drop struct members written as (*name)(...)
    return sorted(n for n in names if not re.search(r"\(\*\s*" + n + r"\)", src))


def test_header_declares_the_entry_points():
    names = declared_functions()
    assert "slate_backend_hip" in names
    assert "slate_hip_matmul_q4k" in names and "slate_hip_llama_step" in names
    assert len(names) >= 35


def test_library_exports_every_declared_symbol():
    lib = slate_amd.load_library()
    out = subprocess.run(["nm", "-D", "--defined-only", slate_amd.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    for n in declared_functions():
        getattr(lib, n)


def test_python_signatures_cover_the_header():
    assert set(declared_functions()) == set(slate_amd.SIGNATURES)


def test_vtable_layout_matches_slate_backend_t():
    """Member order of backend.h:41-99; the extension struct starts with it."""
    order = ["name", "alloc", "release", "copy_h2d", "copy_d2h", "matvec", "linear_batch",
             "matvec_q4k", "rmsnorm_row", "silu_mul", "add_inplace", "embed_lookup",
             "attention_step", "sync"]
    assert [f[0] for f in slate_amd.BackendStruct._fields_] == order
    ps = C.sizeof(C.c_void_p)
    assert C.sizeof(slate_amd.BackendStruct) == 14 * ps
    assert slate_amd.HipBackendStruct.base.offset == 0
    assert slate_amd.HipBackendStruct.matmul_q4k.offset == 14 * ps
    # the C declaration has the same members in the same order
    src = open(HEADER).read()
    body = src[src.index("typedef struct slate_backend {"):src.index("} slate_backend_t;")]
    members = re.findall(r"\(\*(\w+)\)|const char\* (name);", body)
    assert [a or b for a, b in members] == order


def test_engine_structs_match_llama_h():
    """slate_hip_llama_config_t / _layer_t keep llama.h:53-86 field order."""
    cfg = [f[0] for f in slate_amd.LlamaConfig._fields_]
    assert cfg == ["n_layers", "d_model", "ffn_hidden", "n_heads", "n_kv_heads", "head_dim",
                   "max_seq", "vocab", "theta_base", "rms_eps", "tied_output"]
    assert C.sizeof(slate_amd.LlamaLayer) == 9 * C.sizeof(C.c_void_p) + 8 * 4


def test_missing_library_fails_loudly(tmp_path):
    import importlib
    mod = importlib.reload(slate_amd)
    saved = mod._lib
    mod._lib = None
    try:
        with pytest.raises(RuntimeError, match="no CPU fallback"):
            mod.load_library(str(tmp_path / "absent.so"))
    finally:
        mod._lib = saved


class _RecordingLib:
    """Stands in for the library to watch the wrapper's call order."""

    def __init__(self):
        self.calls = []
        self.next = 100

    def slate_hip_llama_session_new(self, h):
        self.next += 1
        self.calls.append(("new", self.next))
        return self.next

    def slate_hip_llama_session_free(self, h):
        self.calls.append(("session_free", h))

    def slate_hip_llama_free(self, h):
        self.calls.append(("engine_free", h))


def test_engine_free_releases_live_sessions_first():
    """A session never reaches slate_hip_llama_session_free after its engine
    is gone (the engine's slot list would be freed memory by then)."""
    lib = _RecordingLib()
    m = object.__new__(slate_amd.Llama)
    m.lib, m.h, m._sessions = lib, 7, __import__("weakref").WeakSet()
    a, b = slate_amd.Session(m), slate_amd.Session(m)
    a.free()
    m.free()
    b.free()            # after the engine: no call
    del a, b
    assert lib.calls == [("new", 101), ("new", 102), ("session_free", 101), ("session_free", 102),
                         ("engine_free", 7)]
