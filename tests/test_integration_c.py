"""The boundary as a C compiler sees it (CPU only, needs slate's include/):

* include/slate_hip.h and slate's include/slate/backend.h in either order,
  in C11 and C++, with slate's factories (backend.h:104-110) and the HIP
  one both declared;
* the loader binding slate_amd/bind/slate_llama_to_hip.c, whose text is the
  C block of the integration guide's LLaMA section, compiles against slate's
  llama.h with its struct-layout asserts, and the built binding library
  exports it;
* the default chooser slate_amd/bind/backend_default_hip.c, whose text is
  the first C block of the guide's vtable section, compiles against slate's
  backend.h, picks the compat vtable (never the device-pointer one) and is
  the chooser the harness library exports.
"""
import os
import re
import subprocess

import pytest

from tests.conftest import ROOT

REF_INCLUDE = "/root/reference/include"
BIND = os.path.join(ROOT, "slate_amd", "bind", "slate_llama_to_hip.c")
CHOOSER = os.path.join(ROOT, "slate_amd", "bind", "backend_default_hip.c")

pytestmark = pytest.mark.skipif(not os.path.isdir(REF_INCLUDE), reason="slate's headers are not mounted here")


def compile_c(tmp_path, src, lang="c"):
    f = tmp_path / ("t.c" if lang == "c" else "t.cpp")
    f.write_text(src)
    cc = ["gcc", "-std=c11"] if lang == "c" else ["g++", "-std=c++17"]
    r = subprocess.run(cc + ["-Wall", "-Werror", "-c", "-I", REF_INCLUDE, "-I", os.path.join(ROOT, "include"),
                             str(f), "-o", str(tmp_path / "t.o")], capture_output=True, text=True)
    return r.returncode, r.stderr


USE_BOTH = """
const slate_backend_t* pick(void) {
    const slate_backend_t* b = slate_backend_hip();
    return b ? b : slate_backend_cpu();
}
"""


@pytest.mark.parametrize("lang", ["c", "c++"])
@pytest.mark.parametrize("first", ["slate_hip.h", "slate/backend.h"])
def test_headers_in_either_order(tmp_path, lang, first):
    second = "slate/backend.h" if first == "slate_hip.h" else "slate_hip.h"
    rc, err = compile_c(tmp_path, f'#include "{first}"\n#include "{second}"\n' + USE_BOTH, lang)
    assert rc == 0, err


def test_header_alone_declares_the_vtable(tmp_path):
    """Without slate's include/ on the path the header declares the struct
    itself (and never slate's include guard)."""
    f = tmp_path / "u.c"
    f.write_text('#include "slate_hip.h"\nconst slate_backend_t* p(void) { return slate_backend_hip(); }\n'
                 "#ifdef SLATE_BACKEND_H\n#error the slate include guard must stay undefined\n#endif\n")
    r = subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-c", "-I", os.path.join(ROOT, "include"), str(f),
                        "-o", str(tmp_path / "u.o")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_integration_binding_is_the_shipped_file_and_compiles(tmp_path):
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    sec = doc[doc.index("## 2. The LLaMA path"):doc.index("## 3.")]
    blocks = re.findall(r"```c\n(.*?)```", sec, flags=re.S)
    assert blocks and blocks[0] == open(BIND).read()
    rc, err = compile_c(tmp_path, blocks[0])
    assert rc == 0, err
    # two same-typed config fields swapped in a copy of the header (a memcpy
    # would silently exchange the RoPE base and the RMSNorm epsilon): the
    # binding's layout asserts reject it
    hdr = open(os.path.join(ROOT, "include", "slate_hip.h")).read()
    assert "float theta_base, rms_eps;" in hdr
    inc = tmp_path / "swapped"
    inc.mkdir()
    (inc / "slate_hip.h").write_text(hdr.replace("float theta_base, rms_eps;", "float rms_eps, theta_base;"))
    f = tmp_path / "b.c"
    f.write_text(blocks[0])
    r = subprocess.run(["gcc", "-std=c11", "-c", "-I", REF_INCLUDE, "-I", str(inc), str(f), "-o",
                        str(tmp_path / "b.o")], capture_output=True, text=True)
    assert r.returncode != 0 and "theta_base" in r.stderr


def test_integration_chooser_is_the_shipped_file_and_compiles(tmp_path):
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    sec = doc[doc.index("## 1. The backend vtables"):doc.index("## 2.")]
    blocks = re.findall(r"```c\n(.*?)```", sec, flags=re.S)
    assert blocks and blocks[0] == open(CHOOSER).read()
    code = blocks[0]
    # slate's callers of the default hand it host pointers: the chooser must
    # return the compat vtable, and no line of it may call the device one
    assert "slate_backend_hip_compat()" in code
    assert not re.search(r"slate_backend_hip\s*\(", code)
    rc, err = compile_c(tmp_path, code)
    assert rc == 0, err


def test_default_harness_library_exports_the_chooser():
    so = os.path.join(ROOT, "oracle", "_ref", "libslate_default_hip.so")
    if not os.path.exists(so):
        pytest.skip("oracle/_ref not built")
    out = subprocess.run(["nm", "-D", so], capture_output=True, text=True, check=True).stdout
    assert re.search(r" T slate_backend_default$", out, flags=re.M)
    assert re.search(r" U slate_backend_hip_compat$", out, flags=re.M)


def test_binding_library_exports_the_binding():
    so = os.path.join(ROOT, "oracle", "_ref", "libslate_bind.so")
    if not os.path.exists(so):
        pytest.skip("oracle/_ref not built")
    out = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True, check=True).stdout
    assert re.search(r" T slate_llama_to_hip$", out, flags=re.M)


INFER_API = ["slate_infer_engine_free", "slate_infer_engine_vocab", "slate_infer_engine_max_seq",
             "slate_infer_session_new", "slate_infer_session_free", "slate_infer_session_reset",
             "slate_infer_session_position", "slate_infer_prefill", "slate_infer_decode_step",
             "slate_infer_batch_new", "slate_infer_batch_free", "slate_infer_batch_step"]


def test_infer_library_exports_slate_infer_api():
    """libslate_hip_infer.so defines every infer.h entry a LLaMA caller uses
    (all but the slate_module_t constructors, infer.h:74-96) plus its own
    constructor; it is linked with --no-undefined."""
    so = os.path.join(ROOT, "slate_amd", "libslate_hip_infer.so")
    out = subprocess.run(["nm", "-D", "--defined-only", so], capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert set(INFER_API) | {"slate_hip_infer_engine_new"} <= exported
    api = open(os.path.join(REF_INCLUDE, "slate", "infer.h")).read()
    declared = set(re.findall(r"\b(slate_infer_\w+)\s*\(", api))
    assert declared - set(INFER_API) == {"slate_infer_engine_new", "slate_infer_engine_new_ex"}


def test_infer_headers_compile_together(tmp_path):
    """slate's infer.h and slate_hip_infer.h declare the same opaque types,
    so a caller such as scheduler.c can use both (in C: slate's runtime.h,
    which infer.h includes, is not valid C++)."""
    src = ('#include "slate/infer.h"\n#include "slate_hip_infer.h"\n'
           "int run(slate_hip_llama_t* m, const int32_t* t, float* lg) {\n"
           "    slate_infer_engine_t* e = slate_hip_infer_engine_new(m);\n"
           "    slate_infer_batch_t* b = slate_infer_batch_new(e, 4);\n"
           "    slate_infer_session_t* s = slate_infer_session_new(e);\n"
           "    int rc = slate_infer_batch_step(b, &s, 1, t, lg);\n"
           "    slate_infer_session_free(s); slate_infer_batch_free(b); slate_infer_engine_free(e);\n"
           "    return rc;\n}\n")
    rc, err = compile_c(tmp_path, src)
    assert rc == 0, err
