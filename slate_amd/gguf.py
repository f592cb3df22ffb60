"""GGUF v3 writer/reader for LLaMA-format models (host side).

Writes files that slate's own loader opens unchanged (src/loader/gguf.c:122-186,
src/loader/llama.c:42-140): little-endian header, typed key/value metadata,
tensor-info table with dims stored innermost-first, data aligned to
``general.alignment``.  ``llama.vocab_size`` is always written because the
loader's fallback reads ``shape[0]``, which is the innermost dim
(llama.c:103-106 with gguf.c:164-167).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = 0x46554747
T_U32, T_F32, T_STRING = 4, 6, 8
GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K = 0, 1, 8, 12
# slate_dtype_t values (include/slate/types.h:29-39)
SLATE_F32, SLATE_F16, SLATE_Q8_0, SLATE_Q4_K = 0, 1, 16, 18
_GGML_TO_SLATE = {GGML_F32: SLATE_F32, GGML_F16: SLATE_F16,
                  GGML_Q8_0: SLATE_Q8_0, GGML_Q4_K: SLATE_Q4_K}


def _nbytes(ggml_type: int, numel: int) -> int:
    if ggml_type == GGML_F32:
        return numel * 4
    if ggml_type == GGML_F16:
        return numel * 2
    if ggml_type == GGML_Q8_0:
        return numel // 32 * 34
    if ggml_type == GGML_Q4_K:
        return numel // 256 * 144
    raise ValueError(f"unsupported ggml type {ggml_type}")


@dataclass
class TensorEntry:
    name: str
    shape: tuple          # outermost-first, e.g. (out, in)
    ggml_type: int
    data: object          # bytes, or a callable returning an array or bytes


@dataclass
class GGUFWriter:
    alignment: int = 32
    kv: list = field(default_factory=list)
    tensors: list = field(default_factory=list)

    def add_u32(self, key, v):
        self.kv.append((key, T_U32, int(v)))

    def add_f32(self, key, v):
        self.kv.append((key, T_F32, float(v)))

    def add_str(self, key, v):
        self.kv.append((key, T_STRING, str(v)))

    def add_tensor(self, name, shape, ggml_type, data):
        """data: an array or bytes, or a callable returning one, called when
        the file is written (so a large model streams through host memory one
        tensor at a time)."""
        numel = int(np.prod(shape))
        if callable(data):
            raw = data
        else:
            raw = data.tobytes() if isinstance(data, np.ndarray) else bytes(data)
            if len(raw) != _nbytes(ggml_type, numel):
                raise ValueError(f"{name}: {len(raw)} bytes, expected {_nbytes(ggml_type, numel)}")
        self.tensors.append(TensorEntry(name, tuple(int(s) for s in shape), ggml_type, raw))

    @staticmethod
    def _payload(te):
        """The tensor's bytes (fetched now for a lazy tensor), size-checked."""
        data = te.data() if callable(te.data) else te.data
        mv = memoryview(np.ascontiguousarray(data) if isinstance(data, np.ndarray) else data).cast("B")
        want = _nbytes(te.ggml_type, int(np.prod(te.shape)))
        if mv.nbytes != want:
            raise ValueError(f"{te.name}: {mv.nbytes} bytes, expected {want}")
        return mv

    @staticmethod
    def _str(s: str) -> bytes:
        b = s.encode()
        return struct.pack("<Q", len(b)) + b

    def write(self, path):
        hdr = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, 3, len(self.tensors), len(self.kv) + 1))
        hdr += self._str("general.alignment") + struct.pack("<II", T_U32, self.alignment)
        for key, t, v in self.kv:
            hdr += self._str(key) + struct.pack("<I", t)
            if t == T_U32:
                hdr += struct.pack("<I", v)
            elif t == T_F32:
                hdr += struct.pack("<f", v)
            else:
                hdr += self._str(v)
        off = 0
        offsets = []
        for te in self.tensors:
            off = (off + self.alignment - 1) // self.alignment * self.alignment
            offsets.append(off)
            off += _nbytes(te.ggml_type, int(np.prod(te.shape)))
        for te, o in zip(self.tensors, offsets):
            hdr += self._str(te.name) + struct.pack("<I", len(te.shape))
            for d in reversed(te.shape):          # innermost first
                hdr += struct.pack("<Q", d)
            hdr += struct.pack("<IQ", te.ggml_type, o)
        pad = (-len(hdr)) % self.alignment
        hdr += b"\0" * pad
        with open(path, "wb") as f:
            f.write(hdr)
            pos = 0
            for te, o in zip(self.tensors, offsets):
                f.write(b"\0" * (o - pos))
                mv = self._payload(te)
                f.write(mv)
                pos = o + mv.nbytes
                del mv


class GGUFFile:
    """Minimal reader (memory-mapped) used by tests and the model loader."""

    def __init__(self, path):
        self.path = path
        self.buf = np.memmap(path, dtype=np.uint8, mode="r")
        mv = memoryview(self.buf)
        p = 0

        def rd(fmt):
            nonlocal p
            v = struct.unpack_from(fmt, mv, p)
            p += struct.calcsize(fmt)
            return v

        def rstr():
            (n,) = rd("<Q")
            nonlocal p
            s = bytes(mv[p:p + n]).decode()
            p += n
            return s

        magic, version, n_t, n_kv = rd("<IIQQ")
        if magic != GGUF_MAGIC or version not in (2, 3):
            raise ValueError("not a GGUF v2/v3 file")
        self.kv = {}
        self.alignment = 32
        for _ in range(n_kv):
            key = rstr()
            (t,) = rd("<I")
            if t == T_U32:
                (v,) = rd("<I")
            elif t == T_F32:
                (v,) = rd("<f")
            elif t == T_STRING:
                v = rstr()
            else:
                raise ValueError(f"unsupported kv type {t} for {key}")
            self.kv[key] = v
            if key == "general.alignment":
                self.alignment = v
        self.tensors = {}
        for _ in range(n_t):
            name = rstr()
            (nd,) = rd("<I")
            dims = rd("<" + "Q" * nd)
            t, off = rd("<IQ")
            self.tensors[name] = (tuple(reversed(dims)), t, off)
        self.data_off = (p + self.alignment - 1) // self.alignment * self.alignment

    def raw(self, name) -> np.ndarray:
        shape, t, off = self.tensors[name]
        n = _nbytes(t, int(np.prod(shape)))
        a = self.data_off + off
        return self.buf[a:a + n]

    def slate_dtype(self, name) -> int:
        return _GGML_TO_SLATE[self.tensors[name][1]]
