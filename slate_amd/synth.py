"""Seeded synthetic LLaMA-shaped models and host-side Q4_K / Q8_0 quantizers.

The quantizer writes slate's Q4_K layout (src/util/quant.c:135-166): 144-byte
super-blocks of [f16 d][f16 dmin][12-byte packed 6-bit scales/mins][128 bytes
of nibbles], where sub-block j takes qs[16j..16j+15] with the low nibble of
byte i as element i and the high nibble as element i+16.  The scale/min
search is this project's own (per sub-block min/max, then 6-bit codes against
the block maxima); any valid encoding serves, since parity is checked on the
bytes it produces.  Q8_0 (quant.c:12-25) is 34-byte blocks of [f16 d][32 x
int8 q] with w = d * q; the encoder takes d = max|w| / 127 per block.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .gguf import GGML_F32, GGML_Q4_K, GGML_Q8_0, GGUFWriter, SLATE_F32, SLATE_Q4_K, SLATE_Q8_0

QK = 256
BLOCK_BYTES = 144
Q8_ELEMS = 32
Q8_BYTES = 34


def pack_scales(qsc: np.ndarray, qmn: np.ndarray) -> np.ndarray:
    """[..., 8] 6-bit scale/min codes -> [..., 12] bytes (inverse of
    quant.c:157-166)."""
    qsc = qsc.astype(np.uint8)
    qmn = qmn.astype(np.uint8)
    s = np.zeros(qsc.shape[:-1] + (12,), np.uint8)
    for j in range(4):
        s[..., j] = (qsc[..., j] & 63) | ((qsc[..., j + 4] >> 4) << 6)
        s[..., j + 4] = (qmn[..., j] & 63) | ((qmn[..., j + 4] >> 4) << 6)
        s[..., j + 8] = (qsc[..., j + 4] & 15) | ((qmn[..., j + 4] & 15) << 4)
    return s


def quantize_q4k(w: np.ndarray) -> bytes:
    """Quantize f32 [M, K] (K % 256 == 0) row-major to Q4_K bytes."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    M, K = w.shape
    assert K % QK == 0
    nb = K // QK
    x = w.reshape(M, nb, 8, 32)
    wmin = x.min(-1)
    wmax = x.max(-1)
    mn = np.maximum(-wmin, 0.0).astype(np.float32)          # offset >= 0
    sc = ((wmax + mn) / 15.0).astype(np.float32)             # step >= 0
    d16 = (sc.max(-1) / 63.0).astype(np.float16)
    dm16 = (mn.max(-1) / 63.0).astype(np.float16)
    d = d16.astype(np.float32)[..., None]
    dm = dm16.astype(np.float32)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        qsc = np.where(d > 0, np.clip(np.rint(sc / d), 0, 63), 0).astype(np.uint8)
        qmn = np.where(dm > 0, np.clip(np.rint(mn / dm), 0, 63), 0).astype(np.uint8)
        step = (d * qsc.astype(np.float32))[..., None]
        off = (dm * qmn.astype(np.float32))[..., None]
        q = np.where(step > 0, np.clip(np.rint((x + off) / step), 0, 15), 0).astype(np.uint8)
    out = np.zeros((M, nb, BLOCK_BYTES), np.uint8)
    out[..., 0:2] = d16.view(np.uint8).reshape(M, nb, 2)
    out[..., 2:4] = dm16.view(np.uint8).reshape(M, nb, 2)
    out[..., 4:16] = pack_scales(qsc, qmn)
    qs = (q[..., :16] | (q[..., 16:] << 4)).reshape(M, nb, 128)
    out[..., 16:] = qs
    return out.tobytes()


def quantize_q8_0(w: np.ndarray) -> bytes:
    """Quantize f32 [M, K] (K % 32 == 0) row-major to Q8_0 bytes."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    M, K = w.shape
    assert K % Q8_ELEMS == 0
    x = w.reshape(M, K // Q8_ELEMS, Q8_ELEMS)
    d16 = (np.abs(x).max(-1) / 127.0).astype(np.float16)
    d = d16.astype(np.float32)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(d > 0, np.clip(np.rint(x / d), -127, 127), 0).astype(np.int8)
    out = np.zeros((M, K // Q8_ELEMS, Q8_BYTES), np.uint8)
    out[..., 0:2] = d16.view(np.uint8).reshape(M, K // Q8_ELEMS, 2)
    out[..., 2:] = q.view(np.uint8)
    return out.tobytes()


def dequantize_q8_0(raw, M: int, K: int) -> np.ndarray:
    """numpy dequant with quant.c:12-25's arithmetic (one exact f32 product)."""
    b = np.frombuffer(bytes(raw), np.uint8).reshape(M, K // Q8_ELEMS, Q8_BYTES)
    d = b[..., 0:2].copy().view(np.float16).astype(np.float32)
    q = b[..., 2:].copy().view(np.int8).astype(np.float32)
    return (d * q).reshape(M, K)


def dequantize_q4k(raw, M: int, K: int) -> np.ndarray:
    """Vectorised numpy dequant (same arithmetic as quant.c:168-202: one f32
    product, one f32 subtraction)."""
    b = np.frombuffer(bytes(raw), np.uint8).reshape(M, K // QK, BLOCK_BYTES)
    d = b[..., 0:2].copy().view(np.float16).astype(np.float32)
    dm = b[..., 2:4].copy().view(np.float16).astype(np.float32)
    s = b[..., 4:16].astype(np.uint16)
    sc = np.zeros(b.shape[:2] + (8,), np.float32)
    mn = np.zeros_like(sc)
    for j in range(8):
        if j < 4:
            sc[..., j] = s[..., j] & 63
            mn[..., j] = s[..., j + 4] & 63
        else:
            sc[..., j] = (s[..., j + 4] & 15) | ((s[..., j - 4] >> 6) << 4)
            mn[..., j] = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
    qs = b[..., 16:].reshape(M, K // QK, 8, 16)
    q = np.concatenate([qs & 15, qs >> 4], axis=-1).astype(np.float32)   # [M, nb, 8, 32]
    sd = (d * sc)[..., None].astype(np.float32)                         # d*sc in f32
    sm = (dm * mn)[..., None].astype(np.float32)
    return (sd * q - sm).astype(np.float32).reshape(M, K)


@dataclass
class LlamaShape:
    n_layers: int
    d_model: int
    n_heads: int
    n_kv_heads: int
    ffn: int
    vocab: int
    max_seq: int
    theta: float = 10000.0
    eps: float = 1e-5

    @property
    def head_dim(self):
        return self.d_model // self.n_heads

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim


LINEARS = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


def linear_shape(s: LlamaShape, name: str):
    D, H, kv = s.d_model, s.ffn, s.kv_dim
    return {"attn_q": (D, D), "attn_k": (kv, D), "attn_v": (kv, D),
            "attn_output": (D, D), "ffn_gate": (H, D), "ffn_up": (H, D),
            "ffn_down": (D, H)}[name]


def make_llama(shape: LlamaShape, seed: int, quant: str = "f32", output_quant: str | None = None,
               std: float = 0.02):
    """Return {name: (array_or_bytes, slate_dtype, (out, in) shape)} with
    weights ~ N(0, std) from ``numpy.random.default_rng(seed)`` and norms 1.0
    (as slate's fixtures do).  ``quant`` ("f32", "q4k" or "q8_0") applies to
    the seven block linears, ``output_quant`` (default: same) to the LM head."""
    rng = np.random.default_rng(seed)
    oq = quant if output_quant is None else output_quant

    def w(shp):
        return rng.normal(0.0, std, shp).astype(np.float32)

    def lin(shp, q):
        a = w(shp)
        if q == "q4k":
            return (np.frombuffer(quantize_q4k(a), np.uint8), SLATE_Q4_K, shp)
        if q == "q8_0":
            return (np.frombuffer(quantize_q8_0(a), np.uint8), SLATE_Q8_0, shp)
        return (a, SLATE_F32, shp)

    t = {}
    t["token_embd.weight"] = (w((shape.vocab, shape.d_model)), SLATE_F32, (shape.vocab, shape.d_model))
    t["output_norm.weight"] = (np.ones(shape.d_model, np.float32), SLATE_F32, (shape.d_model,))
    t["output.weight"] = lin((shape.vocab, shape.d_model), oq)
    for i in range(shape.n_layers):
        t[f"blk.{i}.attn_norm.weight"] = (np.ones(shape.d_model, np.float32), SLATE_F32, (shape.d_model,))
        t[f"blk.{i}.ffn_norm.weight"] = (np.ones(shape.d_model, np.float32), SLATE_F32, (shape.d_model,))
        for n in LINEARS:
            t[f"blk.{i}.{n}.weight"] = lin(linear_shape(shape, n), quant)
    return t


def write_llama_gguf(path, shape: LlamaShape, tensors: dict):
    g = GGUFWriter()
    g.add_str("general.architecture", "llama")
    g.add_u32("llama.block_count", shape.n_layers)
    g.add_u32("llama.embedding_length", shape.d_model)
    g.add_u32("llama.feed_forward_length", shape.ffn)
    g.add_u32("llama.attention.head_count", shape.n_heads)
    g.add_u32("llama.attention.head_count_kv", shape.n_kv_heads)
    g.add_u32("llama.context_length", shape.max_seq)
    g.add_u32("llama.vocab_size", shape.vocab)
    g.add_f32("llama.rope.freq_base", shape.theta)
    g.add_f32("llama.attention.layer_norm_rms_epsilon", shape.eps)
    for name, (arr, dt, shp) in tensors.items():
        g.add_tensor(name, shp, {SLATE_Q4_K: GGML_Q4_K, SLATE_Q8_0: GGML_Q8_0}.get(dt, GGML_F32), arr)
    g.write(path)


def engine_tensors(m, shape: LlamaShape, lazy: bool = False) -> dict:
    """The weights of a device engine (slate_amd.Llama) copied back to the
    host in make_llama's form {name: (array, slate dtype, (out, in) shape)},
    Q4_K and Q8_0 in slate's row layout, ready for write_llama_gguf or the
    oracle.  lazy=True: each array is a callable that copies the tensor when
    called (write_llama_gguf then holds one tensor at a time)."""
    t = {}

    def fetch(name, dt):
        raw, got = m.get_tensor(name)
        assert got == dt
        return raw.view(np.float32) if dt == SLATE_F32 else raw

    def get(name, key, shp):
        if lazy:
            dt = m.tensor_dtype(name)
            t[key] = ((lambda n=name, d=dt: fetch(n, d)), dt, shp)
            return
        raw, dt = m.get_tensor(name)
        t[key] = (raw.view(np.float32) if dt == SLATE_F32 else raw, dt, shp)

    D = shape.d_model
    get("token_embd", "token_embd.weight", (shape.vocab, D))
    get("output_norm", "output_norm.weight", (D,))
    get("output", "output.weight", (shape.vocab, D))
    for i in range(shape.n_layers):
        for n in ("attn_norm", "ffn_norm"):
            get(f"blk.{i}.{n}", f"blk.{i}.{n}.weight", (D,))
        for n in LINEARS:
            get(f"blk.{i}.{n}", f"blk.{i}.{n}.weight", linear_shape(shape, n))
    return t
