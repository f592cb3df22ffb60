"""Shared test constants and helpers (test infrastructure)."""
import hashlib

import numpy as np

from slate_amd.synth import LlamaShape

# The tiny f32 LLaMA and its continuous-batching workload: 2 layers, d_model 64,
# 4 Q / 2 KV heads (head_dim 16), SwiGLU 172, vocab 256, RMSNorm eps 1e-5,
# RoPE theta 10000; 4 sequences with prompts of 8..32 uniform ids, 32 greedy
# tokens each.
TINY = LlamaShape(n_layers=2, d_model=64, n_heads=4, n_kv_heads=2, ffn=172, vocab=256, max_seq=128)
TINY_SEED = 0xCAFE
WORK_SEED = 0x51A7E
N_SEQ, N_GEN = 4, 32
# A small Q4_K model (every linear K is a multiple of 256), GQA 4/2.
Q4 = LlamaShape(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, ffn=512, vocab=64, max_seq=128)
Q4_SEED = 0xBEEF
Q4_PROMPT = np.array([1, 7, 13, 25, 3], np.int32)     # the prompt of slate's Q4_K fixture


def tensors_digest(t):
    h = hashlib.sha256()
    for name in sorted(t):
        h.update(name.encode())
        h.update(np.ascontiguousarray(t[name][0]).tobytes())
    return h.hexdigest()


def relerr(a, b):
    """Normwise relative error max|a-b| / max|b|."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def tiny_prompts():
    wr = np.random.default_rng(WORK_SEED)
    lens = wr.integers(8, 33, N_SEQ)
    return [wr.integers(0, TINY.vocab, n).astype(np.int32) for n in lens]


def same_floats(a, b):
    """Bitwise equal, except that any NaN matches any NaN (NaN payloads of
    inf*0 and the like differ between x86 and the GPU)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all((a.view(np.uint32) == b.view(np.uint32)) | nan))
