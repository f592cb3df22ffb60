#!/usr/bin/env python3
"""Benchmark: LLaMA-3-8B-shaped Q4_K decode under ragged continuous batching.

Workload (one MI355X): 32 layers, d_model 4096, 32 Q / 8 KV heads, head_dim
128, SwiGLU 14336, vocab 128256; every linear weight Q4_K drawn N(0, 0.02)
on the device from a fixed seed, embeddings f32, norms 1.  B = 16 sequences;
contexts prefilled to U[128, 2048] tokens (untimed); each sequence stops after
U[32, 256] generated tokens and its slot is taken by a new arrival whose
U[64, 512]-token prompt is prefilled inside the next ragged step (timed, mixed
prefill + decode).  A step = one pass of the engine over the packed batch;
each step produces one token per sequence.

Printed: one JSON line.  value = generated tokens / wall time over K timed
steps (weights and KV resident in HBM).  roofline = the dominant kernel class
of the decode steps by device time (decode-shaped Q4_K matmuls or decode
attention), from HIP events that the kernel dispatches record themselves, in
every 8th timed step: achieved = algorithmic bytes / device time; traffic =
HBM bytes per launch from the committed rocprofv3 PMC summary.  cpu_baseline =
slate's own C decode step (slate_llama_decode_step, single thread as wired)
on the same weights and KV state, for one step of all 16 sequences.
kernels.hbm_copy_GBs = a measured 1 GiB device copy (read + write bytes /
time) beside the nominal 8 TB/s.

--ops instead prints the op-level figures (one JSON object): the Q4_K and
Q8_0 matmuls through the C ABI (pre-tiled weights) at (M, K) in {(4096, 4096), (14336, 4096), (4096, 14336)}
and B in {1, 4, 16, 64}, rotating over enough weight copies (> 300 MB) that
the 256 MB Infinity Cache cannot hold them; and ragged GQA attention with
B = 64 sequences, 32 q / 8 kv heads, head_dim 128, lengths
clip(round(exp(N(ln 1024, 1))), 16, 16384).  Each figure is the device time
of a captured graph of many calls (no host launch gaps) divided by the calls.
--copy-calibration instead runs a plain device copy of known size (for
scaling the PMC byte counters).  --shape 70b runs the same workload with the
70B layer shapes (80 layers, d_model 8192, 64 Q / 8 KV heads, SwiGLU 28672;
no CPU baseline, no traffic figure: the PMC summary is of the 8B shape).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s at B=16 ragged, 8B-shape Q4_K; Q4_K matmul HBM GB/s"
HBM_PEAK_GBS = 8000.0
PROFILE_EVERY = 8


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Workload:
    """Continuous-batching driver over the engine's ragged step."""

    def __init__(self, m, shape, B, seed, max_tokens):
        self.m, self.shape, self.B = m, shape, B
        self.rng = np.random.default_rng(seed)
        self.max_tokens = max_tokens
        self.sess = [None] * B
        self.pending = [None] * B      # prompt still to prefill
        self.last = [0] * B            # last generated token
        self.gen = [0] * B
        self.stop = [0] * B
        self.arrivals = 0

    def new_prompt(self, lo, hi):
        n = int(self.rng.integers(lo, hi + 1))
        return self.rng.integers(0, self.shape.vocab, n).astype(np.int32)

    def start(self, i, prompt):
        if self.sess[i] is not None:
            self.sess[i].free()
        self.sess[i] = self.m.session()
        self.pending[i] = prompt
        self.gen[i] = 0
        self.stop[i] = int(self.rng.integers(32, 257))

    def prefill_all(self):
        """Untimed: initial contexts U[128, 2048], packed several per step."""
        for i in range(self.B):
            self.start(i, self.new_prompt(128, 2048))
        todo = list(range(self.B))
        while todo:
            group, T = [], 0
            for i in todo:
                if T + len(self.pending[i]) <= self.max_tokens:
                    group.append(i)
                    T += len(self.pending[i])
            todo = [i for i in todo if i not in group]
            rc, _, nxt = self.m.step([self.sess[i] for i in group], [len(self.pending[i]) for i in group],
                                     np.concatenate([self.pending[i] for i in group]), want_logits=False)
            assert rc == 0, f"prefill step rc={rc}"
            for i, t in zip(group, nxt):
                self.pending[i] = None
                self.last[i] = int(t)
                self.gen[i] = 1

    def step(self, want_logits=False):
        n_new, toks = [], []
        for i in range(self.B):
            if self.pending[i] is not None:
                n_new.append(len(self.pending[i]))
                toks.append(self.pending[i])
            else:
                n_new.append(1)
                toks.append(np.array([self.last[i]], np.int32))
        mixed = any(n > 1 for n in n_new)
        rc, lg, nxt = self.m.step(self.sess, n_new, np.concatenate(toks), want_logits=want_logits)
        assert rc == 0, f"step rc={rc}"
        for i in range(self.B):
            self.pending[i] = None
            self.last[i] = int(nxt[i])
            self.gen[i] += 1
            if self.gen[i] >= self.stop[i]:
                self.arrivals += 1
                self.start(i, self.new_prompt(64, 512))
        return mixed, lg


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--layers", type=int, default=None, help="layers (default: the shape's own)")
    ap.add_argument("--shape", choices=("8b", "70b"), default="8b",
                    help="model shape: 8b (the headline line) or 70b (same workload, 70B layer shapes)")
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU reference baseline")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a 1 GiB device-to-device copy 5 times and exit")
    ap.add_argument("--ops", action="store_true", help="op-level Q4_K / Q8_0 matmul and ragged attention figures")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        n = 1 << 28                                  # 2^28 f32 = 1 GiB each way
        a = torch.ones(n, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": 4 * n, "copy_bytes_written": 4 * n, "launches": 5}))
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU; sequence-level data parallelism over "
                                   "several GPUs is designed but not executed", "n_gpus": args.gpus}))
        return 2
    if args.ops:
        print(json.dumps(run_ops(args.seed)), flush=True)
        return 0
    try:   # torch (for the copy-bandwidth figure) must initialise HIP before the library does
        import torch  # noqa: F401
    except ImportError:
        pass

    import slate_amd
    from slate_amd.synth import LlamaShape
    big = args.shape == "70b"
    if args.layers is None:
        args.layers = 80 if big else 32
    if big:
        shape = LlamaShape(n_layers=args.layers, d_model=8192, n_heads=64, n_kv_heads=8, ffn=28672,
                           vocab=128256, max_seq=2304)
        args.no_cpu = True    # the reference's C decode step needs ~13 s per token per core at this shape
    else:
        shape = LlamaShape(n_layers=args.layers, d_model=4096, n_heads=32, n_kv_heads=8, ffn=14336,
                           vocab=128256, max_seq=2304)
    max_tokens = 4096
    t0 = time.perf_counter()
    m = slate_amd.Llama.synthetic(shape, seed=args.seed, quant=18, max_slots=args.batch + 1,
                                  max_tokens=max_tokens)
    log(f"synthetic {args.shape.upper()}-shape Q4_K model on device in {time.perf_counter() - t0:.1f} s")
    wl = Workload(m, shape, args.batch, args.seed + 1, max_tokens)
    t0 = time.perf_counter()
    wl.prefill_all()
    ctx0 = [s.position for s in wl.sess]
    log(f"prefilled {sum(ctx0)} context tokens in {time.perf_counter() - t0:.1f} s")
    for _ in range(args.warmup):
        wl.step()
    lib = slate_amd.load_library()
    m.profile(True)
    m.profile(False)
    lib.slate_hip_sync()
    arrivals0 = wl.arrivals
    mixed_steps = 0
    step_s, step_mixed, step_prof = [], [], []
    t0 = time.perf_counter()
    for i in range(args.steps):
        # one step in PROFILE_EVERY is launched kernel by kernel with
        # dispatch-recorded events (the roofline); the others replay graphs
        prof = i % PROFILE_EVERY == 0
        if prof:
            m.profile(True, reset=False)
        ts = time.perf_counter()
        mixed = wl.step()[0]
        step_s.append(time.perf_counter() - ts)
        if prof:
            m.profile(False)
        step_mixed.append(mixed)
        step_prof.append(prof)
        mixed_steps += mixed
    lib.slate_hip_sync()
    dt = time.perf_counter() - t0
    raw = m.profile_read()
    tokens = args.batch * args.steps
    value = tokens / dt
    dec_s = [t for t, mx, p in zip(step_s, step_mixed, step_prof) if not mx and not p]
    mix_s = [t for t, mx in zip(step_s, step_mixed) if mx]
    log(f"{args.steps} steps in {dt:.3f} s, {mixed_steps} with arrivals ({wl.arrivals - arrivals0} arrivals); "
        f"decode-only step median {1e3 * np.median(dec_s) if dec_s else 0:.2f} ms, "
        f"mixed steps {[round(1e3 * t, 1) for t in mix_s]} ms")
    for k, (ms, by, n) in raw.items():
        log(f"  {k:13s} {ms:9.2f} ms  {n:6d} launches  {by / max(ms, 1e-9) / 1e6:8.1f} GB/s")
    # roofline: the dominant kernel class of the decode steps by device time
    # (decode-shaped Q4_K matmuls vs decode attention)
    dom = max(("q4k_mm", "attention"), key=lambda k: raw[k][0])
    ms, by, n = raw[dom]
    achieved = by / (ms * 1e-3) / 1e9
    kname = "q4k_dec_kernel" if dom == "q4k_mm" else "attn_dec_kernel+attn_merge_kernel"
    roofline = {"bound": "hbm", "kernel": kname,
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": None if big else measured_traffic(kname),   # the PMC summary is of the 8B shape
                "launches": n, "avg_launch_us": round(ms * 1e3 / max(n, 1), 2),
                "algorithmic_bytes_per_launch": round(by / max(n, 1))}
    other = "attention" if dom == "q4k_mm" else "q4k_mm"
    oms, oby, on = raw[other]
    step_ms, _, step_n = raw["step"]
    pf_ms, pf_by, pf_n = raw["q4k_mm_pf"]
    result = {
        "metric": METRIC.replace("8B-shape", "70B-shape") if big else METRIC, "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3 / args.steps, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": ("LLaMA-70B-shaped" if big else "LLaMA-3-8B-shaped") +
                               f" Q4_K decode, ragged continuous batching B={args.batch} "
                               "(contexts U[128,2048], stop U[32,256], arrivals with U[64,512]-token prompts)",
                   "layers": args.layers, "d_model": shape.d_model,
                   "heads": f"{shape.n_heads}q/{shape.n_kv_heads}kv", "ffn": shape.ffn, "vocab": shape.vocab,
                   "weights": "q4_k", "kv_cache": "f16" if lib.slate_hip_llama_kv_f16(m.h) == 1 else "f32",
                   "batch": args.batch,
                   "mixed_prefill_steps": mixed_steps, "arrivals": wl.arrivals - arrivals0,
                   "mean_context_start": round(float(np.mean(ctx0)), 1)},
        "roofline": roofline,
        "kernels": {"other_decode_class": other, f"{other}_GBs": round(oby / max(oms, 1e-9) / 1e6, 1),
                    f"{other}_ms": round(oms, 2),
                    "decode_step_device_ms": round(step_ms / max(step_n, 1), 3),
                    "decode_step_median_ms": round(1e3 * float(np.median(dec_s)), 3) if dec_s else None,
                    "mixed_step_ms": [round(1e3 * t, 1) for t in mix_s],
                    "prefill_q4k_ms": round(pf_ms, 2), "prefill_q4k_launches": pf_n},
    }
    try:
        result["kernels"]["hbm_copy_GBs"] = round(copy_bandwidth(), 1)
    except Exception as e:  # reported beside the nominal peak, never required
        result["kernels"]["hbm_copy_GBs"] = None
        log(f"copy bandwidth not measured: {e}")
    if not args.no_cpu:
        try:
            result["cpu_baseline"] = cpu_baseline_and_parity(m, shape, wl)
        except Exception as e:  # the baseline is reported, never required
            result["cpu_baseline"] = {"error": str(e)}
    print(json.dumps(result), flush=True)
    return 0


def copy_bandwidth(reps=10):
    """Device copy of 1 GiB (read + written bytes / device time), GB/s."""
    import torch
    n = 1 << 28
    a = torch.ones(n, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        b.copy_(a)
    e1.record()
    e1.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del a, b
    return 2 * 4 * n / (ms * 1e-3) / 1e9


def graph_time_us(fn, calls, stream, result):
    """Device microseconds per call of fn (which enqueues on the backend
    stream), from a graph of `calls` captured calls replayed three times, and
    whether every replay left `result` (the output tensor, the same for every
    call) equal to the eager call's."""
    import torch
    fn(0)                                        # eager; grows scratch outside the capture
    torch.cuda.synchronize()
    ref = result.clone()
    same = True
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(calls):
            fn(i)
    best = None
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record()
            g.replay()
            e1.record()
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / calls
        best = us if best is None else min(best, us)
        same = same and bool(torch.equal(result, ref))
        result.zero_()
        torch.cuda.synchronize()
    del g
    return best, same


def run_ops(seed):
    """C2 (Q4_K and Q8_0 matmuls at the 8B linear shapes) and C3 (ragged
    attention) op figures."""
    import torch
    import slate_amd
    lib = slate_amd.load_library()
    slate_amd.Backend()
    stream = torch.cuda.ExternalStream(lib.slate_hip_stream())
    out = {"metric": "op-level device time per call", "hbm_peak_GBs": HBM_PEAK_GBS,
           "mfma_f16_peak_TFLOPs": 2500.0, "hbm_copy_GBs": round(copy_bandwidth(), 1), "q4k": [], "q8_0": [],
           "attention": None}
    gen = torch.Generator(device="cuda").manual_seed(seed)
    # (block elements, block bytes, high byte of each f16 scale, tiler, tiled matmul)
    formats = {"q4k": (256, 144, (1, 3), lib.slate_hip_q4k_tiled_bytes, lib.slate_hip_q4k_tile,
                       lib.slate_hip_matmul_q4k_tiled),
               "q8_0": (32, 34, (1,), lib.slate_hip_q8_0_tiled_bytes, lib.slate_hip_q8_0_tile,
                        lib.slate_hip_matmul_q8_0_tiled)}
    for fmt, (qk, qb, hi, tiled_bytes, tile, matmul) in formats.items():
        for M, K in ((4096, 4096), (14336, 4096), (4096, 14336)):
            nblk = M * K // qk
            raw = torch.randint(0, 256, (nblk, qb), dtype=torch.uint8, device="cuda", generator=gen)
            for b in hi:                                 # finite, moderate scales
                raw[:, b] = (raw[:, b] & 0x1F) | 0x10
            tb = tiled_bytes(M, K)
            # rotate over > 300 MB of copies so every call streams from HBM
            ncopy = max(32, -(-300_000_000 // tb) + 1)
            copies = torch.empty((ncopy, tb), dtype=torch.uint8, device="cuda")
            torch.cuda.synchronize()
            for c in range(ncopy):
                slate_amd.check(tile(copies[c].data_ptr(), raw.data_ptr(), M, K), fmt + " tile")
            lib.slate_hip_sync()
            del raw
            for B in (1, 4, 16, 64):
                X = torch.randn(B, K, device="cuda", generator=gen)
                Y = torch.empty(B, M, device="cuda")
                torch.cuda.synchronize()

                def call(i, X=X, Y=Y, B=B):
                    slate_amd.check(matmul(Y.data_ptr(), copies[i % ncopy].data_ptr(), X.data_ptr(), B, M, K),
                                    fmt + " matmul")
                us, same = graph_time_us(call, 2 * ncopy, stream, Y)
                alg = nblk * qb + 4 * B * K + 4 * B * M
                flops = 2.0 * B * M * K
                out[fmt].append({"M": M, "K": K, "B": B, "us": round(us, 2),
                                 "GBs": round(alg / us / 1e3, 1), "frac_hbm": round(alg / us / 1e3 / HBM_PEAK_GBS, 3),
                                 "TFLOPs": round(flops / us / 1e6, 1),
                                 "frac_mfma": round(flops / us / 1e6 / 2500.0, 4), "replays_match_eager": same})
                log(fmt, out[fmt][-1])
            del copies
            torch.cuda.empty_cache()
    # C3: ragged attention
    rng = np.random.default_rng(seed)
    Bq, Hq, Hkv, hd = 64, 32, 8, 128
    L = np.clip(np.round(np.exp(rng.normal(np.log(1024.0), 1.0, Bq))), 16, 16384).astype(np.int64)
    max_seq = int(L.max())
    head_stride = max_seq * hd
    slot = Hkv * head_stride
    Kp = torch.randn(Bq * slot, device="cuda", generator=gen)
    Vp = torch.randn(Bq * slot, device="cuda", generator=gen)
    q = torch.randn(Bq, Hq * hd, device="cuda", generator=gen)
    o = torch.empty_like(q)
    t2s = torch.arange(Bq, dtype=torch.int32, device="cuda")
    pos = torch.tensor(L - 1, dtype=torch.int32, device="cuda")
    kvb = torch.arange(Bq, dtype=torch.int64, device="cuda") * slot
    torch.cuda.synchronize()

    def att(i):
        slate_amd.check(lib.slate_hip_attention_ragged(o.data_ptr(), q.data_ptr(), Kp.data_ptr(), Vp.data_ptr(),
                                                       t2s.data_ptr(), pos.data_ptr(), kvb.data_ptr(), Bq, Hq,
                                                       Hkv, hd, head_stride, max_seq), "attention_ragged")
    us, same = graph_time_us(att, 20, stream, o)
    alg = int(L.sum()) * 2 * Hkv * hd * 4 + 2 * Bq * Hq * hd * 4
    out["attention"] = {"B": Bq, "Hq": Hq, "Hkv": Hkv, "head_dim": hd, "sum_L": int(L.sum()),
                        "max_L": max_seq, "us": round(us, 2), "GBs": round(alg / us / 1e3, 1),
                        "frac_hbm": round(alg / us / 1e3 / HBM_PEAK_GBS, 3), "replays_match_eager": same}
    log(out["attention"])
    return out


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed PMC summary
    (profiles/q4k_dec_traffic.txt: FETCH_SIZE + WRITE_SIZE per dispatch,
    scaled by a copy kernel of known size), or None when there is none."""
    path = os.path.join(ROOT, "profiles", "q4k_dec_traffic.txt")
    if kernel != "q4k_dec_kernel" or not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return round(float(line.split(":", 1)[1]))
    return None


def cpu_baseline_and_parity(m, shape, wl):
    """Snapshot KV of every decoding sequence, run the CPU reference step from
    that state, then the GPU step; compare the two sets of logits."""
    snap = [(i, wl.sess[i].kv(), wl.sess[i].position, wl.last[i]) for i in range(wl.B)
            if wl.pending[i] is None]
    _, lg, _ = wl.m.step([wl.sess[i] for i, *_ in snap], [1] * len(snap),
                         [t for *_, t in snap], want_logits=True)
    gpu = {i: lg[k] for k, (i, *_) in enumerate(snap)}
    return cpu_baseline_from(m, shape, snap, gpu)


def cpu_baseline_from(m, shape, snap, gpu, budget_s=40.0):
    from oracle.pyoracle import Ref, RefLlama, ref_available
    from slate_amd.gguf import GGML_F32, GGML_Q4_K, GGUFWriter
    if not ref_available():
        return {"error": "oracle/_ref not built"}
    ref = Ref()
    path = "/dev/shm/slate_amd_bench_8b.gguf"
    g = GGUFWriter()
    g.add_str("general.architecture", "llama")
    for k, v in (("block_count", shape.n_layers), ("embedding_length", shape.d_model),
                 ("feed_forward_length", shape.ffn), ("attention.head_count", shape.n_heads),
                 ("attention.head_count_kv", shape.n_kv_heads), ("context_length", shape.max_seq),
                 ("vocab_size", shape.vocab)):
        g.add_u32("llama." + k, v)
    g.add_f32("llama.rope.freq_base", shape.theta)
    g.add_f32("llama.attention.layer_norm_rms_epsilon", shape.eps)
    D, H, kv = shape.d_model, shape.ffn, shape.kv_dim
    dims = {"attn_q": (D, D), "attn_k": (kv, D), "attn_v": (kv, D), "attn_output": (D, D),
            "ffn_gate": (H, D), "ffn_up": (H, D), "ffn_down": (D, H)}

    def add(name, gname, shp):
        raw, dt = m.get_tensor(name)
        g.add_tensor(gname, shp, GGML_Q4_K if dt == 18 else GGML_F32, raw)

    add("token_embd", "token_embd.weight", (shape.vocab, D))
    add("output_norm", "output_norm.weight", (D,))
    add("output", "output.weight", (shape.vocab, D))
    for i in range(shape.n_layers):
        add(f"blk.{i}.attn_norm", f"blk.{i}.attn_norm.weight", (D,))
        add(f"blk.{i}.ffn_norm", f"blk.{i}.ffn_norm.weight", (D,))
        for n, shp in dims.items():
            add(f"blk.{i}.{n}", f"blk.{i}.{n}.weight", shp)
    g.write(path)
    del g
    rm = RefLlama(ref, path)
    t_cpu, n_tok, worst = 0.0, 0, 0.0
    try:
        for i, (K, V), pos, tok in snap:
            rs = rm.session()
            assert rs.set_state(K, V, pos) == 0
            t0 = time.perf_counter()
            rc, lg = rs.decode(tok)
            t_cpu += time.perf_counter() - t0
            rs.free()
            assert rc == 0
            n_tok += 1
            worst = max(worst, float(np.abs(lg - gpu[i]).max() / max(np.abs(lg).max(), 1e-30)))
            if t_cpu > budget_s:
                break
    finally:
        rm.close()
        os.unlink(path)
    return dict(value=round(n_tok / t_cpu, 4), unit="tok/s", cores=1, kind="reference",
                sample=f"slate_llama_decode_step (slate's C, built from its sources, single thread as wired) "
                       f"on the benchmark's weights and KV state: one decode step of {n_tok} sequences, "
                       f"{t_cpu:.1f} s",
                host_cores_available=os.cpu_count(), host_cpu=cpu_model(), logits_max_rel_vs_gpu=worst)


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


if __name__ == "__main__":
    sys.exit(main())
