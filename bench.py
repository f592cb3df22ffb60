#!/usr/bin/env python3
"""Benchmark: LLaMA-3-8B-shaped Q4_K decode under ragged continuous batching.

Workload (one MI355X): 32 layers, d_model 4096, 32 Q / 8 KV heads, head_dim
128, SwiGLU 14336, vocab 128256; every linear weight Q4_K drawn N(0, 0.02)
on the device from a fixed seed, embeddings f32, norms 1.  B = 16 sequences;
contexts prefilled to U[128, 2048] tokens (untimed); each sequence stops
after U[32, 256] generated tokens and its slot is taken by a new arrival
whose U[64, 512]-token prompt is prefilled inside the next ragged step
(mixed prefill + decode).  The workload starts in steady state: after the
context prefill each sequence is placed at a point of its generation drawn
from the stop-and-replace process's equilibrium law, stratified over the
sequences, so every window of n steps holds about n * B / E[stop] arrivals
(prompts prefilled in mixed steps) from the first timed step on.  A step =
one pass of the engine over the packed batch; each step produces one token
per sequence.

Printed: one JSON line.  value = generated tokens / wall time over the K
timed steps (weights and KV resident in HBM; each step's descriptor upload
and next-token download are inside).  decode_only_tok_s is the same over
the steps without prompt chunks.  roofline.step_frac = the timed steps'
algorithmic bytes (every weight byte once per step, K/V rows read once per
sequence per step and the new rows written, embedding rows in, logits out)
/ wall time / 8 TB/s; decode_step_frac the same over decode-only steps.
roofline.achieved / frac: the dominant kernel class of the decode steps by
device time (decode-shaped Q4_K matmuls or decode attention), from HIP
events that the kernel dispatches record themselves, measured in a separate
window of steps after the timed one (so event recording never slows the
headline); traffic = HBM bytes per launch from the committed rocprofv3 PMC
summary.  cpu_baseline = slate's own C decode step (slate_llama_decode_step)
on the same weights and KV state, one step of the sequences, single thread
as wired, plus a harness-level variant over slate's threadpool.
kernels.hbm_copy_GBs = a measured 1 GiB device copy (read + write bytes /
time) beside the nominal 8 TB/s.

--shape 70b runs the 70B configuration's own workload instead: LLaMA-3-70B
shapes (80 layers, d_model 8192, 64 Q / 8 KV heads, SwiGLU 28672, vocab
128256, Q4_K), requests arriving as a Poisson process at 4 per second of
wall time, prompts U[256, 4096], outputs U[64, 512], greedy, at most 32 in
flight; prompts are prefilled in chunks of at most --prefill-chunk tokens
per step inside the ragged steps next to the decode rows (so the decode rows
keep stepping while prompts stream in).  value = generated tokens / wall
time over --duration seconds after --warmup-s seconds.

--ops instead prints the op-level figures (one JSON object): the Q4_K and
Q8_0 matmuls through the C ABI (pre-tiled weights) at (M, K) in {(4096, 4096), (14336, 4096), (4096, 14336)}
and B in {1, 4, 16, 32, 64}, rotating over enough weight copies (> 300 MB)
that the 256 MB Infinity Cache cannot hold them; and ragged GQA attention
with B = 64 sequences, 32 q / 8 kv heads, head_dim 128, lengths
clip(round(exp(N(ln 1024, 1))), 16, 16384).  Each figure is the device time
of a captured graph of many calls (no host launch gaps) divided by the calls.
--copy-calibration instead runs a plain device copy of known size (for
scaling the PMC byte counters).
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
HOST_THREADS = 16            # the host cores one GPU's share of the box offers


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def weight_bytes(shape):
    """Algorithmic weight bytes per step: every Q4_K linear and the Q4_K LM
    head once (slate's 144-byte blocks), the f32 norm vectors once."""
    D, H, kv = shape.d_model, shape.ffn, shape.kv_dim
    q4 = lambda M, K: M * (K // 256) * 144
    per_layer = q4(D, D) * 2 + q4(kv, D) * 2 + q4(H, D) * 2 + q4(D, H) + 2 * D * 4
    return shape.n_layers * per_layer + q4(shape.vocab, D) + D * 4


def step_bytes(shape, pos0, n_new):
    """Algorithmic HBM bytes of one ragged step: weights once, each sequence's
    K/V rows 0 .. pos0+n_new-1 read once and its n_new new rows written
    (2 * layers * kv_dim f32 per row), embedding rows in, logits out."""
    row = 2 * shape.n_layers * shape.kv_dim * 4
    T = int(sum(n_new))
    kv = sum((p + n) * row + n * row for p, n in zip(pos0, n_new))
    return weight_bytes(shape) + kv + T * shape.d_model * 4 + len(n_new) * shape.vocab * 4


class Workload:
    """Continuous-batching driver over the engine's ragged step (B fixed)."""

    def __init__(self, m, shape, B, seed, max_tokens):
        self.m, self.shape, self.B = m, shape, B
        self.rng = np.random.default_rng(seed)
        self.max_tokens = max_tokens
        self.sess = [None] * B
        self.pending = [None] * B      # prompt still to prefill
        self.last = [0] * B            # last generated token
        self.gen = [0] * B
        self.stop = [0] * B
        self.arrivals = 0              # sequences replaced (their prompt goes into the next step)
        self.prompts = 0               # prompts prefilled inside steps
        self.prompt_tokens = 0

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

    def steady_state_positions(self):
        """(stop, generated) per slot at the steady state of the
        stop-and-replace process, stratified over the slots.  A slot's
        remaining tokens R = stop - generated follow the equilibrium
        residual-life law of stop ~ U[32, 256] with generated >= 1:
        P(R = r) proportional to P(stop > r), r = 1 .. 255.  The B slots
        take the R quantiles (k + u0) / B, k = 0 .. B-1, for one uniform u0,
        in random order (systematic sampling: every window of n steps holds
        about n * B / E[stop] finishing sequences, as a long-running server
        sees, instead of whatever one seed gives); then stop ~ U[max(32,
        R + 1), 256] (the law of stop given R) and generated = stop - R."""
        lo, hi = 32, 256
        r = np.arange(1, hi)
        w = np.where(r < lo, 1.0, (hi - r) / (hi - lo + 1.0))   # P(stop > r)
        cdf = np.cumsum(w) / w.sum()
        u = (np.arange(self.B) + self.rng.random()) / self.B
        R = r[np.minimum(np.searchsorted(cdf, u, side="right"), len(r) - 1)]
        R = R[self.rng.permutation(self.B)]
        stop = np.array([int(self.rng.integers(max(lo, x + 1), hi + 1)) for x in R])
        return stop, stop - R

    def prefill_all(self):
        """Untimed: initial contexts U[128, 2048], packed several per step;
        then each sequence is placed where the steady state of the
        stop-and-replace process puts it (steady_state_positions)."""
        stop, gen = self.steady_state_positions()
        for i in range(self.B):
            self.start(i, self.new_prompt(128, 2048))
            self.stop[i] = int(stop[i])
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
                self.gen[i] = int(gen[i])

    def step(self, want_logits=False):
        """One ragged step; returns (mixed, logits, pos0, n_new)."""
        n_new, toks, pos0 = [], [], []
        for i in range(self.B):
            pos0.append(self.sess[i].position)
            if self.pending[i] is not None:
                n_new.append(len(self.pending[i]))
                toks.append(self.pending[i])
            else:
                n_new.append(1)
                toks.append(np.array([self.last[i]], np.int32))
        mixed = any(n > 1 for n in n_new)
        self.prompts += sum(1 for n in n_new if n > 1)
        self.prompt_tokens += sum(n for n in n_new if n > 1)
        rc, lg, nxt = self.m.step(self.sess, n_new, np.concatenate(toks), want_logits=want_logits)
        assert rc == 0, f"step rc={rc}"
        for i in range(self.B):
            self.pending[i] = None
            self.last[i] = int(nxt[i])
            self.gen[i] += 1
            if self.gen[i] >= self.stop[i]:
                self.arrivals += 1
                self.start(i, self.new_prompt(64, 512))
        return mixed, lg, pos0, n_new


def run_c4(args, shape):
    import slate_amd
    max_tokens = 4096
    t0 = time.perf_counter()
    m = slate_amd.Llama.synthetic(shape, seed=args.seed, quant=18, max_slots=args.batch + 1,
                                  max_tokens=max_tokens)
    log(f"synthetic 8B-shape Q4_K model on device in {time.perf_counter() - t0:.1f} s")
    wl = Workload(m, shape, args.batch, args.seed + 1, max_tokens)
    t0 = time.perf_counter()
    wl.prefill_all()
    ctx0 = [s.position for s in wl.sess]
    log(f"prefilled {sum(ctx0)} context tokens in {time.perf_counter() - t0:.1f} s")
    for _ in range(args.warmup):
        wl.step()
    lib = slate_amd.load_library()
    lib.slate_hip_sync()
    prompts0, ptok0 = wl.prompts, wl.prompt_tokens
    step_s, step_mixed, step_by, step_tok = [], [], [], []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ts = time.perf_counter()
        mixed, _, pos0, n_new = wl.step()
        step_s.append(time.perf_counter() - ts)
        step_mixed.append(mixed)
        step_by.append(step_bytes(shape, pos0, n_new))
        step_tok.append(args.batch)
    lib.slate_hip_sync()
    dt = time.perf_counter() - t0
    arrivals = wl.prompts - prompts0          # prompts prefilled inside the timed steps
    prompt_tokens = wl.prompt_tokens - ptok0
    tokens = int(sum(step_tok))
    value = tokens / dt
    dec = [i for i, mx in enumerate(step_mixed) if not mx]
    dec_s = sum(step_s[i] for i in dec)
    dec_tok_s = sum(step_tok[i] for i in dec) / dec_s if dec else None
    step_frac = sum(step_by) / dt / (HBM_PEAK_GBS * 1e9)
    dec_frac = sum(step_by[i] for i in dec) / dec_s / (HBM_PEAK_GBS * 1e9) if dec else None
    mix_ms = [round(1e3 * t, 1) for t, mx in zip(step_s, step_mixed) if mx]
    log(f"{args.steps} steps in {dt:.3f} s, {sum(step_mixed)} mixed ({arrivals} prompts, {prompt_tokens} prompt "
        f"tokens); decode-only steps "
        f"{1e3 * np.median([step_s[i] for i in dec]) if dec else 0:.2f} ms median; mixed steps {mix_ms} ms; "
        f"step_frac {step_frac:.3f}, decode_step_frac {dec_frac if dec_frac is None else round(dec_frac, 3)}")
    # kernel-class timing in its own window (events recorded by every dispatch)
    m.profile(True)
    for _ in range(args.profile_steps):
        wl.step()
    m.profile(False)
    lib.slate_hip_sync()
    raw = m.profile_read()
    for k, (ms, by, n) in raw.items():
        log(f"  {k:13s} {ms:9.2f} ms  {n:6d} launches  {by / max(ms, 1e-9) / 1e6:8.1f} GB/s")
    dom = max(("q4k_mm", "attention"), key=lambda k: raw[k][0])
    ms, by, n = raw[dom]
    achieved = by / (ms * 1e-3) / 1e9
    kname = "q4k_dec_kernel" if dom == "q4k_mm" else "attn_dec_kernel+attn_merge_kernel"
    roofline = {"bound": "hbm", "kernel": kname,
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(kname),
                "launches": n, "avg_launch_us": round(ms * 1e3 / max(n, 1), 2),
                "algorithmic_bytes_per_launch": round(by / max(n, 1)),
                "step_frac": round(step_frac, 4),
                "decode_step_frac": None if dec_frac is None else round(dec_frac, 4),
                "step_bytes_mean": round(float(np.mean(step_by)))}
    other = "attention" if dom == "q4k_mm" else "q4k_mm"
    oms, oby, on = raw[other]
    step_ms, _, step_n = raw["step"]
    pf_ms, _, pf_n = raw["q4k_mm_pf"]
    result = {
        "metric": METRIC, "value": round(value, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3 / args.steps, 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "LLaMA-3-8B-shaped Q4_K decode, ragged continuous batching "
                               f"B={args.batch} (contexts U[128,2048], stop U[32,256], steady-state "
                               "arrivals with U[64,512]-token prompts)",
                   "layers": shape.n_layers, "d_model": shape.d_model,
                   "heads": f"{shape.n_heads}q/{shape.n_kv_heads}kv", "ffn": shape.ffn, "vocab": shape.vocab,
                   "weights": "q4_k", "kv_cache": "f16" if lib.slate_hip_llama_kv_f16(m.h) == 1 else "f32",
                   "batch": args.batch, "mixed_prefill_steps": int(sum(step_mixed)), "arrivals": arrivals,
                   "prompt_tokens": prompt_tokens,
                   "mean_context_start": round(float(np.mean(ctx0)), 1)},
        "decode_only_tok_s": None if dec_tok_s is None else round(dec_tok_s, 1),
        "roofline": roofline,
        "kernels": {"profiled_steps": args.profile_steps, "other_decode_class": other,
                    f"{other}_GBs": round(oby / max(oms, 1e-9) / 1e6, 1), f"{other}_ms": round(oms, 2),
                    "decode_step_device_ms": round(step_ms / max(step_n, 1), 3),
                    "decode_step_median_ms": round(1e3 * float(np.median([step_s[i] for i in dec])), 3)
                    if dec else None,
                    "mixed_step_ms": mix_ms, "prefill_q4k_ms": round(pf_ms, 2), "prefill_q4k_launches": pf_n},
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
    return result


class PoissonWorkload:
    """Open-loop serving: requests arrive as a Poisson process in wall time,
    wait for one of max_batch slots, prefill their prompt in chunks inside
    the ragged steps (the step's token budget minus its decode rows) and
    then decode until their output length."""

    def __init__(self, m, shape, max_batch, rate, seed, max_tokens, prefill_chunk, prompt=(256, 4096), out=(64, 512)):
        self.m, self.shape, self.max_batch, self.rate = m, shape, max_batch, rate
        self.rng = np.random.default_rng(seed)
        self.max_tokens, self.prompt_rng, self.out_rng = max_tokens, prompt, out
        self.prefill_chunk = prefill_chunk
        self.queue, self.active = [], []
        self.next_arrival = float(self.rng.exponential(1.0 / rate))
        self.arrived = self.completed = self.generated = 0

    def admit(self, now):
        while self.next_arrival <= now:
            n = int(self.rng.integers(self.prompt_rng[0], self.prompt_rng[1] + 1))
            self.queue.append({"prompt": self.rng.integers(0, self.shape.vocab, n).astype(np.int32),
                               "out": int(self.rng.integers(self.out_rng[0], self.out_rng[1] + 1)),
                               "t": self.next_arrival})
            self.arrived += 1
            self.next_arrival += float(self.rng.exponential(1.0 / self.rate))
        while self.queue and len(self.active) < self.max_batch:
            r = self.queue.pop(0)
            r.update(sess=self.m.session(), done=0, gen=0, last=0)
            self.active.append(r)

    def step(self, now):
        """One ragged step at wall time `now`; returns (tokens generated, step ran)."""
        self.admit(now)
        if not self.active:
            return 0, False
        n_dec = sum(1 for r in self.active if r["done"] == len(r["prompt"]))
        budget = min(self.prefill_chunk, self.max_tokens - n_dec)
        rows, n_new, toks = [], [], []
        for r in self.active:
            left = len(r["prompt"]) - r["done"]
            if left == 0:
                rows.append(r)
                n_new.append(1)
                toks.append(np.array([r["last"]], np.int32))
            elif budget > 0:
                c = min(left, budget)
                budget -= c
                rows.append(r)
                n_new.append(c)
                toks.append(r["prompt"][r["done"]:r["done"] + c])
        rc, _, nxt = self.m.step([r["sess"] for r in rows], n_new, np.concatenate(toks), want_logits=False)
        assert rc == 0, f"step rc={rc}"
        gen = 0
        for r, n, t in zip(rows, n_new, nxt):
            if r["done"] < len(r["prompt"]):
                r["done"] += n
                if r["done"] < len(r["prompt"]):
                    continue                       # prompt not finished: no token yet
            r["last"] = int(t)
            r["gen"] += 1
            gen += 1
        done = [r for r in self.active if r["gen"] >= r["out"]]
        for r in done:
            r["sess"].free()
        self.active = [r for r in self.active if r["gen"] < r["out"]]
        self.completed += len(done)
        self.generated += gen
        return gen, True


def run_c5(args, shape):
    import slate_amd
    max_tokens, max_batch, rate = 4096, 32, 4.0
    t0 = time.perf_counter()
    m = slate_amd.Llama.synthetic(shape, seed=args.seed, quant=18, max_slots=max_batch, max_tokens=max_tokens)
    log(f"synthetic 70B-shape Q4_K model on device in {time.perf_counter() - t0:.1f} s")
    wl = PoissonWorkload(m, shape, max_batch, rate, args.seed + 1, max_tokens, args.prefill_chunk)
    lib = slate_amd.load_library()
    start = time.perf_counter()
    now = 0.0
    while now < args.warmup_s:                     # fill the system from empty
        wl.step(now)
        now = time.perf_counter() - start
    lib.slate_hip_sync()
    g0, a0, c0 = wl.generated, wl.arrived, wl.completed
    steps, batch_sum, t_begin = 0, 0, time.perf_counter()
    while time.perf_counter() - t_begin < args.duration:
        now = time.perf_counter() - start
        ran = wl.step(now)[1]
        steps += ran
        batch_sum += len(wl.active)
        if not ran:
            time.sleep(0.001)
    lib.slate_hip_sync()
    dt = time.perf_counter() - t_begin
    tokens = wl.generated - g0
    log(f"{steps} steps in {dt:.1f} s: {tokens} tokens, {wl.arrived - a0} arrivals, "
        f"{wl.completed - c0} completed, mean batch {batch_sum / max(steps, 1):.1f}, queue {len(wl.queue)}")
    return {
        "metric": "generated tok/s, 70B-shape Q4_K, Poisson 4 req/s, B<=32 (mixed prefill + decode)",
        "value": round(tokens / dt, 1), "unit": "tok/s", "n_gpus": 1, "steps": steps, "warmup_s": args.warmup_s,
        "duration_s": round(dt, 2), "ms_per_step": round(dt * 1e3 / max(steps, 1), 3), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "LLaMA-3-70B-shaped Q4_K serving: Poisson arrivals at 4 req/s, prompts "
                               "U[256,4096], outputs U[64,512], greedy, at most 32 in flight, prompts "
                               f"chunked into the ragged steps ({args.prefill_chunk} prompt tokens per step)",
                   "layers": shape.n_layers, "d_model": shape.d_model,
                   "heads": f"{shape.n_heads}q/{shape.n_kv_heads}kv", "ffn": shape.ffn, "vocab": shape.vocab,
                   "weights": "q4_k", "max_batch": max_batch, "arrivals": wl.arrived - a0,
                   "completed": wl.completed - c0, "mean_batch": round(batch_sum / max(steps, 1), 2),
                   "queued_at_end": len(wl.queue)},
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--profile-steps", type=int, default=8,
                    help="event-timed steps after the timed window (at least 1: the roofline comes from them)")
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--layers", type=int, default=None, help="layers (default: the shape's own)")
    ap.add_argument("--shape", choices=("8b", "70b"), default="8b",
                    help="8b (the headline line) or 70b (the 70B serving workload)")
    ap.add_argument("--duration", type=float, default=60.0, help="70b: timed seconds")
    ap.add_argument("--warmup-s", type=float, default=20.0, help="70b: untimed seconds from an empty system")
    ap.add_argument("--prefill-chunk", type=int, default=384,
                    help="70b: prompt tokens carried per step next to the decode rows (chunked prefill)")
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU reference baseline")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a 1 GiB device-to-device copy 5 times and exit")
    ap.add_argument("--ops", action="store_true", help="op-level Q4_K / Q8_0 matmul and ragged attention figures")
    args = ap.parse_args()
    if args.profile_steps < 1:
        ap.error("--profile-steps must be at least 1")
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
    from slate_amd.synth import LlamaShape
    if args.shape == "70b":
        shape = LlamaShape(n_layers=args.layers or 80, d_model=8192, n_heads=64, n_kv_heads=8, ffn=28672,
                           vocab=128256, max_seq=4096 + 512)
        result = run_c5(args, shape)
    else:
        shape = LlamaShape(n_layers=args.layers or 32, d_model=4096, n_heads=32, n_kv_heads=8, ffn=14336,
                           vocab=128256, max_seq=2304)
        result = run_c4(args, shape)
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
            if fmt == "q4k":
                # one activation row on slate's own row layout (the vtable's
                # matvec_q4k, backend.h:63-70): the one-kernel GEMV
                rows = torch.empty((ncopy, nblk * qb), dtype=torch.uint8, device="cuda")
                rows.copy_(raw.reshape(1, -1).expand(ncopy, -1))
                X = torch.randn(1, K, device="cuda", generator=gen)
                Y = torch.empty(1, M, device="cuda")
                torch.cuda.synchronize()

                def call_row(i, X=X, Y=Y):
                    slate_amd.check(lib.slate_hip_matmul_q4k(Y.data_ptr(), rows[i % ncopy].data_ptr(),
                                                             X.data_ptr(), 1, M, K), "q4k matmul (row layout)")
                us, same = graph_time_us(call_row, 2 * ncopy, stream, Y)
                alg = nblk * qb + 4 * K + 4 * M
                out["q4k_row_B1"] = out.get("q4k_row_B1", []) + [
                    {"M": M, "K": K, "B": 1, "layout": "row", "us": round(us, 2), "GBs": round(alg / us / 1e3, 1),
                     "frac_hbm": round(alg / us / 1e3 / HBM_PEAK_GBS, 3), "replays_match_eager": same}]
                log(fmt, out["q4k_row_B1"][-1])
                del rows
            del raw
            for B in (1, 4, 16, 32, 64):
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
    """Snapshot the KV of every decoding sequence, run slate's C decode step
    from that state (single thread as wired, then the harness-level
    threadpool variant), then the GPU step; compare the logits."""
    snap = [i for i in range(wl.B) if wl.pending[i] is None]
    kv = {i: (wl.sess[i].kv(), wl.sess[i].position, wl.last[i]) for i in snap}
    _, lg, _ = wl.m.step([wl.sess[i] for i in snap], [1] * len(snap), [wl.last[i] for i in snap],
                         want_logits=True)
    gpu = {i: lg[k] for k, i in enumerate(snap)}
    return cpu_baseline_from(m, shape, [(i, *kv[i]) for i in snap], gpu)


def cpu_baseline_from(m, shape, snap, gpu, budget_s=30.0):
    """slate_llama_decode_step (oracle/_ref) on the engine's weights and the
    given KV states: one session at a time on one thread (as slate wires
    it), then all of them over slate's own threadpool (harness level)."""
    host_threads = min(HOST_THREADS, len(os.sched_getaffinity(0)))
    os.environ.setdefault("SLATE_NUM_THREADS", str(host_threads))
    from oracle.pyoracle import Ref, RefLlama, ref_available
    import slate_amd
    from slate_amd.synth import engine_tensors, write_llama_gguf
    if not ref_available():
        return {"error": "oracle/_ref not built"}
    ref = Ref()
    path = "/dev/shm/slate_amd_bench.gguf"
    write_llama_gguf(path, shape, engine_tensors(m, shape))
    rm = RefLlama(ref, path)
    t_cpu, n_tok, worst = 0.0, 0, 0.0
    pool = {}
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
        # harness level: every snapshot session decoded at once over the pool
        rss = []
        for i, (K, V), pos, tok in snap:
            rs = rm.session()
            assert rs.set_state(K, V, pos) == 0
            rss.append(rs)
        n = len(rss)
        toks = np.array([tok for *_, tok in snap], np.int32)
        out = np.empty((n, shape.vocab), np.float32)
        rcs = np.zeros(n, np.int32)
        arr = (slate_amd.vp * n)(*[r.h for r in rss])
        t0 = time.perf_counter()
        ref.lib.ref_decode_sessions_parallel(arr, toks.ctypes.data_as(slate_amd.i32p), n,
                                             out.ctypes.data_as(slate_amd.f32p), rcs.ctypes.data_as(slate_amd.i32p))
        tp = time.perf_counter() - t0
        assert not rcs.any()
        for k, (i, *_rest) in enumerate(snap):
            worst = max(worst, float(np.abs(out[k] - gpu[i]).max() / max(np.abs(out[k]).max(), 1e-30)))
        for r in rss:
            r.free()
        pool = dict(value=round(n / tp, 4), unit="tok/s", cores=int(ref.lib.ref_pool_threads()),
                    sample=f"one decode step of {n} sequences, sessions spread over slate_threadpool_parallel_for "
                           f"(threadpool.c:122-142; harness-level, not wired in slate's LLaMA path), {tp:.1f} s")
    finally:
        rm.close()
        os.unlink(path)
    return dict(value=round(n_tok / t_cpu, 4), unit="tok/s", cores=1, kind="reference",
                sample=f"slate_llama_decode_step (slate's C, built from its sources, single thread as wired) "
                       f"on the benchmark's weights and KV state: one decode step of {n_tok} sequences, "
                       f"{t_cpu:.1f} s",
                threadpool=pool, host_cores_available=len(os.sched_getaffinity(0)),
                host_cores_used_max=host_threads, host_cpu=cpu_model(), logits_max_rel_vs_gpu=worst)


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
