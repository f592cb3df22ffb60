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

--summarize DIR writes the summaries in profiles/ from the rocprofv3 output
of the runs each summary names at its top (run with -d DIR/<name>), with no
GPU: kernel-trace breakdowns per step (steps split at each
pack_batch_kernel), per-shape Q4_K decode matmul figures, and the PMC
traffic table whose per-launch figure the bench line reports as
roofline.traffic.
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
        "operands": "Q4_K weights dequantised exactly to f16 (q * scale) against f32 activations split into two "
                    "f16 halves (hi + lo, ~22-bit significands), f32 accumulation; f32 K/V cache and attention",
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
        self.arrived = self.completed = self.generated = self.prompt_tokens = 0
        self.last_rows = self.last_seqs = 0

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
        self.last_rows, self.last_seqs = int(sum(n_new)), len(rows)
        self.prompt_tokens += sum(n for r, n in zip(rows, n_new) if r["done"] < len(r["prompt"]))
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
    g0, a0, c0, p0 = wl.generated, wl.arrived, wl.completed, wl.prompt_tokens
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
    prompt_tok = wl.prompt_tokens - p0
    queued = len(wl.queue)
    log(f"{steps} steps in {dt:.1f} s: {tokens} tokens, {prompt_tok} prompt tokens, {wl.arrived - a0} arrivals, "
        f"{wl.completed - c0} completed, mean batch {batch_sum / max(steps, 1):.1f}, queue {queued}")
    # the Q4_K matmuls of a few steps after the window, event-timed: useful
    # flops 2 * rows * (linear weights of the layers) + 2 * sequences * (LM
    # head weights) per step over their device time
    D, H, kvd = shape.d_model, shape.ffn, shape.kv_dim
    layer_w = shape.n_layers * (D * D * 2 + kvd * D * 2 + 3 * H * D)
    flops = 0.0
    m.profile(True)
    for _ in range(args.profile_steps):
        if wl.step(time.perf_counter() - start)[1]:
            flops += 2.0 * (wl.last_rows * layer_w + wl.last_seqs * shape.vocab * D)
    m.profile(False)
    lib.slate_hip_sync()
    raw = m.profile_read()
    mm_ms = raw["q4k_mm"][0] + raw["q4k_mm_pf"][0]
    tflops = flops / (mm_ms * 1e-3) / 1e12 if mm_ms > 0 else None
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
                   "queued_at_end": queued, "prompt_tok_s": round(prompt_tok / dt, 1)},
        "operands": "Q4_K weights dequantised exactly to f16 (q * scale) against f32 activations split into two "
                    "f16 halves (hi + lo, ~22-bit significands), f32 accumulation; f32 K/V and attention",
        "prompt_matmul": {"profiled_steps": args.profile_steps, "device_ms": round(mm_ms, 2),
                          "useful_TFLOPs": None if tflops is None else round(tflops, 1),
                          "frac_f16_peak": None if tflops is None else round(tflops / 2500.0, 4),
                          "note": "every Q4_K matmul launch of the profiled steps; two f16 MFMAs per product"},
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
    ap.add_argument("--summarize", metavar="DIR",
                    help="write the profiles/ summaries from the rocprofv3 output under DIR (no GPU needed)")
    args = ap.parse_args()
    if args.summarize:
        return summarize(args.summarize)
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


# ---------------------------------------------------------------------------
# Profile summaries (--summarize DIR): the text files under profiles/ from
# the rocprofv3 output of the runs listed at the top of each file.

D8, H8, KV8, V8 = 4096, 14336, 1024, 128256
DEC_SHAPES = ("QKV 6144x4096", "O 4096x4096", "gate+up 2x14336x4096", "down 4096x14336", "lm_head 128256x4096")
PROFILE_CMDS = {
    "trace": "rocprofv3 --kernel-trace --stats --output-format csv -d $PROF/trace -o run -- "
             "python3 bench.py --steps 64 --warmup 4 --no-cpu",
    "pmc_fetch": "rocprofv3 --pmc FETCH_SIZE --output-format csv -d $PROF/pmc_fetch -o run -- "
                 "python3 bench.py --steps 8 --warmup 2 --no-cpu",
    "pmc_write": "rocprofv3 --pmc WRITE_SIZE --output-format csv -d $PROF/pmc_write -o run -- "
                 "python3 bench.py --steps 8 --warmup 2 --no-cpu",
    "cal_fetch": "rocprofv3 --pmc FETCH_SIZE --output-format csv -d $PROF/cal_fetch -o run -- "
                 "python3 bench.py --copy-calibration",
    "cal_write": "rocprofv3 --pmc WRITE_SIZE --output-format csv -d $PROF/cal_write -o run -- "
                 "python3 bench.py --copy-calibration",
    "ops": "python3 bench.py --ops > $PROF/ops.json",
    "ops_trace": "rocprofv3 --kernel-trace --stats --output-format csv -d $PROF/ops_trace -o run -- "
                 "python3 bench.py --ops",
    "trace70": "rocprofv3 --kernel-trace --stats --output-format csv -d $PROF/trace70 -o run -- "
               "python3 bench.py --shape 70b --duration 15 --warmup-s 5 > $PROF/trace70.json",
}


def _q4(M, K):
    return M * K // 256 * 144


def dec_alg_bytes(name, T=16):
    """Algorithmic bytes of one 16-row decode matmul launch of the 8B shape:
    weights once, activations in and out once."""
    D, H, V = D8, H8, V8
    return {"QKV 6144x4096": _q4(6144, D) + 4 * T * D + 4 * T * 6144,
            "O 4096x4096": _q4(D, D) + 4 * T * D + 4 * T * D,
            "gate+up 2x14336x4096": 2 * _q4(H, D) + 4 * T * D + 4 * T * 2 * H,
            "down 4096x14336": _q4(D, H) + 4 * T * H + 4 * T * D,
            "lm_head 128256x4096": _q4(V, D) + 4 * T * D + 4 * T * V}[name]


def _one(pattern):
    import glob
    got = glob.glob(pattern, recursive=True)
    if not got:
        raise FileNotFoundError(pattern)
    return got[0]


def _kname(name):
    return name.replace("void ", "").replace("slate_hip::", "").split("(")[0]


def _dur_us(r):
    return (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3


def trace_steps(path):
    """Kernel-trace rows of a bench run split into engine steps (each step
    starts with its pack_batch_kernel; the last, possibly cut, is dropped)."""
    import csv
    rows = list(csv.DictReader(open(_one(path + "/**/*kernel_trace.csv"))))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    steps, cur = [], None
    for r in rows:
        if "pack_batch_kernel" in r["Kernel_Name"]:
            cur = []
            steps.append(cur)
        if cur is not None:
            cur.append(r)
    return steps[:-1]


def has_prompt(step):
    return any("q4k_pf_kernel" in r["Kernel_Name"] for r in step)


def dec_launches(step):
    """(row, shape) of the decode matmul launches of a decode step: QKV, O,
    gate+up, down per layer in that order, then the LM head."""
    ks = [r for r in step if _kname(r["Kernel_Name"]).startswith("q4k_dec_kernel")]
    return [(r, DEC_SHAPES[4] if i == len(ks) - 1 else DEC_SHAPES[i % 4]) for i, r in enumerate(ks)]


def step_breakdown(steps, top=14):
    import collections
    n = len(steps)
    agg = collections.defaultdict(lambda: [0.0, 0])
    span = busy = 0.0
    for s in steps:
        span += (max(int(r["End_Timestamp"]) for r in s) - int(s[0]["Start_Timestamp"])) / 1e3
        for r in s:
            busy += _dur_us(r)
            a = agg[_kname(r["Kernel_Name"])]
            a[0] += _dur_us(r)
            a[1] += 1
    out = [f"per step: span {span / n:.1f} us, kernel busy {busy / n:.1f} us, "
           f"dispatches {sum(v[1] for v in agg.values()) / n:.1f}",
           "  us/step calls/step   us/call  kernel"]
    for k, (d, c) in sorted(agg.items(), key=lambda kv: -kv[1][0])[:top]:
        out.append(f"  {d / n:9.1f}   {c / n:8.1f}  {d / c:8.2f}  {k}")
    return out, agg


def stats_lines(path, top=12):
    import csv
    out = ["  calls     avg us   total ms      %  kernel"]
    for r in list(csv.DictReader(open(_one(path + "/**/*kernel_stats.csv"))))[:top]:
        out.append(f"  {int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:10.2f} "
                   f"{float(r['TotalDurationNs']) / 1e6:10.2f} {float(r['Percentage']):6.2f}  {_kname(r['Name'])}")
    return out


def _header(title, keys, extra=()):
    out = [f"# {title}\n", "Commands (from the repository root, TMPDIR=/tmp, PROF = an output directory):"]
    out += ["  " + PROFILE_CMDS[k] for k in keys]
    out += ["  python3 bench.py --summarize $PROF", ""]
    return out + list(extra)


def summary_decode(prof):
    import collections
    import statistics
    steps = trace_steps(prof + "/trace")
    dec = [s for s in steps if not has_prompt(s)][2:]
    n = len(dec)
    out = _header("Decode step kernels, 8B-shape Q4_K engine, B=16 ragged (MI355X, one GPU)", ["trace"], [
        "Per-step figures: dispatches of the kernel trace split into engine steps at each pack_batch_kernel;",
        "decode-only steps (no q4k_pf_kernel, i.e. no prompt chunk) after the first two; 'alg' = algorithmic",
        "bytes (weights once, activations in and out once) of each launch.  Kernel durations under the tracer",
        "include its per-dispatch overhead (about 1 us); spans include the host time between steps.\n",
        f"decode-only steps analysed: {n} (of {len(steps)} steps in the run)"])
    b, _ = step_breakdown(dec)
    out += b
    per = collections.defaultdict(list)
    for s in dec:
        for r, name in dec_launches(s):
            per[name].append(_dur_us(r))
    out += ["\nq4k_dec_kernel by shape (decode steps, T=16 rows):",
            "shape                      avg us   alg MB  alg GB/s  of 8 TB/s"]
    tot_t = tot_b = cnt = 0
    for name in DEC_SHAPES:
        v, a = per[name], dec_alg_bytes(name)
        m = statistics.mean(v)
        out.append(f"{name:26s} {m:7.2f} {a / 1e6:8.2f} {a / m / 1e3:9.1f} {a / m / 1e3 / HBM_PEAK_GBS:10.3f}")
        tot_t += sum(v)
        tot_b += a * len(v)
        cnt += len(v)
    out.append(f"all q4k_dec launches: {cnt / n:.0f}/step, avg {tot_t / cnt:.2f} us, avg alg bytes "
               f"{tot_b / cnt / 1e6:.2f} MB, {tot_b / tot_t / 1e3:.1f} GB/s ({tot_b / tot_t / 1e3 / HBM_PEAK_GBS:.3f})")
    out.append("\nrocprofv3 --stats over the whole run (includes the untimed context prefill):")
    out += stats_lines(prof + "/trace")
    return "decode_step_8b_b16_kernels.txt", out


def summary_prefill(prof):
    import re
    log_text = open(prof + "/trace.log").read() if os.path.exists(prof + "/trace.log") else ""
    m = re.search(r"prefilled (\d+) context tokens", log_text)
    steps = trace_steps(prof + "/trace")
    first_dec = next(i for i, s_ in enumerate(steps) if not has_prompt(s_))
    pre = steps[:first_dec]
    mixed = [s for s in steps[first_dec:] if has_prompt(s)]
    out = _header("Prompt steps, 8B-shape Q4_K engine (MI355X, one GPU)", ["trace"], [
        "(trace.log: the run's stderr, for the count of context tokens)\n",
        "Part 1: the steps before the first decode-only step: the bench's untimed context prefill, 16",
        "sequences x U[128,2048] tokens packed into steps of up to 4096 tokens.  q4k_pf_kernel: 2*T*M*K",
        "algorithmic flops per launch (T tokens of the step); every product runs as two f16 MFMAs (activation",
        "hi and lo halves).  attn_prompt_kernel: the prompt tokens' attention on MFMA.\n",
        f"== {len(pre)} context-prefill steps"])
    b, agg = step_breakdown(pre, 10)
    out += b
    pf = sum(d for k, (d, c) in agg.items() if k.startswith("q4k_pf_kernel"))
    att = sum(d for k, (d, c) in agg.items() if k.startswith("attn_prompt_kernel") or k.startswith("attn_merge"))
    if m:
        tokens = int(m.group(1))
        lin = 6144 * D8 + D8 * D8 + 2 * H8 * D8 + D8 * H8
        flops = 2.0 * tokens * lin * 32
        out.append(f"\n{tokens} context tokens.  q4k_pf_kernel over these steps: {pf / 1e3:.1f} ms for "
                   f"{flops / 1e12:.1f} TFLOP of linear layers -> {flops / pf / 1e6:.0f} TFLOP/s useful "
                   f"({flops / pf / 1e6 / 2500:.3f} of the 2.5 PFLOP/s f16 peak; {2 * flops / pf / 1e6 / 2500:.3f} "
                   "counting both MFMAs of each product)")
        out.append(f"prompt attention (attn_prompt_kernel + attn_merge_kernel): {att / len(pre) / 1e3:.2f} ms per "
                   f"step ({att / 1e3 / tokens * 1e3:.1f} us per 1k prompt tokens)")
    out.append(f"\nPart 2: the {len(mixed)} steps with a prompt inside the timed window (the decode tokens and an")
    out.append("arrival's 64-512-token prompt); attention per step on the MFMA prompt kernel or, where the")
    out.append("decode tokens' K/V streaming outweighs the prompt work, on the tokenwise decode kernels")
    if mixed:
        b, _ = step_breakdown(mixed, 10)
        out += b
    return "prefill_chunks_8b_kernels.txt", out


def summary_traffic(prof):
    import collections
    import csv

    def pmc(path):
        return list(csv.DictReader(open(_one(path + "/**/*counter_collection.csv"))))

    def copyk(rows):
        return max(float(r["Counter_Value"]) for r in rows
                   if "copy" in r["Kernel_Name"].lower() or "elementwise" in r["Kernel_Name"])

    cf, cw = copyk(pmc(prof + "/cal_fetch")), copyk(pmc(prof + "/cal_write"))
    sf, sw = 1024 * 1024 / cf, 1024 * 1024 / cw          # 1 GiB in KiB / counter

    def dec_rows(rows):
        rows = sorted(rows, key=lambda r: int(r["Dispatch_Id"]))
        steps, cur = [], None
        for r in rows:
            if "pack_batch_kernel" in r["Kernel_Name"]:
                cur = []
                steps.append(cur)
            if cur is not None:
                cur.append(r)
        dec = [s for s in steps[:-1] if not has_prompt(s)][1:]
        return [(name, float(r["Counter_Value"])) for s in dec for r, name in dec_launches(s)]

    fr, wr = dec_rows(pmc(prof + "/pmc_fetch")), dec_rows(pmc(prof + "/pmc_write"))
    if len(fr) != len(wr) or any(a[0] != b[0] for a, b in zip(fr, wr)):
        raise ValueError("the FETCH_SIZE and WRITE_SIZE runs dispatched different decode launches")
    per = collections.defaultdict(lambda: [0, 0.0, 0.0])
    for (name, a), (_, b) in zip(fr, wr):
        p = per[name]
        p[0] += 1
        p[1] += a * 1024 * sf
        p[2] += b * 1024 * sw
    out = _header("HBM traffic of q4k_dec_kernel (decode-shaped Q4_K matmul), 8B-shape engine, B=16",
                  ["pmc_fetch", "pmc_write", "cal_fetch", "cal_write"], [
        "Each counter in its own run.  Counters are KiB per dispatch; each is scaled by what it reads for a",
        "plain 1 GiB device copy (torch copy_, 1 GiB read + 1 GiB written).  Launches: the q4k_dec_kernel",
        "dispatches of the decode-only steps (shape from the position in the step: QKV, O, gate+up, down per",
        "layer, then the LM head).  traffic = fetch + write; 'alg' = algorithmic bytes.  Extra traffic over",
        "'alg': split-K partial writes and one fetch of the activation operand per XCD.\n",
        f"copy-kernel calibration: FETCH_SIZE {cf:.0f} KiB, WRITE_SIZE {cw:.0f} KiB per 1 GiB copy -> scale "
        f"read x{sf:.4f}, write x{sw:.4f}",
        "shape                    launches  fetch MB  write MB traffic MB   alg MB traffic/alg"])
    tl = ta = tc = 0
    for name in DEC_SHAPES:
        c, a, b = per[name]
        if not c:
            continue
        fa, wb, al = a / c, b / c, dec_alg_bytes(name)
        out.append(f"{name:24s} {c:8d} {fa / 1e6:9.2f} {wb / 1e6:9.2f} {(fa + wb) / 1e6:10.2f} {al / 1e6:8.2f} "
                   f"{(fa + wb) / al:11.3f}")
        tl += a + b
        ta += al * c
        tc += c
    out.append(f"all decode-step launches: {tc}, mean traffic {tl / tc / 1e6:.2f} MB, mean algorithmic "
               f"{ta / tc / 1e6:.2f} MB, ratio {tl / ta:.3f}")
    out.append(f"traffic_bytes_per_launch: {tl / tc:.0f}")
    return "q4k_dec_traffic.txt", out


def summary_ops(prof):
    o = json.load(open(prof + "/ops.json"))
    out = _header("Op-level figures: Q4_K and Q8_0 matmuls through the C ABI (C2) and ragged GQA attention (C3), "
                  "MI355X", ["ops", "ops_trace"], [
        "Per call: device time of a captured graph of many calls / calls (the table comes from the run without",
        "the tracer).  Weights rotate over > 300 MB of copies (the Infinity Cache holds 256 MB); algorithmic",
        "bytes = weights + 4*B*K + 4*B*M; ragged attention bytes = K/V once per kv head and sequence + q in and",
        "out.", f"Measured 1 GiB device copy: {o['hbm_copy_GBs']:.0f} GB/s (nominal 8000).\n"])
    if o.get("q4k_row_B1"):
        out.append("q4k, one activation row on slate's row layout (the vtable's matvec_q4k):")
        out.append("          M      K   B  us/call     GB/s of 8 TB/s")
        for r in o["q4k_row_B1"]:
            out.append(f"       {r['M']:6d} {r['K']:6d} {r['B']:3d} {r['us']:8.2f} {r['GBs']:8.1f} {r['frac_hbm']:9.3f}")
        out.append("")
    for fmt in ("q4k", "q8_0"):
        out.append(f"{fmt} (tiled weights):      M      K   B  us/call     GB/s of 8 TB/s  TFLOP/s")
        for r in o[fmt]:
            out.append(f"                     {r['M']:6d} {r['K']:6d} {r['B']:3d} {r['us']:8.2f} {r['GBs']:8.1f} "
                       f"{r['frac_hbm']:9.3f} {r['TFLOPs']:8.1f}")
        out.append("")
    a = o["attention"]
    out.append(f"ragged attention B={a['B']} Hq={a['Hq']} Hkv={a['Hkv']} hd={a['head_dim']}, lengths "
               "clip(round(exp(N(ln 1024, 1))), 16, 16384):")
    out.append(f"  sum_L={a['sum_L']} max_L={a['max_L']}: {a['us']:.1f} us/call, {a['GBs']:.1f} GB/s "
               f"({a['frac_hbm']:.3f} of 8 TB/s)")
    out.append("\nrocprofv3 --stats of the --ops run (tracer durations):")
    out += stats_lines(prof + "/ops_trace")
    return "ops_q4k_c2_attention_c3.txt", out


def summary_c5(prof):
    steps = trace_steps(prof + "/trace70")
    res = json.loads(open(prof + "/trace70.json").read().strip().splitlines()[-1])
    n = len(steps)
    body = steps[n // 3:]                       # after the warm-up has filled the batch
    out = _header("Serving steps, 70B-shape Q4_K engine (80 layers, d 8192, 64q/8kv, SwiGLU 28672), Poisson "
                  "arrivals (MI355X, one GPU)", ["trace70"], [
        "Steps split at each pack_batch_kernel; the last two thirds of the run (the batch has filled).",
        f"Run under the tracer: {res['steps']} timed steps, {res['value']} generated tok/s, "
        f"{res['config'].get('prompt_tok_s', '?')} prompt tok/s.\n",
        f"steps analysed: {len(body)} of {n}"])
    b, _ = step_breakdown(body, 14)
    out += b
    out.append("\nrocprofv3 --stats over the whole run:")
    out += stats_lines(prof + "/trace70")
    return "serving_70b_c5_kernels.txt", out


def summarize(prof):
    """Write every profiles/ summary whose inputs exist under prof."""
    made = 0
    for fn in (summary_decode, summary_prefill, summary_traffic, summary_ops, summary_c5):
        try:
            name, lines = fn(prof)
        except (FileNotFoundError, StopIteration, KeyError) as e:
            log(f"{fn.__name__}: skipped ({e})")
            continue
        with open(os.path.join(ROOT, "profiles", name), "w") as f:
            f.write("\n".join(lines) + "\n")
        log(f"wrote profiles/{name}")
        made += 1
    return 0 if made else 1


if __name__ == "__main__":
    sys.exit(main())
