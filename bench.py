#!/usr/bin/env python
"""Benchmark of the speculative-decoding verify step on one MI355X.

Workload (the full verify step): Qwen3-0.6B architecture (28 layers, hidden
1024, 16 Q / 8 KV heads, head_dim 128, MLP 3072, vocab 151936, tied
embeddings), random-init weights (every parameter N(0, 0.02^2), seed 0, in the
reference's registration order) cast to bf16 and quantised per output row to
int8, int8 paged KV (16-token blocks, bf16 scales), 64 sequences whose 64-token
prompts repeat a seeded 16-token motif of ids in [0, 512) four times, n-gram
(n <= 3) drafting with k = 4, greedy verification, 128 output tokens per
sequence.  Synthetic data: no checkpoint or dataset is read.

One step = one batched verify step over the 64 sequences (draft, reserve KV,
forward over 64 x 5 rows, LM head, acceptance, rollback).  The fixed-shape device
part of the step (packing, forward, LM head, acceptance) is captured once as a HIP
graph and replayed, as the reference's NANOENGINE_CUDA_GRAPHS setting does for
decode; --eager launches it kernel by kernel.  W untimed steps, then
K timed steps bracketed by device synchronisation; ``value`` is accepted tokens
per second (tokens emitted by the timed steps / elapsed).

Also reported on the same line:
  roofline       the paged verify attention (the kernel the metric's GB/s names)
                 at the kernel-only int8 configuration: 64 sequences, context
                 U{128..1024} (seed 1), 5 queries, fp16 scales, a 4096-block pool,
                 28 distinct layer pools so the last-level cache cannot hold them.
                 achieved = algorithmic bytes per launch / average launch time from
                 HIP events on the launching stream; traffic = HBM bytes per launch
                 from two rocprofv3 --pmc child runs (FETCH_SIZE, WRITE_SIZE), each
                 scaled by what the counter reads for a 256 MiB copy.  The verify step's
                 sequence is timed: one plan per pass of the 28 pools, then 28 planned
                 calls; `unplanned_avg_us` times the entry point that plans inside.
                 Also under roofline: `bf16_config` (16 seqs, ctx U{256..2048}, bf16 KV)
                 and `long_context_config` (32 seqs sharing a 1024-token prefix, suffixes
                 U{4096..16384}, 9 queries for k = 8), both kernel-only.
  sampled        the same verify step with temperature-0.8 rejection sampling on seeded
                 uniforms (10 timed steps): step time, tok/s, accepted-per-step histogram
  long_context_verify
                 the full verify step for 32 sequences sharing a 1024-token prefix
                 (served from the prefix cache) with U{4096..16384}-token suffixes,
                 k = 8, greedy (10 timed steps after 2 warm-up steps; prefill untimed)
  gemm           the W8A16 projections (QKV, gate|up with SwiGLU, o and down split-K)
                 and the LM head at the step's 320 rows, kernel-only: 28 calls with
                 distinct weights replayed from a HIP graph (no host launch cost);
                 achieved/frac are MFMA TFLOP/s over QKV + gate|up
  torch_baseline the reference's verify step composed from its own PyTorch ops on
                 this GPU (dequantise-then-linear, gather + dequant + masked GQA
                 attention, logits on every row, a per-sequence verify loop with
                 host syncs), batched over the same 64 sequences
  cpu_baseline   the oracle's restatement of the reference CPU path (fp32, batch 1,
                 64-token motif prompt, n-gram k = 4, greedy, 128 tokens,
                 contiguous KV) on this host's cores
"""

from __future__ import annotations

import argparse
import csv
import json
import math
import os
import shutil
import subprocess
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "inference-engine-from-scratch_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
PROMPT_MOTIF = 16
PROMPT_REPEATS = 4
OUTPUT_TOKENS = 128
NUM_SEQS = 64
K_DRAFT = 4
CALIBRATION_BYTES = 256 << 20


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def motif_prompts(n: int, seed: int = 0) -> list[list[int]]:
    import torch

    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, 512, (PROMPT_MOTIF,), generator=g).tolist() * PROMPT_REPEATS for _ in range(n)]


def attention_bytes(ctx_lens, rows, kv_heads=8, q_heads=16, head_dim=128, int8=True, scale_bytes=2):
    per_token = kv_heads * 2 * (head_dim + scale_bytes if int8 else head_dim * 2)
    return sum(ctx_lens) * per_token + 2 * rows * q_heads * head_dim * 2


def gemm_traffic(m, n, k):
    """int8 weight + bf16 scale + bf16 activations in and out."""
    return n * k + 2 * n + 2 * m * k + 2 * m * n


def speculation_stats(tokens: int, proposed: int, accepted: int) -> dict:
    """The reference benchmark's figures (benchmarks/speculative.py:104-114): acceptance =
    accepted / proposed guesses; a target pass emits its kept guesses plus one token, so
    passes = tokens - accepted and tokens per target pass = tokens / passes."""
    return {"proposed": proposed, "accepted": accepted,
            "acceptance_rate": round(accepted / proposed, 4) if proposed else 0.0,
            "tokens_per_target_pass": round(tokens / max(tokens - accepted, 1), 4)}


def run_verify(args, torch, temperature: float | None = None, steps: int | None = None,
               warmup: int | None = None, draft: bool = False, to_completion: bool = False):
    """The verify step at 64 sequences, k = 4.  draft=True: guesses from a draft model
    (DraftModelProposer) with the target's own weights as the draft (the reference's
    default draft model id names the same Qwen3-0.6B), so every guess a greedy target
    would make is proposed and the step pays four draft forwards.  to_completion=True:
    the 128-token generation from its first verify step until every sequence has
    finished, each step timed (the batch shrinks as sequences end)."""
    from nanoengine_amd import _native
    from nanoengine_amd.config import EngineSettings
    from nanoengine_amd.interface import GenerationRequest, SamplingParams
    from nanoengine_amd.qwen3 import QWEN3_0_6B, random_state_dict
    from nanoengine_amd.runtime import create_verify_engine
    from nanoengine_amd.sequence_state import Sequence

    cfg = QWEN3_0_6B
    temperature = args.temperature if temperature is None else temperature
    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    total_steps = warmup + steps
    # every sequence must still be generating in the last timed step: a step emits at
    # most k + 1 tokens, so 128 tokens last >= 26 steps; longer runs get longer outputs
    max_new = OUTPUT_TOKENS if to_completion else max(OUTPUT_TOKENS, (K_DRAFT + 1) * total_steps + 2)
    max_len = PROMPT_MOTIF * PROMPT_REPEATS + max_new + K_DRAFT + 1
    t0 = time.perf_counter()
    state = random_state_dict(cfg, seed=0, std=0.02)
    log(f"random init {time.perf_counter() - t0:.1f}s")
    settings = EngineSettings(device="cuda", dtype="bfloat16", kv_cache="paged", scheduler="continuous",
                              quantization="int8", kv_cache_dtype="int8",
                              speculative="draft" if draft else "ngram",
                              num_speculative_tokens=K_DRAFT, ngram_max_size=3, max_num_seqs=NUM_SEQS,
                              max_model_len=max_len, kv_cache_memory_mb=2048, cuda_graphs=args.graph,
                              cuda_graph_max_batch=NUM_SEQS, cuda_graph_max_context=max_len + K_DRAFT + 1)
    eng = create_verify_engine(cfg, state, settings, max_prefill_rows=NUM_SEQS * PROMPT_MOTIF * PROMPT_REPEATS,
                               draft_config=cfg if draft else None, draft_state_dict=state if draft else None)
    del state
    log(f"engine ready {time.perf_counter() - t0:.1f}s")
    params = SamplingParams(max_new_tokens=max_new, temperature=temperature, seed=0, ignore_eos=True)
    prompts = motif_prompts(NUM_SEQS, seed=0)
    seqs = [Sequence.from_request(GenerationRequest(f"s{i}", p, params)) for i, p in enumerate(prompts)]
    eng.runner.add(seqs)
    torch.cuda.synchronize()
    log("prefill done")
    for _ in range(warmup):
        eng.runner.step()
    # no step in flight when the clock starts: the runner may have launched one ahead
    eng.runner.drain()
    while eng.runner.pending:
        eng.runner.step()
    ctx_per_step, lengths_per_step = [], []
    # HIP events around each step's device work (graph replay, or the eager launches) on
    # the stream it runs on: the step's wall time minus this is the host's share
    device_events = []
    device_step = eng.runner._run_device_step

    def timed_device_step():
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record()
        device_step()
        end.record()
        device_events.append((begin, end))

    eng.runner._run_device_step = timed_device_step
    torch.cuda.synchronize()
    start = time.perf_counter()
    # per step: the runner's slot lengths before it (its host mirror of each sequence's
    # token count) and what it emitted; the statistics are tallied after the timed loop
    records = []
    if to_completion:
        while eng.runner.active_slots:
            lengths = eng.runner.np_len.copy()
            records.append((lengths, eng.runner.step()))
    else:
        for _ in range(steps):
            lengths = eng.runner.np_len.copy()
            records.append((lengths, eng.runner.step()))
    # step() returns once its step's outputs are on the host; the runner may already
    # have launched the next step (its outputs are not counted, so neither is its time)
    elapsed = time.perf_counter() - start
    eng.runner.drain()
    torch.cuda.synchronize()
    eng.runner._run_device_step = device_step
    device_events = device_events[: len(records)]
    device_us = 1e3 * sum(b.elapsed_time(e) for b, e in device_events) / max(len(device_events), 1)
    tokens = proposed = accepted = 0
    kept_hist: dict[int, int] = {}
    for lengths, results in records:
        # context of sequence b in this step = its length before the step + its guesses
        ctx_per_step.append([int(lengths[i]) + r.num_guesses for i, r in results.items()])
        lengths_per_step.append([int(lengths[i]) for i in results])
        for r in results.values():
            tokens += len(r.tokens)
            proposed += r.num_guesses
            accepted += r.num_kept
            kept_hist[r.num_kept] = kept_hist.get(r.num_kept, 0) + 1
    active = sum(1 for s in eng.runner.slots if s is not None)
    return {
        "elapsed": elapsed,
        "steps": len(records),
        "device_us_per_step": device_us,
        "host_us_per_step": 1e6 * elapsed / max(len(records), 1) - device_us,
        "tokens": tokens,
        "kept_hist": kept_hist,
        "active_at_end": active,
        "max_new": max_new,
        "stats": speculation_stats(tokens, proposed, accepted),
        "mean_context": sum(sum(c) for c in ctx_per_step) / max(1, sum(len(c) for c in ctx_per_step)),
    }


LONG_SEQS = 32
LONG_PREFIX = 1024
LONG_K = 8
LONG_PREFILL_ROWS = 8192


def long_prompts(seed: int = 1) -> list[list[int]]:
    """32 prompts: a shared 1024-token prefix (a seeded 16-token motif repeated) and a
    suffix of U{4096..16384} tokens (the same length draw as the kernel-only long
    attention workload) repeating each prompt's own motif; ids in [0, 512)."""
    import numpy as np
    import torch

    lengths = np.random.default_rng(seed).integers(4096, 16385, size=LONG_SEQS)
    g = torch.Generator().manual_seed(seed)
    prefix = torch.randint(0, 512, (PROMPT_MOTIF,), generator=g).tolist() * (LONG_PREFIX // PROMPT_MOTIF)
    prompts = []
    for n in lengths:
        motif = torch.randint(0, 512, (PROMPT_MOTIF,), generator=g).tolist()
        prompts.append(prefix + (motif * (int(n) // PROMPT_MOTIF + 1))[: int(n)])
    return prompts


def run_verify_long(args, torch, steps: int = 10, warmup: int = 2):
    """The full verify step at long context with a shared prefix (k = 8, greedy): the
    first request prefills and registers the 1024-token prefix; the other 31 take its
    64 blocks from the prefix cache and prefill only their suffixes (chunks of 8192
    rows).  Timed like the main leg (HIP graph replay unless --eager)."""
    from nanoengine_amd.config import EngineSettings
    from nanoengine_amd.interface import GenerationRequest, SamplingParams
    from nanoengine_amd.qwen3 import QWEN3_0_6B, random_state_dict
    from nanoengine_amd.runtime import create_verify_engine
    from nanoengine_amd.sequence_state import Sequence

    cfg = QWEN3_0_6B
    prompts = long_prompts()
    max_new = (LONG_K + 1) * (steps + warmup) + 2
    max_len = max(len(p) for p in prompts) + max_new + LONG_K + 1
    tokens_needed = LONG_PREFIX + sum(len(p) - LONG_PREFIX for p in prompts) + LONG_SEQS * (max_new + 2 * 16 + LONG_K)
    per_token = 2 * cfg.num_hidden_layers * cfg.num_key_value_heads * (cfg.head_dim + 2)
    state = random_state_dict(cfg, seed=0, std=0.02)
    settings = EngineSettings(device="cuda", dtype="bfloat16", kv_cache="paged", scheduler="continuous",
                              quantization="int8", kv_cache_dtype="int8", speculative="ngram",
                              num_speculative_tokens=LONG_K, ngram_max_size=3, max_num_seqs=LONG_SEQS,
                              max_model_len=max_len, prefix_cache=True, cuda_graphs=args.graph,
                              cuda_graph_max_batch=LONG_SEQS, cuda_graph_max_context=max_len + LONG_K + 1,
                              kv_cache_memory_mb=int(math.ceil(tokens_needed * per_token / 2**20)) + 64)
    eng = create_verify_engine(cfg, state, settings, max_prefill_rows=LONG_PREFILL_ROWS)
    del state
    params = SamplingParams(max_new_tokens=max_new, seed=0, ignore_eos=True)
    seqs = [Sequence.from_request(GenerationRequest(f"l{i}", p, params)) for i, p in enumerate(prompts)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    eng.runner.add(seqs[:1])
    eng.runner.add(seqs[1:])
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    log(f"long prefill {prefill_s:.1f}s, prefix hits {eng.allocator.num_prefix_hit_tokens} tokens")
    for _ in range(warmup):
        eng.runner.step()
    torch.cuda.synchronize()
    ctx = []
    tokens = proposed = accepted = 0
    kept_hist: dict[int, int] = {}
    start = time.perf_counter()
    for _ in range(steps):
        lengths = {i: s.num_tokens for i, s in enumerate(eng.runner.slots) if s is not None}
        results = eng.runner.step()
        ctx += [lengths[i] + results[i].num_guesses for i in lengths]
        for r in results.values():
            tokens += len(r.tokens)
            proposed += r.num_guesses
            accepted += r.num_kept
            kept_hist[r.num_kept] = kept_hist.get(r.num_kept, 0) + 1
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    out = {
        "workload": "full verify step, Qwen3-0.6B architecture, 32 seqs sharing a 1024-token prefix "
                    "(prefix cache) + U{4096..16384}-token suffixes (seed 1), n-gram k=8, greedy, "
                    "int8 W + int8 paged KV",
        "steps": steps, "warmup": warmup,
        "verify_step_us": round(1e6 * elapsed / steps, 1),
        "accepted_tok_s": round(tokens / elapsed, 1),
        "mean_context": round(sum(ctx) / max(len(ctx), 1), 1),
        "prefix_hit_tokens": eng.allocator.num_prefix_hit_tokens,
        "prefill_s": round(prefill_s, 2),
        "active_at_end": sum(1 for s in eng.runner.slots if s is not None),
        "accepted_per_step_hist": {str(k): v for k, v in sorted(kept_hist.items())},
        **speculation_stats(tokens, proposed, accepted),
        "hip_graph": bool(args.graph),
    }
    del eng
    torch.cuda.empty_cache()
    return out


class AttentionWorkload:
    """Kernel-only verify attention over `layers` distinct pools, tables from a seeded
    permutation of the pool's blocks.

    int8: 64 seqs, ctx U{128..1024} (seed 1), 5 queries, fp16 scales, 4096-block pool.
    bf16: 16 seqs, ctx U{256..2048} (seed 1), 5 queries, Q/K/V ~ N(0, 1), 4096-block pool.
    bf16_step: 64 seqs, ctx U{64..192} (seed 2), 5 queries: a verify step's contexts on a
          bf16 pool.
    long: 32 seqs sharing a 1024-token prefix (the same 64 blocks at the head of every
          table), then a suffix of U{4096..16384} tokens (seed 1); 9 queries (k = 8),
          int8 KV with bf16 scales."""

    def __init__(self, torch, layers: int = 28, kind: str = "int8", ctx=None):
        import numpy as np

        from nanoengine_amd import kernels

        dev = torch.device("cuda")
        bs, hkv, hq = 16, 8, 16
        rng = np.random.default_rng(1)
        self.kind = kind
        shared = 0
        if kind == "int8":
            # ctx: other contexts for the int8 shape (the context sweep)
            drawn = rng.integers(128, 1025, size=NUM_SEQS)
            self.ctx = (drawn if ctx is None else np.asarray(ctx)).astype(np.int32)
            self.ql = 5
        elif kind == "bf16":
            self.ctx = rng.integers(256, 2049, size=16).astype(np.int32)
            self.ql = 5
        elif kind == "bf16_step":
            self.ctx = np.random.default_rng(2).integers(64, 193, size=NUM_SEQS).astype(np.int32)
            self.ql = 5
        else:
            shared = 1024
            self.ctx = (shared + rng.integers(4096, 16385, size=32)).astype(np.int32)
            self.ql = 9
        b = len(self.ctx)
        own = [int(math.ceil((c - shared) / bs)) for c in self.ctx]
        blocks = max(4096, shared // bs + sum(own) + 1)
        g = torch.Generator().manual_seed(1)
        perm = torch.randperm(blocks, generator=g).to(torch.int32)
        max_blocks = int(math.ceil(self.ctx.max() / bs))
        tables = torch.zeros(b, max_blocks, dtype=torch.int32)
        prefix = perm[: shared // bs]
        cur = shared // bs
        for i, n in enumerate(own):
            tables[i, : shared // bs] = prefix
            tables[i, shared // bs : shared // bs + n] = perm[cur : cur + n]
            cur += n
        slots = blocks * bs + 1
        self.pools = []
        for _ in range(layers):
            if kind.startswith("bf16"):
                kc = torch.randn(slots, hkv, 128, device=dev).to(torch.bfloat16)
                vc = torch.randn(slots, hkv, 128, device=dev).to(torch.bfloat16)
                self.pools.append((kc, vc, None, None))
            else:
                sdt = torch.float16 if kind == "int8" else torch.bfloat16
                kc = torch.randint(-127, 128, (slots, hkv, 128), dtype=torch.int8, device=dev)
                vc = torch.randint(-127, 128, (slots, hkv, 128), dtype=torch.int8, device=dev)
                ks = (torch.rand(slots, hkv, device=dev) * 0.03 + 0.005).to(sdt)
                vs = (torch.rand(slots, hkv, device=dev) * 0.03 + 0.005).to(sdt)
                self.pools.append((kc, vc, ks, vs))
        self.rows = b * self.ql
        self.q = torch.randn(self.rows, hq, 128, device=dev).to(torch.bfloat16)
        self.out = torch.empty_like(self.q)
        self.tables = tables.to(dev)
        self.ctx_d = torch.as_tensor(self.ctx).to(dev)
        self.q_start = torch.arange(b, dtype=torch.int32, device=dev) * self.ql
        self.q_len = torch.full((b,), self.ql, dtype=torch.int32, device=dev)
        self.ws = kernels.AttentionWorkspace()
        int8 = not kind.startswith("bf16")
        self.bytes_per_launch = attention_bytes(self.ctx.tolist(), self.rows, int8=int8) + tables.numel() * 4
        pool = self.pools[0]
        self.plannable = kernels.plan_supported(hq, hkv, self.ql, b, pool[0].dtype,
                                                None if pool[2] is None else pool[2].dtype)
        self._kernels = kernels

    def plan(self) -> None:
        """The per-step work plan every layer's planned call reads (same metadata for all pools)."""
        self._kernels.paged_attention_plan(self.tables, 16, self.ctx_d, self.q_start, self.q_len, 16, 8, self.ql,
                                           int(self.ctx.max()), self.ws)

    def launch(self, pool, planned: bool = False) -> None:
        self._kernels.paged_verify_attention(
            self.q, pool[0], pool[1], pool[2], pool[3], self.tables, 16, self.ctx_d, self.q_start,
            self.q_len, self.ql, int(self.ctx.max()), out=self.out, workspace=self.ws, planned=planned)

    def stream(self, pool) -> None:
        """The planned call's K/V reads alone, on the current plan (the memory ceiling)."""
        self._kernels.paged_kv_stream_planned(pool[0], pool[1], pool[2], pool[3], len(self.ctx), 16, self.ql,
                                              int(self.ctx.max()), self.ws)

    def runs_plan(self) -> None:
        """Balanced whole-slot runs of the same tiles, in place of the work plan."""
        self._kernels.paged_kv_runs_plan(self.tables, 16, self.ctx_d, 16, 8, self.ql, int(self.ctx.max()), self.ws)

    def stream_runs(self, pool) -> None:
        """The same K/V bytes read in the runs (all 8 KV heads of a tile per work-group)."""
        self._kernels.paged_kv_stream_runs(pool[0], pool[1], pool[2], pool[3], len(self.ctx), 16, self.ql,
                                           int(self.ctx.max()), self.ws)


def stream_ceiling(torch, w: AttentionWorkload, reps: int) -> dict:
    """Time per call of the planned call's K/V streamed alone (ne_paged_kv_stream_planned,
    same plan, tiles, ring and copies, no arithmetic) over the same pools, from HIP events
    on the launching stream: what the access pattern costs the memory system.  Beside it,
    `whole_slot_runs`: the same bytes through the same ring and copies in balanced runs
    that cross sequences, each work-group reading all 8 KV heads of its tiles
    (ne_paged_kv_runs_plan + ne_paged_kv_stream_runs)."""
    from nanoengine_amd import _native

    w.plan()
    for p in w.pools:
        w.stream(p)
    torch.cuda.synchronize()
    timer = _native.LaunchTimer()
    _native.set_launch_timer("ne_paged_kv_stream_planned", timer)
    for _ in range(reps):
        for p in w.pools:
            w.stream(p)
    torch.cuda.synchronize()
    _native.set_launch_timer("ne_paged_kv_stream_planned", None)
    dur = timer.durations_ms()
    us = 1e3 * sum(dur) / len(dur)
    kv_bytes = attention_bytes(w.ctx.tolist(), 0, int8=w.pools[0][2] is not None)
    # the same bytes in balanced whole-slot runs across sequences: is the ceiling the
    # planned split's or the memory system's?
    w.runs_plan()
    for p in w.pools:
        w.stream_runs(p)
    torch.cuda.synchronize()
    runs_timer = _native.LaunchTimer()
    _native.set_launch_timer("ne_paged_kv_stream_runs", runs_timer)
    for _ in range(reps):
        for p in w.pools:
            w.stream_runs(p)
    torch.cuda.synchronize()
    _native.set_launch_timer("ne_paged_kv_stream_runs", None)
    runs = runs_timer.durations_ms()
    runs_us = 1e3 * sum(runs) / len(runs)
    if w.ws.error_flag() != 0:
        raise RuntimeError("the K/V stream raised the workspace error flag")
    w.plan()  # the runs took the work plan's place
    return {"us": round(us, 2), "kv_bytes": int(kv_bytes), "GB_s": round(kv_bytes / us / 1e3, 1),
            "frac_of_peak": round(kv_bytes / us / 1e3 / HBM_PEAK_GBS, 4),
            "whole_slot_runs": {"us": round(runs_us, 2), "GB_s": round(kv_bytes / runs_us / 1e3, 1),
                                "frac_of_peak": round(kv_bytes / runs_us / 1e3 / HBM_PEAK_GBS, 4),
                                "split": "the sequences' tiles in order, cut into the plan grid's near-equal "
                                         "runs across sequences; a work-group reads all 8 KV heads of its run"}}


ATTENTION_WORKLOADS = {
    "bf16": "bf16 KV, 16 seqs, ctx U{256..2048} seed 1, q=5, Q/K/V N(0,1), 4096-block pool",
    "bf16_step": "bf16 KV, 64 seqs, ctx U{64..192} seed 2, q=5 (a verify step's contexts), 4096-block pool",
    "long": "int8 KV (bf16 scales), 32 seqs sharing a 1024-token prefix + U{4096..16384} suffix seed 1, "
            "q=9 (k=8)",
}


def run_attention_kernel_only(torch, kind: str, layers: int, reps: int = 3):
    """Average time per attention call (HIP events around each call on its stream) for the
    bf16 and long-context workloads: the planned call a step makes (the plan's time spread
    over its pass of `layers` calls), and the entry point that plans inside the kernel."""
    from nanoengine_amd import _native

    w = AttentionWorkload(torch, layers=layers, kind=kind)
    for p in w.pools:
        w.launch(p)
    torch.cuda.synchronize()
    timers = {name: _native.LaunchTimer() for name in
              ("ne_paged_attention_plan", "ne_paged_verify_attention_planned", "ne_paged_verify_attention")}
    for name, t in timers.items():
        _native.set_launch_timer(name, t)
    for _ in range(reps):
        for p in w.pools:
            w.launch(p)
    if w.plannable:
        for _ in range(reps):
            w.plan()
            for p in w.pools:
                w.launch(p, planned=True)
    torch.cuda.synchronize()
    for name in timers:
        _native.set_launch_timer(name, None)
    if w.ws.error_flag() != 0:
        raise RuntimeError(f"{kind} attention workload raised the workspace error flag (keys dropped)")
    unplanned = timers["ne_paged_verify_attention"].durations_ms()
    unplanned_ms = sum(unplanned) / len(unplanned)
    avg_ms = unplanned_ms
    ceiling = None
    if w.plannable:
        calls = timers["ne_paged_verify_attention_planned"].durations_ms()
        avg_ms = (sum(timers["ne_paged_attention_plan"].durations_ms()) + sum(calls)) / len(calls)
        ceiling = stream_ceiling(torch, w, reps)
    achieved = w.bytes_per_launch / (avg_ms * 1e-3) / 1e9
    out = {"workload": ATTENTION_WORKLOADS[kind], "achieved": round(achieved, 1), "unit": "GB/s",
           "frac": round(achieved / HBM_PEAK_GBS, 4), "avg_us": round(avg_ms * 1e3, 2),
           "call": "plan + planned" if w.plannable else "unplanned",
           "unplanned_avg_us": round(unplanned_ms * 1e3, 2), "kv_stream_ceiling": ceiling,
           "bytes_per_launch": int(w.bytes_per_launch), "sum_ctx": int(w.ctx.sum()), "launches": len(unplanned)}
    del w
    torch.cuda.empty_cache()
    return out


def run_attention_ctx_sweep(torch, reps: int = 5) -> dict:
    """The int8 planned call (64 seqs, 5 queries, fp16 scales, 28 pools) over several
    context draws: U{128..1024} (seed 1, the kernel-only int8 shape), uniform contexts of
    the same total, and uniform 128, 256, 512 and 1024.  A line through the uniform 128..1024
    draws' (K/V bytes, us) splits a call into a fixed part and a rate per added byte; the
    seeded draw against the uniform one of its total is what its spread of lengths costs.
    Each draw also times the K/V stream alone (the same plan and copies)."""
    import numpy as np

    from nanoengine_amd import _native

    base = np.random.default_rng(1).integers(128, 1025, size=NUM_SEQS)
    mean = int(round(float(base.mean())))
    draws = [("ctx U{128..1024} seed 1", base), (f"uniform {mean}", np.full(NUM_SEQS, mean))]
    draws += [(f"uniform {c}", np.full(NUM_SEQS, c)) for c in (128, 256, 512, 1024)]
    rows = []
    for name, ctx in draws:
        w = AttentionWorkload(torch, layers=28, kind="int8", ctx=ctx)
        w.plan()
        for p in w.pools:
            w.launch(p, planned=True)
        torch.cuda.synchronize()
        timer = _native.LaunchTimer()
        _native.set_launch_timer("ne_paged_verify_attention_planned", timer)
        for _ in range(reps):
            w.plan()
            for p in w.pools:
                w.launch(p, planned=True)
        torch.cuda.synchronize()
        _native.set_launch_timer("ne_paged_verify_attention_planned", None)
        if w.ws.error_flag() != 0:
            raise RuntimeError(f"attention sweep ({name}) raised the workspace error flag")
        dur = timer.durations_ms()
        us = 1e3 * sum(dur) / len(dur)
        kv = attention_bytes(w.ctx.tolist(), 0)
        rows.append({"contexts": name, "sum_ctx": int(w.ctx.sum()), "max_ctx": int(w.ctx.max()),
                     "kv_bytes": int(kv), "planned_us": round(us, 2),
                     "GB_s": round(w.bytes_per_launch / us / 1e3, 1),
                     "stream_us": stream_ceiling(torch, w, reps)["us"]})
        del w
        torch.cuda.empty_cache()
    xs = np.array([r["kv_bytes"] for r in rows[2:]], dtype=np.float64)
    ys = np.array([r["planned_us"] for r in rows[2:]], dtype=np.float64)
    slope, icpt = np.polyfit(xs, ys, 1)
    return {"workload": "int8 KV, 64 seqs, q=5, fp16 scales, 28 pools, planned call; context draws below",
            "draws": rows,
            "uniform_fit": {"fixed_us": round(float(icpt), 2), "TB_s_per_added_byte": round(1e-6 / slope, 2)}}


def run_attention_roofline(torch, reps: int = 5):
    """Average time per attention call over `reps` passes of the 28 pools, from HIP events
    recorded on the launching stream around each entry point.  A pass is what a verify step
    does: one plan (ne_paged_attention_plan) and 28 planned calls (the main kernel, plus the
    merge kernel when the plan splits sequences); the
    plan's time is counted and spread over the pass's calls.  The in-kernel-plan entry point
    (ne_paged_verify_attention) is timed the same way for comparison."""
    from nanoengine_amd import _native

    w = AttentionWorkload(torch)
    for p in w.pools:
        w.launch(p)
    w.plan()
    for p in w.pools:
        w.launch(p, planned=True)
    torch.cuda.synchronize()
    timers = {name: _native.LaunchTimer() for name in
              ("ne_paged_attention_plan", "ne_paged_verify_attention_planned", "ne_paged_verify_attention")}
    for name, t in timers.items():
        _native.set_launch_timer(name, t)
    for _ in range(reps):
        w.plan()
        for p in w.pools:
            w.launch(p, planned=True)
    for _ in range(reps):
        for p in w.pools:
            w.launch(p)
    torch.cuda.synchronize()
    for name in timers:
        _native.set_launch_timer(name, None)
    if w.ws.error_flag() != 0:
        raise RuntimeError("int8 attention workload raised the workspace error flag (keys dropped)")
    plan_ms = sum(timers["ne_paged_attention_plan"].durations_ms())
    calls = timers["ne_paged_verify_attention_planned"].durations_ms()
    avg_ms = (plan_ms + sum(calls)) / len(calls)
    unplanned = timers["ne_paged_verify_attention"].durations_ms()
    achieved = w.bytes_per_launch / (avg_ms * 1e-3) / 1e9
    ceiling = stream_ceiling(torch, w, reps)
    return {"kernel": "paged_attention_dma_kernel<fp16 scales, planned> (whole-sequence items, 4 work-groups "
                      "per sequence, no merge kernel at this shape)",
            "workload": "int8 KV, 64 seqs, ctx U{128..1024} seed 1, q=5, fp16 scales, 28 pools",
            "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "avg_us": round(avg_ms * 1e3, 2),
            "plan_us": round(plan_ms * 1e3 / reps, 2),
            "unplanned_avg_us": round(1e3 * sum(unplanned) / len(unplanned), 2),
            "kv_stream_ceiling": ceiling,
            "bytes_per_launch": int(w.bytes_per_launch), "launches": len(calls),
            "sum_ctx": int(w.ctx.sum())}


class GemmWorkload:
    """The verify step's projections at M = 64 x 5 = 320 rows and its LM head, each over
    `layers` distinct random weights (so the last-level cache cannot hold them):

      qkv_fused      QKV projection with QK-norm, RoPE and the int8 KV write in its epilogue
                     (the call the step makes), N = 4096, K = 1024
      gate_up_swiglu gate|up with the SwiGLU epilogue, N = 6144 (paired rows), K = 1024
      o_proj         N = 1024, K = 2048, with its residual add + RMSNorm
      down_proj      N = 1024, K = 3072, with its residual add + RMSNorm
      lm_head        bf16 [151936, 1024] tied embedding, argmax partials only

    Each launch function runs one call of its shape on layer `i`'s weights exactly as
    Qwen3VerifyModel.forward does."""

    def __init__(self, torch, layers: int = 28):
        from nanoengine_amd import kernels
        from nanoengine_amd.qwen3 import QWEN3_0_6B as cfg

        self.torch = torch
        self.kernels = kernels
        self.layers = layers
        dev = torch.device("cuda")
        self.m = m = NUM_SEQS * (K_DRAFT + 1)
        h, inter = cfg.hidden_size, cfg.intermediate_size
        hq, hkv = cfg.num_attention_heads, cfg.num_key_value_heads
        self.hq, self.hkv, self.eps = hq, hkv, cfg.rms_norm_eps
        qkv = (hq + 2 * hkv) * cfg.head_dim
        o_in = hq * cfg.head_dim
        self.shapes = {"qkv_fused": (qkv, h), "gate_up_swiglu": (2 * inter, h), "o_proj": (h, o_in),
                       "down_proj": (h, inter)}
        self.weights = {}
        for name, (n, k) in self.shapes.items():
            self.weights[name] = [(torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev),
                                   (torch.rand(n, device=dev) * 0.01 / math.sqrt(k)).to(torch.bfloat16))
                                  for _ in range(layers)]
        self.x = {k: torch.randn(m, k, device=dev).to(torch.bfloat16) for k in {h, o_in, inter}}
        self.y = {"gate_up_swiglu": torch.empty(m, inter, dtype=torch.bfloat16, device=dev)}
        self.res = torch.randn(m, h, device=dev).to(torch.bfloat16)
        self.normed = torch.empty(m, h, dtype=torch.bfloat16, device=dev)
        self.delta = torch.empty(m, h, dtype=torch.bfloat16, device=dev)
        self.norm_w = torch.ones(h, dtype=torch.bfloat16, device=dev)
        self.splits = {"o_proj": kernels.splitk_splits(m, h, o_in), "down_proj": kernels.splitk_splits(m, h, inter)}
        self.partials = torch.empty(max(self.splits.values()) * m * h, dtype=torch.float32, device=dev)
        # the fused QKV epilogue writes this step's keys/values into a 64-sequence pool
        slots = 4096 * 16 + 1
        self.kv = (torch.zeros(slots, hkv, 128, dtype=torch.int8, device=dev),
                   torch.zeros(slots, hkv, 128, dtype=torch.int8, device=dev),
                   torch.zeros(slots, hkv, dtype=torch.bfloat16, device=dev),
                   torch.zeros(slots, hkv, dtype=torch.bfloat16, device=dev))
        g = torch.Generator().manual_seed(3)
        self.positions = torch.randint(64, 200, (m,), generator=g, dtype=torch.int32).to(dev)
        self.slot_mapping = torch.randperm(slots - 1, generator=g)[:m].to(torch.int32).to(dev)
        self.rope = kernels.rope_table(4096, cfg.rope_theta).to(dev)
        self.q_out = torch.empty(m, hq, 128, dtype=torch.bfloat16, device=dev)
        self.ones128 = torch.ones(128, dtype=torch.bfloat16, device=dev)
        self.vocab = cfg.vocab_size
        self.embed = (torch.randn(cfg.vocab_size, h, device=dev) * 0.02).to(torch.bfloat16)
        self.hidden = (torch.randn(m, h, device=dev) * 0.02).to(torch.bfloat16)
        self.argmax = torch.empty(m, kernels.lm_head_num_tiles(cfg.vocab_size), dtype=torch.int64, device=dev)

    def flops(self, name: str) -> int:
        if name == "lm_head":
            return 2 * self.m * self.vocab * self.hidden.shape[1]
        n, k = self.shapes[name]
        return 2 * self.m * n * k

    def weight_bytes(self, name: str) -> int:
        if name == "lm_head":
            return self.embed.numel() * 2
        n, k = self.shapes[name]
        return n * k + 2 * n

    def launch(self, name: str, i: int) -> None:
        from nanoengine_amd._native import EPILOGUE_SWIGLU

        kernels = self.kernels
        if name == "lm_head":
            kernels.lm_head(self.hidden, self.embed, logits=False, argmax_partials=self.argmax)
            return
        w, s = self.weights[name][i]
        n, k = self.shapes[name]
        x = self.x[k]
        if name == "qkv_fused":
            kernels.w8a16_qkv_norm_rope_kv(x, w, s, self.hq, self.hkv, self.ones128, self.ones128, self.eps,
                                           self.positions, self.rope, self.slot_mapping, *self.kv, q_out=self.q_out)
        elif name == "gate_up_swiglu":
            kernels.w8a16_gemm(x, w, s, epilogue=EPILOGUE_SWIGLU, out=self.y[name])
        else:
            splits = self.splits[name]
            if splits > 1:
                parts = self.partials[: splits * self.m * n]
                kernels.w8a16_gemm_splitk(x, w, s, splits, out=parts)
                kernels.splitk_add_rmsnorm(self.res, parts, splits, self.norm_w, self.eps, out=self.normed)
            else:
                kernels.w8a16_gemm(x, w, s, out=self.delta)
                kernels.add_rmsnorm(self.res, self.delta, self.norm_w, self.eps, out=self.normed)

    def launch_all(self, name: str) -> None:
        for i in range(1 if name == "lm_head" else self.layers):
            self.launch(name, i)


def run_accept_sampled_kernel_only(torch, reps: int = 20) -> dict:
    """Sampled acceptance alone (ne_accept) at the verify step's shape: 64 sequences x 5
    rows x 151,936 bf16 logits, 4 n-gram guesses each, T = 0.8, top-p 1 and 0.9.  Logits
    N(0, 1) with one token per row raised to 10.6 (about 0.63 of the row's probability at
    T = 0.8); a guess is that token with probability 0.8, else a random one, so that
    sequences keep 0..4 guesses.  HIP-graph replays, timed with events on the replay
    stream; reports the kept-guess histogram of the call."""
    from nanoengine_amd import kernels
    from nanoengine_amd.qwen3 import QWEN3_0_6B as cfg

    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(5)
    vocab, b, k = cfg.vocab_size, NUM_SEQS, K_DRAFT
    logits = torch.randn(b * (k + 1), vocab, generator=g)
    top = torch.randint(0, vocab, (b * (k + 1),), generator=g)
    logits[torch.arange(b * (k + 1)), top] = 10.6
    logits = logits.to(torch.bfloat16)
    targets = top.view(b, k + 1)[:, :k].to(torch.int32)
    drafts = torch.where(torch.rand(b, k, generator=g) < 0.8, targets,
                         torch.randint(0, vocab, (b, k), generator=g, dtype=torch.int32))
    d = lambda t: t.contiguous().to(dev)
    logits, drafts = d(logits), d(drafts)
    nd = d(torch.full((b,), k, dtype=torch.int32))
    rs = d(torch.arange(b, dtype=torch.int32) * (k + 1))
    seeds = d(torch.arange(b, dtype=torch.int64) * 1000003 + 17)
    steps = d(torch.zeros(b, dtype=torch.int64))
    temps = d(torch.full((b,), 0.8, dtype=torch.float32))
    out = {"workload": f"ne_accept, {b} seqs x {k + 1} rows x {vocab} bf16 logits N(0, 1), one token per row at "
                       f"10.6, {k} guesses per sequence (that token w.p. 0.8, else random), T = 0.8"}
    for top_p in (1.0, 0.9):
        tops = d(torch.full((b,), top_p, dtype=torch.float32))
        o = torch.empty(b, k + 1, dtype=torch.int32, device=dev)
        n = torch.empty(b, dtype=torch.int32, device=dev)

        def body():
            kernels.accept(drafts, nd, rs, vocab, logits=logits, temperature=temps, top_p=tops, any_sampled=True,
                           seeds=seeds, steps=steps, out_tokens=o, num_out=n)

        us = _graph_time_us(torch, body, reps)
        kept = (n.cpu() - 1).tolist()
        out[f"top_p_{top_p}"] = {"avg_us": round(us, 2),
                                 "kept_hist": {str(c): kept.count(c) for c in range(k + 1)}}
    return out


GEMM_NAMES = ("qkv_fused", "gate_up_swiglu", "o_proj", "down_proj", "lm_head")


def run_gemm_roofline(torch, layers: int = 28, reps: int = 10, counters: dict | None = None):
    """The W8A16 projections and the LM head of the verify step at M = 64 x 5 = 320 rows,
    kernel-only: `layers` calls with distinct random weights captured in one HIP graph
    and replayed `reps` times, so the time is GPU time without host launch cost.  o_proj
    and down_proj include their residual add + RMSNorm (what the step runs after them).
    `counters` (from measure_counters) adds each shape's rocprofv3 counter readings."""
    w = GemmWorkload(torch, layers=layers)
    out = {}
    for name in GEMM_NAMES:
        calls = 1 if name == "lm_head" else layers
        us = _graph_time_us(torch, lambda: w.launch_all(name), reps) / calls
        flops = w.flops(name)
        entry = {"avg_us": round(us, 2), "TFLOP_s": round(flops / us / 1e6, 1),
                 "mfma_frac": round(flops / us / 1e6 / BF16_PEAK_TFLOPS, 4),
                 "weight_GB_s": round(w.weight_bytes(name) / us / 1e3, 1)}
        if name != "lm_head":
            entry["n"], entry["k"] = w.shapes[name]
        entry["m"] = w.m
        if counters is not None and name in counters:
            entry["counters"] = counters[name]
        out[name] = entry
    # at most 80 rows the LM head runs its small-batch kernel (a draft model's 64-row decode)
    from nanoengine_amd import kernels

    h64, a64 = w.hidden[:64], w.argmax[:64]
    us = _graph_time_us(torch, lambda: kernels.lm_head(h64, w.embed, logits=False, argmax_partials=a64), reps)
    out["lm_head_64_rows"] = {"avg_us": round(us, 2), "weight_GB_s": round(w.weight_bytes("lm_head") / us / 1e3, 1),
                              "m": 64, "kernel": "lm_head_small_kernel"}
    del w
    torch.cuda.empty_cache()
    proj = [n for n in GEMM_NAMES if n != "lm_head"]
    flops = sum(2 * out[n]["m"] * out[n]["n"] * out[n]["k"] for n in proj)
    us = sum(out[n]["avg_us"] for n in proj)
    return {"kernel": "W8A16 projections (qkv fused, gate|up SwiGLU, o, down incl. add+RMSNorm) and lm_head_kernel",
            "bound": "mfma", "achieved": round(flops / us / 1e6, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(flops / us / 1e6 / BF16_PEAK_TFLOPS, 4),
            "per_layer_us": round(us, 2),
            "note": "achieved/frac over one layer's four projection calls (MFMA TFLOP/s at M=320); per-shape "
                    "detail, counter traffic and MFMA busy below",
            "shapes": out}


def _graph_time_us(torch, body, reps: int) -> float:
    """Average GPU time of `body` (a fixed sequence of launches) from replays of a HIP
    graph that holds it, timed with events on the replay stream."""
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        body()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=st):
            body()
        graph.replay()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(st)
        for _ in range(reps):
            graph.replay()
        stop.record(st)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) * 1e3 / reps


MARKER_BYTES = 4096
# counter passes, each its own child run (rocprofv3 does not split counters over passes):
# HBM bytes, then MFMA / LDS activity, then vector-L1 -> L2 requests and L2 hits
PMC_PASSES = {
    "fetch": ("FETCH_SIZE",),
    "write": ("WRITE_SIZE",),
    "sq": ("MfmaUtil", "SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE",
           "SQ_BUSY_CU_CYCLES"),
    "l2": ("TCP_TCC_READ_REQ_sum", "TCP_TCC_READ_REQ_LATENCY_sum", "TCC_HIT_sum", "TCC_MISS_sum"),
}
PMC_GROUPS = ("attention",) + GEMM_NAMES


def pmc_child(torch, groups: tuple[str, ...]) -> int:
    """What the rocprofv3 --pmc passes profile: each group's calls (attention: one plan and
    28 planned calls; each projection: 28 distinct-weight calls; the LM head: one call),
    every group followed by a MARKER_BYTES copy, then a copy of CALIBRATION_BYTES whose
    counter reading calibrates the byte counters."""
    import ctypes

    from nanoengine_amd import _native

    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    m = torch.empty(MARKER_BYTES, dtype=torch.uint8, device="cuda")
    marker = lambda: _native.call("ne_copy_bytes", ctypes.c_void_p(m.data_ptr()),
                                  ctypes.c_void_p(m.data_ptr() + MARKER_BYTES // 2), MARKER_BYTES // 2, stream())
    calls = {}
    if "attention" in groups:
        w = AttentionWorkload(torch)
        w.plan()
        for p in w.pools:
            w.launch(p, planned=True)
        torch.cuda.synchronize()
        marker()
        calls["attention"] = len(w.pools)
        del w
    gemm = [g for g in groups if g in GEMM_NAMES]
    if gemm:
        gw = GemmWorkload(torch)
        for name in gemm:
            gw.launch_all(name)
            torch.cuda.synchronize()
            marker()
            calls[name] = 1 if name == "lm_head" else gw.layers
        del gw
    torch.cuda.empty_cache()
    a = torch.empty(CALIBRATION_BYTES, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    _native.call("ne_copy_bytes", ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()), a.numel(), stream())
    torch.cuda.synchronize()
    print(json.dumps({"pmc_child": "done", "calls": calls}), flush=True)
    return 0


def _pmc_run(prof: str, counters: tuple[str, ...], groups: tuple[str, ...]) -> list[dict] | None:
    """One rocprofv3 --pmc child run; the per-dispatch rows of our kernels in dispatch order."""
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as tmp:
        cmd = ["timeout", "-s", "KILL", "150", prof, "--pmc", *counters, "--output-format", "csv", "-d", tmp,
               "-o", "run", "--", sys.executable, str(ROOT / "bench.py"), "--pmc-child", "--pmc-groups",
               ",".join(groups)]
        log(f"pmc pass {' '.join(counters)}")
        r = subprocess.run(cmd, capture_output=True, text=True)
        found = list(Path(tmp).rglob("*counter_collection.csv"))
        if r.returncode != 0 and not found:
            log(f"pmc pass failed ({r.returncode}): {r.stderr[-400:]}")
            return None
        rows = list(csv.DictReader(open(found[0])))
    rows = [x for x in rows if x["Kernel_Name"].removeprefix("void ").startswith("ne::")]
    rows.sort(key=lambda x: int(x["Dispatch_Id"]))
    return rows


def _split_groups(rows: list[dict], groups: tuple[str, ...]):
    """Dispatches between marker copies, by group, plus the calibration copy's rows."""
    by_dispatch: dict[int, list[dict]] = {}
    for x in rows:
        by_dispatch.setdefault(int(x["Dispatch_Id"]), []).append(x)
    out = {g: [] for g in groups}
    gi = 0
    calib = None
    for did in sorted(by_dispatch):
        recs = by_dispatch[did]
        if "copy_kernel" in recs[0]["Kernel_Name"]:
            if gi < len(groups):
                gi += 1
            else:
                calib = recs
            continue
        if gi < len(groups):
            out[groups[gi]].append(recs)
    return out, calib


def measure_counters(groups: tuple[str, ...] = PMC_GROUPS) -> dict | None:
    """Per-call counter readings of each group's kernels from the PMC_PASSES rocprofv3
    runs over `--pmc-child` (made before this process touches the GPU).

    fetch_bytes / write_bytes: HBM bytes per call, FETCH_SIZE / WRITE_SIZE scaled by
    the reading each gives for the CALIBRATION_BYTES copy (which reads and writes that
    many bytes).  mfma_util: MfmaUtil (MFMA busy cycles over GPU-active cycles x SIMDs),
    averaged over the group's GEMM dispatches.  l1_l2_read_bytes: vector-L1 -> L2 read
    requests per call, scaled to bytes by the copy's requests per byte."""
    prof = shutil.which("rocprofv3")
    if prof is None:
        log("rocprofv3 not found: counters not measured")
        return None
    res: dict[str, dict] = {g: {"calls": 0} for g in groups}
    for pass_name, counters in PMC_PASSES.items():
        rows = _pmc_run(prof, counters, groups)
        if rows is None:
            return None
        per_group, calib = _split_groups(rows, groups)
        if calib is None:
            log(f"pmc pass {pass_name}: calibration copy not found")
            return None

        def total(recs_list, name):
            return sum(float(r["Counter_Value"]) for recs in recs_list for r in recs if r["Counter_Name"] == name)

        for g in groups:
            disp = per_group[g]
            calls = 1 if g == "lm_head" else 28
            res[g]["calls"] = calls
            res[g]["dispatches_per_call"] = round(len(disp) / calls, 2)
            if pass_name == "fetch":
                scale = (CALIBRATION_BYTES / 1024.0) / total([calib], "FETCH_SIZE")
                res[g]["fetch_bytes"] = int(total(disp, "FETCH_SIZE") * scale * 1024 / calls)
                res[g]["fetch_scale"] = round(scale, 4)
            elif pass_name == "write":
                scale = (CALIBRATION_BYTES / 1024.0) / total([calib], "WRITE_SIZE")
                res[g]["write_bytes"] = int(total(disp, "WRITE_SIZE") * scale * 1024 / calls)
                res[g]["write_scale"] = round(scale, 4)
            elif pass_name == "sq":
                # the main (longest) kernel of each call: the first dispatch of the call
                mains = [recs for recs in disp if not any(s in recs[0]["Kernel_Name"] for s in
                                                          ("rmsnorm", "plan_kernel", "merge"))]
                util = [float(r["Counter_Value"]) for recs in mains for r in recs if r["Counter_Name"] == "MfmaUtil"]
                res[g]["mfma_util_pct"] = round(sum(util) / len(util), 2) if util else None
                res[g]["mfma_mops_bf16"] = int(total(disp, "SQ_INSTS_VALU_MFMA_MOPS_BF16") / calls)
                res[g]["lds_bank_conflict_cycles"] = int(total(disp, "SQ_LDS_BANK_CONFLICT") / calls)
                res[g]["lds_active_cycles"] = int(total(disp, "SQ_LDS_IDX_ACTIVE") / calls)
                res[g]["busy_cu_quad_cycles"] = int(total(disp, "SQ_BUSY_CU_CYCLES") / calls)
            else:
                per_byte = total([calib], "TCP_TCC_READ_REQ_sum") / CALIBRATION_BYTES
                req = total(disp, "TCP_TCC_READ_REQ_sum")
                res[g]["l1_l2_read_req"] = int(req / calls)
                res[g]["l1_l2_read_bytes"] = int(req / per_byte / calls) if per_byte else None
                res[g]["l2_hit_pct"] = round(100 * total(disp, "TCC_HIT_sum") / max(
                    total(disp, "TCC_HIT_sum") + total(disp, "TCC_MISS_sum"), 1), 2)
                res[g]["l1_l2_read_latency_cycles"] = round(total(disp, "TCP_TCC_READ_REQ_LATENCY_sum") / max(req, 1), 1)
    for g in groups:
        if "fetch_bytes" in res[g] and "write_bytes" in res[g]:
            res[g]["traffic"] = res[g]["fetch_bytes"] + res[g]["write_bytes"]
    return res


class TorchReferenceStep:
    """The reference's verify step composed from its own PyTorch ops, batched over the
    benchmark's 64 sequences, on this GPU with no HIP kernel of this library:

      build_step_inputs      host lists -> token/position/slot/mask tensors each step
                             (ne/engine/generation/batch_builder.py:22-65,
                             ne/engine/memory/paged_allocator.py:69-79)
      Int8Linear.forward     dequantise the whole weight, then F.linear
                             (ne/models/int8_quantization.py:55-57)
      RMSNorm, RoPE, QK-norm ne/models/qwen3.py:31-68, 89-115
      run_cached_attention   quantise + index_copy_ the new K/V, gather the padded
                             context, dequantise, masked GQA attention
                             (ne/models/attention_context.py:42-109)
      compute_logits         every row of the step (ne/models/qwen3.py:197-203)
      verify_proposal        per sequence, one-hot target and draft, .item() per guess
                             (ne/engine/speculative/verifier.py:27-60)

    Attention runs SDPA's math path written out (scores, masked softmax, weighted
    sum) with the key operand made contiguous: torch's bf16 batched matmul with a
    transposed right operand is not safe on this platform."""

    def __init__(self, torch, state: dict, ctx_len: int, block_size: int = 16):
        from nanoengine_amd.qwen3 import QWEN3_0_6B, quantize_rows

        self.torch = torch
        self.F = torch.nn.functional
        self.c = QWEN3_0_6B
        dev = torch.device("cuda")
        bf = torch.bfloat16
        self.layers = []
        for i in range(self.c.num_hidden_layers):
            p = f"model.layers.{i}."
            lw = {}
            for name in ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                         "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"):
                q8, s = quantize_rows(state[p + name + ".weight"].to(bf))
                lw[name] = (q8.to(dev), s.to(dev))
            for name in ("self_attn.q_norm", "self_attn.k_norm", "input_layernorm", "post_attention_layernorm"):
                lw[name] = state[p + name + ".weight"].to(bf).to(dev)
            self.layers.append(lw)
        self.embed = state["model.embed_tokens.weight"].to(bf).to(dev)
        self.norm = state["model.norm.weight"].to(bf).to(dev)
        self.bs = block_size
        self.ctx_len = ctx_len  # tokens per sequence before the step's guesses
        blocks_per_seq = math.ceil((ctx_len + K_DRAFT + 1) / block_size)
        self.num_slots = NUM_SEQS * blocks_per_seq * block_size
        shape = (self.num_slots + 1, self.c.num_key_value_heads, self.c.head_dim)
        self.kc = [torch.zeros(shape, dtype=torch.int8, device=dev) for _ in self.layers]
        self.vc = [torch.zeros(shape, dtype=torch.int8, device=dev) for _ in self.layers]
        self.ks = [torch.zeros(shape[:2] + (1,), dtype=bf, device=dev) for _ in self.layers]
        self.vs = [torch.zeros(shape[:2] + (1,), dtype=bf, device=dev) for _ in self.layers]
        # block tables as the paged allocator leaves them: FIFO blocks per sequence
        self.tables = [list(range(b * blocks_per_seq, (b + 1) * blocks_per_seq)) for b in range(NUM_SEQS)]
        g = torch.Generator().manual_seed(5)
        self.history = [torch.randint(0, 512, (ctx_len,), generator=g).tolist() for _ in range(NUM_SEQS)]
        self.guesses = [h[-K_DRAFT:] for h in self.history]
        self.dev = dev

    # ---- reference ops ----
    def rmsnorm(self, x, w):
        dt = x.dtype
        x = x.float()
        x = x * self.torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.c.rms_norm_eps)
        return w * x.to(dt)

    def int8_linear(self, x, wq):
        q8, s = wq
        return self.F.linear(x, q8.to(x.dtype) * s[:, None])

    def quantize(self, x):
        s = x.abs().amax(-1, keepdim=True).float().clamp(min=1e-8) / 127
        return self.torch.round(x.float() / s).clamp(-127, 127).to(self.torch.int8), s.to(x.dtype)

    def rope(self, x, cos, sin):
        a, b = x.chunk(2, dim=-1)
        return x * cos + self.torch.cat((-b, a), dim=-1) * sin

    def step(self) -> list[list[int]]:
        torch, c = self.torch, self.c
        q_rows = K_DRAFT + 1
        # build_step_inputs: host lists -> tensors
        tok_rows, pos_rows = [], []
        for h, gs in zip(self.history, self.guesses):
            L = len(h)
            tok_rows.append([h[-1]] + gs)
            pos_rows.append(list(range(L - 1, L - 1 + q_rows)))
        ctx = self.ctx_len + K_DRAFT
        per_row = math.ceil(ctx / self.bs)
        tables = torch.tensor([t[:per_row] for t in self.tables], dtype=torch.int64)
        kpos = torch.arange(ctx)
        context_slots = (tables[:, kpos // self.bs] * self.bs + kpos % self.bs).to(self.dev)
        tokens = torch.tensor(tok_rows, device=self.dev)
        positions = torch.tensor(pos_rows, device=self.dev)
        slot_mapping = context_slots.gather(1, positions)
        mask = ((kpos.to(self.dev)[None, None, :] <= positions[:, :, None])
                & (kpos.to(self.dev)[None, None, :] < ctx)).unsqueeze(1)
        # forward
        x = self.embed[tokens]
        exps = torch.arange(0, c.head_dim, 2, device=self.dev, dtype=torch.float32) / c.head_dim
        ang = positions.float()[..., None] * (1.0 / (c.rope_theta ** exps))
        ang = torch.cat((ang, ang), -1).unsqueeze(1)
        cos, sin = ang.cos().to(x.dtype), ang.sin().to(x.dtype)
        b, s = tokens.shape
        nh, nkv, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        for i, lw in enumerate(self.layers):
            h = self.rmsnorm(x, lw["input_layernorm"])
            q = self.rmsnorm(self.int8_linear(h, lw["self_attn.q_proj"]).view(b, s, nh, d),
                             lw["self_attn.q_norm"]).transpose(1, 2)
            k = self.rmsnorm(self.int8_linear(h, lw["self_attn.k_proj"]).view(b, s, nkv, d),
                             lw["self_attn.k_norm"]).transpose(1, 2)
            v = self.int8_linear(h, lw["self_attn.v_proj"]).view(b, s, nkv, d).transpose(1, 2)
            q, k = self.rope(q, cos, sin), self.rope(k, cos, sin)
            target = slot_mapping.reshape(-1)
            for cache, scales, vec in ((self.kc[i], self.ks[i], k), (self.vc[i], self.vs[i], v)):
                qv, sv = self.quantize(vec.transpose(1, 2).reshape(-1, nkv, d))
                cache.index_copy_(0, target, qv)
                scales.index_copy_(0, target, sv)
            ck = (self.kc[i][context_slots].to(x.dtype) * self.ks[i][context_slots]).transpose(1, 2)
            cv = (self.vc[i][context_slots].to(x.dtype) * self.vs[i][context_slots]).transpose(1, 2)
            ck = ck.repeat_interleave(nh // nkv, dim=1)
            cv = cv.repeat_interleave(nh // nkv, dim=1).contiguous()
            scores = torch.matmul(q.contiguous(), ck.transpose(-1, -2).contiguous()) * (1.0 / math.sqrt(d))
            scores = scores.masked_fill(~mask, float("-inf"))
            attn = torch.matmul(torch.softmax(scores, dim=-1), cv)
            x = x + self.int8_linear(attn.transpose(1, 2).reshape(b, s, -1), lw["self_attn.o_proj"])
            h2 = self.rmsnorm(x, lw["post_attention_layernorm"])
            mlp = self.F.silu(self.int8_linear(h2, lw["mlp.gate_proj"])) * self.int8_linear(h2, lw["mlp.up_proj"])
            x = x + self.int8_linear(mlp, lw["mlp.down_proj"])
        hidden = self.rmsnorm(x, self.norm)
        logits = self.F.linear(hidden, self.embed)  # [b, k+1, V]
        # verify_proposal per sequence, greedy, one-hot draft
        out = []
        vocab = logits.shape[-1]
        for bi in range(b):
            target = self.F.one_hot(torch.argmax(logits[bi], dim=-1), vocab).float()
            kept = []
            for j, guess in enumerate(self.guesses[bi]):
                draft = self.F.one_hot(torch.tensor(guess, device=self.dev), vocab).float()
                acc = (target[j, guess] / draft[guess].clamp(min=1e-12)).clamp(max=1.0).item()
                if acc >= 1.0:
                    kept.append(guess)
                    continue
                residual = (target[j] - draft).clamp(min=0.0)
                if residual.sum() <= 0:
                    residual = target[j]
                residual = residual / residual.sum()
                kept.append(int(torch.argmax(residual).item()))
                break
            else:
                kept.append(int(torch.argmax(target[len(self.guesses[bi])]).item()))
            out.append(kept)
        return out


def run_torch_baseline(torch, state, ctx_len: int, steps: int = 5, warmup: int = 2):
    t0 = time.perf_counter()
    ref = TorchReferenceStep(torch, state, ctx_len)
    log(f"torch baseline ready {time.perf_counter() - t0:.1f}s")
    for _ in range(warmup):
        ref.step()
    torch.cuda.synchronize()
    start = time.perf_counter()
    for _ in range(steps):
        ref.step()
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - start) / steps
    return {"verify_step_us": round(step_s * 1e6, 1), "steps": steps, "context_tokens": ctx_len,
            "workload": f"64 seqs x (1 + {K_DRAFT}) rows, context {ctx_len} + {K_DRAFT} tokens each, int8 W + int8 "
                        "paged KV, eager PyTorch ops of the reference on this GPU"}


def run_cpu_baseline(torch):
    """The oracle's restatement of the reference CPU path, batch 1 (see module doc)."""
    from oracle import model as om
    from oracle.paging import ContiguousSlotAllocator
    from oracle.verify import ModelRunner, Sequence, SpeculativeStats, generate_speculative

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    t0 = time.perf_counter()
    model = om.build_random_model(om.QWEN3_0_6B, seed=0, std=0.02, dtype=torch.float32)
    log(f"cpu baseline model built {time.perf_counter() - t0:.1f}s on {cores} threads")
    prompt = motif_prompts(1, seed=0)[0]
    max_len = len(prompt) + OUTPUT_TOKENS + K_DRAFT + 1
    pool = om.KVCachePool(om.QWEN3_0_6B, max_len, torch.float32)
    runner = ModelRunner(model, pool, ContiguousSlotAllocator(1, max_len))
    seq = Sequence("cpu", list(prompt), len(prompt), OUTPUT_TOKENS)
    stats = SpeculativeStats()
    start = time.perf_counter()
    out = generate_speculative(runner, seq, K_DRAFT, 3, stats=stats)
    seconds = time.perf_counter() - start
    steps = sorted(stats.step_seconds)
    return {"value": round(len(out) / seconds, 3), "unit": "accepted tok/s", "cores": cores,
            "kind": "port",
            "sample": (f"fp32 Qwen3-0.6B (random N(0,0.02), seed 0), batch 1, 64-token motif prompt, "
                       f"n-gram k=4 greedy, {len(out)} tokens, contiguous KV; {seconds:.1f}s total incl. "
                       "prefill"),
            "verify_step_us_mean": round(1e6 * sum(steps) / max(len(steps), 1), 1),
            "verify_step_us_median": round(1e6 * steps[len(steps) // 2], 1) if steps else None,
            "acceptance": round(stats.accepted / stats.proposed, 4) if stats.proposed else 0.0,
            "tokens_per_pass": round(len(out) / max(len(out) - stats.accepted, 1), 3)}


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--temperature", type=float, default=0.0)
    parser.add_argument("--eager", dest="graph", action="store_false",
                        help="launch the step's kernels one by one instead of replaying a HIP graph")
    parser.add_argument("--only", choices=("all", "verify", "attention", "gemm", "baseline", "long", "draft",
                                           "accept", "attention_sweep"),
                        default="all")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-torch-baseline", action="store_true")
    parser.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 --pmc passes")
    parser.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    parser.add_argument("--pmc-groups", default=",".join(PMC_GROUPS), help=argparse.SUPPRESS)
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the verify step "
              "shards by sequence with no exchange; run one process per GPU)", file=sys.stderr)
        return 2
    if args.pmc_child:
        import torch

        return pmc_child(torch, tuple(args.pmc_groups.split(",")))
    # counter passes first, as child processes, before this process initialises the GPU
    counters = None
    if args.only in ("all", "attention", "gemm") and not args.no_traffic:
        groups = PMC_GROUPS if args.only == "all" else (("attention",) if args.only == "attention" else GEMM_NAMES)
        counters = measure_counters(groups)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    res = None
    if args.only in ("all", "verify"):
        res = run_verify(args, torch)
        log(f"verify: {res['tokens']} tokens in {res['elapsed']:.3f}s")
    attention = None
    if args.only in ("all", "attention"):
        attention = run_attention_roofline(torch)
        attention["traffic"] = None
        if counters is not None and "attention" in counters:
            attention["traffic"] = counters["attention"].get("traffic")
            attention["counters"] = counters["attention"]
        log(f"attention: {attention['avg_us']} us, {attention['achieved']} GB/s")
        attention["bf16_config"] = run_attention_kernel_only(torch, "bf16", layers=28)
        log(f"attention bf16: {attention['bf16_config']['avg_us']} us")
        attention["bf16_step_config"] = run_attention_kernel_only(torch, "bf16_step", layers=28)
        log(f"attention bf16 at step contexts: {attention['bf16_step_config']['avg_us']} us")
        attention["long_context_config"] = run_attention_kernel_only(torch, "long", layers=8)
        log(f"attention long context: {attention['long_context_config']['avg_us']} us")
    gemm = None
    if args.only in ("all", "gemm"):
        gemm = run_gemm_roofline(torch, counters=counters)
        log(f"gemm: {gemm['achieved']} TFLOP/s over QKV and gate|up")
    if args.only == "attention_sweep":  # the attention call's fixed part and per-byte rate
        print(json.dumps({"attention_ctx_sweep": run_attention_ctx_sweep(torch)}), flush=True)
        return 0
    if args.only == "accept":  # the sampled acceptance kernel alone, and the T = 0.8 step
        s_res = run_verify(args, torch, temperature=0.8, steps=args.steps, warmup=args.warmup)
        print(json.dumps({"accept_kernel_only": run_accept_sampled_kernel_only(torch),
                          "sampled_verify_step_us": round(1e6 * s_res["elapsed"] / args.steps, 1),
                          "sampled_device_step_us": round(s_res["device_us_per_step"], 1)}), flush=True)
        return 0
    torch_base = None
    if args.only in ("all", "baseline") and not args.no_torch_baseline:
        from nanoengine_amd.qwen3 import QWEN3_0_6B, random_state_dict

        ctx_len = int(round(res["mean_context"])) if res else PROMPT_MOTIF * PROMPT_REPEATS + 32
        torch_base = run_torch_baseline(torch, random_state_dict(QWEN3_0_6B, seed=0, std=0.02), ctx_len)
        log(f"torch baseline: {torch_base['verify_step_us']} us per step")
    sampled = None
    if args.only == "all":
        # the same step with temperature-0.8 rejection sampling on seeded uniforms
        s_res = run_verify(args, torch, temperature=0.8, steps=10, warmup=2)
        s_step_us = 1e6 * s_res["elapsed"] / 10
        sampled = {"temperature": 0.8, "steps": 10, "verify_step_us": round(s_step_us, 1),
                   "accepted_tok_s": round(s_res["tokens"] / s_res["elapsed"], 1),
                   "accepted_per_step_hist": {str(k): v for k, v in sorted(s_res["kept_hist"].items())},
                   **s_res["stats"]}
        log(f"sampled: {sampled['verify_step_us']} us per step")
        sampled["accept_kernel_only"] = run_accept_sampled_kernel_only(torch)
        log(f"sampled acceptance kernel-only: {sampled['accept_kernel_only']}")
    draft_verify = None
    if args.only in ("all", "draft"):
        # draft-model speculation (the target's own weights as the draft), greedy
        d_res = run_verify(args, torch, temperature=0.0, steps=10, warmup=2, draft=True)
        d_step_us = 1e6 * d_res["elapsed"] / 10
        draft_verify = {"workload": "verify step with a draft model (DraftModelProposer; Qwen3-0.6B architecture, "
                                    "the target's weights as the draft), 64 seqs, k=4, greedy, int8 W + KV",
                        "steps": 10, "verify_step_us": round(d_step_us, 1),
                        "accepted_tok_s": round(d_res["tokens"] / d_res["elapsed"], 1),
                        "accepted_per_step_hist": {str(k): v for k, v in sorted(d_res["kept_hist"].items())},
                        **d_res["stats"]}
        log(f"draft-model verify: {draft_verify['verify_step_us']} us per step")
    full_generation = None
    if args.only in ("all", "verify"):
        # the whole 128-token generation, first verify step to last, so that the later,
        # longer-context steps (and the shrinking batch at the end) are measured too
        f_res = run_verify(args, torch, warmup=0, to_completion=True)
        full_generation = {
            "workload": "64 seqs x 64-token motif prompts, 128 output tokens each, every verify step from the "
                        "first until all sequences finished, n-gram k=4, greedy, int8 W + int8 paged KV",
            "steps": f_res["steps"], "verify_step_us_mean": round(1e6 * f_res["elapsed"] / max(f_res["steps"], 1), 1),
            "device_step_us_mean": round(f_res["device_us_per_step"], 1),
            "host_us_per_step": round(f_res["host_us_per_step"], 1),
            "accepted_tok_s": round(f_res["tokens"] / f_res["elapsed"], 1), "tokens": f_res["tokens"],
            "mean_context": round(f_res["mean_context"], 1),
            "accepted_per_step_hist": {str(k): v for k, v in sorted(f_res["kept_hist"].items())},
            **f_res["stats"]}
        log(f"full generation: {full_generation['steps']} steps, {full_generation['accepted_tok_s']} tok/s")
    long_verify = None
    if args.only in ("all", "long"):
        long_verify = run_verify_long(args, torch)
        log(f"long-context verify: {long_verify['verify_step_us']} us per step")
    cpu = None
    if args.only == "all" and not args.no_cpu_baseline:
        cpu = run_cpu_baseline(torch)
        log(f"cpu baseline: {cpu['value']} tok/s")
    if res is None:
        print(json.dumps({"attention": attention, "gemm": gemm, "torch_baseline": torch_base,
                          "long_context_verify": long_verify, "draft_verify": draft_verify}), flush=True)
        return 0
    value = res["tokens"] / res["elapsed"]
    step_us = 1e6 * res["elapsed"] / args.steps
    if torch_base is not None:
        torch_base["speedup"] = round(torch_base["verify_step_us"] / step_us, 2)
        torch_base["accepted_tok_s_at_same_acceptance"] = round(res["tokens"] / args.steps
                                                                / (torch_base["verify_step_us"] * 1e-6), 1)
    line = {
        "metric": "verify-step us + accepted tok/s (64 seqs, k=4, int8 W+KV); attn HBM GB/s",
        "value": round(value, 1),
        "unit": "accepted tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_us / 1e3, 4),
        "verify_step_us": round(step_us, 1),
        "device_step_us": round(res["device_us_per_step"], 1),
        "host_us_per_step": round(res["host_us_per_step"], 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 activations, int8 weights + KV (W8A16 on bf16 MFMA)",
        "data": "synthetic (random-init weights, seeded motif prompts)",
        "config": {"workload": "full verify step, Qwen3-0.6B architecture, 64 seqs x 64-token motif prompts, "
                               f"{res['max_new']} output tokens, n-gram k=4, "
                               f"{'greedy' if args.temperature == 0 else f'T={args.temperature}'}, "
                               "int8 W + int8 paged KV",
                   "global_batch": NUM_SEQS, "seq_len": PROMPT_MOTIF * PROMPT_REPEATS, "parallelism": "single GPU",
                   "hip_graph": bool(args.graph)},
        "accepted_per_step_hist": {str(k): v for k, v in sorted(res["kept_hist"].items())},
        **res["stats"],
        "full_generation": full_generation,
        "roofline": attention,
        "gemm": gemm,
        "sampled": sampled,
        "draft_verify": draft_verify,
        "long_context_verify": long_verify,
        "torch_baseline": torch_base,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
