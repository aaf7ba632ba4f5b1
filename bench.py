#!/usr/bin/env python
"""Benchmark of the speculative-decoding verify step on one MI355X.

Workload (the full-verify-step configuration): Qwen3-0.6B architecture (28
layers, hidden 1024, 16 Q / 8 KV heads, head_dim 128, MLP 3072, vocab 151936,
tied embeddings), random-init weights (every parameter N(0, 0.02^2), seed 0, in
the reference's registration order) cast to bf16 and quantised per output row
to int8, int8 paged KV (16-token blocks, bf16 scales), 64 sequences whose
64-token prompts repeat a seeded 16-token motif of ids in [0, 512) four times,
n-gram (n <= 3) drafting with k = 4, greedy verification, 128 output tokens per
sequence.  Synthetic data: no checkpoint or dataset is read.

One step = one batched verify step over the 64 sequences (draft, reserve KV,
forward over 64 x 5 rows, LM head, acceptance, rollback).  W untimed steps, then
K timed steps bracketed by device synchronisation; ``value`` is accepted tokens
per second (tokens emitted by the timed steps / elapsed).

Also reported on the same line:
  roofline      the dominant kernel's algorithmic bytes (or flops) per launch over
                its average launch time, from HIP events around each launch in
                the timed region (eager launches; see --graph)
  attention     the paged verify attention at the kernel-only int8 configuration
                (64 sequences, context U{128..1024}, 5 queries, fp16 scales,
                4096-block pool) over 28 distinct layer pools
  cpu_baseline  the oracle's restatement of the reference CPU path (fp32, batch 1,
                64-token motif prompt, n-gram k = 4, greedy, 128 tokens,
                contiguous KV) on this host's cores
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
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


def run_verify(args, torch):
    from nanoengine_amd import _native
    from nanoengine_amd.config import EngineSettings
    from nanoengine_amd.interface import GenerationRequest, SamplingParams
    from nanoengine_amd.qwen3 import QWEN3_0_6B, random_state_dict
    from nanoengine_amd.runtime import create_verify_engine
    from nanoengine_amd.sequence_state import Sequence

    cfg = QWEN3_0_6B
    total_steps = args.warmup + args.steps
    # every sequence must still be generating in the last timed step: a step emits at
    # most k + 1 tokens, so 128 tokens last >= 26 steps; longer runs get longer outputs
    max_new = max(OUTPUT_TOKENS, (K_DRAFT + 1) * total_steps + 2)
    max_len = PROMPT_MOTIF * PROMPT_REPEATS + max_new + K_DRAFT + 1
    t0 = time.perf_counter()
    state = random_state_dict(cfg, seed=0, std=0.02)
    log(f"random init {time.perf_counter() - t0:.1f}s")
    settings = EngineSettings(device="cuda", dtype="bfloat16", kv_cache="paged", scheduler="continuous",
                              quantization="int8", kv_cache_dtype="int8", speculative="ngram",
                              num_speculative_tokens=K_DRAFT, ngram_max_size=3, max_num_seqs=NUM_SEQS,
                              max_model_len=max_len, kv_cache_memory_mb=2048, cuda_graphs=args.graph)
    eng = create_verify_engine(cfg, state, settings, max_prefill_rows=NUM_SEQS * PROMPT_MOTIF * PROMPT_REPEATS)
    del state
    log(f"engine ready {time.perf_counter() - t0:.1f}s")
    params = SamplingParams(max_new_tokens=max_new, temperature=args.temperature, seed=0, ignore_eos=True)
    prompts = motif_prompts(NUM_SEQS, seed=0)
    seqs = [Sequence.from_request(GenerationRequest(f"s{i}", p, params)) for i, p in enumerate(prompts)]
    eng.runner.add(seqs)
    torch.cuda.synchronize()
    log("prefill done")
    for _ in range(args.warmup):
        eng.runner.step()
    timer_name = {"attention": "ne_paged_verify_attention", "gemm": "ne_w8a16_gemm",
                  "lm_head": "ne_lm_head"}[args.roofline_kernel]
    timer = _native.LaunchTimer() if not args.graph else None
    ctx_per_step, lengths_per_step = [], []
    if timer is not None:
        _native.set_launch_timer(timer_name, timer)
    torch.cuda.synchronize()
    start = time.perf_counter()
    tokens = 0
    kept_hist: dict[int, int] = {}
    for _ in range(args.steps):
        lengths = {i: s.num_tokens for i, s in enumerate(eng.runner.slots) if s is not None}
        results = eng.runner.step()
        # context of sequence b in this step = its length before the step + its guesses
        ctx_per_step.append([lengths[i] + results[i].num_guesses for i in lengths])
        lengths_per_step.append([lengths[i] for i in lengths])
        for r in results.values():
            tokens += len(r.tokens)
            kept_hist[r.num_kept] = kept_hist.get(r.num_kept, 0) + 1
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start
    _native.set_launch_timer(timer_name, None)
    roofline = None
    if timer is not None:
        durations = timer.durations_ms()
        roofline = summarize_roofline(args.roofline_kernel, durations, ctx_per_step, lengths_per_step, cfg)
    active = sum(1 for s in eng.runner.slots if s is not None)
    return {
        "elapsed": elapsed,
        "tokens": tokens,
        "kept_hist": kept_hist,
        "roofline": roofline,
        "active_at_end": active,
        "max_new": max_new,
    }


def summarize_roofline(kind, durations_ms, ctx_per_step, lengths_per_step, cfg):
    layers = cfg.num_hidden_layers
    rows = NUM_SEQS * (K_DRAFT + 1)
    if kind == "attention":
        # one launch per layer per step; context of sequence b = its length + its guesses (<= k)
        # query rows read and output rows written: one per real query (1 + guesses)
        per_step_bytes = [attention_bytes(ctxs, len(ctxs) + sum(ctxs) - sum(lens))
                          for ctxs, lens in zip(ctx_per_step, lengths_per_step, strict=True)]
        total_bytes = sum(b * layers for b in per_step_bytes)
        total_ms = sum(durations_ms)
        achieved = total_bytes / (total_ms * 1e-3) / 1e9
        return {"kernel": "paged_attention_kernel<int8>", "bound": "hbm", "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "launches": len(durations_ms), "avg_us": round(1e3 * total_ms / len(durations_ms), 2),
                "bytes_per_launch": int(total_bytes / len(durations_ms))}
    if kind == "gemm":
        h, i = cfg.hidden_size, cfg.intermediate_size
        q = cfg.num_attention_heads * cfg.head_dim
        qkv = q + 2 * cfg.num_key_value_heads * cfg.head_dim
        shapes = [(rows, qkv, h), (rows, h, q), (rows, 2 * i, h), (rows, h, i)]
        flops = sum(2 * m * n * k for m, n, k in shapes) * layers * len(ctx_per_step)
        total_s = sum(durations_ms) * 1e-3
        achieved = flops / total_s / 1e12
        traffic = sum(gemm_traffic(m, n, k) for m, n, k in shapes)
        return {"kernel": "gemm_kernel<w8a16>", "bound": "mfma", "achieved": round(achieved, 1),
                "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
                "launches": len(durations_ms), "avg_us": round(1e3 * sum(durations_ms) / len(durations_ms), 2),
                "hbm_GBps": round(traffic * layers * len(ctx_per_step) / total_s / 1e9, 1)}
    v, h = cfg.vocab_size, cfg.hidden_size
    total_s = sum(durations_ms) * 1e-3
    per_launch = 2 * v * h + 2 * rows * h + rows * (v // 64) * 8
    achieved = per_launch * len(durations_ms) / total_s / 1e9
    return {"kernel": "gemm_kernel<lm_head>", "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "launches": len(durations_ms),
            "avg_us": round(1e3 * sum(durations_ms) / len(durations_ms), 2)}


def run_attention_roofline(torch, reps: int = 5):
    """Kernel-only int8 verify attention (64 seqs, ctx U{128..1024} seed 1, 5 queries, fp16
    scales, 4096-block pool) over 28 distinct pools so the 256 MB last-level cache cannot
    hold the working set; HIP events around every launch."""
    import numpy as np

    from nanoengine_amd import _native, kernels

    dev = torch.device("cuda")
    layers, blocks, bs, hkv, hq = 28, 4096, 16, 8, 16
    rng = np.random.default_rng(1)
    ctx = rng.integers(128, 1025, size=NUM_SEQS).astype(np.int32)
    g = torch.Generator().manual_seed(1)
    perm = torch.randperm(blocks, generator=g).to(torch.int32)
    max_blocks = int(math.ceil(ctx.max() / bs))
    tables = torch.zeros(NUM_SEQS, max_blocks, dtype=torch.int32)
    cur = 0
    for b, c in enumerate(ctx):
        nb = int(math.ceil(c / bs))
        tables[b, :nb] = perm[cur : cur + nb]
        cur += nb
    slots = blocks * bs + 1
    pools = []
    for _ in range(layers):
        kc = torch.randint(-127, 128, (slots, hkv, 128), dtype=torch.int8, device=dev)
        vc = torch.randint(-127, 128, (slots, hkv, 128), dtype=torch.int8, device=dev)
        ks = (torch.rand(slots, hkv, device=dev) * 0.03 + 0.005).to(torch.float16)
        vs = (torch.rand(slots, hkv, device=dev) * 0.03 + 0.005).to(torch.float16)
        pools.append((kc, vc, ks, vs))
    rows = NUM_SEQS * 5
    q = torch.randn(rows, hq, 128, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    d = lambda a: torch.as_tensor(a).to(dev)
    t_d, c_d = tables.to(dev), d(ctx)
    qs, ql = d(np.arange(NUM_SEQS, dtype=np.int32) * 5), d(np.full(NUM_SEQS, 5, dtype=np.int32))
    ws = kernels.AttentionWorkspace()

    def launch(p):
        kernels.paged_verify_attention(q, p[0], p[1], p[2], p[3], t_d, bs, c_d, qs, ql, 5, int(ctx.max()),
                                       out=out, workspace=ws)

    for p in pools:
        launch(p)
    torch.cuda.synchronize()
    timer = _native.LaunchTimer()
    _native.set_launch_timer("ne_paged_verify_attention", timer)
    for _ in range(reps):
        for p in pools:
            launch(p)
    torch.cuda.synchronize()
    _native.set_launch_timer("ne_paged_verify_attention", None)
    dur = timer.durations_ms()
    avg_ms = sum(dur) / len(dur)
    nbytes = attention_bytes(ctx.tolist(), rows) + tables.numel() * 4
    achieved = nbytes / (avg_ms * 1e-3) / 1e9
    return {"workload": "int8 KV, 64 seqs, ctx U{128..1024} seed 1, q=5, fp16 scales",
            "bytes_per_launch": int(nbytes), "avg_us": round(avg_ms * 1e3, 2),
            "achieved": round(achieved, 1), "unit": "GB/s", "peak": HBM_PEAK_GBS,
            "frac": round(achieved / HBM_PEAK_GBS, 4), "launches": len(dur), "sum_ctx": int(ctx.sum())}


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
    parser.add_argument("--graph", action="store_true", help="replay the fixed-shape step as a HIP graph")
    parser.add_argument("--roofline-kernel", choices=("attention", "gemm", "lm_head"), default="gemm")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-attention", action="store_true")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the verify step "
              "shards by sequence with no exchange; run one process per GPU)", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    res = run_verify(args, torch)
    log(f"verify: {res['tokens']} tokens in {res['elapsed']:.3f}s")
    attention = None if args.no_attention else run_attention_roofline(torch)
    if attention:
        log(f"attention: {attention['avg_us']} us, {attention['achieved']} GB/s")
    cpu = None if args.no_cpu_baseline else run_cpu_baseline(torch)
    if cpu:
        log(f"cpu baseline: {cpu['value']} tok/s")
    value = res["tokens"] / res["elapsed"]
    line = {
        "metric": "verify-step us + accepted tok/s (64 seqs, k=4, int8 W+KV); attn HBM GB/s",
        "value": round(value, 1),
        "unit": "accepted tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * res["elapsed"] / args.steps, 4),
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
        "roofline": res["roofline"],
        "attention": attention,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
