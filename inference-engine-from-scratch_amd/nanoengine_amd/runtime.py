"""Build the HIP verify engine from settings (the part of create_engine,
ne/engine/runtime.py:54-182, that selects pool, allocator, quantisation and the
speculative generator)."""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from nanoengine_amd.config import TORCH_DTYPES, EngineSettings
from nanoengine_amd.draft import DraftModelProposer
from nanoengine_amd.memory import KVCachePool, PagedSlotAllocator, PrefixCachingSlotAllocator, slots_for_budget
from nanoengine_amd.metrics import EngineMetrics
from nanoengine_amd.qwen3 import Qwen3Config, Qwen3VerifyModel, Qwen3Weights
from nanoengine_amd.runner import VerifyRunner
from nanoengine_amd.speculative import BatchedSpeculativeGenerator, SpeculativeGenerator


@dataclass
class VerifyEngine:
    settings: EngineSettings
    model: Qwen3VerifyModel
    pool: KVCachePool
    allocator: PagedSlotAllocator
    runner: VerifyRunner
    metrics: EngineMetrics

    def serial_generator(self) -> SpeculativeGenerator:
        return SpeculativeGenerator(self.runner, self.metrics)

    def batched_generator(self) -> BatchedSpeculativeGenerator:
        return BatchedSpeculativeGenerator(self.runner, self.metrics)


def create_verify_engine(config: Qwen3Config, state_dict: dict[str, torch.Tensor], settings: EngineSettings,
                         stop_token_ids: frozenset[int] = frozenset(), max_prefill_rows: int | None = None,
                         draft_config: Qwen3Config | None = None,
                         draft_state_dict: dict[str, torch.Tensor] | None = None) -> VerifyEngine:
    """Pool sized from ``kv_cache_memory_mb`` (runtime.py:81-95), int8 weights
    (runtime.py:140-141), one VerifyRunner with ``max_num_seqs`` slots.  With
    ``speculative="draft"`` the draft model (``draft_config`` / ``draft_state_dict``, the
    weights ``draft_model_id`` names) gets its own paged pool with room for every slot's
    full length and a ``DraftModelProposer`` (runtime.py:116-129)."""
    problem = settings.hip_verify_path_error()
    if problem is not None:
        raise ValueError(f"the HIP verify path needs other settings: {problem}")
    device = torch.device(settings.device)
    dtype = TORCH_DTYPES[settings.dtype]
    budget = slots_for_budget(config.num_hidden_layers, config.num_key_value_heads, config.head_dim, dtype,
                              settings.kv_cache_memory_mb, settings.is_int8_kv_cache)
    num_blocks = budget // settings.kv_block_size
    if num_blocks * settings.kv_block_size < settings.max_model_len:
        raise ValueError(
            f"kv_cache_memory_mb={settings.kv_cache_memory_mb} holds fewer tokens than "
            f"max_model_len={settings.max_model_len}; raise the budget"
        )
    allocator_type = PrefixCachingSlotAllocator if settings.prefix_cache else PagedSlotAllocator  # runtime.py:93-94
    allocator = allocator_type(num_blocks, settings.kv_block_size, device)
    pool = KVCachePool(config.num_hidden_layers, config.num_key_value_heads, config.head_dim,
                       num_blocks * settings.kv_block_size, device, dtype, settings.is_int8_kv_cache,
                       settings.kv_block_size)
    weights = Qwen3Weights.from_state_dict(config, state_dict, device, dtype)
    max_seqs = settings.max_num_seqs if settings.is_batched else 1
    rows = max(max_seqs * (settings.num_speculative_tokens + 1), max_prefill_rows or settings.max_prefill_tokens)
    model = Qwen3VerifyModel(weights, rows, device)
    proposer = None
    if settings.speculative == "draft":
        if draft_config is None or draft_state_dict is None:
            raise ValueError("speculative='draft' needs the draft model's config and weights")
        if draft_config.vocab_size != config.vocab_size:
            raise ValueError("the draft model must share the target's vocabulary")
        tokens = settings.max_model_len + settings.num_speculative_tokens + 1
        draft_blocks = max_seqs * math.ceil(tokens / settings.kv_block_size)
        draft_pool = KVCachePool(draft_config.num_hidden_layers, draft_config.num_key_value_heads,
                                 draft_config.head_dim, draft_blocks * settings.kv_block_size, device, dtype,
                                 settings.is_int8_kv_cache, settings.kv_block_size)
        draft_weights = Qwen3Weights.from_state_dict(draft_config, draft_state_dict, device, dtype)
        draft_model = Qwen3VerifyModel(draft_weights, rows, device)
        draft_allocator = PagedSlotAllocator(draft_blocks, settings.kv_block_size, device)
        proposer = DraftModelProposer(draft_model, draft_pool, draft_allocator, max_seqs, tokens, device,
                                      k=settings.num_speculative_tokens, use_graph=settings.cuda_graphs)
    runner = VerifyRunner(model, pool, allocator, max_seqs, settings.num_speculative_tokens,
                          settings.ngram_max_size, settings.max_model_len, stop_token_ids,
                          use_graph=settings.cuda_graphs, proposer=proposer,
                          graph_max_batch=settings.cuda_graph_max_batch,
                          graph_max_context=settings.cuda_graph_max_context)
    if settings.cuda_graphs:
        runner.capture_graph()
    return VerifyEngine(settings, model, pool, allocator, runner, EngineMetrics())
