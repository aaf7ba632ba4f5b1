"""Host side of the reference seams (no GPU): the padded step inputs equal the oracle's
``build_step_inputs`` (ne/engine/generation/batch_builder.py:22-65) field by field, the
block tables handed to the kernels give back the context slots, weight quantisation of
``Int8Linear.from_linear`` equals the oracle's, and the HIP-only entry points refuse what
they cannot run instead of computing it some other way."""

from __future__ import annotations

import math

import pytest
import torch

from oracle import paging as op
from oracle.quant import quantize_vectors as oracle_quantize
from nanoengine_amd.attention_context import AttentionContext, run_cached_attention
from nanoengine_amd.int8_quantization import Int8Linear
from nanoengine_amd.interface import GenerationRequest, SamplingParams
from nanoengine_amd.memory import KVCachePool, PagedSlotAllocator
from nanoengine_amd.model_runner import build_step_inputs
from nanoengine_amd.sequence_state import Sequence


def _sequence(rid: str, tokens: list[int]) -> Sequence:
    return Sequence.from_request(GenerationRequest(rid, tokens, SamplingParams(max_new_tokens=8)))


@pytest.mark.parametrize("cached,counts", [([37, 130, 16], [5, 3, 1]), ([0, 0], [64, 17]), ([15], [1])])
def test_step_inputs_equal_oracle(cached, counts):
    g = torch.Generator().manual_seed(sum(cached) + sum(counts))
    dev = torch.device("cpu")
    pool = KVCachePool(1, 8, 128, 64 * 16, dev, torch.bfloat16, True, 16)
    ours = PagedSlotAllocator(64, 16, dev)
    theirs = op.PagedSlotAllocator(64, 16)
    seqs = [_sequence(f"s{i}", torch.randint(0, 4096, (c + n,), generator=g).tolist())
            for i, (c, n) in enumerate(zip(cached, counts))]
    for s, c, n in zip(seqs, cached, counts):
        ours.reserve(s, c + n)
        theirs.reserve(s.request_id, c + n)
        s.num_cached_tokens = c
    got = build_step_inputs(seqs, ours, pool, dev, counts)
    want = op.build_step_inputs([s.token_ids for s in seqs], cached, counts,
                                lambda c: theirs.build_context_slots([s.request_id for s in seqs], c),
                                pool.scratch_slot)
    assert torch.equal(got.token_ids, want.token_ids)
    assert torch.equal(got.context.positions, want.positions)
    assert torch.equal(got.context.slot_mapping, want.slot_mapping)
    assert torch.equal(got.context.context_slots, want.context_slots)
    assert torch.equal(got.context.attention_mask, want.attention_mask)
    assert torch.equal(got.last_token_indices, want.last_token_indices)
    # the kernels' block tables address exactly the context slots
    ctx = got.context
    assert ctx.query_lengths.tolist() == counts
    assert ctx.context_lengths.tolist() == [c + n for c, n in zip(cached, counts)]
    for i, end in enumerate(ctx.context_lengths.tolist()):
        pos = torch.arange(end)
        slots = ctx.block_tables[i].long()[pos // ctx.block_size] * ctx.block_size + pos % ctx.block_size
        assert torch.equal(slots, want.context_slots[i, :end])
    assert ctx.block_tables.shape[1] == math.ceil(max(ctx.context_lengths.tolist()) / 16)


def test_int8_linear_codes_and_refusals():
    g = torch.Generator().manual_seed(3)
    linear = torch.nn.Linear(256, 128, bias=False)
    with torch.no_grad():
        linear.weight.copy_(torch.randn(128, 256, generator=g))
    layer = Int8Linear.from_linear(linear.to(torch.bfloat16))
    codes, scales = oracle_quantize(linear.weight.detach())
    assert torch.equal(layer.weight_int8, codes) and torch.equal(layer.weight_scale, scales.squeeze(-1))
    with pytest.raises(RuntimeError, match="GPU"):
        layer(torch.zeros(4, 256, dtype=torch.bfloat16))


def test_cached_attention_needs_kernel_metadata():
    t = torch.zeros(1, 1)
    ctx = AttentionContext(t, t, t, t, [t], [t])
    with pytest.raises(ValueError, match="build_step_inputs"):
        run_cached_attention(torch.zeros(1, 16, 1, 128), torch.zeros(1, 8, 1, 128), torch.zeros(1, 8, 1, 128),
                             ctx, 0)
