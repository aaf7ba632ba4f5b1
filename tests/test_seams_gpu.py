"""The reference's Python seams on the HIP kernels, each against the oracle's restatement:

  * ``Int8Linear`` (ne/models/int8_quantization.py:37-57): codes and scales of
    ``from_linear`` bit-exact with ``quantize_vectors``; ``forward`` within 2e-2
    relative error of the fp32 product (and of the reference's bf16 layer);
  * ``run_cached_attention`` (ne/models/attention_context.py:66-109) on a padded batch
    built by ``build_step_inputs``: the cache bytes written for the step bit-exact with
    the oracle's ``write_to_cache``, real rows within 2e-2 relative error of the oracle's
    masked SDPA, padding rows zero; int8 and bf16 pools;
  * ``ModelRunner.score_tokens`` / ``run_step`` (ne/engine/generation/model_runner.py:33-62):
    logits after each guess within 1e-2 max-abs and 2e-2 relative error of the oracle's
    runner (2 layers of Qwen3-0.6B's shape, vocabulary 4096), greedy tokens equal where
    the oracle's top-2 margin is clear.
"""

from __future__ import annotations

import pytest
import torch

from oracle import model as om
from oracle.attention import run_cached_attention as oracle_attention
from oracle.paging import PagedSlotAllocator as OraclePaged
from oracle.quant import int8_linear, quantize_vectors as oracle_quantize
from oracle.verify import ModelRunner as OracleRunner
from oracle.verify import Sequence as OracleSequence
from nanoengine_amd.attention_context import run_cached_attention
from nanoengine_amd.int8_quantization import Int8Linear
from nanoengine_amd.interface import GenerationRequest, SamplingParams
from nanoengine_amd.memory import KVCachePool, PagedSlotAllocator
from nanoengine_amd.model_runner import ModelRunner, build_step_inputs
from nanoengine_amd.qwen3 import Qwen3Config, Qwen3VerifyModel, Qwen3Weights, random_state_dict
from nanoengine_amd.sequence_state import Sequence

pytestmark = pytest.mark.gpu

CFG = Qwen3Config(4096, 1024, 3072, 2, 16, 8, 128, 1e-6, 1e6, True)
OCFG = om.Qwen3Config(4096, 1024, 3072, 2, 16, 8, 128, 1e-6, 1e6, True)


def rel(got: torch.Tensor, ref: torch.Tensor) -> float:
    return float((got.float() - ref.float()).norm() / ref.float().norm())


@pytest.mark.parametrize("n,k,lead", [(1024, 1024, (37,)), (3072, 1024, (5, 3)), (1024, 3072, (320,))])
def test_int8_linear_matches_reference_layer(n, k, lead):
    g = torch.Generator().manual_seed(n + k)
    linear = torch.nn.Linear(k, n, bias=False)
    with torch.no_grad():
        linear.weight.copy_(torch.randn(n, k, generator=g) * 0.02)
    linear = linear.to(torch.bfloat16)
    x = torch.randn(*lead, k, generator=g).to(torch.bfloat16)
    codes, scales = oracle_quantize(linear.weight.detach().clone())
    layer = Int8Linear.from_linear(linear.cuda())
    assert torch.equal(layer.weight_int8.cpu(), codes)
    assert torch.equal(layer.weight_scale.cpu(), scales.squeeze(-1))
    y = layer(x.cuda())
    torch.cuda.synchronize()
    assert y.shape == (*lead, n) and y.dtype == torch.bfloat16
    ref = int8_linear(x.float(), codes, scales.squeeze(-1).float())
    assert rel(y.cpu(), ref) <= 2e-2
    ref_bf16 = om.Int8Linear(codes, scales.squeeze(-1))(x)
    assert rel(y.cpu(), ref_bf16) <= 2e-2


def _sequence(rid: str, tokens: list[int]) -> Sequence:
    return Sequence.from_request(GenerationRequest(rid, tokens, SamplingParams(max_new_tokens=64)))


@pytest.mark.parametrize("int8", [True, False], ids=["int8-pool", "bf16-pool"])
def test_run_cached_attention_matches_oracle(int8):
    g = torch.Generator().manual_seed(7)
    dev = torch.device("cuda")
    layers, kvh, hq, d = 2, 8, 16, 128
    pool = KVCachePool(layers, kvh, d, 64 * 16, dev, torch.bfloat16, int8, 16)
    alloc = PagedSlotAllocator(64, 16, dev)
    # three sequences with cached contexts of 37, 130 and 16 tokens and 5, 3 and 1 new ones
    cached, new = [37, 130, 16], [5, 3, 1]
    seqs = [_sequence(f"s{i}", torch.randint(0, 4096, (c + n,), generator=g).tolist())
            for i, (c, n) in enumerate(zip(cached, new))]
    for s, c, n in zip(seqs, cached, new):
        alloc.reserve(s, c + n)
        s.num_cached_tokens = c
    # earlier keys / values already in the pool
    for layer in range(layers):
        for cache, scales in ((pool.key_caches[layer], pool.key_scales), (pool.value_caches[layer], pool.value_scales)):
            vec = torch.randn(cache.shape[0], kvh, d, generator=g).to(torch.bfloat16)
            if int8:
                codes, sc = oracle_quantize(vec)
                cache.copy_(codes.to(dev))
                scales[layer].copy_(sc.to(dev))
            else:
                cache.copy_(vec.to(dev))
    inputs = build_step_inputs(seqs, alloc, pool, dev, new)
    ctx = inputs.context
    b, q = inputs.token_ids.shape
    queries = torch.randn(b, hq, q, d, generator=g).to(torch.bfloat16)
    keys = torch.randn(b, kvh, q, d, generator=g).to(torch.bfloat16)
    values = torch.randn(b, kvh, q, d, generator=g).to(torch.bfloat16)
    layer = 1
    ref_k = pool.key_caches[layer].cpu().clone()
    ref_v = pool.value_caches[layer].cpu().clone()
    ref_ks = pool.key_scales[layer].cpu().clone() if int8 else None
    ref_vs = pool.value_scales[layer].cpu().clone() if int8 else None
    out = run_cached_attention(queries.cuda(), keys.cuda(), values.cuda(), ctx, layer)
    torch.cuda.synchronize()
    ref = oracle_attention(queries, keys, values, ctx.positions.cpu(), ctx.slot_mapping.cpu(),
                           ctx.context_slots.cpu(), ctx.attention_mask.cpu(), ref_k, ref_v, ref_ks, ref_vs)
    # the step's keys / values land in the same bytes; every padding row writes the scratch
    # slot (the last), whose final contents depend on write order on both sides
    real = slice(0, pool.scratch_slot)
    assert torch.equal(pool.key_caches[layer].cpu()[real], ref_k[real])
    assert torch.equal(pool.value_caches[layer].cpu()[real], ref_v[real])
    if int8:
        assert torch.equal(pool.key_scales[layer].cpu()[real], ref_ks[real])
        assert torch.equal(pool.value_scales[layer].cpu()[real], ref_vs[real])
    out = out.cpu()
    for i, n in enumerate(new):
        assert rel(out[i, :, :n], ref[i, :, :n]) <= 2e-2, f"sequence {i}"
        assert float(out[i, :, n:].abs().max() if n < q else 0.0) == 0.0


def _build(state):
    dev = torch.device("cuda")
    weights = Qwen3Weights.from_state_dict(CFG, state, dev, torch.bfloat16)
    model = Qwen3VerifyModel(weights, 160, dev)
    pool = KVCachePool(CFG.num_hidden_layers, CFG.num_key_value_heads, CFG.head_dim, 64 * 16, dev,
                       torch.bfloat16, True, 16)
    return ModelRunner(model, pool, PagedSlotAllocator(64, 16, dev), dev)


def _oracle(state):
    model = om.Qwen3ForCausalLM(OCFG)
    model.load_state_dict(state)
    model = model.to(torch.bfloat16).eval()
    om.quantize_linear_layers(model)
    pool = om.KVCachePool(OCFG, 64 * 16, torch.bfloat16, is_int8=True)
    return OracleRunner(model, pool, OraclePaged(64, 16))


def test_score_tokens_and_run_step_match_oracle():
    state = random_state_dict(CFG, seed=0, std=0.02)
    for name in state:  # O(1) activations, the sharper test of relative accuracy
        if name.endswith("norm.weight") or "layernorm" in name:
            state[name] = torch.ones_like(state[name])
    runner, oracle = _build(state), _oracle(state)
    g = torch.Generator().manual_seed(11)
    prompts = [torch.randint(0, 4096, (n,), generator=g).tolist() for n in (40, 64, 17)]
    seqs = [_sequence(f"r{i}", p) for i, p in enumerate(prompts)]
    oseqs = [OracleSequence(f"o{i}", list(p), len(p), 64) for i, p in enumerate(prompts)]
    for s, o in zip(seqs, oseqs):
        runner.allocator.reserve(s, s.num_tokens)
        oracle.allocator.reserve(o.request_id, len(o.token_ids))
    # one padded prefill step of all three prompts
    ours = runner.run_step(seqs)
    theirs = oracle.run_step(oseqs)
    assert [s.num_cached_tokens for s in seqs] == [len(p) for p in prompts]
    # then five guesses each, scored one sequence at a time
    for s, o, tok, otok in zip(seqs, oseqs, ours, theirs):
        guesses = torch.randint(0, 4096, (4,), generator=g).tolist()
        s.token_ids += [otok] + guesses
        o.token_ids += [otok] + guesses
        runner.allocator.reserve(s, s.num_tokens)
        oracle.allocator.reserve(o.request_id, len(o.token_ids))
        got = runner.score_tokens(s, 5).float().cpu()
        ref = oracle.score_tokens(o, 5).float()
        scale = float(ref.abs().max())
        assert float((got - ref).abs().max()) <= max(1e-2, 2e-2 * scale)
        assert rel(got, ref) <= 2e-2
        assert s.num_cached_tokens == o.num_cached_tokens == s.num_tokens
    # greedy picks of the prefill step agree wherever the oracle's choice is clear
    ref_model = oracle.model
    for p, tok, otok in zip(prompts, ours, theirs):
        with torch.no_grad():
            logits = ref_model.compute_logits(ref_model(torch.tensor([p]))[0, -1:]).float()[0]
        top2 = torch.topk(logits, 2).values
        if float(top2[0] - top2[1]) > 2e-2 * float(logits.abs().max()):
            assert tok == otok
