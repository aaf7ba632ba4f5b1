"""A8 / A8b: the W8A16 projection GEMMs and the bf16 LM head against the oracle.

W8A16 is checked against the reference's Int8Linear (ne/models/int8_quantization.py:55-57,
dequantise then F.linear) evaluated in fp32 on the CPU: relative error <= 2e-2.
The LM head is checked against an fp32 product: logits within 1e-2 max-abs at the
model's scale (hidden ~ N(0,1) * 0.02-scale norm weight, embedding ~ N(0, 0.02)),
relative error <= 2e-2, and its fused argmax partials reduce to exactly the argmax of
the kernel's own bf16 logits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import rel_err
from oracle.quant import int8_linear, quantize_linear
from nanoengine_amd import kernels
from nanoengine_amd._native import EPILOGUE_SWIGLU

pytestmark = pytest.mark.gpu

TOL = 2e-2
# (N, K) of q, k, v, o, gate, up, down in Qwen3-0.6B, plus the fused qkv and gate|up shapes
PROJECTIONS = [(2048, 1024), (1024, 1024), (1024, 1024), (1024, 2048), (3072, 1024), (3072, 1024),
               (1024, 3072), (4096, 1024)]


def make_weight(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    return quantize_linear(w)


@pytest.mark.parametrize("n,k", PROJECTIONS)
@pytest.mark.parametrize("m", [320, 37, 5])
def test_w8a16_matches_int8_linear(device, m, n, k):
    wq, ws = make_weight(n, k, seed=n + k)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
    ref = int8_linear(x.float(), wq, ws.float())
    ref_bf16 = int8_linear(x, wq, ws)  # the reference's own bf16 path
    out = kernels.w8a16_gemm(x.to(device), wq.to(device), ws.to(device))
    torch.cuda.synchronize()
    assert rel_err(out, ref) < TOL
    assert rel_err(out, ref_bf16) < TOL


@pytest.mark.parametrize("m,n,k,splits", [(320, 1024, 2048, 4), (320, 1024, 3072, 4), (37, 1024, 3072, 3),
                                          (5, 512, 1024, 2), (160, 1024, 1024, 1)])
def test_w8a16_splitk_partials(device, m, n, k, splits):
    """Summed split-K partials equal Int8Linear in fp32 (2e-2 relative), and each part is
    the product over its own K range."""
    wq, ws = make_weight(n, k, seed=7 * n + k)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m + k)).to(torch.bfloat16)
    parts = kernels.w8a16_gemm_splitk(x.to(device), wq.to(device), ws.to(device), splits)
    torch.cuda.synchronize()
    parts = parts.cpu()
    assert parts.shape == (splits, m, n)
    assert rel_err(parts.sum(0), int8_linear(x.float(), wq, ws.float())) < TOL
    kp = k // splits
    for s in range(splits):
        ref = int8_linear(x[:, s * kp:(s + 1) * kp].float(), wq[:, s * kp:(s + 1) * kp], ws.float())
        assert rel_err(parts[s], ref) < TOL


def test_splitk_choice_targets_one_work_group_per_cu():
    assert kernels.splitk_splits(320, 1024, 2048) == 2  # 7 x 16 tiles of 48 rows
    assert kernels.splitk_splits(320, 1024, 3072) == 2
    assert kernels.splitk_splits(64, 1024, 3072) == 4  # 2 x 16 tiles
    assert kernels.splitk_splits(320, 4096, 1024) == 1
    assert kernels.splitk_splits(4096, 1024, 3072) == 1
    assert kernels.splitk_splits(80, 1024, 384) == 3  # 3 parts of 128; 4 would not divide k


def test_w8a16_fp16_overflow_free(device):
    """int8_quantization.py:41-43: large activations must not overflow (scale is applied in fp32)."""
    wq, ws = make_weight(256, 1024, seed=3)
    x = (torch.randn(16, 1024) * 60).to(torch.bfloat16)
    out = kernels.w8a16_gemm(x.to(device), wq.to(device), ws.to(device))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert rel_err(out, int8_linear(x.float(), wq, ws.float())) < TOL


def pair_gate_up(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Interleave rows in groups of 32: 16 gate rows then the same 16 up rows."""
    n, k = gate.shape
    return torch.stack([gate.view(n // 16, 16, k), up.view(n // 16, 16, k)], dim=1).reshape(2 * n, k)


@pytest.mark.parametrize("m", [320, 21])
def test_swiglu_epilogue(device, m):
    gq, gs = make_weight(3072, 1024, seed=11)
    uq, us = make_weight(3072, 1024, seed=12)
    wq = pair_gate_up(gq, uq)
    ws = pair_gate_up(gs[:, None], us[:, None])[:, 0].contiguous()
    x = torch.randn(m, 1024).to(torch.bfloat16)
    gate = int8_linear(x.float(), gq, gs.float())
    up = int8_linear(x.float(), uq, us.float())
    ref = torch.nn.functional.silu(gate) * up
    out = kernels.w8a16_gemm(x.to(device), wq.to(device), ws.to(device), epilogue=EPILOGUE_SWIGLU)
    torch.cuda.synchronize()
    assert out.shape == (m, 3072)
    assert rel_err(out, ref) < TOL


@pytest.mark.parametrize("m,vocab", [(320, 151936), (5, 4096), (70, 8192), (400, 16512), (8, 180224)])
def test_lm_head_logits_and_argmax(device, m, vocab):
    g = torch.Generator().manual_seed(vocab + m)
    hidden = (torch.randn(m, 1024, generator=g) * 0.02).to(torch.bfloat16)
    embed = (torch.randn(vocab, 1024, generator=g) * 0.02).to(torch.bfloat16)
    ref = hidden.float() @ embed.float().T
    logits, partials = kernels.lm_head(hidden.to(device), embed.to(device), logits=True,
                                       argmax_partials=True)
    torch.cuda.synchronize()
    assert float((logits.float().cpu() - ref).abs().max()) < 1e-2
    assert rel_err(logits, ref) < TOL
    # partial argmax reduces to the first-index argmax of the kernel's own bf16 logits;
    # keys order as unsigned 64-bit integers (a set with no columns holds key 0)
    p = partials.cpu().numpy().view(np.uint64)
    best = torch.from_numpy((p.max(axis=1) & np.uint64(0xFFFFFFFF)).astype(np.int64))
    idx = 0xFFFFFFFF - best
    assert torch.equal(idx, torch.argmax(logits.float().cpu(), dim=1))
    # and equals the fp32 argmax wherever the top-2 margin exceeds the bf16 error
    top2 = torch.topk(ref, 2, dim=1).values
    clear = (top2[:, 0] - top2[:, 1]) > 2e-3
    assert torch.equal(idx[clear], torch.argmax(ref, dim=1)[clear])


def test_lm_head_argmax_ties_pick_the_first_column(device):
    """Exact ties: copies of a winning embedding row placed after it -- in the same lane,
    the next 16 columns, other blocks of the range and other work-groups' ranges -- must
    lose to the first copy (torch.argmax's first-index rule)."""
    vocab, m = 16512, 24
    g = torch.Generator().manual_seed(7)
    embed = (torch.randn(vocab, 1024, generator=g) * 0.02).to(torch.bfloat16)
    targets = torch.randint(0, vocab - 4096, (m,), generator=g)
    for j, t in enumerate(targets.tolist()):
        for off in (1, 2, 17, 64, 130, 256 + j, 700, 4000):
            embed[t + off] = embed[t]
    # a copy may land on another row's target: the winner is the first row equal to the
    # (final) target row, whose own logit 40 |e|^2 ~ 16 dwarfs any other row's (~N(0, 0.5))
    first = torch.tensor([int((embed == embed[t]).all(dim=1).nonzero().min()) for t in targets.tolist()])
    assert len(set(first.tolist())) > m // 2
    hidden = (embed[targets].float() * 40).to(torch.bfloat16)
    logits, partials = kernels.lm_head(hidden.to(device), embed.to(device), logits=True, argmax_partials=True)
    torch.cuda.synchronize()
    p = partials.cpu().numpy().view(np.uint64)
    idx = torch.from_numpy((0xFFFFFFFF - (p.max(axis=1) & np.uint64(0xFFFFFFFF))).astype(np.int64))
    assert torch.equal(idx, torch.argmax(logits.float().cpu(), dim=1))
    assert torch.equal(idx, first)


@pytest.mark.parametrize("m", [80, 64, 5, 1])
def test_lm_head_small_batch_kernel_equals_the_320_row_kernel(device, m):
    """At most 80 rows run their own LM-head kernel (each wave 32 columns x all rows, a
    three-stage ring); it sums every logit in the 320-row kernel's order, so its logits and
    argmax partials equal, bit for bit, those the 320-row kernel gives the same rows (81
    rows select that kernel).  Full vocabulary, short last blocks included."""
    vocab = 151936
    g = torch.Generator().manual_seed(500 + m)
    hidden = (torch.randn(81, 1024, generator=g) * 0.5).to(torch.bfloat16).to(device)
    embed = (torch.randn(vocab, 1024, generator=g) * 0.02).to(torch.bfloat16).to(device)
    big_logits, big_parts = kernels.lm_head(hidden, embed, logits=True, argmax_partials=True)
    logits, parts = kernels.lm_head(hidden[:m].contiguous(), embed, logits=True, argmax_partials=True)
    _, parts_only = kernels.lm_head(hidden[:m].contiguous(), embed, logits=False, argmax_partials=True)
    torch.cuda.synchronize()
    assert torch.equal(logits, big_logits[:m])
    assert torch.equal(parts, big_parts[:m]) and torch.equal(parts_only, parts)


def test_lm_head_argmax_only_matches_logits_path(device):
    hidden = (torch.randn(64, 1024) * 0.02).to(torch.bfloat16).to(device)
    embed = (torch.randn(8192, 1024) * 0.02).to(torch.bfloat16).to(device)
    logits, p1 = kernels.lm_head(hidden, embed, logits=True, argmax_partials=True)
    _, p2 = kernels.lm_head(hidden, embed, logits=False, argmax_partials=True)
    torch.cuda.synchronize()
    assert torch.equal(p1, p2)


@pytest.mark.parametrize("kv", ["int8-bf16-scales", "int8-fp16-scales", "bf16"])
@pytest.mark.parametrize("m", [320, 37, 1])
def test_fused_qkv_epilogue_equals_gemm_then_row_kernel(device, kv, m):
    """ne_w8a16_qkv_norm_rope_kv writes the same bits (q_out, cache codes, scales) as
    ne_w8a16_gemm followed by ne_qk_norm_rope_kv_write; the latter is checked against
    the oracle in test_rowwise_gpu.py and the GEMM above."""
    hq, hkv, k = 16, 8, 1024
    g = torch.Generator().manual_seed(1000 + m)
    wq, ws = make_weight((hq + 2 * hkv) * 128, k, seed=7)
    wq, ws = wq.to(device), ws.to(device)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(device)
    q_norm = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(device)
    k_norm = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(device)
    positions = torch.randint(0, 3000, (m,), generator=g, dtype=torch.int32).to(device)
    rope = kernels.rope_table(4096, 1e6).to(device)
    num_slots = 2048
    slots = torch.randperm(num_slots, generator=g)[:m].to(torch.int32).to(device)

    def pool():
        if kv == "bf16":
            return (torch.zeros(num_slots, hkv, 128, dtype=torch.bfloat16, device=device),
                    torch.zeros(num_slots, hkv, 128, dtype=torch.bfloat16, device=device), None, None)
        sdt = torch.bfloat16 if kv == "int8-bf16-scales" else torch.float16
        return (torch.zeros(num_slots, hkv, 128, dtype=torch.int8, device=device),
                torch.zeros(num_slots, hkv, 128, dtype=torch.int8, device=device),
                torch.zeros(num_slots, hkv, dtype=sdt, device=device),
                torch.zeros(num_slots, hkv, dtype=sdt, device=device))

    a, b = pool(), pool()
    qkv = kernels.w8a16_gemm(x, wq, ws)
    q_ref = kernels.qk_norm_rope_kv_write(qkv, hq, hkv, q_norm, k_norm, 1e-6, positions, rope, slots, *a)
    q_out = torch.empty(m, hq, 128, dtype=torch.bfloat16, device=device)
    assert kernels.qkv_fusion_supported(b[0], b[2])
    kernels.w8a16_qkv_norm_rope_kv(x, wq, ws, hq, hkv, q_norm, k_norm, 1e-6, positions, rope, slots, *b,
                                   q_out=q_out)
    torch.cuda.synchronize()
    assert torch.equal(q_out.view(torch.int16), q_ref.view(torch.int16))
    for ta, tb in zip(a, b):
        if ta is not None:
            assert torch.equal(ta.view(torch.uint8), tb.view(torch.uint8))
    assert int(a[0].view(torch.uint8).ne(0).sum()) > 0  # something was written
