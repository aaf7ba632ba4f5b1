"""RMSNorm variants, fused QK-norm + RoPE + KV write, and the A7 KV write/quantise,
against the oracle's restatement of ne/models/qwen3.py:31-115 and
ne/models/int8_quantization.py:30-34.

The standalone int8 KV write must be bit-exact (codes and scales) against
quantize_vectors.  Norm/RoPE outputs are bf16 and compared within 2e-2 relative
(a summation-order difference can move a bf16 result by one ulp).
"""

from __future__ import annotations

import pytest
import torch

from helpers import rel_err
from oracle.model import RMSNorm, apply_rotary_embedding, build_rotary_tables
from oracle.quant import quantize_vectors
from nanoengine_amd import kernels

pytestmark = pytest.mark.gpu

TOL = 2e-2
EPS = 1e-6


def oracle_norm(x, w):
    norm = RMSNorm(x.shape[-1], EPS)
    norm.weight.data = w.clone()
    return norm.to(torch.bfloat16)(x)


def test_rmsnorm(device):
    x = torch.randn(37, 1024).to(torch.bfloat16)
    w = (torch.randn(1024) * 0.02).to(torch.bfloat16)
    out = kernels.rmsnorm(x.to(device), w.to(device), EPS)
    torch.cuda.synchronize()
    assert rel_err(out, oracle_norm(x, w)) < TOL


def test_add_rmsnorm_updates_residual(device):
    r = torch.randn(320, 1024).to(torch.bfloat16)
    dlt = torch.randn(320, 1024).to(torch.bfloat16)
    w = torch.randn(1024).to(torch.bfloat16)
    rd = r.to(device)
    out = kernels.add_rmsnorm(rd, dlt.to(device), w.to(device), EPS)
    torch.cuda.synchronize()
    new_r = r + dlt  # bf16 add, as the reference's residual connection
    assert torch.equal(rd.cpu(), new_r)
    assert rel_err(out, oracle_norm(new_r, w)) < TOL


@pytest.mark.parametrize("splits", [1, 3, 4])
def test_splitk_add_rmsnorm_equals_add_of_summed_partials(device, splits):
    """delta = bf16(p[0] + p[1] + ... in order, fp32), then exactly ne_add_rmsnorm."""
    rows, hidden = 37, 1024
    parts = torch.randn(splits, rows, hidden) * 0.5
    r = torch.randn(rows, hidden).to(torch.bfloat16)
    w = torch.randn(hidden).to(torch.bfloat16)
    acc = parts[0].numpy().copy()
    for s in range(1, splits):
        acc += parts[s].numpy()  # numpy fp32, sequential: the kernel's order
    delta = torch.from_numpy(acc).to(torch.bfloat16)
    r1, r2 = r.to(device), r.to(device)
    want = kernels.add_rmsnorm(r1, delta.to(device), w.to(device), EPS)
    got = kernels.splitk_add_rmsnorm(r2, parts.to(device), splits, w.to(device), EPS)
    torch.cuda.synchronize()
    assert torch.equal(r2.cpu(), r1.cpu())
    assert torch.equal(got.cpu(), want.cpu())
    assert torch.equal(r2.cpu(), r + delta)


def test_embed_rmsnorm(device):
    emb = (torch.randn(5000, 1024) * 0.02).to(torch.bfloat16)
    w = (torch.randn(1024) * 0.02).to(torch.bfloat16)
    tok = torch.randint(0, 5000, (64,), dtype=torch.int32)
    res, out = kernels.embed_rmsnorm(tok.to(device), emb.to(device), w.to(device), EPS)
    torch.cuda.synchronize()
    assert torch.equal(res.cpu(), emb[tok.long()])
    assert rel_err(out, oracle_norm(emb[tok.long()], w)) < TOL


@pytest.mark.parametrize("vec_dtype", [torch.bfloat16, torch.float16])
def test_kv_write_int8_bit_exact(device, vec_dtype):
    n, heads = 40, 8
    vectors = (torch.randn(n, heads, 128) * torch.rand(n, heads, 1) * 4).to(vec_dtype)
    vectors[3, 2] = 0  # all-zero vector: scale clamps to 1e-8 / 127
    # exact rounding ties: max 127 / 8 gives scale 1 / 8, so x / s = k + 0.5 (rint: to even)
    ties = (torch.arange(128) % 64 - 32 + 0.5) / 8
    ties[0] = 127 / 8
    vectors[5, 1] = ties.to(vec_dtype)
    vectors[6, 4] = (-ties).to(vec_dtype)
    # quotients near k + 0.5 for a scale that is not a power of two
    near = ((torch.arange(128) % 100) - 50 + 0.5) * (3.7 / 127)
    near[0] = 3.7
    vectors[7, 0] = near.to(vec_dtype)
    slots = torch.randperm(100)[:n].to(torch.int32)
    cache = torch.zeros(101, heads, 128, dtype=torch.int8, device=device)
    scales = torch.zeros(101, heads, dtype=vec_dtype, device=device)
    kernels.kv_write(vectors.to(device), slots.to(device), cache, scales)
    torch.cuda.synchronize()
    q, s = quantize_vectors(vectors)
    assert torch.equal(cache.cpu()[slots.long()], q)
    assert torch.equal(scales.cpu()[slots.long()], s[..., 0])


def test_kv_write_bf16_scatter(device):
    vectors = torch.randn(10, 8, 128).to(torch.bfloat16)
    slots = torch.tensor([5, 1, 9, 0, 3, 7, 2, 8, 6, 4], dtype=torch.int32)
    cache = torch.zeros(11, 8, 128, dtype=torch.bfloat16, device=device)
    kernels.kv_write(vectors.to(device), slots.to(device), cache, None)
    torch.cuda.synchronize()
    assert torch.equal(cache.cpu()[slots.long()], vectors)


@pytest.mark.parametrize("kv_dtype", ["int8", "bf16"])
def test_qk_norm_rope_kv_write(device, kv_dtype):
    rows, hq, hkv = 45, 16, 8
    qkv = torch.randn(rows, (hq + 2 * hkv) * 128).to(torch.bfloat16)
    qn = (torch.randn(128) * 0.5 + 1).to(torch.bfloat16)
    kn = (torch.randn(128) * 0.5 + 1).to(torch.bfloat16)
    positions = torch.randint(0, 17000, (rows,), dtype=torch.int32)
    slots = torch.randperm(200)[:rows].to(torch.int32)
    rope = kernels.rope_table(17000, 1e6)
    is_int8 = kv_dtype == "int8"
    cdt = torch.int8 if is_int8 else torch.bfloat16
    kc = torch.zeros(201, hkv, 128, dtype=cdt, device=device)
    vc = torch.zeros(201, hkv, 128, dtype=cdt, device=device)
    ks = torch.zeros(201, hkv, dtype=torch.bfloat16, device=device) if is_int8 else None
    vs = torch.zeros(201, hkv, dtype=torch.bfloat16, device=device) if is_int8 else None
    q_out = kernels.qk_norm_rope_kv_write(
        qkv.to(device), hq, hkv, qn.to(device), kn.to(device), EPS, positions.to(device),
        rope.to(device), slots.to(device), kc, vc, ks, vs)
    torch.cuda.synchronize()
    # oracle: q_norm / k_norm then RoPE in bf16 (qwen3.py:100-104)
    q = qkv[:, : hq * 128].view(1, rows, hq, 128)
    k = qkv[:, hq * 128 : (hq + hkv) * 128].view(1, rows, hkv, 128)
    v = qkv[:, (hq + hkv) * 128 :].view(rows, hkv, 128)
    cos, sin = build_rotary_tables(positions.long()[None], 128, 1e6, torch.bfloat16)
    q_ref = apply_rotary_embedding(oracle_norm(q, qn).transpose(1, 2), cos, sin).transpose(1, 2)[0]
    k_ref = apply_rotary_embedding(oracle_norm(k, kn).transpose(1, 2), cos, sin).transpose(1, 2)[0]
    assert rel_err(q_out, q_ref) < TOL
    sl = slots.long()
    if is_int8:
        k_deq = kc.cpu()[sl].float() * ks.cpu()[sl].float()[..., None]
        v_deq = vc.cpu()[sl].float() * vs.cpu()[sl].float()[..., None]
        assert rel_err(k_deq, k_ref) < TOL
        assert rel_err(v_deq, v) < TOL
        vq, vsc = quantize_vectors(v)  # values are not transformed: codes are exact
        assert torch.equal(vc.cpu()[sl], vq)
        assert torch.equal(vs.cpu()[sl], vsc[..., 0])
    else:
        assert rel_err(kc.cpu()[sl], k_ref) < TOL
        assert torch.equal(vc.cpu()[sl], v)
