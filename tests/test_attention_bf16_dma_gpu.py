"""A6 with a bf16 pool on the DMA-fed kernel (two-tile LDS rings, bf16 MFMA scores) against
the oracle (fp32 gather + masked softmax, ne/models/attention_context.py:57-109).

Covered: the bf16 kernel-only configuration (16 sequences, context U{256..2048} seed 1,
5 queries) through the per-step plan and the planned call, which split sequences and
merge partials; whole-sequence items served by 4 or 2 work-groups (4 or 2 waves per KV
head merged in LDS); two row tiles per KV head (k = 8); and a pool whose every slot
outside the contexts holds NaN, where the tails of partial tiles must not reach the
output.  Bar: relative error <= 2e-2 on the rows of real queries, no error flag.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import make_batch, make_pool, real_rows, rel_err
from oracle.attention import paged_attention_reference
from nanoengine_amd import kernels

pytestmark = pytest.mark.gpu

TOL = 2e-2
HQ, HKV = 16, 8


def _run(device, ctx, q_lens, num_blocks=None, pool=None, seed=0):
    num_blocks = num_blocks or sum((c + 15) // 16 for c in ctx) + 8
    kc, vc, _, _ = pool if pool is not None else make_pool(num_blocks, 16, HKV, "bf16", seed=seed)
    tables, ctx_t, qs, ql, rows = make_batch(ctx, q_lens, num_blocks, 16, seed=seed + 1)
    q = torch.randn(rows, HQ, 128, generator=torch.Generator().manual_seed(seed + 2)).to(torch.bfloat16)
    d = lambda t: t.to(device)
    tables_d, ctx_d, qs_d, ql_d = d(tables), d(ctx_t), d(qs), d(ql)
    args = (d(q), d(kc), d(vc), None, None, tables_d, 16, ctx_d, qs_d, ql_d)
    assert kernels.plan_supported(HQ, HKV, max(q_lens), len(ctx), torch.bfloat16, None)
    ws = kernels.AttentionWorkspace()
    unplanned = kernels.paged_verify_attention(*args, max_q_len=max(q_lens), max_ctx_len=max(ctx), workspace=ws)
    torch.cuda.synchronize()
    assert ws.error_flag() == 0
    kernels.paged_attention_plan(tables_d, 16, ctx_d, qs_d, ql_d, HQ, HKV, max(q_lens), max(ctx), ws)
    planned = kernels.paged_verify_attention(*args, max_q_len=max(q_lens), max_ctx_len=max(ctx), workspace=ws,
                                             planned=True)
    torch.cuda.synchronize()
    assert ws.error_flag() == 0
    idx = real_rows(qs, ql)
    ref = paged_attention_reference(q, kc, vc, None, None, tables, 16, ctx_t, qs, ql, model_dtype=torch.bfloat16)
    return unplanned.cpu()[idx], planned.cpu()[idx], ref[idx]


def test_bf16_16_seqs_ctx_256_to_2048_plan_and_planned(device):
    """16 sequences, context U{256..2048} (seed 1), 5 queries, 4096-block pool: split items
    and the partial merge, planned and unplanned (the same items, the same bits)."""
    ctx = np.random.default_rng(1).integers(256, 2049, size=16).tolist()
    unplanned, planned, ref = _run(device, ctx, [5] * 16, num_blocks=4096)
    assert rel_err(planned, ref) < TOL
    assert torch.equal(planned, unplanned)


@pytest.mark.parametrize("num_seqs,max_ctx", [(64, 256), (100, 1024), (64, 1024)])
def test_whole_sequence_items(device, num_seqs, max_ctx):
    """Contexts of at most 1024 keys: one item per sequence over 4 (64 sequences) or 2 (100)
    work-groups; contexts of 1..17 keys leave some waves without tiles."""
    rng = np.random.default_rng(num_seqs + max_ctx)
    ctx = [int(c) for c in rng.integers(1, max_ctx + 1, size=num_seqs)]
    ctx[:6] = [1, 2, 15, 16, 17, max_ctx]
    q_lens = [int(min(c, 5)) for c in ctx]
    unplanned, planned, ref = _run(device, ctx, q_lens, seed=5)
    assert rel_err(planned, ref) < TOL
    assert rel_err(unplanned, ref) < TOL


def test_k8_two_row_tiles(device):
    ctx = [300, 1500, 2100, 40, 9]
    unplanned, planned, ref = _run(device, ctx, [9, 9, 7, 9, 9], seed=9)
    assert rel_err(planned, ref) < TOL
    assert torch.equal(planned, unplanned)


def test_nan_outside_the_contexts_stays_out(device):
    """Every slot no context covers holds NaN: the keys past a context's end inside its last
    tile, and the tiles a split re-reads past its end, must contribute nothing."""
    ctx = [17, 33, 250, 1000, 513, 7]
    q_lens = [5, 5, 5, 5, 5, 5]
    num_blocks = sum((c + 15) // 16 for c in ctx) + 8
    kc, vc, _, _ = make_pool(num_blocks, 16, HKV, "bf16", seed=3)
    tables, ctx_t, _, _, _ = make_batch(ctx, q_lens, num_blocks, 16, seed=4)
    covered = torch.zeros(kc.shape[0], dtype=torch.bool)
    for b, c in enumerate(ctx):
        pos = torch.arange(c)
        covered[tables[b, pos // 16].long() * 16 + pos % 16] = True
    kc[~covered] = float("nan")
    vc[~covered] = float("nan")
    unplanned, planned, ref = _run(device, ctx, q_lens, num_blocks=num_blocks, pool=(kc, vc, None, None), seed=3)
    assert torch.isfinite(ref).all()
    assert torch.isfinite(planned).all() and torch.isfinite(unplanned).all()
    assert rel_err(planned, ref) < TOL
    assert rel_err(unplanned, ref) < TOL


@pytest.mark.parametrize("kv_dtype", ["int8", "bf16"])
def test_kv_stream_follows_the_plan(device, kv_dtype):
    """The measurement entry point (the planned call's K/V reads alone) runs on the same plan
    for both cache dtypes, whole-sequence and split items, without raising the flag."""
    for ctx in (np.random.default_rng(1).integers(128, 1025, size=64).tolist(),
                np.random.default_rng(1).integers(256, 2049, size=16).tolist()):
        num_blocks = sum((c + 15) // 16 for c in ctx) + 8
        kc, vc, ks, vs = make_pool(num_blocks, 16, HKV, kv_dtype, torch.float16, seed=1)
        tables, ctx_t, qs, ql, _ = make_batch(ctx, [5] * len(ctx), num_blocks, 16, seed=2)
        d = lambda t: None if t is None else t.to(device)
        ws = kernels.AttentionWorkspace()
        kernels.paged_attention_plan(d(tables), 16, d(ctx_t), d(qs), d(ql), HQ, HKV, 5, max(ctx), ws)
        kernels.paged_kv_stream_planned(d(kc), d(vc), d(ks), d(vs), len(ctx), HQ, 5, max(ctx), ws)
        torch.cuda.synchronize()
        assert ws.error_flag() == 0


def _runs_in_workspace(ws, grid):
    """The runs' items [grid][8] and slot lists [grid][512] (int32): the workspace's last two
    regions, each starting on a 256-byte boundary, the slot lists last."""
    slots_bytes = grid * 512 * 4
    items_bytes = -(-grid * 8 * 4 // 256) * 256
    buf = ws.buffer.cpu()
    slots = buf[buf.numel() - slots_bytes:].view(torch.int32).view(grid, 512)
    items = buf[buf.numel() - slots_bytes - items_bytes:][: grid * 32].view(torch.int32).view(grid, 8)
    return items, slots


@pytest.mark.parametrize("kv_dtype", ["int8", "bf16"])
@pytest.mark.parametrize("case", ["64_seqs_with_empty_ones", "4_short_seqs"])
def test_kv_stream_runs_cover_every_tile_once_in_order(device, kv_dtype, case):
    """The whole-slot runs (measurement entry points): the sequences' 16-key tiles in order,
    cut into the plan grid's near-equal runs across sequence boundaries, empty sequences
    (inside the order and at its end) and empty runs included; the stream over them leaves
    no error flag, and a planned call afterwards is refused until the plan is written again."""
    from nanoengine_amd import _native

    if case == "64_seqs_with_empty_ones":
        ctx = np.random.default_rng(5).integers(1, 1025, size=64).tolist()
        ctx[3] = ctx[40] = ctx[63] = 0
    else:
        ctx = [17, 0, 5, 40]
    num_blocks = sum((c + 15) // 16 for c in ctx) + 8
    kc, vc, ks, vs = make_pool(num_blocks, 16, HKV, kv_dtype, torch.float16, seed=3)
    tables, ctx_t, qs, ql, _ = make_batch(ctx, [5] * len(ctx), num_blocks, 16, seed=4)
    d = lambda t: None if t is None else t.to(device)
    ws = kernels.AttentionWorkspace()
    kernels.paged_kv_runs_plan(d(tables), 16, d(ctx_t), HQ, HKV, 5, max(ctx), ws)
    torch.cuda.synchronize()
    assert ws.error_flag() == 0
    assert ws.buffer.numel() == _native.load().ne_paged_attention_workspace_size(len(ctx), HQ, HKV, 5, max(ctx), 0)
    grid = 256  # max(256, 2 B, B + ceil(B * max_tiles / 512)) at these shapes
    items, slots = _runs_in_workspace(ws, grid)
    expected = [int(tables[b, j]) * 16 for b, c in enumerate(ctx) for j in range((c + 15) // 16)]
    T = len(expected)
    sizes = [T * (w + 1) // grid - T * w // grid for w in range(grid)]
    assert items[:, 7].tolist() == sizes
    assert items[:, 3].tolist() == [0] * grid
    assert items[:, 0].tolist() == [0 if n > 0 else -1 for n in sizes]
    got = [int(x) for w in range(grid) for x in slots[w, : sizes[w]]]
    assert got == expected
    kernels.paged_kv_stream_runs(d(kc), d(vc), d(ks), d(vs), len(ctx), HQ, 5, max(ctx), ws)
    torch.cuda.synchronize()
    assert ws.error_flag() == 0
    q = torch.zeros(5 * len(ctx), HQ, 128, dtype=torch.bfloat16, device=device)
    args = (q, d(kc), d(vc), d(ks), d(vs), d(tables), 16, d(ctx_t), d(qs), d(ql))
    with pytest.raises(ValueError, match="paged_attention_plan"):
        kernels.paged_verify_attention(*args, max_q_len=5, max_ctx_len=max(ctx), workspace=ws, planned=True)
