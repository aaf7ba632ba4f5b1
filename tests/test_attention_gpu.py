"""A6: the HIP paged verify attention against the oracle (fp32 restatement of the reference's
gather + dequant + masked SDPA, ne/models/attention_context.py:57-109).

Bar: relative error <= 2e-2 (bf16), checked on the rows of real queries.  Shapes
follow the kernel-only attention configurations: 16 Q / 8 KV heads, head_dim 128,
16-token blocks drawn from a seeded permutation of a 4096-block pool, 5 query
tokens per sequence with causal masking among them.
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


def run_case(device, ctx_lens, q_lens, kv_dtype, scale_dtype=torch.bfloat16, block_size=16,
             num_blocks=None, split_len=0, padded_q=None, seed=0):
    num_blocks = num_blocks or max(64, sum((c + block_size - 1) // block_size for c in ctx_lens) + 8)
    kc, vc, ks, vs = make_pool(num_blocks, block_size, HKV, kv_dtype, scale_dtype, seed=seed)
    tables, ctx, qs, ql, rows = make_batch(ctx_lens, q_lens, num_blocks, block_size, seed=seed + 1,
                                           padded_q=padded_q)
    g = torch.Generator().manual_seed(seed + 2)
    q = torch.randn(rows, HQ, 128, generator=g).to(torch.bfloat16)
    ref = paged_attention_reference(q, kc, vc, ks, vs, tables, block_size, ctx, qs, ql,
                                    model_dtype=scale_dtype if kv_dtype == "int8" else torch.bfloat16)
    d = lambda t: None if t is None else t.to(device)
    out = kernels.paged_verify_attention(
        d(q), d(kc), d(vc), d(ks), d(vs), d(tables), block_size, d(ctx), d(qs), d(ql),
        max_q_len=max(q_lens), max_ctx_len=max(ctx_lens), split_len=split_len,
    )
    torch.cuda.synchronize()
    idx = real_rows(qs, ql)
    return out.cpu()[idx], ref[idx], out


@pytest.mark.parametrize("kv_dtype", ["bf16", "int8"])
def test_small_ragged_batch(device, kv_dtype):
    got, ref, _ = run_case(device, [5, 17, 40, 129, 300], [5, 1, 3, 5, 2], kv_dtype)
    assert rel_err(got, ref) < TOL


@pytest.mark.parametrize("kv_dtype", ["bf16", "int8"])
@pytest.mark.parametrize("split_len", [128, 256])
def test_split_k_merge_and_fully_masked_split_rows(device, kv_dtype, split_len):
    # contexts just past a split boundary: the last split holds keys that early
    # queries may not see, so some rows of that split are fully masked
    ctx = [split_len + 1, split_len + 3, 2 * split_len + 2, 3 * split_len, 1000]
    got, ref, _ = run_case(device, ctx, [5, 5, 5, 5, 5], kv_dtype, split_len=split_len)
    assert rel_err(got, ref) < TOL


@pytest.mark.parametrize("scale_dtype", [torch.float16, torch.bfloat16])
def test_int8_scale_dtypes(device, scale_dtype):
    got, ref, _ = run_case(device, [64, 200, 513], [5, 5, 5], "int8", scale_dtype=scale_dtype)
    assert rel_err(got, ref) < TOL


def test_padded_layout_and_block_size_32(device):
    got, ref, _ = run_case(device, [33, 90, 250], [4, 5, 1], "int8", block_size=32, padded_q=5)
    assert rel_err(got, ref) < TOL


def test_prefill_shape_many_query_rows(device):
    # q_len 64 -> 128 query rows per KV head: eight 16-row M tiles with per-tile key bounds
    got, ref, _ = run_case(device, [64, 100], [64, 37], "bf16")
    assert rel_err(got, ref) < TOL


def test_k8_drafts_use_two_row_tiles(device):
    got, ref, _ = run_case(device, [300, 1500], [9, 9], "int8")
    assert rel_err(got, ref) < TOL


def test_deterministic(device):
    _, _, a = run_case(device, [100, 700, 1500], [5, 5, 5], "int8", split_len=128)
    _, _, b = run_case(device, [100, 700, 1500], [5, 5, 5], "int8", split_len=128)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_bf16_16_seqs_ctx_256_to_2048_full_shape(device):
    """16 sequences, context U{256..2048} (seed 1), 5 queries, bf16 KV, 4096-block pool."""
    rng = np.random.default_rng(1)
    ctx = rng.integers(256, 2049, size=16).tolist()
    got, ref, _ = run_case(device, ctx, [5] * 16, "bf16", num_blocks=4096)
    assert rel_err(got, ref) < TOL


def test_int8_64_seqs_ctx_128_to_1024_full_shape(device):
    """64 sequences, context U{128..1024}, int8 KV with fp16 scales, 4096-block pool."""
    rng = np.random.default_rng(1)
    ctx = rng.integers(128, 1025, size=64).tolist()
    got, ref, _ = run_case(device, ctx, [5] * 64, "int8", scale_dtype=torch.float16, num_blocks=4096)
    assert rel_err(got, ref) < TOL


def test_workspace_error_flag_stays_clear(device):
    ws = kernels.AttentionWorkspace()
    kc, vc, ks, vs = make_pool(64, 16, HKV, "int8")
    tables, ctx, qs, ql, rows = make_batch([500, 20], [5, 5], 64, 16)
    q = torch.randn(rows, HQ, 128).to(torch.bfloat16)
    d = lambda t: t.to(device)
    kernels.paged_verify_attention(d(q), d(kc), d(vc), d(ks), d(vs), d(tables), 16, d(ctx), d(qs), d(ql),
                                   max_q_len=5, max_ctx_len=500, workspace=ws, split_len=128)
    torch.cuda.synchronize()
    assert ws.error_flag() == 0


def test_workspace_error_flag_reports_context_past_max(device):
    # ctx 500 with max_ctx_len 200 and 128-key splits: the split grid covers 256 keys,
    # so the call reads only in-range blocks, drops the rest and raises the flag
    ws = kernels.AttentionWorkspace()
    kc, vc, ks, vs = make_pool(64, 16, HKV, "int8")
    tables, ctx, qs, ql, rows = make_batch([500, 20], [5, 5], 64, 16)
    q = torch.randn(rows, HQ, 128).to(torch.bfloat16)
    d = lambda t: t.to(device)
    kernels.paged_verify_attention(d(q), d(kc), d(vc), d(ks), d(vs), d(tables), 16, d(ctx), d(qs), d(ql),
                                   max_q_len=5, max_ctx_len=200, workspace=ws, split_len=128)
    torch.cuda.synchronize()
    assert ws.error_flag() != 0


@pytest.mark.parametrize("ctx,q_lens,split_len,scale_dtype", [
    ([5, 17, 40, 129, 300, 1000], [5, 1, 3, 5, 2, 5], 0, torch.bfloat16),
    ([129, 259, 514, 1000, 2047], [5, 5, 4, 5, 5], 256, torch.float16),
    ([65, 700, 128, 1500, 16, 900, 256, 1024], [5] * 8, 128, torch.bfloat16),
    ([300, 1500, 2100, 40, 9], [9, 9, 7, 9, 9], 0, torch.float16),  # k = 8: two row tiles per KV head
])
def test_planned_matches_unplanned(device, ctx, q_lens, split_len, scale_dtype):
    """The per-step plan gives the same work items as the in-kernel plan: identical bits.
    Where the plan makes whole-sequence items instead (at most 64 tiles of context, no
    fixed split, one row tile, few sequences), the values agree up to the fp32 order."""
    num_blocks = max(64, sum((c + 15) // 16 for c in ctx) + 8)
    kc, vc, ks, vs = make_pool(num_blocks, 16, HKV, "int8", scale_dtype, seed=3)
    tables, ctx_t, qs, ql, rows = make_batch(ctx, q_lens, num_blocks, 16, seed=4)
    q = torch.randn(rows, HQ, 128, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    d = lambda t: t.to(device)
    tables_d, ctx_d, qs_d, ql_d = d(tables), d(ctx_t), d(qs), d(ql)
    args = (d(q), d(kc), d(vc), d(ks), d(vs), tables_d, 16, ctx_d, qs_d, ql_d)
    ws = kernels.AttentionWorkspace()
    a = kernels.paged_verify_attention(*args, max_q_len=max(q_lens), max_ctx_len=max(ctx), workspace=ws,
                                       split_len=split_len)
    kernels.paged_attention_plan(tables_d, 16, ctx_d, qs_d, ql_d, HQ, HKV, max(q_lens), max(ctx), ws,
                                 split_len=split_len)
    b = kernels.paged_verify_attention(*args, max_q_len=max(q_lens), max_ctx_len=max(ctx), workspace=ws,
                                       split_len=split_len, planned=True)
    torch.cuda.synchronize()
    idx = real_rows(qs, ql)
    whole = split_len == 0 and max(q_lens) * HQ // HKV <= 16 and (max(ctx) + 15) // 16 <= 64
    if whole:
        diff = float((a.cpu()[idx].float() - b.cpu()[idx].float()).abs().max())
        assert diff <= 2e-2 * float(a.cpu()[idx].float().abs().max())
    else:
        assert torch.equal(a.cpu()[idx], b.cpu()[idx])
    assert ws.error_flag() == 0
    ref = paged_attention_reference(q, kc, vc, ks, vs, tables, 16, ctx_t, qs, ql, model_dtype=scale_dtype)
    assert rel_err(b.cpu()[idx], ref[idx]) < TOL


def test_planned_path_in_a_captured_graph_replays_like_eager(device):
    """Plan + planned attention captured in a HIP graph, replayed several times with eager work
    in between: every replay equals the eager result."""
    ctx, q_lens = [300, 77, 1000, 513], [5, 5, 5, 5]
    num_blocks = 128
    kc, vc, ks, vs = make_pool(num_blocks, 16, HKV, "int8", torch.float16, seed=6)
    tables, ctx_t, qs, ql, rows = make_batch(ctx, q_lens, num_blocks, 16, seed=7)
    q = torch.randn(rows, HQ, 128, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    d = lambda t: t.to(device)
    tables, ctx_t, qs, ql, q, kc, vc, ks, vs = map(d, (tables, ctx_t, qs, ql, q, kc, vc, ks, vs))
    out = torch.empty_like(q)
    ws = kernels.AttentionWorkspace()

    def body():
        kernels.paged_attention_plan(tables, 16, ctx_t, qs, ql, HQ, HKV, 5, max(ctx), ws)
        kernels.paged_verify_attention(q, kc, vc, ks, vs, tables, 16, ctx_t, qs, ql, max_q_len=5,
                                       max_ctx_len=max(ctx), out=out, workspace=ws, planned=True)

    body()
    torch.cuda.synchronize()
    eager = out.clone()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        body()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            body()
    idx = real_rows(qs.cpu(), ql.cpu())
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.cpu()[idx], eager.cpu()[idx]), f"replay {i}"
        _ = (q.float() * 2).sum().item()  # eager work between replays


@pytest.mark.parametrize("split_len", [0, 128])
def test_k8_long_contexts_with_a_shared_prefix(device, split_len):
    """k = 8 (9 queries, 18 rows per KV head) over long contexts whose first 64 blocks are the
    same physical blocks in every table (a shared prefix), int8 with bf16 scales."""
    bs, shared = 16, 1024
    ctx = [shared + 300, shared + 2500, shared + 17, shared + 1200]
    own = [(c - shared + bs - 1) // bs for c in ctx]
    num_blocks = shared // bs + sum(own) + 8
    kc, vc, ks, vs = make_pool(num_blocks, bs, HKV, "int8", torch.bfloat16, seed=11)
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(12)).to(torch.int32)
    tables = torch.zeros(len(ctx), max((c + bs - 1) // bs for c in ctx), dtype=torch.int32)
    cur = shared // bs
    for i, n in enumerate(own):
        tables[i, : shared // bs] = perm[: shared // bs]
        tables[i, shared // bs : shared // bs + n] = perm[cur : cur + n]
        cur += n
    ql = torch.full((len(ctx),), 9, dtype=torch.int32)
    qs = torch.arange(len(ctx), dtype=torch.int32) * 9
    ctx_t = torch.tensor(ctx, dtype=torch.int32)
    q = torch.randn(9 * len(ctx), HQ, 128, generator=torch.Generator().manual_seed(13)).to(torch.bfloat16)
    ref = paged_attention_reference(q, kc, vc, ks, vs, tables, bs, ctx_t, qs, ql, model_dtype=torch.bfloat16)
    d = lambda t: t.to(device)
    out = kernels.paged_verify_attention(d(q), d(kc), d(vc), d(ks), d(vs), d(tables), bs, d(ctx_t), d(qs), d(ql),
                                         max_q_len=9, max_ctx_len=max(ctx), split_len=split_len)
    torch.cuda.synchronize()
    assert rel_err(out.cpu(), ref) < TOL


@pytest.mark.parametrize("num_seqs,max_ctx", [(64, 256), (100, 256), (200, 256), (64, 1024), (128, 1024),
                                              (64, 1025)])
def test_head_split_planned_path(device, num_seqs, max_ctx):
    """Contexts of at most 1024 keys: the planned kernel gives every sequence one item
    served by 4 (64 sequences) or 2 (100, 128) work-groups, each over 2 or 4 KV heads, a
    head's waves taking consecutive parts of its tiles and merging through LDS; 200
    sequences, or a 1025-key context, keep the split plan.  Contexts of 1..17 keys leave
    some waves without tiles."""
    rng = np.random.default_rng(num_seqs + max_ctx)
    ctx = [int(c) for c in rng.integers(1, max_ctx + 1, size=num_seqs)]
    ctx[:6] = [1, 2, 15, 16, 17, max_ctx]
    q_lens = [int(min(c, 5)) for c in ctx]
    num_blocks = sum((c + 15) // 16 for c in ctx) + 8
    kc, vc, ks, vs = make_pool(num_blocks, 16, HKV, "int8", torch.bfloat16, seed=11)
    tables, ctx_t, qs, ql, rows = make_batch(ctx, q_lens, num_blocks, 16, seed=12)
    q = torch.randn(rows, HQ, 128, generator=torch.Generator().manual_seed(13)).to(torch.bfloat16)
    d = lambda t: t.to(device)
    tables_d, ctx_d, qs_d, ql_d = d(tables), d(ctx_t), d(qs), d(ql)
    args = (d(q), d(kc), d(vc), d(ks), d(vs), tables_d, 16, ctx_d, qs_d, ql_d)
    ws = kernels.AttentionWorkspace()
    a = kernels.paged_verify_attention(*args, max_q_len=5, max_ctx_len=max(ctx), workspace=ws)
    kernels.paged_attention_plan(tables_d, 16, ctx_d, qs_d, ql_d, HQ, HKV, 5, max(ctx), ws)
    b = kernels.paged_verify_attention(*args, max_q_len=5, max_ctx_len=max(ctx), workspace=ws, planned=True)
    torch.cuda.synchronize()
    assert ws.error_flag() == 0
    idx = real_rows(qs, ql)
    ref = paged_attention_reference(q, kc, vc, ks, vs, tables, 16, ctx_t, qs, ql, model_dtype=torch.bfloat16)
    assert rel_err(b.cpu()[idx], ref[idx]) < TOL
    # the same values as one wave per head, up to the order of the fp32 sums (bf16 output)
    assert float((b.cpu()[idx].float() - a.cpu()[idx].float()).abs().max()) <= 2e-2 * float(a.cpu()[idx].float().abs().max())


@pytest.mark.parametrize("kv_dtype", ["int8", "bf16"])
def test_odd_last_tiles_ignore_what_the_previous_call_left_in_lds(device, kv_dtype):
    """A wave copies no tile past its last one, so when its tile count is odd the second ring
    slot of its last iteration holds whatever the previous kernel on that CU left in LDS.
    Calls over a pool of NaN (every K / V value, or every int8 scale) run first and fill
    the rings with NaN; the same batch over a clean pool, with 0 to 6 tiles per wave (64
    sequences, 4 waves per KV head in the planned call), must still match the oracle, and so
    must the unplanned entry point (one wave per head over splits of odd tile counts)."""
    tiles = [1, 2, 3, 5, 6, 7, 9, 11, 13, 17, 19, 21, 23, 25, 4, 8]
    ctx = [16 * t - (i % 7) for i, t in enumerate(tiles * 4)]
    q_lens = [min(5, c) for c in ctx]
    sdt = torch.float16 if kv_dtype == "int8" else torch.bfloat16
    num_blocks = sum((c + 15) // 16 for c in ctx) + 8
    kc, vc, ks, vs = make_pool(num_blocks, 16, HKV, kv_dtype, sdt, seed=21)
    tables, ctx_t, qs, ql, rows = make_batch(ctx, q_lens, num_blocks, 16, seed=22)
    q = torch.randn(rows, HQ, 128, generator=torch.Generator().manual_seed(23)).to(torch.bfloat16)
    d = lambda t: None if t is None else t.to(device)
    tables_d, ctx_d, qs_d, ql_d, q_d = d(tables), d(ctx_t), d(qs), d(ql), d(q)
    if kv_dtype == "bf16":
        poison = (torch.full_like(d(kc), float("nan")), torch.full_like(d(vc), float("nan")), None, None)
    else:
        poison = (d(kc), d(vc), torch.full_like(d(ks), float("nan")), torch.full_like(d(vs), float("nan")))
    clean = (d(kc), d(vc), d(ks), d(vs))
    ws = kernels.AttentionWorkspace()
    kernels.paged_attention_plan(tables_d, 16, ctx_d, qs_d, ql_d, HQ, HKV, 5, max(ctx), ws)
    call = lambda pool, planned, split_len=0: kernels.paged_verify_attention(
        q_d, *pool, tables_d, 16, ctx_d, qs_d, ql_d, max_q_len=5, max_ctx_len=max(ctx), workspace=ws,
        planned=planned, split_len=split_len)
    idx = real_rows(qs, ql)
    ref = paged_attention_reference(q, kc, vc, ks, vs, tables, 16, ctx_t, qs, ql, model_dtype=sdt)
    for planned, split_len in ((True, 0), (False, 128)):
        call(poison, planned, split_len)
        out = call(clean, planned, split_len)
        torch.cuda.synchronize()
        got = out.cpu()[idx]
        assert bool(torch.isfinite(got.float()).all()), (planned, split_len)
        assert rel_err(got, ref[idx]) < TOL, (planned, split_len)
    assert ws.error_flag() == 0


def _random_int8_pool(num_slots, scale_dtype, seed):
    """int8 codes U{-127..127} and per-(slot, head) scales in [0.005, 0.035): the layout the
    reference's int8 KV pool holds (ne/engine/memory/kv_cache_pool.py:49-69)."""
    g = torch.Generator().manual_seed(seed)
    kc = torch.randint(-127, 128, (num_slots, HKV, 128), generator=g, dtype=torch.int8)
    vc = torch.randint(-127, 128, (num_slots, HKV, 128), generator=g, dtype=torch.int8)
    ks = (torch.rand(num_slots, HKV, generator=g) * 0.03 + 0.005).to(scale_dtype)
    vs = (torch.rand(num_slots, HKV, generator=g) * 0.03 + 0.005).to(scale_dtype)
    return kc, vc, ks, vs


def test_long_context_32_seqs_shared_prefix_plan_and_unplanned(device):
    """The long-context + prefix-sharing configuration: 32 sequences whose tables start with
    the same 64 blocks (a 1024-token shared prefix) followed by U{4096..16384} own tokens
    (seed 1), k = 8 (9 queries), int8 KV with bf16 scales; one sequence is stretched to
    17,408 keys so the plan splits contexts above 8,192 keys over more than one split
    grid.  The per-step plan + planned call and the unplanned call both match the oracle
    (gather + dequant + masked softmax in fp32), agree bit for bit, and raise no error flag."""
    bs, shared, q = 16, 1024, 9
    rng = np.random.default_rng(1)
    ctx = [int(shared + s) for s in rng.integers(4096, 16385, size=32)]
    ctx[7] = 17408
    own = [(c - shared + bs - 1) // bs for c in ctx]
    num_blocks = shared // bs + sum(own) + 1
    kc, vc, ks, vs = _random_int8_pool(num_blocks * bs + 1, torch.bfloat16, seed=21)
    perm = torch.randperm(num_blocks, generator=torch.Generator().manual_seed(1)).to(torch.int32)
    tables = torch.zeros(32, max((c + bs - 1) // bs for c in ctx), dtype=torch.int32)
    cur = shared // bs
    for i, n in enumerate(own):
        tables[i, : shared // bs] = perm[: shared // bs]
        tables[i, shared // bs : shared // bs + n] = perm[cur : cur + n]
        cur += n
    ctx_t = torch.tensor(ctx, dtype=torch.int32)
    ql = torch.full((32,), q, dtype=torch.int32)
    qs = torch.arange(32, dtype=torch.int32) * q
    qt = torch.randn(32 * q, HQ, 128, generator=torch.Generator().manual_seed(22)).to(torch.bfloat16)
    d = lambda t: t.to(device)
    tables_d, ctx_d, qs_d, ql_d = d(tables), d(ctx_t), d(qs), d(ql)
    args = (d(qt), d(kc), d(vc), d(ks), d(vs), tables_d, bs, ctx_d, qs_d, ql_d)
    ws = kernels.AttentionWorkspace()
    unplanned = kernels.paged_verify_attention(*args, max_q_len=q, max_ctx_len=max(ctx), workspace=ws)
    torch.cuda.synchronize()
    assert ws.error_flag() == 0
    kernels.paged_attention_plan(tables_d, bs, ctx_d, qs_d, ql_d, HQ, HKV, q, max(ctx), ws)
    planned = kernels.paged_verify_attention(*args, max_q_len=q, max_ctx_len=max(ctx), workspace=ws, planned=True)
    torch.cuda.synchronize()
    assert ws.error_flag() == 0
    assert torch.equal(planned.cpu(), unplanned.cpu())
    ref = paged_attention_reference(qt, kc, vc, ks, vs, tables, bs, ctx_t, qs, ql, model_dtype=torch.bfloat16)
    assert rel_err(planned.cpu(), ref) < TOL
    for b in (7, int(np.argmin(ctx))):  # the longest and the shortest sequence on their own
        rows = slice(b * q, (b + 1) * q)
        assert rel_err(planned.cpu()[rows], ref[rows]) < TOL, f"sequence {b} ({ctx[b]} keys)"


def test_int8_64_seqs_planned_fp16_scales_roofline_variant(device):
    """The call the attention roofline times: the per-step plan and the planned call at the
    int8 configuration (64 sequences, context U{128..1024} seed 1, 5 queries, fp16 scales,
    4096-block pool), which serves each sequence as one whole item over 4 work-groups with
    4 waves per KV head merged in LDS."""
    rng = np.random.default_rng(1)
    ctx = rng.integers(128, 1025, size=64).tolist()
    kc, vc, ks, vs = make_pool(4096, 16, HKV, "int8", torch.float16, seed=0)
    tables, ctx_t, qs, ql, rows = make_batch(ctx, [5] * 64, 4096, 16, seed=1)
    qt = torch.randn(rows, HQ, 128, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    d = lambda t: t.to(device)
    tables_d, ctx_d, qs_d, ql_d = d(tables), d(ctx_t), d(qs), d(ql)
    assert kernels.plan_supported(HQ, HKV, 5, 64, torch.int8, torch.float16)
    ws = kernels.AttentionWorkspace()
    kernels.paged_attention_plan(tables_d, 16, ctx_d, qs_d, ql_d, HQ, HKV, 5, max(ctx), ws)
    out = kernels.paged_verify_attention(d(qt), d(kc), d(vc), d(ks), d(vs), tables_d, 16, ctx_d, qs_d, ql_d,
                                         max_q_len=5, max_ctx_len=max(ctx), workspace=ws, planned=True)
    torch.cuda.synchronize()
    assert ws.error_flag() == 0
    ref = paged_attention_reference(qt, kc, vc, ks, vs, tables, 16, ctx_t, qs, ql, model_dtype=torch.float16)
    assert rel_err(out.cpu(), ref) < TOL
