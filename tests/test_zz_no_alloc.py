"""The allocation-free attention entry point against the workspace one, through the C ABI.

ne_paged_verify_attention_noalloc runs the same kernels as ne_paged_verify_attention with
the work plan and split partials in the library's per-GPU scratch instead of a caller
workspace, so on the same inputs its output is identical bit for bit.  Checked on two
calls in a row, the second with a smaller input (the scratch keeps the first call's
contents), on the int8 DMA path and the bf16 register path, plus the error flag in the
caller's word and the refusal of shapes beyond the scratch.  Runs last: it leaves the
scratch allocated for the rest of the process.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from helpers import make_batch, make_pool, real_rows, rel_err
from oracle.attention import paged_attention_reference
from nanoengine_amd import _native, kernels

pytestmark = pytest.mark.gpu

HQ, HKV = 16, 8


def _vp(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _args(q, kc, vc, ks, vs, tables, ctx, qs, ql, max_q, max_ctx, out, split_len):
    return [_vp(q), q.stride(0), q.stride(1), _vp(kc), _vp(vc), _vp(ks), _vp(vs),
            3 if kc.dtype == torch.int8 else 0,
            (1 if ks.dtype == torch.float16 else 0) if ks is not None else 0,
            _vp(tables), tables.stride(0), 16, _vp(ctx), _vp(qs), _vp(ql), ctx.shape[0], HQ, HKV, 128, max_q,
            max_ctx, ctypes.c_float(1.0 / 128 ** 0.5), _vp(out), out.stride(0), out.stride(1), split_len]


def _case(device, ctx_lens, q_lens, kv, seed, split_len=0, scale_dtype=torch.float16):
    num_blocks = sum((c + 15) // 16 for c in ctx_lens) + 8
    kc, vc, ks, vs = make_pool(num_blocks, 16, HKV, kv, scale_dtype, seed=seed)
    tables, ctx, qs, ql, rows = make_batch(ctx_lens, q_lens, num_blocks, 16, seed=seed + 1)
    q = torch.randn(rows, HQ, 128, generator=torch.Generator().manual_seed(seed + 2)).to(torch.bfloat16)
    d = lambda t: None if t is None else t.to(device)
    return [d(t) for t in (q, kc, vc, ks, vs, tables, ctx, qs, ql)], (q, kc, vc, ks, vs, tables, ctx, qs, ql)


def _both(device, tensors, max_q, max_ctx, split_len=0):
    q, kc, vc, ks, vs, tables, ctx, qs, ql = tensors
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    lib = _native.load()
    nbytes = lib.ne_paged_attention_workspace_size(ctx.shape[0], HQ, HKV, max_q, max_ctx, split_len)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
    ref = torch.full_like(q, 7.0)
    _native.call("ne_paged_verify_attention",
                 *_args(q, kc, vc, ks, vs, tables, ctx, qs, ql, max_q, max_ctx, ref, split_len),
                 _vp(ws), ctypes.c_size_t(nbytes), stream)
    flag = torch.zeros(1, dtype=torch.int32, device=device)
    got = torch.full_like(q, -7.0)
    _native.call("ne_paged_verify_attention_noalloc",
                 *_args(q, kc, vc, ks, vs, tables, ctx, qs, ql, max_q, max_ctx, got, split_len), _vp(flag), stream)
    torch.cuda.synchronize()
    return ref, got, int(ws[:4].view(torch.int32).item()), int(flag.item())


@pytest.mark.parametrize("kv,scale_dtype", [("int8", torch.float16), ("int8", torch.bfloat16), ("bf16", None)])
def test_noalloc_matches_the_workspace_entry_point_twice(device, kv, scale_dtype):
    """Two calls in a row, the second smaller: identical to the workspace entry point on
    each (and, for the record, within the attention bar of the oracle)."""
    rng = np.random.default_rng(5)
    first = rng.integers(128, 1025, size=64).tolist()
    second = rng.integers(16, 300, size=9).tolist()
    for i, ctx_lens in enumerate((first, second)):
        q_lens = [5] * len(ctx_lens)
        dev_t, cpu_t = _case(device, ctx_lens, q_lens, kv, seed=40 + i, scale_dtype=scale_dtype or torch.bfloat16)
        ref, got, ws_flag, flag = _both(device, dev_t, 5, max(ctx_lens))
        assert torch.equal(got.cpu(), ref.cpu()), f"call {i}"
        assert ws_flag == 0 and flag == 0
        q, kc, vc, ks, vs, tables, ctx, qs, ql = cpu_t
        want = paged_attention_reference(q, kc, vc, ks, vs, tables, 16, ctx, qs, ql,
                                         model_dtype=scale_dtype or torch.bfloat16)
        idx = real_rows(qs, ql)
        assert rel_err(got.cpu()[idx], want[idx]) < 2e-2


def test_noalloc_error_flag_goes_to_the_callers_word(device):
    """A context past max_ctx_len with 128-key splits: the keys past the split grid are
    dropped and the flag is raised in the caller's word, as in the workspace's."""
    dev_t, _ = _case(device, [500, 20], [5, 5], "int8", seed=50)
    ref, got, ws_flag, flag = _both(device, dev_t, 5, 200, split_len=128)
    assert ws_flag != 0 and flag == ws_flag
    assert torch.equal(got.cpu(), ref.cpu())


def test_noalloc_refuses_shapes_beyond_its_scratch(device):
    """A shape whose plan and partials exceed NOALLOC_SCRATCH_BYTES is refused before any
    launch, with the sizes in the message; the wrapper takes the same path."""
    lib = _native.load()
    assert lib.ne_paged_attention_workspace_size(32, HQ, HKV, 9, 17426, 0) > _native.NOALLOC_SCRATCH_BYTES
    p = ctypes.c_void_p(256)
    flag = torch.zeros(1, dtype=torch.int32, device=device)
    rc = lib.ne_paged_verify_attention_noalloc(p, 2048, 128, p, p, p, p, 3, 0, p, 1100, 16, p, p, p, 32, 16, 8, 128,
                                                9, 17426, ctypes.c_float(0.088), p, 2048, 128, 0,
                                                ctypes.c_void_p(flag.data_ptr()), ctypes.c_void_p(0))
    assert rc == -4 and b"allocation-free" in lib.ne_last_error()
    dev_t, _ = _case(device, [300, 40], [5, 5], "int8", seed=60)
    q, kc, vc, ks, vs, tables, ctx, qs, ql = dev_t
    out = torch.empty_like(q)
    kernels.paged_verify_attention_noalloc(q, kc, vc, ks, vs, tables, 16, ctx, qs, ql, 5, 300, flag, out)
    torch.cuda.synchronize()
    assert int(flag.item()) == 0
