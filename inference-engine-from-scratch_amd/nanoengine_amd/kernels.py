"""Tensor-level wrappers over the C ABI: shape/dtype/device checks, then one launch.

Every function here requires device tensors on a ROCm GPU and launches on the
current torch stream of that device.  None of them has a CPU or PyTorch
fallback; a missing library or a CPU tensor raises.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import torch

from nanoengine_amd import _native
from nanoengine_amd._native import (
    DTYPE_BF16,
    DTYPE_FP16,
    DTYPE_FP32,
    DTYPE_INT8,
    EPILOGUE_STORE,
    EPILOGUE_SWIGLU,
)

_DTYPE_CODES = {
    torch.bfloat16: DTYPE_BF16,
    torch.float16: DTYPE_FP16,
    torch.float32: DTYPE_FP32,
    torch.int8: DTYPE_INT8,
}

HEAD_DIM = 128


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError as error:
        raise TypeError(f"unsupported dtype {dtype}") from error


def _ptr(tensor: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def _require_gpu(*tensors: torch.Tensor | None) -> torch.device:
    device = None
    for tensor in tensors:
        if tensor is None:
            continue
        if tensor.device.type != "cuda":
            raise RuntimeError(
                f"nanoengine HIP kernels need GPU tensors; got one on {tensor.device}"
            )
        if device is None:
            device = tensor.device
        elif tensor.device != device:
            raise RuntimeError(f"tensors on different devices: {device} and {tensor.device}")
    if device is None:
        raise RuntimeError("no GPU tensor given")
    return device


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _check(cond: bool, message: str) -> None:
    if not cond:
        raise ValueError(message)


def _contig(tensor: torch.Tensor, name: str) -> None:
    _check(tensor.is_contiguous(), f"{name} must be contiguous")


def _int32(tensor: torch.Tensor, name: str) -> None:
    _check(tensor.dtype == torch.int32, f"{name} must be int32, got {tensor.dtype}")
    _contig(tensor, name)


# --------------------------------------------------------------------------- A1
def ngram_propose(
    history: torch.Tensor,
    history_len: torch.Tensor,
    num_tokens: torch.Tensor,
    max_ngram: int,
    max_drafts: int,
    min_ngram: int = 1,
    drafts: torch.Tensor | None = None,
    num_drafts: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Drafts ``[b, max_drafts]`` (tail unused) and their counts ``[b]`` from each history."""
    device = _require_gpu(history, history_len, num_tokens)
    _int32(history, "history")
    _int32(history_len, "history_len")
    _int32(num_tokens, "num_tokens")
    _check(history.dim() == 2, "history must be [num_seqs, capacity]")
    num_seqs = history.shape[0]
    if drafts is None:
        drafts = torch.zeros((num_seqs, max_drafts), dtype=torch.int32, device=device)
    if num_drafts is None:
        num_drafts = torch.empty((num_seqs,), dtype=torch.int32, device=device)
    _native.call(
        "ne_ngram_propose",
        _ptr(history), history.stride(0), _ptr(history_len), _ptr(num_tokens), num_seqs,
        max_ngram, min_ngram, max_drafts, _ptr(drafts), _ptr(num_drafts), _stream(device),
    )
    return drafts, num_drafts


# --------------------------------------------------------------------------- A7
def kv_write(
    vectors: torch.Tensor,
    slot_mapping: torch.Tensor,
    cache: torch.Tensor,
    scales: torch.Tensor | None,
) -> None:
    """Write ``vectors [n, heads, 128]`` to ``cache`` at ``slot_mapping`` (quantising to int8)."""
    device = _require_gpu(vectors, slot_mapping, cache, scales)
    _contig(vectors, "vectors")
    _int32(slot_mapping, "slot_mapping")
    _check(vectors.dim() == 3 and vectors.shape[2] == HEAD_DIM, "vectors must be [n, heads, 128]")
    _check(cache.dim() == 3 and cache.shape[1:] == vectors.shape[1:], "cache shape mismatch")
    _check(slot_mapping.numel() == vectors.shape[0], "one slot per vector row")
    if cache.dtype == torch.int8:
        _check(scales is not None and scales.shape[0] == cache.shape[0], "int8 cache needs scales")
    _native.call(
        "ne_kv_write",
        _ptr(vectors), dtype_code(vectors.dtype), vectors.shape[0], vectors.shape[1], HEAD_DIM,
        _ptr(slot_mapping), _ptr(cache), dtype_code(cache.dtype), _ptr(scales),
        dtype_code(scales.dtype) if scales is not None else DTYPE_BF16, _stream(device),
    )


# --------------------------------------------------------------------------- A6
@dataclass
class AttentionWorkspace:
    """Caller-owned scratch for split-K attention; re-zeroed when its layout changes.

    ``plan_key`` names the metadata the last :func:`paged_attention_plan` call used, so
    that a planned attention call on other metadata is refused.  ``frozen`` is set once a
    captured HIP graph holds the buffer's address: from then on a call that would need a
    larger buffer raises instead of reallocating under the graph."""

    buffer: torch.Tensor | None = None
    layout: tuple | None = None
    plan_key: tuple | None = None
    runs_key: tuple | None = None  # metadata of the last paged_kv_runs_plan (measurement)
    frozen: bool = False

    def get(self, device: torch.device, nbytes: int, layout: tuple) -> torch.Tensor:
        if self.buffer is None or self.buffer.numel() < nbytes or self.buffer.device != device:
            if self.frozen:
                have = 0 if self.buffer is None else self.buffer.numel()
                raise RuntimeError(f"attention workspace of {have} bytes is held by a captured HIP graph; "
                                   f"this call needs {nbytes} bytes on {device}: size it before capture")
            self.buffer = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
            self.layout = layout
            self.plan_key = self.runs_key = None
        elif self.layout != layout:
            self.buffer.zero_()
            self.layout = layout
            self.plan_key = self.runs_key = None
        return self.buffer

    def error_flag(self) -> int:
        if self.buffer is None:
            return 0
        return int(self.buffer[:4].view(torch.int32).item())


_default_workspaces: dict[torch.device, AttentionWorkspace] = {}


def default_workspace(device: torch.device) -> AttentionWorkspace:
    return _default_workspaces.setdefault(device, AttentionWorkspace())


def paged_verify_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_scale: torch.Tensor | None,
    v_scale: torch.Tensor | None,
    block_tables: torch.Tensor,
    block_size: int,
    ctx_len: torch.Tensor,
    q_start: torch.Tensor,
    q_len: torch.Tensor,
    max_q_len: int,
    max_ctx_len: int,
    softmax_scale: float | None = None,
    out: torch.Tensor | None = None,
    workspace: AttentionWorkspace | None = None,
    split_len: int = 0,
    planned: bool = False,
) -> torch.Tensor:
    """Paged multi-query attention; ``q``/``out`` are ``[rows, q_heads, 128]`` bf16.

    ``planned=True`` reads the work plan that :func:`paged_attention_plan` wrote into
    the same ``workspace`` for the same metadata (once per step, shared by the layers)."""
    device = _require_gpu(q, k_cache, v_cache, k_scale, v_scale, block_tables, ctx_len, q_start,
                          q_len)
    _check(q.dtype == torch.bfloat16 and q.dim() == 3 and q.shape[2] == HEAD_DIM,
           "q must be [rows, heads, 128] bf16")
    _check(q.stride(2) == 1, "q head_dim must be contiguous")
    _check(k_cache.shape == v_cache.shape and k_cache.dim() == 3, "k/v cache shape mismatch")
    _check(k_cache.is_contiguous() and v_cache.is_contiguous(), "caches must be contiguous")
    is_int8 = k_cache.dtype == torch.int8
    if is_int8:
        _check(k_scale is not None and v_scale is not None, "int8 cache needs scales")
        _check(k_scale.is_contiguous() and v_scale.is_contiguous(), "scales must be contiguous")
        _check(k_scale.numel() == k_cache.shape[0] * k_cache.shape[1], "k_scale shape mismatch")
    else:
        _check(k_cache.dtype == torch.bfloat16, "cache must be int8 or bf16")
    _int32(block_tables, "block_tables")
    for name, t in (("ctx_len", ctx_len), ("q_start", q_start), ("q_len", q_len)):
        _int32(t, name)
    num_seqs = ctx_len.shape[0]
    num_q_heads = q.shape[1]
    num_kv_heads = k_cache.shape[1]
    if out is None:
        out = torch.empty_like(q)
    _check(out.shape == q.shape and out.dtype == torch.bfloat16 and out.stride(2) == 1,
           "out must match q")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(HEAD_DIM)
    nbytes = _native.load().ne_paged_attention_workspace_size(
        num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len, split_len
    )
    _check(nbytes > 0, "bad attention shape")
    workspace = workspace or default_workspace(device)
    ws = workspace.get(device, nbytes, (num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len, split_len))
    if planned:
        _check(workspace.plan_key == _plan_key(block_tables, block_size, ctx_len, q_start, q_len, max_q_len,
                                               max_ctx_len, split_len),
               "planned attention needs paged_attention_plan on the same metadata and workspace first")
    _native.call(
        "ne_paged_verify_attention_planned" if planned else "ne_paged_verify_attention",
        _ptr(q), q.stride(0), q.stride(1),
        _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale),
        dtype_code(k_cache.dtype), dtype_code(k_scale.dtype) if is_int8 else DTYPE_BF16,
        _ptr(block_tables), block_tables.stride(0), block_size,
        _ptr(ctx_len), _ptr(q_start), _ptr(q_len),
        num_seqs, num_q_heads, num_kv_heads, HEAD_DIM, max_q_len, max_ctx_len,
        float(softmax_scale),
        _ptr(out), out.stride(0), out.stride(1),
        split_len, _ptr(ws), ws.numel(), _stream(device),
    )
    return out


def paged_verify_attention_noalloc(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_scale: torch.Tensor | None,
    v_scale: torch.Tensor | None,
    block_tables: torch.Tensor,
    block_size: int,
    ctx_len: torch.Tensor,
    q_start: torch.Tensor,
    q_len: torch.Tensor,
    max_q_len: int,
    max_ctx_len: int,
    error_flag: torch.Tensor,
    out: torch.Tensor,
    softmax_scale: float | None = None,
    split_len: int = 0,
) -> torch.Tensor:
    """:func:`paged_verify_attention` without a workspace: the work plan and split partials
    live in the library's per-GPU scratch (``NOALLOC_SCRATCH_BYTES``), ``error_flag`` is a
    caller-owned int32 device word that receives the error bits, and ``out`` is given, so
    the call allocates nothing (usable where allocation is not allowed).  Calls that
    overlap on one GPU share the scratch and race."""
    device = _require_gpu(q, k_cache, v_cache, k_scale, v_scale, block_tables, ctx_len, q_start, q_len,
                          error_flag, out)
    _check(q.dtype == torch.bfloat16 and q.dim() == 3 and q.shape[2] == HEAD_DIM and q.stride(2) == 1,
           "q must be [rows, heads, 128] bf16")
    _check(out.shape == q.shape and out.dtype == torch.bfloat16 and out.stride(2) == 1, "out must match q")
    _check(error_flag.dtype == torch.int32 and error_flag.numel() >= 1, "error_flag must be an int32 word")
    is_int8 = k_cache.dtype == torch.int8
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(HEAD_DIM)
    _native.call(
        "ne_paged_verify_attention_noalloc",
        _ptr(q), q.stride(0), q.stride(1),
        _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale),
        dtype_code(k_cache.dtype), dtype_code(k_scale.dtype) if is_int8 else DTYPE_BF16,
        _ptr(block_tables), block_tables.stride(0), block_size,
        _ptr(ctx_len), _ptr(q_start), _ptr(q_len),
        ctx_len.shape[0], q.shape[1], k_cache.shape[1], HEAD_DIM, max_q_len, max_ctx_len,
        float(softmax_scale),
        _ptr(out), out.stride(0), out.stride(1),
        split_len, _ptr(error_flag), _stream(device),
    )
    return out


def _plan_key(block_tables, block_size, ctx_len, q_start, q_len, max_q_len, max_ctx_len, split_len) -> tuple:
    return (block_tables.data_ptr(), tuple(block_tables.shape), block_tables.stride(0), block_size,
            ctx_len.data_ptr(), q_start.data_ptr(), q_len.data_ptr(), ctx_len.shape[0], max_q_len, max_ctx_len,
            split_len)


def paged_attention_plan(
    block_tables: torch.Tensor,
    block_size: int,
    ctx_len: torch.Tensor,
    q_start: torch.Tensor,
    q_len: torch.Tensor,
    num_q_heads: int,
    num_kv_heads: int,
    max_q_len: int,
    max_ctx_len: int,
    workspace: AttentionWorkspace,
    split_len: int = 0,
) -> None:
    """Write the attention work plan for this metadata into ``workspace`` (8 KV heads and
    at most 32 query rows per KV head; bf16 pools or int8 ones with 2-byte scales)."""
    device = _require_gpu(block_tables, ctx_len, q_start, q_len)
    _int32(block_tables, "block_tables")
    for name, t in (("ctx_len", ctx_len), ("q_start", q_start), ("q_len", q_len)):
        _int32(t, name)
    num_seqs = ctx_len.shape[0]
    nbytes = _native.load().ne_paged_attention_workspace_size(
        num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len, split_len
    )
    _check(nbytes > 0, "bad attention shape")
    ws = workspace.get(device, nbytes, (num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len, split_len))
    _native.call(
        "ne_paged_attention_plan",
        _ptr(block_tables), block_tables.stride(0), block_size, _ptr(ctx_len), _ptr(q_start), _ptr(q_len),
        num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len, split_len, _ptr(ws), ws.numel(),
        _stream(device),
    )
    workspace.plan_key = _plan_key(block_tables, block_size, ctx_len, q_start, q_len, max_q_len, max_ctx_len,
                                   split_len)
    workspace.runs_key = None


def paged_kv_stream_planned(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_scale: torch.Tensor | None,
    v_scale: torch.Tensor | None,
    num_seqs: int,
    num_q_heads: int,
    max_q_len: int,
    max_ctx_len: int,
    workspace: AttentionWorkspace,
    split_len: int = 0,
) -> None:
    """Measurement: the K/V reads of the planned attention call alone (its plan, tiles, ring
    and copies; nothing computed or stored), on the plan ``workspace`` holds for the same
    metadata.  Its time is the memory ceiling of that call's access pattern."""
    device = _require_gpu(k_cache, v_cache, k_scale, v_scale)
    _check(workspace.buffer is not None and workspace.plan_key is not None,
           "the stream reads the plan paged_attention_plan wrote into the workspace")
    num_kv_heads = k_cache.shape[1]
    is_int8 = k_cache.dtype == torch.int8
    _native.call(
        "ne_paged_kv_stream_planned",
        _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale), dtype_code(k_cache.dtype),
        dtype_code(k_scale.dtype) if is_int8 else DTYPE_BF16, num_seqs, num_q_heads, num_kv_heads, max_q_len,
        max_ctx_len, split_len, _ptr(workspace.buffer), workspace.buffer.numel(), _stream(device),
    )


def paged_kv_runs_plan(
    block_tables: torch.Tensor,
    block_size: int,
    ctx_len: torch.Tensor,
    num_q_heads: int,
    num_kv_heads: int,
    max_q_len: int,
    max_ctx_len: int,
    workspace: AttentionWorkspace,
) -> None:
    """Measurement: cut the sequences' 16-key tiles, in order, into the workspace's
    plan_grid runs of near-equal length across sequence boundaries, for
    :func:`paged_kv_stream_runs`.  The runs take the place of the attention work plan,
    so a planned call afterwards needs :func:`paged_attention_plan` again."""
    device = _require_gpu(block_tables, ctx_len)
    _int32(block_tables, "block_tables")
    _int32(ctx_len, "ctx_len")
    num_seqs = ctx_len.shape[0]
    nbytes = _native.load().ne_paged_attention_workspace_size(
        num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len, 0
    )
    _check(nbytes > 0, "bad attention shape")
    ws = workspace.get(device, nbytes, (num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len, 0))
    _native.call(
        "ne_paged_kv_runs_plan",
        _ptr(block_tables), block_tables.stride(0), block_size, _ptr(ctx_len), num_seqs, num_q_heads,
        num_kv_heads, max_q_len, max_ctx_len, _ptr(ws), ws.numel(), _stream(device),
    )
    workspace.plan_key = None
    workspace.runs_key = (num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len)


def paged_kv_stream_runs(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_scale: torch.Tensor | None,
    v_scale: torch.Tensor | None,
    num_seqs: int,
    num_q_heads: int,
    max_q_len: int,
    max_ctx_len: int,
    workspace: AttentionWorkspace,
) -> None:
    """Measurement: the same K/V bytes as the planned call, read in the balanced whole-slot
    runs that :func:`paged_kv_runs_plan` wrote (work-group w reads all 8 KV heads of every
    tile of run w through the planned call's ring and copies; nothing computed or stored)."""
    device = _require_gpu(k_cache, v_cache, k_scale, v_scale)
    num_kv_heads = k_cache.shape[1]
    _check(workspace.buffer is not None
           and workspace.runs_key == (num_seqs, num_q_heads, num_kv_heads, max_q_len, max_ctx_len),
           "the stream reads the runs paged_kv_runs_plan wrote into the workspace for this shape")
    is_int8 = k_cache.dtype == torch.int8
    _native.call(
        "ne_paged_kv_stream_runs",
        _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale), dtype_code(k_cache.dtype),
        dtype_code(k_scale.dtype) if is_int8 else DTYPE_BF16, num_seqs, num_q_heads, num_kv_heads, max_q_len,
        max_ctx_len, _ptr(workspace.buffer), workspace.buffer.numel(), _stream(device),
    )


def plan_supported(num_q_heads: int, num_kv_heads: int, max_q_len: int, num_seqs: int, kv_dtype, scale_dtype) -> bool:
    """Whether :func:`paged_attention_plan` / ``planned=True`` serve this shape."""
    cache_ok = kv_dtype == torch.bfloat16 or (kv_dtype == torch.int8 and scale_dtype in (torch.bfloat16,
                                                                                        torch.float16))
    return (cache_ok and num_kv_heads == 8 and num_q_heads % num_kv_heads == 0
            and (num_q_heads // num_kv_heads) * max_q_len <= 32 and num_seqs <= 1024)


# --------------------------------------------------------------------------- A8
def w8a16_gemm(
    x: torch.Tensor,
    weight_int8: torch.Tensor,
    weight_scale: torch.Tensor,
    epilogue: int = EPILOGUE_STORE,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``bf16(x @ (int8 * scale).T)``; SwiGLU epilogue pairs 16 gate rows with 16 up rows."""
    device = _require_gpu(x, weight_int8, weight_scale)
    _check(x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1, "x must be [m, k] bf16")
    _check(weight_int8.dtype == torch.int8 and weight_int8.dim() == 2, "weight must be [n, k] int8")
    _contig(weight_int8, "weight_int8")
    _contig(weight_scale, "weight_scale")
    m, k = x.shape
    n = weight_int8.shape[0]
    _check(weight_int8.shape[1] == k, f"k mismatch: x has {k}, weight {weight_int8.shape[1]}")
    _check(weight_scale.numel() == n, "one scale per weight row")
    n_out = n // 2 if epilogue == EPILOGUE_SWIGLU else n
    if out is None:
        out = torch.empty((m, n_out), dtype=torch.bfloat16, device=device)
    _check(out.shape == (m, n_out) and out.stride(1) == 1, "bad out shape")
    _native.call(
        "ne_w8a16_gemm",
        _ptr(x), x.stride(0), _ptr(weight_int8), _ptr(weight_scale),
        dtype_code(weight_scale.dtype), m, n, k, _ptr(out), out.stride(0), epilogue,
        _stream(device),
    )
    return out


PROJ_TILE_ROWS = 80  # token rows per work-group of the W8A16 kernels
SPLITK_TILE_ROWS = 48  # token rows per work-group of the split-K product
PROJ_TILE_COLS = 64  # weight rows per work-group of the store / split-K kernels
TARGET_WORK_GROUPS = 256  # one per CU


def splitk_splits(m: int, n: int, k: int, max_splits: int = 4) -> int:
    """K splits that bring a narrow projection to about one work-group per CU (at most; 320
    rows of o / down give 7 x 16 tiles of 48 rows and 2 splits)."""
    tiles = -(-m // SPLITK_TILE_ROWS) * (n // PROJ_TILE_COLS)
    splits = max(1, min(max_splits, TARGET_WORK_GROUPS // max(tiles, 1)))
    while splits > 1 and k % (128 * splits):
        splits -= 1
    return splits


def w8a16_gemm_splitk(
    x: torch.Tensor,
    weight_int8: torch.Tensor,
    weight_scale: torch.Tensor,
    splits: int,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """fp32 ``[splits, m, n]`` partial products over K parts (scale applied), summed by
    ``splitk_add_rmsnorm``."""
    device = _require_gpu(x, weight_int8, weight_scale)
    _check(x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1, "x must be [m, k] bf16")
    _check(weight_int8.dtype == torch.int8 and weight_int8.dim() == 2, "weight must be [n, k] int8")
    _contig(weight_int8, "weight_int8")
    _contig(weight_scale, "weight_scale")
    m, k = x.shape
    n = weight_int8.shape[0]
    _check(weight_int8.shape[1] == k, f"k mismatch: x has {k}, weight {weight_int8.shape[1]}")
    _check(weight_scale.numel() == n, "one scale per weight row")
    if out is None:
        out = torch.empty((splits, m, n), dtype=torch.float32, device=device)
    _check(out.dtype == torch.float32 and out.is_contiguous() and out.numel() >= splits * m * n,
           "partials must be contiguous fp32 with room for [splits, m, n]")
    _native.call(
        "ne_w8a16_gemm_splitk",
        _ptr(x), x.stride(0), _ptr(weight_int8), _ptr(weight_scale),
        dtype_code(weight_scale.dtype), m, n, k, splits, _ptr(out), _stream(device),
    )
    return out


def lm_head_num_tiles(vocab: int) -> int:
    return int(_native.load().ne_lm_head_num_tiles(vocab))


def lm_head(
    x: torch.Tensor,
    weight: torch.Tensor,
    logits: torch.Tensor | bool = True,
    argmax_partials: torch.Tensor | bool = False,
) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """``x [m, k] @ weight[n, k].T`` in bf16; optionally only per-tile argmax partials."""
    device = _require_gpu(x, weight)
    _check(x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16, "bf16 inputs required")
    _check(x.dim() == 2 and x.stride(1) == 1, "x must be [m, k]")
    _contig(weight, "weight")
    m, k = x.shape
    _check(weight.dim() == 2 and weight.shape[1] == k, f"k mismatch: x has {k}, weight {tuple(weight.shape)}")
    n = weight.shape[0]
    if logits is True:
        logits = torch.empty((m, n), dtype=torch.bfloat16, device=device)
    elif logits is False:
        logits = None
    if argmax_partials is True:
        argmax_partials = torch.empty((m, lm_head_num_tiles(n)), dtype=torch.int64, device=device)
    elif argmax_partials is False:
        argmax_partials = None
    _native.call(
        "ne_lm_head",
        _ptr(x), x.stride(0), _ptr(weight), m, n, k, _ptr(logits),
        logits.stride(0) if logits is not None else 0, _ptr(argmax_partials), _stream(device),
    )
    return logits, argmax_partials


# ------------------------------------------------------------------- norms, RoPE
def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, out=None) -> torch.Tensor:
    device = _require_gpu(x, weight)
    _contig(x, "x")
    out = torch.empty_like(x) if out is None else out
    rows, hidden = x.shape
    _native.call("ne_rmsnorm", _ptr(x), _ptr(weight), _ptr(out), rows, hidden, float(eps),
                 _stream(device))
    return out


def add_rmsnorm(residual: torch.Tensor, delta: torch.Tensor, weight: torch.Tensor, eps: float,
                out=None) -> torch.Tensor:
    """``residual += delta`` (bf16) in place, then RMSNorm of the new residual."""
    device = _require_gpu(residual, delta, weight)
    _contig(residual, "residual")
    _contig(delta, "delta")
    out = torch.empty_like(residual) if out is None else out
    rows, hidden = residual.shape
    _native.call("ne_add_rmsnorm", _ptr(residual), _ptr(delta), _ptr(weight), _ptr(out), rows,
                 hidden, float(eps), _stream(device))
    return out


def splitk_add_rmsnorm(residual: torch.Tensor, partials: torch.Tensor, splits: int, weight: torch.Tensor,
                       eps: float, out=None) -> torch.Tensor:
    """``residual += bf16(sum of the split-K partials)`` in place, then RMSNorm."""
    device = _require_gpu(residual, partials, weight)
    _contig(residual, "residual")
    rows, hidden = residual.shape
    _check(partials.dtype == torch.float32 and partials.is_contiguous()
           and partials.numel() >= splits * rows * hidden, "partials must be fp32 [splits, rows, hidden]")
    out = torch.empty_like(residual) if out is None else out
    _native.call("ne_splitk_add_rmsnorm", _ptr(residual), _ptr(partials), splits, _ptr(weight), _ptr(out),
                 rows, hidden, float(eps), _stream(device))
    return out


def embed_rmsnorm(tokens: torch.Tensor, embed: torch.Tensor, weight: torch.Tensor, eps: float,
                  residual=None, out=None) -> tuple[torch.Tensor, torch.Tensor]:
    device = _require_gpu(tokens, embed, weight)
    _int32(tokens, "tokens")
    rows = tokens.numel()
    hidden = embed.shape[1]
    if residual is None:
        residual = torch.empty((rows, hidden), dtype=embed.dtype, device=device)
    if out is None:
        out = torch.empty((rows, hidden), dtype=embed.dtype, device=device)
    _native.call("ne_embed_rmsnorm", _ptr(tokens), _ptr(embed), _ptr(weight), _ptr(residual),
                 _ptr(out), rows, hidden, float(eps), _stream(device))
    return residual, out


def rope_table(positions: int, rope_theta: float, head_dim: int = HEAD_DIM) -> torch.Tensor:
    """[positions, 2, head_dim / 2] bf16 cos | sin on the CPU, built exactly as
    build_rotary_tables does (ne/models/qwen3.py:47-57): fp32 inverse frequencies,
    fp32 angles position * inv_freq, cos/sin in fp32, then rounded to bf16."""
    exps = torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim
    inv_freq = 1.0 / (rope_theta**exps)
    angles = torch.arange(positions).float()[:, None] * inv_freq
    return torch.stack([angles.cos(), angles.sin()], dim=1).to(torch.bfloat16).contiguous()


def qk_norm_rope_kv_write(
    qkv: torch.Tensor,
    num_q_heads: int,
    num_kv_heads: int,
    q_norm_weight: torch.Tensor,
    k_norm_weight: torch.Tensor,
    eps: float,
    positions: torch.Tensor,
    rope_cos_sin: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_scale: torch.Tensor | None,
    v_scale: torch.Tensor | None,
    q_out: torch.Tensor | None = None,
) -> torch.Tensor:
    device = _require_gpu(qkv, q_norm_weight, k_norm_weight, positions, rope_cos_sin, slot_mapping,
                          k_cache, v_cache)
    _contig(qkv, "qkv")
    _int32(positions, "positions")
    _int32(slot_mapping, "slot_mapping")
    _check(rope_cos_sin.dtype == torch.bfloat16 and rope_cos_sin.dim() == 3 and rope_cos_sin.shape[1:] == (2, 64)
           and rope_cos_sin.is_contiguous(), "rope_cos_sin must be contiguous [positions, 2, 64] bf16")
    rows = qkv.shape[0]
    _check(qkv.shape[1] == (num_q_heads + 2 * num_kv_heads) * HEAD_DIM, "qkv width mismatch")
    if q_out is None:
        q_out = torch.empty((rows, num_q_heads, HEAD_DIM), dtype=torch.bfloat16, device=device)
    is_int8 = k_cache.dtype == torch.int8
    _native.call(
        "ne_qk_norm_rope_kv_write",
        _ptr(qkv), rows, num_q_heads, num_kv_heads, HEAD_DIM,
        _ptr(q_norm_weight), _ptr(k_norm_weight), float(eps),
        _ptr(positions), _ptr(rope_cos_sin), rope_cos_sin.shape[0], _ptr(slot_mapping),
        _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale),
        dtype_code(k_cache.dtype), dtype_code(k_scale.dtype) if is_int8 else DTYPE_BF16,
        _ptr(q_out), _stream(device),
    )
    return q_out


def w8a16_qkv_norm_rope_kv(
    x: torch.Tensor,
    w_int8: torch.Tensor,
    w_scale: torch.Tensor,
    num_q_heads: int,
    num_kv_heads: int,
    q_norm_weight: torch.Tensor,
    k_norm_weight: torch.Tensor,
    eps: float,
    positions: torch.Tensor,
    rope_cos_sin: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k_scale: torch.Tensor | None,
    v_scale: torch.Tensor | None,
    q_out: torch.Tensor,
) -> torch.Tensor:
    """The QKV projection with QK-norm, RoPE and the KV write fused into its epilogue:
    the same bits as :func:`w8a16_gemm` followed by :func:`qk_norm_rope_kv_write`."""
    device = _require_gpu(x, w_int8, w_scale, q_norm_weight, k_norm_weight, positions, rope_cos_sin,
                          slot_mapping, k_cache, v_cache, q_out)
    _check(x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1, "x must be [m, k] bf16")
    _check(w_int8.dtype == torch.int8 and w_int8.is_contiguous(), "w must be contiguous int8")
    _int32(positions, "positions")
    _int32(slot_mapping, "slot_mapping")
    _check(rope_cos_sin.dtype == torch.bfloat16 and rope_cos_sin.dim() == 3 and rope_cos_sin.shape[1:] == (2, 64)
           and rope_cos_sin.is_contiguous(), "rope_cos_sin must be contiguous [positions, 2, 64] bf16")
    rows, kdim = x.shape
    _check(w_int8.shape == ((num_q_heads + 2 * num_kv_heads) * HEAD_DIM, kdim), "w shape mismatch")
    _check(q_out.shape == (rows, num_q_heads, HEAD_DIM) and q_out.dtype == torch.bfloat16 and q_out.is_contiguous(),
           "q_out must be contiguous [rows, q_heads, 128] bf16")
    is_int8 = k_cache.dtype == torch.int8
    _native.call(
        "ne_w8a16_qkv_norm_rope_kv",
        _ptr(x), x.stride(0), _ptr(w_int8), _ptr(w_scale), dtype_code(w_scale.dtype), rows,
        num_q_heads, num_kv_heads, kdim,
        _ptr(q_norm_weight), _ptr(k_norm_weight), float(eps),
        _ptr(positions), _ptr(rope_cos_sin), rope_cos_sin.shape[0], _ptr(slot_mapping),
        dtype_code(k_cache.dtype), _ptr(k_cache), _ptr(v_cache), _ptr(k_scale), _ptr(v_scale),
        dtype_code(k_scale.dtype) if is_int8 else DTYPE_BF16,
        _ptr(q_out), _stream(device),
    )
    return q_out


def qkv_fusion_supported(k_cache: torch.Tensor, k_scale: torch.Tensor | None) -> bool:
    """Whether :func:`w8a16_qkv_norm_rope_kv` takes this cache (bf16, or int8 with bf16/fp16 scales)."""
    if k_cache.dtype == torch.bfloat16:
        return True
    return k_cache.dtype == torch.int8 and k_scale is not None and k_scale.dtype in (torch.bfloat16, torch.float16)


# ------------------------------------------------------------------------ A9/A10
def accept(
    drafts: torch.Tensor,
    num_drafts: torch.Tensor,
    row_start: torch.Tensor,
    vocab: int,
    logits: torch.Tensor | None = None,
    argmax_partials: torch.Tensor | None = None,
    temperature: float | torch.Tensor = 0.0,
    top_p: float | torch.Tensor = 1.0,
    seeds: torch.Tensor | None = None,
    steps: torch.Tensor | None = None,
    out_tokens: torch.Tensor | None = None,
    num_out: torch.Tensor | None = None,
    history: torch.Tensor | None = None,
    history_len: torch.Tensor | None = None,
    num_cached: torch.Tensor | None = None,
    draft_logits: torch.Tensor | None = None,
    draft_probs: torch.Tensor | None = None,
    draft_row_start: torch.Tensor | None = None,
    any_sampled: bool | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Accepted guesses plus one target token per sequence: ``(out_tokens [b, k+1], num_out [b])``.

    ``temperature`` / ``top_p``: one value for every sequence, or per-sequence fp32 device
    tensors (0 = greedy); with tensors, ``any_sampled`` says whether any temperature is
    positive (the host knows it without reading the device).  The draft distribution of
    each guess (sampled sequences): ``draft_logits`` (bf16, the draft model's logits; its
    distribution is the same temperature/top-p softmax) or ``draft_probs`` (fp32
    probabilities used as given), row ``draft_row_start[b] + i`` for guess i of sequence b;
    neither: the guesses count as deterministic (one-hot draft distribution)."""
    device = _require_gpu(drafts, num_drafts, row_start, logits, argmax_partials)
    _int32(drafts, "drafts")
    _int32(num_drafts, "num_drafts")
    _int32(row_start, "row_start")
    num_seqs, max_drafts = drafts.shape
    if isinstance(temperature, torch.Tensor):
        _check(temperature.dtype == torch.float32 and temperature.numel() >= num_seqs, "temperature [b] fp32")
        _check(any_sampled is not None, "per-sequence temperatures need any_sampled")
        temps = temperature
    else:
        any_sampled = float(temperature) > 0.0
        temps = torch.full((num_seqs,), float(temperature), dtype=torch.float32, device=device) if any_sampled \
            else None
    if isinstance(top_p, torch.Tensor):
        _check(top_p.dtype == torch.float32 and top_p.numel() >= num_seqs, "top_p [b] fp32")
        top_ps = top_p
    else:
        top_ps = None if float(top_p) >= 1.0 else torch.full((num_seqs,), float(top_p), dtype=torch.float32,
                                                                device=device)
    if logits is not None:
        _check(logits.dtype == torch.bfloat16 and logits.stride(1) == 1, "logits must be bf16 rows")
        _check(logits.shape[1] == vocab, "logits width must equal vocab")
    if any_sampled:
        _check(logits is not None, "sampled acceptance needs logits")
        _check(seeds is not None and steps is not None, "sampled acceptance needs seeds and steps")
        _check(seeds.dtype == torch.int64 and steps.dtype == torch.int64, "seeds/steps int64")
    _check(draft_logits is None or draft_probs is None, "give draft logits or draft probabilities, not both")
    draft = draft_logits if draft_logits is not None else draft_probs
    draft_dtype = DTYPE_BF16
    if draft is not None:
        _check(any_sampled, "draft distributions need sampled acceptance")
        want = torch.bfloat16 if draft_logits is not None else torch.float32
        _check(draft.dtype == want and draft.stride(1) == 1, f"draft rows must be {want} rows")
        _check(draft.shape[1] == vocab, "draft rows' width must equal vocab")
        _check(draft_row_start is not None, "draft rows need draft_row_start")
        _int32(draft_row_start, "draft_row_start")
        draft_dtype = dtype_code(draft.dtype)
    if out_tokens is None:
        out_tokens = torch.empty((num_seqs, max_drafts + 1), dtype=torch.int32, device=device)
    if num_out is None:
        num_out = torch.empty((num_seqs,), dtype=torch.int32, device=device)
    num_tiles = argmax_partials.shape[1] if argmax_partials is not None else 0
    _native.call(
        "ne_accept",
        _ptr(logits), logits.stride(0) if logits is not None else 0,
        _ptr(argmax_partials), num_tiles, vocab,
        _ptr(drafts), max_drafts, _ptr(num_drafts), _ptr(row_start), num_seqs,
        _ptr(temps), _ptr(top_ps), int(bool(any_sampled)), _ptr(seeds), _ptr(steps),
        _ptr(out_tokens), _ptr(num_out),
        _ptr(history), history.stride(0) if history is not None else 0,
        _ptr(history_len), _ptr(num_cached),
        _ptr(draft), draft_dtype, draft.stride(0) if draft is not None else 0, _ptr(draft_row_start),
        _stream(device),
    )
    return out_tokens, num_out


def prepare_verify_step(
    history: torch.Tensor,
    history_len: torch.Tensor,
    drafts: torch.Tensor,
    num_drafts: torch.Tensor,
    block_tables: torch.Tensor,
    block_size: int,
    scratch_slot: int,
    tokens: torch.Tensor,
    positions: torch.Tensor,
    slot_mapping: torch.Tensor,
    q_start: torch.Tensor,
    q_len: torch.Tensor,
    ctx_len: torch.Tensor,
) -> None:
    """Pack a batched verify step on the device: rows, positions, slots, attention metadata."""
    device = _require_gpu(history, history_len, drafts, num_drafts, block_tables, tokens, positions,
                          slot_mapping, q_start, q_len, ctx_len)
    for name, t in (("history", history), ("history_len", history_len), ("drafts", drafts),
                    ("num_drafts", num_drafts), ("block_tables", block_tables), ("tokens", tokens),
                    ("positions", positions), ("slot_mapping", slot_mapping), ("q_start", q_start),
                    ("q_len", q_len), ("ctx_len", ctx_len)):
        _int32(t, name)
    num_seqs, max_drafts = drafts.shape
    _check(tokens.numel() >= num_seqs * (max_drafts + 1), "tokens too small for the padded rows")
    _native.call(
        "ne_prepare_verify_step",
        _ptr(history), history.stride(0), _ptr(history_len), _ptr(drafts), max_drafts, _ptr(num_drafts),
        _ptr(block_tables), block_tables.stride(0), block_size, scratch_slot, num_seqs,
        _ptr(tokens), _ptr(positions), _ptr(slot_mapping), _ptr(q_start), _ptr(q_len), _ptr(ctx_len),
        _stream(device),
    )


def advance_step_counts(history_len: torch.Tensor, num_out: torch.Tensor, max_new_tokens: torch.Tensor,
                        num_generated: torch.Tensor, steps: torch.Tensor, num_guesses: torch.Tensor,
                        k: int) -> None:
    """After a verify step: active sequences add their emitted tokens to the generated
    count, advance the sampling step and get the next step's guess count
    (speculative_generator.py:71-72); inactive ones (history_len 0) get 0 guesses."""
    device = _require_gpu(history_len, num_out, max_new_tokens, num_generated, steps, num_guesses)
    for name, t in (("history_len", history_len), ("num_out", num_out), ("max_new_tokens", max_new_tokens),
                    ("num_generated", num_generated), ("num_guesses", num_guesses)):
        _int32(t, name)
    _check(steps.dtype == torch.int64 and steps.is_contiguous(), "steps must be contiguous int64")
    n = history_len.numel()
    _check(all(t.numel() >= n for t in (num_out, max_new_tokens, num_generated, steps, num_guesses)),
           "per-sequence arrays shorter than history_len")
    _native.call("ne_advance_step_counts", _ptr(history_len), _ptr(num_out), _ptr(max_new_tokens),
                 _ptr(num_generated), _ptr(steps), _ptr(num_guesses), k, n, _stream(device))


def advance_and_propose(history: torch.Tensor, history_len: torch.Tensor, num_out: torch.Tensor,
                        max_new_tokens: torch.Tensor, num_generated: torch.Tensor, steps: torch.Tensor,
                        num_guesses: torch.Tensor, k: int, max_ngram: int, drafts: torch.Tensor,
                        num_drafts: torch.Tensor, min_ngram: int = 1) -> None:
    """:func:`advance_step_counts` then :func:`ngram_propose` with ``num_tokens =
    num_guesses`` in one launch (the same results): the tail of a verify step."""
    device = _require_gpu(history, history_len, num_out, max_new_tokens, num_generated, steps, num_guesses,
                          drafts, num_drafts)
    for name, t in (("history", history), ("history_len", history_len), ("num_out", num_out),
                    ("max_new_tokens", max_new_tokens), ("num_generated", num_generated),
                    ("num_guesses", num_guesses), ("drafts", drafts), ("num_drafts", num_drafts)):
        _int32(t, name)
    _check(steps.dtype == torch.int64 and steps.is_contiguous(), "steps must be contiguous int64")
    _check(history.dim() == 2 and drafts.dim() == 2 and drafts.is_contiguous(),
           "history [num_seqs, capacity], drafts [num_seqs, max_drafts]")
    n = history.shape[0]
    _check(all(t.numel() >= n for t in (history_len, num_out, max_new_tokens, num_generated, steps, num_guesses,
                                        num_drafts)) and drafts.shape[0] >= n,
           "per-sequence arrays shorter than the histories")
    _native.call("ne_advance_and_propose", _ptr(history), history.stride(0), _ptr(history_len), _ptr(num_out),
                 _ptr(max_new_tokens), _ptr(num_generated), _ptr(steps), _ptr(num_guesses), k, n, max_ngram,
                 min_ngram, drafts.shape[1], _ptr(drafts), _ptr(num_drafts), _stream(device))


def copy_bytes(src: torch.Tensor, dst: torch.Tensor) -> None:
    device = _require_gpu(src, dst)
    nbytes = src.numel() * src.element_size()
    _check(dst.numel() * dst.element_size() >= nbytes, "dst too small")
    _native.call("ne_copy_bytes", _ptr(src), _ptr(dst), nbytes, _stream(device))
