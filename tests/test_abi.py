"""The C-ABI library (CPU only): it loads, exports every entry point that
include/nanoengine_hip.h declares, and its host-side argument checks reject bad
calls before any launch.  No kernel is launched here."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from nanoengine_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "nanoengine_hip.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ne_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _native.library_path().exists():
        pytest.skip("libnanoengine_hip.so is not built (run __graft_entry__.build())")
    return _native.load()


def test_header_and_binding_declare_the_same_entry_points():
    assert declared_functions() == sorted(_native.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing
    assert lib.ne_abi_version() == _native.ABI_VERSION


def test_host_checks_reject_bad_arguments_without_launching(lib):
    null = ctypes.c_void_p(0)
    rc = lib.ne_ngram_propose(null, 8, null, null, -1, 3, 1, 4, null, null, null)
    assert rc == -1 and b"num_seqs" in lib.ne_last_error()
    rc = lib.ne_ngram_propose(null, 8, null, null, 2, 3, 1, 4, null, null, null)
    assert rc == -1 and b"null" in lib.ne_last_error()
    rc = lib.ne_ngram_propose(ctypes.c_void_p(16), 8, ctypes.c_void_p(16), ctypes.c_void_p(16), 2, 17, 1, 4,
                              ctypes.c_void_p(16), ctypes.c_void_p(16), null)
    assert rc == -2  # max_ngram above the kernel's limit: unsupported, nothing launched
    # attention: head_dim other than 128 is unsupported
    p = ctypes.c_void_p(256)
    rc = lib.ne_paged_verify_attention(p, 2048, 128, p, p, p, p, 3, 0, p, 8, 16, p, p, p, 4, 16, 8, 64,
                                       5, 100, 0.125, p, 2048, 128, 0, p, 1 << 20, null)
    assert rc == -2 and b"head_dim" in lib.ne_last_error()
    # W8A16 GEMM: k must be a multiple of 128
    rc = lib.ne_w8a16_gemm(p, 1000, p, p, 0, 320, 1024, 1000, p, 1024, 0, null)
    assert rc == -2
    rc = lib.ne_accept(null, 0, p, 10, 100, p, 0, p, p, 2, null, null, 0, null, null, p, p, null, 0, null, null,
                       null, 0, 0, null, null)
    assert rc == -1 and b"max_drafts" in lib.ne_last_error()
    # sampled sequences need per-sequence temperatures and logits
    rc = lib.ne_accept(null, 0, p, 10, 100, p, 4, p, p, 2, null, null, 1, p, p, p, p, null, 0, null, null,
                       null, 0, 0, null, null)
    assert rc == -1 and b"temperature" in lib.ne_last_error()
    # draft rows must be bf16 logits or fp32 probabilities
    rc = lib.ne_accept(p, 100, null, 0, 100, p, 4, p, p, 2, p, null, 1, p, p, p, p, null, 0, null, null,
                       p, 3, 100, p, null)
    assert rc == -1 and b"draft rows" in lib.ne_last_error()
    # next-step counters: sizes and pointers are checked before any launch
    rc = lib.ne_advance_step_counts(p, p, p, p, p, p, -1, 4, null)
    assert rc == -1 and b"bad sizes" in lib.ne_last_error()
    rc = lib.ne_advance_step_counts(p, null, p, p, p, p, 4, 4, null)
    assert rc == -1 and b"null" in lib.ne_last_error()
    assert lib.ne_advance_step_counts(null, null, null, null, null, null, 4, 0, null) == 0  # nothing to do


def test_workspace_and_tile_queries(lib):
    assert lib.ne_lm_head_num_tiles(151936) == 2 * 256  # two halves of 256 work-groups' ranges
    assert lib.ne_lm_head_num_tiles(4096) == 2 * (4096 // 64)
    assert lib.ne_paged_attention_workspace_size(0, 16, 8, 5, 1024, 0) == 0
    assert lib.ne_paged_attention_workspace_size(64, 16, 7, 5, 1024, 0) == 0  # 16 % 7 != 0
    one_split = lib.ne_paged_attention_workspace_size(64, 16, 8, 5, 256, 256)
    four_splits = lib.ne_paged_attention_workspace_size(64, 16, 8, 5, 1024, 256)
    # no partial sums: the error flag, the int8 work plan's 65 prefix entries, and the
    # precomputed plan's 64 work items (8 ints) and slot lists (512 ints)
    assert one_split == 256 + 512 + 64 * 8 * 4 + 64 * 512 * 4
    # partials: units x splits x 16 rows x (128 + 2) fp32
    assert four_splits >= 256 + 64 * 8 * 4 * 16 * 130 * 4


def test_plan_entry_points_refuse_shapes_off_the_planned_path(lib):
    """The precomputed plan serves 8 KV heads and <= 32 query rows per KV head (int8 with
    2-byte scales for the attention call); anything else is refused before a launch."""
    p = ctypes.c_void_p(256)
    null = ctypes.c_void_p(0)
    ws = ctypes.c_size_t(1 << 30)
    # 4 KV heads
    rc = lib.ne_paged_attention_plan(p, 64, 16, p, p, p, 8, 16, 4, 5, 1024, 0, p, ws, null)
    assert rc == -2 and b"8 KV heads" in lib.ne_last_error()
    # 2 q heads per KV head x 17 queries = 34 rows per KV head
    rc = lib.ne_paged_attention_plan(p, 64, 16, p, p, p, 8, 16, 8, 17, 1024, 0, p, ws, null)
    assert rc == -2
    # int8 cache with fp32 scales on the planned attention call (bf16 and 2-byte scales only)
    rc = lib.ne_paged_verify_attention_planned(p, 2048, 128, p, p, p, p, 3, 2, p, 64, 16, p, p, p,
                                                8, 16, 8, 128, 5, 1024, 0.088, p, 2048, 128, 0, p, ws, null)
    assert rc == -2 and b"planned path" in lib.ne_last_error()
    # the K/V stream (measurement) follows the planned path's shapes: 4 KV heads refused
    rc = lib.ne_paged_kv_stream_planned(p, p, null, null, 0, 0, 8, 16, 4, 5, 1024, 0, p, ws, null)
    assert rc == -2 and b"planned path" in lib.ne_last_error()
    # a workspace smaller than the plan's layout
    rc = lib.ne_paged_attention_plan(p, 64, 16, p, p, p, 8, 16, 8, 5, 1024, 0, p, ctypes.c_size_t(64), null)
    assert rc == -1 and b"workspace" in lib.ne_last_error()
    # the whole-slot runs (measurement): the same shapes, block sizes and workspace
    rc = lib.ne_paged_kv_runs_plan(p, 64, 16, p, 8, 16, 4, 5, 1024, p, ws, null)
    assert rc == -2 and b"8 KV heads" in lib.ne_last_error()
    rc = lib.ne_paged_kv_runs_plan(p, 64, 24, p, 8, 16, 8, 5, 1024, p, ws, null)
    assert rc == -2 and b"block_size" in lib.ne_last_error()
    rc = lib.ne_paged_kv_runs_plan(p, 64, 16, p, 8, 16, 8, 5, 1024, p, ctypes.c_size_t(64), null)
    assert rc == -1 and b"workspace" in lib.ne_last_error()
    rc = lib.ne_paged_kv_stream_runs(p, p, null, null, 0, 0, 8, 16, 4, 5, 1024, p, ws, null)
    assert rc == -2 and b"planned path" in lib.ne_last_error()
