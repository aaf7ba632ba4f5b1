"""ctypes binding of libnanoengine_hip.so (the C ABI declared in include/nanoengine_hip.h).

The library is loaded lazily on first use.  There is no fallback: if the shared
object is missing or fails to load, every kernel call raises, so a GPU run can
never silently take another code path.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIBRARY_NAME = "libnanoengine_hip.so"
LIBRARY_PATH = Path(__file__).resolve().parent / LIBRARY_NAME
ABI_VERSION = 10

# status codes (nanoengine_hip.h)
NE_OK = 0
STATUS_NAMES = {-1: "NE_EINVAL", -2: "NE_EUNSUPPORTED", -3: "NE_ELAUNCH", -4: "NE_EWORKSPACE"}
NOALLOC_SCRATCH_BYTES = 64 << 20  # NE_NOALLOC_SCRATCH_BYTES

# dtype codes
DTYPE_BF16 = 0
DTYPE_FP16 = 1
DTYPE_FP32 = 2
DTYPE_INT8 = 3

EPILOGUE_STORE = 0
EPILOGUE_SWIGLU = 1

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t
_u64p = ctypes.c_void_p

# name -> (restype, argtypes); mirrors nanoengine_hip.h one to one
SIGNATURES: dict[str, tuple] = {
    "ne_abi_version": (ctypes.c_int, []),
    "ne_last_error": (ctypes.c_char_p, []),
    "ne_ngram_propose": (
        ctypes.c_int,
        [_vp, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp],
    ),
    "ne_kv_write": (ctypes.c_int, [_vp, _i32, _i64, _i32, _i32, _vp, _vp, _i32, _vp, _i32, _vp]),
    "ne_paged_attention_workspace_size": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "ne_paged_verify_attention": (
        ctypes.c_int,
        [
            _vp, _i64, _i64,  # q, strides
            _vp, _vp, _vp, _vp, _i32, _i32,  # caches, scales, dtypes
            _vp, _i32, _i32,  # block tables, stride, block size
            _vp, _vp, _vp,  # ctx_len, q_start, q_len
            _i32, _i32, _i32, _i32, _i32, _i32,  # seqs, heads, kv heads, head dim, max q, max ctx
            _f32,  # softmax scale
            _vp, _i64, _i64,  # out, strides
            _i32,  # split_len
            _vp, _sz, _vp,  # workspace, bytes, stream
        ],
    ),
    "ne_paged_verify_attention_planned": (ctypes.c_int, []),  # filled below: same as ne_paged_verify_attention
    "ne_paged_verify_attention_noalloc": (ctypes.c_int, []),  # filled below
    "ne_paged_attention_plan": (
        ctypes.c_int,
        [_vp, _i32, _i32, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _sz, _vp],
    ),
    "ne_paged_kv_stream_planned": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _sz, _vp],
    ),
    "ne_paged_kv_runs_plan": (
        ctypes.c_int,
        [_vp, _i32, _i32, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _sz, _vp],
    ),
    "ne_paged_kv_stream_runs": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _sz, _vp],
    ),
    "ne_w8a16_gemm": (
        ctypes.c_int,
        [_vp, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _i64, _i32, _vp],
    ),
    "ne_w8a16_gemm_splitk": (
        ctypes.c_int,
        [_vp, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp],
    ),
    "ne_lm_head_num_tiles": (_i32, [_i32]),
    "ne_lm_head": (ctypes.c_int, [_vp, _i64, _vp, _i32, _i32, _i32, _vp, _i64, _u64p, _vp]),
    "ne_rmsnorm": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32, _f32, _vp]),
    "ne_add_rmsnorm": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp]),
    "ne_splitk_add_rmsnorm": (ctypes.c_int, [_vp, _vp, _i32, _vp, _vp, _i32, _i32, _f32, _vp]),
    "ne_embed_rmsnorm": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _f32, _vp]),
    "ne_qk_norm_rope_kv_write": (
        ctypes.c_int,
        [
            _vp, _i32, _i32, _i32, _i32,  # qkv, rows, heads, kv heads, head dim
            _vp, _vp, _f32,  # norm weights, eps
            _vp, _vp, _i32, _vp,  # positions, rope table, its positions, slot mapping
            _vp, _vp, _vp, _vp, _i32, _i32,  # caches, scales, dtypes
            _vp, _vp,  # q_out, stream
        ],
    ),
    "ne_w8a16_qkv_norm_rope_kv": (
        ctypes.c_int,
        [
            _vp, _i64, _vp, _vp, _i32, _i32, _i32, _i32, _i32,  # x, ldx, w, scale, dtype, m, hq, hkv, k
            _vp, _vp, _f32,  # norm weights, eps
            _vp, _vp, _i32, _vp,  # positions, rope table, its positions, slot mapping
            _i32, _vp, _vp, _vp, _vp, _i32,  # kv dtype, caches, scales, scale dtype
            _vp, _vp,  # q_out, stream
        ],
    ),
    "ne_accept": (
        ctypes.c_int,
        [
            _vp, _i64, _u64p, _i32, _i32,  # logits, ld, partials, tiles, vocab
            _vp, _i32, _vp, _vp, _i32,  # drafts, max drafts, num drafts, row start, seqs
            _vp, _vp, _i32, _u64p, _u64p,  # temperatures, top-p, any sampled, seeds, steps
            _vp, _vp,  # out tokens, num out
            _vp, _i64, _vp, _vp,  # history, stride, history len, num cached
            _vp, _i32, _i64, _vp,  # draft rows, their dtype, ld, draft row start
            _vp,  # stream
        ],
    ),
    "ne_prepare_verify_step": (
        ctypes.c_int,
        [_vp, _i64, _vp, _vp, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
    ),
    "ne_advance_step_counts": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u64p, _vp, _i32, _i32, _vp]),
    "ne_advance_and_propose": (
        ctypes.c_int,
        [_vp, _i64, _vp, _vp, _vp, _vp, _u64p, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp],
    ),
    "ne_copy_bytes": (ctypes.c_int, [_vp, _vp, _sz, _vp]),
}
SIGNATURES["ne_paged_verify_attention_planned"] = SIGNATURES["ne_paged_verify_attention"]
# the allocation-free variant: (workspace, bytes) replaced by the caller's error-flag word
SIGNATURES["ne_paged_verify_attention_noalloc"] = (
    ctypes.c_int, SIGNATURES["ne_paged_verify_attention"][1][:-3] + [_vp, _vp])


class NativeError(RuntimeError):
    """A kernel entry point returned a non-zero status."""

    def __init__(self, function: str, status: int, message: str) -> None:
        self.function = function
        self.status = status
        super().__init__(f"{function} failed ({STATUS_NAMES.get(status, status)}): {message}")


_lock = threading.Lock()
_library: ctypes.CDLL | None = None


def library_path() -> Path:
    override = os.environ.get("NANOENGINE_HIP_LIBRARY")
    return Path(override) if override else LIBRARY_PATH


def load() -> ctypes.CDLL:
    """Load the library once; raise if it is missing or has another ABI version."""
    global _library
    with _lock:
        if _library is not None:
            return _library
        path = library_path()
        if not path.exists():
            raise RuntimeError(
                f"{path} is missing: build it with "
                "`python inference-engine-from-scratch_amd/build.py` (hipcc, gfx950)"
            )
        lib = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.ne_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
        _library = lib
        return lib


class LaunchTimer:
    """HIP events recorded on the launching stream around every call of one entry point."""

    def __init__(self) -> None:
        self.pairs: list = []

    def durations_ms(self) -> list[float]:
        return [start.elapsed_time(stop) for start, stop in self.pairs]


_timers: dict[str, LaunchTimer] = {}


def set_launch_timer(name: str, timer: LaunchTimer | None) -> None:
    """Time every launch of ``name`` (events on torch's current stream, which is the
    stream the wrappers launch on); ``None`` stops timing."""
    if timer is None:
        _timers.pop(name, None)
    else:
        _timers[name] = timer


def call(name: str, *args) -> None:
    """Call an entry point and raise NativeError on a non-zero status."""
    lib = load()
    timer = _timers.get(name)
    if timer is not None:
        import torch

        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        status = getattr(lib, name)(*args)
        stop.record()
        timer.pairs.append((start, stop))
    else:
        status = getattr(lib, name)(*args)
    if status != NE_OK:
        message = lib.ne_last_error().decode("utf-8", "replace")
        raise NativeError(name, status, message)


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
