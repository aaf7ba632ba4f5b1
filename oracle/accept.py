"""Acceptance under the library's explicit-uniform contract (test infrastructure only).

Greedy (ne/engine/speculative/verifier.py:27-60 with one-hot p and q): keep guesses
while they equal the row argmax (first index on ties, numpy/torch order), then
append the argmax of the first mismatching row or of the bonus row.

Sampled: the C oracle in ``csrc/accept_oracle.c`` (built by ``oracle/Makefile``)
restates the contract documented in the HIP kernel; this module loads it.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "_build" / "libaccept_oracle.so"

_lib: ctypes.CDLL | None = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        handle = ctypes.CDLL(str(LIB_PATH))
        handle.oracle_cephes_exp.restype = ctypes.c_float
        handle.oracle_cephes_exp.argtypes = [ctypes.c_float]
        handle.oracle_uniform.restype = ctypes.c_float
        handle.oracle_uniform.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int]
        handle.oracle_philox4x32_10.restype = None
        handle.oracle_philox4x32_10.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        handle.oracle_accept_sampled_draft.restype = ctypes.c_int
        handle.oracle_accept_sampled_draft.argtypes = [
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p,
            ctypes.c_int, ctypes.c_float, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p,
        ]
        handle.oracle_accept_sampled_v2.restype = ctypes.c_int
        handle.oracle_accept_sampled_v2.argtypes = [
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_float,
            ctypes.c_float, ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint64,
            ctypes.c_void_p, ctypes.c_void_p,
        ]
        handle.oracle_top_p_kept.restype = ctypes.c_float
        handle.oracle_top_p_kept.argtypes = [
            ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p,
        ]
        handle.oracle_accept_sampled.restype = ctypes.c_int
        handle.oracle_accept_sampled.argtypes = [
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
            ctypes.c_float, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p,
        ]
        handle.oracle_exp3.restype = ctypes.c_float
        handle.oracle_exp3.argtypes = [ctypes.c_float]
        handle.oracle_v3_scratch_bytes.restype = ctypes.c_size_t
        handle.oracle_v3_scratch_bytes.argtypes = []
        handle.oracle_accept_sampled_v3.restype = ctypes.c_int
        handle.oracle_accept_sampled_v3.argtypes = [
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_float,
            ctypes.c_float, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p,
        ]
        handle.oracle_v3_row.restype = ctypes.c_uint64
        handle.oracle_v3_row.argtypes = [
            ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ]
        handle.oracle_v3_weight.restype = ctypes.c_uint32
        handle.oracle_v3_weight.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_uint32,
                                            ctypes.c_void_p]
        _lib = handle
    return _lib


def _v3_scratch() -> np.ndarray:
    return np.zeros(int(lib().oracle_v3_scratch_bytes()) // 8 + 1, dtype=np.uint64)


def exp3(x: float) -> float:
    """The integer-mass contract's exp (Cephes' reduction and polynomial, one fmaf per step)."""
    return float(lib().oracle_exp3(ctypes.c_float(x)))


def cephes_exp(x: float) -> float:
    return float(lib().oracle_cephes_exp(ctypes.c_float(x)))


def philox4x32_10(counter: list[int], key: list[int]) -> list[int]:
    ctr = (ctypes.c_uint32 * 4)(*counter)
    k = (ctypes.c_uint32 * 2)(*key)
    lib().oracle_philox4x32_10(ctr, k)
    return list(ctr)


def uniform(seed: int, step: int, j: int) -> float:
    return float(lib().oracle_uniform(seed, step, j))


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """float32 values that are exact bf16 -> their 16-bit patterns."""
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    return (bits >> 16).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def greedy_accept(rows: np.ndarray, drafts: list[int]) -> list[int]:
    """``rows [g+1, V]`` float logits (already bf16-rounded) -> kept guesses + target token."""
    targets = np.argmax(rows, axis=-1)
    kept: list[int] = []
    for i, guess in enumerate(drafts):
        if guess != int(targets[i]):
            return [*kept, int(targets[i])]
        kept.append(guess)
    return [*kept, int(targets[len(drafts)])]


def sampled_accept(row_bits: np.ndarray, drafts: list[int], temperature: float, seed: int,
                   step: int) -> list[int]:
    """``row_bits [g+1, V]`` uint16 bf16 patterns -> kept guesses + drawn token (C oracle)."""
    rows = np.ascontiguousarray(row_bits, dtype=np.uint16)
    g = len(drafts)
    assert rows.shape[0] == g + 1
    vocab = rows.shape[1]
    d = np.ascontiguousarray(np.asarray(drafts, dtype=np.int32))
    out = np.zeros(g + 1, dtype=np.int32)
    scratch = np.zeros(vocab, dtype=np.float32)
    n = lib().oracle_accept_sampled(
        rows.ctypes.data, vocab, vocab, d.ctypes.data if g else None, g, ctypes.c_float(temperature),
        seed, step, out.ctypes.data, scratch.ctypes.data,
    )
    return out[:n].tolist()


def sampled_accept_draft(row_bits: np.ndarray, draft_bits: np.ndarray, drafts: list[int], temperature: float,
                         seed: int, step: int) -> list[int]:
    """Target rows ``[g+1, V]`` and the draft model's rows ``[g, V]`` (uint16 bf16 patterns)
    -> kept guesses + drawn token (C oracle, verifier.py:36-56 with draft distributions)."""
    rows = np.ascontiguousarray(row_bits, dtype=np.uint16)
    drows = np.ascontiguousarray(draft_bits, dtype=np.uint16)
    g = len(drafts)
    assert rows.shape[0] == g + 1 and drows.shape[0] >= g
    vocab = rows.shape[1]
    d = np.ascontiguousarray(np.asarray(drafts, dtype=np.int32))
    out = np.zeros(g + 1, dtype=np.int32)
    scratch = np.zeros(3 * vocab, dtype=np.float32)
    n = lib().oracle_accept_sampled_draft(
        rows.ctypes.data, vocab, drows.ctypes.data, vocab, vocab, d.ctypes.data if g else None, g,
        ctypes.c_float(temperature), seed, step, out.ctypes.data, scratch.ctypes.data,
    )
    return out[:n].tolist()


def sampled_accept_v2(row_bits: np.ndarray, drafts: list[int], temperature: float, top_p: float, seed: int,
                      step: int, draft_bits: np.ndarray | None = None,
                      draft_probs: np.ndarray | None = None) -> list[int]:
    """The contract with top-p and an optional draft distribution per guess (C oracle):
    ``row_bits [g+1, V]`` target bf16 patterns; ``draft_bits [g, V]`` the draft model's
    bf16 logits (its distribution: the same top-p softmax) or ``draft_probs [g, V]``
    fp32 probabilities used as given; neither: one-hot (n-gram) guesses."""
    rows = np.ascontiguousarray(row_bits, dtype=np.uint16)
    g = len(drafts)
    assert rows.shape[0] == g + 1
    vocab = rows.shape[1]
    d = np.ascontiguousarray(np.asarray(drafts, dtype=np.int32))
    out = np.zeros(g + 1, dtype=np.int32)
    scratch = np.zeros(4 * vocab + vocab // 2 + 1, dtype=np.float32)
    if draft_bits is not None:
        dr = np.ascontiguousarray(draft_bits, dtype=np.uint16)
        is_probs = 0
    elif draft_probs is not None:
        dr = np.ascontiguousarray(draft_probs, dtype=np.float32)
        is_probs = 1
    else:
        dr, is_probs = None, 0
    assert dr is None or (dr.shape[0] >= g and dr.shape[1] == vocab)
    n = lib().oracle_accept_sampled_v2(
        rows.ctypes.data, vocab, vocab, d.ctypes.data if g else None, g, ctypes.c_float(temperature),
        ctypes.c_float(top_p), None if dr is None else dr.ctypes.data, is_probs, vocab, seed, step,
        out.ctypes.data, scratch.ctypes.data,
    )
    return out[:n].tolist()


def top_p_kept(row_bits: np.ndarray, temperature: float, top_p: float) -> tuple[np.ndarray, float, int, int]:
    """Kept flags of one row under the contract's top-p, with K, the threshold key and
    the count of threshold ties kept."""
    row = np.ascontiguousarray(row_bits, dtype=np.uint16)
    vocab = row.shape[0]
    kept = np.zeros(vocab, dtype=np.uint8)
    w = np.zeros(vocab, dtype=np.float32)
    tau = ctypes.c_uint32(0)
    m = ctypes.c_int(0)
    k = lib().oracle_top_p_kept(row.ctypes.data, vocab, ctypes.c_float(temperature), ctypes.c_float(top_p),
                                kept.ctypes.data, w.ctypes.data, ctypes.byref(tau), ctypes.byref(m))
    return kept.astype(bool), float(k), int(tau.value), int(m.value)


def sampled_accept_v3(row_bits: np.ndarray, drafts: list[int], temperature: float, top_p: float, seed: int,
                      step: int) -> list[int]:
    """The integer-mass contract for one-hot (n-gram) guesses (C oracle): ``row_bits
    [g+1, V]`` bf16 patterns -> kept guesses + drawn token."""
    rows = np.ascontiguousarray(row_bits, dtype=np.uint16)
    g = len(drafts)
    assert rows.shape[0] == g + 1
    vocab = rows.shape[1]
    d = np.ascontiguousarray(np.asarray(drafts, dtype=np.int32))
    out = np.zeros(g + 1, dtype=np.int32)
    scratch = _v3_scratch()
    n = lib().oracle_accept_sampled_v3(
        rows.ctypes.data, vocab, vocab, d.ctypes.data if g else None, g, ctypes.c_float(temperature),
        ctypes.c_float(top_p), seed, step, out.ctypes.data, scratch.ctypes.data,
    )
    return out[:n].tolist()


def v3_row(row_bits: np.ndarray, temperature: float, top_p: float) -> tuple[np.ndarray, int, int, int, int]:
    """(kept flags, K, Z, tau, m) of one row under the integer-mass contract."""
    row = np.ascontiguousarray(row_bits, dtype=np.uint16)
    vocab = row.shape[0]
    kept = np.zeros(vocab, dtype=np.uint8)
    z, tau, m = ctypes.c_uint64(0), ctypes.c_uint32(0), ctypes.c_uint32(0)
    scratch = _v3_scratch()  # held by name: the C call writes into it
    k = lib().oracle_v3_row(row.ctypes.data, vocab, ctypes.c_float(temperature), ctypes.c_float(top_p),
                            kept.ctypes.data, ctypes.byref(z), ctypes.byref(tau), ctypes.byref(m),
                            scratch.ctypes.data)
    return kept.astype(bool), int(k), int(z.value), int(tau.value), int(m.value)


def v3_weight(row_bits: np.ndarray, temperature: float, key: int) -> int:
    """E(key) of a row: the integer weight of a token whose bf16 order key is ``key``."""
    row = np.ascontiguousarray(row_bits, dtype=np.uint16)
    scratch = _v3_scratch()  # held by name: the C call writes into it
    return int(lib().oracle_v3_weight(row.ctypes.data, row.shape[0], ctypes.c_float(temperature), key,
                                      scratch.ctypes.data))


def key16(bits: np.ndarray) -> np.ndarray:
    """16-bit order keys of bf16 bit patterns (larger value, larger key; -0 as +0)."""
    b = np.asarray(bits, dtype=np.uint32)
    b = np.where((b & 0x7FFF) == 0, 0, b)
    return np.where(b & 0x8000, (~b) & 0xFFFF, b | 0x8000).astype(np.uint32)
