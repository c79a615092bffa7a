"""ctypes binding of oracle/liboracle.so (the CPU checker; test infrastructure).

Builds the oracle on first use if it is missing (gcc is on both the build
container and the GPU box). Only tests, the smoke check and bench.py's
cpu_baseline leg use this module.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_double, c_float, c_int, c_int64, c_size_t, c_uint16, c_uint32, c_void_p

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "liboracle.so")

_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    src = os.path.join(ORACLE_DIR, "oracle.c")
    if not os.path.exists(ORACLE_SO) or os.path.getmtime(ORACLE_SO) < os.path.getmtime(src):
        subprocess.run(["make", "-C", ORACLE_DIR], check=True, capture_output=True)
    lib = ctypes.CDLL(ORACLE_SO)
    sig = {
        "orc_f16_to_f32": (c_float, [c_uint16]),
        "orc_f16_from_f32": (c_uint16, [c_float]),
        "orc_f16_round": (c_float, [c_float]),
        "orc_bf16_from_f32": (c_uint16, [c_float]),
        "orc_bf16_to_f32": (c_float, [c_uint16]),
        "orc_f16_array_to_f32": (None, [c_void_p, c_void_p, c_size_t]),
        "orc_f32_array_to_f16": (None, [c_void_p, c_void_p, c_size_t]),
        "orc_silu": (c_float, [c_float]),
        "orc_gemm_nt_f16": (
            None,
            [c_void_p, c_uint32, c_void_p, c_uint32, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32, c_void_p,
             c_int],
        ),
        "orc_gemm_nt": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32]),
        "orc_swiglu_interleaved": (None, [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32]),
        "orc_rmsnorm": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_int, c_float]),
        "orc_final_head": (
            None,
            [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_float],
        ),
        "orc_interleave_gate_up": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32]),
        "orc_deinterleave_q_gate": (None, [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32]),
        "orc_gemm_f32_fast": (None, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_int]),
        "orc_rel_frobenius": (c_double, [c_void_p, c_void_p, c_size_t]),
        "orc_assert_close": (c_int64, [c_void_p, c_void_p, c_size_t, c_float, c_float]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def gemm_nt_f16(x: np.ndarray, w: np.ndarray, rows: np.ndarray | None = None, threads: int = 0) -> np.ndarray:
    """cpu_ref::gemm_nt on fp16 inputs: y[i][j] = Σ_k x[i][k]·w[j][k] (f64 sum in k order) → f32.

    ``x`` fp16 [M, K], ``w`` fp16 [N, K]; ``rows`` selects rows of x."""
    x = np.ascontiguousarray(x, dtype=np.float16)
    w = np.ascontiguousarray(w, dtype=np.float16)
    m, k = x.shape
    n = w.shape[0]
    assert w.shape[1] == k
    r = None if rows is None else np.ascontiguousarray(rows, dtype=np.uint32)
    mo = m if r is None else len(r)
    y = np.empty((mo, n), dtype=np.float32)
    load().orc_gemm_nt_f16(_p(x.view(np.uint16)), k, _p(w.view(np.uint16)), k, _p(y), n, mo, n, k,
                           None if r is None else _p(r), threads)
    return y


def gemm_nt(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    load().orc_gemm_nt(_p(x), _p(w), _p(y), m, n, k)
    return y


def swiglu_interleaved(y: np.ndarray, blk: int = 16) -> np.ndarray:
    y = np.ascontiguousarray(y, dtype=np.float32)
    m, n2 = y.shape
    out = np.empty((m, n2 // 2), dtype=np.float32)
    load().orc_swiglu_interleaved(_p(y), _p(out), m, n2, blk)
    return out


def rmsnorm(x: np.ndarray, w: np.ndarray, add_one: bool, eps: float = 1e-6) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, h = x.shape
    out = np.empty_like(x)
    load().orc_rmsnorm(_p(x), _p(w), _p(out), rows, h, 1 if add_one else 0, eps)
    return out


def final_head(x: np.ndarray, w: np.ndarray, table_bits: np.ndarray, cand: np.ndarray, ncand: np.ndarray,
               max_cand: int, eps: float = 1e-6) -> np.ndarray:
    """cpu_ref::final_head; returns logits [rows, max_cand] with NaN where not written."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    table_bits = np.ascontiguousarray(table_bits, dtype=np.uint16)
    cand = np.ascontiguousarray(cand, dtype=np.uint32)
    ncand = np.ascontiguousarray(ncand, dtype=np.uint32)
    rows, hidden = x.shape
    logits = np.full((rows, max_cand), np.nan, dtype=np.float32)
    load().orc_final_head(_p(x), _p(w), _p(table_bits), _p(cand), _p(ncand), _p(logits), rows, hidden, max_cand,
                          eps)
    return logits


def interleave_gate_up(gate: np.ndarray, up: np.ndarray, block: int = 16) -> np.ndarray:
    gate = np.ascontiguousarray(gate, dtype=np.uint16)
    up = np.ascontiguousarray(up, dtype=np.uint16)
    n, k = gate.shape
    out = np.empty((2 * n, k), dtype=np.uint16)
    load().orc_interleave_gate_up(_p(gate), _p(up), _p(out), n, k, block)
    return out


def deinterleave_q_gate(src: np.ndarray, heads: int, head_dim: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint16)
    k = src.shape[1]
    out = np.empty_like(src)
    load().orc_deinterleave_q_gate(_p(src), _p(out), heads, head_dim, k)
    return out


def gemm_f32_fast(x: np.ndarray, w: np.ndarray, threads: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), dtype=np.float32)
    load().orc_gemm_f32_fast(_p(x), _p(w), _p(y), m, n, k, threads)
    return y


def rel_frobenius(got: np.ndarray, want: np.ndarray) -> float:
    got = np.ascontiguousarray(got, dtype=np.float32)
    want = np.ascontiguousarray(want, dtype=np.float32)
    assert got.shape == want.shape
    return float(load().orc_rel_frobenius(_p(got), _p(want), got.size))


def assert_close(name: str, got: np.ndarray, want: np.ndarray, atol: float, rtol: float) -> None:
    """testutil::assert_close: |g − w| <= atol + rtol·|w| element-wise; NaN fails."""
    got = np.ascontiguousarray(got, dtype=np.float32)
    want = np.ascontiguousarray(want, dtype=np.float32)
    assert got.shape == want.shape, f"{name}: shape {got.shape} vs {want.shape}"
    i = load().orc_assert_close(_p(got), _p(want), got.size, atol, rtol)
    if i >= 0:
        raise AssertionError(f"{name}: element {i}: got {got.flat[i]} want {want.flat[i]} (atol {atol}, rtol {rtol})")


def f16_round(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    bits = np.empty(a.shape, dtype=np.uint16)
    load().orc_f32_array_to_f16(_p(a), _p(bits), a.size)
    out = np.empty(a.shape, dtype=np.float32)
    load().orc_f16_array_to_f32(_p(bits), _p(out), a.size)
    return out
