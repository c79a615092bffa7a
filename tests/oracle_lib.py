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
# DH_ORACLE_LIB names another build of the checker (oracle/Makefile's `sanitized` target); unset, the in-tree one
ORACLE_SO = os.environ.get("DH_ORACLE_LIB") or os.path.join(ORACLE_DIR, "liboracle.so")

_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    srcs = [os.path.join(ORACLE_DIR, f) for f in ("oracle.c", "oracle_mixer.c", "Makefile")]
    if not os.path.exists(ORACLE_SO) or os.path.getmtime(ORACLE_SO) < max(os.path.getmtime(f) for f in srcs):
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
        "orc_softplus": (c_float, [c_float]),
        "orc_inv_freq": (None, [c_void_p]),
        "orc_conv_silu_l2": (None, [c_void_p, c_uint32, c_uint32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
        "orc_conv_state_update": (None, [c_void_p, c_uint32, c_uint32, c_void_p, c_void_p]),
        "orc_gated_delta": (None, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_void_p,
                                   c_void_p, c_uint32, c_void_p]),
        "orc_gated_rmsnorm_silu": (None, [c_void_p, c_void_p, c_uint32, c_void_p, c_uint32, c_void_p]),
        "orc_head_norm_rope": (None, [c_void_p, c_void_p, c_uint32, c_void_p]),
        "orc_attention": (None, [c_void_p, c_void_p, c_uint32, c_void_p, c_void_p, c_void_p, c_uint32, c_void_p]),
        "orc_embed_bf16": (None, [c_void_p, c_void_p, c_uint32, c_uint32, c_void_p]),
        "orc_normal_at": (c_float, [ctypes.c_uint64, ctypes.c_uint64, c_float, c_float]),
        "orc_fill_normal": (None, [c_void_p, ctypes.c_uint64, ctypes.c_uint64, c_float, c_float, c_uint32, c_int]),
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


# ---- the non-GEMM forward pieces (oracle_mixer.c; cpu_ref.rs:55-188)
NK, DK, NV, DV = 16, 128, 32, 128
KEY_DIM, VALUE_DIM, CONV_DIM = NK * DK, NV * DV, 2 * NK * DK + NV * DV
NQ, NKV, HEAD_DIM = 16, 4, 256
Q_DIM, KV_DIM = NQ * HEAD_DIM, NKV * HEAD_DIM


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def softplus(x: float) -> float:
    return float(load().orc_softplus(x))


def inv_freq() -> np.ndarray:
    out = np.empty(32, np.float32)
    load().orc_inv_freq(_p(out))
    return out


def conv_silu_l2(p: np.ndarray, t: int, prev: np.ndarray, w: np.ndarray):
    """cpu_ref::conv_silu_l2 over the first CONV_DIM columns of p [t, ldp] → (q [t,16,128], k, v [t,32,128])."""
    p, prev, w = _f32(p), _f32(prev), _f32(w)
    q = np.empty((t, NK, DK), np.float32)
    k = np.empty((t, NK, DK), np.float32)
    v = np.empty((t, NV, DV), np.float32)
    load().orc_conv_silu_l2(_p(p), p.shape[1], t, _p(prev), _p(w), _p(q), _p(k), _p(v))
    return q, k, v


def conv_state_update(p: np.ndarray, t: int, prev: np.ndarray) -> np.ndarray:
    p, prev = _f32(p), _f32(prev)
    out = np.empty((3, CONV_DIM), np.float32)
    load().orc_conv_state_update(_p(p), p.shape[1], t, _p(prev), _p(out))
    return out


def gated_delta(q, k, v, a, b, a_log, dt_bias, state, t: int):
    """cpu_ref::gated_delta; a, b are [t, ldab] (head h at column h). Returns (o [t,32,128], new state)."""
    q, k, v, a, b = _f32(q), _f32(k), _f32(v), _f32(a), _f32(b)
    assert a.shape == b.shape, "a and b share one row stride"
    st = _f32(state).copy()
    o = np.empty((t, NV, DV), np.float32)
    load().orc_gated_delta(_p(q), _p(k), _p(v), _p(a), _p(b), a.shape[1], _p(_f32(a_log)), _p(_f32(dt_bias)),
                           _p(st), t, _p(o))
    return o, st


def gated_rmsnorm_silu(o, z, w, t: int) -> np.ndarray:
    o, z, w = _f32(o), _f32(z), _f32(w)
    y = np.empty((t, VALUE_DIM), np.float32)
    load().orc_gated_rmsnorm_silu(_p(o), _p(z), z.shape[1], _p(w), t, _p(y))
    return y


def head_norm_rope(seg, w, pos: int) -> np.ndarray:
    seg, w = _f32(seg), _f32(w)
    out = np.empty(HEAD_DIM, np.float32)
    load().orc_head_norm_rope(_p(seg), _p(w), pos, _p(out))
    return out


def attention(q, qpos, kc, vc, gate) -> np.ndarray:
    """cpu_ref::attention: q [rows,16,256], kc/vc [npos,4,256], gate [rows, ldg] → [rows, 4096]."""
    q, kc, vc, gate = _f32(q), _f32(kc), _f32(vc), _f32(gate)
    qpos = np.ascontiguousarray(qpos, dtype=np.uint32)
    rows = len(qpos)
    out = np.empty((rows, Q_DIM), np.float32)
    load().orc_attention(_p(q), _p(qpos), rows, _p(kc), _p(vc), _p(gate), gate.shape[1], _p(out))
    return out


def embed_bf16(ids, table_bits) -> np.ndarray:
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    table_bits = np.ascontiguousarray(table_bits, dtype=np.uint16)
    out = np.empty((len(ids), table_bits.shape[1]), np.float32)
    load().orc_embed_bf16(_p(ids), _p(table_bits), len(ids), table_bits.shape[1], _p(out))
    return out


def fill_normal(n: int, seed: int, mean: float, sd: float, dtype: int, threads: int = 0) -> np.ndarray:
    """The library's random-init stream restated (orc_fill_normal): n values ~ N(mean, sd) as fp16 (dtype 0),
    bf16 bits as uint16 (1) or fp32 (2); element i depends only on (seed, i)."""
    out = np.empty(n, dtype={0: np.float16, 1: np.uint16, 2: np.float32}[dtype])
    load().orc_fill_normal(_p(out), n, seed & (2**64 - 1), mean, sd, dtype, threads)
    return out
