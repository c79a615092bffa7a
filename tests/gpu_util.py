"""Helpers shared by the GPU parity tests: device copies and parity checks."""

from __future__ import annotations

import numpy as np

import oracle_lib as orc
from decide_amd.hip import DeviceArray, synchronize

# BASELINE tolerance for one GEMM: relative Frobenius error against the fp32
# CPU computation of the same inputs.
GEMM_REL_FROB = 1e-3


def to_dev(a: np.ndarray) -> DeviceArray:
    return DeviceArray.from_numpy(np.ascontiguousarray(a))


def to_host(t: DeviceArray) -> np.ndarray:
    return t.numpy()


def empty(shape, dtype) -> DeviceArray:
    return DeviceArray(shape, dtype)


def full(shape, dtype, value) -> DeviceArray:
    return DeviceArray.full(shape, dtype, value)


def sync() -> None:
    synchronize()


def sample_rows(m: int, count: int = 48, seed: int = 0) -> np.ndarray:
    """Rows to check at full size: the first and last 16-row fragments' edges, the last row, random others."""
    fixed = {0, 1, 15, 16, min(m - 1, 31), m - 1, max(0, m - 2), max(0, m - 17), m // 2}
    rng = np.random.default_rng(seed)
    extra = rng.choice(m, size=min(m, count), replace=False)
    rows = sorted({r for r in fixed if 0 <= r < m} | set(int(r) for r in extra))
    return np.array(rows, dtype=np.uint32)


def check_gemm(name: str, got: np.ndarray, want: np.ndarray, rel: float = GEMM_REL_FROB) -> float:
    got = np.asarray(got, dtype=np.float32)
    want = np.asarray(want, dtype=np.float32)
    assert got.shape == want.shape, f"{name}: shape {got.shape} vs {want.shape}"
    assert np.isfinite(got).all(), f"{name}: non-finite output"
    e = orc.rel_frobenius(got, want)
    assert e <= rel, f"{name}: relative Frobenius error {e:.3e} > {rel:.1e}"
    return e


def swiglu_f16(y_f32: np.ndarray) -> np.ndarray:
    """The oracle's SwiGLU of f32 GEMM rows, rounded to fp16 (decide's `mlp` buffer is fp16)."""
    return orc.f16_round(orc.swiglu_interleaved(y_f32))
