"""Seeded synthetic inputs for the GEMM path, on the host.

decide's tests draw uniform inputs from ``StdRng`` (testutil.rs:4-8); the
BASELINE shapes ask for Gaussians instead (X ~ N(0, 1), W ~ N(0, 0.02)), so
this module defines its own portable generator (the library's device fills,
``dh_fill_normal`` and ``dh_model_init_random``, use the same stream):

* uniform u64 stream: ``mix64(seed + φ·(i + 1))`` with splitmix64's finaliser
  and φ = 0x9e3779b97f4a7c15 (all arithmetic mod 2⁶⁴);
* pair p of normals from u64s 2p and 2p + 1: 24-bit uniforms in (0, 1),
  Box–Muller, cos branch for even elements and sin branch for odd ones.

This host version computes Box–Muller in float64 with numpy's log/cos/sin. The
device computes it in fp32 from IEEE-rounded +, −, ×, ÷ and sqrt only
(``decide_amd/csrc/normal_gen.h``), so the two agree to about 1e-6 (1e-4 where
u₁'s fp32 rounding matters, next to 1), not bit for bit: tests that compare
the GPU with the oracle feed both the same fp16 arrays, or rebuild device
fills with the oracle's bit-exact restatement of the device steps.
"""

from __future__ import annotations

import numpy as np

PHI = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def mix64(z: np.ndarray) -> np.ndarray:
    z = z.astype(np.uint64, copy=True)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def uniform24(seed: int, idx: np.ndarray) -> np.ndarray:
    """24-bit uniforms in (0, 1) for stream positions ``idx``."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + PHI * (idx.astype(np.uint64) + np.uint64(1))
    return ((mix64(z) >> np.uint64(40)).astype(np.float64) + 0.5) / 16777216.0


def normal(seed: int, n: int, std: float = 1.0, chunk: int = 1 << 22) -> np.ndarray:
    """n float64 values ~ N(0, std) (element i depends only on (seed, i))."""
    out = np.empty(n, dtype=np.float64)
    for s in range(0, n, chunk):
        i = np.arange(s, min(n, s + chunk), dtype=np.uint64)
        p = i >> np.uint64(1)
        u1 = uniform24(seed, np.uint64(2) * p)
        u2 = uniform24(seed, np.uint64(2) * p + np.uint64(1))
        rad = np.sqrt(-2.0 * np.log(u1))
        ang = 2.0 * np.pi * u2
        z = np.where((i & np.uint64(1)) == 0, rad * np.cos(ang), rad * np.sin(ang))
        out[s:s + len(i)] = z * std
    return out


def normal_f16(seed: int, shape, std: float = 1.0) -> np.ndarray:
    """fp16 array of ``shape`` ~ N(0, std), rounded to nearest even."""
    n = int(np.prod(shape))
    return normal(seed, n, std).astype(np.float16).reshape(shape)


def normal_f32(seed: int, shape, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    return normal(seed, n, std).astype(np.float32).reshape(shape)


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """float32 → bf16 bit patterns (uint16), round to nearest even."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    return ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def uniform_ids(seed: int, n: int, vocab: int) -> np.ndarray:
    """n token ids uniform over [0, vocab) (u32)."""
    i = np.arange(n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + PHI * (i + np.uint64(1))
    return (mix64(z) % np.uint64(vocab)).astype(np.uint32)


# Tensor seeds: 0xDEC1DE xor a per-tensor id.
SEED_BASE = 0xDEC1DE


def seed_for(tensor_id: int) -> int:
    return SEED_BASE ^ tensor_id
