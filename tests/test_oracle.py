"""Pins the CPU oracle (oracle/oracle.c) independently of itself.

Every oracle function is checked against something it does not compute:
decide's own known-answer tests (cpu_ref.rs:204-221), numpy's IEEE float16
and float64 routines, closed forms and the committed golden fixtures
(tests/golden/, written by tests/golden/make_golden.py with numpy float64).
Each check is chosen so a plausible mistake fails it: a transposed operand,
a dropped term, a wrong SwiGLU block pairing, a missing (1 + w).
"""

import json
import os

import numpy as np
import pytest

import oracle_lib as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def silu64(x):
    return x / (1.0 + np.exp(-x))


# ---------------------------------------------------------------- rounding
def test_f16_decode_matches_numpy_for_every_bit_pattern():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    lib = orc.load()
    got = np.empty(65536, dtype=np.float32)
    lib.orc_f16_array_to_f32(bits.ctypes.data, got.ctypes.data, 65536)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_encode_matches_numpy_rne():
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 200000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, 1e9, -1e9, 2.0**-24, 2.0**-25, 2.0**-25 * 1.0001,
                  2.0**-14, 2.0**-14 * (1 - 2**-11), 3 * 2.0**-25, np.inf, -np.inf], dtype=np.float32),
    ])
    # every halfway point between consecutive halves (ties go to even)
    h = np.arange(0x7BFF, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    vals = np.ascontiguousarray(np.concatenate([vals, mids, -mids]), dtype=np.float32)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.empty(vals.shape, dtype=np.uint16)
    orc.load().orc_f32_array_to_f16(vals.ctypes.data, got.ctypes.data, vals.size)
    assert np.array_equal(got, want)


def test_bf16_rounding_closed_form():
    lib = orc.load()
    # 1 + 2^-8 is exactly halfway between bf16 1.0 and 1 + 2^-7: ties to even → 1.0
    assert lib.orc_bf16_from_f32(np.float32(1 + 2.0**-8)) == 0x3F80
    # 1 + 3·2^-8 is halfway between 1 + 2^-7 (odd mantissa 1) and 1 + 2^-6: → 1 + 2^-6
    assert lib.orc_bf16_from_f32(np.float32(1 + 3 * 2.0**-8)) == 0x3F82
    assert lib.orc_bf16_to_f32(0x4049) == pytest.approx(3.140625)
    assert lib.orc_bf16_to_f32(0xC000) == -2.0


# ---------------------------------------------------------------- GEMM
def test_gemm_known_answer_tiny():
    # x = [[1, 2], [3, 4]], w rows [1, 0], [0, 1], [1, 1]:  y = x · wᵀ
    x = np.array([[1, 2], [3, 4]], dtype=np.float32)
    w = np.array([[1, 0], [0, 1], [1, 1]], dtype=np.float32)
    np.testing.assert_array_equal(orc.gemm_nt(x, w), [[1, 2, 3], [3, 4, 7]])
    # the fp16-input form agrees
    np.testing.assert_array_equal(orc.gemm_nt_f16(x.astype(np.float16), w.astype(np.float16)),
                                  [[1, 2, 3], [3, 4, 7]])


@pytest.mark.parametrize("m,n,k", [(1, 32, 32), (7, 64, 96), (17, 32, 64), (33, 96, 160)])
def test_gemm_matches_numpy_float64_brute_force(m, n, k):
    rng = np.random.default_rng(m * 1000 + n + k)
    x = rng.standard_normal((m, k)).astype(np.float16)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
    want = (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)
    got = orc.gemm_nt_f16(x, w)
    # f64 sums in different orders agree to far below one f32 ulp
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-9)


def test_gemm_exact_on_integer_inputs():
    # integer-valued fp16 in [-4, 4]: every partial sum is an integer < 2^24, so exact
    rng = np.random.default_rng(3)
    x = rng.integers(-4, 5, (19, 256)).astype(np.float16)
    w = rng.integers(-4, 5, (64, 256)).astype(np.float16)
    want = (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)
    np.testing.assert_array_equal(orc.gemm_nt_f16(x, w), want)


def test_gemm_one_hot_rows_copy_columns_and_linearity():
    rng = np.random.default_rng(4)
    k, m = 64, 5
    x = rng.standard_normal((m, k)).astype(np.float16)
    w = np.zeros((32, k), dtype=np.float16)
    for j in range(32):
        w[j, (j * 7) % k] = 1.0
    y = orc.gemm_nt_f16(x, w)
    for j in range(32):
        np.testing.assert_array_equal(y[:, j], x[:, (j * 7) % k].astype(np.float32))
    # linearity in W: y(w1 + w2) = y(w1) + y(w2) for integer data (exact)
    w1 = rng.integers(-3, 4, (32, k)).astype(np.float16)
    w2 = rng.integers(-3, 4, (32, k)).astype(np.float16)
    xi = rng.integers(-3, 4, (m, k)).astype(np.float16)
    np.testing.assert_array_equal(orc.gemm_nt_f16(xi, (w1 + w2)),
                                  orc.gemm_nt_f16(xi, w1) + orc.gemm_nt_f16(xi, w2))


def test_gemm_row_selection_and_threads_do_not_change_results():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((40, 128)).astype(np.float16)
    w = rng.standard_normal((64, 128)).astype(np.float16)
    full1 = orc.gemm_nt_f16(x, w, threads=1)
    full8 = orc.gemm_nt_f16(x, w, threads=8)
    assert np.array_equal(full1, full8)
    rows = np.array([39, 0, 17], dtype=np.uint32)
    assert np.array_equal(orc.gemm_nt_f16(x, w, rows=rows), full1[rows])


def test_fast_f32_gemm_agrees_with_oracle():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((9, 200)).astype(np.float32)
    w = rng.standard_normal((40, 200)).astype(np.float32)
    np.testing.assert_allclose(orc.gemm_f32_fast(x, w), orc.gemm_nt(x, w), rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------- SwiGLU
def test_swiglu_pairs_blocks_decide_kat():
    # decide's swiglu_pairs_blocks (cpu_ref.rs:212-221)
    y = np.zeros((1, 32), dtype=np.float32)
    y[0, 3] = 1.0  # gate col 3
    y[0, 16 + 3] = 2.0  # up col 3
    out = orc.swiglu_interleaved(y)
    assert abs(out[0, 3] - silu64(1.0) * 2.0) < 1e-6
    assert all(v == 0.0 for i, v in enumerate(out[0]) if i != 3)


def test_swiglu_second_block_closed_form():
    # row of 64 = blocks (gate 0..15 | up 0..15 | gate 16..31 | up 16..31)
    y = np.zeros((2, 64), dtype=np.float32)
    y[1, 32 + 5] = -1.5  # gate of output 21
    y[1, 48 + 5] = 4.0  # up of output 21
    y[0, 10] = 3.0  # gate of output 10 with no up → 0
    out = orc.swiglu_interleaved(y)
    assert out.shape == (2, 32)
    assert abs(out[1, 21] - silu64(-1.5) * 4.0) < 1e-6
    assert np.count_nonzero(out) == 1


# ---------------------------------------------------------------- RMSNorm
def test_rmsnorm_by_hand_decide_kat():
    # decide's rmsnorm_by_hand (cpu_ref.rs:204-210)
    y = orc.rmsnorm(np.array([[3.0, 4.0]]), np.array([1.0, 1.0]), add_one=True)
    want = np.array([3.0, 4.0]) * 2.0 / np.sqrt(12.5)
    np.testing.assert_allclose(y[0], want, atol=1e-5)
    # without add_one the weight is used as is
    y = orc.rmsnorm(np.array([[3.0, 4.0]]), np.array([1.0, 1.0]), add_one=False)
    np.testing.assert_allclose(y[0], np.array([3.0, 4.0]) / np.sqrt(12.5), atol=1e-5)


def test_rmsnorm_scale_invariance():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((3, 2560)).astype(np.float32)
    w = (rng.standard_normal(2560) * 0.02).astype(np.float32)
    a = orc.rmsnorm(x, w, True)
    b = orc.rmsnorm(x * np.float32(4.0), w, True)  # eps is negligible at this scale
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- layouts
def test_interleave_gate_up_kat():
    k = 3
    gate = np.arange(32 * k, dtype=np.uint16).reshape(32, k)
    up = (1000 + np.arange(32 * k)).astype(np.uint16).reshape(32, k)
    out = orc.interleave_gate_up(gate, up, 16)
    assert np.array_equal(out[0:16], gate[0:16])
    assert np.array_equal(out[16:32], up[0:16])
    assert np.array_equal(out[32:48], gate[16:32])
    assert np.array_equal(out[48:64], up[16:32])


def test_deinterleave_q_gate_kat():
    heads, hd, k = 3, 2, 4
    # HF rows per head: [q_h (hd rows); gate_h (hd rows)]; value = 100·h + 10·part + d
    src = np.zeros((heads * 2 * hd, k), dtype=np.uint16)
    for h in range(heads):
        for part in range(2):
            for d in range(hd):
                src[(h * 2 + part) * hd + d] = 100 * h + 10 * part + d
    out = orc.deinterleave_q_gate(src, heads, hd)
    want = [100 * h + d for h in range(heads) for d in range(hd)] + \
           [100 * h + 10 + d for h in range(heads) for d in range(hd)]
    assert list(out[:, 0]) == want


# ---------------------------------------------------------------- golden fixtures
def _golden(name):
    path = os.path.join(GOLDEN, name)
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_golden_gemm_fixtures():
    with open(os.path.join(GOLDEN, "index.json")) as f:
        index = json.load(f)
    for case in index["gemm"]:
        z = _golden(case["file"])
        x, w = z["x"].astype(np.float16), z["w"].astype(np.float16)
        got = orc.gemm_nt_f16(x, w)
        np.testing.assert_allclose(got, z["y"], rtol=1e-6, atol=1e-9, err_msg=case["file"])
        if "swiglu" in z:
            np.testing.assert_allclose(orc.swiglu_interleaved(got), z["swiglu"], rtol=1e-5, atol=1e-6)


def test_golden_head_fixture():
    z = _golden("head_small.npz")
    got = orc.final_head(z["x"], z["w"], z["table"], z["cand"], z["ncand"], int(z["max_cand"]))
    want = z["logits"]
    written = ~np.isnan(want)
    assert np.array_equal(~np.isnan(got), written)
    np.testing.assert_allclose(got[written], want[written], rtol=1e-5, atol=1e-6)
