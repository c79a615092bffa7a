"""dh_gemm_add_rmsnorm: a residual-adding projection and the norm that reads the new rows next, as one call.

Its results are defined as those of the two calls it replaces, dh_gemm_nt with the AddF32 epilogue (decide's
x += a·wᵀ, forward.rs:1256-1282) followed by dh_rmsnorm_rows over the same rows (norm.rs:26-33). Both of those
are checked against the oracle elsewhere (test_gemm_gpu.py, test_rows_gpu.py); here the fused call must equal them
bit for bit, in y and in h, on the split-K path where one kernel does the reduce, the residual add and the norm,
and on the paths that keep two kernels (no split, or rows the fused kernel does not take).
"""

import numpy as np
import pytest

from decide_amd import synth
from decide_amd.kernels import Epilogue
from gpu_util import full, sync, to_dev, to_host

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _case(kernels, m, n, k, ldy, ldh, add_one, seed, force=None):
    x = synth.normal_f16(synth.seed_for(seed), (m, k), 1.0)
    w = synth.normal_f16(synth.seed_for(seed + 1), (n, k), 0.02)
    y0 = np.full((m, ldy), np.nan, np.float32)
    y0[:, :n] = synth.normal_f32(synth.seed_for(seed + 2), (m, n), 1.0)
    nw = synth.normal_f32(synth.seed_for(seed + 3), (n,), 0.02) + (0.0 if add_one else 1.0)
    dx, dw, dnw = to_dev(x), to_dev(w), to_dev(nw.astype(np.float32))
    rowmap = to_dev(np.arange(m, dtype=np.uint32))
    g = kernels.gemm
    if force is not None:
        g.force(*force)
    try:
        # the two calls
        ya = to_dev(y0)
        ha = full((m, ldh), np.float16, np.nan)
        g.gemm(0, (dx, 0), (dw, 0), (ya, 0), m, n, k, k, k, ldy, Epilogue.AddF32)
        kernels.norm.rmsnorm(0, (ya, 0), (dnw, 0), (ha, 0), (rowmap, 0), m, n, ldy, ldh, add_one, EPS)
        # the fused call
        yb = to_dev(y0)
        hb = full((m, ldh), np.float16, np.nan)
        g.gemm_add_rmsnorm(0, (dx, 0), (dw, 0), (yb, 0), m, n, k, k, k, ldy, (dnw, 0), (hb, 0), ldh, add_one, EPS)
        sync()
    finally:
        if force is not None:
            g.force(None)
    a_y, b_y, a_h, b_h = to_host(ya), to_host(yb), to_host(ha), to_host(hb)
    np.testing.assert_array_equal(b_y.view(np.uint32), a_y.view(np.uint32), err_msg="y")
    np.testing.assert_array_equal(b_h.view(np.uint16), a_h.view(np.uint16), err_msg="h")
    # padding columns of h stay untouched
    assert np.isnan(b_h[:, n:].astype(np.float32)).all()
    assert np.isfinite(b_h[:, :n].astype(np.float32)).all()


@pytest.mark.parametrize("m,k", [(603, 9216), (603, 4096), (276, 4096), (37, 9216), (1024, 4096)])
def test_planner_shapes_equal_the_two_calls(gpu, kernels, m, k):
    """The engine's N = 2560 residual projections at prompt lengths where the planner splits K (and 37 rows)."""
    plan = kernels.gemm.plan(m, 2560, k, Epilogue.AddF32)
    _case(kernels, m, 2560, k, 2560, 2560, True, seed=900 + m + k)
    print(f"M {m} K {k}: plan {plan}")


def test_unsplit_plan_equals_the_two_calls(gpu, kernels):
    """M = 2,307: the planner does not split K, so the call runs the projection and the norm kernel."""
    assert kernels.gemm.plan(2307, 2560, 4096, Epilogue.AddF32)["splits"] == 1
    _case(kernels, 2307, 2560, 4096, 2560, 2560, True, seed=950)


@pytest.mark.parametrize("splits", [2, 3, 4, 5, 6, 7, 8])
def test_every_split_count(gpu, kernels, splits):
    """The fused kernel for each split count it is compiled for (160 x 160 tiles, forced)."""
    _case(kernels, 130, 2560, 32 * 64, 2560, 2560, True, seed=960 + splits, force=(14, splits))


@pytest.mark.parametrize("n,ldy,ldh,add_one", [(2528, 2600, 2536, True), (1024, 1024, 1032, False),
                                              (64, 68, 64, True), (3072, 3072, 3072, True)])
def test_ragged_rows_and_strides(gpu, kernels, n, ldy, ldh, add_one):
    """Row widths below a full 64-lane pass, padded strides, the plain weight, and a row too wide for the
    fused kernel (3,072 > 2,560: the two kernels)."""
    _case(kernels, 77, n, 1024, ldy, ldh, add_one, seed=980 + n, force=(14, 4))


def test_refuses_a_zero_width_row(gpu, kernels):
    x = to_dev(np.zeros((4, 64), np.float16))
    y = to_dev(np.zeros((4, 32), np.float32))
    h = to_dev(np.zeros((4, 32), np.float16))
    with pytest.raises(AssertionError, match="N must be at least 32"):
        kernels.gemm.gemm_add_rmsnorm(0, (x, 0), (x, 0), (y, 0), 4, 0, 64, 64, 64, 32, (y, 0), (h, 0), 32)
