"""dh_gemm_nt_noalloc: the GEMM entry point that allocates nothing (its split-K partials live in the library's
file-scope device scratch) against dh_gemm_nt on the same inputs. Two calls in a row, the second smaller, so the
second runs over the first's leftovers in the shared scratch; a plan whose partials exceed the scratch is refused
before anything is launched; and the device's free memory does not move across the calls."""

import ctypes

import numpy as np
import pytest

from decide_amd import _lib, synth
from decide_amd.hip import rt
from decide_amd.kernels import Epilogue, Kernels, addr
from gpu_util import check_gemm, full, sync, to_dev, to_host

pytestmark = pytest.mark.gpu

# (m, n, k, epi): C2's down projection (split-K 4: 24.7 MB of partials), then a smaller split-K call
CALLS = [(603, 2560, 9216, Epilogue.AddF32), (163, 2560, 4096, Epilogue.AddF32)]


def _noalloc(k, x, w, y, m, n, kk, ldy, epi):
    return _lib.load().dh_gemm_nt_noalloc(k.ctx.handle, None, addr(x), kk, addr(w), kk, addr(y), ldy, m, n, kk,
                                          int(epi))


def _free_bytes():
    r = rt()
    r.hipMemGetInfo.restype = ctypes.c_int
    r.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert r.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_noalloc_matches_gemm_nt_on_two_calls(gpu):
    k = Kernels()
    data = []
    for i, (m, n, kk, epi) in enumerate(CALLS):
        x = synth.normal_f16(synth.seed_for(900 + i), (m, kk), 1.0)
        w = synth.normal_f16(synth.seed_for(910 + i), (n, kk), 0.02)
        y0 = synth.normal_f32(synth.seed_for(920 + i), (m, n), 1.0)
        assert k.gemm.plan(m, n, kk, epi)["splits"] > 1, "both calls must exercise the split-K scratch"
        data.append((to_dev(x), to_dev(w), y0))
    # dh_gemm_nt's results (its own, context-owned workspace)
    want = []
    for (m, n, kk, epi), (xd, wd, y0) in zip(CALLS, data):
        y = to_dev(y0)
        k.gemm.gemm(0, (xd, 0), (wd, 0), (y, 0), m, n, kk, kk, kk, n, epi)
        sync()
        want.append(to_host(y))
    # warm pass of the no-alloc path (first launches may load code), then the measured pair back to back
    ys = [to_dev(y0) for (_, _, y0) in data]
    for (m, n, kk, epi), (xd, wd, _), y in zip(CALLS, data, ys):
        assert _noalloc(k, (xd, 0), (wd, 0), (y, 0), m, n, kk, n, epi) == 0, _lib.last_error()
    sync()
    ys = [to_dev(y0) for (_, _, y0) in data]
    sync()
    before = _free_bytes()
    for (m, n, kk, epi), (xd, wd, _), y in zip(CALLS, data, ys):
        assert _noalloc(k, (xd, 0), (wd, 0), (y, 0), m, n, kk, n, epi) == 0, _lib.last_error()
    sync()
    after = _free_bytes()
    # nothing allocated (a free the runtime completes late may only raise the figure)
    assert after >= before, f"device free memory fell by {before - after} bytes"
    for (m, n, kk, epi), y, w_, (_, _, y0) in zip(CALLS, ys, want, data):
        got = to_host(y)
        # the same plan as dh_gemm_nt (its partials fit the scratch), so the same bits
        np.testing.assert_array_equal(got, w_, err_msg=f"m {m}")
        check_gemm(f"noalloc m{m}", got - y0, w_ - y0)
    k.ctx.close()


def test_noalloc_refuses_a_plan_beyond_its_scratch(gpu):
    k = Kernels()
    m, n, kk = 2307, 18432, 2560
    x = to_dev(synth.normal_f16(synth.seed_for(930), (m, kk), 1.0))
    w = to_dev(synth.normal_f16(synth.seed_for(931), (n, kk), 0.02))
    y = full((m, n // 2), np.float16, 5.0)
    k.gemm.force(0, 8)  # 8 splits x 2307 x 18432 fp32 partials: 1.36 GB
    try:
        rc = _noalloc(k, (x, 0), (w, 0), (y, 0), m, n, kk, n // 2, Epilogue.SwigluF16)
        err = _lib.last_error()  # read before dh_gemm_force clears it
    finally:
        k.gemm.force(None)
    assert rc == _lib.DH_EINVAL
    assert "bytes of scratch" in err, err
    sync()
    assert (to_host(y) == 5.0).all(), "nothing may be launched after a refusal"
    # the planner itself stays within the scratch for the same shape
    rc = _noalloc(k, (x, 0), (w, 0), (y, 0), m, n, kk, n // 2, Epilogue.SwigluF16)
    assert rc == 0, _lib.last_error()
    sync()
    assert np.isfinite(to_host(y).astype(np.float32)).all()
    k.ctx.close()
