"""One context shared by streams and host threads (decide: Gemm is Sync, its pipeline cache behind a mutex,
kernels/gemm.rs:46-55, 115-124). Each stream gets its own split-K and forward workspaces, so overlapping calls on
different streams must give the bits the same calls give one after another; a workspace that would have to grow
on a stream being captured is refused before anything is enqueued."""

import ctypes
import threading

import numpy as np
import pytest

from decide_amd import synth
from decide_amd.forward import Model, ModelConfig
from decide_amd.hip import Stream, check, rt
from decide_amd.kernels import Epilogue, Kernels
from gpu_util import full, sync, to_dev, to_host

pytestmark = pytest.mark.gpu

# Two split-K shapes of the engine (C2 down, C3 out at 603 rows) with the residual-add epilogue.
SHAPES = [(603, 2560, 9216), (603, 2560, 4096)]


def _operands(m, n, k, seed):
    x = to_dev(synth.normal_f16(synth.seed_for(seed), (m, k), 1.0))
    w = to_dev(synth.normal_f16(synth.seed_for(seed + 1), (n, k), 0.02))
    y0 = synth.normal_f32(synth.seed_for(seed + 2), (m, n), 1.0)
    return x, w, y0


def test_split_k_gemms_overlap_on_two_streams(gpu, kernels):
    for (m, n, k) in SHAPES:
        assert kernels.gemm.plan(m, n, k, Epilogue.AddF32)["splits"] > 1
    ops = [_operands(m, n, k, 700 + 10 * i) for i, (m, n, k) in enumerate(SHAPES)]
    reps = 12
    # sequential reference: `reps` accumulations of each GEMM on stream 0
    want = []
    for (m, n, k), (x, w, y0) in zip(SHAPES, ops):
        y = to_dev(y0)
        for _ in range(reps):
            kernels.gemm.gemm(0, (x, 0), (w, 0), (y, 0), m, n, k, k, k, n, Epilogue.AddF32)
        sync()
        want.append(to_host(y))
    streams = [Stream(), Stream()]
    ys = [to_dev(y0) for (_, _, y0) in ops]
    for _ in range(reps):  # interleaved enqueues, no synchronisation between the streams
        for (m, n, k), (x, w, _), y, st in zip(SHAPES, ops, ys, streams):
            kernels.gemm.gemm(st.handle, (x, 0), (w, 0), (y, 0), m, n, k, k, k, n, Epilogue.AddF32)
    for st in streams:
        st.synchronize()
    for got, ref in zip(ys, want):
        np.testing.assert_array_equal(to_host(got), ref)
    for st in streams:
        st.destroy()


def test_two_threads_two_streams(gpu, kernels):
    """Host threads calling into one context at once (ctypes releases the GIL in foreign calls)."""
    (m, n, k) = SHAPES[0]
    x, w, y0 = _operands(m, n, k, 800)
    reps = 16
    ref = to_dev(y0)
    for _ in range(reps):
        kernels.gemm.gemm(0, (x, 0), (w, 0), (ref, 0), m, n, k, k, k, n, Epilogue.AddF32)
    sync()
    want = to_host(ref)
    streams = [Stream() for _ in range(2)]
    ys = [to_dev(y0) for _ in streams]
    errors = []

    def work(st, y):
        try:
            for _ in range(reps):
                kernels.gemm.gemm(st.handle, (x, 0), (w, 0), (y, 0), m, n, k, k, k, n, Epilogue.AddF32)
            st.synchronize()
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    threads = [threading.Thread(target=work, args=(st, y)) for st, y in zip(streams, ys)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for y in ys:
        np.testing.assert_array_equal(to_host(y), want)
    for st in streams:
        st.destroy()


def _forward(model, st, ids, ans, cand, ncand, logits):
    model.forward(st, (ids, 0), ids.shape[0], (ans, 0), ans.shape[0], (cand, 0), (ncand, 0), (logits, 0))


def test_two_models_forward_concurrently_through_one_context(gpu, kernels):
    """Two 4-layer models at 400 tokens (the chunked recurrence and attention both use the forward workspace)
    running at once on two streams of one context give the bits each gives alone."""
    t, n_ans, n_cand = 400, 2, 4
    cfg = ModelConfig(layers=4, vocab=1000, max_tokens=t, max_answers=n_ans, max_cand=n_cand)
    models = [Model(kernels.ctx, cfg) for _ in range(2)]
    reqs = []
    for i, model in enumerate(models):
        model.init_random(0, seed=4200 + i)
        ids = to_dev(synth.uniform_ids(synth.seed_for(4300 + i), t, cfg.vocab).astype(np.uint32))
        ans = to_dev(np.array([t // 2, t - 1], np.uint32))
        cand = to_dev(synth.uniform_ids(synth.seed_for(4400 + i), n_ans * n_cand, cfg.vocab).astype(np.uint32))
        ncand = to_dev(np.full(n_ans, n_cand, np.uint32))
        reqs.append((ids, ans, cand, ncand))
    sync()
    want = []
    for model, req in zip(models, reqs):
        logits = full((n_ans, n_cand), np.float32, np.nan)
        _forward(model, 0, *req, logits)
        sync()
        want.append(to_host(logits))
    streams = [Stream(), Stream()]
    outs = [full((n_ans, n_cand), np.float32, np.nan) for _ in models]
    for _ in range(3):
        for model, req, st, out in zip(models, reqs, streams, outs):
            _forward(model, st.handle, *req, out)
    for st in streams:
        st.synchronize()
    for got, ref in zip(outs, want):
        np.testing.assert_array_equal(to_host(got), ref)
    for model in models:
        model.close()
    for st in streams:
        st.destroy()


def test_growth_under_capture_is_refused(gpu):
    """A split-K GEMM on a stream whose workspace was never sized, while that stream is captured, is refused
    (DH_EINVAL, nothing enqueued); after one eager call of that size on the stream, the same call captures and
    its graph replays to the eager result. A fresh context, so no earlier stream's workspace is in it."""
    kernels = Kernels()
    (m, n, k) = SHAPES[1]
    x, w, y0 = _operands(m, n, k, 900)
    st = Stream()
    y = to_dev(y0)
    graph = ctypes.c_void_p()
    check(rt().hipStreamBeginCapture(st.handle, 2), "hipStreamBeginCapture")  # relaxed mode
    with pytest.raises(AssertionError, match="being captured"):
        kernels.gemm.gemm(st.handle, (x, 0), (w, 0), (y, 0), m, n, k, k, k, n, Epilogue.AddF32)
    check(rt().hipStreamEndCapture(st.handle, ctypes.byref(graph)), "hipStreamEndCapture")
    if graph.value:
        check(rt().hipGraphDestroy(graph), "hipGraphDestroy")
    # size the workspace eagerly on this stream, then capture the same call
    kernels.gemm.gemm(st.handle, (x, 0), (w, 0), (y, 0), m, n, k, k, k, n, Epilogue.AddF32)
    st.synchronize()
    once = to_host(y)
    y.copy_from(y0)
    check(rt().hipStreamBeginCapture(st.handle, 2), "hipStreamBeginCapture")
    kernels.gemm.gemm(st.handle, (x, 0), (w, 0), (y, 0), m, n, k, k, k, n, Epilogue.AddF32)
    graph = ctypes.c_void_p()
    check(rt().hipStreamEndCapture(st.handle, ctypes.byref(graph)), "hipStreamEndCapture")
    exe = ctypes.c_void_p()
    check(rt().hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0), "hipGraphInstantiate")
    check(rt().hipGraphLaunch(exe, st.handle), "hipGraphLaunch")
    st.synchronize()
    np.testing.assert_array_equal(to_host(y), once)
    check(rt().hipGraphExecDestroy(exe), "hipGraphExecDestroy")
    check(rt().hipGraphDestroy(graph), "hipGraphDestroy")
    st.destroy()
    kernels.ctx.close()
