"""The whole hybrid decoder forward on the GPU (dh_model_forward) against the oracle's forward built from
cpu_ref.rs pieces with decide's rounding points, on a reduced random-init model (same layer shapes, fewer
layers, small vocab and prompt). Bar: max |Δlogit| <= 0.01.
The forward at its stated size (36 layers, 2,307 tokens, vocab 151,936) is checked in test_forward_c5_gpu.py:
against the oracle at full depth (T = 256) and at full length (4 layers, T = 2,307), and at the full shape
through determinism, graph replay, pruning, an independent GPU implementation and a closed form."""

import numpy as np
import pytest

import oracle_forward
from decide_amd import synth
from decide_amd.forward import Model, ModelConfig
from gpu_util import full, sync, to_dev, to_host

pytestmark = pytest.mark.gpu

MAX_LOGIT_DIFF = 0.01  # BASELINE config 5 tolerance


def _names(layers):
    names = ["embed", "final_norm"]
    for l in range(layers):
        pre = f"L{l}."
        names += [pre + n for n in ("in_norm", "w_in", "w_out", "post_norm", "w_gu", "w_down")]
        if (l + 1) % 4 == 0:
            names += [pre + "q_norm", pre + "k_norm"]
        else:
            names += [pre + n for n in ("conv_w", "a_log", "dt_bias", "gnorm")]
    return names


def _shape(name, n):
    two_d = {"embed": 2560, "w_in": 2560, "w_gu": 2560, "w_out": None, "w_down": 9216, "conv_w": 4}
    key = name.split(".")[-1]
    if key == "w_out":
        return (2560, n // 2560)
    if key in two_d:
        return (n // two_d[key], two_d[key])
    return (n,)


def _request(t, vocab, n_ans, max_cand, seed):
    ids = synth.uniform_ids(synth.seed_for(seed), t, vocab).astype(np.uint32)
    ans = np.linspace(t // 3, t - 1, n_ans).astype(np.uint32)
    cand = synth.uniform_ids(synth.seed_for(seed + 1), n_ans * max_cand, vocab).astype(np.uint32).reshape(n_ans,
                                                                                                          max_cand)
    ncand = np.full(n_ans, max_cand, np.uint32)
    ncand[0] = max_cand - 3  # ragged
    return ids, ans, cand, ncand


def _run(model, kernels, ids, ans, cand, ncand, max_cand, prune):
    logits = full((len(ans), max_cand), np.float32, np.nan)
    model.forward(0, (to_dev(ids), 0), len(ids), (to_dev(ans), 0), len(ans), (to_dev(cand), 0), (to_dev(ncand), 0),
                  (logits, 0), prune=prune)
    sync()
    return to_host(logits)


# (4, 330): past DH_DELTA_CHUNK_MIN_T, so the default context runs the chunked recurrence end to end
@pytest.mark.parametrize("layers,t,prune", [(4, 48, True), (4, 40, False), (8, 70, True), (4, 330, True)])
def test_forward_matches_oracle(gpu, kernels, layers, t, prune):
    cfg = ModelConfig(layers=layers, vocab=1000, max_tokens=max(96, t), max_answers=4, max_cand=8)
    model = Model(kernels.ctx, cfg)
    kernels.gemm.warm_up(0, max_m=cfg.max_tokens)
    model.init_random(0, seed=1234 + layers)
    sync()
    W = {}
    for name in _names(layers):
        W[name] = model.download(name).reshape(_shape(name, model.tensor(name)[1]))
    ids, ans, cand, ncand = _request(t, cfg.vocab, 3, cfg.max_cand, 300 + layers)
    got = _run(model, kernels, ids, ans, cand, ncand, cfg.max_cand, prune)
    want = oracle_forward.forward(W, layers, ids, ans, cand, ncand, cfg.max_cand, prune=prune)
    written = ~np.isnan(want)
    assert np.array_equal(~np.isnan(got), written), "entries past ncand must stay untouched"
    diff = np.abs(got[written] - want[written])
    assert np.isfinite(got[written]).all()
    assert diff.max() <= MAX_LOGIT_DIFF, f"max |Δlogit| {diff.max():.4g} (logits up to {np.abs(want[written]).max():.3g})"
    model.close()


def test_forward_pruned_equals_unpruned_within_tolerance(gpu, kernels):
    """Pruning the last layer to the answer rows changes only which rows are computed (forward.rs:1144-1150)."""
    cfg = ModelConfig(layers=4, vocab=500, max_tokens=64, max_answers=4, max_cand=6)
    model = Model(kernels.ctx, cfg)
    model.init_random(0, seed=77)
    ids, ans, cand, ncand = _request(50, cfg.vocab, 4, cfg.max_cand, 410)
    a = _run(model, kernels, ids, ans, cand, ncand, cfg.max_cand, True)
    b = _run(model, kernels, ids, ans, cand, ncand, cfg.max_cand, False)
    w = ~np.isnan(a)
    assert np.abs(a[w] - b[w]).max() <= 1e-3
    model.close()


def test_forward_is_deterministic_and_answer_rows_are_independent(gpu, kernels):
    cfg = ModelConfig(layers=4, vocab=500, max_tokens=64, max_answers=4, max_cand=6)
    model = Model(kernels.ctx, cfg)
    model.init_random(0, seed=78)
    ids, ans, cand, ncand = _request(60, cfg.vocab, 4, cfg.max_cand, 420)
    a = _run(model, kernels, ids, ans, cand, ncand, cfg.max_cand, True)
    b = _run(model, kernels, ids, ans, cand, ncand, cfg.max_cand, True)
    np.testing.assert_array_equal(a, b)
    # the pruned layer's GEMMs run at M = answers, so a different count may take a different GEMM plan:
    # equal within the parity tolerance, not bitwise
    one = _run(model, kernels, ids, ans[2:3], cand[2:3], ncand[2:3], cfg.max_cand, True)
    w = ~np.isnan(a[2])
    assert np.abs(one[0][w] - a[2][w]).max() <= 1e-3
    model.close()


def test_captured_forward_replays_match_eager(gpu, kernels):
    """The whole forward captured as one HIP graph: every replay (with eager forwards and new inputs in
    between) reproduces the eager forward bit for bit."""
    from decide_amd.hip import Stream

    cfg = ModelConfig(layers=4, vocab=700, max_tokens=64, max_answers=4, max_cand=6)
    model = Model(kernels.ctx, cfg)
    st = Stream()
    s = st.handle
    model.init_random(s, seed=91)
    kernels.gemm.warm_up(s, max_m=cfg.max_tokens)
    ids_a, ans, cand, ncand = _request(56, cfg.vocab, 3, cfg.max_cand, 430)
    ids_b = _request(56, cfg.vocab, 3, cfg.max_cand, 431)[0]
    dev = {"ids": to_dev(ids_a), "ans": to_dev(ans), "cand": to_dev(cand), "ncand": to_dev(ncand)}
    logits = full((3, cfg.max_cand), np.float32, np.nan)
    graph = model.capture(s, (dev["ids"], 0), 56, (dev["ans"], 0), 3, (dev["cand"], 0), (dev["ncand"], 0),
                          (logits, 0))
    st.synchronize()
    eager_a = _run(model, kernels, ids_a, ans, cand, ncand, cfg.max_cand, True)
    eager_b = _run(model, kernels, ids_b, ans, cand, ncand, cfg.max_cand, True)
    for i, (ids, want) in enumerate([(ids_a, eager_a), (ids_b, eager_b), (ids_a, eager_a)]):
        dev["ids"].copy_from(ids)
        logits.copy_from(np.full((3, cfg.max_cand), np.nan, np.float32))
        graph.launch(s)
        st.synchronize()
        np.testing.assert_array_equal(to_host(logits), want, err_msg=f"replay {i}")
        _run(model, kernels, ids_b, ans, cand, ncand, cfg.max_cand, True)  # eager work between replays
    graph.close()
    st.destroy()
    model.close()


def test_forward_delta_implementations_agree(gpu, kernels, kernels_delta_sequential):
    """From DH_DELTA_CHUNK_MIN_T tokens on the default context runs the chunked recurrence; the same model
    forward with the token-by-token kernel agrees within the parity tolerance (both are pinned against the
    oracle's recurrence in test_mixer_gpu.py)."""
    cfg = ModelConfig(layers=4, vocab=800, max_tokens=400, max_answers=3, max_cand=5)
    ids, ans, cand, ncand = _request(400, cfg.vocab, 3, cfg.max_cand, 440)
    out = []
    for k in (kernels, kernels_delta_sequential):
        model = Model(k.ctx, cfg)
        model.init_random(0, seed=93)
        out.append(_run(model, k, ids, ans, cand, ncand, cfg.max_cand, True))
        model.close()
    w = ~np.isnan(out[0])
    assert np.array_equal(w, ~np.isnan(out[1]))
    assert np.abs(out[0][w] - out[1][w]).max() <= MAX_LOGIT_DIFF


def test_graph_survives_workspace_growth(gpu):
    """A graph keeps the raw workspace pointers it was captured with. Capture at T = 603 (split-K down and out
    projections), then run an eager forward at T = 1146 on a fresh context without warm-up, which grows the split-K
    workspace: the replayed graph must still reproduce the eager T = 603 forward (the replaced workspace stays
    allocated until the context is destroyed)."""
    from decide_amd.hip import Stream
    from decide_amd.kernels import Kernels

    k = Kernels()
    cfg = ModelConfig(layers=4, vocab=600, max_tokens=1146, max_answers=3, max_cand=5)
    model = Model(k.ctx, cfg)
    st = Stream()
    s = st.handle
    model.init_random(s, seed=95)
    ids, ans, cand, ncand = _request(603, cfg.vocab, 3, cfg.max_cand, 450)
    dev = [to_dev(a) for a in (ids, ans, cand, ncand)]
    logits = full((3, cfg.max_cand), np.float32, np.nan)
    graph = model.capture(s, (dev[0], 0), 603, (dev[1], 0), 3, (dev[2], 0), (dev[3], 0), (logits, 0))
    st.synchronize()
    eager = to_host(logits)
    before = k.gemm.plan(1146, 2560, 9216, 2)["ws_bytes"]
    long_ids, long_ans, long_cand, long_ncand = _request(1146, cfg.vocab, 3, cfg.max_cand, 451)
    _run(model, k, long_ids, long_ans, long_cand, long_ncand, cfg.max_cand, True)
    assert before > k.gemm.plan(603, 2560, 9216, 2)["ws_bytes"], "the T = 1146 forward must need a larger workspace"
    for i in range(2):
        logits.copy_from(np.full((3, cfg.max_cand), np.nan, np.float32))
        graph.launch(s)
        st.synchronize()
        np.testing.assert_array_equal(to_host(logits), eager, err_msg=f"replay {i}")
    graph.close()
    st.destroy()
    model.close()
    k.ctx.close()
