"""BASELINE config 5 at the size its targets are stated on: the 4B-shaped hybrid forward (36 layers, every 4th
full attention, d 2560, d_ff 9216) over a 2,307-token prompt, bar max |Δlogit| <= 0.01.

The stated shape itself (36 layers, T = 2,307, vocab 151,936, 3 answers x 8 candidates, one list ragged) against
the oracle: the random-init model is rebuilt bit for bit on the host (the device fill's steps restated in
orc_fill_normal) and tests/golden/c5_full_logits.npz holds the oracle forward's logits for it (tests/oracle_forward.py:
cpu_ref.rs pieces with decide's rounding points, forward.rs:1118-1310), with f64 GEMM sums and, as the fp32 noise
floor at this shape, with fp32 sums (tests/golden/make_forward_logits.py c5). Measured: GPU 0.0084, fp32-sum oracle
0.0093.
The live oracle also runs at the extremes the CPU finishes in well under a minute each:
  * length: 4 layers at T = 2,307 (the chunked recurrence over 2,307 steps and 2,307-key causal attention over every
    row, no pruning);
  * depth: 24 and 36 layers at T = 256 (the last one pruned to 3 answer rows), the latter beside the fp32-sum oracle;
  * 8 layers at T = 603, the shorter prompt length BASELINE reports;
all at the bar 0.01.
The full shape is further checked through properties that need no oracle: bitwise run-to-run determinism, graph
replay equal to eager, pruned within 1e-3 of unpruned, agreement with an independent GPU implementation (the
M-independent reference GEMM kernel and the token-by-token recurrence) within 0.025 (at this length a one-ulp change
in a fraction of the fp16 activations alone moves the logits by up to 0.009; see IMPL_NOISE_BOUND), and one closed
form of the layer wiring: with every w_out and w_down zero the residual stream never leaves the embedding rows, so
the logits are final_head of the answers' embedding rows."""

import os

import numpy as np
import pytest

import oracle_forward
import oracle_lib as orc
from decide_amd import synth
from decide_amd.forward import Model, ModelConfig
from decide_amd.hip import rt
from decide_amd.kernels import GemmImpl, Kernels
from gpu_util import full, sync, to_dev, to_host
from test_forward_gpu import MAX_LOGIT_DIFF, _names, _shape

pytestmark = pytest.mark.gpu

LAYERS, T_FULL, VOCAB, ANSWERS, CANDS = 36, 2307, 151936, 3, 8
# Two fp32 implementations on the GPU differ by more than either differs from the f64 oracle, since each sits on its
# own side of it. At the stated shape the fast path is 0.0084 from the oracle and the fp32-sum oracle 0.0093
# (test_full_shape_matches_the_oracle); the fast path and the reference implementations (M-independent GEMM kernel,
# token-by-token recurrence) measure 0.0153 apart in this test. The bar below was set before the stated-shape oracle
# existed; the oracle comparison above is the parity test of record.
IMPL_NOISE_BOUND = 0.025


def _request(t, vocab, seed, answers=ANSWERS, cands=CANDS):
    ids = synth.uniform_ids(synth.seed_for(seed), t, vocab).astype(np.uint32)
    ans = np.array([t // 3, (2 * t) // 3, t - 1], np.uint32)[:answers]
    cand = synth.uniform_ids(synth.seed_for(seed + 1), answers * cands, vocab).astype(np.uint32).reshape(answers,
                                                                                                         cands)
    ncand = np.full(answers, cands, np.uint32)
    ncand[1] = cands - 2  # ragged
    return ids, ans, cand, ncand


def _forward(model, ids, ans, cand, ncand, prune=True):
    logits = full((len(ans), model.cfg.max_cand), np.float32, np.nan)
    model.forward(0, (to_dev(ids), 0), len(ids), (to_dev(ans), 0), len(ans), (to_dev(cand), 0), (to_dev(ncand), 0),
                  (logits, 0), prune=prune)
    sync()
    return to_host(logits)


def _weights(model, layers):
    return {name: model.download(name).reshape(_shape(name, model.tensor(name)[1])) for name in _names(layers)}


def _gemm_fp32_sums(x, w):
    """The oracle's GEMM with fp32 sums (blocked, OpenMP) instead of f64: a second correct fp32 implementation."""
    return orc.gemm_f32_fast(np.asarray(x, np.float16).astype(np.float32), np.asarray(w, np.float16).astype(np.float32))


def _oracle_drift(kernels, layers, t, prune, seed, noise_floor=False):
    """(GPU vs f64 oracle, fp32-sum oracle vs f64 oracle or None) max |Δlogit| over the written logits."""
    cfg = ModelConfig(layers=layers, vocab=4096, max_tokens=t, max_answers=ANSWERS, max_cand=CANDS)
    model = Model(kernels.ctx, cfg)
    kernels.gemm.warm_up(0, max_m=t)
    model.init_random(0, seed=seed)
    sync()
    ids, ans, cand, ncand = _request(t, cfg.vocab, seed + 7)
    got = _forward(model, ids, ans, cand, ncand, prune)
    W = _weights(model, layers)
    model.close()
    want = oracle_forward.forward(W, layers, ids, ans, cand, ncand, cfg.max_cand, prune=prune)
    written = ~np.isnan(want)
    assert np.array_equal(~np.isnan(got), written), "entries past ncand must stay untouched"
    assert np.isfinite(got[written]).all()
    diff = float(np.abs(got[written] - want[written]).max())
    floor = None
    if noise_floor:
        alt = oracle_forward.forward(W, layers, ids, ans, cand, ncand, cfg.max_cand, prune=prune,
                                     gemm=_gemm_fp32_sums)
        floor = float(np.abs(alt[written] - want[written]).max())
    print(f"layers {layers} T {t}: GPU max |Δlogit| {diff:.4f}" +
          ("" if floor is None else f", fp32-sum oracle {floor:.4f}") +
          f" (logits up to {np.abs(want[written]).max():.3g})")
    return diff, floor


def test_forward_matches_oracle_at_length(gpu, kernels):
    """4 layers (three Gated-DeltaNet on the chunked recurrence, then full attention over all 2,307 rows)."""
    diff, _ = _oracle_drift(kernels, 4, T_FULL, False, seed=5200)
    assert diff <= MAX_LOGIT_DIFF, f"max |Δlogit| {diff:.4g}"


def test_forward_matches_oracle_at_depth(gpu, kernels):
    """24 layers (18 Gated-DeltaNet, 6 gated attention; the last one pruned) at T = 256."""
    diff, _ = _oracle_drift(kernels, 24, 256, True, seed=5100)
    assert diff <= MAX_LOGIT_DIFF, f"max |Δlogit| {diff:.4g}"


def test_forward_matches_oracle_at_603_tokens(gpu, kernels):
    """8 layers (6 Gated-DeltaNet, 2 gated attention) at BASELINE's shorter prompt length, where the residual
    projections split K and their partials meet the residual and the next norm in one kernel."""
    diff, _ = _oracle_drift(kernels, 8, 603, True, seed=5400)
    assert diff <= MAX_LOGIT_DIFF, f"max |Δlogit| {diff:.4g}"


def test_forward_at_full_depth_is_within_the_fp32_noise_floor(gpu, kernels):
    """All 36 layers at T = 256 against the f64 oracle, beside the same oracle with fp32 GEMM sums."""
    diff, floor = _oracle_drift(kernels, LAYERS, 256, True, seed=5100, noise_floor=True)
    assert floor > 0.0
    assert diff <= MAX_LOGIT_DIFF, f"max |Δlogit| {diff:.4g} (fp32-sum oracle: {floor:.4g})"


@pytest.fixture(scope="module")
def full_model(kernels):
    cfg = ModelConfig(layers=LAYERS, vocab=VOCAB, max_tokens=T_FULL, max_answers=ANSWERS, max_cand=CANDS)
    model = Model(kernels.ctx, cfg)
    kernels.gemm.warm_up(0, max_m=T_FULL)
    model.init_random(0, seed=0xDEC1DE)
    sync()
    yield model
    model.close()


@pytest.fixture(scope="module")
def full_request():
    return _request(T_FULL, VOCAB, 5300)


def test_full_shape_matches_the_oracle(gpu, full_model, full_request):
    """The stated shape itself against the oracle: tests/golden/c5_full_logits.npz holds the oracle forward's logits
    for this model (dh_model_init_random(0xDEC1DE), rebuilt bit for bit on the host) and this request, with f64 GEMM
    sums and, as the fp32 noise floor at this shape, with fp32 sums (tests/golden/make_forward_logits.py c5)."""
    fx = np.load(os.path.join(os.path.dirname(__file__), "golden", "c5_full_logits.npz"))
    layers, t, vocab, answers, cands, init_seed = (int(v) for v in fx["meta"][:6])
    assert (layers, t, vocab, answers, cands, init_seed) == (LAYERS, T_FULL, VOCAB, ANSWERS, CANDS, 0xDEC1DE)
    for name, a in zip(("ids", "ans", "cand", "ncand"), full_request):
        np.testing.assert_array_equal(a, fx[name], err_msg=name)
    got = _forward(full_model, *full_request)
    want, alt = fx["logits_f64"], fx["logits_f32sum"]
    written = ~np.isnan(want)
    assert np.array_equal(~np.isnan(got), written)
    diff = float(np.abs(got[written] - want[written]).max())
    floor = float(np.abs(alt[written] - want[written]).max())
    print(f"36 layers, T 2307: GPU max |Δlogit| {diff:.4f}, fp32-sum oracle {floor:.4f} "
          f"(logits up to {np.abs(want[written]).max():.3g})")
    assert diff <= MAX_LOGIT_DIFF, f"max |Δlogit| {diff:.4g} (fp32-sum oracle: {floor:.4g})"


def test_full_shape_is_finite_and_deterministic(gpu, full_model, full_request):
    a = _forward(full_model, *full_request)
    b = _forward(full_model, *full_request)
    written = ~np.isnan(a)
    assert written.sum() == ANSWERS * CANDS - 2
    assert np.isfinite(a[written]).all()
    np.testing.assert_array_equal(a, b)


def test_full_shape_graph_replays_equal_eager(gpu, full_model, full_request):
    from decide_amd.hip import Stream

    ids, ans, cand, ncand = full_request
    eager = _forward(full_model, ids, ans, cand, ncand)
    st = Stream()
    dev = [to_dev(a) for a in (ids, ans, cand, ncand)]
    logits = full((ANSWERS, CANDS), np.float32, np.nan)
    graph = full_model.capture(st.handle, (dev[0], 0), T_FULL, (dev[1], 0), ANSWERS, (dev[2], 0), (dev[3], 0),
                               (logits, 0))
    for i in range(3):
        logits.copy_from(np.full((ANSWERS, CANDS), np.nan, np.float32))
        graph.launch(st.handle)
        st.synchronize()
        np.testing.assert_array_equal(to_host(logits), eager, err_msg=f"replay {i}")
        _forward(full_model, ids[:600], ans[:1] % 600, cand[:1], ncand[:1])  # eager work of another size between
    graph.close()
    st.destroy()


def test_full_shape_pruned_equals_unpruned(gpu, full_model, full_request):
    a = _forward(full_model, *full_request, prune=True)
    b = _forward(full_model, *full_request, prune=False)
    w = ~np.isnan(a)
    assert np.array_equal(w, ~np.isnan(b))
    assert np.abs(a[w] - b[w]).max() <= 1e-3


def test_full_shape_agrees_with_the_reference_implementations(gpu, full_model, full_request):
    """The fast path against a context whose GEMMs run the M-independent reference kernel (fp32 FMA over K in order)
    and whose recurrence runs token by token, on the same random-init weights."""
    fast = _forward(full_model, *full_request)
    ref = Kernels(GemmImpl.Baseline, delta="sequential")
    model = Model(ref.ctx, full_model.cfg)
    model.init_random(0, seed=0xDEC1DE)
    slow = _forward(model, *full_request)
    model.close()
    ref.ctx.close()
    w = ~np.isnan(fast)
    assert np.array_equal(w, ~np.isnan(slow))
    diff = np.abs(fast[w] - slow[w]).max()
    print(f"fast vs reference implementations: max |Δlogit| {diff:.4f}")
    assert diff <= IMPL_NOISE_BOUND


def test_zero_projections_leave_the_embedding(gpu, kernels, full_request):
    """Closed form of the composition: every mixer and MLP output enters x only through w_out and w_down
    (x += g·w_outᵀ, x += mlp·w_downᵀ; forward.rs:1256-1282), so with both zero the answer rows reach the head as
    their embedding rows, and the logits are final_head(embed[ids[ans]]) (cpu_ref.rs:190-198)."""
    cfg = ModelConfig(layers=LAYERS, vocab=VOCAB, max_tokens=T_FULL, max_answers=ANSWERS, max_cand=CANDS)
    model = Model(kernels.ctx, cfg)
    model.init_random(0, seed=0xC105ED)
    for l in range(LAYERS):
        for name in ("w_out", "w_down"):
            ptr, n, dtype = model.tensor(f"L{l}.{name}")
            assert rt().hipMemset(ptr, 0, n * np.dtype(dtype).itemsize) == 0
    sync()
    ids, ans, cand, ncand = full_request
    got = _forward(model, ids, ans, cand, ncand)
    table = model.download("embed").reshape(VOCAB, 2560)
    x = orc.embed_bf16(ids[ans], table)
    want = orc.final_head(x, model.download("final_norm"), table, cand, ncand, CANDS)
    model.close()
    w = ~np.isnan(want)
    assert np.array_equal(w, ~np.isnan(got))
    diff = np.abs(got[w] - want[w]).max()
    assert diff <= 1e-4, f"max |Δlogit| {diff:.3g}"
