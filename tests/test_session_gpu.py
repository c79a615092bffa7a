"""Requests (dh_model_logits and friends) against decide's request layer (Forward::logits, build_snapshot
and the state cache, forward.rs:641-1116) on a reduced random-init model.

What is pinned, and how:
  * the math of every route: chunked runs, snapshot runs and follow-ups from a cached state match the
    oracle's whole-sequence forward within BASELINE's max |Δlogit| 0.01, and each other within 5e-3 (the
    fast GEMM picks its kernel and split by M, so rows' rounding depends on the chunking, as decide notes
    at forward.rs:606-611; through the fp16 rounding points that reaches ~2.5e-3 on logits of size ~3);
  * route choice (snapshot / full / state_cache), the first computed position, the LRU order and
    eviction, and decide's refusals, as forward.rs states them;
  * the K/V bookkeeping (restore of the prefix rows and of an entry's rows after another run has
    overwritten them) bitwise: the same request on the same route gives the same logits bit for bit;
  * tail truncation bitwise: ids after the last answer row never run.
"""

import numpy as np
import pytest

import oracle_forward
from decide_amd import synth
from decide_amd.forward import STATE_MARKER, Model, ModelConfig
from gpu_util import sync
from test_forward_gpu import _names, _shape

pytestmark = pytest.mark.gpu

CFG = ModelConfig(layers=4, vocab=600, max_tokens=128, max_answers=4, max_cand=6)
ROUTE_TOL = 5e-3
ORACLE_TOL = 0.01
MARKER = [591, 592, 593]  # a state marker no random id below 590 can form


@pytest.fixture(scope="module")
def model(kernels):
    m = Model(kernels.ctx, CFG)
    kernels.gemm.warm_up(0, max_m=CFG.max_tokens)
    m.init_random(0, seed=2024)
    sync()
    m.set_state_marker(MARKER)
    yield m
    m.close()


@pytest.fixture(scope="module")
def weights(model):
    return {n: model.download(n).reshape(_shape(n, model.tensor(n)[1])) for n in _names(CFG.layers)}


def _ids(n, seed):
    return [int(x) for x in synth.uniform_ids(synth.seed_for(seed), n, 590)]


def _answers(rows, seed, ragged=True):
    out = []
    for i, r in enumerate(rows):
        c = [int(x) for x in synth.uniform_ids(synth.seed_for(seed + i), CFG.max_cand, CFG.vocab)]
        out.append((r, c[: CFG.max_cand - (i % 3 if ragged else 0)]))
    return out


def _oracle(weights, ids, answers):
    n = len(answers)
    cand = np.zeros((n, CFG.max_cand), np.uint32)
    ncand = np.zeros(n, np.uint32)
    for i, (_, c) in enumerate(answers):
        cand[i, : len(c)] = c
        ncand[i] = len(c)
    rows = np.array([r for r, _ in answers], np.uint32)
    want = oracle_forward.forward(weights, CFG.layers, np.array(ids, np.uint32), rows, cand, ncand, CFG.max_cand,
                                  prune=True)
    return [want[i, : len(c)].tolist() for i, (_, c) in enumerate(answers)]


def _close(a, b, tol):
    d = max(float(np.abs(np.array(x) - np.array(y)).max()) for x, y in zip(a, b))
    assert d <= tol, f"max |Δlogit| {d:.3g} > {tol}"


@pytest.fixture(autouse=True)
def _reset(model):
    model.set_chunk(CFG.max_tokens)
    model.set_pruning(True)
    model.set_state_cache(2)
    model.forget_states()
    yield


def test_chunked_full_route_matches_oracle(gpu, model, weights):
    ids = _ids(90, 1)
    answers = _answers([89, 40, 61], 10)  # unsorted on purpose
    want = _oracle(weights, ids, answers)
    one = model.logits_full(0, ids, answers)
    assert model.last_route() == "full" and model.last_start() == 0
    _close(one, want, ORACLE_TOL)
    for chunk in (17, 5, 40):
        model.set_chunk(chunk)
        got = model.logits_full(0, ids, answers)
        _close(got, want, ORACLE_TOL)
        _close(got, one, ROUTE_TOL)


def test_chunks_carry_the_conv_state_into_the_fused_recurrence(gpu, kernels_delta_chunked, weights):
    """On a context that always runs the chunked recurrence, every chunk of a Gated-DeltaNet layer takes the fused
    conv + recurrence call, which reads the carried conv state and only then lets the next chunk's state replace it:
    chunked requests still match the oracle's whole-sequence forward."""
    m = Model(kernels_delta_chunked.ctx, CFG)
    kernels_delta_chunked.gemm.warm_up(0, max_m=CFG.max_tokens)
    m.init_random(0, seed=2024)  # the module model's weights, so `weights` is its oracle copy
    sync()
    try:
        ids = _ids(90, 1)
        answers = _answers([89, 40, 61], 10)
        want = _oracle(weights, ids, answers)
        for chunk in (90, 17, 40):
            m.set_chunk(chunk)
            _close(m.logits_full(0, ids, answers), want, ORACLE_TOL)
    finally:
        m.close()


def test_unpruned_chunked_matches_pruned(gpu, model):
    ids = _ids(70, 2)
    answers = _answers([30, 69], 20)
    model.set_chunk(23)
    a = model.logits_full(0, ids, answers)
    model.set_pruning(False)
    assert not model.pruning()
    b = model.logits_full(0, ids, answers)
    _close(a, b, ROUTE_TOL)


def test_rows_after_the_last_answer_never_run(gpu, model):
    ids = _ids(80, 3)
    answers = _answers([50, 60], 30)
    a = model.logits_full(0, ids, answers)
    tail = ids[:61] + _ids(19, 4)
    b = model.logits_full(0, tail, answers)
    assert a == b


def test_snapshot_route_and_prefix_restore(gpu, model, weights):
    prefix = _ids(24, 5)
    model.build_snapshot(0, prefix)
    assert model.prefix_len() == 24
    ids = prefix + _ids(50, 6)
    answers = _answers([73, 30], 40)
    model.set_chunk(13)
    snap = model.logits(0, ids, answers)
    assert model.last_route() == "snapshot" and model.last_start() == 24
    _close(snap, _oracle(weights, ids, answers), ORACLE_TOL)
    _close(snap, model.logits_full(0, ids, answers), ROUTE_TOL)
    # ids that do not start with the prefix, or an answer inside it: the full route
    other = _ids(60, 7)
    model.logits(0, other, _answers([59], 50))
    assert model.last_route() == "full" and model.last_start() == 0
    model.logits(0, ids, _answers([10, 70], 55))
    assert model.last_route() == "full"
    # the full runs overwrote the prefix's K/V rows; the snapshot route puts them back
    again = model.logits(0, ids, answers)
    assert model.last_route() == "snapshot"
    assert again == snap


def _state_prompt(prefix, seed, state_len=20, question_len=15):
    state = _ids(state_len, seed)
    question = _ids(question_len, seed + 1)
    ids = prefix + state + MARKER + question
    return ids, len(prefix) + state_len + len(MARKER)


@pytest.mark.parametrize("chunk", [128, 16, 9])
def test_state_capture_and_follow_up(gpu, model, weights, chunk):
    prefix = _ids(12, 8)
    model.build_snapshot(0, prefix)
    model.set_chunk(chunk)
    ids, boundary = _state_prompt(prefix, 9)
    answers = _answers([len(ids) - 1, boundary + 3], 60)
    first = model.logits(0, ids, answers)
    assert model.last_route() == "snapshot"
    assert model.cached_states() == [boundary]
    _close(first, model.logits_full(0, ids, answers), ROUTE_TOL)
    # a follow-up: the same state, another question
    follow = ids[:boundary] + _ids(18, 11)
    fa = _answers([boundary + 5, len(follow) - 1], 70)
    got = model.logits(0, follow, fa)
    assert model.last_route() == "state_cache" and model.last_start() == boundary
    _close(got, _oracle(weights, follow, fa), ORACLE_TOL)
    _close(got, model.logits_full(0, follow, fa), ROUTE_TOL)
    # the full run above overwrote the entry's K/V rows: the follow-up puts them back, bit for bit
    assert model.logits(0, follow, fa) == got
    assert model.last_route() == "state_cache"


def test_state_boundary_at_a_chunk_end(gpu, model):
    prefix = _ids(10, 12)
    model.build_snapshot(0, prefix)
    ids, boundary = _state_prompt(prefix, 13, state_len=17)  # boundary = 10 + 17 + 3 = 30
    model.set_chunk(20)  # chunks from 10: [10, 30), [30, ...): the state ends exactly at a chunk end
    answers = _answers([len(ids) - 1], 80)
    model.logits(0, ids, answers)
    assert model.cached_states() == [boundary]
    follow = ids[:boundary] + _ids(9, 14)
    fa = _answers([len(follow) - 1], 90)
    got = model.logits(0, follow, fa)
    assert model.last_route() == "state_cache"
    _close(got, model.logits_full(0, follow, fa), ROUTE_TOL)


def test_lru_eviction_capacity_and_forgetting(gpu, model):
    prefix = _ids(8, 15)
    model.build_snapshot(0, prefix)
    model.set_state_cache(2)
    prompts = [_state_prompt(prefix, 100 + 10 * i, state_len=10 + i) for i in range(3)]
    for ids, _ in prompts:
        model.logits(0, ids, _answers([len(ids) - 1], 95))
    lens = [b for _, b in prompts]
    assert model.cached_states() == [lens[2], lens[1]]  # most recent first; the oldest was evicted
    # a follow-up on the evicted state runs from the snapshot and captures it again
    ids0, b0 = prompts[0]
    model.logits(0, ids0[:b0] + _ids(5, 16), _answers([b0 + 4], 96))
    assert model.last_route() == "snapshot"
    assert model.cached_states() == [lens[0], lens[2]]
    # a hit moves its entry to the front
    ids2, b2 = prompts[2]
    model.logits(0, ids2[:b2] + _ids(5, 17), _answers([b2 + 4], 97))
    assert model.last_route() == "state_cache"
    assert model.cached_states() == [lens[2], lens[0]]
    model.set_state_cache(1)
    assert model.cached_states() == [lens[2]]
    model.forget_states()
    assert model.cached_states() == []
    model.logits(0, ids2[:b2] + _ids(5, 17), _answers([b2 + 4], 97))
    assert model.last_route() == "snapshot"
    model.set_state_cache(0)
    model.forget_states()
    model.logits(0, ids2, _answers([len(ids2) - 1], 98))
    assert model.cached_states() == []
    with pytest.raises(AssertionError, match="at most 4"):
        model.set_state_cache(5)
    assert model.state_cache_capacity() == 0


def test_snapshot_rebuild_empties_the_cache(gpu, model):
    prefix = _ids(9, 18)
    model.build_snapshot(0, prefix)
    ids, b = _state_prompt(prefix, 19)
    model.logits(0, ids, _answers([len(ids) - 1], 99))
    assert model.cached_states() == [b]
    model.build_snapshot(0, prefix)
    assert model.cached_states() == []


@pytest.mark.parametrize("call,message", [
    (lambda m: m.logits(0, [], [(0, [1])]), "no input tokens"),
    (lambda m: m.logits(0, [1] * 129, [(0, [1])]), "at most 128"),
    (lambda m: m.logits(0, [1, 600], [(0, [1])]), "token id 600 is outside the 600-token vocabulary"),
    (lambda m: m.logits(0, [1, 2], []), "0 answers; a request has 1 to 4"),
    (lambda m: m.logits(0, [1, 2], [(0, [1])] * 5), "5 answers"),
    (lambda m: m.logits(0, [1, 2], [(2, [1])]), "answer 0: logit row 2 is past the 2-token input"),
    (lambda m: m.logits(0, [1, 2], [(1, [1]), (0, [])]), "answer 1: 0 candidates; a field has 1 to 6"),
    (lambda m: m.logits(0, [1, 2], [(1, [1] * 7)]), "answer 0: 7 candidates"),
    (lambda m: m.logits(0, [1, 2], [(1, [3, 600])]), "answer 0: candidate 600 is outside"),
    (lambda m: m.set_chunk(0), "chunk of 0 rows; the buffers hold 1 to 128"),
    (lambda m: m.set_chunk(129), "chunk of 129 rows"),
    (lambda m: m.build_snapshot(0, [1] * 128), "a 128-token prefix leaves no room for a request"),
    (lambda m: m.set_state_marker([]), "an empty state marker"),
])
def test_request_refusals(gpu, model, call, message):
    with pytest.raises(AssertionError, match=message):
        call(model)


def test_default_marker_and_chunk(gpu, kernels):
    m = Model(kernels.ctx, ModelConfig(layers=4, vocab=100, max_tokens=32, max_answers=2, max_cand=3))
    assert m.chunk() == 32 and m.pruning() and m.state_cache_capacity() == 2
    assert m.prefix_len() is None and m.last_route() is None and m.last_start() is None
    assert tuple(STATE_MARKER) == (550, 39087, 10485, 198)
    m.close()
