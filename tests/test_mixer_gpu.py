"""Parity of the forward kernels beside the GEMMs (embedding, conv, gated delta, gated norm, RoPE,
attention) on the GPU against the oracle's restatement of cpu_ref.rs, through the C ABI.

Tolerances (each written at its check): fp32 kernels that use the hardware exp (decide's fast-math
silu/sigmoid, common.h:5-8) are held to rtol 1e-4; fp16 outputs to one fp16 rounding of the oracle
plus that; the recurrence to a relative Frobenius error of 1e-4 (fp32 state vs the oracle's f64 dots);
attention to 2e-3 relative Frobenius (P is rounded to fp16 as the P·V operand, as in decide's kernel).
Gathers and copies are bit-exact."""

import numpy as np
import pytest

import oracle_lib as orc
from decide_amd import synth
from gpu_util import empty, full, sync, to_dev, to_host

pytestmark = pytest.mark.gpu

NK, DK, NV, DV = orc.NK, orc.DK, orc.NV, orc.DV
CONV_DIM, KEY_DIM, VALUE_DIM = orc.CONV_DIM, orc.KEY_DIM, orc.VALUE_DIM
LIN_IN_N, LIN_Z, LIN_B, LIN_A = 12352, 8192, 12288, 12320
ATT_IN_N, ATT_K, ATT_V = 10240, 8192, 9216


def u32(a):
    return to_dev(np.ascontiguousarray(a, dtype=np.uint32))


def test_embed_is_a_bitwise_widening(gpu, kernels, stream):
    vocab, h, t = 3001, 2560, 41
    table = synth.bf16_bits(synth.normal_f32(synth.seed_for(100), (vocab, h), 0.02))
    ids = synth.uniform_ids(synth.seed_for(101), t, vocab).astype(np.uint32)
    ids[:3] = [0, vocab - 1, 0]
    out = empty((t, h), np.float32)
    kernels.embed.embed(stream, (u32(ids), 0), (to_dev(table), 0), (out, 0), t, h)
    sync()
    np.testing.assert_array_equal(to_host(out).view(np.uint32), orc.embed_bf16(ids, table).view(np.uint32))


@pytest.mark.parametrize("t", [1, 2, 37])
def test_conv_silu_l2_matches_oracle(gpu, kernels, stream, t):
    p = synth.normal_f32(synth.seed_for(110), (t, LIN_IN_N), 1.0)
    prev = synth.normal_f32(synth.seed_for(111), (3, CONV_DIM), 1.0)
    w = synth.normal_f32(synth.seed_for(112), (CONV_DIM, 4), 0.5)
    q, k, v = (empty(s, np.float32) for s in ((t, NK, DK), (t, NK, DK), (t, NV, DV)))
    kernels.conv.conv_silu_l2(stream, (to_dev(p), 0), (to_dev(prev), 0), (to_dev(w), 0), (q, 0), (k, 0), (v, 0), t,
                              LIN_IN_N)
    sync()
    wq, wk, wv = orc.conv_silu_l2(p, t, prev, w)
    orc.assert_close("conv q", to_host(q), wq, atol=1e-6, rtol=1e-4)  # hardware exp in silu
    orc.assert_close("conv k", to_host(k), wk, atol=1e-6, rtol=1e-4)
    orc.assert_close("conv v", to_host(v), wv, atol=1e-6, rtol=1e-4)


@pytest.mark.parametrize("t", [1, 2, 3, 9])
def test_conv_state_update_is_exact_and_may_run_in_place(gpu, kernels, stream, t):
    p = synth.normal_f32(synth.seed_for(120), (t, LIN_IN_N), 1.0)
    prev = synth.normal_f32(synth.seed_for(121), (3, CONV_DIM), 1.0)
    pd, prev_d = to_dev(p), to_dev(prev)
    out = empty((3, CONV_DIM), np.float32)
    kernels.conv.conv_state_update(stream, (pd, 0), (prev_d, 0), (out, 0), t, LIN_IN_N)
    kernels.conv.conv_state_update(stream, (pd, 0), (prev_d, 0), (prev_d, 0), t, LIN_IN_N)  # in place
    sync()
    want = orc.conv_state_update(p, t, prev)
    np.testing.assert_array_equal(to_host(out), want)
    np.testing.assert_array_equal(to_host(prev_d), want)


def _delta_inputs(t, seed, a_log_std=0.5, a_shift=0.0):
    q = synth.normal_f32(synth.seed_for(seed), (t, NK, DK), 0.09)
    k = synth.normal_f32(synth.seed_for(seed + 1), (t, NK, DK), 0.09)
    v = synth.normal_f32(synth.seed_for(seed + 2), (t, NV, DV), 1.0)
    p = synth.normal_f32(synth.seed_for(seed + 3), (t, LIN_IN_N), 1.0)  # a, b read from P's columns
    p[:, LIN_A:LIN_A + NV] += a_shift
    a_log = synth.normal_f32(synth.seed_for(seed + 4), (NV,), a_log_std)
    dt_bias = synth.normal_f32(synth.seed_for(seed + 5), (NV,), 0.5)
    s0 = synth.normal_f32(synth.seed_for(seed + 6), (NV, DV, DK), 0.05)
    return q, k, v, p, a_log, dt_bias, s0


def _run_delta(kernels, stream, q, k, v, p, a_log, dt_bias, s0, t, in_place=False, write=True):
    qd, kd, vd, pd = to_dev(q), to_dev(k), to_dev(v), to_dev(p)
    sin = to_dev(s0)
    sout = sin if in_place else full(s0.shape, np.float32, np.nan)
    o = empty((t, NV, DV), np.float32)
    kernels.delta.gated_delta(stream, (qd, 0), (kd, 0), (vd, 0), (pd, LIN_A * 4), (pd, LIN_B * 4), (to_dev(a_log), 0),
                              (to_dev(dt_bias), 0), (sin, 0), (sout, 0), (o, 0), t, LIN_IN_N, write)
    sync()
    return to_host(o), to_host(sout)


@pytest.mark.parametrize("t", [1, 5, 64, 70, 200, 1000])
@pytest.mark.parametrize("impl", ["chunked", "sequential"])
def test_gated_delta_matches_oracle(gpu, kernels_delta_sequential, kernels_delta_chunked, stream, t, impl):
    q, k, v, p, a_log, dt_bias, s0 = _delta_inputs(t, 130)
    ks = kernels_delta_chunked if impl == "chunked" else kernels_delta_sequential
    o, s1 = _run_delta(ks, stream, q, k, v, p, a_log, dt_bias, s0, t)
    wo, ws = orc.gated_delta(q, k, v, p[:, LIN_A:LIN_A + NV], p[:, LIN_B:LIN_B + NV], a_log, dt_bias, s0, t)
    assert orc.rel_frobenius(o, wo) <= 1e-4, orc.rel_frobenius(o, wo)  # fp32 state vs f64 dots
    assert orc.rel_frobenius(s1, ws) <= 1e-4, orc.rel_frobenius(s1, ws)


@pytest.mark.parametrize("impl", ["chunked", "sequential"])
def test_gated_delta_unit_gate_known_answer(gpu, kernels_delta_sequential, kernels_delta_chunked, stream, impl):
    """decide's known answer (cpu_ref.rs:224-236) through both GPU implementations: one step, beta = 1 (b = 50),
    g = 1 (A_log = -inf), k = q = e_0 and v = 3 e_5 in head 0: o = v and S = v kᵀ exactly, all else zero."""
    kernels = kernels_delta_chunked if impl == "chunked" else kernels_delta_sequential
    t = 1
    q = np.zeros((t, NK, DK), np.float32)
    q[0, 0, 0] = 1.0
    k = q.copy()
    v = np.zeros((t, NV, DV), np.float32)
    v[0, 0, 5] = 3.0
    p = np.zeros((t, LIN_IN_N), np.float32)
    p[:, LIN_B:LIN_B + NV] = 50.0
    a_log = np.full(NV, -np.inf, np.float32)
    o, s1 = _run_delta(kernels, stream, q, k, v, p, a_log, np.zeros(NV, np.float32),
                       np.zeros((NV, DV, DK), np.float32), t)
    want_o = np.zeros_like(o)
    want_o[0, 0, 5] = 3.0
    want_s = np.zeros_like(s1)
    want_s[0, 5, 0] = 3.0
    np.testing.assert_array_equal(o, want_o)
    np.testing.assert_array_equal(s1, want_s)


@pytest.mark.parametrize("impl", ["chunked", "sequential"])
def test_gated_delta_renormalises_a_fast_decay(gpu, kernels_delta_sequential, kernels_delta_chunked, stream, impl):
    """g ≈ e^-37 per token: the sequential kernel's running scale drops below 2^-60 within two tokens,
    the chunked kernel's within-chunk ratios γ_i/γ_j underflow to 0."""
    kernels = kernels_delta_chunked if impl == "chunked" else kernels_delta_sequential
    t = 12
    q, k, v, p, a_log, dt_bias, s0 = _delta_inputs(t, 140, a_log_std=0.0, a_shift=0.0)
    a_log[:] = 2.0
    p[:, LIN_A:LIN_A + NV] = 5.0
    dt_bias[:] = 0.0
    o, s1 = _run_delta(kernels, stream, q, k, v, p, a_log, dt_bias, s0, t)
    wo, ws = orc.gated_delta(q, k, v, p[:, LIN_A:LIN_A + NV], p[:, LIN_B:LIN_B + NV], a_log, dt_bias, s0, t)
    assert np.isfinite(o).all() and np.isfinite(s1).all()
    assert orc.rel_frobenius(o, wo) <= 1e-4
    assert orc.rel_frobenius(s1, ws) <= 1e-4


@pytest.mark.parametrize("impl", ["chunked", "sequential"])
def test_gated_delta_in_place_chunks_and_no_write(gpu, kernels_delta_sequential, kernels_delta_chunked, stream, impl):
    kernels = kernels_delta_chunked if impl == "chunked" else kernels_delta_sequential
    t1, t2 = 40, 30
    q, k, v, p, a_log, dt_bias, s0 = _delta_inputs(t1 + t2, 150)
    whole_o, whole_s = _run_delta(kernels, stream, q, k, v, p, a_log, dt_bias, s0, t1 + t2)
    o1, s_mid = _run_delta(kernels, stream, q[:t1], k[:t1], v[:t1], p[:t1], a_log, dt_bias, s0, t1, in_place=True)
    o2, s_end = _run_delta(kernels, stream, q[t1:], k[t1:], v[t1:], p[t1:], a_log, dt_bias, s_mid, t2, in_place=True)
    assert orc.rel_frobenius(np.concatenate([o1, o2]), whole_o) <= 1e-5
    assert orc.rel_frobenius(s_end, whole_s) <= 1e-5
    _, untouched = _run_delta(kernels, stream, q, k, v, p, a_log, dt_bias, s0, 3, write=False)
    assert np.isnan(untouched).all(), "write_state = 0 must leave state_out untouched"


@pytest.mark.parametrize("t", [1, 70, 2307])
def test_conv_gated_delta_chunked_equals_the_two_steps(gpu, kernels_delta_chunked, stream, t):
    """dh_conv_gated_delta_chunked, whose prep kernel forms q, k and v from p itself, against dh_conv_silu_l2 then
    dh_gated_delta on the chunked path: q, o and the final state bit for bit, from a nonzero conv state (raw rows
    before the first) and a nonzero state; t = 70 and 2,307 end inside a chunk."""
    ks = kernels_delta_chunked
    p = synth.normal_f32(synth.seed_for(190), (t, LIN_IN_N), 1.0)
    prev = synth.normal_f32(synth.seed_for(191), (3, CONV_DIM), 1.0)
    w = synth.normal_f32(synth.seed_for(192), (CONV_DIM, 4), 0.5)
    a_log = synth.normal_f32(synth.seed_for(193), (NV,), 0.5)
    dt_bias = synth.normal_f32(synth.seed_for(194), (NV,), 0.5)
    s0 = synth.normal_f32(synth.seed_for(195), (NV, DV, DK), 0.05)
    pd, prevd, wd, ad, dd, sd = (to_dev(x) for x in (p, prev, w, a_log, dt_bias, s0))
    q1, k1, v1 = (empty(s, np.float32) for s in ((t, NK, DK), (t, NK, DK), (t, NV, DV)))
    o1, o2 = empty((t, NV, DV), np.float32), empty((t, NV, DV), np.float32)
    s1, s2 = full(s0.shape, np.float32, np.nan), full(s0.shape, np.float32, np.nan)
    q2 = full((t, NK, DK), np.float32, np.nan)
    ks.conv.conv_silu_l2(stream, (pd, 0), (prevd, 0), (wd, 0), (q1, 0), (k1, 0), (v1, 0), t, LIN_IN_N)
    ks.delta.gated_delta(stream, (q1, 0), (k1, 0), (v1, 0), (pd, LIN_A * 4), (pd, LIN_B * 4), (ad, 0), (dd, 0),
                         (sd, 0), (s1, 0), (o1, 0), t, LIN_IN_N, True)
    ks.delta.conv_gated_delta_chunked(stream, (pd, 0), (prevd, 0), (wd, 0), (q2, 0), (pd, LIN_A * 4),
                                      (pd, LIN_B * 4), (ad, 0), (dd, 0), (sd, 0), (s2, 0), (o2, 0), t, LIN_IN_N,
                                      LIN_IN_N, True)
    sync()
    for name, a, b in (("q", q1, q2), ("o", o1, o2), ("state", s1, s2)):
        np.testing.assert_array_equal(to_host(b).view(np.uint32), to_host(a).view(np.uint32), err_msg=name)


@pytest.mark.parametrize("t", [1, 33])
def test_gated_rmsnorm_silu_matches_oracle(gpu, kernels, stream, t):
    o = synth.normal_f32(synth.seed_for(160), (t, NV, DV), 1.0)
    p = synth.normal_f32(synth.seed_for(161), (t, LIN_IN_N), 1.0)
    w = synth.normal_f32(synth.seed_for(162), (DV,), 1.0)
    y = empty((t, VALUE_DIM), np.float16)
    pd = to_dev(p)
    kernels.gnorm.gated_rmsnorm_silu(stream, (to_dev(o), 0), (pd, LIN_Z * 4), (to_dev(w), 0), (y, 0), t, LIN_IN_N)
    sync()
    want = orc.gated_rmsnorm_silu(o, p[:, LIN_Z:], w, t)
    got = to_host(y).astype(np.float32)
    orc.assert_close("gnorm", got, orc.f16_round(want), atol=2e-3, rtol=2e-3)  # one fp16 rounding + hardware exp


def _inv_freq_dev():
    return to_dev(orc.inv_freq())


@pytest.mark.parametrize("rows", [1, 19])
def test_q_norm_rope_matches_oracle(gpu, kernels, stream, rows):
    pq = synth.normal_f32(synth.seed_for(170), (rows, ATT_IN_N), 1.5)
    qw = synth.normal_f32(synth.seed_for(171), (256,), 0.1)
    qpos = np.array([(7919 * r) % 8192 for r in range(rows)], np.uint32)
    qo = empty((rows, 16, 256), np.float16)
    kernels.rope.q_norm_rope(stream, (to_dev(pq), 0), (to_dev(qw), 0), (_inv_freq_dev(), 0), (u32(qpos), 0), (qo, 0),
                             rows, ATT_IN_N)
    sync()
    got = to_host(qo).astype(np.float32)
    for r in range(rows):
        for h in range(16):
            want = orc.head_norm_rope(pq[r, h * 256:(h + 1) * 256], qw, int(qpos[r]))
            orc.assert_close(f"q_norm_rope r{r} h{h}", got[r, h], orc.f16_round(want), atol=2e-3, rtol=2e-3)


def test_kv_norm_rope_matches_oracle(gpu, kernels, stream):
    rows, pos0 = 13, 8000
    pkv = synth.normal_f32(synth.seed_for(180), (rows, ATT_IN_N), 1.5)
    kw = synth.normal_f32(synth.seed_for(181), (256,), 0.1)
    kc = full((8192, 4, 256), np.float16, 0)
    vc = full((8192, 4, 256), np.float16, 0)
    kernels.rope.kv_norm_rope(stream, (to_dev(pkv), 0), (to_dev(kw), 0), (_inv_freq_dev(), 0), (kc, 0), (vc, 0), rows,
                              ATT_IN_N, ATT_K, ATT_V, pos0)
    sync()
    kh, vh = to_host(kc), to_host(vc)
    assert not kh[:pos0].any() and not vh[:pos0].any(), "rows before pos0 must stay untouched"
    for r in range(rows):
        for j in range(4):
            want = orc.head_norm_rope(pkv[r, ATT_K + j * 256:ATT_K + (j + 1) * 256], kw, pos0 + r)
            orc.assert_close(f"k r{r} j{j}", kh[pos0 + r, j].astype(np.float32), orc.f16_round(want), atol=2e-3,
                             rtol=2e-3)
            np.testing.assert_array_equal(vh[pos0 + r, j],
                                          pkv[r, ATT_V + j * 256:ATT_V + (j + 1) * 256].astype(np.float16))


def _attention_case(rows, npos, qpos, seed):
    q = synth.normal_f16(synth.seed_for(seed), (rows, 16, 256), 1.0)
    kc = synth.normal_f16(synth.seed_for(seed + 1), (npos, 4, 256), 1.0)
    vc = synth.normal_f16(synth.seed_for(seed + 2), (npos, 4, 256), 1.0)
    pq = synth.normal_f32(synth.seed_for(seed + 3), (rows, ATT_IN_N), 1.0)
    return q, kc, vc, pq, np.asarray(qpos, np.uint32)


# (2307, 2307): config 5's full prompt, 2,307-key causal attention over every row, its long query blocks cut into
# two key pieces; (70, 1200, "scattered"): positions in no order, so one workgroup's 32 rows reach very different
# key counts; (600, 2307, "scattered"): every query block cut into five pieces, the last one long, with rows that
# see no key of some pieces; (300, 300): five pieces per query block
@pytest.mark.parametrize("rows,npos,kind", [(37, 37, "prefill"), (300, 300, "prefill"), (3, 900, "answers"),
                                            (16, 16, "prefill"), (1, 1, "prefill"), (2307, 2307, "prefill"),
                                            (70, 1200, "scattered"), (600, 2307, "scattered")])
def test_attention_matches_oracle(gpu, kernels, stream, rows, npos, kind):
    if kind == "prefill":
        qpos = np.arange(rows)
    elif kind == "answers":
        qpos = np.array([899, 17, 512])[:rows]
    else:
        qpos = np.random.default_rng(7).integers(0, npos, rows)
    q, kc, vc, pq, qpos = _attention_case(rows, npos, qpos, 190)
    y = empty((rows, 4096), np.float16)
    kernels.attn.attention(stream, (to_dev(q), 0), (to_dev(kc), 0), (to_dev(vc), 0), (to_dev(pq), 0), (u32(qpos), 0),
                           (y, 0), rows, ATT_IN_N)
    sync()
    want = orc.attention(q.astype(np.float32), qpos, kc.astype(np.float32), vc.astype(np.float32), pq[:, 4096:])
    got = to_host(y).astype(np.float32)
    assert np.isfinite(got).all()
    e = orc.rel_frobenius(got, want)
    assert e <= 2e-3, f"attention rel. Frobenius {e:.2e}"  # fp16 P operand and fp16 output


def test_attention_key_pieces_keep_rows_independent(gpu, kernels, stream):
    """96 rows at scattered positions: their query blocks' keys are cut into pieces (every 64 keys at the shortest)
    and merged. A row whose position is below 64 sees one piece only and gets bit for bit the result of a call
    with that row alone (never cut); a row past it matches the one-row call within one fp16 rounding."""
    rows = 96
    qpos = np.random.default_rng(11).integers(0, 1200, rows)
    qpos[::7] = np.arange(0, 64, 64 / len(qpos[::7])).astype(np.int64)[:len(qpos[::7])]
    q, kc, vc, pq, qpos = _attention_case(rows, 1200, qpos, 210)
    y = empty((rows, 4096), np.float16)
    args = ((to_dev(kc), 0), (to_dev(vc), 0))
    kernels.attn.attention(stream, (to_dev(q), 0), *args, (to_dev(pq), 0), (u32(qpos), 0), (y, 0), rows, ATT_IN_N)
    sync()
    got = to_host(y)
    early = [r for r in range(rows) if qpos[r] < 64]
    late = [r for r in range(rows) if qpos[r] >= 64][:12]
    assert len(early) >= 8 and len(late) == 12
    for r in early + late:
        y1 = empty((1, 4096), np.float16)
        kernels.attn.attention(stream, (to_dev(q[r:r + 1]), 0), *args, (to_dev(pq[r:r + 1]), 0),
                               (u32(qpos[r:r + 1]), 0), (y1, 0), 1, ATT_IN_N)
        sync()
        one = to_host(y1)[0]
        if qpos[r] < 64:
            np.testing.assert_array_equal(got[r], one, err_msg=f"row {r} at {qpos[r]}")
        else:
            np.testing.assert_allclose(got[r].astype(np.float32), one.astype(np.float32), rtol=1e-3, atol=1e-4,
                                       err_msg=f"row {r} at {qpos[r]}")


def test_attention_rows_are_independent_of_their_neighbours(gpu, kernels, stream):
    """Row r's output depends only on its own query, position and cache rows 0..=qpos[r]."""
    rows = 40
    q, kc, vc, pq, qpos = _attention_case(rows, 300, np.arange(200, 240), 200)
    y = empty((rows, 4096), np.float16)
    args = ((to_dev(kc), 0), (to_dev(vc), 0))
    kernels.attn.attention(stream, (to_dev(q), 0), *args, (to_dev(pq), 0), (u32(qpos), 0), (y, 0), rows, ATT_IN_N)
    y1 = empty((1, 4096), np.float16)
    r = 21
    kernels.attn.attention(stream, (to_dev(q[r:r + 1]), 0), *args, (to_dev(pq[r:r + 1]), 0), (u32(qpos[r:r + 1]), 0),
                           (y1, 0), 1, ATT_IN_N)
    sync()
    np.testing.assert_array_equal(to_host(y)[r], to_host(y1)[0])
