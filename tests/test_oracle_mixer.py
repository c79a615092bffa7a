"""Pins the oracle's restatement of decide's non-GEMM forward pieces (cpu_ref.rs:55-188) with closed
forms, known answers and independent float64 computations, so that a dropped term, a wrong index or a
swapped operand in oracle/oracle_mixer.c fails here. CPU only."""

import numpy as np
import pytest

import oracle_lib as orc
from decide_amd import synth

NK, DK, NV, DV = orc.NK, orc.DK, orc.NV, orc.DV
CONV_DIM, KEY_DIM, VALUE_DIM = orc.CONV_DIM, orc.KEY_DIM, orc.VALUE_DIM


def silu64(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def sig64(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


# ---- conv_silu_l2 / conv_state_update (cpu_ref.rs:55-95)

def _conv_inputs(t, seed=1):
    p = synth.normal_f32(synth.seed_for(seed), (t, CONV_DIM + 64), 1.0)
    prev = synth.normal_f32(synth.seed_for(seed + 1), (3, CONV_DIM), 1.0)
    return p, prev


@pytest.mark.parametrize("tap", [3, 0, 1])
def test_conv_one_tap_kernel_is_a_shifted_silu(tap):
    t = 6
    p, prev = _conv_inputs(t)
    w = np.zeros((CONV_DIM, 4), np.float32)
    w[:, tap] = 1.0
    q, k, v = orc.conv_silu_l2(p, t, prev, w)
    shift = 3 - tap
    for s in range(t):
        src = p[s - shift, :CONV_DIM] if s - shift >= 0 else prev[3 + s - shift]
        want = silu64(src)
        np.testing.assert_allclose(v[s].ravel(), want[2 * KEY_DIM:], rtol=2e-6, atol=1e-7)
        for h in range(NK):
            seg = want[h * DK:(h + 1) * DK]
            np.testing.assert_allclose(q[s, h], seg / np.sqrt((seg ** 2).sum() + 1e-6) / np.sqrt(DK), rtol=1e-5,
                                       atol=1e-7)
            seg = want[KEY_DIM + h * DK:KEY_DIM + (h + 1) * DK]
            np.testing.assert_allclose(k[s, h], seg / np.sqrt((seg ** 2).sum() + 1e-6), rtol=1e-5, atol=1e-7)


def test_conv_q_k_are_unit_vectors_and_taps_are_ordered_oldest_first():
    t = 5
    p, prev = _conv_inputs(t, 5)
    w = synth.normal_f32(synth.seed_for(7), (CONV_DIM, 4), 0.5)
    q, k, v = orc.conv_silu_l2(p, t, prev, w)
    np.testing.assert_allclose(np.linalg.norm(q.astype(np.float64), axis=-1) * np.sqrt(DK), 1.0, atol=1e-5)
    np.testing.assert_allclose(np.linalg.norm(k.astype(np.float64), axis=-1), 1.0, atol=1e-5)
    # channel c of row s = silu(Σ_j w[c, j] · raw[s − 3 + j])
    raw = np.concatenate([prev, p[:, :CONV_DIM]], axis=0).astype(np.float64)
    acc = sum(w[:, j].astype(np.float64) * raw[3 - 3 + j: 3 - 3 + j + t] for j in range(4))
    np.testing.assert_allclose(v.reshape(t, -1), silu64(acc)[:, 2 * KEY_DIM:], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("t", [1, 2, 3, 7])
def test_conv_state_update_keeps_the_last_three_raw_rows(t):
    p, prev = _conv_inputs(t, 9)
    out = orc.conv_state_update(p, t, prev)
    raw = np.concatenate([prev, p[:, :CONV_DIM]], axis=0)
    np.testing.assert_array_equal(out, raw[-3:])


# ---- gated_delta (cpu_ref.rs:101-129)

def _delta_inputs(t, seed, state_std=0.0):
    q = synth.normal_f32(synth.seed_for(seed), (t, NK, DK), 0.1)
    k = synth.normal_f32(synth.seed_for(seed + 1), (t, NK, DK), 0.1)
    v = synth.normal_f32(synth.seed_for(seed + 2), (t, NV, DV), 1.0)
    ab = synth.normal_f32(synth.seed_for(seed + 3), (t, 2 * NV), 1.0)
    a_log = synth.normal_f32(synth.seed_for(seed + 4), (NV,), 0.5)
    dt_bias = synth.normal_f32(synth.seed_for(seed + 5), (NV,), 0.5)
    st = synth.normal_f32(synth.seed_for(seed + 6), (NV, DV, DK), state_std) if state_std else np.zeros(
        (NV, DV, DK), np.float32)
    return q, k, v, ab[:, :NV], ab[:, NV:], a_log, dt_bias, st


def _gate(a, dt_bias, a_log):
    x = np.float64(a) + np.float64(dt_bias)
    sp = x if x > 20 else np.log1p(np.exp(x))
    return np.exp(-np.exp(np.float64(a_log)) * sp)


def test_delta_one_token_from_zero_state_closed_form():
    q, k, v, a, b, a_log, dt_bias, st = _delta_inputs(1, 20)
    o, s1 = orc.gated_delta(q, k, v, a, b, a_log, dt_bias, st, 1)
    for h in range(NV):
        hk = h // 2
        beta = sig64(b[0, h])
        kq = np.dot(k[0, hk].astype(np.float64), q[0, hk].astype(np.float64))
        np.testing.assert_allclose(o[0, h], beta * kq * v[0, h].astype(np.float64), rtol=1e-4, atol=1e-7)
        # S = β v kᵀ (row dv = β v[dv] k)
        np.testing.assert_allclose(s1[h], beta * np.outer(v[0, h], k[0, hk]), rtol=1e-5, atol=1e-8)


def test_delta_rule_with_unit_gate_is_a_delta_update():
    """decide's own known answer (cpu_ref.rs:224-236): one step with beta = 1 (b = 50) and g = 1 (A_log = -inf,
    so exp(A_log) = 0): S = v kᵀ with k = e_0, so o = S q = v; every other value stays zero."""
    t = 1
    q = np.zeros((t, NK, DK), np.float32)
    q[0, 0, 0] = 1.0
    k = q.copy()
    v = np.zeros((t, NV, DV), np.float32)
    v[0, 0, 5] = 3.0  # head 0, column 5
    a, b = np.zeros((t, NV), np.float32), np.full((t, NV), 50.0, np.float32)
    st = np.zeros((NV, DV, DK), np.float32)
    o, s1 = orc.gated_delta(q, k, v, a, b, np.full(NV, -np.inf, np.float32), np.zeros(NV, np.float32), st, t)
    assert abs(o[0, 0, 5] - 3.0) < 1e-5
    assert abs(s1[0, 5, 0] - 3.0) < 1e-5  # state[5 * DK]: head 0, value row 5, key column 0
    o[0, 0, 5] = 0.0
    s1[0, 5, 0] = 0.0
    assert not o.any() and not s1.any()


def test_delta_without_writes_only_decays_the_state():
    t = 4
    q, k, v, a, b, a_log, dt_bias, st = _delta_inputs(t, 30, state_std=0.3)
    b[:] = -200.0  # β = σ(−200) = 0 in f32: nothing is written
    o, s_t = orc.gated_delta(q, k, v, a, b, a_log, dt_bias, st, t)
    s = st.astype(np.float64)
    for s_i in range(t):
        for h in range(NV):
            g = _gate(a[s_i, h], dt_bias[h], a_log[h])
            s[h] *= g
            np.testing.assert_allclose(o[s_i, h], s[h] @ q[s_i, h // 2].astype(np.float64), rtol=2e-4, atol=1e-6)
    np.testing.assert_allclose(s_t, s, rtol=1e-4, atol=1e-8)


def test_delta_matches_a_matrix_form_recurrence():
    """Independent float64 restatement in matrix form: S ← g·S; S ← S + β (v − S k) kᵀ; o = S q."""
    t = 6
    q, k, v, a, b, a_log, dt_bias, st = _delta_inputs(t, 40, state_std=0.05)
    o, s_t = orc.gated_delta(q, k, v, a, b, a_log, dt_bias, st, t)
    s = st.astype(np.float64)
    for s_i in range(t):
        for h in range(NV):
            kk, qq = k[s_i, h // 2].astype(np.float64), q[s_i, h // 2].astype(np.float64)
            s[h] *= _gate(a[s_i, h], dt_bias[h], a_log[h])
            s[h] += sig64(b[s_i, h]) * np.outer(v[s_i, h] - s[h] @ kk, kk)
            np.testing.assert_allclose(o[s_i, h], s[h] @ qq, rtol=1e-3, atol=1e-5)
    np.testing.assert_allclose(s_t, s, rtol=1e-3, atol=1e-6)


def test_softplus_branches():
    assert orc.softplus(25.0) == 25.0
    assert abs(orc.softplus(0.0) - np.log(2.0)) < 1e-7
    assert abs(orc.softplus(-5.0) - np.log1p(np.exp(-5.0))) < 1e-7


# ---- gated_rmsnorm_silu (cpu_ref.rs:132-145)

def test_gated_rmsnorm_silu_known_answer():
    t = 2
    o = np.full((t, NV, DV), 2.0, np.float32)
    z = np.zeros((t, VALUE_DIM + 8), np.float32)
    z[0, :] = 1.0
    w = np.full(DV, 1.5, np.float32)
    y = orc.gated_rmsnorm_silu(o, z, w, t)
    want = 2.0 / np.sqrt(4.0 + 1e-6) * 1.5 * (1.0 / (1.0 + np.exp(-1.0)))
    np.testing.assert_allclose(y[0], want, rtol=1e-6)
    np.testing.assert_array_equal(y[1], 0.0)  # silu(0) = 0


def test_gated_rmsnorm_silu_uses_its_own_head_segment():
    t = 1
    o = synth.normal_f32(synth.seed_for(50), (t, NV, DV), 1.0)
    o[0, 7] *= 100.0  # one loud head must not change the others
    z = synth.normal_f32(synth.seed_for(51), (t, VALUE_DIM), 1.0)
    w = synth.normal_f32(synth.seed_for(52), (DV,), 1.0)
    y = orc.gated_rmsnorm_silu(o, z, w, t).reshape(NV, DV)
    for h in (0, 7, 31):
        seg = o[0, h].astype(np.float64)
        want = seg / np.sqrt((seg ** 2).mean() + 1e-6) * w * silu64(z[0, h * DV:(h + 1) * DV])
        np.testing.assert_allclose(y[h], want, rtol=1e-5, atol=1e-6)


# ---- head_norm_rope (cpu_ref.rs:149-162)

def test_inv_freq_formula():
    f = orc.inv_freq()
    np.testing.assert_allclose(f, 1.0 / (1e7 ** (np.arange(32) * 2 / 64.0)), rtol=1e-6)
    assert f[0] == 1.0


def test_rope_at_position_zero_is_the_plain_norm():
    seg = synth.normal_f32(synth.seed_for(60), (256,), 2.0)
    w = synth.normal_f32(synth.seed_for(61), (256,), 0.1)
    out = orc.head_norm_rope(seg, w, 0)
    s = seg.astype(np.float64)
    np.testing.assert_allclose(out, s / np.sqrt((s ** 2).mean() + 1e-6) * (1.0 + w), rtol=1e-5)


def test_rope_rotates_pairs_i_and_i_plus_32():
    seg = synth.normal_f32(synth.seed_for(62), (256,), 1.0)
    w = np.zeros(256, np.float32)
    base = orc.head_norm_rope(seg, w, 0)
    for pos in (1, 1000, 2306):
        out = orc.head_norm_rope(seg, w, pos)
        np.testing.assert_array_equal(out[64:], base[64:])  # dims past ROT_DIM untouched
        np.testing.assert_allclose(out[:32] ** 2 + out[32:64] ** 2, base[:32] ** 2 + base[32:64] ** 2, rtol=1e-5)
        ang = pos * orc.inv_freq().astype(np.float64)
        np.testing.assert_allclose(out[:32], base[:32] * np.cos(ang) - base[32:64] * np.sin(ang), atol=2e-5)
        np.testing.assert_allclose(out[32:64], base[32:64] * np.cos(ang) + base[:32] * np.sin(ang), atol=2e-5)


# ---- attention (cpu_ref.rs:167-188)

def test_attention_first_position_sees_only_itself():
    q = synth.normal_f32(synth.seed_for(70), (1, 16, 256), 1.0)
    kc = synth.normal_f32(synth.seed_for(71), (3, 4, 256), 1.0)
    vc = synth.normal_f32(synth.seed_for(72), (3, 4, 256), 1.0)
    gate = synth.normal_f32(synth.seed_for(73), (1, 4096), 1.0)
    out = orc.attention(q, [0], kc, vc, gate).reshape(16, 256)
    for h in range(16):
        np.testing.assert_allclose(out[h], vc[0, h // 4] * sig64(gate[0, h * 256:(h + 1) * 256]), rtol=1e-6)


def test_attention_equal_scores_average_the_values():
    kc = np.tile(synth.normal_f32(synth.seed_for(74), (1, 4, 256), 1.0), (6, 1, 1))
    vc = synth.normal_f32(synth.seed_for(75), (6, 4, 256), 1.0)
    q = synth.normal_f32(synth.seed_for(76), (2, 16, 256), 1.0)
    gate = np.full((2, 4096), 50.0, np.float32)  # σ(50) = 1 in f32
    out = orc.attention(q, [5, 2], kc, vc, gate).reshape(2, 16, 256)
    for h in range(16):
        np.testing.assert_allclose(out[0, h], vc[:6, h // 4].astype(np.float64).mean(0), rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(out[1, h], vc[:3, h // 4].astype(np.float64).mean(0), rtol=1e-5, atol=1e-6)


def test_attention_matches_numpy_softmax():
    npos = 7
    q = synth.normal_f32(synth.seed_for(77), (3, 16, 256), 0.3)
    kc = synth.normal_f32(synth.seed_for(78), (npos, 4, 256), 0.3)
    vc = synth.normal_f32(synth.seed_for(79), (npos, 4, 256), 1.0)
    gate = synth.normal_f32(synth.seed_for(80), (3, 4096 + 32), 1.0)
    qpos = [6, 0, 3]
    out = orc.attention(q, qpos, kc, vc, gate).reshape(3, 16, 256)
    for r, pos in enumerate(qpos):
        for h in range(16):
            s = kc[:pos + 1, h // 4].astype(np.float64) @ q[r, h].astype(np.float64) / 16.0
            p = np.exp(s - s.max())
            want = (p / p.sum()) @ vc[:pos + 1, h // 4].astype(np.float64) * sig64(gate[r, h * 256:(h + 1) * 256])
            np.testing.assert_allclose(out[r, h], want, rtol=1e-5, atol=1e-6)


# ---- embedding gather

def test_embed_widens_bf16_bitwise():
    table = synth.bf16_bits(synth.normal_f32(synth.seed_for(90), (50, 64), 0.02))
    ids = np.array([3, 0, 49, 3], np.uint32)
    out = orc.embed_bf16(ids, table)
    want = (table[ids].astype(np.uint32) << 16).view(np.float32)
    np.testing.assert_array_equal(out.view(np.uint32), want.view(np.uint32))


def chunked_delta64(q, k, v, a, b, a_log, dt_bias, s0, C=64):
    """The chunked (WY-form) gated delta rule in float64, the formulation the GPU kernel uses:
    per chunk, A_ij = β_i (γ_i/γ_j) k_i·k_j (i > j), T = (I + A)⁻¹, W = T diag(βγ) K, U = T diag(β) V,
    V' = U − W Sᵀ, O = diag(γ) Q Sᵀ + (Q Kᵀ ⊙ Γ) V' (Γ_ij = γ_i/γ_j, i ≥ j), S ← γ_C S + V'ᵀ diag(γ_C/γ) K."""
    t = q.shape[0]
    S = s0.astype(np.float64).copy()
    o = np.zeros((t, NV, DV))
    A_ = np.exp(a_log.astype(np.float64))
    for c0 in range(0, t, C):
        n = min(C, t - c0)
        for h in range(NV):
            hk = h // 2
            x = a[c0:c0 + n, h].astype(np.float64) + dt_bias[h]
            lam = -A_[h] * np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))
            Lg = np.cumsum(lam)
            beta = sig64(b[c0:c0 + n, h])
            K = k[c0:c0 + n, hk].astype(np.float64)
            Q = q[c0:c0 + n, hk].astype(np.float64)
            V = v[c0:c0 + n, h].astype(np.float64)
            R = np.exp(Lg[:, None] - Lg[None, :])
            Am = np.tril(beta[:, None] * R * (K @ K.T), -1)
            T = np.linalg.inv(np.eye(n) + Am)
            W = T @ (beta[:, None] * np.exp(Lg)[:, None] * K)
            U = T @ (beta[:, None] * V)
            Vp = U - W @ S[h].T
            M = np.tril(R * (Q @ K.T))
            o[c0:c0 + n, h] = np.exp(Lg)[:, None] * (Q @ S[h].T) + M @ Vp
            S[h] = np.exp(Lg[-1]) * S[h] + Vp.T @ (np.exp(Lg[-1] - Lg)[:, None] * K)
    return o, S


@pytest.mark.parametrize("t", [1, 5, 64, 150])
def test_chunked_delta_formulation_equals_the_recurrence(t):
    """Pins the chunked form the GPU's chunk kernels implement against the oracle's token-by-token rule."""
    q, k, v, a, b, a_log, dt_bias, st = _delta_inputs(t, 60, state_std=0.05)
    o_ref, s_ref = orc.gated_delta(q, k, v, a, b, a_log, dt_bias, st, t)
    o, s = chunked_delta64(q, k, v, a, b, a_log, dt_bias, st)
    np.testing.assert_allclose(o, o_ref, rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(s, s_ref, rtol=1e-4, atol=1e-7)
