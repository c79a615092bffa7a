"""GPU parity of the GEMM operator (dh_gemm_nt / dh_gemm_nt_grouped) against the oracle.

Everything goes through the C ABI (decide_amd.kernels wraps it with ctypes);
device memory comes from decide_amd.hip (the same HIP runtime the library links). Oracle: cpu_ref::gemm_nt restated in C
(f64 sums, fp32 result) on the same fp16 inputs. Bars: relative Frobenius
error <= 1e-3 per GEMM (BASELINE), bit-exact where the mathematics makes the
fp32 result exact (integer-valued inputs).
"""

import numpy as np
import pytest

import oracle_lib as orc
from decide_amd import synth
from decide_amd.kernels import Epilogue, variants
from gpu_util import check_gemm, empty, full, sample_rows, swiglu_f16, sync, to_dev, to_host

pytestmark = pytest.mark.gpu

SMALL = [(1, 32, 32), (7, 64, 96), (17, 32, 64), (33, 96, 160), (5, 128, 320), (64, 256, 512), (203, 288, 128)]


def run_gemm(kernels, stream, x, w, epi, y0=None, ldy=None):
    m, k = x.shape
    n = w.shape[0]
    out_cols = n // 2 if epi == Epilogue.SwigluF16 else n
    ldy = ldy or out_cols
    dt = np.float32 if epi in (Epilogue.StoreF32, Epilogue.AddF32) else np.float16
    if y0 is not None:
        y = to_dev(y0)
    else:
        y = full((m, ldy), dt, np.nan)
    xd, wd = to_dev(x), to_dev(w)
    kernels.gemm.gemm(stream, (xd, 0), (wd, 0), (y, 0), m, n, k, k, k, ldy, epi)
    sync()
    return to_host(y)[:, :out_cols].astype(np.float32)


def oracle_epi(x, w, epi, y0=None):
    y = orc.gemm_nt_f16(x, w)
    if epi == Epilogue.StoreF32:
        return y
    if epi == Epilogue.StoreF16:
        return orc.f16_round(y)
    if epi == Epilogue.AddF32:
        return y0 + y
    return swiglu_f16(y)


def inputs(m, n, k, seed):
    x = synth.normal_f16(synth.seed_for(seed), (m, k), 1.0)
    w = synth.normal_f16(synth.seed_for(seed + 1), (n, k), 0.02)
    return x, w


@pytest.mark.parametrize("m,n,k", SMALL)
@pytest.mark.parametrize("epi", list(Epilogue))
def test_small_shapes_planner(gpu, kernels, stream, m, n, k, epi):
    x, w = inputs(m, n, k, 10 + m)
    y0 = synth.normal_f32(synth.seed_for(99), (m, n), 1.0) if epi == Epilogue.AddF32 else None
    got = run_gemm(kernels, stream, x, w, epi, y0)
    want = oracle_epi(x, w, epi, y0)
    check_gemm(f"m{m} n{n} k{k} {epi.name}", got, want)
    tol = 2e-3 if epi in (Epilogue.StoreF16, Epilogue.SwigluF16) else 1e-4
    orc.assert_close(f"m{m} n{n} k{k} {epi.name}", got, want, atol=tol, rtol=tol)


# the weight-streaming kernel (M <= 16, K % 128 == 0): split-K and single-pass shapes, ragged M, N tails
STREAM = [(1, 32, 128), (3, 2560, 9216), (16, 4096, 2560), (7, 96, 384), (16, 64, 1024), (13, 2048, 2560),
          (2, 160, 4096)]


@pytest.mark.parametrize("m,n,k", STREAM)
@pytest.mark.parametrize("epi", list(Epilogue))
def test_weight_streaming_kernel(gpu, kernels, stream, m, n, k, epi):
    from decide_amd import _lib

    assert kernels.gemm.plan(m, n, k, epi)["variant"] == _lib.DH_GEMM_STREAM_VARIANT
    x, w = inputs(m, n, k, 700 + m + n)
    y0 = synth.normal_f32(synth.seed_for(98), (m, n), 1.0) if epi == Epilogue.AddF32 else None
    got = run_gemm(kernels, stream, x, w, epi, y0)
    want = oracle_epi(x, w, epi, y0)
    check_gemm(f"stream m{m} n{n} k{k} {epi.name}", got, want)
    tol = 2e-3 if epi in (Epilogue.StoreF16, Epilogue.SwigluF16) else 1e-4
    orc.assert_close(f"stream m{m} n{n} k{k} {epi.name}", got, want, atol=tol, rtol=tol)
    assert np.array_equal(got, run_gemm(kernels, stream, x, w, epi, y0)), "not deterministic"


def test_weight_streaming_grouped(gpu, kernels, stream):
    """A grouped launch of three members (SwiGLU, fp32 and fp16) at M = 3 on the streaming kernel."""
    from decide_amd import _lib
    from decide_amd.kernels import addr

    m, k = 3, 2560
    x = synth.normal_f16(synth.seed_for(801), (m, k), 1.0)
    ws = [synth.normal_f16(synth.seed_for(802 + i), (n, k), 0.02) for i, n in enumerate((512, 224, 96))]
    epis = [Epilogue.SwigluF16, Epilogue.StoreF32, Epilogue.StoreF16]
    outs, members = [], []
    for w, epi in zip(ws, epis):
        cols = w.shape[0] // 2 if epi == Epilogue.SwigluF16 else w.shape[0]
        y = full((m, cols), np.float32 if epi == Epilogue.StoreF32 else np.float16, np.nan)
        wd = to_dev(w)
        outs.append((y, wd))
        members.append(_lib.DhGemmMember(addr((wd, 0)), addr((y, 0)), k, cols, w.shape[0], int(epi)))
    arr = (_lib.DhGemmMember * 3)(*members)
    xd = to_dev(x)
    assert _lib.load().dh_gemm_nt_grouped(kernels.ctx.handle, None, addr((xd, 0)), k, m, k, arr, 3) == 0
    sync()
    for (y, _), w, epi in zip(outs, ws, epis):
        got = to_host(y).astype(np.float32)
        want = oracle_epi(x, w, epi)
        check_gemm(f"grouped stream {epi.name}", got, want)


@pytest.mark.parametrize("variant", range(len(variants())))
def test_every_variant_and_split_on_integer_inputs_is_exact(gpu, kernels, stream, variant):
    """Integer-valued fp16 in [-4, 4] at K = 288 (4 full stages and a 32-wide tail): every partial
    sum is an integer below 2^24, so any summation order gives the exact fp32 result."""
    rng = np.random.default_rng(variant)
    m, k = 45, 288
    n = 2 * variants()[variant]["bn"]
    x = rng.integers(-4, 5, (m, k)).astype(np.float16)
    w = rng.integers(-4, 5, (n, k)).astype(np.float16)
    want = (x.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32)
    try:
        for splits in (1, 2, 3):
            kernels.gemm.force(variant, splits)
            got = run_gemm(kernels, stream, x, w, Epilogue.StoreF32)
            assert np.array_equal(got, want), f"variant {variant} splits {splits}"
    finally:
        kernels.gemm.force(None)


@pytest.mark.parametrize("variant", range(len(variants())))
def test_every_variant_swiglu_and_add(gpu, kernels, stream, variant):
    """Ragged in every direction: m = 37 leaves a partial row tile, n = 2·BN + 96 a last column stripe
    holding only 3 gate|up pairs (columns past N re-read row N-1 of W and are never stored)."""
    m, k = 37, 192
    n = 2 * variants()[variant]["bn"] + 96
    x, w = inputs(m, n, k, 200 + variant)
    y0 = synth.normal_f32(synth.seed_for(300 + variant), (m, n), 1.0)
    try:
        for splits in (1, 2):
            kernels.gemm.force(variant, splits)
            for epi in (Epilogue.SwigluF16, Epilogue.AddF32, Epilogue.StoreF16):
                got = run_gemm(kernels, stream, x, w, epi, y0 if epi == Epilogue.AddF32 else None)
                check_gemm(f"variant {variant} splits {splits} {epi.name}", got, oracle_epi(x, w, epi, y0))
    finally:
        kernels.gemm.force(None)


def test_every_variant_stores_the_same_bits(gpu, kernels, stream):
    """Every tile variant sums K in the same order (64-wide stages, two 32-wide MFMA steps, the same lane
    split of k), so without split-K they store identical bits for every epilogue, whatever the tiling:
    the 2 x 2 tile's SwiGLU pair that straddles its two N halves included (n covers 9 tiles of 256 and
    8 of 288 columns, m several row tiles with a ragged last one)."""
    m, n, k = 203, 2304, 320
    x, w = inputs(m, n, k, 77)
    y0 = synth.normal_f32(synth.seed_for(78), (m, n), 1.0)
    try:
        for epi in (Epilogue.SwigluF16, Epilogue.StoreF32, Epilogue.AddF32, Epilogue.StoreF16):
            ref = None
            for v in range(len(variants())):
                kernels.gemm.force(v, 1)
                got = run_gemm(kernels, stream, x, w, epi, y0 if epi == Epilogue.AddF32 else None)
                if ref is None:
                    ref = got
                    check_gemm(f"variant 0 {epi.name}", got, oracle_epi(x, w, epi, y0))
                else:
                    assert np.array_equal(got.view(np.uint8), ref.view(np.uint8)), f"variant {v} {epi.name}"
    finally:
        kernels.gemm.force(None)


@pytest.mark.parametrize("m", [3, 203])
def test_empty_k_and_n(gpu, kernels, stream, m):
    """K = 0 stores the empty sum (zeros; AddF32 leaves the residual as it was); N = 0 launches nothing.
    decide's contract admits both (gemm.rs:140-144)."""
    x, w = to_dev(np.ones((m, 64), np.float16)), to_dev(np.ones((64, 64), np.float16))
    y0 = synth.normal_f32(synth.seed_for(71), (m, 64), 1.0)
    for epi in Epilogue:
        out_cols = 32 if epi == Epilogue.SwigluF16 else 64
        dt = np.float32 if epi in (Epilogue.StoreF32, Epilogue.AddF32) else np.float16
        start = y0.astype(dt)[:, :out_cols].copy()
        y = to_dev(start)
        kernels.gemm.gemm(stream, (x, 0), (w, 0), (y, 0), m, 64, 0, 64, 64, out_cols, epi)
        sync()
        want = start if epi == Epilogue.AddF32 else np.zeros_like(start)
        assert np.array_equal(to_host(y).view(np.uint8), want.view(np.uint8)), f"K = 0 {epi.name}"
        y = to_dev(start)
        kernels.gemm.gemm(stream, (x, 0), (w, 0), (y, 0), m, 0, 64, 64, 64, out_cols, epi)
        sync()
        assert np.array_equal(to_host(y).view(np.uint8), start.view(np.uint8)), f"N = 0 {epi.name}"

def test_reference_kernel_matches_oracle(gpu, kernels_ref, stream):
    for (m, n, k) in [(5, 64, 96), (33, 96, 160), (70, 128, 2560)]:
        x, w = inputs(m, n, k, 400 + m)
        for epi in Epilogue:
            y0 = synth.normal_f32(synth.seed_for(401), (m, n), 1.0) if epi == Epilogue.AddF32 else None
            got = run_gemm(kernels_ref, stream, x, w, epi, y0)
            check_gemm(f"reference m{m} {epi.name}", got, oracle_epi(x, w, epi, y0))


def test_reference_kernel_takes_what_decides_baseline_takes(gpu, kernels, kernels_ref, stream):
    """decide's baseline returns before the fast path's alignment asserts (gemm.rs:150-163): strides that are not
    multiples of 8, x/w at 2-byte offsets and y at element offsets are accepted there and computed correctly;
    the fast context still refuses them."""
    m, n, k = 21, 64, 96
    ldx, ldw = k + 2, k + 6  # not multiples of 8
    rng = np.random.default_rng(12)
    xbig = rng.standard_normal((m + 1, ldx)).astype(np.float16)
    wbig = (rng.standard_normal((n + 1, ldw)) * 0.05).astype(np.float16)
    xd, wd = to_dev(xbig), to_dev(wbig)
    x_off, w_off = ldx * 2 + 2, 2  # row 1 column 1; row 0 column 1: 2-byte aligned only
    x = xbig.reshape(-1)[x_off // 2:x_off // 2 + (m - 1) * ldx + k]
    x = np.stack([x[i * ldx:i * ldx + k] for i in range(m)])
    w = wbig.reshape(-1)[w_off // 2:w_off // 2 + (n - 1) * ldw + k]
    w = np.stack([w[j * ldw:j * ldw + k] for j in range(n)])
    for epi in Epilogue:
        out_cols = n // 2 if epi == Epilogue.SwigluF16 else n
        ldy = out_cols + 1  # odd
        dt = np.float32 if epi in (Epilogue.StoreF32, Epilogue.AddF32) else np.float16
        y0 = synth.normal_f32(synth.seed_for(402), (m, out_cols), 1.0)
        ybig = np.full((m + 1, ldy), 3.0, dt)
        ybig[:m, 1:1 + out_cols] = y0.astype(dt)
        y = to_dev(ybig)
        y_off = np.dtype(dt).itemsize  # column 1
        kernels_ref.gemm.gemm(stream, (xd, x_off), (wd, w_off), (y, y_off), m, n, k, ldx, ldw, ldy, epi)
        sync()
        got = to_host(y)[:m, 1:1 + out_cols].astype(np.float32)
        check_gemm(f"reference unaligned {epi.name}", got,
                   oracle_epi(x, w, epi, y0.astype(dt).astype(np.float32)))
        with pytest.raises(AssertionError, match="gemm \\(fast\\)"):
            kernels.gemm.gemm(stream, (xd, x_off), (wd, w_off), (y, y_off), m, n, k, ldx, ldw, ldy, epi)


def test_strides_and_offsets(gpu, kernels, stream):
    """Row strides wider than K / N and operands addressed at byte offsets inside larger buffers,
    as decide's forward does (e.g. the k|v rows of w_in at ATT_K·HIDDEN·2, forward.rs:1157-1158)."""
    m, n, k = 50, 128, 256
    ldx, ldw, ldy = 320, 264, 160
    rng = np.random.default_rng(11)
    xbig = rng.standard_normal((m + 3, ldx)).astype(np.float16)
    wbig = (rng.standard_normal((n + 64, ldw)) * 0.05).astype(np.float16)
    xd, wd = to_dev(xbig), to_dev(wbig)
    y = full((m + 2, ldy), np.float32, 7.0)
    x_off = 3 * ldx * 2  # start at row 3
    w_off = 64 * ldw * 2  # weight rows 64..
    y_off = 2 * ldy * 4 + 16 * 4  # row 2, column 16
    kernels.gemm.gemm(stream, (xd, x_off), (wd, w_off), (y, y_off), m, n, k, ldx, ldw, ldy, Epilogue.StoreF32)
    sync()
    yh = to_host(y)
    want = orc.gemm_nt_f16(xbig[3:, :k], wbig[64:, :k])
    check_gemm("strided", yh[2:, 16:16 + n], want)
    orc.assert_close("strided", yh[2:, 16:16 + n], want, 1e-4, 1e-4)
    # nothing outside the output window is touched
    assert (yh[:2] == 7.0).all() and (yh[2:, :16] == 7.0).all()


def test_deterministic_and_m_independent_rows(gpu, kernels, stream):
    x, w = inputs(603, 512, 2560, 500)
    a = run_gemm(kernels, stream, x, w, Epilogue.StoreF32)
    b = run_gemm(kernels, stream, x, w, Epilogue.StoreF32)
    assert np.array_equal(a, b)
    # with the plan pinned, the first rows do not depend on how many rows follow
    p = kernels.gemm.plan(603, 512, 2560, Epilogue.StoreF32)
    try:
        kernels.gemm.force(p["variant"], p["splits"])
        c = run_gemm(kernels, stream, x[:17].copy(), w, Epilogue.StoreF32)
        assert np.array_equal(c, a[:17])
    finally:
        kernels.gemm.force(None)


# ------------------------------------------------------------------ BASELINE configs
def test_config1_single_gemm_m276(gpu, kernels, stream):
    """C1: Y = X·Wᵀ, M = 276, K = 2560, N = 9216, fp32 out; checked against the fp32 CPU matmul."""
    m, n, k = 276, 9216, 2560
    x, w = inputs(m, n, k, 1)
    got = run_gemm(kernels, stream, x, w, Epilogue.StoreF32)
    want = orc.gemm_nt_f16(x, w)  # all rows: ~6.5 G MAC, a few seconds on the host
    check_gemm("C1", got, want)
    orc.assert_close("C1", got, want, atol=1e-4, rtol=1e-4)
    got16 = run_gemm(kernels, stream, x, w, Epilogue.StoreF16)
    check_gemm("C1 f16", got16, orc.f16_round(want))


def test_config2_fused_mlp_m603(gpu, kernels, stream):
    """C2: gate|up [603×2560]·[18432×2560]ᵀ with SwiGLU → fp16 [603, 9216]; down [603×9216]·[2560×9216]ᵀ
    added into the fp32 residual. Each GEMM against the oracle on the GPU's own inputs (sampled rows),
    the whole block against the oracle chain."""
    m, d, f = 603, 2560, 9216
    x = synth.normal_f16(synth.seed_for(21), (m, d), 1.0)
    wgu = synth.normal_f16(synth.seed_for(22), (2 * f, d), 0.02)
    wdn = synth.normal_f16(synth.seed_for(23), (d, f), 0.02)
    x0 = synth.normal_f32(synth.seed_for(24), (m, d), 1.0)
    xd, wgud, wdnd = to_dev(x), to_dev(wgu), to_dev(wdn)
    mlp = empty((m, f), np.float16)
    res = to_dev(x0)
    kernels.gemm.gemm(stream, (xd, 0), (wgud, 0), (mlp, 0), m, 2 * f, d, d, d, f, Epilogue.SwigluF16)
    kernels.gemm.gemm(stream, (mlp, 0), (wdnd, 0), (res, 0), m, d, f, f, f, d, Epilogue.AddF32)
    sync()
    mlp_h = to_host(mlp)
    res_h = to_host(res)
    rows = sample_rows(m)
    # (1) gate|up + SwiGLU on the sampled rows
    want_mlp = swiglu_f16(orc.gemm_nt_f16(x, wgu, rows=rows))
    check_gemm("C2 gate|up swiglu", mlp_h[rows].astype(np.float32), want_mlp)
    orc.assert_close("C2 gate|up swiglu", mlp_h[rows].astype(np.float32), want_mlp, atol=2e-3, rtol=4e-3)
    # (2)+(3) down + residual on the GPU's own fp16 activations
    want_down = orc.gemm_nt_f16(mlp_h, wdn, rows=rows)
    check_gemm("C2 down (delta)", res_h[rows] - x0[rows], want_down)
    orc.assert_close("C2 down + residual", res_h[rows], x0[rows] + want_down, atol=1e-4, rtol=1e-4)
    # end to end through the oracle's own activations
    want_chain = x0[rows] + orc.gemm_nt_f16(want_mlp.astype(np.float16), wdn)
    check_gemm("C2 chain (delta)", res_h[rows] - x0[rows], want_chain - x0[rows], rel=2e-3)


def rmsnorm_h(kernels, stream, xin, wn):
    m, d = xin.shape
    xdv = to_dev(xin)
    h = empty((m, d), np.float16)
    iota = to_dev(np.arange(m, dtype=np.uint32).view(np.int32))
    kernels.norm.rmsnorm(stream, (xdv, 0), (to_dev(wn), 0), (h, 0), (iota, 0), m, d, d, d, True)
    return h


@pytest.mark.parametrize("group", ["attention_6144", "attention_10240", "gdn_12352"])
def test_config3_grouped_projections_m603(gpu, kernels, stream, group):
    """C3: the projections sharing one RMSNormed activation as ONE grouped launch, then the out
    projection (AddF32). Attention (BASELINE): Q 4096, K 1024, V 1024; attention (decide, gated):
    q|gate 8192, k 1024, v 1024; GDN: qkv 8192, z 4096, b 32, a 32 (decide's column order)."""
    m, d = 603, 2560
    widths = {"attention_6144": [4096, 1024, 1024], "attention_10240": [8192, 1024, 1024],
              "gdn_12352": [8192, 4096, 32, 32]}[group]
    xin = synth.normal_f32(synth.seed_for(31), (m, d), 1.0)
    wn = synth.normal_f32(synth.seed_for(32), (d,), 0.02)
    h = rmsnorm_h(kernels, stream, xin, wn)
    ws = [synth.normal_f16(synth.seed_for(40 + i), (n, d), 0.02) for i, n in enumerate(widths)]
    wds = [to_dev(w) for w in ws]
    ys = [full((m, n), np.float32, np.nan) for n in widths]
    members = [((wd, 0), d, n, (y, 0), n, Epilogue.StoreF32) for wd, n, y in zip(wds, widths, ys)]
    kernels.gemm.gemm_grouped(stream, (h, 0), d, m, d, members)
    sync()
    hh = to_host(h)
    rows = sample_rows(m)
    for i, (w, y) in enumerate(zip(ws, ys)):
        want = orc.gemm_nt_f16(hh, w, rows=rows)
        got = to_host(y)[rows]
        check_gemm(f"C3 {group} member {i}", got, want)
        orc.assert_close(f"C3 {group} member {i}", got, want, 1e-4, 1e-4)
    # the out projection: g fp16 [603, 4096] · W_o [2560, 4096]ᵀ added into x
    g = synth.normal_f16(synth.seed_for(50), (m, 4096), 1.0)
    wo = synth.normal_f16(synth.seed_for(51), (d, 4096), 0.02)
    x0 = synth.normal_f32(synth.seed_for(52), (m, d), 1.0)
    res = to_dev(x0)
    kernels.gemm.gemm(stream, (to_dev(g), 0), (to_dev(wo), 0), (res, 0), m, d, 4096, 4096, 4096,
                      d, Epilogue.AddF32)
    sync()
    want = orc.gemm_nt_f16(g, wo, rows=rows)
    check_gemm(f"C3 {group} out", to_host(res)[rows] - x0[rows], want)


def test_grouped_qkv_m2307_member_stripes(gpu, kernels, stream):
    """BASELINE's Q|K|V group at M = 2307: its members round up to whole column stripes each, which for
    the single-GEMM choice at N = 6144 would add a round of tiles, so the grouped planner re-plans; the
    re-planned launch still matches the oracle on every member (sampled rows)."""
    m, d, widths = 2307, 2560, [4096, 1024, 1024]
    x = synth.normal_f16(synth.seed_for(33), (m, d), 1.0)
    ws = [synth.normal_f16(synth.seed_for(43 + i), (n, d), 0.02) for i, n in enumerate(widths)]
    ys = [full((m, n), np.float32, np.nan) for n in widths]
    members = [((to_dev(w), 0), d, n, (y, 0), n, Epilogue.StoreF32) for w, n, y in zip(ws, widths, ys)]
    kernels.gemm.gemm_grouped(stream, (to_dev(x), 0), d, m, d, members)
    sync()
    rows = sample_rows(m)
    for i, (w, y) in enumerate(zip(ws, ys)):
        got = to_host(y)
        assert np.isfinite(got).all(), f"member {i}: rows left unwritten"
        want = orc.gemm_nt_f16(x, w, rows=rows)
        check_gemm(f"Q|K|V m2307 member {i}", got[rows], want)
        orc.assert_close(f"Q|K|V m2307 member {i}", got[rows], want, 1e-4, 1e-4)

def test_grouped_equals_fused_single_gemm(gpu, kernels, stream):
    """A grouped launch over [W_a; W_b] gives the same bits as one GEMM over the concatenated rows when
    both use the same tile variant (decide fuses by concatenation, convert.rs:204-245)."""
    m, d = 96, 512
    wa = synth.normal_f16(synth.seed_for(60), (256, d), 0.02)
    wb = synth.normal_f16(synth.seed_for(61), (512, d), 0.02)
    x = synth.normal_f16(synth.seed_for(62), (m, d), 1.0)
    xd = to_dev(x)
    cat = to_dev(np.concatenate([wa, wb]))
    v = kernels.gemm.plan(m, 768, d, Epilogue.StoreF32)["variant"]
    try:
        kernels.gemm.force(v, 1)
        yf = empty((m, 768), np.float32)
        kernels.gemm.gemm(stream, (xd, 0), (cat, 0), (yf, 0), m, 768, d, d, d, 768, Epilogue.StoreF32)
        ya, yb = empty((m, 256), np.float32), empty((m, 512), np.float32)
        kernels.gemm.gemm_grouped(stream, (xd, 0), d, m, d, [((to_dev(wa), 0), d, 256, (ya, 0), 256,
                                                              Epilogue.StoreF32),
                                                             ((to_dev(wb), 0), d, 512, (yb, 0), 512,
                                                              Epilogue.StoreF32)])
        sync()
    finally:
        kernels.gemm.force(None)
    f = to_host(yf)
    assert np.array_equal(f[:, :256], to_host(ya))
    assert np.array_equal(f[:, 256:], to_host(yb))


@pytest.mark.parametrize("kn", [(2560, 12352), (2560, 10240), (2560, 18432), (4096, 2560), (9216, 2560)])
def test_config4_projections_m2307(gpu, kernels, stream, kn):
    """C4: every projection GEMM of one hybrid layer at M = 2,307 (sampled rows against the oracle)."""
    k, n = kn
    m = 2307
    x, w = inputs(m, n, k, 70 + n)
    epi = Epilogue.SwigluF16 if n == 18432 else (Epilogue.AddF32 if n == 2560 else Epilogue.StoreF32)
    y0 = synth.normal_f32(synth.seed_for(71), (m, n), 1.0) if epi == Epilogue.AddF32 else None
    got = run_gemm(kernels, stream, x, w, epi, y0)
    rows = sample_rows(m, 40, seed=n)
    y = orc.gemm_nt_f16(x, w, rows=rows)
    if epi == Epilogue.SwigluF16:
        want = swiglu_f16(y)
    elif epi == Epilogue.AddF32:
        want = y0[rows] + y
    else:
        want = y
    check_gemm(f"C4 k{k} n{n}", got[rows], want)


# One shape per tile work order the planner picks (dh_gemm_plan.order: 0 = M tiles fastest, g = column stripes
# in groups of g), each a single planned launch without split-K.
ORDER_SHAPES = {0: (603, 18432, 2560), 2: (800, 2048, 2560), 3: (2000, 2048, 2560), 4: (1500, 2560, 4096),
                6: (2307, 2560, 4096), 8: (1024, 3072, 1024)}


@pytest.mark.parametrize("order", sorted(ORDER_SHAPES))
def test_every_tile_order_is_exact(gpu, kernels, stream, order):
    """The work order only decides which workgroup computes which tile, so every tile must still be computed
    once, in place: integer-valued fp16 in [-4, 4] make every partial sum an integer below 2^24, so the fp32
    result is exact whatever the order (the f64 product is the exact answer)."""
    m, n, k = ORDER_SHAPES[order]
    p = kernels.gemm.plan(m, n, k, Epilogue.StoreF32)
    assert p["order"] == order and p["splits"] == 1, p
    rng = np.random.default_rng(order)
    x = rng.integers(-4, 5, (m, k)).astype(np.float16)
    w = rng.integers(-4, 5, (n, k)).astype(np.float16)
    want = (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)
    got = run_gemm(kernels, stream, x, w, Epilogue.StoreF32)
    assert np.array_equal(got, want), f"order {order}: {int((got != want).sum())} outputs differ"


def random_shapes(count: int, seed: int):
    """Seeded shapes across the planner's range: M from 1 (the weight-streaming kernel) to ~1300, N and K
    any multiple of 32 (so K % 64 == 32 leaves a half stage, split-K included), row strides padded past
    K and the output width, every epilogue. M·N·K stays small enough for the oracle."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        r = rng.random()
        m = int(rng.integers(1, 17)) if r < 0.2 else int(rng.integers(17, 420)) if r < 0.8 else int(rng.integers(420, 1300))
        n = 32 * int(rng.integers(1, 72))
        k = 32 * int(rng.integers(1, 90))
        if m * n * k > 6e8:
            continue
        epi = Epilogue(int(rng.integers(0, 4)))
        pads = [8 * int(rng.integers(0, 3)) for _ in range(3)]  # extra elements of ldx, ldw, ldy
        forced = (int(rng.integers(0, len(variants()))), int(rng.integers(1, 5)))
        out.append((m, n, k, epi, pads, forced))
    return out


@pytest.mark.parametrize("case", range(32))
def test_random_shapes_planner_and_forced(gpu, kernels, stream, case):
    """One seeded shape through the planner's own choice and through one forced (variant, split-K) pair:
    both within the GEMM bar of the oracle, and nothing outside the output window written."""
    m, n, k, epi, (px, pw, py), forced = random_shapes(32, 2024)[case]
    ldx, ldw = k + px, k + pw
    out_cols = n // 2 if epi == Epilogue.SwigluF16 else n
    ldy = out_cols + py
    dt = np.float32 if epi in (Epilogue.StoreF32, Epilogue.AddF32) else np.float16
    x, w = inputs(m, n, k, 900 + case)
    xbig = np.zeros((m, ldx), np.float16)
    wbig = np.zeros((n, ldw), np.float16)
    xbig[:, :k], wbig[:, :k] = x, w
    xbig[:, k:], wbig[:, k:] = np.float16(np.inf), np.float16(np.inf)  # must never reach a sum
    y0 = synth.normal_f32(synth.seed_for(950 + case), (m, ldy), 1.0).astype(dt)
    if epi != Epilogue.AddF32:
        y0[:] = 7.0
    want = oracle_epi(x, w, epi, y0[:, :n].astype(np.float32) if epi == Epilogue.AddF32 else None)
    xd, wd = to_dev(xbig), to_dev(wbig)
    name = f"case {case}: m{m} n{n} k{k} {epi.name} ld {ldx}/{ldw}/{ldy}"
    tol = 2e-3 if epi in (Epilogue.StoreF16, Epilogue.SwigluF16) else 1e-4
    try:
        for pin in (None, forced):
            if pin is not None:
                kernels.gemm.force(*pin)
            plan = kernels.gemm.plan(m, n, k, epi)
            label = f"{name} variant {plan['variant']} splits {plan['splits']}"
            print(label, flush=True)
            y = to_dev(y0)
            kernels.gemm.gemm(stream, (xd, 0), (wd, 0), (y, 0), m, n, k, ldx, ldw, ldy, epi)
            sync()
            got = to_host(y)
            check_gemm(label, got[:, :out_cols].astype(np.float32), want)
            orc.assert_close(label, got[:, :out_cols].astype(np.float32), want, atol=tol, rtol=tol)
            assert np.array_equal(got[:, out_cols:].view(np.uint8), y0[:, out_cols:].view(np.uint8)), label
    finally:
        kernels.gemm.force(None)


@pytest.mark.parametrize("variant", range(len(variants())))
def test_grouped_ragged_members_every_variant(gpu, kernels, stream, variant):
    """One grouped launch per tile variant over members of mixed epilogues and widths that end mid-stripe
    (96, 32 and 160 columns), K = 224 (three 64-wide stages and a 32-wide half stage), M = 41: every member
    against the oracle, and the columns past each member's output untouched."""
    m, k = 41, 224
    specs = [(96, Epilogue.StoreF32), (32, Epilogue.AddF32), (160, Epilogue.SwigluF16)]
    x = synth.normal_f16(synth.seed_for(81), (m, k), 1.0)
    ws = [synth.normal_f16(synth.seed_for(82 + i), (n, k), 0.02) for i, (n, _) in enumerate(specs)]
    ys, starts = [], []
    for i, (n, epi) in enumerate(specs):
        cols = n // 2 if epi == Epilogue.SwigluF16 else n
        dt = np.float16 if epi == Epilogue.SwigluF16 else np.float32
        start = synth.normal_f32(synth.seed_for(90 + i), (m, cols + 8), 1.0).astype(dt)
        starts.append(start)
        ys.append(to_dev(start))
    members = [((to_dev(w), 0), k, n, (y, 0), s.shape[1], epi) for w, (n, epi), y, s in zip(ws, specs, ys, starts)]
    try:
        kernels.gemm.force(variant, 1)
        kernels.gemm.gemm_grouped(stream, (to_dev(x), 0), k, m, k, members)
        sync()
    finally:
        kernels.gemm.force(None)
    for i, ((n, epi), w, y, start) in enumerate(zip(specs, ws, ys, starts)):
        got = to_host(y)
        cols = n // 2 if epi == Epilogue.SwigluF16 else n
        y0 = start[:, :n].astype(np.float32) if epi == Epilogue.AddF32 else None
        want = oracle_epi(x, w, epi, y0)
        check_gemm(f"variant {variant} member {i} {epi.name}", got[:, :cols].astype(np.float32), want)
        assert np.array_equal(got[:, cols:].view(np.uint8), start[:, cols:].view(np.uint8)), f"member {i} padding"
