"""GPU parity of the row kernels: gathers (bit-exact), candidate head, RMSNorm, N(0, σ) fill."""

import numpy as np
import pytest

import oracle_lib as orc
from decide_amd import synth
from decide_amd.kernels import fill_normal_f16
from gpu_util import empty, full, sync, to_dev, to_host

pytestmark = pytest.mark.gpu


def u32(a):
    return to_dev(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32))


@pytest.mark.parametrize("h", [2560, 7, 1, 4096])
def test_gather_rows_bit_exact(gpu, kernels, stream, h):
    rng = np.random.default_rng(h)
    src32 = rng.standard_normal((300, h)).astype(np.float32)
    src32[5, 0] = np.nan  # payloads and signs must survive: bitwise copy
    src32[6, 0] = -0.0
    src16 = rng.integers(0, 65536, (300, h)).astype(np.uint16)
    rowmap = rng.integers(0, 300, 57).astype(np.uint32)
    rowmap[:3] = [299, 5, 6]
    out32 = empty((57, h), np.float32)
    out16 = empty((57, h), np.int16)
    kernels.head.gather_rows_f32(stream, (to_dev(src32), 0), (u32(rowmap), 0), (out32, 0), 57, h)
    kernels.head.gather_rows_f16(stream, (to_dev(src16.view(np.int16)), 0), (u32(rowmap), 0),
                                 (out16, 0), 57, h)
    sync()
    assert np.array_equal(to_host(out32).view(np.uint32), src32[rowmap].view(np.uint32))
    assert np.array_equal(to_host(out16).view(np.uint16), src16[rowmap])


def test_gather_zero_rows_is_a_no_op(gpu, kernels, stream):
    out = full((4, 8), np.float32, 3.0)
    kernels.head.gather_rows_f32(stream, (out, 0), (u32(np.zeros(1)), 0), (out, 0), 0, 8)
    sync()
    assert (to_host(out) == 3.0).all()


def test_gather_bf16_candidate_rows_from_a_151936_vocab(gpu, kernels, stream):
    """C4's candidate gather: 24 answer rows × 64 ids uniform over 151,936; rows copied bitwise."""
    vocab, hidden = 151936, 2560
    table = to_dev(np.zeros((vocab, hidden), dtype=np.int16))
    kernels_fill = synth.seed_for(80)
    fill_normal_f16(kernels.ctx, stream, (table, 0), vocab * hidden, kernels_fill, 0.02)
    ids = synth.uniform_ids(synth.seed_for(81), 24 * 64, vocab)
    out = empty((24 * 64, hidden), np.int16)
    kernels.head.gather_rows_f16(stream, (table, 0), (u32(ids), 0), (out, 0), 24 * 64, hidden)
    sync()
    t = to_host(table)
    assert np.array_equal(to_host(out), t[ids])


@pytest.mark.parametrize("rows,hidden,max_cand", [(24, 2560, 64), (3, 2560, 8), (6, 256, 8), (16, 2560, 62),
                                                    (5, 2560, 13), (4, 512, 1), (7, 1024, 17)])
def test_final_head_matches_oracle(gpu, kernels, stream, rows, hidden, max_cand):
    vocab = 151936 if hidden == 2560 else 1000
    x = synth.normal_f32(synth.seed_for(90), (rows, hidden), 3.0)
    w = synth.normal_f32(synth.seed_for(91), (hidden,), 0.02)
    table = synth.bf16_bits(synth.normal_f32(synth.seed_for(92), (vocab, hidden), 0.02))
    cand = synth.uniform_ids(synth.seed_for(93), rows * max_cand, vocab).reshape(rows, max_cand)
    ncand = np.full(rows, max_cand, dtype=np.uint32)
    ncand[0] = 0  # ragged: none, one, more than max
    if rows > 1:
        ncand[1] = 1
    if rows > 2:
        ncand[2] = max_cand + 5
    logits = full((rows, max_cand), np.float32, np.nan)
    kernels.head.final_head(stream, (to_dev(x), 0), (to_dev(w), 0),
                            (to_dev(table.view(np.int16)), 0), (u32(cand), 0),
                            (u32(ncand), 0), (logits, 0), rows, hidden, max_cand)
    sync()
    got = to_host(logits)
    want = orc.final_head(x, w, table, cand, ncand, max_cand)
    written = ~np.isnan(want)
    assert np.array_equal(~np.isnan(got), written), "entries past ncand must stay untouched"
    orc.assert_close("final_head", got[written], want[written], atol=1e-4, rtol=1e-4)


def test_golden_head_fixture_on_gpu(gpu, kernels, stream):
    import os

    with np.load(os.path.join(os.path.dirname(__file__), "golden", "head_small.npz"), allow_pickle=False) as z:
        x, w, table, cand, ncand, want = (z[k] for k in ("x", "w", "table", "cand", "ncand", "logits"))
        max_cand = int(z["max_cand"])
    rows, hidden = x.shape
    logits = full((rows, max_cand), np.float32, np.nan)
    kernels.head.final_head(stream, (to_dev(x), 0), (to_dev(w), 0),
                            (to_dev(table.view(np.int16)), 0), (u32(cand), 0),
                            (u32(ncand), 0), (logits, 0), rows, hidden, max_cand)
    sync()
    got = to_host(logits)
    written = ~np.isnan(want)
    assert np.array_equal(~np.isnan(got), written)
    np.testing.assert_allclose(got[written], want[written], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("add_one", [True, False])
def test_rmsnorm_rows_matches_oracle(gpu, kernels, stream, add_one):
    rows, h, ld_in, ld_out = 37, 2560, 2600, 2568
    x = synth.normal_f32(synth.seed_for(100), (rows + 5, ld_in), 2.0)
    w = synth.normal_f32(synth.seed_for(101), (h,), 0.3)
    rowmap = np.array([(i * 7) % (rows + 5) for i in range(rows)], dtype=np.uint32)
    y = full((rows, ld_out), np.float16, 0)
    kernels.norm.rmsnorm(stream, (to_dev(x), 0), (to_dev(w), 0), (y, 0), (u32(rowmap), 0),
                         rows, h, ld_in, ld_out, add_one)
    sync()
    got = to_host(y)[:, :h].astype(np.float32)
    want = orc.f16_round(orc.rmsnorm(x[rowmap, :h], w, add_one))
    # one fp16 rounding step apart at most
    orc.assert_close("rmsnorm", got, want, atol=1e-3, rtol=2e-3)
    assert (to_host(y)[:, h:] == 0).all()


def test_rmsnorm_kat_on_gpu(gpu, kernels, stream):
    """decide's rmsnorm_by_hand (cpu_ref.rs:204-210) on the GPU: [3, 4], w = [1, 1], add_one → 2·x/√12.5."""
    x = np.array([[3.0, 4.0]], dtype=np.float32)
    y = full((1, 2), np.float16, 0)
    kernels.norm.rmsnorm(stream, (to_dev(x), 0), (to_dev(np.ones(2, np.float32)), 0), (y, 0),
                         (u32(np.zeros(1)), 0), 1, 2, 2, 2, True)
    sync()
    want = np.array([3.0, 4.0]) * 2.0 / np.sqrt(12.5)
    np.testing.assert_allclose(to_host(y)[0].astype(np.float64), want, atol=2e-3)


def test_fill_normal_statistics_and_reproducibility(gpu, kernels, stream):
    n = 1 << 22
    a = empty((n,), np.float16)
    b = empty((n,), np.float16)
    fill_normal_f16(kernels.ctx, stream, (a, 0), n, 1234, 0.02)
    fill_normal_f16(kernels.ctx, stream, (b, 0), n, 1234, 0.02)
    sync()
    ah = to_host(a).astype(np.float64)
    assert np.array_equal(ah, to_host(b).astype(np.float64))
    assert abs(ah.mean()) < 1e-4
    assert abs(ah.std() - 0.02) < 2e-4
    # agrees with the host generator to within fp16 rounding
    host = synth.normal(1234, 4096, 0.02)
    np.testing.assert_allclose(ah[:4096], host, atol=2e-5, rtol=2e-3)
