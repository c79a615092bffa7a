"""The device's seeded Gaussian fills (dh_fill_normal, dh_fill_normal_f16, dh_model_init_random) equal the oracle's
host restatement (orc_fill_normal) bit for bit, so a random-init model can be rebuilt on the host exactly. The host
restatement itself is pinned in test_normal_gen.py."""

import numpy as np
import pytest

import oracle_forward
import oracle_lib as orc
from decide_amd.forward import Model, ModelConfig
from decide_amd.kernels import fill_normal, fill_normal_f16
from gpu_util import empty, sync, to_host

pytestmark = pytest.mark.gpu

N = 3_000_001  # odd: the last element is the cos half of an unfinished pair


@pytest.mark.parametrize("dtype,name,np_dtype", [(0, "f16", np.uint16), (1, "bf16", np.uint16), (2, "f32", np.uint32)])
@pytest.mark.parametrize("seed,mean,std", [(0xDEC1DE, 0.0, 0.02), (2**64 - 3, 0.5, 0.5), (7, 1.0, 0.3)])
def test_fill_normal_equals_host(gpu, kernels, dtype, name, np_dtype, seed, mean, std):
    out = empty((N,), np.float32 if dtype == 2 else np.uint16)
    fill_normal(kernels.ctx, 0, (out, 0), N, seed, mean, std, name)
    sync()
    got = to_host(out).view(np_dtype)
    want = orc.fill_normal(N, seed, mean, std, dtype).view(np_dtype)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} of {N} differ, first at {bad[:5]}"


def test_fill_normal_f16_equals_host(gpu, kernels):
    out = empty((N,), np.uint16)
    fill_normal_f16(kernels.ctx, 0, (out, 0), N, 0x5EED, 0.02)
    sync()
    np.testing.assert_array_equal(to_host(out), orc.fill_normal(N, 0x5EED, 0.0, 0.02, 0).view(np.uint16))


def test_model_init_random_is_rebuilt_on_the_host(gpu, kernels):
    """Every tensor of a 5-layer model (both mixer kinds) after dh_model_init_random, in the registry order the host
    rebuild assumes."""
    layers, vocab, seed = 5, 1000, 0xC0FFEE
    model = Model(kernels.ctx, ModelConfig(layers=layers, vocab=vocab, max_tokens=64, max_answers=2, max_cand=4))
    model.init_random(0, seed=seed)
    sync()
    reg = oracle_forward.random_init_registry(layers, vocab)
    assert model.tensor_names() == [r[0] for r in reg]
    host = oracle_forward.RandomInitWeights(seed, layers, vocab)
    for name, shape, dt, _, _ in reg:
        got = model.download(name)
        want = host[name]
        assert got.size == want.size, name
        np.testing.assert_array_equal(got.reshape(-1).view(np.uint8), np.ascontiguousarray(want).reshape(-1).view(np.uint8),
                                      err_msg=name)
    model.close()
