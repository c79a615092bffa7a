"""decide-weights-v1 round trip and the loader's checks (decide: Weights::open, weights.rs:105-183):
a random-init model saved in decide's converted layout and loaded into a fresh model gives bitwise the
same tensors and logits; a bad index, offset, dtype, size or blob is refused with decide's messages."""

import json
import os

import numpy as np
import pytest

from decide_amd import weights
from decide_amd.forward import Model, ModelConfig
from gpu_util import full, sync, to_dev, to_host
from test_forward_gpu import _request

pytestmark = pytest.mark.gpu

CFG = ModelConfig(layers=4, vocab=300, max_tokens=40, max_answers=2, max_cand=4)


def _logits(model, ids, ans, cand, ncand):
    logits = full((len(ans), CFG.max_cand), np.float32, np.nan)
    model.forward(0, (to_dev(ids), 0), len(ids), (to_dev(ans), 0), len(ans), (to_dev(cand), 0), (to_dev(ncand), 0),
                  (logits, 0))
    sync()
    return to_host(logits)


@pytest.fixture(scope="module")
def saved(kernels, tmp_path_factory):
    d = str(tmp_path_factory.mktemp("weights"))
    a = Model(kernels.ctx, CFG)
    a.init_random(0, seed=5)
    sync()
    index = weights.save(a, d)
    yield a, d, index
    a.close()


def test_round_trip_is_bitwise(gpu, kernels, saved):
    a, d, index = saved
    assert index["format"] == "decide-weights-v1"
    assert all(e["offset"] % (16 * 1024) == 0 for e in index["tensors"].values())
    b = Model(kernels.ctx, CFG)
    b.load(d)
    for name in a.tensor_names():
        np.testing.assert_array_equal(a.download(name).view(np.uint8), b.download(name).view(np.uint8), err_msg=name)
    ids, ans, cand, ncand = _request(37, CFG.vocab, 2, CFG.max_cand, 600)
    np.testing.assert_array_equal(_logits(a, ids, ans, cand, ncand), _logits(b, ids, ans, cand, ncand))
    b.close()


def _broken(d, tmp_path, edit):
    out = tmp_path / "broken"
    out.mkdir()
    for f in os.listdir(d):
        if f != "decide-index.json":
            os.symlink(os.path.join(d, f), out / f)
    index = json.load(open(os.path.join(d, "decide-index.json")))
    edit(index)
    json.dump(index, open(out / "decide-index.json", "w"))
    return str(out)


@pytest.mark.parametrize("edit,message", [
    (lambda ix: ix.update(format="decide-weights-v0"), "expected decide-weights-v1"),
    (lambda ix: ix["tensors"]["L1.w_gu"].update(offset=ix["tensors"]["L1.w_gu"]["offset"] + 2), "aligned"),
    (lambda ix: ix["tensors"]["L0.in_norm"].update(dtype="f16"), "the model holds it"),
    (lambda ix: ix["tensors"]["L2.a_log"].update(dtype="f64"), "unknown dtype"),
    (lambda ix: ix["tensors"]["L3.w_down"].update(shape=[2560, 9215]), "elements"),
    (lambda ix: ix["tensors"].pop("L3.k_norm"), "no tensor L3.k_norm"),
    (lambda ix: ix["tensors"]["final_norm"].update(offset=1 << 40), "runs past the end"),
    # 2^64 - 16 KiB is 16 KiB-aligned and exact as a double: offset + bytes would wrap below the blob length
    (lambda ix: ix["tensors"]["L1.w_gu"].update(offset=(1 << 64) - 16384), "bad offset"),
    (lambda ix: ix["tensors"]["L1.w_gu"].update(offset=16384.5), "bad offset"),
    (lambda ix: ix["tensors"]["L3.w_down"].update(shape=[1 << 32, 1 << 32]), "overflows"),
    (lambda ix: ix["tensors"]["L3.w_down"].update(shape=[2560, 9216.5]), "bad shape"),
    (lambda ix: ix["tensors"]["embed"].update(blob="decide-l99.bin"), "not in the blob list"),
])
def test_loader_refuses_bad_indexes(gpu, kernels, saved, tmp_path, edit, message):
    _, d, _ = saved
    b = Model(kernels.ctx, CFG)
    with pytest.raises(AssertionError, match=message):
        b.load(_broken(d, tmp_path, edit))
    b.close()


def test_loader_needs_an_index(gpu, kernels, tmp_path):
    b = Model(kernels.ctx, CFG)
    with pytest.raises(AssertionError, match="does not exist"):
        b.load(str(tmp_path))
    b.close()
