"""Write a model's weights as a decide-weights-v1 directory (the layout decide's converter writes,
crates/decide-engine/src/convert.rs:140-200, 300-400), so a set can be saved and re-loaded with
``Model.load`` / ``dh_model_load``.

Layout: ``decide-index.json`` = {"format": "decide-weights-v1", "blobs": [...], "tensors": {name:
{"blob", "offset", "dtype", "shape"}}}; blob ``decide-embed.bin`` holds the bf16 embedding, blobs
``decide-lNN.bin`` hold layers NN .. NN+7 in forward order, ``final_norm`` closes the last blob; every
tensor starts at a 16 KiB boundary and every blob is zero-padded to one.
"""

from __future__ import annotations

import json
import os

import numpy as np

from .forward import Model

ALIGN = 16 * 1024
FORMAT = "decide-weights-v1"
EMBED_BLOB = "decide-embed.bin"
LAYERS_PER_BLOB = 8
DTYPE_NAMES = {np.float16: "f16", np.uint16: "bf16", np.float32: "f32"}


def _shape(name: str, n: int) -> list[int]:
    key = name.split(".")[-1]
    cols = {"embed": 2560, "w_in": 2560, "w_gu": 2560, "w_down": 9216, "conv_w": 4, "w_out": None}
    if key == "w_out":
        return [2560, n // 2560]
    if key in cols:
        return [n // cols[key], cols[key]]
    return [n]


def save(model: Model, directory: str) -> dict:
    """Write every tensor of ``model`` to ``directory``; returns the index."""
    os.makedirs(directory, exist_ok=True)
    layers = model.cfg.layers
    blob_names = [EMBED_BLOB] + [f"decide-l{l:02d}.bin" for l in range(0, layers, LAYERS_PER_BLOB)]
    files = {b: open(os.path.join(directory, b), "wb") for b in blob_names}
    lengths = {b: 0 for b in blob_names}
    tensors = {}

    def put(blob: str, name: str):
        data = model.download(name)
        f = files[blob]
        pad = -lengths[blob] % ALIGN
        f.write(b"\0" * pad)
        lengths[blob] += pad
        tensors[name] = {"blob": blob, "offset": lengths[blob], "dtype": DTYPE_NAMES[data.dtype.type],
                         "shape": _shape(name, data.size)}
        f.write(data.tobytes())
        lengths[blob] += data.nbytes

    names = model.tensor_names()
    put(EMBED_BLOB, "embed")
    for l in range(layers):
        blob = blob_names[1 + l // LAYERS_PER_BLOB]
        for name in names:
            if name.startswith(f"L{l}."):
                put(blob, name)
    put(blob_names[-1], "final_norm")
    for b, f in files.items():
        f.write(b"\0" * (-lengths[b] % ALIGN))
        f.close()
    index = {"format": FORMAT, "blobs": blob_names, "tensors": tensors}
    with open(os.path.join(directory, "decide-index.json"), "w") as f:
        json.dump(index, f, indent=1)
    return index
