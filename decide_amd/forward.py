"""Host mirror of decide's ``Forward`` (crates/decide-engine/src/forward.rs) over the C ABI.

The model owns its weights and activation buffers in device memory (``dh_model_create``), named as in
decide's ``decide-weights-v1`` index (convert.rs:158-245). ``forward`` enqueues one full-route forward
(embedding, every layer, the pruned last layer, the candidate head) on a stream. The request methods
(``logits``, ``build_snapshot``, the state cache; forward.rs:641-1116) take host ids and answers, run in
chunks from the prefix snapshot or a cached state, and wait for their result, as decide's do. Nothing
here computes anything itself.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .kernels import Arg, Context, _call, addr

DTYPES = {0: np.float16, 1: np.uint16, 2: np.float32}  # bf16 weights are returned as raw bits

# decide's Route (forward.rs:196-207)
ROUTES = {_lib.DH_ROUTE_SNAPSHOT: "snapshot", _lib.DH_ROUTE_FULL: "full", _lib.DH_ROUTE_STATE_CACHE: "state_cache"}
MAX_STATE_ENTRIES = 4  # forward.rs:70
STATE_MARKER = (550, 39087, 10485, 198)  # forward.rs:68


def _u32(values) -> ctypes.Array:
    a = np.ascontiguousarray(np.asarray(values, dtype=np.int64))
    if a.size and (a.min() < 0 or a.max() > 0xFFFFFFFF):
        raise ValueError("ids must be unsigned 32-bit")
    return (ctypes.c_uint32 * max(a.size, 1))(*a.tolist())


def state_boundary(ids, prefix: int, marker, limit: int):
    """Where a prompt's state ends: one past the first ``marker`` in ``ids[prefix:limit]``, or None
    (decide: state_boundary, forward.rs:1503-1515). Host code of the library, no GPU involved."""
    lib = _lib.load()
    ids, marker = list(ids), list(marker)
    b, found = ctypes.c_uint32(), ctypes.c_int()
    _call(lib.dh_state_boundary(_u32(ids), len(ids), prefix, _u32(marker), len(marker), limit, ctypes.byref(b),
                                ctypes.byref(found)))
    return int(b.value) if found.value else None


@dataclass
class ModelConfig:
    """decide's model shape parameters that BASELINE varies (config.rs:4-37)."""

    layers: int = 36
    vocab: int = 151936
    max_tokens: int = 2307
    max_answers: int = 16
    max_cand: int = 62


def is_full_attention(layer: int) -> bool:
    """config.rs:39-41."""
    return (layer + 1) % 4 == 0


class Model:
    def __init__(self, ctx: Context, cfg: ModelConfig):
        self.ctx = ctx
        self.cfg = cfg
        self.lib = ctx.lib
        c = _lib.DhModelConfig(cfg.layers, cfg.vocab, cfg.max_tokens, cfg.max_answers, cfg.max_cand)
        h = ctypes.c_void_p()
        _call(self.lib.dh_model_create(ctx.handle, ctypes.byref(c), ctypes.byref(h)))
        self.handle = h

    def close(self) -> None:
        if self.handle:
            self.lib.dh_model_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass

    def tensor(self, name: str) -> tuple[int, int, type]:
        """(device address, elements, numpy dtype) of a weight."""
        ptr, n, dt = ctypes.c_void_p(), ctypes.c_uint64(), ctypes.c_uint32()
        _call(self.lib.dh_model_tensor(self.handle, name.encode(), ctypes.byref(ptr), ctypes.byref(n),
                                       ctypes.byref(dt)))
        return int(ptr.value), int(n.value), DTYPES[dt.value]

    def download(self, name: str) -> np.ndarray:
        """A weight's values on the host (bf16 as raw uint16 bits)."""
        from .hip import D2H, check, rt

        ptr, n, dtype = self.tensor(name)
        out = np.empty(n, dtype=dtype)
        check(rt().hipMemcpy(out.ctypes.data, ptr, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def tensor_names(self) -> list[str]:
        names, i = [], 0
        while True:
            n = self.lib.dh_model_tensor_name(self.handle, i)
            if n is None:
                return names
            names.append(n.decode())
            i += 1

    def load(self, directory: str) -> None:
        """Fill every weight from a decide-weights-v1 directory (decide: Weights::open, weights.rs:105-183)."""
        _call(self.lib.dh_model_load(self.handle, directory.encode()))

    def init_random(self, stream: int, seed: int) -> None:
        _call(self.lib.dh_model_init_random(self.handle, ctypes.c_void_p(stream), seed))

    def capture(self, stream: int, ids: Arg, t: int, ans_rows: Arg, n_ans: int, cand: Arg, ncand: Arg, logits: Arg,
                prune: bool = True) -> "Graph":
        """Run one forward eagerly, then capture the next into a replayable graph (same buffers and sizes)."""
        flags = 0 if prune else _lib.DH_FORWARD_NO_PRUNE
        g = ctypes.c_void_p()
        _call(self.lib.dh_model_capture(self.handle, ctypes.c_void_p(stream), addr(ids), t, addr(ans_rows), n_ans,
                                        addr(cand), addr(ncand), addr(logits), flags, ctypes.byref(g)))
        return Graph(self.lib, g)

    def forward(self, stream: int, ids: Arg, t: int, ans_rows: Arg, n_ans: int, cand: Arg, ncand: Arg,
                logits: Arg, prune: bool = True) -> None:
        """decide's Forward::logits for the full route, enqueued on ``stream`` (no synchronisation)."""
        flags = 0 if prune else _lib.DH_FORWARD_NO_PRUNE
        _call(self.lib.dh_model_forward(self.handle, ctypes.c_void_p(stream), addr(ids), t, addr(ans_rows), n_ans,
                                        addr(cand), addr(ncand), addr(logits), flags))


    # ---- requests (decide: Forward, forward.rs:641-1116); host ids, synchronous
    def logits(self, stream: int, ids, answers, full: bool = False) -> list[list[float]]:
        """Logits of each answer's candidates: ``answers`` is a list of (absolute logit row, candidate ids);
        one row of logits per answer, in the given order (decide: logits / logits_full, forward.rs:696-815)."""
        ids = list(ids)
        arr = (_lib.DhAnswer * max(len(answers), 1))()
        keep = []
        for i, (row, cand) in enumerate(answers):
            c = _u32(list(cand))
            keep.append(c)
            arr[i].row = int(row)
            arr[i].ncand = len(cand)
            arr[i].cand = ctypes.cast(c, ctypes.POINTER(ctypes.c_uint32))
        mc = self.cfg.max_cand
        out = np.full(max(len(answers), 1) * mc, np.nan, dtype=np.float32)
        flags = _lib.DH_LOGITS_FULL if full else 0
        _call(self.lib.dh_model_logits(self.handle, ctypes.c_void_p(stream), _u32(ids), len(ids), arr, len(answers),
                                       out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), flags))
        return [out[i * mc:i * mc + len(c)].tolist() for i, (_, c) in enumerate(answers)]

    def logits_full(self, stream: int, ids, answers) -> list[list[float]]:
        """``logits`` by the full path whatever the ids (decide: logits_full, forward.rs:809-815)."""
        return self.logits(stream, ids, answers, full=True)

    def build_snapshot(self, stream: int, prefix_ids) -> None:
        """Run the constant prompt prefix from zero state and keep the state after it (forward.rs:641-675)."""
        ids = list(prefix_ids)
        _call(self.lib.dh_model_build_snapshot(self.handle, ctypes.c_void_p(stream), _u32(ids), len(ids)))

    def prefix_len(self):
        n, has = ctypes.c_uint32(), ctypes.c_int()
        _call(self.lib.dh_model_prefix_len(self.handle, ctypes.byref(n), ctypes.byref(has)))
        return int(n.value) if has.value else None

    def last_route(self):
        """"snapshot", "full" or "state_cache" for the last ``logits`` call (None before the first)."""
        r, s = ctypes.c_int32(), ctypes.c_int64()
        _call(self.lib.dh_model_last_route(self.handle, ctypes.byref(r), ctypes.byref(s)))
        return ROUTES.get(r.value)

    def last_start(self):
        """The first position the last ``logits`` call computed (forward.rs:688-694)."""
        r, s = ctypes.c_int32(), ctypes.c_int64()
        _call(self.lib.dh_model_last_route(self.handle, ctypes.byref(r), ctypes.byref(s)))
        return None if s.value < 0 else int(s.value)

    def chunk(self) -> int:
        return int(self.lib.dh_model_chunk(self.handle))

    def set_chunk(self, rows: int) -> None:
        _call(self.lib.dh_model_set_chunk(self.handle, rows))

    def pruning(self) -> bool:
        return bool(self.lib.dh_model_pruning(self.handle))

    def set_pruning(self, on: bool) -> None:
        self.lib.dh_model_set_pruning(self.handle, 1 if on else 0)

    def set_state_cache(self, entries: int) -> None:
        _call(self.lib.dh_model_set_state_cache(self.handle, entries))

    def state_cache_capacity(self) -> int:
        return int(self.lib.dh_model_state_cache_capacity(self.handle))

    def forget_states(self) -> None:
        self.lib.dh_model_forget_states(self.handle)

    def cached_states(self) -> list[int]:
        buf = (ctypes.c_uint32 * MAX_STATE_ENTRIES)()
        n = self.lib.dh_model_cached_states(self.handle, buf, MAX_STATE_ENTRIES)
        return [int(buf[i]) for i in range(min(n, MAX_STATE_ENTRIES))]

    def set_state_marker(self, marker) -> None:
        m = list(marker)
        _call(self.lib.dh_model_set_state_marker(self.handle, _u32(m), len(m)))


class Graph:
    """A captured whole forward (dh_model_capture): one launch replays every kernel of the forward."""

    def __init__(self, lib, handle):
        self.lib = lib
        self.handle = handle

    def launch(self, stream: int) -> None:
        _call(self.lib.dh_graph_launch(self.handle, ctypes.c_void_p(stream)))

    def close(self) -> None:
        if self.handle:
            self.lib.dh_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover
        try:
            self.close()
        except Exception:
            pass


def main():
    """Time random-init forwards: python -m decide_amd.forward [--layers 36] [--tokens 2307] [--runs 5]."""
    import argparse
    import json

    from . import hip, synth
    from .hip import DeviceArray, Event, Stream
    from .kernels import Kernels

    ap = argparse.ArgumentParser(description=main.__doc__)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--vocab", type=int, default=151936)
    ap.add_argument("--tokens", type=int, default=2307)
    ap.add_argument("--runs", type=int, default=5)
    ap.add_argument("--no-prune", action="store_true")
    ap.add_argument("--delta", choices=["auto", "chunked", "sequential"], default="auto",
                    help="gated delta implementation (auto: chunked from DH_DELTA_CHUNK_MIN_T tokens)")
    args = ap.parse_args()
    if not hip.available():
        raise SystemExit("no GPU")
    k = Kernels(delta=args.delta)
    st = Stream()
    s = st.handle
    t = args.tokens
    model = Model(k.ctx, ModelConfig(args.layers, args.vocab, t, 3, 8))
    model.init_random(s, seed=0xDEC1DE)
    k.gemm.warm_up(s, max_m=t)
    ids = DeviceArray.from_numpy(synth.uniform_ids(synth.seed_for(500 + t), t, args.vocab).astype(np.uint32))
    ans = DeviceArray.from_numpy(np.array([t - 3, t - 2, t - 1], np.uint32))
    cand = DeviceArray.from_numpy(synth.uniform_ids(synth.seed_for(501 + t), 24, args.vocab).astype(np.uint32))
    ncand = DeviceArray.from_numpy(np.full(3, 8, np.uint32))
    logits = DeviceArray((3, 8), np.float32)
    times = []
    for i in range(args.runs + 1):
        e0, e1 = Event(), Event()
        e0.record(s)
        model.forward(s, (ids, 0), t, (ans, 0), 3, (cand, 0), (ncand, 0), (logits, 0), prune=not args.no_prune)
        e1.record(s)
        e1.synchronize()
        if i:
            times.append(e0.elapsed_ms(e1))
    print(json.dumps({"layers": args.layers, "tokens": t, "runs": args.runs, "delta": args.delta,
                      "p50_ms": float(np.median(times)),
                      "logits": logits.numpy().round(4).tolist()}), flush=True)
    model.close()


if __name__ == "__main__":
    main()
