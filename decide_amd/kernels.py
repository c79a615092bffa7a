"""Host-side mirror of decide-engine's GEMM-path kernel wrappers over the C ABI.

decide's Rust layer (crates/decide-engine/src/kernels/) exposes one struct per
kernel family with one method per kernel; methods only encode onto the
caller's serial encoder and take buffers as ``Arg = (&Buffer, byte offset)``
(kernels/mod.rs:32). This module keeps those names, argument meanings and
error behaviour, with a HIP stream in place of the encoder:

* ``Arg`` is ``(device_buffer, byte_offset)``, where ``device_buffer`` is an
  integer device address or any object with ``data_ptr()``.
* ``stream`` is a hipStream_t handle (an int; 0 = the default stream).
* Contract violations raise ``AssertionError`` with decide's wording (decide
  panics through ``assert!``, gemm.rs:140-163); runtime failures raise
  ``DecideHipError``.

It is the Python face of the same library a Rust ``decide-hip`` crate binds
(see INTEGRATION.md); nothing here computes anything itself.
"""

from __future__ import annotations

import ctypes
import enum
from typing import Iterable, Sequence, Tuple, Union

from . import _lib

Buffer = Union[int, object]
Arg = Tuple[Buffer, int]


class Epilogue(enum.IntEnum):
    """decide's ``Epilogue`` (kernels/gemm.rs:15-26), same codes."""

    StoreF32 = 0
    StoreF16 = 1
    AddF32 = 2
    SwigluF16 = 3


class GemmImpl(enum.Enum):
    """decide's ``GemmImpl`` (kernels/gemm.rs:28-35)."""

    Fast = "fast"
    Baseline = "baseline"


SWIGLU_BLOCK = 16


def addr(a: Arg) -> int:
    """Device address of an ``Arg``."""
    buf, off = a
    base = buf if isinstance(buf, int) else int(buf.data_ptr())
    return base + int(off)


def _call(rc: int) -> None:
    if rc == _lib.DH_EINVAL:
        raise AssertionError(_lib.last_error())
    _lib.check(rc)


class Context:
    """One library context (the analog of the pipelines ``Kernels::new`` builds)."""

    def __init__(self, imp: GemmImpl = GemmImpl.Fast, delta: str = "auto"):
        lib = _lib.load()
        h = ctypes.c_void_p()
        flags = _lib.DH_GEMM_REFERENCE if imp == GemmImpl.Baseline else 0
        # the recurrence's implementation (decide's DECIDE_DELTA, kernels/delta.rs:36-49): "auto" picks by T
        flags |= {"auto": 0, "chunked": _lib.DH_DELTA_CHUNKED, "sequential": _lib.DH_DELTA_SEQUENTIAL}[delta]
        _lib.check(lib.dh_ctx_create(flags, ctypes.byref(h)))
        self.handle = h
        self.imp = imp
        self.lib = lib

    def close(self) -> None:
        if self.handle:
            self.lib.dh_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):  # pragma: no cover - interpreter shutdown order
        try:
            self.close()
        except Exception:
            pass


class Gemm:
    """decide's ``Gemm`` (kernels/gemm.rs:46-176)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    @classmethod
    def new(cls, ctx: Context) -> "Gemm":
        return cls(ctx)

    def implementation(self) -> GemmImpl:
        return self.ctx.imp

    def warm_up(self, stream: int = 0, max_m: int = 2560) -> None:
        """Loads every kernel and sizes the split-K workspace (gemm.rs:87-107)."""
        _lib.check(self.lib.dh_warm_up(self.ctx.handle, ctypes.c_void_p(stream), max_m))

    def fast_pipelines(self) -> int:
        """Kernels launched so far; must not grow after ``warm_up`` (gemm.rs:109-113)."""
        return int(self.lib.dh_variants_loaded(self.ctx.handle))

    def gemm(self, stream: int, x: Arg, w: Arg, y: Arg, m: int, n: int, k: int, ldx: int, ldw: int, ldy: int,
             epi: Epilogue) -> None:
        """``Y = X · Wᵀ``, then ``epi`` (gemm.rs:126-176). X fp16 [M, K] (row stride ldx), W fp16
        [N, K] (row stride ldw), ldy in elements of Y's type; fp32 accumulation."""
        _call(self.lib.dh_gemm_nt(self.ctx.handle, ctypes.c_void_p(stream), addr(x), ldx, addr(w), ldw, addr(y),
                                  ldy, m, n, k, int(epi)))

    def gemm_add_rmsnorm(self, stream: int, x: Arg, w: Arg, y: Arg, m: int, n: int, k: int, ldx: int, ldw: int,
                         ldy: int, norm_w: Arg, h: Arg, ldh: int, add_one: bool = True, eps: float = 1e-6) -> None:
        """``y += X · Wᵀ`` (fp32 y, the AddF32 epilogue), then ``h = rmsnorm(y)`` fp16 row by row: bitwise
        ``gemm(..., AddF32)`` followed by the row norm, one kernel for both where K is split."""
        _call(self.lib.dh_gemm_add_rmsnorm(self.ctx.handle, ctypes.c_void_p(stream), addr(x), ldx, addr(w), ldw,
                                           addr(y), ldy, m, n, k, addr(norm_w), 1 if add_one else 0, eps, addr(h),
                                           ldh))

    def gemm_grouped(self, stream: int, x: Arg, ldx: int, m: int, k: int,
                     members: Sequence[Tuple[Arg, int, int, Arg, int, Epilogue]]) -> None:
        """Every member ``(w, ldw, n, y, ldy, epi)`` shares X; one launch."""
        arr = (_lib.DhGemmMember * len(members))()
        for i, (w, ldw, n, y, ldy, epi) in enumerate(members):
            arr[i] = _lib.DhGemmMember(addr(w), addr(y), ldw, ldy, n, int(epi))
        _call(self.lib.dh_gemm_nt_grouped(self.ctx.handle, ctypes.c_void_p(stream), addr(x), ldx, m, k, arr,
                                          len(members)))

    def plan(self, m: int, n: int, k: int, epi: Epilogue) -> dict:
        p = _lib.DhGemmPlan()
        _call(self.lib.dh_gemm_plan_for(self.ctx.handle, m, n, k, int(epi), ctypes.byref(p)))
        return {f: getattr(p, f) for f, _ in _lib.DhGemmPlan._fields_}

    def force(self, variant: int | None, splits: int = 1) -> None:
        """Pin the tile variant / split-K (tuning only); ``None`` restores the planner."""
        v = 0xFFFFFFFF if variant is None else variant
        _call(self.lib.dh_gemm_force(self.ctx.handle, v, splits))


def plan_for(m: int, n: int, k: int, epi: Epilogue) -> dict:
    """The planner's choice without a context or a device."""
    lib = _lib.load()
    p = _lib.DhGemmPlan()
    _call(lib.dh_gemm_plan_for(None, m, n, k, int(epi), ctypes.byref(p)))
    return {f: getattr(p, f) for f, _ in _lib.DhGemmPlan._fields_}


def variants() -> list:
    """Geometry of every compiled tile variant: dicts of bm, bn, waves, wave_cols."""
    lib = _lib.load()
    out = []
    for v in range(lib.dh_gemm_variant_count()):
        vals = [ctypes.c_uint32() for _ in range(4)]
        _lib.check(lib.dh_gemm_variant_info(v, *[ctypes.byref(x) for x in vals]))
        out.append(dict(zip(("bm", "bn", "waves", "wave_cols"), (x.value for x in vals))))
    return out


class Head:
    """decide's ``Head`` (kernels/head.rs:14-60): row gathers and the candidate head."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def gather_rows_f32(self, stream: int, x: Arg, rowmap: Arg, out: Arg, rows: int, h: int) -> None:
        """out[i] = x[rowmap[i]] for ``rows`` fp32 rows of ``h`` elements."""
        _call(self.lib.dh_gather_rows_f32(self.ctx.handle, ctypes.c_void_p(stream), addr(x), addr(rowmap),
                                          addr(out), rows, h))

    def gather_rows_f16(self, stream: int, x: Arg, rowmap: Arg, out: Arg, rows: int, h: int) -> None:
        """out[i] = x[rowmap[i]] for ``rows`` 16-bit rows (fp16 or bf16) of ``h`` elements."""
        _call(self.lib.dh_gather_rows_f16(self.ctx.handle, ctypes.c_void_p(stream), addr(x), addr(rowmap),
                                          addr(out), rows, h))

    def final_head(self, stream: int, x: Arg, w: Arg, table: Arg, cand: Arg, ncand: Arg, logits: Arg, rows: int,
                   hidden: int = 2560, max_cand: int = 62, eps: float = 1e-6) -> None:
        """``cpu_ref::final_head``: zero-centred RMSNorm of each row, then fp32 logits against its
        bf16 candidate rows. decide fixes hidden 2560 / 62 candidates; both are parameters here."""
        _call(self.lib.dh_final_head(self.ctx.handle, ctypes.c_void_p(stream), addr(x), addr(w), addr(table),
                                     addr(cand), addr(ncand), addr(logits), rows, hidden, max_cand, eps))


class Norm:
    """decide's ``Norm`` (kernels/norm.rs:11-33)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def rmsnorm(self, stream: int, x: Arg, w: Arg, y: Arg, rowmap: Arg, rows: int, h: int, ld_in: int, ld_out: int,
                add_one: bool, eps: float = 1e-6) -> None:
        """y[r] = rmsnorm(x[rowmap[r]]) · (w or 1 + w) as fp16."""
        _call(self.lib.dh_rmsnorm_rows(self.ctx.handle, ctypes.c_void_p(stream), addr(x), addr(w), addr(y),
                                       addr(rowmap), rows, h, ld_in, ld_out, 1 if add_one else 0, eps))


class Embed:
    """decide's ``Embed`` (kernels/embed.rs:11-24)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def embed(self, stream: int, ids: Arg, table: Arg, out: Arg, t: int, h: int = 2560) -> None:
        """out[t] = embed[ids[t]] (bf16 → f32), rows [t, h]."""
        _call(self.lib.dh_embed_bf16(self.ctx.handle, ctypes.c_void_p(stream), addr(ids), addr(table), addr(out), t,
                                     h))


class Conv:
    """decide's ``Conv`` (kernels/conv.rs:11-48)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def conv_silu_l2(self, stream: int, p: Arg, prev: Arg, w: Arg, q: Arg, k: Arg, v: Arg, t: int, ldp: int) -> None:
        _call(self.lib.dh_conv_silu_l2(self.ctx.handle, ctypes.c_void_p(stream), addr(p), addr(prev), addr(w),
                                       addr(q), addr(k), addr(v), t, ldp))

    def conv_state_update(self, stream: int, p: Arg, prev_in: Arg, prev_out: Arg, t: int, ldp: int) -> None:
        _call(self.lib.dh_conv_state_update(self.ctx.handle, ctypes.c_void_p(stream), addr(p), addr(prev_in),
                                            addr(prev_out), t, ldp))


class Delta:
    """decide's ``Delta`` (kernels/delta.rs:28-80)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def gated_delta(self, stream: int, q: Arg, k: Arg, v: Arg, a: Arg, b: Arg, a_log: Arg, dt_bias: Arg,
                    state_in: Arg, state_out: Arg, o: Arg, t: int, ldab: int, write_state: bool) -> None:
        _call(self.lib.dh_gated_delta(self.ctx.handle, ctypes.c_void_p(stream), addr(q), addr(k), addr(v), addr(a),
                                      addr(b), addr(a_log), addr(dt_bias), addr(state_in), addr(state_out), addr(o),
                                      t, ldab, 1 if write_state else 0))

    def conv_gated_delta_chunked(self, stream: int, p: Arg, prev: Arg, w: Arg, q: Arg, a: Arg, b: Arg, a_log: Arg,
                                 dt_bias: Arg, state_in: Arg, state_out: Arg, o: Arg, t: int, ldp: int, ldab: int,
                                 write_state: bool) -> None:
        """``Conv::conv_silu_l2`` then ``gated_delta`` in one call on the chunked recurrence (only q is written
        of the conv outputs)."""
        _call(self.lib.dh_conv_gated_delta_chunked(self.ctx.handle, ctypes.c_void_p(stream), addr(p), addr(prev),
                                                   addr(w), addr(q), addr(a), addr(b), addr(a_log), addr(dt_bias),
                                                   addr(state_in), addr(state_out), addr(o), t, ldp, ldab,
                                                   1 if write_state else 0))


class GNorm:
    """decide's ``GNorm`` (kernels/gnorm.rs:10-31)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def gated_rmsnorm_silu(self, stream: int, o: Arg, z: Arg, w: Arg, y: Arg, t: int, ldz: int) -> None:
        _call(self.lib.dh_gated_rmsnorm_silu(self.ctx.handle, ctypes.c_void_p(stream), addr(o), addr(z), addr(w),
                                             addr(y), t, ldz))


class Rope:
    """decide's ``Rope`` (kernels/rope.rs:16-54)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def q_norm_rope(self, stream: int, pq: Arg, qw: Arg, inv_freq: Arg, qpos: Arg, qo: Arg, rows: int,
                    ldq: int) -> None:
        _call(self.lib.dh_q_norm_rope(self.ctx.handle, ctypes.c_void_p(stream), addr(pq), addr(qw), addr(inv_freq),
                                      addr(qpos), addr(qo), rows, ldq))

    def kv_norm_rope(self, stream: int, pkv: Arg, kw: Arg, inv_freq: Arg, kc: Arg, vc: Arg, rows: int, ldkv: int,
                     kcol: int, vcol: int, pos0: int) -> None:
        _call(self.lib.dh_kv_norm_rope(self.ctx.handle, ctypes.c_void_p(stream), addr(pkv), addr(kw), addr(inv_freq),
                                       addr(kc), addr(vc), rows, ldkv, kcol, vcol, pos0))


class Attn:
    """decide's ``Attn`` (kernels/attn.rs:44-125)."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib

    def attention(self, stream: int, q: Arg, kc: Arg, vc: Arg, pq: Arg, qpos: Arg, y: Arg, rows: int,
                  ldq: int) -> None:
        _call(self.lib.dh_attention(self.ctx.handle, ctypes.c_void_p(stream), addr(q), addr(kc), addr(vc), addr(pq),
                                    addr(qpos), addr(y), rows, ldq))


def fill_normal(ctx: Context, stream: int, out: Arg, n: int, seed: int, mean: float, std: float, dtype: str) -> None:
    """N(mean, std) fill of fp16 / bf16 / fp32 values from the counter-based generator."""
    code = {"f16": 0, "bf16": 1, "f32": 2}[dtype]
    _call(ctx.lib.dh_fill_normal(ctx.handle, ctypes.c_void_p(stream), addr(out), n, seed, mean, std, code))


def fill_normal_f16(ctx: Context, stream: int, out: Arg, n: int, seed: int, std: float) -> None:
    """N(0, std) fp16 fill from a counter-based generator (reproducible per (seed, index))."""
    _call(ctx.lib.dh_fill_normal_f16(ctx.handle, ctypes.c_void_p(stream), addr(out), n, seed, std))


class Kernels:
    """decide's ``Kernels`` registry (kernels/mod.rs:40-67): the GEMM path and the forward kernels beside it."""

    def __init__(self, imp: GemmImpl = GemmImpl.Fast, delta: str = "auto"):
        self.ctx = Context(imp, delta)
        self.gemm = Gemm(self.ctx)
        self.head = Head(self.ctx)
        self.norm = Norm(self.ctx)
        self.embed = Embed(self.ctx)
        self.conv = Conv(self.ctx)
        self.delta = Delta(self.ctx)
        self.gnorm = GNorm(self.ctx)
        self.rope = Rope(self.ctx)
        self.attn = Attn(self.ctx)
