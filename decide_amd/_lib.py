"""ctypes binding of libdecide_hip.so, the C ABI declared in include/decide_hip.h.

The library is loaded from this package directory only (it is built in-tree by
``decide_amd/csrc/Makefile``); a missing or stale library raises instead of
falling back to anything else.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_uint16, c_uint32, c_uint64, c_void_p

# DH_LIB names another build of the same library (the sanitizer builds of decide_amd/csrc/Makefile); unset, the
# in-tree library is the one loaded.
LIB_PATH = os.environ.get("DH_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), "libdecide_hip.so")

DH_OK = 0
DH_EINVAL = 1
DH_ELAUNCH = 2
DH_ENOMEM = 3
DH_EDEVICE = 4

DH_GEMM_REFERENCE = 1
DH_GEMM_STREAM_VARIANT = 64
DH_DELTA_CHUNKED = 2
DH_DELTA_SEQUENTIAL = 4
DH_DELTA_CHUNK_MIN_T = 320


class DhGemmMember(ctypes.Structure):
    """``dh_gemm_member`` (include/decide_hip.h)."""

    _fields_ = [
        ("w", c_void_p),
        ("y", c_void_p),
        ("ldw", c_uint32),
        ("ldy", c_uint32),
        ("n", c_uint32),
        ("epi", c_uint32),
    ]


class DhGemmPlan(ctypes.Structure):
    """``dh_gemm_plan`` (include/decide_hip.h)."""

    _fields_ = [
        ("variant", c_uint32),
        ("bm", c_uint32),
        ("bn", c_uint32),
        ("waves", c_uint32),
        ("splits", c_uint32),
        ("workgroups", c_uint32),
        ("ws_bytes", c_uint64),
        ("order", c_uint32),
    ]


# name -> (restype, argtypes); every symbol include/decide_hip.h declares.
class DhModelConfig(ctypes.Structure):
    _fields_ = [("layers", c_uint32), ("vocab", c_uint32), ("max_tokens", c_uint32), ("max_answers", c_uint32),
                ("max_cand", c_uint32)]


class DhAnswer(ctypes.Structure):
    """``dh_answer`` (include/decide_hip.h): one answer row and its host candidate ids."""

    _fields_ = [("row", c_uint32), ("ncand", c_uint32), ("cand", POINTER(c_uint32))]


DH_FORWARD_NO_PRUNE = 1
DH_LOGITS_FULL = 1
DH_ROUTE_SNAPSHOT = 0
DH_ROUTE_FULL = 1
DH_ROUTE_STATE_CACHE = 2

PROTOTYPES = {
    "dh_ctx_create": (c_int, [c_uint32, POINTER(c_void_p)]),
    "dh_ctx_destroy": (None, [c_void_p]),
    "dh_last_error": (c_char_p, []),
    "dh_version": (c_char_p, []),
    "dh_warm_up": (c_int, [c_void_p, c_void_p, c_uint32]),
    "dh_variants_loaded": (c_uint32, [c_void_p]),
    "dh_gemm_nt": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_uint32, c_void_p, c_uint32, c_uint32, c_uint32,
         c_uint32, c_uint32],
    ),
    "dh_gemm_nt_noalloc": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_uint32, c_void_p, c_uint32, c_uint32, c_uint32,
         c_uint32, c_uint32],
    ),
    "dh_gemm_nt_grouped": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, POINTER(DhGemmMember), c_uint32],
    ),
    "dh_gemm_plan_for": (c_int, [c_void_p, c_uint32, c_uint32, c_uint32, c_uint32, POINTER(DhGemmPlan)]),
    "dh_gemm_ws_need": (c_int, [c_void_p, c_uint32, c_uint32, c_uint32, POINTER(c_uint64)]),
    "dh_gemm_force": (c_int, [c_void_p, c_uint32, c_uint32]),
    "dh_gemm_variant_count": (c_uint32, []),
    "dh_gemm_variant_info": (
        c_int,
        [c_uint32, POINTER(c_uint32), POINTER(c_uint32), POINTER(c_uint32), POINTER(c_uint32)],
    ),
    "dh_gather_rows_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32]),
    "dh_gather_rows_f16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32]),
    "dh_final_head": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32,
         c_uint32, c_float],
    ),
    "dh_rmsnorm_rows": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32,
         c_uint32, c_float],
    ),
    "dh_gemm_add_rmsnorm": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_uint32, c_void_p, c_uint32, c_uint32, c_uint32,
         c_uint32, c_void_p, c_uint32, c_float, c_void_p, c_uint32],
    ),
    "dh_fill_normal_f16": (c_int, [c_void_p, c_void_p, c_void_p, c_uint64, c_uint64, c_float]),
    "dh_interleave_gate_up": (c_int, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32]),
    "dh_deinterleave_q_gate": (c_int, [c_void_p, c_void_p, c_uint32, c_uint32, c_uint32]),
    "dh_bf16_to_f16": (c_int, [c_void_p, c_void_p, c_uint64, POINTER(c_uint64)]),
    "dh_embed_bf16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32]),
    "dh_conv_silu_l2": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32],
    ),
    "dh_conv_state_update": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32]),
    "dh_gated_delta": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_uint32, c_uint32, c_uint32],
    ),
    "dh_conv_gated_delta_chunked": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32],
    ),
    "dh_gated_rmsnorm_silu": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32]),
    "dh_q_norm_rope": (
        c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32]),
    "dh_kv_norm_rope": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32,
         c_uint32, c_uint32],
    ),
    "dh_attention": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32],
    ),
    "dh_fill_normal": (c_int, [c_void_p, c_void_p, c_void_p, c_uint64, c_uint64, c_float, c_float, c_uint32]),
    "dh_model_create": (c_int, [c_void_p, POINTER(DhModelConfig), POINTER(c_void_p)]),
    "dh_model_destroy": (None, [c_void_p]),
    "dh_model_tensor": (c_int, [c_void_p, c_char_p, POINTER(c_void_p), POINTER(c_uint64), POINTER(c_uint32)]),
    "dh_model_init_random": (c_int, [c_void_p, c_void_p, c_uint64]),
    "dh_model_tensor_name": (c_char_p, [c_void_p, c_uint32]),
    "dh_model_load": (c_int, [c_void_p, c_char_p]),
    "dh_model_capture": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_uint32, c_void_p, c_void_p, c_void_p, c_uint32,
         POINTER(c_void_p)],
    ),
    "dh_graph_launch": (c_int, [c_void_p, c_void_p]),
    "dh_graph_destroy": (None, [c_void_p]),
    "dh_model_forward": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_uint32, c_void_p, c_void_p, c_void_p, c_uint32],
    ),
    "dh_model_logits": (
        c_int, [c_void_p, c_void_p, POINTER(c_uint32), c_uint32, POINTER(DhAnswer), c_uint32, POINTER(c_float), c_uint32]),
    "dh_model_build_snapshot": (c_int, [c_void_p, c_void_p, POINTER(c_uint32), c_uint32]),
    "dh_model_prefix_len": (c_int, [c_void_p, POINTER(c_uint32), POINTER(c_int)]),
    "dh_model_last_route": (c_int, [c_void_p, POINTER(ctypes.c_int32), POINTER(ctypes.c_int64)]),
    "dh_model_set_chunk": (c_int, [c_void_p, c_uint32]),
    "dh_model_chunk": (c_uint32, [c_void_p]),
    "dh_model_set_pruning": (None, [c_void_p, c_int]),
    "dh_model_pruning": (c_int, [c_void_p]),
    "dh_model_set_state_cache": (c_int, [c_void_p, c_uint32]),
    "dh_model_state_cache_capacity": (c_uint32, [c_void_p]),
    "dh_model_forget_states": (None, [c_void_p]),
    "dh_model_cached_states": (c_uint32, [c_void_p, POINTER(c_uint32), c_uint32]),
    "dh_model_set_state_marker": (c_int, [c_void_p, POINTER(c_uint32), c_uint32]),
    "dh_state_boundary": (
        c_int, [POINTER(c_uint32), c_uint32, c_uint32, POINTER(c_uint32), c_uint32, c_uint32, POINTER(c_uint32),
                POINTER(c_int)]),
}

_lib = None


class DecideHipError(RuntimeError):
    """A DH_E* status from the library, with its message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


def load() -> ctypes.CDLL:
    """The loaded library (loaded once). Raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built: run `make -C decide_amd/csrc` (or __graft_entry__.build()). "
            "There is no fallback path."
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().dh_last_error().decode()


def check(rc: int) -> None:
    """Raise DecideHipError for a non-DH_OK status."""
    if rc != DH_OK:
        raise DecideHipError(rc, last_error())
