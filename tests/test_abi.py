"""CPU-only checks of the C ABI: the library loads, exports every declared symbol, and rejects
contract violations before touching a device (decide's Gemm::gemm asserts, gemm.rs:140-163).
No compute call is made here."""

import ctypes
import os
import re

import numpy as np
import pytest

from decide_amd import _lib
from decide_amd.kernels import Epilogue, plan_for, variants

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    with open(os.path.join(ROOT, "include", "decide_hip.h")) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
    # and the binding covers exactly the header
    assert sorted(_lib.PROTOTYPES) == names


def test_version_string():
    assert b"gfx950" in _lib.load().dh_version()


def bad_gemm(**kw):
    args = dict(x=16, ldx=64, w=16, ldw=64, y=16, ldy=64, m=4, n=64, k=64, epi=0)
    args.update(kw)
    lib = _lib.load()
    rc = lib.dh_gemm_nt(None, None, args["x"], args["ldx"], args["w"], args["ldw"], args["y"], args["ldy"],
                        args["m"], args["n"], args["k"], args["epi"])
    return rc, _lib.last_error()


@pytest.mark.parametrize("kw,msg", [
    (dict(n=48), "multiples of 32"),
    (dict(k=40), "multiples of 32"),
    (dict(m=0), "M must be at least 1"),
    (dict(ldx=32), "must cover K"),
    (dict(ldw=32), "must cover K"),
    (dict(ldy=32), "must cover the 64 output columns"),
    (dict(ldx=68, k=64), "multiples of 8"),
    (dict(x=24), "multiples of 16"),
    (dict(w=8), "multiples of 16"),
    (dict(ldy=65), "must be even"),
    (dict(y=4, epi=0), "multiple of 8"),
    (dict(y=2, epi=3, ldy=32), "multiple of 4"),
    (dict(epi=4), "epilogue"),
    (dict(m=233017, ldx=9216, ldw=9216, k=9216), "X rows span more than 4 GiB"),
    (dict(n=262144, ldx=8192, ldw=8192, ldy=262144, k=8192), "W rows span more than 4 GiB"),
])
def test_gemm_contract_violations_are_rejected(kw, msg):
    rc, err = bad_gemm(**kw)
    assert rc == _lib.DH_EINVAL
    assert msg in err, err


def test_swiglu_output_width_is_half_n():
    rc, err = bad_gemm(epi=3, ldy=32)  # n = 64 → 32 output columns: ok contract, then null ctx
    assert rc == _lib.DH_EINVAL and "null context" in err


def test_valid_call_without_context_fails_cleanly():
    rc, err = bad_gemm()
    assert rc == _lib.DH_EINVAL and "null context" in err


def test_rmsnorm_contract():
    lib = _lib.load()
    rc = lib.dh_rmsnorm_rows(None, None, 16, 16, 16, 16, 4, 2600, 2560, 2560, 1, 1e-6)
    assert rc == _lib.DH_EINVAL and "exceeds a row stride" in _lib.last_error()


def test_final_head_contract():
    lib = _lib.load()
    rc = lib.dh_final_head(None, None, 16, 16, 16, 16, 16, 16, 3, 2561, 62, 1e-6)
    assert rc == _lib.DH_EINVAL and "multiple of 8" in _lib.last_error()
    rc = lib.dh_final_head(None, None, 16, 16, 16, 16, 16, 16, 3, 2560, 0, 1e-6)
    assert rc == _lib.DH_EINVAL and "max_cand" in _lib.last_error()
    rc = lib.dh_final_head(None, None, 16, 16, 16, 16, 16, 16, 3, 2560, 524281, 1e-6)
    assert rc == _lib.DH_EINVAL and "max_cand" in _lib.last_error()


def test_grouped_member_errors_name_the_member():
    lib = _lib.load()
    arr = (_lib.DhGemmMember * 2)()
    arr[0] = _lib.DhGemmMember(16, 16, 64, 64, 64, 0)
    arr[1] = _lib.DhGemmMember(16, 16, 64, 64, 48, 0)
    rc = lib.dh_gemm_nt_grouped(None, None, 16, 64, 4, 64, arr, 2)
    assert rc == _lib.DH_EINVAL and _lib.last_error().startswith("member 1:")
    rc = lib.dh_gemm_nt_grouped(None, None, 16, 64, 4, 64, arr, 9)
    assert rc == _lib.DH_EINVAL and "count" in _lib.last_error()


def test_variant_menu_geometry():
    vs = variants()
    assert len(vs) >= 8
    for v in vs:
        assert v["bm"] % 16 == 0 and v["bn"] % 32 == 0  # a tile holds whole gate|up pairs (2 x 16 columns)
        # 4 waves, or 8 (two per SIMD, each 2 x 2 position's block split between them)
        assert v["wave_cols"] % 16 == 0 and v["waves"] in (4, 8)
        assert v["bn"] % v["wave_cols"] == 0 and v["bm"] % 16 == 0


@pytest.mark.parametrize("m", [1, 8, 16, 163, 276, 300, 493, 512, 603, 2307])
@pytest.mark.parametrize("kn", [(2560, 12352), (2560, 10240), (2560, 18432), (4096, 2560), (9216, 2560),
                                (2560, 2048), (2560, 8192), (2560, 6144), (2560, 9216)])
def test_planner_covers_engine_shapes(m, kn):
    """Like decide's plan-covers-every-engine-shape test (gemm_configs.rs:385-400), with this build's M set."""
    k, n = kn
    for epi in Epilogue:
        p = plan_for(m, n, k, epi)
        if p["variant"] == _lib.DH_GEMM_STREAM_VARIANT:  # the weight-streaming kernel: M <= 16 only
            assert m <= 16 and n <= 4096 and k % 128 == 0 and p["bm"] == 16 and p["bn"] == 32 and p["waves"] == 4
        else:
            v = variants()[p["variant"]]
            assert p["bm"] == v["bm"] and p["bn"] == v["bn"]
        assert 1 <= p["splits"] <= 8
        # the grid covers the output exactly once per split
        assert p["workgroups"] == -(-m // p["bm"]) * -(-n // p["bn"]) * p["splits"]
        assert (p["ws_bytes"] == 0) == (p["splits"] == 1)
        assert p["ws_bytes"] <= 512 << 20


def test_planner_invariants_on_random_shapes():
    """Any legal shape gets a plan whose grid covers the output once per split, with no empty split
    (splits <= the 64-wide K stages, or the 128-wide ones of the weight-streaming kernel), a workspace
    of exactly splits x M x N fp32 partials when split, and the workspace cap respected."""
    rng = np.random.default_rng(7)
    vs = variants()
    for _ in range(400):
        m = int(rng.choice([rng.integers(1, 17), rng.integers(17, 700), rng.integers(700, 4097)]))
        n = 32 * int(rng.integers(1, 1025))
        k = 32 * int(rng.integers(1, 513))
        epi = Epilogue(int(rng.integers(0, 4)))
        p = plan_for(m, n, k, epi)
        name = f"m{m} n{n} k{k} {epi.name}: {p}"
        if p["variant"] == _lib.DH_GEMM_STREAM_VARIANT:
            assert m <= 16 and k % 128 == 0 and p["bm"] == 16 and p["bn"] == 32, name
            assert p["splits"] <= k // 128, name
        else:
            v = vs[p["variant"]]
            assert p["bm"] == v["bm"] and p["bn"] == v["bn"] and p["waves"] == v["waves"], name
            assert p["splits"] <= -(-k // 64), name
        assert p["splits"] >= 1, name
        assert p["workgroups"] == -(-m // p["bm"]) * -(-n // p["bn"]) * p["splits"], name
        assert p["ws_bytes"] == (p["splits"] * m * n * 4 if p["splits"] > 1 else 0), name
        assert p["ws_bytes"] <= 512 << 20, name
        # the work order: M tiles fastest, or column stripes in groups narrower than the stripe count
        assert p["order"] in (0, 1, 2, 3, 4, 6, 8), name
        assert p["order"] == 0 or p["order"] < -(-n // p["bn"]), name
        if p["variant"] == _lib.DH_GEMM_STREAM_VARIANT:
            assert p["order"] == 0, name


def test_tile_order_gives_each_xcd_a_compact_block():
    """The 8 XCDs each take a contiguous run of work ids. At M = 2,307 the down and out projections make
    15 x 16 tiles of 160 x 160 (30 per XCD): in M-fastest order each XCD's run covers all 15 row blocks of X
    and 2 column stripes of W (17 tile loads per XCD), in groups of 6 stripes 5 row blocks x 6 stripes (11; on the
    two XCDs that share the last group, of 4 stripes, 8 row blocks x 4 stripes: 12).
    At M = 603 the 4 row blocks per stripe already make compact runs, and the order stays M-fastest."""
    assert plan_for(2307, 2560, 9216, Epilogue.AddF32)["order"] == 6
    assert plan_for(2307, 2560, 4096, Epilogue.AddF32)["order"] == 6
    for n, k in ((18432, 2560), (12352, 2560), (2560, 9216)):
        assert plan_for(603, n, k, Epilogue.StoreF32)["order"] == 0, (n, k)


@pytest.mark.parametrize("m", [1, 4, 603, 2307])
def test_planner_handles_empty_n_and_k(m):
    """decide's contract admits N = 0 and K = 0 (gemm.rs:140-144): N = 0 plans no workgroup at all, K = 0
    one split of no stages whose tiles store the empty sum (zeros, or the residual unchanged)."""
    for epi in Epilogue:
        p = plan_for(m, 0, 128, epi)
        assert p["workgroups"] == 0 and p["ws_bytes"] == 0, p
        p = plan_for(m, 64, 0, epi)
        assert p["splits"] == 1 and p["ws_bytes"] == 0 and p["workgroups"] == -(-m // p["bm"]), p
    rc, err = bad_gemm(n=0)
    assert rc == _lib.DH_EINVAL and "null context" in err  # the contract itself accepts N = 0

def test_layout_functions_match_oracle():
    import oracle_lib as orc

    lib = _lib.load()
    rng = np.random.default_rng(1)
    gate = rng.integers(0, 65536, (64, 40)).astype(np.uint16)
    up = rng.integers(0, 65536, (64, 40)).astype(np.uint16)
    out = np.empty((128, 40), dtype=np.uint16)
    assert lib.dh_interleave_gate_up(gate.ctypes.data, up.ctypes.data, out.ctypes.data, 64, 40, 16) == 0
    assert np.array_equal(out, orc.interleave_gate_up(gate, up, 16))
    src = rng.integers(0, 65536, (4 * 2 * 8, 24)).astype(np.uint16)
    out = np.empty_like(src)
    assert lib.dh_deinterleave_q_gate(src.ctypes.data, out.ctypes.data, 4, 8, 24) == 0
    assert np.array_equal(out, orc.deinterleave_q_gate(src, 4, 8))
    assert lib.dh_interleave_gate_up(gate.ctypes.data, up.ctypes.data, out.ctypes.data, 60, 40, 16) != 0


def test_bf16_to_f16_rne_and_overflow_gate():
    lib = _lib.load()
    # every bf16 bit pattern that is finite and fits fp16: compare with numpy's IEEE RNE
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f32 = (bits.astype(np.uint32) << 16).view(np.float32)
    ok = np.isfinite(f32) & (np.abs(f32) < 65504)
    src = bits[ok]
    out = np.empty_like(src)
    counts = (ctypes.c_uint64 * 4)()
    assert lib.dh_bf16_to_f16(src.ctypes.data, out.ctypes.data, src.size, counts) == 0
    assert np.array_equal(out, f32[ok].astype(np.float16).view(np.uint16))
    assert counts[0] == src.size and counts[3] == 0
    assert counts[2] > 0 and counts[1] > 0  # tiny values flush / become subnormal
    # an overflowing value aborts (decide's convert refuses it, convert.rs:168-173)
    big = np.array([0x4780], dtype=np.uint16)  # 65536.0
    o = np.empty_like(big)
    assert lib.dh_bf16_to_f16(big.ctypes.data, o.ctypes.data, 1, counts) == _lib.DH_EINVAL
    assert counts[3] == 1


def _split_args(text):
    """Top-level comma-separated arguments of one parameter list."""
    args, depth, cur = [], 0, ""
    for ch in text:
        if ch in "([<":
            depth += 1
        elif ch in ")]>":
            depth -= 1
        if ch == "," and depth == 0:
            args.append(cur)
            cur = ""
        else:
            cur += ch
    if cur.strip():
        args.append(cur)
    return [a.strip() for a in args if a.strip() and a.strip() != "void"]


def header_prototypes():
    """{name: argument count} of every function include/decide_hip.h declares."""
    with open(os.path.join(ROOT, "include", "decide_hip.h")) as f:
        text = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
    protos = {}
    for m in re.finditer(r"\b(dh_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        protos[m.group(1)] = len(_split_args(m.group(2)))
    return protos


def rust_prototypes():
    """{name: argument count} of the `extern "C"` block INTEGRATION.md shows for the decide-hip crate."""
    with open(os.path.join(ROOT, "INTEGRATION.md")) as f:
        text = f.read()
    start = text.index('extern "C" {')
    body = text[start:text.index("\n}\n", start)]
    protos = {}
    for m in re.finditer(r"pub fn (dh_[a-z0-9_]+)\s*\((.*?)\)\s*(->[^;]*)?;", body, flags=re.S):
        assert m.group(1) not in protos, f"{m.group(1)} is bound twice"
        protos[m.group(1)] = len(_split_args(m.group(2)))
    return protos


def test_rust_binding_matches_the_header():
    header, rust = header_prototypes(), rust_prototypes()
    assert sorted(header) == declared_symbols()
    assert sorted(rust) == sorted(header), (sorted(set(header) - set(rust)), sorted(set(rust) - set(header)))
    for name, n in header.items():
        assert rust[name] == n, f"{name}: {rust[name]} arguments in the Rust binding, {n} in the header"


@pytest.mark.parametrize("kn", [(9216, 2560), (4096, 2560), (2560, 18432)])
def test_workspace_need_covers_every_m(kn):
    """dh_gemm_ws_need (what dh_warm_up holds) is the maximum of every plan's workspace for M in 1..max_m:
    the planner's table switches split counts between measured rows, so the need is not monotone in M."""
    k, n = kn
    lib = _lib.load()
    max_m = 1200
    need = ctypes.c_uint64()
    _lib.check(lib.dh_gemm_ws_need(None, max_m, n, k, ctypes.byref(need)))
    brute = 0
    for m in range(1, max_m + 1):
        for epi in range(4):
            brute = max(brute, plan_for(m, n, k, Epilogue(epi))["ws_bytes"])
    assert need.value == brute
    # the point of the sweep: a larger M can need less than a smaller one
    if kn == (9216, 2560):
        assert plan_for(1146, n, k, Epilogue.AddF32)["ws_bytes"] > plan_for(2307, n, k, Epilogue.AddF32)["ws_bytes"]


def test_workspace_need_refuses_an_unbounded_sweep():
    """dh_gemm_ws_need runs the planner once per M, so max_m is capped (DH_PLAN_MAX_ROWS = 65,536): beyond it the
    call is refused at once instead of spending hours of host time."""
    lib = _lib.load()
    need = ctypes.c_uint64(7)
    assert lib.dh_gemm_ws_need(None, 0xFFFFFFFF, 2560, 9216, ctypes.byref(need)) == _lib.DH_EINVAL
    assert "DH_PLAN_MAX_ROWS" in _lib.last_error()
    assert lib.dh_gemm_ws_need(None, 65537, 2560, 9216, ctypes.byref(need)) == _lib.DH_EINVAL
    assert need.value == 7  # untouched
    assert lib.dh_warm_up(None, None, 65537) == _lib.DH_EINVAL  # null context is reported first, without a device
