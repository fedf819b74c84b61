"""The C-ABI boundary, checked on the CPU (no GPU call is made).

* libwhetstone_hip.so exports every function include/whetstone.h and
  include/whetstone_ext.h declare; libwhetstone_engine.so every function of
  include/whetstone_engine.h.
* Argument checks run before any device work and report through the status
  code and wst_last_error (whetstone.h:3-28), as the reference's WST_REQUIRE
  does (common.cuh:15-26).
* The symbols the reference binds but this build does not implement (g128,
  variants, probes, MoE) return WST_ERR_UNSUPPORTED_ARCH with a message.
* Nothing in the product -- the two libraries and the whetstone_amd package --
  links, loads or imports the CPU oracle.
"""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
INC = ROOT / "include"
LIBDIR = ROOT / "whetstone_amd" / "lib"
HIP_LIB = LIBDIR / "libwhetstone_hip.so"
ENG_LIB = LIBDIR / "libwhetstone_engine.so"

WST_OK, WST_ERR_INVALID_ARG, WST_ERR_UNSUPPORTED_ARCH, WST_ERR_SHAPE = 0, 2, 3, 5


def declared(header: Path, prefix: str) -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return set(re.findall(rf"\b({prefix}\w+)\s*\(", text))


def exported(lib: Path) -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True,
                         text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


@pytest.fixture(scope="module")
def hip():
    if not HIP_LIB.exists():
        pytest.fail(f"{HIP_LIB} is not built (python -m whetstone_amd.build)")
    return C.CDLL(str(HIP_LIB))


def test_headers_declare_the_reference_decode_surface():
    names = declared(INC / "whetstone.h", "wst_")
    for must in ["wst_gemv_int4_hier_ex", "wst_gemv_hier_set_rule", "wst_gemv_hier_get_rule",
                 "wst_embed_int4_hier", "wst_rmsnorm", "wst_rope_cache", "wst_attn_decode",
                 "wst_attn_partial_floats", "wst_swiglu", "wst_argmax", "wst_head_threshold",
                 "wst_head_compact", "wst_head_rescore", "wst_advance_pos",
                 "wst_graph_capture_begin", "wst_graph_capture_end", "wst_graph_launch",
                 "wst_gemm_int4_hier", "wst_attn_chunk", "wst_nll", "wst_last_error"]:
        assert must in names, must


def test_every_declared_function_is_exported():
    have = exported(HIP_LIB)
    for h in ("whetstone.h", "whetstone_ext.h"):
        missing = declared(INC / h, "wst_") - have
        assert not missing, f"{h}: {sorted(missing)}"
    missing = declared(INC / "whetstone_engine.h", "wse_") - exported(ENG_LIB)
    assert not missing, sorted(missing)


def test_product_libraries_do_not_contain_or_link_the_oracle():
    for lib in (HIP_LIB, ENG_LIB):
        assert not any(s.startswith("orc_") for s in exported(lib)), lib
        ldd = subprocess.run(["ldd", str(lib)], capture_output=True, text=True).stdout
        assert "liboracle" not in ldd
    for py in (ROOT / "whetstone_amd").rglob("*.py"):
        src = py.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", src, re.M), py


def test_refusals_come_before_any_device_work(hip):
    hip.wst_last_error.restype = C.c_char_p
    f = hip.wst_gemv_int4_hier_ex
    f.restype = C.c_int
    f.argtypes = [C.c_void_p] * 6 + [C.c_int32, C.c_int32, C.c_int32]
    assert f(None, None, None, None, None, None, 896, 1152, 0) == WST_ERR_INVALID_ARG
    assert hip.wst_last_error()
    dummy = C.c_void_p(0x1000)
    st = f(dummy, dummy, dummy, dummy, None, dummy, 100, 8, 0)  # in_f not a multiple of 32
    assert st in (WST_ERR_INVALID_ARG, WST_ERR_SHAPE), st
    assert b"32" in hip.wst_last_error()

    r = hip.wst_rmsnorm
    r.restype = C.c_int
    r.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int32, C.c_float]
    assert r(None, None, None, 896, 1e-6) == WST_ERR_INVALID_ARG

    a = hip.wst_attn_decode
    a.restype = C.c_int
    a.argtypes = [C.c_void_p] * 5 + [C.c_int32] * 3 + [C.c_void_p, C.c_int32, C.c_float]
    # 14 query heads over 3 kv heads: refused
    assert a(dummy, dummy, dummy, dummy, dummy, 14, 3, 64, dummy, 128, 0.125) != WST_OK
    assert b"multiple" in hip.wst_last_error()


def test_unsupported_reference_symbols_report_unsupported(hip):
    hip.wst_last_error.restype = C.c_char_p
    stubs = sorted(n for n in declared(INC / "whetstone.h", "wst_")
                   if re.search(r"g128|variant|probe|moe", n))
    assert stubs, "expected the g128/variant/probe/MoE surface to be declared"
    g = hip.wst_gemv_int4_g128
    g.restype = C.c_int
    assert g(None, None, None, None, None, None, 0, 0, 0) == WST_ERR_UNSUPPORTED_ARCH
    assert hip.wst_last_error()


def test_python_binding_refuses_bad_shapes_before_the_boundary():
    from whetstone_amd import ffi
    from whetstone_amd.kernels import QuantLinearHier
    with pytest.raises(ffi.ShapeError):
        QuantLinearHier([0] * 12, [0] * 3, [0] * 1, 100, 1)


def test_attention_slice_length_rule(hip):
    """Positions per attention slice: 16384 / head_dim."""
    f = hip.wst_attn_slice_positions
    f.restype = C.c_int32
    f.argtypes = [C.c_int32, C.c_int32]
    cases = {(128, 1024): 128, (128, 2312): 128, (128, 40000): 128, (64, 776): 256,
             (64, 40000): 256, (256, 300): 64, (256, 5000): 64, (100, 10): 0, (128, 0): 0}
    for (hd, ms), want in cases.items():
        assert f(hd, ms) == want, (hd, ms)
