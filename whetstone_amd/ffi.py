"""ctypes binding of libwhetstone_hip.so -- the Python twin of the reference's
extern block (crates/whetstone-kernels/src/ffi.rs:134-473).

The library must be built (python -m whetstone_amd.build). There is no fallback:
if the shared object is missing, importing the product path raises.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "lib"
HIP_LIB = LIB_DIR / "libwhetstone_hip.so"
ENGINE_LIB = LIB_DIR / "libwhetstone_engine.so"

WST_OK = 0
WST_ERR_CUDA = 1
WST_ERR_INVALID_ARG = 2
WST_ERR_UNSUPPORTED_ARCH = 3
WST_ERR_OOM = 4
WST_ERR_SHAPE = 5

P = C.c_void_p
I32 = C.c_int32
I64 = C.c_int64
U64 = C.c_uint64
F32 = C.c_float
SZ = C.c_size_t


class DeviceInfo(C.Structure):
    """wst_device_info_t (whetstone.h:32-57)."""
    _fields_ = [
        ("name", C.c_char * 256), ("major", I32), ("minor", I32), ("sm_count", I32),
        ("clock_khz", I32), ("mem_clock_khz", I32), ("mem_bus_width", I32),
        ("max_threads_per_block", I32), ("max_smem_per_block", I32), ("warp_size", I32),
        ("l2_bytes", I32), ("mem_total", C.c_uint64), ("mem_free", C.c_uint64),
        ("bandwidth_gbs", C.c_double), ("has_tensor_cores", I32), ("has_imma", I32),
        ("has_bmma_xor", I32), ("has_bmma_and", I32), ("has_cp_async", I32),
        ("has_sparse_tc", I32), ("has_fp8", I32),
    ]


class ProbeResult(C.Structure):
    _fields_ = [("fp16_wmma_tflops", C.c_double), ("int8_wmma_tops", C.c_double),
                ("int4_wmma_tops", C.c_double), ("bin_bmma_tops", C.c_double),
                ("dp4a_tops", C.c_double), ("popc_tops", C.c_double),
                ("xnor_identity_ok", I32)]


class AbiLayout(C.Structure):
    _fields_ = [("device_info_size", C.c_uint32), ("device_info_align", C.c_uint32),
                ("probe_size", C.c_uint32), ("probe_align", C.c_uint32)]


# name -> (restype, argtypes). Every symbol declared in include/whetstone.h and
# include/whetstone_ext.h.
ABI = {
    "wst_last_error": (C.c_char_p, []),
    "wst_abi_layout": (None, [C.POINTER(AbiLayout)]),
    "wst_device_count": (I32, [C.POINTER(I32)]),
    "wst_device_set": (I32, [I32]),
    "wst_device_info": (I32, [I32, C.POINTER(DeviceInfo)]),
    "wst_device_synchronize": (I32, []),
    "wst_malloc": (I32, [C.POINTER(P), SZ]),
    "wst_free": (I32, [P]),
    "wst_malloc_host": (I32, [C.POINTER(P), SZ]),
    "wst_host_alloc_supported": (I32, []),
    "wst_memset": (I32, [P, I32, SZ]),
    "wst_memcpy_h2d": (I32, [P, P, SZ]),
    "wst_memcpy_d2h": (I32, [P, P, SZ]),
    "wst_memcpy_d2d": (I32, [P, P, SZ]),
    "wst_probe": (I32, [C.POINTER(ProbeResult), I32]),
    "wst_bench_bandwidth": (I32, [SZ, I32, C.POINTER(C.c_double)]),
    "wst_gemv_int4_g128": (I32, [P, P, P, P, I32, I32]),
    "wst_bench_gemv": (I32, [I32, I32, I32, I32, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    "wst_gemv_int4_g128_ex": (I32, [P, P, P, P, P, I32, I32, I32]),
    "wst_gemv_variant_count": (I32, []),
    "wst_gemv_default_variant": (I32, []),
    "wst_gemv_variant_for_shape": (I32, [I32, I32]),
    "wst_gemv_set_shape_rule": (None, [I32, I32, I32]),
    "wst_gemv_get_shape_rule": (None, [C.POINTER(I32)]),
    "wst_gemv_variant_name": (C.c_char_p, [I32]),
    "wst_gemv_int4_variant": (I32, [I32, P, P, P, P, P, I32, I32, I32]),
    "wst_bench_gemv_variant": (I32, [I32, I32, I32, I32, C.POINTER(C.c_double),
                                     C.POINTER(C.c_double)]),
    "wst_embed_int4_g128": (I32, [P, P, P, P, I32, I32]),
    "wst_embed_int4_g128_chunk": (I32, [P, P, P, P, I32, I32, I32]),
    "wst_gemv_fp16": (I32, [P, P, P, I32, I32]),
    "wst_gemv_fp16_ex": (I32, [P, P, P, P, I32, I32, I32]),
    "wst_gemv_int4_hier_ex": (I32, [P, P, P, P, P, P, I32, I32, I32]),
    "wst_gemv_hier_set_rule": (None, [I32, I32, I32]),
    "wst_gemv_hier_get_rule": (None, [C.POINTER(I32)]),
    "wst_embed_int4_hier": (I32, [P, P, P, P, P, I32, I32]),
    "wst_rmsnorm": (I32, [P, P, P, I32, F32]),
    "wst_rope_cache": (I32, [P, P, P, P, P, I32, I32, I32, P, I32, P, P, F32]),
    "wst_attn_decode": (I32, [P, P, P, P, P, I32, I32, I32, P, I32, F32]),
    "wst_attn_partial_floats": (I32, [I32, I32, I32]),
    "wst_attn_slice_positions": (I32, [I32, I32]),
    "wst_swiglu": (I32, [P, P, I32]),
    "wst_embed_fp16": (I32, [P, P, P, I32, I32]),
    "wst_graph_capture_begin": (I32, []),
    "wst_graph_capture_end": (I32, [C.POINTER(P)]),
    "wst_graph_launch": (I32, [P]),
    "wst_graph_destroy": (I32, [P]),
    "wst_stream_sync": (I32, []),
    "wst_event_create": (I32, [C.POINTER(P)]),
    "wst_event_record": (I32, [P]),
    "wst_event_elapsed_ms": (I32, [P, P, C.POINTER(F32)]),
    "wst_event_destroy": (I32, [P]),
    "wst_advance_pos": (I32, [P, I32]),
    "wst_argmax": (I32, [P, P, I32]),
    "wst_nll": (I32, [P, I32, P, I32]),
    "wst_head_threshold": (I32, [P, I32, I32, I32, P, I32, P, P]),
    "wst_head_compact": (I32, [P, I32, P, P, P, I32]),
    "wst_head_rescore": (I32, [P, P, P, P, P, I32, I32, I32]),
    "wst_moe_router": (I32, [P, I32, I32, I32, P, P]),
    "wst_moe_accumulate": (I32, [P, P, P, I32, I32]),
    "wst_chunk_max_tokens": (I32, []),
    "wst_gemm_int4_hier": (I32, [P, P, P, P, P, P, I32, I32, I32, I32]),
    "wst_gemm_int4_hier_noalloc": (I32, [P, P, P, P, P, P, I32, I32, I32, I32]),
    "wst_stream_read": (I32, [P, C.c_size_t, P]),
    "wst_gemm_fp16": (I32, [P, P, P, P, I32, I32, I32, I32]),
    "wst_rmsnorm_chunk": (I32, [P, P, P, I32, I32, F32]),
    "wst_rope_cache_chunk": (I32, [P, P, P, P, P, I32, I32, I32, I32, I32, I32, P, P, F32]),
    "wst_attn_chunk": (I32, [P, P, P, P, I32, I32, I32, I32, I32, I32, F32]),
    "wst_swiglu_chunk": (I32, [P, P, I32, I32]),
    "wst_embed_fp16_chunk": (I32, [P, P, P, I32, I32, I32]),
    "wst_embed_int4_hier_chunk": (I32, [P, P, P, P, P, I32, I32, I32]),
    "wst_argmax_chunk": (I32, [P, P, I32, I32]),
    # whetstone_ext.h
    "wst_fixture_normal_f32": (I32, [P, SZ, U64, U64, U64, F32]),
    "wst_fixture_normal_f16": (I32, [P, SZ, U64, U64, U64, F32, F32]),
    "wst_fixture_pack_hier": (I32, [P, P, P, I64, I64, I64, U64, U64, F32]),
    "wst_quantize_int4_hier": (I32, [P, P, P, P, I64, I64]),
    "wst_fixture_fill_kv": (I32, [P, P, I32, I32, I32, I32, U64, U64]),
    "wst_gemv_hier_rmsnorm": (I32, [P, P, P, P, P, F32, P, P, P, I32, I32, I32]),
    "wst_gemv_hier_rmsnorm_argmax": (I32, [P, P, P, P, P, F32, P, P, I32, I32, P, P, I32]),
    "wst_gemv_hier_swiglu": (I32, [P, P, P, P, P, F32, P, I32, I32]),
    "wst_attn_decode_fused": (I32, [P, P, P, P, P, P, P, I32, I32, I32, P, I32, F32, P, P, F32]),
    "wst_argmax_advance": (I32, [P, P, I32, P, I32]),
    "wst_head_rescore_fused": (I32, [P, P, P, I32, I32, I32, I32, P, I32]),
    "wst_gemm_hier_swiglu_chunk": (I32, [P, P, P, P, P, I32, I32, I32]),
    "wst_attn_decode_slices": (I32, [P, P, P, P, P, P, I32, I32, I32, P, I32, F32, P, P, F32]),
    "wst_hier_xq_table": (I32, [P, P, I32]),
    "wst_gemv_hier_xq": (I32, [P, P, P, P, P, P, I32, I32, I32]),
    "wst_gemv_hier_swiglu_xq": (I32, [P, P, P, P, P, F32, P, P, I32, I32]),
    "wst_attn_decode_fused_xq": (I32, [P, P, P, P, P, P, P, P, I32, I32, I32, P, I32, F32, P, P, F32]),
    "wst_gemv_hier_attn": (I32, [P, P, P, P, P, I32, I32, P, I32, I32, I32]),
    "wst_gemm_hier_norm_chunk": (I32, [P, P, P, P, P, P, I32, I32, I32, I32, P, F32, P]),
    "wst_gemm_hier_rope_chunk": (I32, [P, P, P, P, P, P, I32, P, P, P, P, I32, I32, I32, I32, I32,
                                       I32, P, P, F32]),
}


class WstError(RuntimeError):
    """A non-OK wst_status_t, with the library's thread-local message
    (the Python face of the reference's Error enum, kernels/src/lib.rs:47-98)."""

    NAMES = {1: "Cuda", 2: "InvalidArg", 3: "UnsupportedArch", 4: "Oom", 5: "Shape"}

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"{self.NAMES.get(status, status)}: {message}")


class ShapeError(ValueError):
    """Raised by the safe wrappers before any call crosses the boundary."""


_lib = None


def lib():
    """The loaded C ABI. Raises if the library was not built: there is no
    CPU fallback behind this binding."""
    global _lib
    if _lib is None:
        if not HIP_LIB.exists():
            raise FileNotFoundError(
                f"{HIP_LIB} is missing; build it with `python -m whetstone_amd.build`")
        L = C.CDLL(str(HIP_LIB))
        for name, (res, args) in ABI.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != WST_OK:
        raise WstError(status, lib().wst_last_error().decode(errors="replace"))


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
