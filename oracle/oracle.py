"""ctypes view of the CPU oracle (oracle/liboracle.so). TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the checker or the timed CPU baseline. The product path never
does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")


class Config(C.Structure):
    _fields_ = [
        ("n_layers", C.c_int32), ("hidden", C.c_int32), ("n_q", C.c_int32),
        ("n_kv", C.c_int32), ("head_dim", C.c_int32), ("inter", C.c_int32),
        ("vocab", C.c_int32), ("tied", C.c_int32), ("qkv_bias", C.c_int32),
        ("qk_norm", C.c_int32), ("rescore_k", C.c_int32), ("eps", C.c_float),
        ("rope_theta", C.c_double),
    ]


def build(force: bool = False) -> Path:
    """Compiles liboracle.so with the committed Makefile."""
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "-B" if force else "liboracle.so"],
                       check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    build()
    L = C.CDLL(str(LIB_PATH))
    sig = {
        "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
        "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_f32_to_f16_n": (None, [_f32p, _u16p, C.c_size_t]),
        "orc_f16_to_f32_n": (None, [_u16p, _f32p, C.c_size_t]),
        "orc_splitmix64": (C.c_uint64, [C.c_uint64]),
        "orc_fixture_normal": (C.c_float, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float]),
        "orc_fixture_normal_n": (None, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, _f32p,
                                        C.c_size_t]),
        "orc_quantize_int4_hier": (C.c_int, [_f32p, C.c_int64, C.c_int64, _u32p, _u8p, _u32p,
                                             C.POINTER(C.c_double), C.POINTER(C.c_double)]),
        "orc_fit_group": (None, [_f32p, C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_float)]),
        "orc_shared_scale": (C.c_uint16, [C.c_float]),
        "orc_dequantize_int4_hier": (None, [_u32p, _u8p, _u32p, C.c_int64, C.c_int64, _f32p]),
        "orc_gemv_int4_hier": (None, [_u32p, _u8p, _u32p, _u16p, C.c_void_p, _f32p, C.c_int64,
                                      C.c_int64, C.c_int]),
        "orc_gemv_fp16": (None, [_u16p, _u16p, C.c_void_p, _f32p, C.c_int64, C.c_int64, C.c_int]),
        "orc_rmsnorm": (None, [_f32p, _u16p, _u16p, C.c_int, C.c_float]),
        "orc_rope_table": (None, [C.c_int, C.c_int, C.c_double, _f32p, _f32p]),
        "orc_rope_cache": (None, [_f32p, _u16p, _u16p, _f32p, _f32p, C.c_int, C.c_int, C.c_int,
                                  C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_float]),
        "orc_attn_decode": (None, [_f32p, _u16p, _u16p, _u16p, C.c_int, C.c_int, C.c_int, C.c_int,
                                   C.c_int, C.c_float]),
        "orc_swiglu": (None, [_f32p, _u16p, C.c_int]),
        "orc_argmax": (C.c_int32, [_f32p, C.c_int]),
        "orc_argmax_key": (C.c_uint64, [C.c_float, C.c_int32]),
        "orc_head_threshold": (C.c_float, [_f32p, C.c_int, C.c_int, C.c_int,
                                           C.POINTER(C.c_int32), C.POINTER(C.c_int32)]),
        "orc_head_rescore": (None, [_u16p, _u16p, _f32p, C.c_int, C.c_int, C.c_float]),
        "orc_model_synthetic": (C.c_void_p, [C.POINTER(Config), C.c_uint64]),
        "orc_model_alloc": (C.c_void_p, [C.POINTER(Config), C.c_uint64]),
        "orc_model_free": (None, [C.c_void_p]),
        "orc_model_tensor": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_void_p),
                                       C.POINTER(C.c_void_p), C.POINTER(C.c_void_p),
                                       C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
        "orc_model_fp16": (C.c_void_p, [C.c_void_p, C.c_char_p, C.POINTER(C.c_int64)]),
        "orc_model_set_dense": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p]),
        "orc_state_new": (C.c_void_p, [C.c_void_p, C.c_int, C.c_int]),
        "orc_state_free": (None, [C.c_void_p]),
        "orc_state_pos": (C.c_int, [C.c_void_p]),
        "orc_state_set_pos": (None, [C.c_void_p, C.c_int]),
        "orc_step": (C.c_int32, [C.c_void_p, C.c_int32, _f32p]),
        "orc_state_fill_kv": (None, [C.c_void_p, C.c_uint64, C.c_int]),
        "orc_forward_full": (None, [C.c_void_p, _i32p, C.c_int, _f64p]),
        "orc_threads": (C.c_int, []),
        "orc_set_variant": (None, [C.c_int, C.c_int]),
        "orc_xq14": (None, [_u16p, C.c_int64, _f64p]),
        "orc_set_ref_sms": (None, [C.c_int]),
        "orc_ref_attn_splits": (C.c_int, [C.c_int, C.c_int]),
        "orc_d2h": (C.c_uint16, [C.c_double]),
        "orc_ref_hadd": (C.c_uint16, [C.c_uint16, C.c_uint16]),
        "orc_ref_hfma": (C.c_uint16, [C.c_uint16, C.c_uint16, C.c_uint16]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data


# ----------------------------------------------------------------- helpers

def f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    out = np.empty(x.size, np.uint16)
    lib().orc_f32_to_f16_n(x, out, x.size)
    return out


def f16_value(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16).ravel()
    out = np.empty(b.size, np.float32)
    lib().orc_f16_to_f32_n(b, out, b.size)
    return out


def fixture_normal(seed: int, stream: int, n: int, std: float = 0.02, index0: int = 0):
    out = np.empty(n, np.float32)
    lib().orc_fixture_normal_n(seed, stream, index0, std, out, n)
    return out


class Packed:
    """A packed int4-hier-g32 matrix: qw [out][in/8] u32, si [out][in/32] u8, sb [out] u32."""

    def __init__(self, qw, si, sb, in_f, out_f):
        self.qw, self.si, self.sb = qw, si, sb
        self.in_f, self.out_f = int(in_f), int(out_f)

    def nbytes(self) -> int:
        return self.qw.nbytes + self.si.nbytes + self.sb.nbytes


def quantize(w: np.ndarray, in_f: int, out_f: int):
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    qw = np.zeros(out_f * in_f // 8, np.uint32)
    si = np.zeros(out_f * in_f // 32, np.uint8)
    sb = np.zeros(out_f, np.uint32)
    num, den = C.c_double(), C.c_double()
    st = lib().orc_quantize_int4_hier(w, in_f, out_f, qw, si, sb, C.byref(num), C.byref(den))
    if st != 0:
        raise ValueError(f"quantize: bad shape in={in_f} out={out_f} n={w.size}")
    rel = 0.0 if den.value == 0 else float(np.sqrt(num.value / den.value))
    return Packed(qw, si, sb, in_f, out_f), rel


def dequantize(p: Packed) -> np.ndarray:
    out = np.empty(p.in_f * p.out_f, np.float32)
    lib().orc_dequantize_int4_hier(p.qw, p.si, p.sb, p.in_f, p.out_f, out)
    return out.reshape(p.out_f, p.in_f)


def fit_group(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    s, m = C.c_float(), C.c_float()
    lib().orc_fit_group(x, x.size, C.byref(s), C.byref(m))
    return s.value, m.value


def gemv(p: Packed, x_bits, bias_bits=None, y=None, accum=False):
    y = np.zeros(p.out_f, np.float32) if y is None else np.array(y, np.float32)
    bias = None if bias_bits is None else np.ascontiguousarray(bias_bits, np.uint16)
    lib().orc_gemv_int4_hier(p.qw, p.si, p.sb, np.ascontiguousarray(x_bits, np.uint16),
                             _ptr(bias), y, p.in_f, p.out_f, int(accum))
    return y


def rmsnorm(x, w_bits, eps):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size, np.uint16)
    lib().orc_rmsnorm(x, np.ascontiguousarray(w_bits, np.uint16), out, x.size, eps)
    return out


def rope_table(max_seq, head_dim, theta):
    c = np.empty(max_seq * (head_dim // 2), np.float32)
    s = np.empty_like(c)
    lib().orc_rope_table(max_seq, head_dim, theta, c, s)
    return c, s


def argmax(logits) -> int:
    v = np.ascontiguousarray(logits, np.float32)
    return int(lib().orc_argmax(v, v.size))


def head_threshold(logits, k, cap):
    v = np.ascontiguousarray(logits, np.float32)
    cnt, rung = C.c_int32(), C.c_int32()
    t = lib().orc_head_threshold(v, v.size, k, cap, C.byref(cnt), C.byref(rung))
    return float(np.float32(t)), cnt.value, rung.value


# ------------------------------------------------------------------- model

QWEN05B = dict(n_layers=24, hidden=896, n_q=14, n_kv=2, head_dim=64, inter=4864,
               vocab=151936, tied=1, qkv_bias=1, qk_norm=0, rescore_k=0, eps=1e-6,
               rope_theta=1e6)
QWEN7B = dict(n_layers=28, hidden=3584, n_q=28, n_kv=4, head_dim=128, inter=18944,
              vocab=152064, tied=0, qkv_bias=1, qk_norm=0, rescore_k=0, eps=1e-6,
              rope_theta=1e6)
TINY = dict(n_layers=2, hidden=256, n_q=4, n_kv=2, head_dim=64, inter=512, vocab=4096,
            tied=1, qkv_bias=1, qk_norm=0, rescore_k=0, eps=1e-6, rope_theta=1e6)


def make_config(**kw) -> Config:
    return Config(**kw)


class Model:
    """A seeded synthetic model packed by the oracle's quantiser."""

    def __init__(self, cfg: dict, seed: int = 0, pack: bool = True):
        """pack=False leaves the packed matrices zero, for a caller that copies
        packed bytes in through tensor()'s (writable) views."""
        self.cfg = dict(cfg)
        self._c = make_config(**self.cfg)
        make = lib().orc_model_synthetic if pack else lib().orc_model_alloc
        self.h = make(C.byref(self._c), seed)
        self.seed = seed

    def close(self):
        if self.h:
            lib().orc_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor(self, name: str) -> Packed:
        qw, si, sb = C.c_void_p(), C.c_void_p(), C.c_void_p()
        i, o = C.c_int64(), C.c_int64()
        st = lib().orc_model_tensor(self.h, name.encode(), C.byref(qw), C.byref(si), C.byref(sb),
                                    C.byref(i), C.byref(o))
        if st != 0:
            raise KeyError(name)
        i, o = i.value, o.value
        a = lambda p, n, t: np.ctypeslib.as_array(C.cast(p, C.POINTER(t)), (n,))
        return Packed(a(qw, o * i // 8, C.c_uint32), a(si, o * i // 32, C.c_uint8),
                      a(sb, o, C.c_uint32), i, o)

    def fp16(self, name: str):
        n = C.c_int64()
        p = lib().orc_model_fp16(self.h, name.encode(), C.byref(n))
        if not p or n.value == 0:
            return None
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), (n.value,))

    def set_dense(self, which: str, table_bits) -> None:
        """Dense f16 [vocab][hidden] embedding ("embed") or head ("head")."""
        t = np.ascontiguousarray(table_bits, np.uint16)
        if t.size != self.cfg["vocab"] * self.cfg["hidden"]:
            raise ValueError("table must be [vocab][hidden]")
        if lib().orc_model_set_dense(self.h, which.encode(), t.ctypes.data) != 0:
            raise KeyError(which)

    def forward_full(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.int32)
        out = np.empty(self.cfg["vocab"], np.float64)
        lib().orc_forward_full(self.h, ids, ids.size, out)
        return out


class State:
    """Incremental decode state. mode 0 = precision-mirrored, 1 = textbook f64."""

    def __init__(self, model: Model, max_seq: int, mode: int = 0):
        self.model = model
        self.h = lib().orc_state_new(model.h, max_seq, mode)

    def close(self):
        if self.h:
            lib().orc_state_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def pos(self) -> int:
        return lib().orc_state_pos(self.h)

    @pos.setter
    def pos(self, p: int):
        lib().orc_state_set_pos(self.h, p)

    def fill_kv(self, seed: int, n: int):
        lib().orc_state_fill_kv(self.h, seed, n)

    def step(self, token: int):
        logits = np.empty(self.model.cfg["vocab"], np.float32)
        nxt = lib().orc_step(self.h, token, logits)
        return int(nxt), logits


ACC_F64, ACC_F32_SEQ, ACC_F32_LANE, ACC_REF = 0, 1, 2, 3


class variant:
    """Context manager for the oracle's arithmetic variants (process-wide):
    `acc` picks how reductions are summed (ACC_F64 default, or f32 in
    ascending order / as 64 lane partials and a tree, or ACC_REF: the
    reference CUDA kernels' own f16 group sums and reduction orders), `xq` rounds int4-GEMV
    activations to the GPU activation table's 14-bit per-group fixed point."""

    def __init__(self, acc: int = ACC_F64, xq: bool = False):
        self.acc, self.xq = int(acc), int(bool(xq))

    def __enter__(self):
        lib().orc_set_variant(self.acc, self.xq)
        return self

    def __exit__(self, *exc):
        lib().orc_set_variant(ACC_F64, 0)
        return False


def xq14(x_bits) -> np.ndarray:
    """The activation table's value of each f16 activation (float64)."""
    b = np.ascontiguousarray(x_bits, np.uint16)
    out = np.empty(b.size, np.float64)
    lib().orc_xq14(b, b.size, out)
    return out


def top2_margin(logits) -> float:
    v = np.sort(np.asarray(logits, np.float64))
    return float(v[-1] - v[-2])


if __name__ == "__main__":  # pragma: no cover
    build(force=True)
    print("oracle threads:", lib().orc_threads(), os.cpu_count())
