"""Safe wrappers over the C ABI -- the Python twin of the reference's
whetstone-kernels crate (crates/whetstone-kernels/src/{lib,gemv,decode,rescore}.rs).

Every wrapper validates shapes against the real buffer lengths before a call
crosses the boundary, as the Rust wrappers do, and raises ShapeError instead of
letting a kernel read out of bounds.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np

from . import ffi
from .ffi import ShapeError, call, lib

# ----------------------------------------------------------------- device


def device_count() -> int:
    n = C.c_int32()
    ffi.check(lib().wst_device_count(C.byref(n)))
    return n.value


def device_info(ordinal: int = 0) -> ffi.DeviceInfo:
    info = ffi.DeviceInfo()
    ffi.check(lib().wst_device_info(ordinal, C.byref(info)))
    return info


def synchronize() -> None:
    call("wst_device_synchronize")


def stream_sync() -> None:
    call("wst_stream_sync")


class DeviceBuffer:
    """An owned device allocation of `n` elements of `dtype`
    (kernels/src/lib.rs:235-504). Freed on close/GC."""

    def __init__(self, n: int, dtype, zero: bool = True):
        self.dtype = np.dtype(dtype)
        self.n = int(n)
        self.ptr = C.c_void_p()
        if self.nbytes:
            ffi.check(lib().wst_malloc(C.byref(self.ptr), self.nbytes))
            if zero:
                ffi.check(lib().wst_memset(self.ptr, 0, self.nbytes))

    @classmethod
    def from_array(cls, a) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.size, a.dtype, zero=False)
        if a.nbytes:
            ffi.check(lib().wst_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes))
        return b

    @property
    def nbytes(self) -> int:
        return self.n * self.dtype.itemsize

    def __len__(self) -> int:
        return self.n

    def copy_from(self, a) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        if a.size != self.n:
            raise ShapeError(f"copy_from: {a.size} elements into a buffer of {self.n}")
        if a.nbytes:
            ffi.check(lib().wst_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes))

    def numpy(self) -> np.ndarray:
        out = np.empty(self.n, self.dtype)
        if self.nbytes:
            ffi.check(lib().wst_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes))
        return out

    def at(self, offset_elems: int) -> int:
        """Raw device address of element `offset_elems` (for sub-views)."""
        if not 0 <= offset_elems <= self.n:
            raise ShapeError(f"offset {offset_elems} outside a buffer of {self.n}")
        return self.ptr.value + offset_elems * self.dtype.itemsize

    def close(self) -> None:
        if getattr(self, "ptr", None) is not None and self.ptr.value:
            lib().wst_free(self.ptr)
            self.ptr = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _need(buf: DeviceBuffer, n: int, what: str, dtype=None) -> None:
    if len(buf) != n:
        raise ShapeError(f"{what} has {len(buf)} elements, expected {n}")
    if dtype is not None and buf.dtype != np.dtype(dtype):
        raise ShapeError(f"{what} is {buf.dtype}, expected {np.dtype(dtype)}")


# ------------------------------------------------------------------- GEMV

HGROUP = 32


class QuantLinearHier:
    """An int4-hier-g32 matrix resident on the device (gemv.rs:460-600)."""

    def __init__(self, qw, si, sb, in_features: int, out_features: int):
        if in_features <= 0 or out_features <= 0 or in_features % HGROUP:
            raise ShapeError(f"in_features {in_features} must be a positive multiple of 32")
        if len(qw) != out_features * in_features // 8:
            raise ShapeError("qw length does not match the shape")
        if len(si) != out_features * in_features // HGROUP:
            raise ShapeError("si length does not match the shape")
        if len(sb) != out_features:
            raise ShapeError("sb length does not match the shape")
        conv = lambda a, t: a if isinstance(a, DeviceBuffer) else DeviceBuffer.from_array(
            np.asarray(a, t))
        self.qw, self.si, self.sb = conv(qw, np.uint32), conv(si, np.uint8), conv(sb, np.uint32)
        self.in_features, self.out_features = int(in_features), int(out_features)

    @classmethod
    def from_packed(cls, p) -> "QuantLinearHier":
        return cls(p.qw, p.si, p.sb, p.in_f, p.out_f)

    def bytes(self) -> int:
        return self.qw.nbytes + self.si.nbytes + self.sb.nbytes

    def gemv_ex(self, x: DeviceBuffer, bias: DeviceBuffer | None, y: DeviceBuffer,
                accumulate: bool = False) -> None:
        _need(x, self.in_features, "x", np.float16)
        _need(y, self.out_features, "y", np.float32)
        if bias is not None:
            _need(bias, self.out_features, "bias", np.float16)
        call("wst_gemv_int4_hier_ex", self.qw.ptr, self.si.ptr, self.sb.ptr, x.ptr,
             None if bias is None else bias.ptr, y.ptr, self.in_features, self.out_features,
             int(accumulate))

    def gemv(self, x: DeviceBuffer, y: DeviceBuffer) -> None:
        self.gemv_ex(x, None, y, False)

    def gather_row(self, row: "DeviceCursor", out: DeviceBuffer) -> None:
        _need(out, self.in_features, "gather_row output", np.float32)
        call("wst_embed_int4_hier", self.qw.ptr, self.si.ptr, self.sb.ptr, row.buf.ptr,
             out.ptr, self.in_features, self.out_features)

    def gather_rows(self, tokens: DeviceBuffer, out: DeviceBuffer, n: int) -> None:
        _need(out, n * self.in_features, "gather_rows output", np.float32)
        if len(tokens) < n:
            raise ShapeError("fewer token ids than rows requested")
        call("wst_embed_int4_hier_chunk", self.qw.ptr, self.si.ptr, self.sb.ptr, tokens.ptr,
             out.ptr, self.in_features, self.out_features, n)

    def gemm(self, x: DeviceBuffer, bias, y: DeviceBuffer, n: int, accumulate=False) -> None:
        _need(x, n * self.in_features, "x", np.float16)
        _need(y, n * self.out_features, "y", np.float32)
        call("wst_gemm_int4_hier", self.qw.ptr, self.si.ptr, self.sb.ptr, x.ptr,
             None if bias is None else bias.ptr, y.ptr, self.in_features, self.out_features, n,
             int(accumulate))


def hier_set_rule(wide: int, huge: int, other: int) -> None:
    lib().wst_gemv_hier_set_rule(wide, huge, other)


def hier_get_rule() -> list[int]:
    out = (C.c_int32 * 3)()
    lib().wst_gemv_hier_get_rule(out)
    return list(out)


def gemv_fp16(w: DeviceBuffer, x: DeviceBuffer, bias, y: DeviceBuffer, in_f: int, out_f: int,
              accumulate: bool = False) -> None:
    _need(w, in_f * out_f, "w", np.float16)
    _need(x, in_f, "x", np.float16)
    _need(y, out_f, "y", np.float32)
    call("wst_gemv_fp16_ex", w.ptr, x.ptr, None if bias is None else bias.ptr, y.ptr, in_f,
         out_f, int(accumulate))


# ---------------------------------------------------------- decode layers


def rmsnorm(x: DeviceBuffer, w: DeviceBuffer, out: DeviceBuffer, eps: float) -> None:
    """decode.rs:24-41"""
    n = len(x)
    _need(w, n, "norm weight", np.float16)
    _need(out, n, "rmsnorm output", np.float16)
    call("wst_rmsnorm", x.ptr, w.ptr, out.ptr, n, eps)


def swiglu(gate_up: DeviceBuffer, out: DeviceBuffer) -> None:
    n = len(out)
    _need(gate_up, 2 * n, "gate_up", np.float32)
    call("wst_swiglu", gate_up.ptr, out.ptr, n)


class RopeTable:
    """cos/sin [max_seq][head_dim/2] f32, built in f64 on the host
    (decode.rs:95-147, no frequency scaling)."""

    def __init__(self, max_seq: int, head_dim: int, theta: float):
        if head_dim <= 0 or head_dim % 2:
            raise ShapeError(f"rope: head_dim {head_dim} must be even")
        half = head_dim // 2
        j = np.arange(half, dtype=np.float64)
        invf = np.power(float(theta), -j / half)
        ang = np.arange(max_seq, dtype=np.float64)[:, None] * invf[None, :]
        self.cos = DeviceBuffer.from_array(np.cos(ang).astype(np.float32))
        self.sin = DeviceBuffer.from_array(np.sin(ang).astype(np.float32))
        self.max_seq, self.half_dim = max_seq, half


class KvCache:
    """[n_kv][max_seq][head_dim] f16 keys and values plus the split partials
    (decode.rs:162-212)."""

    def __init__(self, n_kv: int, n_q: int, head_dim: int, max_seq: int):
        n = n_kv * max_seq * head_dim
        self.k = DeviceBuffer(n, np.float16)
        self.v = DeviceBuffer(n, np.float16)
        floats = lib().wst_attn_partial_floats(n_q, head_dim, max_seq)
        self.partials = DeviceBuffer(max(floats, 1), np.float32)
        self.n_kv, self.head_dim, self.max_seq = n_kv, head_dim, max_seq


class DeviceCursor:
    """A device-resident i32 (decode.rs:221-256)."""

    def __init__(self, value: int = 0):
        self.buf = DeviceBuffer.from_array(np.array([value], np.int32))

    def set(self, value: int) -> None:
        self.buf.copy_from(np.array([value], np.int32))

    def get(self) -> int:
        return int(self.buf.numpy()[0])

    def advance(self, max_seq: int) -> None:
        call("wst_advance_pos", self.buf.ptr, max_seq)


def rope_cache(qkv: DeviceBuffer, cache: KvCache, table: RopeTable, n_q: int,
               pos: DeviceCursor, qk_norm=None) -> None:
    """decode.rs:305-365. qk_norm = (q_gain f16 buffer, k_gain f16 buffer, eps)."""
    hd, n_kv = cache.head_dim, cache.n_kv
    _need(qkv, (n_q + 2 * n_kv) * hd, "qkv", np.float32)
    if table.half_dim * 2 != hd or table.max_seq < cache.max_seq:
        raise ShapeError("rope table does not match the cache")
    qn = kn = None
    eps = 0.0
    if qk_norm is not None:
        qn, kn, eps = qk_norm
        _need(qn, hd, "q_norm", np.float16)
        _need(kn, hd, "k_norm", np.float16)
    call("wst_rope_cache", qkv.ptr, cache.k.ptr, cache.v.ptr, table.cos.ptr, table.sin.ptr, n_q,
         n_kv, hd, pos.buf.ptr, cache.max_seq, None if qn is None else qn.ptr,
         None if kn is None else kn.ptr, eps)


def attn_decode(q: DeviceBuffer, cache: KvCache, out: DeviceBuffer, n_q: int,
                pos: DeviceCursor, q_offset: int = 0) -> None:
    """decode.rs:368-405; q is the leading n_q*head_dim of `q` (e.g. qkv)."""
    hd = cache.head_dim
    if len(q) < q_offset + n_q * hd:
        raise ShapeError("q is shorter than n_q * head_dim")
    _need(out, n_q * hd, "attention output", np.float16)
    call("wst_attn_decode", q.at(q_offset), cache.k.ptr, cache.v.ptr, cache.partials.ptr,
         out.ptr, n_q, cache.n_kv, hd, pos.buf.ptr, cache.max_seq, 1.0 / math.sqrt(hd))


def argmax(logits: DeviceBuffer, out: DeviceBuffer) -> None:
    _need(out, 1, "argmax output", np.int32)
    call("wst_argmax", logits.ptr, out.ptr, len(logits))


def nll(logits: DeviceBuffer, target: int, acc: DeviceBuffer) -> None:
    _need(acc, 2, "nll accumulator", np.float32)
    call("wst_nll", logits.ptr, target, acc.ptr, len(logits))


# ---------------------------------------------------------------- rescore


class HeadRescore:
    """fp16 head copy + scratch for the top-k rescore (rescore.rs:75-184)."""

    def __init__(self, head_f16, vocab: int, hidden: int, k: int):
        if len(head_f16) != vocab * hidden:
            raise ShapeError(
                f"head rescore: got {len(head_f16)} elements for a [{vocab}, {hidden}] head")
        if k <= 0 or k > vocab:
            raise ShapeError(f"head rescore: k {k} must be in 1..={vocab}")
        self.cap = max(min(k * 16, vocab), k)
        self.grid = min(self.cap, 256)
        self.nblocks = min(max((vocab + 255) // 256, 1), 512)
        self.head = head_f16 if isinstance(head_f16, DeviceBuffer) else DeviceBuffer.from_array(
            np.asarray(head_f16, np.float16))
        self.thresh = DeviceBuffer(1, np.float32)
        self.scratch = DeviceBuffer(self.nblocks + 1 + 12, np.float32)
        self.count = DeviceBuffer(1, np.int32)
        self.idx = DeviceBuffer(self.cap, np.int32)
        self.k, self.hidden, self.vocab = k, hidden, vocab

    def apply(self, logits: DeviceBuffer, x: DeviceBuffer) -> None:
        _need(logits, self.vocab, "logits", np.float32)
        _need(x, self.hidden, "activation", np.float16)
        call("wst_head_threshold", logits.ptr, self.vocab, self.k, self.cap, self.scratch.ptr,
             self.nblocks, self.thresh.ptr, self.count.ptr)
        call("wst_head_compact", logits.ptr, self.vocab, self.thresh.ptr, self.count.ptr,
             self.idx.ptr, self.cap)
        call("wst_head_rescore", self.head.ptr, x.ptr, self.idx.ptr, self.count.ptr, logits.ptr,
             self.hidden, self.cap, self.grid)

    def last_count(self) -> int:
        return int(self.count.numpy()[0])

    def last_threshold(self) -> float:
        return float(self.thresh.numpy()[0])


# ------------------------------------------------------------ graphs/events


class Graph:
    """Capture of the calling thread's stream (decode.rs:558-588)."""

    def __init__(self, exec_ptr):
        self.exec = exec_ptr

    @classmethod
    def capture(cls, fn) -> "Graph":
        call("wst_graph_capture_begin")
        try:
            fn()
        finally:
            out = C.c_void_p()
            st = lib().wst_graph_capture_end(C.byref(out))
        ffi.check(st)
        return cls(out)

    def launch(self) -> None:
        call("wst_graph_launch", self.exec)

    def close(self) -> None:
        if self.exec is not None and self.exec.value:
            lib().wst_graph_destroy(self.exec)
            self.exec = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        self.h = C.c_void_p()
        call("wst_event_create", C.byref(self.h))

    def record(self) -> None:
        call("wst_event_record", self.h)

    def elapsed_ms(self, later: "Event") -> float:
        out = C.c_float()
        call("wst_event_elapsed_ms", self.h, later.h, C.byref(out))
        return out.value

    def __del__(self):
        try:
            lib().wst_event_destroy(self.h)
        except Exception:
            pass


def bench_bandwidth(nbytes: int, reps: int) -> float:
    out = C.c_double()
    call("wst_bench_bandwidth", nbytes, reps, C.byref(out))
    return out.value
