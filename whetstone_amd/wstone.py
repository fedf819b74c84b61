"""The `.wstone` converted-model container: writer, and the convert tool.

reference: crates/whetstone-quant/src/format.rs (Writer, 236-419; layout and
header, 1-223), crates/whetstone-cli/src/convert.rs (build_plan 111-158, run
160-398, pack_one/write_fp16 423-483), docs/FORMAT.md.

Files written here are byte-for-byte what the reference writer produces from
the same tensors:

* a 32-byte prefix (magic "WHETSTON", version 1, flags 0, header length,
  header hash), the JSON header, zero padding to the first payload, then each
  blob at the next 256-byte boundary in the order written;
* the header is serde_json's compact serialisation of the reference's Header
  struct: its fields in declaration order, maps (quant, blobs, extras and the
  embedded model_config) with sorted keys, integers verbatim and floats in
  ryu's shortest form and layout;
* tensor entries sorted by name; blob hashes and the header hash are the
  container's FNV-1a-shaped hash (multiplier 0x1000000001B3).

The reader and loader are C++ (libwhetstone_engine.so: wse_wstone_check,
wse_model_load_wstone); hashing goes through the same library.

`convert` quantises on the GPU with the device packer (wst_quantize_int4_hier),
which reproduces the reference quantiser's bytes. There is no CPU quantiser in
the product: without the HIP library, convert raises.
"""
from __future__ import annotations

import ctypes as C
import json
import math
import os
from pathlib import Path

import numpy as np

MAGIC = b"WHETSTON"
VERSION = 1
ALIGN = 256
PREFIX = 32
RESCORE_SUFFIX = ".rescore"
PRODUCER = "whetstone-quant 0.6.0"  # concat!("whetstone-quant ", CARGO_PKG_VERSION), Cargo.toml:11
HGROUP = 32


class WstoneError(RuntimeError):
    pass


def fnv1a(data) -> int:
    """The container hash of a bytes-like object or a contiguous numpy array."""
    from . import engine
    a = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray))
                             else data)
    return int(engine.lib().wse_fnv1a(C.c_void_p(a.ctypes.data), a.nbytes))


# ------------------------------------------------------------ serde_json compact


class Struct(list):
    """A JSON object serialised in the given field order (a Rust struct);
    plain dicts are maps and serialise with sorted keys (serde_json's Map is a
    BTreeMap without the preserve_order feature)."""


def ryu(x: float) -> str:
    """f64 formatted as serde_json does (ryu's shortest digits, its layout)."""
    if x == 0.0:
        return "-0.0" if math.copysign(1.0, x) < 0 else "0.0"
    if not math.isfinite(x):
        return "null"  # serde_json writes non-finite floats as null
    sign = "-" if x < 0 else ""
    r = repr(abs(x))  # Python's repr is also the shortest round-trip digit string
    mant, _, exp = r.partition("e")
    e10 = int(exp) if exp else 0
    ip, _, fp = mant.partition(".")
    if fp == "0":
        fp = ""
    digits = (ip + fp).lstrip("0")
    k = e10 - len(fp)  # value = int(digits_with_zeros) * 10^k
    stripped = digits.rstrip("0")
    k += len(digits) - len(stripped)
    d = stripped
    n = len(d)
    kk = n + k  # position of the decimal point relative to the digits
    if 0 <= k and kk <= 16:
        out = d + "0" * k + ".0"
    elif 0 < kk <= 16:
        out = d[:kk] + "." + d[kk:]
    elif -5 < kk <= 0:
        out = "0." + "0" * (-kk) + d
    elif n == 1:
        out = d + "e" + str(kk - 1)
    else:
        out = d[0] + "." + d[1:] + "e" + str(kk - 1)
    return sign + out


def json_str(s: str) -> str:
    out = ['"']
    for ch in s:
        o = ord(ch)
        if ch == '"':
            out.append('\\"')
        elif ch == "\\":
            out.append("\\\\")
        elif o < 0x20:
            out.append({8: "\\b", 9: "\\t", 10: "\\n", 12: "\\f", 13: "\\r"}.get(o, "\\u%04x" % o))
        else:
            out.append(ch)
    out.append('"')
    return "".join(out)


def to_json(v) -> str:
    if v is None:
        return "null"
    if v is True:
        return "true"
    if v is False:
        return "false"
    if isinstance(v, int):
        return str(v)
    if isinstance(v, float):
        return ryu(v)
    if isinstance(v, str):
        return json_str(v)
    if isinstance(v, Struct):
        return "{" + ",".join(json_str(k) + ":" + to_json(x) for k, x in v) + "}"
    if isinstance(v, dict):
        return "{" + ",".join(json_str(k) + ":" + to_json(v[k]) for k in sorted(v)) + "}"
    if isinstance(v, (list, tuple)):
        return "[" + ",".join(to_json(x) for x in v) + "]"
    raise TypeError(f"cannot serialise {type(v).__name__}")


# ------------------------------------------------------------------- writer


def _align_up(n: int, a: int) -> int:
    return -(-n // a) * a


class Writer:
    """Streams a .wstone file (format.rs:236-419): payloads first, the header
    patched in at the end into `header_reserve` bytes set aside after the
    prefix."""

    def __init__(self, path, model_config: dict, header_reserve: int):
        self.path = Path(path)
        self.f = open(self.path, "wb")
        self.cursor = _align_up(PREFIX + header_reserve, ALIGN)
        self.f.seek(self.cursor)
        self.entries: list[tuple[str, str, list[int], dict]] = []
        self.extras: dict = {}
        self.model_config = model_config
        self.quant: dict = {}
        self.header_reserve = header_reserve

    def set_quant_meta(self, key: str, value: str) -> None:
        self.quant[key] = value

    def _blob(self, data) -> Struct:
        a = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray))
                                 else data)
        pad = _align_up(self.cursor, ALIGN) - self.cursor
        if pad:
            self.f.write(b"\0" * pad)
            self.cursor += pad
        off = self.cursor
        self.f.write(memoryview(a).cast("B"))
        self.cursor += a.nbytes
        return Struct([("offset", off), ("len", a.nbytes), ("hash", fnv1a(a))])

    def write_int4_hier(self, name: str, qw, si, sb, out_features: int, in_features: int) -> None:
        qw, si, sb = (np.ascontiguousarray(qw, np.uint32), np.ascontiguousarray(si, np.uint8),
                      np.ascontiguousarray(sb, np.uint32))
        if (qw.size != out_features * in_features // 8 or si.size != out_features * in_features // 32
                or sb.size != out_features):
            raise WstoneError(f"{name}: packed sizes do not match [{out_features}, {in_features}]")
        blobs = {"qw": self._blob(qw), "si": self._blob(si), "sb": self._blob(sb)}
        self.entries.append((name, "int4_hier_g32", [out_features, in_features], blobs))

    def write_int4(self, name: str, qw, sz, out_features: int, in_features: int) -> None:
        """An int4 group-128 tensor (the 0.3.0 kind; kept for file compatibility)."""
        blobs = {"qw": self._blob(np.ascontiguousarray(qw, np.uint32)),
                 "sz": self._blob(np.ascontiguousarray(sz, np.uint32))}
        self.entries.append((name, "int4_g128", [out_features, in_features], blobs))

    def write_fp16(self, name: str, bits, shape) -> None:
        bits = np.ascontiguousarray(bits).view(np.uint16).reshape(-1)
        expect = int(np.prod(shape)) if len(shape) else 1
        if bits.size != expect:
            raise WstoneError(f"{name}: {bits.size} elements for shape {list(shape)} "
                              f"(expected {expect})")
        self.entries.append((name, "fp16", [int(d) for d in shape], {"data": self._blob(bits)}))

    def write_extra(self, name: str, data: bytes) -> None:
        self.extras[name] = self._blob(bytes(data))

    def header(self) -> Struct:
        tensors = [Struct([("name", n), ("kind", k), ("shape", s), ("blobs", b)])
                   for n, k, s, b in sorted(self.entries, key=lambda e: e[0].encode())]
        return Struct([("format", "wstone"), ("version", VERSION), ("producer", PRODUCER),
                       ("model_config", self.model_config), ("quant", self.quant),
                       ("tensors", tensors), ("extras", self.extras)])

    def finish(self) -> bytes:
        """Writes the header; returns its JSON bytes."""
        js = to_json(self.header()).encode()
        if len(js) > self.header_reserve:
            self.f.close()
            raise WstoneError(
                f"header is {len(js)} bytes but only {self.header_reserve} were reserved; pass a "
                "larger header_reserve (tensor payloads are already written, so the directory "
                "cannot be grown in place)")
        prefix = (MAGIC + VERSION.to_bytes(4, "little") + (0).to_bytes(4, "little")
                  + len(js).to_bytes(8, "little") + fnv1a(js).to_bytes(8, "little"))
        self.f.seek(0)
        self.f.write(prefix + js)
        self.f.close()
        return js


# ------------------------------------------------------------- safetensors


_ST_DTYPES = {"F32": (np.float32, 4), "F16": (np.float16, 2), "BF16": (np.uint16, 2)}


class Checkpoint:
    """Tensors of a Hugging Face checkpoint directory (model.safetensors or a
    sharded index), read by memory map; bf16 and f16 widen to f32 exactly.
    The safetensors layout: an 8-byte little-endian header length, a JSON
    header of {name: {dtype, shape, data_offsets}}, then the data."""

    def __init__(self, model_dir):
        d = Path(model_dir)
        idx = d / "model.safetensors.index.json"
        if idx.exists():
            files = sorted(set(json.loads(idx.read_text())["weight_map"].values()))
            self.files = [d / f for f in files]
        elif (d / "model.safetensors").exists():
            self.files = [d / "model.safetensors"]
        else:
            raise WstoneError(f"no model.safetensors (or index) in {d}")
        self.entries = {}
        for f in self.files:
            with open(f, "rb") as fh:
                n = int.from_bytes(fh.read(8), "little")
                hdr = json.loads(fh.read(n))
            for name, e in hdr.items():
                if name == "__metadata__":
                    continue
                if e["dtype"] not in _ST_DTYPES:
                    raise WstoneError(f"{name}: dtype {e['dtype']} is not f32, f16 or bf16")
                self.entries[name] = (f, 8 + n, e)

    def has(self, name: str) -> bool:
        return name in self.entries

    def shape(self, name: str) -> list[int]:
        return list(self.entries[name][2]["shape"])

    def f32(self, name: str) -> np.ndarray:
        f, base, e = self.entries[name]
        dt, size = _ST_DTYPES[e["dtype"]]
        b0, b1 = e["data_offsets"]
        n = int(np.prod(e["shape"])) if e["shape"] else 1
        if b1 - b0 != n * size:
            raise WstoneError(f"{name}: data range does not match its shape")
        raw = np.memmap(f, dtype=np.uint8, mode="r", offset=base + b0, shape=(b1 - b0,))
        a = np.frombuffer(raw, dtype=dt, count=n)
        if e["dtype"] == "BF16":
            return (a.astype(np.uint32) << 16).view(np.float32)
        return a.astype(np.float32)


# ------------------------------------------------------------------ convert

LINEAR_SUFFIXES = ["self_attn.q_proj.weight", "self_attn.k_proj.weight",
                   "self_attn.v_proj.weight", "self_attn.o_proj.weight",
                   "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight"]
EMBED = "model.embed_tokens.weight"


def build_plan(cfg: dict, st: Checkpoint) -> list[tuple[str, str]]:
    """(name, role) in the order convert emits them (convert.rs:111-158)."""
    plan = []
    for layer in range(int(cfg["num_hidden_layers"])):
        p = f"model.layers.{layer}."
        plan += [(p + s, "body") for s in LINEAR_SUFFIXES]
        plan += [(p + s, "dense") for s in ("input_layernorm.weight",
                                            "post_attention_layernorm.weight")]
        for s in ("self_attn.q_proj.bias", "self_attn.k_proj.bias", "self_attn.v_proj.bias",
                  "self_attn.q_norm.weight", "self_attn.k_norm.weight"):
            if st.has(p + s):
                plan.append((p + s, "dense"))
    plan.append(("model.norm.weight", "dense"))
    plan.append((EMBED, "head"))
    if not cfg.get("tie_word_embeddings", False) and st.has("lm_head.weight"):
        plan.append(("lm_head.weight", "head"))
    return plan


def f16_bits(w32: np.ndarray) -> np.ndarray:
    """IEEE round-to-nearest-even narrowing, as the reference's narrow_f16."""
    return np.asarray(w32, np.float32).astype(np.float16).view(np.uint16)


def pack_hier_device(w32: np.ndarray, in_f: int, out_f: int):
    """The device packer (bit-exact with quantize_int4_hier): f32 [out][in] ->
    (qw, si, sb) on the host."""
    from . import ffi, kernels as wk
    w = wk.DeviceBuffer.from_array(np.ascontiguousarray(w32, np.float32).reshape(-1))
    qw = wk.DeviceBuffer(out_f * in_f // 8, np.uint32, zero=False)
    si = wk.DeviceBuffer(out_f * in_f // 32, np.uint8, zero=False)
    sb = wk.DeviceBuffer(out_f, np.uint32, zero=False)
    ffi.call("wst_quantize_int4_hier", w.ptr, qw.ptr, si.ptr, sb.ptr, in_f, out_f)
    out = qw.numpy(), si.numpy(), sb.numpy()
    for b in (w, qw, si, sb):
        b.close()
    return out


def convert(model_dir, out_path, head: str = "fp16", body: str = "int4-hier",
            head_rescore: bool = False, log=print) -> bytes:
    """A Hugging Face checkpoint directory -> .wstone (convert.rs:160-398).

    head: "fp16" (the reference's default) or "int4-hier"; body: "int4-hier" or
    "fp16"; head_rescore also stores the f16 copy of the output projection
    (`<name>.rescore`) for the top-k rescore. Returns the header JSON."""
    from . import engine
    if head not in ("fp16", "int4-hier") or body not in ("fp16", "int4-hier"):
        raise WstoneError("head and body are fp16 or int4-hier in this build")
    d = Path(model_dir)
    raw = (d / "config.json").read_text()
    engine.config_from_json(raw)  # the loader's own validation (config.rs:206-247)
    cfg = json.loads(raw)
    st = Checkpoint(d)
    plan = build_plan(cfg, st)
    w = Writer(out_path, cfg, max(1 << 20, len(plan) * 512))
    w.set_quant_meta("scheme", "int4-hier-g32" if body == "int4-hier" else "fp16")
    w.set_quant_meta("group", "32" if body == "int4-hier" else "128")
    w.set_quant_meta("method", "kqx2-weighted-ls" if body == "int4-hier" else "rtn")
    w.set_quant_meta("source", str(st.files[0]) if st.files else "")
    w.set_quant_meta("head_rescore", "fp16-topk" if head_rescore else "none")
    w.set_quant_meta("lm_head", "fp16" if head == "fp16" else "int4-hier-g32")
    tied = bool(cfg.get("tie_word_embeddings", False))
    for name, role in plan:
        w32, shape = st.f32(name), st.shape(name)
        hier = {"dense": False, "body": body == "int4-hier", "head": head == "int4-hier"}[role]
        if role == "head" and head_rescore and hier and (name != EMBED or tied):
            w.write_fp16(name + RESCORE_SUFFIX, f16_bits(w32), shape)
        if hier and len(shape) == 2 and shape[1] % HGROUP == 0:
            out_f, in_f = shape
            qw, si, sb = pack_hier_device(w32, in_f, out_f)
            w.write_int4_hier(name, qw, si, sb, out_f, in_f)
        else:
            if hier:
                log(f"  {name}: in_features {shape[-1]} not a multiple of {HGROUP}, keeping fp16")
            w.write_fp16(name, f16_bits(w32), shape)
    tok = d / "tokenizer.json"
    if tok.exists():
        w.write_extra("tokenizer.json", tok.read_bytes())
    return w.finish()


def main(argv=None) -> int:
    import argparse
    ap = argparse.ArgumentParser(description="convert a checkpoint directory to .wstone")
    ap.add_argument("model_dir")
    ap.add_argument("-o", "--out", required=True)
    ap.add_argument("--head", default="fp16", choices=("fp16", "int4-hier"))
    ap.add_argument("--body", default="int4-hier", choices=("fp16", "int4-hier"))
    ap.add_argument("--head-rescore", action="store_true")
    a = ap.parse_args(argv)
    convert(a.model_dir, a.out, a.head, a.body, a.head_rescore)
    print(f"wrote {a.out} ({os.path.getsize(a.out) / 1e6:.1f} MB)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
