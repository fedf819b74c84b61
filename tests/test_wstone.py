"""The .wstone container on the CPU: the writer (whetstone_amd/wstone.py) and
the C++ reader/validator (wse_wstone_check, wse_wstone_config).

The reference's own container tests are restated (format.rs:573-720: round
trip, extras and old headers, alignment, foreign/corrupt files, truncation,
header overflow, single-bit flips), plus checks that pin the header bytes to
serde_json's compact serialisation of the reference's Header struct and the
embedded-config rules of config.rs:26-262."""
import json
import math

import numpy as np
import pytest

from whetstone_amd import engine, ffi, wstone

pytestmark = []


def small_config(**kw):
    c = {"hidden_size": 64, "num_hidden_layers": 1, "num_attention_heads": 2,
         "num_key_value_heads": 1, "intermediate_size": 64, "vocab_size": 128,
         "rms_norm_eps": 1e-6, "rope_theta": 1000000.0, "tie_word_embeddings": True,
         "model_type": "qwen2"}
    c.update(kw)
    return c


def packed(rng, out_f, in_f):
    return (rng.integers(0, 2**32, out_f * in_f // 8, dtype=np.uint32),
            rng.integers(0, 256, out_f * in_f // 32, dtype=np.uint8),
            rng.integers(0, 2**32, out_f, dtype=np.uint32))


def write_file(path, cfg=None, reserve=8192, extras=None):
    rng = np.random.default_rng(0)
    w = wstone.Writer(path, cfg or small_config(), reserve)
    w.set_quant_meta("scheme", "int4-hier-g32")
    qw, si, sb = packed(rng, 8, 64)
    w.write_int4_hier("gate", qw, si, sb, 8, 64)
    w.write_fp16("norm", np.full(64, 0x3C00, np.uint16), [64])
    for k, v in (extras or {}).items():
        w.write_extra(k, v)
    js = w.finish()
    return (qw, si, sb), js


def header_of(path):
    b = open(path, "rb").read()
    n = int.from_bytes(b[16:24], "little")
    return b, json.loads(b[32:32 + n])


# ------------------------------------------------------------------ hashing


def test_hash_is_fnv1a_shape_with_the_reference_multiplier():
    # format.rs:225-232: FNV-1a's offset basis and xor-multiply, multiplier
    # 0x1000000001B3. The published FNV-1a 64 of "a" is 0xaf63dc4c8601ec8c; the
    # container's must differ from it (one more hex digit in the multiplier).
    assert wstone.fnv1a(b"") == 0xcbf29ce484222325
    basis, mult = 0xcbf29ce484222325, 0x1000000001B3
    assert wstone.fnv1a(b"a") == ((basis ^ 0x61) * mult) % 2**64
    assert wstone.fnv1a(b"a") != 0xaf63dc4c8601ec8c
    h = basis
    for byte in b"the quick brown fox":
        h = ((h ^ byte) * mult) % 2**64
    assert wstone.fnv1a(b"the quick brown fox") == h


def test_fnv_detects_single_bit_flips():
    a = bytearray(b"the quick brown fox")
    ref = wstone.fnv1a(bytes(a))
    for i in range(len(a)):
        for bit in range(8):
            b = bytearray(a)
            b[i] ^= 1 << bit
            assert wstone.fnv1a(bytes(b)) != ref


# ------------------------------------------------------------- serde output


@pytest.mark.parametrize("x,want", [
    (1e-6, "1e-6"), (1e-5, "0.00001"), (1000000.0, "1000000.0"), (0.02, "0.02"),
    (1e16, "1e16"), (1e15, "1000000000000000.0"), (1.5e-7, "1.5e-7"), (-0.0, "-0.0"),
    (0.0, "0.0"), (123.456, "123.456"), (1.2345678901234568e17, "1.2345678901234568e17"),
    (5e-324, "5e-324"), (10000.0, "10000.0"), (0.1, "0.1"), (-2.5, "-2.5"),
    (1.7976931348623157e308, "1.7976931348623157e308")])
def test_floats_use_ryu_layout(x, want):
    # ryu's pretty format (serde_json's float writer): plain decimal while the
    # decimal point is within 16 digits (".0" for integers), "0.000ddd" down to
    # 1e-5, scientific beyond, exponent without "+" or padding.
    assert wstone.ryu(x) == want


def test_strings_escape_as_serde_json():
    assert wstone.json_str('a"b\\c') == '"a\\"b\\\\c"'
    assert wstone.json_str("\n\t\r\b\f\x01\x1f") == '"\\n\\t\\r\\b\\f\\u0001\\u001f"'
    assert wstone.json_str("é/€") == '"é/€"'  # non-ASCII and '/' verbatim


def test_header_bytes_match_serde_compact_struct_order(tmp_path):
    """The exact header for a small file, from the Header/TensorEntry/Blob
    field order (format.rs:102-161), sorted maps, compact separators."""
    cfg = {"vocab_size": 128, "hidden_size": 64, "rope_theta": 1000000.0, "rms_norm_eps": 1e-06,
           "tie_word_embeddings": True, "architectures": ["Qwen2ForCausalLM"],
           "num_hidden_layers": 1, "num_attention_heads": 2, "intermediate_size": 64}
    p = tmp_path / "h.wstone"
    w = wstone.Writer(p, cfg, 4096)
    w.set_quant_meta("scheme", "int4-hier-g32")
    w.set_quant_meta("group", "32")
    w.write_fp16("z.norm", np.full(4, 0x3C00, np.uint16), [4])
    w.write_fp16("a.norm", np.zeros(2, np.uint16), [2])
    js = w.finish().decode()
    start = 4352  # align_up(32 + 4096, 256)
    hz = wstone.fnv1a(np.full(4, 0x3C00, np.uint16))
    ha = wstone.fnv1a(np.zeros(2, np.uint16))
    want = ('{"format":"wstone","version":1,"producer":"whetstone-quant 0.6.0",'
            '"model_config":{"architectures":["Qwen2ForCausalLM"],"hidden_size":64,'
            '"intermediate_size":64,"num_attention_heads":2,"num_hidden_layers":1,'
            '"rms_norm_eps":1e-6,"rope_theta":1000000.0,"tie_word_embeddings":true,'
            '"vocab_size":128},"quant":{"group":"32","scheme":"int4-hier-g32"},'
            '"tensors":[{"name":"a.norm","kind":"fp16","shape":[2],"blobs":{"data":'
            f'{{"offset":{start + 256},"len":4,"hash":{ha}}}}}}},'
            '{"name":"z.norm","kind":"fp16","shape":[4],"blobs":{"data":'
            f'{{"offset":{start},"len":8,"hash":{hz}}}}}}}],"extras":{{}}}}')
    assert js == want
    b = open(p, "rb").read()
    assert b[:8] == b"WHETSTON"
    assert int.from_bytes(b[8:12], "little") == 1 and int.from_bytes(b[12:16], "little") == 0
    assert int.from_bytes(b[16:24], "little") == len(js)
    assert int.from_bytes(b[24:32], "little") == wstone.fnv1a(js.encode())
    assert b[32 + len(js):start] == b"\0" * (start - 32 - len(js))
    assert len(b) == start + 256 + 4  # no padding after the last blob


# ------------------------------------------- format.rs tests, restated


def test_round_trips_through_a_file(tmp_path):
    p = tmp_path / "m.wstone"
    (qw, si, sb), _ = write_file(p)
    assert engine.wstone_check(p, verify=True) == 2
    b, h = header_of(p)
    assert h["format"] == "wstone" and h["version"] == 1
    assert h["quant"] == {"scheme": "int4-hier-g32"}
    gate = next(t for t in h["tensors"] if t["name"] == "gate")
    assert gate["kind"] == "int4_hier_g32" and gate["shape"] == [8, 64]
    for name, arr in (("qw", qw), ("si", si), ("sb", sb)):
        e = gate["blobs"][name]
        assert b[e["offset"]:e["offset"] + e["len"]] == arr.tobytes()


def test_extras_round_trip_and_old_headers_still_load(tmp_path):
    p = tmp_path / "e.wstone"
    write_file(p, extras={"tokenizer.json": b'{"model":{}}'})
    engine.wstone_check(p, verify=True)
    b, h = header_of(p)
    e = h["extras"]["tokenizer.json"]
    assert b[e["offset"]:e["offset"] + e["len"]] == b'{"model":{}}'
    # A header written before `extras` existed (#[serde(default)]).
    js = json.dumps({"format": "wstone", "version": 1, "producer": "test",
                     "model_config": small_config(), "quant": {}, "tensors": []},
                    separators=(",", ":")).encode()
    old = (b"WHETSTON" + (1).to_bytes(4, "little") + (0).to_bytes(4, "little")
           + len(js).to_bytes(8, "little") + wstone.fnv1a(js).to_bytes(8, "little") + js)
    q = tmp_path / "old.wstone"
    q.write_bytes(old)
    assert engine.wstone_check(q) == 0


def test_payloads_are_aligned_for_vector_loads(tmp_path):
    p = tmp_path / "a.wstone"
    w = wstone.Writer(p, small_config(), 8192)
    rng = np.random.default_rng(1)
    for name in ("a", "b", "c"):
        qw, si, sb = packed(rng, 3, 32)  # odd sizes: every blob needs padding
        w.write_int4_hier(name, qw, si, sb, 3, 32)
    w.finish()
    _, h = header_of(p)
    for t in h["tensors"]:
        for blob in t["blobs"].values():
            assert blob["offset"] % 256 == 0
    engine.wstone_check(p, verify=True)


def check_refused(path, needle):
    with pytest.raises(ffi.WstError) as e:
        engine.wstone_check(path, verify=True)
    assert needle in str(e.value), str(e.value)


def test_rejects_foreign_and_corrupt_files(tmp_path):
    junk = tmp_path / "junk"
    junk.write_bytes(b"GGUF\0\0\0\0" + b"\0" * 504)
    check_refused(junk, "magic")
    short = tmp_path / "short"
    short.write_bytes(b"\0" * 8)
    check_refused(short, "too short")
    p = tmp_path / "flip.wstone"
    write_file(p)
    b = bytearray(p.read_bytes())
    b[32 + 5] ^= 0xFF
    p.write_bytes(bytes(b))
    check_refused(p, "checksum")
    v = tmp_path / "ver.wstone"
    write_file(v)
    b = bytearray(v.read_bytes())
    b[8] = 2
    v.write_bytes(bytes(b))
    check_refused(v, "version 2")


def test_truncation_is_caught_at_header_parse(tmp_path):
    p = tmp_path / "t.wstone"
    write_file(p)
    b = p.read_bytes()
    p.write_bytes(b[:-100])
    check_refused(p, "truncated")
    q = tmp_path / "t2.wstone"
    q.write_bytes(b[:100])  # shorter than the header itself
    check_refused(q, "holds")


def test_header_overflow_is_reported_not_silently_truncated(tmp_path):
    w = wstone.Writer(tmp_path / "o.wstone", small_config(), 16)
    w.write_fp16("a", np.zeros(4, np.uint16), [4])
    with pytest.raises(wstone.WstoneError, match="reserved"):
        w.finish()


def test_payload_corruption_is_caught_by_verify(tmp_path):
    p = tmp_path / "c.wstone"
    write_file(p)
    b, h = header_of(p)
    off = h["tensors"][0]["blobs"]["qw"]["offset"] if h["tensors"][0]["name"] == "gate" else \
        h["tensors"][1]["blobs"]["qw"]["offset"]
    bb = bytearray(b)
    bb[off + 3] ^= 0x10
    p.write_bytes(bytes(bb))
    assert engine.wstone_check(p, verify=False) == 2  # ranges are still valid
    check_refused(p, "checksum mismatch")


def hand_file(tmp_path, header: dict, payload_len=0, name="x.wstone"):
    js = json.dumps(header, separators=(",", ":")).encode()
    b = (b"WHETSTON" + (1).to_bytes(4, "little") + (0).to_bytes(4, "little")
         + len(js).to_bytes(8, "little") + wstone.fnv1a(js).to_bytes(8, "little") + js)
    b += b"\0" * (-len(b) % 256) + b"\0" * payload_len
    p = tmp_path / name
    p.write_bytes(b)
    return p, len(b) - payload_len


def test_hostile_ranges_and_kinds_are_refused(tmp_path):
    base = {"format": "wstone", "version": 1, "producer": "t", "model_config": small_config(),
            "quant": {}}
    blob = lambda off, n: {"offset": off, "len": n, "hash": 0}
    p, start = hand_file(tmp_path, {**base, "tensors": [
        {"name": "a", "kind": "fp16", "shape": [2], "blobs": {"data": blob(2**64 - 8, 16)}}]})
    check_refused(p, "overflows")
    p, start = hand_file(tmp_path, {**base, "tensors": [
        {"name": "a", "kind": "fp16", "shape": [2], "blobs": {"data": blob(264, 4)}}]}, 512)
    check_refused(p, "aligned")
    p, start = hand_file(tmp_path, {**base, "tensors": [
        {"name": "a", "kind": "int4_hier_g32", "shape": [1, 32],
         "blobs": {"qw": blob(256, 16), "sb": blob(512, 4)}}]}, 1024)
    check_refused(p, "requires a \"si\" blob")
    p, start = hand_file(tmp_path, {**base, "tensors": [
        {"name": "a", "kind": "int8", "shape": [1], "blobs": {"data": blob(256, 1)}}]}, 512)
    check_refused(p, "unknown kind")
    p, start = hand_file(tmp_path, {**base, "tensors": [{"name": "a", "kind": "fp16"}]})
    check_refused(p, "malformed header JSON")


# ------------------------------------------------------------ embedded config


def cfg_of(tmp_path, **kw):
    p = tmp_path / "cfg.wstone"
    write_file(p, small_config(**kw))
    return engine.wstone_config(p)


def test_config_fields_and_defaults(tmp_path):
    c = cfg_of(tmp_path)
    assert (c["hidden"], c["n_layers"], c["n_q"], c["n_kv"], c["head_dim"], c["inter"],
            c["vocab"], c["tied"]) == (64, 1, 2, 1, 32, 64, 128, 1)
    assert c["eps"] == np.float32(1e-6) and c["rope_theta"] == 1e6 and c["rope_llama3"] == 0
    # config.rs defaults: MHA without num_key_value_heads, eps 1e-6, theta 1e4,
    # untied, head_dim = hidden / heads unless given.
    d = small_config()
    for k in ("num_key_value_heads", "rms_norm_eps", "rope_theta", "tie_word_embeddings"):
        del d[k]
    d["head_dim"] = 48
    p = tmp_path / "d.wstone"
    write_file(p, d)
    c = engine.wstone_config(p)
    assert c["n_kv"] == 2 and c["eps"] == np.float32(1e-6) and c["rope_theta"] == 1e4
    assert c["tied"] == 0 and c["head_dim"] == 48
    # rope_theta is an f32 in the reference config; the table widens that f32.
    c = cfg_of(tmp_path, rope_theta=500000.3)
    assert c["rope_theta"] == float(np.float32(500000.3))


def test_config_llama3_scaling(tmp_path):
    c = cfg_of(tmp_path, model_type="llama", rope_scaling={
        "rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
        "original_max_position_embeddings": 8192})
    assert c["rope_llama3"] == 1 and c["rope_factor"] == 32.0 and c["rope_orig_max"] == 8192
    c = cfg_of(tmp_path, model_type="llama", rope_scaling={"type": "llama3"})  # older spelling
    assert c["rope_llama3"] == 1 and c["rope_factor"] == 8.0 and c["rope_high_freq"] == 4.0


@pytest.mark.parametrize("kw,needle", [
    ({"model_type": "mixtral"}, "unsupported model_type"),
    ({"model_type": "qwen2", "num_experts": 8}, "mixture-of-experts"),
    ({"hidden_act": "gelu"}, "unsupported activation"),
    ({"rope_scaling": {"rope_type": "yarn", "factor": 4.0}}, "not implemented"),
    ({"num_attention_heads": 3}, "not divisible"),
    ({"num_key_value_heads": 2, "num_attention_heads": 3, "head_dim": 16}, "multiple of"),
    ({"hidden_size": 0}, "non-zero"),
    ({"vocab_size": -1}, "vocab_size"),
    ({"vocab_size": 1.5}, "vocab_size"),
])
def test_config_refusals(tmp_path, kw, needle):
    p = tmp_path / "r.wstone"
    write_file(p, small_config(**kw))
    engine.wstone_check(p)  # the container itself is fine
    with pytest.raises(ffi.WstError) as e:
        engine.wstone_config(p)
    assert needle in str(e.value), str(e.value)
    d = small_config()
    del d["vocab_size"]
    with pytest.raises(ffi.WstError, match="missing field `vocab_size`"):
        engine.config_from_json(json.dumps(d))


def test_plan_order_matches_convert(tmp_path):
    """convert.rs:111-158: per layer the seven projections, the two norms, the
    biases and QK-norm gains that exist; then the final norm, the embedding,
    and lm_head only when untied."""
    class St:
        def __init__(self, names):
            self.n = set(names)

        def has(self, name):
            return name in self.n
    st = St(["model.layers.0.self_attn.q_proj.bias", "model.layers.1.self_attn.k_norm.weight",
             "lm_head.weight"])
    plan = wstone.build_plan({"num_hidden_layers": 2, "tie_word_embeddings": False}, st)
    names = [n for n, _ in plan]
    assert names[:7] == ["model.layers.0." + s for s in wstone.LINEAR_SUFFIXES]
    assert names[7:10] == ["model.layers.0.input_layernorm.weight",
                           "model.layers.0.post_attention_layernorm.weight",
                           "model.layers.0.self_attn.q_proj.bias"]
    assert names[10:19] == (["model.layers.1." + s for s in wstone.LINEAR_SUFFIXES]
                            + ["model.layers.1.input_layernorm.weight",
                               "model.layers.1.post_attention_layernorm.weight"])
    assert names[19:] == ["model.layers.1.self_attn.k_norm.weight", "model.norm.weight",
                          "model.embed_tokens.weight", "lm_head.weight"]
    tied = wstone.build_plan({"num_hidden_layers": 1, "tie_word_embeddings": True}, st)
    assert tied[-1][0] == "model.embed_tokens.weight"
    assert [r for _, r in plan][:7] == ["body"] * 7 and plan[-1][1] == "head"


def test_checkpoint_reader_widens_bf16_exactly(tmp_path):
    """safetensors: 8-byte header length, JSON, data; bf16 is the high half of
    an f32."""
    vals = np.array([1.0, -2.5, 3.140625, 0.0], np.float32)
    bf = (vals.view(np.uint32) >> 16).astype(np.uint16)
    f16 = np.array([0.5, 65504.0], np.float16)
    hdr = {"a": {"dtype": "BF16", "shape": [2, 2], "data_offsets": [0, 8]},
           "b": {"dtype": "F16", "shape": [2], "data_offsets": [8, 12]},
           "__metadata__": {"format": "pt"}}
    js = json.dumps(hdr).encode()
    (tmp_path / "model.safetensors").write_bytes(len(js).to_bytes(8, "little") + js
                                                 + bf.tobytes() + f16.tobytes())
    st = wstone.Checkpoint(tmp_path)
    assert st.shape("a") == [2, 2] and np.array_equal(st.f32("a"), vals)
    assert np.array_equal(st.f32("b"), f16.astype(np.float32))
