"""GPU tests of the .wstone loader (wse_model_load_wstone) and of convert.

* A model written to a .wstone (the synthetic model's tensors, split back into
  the checkpoint's q/k/v and gate/up projections) and loaded again runs the
  same bits as the model it was written from: the loader's row-append fusion
  is exact.
* A file with dense f16 embedding and head (the reference converter's default
  head precision) runs against the mirrored oracle with the same f16 tables,
  to the north-star logit tolerance, with identical greedy tokens.
* convert() of a safetensors checkpoint quantises on the device to exactly the
  oracle quantiser's bytes, and the loaded model decodes.
"""
import json

import numpy as np
import pytest

from whetstone_amd import engine as E
from whetstone_amd import wstone

pytestmark = pytest.mark.gpu

TINY = dict(n_layers=2, hidden=256, n_q=4, n_kv=2, head_dim=64, inter=512, vocab=4096,
            tied=0, qkv_bias=1, qk_norm=0, rescore_k=0, eps=1e-6, rope_theta=1e6)
TINY_QK = dict(TINY, n_q=8, n_kv=2, head_dim=64, tied=1, qkv_bias=0, qk_norm=1, rescore_k=16)


def hf_config(cfg):
    return {"architectures": ["Qwen3ForCausalLM" if cfg["qk_norm"] else "Qwen2ForCausalLM"],
            "model_type": "qwen3" if cfg["qk_norm"] else "qwen2",
            "hidden_size": cfg["hidden"], "num_hidden_layers": cfg["n_layers"],
            "num_attention_heads": cfg["n_q"], "num_key_value_heads": cfg["n_kv"],
            "head_dim": cfg["head_dim"], "intermediate_size": cfg["inter"],
            "vocab_size": cfg["vocab"], "rms_norm_eps": 1e-6, "rope_theta": 1000000.0,
            "tie_word_embeddings": bool(cfg["tied"]), "hidden_act": "silu"}


def write_model(g, cfg, path, dense=None):
    """Writes the device model g as a checkpoint-shaped .wstone. dense: None,
    or {"embed": bits, "head": bits} f16 tables to store instead of int4."""
    H, hd, nq, nkv, I = cfg["hidden"], cfg["head_dim"], cfg["n_q"], cfg["n_kv"], cfg["inter"]
    w = wstone.Writer(path, hf_config(cfg), 1 << 20)
    w.set_quant_meta("scheme", "int4-hier-g32")

    def hier(name, mat, rows=None):
        q, s, b, in_f, n = g.tensor_host(mat, rows)
        w.write_int4_hier(name, q, s, b, n, in_f)

    for l in range(cfg["n_layers"]):
        p = f"model.layers.{l}."
        q0, q1, q2 = nq * hd, (nq + nkv) * hd, (nq + 2 * nkv) * hd
        hier(p + "self_attn.q_proj.weight", f"L{l}.qkv", (0, q0))
        hier(p + "self_attn.k_proj.weight", f"L{l}.qkv", (q0, q1))
        hier(p + "self_attn.v_proj.weight", f"L{l}.qkv", (q1, q2))
        hier(p + "self_attn.o_proj.weight", f"L{l}.o")
        hier(p + "mlp.gate_proj.weight", f"L{l}.gate_up", (0, I))
        hier(p + "mlp.up_proj.weight", f"L{l}.gate_up", (I, 2 * I))
        hier(p + "mlp.down_proj.weight", f"L{l}.down")
        w.write_fp16(p + "input_layernorm.weight", g.vector_host(f"L{l}.in_norm"), [H])
        w.write_fp16(p + "post_attention_layernorm.weight", g.vector_host(f"L{l}.post_norm"), [H])
        if cfg["qkv_bias"]:
            b = g.vector_host(f"L{l}.qkv_bias")
            w.write_fp16(p + "self_attn.q_proj.bias", b[:q0], [q0])
            w.write_fp16(p + "self_attn.k_proj.bias", b[q0:q1], [q1 - q0])
            w.write_fp16(p + "self_attn.v_proj.bias", b[q1:], [q2 - q1])
        if cfg["qk_norm"]:
            w.write_fp16(p + "self_attn.q_norm.weight", g.vector_host(f"L{l}.q_norm"), [hd])
            w.write_fp16(p + "self_attn.k_norm.weight", g.vector_host(f"L{l}.k_norm"), [hd])
    w.write_fp16("model.norm.weight", g.vector_host("final_norm"), [H])
    V = cfg["vocab"]
    head_name = "model.embed_tokens.weight" if cfg["tied"] else "lm_head.weight"
    if cfg["rescore_k"] and not dense:
        w.write_fp16(head_name + ".rescore", g.vector_host("rescore"), [V, H])
    if dense:
        w.write_fp16("model.embed_tokens.weight", dense["embed"], [V, H])
        if not cfg["tied"]:
            w.write_fp16("lm_head.weight", dense["head"], [V, H])
    else:
        hier("model.embed_tokens.weight", "embed")
        if not cfg["tied"]:
            hier("lm_head.weight", "lm_head")
    w.finish()


@pytest.mark.parametrize("cfg", [TINY, TINY_QK], ids=["qwen2-untied-bias", "qknorm-tied-rescore"])
def test_written_then_loaded_model_runs_the_same_bits(tmp_path, cfg):
    g = E.Model(cfg, seed=4)
    p = tmp_path / "m.wstone"
    write_model(g, cfg, p)
    assert E.wstone_check(p, verify=True) > 0
    f = E.Model.load(p, rescore_k=cfg["rescore_k"] or -1)
    for k in ("n_layers", "hidden", "n_q", "n_kv", "head_dim", "inter", "vocab", "tied",
              "qkv_bias", "qk_norm", "rescore_k"):
        assert f.cfg[k] == cfg[k], k
    assert f.weight_bytes() == g.weight_bytes()
    for name in ["embed"] + [f"L{l}.{t}" for l in range(cfg["n_layers"])
                             for t in ("qkv", "o", "gate_up", "down")]:
        a, b = g.tensor_host(name), f.tensor_host(name)
        assert all(np.array_equal(x, y) for x, y in zip(a[:3], b[:3])), name
    ids = np.random.default_rng(7).integers(0, cfg["vocab"], 6).astype(np.int32)
    for mode in (E.STEP_FUSED, E.STEP_REFERENCE):
        e1, e2 = E.Engine(g, 32, mode), E.Engine(f, 32, mode)
        for t in ids:
            e1.forward(int(t))
            e2.forward(int(t))
            assert np.array_equal(e1.logits().view(np.uint32), e2.logits().view(np.uint32))
            assert e1.token() == e2.token()
        e1.close(), e2.close()
    f.close(), g.close()


@pytest.mark.parametrize("cfg", [TINY, TINY_QK], ids=["untied", "tied"])
def test_dense_f16_embedding_and_head_match_oracle(tmp_path, orc, cfg):
    cfg = dict(cfg, rescore_k=0)
    g, o = E.Model(cfg, seed=5), orc.Model(cfg, seed=5)
    emb = orc.f16_bits(orc.dequantize(o.tensor("embed")))
    head = None if cfg["tied"] else orc.f16_bits(orc.dequantize(o.tensor("lm_head")))
    p = tmp_path / "d.wstone"
    write_model(g, cfg, p, dense={"embed": emb, "head": head})
    f = E.Model.load(p)
    o.set_dense("embed", emb)
    if head is not None:
        o.set_dense("head", head)
    eng, st = E.Engine(f, 48), orc.State(o, 48, 0)
    for t in np.random.default_rng(8).integers(0, cfg["vocab"], 24).astype(np.int32):
        eng.forward(int(t))
        _, want = st.step(int(t))
        got = eng.logits()
        assert np.allclose(got, want, rtol=1e-3, atol=1e-2), np.max(np.abs(got - want))
        assert eng.token() == orc.argmax(got)
    # greedy continuation identical over 16 steps
    nxt = eng.token()
    for _ in range(16):
        eng.forward(nxt)
        want_tok, _ = st.step(nxt)
        assert eng.token() == want_tok
        nxt = want_tok
    eng.close(), st.close(), f.close(), g.close(), o.close()


def write_checkpoint(d, cfg, rng):
    """A bf16 safetensors checkpoint with a Qwen2-style config."""
    H, hd, nq, nkv, I, V = (cfg[k] for k in ("hidden", "head_dim", "n_q", "n_kv", "inter", "vocab"))
    tensors = {}
    for l in range(cfg["n_layers"]):
        p = f"model.layers.{l}."
        for name, shape in (("self_attn.q_proj.weight", (nq * hd, H)),
                            ("self_attn.k_proj.weight", (nkv * hd, H)),
                            ("self_attn.v_proj.weight", (nkv * hd, H)),
                            ("self_attn.o_proj.weight", (H, nq * hd)),
                            ("mlp.gate_proj.weight", (I, H)), ("mlp.up_proj.weight", (I, H)),
                            ("mlp.down_proj.weight", (H, I))):
            tensors[p + name] = rng.standard_normal(shape).astype(np.float32) * 0.02
        for name, n in (("self_attn.q_proj.bias", nq * hd), ("self_attn.k_proj.bias", nkv * hd),
                        ("self_attn.v_proj.bias", nkv * hd)):
            tensors[p + name] = rng.standard_normal(n).astype(np.float32) * 0.1
        tensors[p + "input_layernorm.weight"] = 1 + rng.standard_normal(H).astype(np.float32) * 0.05
        tensors[p + "post_attention_layernorm.weight"] = np.ones(H, np.float32)
    tensors["model.norm.weight"] = np.ones(H, np.float32)
    tensors["model.embed_tokens.weight"] = rng.standard_normal((V, H)).astype(np.float32) * 0.02
    tensors["lm_head.weight"] = rng.standard_normal((V, H)).astype(np.float32) * 0.02
    header, blobs, off = {}, [], 0
    for name, a in tensors.items():
        bf = (a.view(np.uint32) >> 16).astype(np.uint16)  # truncation to bf16 is exact data
        header[name] = {"dtype": "BF16", "shape": list(a.shape), "data_offsets": [off, off + bf.nbytes]}
        blobs.append(bf.tobytes())
        off += bf.nbytes
    js = json.dumps(header).encode()
    (d / "model.safetensors").write_bytes(len(js).to_bytes(8, "little") + js + b"".join(blobs))
    (d / "config.json").write_text(json.dumps(hf_config(cfg)))
    (d / "tokenizer.json").write_text('{"model":{}}')
    return {k: (v.view(np.uint32) & 0xFFFF0000).view(np.float32) for k, v in tensors.items()}


def test_convert_quantises_to_the_oracle_bytes_and_loads(tmp_path, orc):
    cfg = dict(TINY, n_layers=1, vocab=1024)
    src = tmp_path / "ckpt"
    src.mkdir()
    w32 = write_checkpoint(src, cfg, np.random.default_rng(11))
    out = tmp_path / "c.wstone"
    wstone.convert(src, out, head="int4-hier", head_rescore=True)
    assert E.wstone_check(out, verify=True) > 0
    b = out.read_bytes()
    h = json.loads(b[32:32 + int.from_bytes(b[16:24], "little")])
    assert h["quant"]["lm_head"] == "int4-hier-g32" and h["quant"]["head_rescore"] == "fp16-topk"
    assert "tokenizer.json" in h["extras"]
    ents = {t["name"]: t for t in h["tensors"]}
    blob = lambda t, k: np.frombuffer(b, np.uint8, t["blobs"][k]["len"], t["blobs"][k]["offset"])
    for name in ("model.layers.0.self_attn.q_proj.weight", "model.layers.0.mlp.down_proj.weight",
                 "lm_head.weight"):
        t = ents[name]
        out_f, in_f = t["shape"]
        p, _ = orc.quantize(w32[name].reshape(-1), in_f, out_f)
        assert np.array_equal(blob(t, "qw").view(np.uint32), p.qw), name
        assert np.array_equal(blob(t, "si"), p.si), name
        assert np.array_equal(blob(t, "sb").view(np.uint32), p.sb), name
    t = ents["model.layers.0.self_attn.q_proj.bias"]
    assert np.array_equal(blob(t, "data").view(np.uint16),
                          orc.f16_bits(w32["model.layers.0.self_attn.q_proj.bias"]))
    assert ents["lm_head.weight.rescore"]["kind"] == "fp16"
    assert ents["model.embed_tokens.weight"]["kind"] == "int4_hier_g32"
    m = E.Model.load(out)
    assert m.cfg["rescore_k"] == 64 and m.cfg["qkv_bias"] == 1
    eng = E.Engine(m, 16)
    for t in (1, 2, 3):
        eng.forward(t)
        lg = eng.logits()
        assert np.all(np.isfinite(lg)) and eng.token() == orc.argmax(lg)
    eng.close(), m.close()
