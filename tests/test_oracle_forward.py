"""Pins the oracle's end-to-end forward (CPU only).

The reference's CPU forward (bench/reference_numpy.py:74-194) is a textbook
float64 Qwen2 decoder. Rather than running it, the oracle's textbook forward is
checked against an independent implementation of the same architecture --
Hugging Face transformers' Qwen2 (and Qwen3 for QK-norm) in float64 -- loaded
with the oracle's dequantised int4 weights, on the same token ids. The
incremental (KV-cache) textbook state must equal the full recompute, and the
precision-mirrored state (f16 at the kernels' narrowing points) must stay
within f16 noise of it.
"""
import numpy as np
import pytest

TINY = dict(n_layers=2, hidden=256, n_q=4, n_kv=2, head_dim=64, inter=512, vocab=4096,
            tied=1, qkv_bias=1, qk_norm=0, rescore_k=0, eps=1e-6, rope_theta=1e6)
TINY_QK = dict(TINY, n_layers=2, hidden=256, n_q=8, n_kv=2, head_dim=64, inter=384,
               vocab=2048, tied=0, qk_norm=1)


@pytest.fixture(scope="module")
def tiny(orc):
    return orc.Model(TINY, seed=21)


def _ids(n, vocab, seed=3):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.int32)


def _hf_model(orc, m, cfg):
    torch = pytest.importorskip("torch")
    transformers = pytest.importorskip("transformers")
    H, hd, nq, nkv, I = cfg["hidden"], cfg["head_dim"], cfg["n_q"], cfg["n_kv"], cfg["inter"]
    common = dict(vocab_size=cfg["vocab"], hidden_size=H, intermediate_size=I,
                  num_hidden_layers=cfg["n_layers"], num_attention_heads=nq,
                  num_key_value_heads=nkv, head_dim=hd, rms_norm_eps=cfg["eps"],
                  rope_theta=cfg["rope_theta"], max_position_embeddings=4096,
                  tie_word_embeddings=bool(cfg["tied"]), hidden_act="silu",
                  attention_dropout=0.0, torch_dtype=torch.float64)
    if cfg["qk_norm"]:
        conf = transformers.Qwen3Config(attention_bias=bool(cfg["qkv_bias"]), **common)
        model = transformers.Qwen3ForCausalLM(conf)
    else:
        conf = transformers.Qwen2Config(**common)
        model = transformers.Qwen2ForCausalLM(conf)
    model = model.to(torch.float64).eval()
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float64))
    dq = lambda name: orc.dequantize(m.tensor(name)).astype(np.float64)
    f16 = lambda name: orc.f16_value(m.fp16(name)).astype(np.float64)
    sd = {"model.embed_tokens.weight": T(dq("embed")), "model.norm.weight": T(f16("final_norm"))}
    if not cfg["tied"]:
        sd["lm_head.weight"] = T(dq("lm_head"))
    for l in range(cfg["n_layers"]):
        p = f"model.layers.{l}."
        qkv, gu = dq(f"L{l}.qkv"), dq(f"L{l}.gate_up")
        sd[p + "self_attn.q_proj.weight"] = T(qkv[:nq * hd])
        sd[p + "self_attn.k_proj.weight"] = T(qkv[nq * hd:(nq + nkv) * hd])
        sd[p + "self_attn.v_proj.weight"] = T(qkv[(nq + nkv) * hd:])
        if cfg["qkv_bias"]:
            b = f16(f"L{l}.qkv_bias")
            sd[p + "self_attn.q_proj.bias"] = T(b[:nq * hd])
            sd[p + "self_attn.k_proj.bias"] = T(b[nq * hd:(nq + nkv) * hd])
            sd[p + "self_attn.v_proj.bias"] = T(b[(nq + nkv) * hd:])
        sd[p + "self_attn.o_proj.weight"] = T(dq(f"L{l}.o"))
        if cfg["qk_norm"] and cfg["qkv_bias"]:  # Qwen3's attention_bias also biases o
            sd[p + "self_attn.o_proj.bias"] = T(np.zeros(H))
        sd[p + "mlp.gate_proj.weight"] = T(gu[:I])
        sd[p + "mlp.up_proj.weight"] = T(gu[I:])
        sd[p + "mlp.down_proj.weight"] = T(dq(f"L{l}.down"))
        sd[p + "input_layernorm.weight"] = T(f16(f"L{l}.in_norm"))
        sd[p + "post_attention_layernorm.weight"] = T(f16(f"L{l}.post_norm"))
        if cfg["qk_norm"]:
            sd[p + "self_attn.q_norm.weight"] = T(f16(f"L{l}.q_norm"))
            sd[p + "self_attn.k_norm.weight"] = T(f16(f"L{l}.k_norm"))
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected, unexpected
    assert all("rotary" in k or (cfg["tied"] and k == "lm_head.weight") for k in missing), missing
    return model


@pytest.mark.parametrize("cfg", [TINY, TINY_QK], ids=["qwen2", "qwen3-qknorm"])
def test_textbook_forward_matches_transformers_float64(orc, cfg):
    import torch
    m = orc.Model(cfg, seed=22)
    ids = _ids(9, cfg["vocab"])
    want = m.forward_full(ids)
    hf = _hf_model(orc, m, cfg)
    with torch.no_grad():
        got = hf(torch.from_numpy(ids.astype(np.int64))[None]).logits[0, -1].numpy()
    # transformers builds its RoPE frequencies in float32 (the oracle in
    # float64), which alone moves the logits by ~1e-7; a dropped term, a wrong
    # sign or a transposed operand moves them by > 1e-2.
    assert np.max(np.abs(got - want)) < 2e-6 * max(1.0, np.max(np.abs(want)))


def test_incremental_textbook_equals_full_recompute(orc, tiny):
    ids = _ids(12, TINY["vocab"], 4)
    st = orc.State(tiny, 32, 1)
    for i, t in enumerate(ids):
        _, lg = st.step(int(t))
        if i in (0, 5, 11):
            full = tiny.forward_full(ids[:i + 1])
            assert np.max(np.abs(lg - full)) < 5e-6 * max(1.0, np.max(np.abs(full)))


def test_mirrored_forward_within_f16_noise_of_textbook(orc, tiny):
    ids = _ids(16, TINY["vocab"], 5)
    a, b = orc.State(tiny, 32, 0), orc.State(tiny, 32, 1)
    for t in ids:
        _, la = a.step(int(t))
        _, lb = b.step(int(t))
        scale = np.sqrt(np.mean(lb.astype(np.float64) ** 2))
        assert np.max(np.abs(la - lb)) < 2e-3 * max(scale, 1.0)


def test_synthetic_context_is_the_seeded_kv_fill(orc, tiny):
    """fill_kv writes f16 N(0,1) from (seed, stream 1000+layer) for positions
    [0, n); decoding from it is deterministic and position-dependent."""
    a, b = orc.State(tiny, 64, 0), orc.State(tiny, 64, 0)
    a.fill_kv(5, 40)
    b.fill_kv(5, 40)
    a.pos = b.pos = 40
    _, la = a.step(7)
    _, lb = b.step(7)
    assert np.array_equal(la, lb)
    c = orc.State(tiny, 64, 0)
    c.fill_kv(6, 40)
    c.pos = 40
    _, lc = c.step(7)
    assert not np.array_equal(la, lc)


def test_golden_fixture_is_reproduced(orc):
    """tests/golden/qwen05b_greedy.json (0.5B shape, seed 0): the oracle
    regenerates the first 6 greedy tokens of the committed stream."""
    import json
    from pathlib import Path
    gold = json.loads((Path(__file__).parent / "golden" / "qwen05b_greedy.json").read_text())
    m = orc.Model(orc.QWEN05B, gold["seed"])
    st = orc.State(m, 64, 0)
    for t in gold["prompt"]:
        nxt, _ = st.step(int(t))
    got = []
    for _ in range(6):
        got.append(nxt)
        nxt, _ = st.step(nxt)
    assert got == gold["tokens"][:6]


def test_mirrored_step_with_dense_f16_tables(orc):
    """Dense f16 embedding / head (a converted model's fp16 tables): set to the
    f16 rounding of the dequantised int4 tables, the logits stay within f16
    noise of the int4 run (and differ from it: the dense tables are used)."""
    for cfg in (TINY, TINY_QK):
        m, d = orc.Model(cfg, seed=31), orc.Model(cfg, seed=31)
        emb = orc.f16_bits(orc.dequantize(m.tensor("embed")))
        d.set_dense("embed", emb)
        if not cfg["tied"]:
            d.set_dense("head", orc.f16_bits(orc.dequantize(m.tensor("lm_head"))))
        a, b = orc.State(m, 16, 0), orc.State(d, 16, 0)
        for t in _ids(6, cfg["vocab"], 9):
            _, la = a.step(int(t))
            _, lb = b.step(int(t))
            scale = np.sqrt(np.mean(la.astype(np.float64) ** 2))
            assert np.max(np.abs(la - lb)) < 3e-3 * max(scale, 1.0)
            assert np.max(np.abs(la - lb)) > 0  # the dense tables are in use
        a.close(), b.close(), m.close(), d.close()
