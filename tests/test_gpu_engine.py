"""End-to-end GPU parity of the decode engine against the CPU oracle.

packed weights and argmax bit-exact; logits
within 1e-2 max-abs / 1e-3 relative, read as |got - ref| <= 1e-2 + 1e-3*|ref|
elementwise (numpy.allclose(rtol=1e-3, atol=1e-2)); greedy streams identical
over 64 steps.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from conftest import assert_streams
from whetstone_amd import engine as E

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"

TINY = dict(n_layers=2, hidden=256, n_q=4, n_kv=2, head_dim=64, inter=512, vocab=4096,
            tied=1, qkv_bias=1, qk_norm=0, rescore_k=0, eps=1e-6, rope_theta=1e6)
TINY_QK = dict(TINY, n_layers=3, hidden=512, n_q=8, n_kv=2, head_dim=128, inter=1024,
               vocab=8192, tied=0, qk_norm=1, rescore_k=16)


def _prompt(seed, n, vocab):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.int32)


@pytest.fixture(scope="module")
def tiny(orc):
    return E.Model(TINY, seed=0), orc.Model(TINY, seed=0)


def test_device_weights_equal_oracle_weights(orc, tiny):
    g, o = tiny
    names = ["embed"] + [f"L{l}.{t}" for l in range(TINY["n_layers"])
                         for t in ("qkv", "o", "gate_up", "down")]
    for name in names:
        q, s, b, i, n = g.tensor_host(name)
        p = o.tensor(name)
        assert np.array_equal(q, p.qw) and np.array_equal(s, p.si) and np.array_equal(b, p.sb), name


def test_decode_logits_match_mirrored_oracle(orc, tiny):
    g, o = tiny
    eng = E.Engine(g, 64)
    st = orc.State(o, 64, 0)
    tb = orc.State(o, 64, 1)
    for t in _prompt(1, 12, TINY["vocab"]):
        eng.forward(int(t))
        nxt, want = st.step(int(t))
        _, text = tb.step(int(t))
        got = eng.logits()
        assert np.allclose(got, want, rtol=1e-3, atol=1e-2), np.max(np.abs(got - want))
        assert np.max(np.abs(got - text)) < 5e-2  # the f64 textbook forward
        assert eng.token() == orc.argmax(got)    # argmax bit-exact on the device logits


@pytest.mark.parametrize("cfg", [TINY, TINY_QK], ids=["qwen2-tiny", "qknorm-rescore-tiny"])
def test_greedy_stream_matches_oracle_64_steps(orc, cfg):
    g, o = E.Model(cfg, seed=3), orc.Model(cfg, seed=3)
    prompt = _prompt(4, 16, cfg["vocab"])
    eng = E.Engine(g, 128)
    got = eng.generate(prompt, 64, chunked=False)
    st = orc.State(o, 128, 0)
    for t in prompt:
        nxt, lg = st.step(int(t))
    want, margins = [], []
    for _ in range(64):
        want.append(nxt)
        margins.append(orc.top2_margin(lg))
        nxt, lg = st.step(nxt)
    assert_streams(got, want, margins)


def test_fused_step_equals_reference_step_bit_for_bit(tiny):
    g, _ = tiny
    a, b = E.Engine(g, 64, E.STEP_FUSED), E.Engine(g, 64, E.STEP_REFERENCE)
    for t in _prompt(7, 10, TINY["vocab"]):
        a.forward(int(t))
        b.forward(int(t))
        assert np.array_equal(a.logits().view(np.uint32), b.logits().view(np.uint32))
        assert a.token() == b.token()


def test_fused_equals_reference_with_qknorm_and_rescore(orc):
    g = E.Model(TINY_QK, seed=1)
    a, b = E.Engine(g, 64, E.STEP_FUSED), E.Engine(g, 64, E.STEP_REFERENCE)
    for t in _prompt(8, 9, TINY_QK["vocab"]):
        a.forward(int(t))
        b.forward(int(t))
        assert np.array_equal(a.logits().view(np.uint32), b.logits().view(np.uint32))


def test_graph_replays_equal_eager_steps(tiny):
    g, _ = tiny
    prompt = _prompt(9, 6, TINY["vocab"])
    a, b = E.Engine(g, 64), E.Engine(g, 64)
    a.prefill(prompt, chunked=False)
    b.prefill(prompt, chunked=False)
    a.capture_graph()
    for _ in range(8):  # replays interleaved with host reads, each checked
        a.step()
        b.step()
        assert np.array_equal(a.logits().view(np.uint32), b.logits().view(np.uint32))
        assert a.token() == b.token() and a.pos == b.pos


def test_chunked_prefill_matches_sequential(orc, tiny):
    """engine.rs:195-199: chunked prefill gives the same greedy output as
    sequential prefill. Two chunks (256 + 44), then 32 greedy tokens from each
    engine, token for token, and both against the oracle's stream."""
    g, o = tiny
    prompt = _prompt(10, 300, TINY["vocab"])
    a, b = E.Engine(g, 512), E.Engine(g, 512)
    ta = a.generate(prompt, 32, chunked=True)
    tb = b.generate(prompt, 32, chunked=False)
    assert a.pos == b.pos == 300 + 31
    st = orc.State(o, 512, 0)
    for t in prompt:
        nxt, lg = st.step(int(t))
    want, margins = [], []
    for _ in range(32):
        want.append(nxt)
        margins.append(orc.top2_margin(lg))
        nxt, lg = st.step(nxt)
    assert_streams(ta, tb, margins)
    assert_streams(ta, want, margins)
    assert_streams(tb, want, margins)
    # the caches the two paths wrote give the same next logits within tolerance
    assert np.allclose(a.logits(), b.logits(), rtol=1e-3, atol=1e-2)


def test_generate_stops_when_the_context_is_full(tiny):
    g, _ = tiny
    eng = E.Engine(g, 24)
    got = eng.generate(_prompt(11, 16, TINY["vocab"]), 20, chunked=False)
    assert len(got) == 24 - 16 + 1   # the last token is picked at the full context
    assert eng.pos == 24
    with pytest.raises(Exception):
        eng.capture_graph()          # no room for the warm-up step


def test_synthetic_context_matches_oracle(orc, tiny):
    g, o = tiny
    eng = E.Engine(g, 300)
    eng.fill_kv(5, 200)
    st = orc.State(o, 300, 0)
    st.fill_kv(5, 200)
    st.pos = 200
    for t in (17, 400, 4095):
        eng.forward(t)
        _, want = st.step(t)
        assert np.max(np.abs(eng.logits() - want)) < 1e-2


def test_step_bytes_match_the_format_arithmetic():
    """The 0.5B algorithmic bytes per token (rows of in/2 + in/32 + 4 bytes):
    weights 264,241,152 + norms/biases 143,104 + 12,288 B per cached token."""
    g = E.Model(E.QWEN05B, seed=0)
    assert g.weight_bytes() == 264_241_152 + 143_104
    eng = E.Engine(g, 1024)
    eng.set_pos(511)
    assert eng.step_bytes() == 264_241_152 + 143_104 + 12_288 * 512


def test_qwen05b_greedy_stream_matches_golden():
    """0.5B shape (config 2's weights), seeded 16-token prompt, 64 greedy
    tokens; golden stream from the precision-mirrored CPU oracle
    (tests/golden/make_golden.py)."""
    gold = json.loads((GOLDEN / "qwen05b_greedy.json").read_text())
    g = E.Model(E.QWEN05B, seed=gold["seed"])
    eng = E.Engine(g, 256)
    got = eng.generate(np.array(gold["prompt"], np.int32), len(gold["tokens"]), chunked=False)
    assert_streams(got, gold["tokens"], gold["margins"])
