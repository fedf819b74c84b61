"""Chunk passes with per-row picks, rewind, and speculative generation
(engine.rs:731-881, speculate.rs:152-260) on the GPU.

The reference's exactness claim for speculation: the emitted stream is the
greedy stream, token for token, because a drafted token is kept only when it
equals the target's own pick at that position. These tests check it against
the engine's plain greedy generation. The claim needs the chunk pass's picks
to equal the decode step's argmax; with a rescored head the decode argmax
follows the f16 rescore and the chunk head does not (as in the reference), so
the equality tests use rescore_k = 0.
"""
import numpy as np
import pytest

from whetstone_amd import engine as E
from whetstone_amd import ffi

pytestmark = pytest.mark.gpu

TINY = dict(n_layers=2, hidden=256, n_q=4, n_kv=2, head_dim=64, inter=512, vocab=4096,
            tied=1, qkv_bias=1, qk_norm=0, rescore_k=0, eps=1e-6, rope_theta=1e6)
TINY_QK = dict(TINY, n_layers=3, hidden=512, n_q=8, n_kv=2, head_dim=128, inter=1024,
               vocab=8192, tied=0, qk_norm=1)


@pytest.fixture(scope="module", params=[TINY, TINY_QK], ids=["qwen2-tiny", "qknorm-tiny"])
def model(request):
    return E.Model(request.param, seed=1)


def _prompt(seed, n, vocab):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.int32)


def test_chunk_picks_match_per_token_decode(model):
    V = model.cfg["vocab"]
    p, x = _prompt(1, 20, V), _prompt(2, 7, V)
    a, b = E.Engine(model, 128), E.Engine(model, 128)
    a.prefill(p)
    b.prefill(p)
    a.forward_chunk(x)
    want = []
    for t in x:
        b.forward(int(t))
        want.append(b.token())
    picks = a.chunk_picks(len(x))
    assert list(picks) == want
    assert a.token() == picks[-1] and a.pos == b.pos == 27
    assert np.allclose(a.logits(), b.logits(), rtol=1e-3, atol=1e-2)
    assert list(a.chunk_picks(3)) == want[:3]


def test_rewind_then_chunk_equals_the_unrejected_history(model):
    V = model.cfg["vocab"]
    p, x1, x2 = _prompt(3, 16, V), _prompt(4, 5, V), _prompt(5, 3, V)
    a, b = E.Engine(model, 128), E.Engine(model, 128)
    a.prefill(p)
    b.prefill(p)
    a.forward_chunk(x1)
    a.rewind(16 + 2)        # keep x1[:2]; x1[2:] is overwritten by x2
    a.forward_chunk(x2)
    b.forward_chunk(x1[:2])
    b.forward_chunk(x2)
    assert a.pos == b.pos == 21
    assert np.array_equal(a.logits().view(np.uint32), b.logits().view(np.uint32))
    assert np.array_equal(a.chunk_picks(3), b.chunk_picks(3))
    a.step()                # a decode step continues from the chunk's state
    b.step()
    assert np.array_equal(a.logits().view(np.uint32), b.logits().view(np.uint32))


def test_chunk_errors(model):
    e = E.Engine(model, 64)
    with pytest.raises(ffi.WstError, match="no chunk pass"):
        e.chunk_picks(1)
    with pytest.raises(ffi.WstError, match="empty chunk"):
        e.forward_chunk(np.zeros(0, np.int32))
    w = e.chunk_width()
    with pytest.raises(ffi.WstError, match="chunk width"):
        e.forward_chunk(np.zeros(w + 1, np.int32))
    e.forward_chunk(np.array([1, 2, 3], np.int32))
    with pytest.raises(ffi.WstError, match="chunk width"):
        e.chunk_picks(w + 1)
    with pytest.raises(ffi.WstError, match="ahead of the current position"):
        e.rewind(4)
    with pytest.raises(ffi.WstError, match="exceeds the 64 token cache"):
        e.forward_chunk(np.zeros(62, np.int32))
    e.rewind(0)
    assert e.pos == 0


@pytest.mark.parametrize("graph", [False, True], ids=["eager", "graph"])
def test_speculation_emits_the_greedy_stream(model, graph):
    V = model.cfg["vocab"]
    base = _prompt(6, 5, V)
    prompt = np.concatenate([base] * 4 + [base[:3]])  # repeats for the draft
    n_new = 64
    ref = E.Engine(model, 256)
    want = ref.generate(prompt, n_new)
    e = E.Engine(model, 256)
    if graph:
        e.capture_graph()
        e.reset()
    got, st = e.speculate(prompt, n_new, E.SpecConfig(draft=4))
    assert list(got) == list(want)
    assert st.rounds > 0 and st.proposed > 0
    assert st.rounds - st.empty_rounds <= st.rounds
    # every round emits its confirmed token plus the accepted drafts
    assert st.rounds + st.accepted >= n_new - 1
    print(f"acceptance {st.acceptance():.2f}, tokens/round {st.tokens_per_round():.2f}")


def test_speculation_at_the_end_of_the_cache(model):
    V = model.cfg["vocab"]
    prompt = np.concatenate([_prompt(7, 4, V)] * 3)
    ref = E.Engine(model, 20)
    want = ref.generate(prompt, 20)  # the cache fills after 20 - 12 + 1 tokens
    e = E.Engine(model, 20)
    got, _ = e.speculate(prompt, 20, E.SpecConfig(draft=8))
    assert len(got) == 9 and list(got) == list(want[:9]) and e.pos == 20


# ------------------------------------------------ Engine::cross_entropy

def _host_nll(logits, target):
    z = np.asarray(logits, np.float64)
    m = z.max()
    return float(m + np.log(np.exp(z - m).sum()) - z[target])


def test_cross_entropy_matches_per_window_decode_and_host_log_softmax(model):
    """engine.rs:585-618: each window from an empty cache, position i predicts
    token i+1; the device sum equals the host log-softmax of the same logits."""
    V, W = model.cfg["vocab"], 9
    toks = _prompt(5, 3 * W + 4, V)  # 3 whole windows and a ragged tail
    a, b = E.Engine(model, 64), E.Engine(model, 64)
    nll, n = a.cross_entropy(toks, W)
    want = 0.0
    for w in range(3):
        b.reset()
        for i in range(W - 1):
            b.forward(int(toks[w * W + i]))
            want += _host_nll(b.logits(), int(toks[w * W + i + 1]))
    assert n == 3 * (W - 1)
    assert abs(nll - want) <= 1e-5 * abs(want) + 1e-3, (nll, want)
    # max_windows bounds the windows; one window is its own (sum, count)
    nll1, n1 = a.cross_entropy(toks, W, max_windows=1)
    assert n1 == W - 1 and 0.0 < nll1 < nll
    # random weights give near-uniform predictions: per-position NLL ~ log V
    assert abs(nll / n - np.log(V)) < 0.5


def test_cross_entropy_refusals(model):
    e = E.Engine(model, 16)
    toks = _prompt(6, 40, model.cfg["vocab"])
    for window in (0, 1, 17):
        with pytest.raises(ffi.WstError):
            e.cross_entropy(toks, window)
    bad = toks.copy()
    bad[3] = model.cfg["vocab"]
    with pytest.raises(ffi.WstError):
        e.cross_entropy(bad, 8)
    assert e.cross_entropy(toks[:5], 8) == (0.0, 0)  # no whole window


def test_cross_entropy_matches_the_oracle():
    """The device NLL against the CPU oracle's mirrored forward on the same
    seeded weights (the device packer is bit-exact with the oracle's): the
    per-position logits agree within the logit tolerance, so the summed NLL
    agrees within a few 1e-3 per position."""
    from oracle import oracle as O
    cfg = dict(TINY, n_layers=2)
    g, o = E.Model(cfg, seed=21), O.Model(cfg, 21)
    V, W = cfg["vocab"], 8
    toks = _prompt(9, 2 * W, V)
    nll, n = E.Engine(g, 32).cross_entropy(toks, W)
    want = 0.0
    for w in range(2):
        st = O.State(o, 32, 0)
        for i in range(W - 1):
            _, lg = st.step(int(toks[w * W + i]))
            want += _host_nll(lg, int(toks[w * W + i + 1]))
        st.close()
    o.close()
    assert n == 2 * (W - 1)
    assert abs(nll - want) <= 3e-3 * n, (nll, want)
