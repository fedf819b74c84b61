"""Engine::sample and generate with a sampler (engine.rs:648-673, 909-956) on
the GPU: the device logits go to the host sampler with the engine's
recent-token window, and the choice goes back to the device cursor."""
import numpy as np
import pytest

from whetstone_amd import engine as E

pytestmark = pytest.mark.gpu

TINY = dict(n_layers=2, hidden=256, n_q=4, n_kv=2, head_dim=64, inter=512, vocab=4096,
            tied=1, qkv_bias=1, qk_norm=0, rescore_k=0, eps=1e-6, rope_theta=1e6)


@pytest.fixture(scope="module")
def model():
    return E.Model(TINY, seed=3)


def _prompt(seed, n):
    return np.random.default_rng(seed).integers(0, TINY["vocab"], n).astype(np.int32)


def test_sample_uses_the_device_logits_and_the_window(model):
    e = E.Engine(model, 64)
    p = _prompt(1, 9)
    e.prefill(p)
    assert e.recent() == [int(t) for t in p]
    cfg = E.SamplingConfig(temperature=1.5, top_p=0.95, top_k=0, repeat_penalty=1.3,
                           repeat_last_n=5, seed=11)
    for step in range(6):
        window = e.recent()
        want, _ = E.sample_with(e.logits(), cfg, step, window)
        got = e.sample(cfg, step)
        assert got == want and e.token() == got
        assert e.recent() == window + [got]
        e.step()
    g = e.sample(None, 99)  # greedy: the device cursor, noted
    assert g == e.token() and e.recent()[-1] == g
    e.reset()
    assert e.recent() == []


def test_generate_sampled(model):
    p = _prompt(2, 12)
    greedy = E.Engine(model, 64).generate(p, 10)
    zero_t = E.SamplingConfig(temperature=0.0, repeat_penalty=1.0, repeat_last_n=0)
    host_greedy = E.Engine(model, 64).generate_sampled(p, 10, zero_t)
    # the host argmax takes the last of equal maxima, the device the first:
    # identical unless the logits tie exactly
    assert list(host_greedy) == list(greedy)
    cfg = E.SamplingConfig(temperature=1.0, top_p=1.0, top_k=0, seed=5)
    a = E.Engine(model, 64).generate_sampled(p, 16, cfg)
    b = E.Engine(model, 64).generate_sampled(p, 16, cfg)
    assert len(a) == 16 and list(a) == list(b)
    cfg.seed = 6
    c = E.Engine(model, 64).generate_sampled(p, 16, cfg)
    assert list(c) != list(a)  # near-uniform logits: another seed draws other tokens
    # the cache end stops generation: 12 prompt + 4 steps fill a 16-token cache
    short = E.Engine(model, 16).generate_sampled(p, 10, cfg)
    assert len(short) == 5
