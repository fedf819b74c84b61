"""Host-side stochastic sampling (wse_sample_with: engine.rs:987-1114) on the
CPU: the reference's own sampler tests restated (engine.rs:1155-1250), the
published SplitMix64 vectors, and an independent pure-Python restatement of
the algorithm compared token for token over random logits, configurations and
steps."""
import math

import numpy as np
import pytest

from whetstone_amd import engine as E


def plain(temperature, top_p, seed):
    """engine.rs:1158-1168: a config that isolates one knob."""
    return E.SamplingConfig(temperature, top_p, 0, 0.0, 1.0, 0, seed)


def draw(l, cfg, step, recent=()):
    return E.sample_with(np.asarray(l, np.float32), cfg, step, recent)[0]


def test_splitmix64_published_vectors():
    # seed 0, then the state after one step (the first two outputs of the
    # published SplitMix64 reference stream)
    assert E.splitmix64(0) == 0xE220A8397B1DCDAF
    assert E.splitmix64(0x9E3779B97F4A7C15) == 0x6E789E6AA1B965F4


def test_greedy_is_what_zero_temperature_means():
    l = np.zeros(64, np.float32)
    l[37] = 5.0
    assert draw(l, plain(0.0, 0.9, 1), 0) == 37


def test_greedy_ties_go_to_the_last_maximum():
    """engine.rs:1098-1105 (max_by keeps the later of equal elements): the
    host argmax is the opposite of the device's low-index rule."""
    l = np.zeros(16, np.float32)
    l[[3, 9]] = 2.0
    assert draw(l, plain(0.0, 1.0, 0), 0) == 9


def test_nucleus_sampling_never_leaves_the_nucleus():
    l = np.full(512, -20.0, np.float32)
    l[100] = 10.0
    for seed in range(32):
        assert draw(l, plain(1.0, 0.9, seed), seed) == 100


def test_sampling_is_reproducible_for_a_seed():
    l = np.array([((i * 37 % 101) / 20.0) for i in range(1024)], np.float32)
    cfg = plain(0.8, 0.95, 7)
    a = [draw(l, cfg, s) for s in range(16)]
    assert a == [draw(l, cfg, s) for s in range(16)]
    assert len(set(a)) > 1


def test_top_k_bounds_what_can_be_drawn():
    l = np.arange(512, dtype=np.float32) * 0.01
    cfg = plain(2.0, 1.0, 0)
    cfg.top_k = 3
    for step in range(64):
        assert draw(l, cfg, step) >= 509


def test_min_p_tightens_when_the_model_is_confident():
    peaked = np.zeros(256, np.float32)
    peaked[9] = 12.0
    cfg = plain(1.0, 1.0, 3)
    cfg.min_p = 0.1
    for step in range(32):
        assert draw(peaked, cfg, step) == 9
    flat = np.ones(256, np.float32)
    assert len({draw(flat, cfg, s) for s in range(64)}) > 1


def test_repetition_penalty_moves_logits_toward_zero_from_both_sides():
    l = np.full(8, -8.0, np.float32)
    l[1], l[2] = 6.0, 5.0
    cfg = plain(0.0, 1.0, 0)
    cfg.repeat_penalty, cfg.repeat_last_n = 2.0, 4
    t, v = E.sample_with(l, cfg, 0, [1])
    assert t == 2 and v[1] < l[1]
    _, v2 = E.sample_with(l, cfg, 0, [0])
    assert v2[0] < l[0]


def test_repetition_penalty_only_looks_back_repeat_last_n():
    l = np.zeros(8, np.float32)
    l[3] = 1.0
    cfg = plain(0.0, 1.0, 0)
    cfg.repeat_penalty, cfg.repeat_last_n = 2.0, 2
    _, v = E.sample_with(l, cfg, 0, [3, 5, 5, 5, 5])
    assert v[3] == l[3]
    # each occurrence in the window counts: two 5s divide twice
    l[5] = 8.0
    _, v = E.sample_with(l, cfg, 0, [3, 5, 5])
    assert v[5] == np.float32(np.float32(8.0 / 2.0) / 2.0)


# ------------------------------------------------ independent restatement

M64 = (1 << 64) - 1


def _splitmix(z):
    z = (z + 0x9E3779B97F4A7C15) & M64
    r = z
    r = ((r ^ (r >> 30)) * 0xBF58476D1CE4E5B9) & M64
    r = ((r ^ (r >> 27)) * 0x94D049BB133111EB) & M64
    return r ^ (r >> 31)


def _py_sample(logits, temperature, top_p, top_k, min_p, pen, last_n, seed, step, recent):
    l = [np.float32(v) for v in logits]
    if pen != 1.0 and last_n > 0:
        for t in list(recent)[-last_n:] if recent else []:
            if 0 <= t < len(l):
                l[t] = np.float32(l[t] / np.float32(pen)) if l[t] > 0 else np.float32(l[t] * np.float32(pen))
    if temperature <= 0:
        best = 0
        for i in range(1, len(l)):
            if not (l[best] > l[i]):
                best = i
        return best
    pool = min(top_k, 512) if top_k > 0 else 512
    order = sorted(range(len(l)), key=lambda i: (-float(l[i]), i))[:min(pool, len(l))]
    mx = float(l[order[0]])
    probs = [math.exp((float(l[i]) - mx) / float(np.float32(temperature))) for i in order]
    total = 0.0
    for p in probs:
        total += p
    cut = len(probs)
    if min_p > 0:
        floor_ = probs[0] * float(np.float32(min_p))
        cut = next((i for i, p in enumerate(probs) if p < floor_), len(probs))
        cut = max(cut, 1)
    if top_p < 1.0:
        acc = 0.0
        for i in range(cut):
            acc += probs[i] / total
            if acc >= float(np.float32(top_p)):
                cut = i + 1
                break
    mass = 0.0
    for p in probs[:cut]:
        mass += p
    u = float(_splitmix(seed ^ ((step * 0x9E3779B97F4A7C15) & M64))) / float(M64) * mass
    acc = 0.0
    for i in range(cut):
        acc += probs[i]
        if acc >= u:
            return order[i]
    return order[max(cut - 1, 0)]


@pytest.mark.parametrize("case", range(12))
def test_sample_with_equals_an_independent_restatement(case):
    rng = np.random.default_rng(100 + case)
    n = int(rng.choice([7, 300, 2000]))
    logits = (rng.standard_normal(n) * rng.choice([0.5, 2.0, 6.0])).astype(np.float32)
    if case % 3 == 0:
        logits[rng.integers(0, n, 5)] = logits.max()  # ties at the top
    cfgs = [(0.7, 0.8, 20, 0.0, 1.05, 64), (1.0, 1.0, 0, 0.0, 1.0, 0), (1.3, 0.95, 0, 0.05, 1.2, 8),
            (0.5, 0.5, 600, 0.0, 1.0, 0), (0.0, 0.9, 0, 0.0, 1.3, 16)]
    recent = [int(v) for v in rng.integers(0, n, 40)]
    for (t, p, k, mp, pen, last) in cfgs:
        cfg = E.SamplingConfig(t, p, k, mp, pen, last, 1000 + case)
        for step in range(6):
            want = _py_sample(logits, t, p, k, mp, pen, last, 1000 + case, step, recent)
            assert draw(logits, cfg, step, recent) == want, (t, p, k, mp, pen, last, step)
