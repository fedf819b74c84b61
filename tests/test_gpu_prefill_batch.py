"""The batched prefill against the chunk-by-chunk one.

A chunked prefill's full chunks go through each layer together, one launch
per op for all of them (engine.cpp chunk_pass), each launch keeping one
chunk's tiling and split-K plan. The contract is bit-identity with running
the same chunks one after the other (WSE_CHUNK_BATCH=0): the last chunk's
logits, its greedy picks, every KV-cache row (seen through the decode steps
that follow), and the greedy stream after the prompt.
"""
import os

import numpy as np
import pytest

from whetstone_amd import engine as E

pytestmark = pytest.mark.gpu


def _run(g, prompt, n_new, batch):
    os.environ["WSE_CHUNK_BATCH"] = "1" if batch else "0"
    try:
        eng = E.Engine(g, len(prompt) + n_new + 8)
        assert eng.chunk_width() == 256
        eng.prefill(prompt, chunked=True)
        logits = eng.logits().copy()
        tok = eng.token()
        picks = eng.chunk_picks(len(prompt) - (len(prompt) - 1) // 256 * 256)
        toks = [tok]
        for _ in range(n_new):
            eng.step()
            toks.append(eng.token())
        eng.close()
    finally:
        os.environ.pop("WSE_CHUNK_BATCH", None)
    return logits, picks, toks


@pytest.mark.parametrize("cfg_name,n_prompt", [("05b_qk_rescore", 1024), ("05b_qk_rescore", 900),
                                               ("05b", 768), ("7b", 512)])
def test_batched_prefill_is_bit_identical_to_chunk_by_chunk(cfg_name, n_prompt):
    cfg = {"05b_qk_rescore": dict(E.QWEN05B, qk_norm=1, rescore_k=32), "05b": E.QWEN05B,
           "7b": dict(E.QWEN7B, n_layers=4)}[cfg_name]
    g = E.Model(cfg, seed=3)
    prompt = np.random.default_rng(n_prompt).integers(0, cfg["vocab"], n_prompt).astype(np.int32)
    print(f"batched prefill: {cfg_name}, {n_prompt} tokens", flush=True)
    a = _run(g, prompt, 8, False)
    b = _run(g, prompt, 8, True)
    g.close()
    assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
    assert np.array_equal(a[1], b[1])
    assert a[2] == b[2]
