"""GPU parity at the chunked-prefill configuration (config 4).

Qwen2.5-0.5B shape with QK-norm and the int4 head rescored from an fp16 copy
(top 32); seeded weights packed on the device; a seeded 4096-token prompt
prefilled in 256-token chunks (16 chunks), then the golden file's greedy
tokens (128: the configuration's decode steps).

The reference's contract for this path (crates/whetstone-core/src/engine.rs:
195-199): chunked prefill gives bit-identical greedy output to sequential
prefill. Checked here three ways, each token for token (a divergence is
allowed only on an oracle near-tie, top-2 margin < 1e-4):
  chunked stream == sequential stream
  chunked stream == the oracle's (tests/golden/qwen05b_qk_rescore_4096.json)
  sequential stream == the oracle's
"""
import json
from pathlib import Path

import numpy as np
import pytest

from conftest import assert_streams
from whetstone_amd import engine as E

pytestmark = pytest.mark.gpu
_PATH = Path(__file__).resolve().parent / "golden" / "qwen05b_qk_rescore_4096.json"
GOLDEN = json.loads(_PATH.read_text()) if _PATH.exists() else {"tokens": []}
CFG = dict(E.QWEN05B, qk_norm=1, rescore_k=32)
N_NEW = len(GOLDEN["tokens"])


@pytest.fixture(scope="module", autouse=True)
def _have_golden():
    if not _PATH.exists():
        pytest.fail(f"{_PATH.name} is missing: python tests/golden/make_golden.py cfg4")


@pytest.fixture(scope="module")
def streams():
    g = E.Model(CFG, seed=GOLDEN["seed"])
    prompt = np.random.default_rng(GOLDEN["prompt_seed"]).integers(
        0, CFG["vocab"], GOLDEN["n_prompt"]).astype(np.int32)
    out = {}
    for chunked in (True, False):
        eng = E.Engine(g, GOLDEN["n_prompt"] + N_NEW + 8)
        if chunked:
            assert eng.chunk_width() == 256
        eng.capture_graph()
        out[chunked] = eng.generate(prompt, N_NEW, chunked=chunked)
        eng.close()
    g.close()
    return out


def test_chunked_prefill_greedy_equals_sequential(streams):
    n = assert_streams(streams[True], streams[False], GOLDEN["margins"])
    print(f"chunked vs sequential prefill: {n}/{N_NEW} greedy tokens identical")


@pytest.mark.parametrize("chunked", [True, False], ids=["chunked", "sequential"])
def test_stream_after_4096_prompt_matches_oracle(streams, chunked):
    n = assert_streams(streams[chunked], GOLDEN["tokens"], GOLDEN["margins"])
    print(f"{'chunked' if chunked else 'sequential'} prefill: {n}/{N_NEW} tokens as the oracle")
