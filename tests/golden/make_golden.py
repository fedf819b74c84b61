"""Writes tests/golden/qwen05b_greedy.json with the CPU oracle.

The oracle (oracle/oracle.c) regenerates the seeded 0.5B-shaped synthetic
model on the host -- the same bytes the device generator packs -- and runs the
precision-mirrored forward: 16 prompt tokens, then 64 greedy tokens, recording
each step's top-2 logit margin (so a divergence on a near-tie can be told from
a bug). No reference code is imported or run.

    python tests/golden/make_golden.py
"""
import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle as O  # noqa: E402

SEED = 0
PROMPT_SEED = 1
N_PROMPT, N_NEW = 16, 64


def main():
    t0 = time.time()
    m = O.Model(O.QWEN05B, SEED)
    t1 = time.time()
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, O.QWEN05B["vocab"], N_PROMPT)
    st = O.State(m, 256, 0)
    for t in prompt:
        nxt, lg = st.step(int(t))
    tokens, margins, top = [], [], []
    for _ in range(N_NEW):
        tokens.append(int(nxt))
        margins.append(O.top2_margin(lg))
        top.append(float(np.max(lg)))
        nxt, lg = st.step(nxt)
    out = dict(config="qwen2.5-0.5b-shape", seed=SEED, prompt_seed=PROMPT_SEED,
               prompt=[int(t) for t in prompt], tokens=tokens, margins=margins, top_logit=top,
               oracle="mirrored", threads=O.lib().orc_threads(),
               seconds=dict(model=round(t1 - t0, 1), decode=round(time.time() - t1, 1)))
    path = Path(__file__).resolve().parent / "qwen05b_greedy.json"
    path.write_text(json.dumps(out, indent=1))
    print(f"wrote {path} in {time.time() - t0:.1f}s; min margin {min(margins):.3g}")


if __name__ == "__main__":
    main()
