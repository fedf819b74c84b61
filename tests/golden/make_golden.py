"""Writes the golden greedy streams under tests/golden/ with the CPU oracle.

The oracle (oracle/oracle.c) regenerates each seeded synthetic model on the
host -- the same bytes the device generator packs (tests/test_gpu_fixture_fused.py
checks the packer byte for byte) -- and runs the precision-mirrored forward,
recording each step's top-2 logit margin so a divergence on a near-tie can be
told from a bug. No reference code is imported or run.

    python tests/golden/make_golden.py [05b] [7b] [cfg2] [cfg4]    (default: 05b)

  05b   qwen05b_greedy.json: 0.5B shape, 16 prompt tokens, 64 greedy tokens.
  7b    qwen7b_ctx2048_greedy.json: the 7B shape of the headline benchmark,
        KV caches filled with the synthetic context (seed 2) for positions
        0..2047, one seeded token at position 2048, 256 greedy tokens (the
        configuration's 2048 -> 2304); plus a
        sample of the first step's logits (the top 64 and every 64th entry)
        and the oracle's two f32 summation orders (first-step logits and
        their 256-token streams). About 4 minutes to pack on 8 threads, 4 s
        per token and form.
  7bref adds to qwen7b_ctx2048_greedy.json the oracle's ORC_ACC_REF forward
        (the reference CUDA kernels' own arithmetic: f16 group sums in the
        GEMV, their reduction orders, attention split for a 30-SM device):
        its first-step logits at the same sample, its full-vector distance
        from the f64-summing oracle, and its 256-token stream with margins;
        the first step also at 132 SMs (another split count). About an hour
        on 8 threads.
  cfg2  qwen05b_ctx512_greedy.json: config 2's workload, the 0.5B shape with a
        seeded 512-token prompt and 256 greedy tokens (context 512 -> 768),
        plus the first generated step's logits under the oracle's two f32
        summation orders (the order-only drift at this depth).
  cfg2ref adds to qwen05b_ctx512_greedy.json the first generated step's
        logits under ORC_ACC_REF (the reference kernels' own arithmetic, 30-SM
        device) after the 512-token prompt: their distance from the mirrored
        oracle, and whether they meet 1e-2 / 1e-3. About 15 minutes.
  cfg4  qwen05b_qk_rescore_4096.json: the chunked-prefill configuration (0.5B
        shape, QK-norm, fp16 head rescore of the top 32), a seeded 4096-token
        prompt, then 128 greedy tokens.
"""
import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import oracle as O  # noqa: E402

HERE = Path(__file__).resolve().parent
SEED = 0
PROMPT_SEED = 1
KV_SEED = 2
N_NEW = 64
N_NEW_7B = 256   # config 3: context 2048 -> 2304
N_NEW_CFG4 = 128  # config 4: 128 decode steps after the prompt


def _decode(st, nxt, lg, n):
    tokens, margins, top = [], [], []
    for _ in range(n):
        tokens.append(int(nxt))
        margins.append(O.top2_margin(lg))
        top.append(float(np.max(lg)))
        nxt, lg = st.step(nxt)
    return tokens, margins, top


def _write(name, out, t0):
    out["threads"] = O.lib().orc_threads()
    out["seconds"] = round(time.time() - t0, 1)
    path = HERE / name
    path.write_text(json.dumps(out, indent=1))
    print(f"wrote {path} in {time.time() - t0:.1f}s; min margin {min(out['margins']):.3g}",
          flush=True)


def golden_05b():
    t0 = time.time()
    m = O.Model(O.QWEN05B, SEED)
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, O.QWEN05B["vocab"], 16)
    st = O.State(m, 256, 0)
    for t in prompt:
        nxt, lg = st.step(int(t))
    tokens, margins, top = _decode(st, nxt, lg, N_NEW)
    _write("qwen05b_greedy.json",
           dict(config="qwen2.5-0.5b-shape", seed=SEED, prompt_seed=PROMPT_SEED,
                prompt=[int(t) for t in prompt], tokens=tokens, margins=margins,
                top_logit=top, oracle="mirrored"), t0)


def golden_7b():
    t0 = time.time()
    ctx = 2048
    cfg = O.QWEN7B
    m = O.Model(cfg, SEED)
    print(f"7b packed in {time.time() - t0:.0f}s", flush=True)
    first = int(np.random.default_rng(PROMPT_SEED).integers(0, cfg["vocab"]))

    def state():
        st = O.State(m, ctx + N_NEW_7B + 8, 0)
        st.fill_kv(KV_SEED, ctx)
        st.pos = ctx
        return st

    drift, variant_tokens, variant_margins = {}, {}, {}
    for name, acc in (("f32_seq", O.ACC_F32_SEQ), ("f32_lane", O.ACC_F32_LANE)):
        with O.variant(acc):
            st = state()
            nxt_v, lg_v = st.step(first)
            drift[name] = lg_v.astype(np.float64)
            toks_v, margins_v, _ = _decode(st, nxt_v, lg_v, N_NEW_7B)
            variant_tokens[name], variant_margins[name] = toks_v, margins_v
            st.close()
        print(f"7b {name} stream done ({time.time() - t0:.0f}s)", flush=True)
    st = state()
    nxt, lg = st.step(first)
    lg0 = lg.copy()
    tokens, margins, top = _decode(st, nxt, lg, N_NEW_7B)
    top64 = np.argsort(-lg0.astype(np.float64), kind="stable")[:64]
    every = np.arange(0, cfg["vocab"], 64)
    sample = np.unique(np.concatenate([top64, every]))
    _write("qwen7b_ctx2048_greedy.json",
           dict(config="qwen2.5-7b-shape", seed=SEED, kv_seed=KV_SEED, context=ctx,
                first_token=first, tokens=tokens, margins=margins, top_logit=top,
                oracle="mirrored",
                first_step_logits=dict(index=[int(i) for i in sample],
                                       value=[float(lg0[i]) for i in sample]),
                # the same stream from the oracle with only its f32 summation
                # order changed (two ways): where these leave the mirrored
                # stream, the reference's own freedom of order decides the token
                order_variant_tokens=variant_tokens,
                order_variant_margins=variant_margins,
                first_step_order_drift=dict(
                    f32_seq_vs_f32_lane=float(np.max(np.abs(drift["f32_seq"] - drift["f32_lane"]))),
                    mirrored_vs_f32_seq=float(np.max(np.abs(lg0 - drift["f32_seq"]))),
                    mirrored_vs_f32_lane=float(np.max(np.abs(lg0 - drift["f32_lane"]))))), t0)


def golden_7b_ref():
    t0 = time.time()
    path = HERE / "qwen7b_ctx2048_greedy.json"
    g = json.loads(path.read_text())
    ctx, cfg = g["context"], O.QWEN7B
    m = O.Model(cfg, g["seed"])
    print(f"7b packed in {time.time() - t0:.0f}s", flush=True)

    def state():
        st = O.State(m, ctx + N_NEW_7B + 8, 0)
        st.fill_kv(g["kv_seed"], ctx)
        st.pos = ctx
        return st

    st = state()
    f64 = st.step(g["first_token"])[1].astype(np.float64)
    st.close()
    idx = np.asarray(g["first_step_logits"]["index"])
    assert np.array_equal(f64[idx].astype(np.float32),
                          np.asarray(g["first_step_logits"]["value"], np.float32))
    lib = O.lib()
    lib.orc_set_ref_sms(132)
    with O.variant(O.ACC_REF):
        st = state()
        ref132 = st.step(g["first_token"])[1].astype(np.float64)
        st.close()
    lib.orc_set_ref_sms(30)
    with O.variant(O.ACC_REF):
        st = state()
        nxt, lg = st.step(g["first_token"])
        ref = lg.astype(np.float64)
        print(f"7b ref first step {time.time() - t0:.0f}s: vs f64 {np.max(np.abs(ref - f64)):.4f}",
              flush=True)
        tokens, margins, top = _decode(st, nxt, lg, N_NEW_7B)
        st.close()
    g["ref"] = dict(
        sms=30,
        first_step_sample=[float(ref[i]) for i in idx],
        first_step_vs_f64=float(np.max(np.abs(ref - f64))),
        first_step_allclose_1e3_1e2=bool(np.allclose(ref, f64, rtol=1e-3, atol=1e-2)),
        first_step_vs_f64_at_132_sms=float(np.max(np.abs(ref132 - f64))),
        first_step_30_vs_132_sms=float(np.max(np.abs(ref - ref132))),
        tokens=tokens, margins=margins, top_logit=top,
        seconds=round(time.time() - t0, 1))
    path.write_text(json.dumps(g, indent=1))
    print(f"wrote {path} in {time.time() - t0:.1f}s", flush=True)


def golden_cfg2():
    t0 = time.time()
    cfg = O.QWEN05B
    n_prompt, n_new = 512, 256
    m = O.Model(cfg, SEED)
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, cfg["vocab"], n_prompt)
    first = {}
    for name, acc in (("f32_seq", O.ACC_F32_SEQ), ("f32_lane", O.ACC_F32_LANE)):
        with O.variant(acc):
            st = O.State(m, n_prompt + 8, 0)
            for t in prompt:
                _, lg = st.step(int(t))
            first[name] = lg.astype(np.float64)
            st.close()
    st = O.State(m, n_prompt + n_new + 8, 0)
    for t in prompt:
        nxt, lg = st.step(int(t))
    lg0 = lg.astype(np.float64)
    tokens, margins, top = _decode(st, nxt, lg, n_new)
    _write("qwen05b_ctx512_greedy.json",
           dict(config="qwen2.5-0.5b-shape", seed=SEED, prompt_seed=PROMPT_SEED,
                n_prompt=n_prompt, tokens=tokens, margins=margins, top_logit=top,
                oracle="mirrored",
                first_step_order_drift=dict(
                    f32_seq_vs_f32_lane=float(np.max(np.abs(first["f32_seq"] - first["f32_lane"]))),
                    mirrored_vs_f32_seq=float(np.max(np.abs(lg0 - first["f32_seq"]))),
                    mirrored_vs_f32_lane=float(np.max(np.abs(lg0 - first["f32_lane"]))))), t0)


def golden_cfg2_ref():
    t0 = time.time()
    path = HERE / "qwen05b_ctx512_greedy.json"
    g = json.loads(path.read_text())
    cfg = O.QWEN05B
    m = O.Model(cfg, g["seed"])
    prompt = np.random.default_rng(g["prompt_seed"]).integers(0, cfg["vocab"], g["n_prompt"])
    lg = {}
    for name, acc in (("f64", O.ACC_F64), ("ref", O.ACC_REF)):
        with O.variant(acc):
            st = O.State(m, g["n_prompt"] + 8, 0)
            for t in prompt:
                nxt, l_ = st.step(int(t))
            lg[name] = (nxt, l_.astype(np.float64))
            st.close()
    assert lg["f64"][0] == g["tokens"][0]
    g["ref"] = dict(sms=30, first_token=int(lg["ref"][0]),
                    first_step_vs_f64=float(np.max(np.abs(lg["ref"][1] - lg["f64"][1]))),
                    first_step_allclose_1e3_1e2=bool(np.allclose(lg["ref"][1], lg["f64"][1],
                                                                 rtol=1e-3, atol=1e-2)),
                    seconds=round(time.time() - t0, 1))
    path.write_text(json.dumps(g, indent=1))
    print(f"wrote {path} in {time.time() - t0:.1f}s: ref vs f64 {g['ref']['first_step_vs_f64']:.4f}",
          flush=True)


def golden_cfg4():
    """The 4096-token prompt, then the configuration's 128 greedy tokens, from
    the mirrored (f64-summing) oracle; with a sample of the first generated
    step's logits (the top 64 and every 64th) and the distance between the
    oracle's two f32 summation orders at that step (each runs the whole
    prompt in its own order), so that a GPU stream's departure from this one
    can be held to a margin two implementations that far apart could split."""
    t0 = time.time()
    cfg = dict(O.QWEN05B, qk_norm=1, rescore_k=32)
    n_prompt = 4096
    m = O.Model(cfg, SEED)
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, cfg["vocab"], n_prompt)

    def run_prompt(tag):
        st = O.State(m, n_prompt + N_NEW_CFG4 + 8, 0)
        for i, t in enumerate(prompt):
            nxt, lg = st.step(int(t))
            if i % 512 == 511:
                print(f"cfg4 {tag} prompt {i + 1}/{n_prompt} ({time.time() - t0:.0f}s)", flush=True)
        return st, nxt, lg

    drift = {}
    for name, acc in (("f32_seq", O.ACC_F32_SEQ), ("f32_lane", O.ACC_F32_LANE)):
        with O.variant(acc):
            st, _, lg_v = run_prompt(name)
            drift[name] = lg_v.astype(np.float64)
            st.close()
    st, nxt, lg = run_prompt("mirrored")
    lg0 = lg.copy().astype(np.float64)
    tokens, margins, top = _decode(st, nxt, lg, N_NEW_CFG4)
    top64 = np.argsort(-lg0, kind="stable")[:64]
    sample = np.unique(np.concatenate([top64, np.arange(0, cfg["vocab"], 64)]))
    _write("qwen05b_qk_rescore_4096.json",
           dict(config="qwen2.5-0.5b-shape, qk_norm, rescore_k=32", seed=SEED,
                prompt_seed=PROMPT_SEED, n_prompt=n_prompt, tokens=tokens, margins=margins,
                top_logit=top, oracle="mirrored",
                first_step_logits=dict(index=[int(i) for i in sample],
                                       value=[float(lg0[i]) for i in sample]),
                first_step_order_drift=dict(
                    f32_seq_vs_f32_lane=float(np.max(np.abs(drift["f32_seq"] - drift["f32_lane"]))),
                    mirrored_vs_f32_seq=float(np.max(np.abs(lg0 - drift["f32_seq"]))),
                    mirrored_vs_f32_lane=float(np.max(np.abs(lg0 - drift["f32_lane"]))))), t0)


def golden_7b_prompt():
    """The 7B shape after a seeded 256-token prompt (one chunk): the f64-
    summing oracle's first-step logits (a sample: the top 64 and every 64th)
    and first token, and the same step in ORC_ACC_REF, the reference CUDA
    build's own arithmetic, with its distance from the f64 oracle; for the
    chunk path's parity at full depth."""
    t0 = time.time()
    cfg = O.QWEN7B
    n_prompt = 256
    m = O.Model(cfg, SEED)
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, cfg["vocab"], n_prompt)
    lg = {}
    for name, acc in (("f64", O.ACC_F64), ("ref", O.ACC_REF)):
        with O.variant(acc):
            st = O.State(m, n_prompt + 8, 0)
            for i, t in enumerate(prompt):
                nxt, l_ = st.step(int(t))
                if i % 64 == 63:
                    print(f"7b prompt {name} {i + 1}/{n_prompt} ({time.time() - t0:.0f}s)", flush=True)
            lg[name] = (int(nxt), l_.astype(np.float64))
            st.close()
    l0 = lg["f64"][1]
    top64 = np.argsort(-l0, kind="stable")[:64]
    sample = np.unique(np.concatenate([top64, np.arange(0, cfg["vocab"], 64)]))
    out = dict(config="qwen2.5-7b-shape", seed=SEED, prompt_seed=PROMPT_SEED, n_prompt=n_prompt,
               first_token=lg["f64"][0], top2_margin=O.top2_margin(l0),
               first_step_logits=dict(index=[int(i) for i in sample],
                                      value=[float(l0[i]) for i in sample]),
               ref=dict(sms=30, first_token=lg["ref"][0],
                        first_step_vs_f64=float(np.max(np.abs(lg["ref"][1] - l0)))),
               oracle="mirrored", threads=O.lib().orc_threads(),
               seconds=round(time.time() - t0, 1))
    path = HERE / "qwen7b_prompt256.json"
    path.write_text(json.dumps(out, indent=1))
    print(f"wrote {path} in {time.time() - t0:.1f}s; ref vs f64 {out['ref']['first_step_vs_f64']:.4f}",
          flush=True)


if __name__ == "__main__":
    which = sys.argv[1:] or ["05b"]
    for w in which:
        {"05b": golden_05b, "7b": golden_7b, "7bref": golden_7b_ref, "cfg2": golden_cfg2,
         "cfg2ref": golden_cfg2_ref,
         "cfg4": golden_cfg4, "7bprompt": golden_7b_prompt}[w]()
