"""Batch=1 int4-hier-g32 decode benchmark on one MI355X.

Workload (default, the configuration the headline metric is quoted on):
Qwen2.5-7B-shaped decoder (28 layers, hidden 3584, 28 q / 4 kv heads of 128,
SwiGLU 18944, vocab 152064, untied int4 lm_head), seeded synthetic weights
packed to int4-hier-g32 on the device, KV caches filled with seeded f16 for
positions 0..2047, then `--steps` greedy tokens (2048 -> 2304 at the default
256), one captured-graph replay and a 4-byte token read back per token, as the
reference's generate loop does.

The line printed carries:
  value      tok/s over the timed steps (inputs resident in HBM)
  roofline   the dominant kernel (largest share of the step's time) timed with
             HIP events over back-to-back launches of all its layer instances;
             achieved = algorithmic bytes per launch / average launch time
  kernels    the same figures for every stage kernel
  cpu_baseline  the CPU oracle (oracle/, a C restatement of the reference's
             dequant + forward) on the same weights and context, timed on the
             host cores for a bounded number of tokens
  cpu_check  the GPU's first-step logits and tokens against that CPU run
  secondary  (config 3 without --no-secondary) the other GPU configurations,
             each measured once after the headline's timed region: config 2
             (0.5B decode, 512-token prefill, 256 steps), config 4 (4096-token
             chunked prefill with counted TFLOP/s, then 128 decode steps),
             config 1 (the 0.5B lm_head GEMV, weights cold)
  config.full_range_tok_s  (config 3, when --steps is not 256) the whole
             2048 -> 2304 range, timed after the headline's steps

The config-3 KV cache always holds the configuration's 2304 positions (+8), so
attention's grid is the configuration's whatever --steps is.

    python bench.py [--steps 256] [--warmup 8] [--config 3|2] [--cpu-seconds 12]

`--config 0` times the CPU reference path (the 0.5B shape, 16 + 32 greedy
tokens, on the host) beside the GPU engine on the same weights.
`--config 1` measures the GEMV alone (lm_head and 0.5B block shapes, weights
cold past the MALL and hot) and prints a line of its own.
`--config 4` instead measures the chunked prefill (0.5B shape with QK-norm and
the int4 head rescored from an fp16 copy, top-32): a 4096-token seeded prompt
in 256-token chunks through the MFMA GEMMs, the 16 chunks batched one launch
per op and layer (and, for comparison, one launch per chunk and op), then 128
greedy decode steps, and prints a line of its own (prefill tok/s and achieved
TFLOP/s, decode tok/s). `--batched-only` skips the per-chunk timing.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "batch=1 decode tok/s + achieved HBM GB/s (% of 8 TB/s), Qwen2.5-0.5B/7B int4"
HBM_PEAK_GBS = 8000.0
KV_SEED, WEIGHT_SEED, PROMPT_SEED = 2, 0, 1
FULL_RANGE = 256  # config 3 decodes context 2048 -> 2304
TIMED_STAGES = ["qkv", "attn", "o", "gate_up", "down", "head"]
KERNEL_NAMES = {  # kernels each stage launches in the fused step (rocprof names)
    "qkv": "gemv_hier_kernel<NG, WPR, XB, 512, NORM=true, SWIGLU=false, PD>",
    "attn": "attn_decode_kernel<HD, ROPE=true> + attn_merge_kernel",
    "o": "gemv_hier_kernel<NG, WPR, XB, NT, NORM=false, SWIGLU=false, PD>",
    "gate_up": "gemv_hier_kernel<NG, WPR, XB, 512, NORM=true, SWIGLU=true, PD>",
    "down": "gemv_hier_kernel<NG, WPR, XB, NT, NORM=false, SWIGLU=false, PD>",
    "head": "gemv_hier_kernel<NG, WPR, XB, 512, NORM=true, SWIGLU=false, PD>",
}
TRAFFIC_FILE = ROOT / "profiles" / "traffic.md"
GEMV_TRAFFIC_FILE = ROOT / "profiles" / "gemv_cfg1_kernel_trace.md"


def log(msg: str) -> None:
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None,
                   help="timed decode steps (default 256; config 4: its 128 decode steps)")
    p.add_argument("--warmup", type=int, default=8)
    p.add_argument("--config", type=int, default=3, choices=(0, 1, 2, 3, 4))
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="CPU baseline budget (tokens are added until it is spent)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-secondary", action="store_true",
                   help="with --config 3: skip the configs 1, 2 and 4 measured after the "
                        "headline's timed region")
    p.add_argument("--stage-reps", type=int, default=20)
    p.add_argument("--no-full-range", action="store_true",
                   help="config 3: skip the timing of the whole 2048 -> 2304 range after the "
                        "headline's steps")
    p.add_argument("--no-graph", action="store_true",
                   help="configs 2 and 3: launch each step's kernels eagerly instead of replaying "
                        "the captured graph (the same kernels; for profiler runs, whose graph "
                        "launch interception can crash)")
    p.add_argument("--max-seq", type=int, default=0,
                   help="KV-cache capacity for configs 2 and 3 (default: the context plus the "
                        "generated tokens plus 8); attention's grid covers the capacity")
    p.add_argument("--batched-only", action="store_true",
                   help="with --config 4: time only the batched prefill (for profiler runs)")
    p.add_argument("--gemm-7b", action="store_true",
                   help="with --config 4: also time the chunk GEMMs at the 7B shapes")
    p.add_argument("--floors", action="store_true",
                   help="with --config 2 or 3: the step's launch structure replayed as a graph "
                        "of plain streaming reads of each kernel's bytes (the floor of that "
                        "structure), beside a graph of the same number of empty launches")
    p.add_argument("--summarize", nargs="+", metavar="DIR",
                   help="print a text summary of rocprofv3 CSV output directories "
                        "(kernel stats, or FETCH_SIZE/WRITE_SIZE counters scaled by a "
                        "--copy-probe run given with --calibration) and exit")
    p.add_argument("--calibration", nargs="*", default=[], metavar="DIR",
                   help="rocprofv3 counter directories of a --copy-probe run (its size in "
                        "MiB by --copy-probe, default 256)")
    p.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                   help="only run the counter calibration: a device-to-device copy, a "
                        "memset and a read sweep of MIB MiB each, then exit")
    a = p.parse_args()
    if a.steps is None:
        a.steps = 128 if a.config == 4 else 256
    return a


def _short(name: str) -> str:
    name = name.replace("HIP_vector_type<unsigned int, 4u>", "uint4")
    return name.split("(")[0].replace("void ", "")[:96]


def summarize(dirs, calibration, copy_mib) -> None:
    """Text summary of rocprofv3 --output-format csv directories."""
    import csv
    import glob
    from collections import defaultdict
    scale = {}
    for d in calibration:  # counter value of the copy kernel vs its known bytes
        for f in glob.glob(os.path.join(d, "*counter_collection.csv")):
            for r in csv.DictReader(open(f)):
                if "copyBuffer" in r["Kernel_Name"]:  # reads and writes copy_mib MiB
                    scale[r["Counter_Name"]] = copy_mib * 1024 / float(r["Counter_Value"])
    for d in dirs:
        for f in sorted(glob.glob(os.path.join(d, "*kernel_stats.csv"))):
            rows = list(csv.DictReader(open(f)))
            print(f"kernel stats ({os.path.basename(f)}): name | calls | avg us | total ms | %")
            for r in rows[:16]:
                print(f"  {_short(r['Name']):96s} | {int(r['Calls']):6d} | "
                      f"{float(r['AverageNs']) / 1e3:9.2f} | {float(r['TotalDurationNs']) / 1e6:9.2f}"
                      f" | {float(r['Percentage']):5.1f}")
        for f in sorted(glob.glob(os.path.join(d, "*counter_collection.csv"))):
            agg = defaultdict(list)
            for r in csv.DictReader(open(f)):
                agg[(r["Counter_Name"], _short(r["Kernel_Name"]), int(r["Grid_Size"]))].append(
                    float(r["Counter_Value"]))
            print(f"counters ({os.path.basename(f)}): counter | kernel | grid | dispatches | "
                  f"avg KiB/dispatch | scale | avg bytes/dispatch")
            for (cn, kn, grid), v in sorted(agg.items(), key=lambda kv: -sum(kv[1]))[:16]:
                sc = scale.get(cn, 1.0)
                avg = sum(v) / len(v)
                print(f"  {cn} | {kn:96s} | {grid:8d} | {len(v):5d} | {avg:12.1f} | {sc:.4f} | "
                      f"{avg * 1024 * sc:14.0f}")
    for cn, sc in sorted(scale.items()):
        print(f"calibration: {cn} reads {1 / sc:.5f} KiB per KiB a copy kernel moves (scale {sc:.5f})")


def copy_probe(mib: int) -> None:
    """Kernels of known traffic, for scaling rocprofv3's FETCH_SIZE and
    WRITE_SIZE readings: a copy reads and writes `mib` MiB, a memset writes
    it, the bandwidth sweep reads it."""
    from whetstone_amd import kernels as wk, ffi
    n = mib << 20
    a = wk.DeviceBuffer(n, np.uint8)
    b = wk.DeviceBuffer(n, np.uint8)
    for _ in range(3):
        ffi.call("wst_memcpy_d2d", b.ptr, a.ptr, n)
        ffi.call("wst_memset", a.ptr, 1, n)
    gbs = wk.bench_bandwidth(n, 3)
    wk.synchronize()
    print(json.dumps({"copy_probe_bytes": n, "bandwidth_sweep_gbs": round(gbs, 1)}), flush=True)


def traffic_for(config: int, stage: str, path=None):
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE + WRITE_SIZE,
    scaled by the same counters' reading for a copy of known size; committed
    in profiles/traffic.md as `traffic cfg<N> <stage>: <bytes>` lines."""
    path = path or TRAFFIC_FILE
    if not path.exists():
        return None
    key = f"traffic cfg{config} {stage}:"
    for line in path.read_text().splitlines():
        line = line.strip().strip("`")
        if line.startswith(key):
            return int(line[len(key):].strip().split()[0])
    return None


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def copy_model_to_oracle(g, o, cfg):
    """Device packed bytes -> the oracle's (zero-initialised) host matrices."""
    from whetstone_amd import ffi
    names = ["embed"] + ([] if cfg["tied"] else ["lm_head"])
    names += [f"L{l}.{t}" for l in range(cfg["n_layers"]) for t in ("qkv", "o", "gate_up", "down")]
    for name in names:
        qw, si, sb, i, n = g.tensor(name)
        p = o.tensor(name)
        assert (p.in_f, p.out_f) == (i, n), name
        for dst, src in ((p.qw, qw), (p.si, si), (p.sb, sb)):
            ffi.check(ffi.lib().wst_memcpy_d2h(dst.ctypes.data, src, dst.nbytes))


def cpu_leg(g, cfg, ctx0, first_token, gpu_tokens, gpu_logits0, budget_s, same_context):
    """Times the oracle's precision-mirrored decode on the same weights and a
    synthetic context of the same length; when that context is the GPU's own
    (same_context), also checks the GPU's first logits and tokens."""
    from oracle import oracle as O
    t0 = time.perf_counter()
    o = O.Model(cfg, WEIGHT_SEED, pack=False)
    copy_model_to_oracle(g, o, cfg)
    st = O.State(o, ctx0 + 64, 0)
    st.fill_kv(KV_SEED, ctx0)
    st.pos = ctx0
    setup_s = time.perf_counter() - t0
    tok, times, toks, lg0 = first_token, [], [], None
    while True:
        t = time.perf_counter()
        nxt, lg = st.step(tok)
        times.append(time.perf_counter() - t)
        if lg0 is None:
            lg0 = lg
        toks.append(nxt)
        tok = nxt
        if sum(times) >= budget_s or len(times) >= 16:
            break
    lg_text = None
    if same_context:  # the f64 textbook forward (no f16 narrowing) for one step
        tb = O.State(o, ctx0 + 64, 1)
        tb.fill_kv(KV_SEED, ctx0)
        tb.pos = ctx0
        _, lg_text = tb.step(first_token)
        tb.close()
        # the same step in the reference CUDA kernels' own arithmetic (f16
        # group sums, their reduction orders): how far the reference itself
        # lands from the precision-mirrored f64 forward
        rf = O.State(o, ctx0 + 64, 0)
        rf.fill_kv(KV_SEED, ctx0)
        rf.pos = ctx0
        with O.variant(O.ACC_REF):
            _, lg_ref = rf.step(first_token)
        rf.close()
    st.close()
    n = len(toks)
    # The reference's CPU path dequantises the model once (whetstone-quant)
    # before its numpy forward: timed here on layer 0's four matrices and the
    # head, projected to the whole model.
    t = time.perf_counter()
    for name in ("L0.qkv", "L0.o", "L0.gate_up", "L0.down"):
        O.dequantize(o.tensor(name))
    layer_s = time.perf_counter() - t
    t = time.perf_counter()
    O.dequantize(o.tensor("embed" if cfg["tied"] else "lm_head"))
    head_s = time.perf_counter() - t
    base = {
        "value": round(n / sum(times), 4),
        "unit": "tok/s",
        "cores": int(O.lib().orc_threads()),
        "kind": "port",
        "nproc": os.cpu_count(),
        "cpu_model": cpu_model(),
        "dequant_s_per_layer": round(layer_s, 3),
        "dequant_s_model_projected": round(layer_s * cfg["n_layers"] + head_s, 2),
        "sample": (f"{n} greedy tokens from a {ctx0}-token context on the same packed weights: "
                   f"oracle/oracle.c precision-mirrored forward (dequant on the fly, f64 dot "
                   f"products), OpenMP over rows; setup {setup_s:.1f}s not timed; the whole-model "
                   f"dequantisation of the reference's CPU path projected from layer 0 and the "
                   f"head on the same threads"),
    }
    o.close()
    if not same_context:
        return base, None
    diff = np.abs(gpu_logits0.astype(np.float64) - lg0)
    rel = diff / np.maximum(np.abs(lg0), 1.0)
    check = {
        "tokens_compared": n,
        "tokens_identical": int(sum(int(a) == int(b) for a, b in zip(toks, gpu_tokens[:n]))),
        "first_step_logits_max_abs": float(diff.max()),
        "first_step_logits_max_rel": float(rel.max()),
        "first_step_within_tolerance": bool(np.allclose(gpu_logits0, lg0, rtol=1e-3, atol=1e-2)),
        "first_step_reference_arithmetic_max_abs": float(np.max(np.abs(lg_ref - lg0))),
        "first_step_gpu_at_most_reference_distance": bool(
            diff.max() <= np.max(np.abs(lg_ref.astype(np.float64) - lg0))),
        "first_step_top2_margin": O.top2_margin(lg0),
        "first_step_gpu_vs_textbook_max_abs": float(np.max(np.abs(gpu_logits0 - lg_text))),
        "first_step_mirrored_vs_textbook_max_abs": float(np.max(np.abs(lg0 - lg_text))),
        "first_step_logit_rms": float(np.sqrt(np.mean(lg_text.astype(np.float64) ** 2))),
    }
    return base, check


def chunk_gemm_times(wk, shapes, n: int = 256, reps: int = 50) -> dict:
    """HIP-event time of each chunk GEMM form over n tokens (weights packed on
    the device, x f16 N(0,1)): name -> (us per call, TFLOP/s counted)."""
    from whetstone_amd import ffi
    out = {}
    for name, (kind, in_f, rows) in shapes.items():
        qw = wk.DeviceBuffer(rows * in_f // 8, np.uint32)
        si = wk.DeviceBuffer(rows * in_f // 32, np.uint8)
        sb = wk.DeviceBuffer(rows, np.uint32)
        ffi.call("wst_fixture_pack_hier", qw.ptr, si.ptr, sb.ptr, in_f, 0, rows, WEIGHT_SEED, 7, 0.02)
        x = wk.DeviceBuffer(n * in_f, np.float16)
        ffi.call("wst_fixture_normal_f16", x.ptr, n * in_f, KV_SEED, 8, 0, 1.0, 0.0)
        y = wk.DeviceBuffer(n * rows, np.float32)
        if kind == "swiglu":
            fn = lambda: ffi.call("wst_gemm_hier_swiglu_chunk", qw.ptr, si.ptr, sb.ptr, x.ptr, y.ptr,
                                  in_f, rows // 2, n)
        else:
            fn = lambda: ffi.call("wst_gemm_int4_hier", qw.ptr, si.ptr, sb.ptr, x.ptr, None, y.ptr,
                                  in_f, rows, n, 1)
        for _ in range(5):
            fn()
        e0, e1 = wk.Event(), wk.Event()
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        wk.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / reps
        out[name] = {"us": round(us, 2), "tflops": round(2 * n * in_f * rows / us / 1e6, 1)}
        del qw, si, sb, x, y
    return out


def prefill_bench(E, wk, n_new: int, gemm_7b: bool = False, gemms: bool = True,
                  emit: bool = True, batched_only: bool = False) -> dict:
    """Config 4: chunked prefill of 4096 tokens (256 per chunk), then n_new
    graph decode steps (none, and no graph capture, for n_new = 0)."""
    cfg = dict(E.QWEN05B, qk_norm=1, rescore_k=32)
    n_prompt, chunk = 4096, 256
    g = E.Model(cfg, seed=WEIGHT_SEED)
    eng = E.Engine(g, n_prompt + n_new + 8)
    ids = np.random.default_rng(PROMPT_SEED).integers(0, cfg["vocab"], n_prompt).astype(np.int32)
    def timed_prefill(batch: bool) -> float:
        # The full chunks share each layer's launches, each planned for all
        # its tokens, unless batch is off (WSE_CHUNK_BATCH=0: one launch per
        # chunk and op). A warm-up prefill first (kernels, buffers, split
        # scratch), then rewind.
        os.environ["WSE_CHUNK_BATCH"] = "1" if batch else "0"
        try:
            eng.set_pos(0)
            eng.prefill(ids, chunked=True)
            eng.set_pos(0)
            wk.synchronize()
            t0 = time.perf_counter()
            eng.prefill(ids, chunked=True)
            wk.synchronize()
            return time.perf_counter() - t0
        finally:
            os.environ.pop("WSE_CHUNK_BATCH", None)

    log(f"prefill {n_prompt} tokens in {chunk}-token chunks, one launch per chunk and op")
    dt_1 = None if batched_only else timed_prefill(False)
    log(f"prefill {n_prompt} tokens in {chunk}-token chunks, the full chunks batched per op")
    dt_p = timed_prefill(True)
    # FLOPs: every layer GEMM on every token (2 per weight), the causal
    # attention (q.k and p.v: 2 * 2 * head_dim per (head, cached position)),
    # and the head on the last token only.
    H, I, hd, nq, nkv, L = (cfg[k] for k in ("hidden", "inter", "head_dim", "n_q", "n_kv",
                                               "n_layers"))
    w_layer = H * (nq + 2 * nkv) * hd + nq * hd * H + H * 2 * I + I * H
    attn = 2 * 2 * hd * nq * n_prompt * (n_prompt + 1) // 2
    flops = L * (2 * w_layer * n_prompt + attn) + 2 * cfg["vocab"] * H
    dt_d = None
    if n_new > 0:
        log("capturing the decode graph")
        eng.capture_graph()
        for _ in range(8):
            eng.step()
            eng.token()
        eng.set_pos(n_prompt)
        wk.synchronize()
        t0 = time.perf_counter()
        for _ in range(n_new):
            eng.step()
            eng.token()
        wk.synchronize()
        dt_d = time.perf_counter() - t0
    shapes = {"0.5b gate_up+swiglu": ("swiglu", H, 2 * I), "0.5b down": ("gemm", I, H),
              "0.5b qkv": ("gemm", H, (nq + 2 * nkv) * hd), "0.5b o": ("gemm", nq * hd, H)}
    if gemm_7b:
        c7 = E.QWEN7B
        H7, I7 = c7["hidden"], c7["inter"]
        shapes.update({"7b gate_up+swiglu": ("swiglu", H7, 2 * I7), "7b down": ("gemm", I7, H7),
                       "7b qkv": ("gemm", H7, (c7["n_q"] + 2 * c7["n_kv"]) * c7["head_dim"]),
                       "7b o": ("gemm", c7["n_q"] * c7["head_dim"], H7)})
    gemms = chunk_gemm_times(wk, shapes, chunk) if gemms else None
    line = {
        "metric": "chunked prefill tok/s (config 4)", "value": round(n_prompt / dt_p, 1),
        "unit": "tok/s", "n_gpus": 1, "higher_is_better": True, "dtype": "int4xf16->f32",
        "data": "synthetic (seeded N(0,0.02) weights packed to int4-hier-g32 on the device; "
                "seeded random prompt)",
        "config": {"workload": f"config 4: Qwen2.5-0.5B-shape (QK-norm, head rescore top-32) "
                               f"chunked prefill of {n_prompt} tokens in {chunk}-token chunks, "
                               f"then {n_new} greedy decode steps",
                   "prefill_ms": round(dt_p * 1e3, 2),
                   "prefill_tflops": round(flops / dt_p / 1e12, 2),
                   "batched": f"each layer's op runs for all {n_prompt // chunk} chunks in "
                              "one launch, its GEMMs planned for all the tokens (f32 sums "
                              "within rounding of one launch per chunk)",
                   "prefill_tok_s_one_launch_per_chunk": round(n_prompt / dt_1, 1) if dt_1 else None,
                   "prefill_ms_one_launch_per_chunk": round(dt_1 * 1e3, 2) if dt_1 else None,
                   "prefill_flops": flops,
                   "decode_steps": n_new,
                   "decode_tok_s": round(n_new / dt_d, 1) if dt_d else None,
                   "chunk_gemms_256_tokens": gemms},
    }
    eng.close()
    g.close()
    if emit:
        print(json.dumps(line), flush=True)
    return line


def decode_05b(E, wk, n_prompt: int = 512, n_new: int = 256, warmup: int = 8) -> dict:
    """Config 2: the 0.5B shape, a seeded n_prompt-token chunked prefill, then
    n_new graph steps (one replay and a 4-byte token read-back each)."""
    cfg = E.QWEN05B
    g = E.Model(cfg, seed=WEIGHT_SEED)
    eng = E.Engine(g, n_prompt + n_new + 8)
    prompt = np.random.default_rng(PROMPT_SEED).integers(0, cfg["vocab"], n_prompt)
    eng.prefill(prompt.astype(np.int32), chunked=True)
    eng.capture_graph()
    tok0 = eng.token()
    for _ in range(warmup):
        eng.step()
        eng.token()
    eng.set_pos(n_prompt)
    eng.set_token(tok0)
    wk.synchronize()
    t0 = time.perf_counter()
    for _ in range(n_new):
        eng.step()
        eng.token()
    wk.synchronize()
    dt = time.perf_counter() - t0
    bts = []
    for i in range(n_new):
        eng.set_pos(n_prompt + i)
        bts.append(eng.step_bytes())
    eng.close()
    g.close()
    b = float(np.mean(bts))
    tok_s = n_new / dt
    return {"workload": f"config 2: 0.5B-shape decode, {n_prompt}-token chunked prefill, "
                        f"context {n_prompt} -> {n_prompt + n_new}, captured graph",
            "tok_s": round(tok_s, 1), "ms_per_token": round(dt / n_new * 1e3, 4),
            "bytes_per_token": int(b), "hbm_gbs": round(b * tok_s / 1e9, 1),
            "frac_of_hbm_peak": round(b * tok_s / 1e9 / HBM_PEAK_GBS, 4),
            "token_roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / b, 1)}


def secondary_configs(E, wk) -> dict:
    """Configs 2, 4 and 1 at their own workloads, each measured once after the
    headline's timed region (nothing here is inside it)."""
    out = {}
    log("secondary: config 2 (0.5B decode after a 512-token prefill, 256 steps)")
    out["config2"] = decode_05b(E, wk)
    log("secondary: config 4 (4096-token chunked prefill, then 128 decode steps)")
    p = prefill_bench(E, wk, 128, gemms=False, emit=False)
    c = p["config"]
    out["config4"] = {"workload": c["workload"], "prefill_tok_s": p["value"],
                      "prefill_ms": c["prefill_ms"], "prefill_tflops": c["prefill_tflops"],
                      "prefill_tok_s_one_launch_per_chunk": c["prefill_tok_s_one_launch_per_chunk"],
                      "decode_tok_s": c["decode_tok_s"]}
    log("secondary: config 1 (lm_head GEMV 896 -> 151936, weights cold)")
    h = gemv_bench(wk, 200, head_only=True, emit=False)["config"]["shapes"]["lm_head"]
    out["config1"] = {"workload": "config 1: int4-hier GEMV 896 -> 151936, weights cold past "
                                  "the MALL", "us_per_call": h["cold"]["us_per_call"],
                      "gbs": h["cold"]["gbs"], "frac_of_hbm_peak": h["cold"]["frac"],
                      "stream_read_floor_us": h["stream_read_floor_cold"]["us_per_call"],
                      "gemv_frac_of_floor": h["gemv_frac_of_floor"]}
    return out


def floors_bench(E, wk, config: int, reps: int) -> None:
    """The floor of the decode step's launch structure: a captured graph with
    one launch per kernel of the fused step (per layer: norm+qkv, attention
    slices, slice merge, o, norm+gate|up+SwiGLU, down; then the head, the
    argmax over its blocks' keys, and the embedding row), each launch replaced by the library's
    plain streaming read (wst_stream_read) of that kernel's algorithmic bytes
    from its own buffer (so the weights stream cold, as in the step); and a
    graph of the same number of minimal launches (16 bytes each), which is
    the cost of the dependent launches alone. (With a cache of at most 8
    attention slices the o GEMV merges them, and there is no merge launch.)
    Prints one JSON line."""
    from whetstone_amd import ffi
    cfg = E.QWEN7B if config == 3 else E.QWEN05B
    H, I, hd, nq, nkv, L, V = (cfg[k] for k in ("hidden", "inter", "head_dim", "n_q", "n_kv",
                                                 "n_layers", "vocab"))
    ctx = 2048 + 128 if config == 3 else 512 + 128
    row = lambda in_f: in_f // 2 + in_f // 32 + 4
    nqkv = (nq + 2 * nkv) * hd
    stage_bytes = {
        "qkv": nqkv * row(H) + H * 6 + nqkv * 6,
        "attn": 2 * nkv * ctx * hd * 2 + nqkv * 4,
        "merge": nq * -(-ctx // (16384 // hd)) * (hd + 2) * 4 + nq * hd * 2,
        "o": H * row(nq * hd) + nq * hd * 2 + H * 8,
        "gate_up": 2 * I * row(H) + H * 6 + I * 2,
        "down": H * row(I) + I * 2 + H * 8,
    }
    if ctx + 136 <= 8 * (16384 // hd):  # short caches: the o GEMV merges the slices itself
        stage_bytes["o"] += stage_bytes.pop("merge") - nq * hd * 2
    head_bytes = V * row(H) + H * 8 + V * 4
    per_layer = [(k, -(-b // 256) * 256) for k, b in stage_bytes.items()]
    keys_bytes = 4096  # the argmax finish: one 8-byte key per head block
    total = sum(b for _, b in per_layer) * L + head_bytes + keys_bytes + H * 4
    buf = wk.DeviceBuffer(total + 4096, np.uint8)
    ffi.call("wst_memset", buf.ptr, 1, total + 4096)
    sink = wk.DeviceBuffer(4, np.float32)
    base = buf.ptr.value
    launches = []
    off = 0
    for _ in range(L):
        for k, b in per_layer:
            launches.append((off, b))
            off += b
    launches.append((off, -(-head_bytes // 256) * 256))
    off += launches[-1][1]
    launches.append((off, keys_bytes))  # the argmax over the head blocks' keys
    off += keys_bytes
    launches.append((off, H * 4))  # the next step's embedding row
    wk.synchronize()

    def run(graph_fn, n_rep):
        g = wk.Graph.capture(graph_fn)
        for _ in range(3):
            g.launch()
        wk.synchronize()
        t0 = time.perf_counter()
        for _ in range(n_rep):
            g.launch()
        wk.synchronize()
        dt = (time.perf_counter() - t0) / n_rep
        g.close()
        return dt

    def stream_graph():
        for o, b in launches:
            ffi.call("wst_stream_read", base + o, b, sink.ptr)

    def empty_graph():
        for _ in launches:
            ffi.call("wst_stream_read", base, 16, sink.ptr)

    t_stream = run(stream_graph, reps)
    t_empty = run(empty_graph, reps)
    n = len(launches)
    line = {
        "metric": f"decode-step launch-structure floors (config {config})",
        "value": round(1.0 / t_stream, 1), "unit": "tok/s", "n_gpus": 1,
        "higher_is_better": True, "data": "synthetic (streaming reads of each kernel's bytes)",
        "config": {"workload": f"config {config}: {n} dependent launches per token "
                               f"({L} layers x {len(per_layer)} + head + argmax + embedding), context "
                               f"{ctx}, as one captured graph",
                   "bytes_per_token": total,
                   "stream_graph_us_per_token": round(t_stream * 1e6, 1),
                   "stream_graph_gbs": round(total / t_stream / 1e9, 1),
                   "empty_graph_us_per_token": round(t_empty * 1e6, 1),
                   "empty_graph_us_per_launch": round(t_empty * 1e6 / n, 3),
                   "hbm_time_at_8tbs_us": round(total / HBM_PEAK_GBS / 1e3, 1),
                   "launches": n, "reps": reps},
    }
    print(json.dumps(line), flush=True)


def cpu_reference_bench(E, wk) -> None:
    """Config 0: the CPU reference path. The 0.5B shape with seeded weights
    (packed on the device, copied to the oracle), a seeded 16-token prompt,
    32 greedy tokens through oracle/oracle.c's precision-mirrored forward on
    the host's OpenMP threads (dequant on the fly, f64 dot products); the
    same prompt through the GPU engine beside it, tokens compared. The value
    is the CPU's tok/s over prompt + generation, as the reference quotes its
    CPU path; the GPU's figure for the same run is in `config`."""
    from oracle import oracle as O
    cfg = E.QWEN05B
    n_prompt, n_new = 16, 32
    g = E.Model(cfg, seed=WEIGHT_SEED)
    ids = np.random.default_rng(PROMPT_SEED).integers(0, cfg["vocab"], n_prompt).astype(np.int32)
    eng = E.Engine(g, n_prompt + n_new + 8)
    eng.generate(ids, 4, chunked=False)  # warm-up
    eng.reset()
    wk.synchronize()
    t0 = time.perf_counter()
    gpu = [int(t) for t in eng.generate(ids, n_new, chunked=False)]
    wk.synchronize()
    gpu_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    o = O.Model(cfg, WEIGHT_SEED, pack=False)
    copy_model_to_oracle(g, o, cfg)
    st = O.State(o, n_prompt + n_new + 8, 0)
    setup_s = time.perf_counter() - t0
    log(f"config 0: CPU path, {n_prompt} prompt + {n_new} greedy tokens")
    t0 = time.perf_counter()
    nxt = None
    for t in ids:
        nxt, _ = st.step(int(t))
    cpu = []
    for _ in range(n_new):
        cpu.append(int(nxt))
        nxt, _ = st.step(int(nxt))
    cpu_s = time.perf_counter() - t0
    st.close()
    # the faithful form of the reference's CPU forward (reference_numpy.py:
    # every token recomputes the whole sequence, f64, no KV cache): one call
    # at the final length, the cost of the last generated token
    t0 = time.perf_counter()
    full = o.forward_full(np.concatenate([ids, np.asarray(cpu, np.int32)]))
    faithful_s = time.perf_counter() - t0
    o.close()
    eng.close()
    g.close()
    steps = n_prompt + n_new
    line = {
        "metric": "CPU reference path tok/s (config 0: Qwen2.5-0.5B shape, 16-token prompt, "
                  "32 greedy tokens)",
        "value": round(steps / cpu_s, 3), "unit": "tok/s", "n_gpus": 1,
        "higher_is_better": True, "dtype": "f32 dequant, f64 dot products",
        "data": "synthetic (seeded N(0,0.02) weights packed to int4-hier-g32; seeded prompt)",
        "config": {"workload": "config 0: oracle/oracle.c mirrored forward, one token at a time "
                               "with a KV cache, on the host; the GPU engine on the same weights",
                   "cores": int(O.lib().orc_threads()), "cpu_seconds": round(cpu_s, 3),
                   "setup_seconds_not_timed": round(setup_s, 2),
                   "gpu_tok_s_same_run": round(steps / gpu_s, 1),
                   "faithful_full_recompute_s_per_token_at_48": round(faithful_s, 3),
                   "faithful_argmax_equals_last_cpu_token": bool(int(np.argmax(full)) == int(nxt)),
                   "tokens_compared": n_new,
                   "tokens_identical": int(sum(a == b for a, b in zip(cpu, gpu)))},
    }
    print(json.dumps(line), flush=True)


def gemv_bench(wk, reps: int, head_only: bool = False, emit: bool = True) -> dict:
    """Config 1: the int4-hier-g32 GEMV alone, y f32 = W x (x f16 N(0,1), W
    N(0,0.02) packed on the device), on the 0.5B lm_head shape and the 0.5B
    block shapes. "cold" cycles through ceil(512 MB / matrix bytes) distinct
    copies so the 256 MB MALL cannot serve the weights; "hot" repeats one copy.
    HIP events on the calling thread's stream around `reps` back-to-back
    launches; bytes per call = packed weights + x + y."""
    from whetstone_amd import ffi
    shapes = [("lm_head", 896, 151936), ("qkv", 896, 1152), ("gate_up", 896, 9728),
              ("down", 4864, 896)]
    if head_only:
        shapes = shapes[:1]
    res = {}
    for name, in_f, out_f in shapes:
        wbytes = out_f * (in_f // 2 + in_f // 32 + 4)
        nbytes = wbytes + 2 * in_f + 4 * out_f
        copies = max(1, -(-512_000_000 // wbytes))
        qw = wk.DeviceBuffer(copies * out_f * in_f // 2, np.uint8)
        si = wk.DeviceBuffer(copies * out_f * in_f // 32, np.uint8)
        sb = wk.DeviceBuffer(copies * out_f * 4, np.uint8)
        base = (qw.ptr.value, si.ptr.value, sb.ptr.value)
        ptrs = [(base[0] + c * out_f * in_f // 2, base[1] + c * out_f * in_f // 32,
                 base[2] + c * out_f * 4) for c in range(copies)]
        for (q, i_, b) in ptrs:
            ffi.call("wst_fixture_pack_hier", q, i_, b, in_f, 0, out_f, WEIGHT_SEED, 1, 0.02)
        x = wk.DeviceBuffer(in_f, np.float16)
        ffi.call("wst_fixture_normal_f16", x.ptr, in_f, KV_SEED, 2, 0, 1.0, 0.0)
        y = wk.DeviceBuffer(out_f, np.float32)
        out = {"in": in_f, "out": out_f, "bytes_per_call": nbytes, "cold_copies": copies}
        for mode in ("cold", "hot"):
            seq = ptrs if mode == "cold" else ptrs[:1]
            for k in range(10):
                q, i_, b = seq[k % len(seq)]
                ffi.call("wst_gemv_int4_hier_ex", q, i_, b, x.ptr, None, y.ptr, in_f, out_f, 0)
            e0, e1 = wk.Event(), wk.Event()
            e0.record()
            for k in range(reps):
                q, i_, b = seq[k % len(seq)]
                ffi.call("wst_gemv_int4_hier_ex", q, i_, b, x.ptr, None, y.ptr, in_f, out_f, 0)
            e1.record()
            wk.synchronize()
            us = e0.elapsed_ms(e1) * 1e3 / reps
            out[mode] = {"us_per_call": round(us, 3), "gbs": round(nbytes / us / 1e3, 1),
                         "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
        if name == "lm_head":
            # the floor: the library's streaming read of the same bytes per
            # call, cycling through as many distinct copies (weights cold)
            buf = wk.DeviceBuffer(copies * nbytes, np.uint8)
            ffi.call("wst_memset", buf.ptr, 1, copies * nbytes)
            sink = wk.DeviceBuffer(4, np.float32)
            for k in range(10):
                ffi.call("wst_stream_read", buf.ptr.value + (k % copies) * nbytes, nbytes, sink.ptr)
            e0, e1 = wk.Event(), wk.Event()
            e0.record()
            for k in range(reps):
                ffi.call("wst_stream_read", buf.ptr.value + (k % copies) * nbytes, nbytes, sink.ptr)
            e1.record()
            wk.synchronize()
            us = e0.elapsed_ms(e1) * 1e3 / reps
            out["stream_read_floor_cold"] = {"us_per_call": round(us, 3),
                                             "gbs": round(nbytes / us / 1e3, 1),
                                             "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
            out["gemv_frac_of_floor"] = round(us / out["cold"]["us_per_call"], 4)
            del buf
        log(f"{name}: {out}")
        res[name] = out
        del qw, si, sb
    head = res["lm_head"]["cold"]
    line = {
        "metric": "int4 hier-g32 GEMV achieved HBM GB/s (config 1: lm_head 896 -> 151936)",
        "value": head["gbs"], "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "int4xf16->f32",
        "data": "synthetic (seeded N(0,0.02) weights packed to int4-hier-g32 on the device; "
                "f16 N(0,1) x)",
        "config": {"workload": "config 1: single int4 hier-g32 GEMV, y[151936] = W x[896], "
                               "plus the 0.5B block shapes; cold = distinct weight copies "
                               "cycling past the MALL", "reps": reps, "shapes": res},
        "roofline": {"bound": "hbm", "achieved": head["gbs"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": head["frac"],
                     "traffic": traffic_for(1, "lm_head", GEMV_TRAFFIC_FILE)},
    }
    if emit:
        print(json.dumps(line), flush=True)
    return line


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {a.gpus} is not supported "
              "(multi-GPU sharding is designed, not built)", file=sys.stderr)
        sys.exit(2)
    if a.summarize:
        summarize(a.summarize, a.calibration, a.copy_probe or 256)
        return
    if a.copy_probe:
        copy_probe(a.copy_probe)
        return
    if (a.steps <= 0 and not (a.config == 4 and a.steps == 0)) or a.warmup < 0:
        sys.exit("bench.py: --steps must be positive (0 allowed with --config 4: prefill only) "
                 "and --warmup non-negative")

    from whetstone_amd import engine as E, kernels as wk  # raises if not built
    if a.config == 0:
        cpu_reference_bench(E, wk)
        return
    if a.config == 1:
        gemv_bench(wk, max(a.steps, 200))
        return
    if a.config == 4:
        prefill_bench(E, wk, a.steps, a.gemm_7b, batched_only=a.batched_only)
        return
    if a.floors:
        floors_bench(E, wk, a.config, max(a.steps, 20))
        return
    cfg = E.QWEN7B if a.config == 3 else E.QWEN05B
    t_gen = time.perf_counter()
    g = E.Model(cfg, seed=WEIGHT_SEED)
    wk.synchronize()
    t_gen = time.perf_counter() - t_gen

    ms_need = None
    if a.config == 3:
        ctx0 = 2048
        # the configuration's cache: context 2048 -> 2304 (the reference CLI's
        # max(ctx, prompt + max_new + 1), run.rs:103), or longer for more steps
        ms_need = ctx0 + max(a.steps, a.warmup, FULL_RANGE) + 8
        eng = E.Engine(g, max(a.max_seq, ms_need))
        eng.fill_kv(KV_SEED, ctx0)
        workload = ("config 3: Qwen2.5-7B-shape int4 hier-g32 batch=1 greedy decode, "
                    f"KV context {ctx0} -> {ctx0 + a.steps}")
    else:
        ctx0 = 512
        ms_need = ctx0 + max(a.steps, a.warmup) + 8
        eng = E.Engine(g, max(a.max_seq, ms_need))
        prompt = np.random.default_rng(PROMPT_SEED).integers(0, cfg["vocab"], ctx0)
        eng.prefill(prompt.astype(np.int32), chunked=True)
        workload = ("config 2: Qwen2.5-0.5B-shape int4 hier-g32 batch=1 greedy decode after a "
                    f"{ctx0}-token chunked prefill, context {ctx0} -> {ctx0 + a.steps}")
    log(f"model ready ({t_gen:.2f}s), context {ctx0}; "
        + ("eager steps" if a.no_graph else "capturing the step graph"))
    if not a.no_graph:
        eng.capture_graph()  # warm-up step + rewind inside
    log("graph captured; warm-up")
    tok0 = eng.token()
    for _ in range(a.warmup):
        eng.step()
        eng.token()
    eng.set_pos(ctx0)
    eng.forward(tok0)  # the first timed step's inputs again, eagerly, for the logits check
    logits0 = eng.logits()
    eng.set_pos(ctx0)
    eng.set_token(tok0)

    log(f"timing {a.steps} steps")
    bytes_steps = []
    tokens = []
    wk.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        eng.step()
        tokens.append(eng.token())
    wk.synchronize()
    dt = time.perf_counter() - t0
    # bytes of each timed step (position ctx0 + i reads ctx0 + i + 1 cached rows)
    for i in range(a.steps):
        eng.set_pos(ctx0 + i)
        bytes_steps.append(eng.step_bytes())
    bytes_tok = float(np.mean(bytes_steps))
    full = None
    if a.config == 3 and a.steps != FULL_RANGE and not a.no_full_range:
        # the configuration's whole range, 2048 -> 2304, outside the timed region
        eng.set_pos(ctx0)
        eng.set_token(tok0)
        wk.synchronize()
        t1 = time.perf_counter()
        for _ in range(FULL_RANGE):
            eng.step()
            eng.token()
        wk.synchronize()
        full = round(FULL_RANGE / (time.perf_counter() - t1), 2)

    log(f"{a.steps / dt:.1f} tok/s; timing each stage kernel")
    # Per-kernel timing at the middle of the timed context range.
    eng.set_pos(ctx0 + a.steps // 2)
    kernels = {}
    launches = {"head": 1}
    for s in TIMED_STAGES:
        us, b = eng.time_stage(s, a.stage_reps)
        n = launches.get(s, cfg["n_layers"])
        kernels[s] = {"kernel": KERNEL_NAMES[s], "us_per_launch": round(us, 3),
                      "bytes_per_launch": b, "gbs": round(b / us / 1e3, 1),
                      "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4),
                      "launches_per_token": n, "us_per_token": round(us * n, 1)}
    dom = max(kernels, key=lambda s: kernels[s]["us_per_token"])
    k = kernels[dom]
    roofline = {"bound": "hbm", "kernel": f"{dom}: {k['kernel']}", "achieved": k["gbs"],
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": k["frac"],
                "traffic": traffic_for(a.config, dom)}

    tok_s = a.steps / dt
    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(dt / a.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xf16->f32",
        "data": "synthetic (seeded N(0,0.02) weights packed to int4-hier-g32 on the device; "
                + ("seeded f16 N(0,1) KV context)" if a.config == 3 else "seeded random prompt)"),
        "config": {"workload": workload, "bytes_per_token": int(bytes_tok),
                   "max_seq": max(a.max_seq, ms_need),
                   "hbm_gbs": round(bytes_tok * tok_s / 1e9, 1),
                   "frac_of_hbm_peak": round(bytes_tok * tok_s / 1e9 / HBM_PEAK_GBS, 4),
                   "token_roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / bytes_tok, 1),
                   "graph": not a.no_graph, "weights_generated_s": round(t_gen, 2)},
        "roofline": roofline,
        "kernels": kernels,
    }
    if full is not None:
        line["config"]["full_range_tok_s"] = full
    if a.no_cpu:
        line["cpu_baseline"] = None
    else:
        log("CPU baseline (oracle) on the same weights")
        base, check = cpu_leg(g, cfg, ctx0, tok0, tokens, logits0, a.cpu_seconds,
                              same_context=a.config == 3)
        line["cpu_baseline"] = base
        line["cpu_check"] = check
    eng.close()
    g.close()
    if a.config == 3 and not a.no_secondary:
        line["secondary"] = secondary_configs(E, wk)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
