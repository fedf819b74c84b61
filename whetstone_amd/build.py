"""Builds the native libraries in-tree with hipcc for gfx950.

    python -m whetstone_amd.build          # compile everything
    python -m whetstone_amd.build --check  # compile, and fail on warnings

Outputs (git-ignored, shipped to the GPU box with the tree):
    whetstone_amd/lib/libwhetstone_hip.so     the C ABI (include/whetstone.h)
    whetstone_amd/lib/libwhetstone_engine.so  the C++ decode engine
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OUT = PKG / "lib"
OBJ = ROOT / "_build" / "obj"

ARCH = os.environ.get("WHETSTONE_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # All launches go to the calling thread's per-thread default stream, as the
    # reference's --default-stream=per-thread (build.rs:494-499).
    "-fgpu-default-stream=per-thread",
    # Packed FP32 ops stay off: plain f32 code only.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]

LIB_SOURCES = [
    "runtime.hip",
    "gemv_hier.hip",
    "decode.hip",
    "attention.hip",
    "sample.hip",
    "head_rescore.hip",
    "fixture.hip",
    "embed_fp16.hip",
    "gemm.hip",
    "chunk.hip",
    "stubs.hip",
]
ENGINE_SOURCES = ["engine.cpp", "wstone.cpp", "speculate.cpp", "sampler.cpp"]

# Per-file code-generation flags. chunk.hip: MFMA accumulators in VGPRs (the
# chunk attention's online softmax rescales and reads them between MFMAs; in
# AGPRs each tile paid ~40 accvgpr moves).
FILE_FLAGS = {"chunk.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    return p


# The engine is plain host C++ that reaches the GPU only through the C ABI.
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{INCLUDE}"]


def _compile(src: Path, obj: Path, extra: list[str]) -> tuple[Path, str]:
    obj.parent.mkdir(parents=True, exist_ok=True)
    if src.suffix == ".cpp":
        cmd = [shutil.which("g++") or "g++", *CXX_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [hipcc(), *HIP_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that note is
    # expected and harmless.
    err = "\n".join(l for l in (r.stderr or "").splitlines()
                    if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{err}")
    return obj, err


def build(verbose: bool = True, jobs: int | None = None) -> dict[str, Path]:
    """Compiles every HIP/C++ source and links the two shared libraries."""
    OUT.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    lib_srcs = [CSRC / s for s in LIB_SOURCES if (CSRC / s).exists()]
    eng_srcs = [CSRC / s for s in ENGINE_SOURCES if (CSRC / s).exists()]
    warnings: list[str] = []
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = {ex.submit(_compile, s, OBJ / (s.stem + ".o"), FILE_FLAGS.get(s.name, [])): s
                for s in lib_srcs + eng_srcs}
        objs = {}
        for f in cf.as_completed(futs):
            obj, err = f.result()
            objs[futs[f]] = obj
            if err.strip():
                warnings.append(f"{futs[f].name}:\n{err}")
    lib = OUT / "libwhetstone_hip.so"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(lib),
           *[str(objs[s]) for s in lib_srcs]]
    subprocess.run(cmd, check=True)
    out = {"hip": lib}
    if eng_srcs:
        eng = OUT / "libwhetstone_engine.so"
        cmd = [shutil.which("g++") or "g++", "-shared", "-fPIC", "-o", str(eng),
               *[str(objs[s]) for s in eng_srcs], f"-L{OUT}", "-lwhetstone_hip",
               "-Wl,-rpath,$ORIGIN"]
        subprocess.run(cmd, check=True)
        out["engine"] = eng
    if verbose:
        for w in warnings:
            print(w, file=sys.stderr)
        for k, v in out.items():
            print(f"built {k}: {v.relative_to(ROOT)}")
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--check", action="store_true", help="fail on compiler warnings")
    a = ap.parse_args(argv)
    build()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
