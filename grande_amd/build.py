"""Builds grande_amd/libomg_hip.so: the gfx950 kernels and the C++ engine
behind include/omg_hip.h, compiled with hipcc in-tree.

    python -m grande_amd.build            # incremental
    python -m grande_amd.build --force    # rebuild every object
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libomg_hip.so"
INCLUDE = PKG.parent / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result", f"-I{INCLUDE}"]
# Device code never uses packed-FP32 VALU instructions.
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

SOURCES = ["gemm.hip", "attention.hip", "norm.hip", "laya.hip", "model.cpp", "gguf.cpp", "state.cpp", "engine.cpp", "laya.cpp", "capi.cpp"]
# Per-file device flags.  The GEMM and attention kernels keep their MFMA
# accumulators in ordinary VGPRs: with the AGPR form the register allocator
# shuffles them between loop iterations (v_accvgpr moves in the main loop).
EXTRA = {name: ["-mllvm", "-amdgpu-mfma-vgpr-form"] for name in ("gemm.hip", "attention.hip", "laya.hip")}
HEADERS = sorted(CSRC.glob("*.h")) + [INCLUDE / "omg_hip.h"]


def _compile(src: Path, force: bool) -> Path:
    obj = OBJ / (src.name + ".o")
    newest_dep = max([src.stat().st_mtime] + [h.stat().st_mtime for h in HEADERS])
    if not force and obj.exists() and obj.stat().st_mtime >= newest_dep:
        return obj
    flags = COMMON + (DEVICE if src.suffix == ".hip" else [f"--offload-arch={ARCH}"]) + EXTRA.get(src.name, [])
    cmd = [HIPCC, *flags, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed on {src.name}")
    return obj


def build(force: bool = False, verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = [CSRC / s for s in SOURCES]
    with ThreadPoolExecutor(max_workers=min(len(srcs), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), srcs))
    if force or not LIB.exists() or LIB.stat().st_mtime < max(o.stat().st_mtime for o in objs):
        tmp = LIB.with_suffix(".so.tmp")
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            sys.stderr.write(res.stdout + res.stderr)
            raise RuntimeError("hipcc link failed")
        os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    a = ap.parse_args()
    build(force=a.force, verbose=True)
