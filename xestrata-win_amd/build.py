"""Build libxsmoe.so (the HIP kernels and the C ABI of include/xs_moe.h) in-tree for gfx950.

    python xestrata-win_amd/build.py [-j N]

Every translation unit is compiled by hipcc with -ffp-contract=off (the canonical arithmetic's products and sums must
round on their own) and with packed fp32 instructions disabled; objects go to xestrata-win_amd/_build/, the shared
library next to this file.  No GPU is needed: hipcc cross-compiles for gfx950.
"""
import argparse
import concurrent.futures
import os
import pathlib
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libxsmoe.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-but-set-variable",
]
SOURCES = ["formats.hip", "quant_act.hip", "experts_decode.hip", "experts_stream.hip", "experts_prefill.hip", "router.hip", "dispatch.hip",
           "combine.hip", "decode_layer.hip", "decode_fused.hip", "decode_t1.hip", "tiers.hip", "noalloc.hip", "mmq.hip", "gemv.hip", "peaks.hip",
           "abi.cpp", "pack.cpp"]


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD / (src.stem + ".o")
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [HIPCC, *FLAGS, *lang, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(jobs: int = 8) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    srcs = [CSRC / s for s in SOURCES]
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=min(8, os.cpu_count() or 1))
    args = ap.parse_args()
    try:
        print(build(args.j))
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
