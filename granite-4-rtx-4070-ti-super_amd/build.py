"""Builds libgranite4_layerops.so (gfx950) in-tree with hipcc.

    python granite-4-rtx-4070-ti-super_amd/build.py [--jobs N]

Each csrc/*.hip is compiled to an object under _build/, then linked into
lib/libgranite4_layerops.so next to this file. Compile flags that matter for
parity: -ffp-contract=off (no silent a*b+c fusion: the reference's host math
rounds every product), -fhip-fp32-correctly-rounded-divide-sqrt (IEEE f32
division and square root), and packed-FP32 instructions disabled.
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIBDIR, "libgranite4_layerops.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIPFLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++20", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    "-I", CSRC, "-I", os.path.join(ROOT, "include"),
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cc")))


# Host-only sources (.cc: the KV page-table controller) build with the host
# compiler; they hold no device code.
CXX = os.environ.get("CXX", "g++")
CXXFLAGS = ["-O2", "-std=c++20", "-fPIC", "-Wall", "-I", os.path.join(ROOT, "include")]


def compile_one(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if src.endswith(".cc"):
        cmd = [CXX, *CXXFLAGS, "-c", src, "-o", obj]
    else:
        cmd = [HIPCC, *HIPFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(jobs=8, verbose=True, out=LIB):
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(os.path.dirname(out), exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = out + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print("built", out)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--out", default=LIB, help="output library path")
    ap.add_argument("--define", action="append", default=[],
                    help="extra preprocessor definition (measurement builds, e.g. G4_TRACE_FP8)")
    ap.add_argument("--build-dir", default=None, help="object directory (default _build/)")
    a = ap.parse_args()
    HIPFLAGS += [f"-D{d}" for d in a.define]
    if a.build_dir:
        BUILD = os.path.abspath(a.build_dir)
    try:
        build(a.jobs, out=os.path.abspath(a.out))
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
