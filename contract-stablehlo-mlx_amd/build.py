"""Build libshlo_hip.so (and the shlo_hip CLI) for gfx950, in-tree.

    python contract-stablehlo-mlx_amd/build.py [-j N]

Every .hip and .cpp under csrc/ (except the gen_* table generators) is
compiled with hipcc for gfx950 and linked into shlo_hip/libshlo_hip.so; the
CLI csrc/cli/shlo_hip_main.cpp links against it as shlo_hip/shlo_hip.

Floating-point flags that the bit-exact kernels rely on:
  -ffp-contract=off                  only explicit fma() fuses
  -fno-gpu-flush-denormals-to-zero   binary32 subnormals are kept (arm64 FPCR.FZ=0)
  -fhip-fp32-correctly-rounded-divide-sqrt
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed FP32 instructions
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "shlo_hip")
OBJ_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libshlo_hip.so")
CLI = os.path.join(OUT_DIR, "shlo_hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17",
    "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument", "-Wno-unknown-warning-option",
    "-Wno-unused-function",
    "-I" + CSRC, "-I" + os.path.join(os.path.dirname(HERE), "include"),
]


def sources():
    out = []
    for f in sorted(os.listdir(CSRC)):
        if f.startswith("gen_"):
            continue
        if f.endswith(".hip") or f.endswith(".cpp"):
            out.append(os.path.join(CSRC, f))
    return out


def compile_one(src):
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC] + COMMON + lang + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    warn = [l for l in r.stderr.splitlines() if "warning" in l and "packed-fp32-ops" not in l]
    return obj, warn


def build(jobs=None, verbose=False):
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for obj, warn in ex.map(compile_one, srcs):
            objs.append(obj)
            if verbose:
                for w in warn:
                    print(w, file=sys.stderr)
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs + ["-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    cli_src = os.path.join(CSRC, "cli", "shlo_hip_main.cpp")
    if os.path.exists(cli_src):
        cmd = [HIPCC] + COMMON + [cli_src, "-o", CLI + ".tmp", "-L" + OUT_DIR, "-lshlo_hip",
                                  "-Wl,-rpath,$ORIGIN"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"CLI link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
        os.replace(CLI + ".tmp", CLI)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.v))
