"""Builds libgeode_verify.so (hipcc, gfx950) in-tree, and the CPU checker under oracle/ (g++).

    python -m geode_amd.build            # everything
    python -m geode_amd.build hip        # the HIP library only
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "geode_amd", "csrc")
OBJ = os.path.join(ROOT, "geode_amd", "_build")
LIB = os.path.join(ROOT, "geode_amd", "libgeode_verify.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
SOURCES = ["misc.hip", "q4.hip", "capi.hip", "model.hip", "sample.hip", "state.hip", "pack.hip", "gdn.hip", "mtp.hip",
           "prefill.hip"]
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-I", os.path.join(ROOT, "include"),
]


def _run(cmd, cwd=ROOT):
    p = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (p.stderr or "").splitlines() if noise not in l)
    if p.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{p.stdout}\n{err}")
    return err


def build_hip(verbose=False):
    os.makedirs(OBJ, exist_ok=True)

    def compile_one(src):
        obj = os.path.join(OBJ, src + ".o")
        _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
        return obj

    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


def build_oracle(verbose=False):
    _run(["make", "-B", "-C", os.path.join(ROOT, "oracle"), "all"])
    if os.path.isdir("/root/reference/engine/src"):
        _run(["make", "-B", "-C", os.path.join(ROOT, "oracle"), "ref"])
    if verbose:
        print("built oracle")


def build_all(verbose=False):
    build_oracle(verbose)
    build_hip(verbose)


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "all"
    {"all": build_all, "hip": build_hip, "oracle": build_oracle}[what](verbose=True)
