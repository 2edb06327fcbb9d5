"""Build librhizome_gdr.so in-tree with hipcc, for gfx950 only.

    python -m rhizome_amd.build        (or rhizome_amd.build.build())

Every .hip / .cpp file under rhizome_amd/csrc is compiled separately (in
parallel) and linked into rhizome_amd/librhizome_gdr.so next to this file.
The C++ restatement of the reference's delta.rs API (rhizome_amd/host) is
linked against it into rhizome_amd/librhizome_ops.so.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "librhizome_gdr.so")
HOST = os.path.join(HERE, "host")
OPS_LIB = os.path.join(HERE, "librhizome_ops.so")
ARCH = "gfx950"

# Packed-FP32 instructions stay off (the compiler emits none of
# v_pk_add/mul/fma_f32 with this feature disabled).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the ROCm toolchain is required to build librhizome_gdr.so")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.basename(src) + ".o")
    cmd = [hipcc()] + HIP_FLAGS + ["-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(jobs: int | None = None) -> str:
    os.makedirs(OBJ, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    build_ops()
    return LIB


def build_ops() -> str:
    """librhizome_ops.so: the delta.rs-shaped C++ API over librhizome_gdr.so."""
    objs = []
    for f in sorted(os.listdir(HOST)):
        if f.endswith(".cpp"):
            obj = os.path.join(OBJ, "host_" + f + ".o")
            cmd = [hipcc(), "-O2", "-fPIC", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"),
                   "-I", HOST, "-c", os.path.join(HOST, f), "-o", obj]
            res = subprocess.run(cmd, capture_output=True, text=True)
            if res.returncode != 0:
                raise RuntimeError(f"hipcc failed on host/{f}:\n{res.stderr}")
            objs.append(obj)
    tmp = OPS_LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", "-o", tmp] + objs + [
        "-L", HERE, "-lrhizome_gdr", "-Wl,-rpath,$ORIGIN"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of librhizome_ops.so failed:\n{res.stderr}")
    os.replace(tmp, OPS_LIB)
    return OPS_LIB


if __name__ == "__main__":
    print(build())
