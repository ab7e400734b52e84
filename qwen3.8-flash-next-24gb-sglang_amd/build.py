"""Build libkvtier.so (the HIP kernels behind the C ABI of include/kvtier.h) for gfx950, in place.

Every .hip file under csrc/ is compiled to an object with hipcc (in parallel), then linked into
``libkvtier.so`` next to this file.  Flags:
  --offload-arch=gfx950                       MI355X only (one code path, no CUDA/HIP dual build)
  -fhip-fp32-correctly-rounded-divide-sqrt    IEEE fp32 division (the quantizers' x / s must be exact)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                              no packed fp32 VALU instructions
  no -ffast-math: rounding must follow IEEE round-to-nearest-even.
Per file: decode_mfma.hip, decode_rows.hip and decode_ref.hip preload the first kernel-argument dwords into SGPRs
(-mllvm -amdgpu-kernarg-preload-count=16; the split-K kernel's arguments are ordered for it).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
LIB_NAME = "libkvtier.so"
BUILD_DIR = os.path.join(HERE, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{CSRC}",
    f"-I{INCLUDE}",
]


EXTRA_CFLAGS = {
    "decode_mfma.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
    "decode_ref.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
    "decode_rows.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
}


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *CFLAGS, *EXTRA_CFLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every kernel source and link libkvtier.so; returns its path.  Always rebuilds."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        objs = list(ex.map(_compile, srcs))
    out = os.path.join(HERE, LIB_NAME)
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    shutil.rmtree(BUILD_DIR, ignore_errors=True)
    if verbose:
        print(f"built {out} from {len(srcs)} sources")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
