"""Build libq6moe.so (HIP, gfx950 only) in-tree with hipcc.

Usage: python data-synth-tpu_amd/build.py [-j N] [-v]

Every .hip file under csrc/ is compiled to an object with hipcc for
--offload-arch=gfx950 and linked into q6moe/libq6moe.so. Packed FP32 VALU
forms are disabled (-packed-fp32-ops) for every device compile.
"""

import argparse
import concurrent.futures
import os
import subprocess
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT_DIR = HERE / "_build"
LIB = HERE / "q6moe" / "libq6moe.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{HERE.parent / 'include'}",
]


def _compile(src, verbose):
    obj = OUT_DIR / (src.stem + ".o")
    cmd = [HIPCC, *DEVICE_FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the device-only feature; drop that one note.
    noise = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip() and verbose:
        print(err)
    return obj


def build(jobs=None, verbose=False):
    """Compile every csrc/*.hip and link q6moe/libq6moe.so. Returns the library path."""
    OUT_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    started = time.time()
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        objects = list(pool.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources in {time.time() - started:.1f}s")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    try:
        build(a.j, True if a.v else False)
    except RuntimeError as exc:
        print(exc, file=sys.stderr)
        sys.exit(1)
