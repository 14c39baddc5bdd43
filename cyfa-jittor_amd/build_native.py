"""Build libcyfa_hip.so for gfx950 from csrc/*.hip (in-tree, no JIT cache).

Usage: python cyfa-jittor_amd/build_native.py [--verbose]
The library lands next to the Python package that loads it:
cyfa-jittor_amd/cyclic_flow_attention/libcyfa_hip.so
"""

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = REPO / "include"
OUT = HERE / "cyclic_flow_attention" / "libcyfa_hip.so"
OBJ_DIR = HERE / "_build"
ARCH = os.environ.get("CYFA_OFFLOAD_ARCH", "gfx950")

# Packed-FP32 instructions are disabled for every HIP translation unit.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.sep not in cand or os.path.exists(cand)):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(str(c) for c in cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(
        line for line in res.stderr.splitlines() if "packed-fp32-ops" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(map(str, cmd))}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose=False):
    """Compile every csrc/*.hip for gfx950 and link libcyfa_hip.so."""
    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objects = [OBJ_DIR / (s.stem + ".o") for s in sources]
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        futures = [
            pool.submit(_run, [hipcc, *HIPCC_FLAGS, "-c", str(s), "-o", str(o)], verbose)
            for s, o in zip(sources, objects)
        ]
        for f in futures:
            f.result()
    tmp = OUT.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)], verbose)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    path = build(verbose="--verbose" in sys.argv)
    print(path)
