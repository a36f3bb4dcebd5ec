"""Builds libraceline_amd.so in-tree with hipcc for gfx950.

    python -m raceline_amd.build            # compile every source under csrc/ and link

The library lands next to this file (raceline_amd/libraceline_amd.so), where the
ctypes loader looks first, so it travels with the source tree. Objects go to
raceline_amd/_build/. Every call recompiles (the driver uses this as its build check).
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
OUT = os.path.join(HERE, "libraceline_amd.so")
BUILD = os.path.join(HERE, "_build")
ARCH = os.environ.get("RLQ_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed fp32 ops are kept out of every kernel (they have given silent wrong results on this pool)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.isfile(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def sources():
    """HIP sources (kernels and their entry points) and host-only C++ (the model file reader)."""
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def _compile(src: str) -> str:
    base = os.path.basename(src)
    obj = os.path.join(BUILD, base.rsplit(".", 1)[0] + (".o" if base.endswith(".hip") else ".cpp.o"))
    cmd = [hipcc(), *HIP_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        noise = "is not a recognized feature for this target"
        err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{err}")
    return obj


def _check_defined(lib: str) -> None:
    """Fails when the library leaves one of its own symbols undefined. A shared library
    links with undefined symbols, and the loader only refuses it at dlopen; clang's host
    pass can drop a kernel's launch stub without a diagnostic (a kernel template whose
    body it skips), which shows up here as an undefined rlq:: symbol."""
    nm = shutil.which("nm")
    if not nm:
        return
    r = subprocess.run([nm, "-u", "-C", lib], capture_output=True, text=True)
    missing = [l.strip() for l in r.stdout.splitlines() if "rlq::" in l or " rlq_" in l]
    if missing:
        raise RuntimeError("library leaves its own symbols undefined:\n  " + "\n  ".join(missing))


def build(verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    _check_defined(tmp)
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources", flush=True)
    return OUT


if __name__ == "__main__":
    build()
    sys.exit(0)
