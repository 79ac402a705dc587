"""Build libravel_em.so for gfx950 with hipcc (run: python -m ravel_em._build).

Each HIP translation unit compiles to an object in parallel, then the objects
link into one shared library next to this file.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)
CSRC = os.path.join(PKG_ROOT, "csrc")
OBJ_DIR = os.path.join(PKG_ROOT, "_build")
SOURCES = [
    "em_api.hip", "em_sort.hip", "em_lookup.hip", "em_sum.hip", "em_cache.hip", "em_backward.hip",
    "em_fuse.hip", "em_addr.hip",
]
ARCH = os.environ.get("RAVEL_EM_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed fp32 instructions are disabled for all device code.
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build(verbose: bool = False) -> str:
    """Compile every HIP source and link libravel_em.so; returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    out = os.path.join(HERE, "libravel_em.so")
    objs = [os.path.join(OBJ_DIR, s.replace(".hip", ".o")) for s in SOURCES]
    cmds = [[HIPCC, *CFLAGS, "-c", os.path.join(CSRC, s), "-o", o] for s, o in zip(SOURCES, objs)]
    with cf.ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 1)) as ex:
        for msg in ex.map(_run, cmds):
            if verbose and msg:
                print(msg, file=sys.stderr)
    tmp = out + ".tmp"
    # --no-undefined: a missing definition fails the build, not the first dlopen
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", tmp, *objs])
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
