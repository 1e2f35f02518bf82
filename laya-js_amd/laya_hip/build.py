"""Compiles libhipbackend.so (gfx950 only) from laya-js_amd/csrc/*.hip.

Objects go to laya-js_amd/_build/ (git-ignored); the shared library lands
next to this file, in-tree, so it travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(ROOT, "csrc")
OUT_DIR = os.path.join(ROOT, "_build")
LIB = os.path.join(PKG, "libhipbackend.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed-FP32 VALU ops are disabled for every kernel (the hardware forms of
# v_pk_{add,mul,fma}_f32 are not used on this target).
CFLAGS = [f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-function",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _stale(src: str, obj: str) -> bool:
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    deps = [src, *glob.glob(os.path.join(CSRC, "*.h")), os.path.join(os.path.dirname(ROOT), "include", "laya_hip.h")]
    return any(os.path.getmtime(d) > t for d in deps if os.path.exists(d))


def _compile(src: str, incremental: bool = False) -> str:
    obj = os.path.join(OUT_DIR, os.path.basename(src).replace(".hip", ".o"))
    if incremental and not _stale(src, obj):
        return obj
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        msg = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops' is not a recognized" not in l)
        raise RuntimeError(f"hipcc failed for {src}:\n{msg}")
    return obj


def build(jobs: int = 8, incremental: bool = False) -> str:
    """Compiles every csrc/*.hip and links libhipbackend.so; returns its path.
    `incremental` recompiles only the sources newer than their objects (or
    than any csrc/*.h or laya_hip.h)."""
    os.makedirs(OUT_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        objs = list(ex.map(lambda s_: _compile(s_, incremental), srcs))
    tmp = LIB + ".tmp"
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    import sys
    print(build(incremental="--incremental" in sys.argv))
