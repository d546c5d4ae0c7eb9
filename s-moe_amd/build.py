"""Build libsmoe_hip.so (gfx950) in-tree.

    python s-moe_amd/build.py            # compile every translation unit, link

Each .hip / .cpp under csrc/ is compiled by hipcc for gfx950 only, objects go
to s-moe_amd/_build/ and the shared library to s-moe_amd/smoe_amd/.  Packed
FP32 instructions are disabled for all device code.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
BUILD = os.path.join(PKG, "_build")
LIBDIR = os.path.join(PKG, "smoe_amd")
LIB = os.path.join(LIBDIR, "libsmoe_hip.so")
HOSTLIB = os.path.join(LIBDIR, "libsmoe_host.so")

ARCH = os.environ.get("SMOE_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result",
          "-I" + os.path.join(ROOT, "include"), "-I" + CSRC]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-munsafe-fp-atomics"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the gfx950 feature flag; that note is noise
    err = "\n".join(l for l in r.stderr.splitlines()
                    if "packed-fp32-ops" not in l or "error" in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}")
    return err


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC)
                  if f.endswith((".hip", ".cpp")))


def host_sources():
    if not os.path.isdir(HOST):
        return []
    return sorted(os.path.join(HOST, f) for f in os.listdir(HOST) if f.endswith(".cpp"))


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    jobs = []
    for src in sources():
        obj = os.path.join(BUILD, os.path.basename(src) + ".o")
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        jobs.append((obj, [HIPCC, *COMMON, *DEVICE, *lang, "-c", src, "-o", obj]))
    workers = min(len(jobs), int(os.environ.get("MAX_JOBS", "8")))
    with cf.ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        for out in ex.map(lambda j: _run(j[1]), jobs):
            if verbose and out:
                print(out, file=sys.stderr)
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[j[0] for j in jobs]])
    os.replace(tmp, LIB)

    hs = host_sources()
    if hs:
        tmp = HOSTLIB + ".tmp"
        _run([HIPCC, *COMMON, "-shared", "-o", tmp, *hs, "-L" + LIBDIR, "-lsmoe_hip",
              "-Wl,-rpath,$ORIGIN"])
        os.replace(tmp, HOSTLIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
