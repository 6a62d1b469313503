"""Build libq8hip.so (the gfx950 Q8 kernels + C ABI) in-tree with hipcc.

    python -m lama32_mojo_amd.build          # -> lama32_mojo_amd/libq8hip.so
    python -m lama32_mojo_amd.build --incremental   # only out-of-date objects

Every source under csrc/ is compiled for gfx950 only, with
  * packed fp32 instructions disabled (-target-feature -packed-fp32-ops),
  * IEEE f32 division and square root (no fast-math), which the bit-exact
    quantizer relies on.
Objects go to lama32_mojo_amd/_build/ and are linked into one shared
library next to this file, so it travels with the source tree.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_PATH = os.path.join(HERE, "libq8hip.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(os.path.dirname(HERE), "include"),
]


def sources():
    return sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC)
        if f.endswith(".hip") or f.endswith(".cpp"))


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 target feature and
    # warns about it; that warning is expected and filtered here.
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out:
        print(out, flush=True)


def _stale(src: str, obj: str) -> bool:
    """An object older than its source or any header it may include."""
    if not os.path.exists(obj):
        return True
    deps = [src] + [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    deps.append(os.path.join(os.path.dirname(HERE), "include", "q8hip.h"))
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(d) > t for d in deps if os.path.exists(d))


def build(verbose: bool = True, jobs: int | None = None, incremental: bool = False) -> str:
    """Compile every csrc/ source and link libq8hip.so; returns its path.
    incremental=True recompiles only sources whose object is out of date."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(BUILD_DIR, os.path.basename(s) + ".o") for s in srcs]
    cmds = []
    for s, o in zip(srcs, objs):
        if incremental and not _stale(s, o):
            continue
        lang = ["-x", "hip"] if s.endswith(".cpp") else []
        cmds.append([HIPCC, *COMMON_FLAGS, *lang, "-c", s, "-o", o])
    jobs = jobs or min(max(len(cmds), 1), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB_PATH + ".tmp"
    # export only the C ABI (q8_*): the version script keeps every internal
    # launcher and helper local to the library
    vscript = os.path.join(CSRC, "libq8hip.map")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,--version-script={vscript}",
          "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB_PATH)
    build_calib(verbose)
    return LIB_PATH


CALIB_SRC = os.path.join(HERE, "calib", "q8_calib.hip")
CALIB_PATH = os.path.join(HERE, "libq8calib.so")


def build_calib(verbose: bool = True) -> str:
    """libq8calib.so: the calibration kernels bench.py --workload calib
    times (empty kernel node, streaming read, few-CU reads, register-only
    MFMA); measurement infrastructure, not part of libq8hip.so."""
    tmp = CALIB_PATH + ".tmp"
    _run([HIPCC, *COMMON_FLAGS, "-shared", "-o", tmp, CALIB_SRC], verbose)
    os.replace(tmp, CALIB_PATH)
    return CALIB_PATH


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv, incremental="--incremental" in sys.argv)
