"""Build libkiln_hip.so (every HIP kernel family + the C ABI) for gfx950.

    python kiln-compiler_amd/build.py [--jobs N] [--verbose]

Each csrc/*.hip file is compiled by hipcc to an object in _build/ (in
parallel), then linked into kiln/hip/libkiln_hip.so, next to the ctypes
binding that loads it. Always rebuilds: the driver's build() check calls this
on every round, and objects of a stale source must never be reused.
"""

from __future__ import annotations

import argparse
import hashlib
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = REPO / "include"
BUILD = HERE / "_build"
LIB = HERE / "kiln" / "hip" / "libkiln_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    # packed fp32 ops off: the compiler must not form v_pk_* fp32 instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the HIP backend needs ROCm's hipcc to build")
    return path


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        noise = "is not a recognized feature for this target"
        err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    return res


def source_digest() -> str:
    """sha256 over every file the library is compiled from (csrc/, include/)
    and the compiler flags: compiled into the library as kh_build_id(), so a
    stored plan is never reused by a library built from other sources."""
    h = hashlib.sha256()
    for f in sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.hpp"), *INCLUDE.glob("*.h")]):
        h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    h.update(" ".join(HIPCC_FLAGS[:-2]).encode())
    return h.hexdigest()[:32]


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    BUILD.mkdir(exist_ok=True)
    cc = hipcc()
    objects = [BUILD / (s.stem + ".o") for s in sources]
    flags = [*HIPCC_FLAGS, f'-DKH_BUILD_ID="{source_digest()}"']
    cmds = [[cc, *flags, "-c", str(s), "-o", str(o)] for s, o in zip(sources, objects)]
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        for fut in [pool.submit(_run, c, verbose) for c in cmds]:
            fut.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)], verbose)
    os.replace(tmp, LIB)
    return LIB


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--jobs", type=int, default=None)
    p.add_argument("--verbose", action="store_true")
    args = p.parse_args(argv)
    lib = build(args.jobs, args.verbose)
    print(f"built {lib}")


if __name__ == "__main__":
    sys.exit(main())
