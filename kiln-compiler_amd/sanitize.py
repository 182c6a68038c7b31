"""Build the library's host code with AddressSanitizer and UBSan and run the
CPU tests that exercise it (plan validation, the host interpreter, the chain
finder's range proofs) against that build.

    python kiln-compiler_amd/sanitize.py [pytest args...]

Host code only: each -fsanitize= flag is passed to hipcc after -Xarch_host,
so the device code is compiled exactly as in build.py (no GPU sanitizer).
The sanitized library goes to kiln/hip/libkiln_hip_asan.so and is loaded by
the tests through KILN_HIP_LIB; the product library is not touched. Python
itself is not instrumented, so the ASan runtime is preloaded into the test
process (leak checking off: the interpreter's own allocations would report).
Any sanitizer report fails the run (halt_on_error, UBSan non-recoverable).
The sanitized library and its objects are deleted afterwards (--keep keeps
them), so they never ship with the tree.
"""

from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import build  # noqa: E402

SAN_LIB = os.path.join(HERE, "kiln", "hip", "libkiln_hip_asan.so")
SAN_BUILD = build.BUILD.with_name("_build_asan")
SAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
             "-Xarch_host", "-g"]
TESTS = ["tests/test_interpret.py", "tests/test_lowering.py"]


def asan_runtime() -> str:
    hits = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        raise RuntimeError("no libclang_rt.asan-x86_64.so under /opt/rocm/lib/llvm")
    return hits[-1]


def build_sanitized(jobs=None) -> str:
    SAN_BUILD.mkdir(exist_ok=True)
    cc = build.hipcc()
    flags = [*build.HIPCC_FLAGS, f'-DKH_BUILD_ID="{build.source_digest()}"', *SAN_FLAGS]
    sources = sorted(build.CSRC.glob("*.hip"))
    objects = [SAN_BUILD / (s.stem + ".o") for s in sources]
    cmds = [[cc, *flags, "-c", str(s), "-o", str(o)] for s, o in zip(sources, objects)]
    with ThreadPoolExecutor(max_workers=jobs or min(len(cmds), os.cpu_count() or 4)) as pool:
        for fut in [pool.submit(build._run, c, False) for c in cmds]:
            fut.result()
    build._run([cc, f"--offload-arch={build.ARCH}", "-shared", "-fPIC", *SAN_FLAGS, *map(str, objects),
                "-o", SAN_LIB], False)
    return SAN_LIB


CHECK = (
    "import sys; sys.path[:0] = ['kiln-compiler_amd']\n"
    "from kiln.hip import lib\n"
    "lib.load()\n"
    "maps = open('/proc/self/maps').read()\n"
    "assert 'libclang_rt.asan' in maps and 'libkiln_hip_asan.so' in maps, 'sanitized library not loaded'\n"
    "print('loaded', lib.library_path())\n")


def main(argv=None):
    argv = list(sys.argv[1:] if argv is None else argv)
    keep = "--keep" in argv
    argv = [a for a in argv if a != "--keep"]
    lib = build_sanitized()
    print(f"built {lib}", flush=True)
    env = dict(os.environ, KILN_HIP_LIB=lib, LD_PRELOAD=asan_runtime(),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:detect_odr_violation=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    root = os.path.dirname(HERE)
    try:
        subprocess.check_call([sys.executable, "-c", CHECK], cwd=root, env=env)
        cmd = [sys.executable, "-m", "pytest", *TESTS, "-q", "-m", "not gpu", "-p", "no:cacheprovider", *argv]
        return subprocess.call(cmd, cwd=root, env=env)
    finally:
        if not keep:
            os.remove(lib)
            shutil.rmtree(SAN_BUILD, ignore_errors=True)


if __name__ == "__main__":
    sys.exit(main())
