"""Build the C oracle: oracle/kiln_oracle.c -> oracle/_build/libkiln_oracle.so.

Test infrastructure: the oracle is the CPU checker (and the timed CPU
baseline), never part of the product path.

    python oracle/build.py
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "kiln_oracle.c"
OUT = HERE / "_build" / "libkiln_oracle.so"


def build(verbose=False) -> Path:
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no C compiler (gcc) for the oracle")
    OUT.parent.mkdir(exist_ok=True)
    tmp = OUT.with_suffix(".so.tmp")
    # -ffp-contract=off keeps every double operation individually rounded.
    cmd = [cc, "-O2", "-ffp-contract=off", "-fPIC", "-shared", "-std=c11", str(SRC), "-o", str(tmp), "-lm"]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
