"""FileCheck tests over textual IR (tests/lit/*.kir), run through kiln-opt.

Each ``// RUN:`` line is executed with ``%kiln-opt`` -> ``python -m
kiln.tools.opt`` and ``%s`` -> the fixture, piped into LLVM's FileCheck
(ROCm ships it); `lit` itself is not needed. The fixtures restate the
reference's lit expectations (its tests/lit/*.kir): fusion partition,
memory-plan offsets (arena 3072 / naive 4096), buffer-assignment strides and
copies, canonicalisation, constant folding, freezing; plus the lowered plan.
"""

import os
import re
import shlex
import shutil
import subprocess
import sys

import pytest

LIT = os.path.join(os.path.dirname(__file__), "lit")
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FILECHECK = shutil.which("FileCheck") or "/opt/rocm/lib/llvm/bin/FileCheck"
FIXTURES = sorted(f for f in os.listdir(LIT) if f.endswith(".kir"))


def run_lines(path):
    out = []
    for line in open(path):
        m = re.match(r"\s*//\s*RUN:\s*(.*)", line)
        if m:
            out.append(m.group(1))
    return out


@pytest.mark.skipif(not os.path.exists(FILECHECK), reason="FileCheck not found")
@pytest.mark.parametrize("fixture", FIXTURES)
def test_filecheck(fixture):
    path = os.path.join(LIT, fixture)
    runs = run_lines(path)
    assert runs, f"{fixture} has no RUN line"
    env = {**os.environ, "PYTHONPATH": os.pathsep.join([os.path.join(ROOT, "kiln-compiler_amd"),
                                                          os.environ.get("PYTHONPATH", "")])}
    for cmd in runs:
        left, right = cmd.split("|", 1)
        opt = shlex.split(left.replace("%kiln-opt", f"{sys.executable} -m kiln.tools.opt").replace("%s", path))
        check = shlex.split(right.replace("FileCheck", FILECHECK).replace("%s", path))
        produced = subprocess.run(opt, capture_output=True, text=True, env=env)
        assert produced.returncode == 0, produced.stderr
        verdict = subprocess.run(check, input=produced.stdout, capture_output=True, text=True)
        assert verdict.returncode == 0, f"{cmd}\n{verdict.stderr}\n--- kiln-opt output ---\n{produced.stdout}"
