"""On-disk store of lowered plans.

A lowered ``Program`` (its ``kh_launch`` descriptors, constant slots and the
recipes of the constants derived at build time) is written once per key and
read back by later compiles, which then skip lowering and GEMM tuning. This
is the counterpart of the reference's content-addressed kernel source cache
(kiln/gpu/runtime.py:53-79), one level further: what is stored is the plan
itself, not source text to recompile.

The key hashes everything the plan depends on: the backend's code (the
lowering and tuner sources, the shipped tuning table, the library's ABI
version, struct sizes and GEMM configuration table), the device (arch, CU
count), the matmul precision, how GEMM configurations were chosen, and the
optimised graph's text (ops, shapes, kernel partition, buffer layouts and
arena offsets). Constant *data* is not part of it: no descriptor depends on
it, derived copies are rebuilt from the recipes.

Files live in ``<cache dir>/plans/<key>.json`` (written to a temporary file,
flushed, then renamed, so a crash never leaves a half-written plan behind),
next to ``<key>.txt``, the human-readable listing. A file that does not parse
or does not match the key is ignored (and rewritten).
"""

from __future__ import annotations

import base64
import hashlib
import json
import os
from pathlib import Path

from kiln.hip import lib as kl

FORMAT = 3


def cache_dir() -> Path:
    base = os.environ.get("KILN_CACHE_DIR") or os.path.join(Path.home(), ".cache", "kiln")
    return Path(base) / "hip"


_BACKEND_FILES = ("lowering.py", "autotune.py", "attention.py", "bf16.py", "tuned_configs.json")
_fingerprint = None


def backend_fingerprint() -> str:
    """Digest of the code that turns a graph into a plan and of the library
    build that reads the plan's descriptors (kh_build_id)."""
    global _fingerprint
    if _fingerprint is None:
        h = hashlib.sha256()
        here = Path(__file__).resolve().parent
        for name in _BACKEND_FILES:
            try:
                h.update((here / name).read_bytes())
            except OSError:
                h.update(b"missing " + name.encode())
        h.update(repr((kl.ABI_VERSION, kl.ctypes.sizeof(kl.LaunchDesc), tuple(kl.gemm_configs()),
                       kl.build_id())).encode())
        _fingerprint = h.hexdigest()
    return _fingerprint


def plan_key(graph_text: str, precision: str, config_source: str, device: dict) -> str:
    h = hashlib.sha256()
    for part in (f"format {FORMAT}", backend_fingerprint(), f"{device.get('arch')}|{device.get('cus')}",
                 precision, config_source, graph_text):
        h.update(part.encode())
        h.update(b"\0")
    return h.hexdigest()[:24]


def _atomic_write(path: Path, text: str):
    path.parent.mkdir(parents=True, exist_ok=True)
    tmp = path.with_name(f".{path.name}.{os.getpid()}.tmp")
    with open(tmp, "w") as f:
        f.write(text)
        f.flush()
        os.fsync(f.fileno())
    os.replace(tmp, path)


def listing_path(key: str) -> Path:
    return cache_dir() / "plans" / f"{key}.txt"


def write_listing(key: str, program) -> Path:
    """The plan's human-readable listing under ``key`` (rewritten only when
    its text changed); returns its path."""
    listing = listing_path(key)
    try:
        fresh = listing.read_text() != program.source
    except OSError:
        fresh = True
    if fresh:
        _atomic_write(listing, program.source)
    return listing


def save(key: str, program, autotune_log=()) -> Path:
    """Store ``program`` under ``key``; returns the listing's path."""
    record = {
        "format": FORMAT, "key": key, "precision": program.precision, "consts": list(program.consts),
        "derived": {name: list(recipe) for name, recipe in program.derived.items()},
        "arena_buffers": [list(b) for b in program.arena_buffers],
        "launches": [{"name": l.name, "kernel": l.kernel, "family": l.family, "summary": l.summary,
                      "flops": l.flops, "bytes": l.bytes,
                      "desc": base64.b64encode(bytes(l.desc)).decode()} for l in program.launches],
        "autotune": [dict(e, shape=list(e["shape"])) for e in autotune_log],
    }
    folder = cache_dir() / "plans"
    _atomic_write(folder / f"{key}.json", json.dumps(record))
    return write_listing(key, program)


def _recipe(r) -> tuple:
    """A derived-constant recipe read back from JSON: (source, offset,
    strides, batch, k, n) and, for the folded LayerNorm constants, the
    (constant, offset, stride) of the vector they fold in."""
    head = (r[0], int(r[1]), tuple(r[2]), int(r[3]), int(r[4]), int(r[5]))
    return head + ((str(r[6][0]), int(r[6][1]), int(r[6][2])),) if len(r) > 6 else head


def load(key: str):
    """(Program, autotune log) stored under ``key``, or None."""
    from kiln.hip.lowering import Launch, Program

    path = cache_dir() / "plans" / f"{key}.json"
    try:
        record = json.loads(path.read_text())
        if record.get("format") != FORMAT or record.get("key") != key:
            return None
        size = kl.ctypes.sizeof(kl.LaunchDesc)
        launches = []
        for item in record["launches"]:
            raw = base64.b64decode(item["desc"])
            if len(raw) != size:
                return None
            launches.append(Launch(item["name"], item["kernel"], int(item["family"]),
                                   kl.LaunchDesc.from_buffer_copy(raw), item["summary"], int(item["flops"]),
                                   int(item["bytes"])))
        program = Program(launches=launches, consts=list(record["consts"]), precision=record["precision"],
                          derived={name: _recipe(r) for name, r in record["derived"].items()},
                          arena_buffers=[(str(b[0]), int(b[1]), int(b[2]), int(b[3]), int(b[4]))
                                         for b in record.get("arena_buffers", [])])
        log = [dict(e, shape=tuple(e["shape"]), source="cache") for e in record.get("autotune", [])]
        return program, log
    except (OSError, ValueError, KeyError, TypeError, IndexError):
        return None
