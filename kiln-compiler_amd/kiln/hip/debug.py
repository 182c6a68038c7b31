"""Arena checks of ``Options(debug=True)``: NaN poison and canaries.

A debug build runs its plan launch by launch and, around every launch,

  * before the launch that first writes an arena buffer, fills the buffer
    with NaN: a launch that reads an intermediate before it is written
    (a missing dependency, a wrong offset) gets NaN, which reaches the
    outputs, also when the memory plan gave the buffer bytes another buffer
    held earlier in the same call;
  * gives every buffer a guard of ``kiln.api.DEBUG_GUARD_BYTES`` after its
    aligned size (the memory plan reserves it), fills the guard and the
    alignment padding with a canary when the buffer's value becomes live,
    and after each launch checks the canaries of every buffer live at that
    launch: a launch that writes past the end of a buffer raises
    RuntimeError naming the launch and the buffer.

The canary is a signalling-NaN bit pattern; arithmetic on the device and
the host produces quiet NaNs only, so no kernel writes it by computing.
The checks are the same for the device arena (torch tensor) and the host
interpreter's (numpy array). The counterpart of the reference's invariant
checking is the pass manager's ``verify`` after every pass
(kiln/passes/manager.py:36-37); these checks are the runtime side.
"""

from __future__ import annotations

import numpy as np

NAN_BITS = 0x7FC00000      # the quiet NaN the poison writes
CANARY = 0x7FBADBAD        # a signalling NaN: never the result of arithmetic
ALIGN = 64


def _align(n: int) -> int:
    return (n + ALIGN - 1) // ALIGN * ALIGN


class ArenaGuards:
    """Per-launch poison and canary checks over one arena (32-bit words)."""

    def __init__(self, program, guard_bytes: int):
        self.program = program
        self.names = [launch.name for launch in program.launches]
        n = len(program.launches)
        self.starts = [[] for _ in range(n)]   # launch -> buffers whose value becomes live there
        self.live = [[] for _ in range(n)]     # launch -> buffers live during it
        self.buffers = []
        for label, off, nbytes, first, last in program.arena_buffers:
            if first < 0 or first >= n:
                continue
            body = (off // 4, (off + nbytes) // 4)
            guard = ((off + nbytes) // 4, (off + _align(nbytes) + guard_bytes) // 4)
            b = len(self.buffers)
            self.buffers.append((label, body, guard))
            self.starts[first].append(b)
            for i in range(first, min(last, n - 1) + 1):
                self.live[i].append(b)

    def words_needed(self) -> int:
        return max([g[1] for _, _, g in self.buffers] + [0])

    # the caller passes the arena as an indexable array of int32 words with
    # fill(lo, hi, value) and differs(lo, hi, value) -> bool helpers
    def before(self, i: int, fill):
        for b in self.starts[i]:
            _, (lo, hi), (glo, ghi) = self.buffers[b]
            fill(lo, hi, NAN_BITS)
            fill(glo, ghi, CANARY)

    def after(self, i: int, differs):
        for b in self.live[i]:
            label, (lo, hi), (glo, ghi) = self.buffers[b]
            if ghi > glo and differs(glo, ghi, CANARY):
                raise RuntimeError(f"debug: launch {i} ({self.names[i]}) wrote past the end of arena buffer "
                                   f"'{label}' (bytes {4 * lo}..{4 * hi}): its guard bytes "
                                   f"{4 * glo}..{4 * ghi} changed")


def numpy_ops(words: np.ndarray):
    """fill / differs over a host arena viewed as int32 words."""
    def fill(lo, hi, value):
        words[lo:hi] = np.int32(np.uint32(value).view(np.int32))

    def differs(lo, hi, value):
        return bool((words[lo:hi] != np.uint32(value).view(np.int32)).any())

    return fill, differs


def torch_ops(words):
    """fill / differs over a device arena viewed as int32 words (each check
    synchronises)."""
    def as_i32(value):
        return int(np.uint32(value).view(np.int32))

    def fill(lo, hi, value):
        words[lo:hi].fill_(as_i32(value))

    def differs(lo, hi, value):
        return bool((words[lo:hi] != as_i32(value)).any().item())

    return fill, differs
