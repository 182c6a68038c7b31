"""Static memory plan: every arena buffer gets a fixed offset in one allocation.

The plan is Kiln's (the reference's kiln/passes/memory_plan.py:43-112): the
memory_plan.kir fixture pins its offsets, and for the GPT-2 block the arena
equals the peak-live lower bound (the reference's
tests/test_memory_plan.py:42-51):

  * a buffer is busy from the kernel that writes it to the last kernel that
    reads it, directly or through a view, both included (kernel indices);
  * buffers are placed one by one, largest first (equal sizes: the earlier
    writer first), each at the lowest 64-byte-aligned offset where it
    overlaps no already placed buffer that is busy at the same time;
  * ``reuse=False`` places them end to end instead (the ablation baseline);
  * ``guard`` (debug builds; 0 otherwise) reserves that many more bytes after
    each buffer's aligned size, so no two buffers abut: the runtime fills the
    gap with a canary and checks it after every launch.

On the MI355X the arena is one device allocation, and the fixed offsets are
what let a whole compiled graph be captured once and replayed as a hipGraph.
"""

from __future__ import annotations

from kiln.ir.core import Graph
from kiln.passes.buffers import ALIGNMENT, compute_layouts, kernel_inputs
from kiln.passes.manager import Pass


def align(nbytes: int) -> int:
    return (nbytes + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT


def live_ranges(graph: Graph) -> dict:
    """{buffer-owning Value: [first kernel, last kernel]} for arena buffers."""
    layouts = compute_layouts(graph)
    kernel_index = {n: i for i, k in enumerate(graph.kernels) for n in k.nodes}
    spans = {}
    for v, lay in layouts.items():
        if lay.base == ("arena", v):
            spans[v] = [kernel_index[v.node], kernel_index[v.node]]
    for i, k in enumerate(graph.kernels):
        for v in kernel_inputs(graph, k):
            lay = layouts.get(v)
            if lay is not None and lay.base[0] == "arena":
                span = spans[lay.base[1]]
                span[1] = max(span[1], i)
    return spans


def overlaps(a, b) -> bool:
    """Do two closed [first, last] kernel intervals share a kernel?"""
    return max(a[0], b[0]) <= min(a[1], b[1])


def peak_live_bytes(ranges) -> int:
    """The most (aligned) bytes busy during any one kernel: no plan can be
    smaller. Computed as a sweep over interval start / end events."""
    events = {}
    for v, (first, last) in ranges.items():
        size = align(v.type.nbytes)
        events[first] = events.get(first, 0) + size
        events[last + 1] = events.get(last + 1, 0) - size
    peak = live = 0
    for t in sorted(events):
        live += events[t]
        peak = max(peak, live)
    return peak


def _lowest_gap(size: int, taken) -> int:
    """Lowest offset where [offset, offset + size) avoids every [lo, hi) in
    ``taken`` (offsets of multiples of the alignment stay aligned)."""
    offset = 0
    for lo, hi in sorted(taken):
        if offset + size <= lo:
            break
        offset = max(offset, hi)
    return offset


class MemoryPlan(Pass):
    name = "memory-plan"

    def __init__(self, reuse: bool = True, guard: int = 0):
        self.reuse = reuse
        self.guard = align(guard)

    def run(self, graph: Graph):
        ranges = live_ranges(graph)
        placements = []   # (offset, size, busy interval)
        end = 0
        for v in sorted(ranges, key=lambda v: (-v.type.nbytes, ranges[v][0])):
            size, busy = align(v.type.nbytes) + self.guard, ranges[v]
            if self.reuse:
                offset = _lowest_gap(size, [(o, o + s) for o, s, b in placements if overlaps(b, busy)])
            else:
                offset = end
            placements.append((offset, size, busy))
            end = max(end, offset + size)
            v.node.attrs["offset"] = offset
        graph.attrs["arena_bytes"] = end
        return {
            "buffers": len(placements),
            "arena_bytes": end,
            "naive_bytes": sum(size for _, size, _ in placements),
            "lower_bound_bytes": peak_live_bytes(ranges),
        }
