"""Static memory planning: pack every arena buffer into one allocation.

Same plan as the reference (kiln/passes/memory_plan.py:43-112), since the
``memory_plan.kir`` fixture pins offsets and the Block's arena must equal the
peak-live lower bound (tests/test_memory_plan.py:42-51):

  * a buffer is live over the closed interval [writer kernel, last reader
    kernel]; reading through a view keeps the viewed buffer alive;
  * buffers are placed largest first (ties by start), each at the lowest
    64-byte-aligned offset that overlaps no placed buffer whose interval
    intersects its own (greedy-by-size first fit);
  * ``reuse=False`` gives every buffer its own slot (the ablation baseline).

On MI355X the arena is one ``hipMalloc`` (a torch uint8 tensor); the plan is
what makes the whole compiled graph replayable as one hipGraph with fixed
addresses.
"""

from __future__ import annotations

from kiln.ir.core import Graph
from kiln.passes.buffers import ALIGNMENT, compute_layouts, kernel_inputs
from kiln.passes.manager import Pass


def align(nbytes: int) -> int:
    return -(-nbytes // ALIGNMENT) * ALIGNMENT


def live_ranges(graph: Graph) -> dict:
    """{owner Value: [first, last]} in kernel indices for every arena buffer."""
    lay = compute_layouts(graph)
    index = {n: i for i, k in enumerate(graph.kernels) for n in k.nodes}
    ranges = {v: [index[v.node]] * 2 for v, l in lay.items() if l.base[0] == "arena" and l.base[1] is v}
    for i, k in enumerate(graph.kernels):
        for v in kernel_inputs(graph, k):
            l = lay.get(v)
            if l is not None and l.base[0] == "arena":
                r = ranges[l.base[1]]
                r[1] = max(r[1], i)
    return ranges


def overlaps(a, b) -> bool:
    return a[0] <= b[1] and b[0] <= a[1]


def peak_live_bytes(ranges) -> int:
    """Lower bound: the most aligned bytes live during any single kernel."""
    if not ranges:
        return 0
    end = max(r[1] for r in ranges.values())
    return max(sum(align(v.type.nbytes) for v, r in ranges.items() if r[0] <= t <= r[1])
               for t in range(end + 1))


class MemoryPlan(Pass):
    name = "memory-plan"

    def __init__(self, reuse: bool = True):
        self.reuse = reuse

    def run(self, graph: Graph):
        ranges = live_ranges(graph)
        placed = []   # (offset, size, range)
        for v in sorted(ranges, key=lambda v: (-v.type.nbytes, ranges[v][0])):
            size = align(v.type.nbytes)
            if self.reuse:
                offset = 0
                for lo, hi in sorted((o, o + s) for o, s, r in placed if overlaps(r, ranges[v])):
                    if offset + size <= lo:
                        break
                    offset = max(offset, hi)
            else:
                offset = sum(s for _, s, _ in placed)
            placed.append((offset, size, ranges[v]))
            v.node.attrs["offset"] = offset
        arena = max((o + s for o, s, _ in placed), default=0)
        graph.attrs["arena_bytes"] = arena
        return {
            "buffers": len(placed),
            "arena_bytes": arena,
            "naive_bytes": sum(s for _, s, _ in placed),
            "lower_bound_bytes": peak_live_bytes(ranges),
        }
