"""Fused attention: recognise scores -> softmax -> (x V) in the fused graph and
merge it into one kernel of kind ``attention`` (the HIP attention family).

After Fusion and BufferAssignment the reference's pipeline turns
``softmax(q @ k^T * c + mask) @ v`` (tests/models/transformer.py:31-42) into
five kernels (kiln/gpu/codegen.py:484-542 then emits one launch each):

    [copy]      K^T made N-contiguous for the matmul (BufferAssignment)
    matmul      scores = q @ k^T, epilogue [* or / scalar] [+ mask]
    reduction   softmax over the last dim: max, sub, exp, sum, div
    matmul      probabilities @ v (no epilogue)
    [copy]      head merge: a transposed view of the result made contiguous

``FuseAttention`` runs after BufferAssignment and before MemoryPlan: it merges
those kernels into one, and drops the storage of the values that become
internal (K^T copy, scores, probabilities, per-head result), so the memory
plan neither reserves the [B, Tq, Tk] scores nor lets the result overlap the
q/k/v buffers that the fused kernel still reads. The graph's nodes and
semantics are unchanged; only the kernel partition and the arena differ from
the reference's pipeline, and only on this backend.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from kiln.hip import lib as kl
from kiln.ir import ops
from kiln.ir.core import Graph, Kernel
from kiln.passes.buffers import compute_layouts, kernel_outputs, order_kernels
from kiln.passes.manager import Pass

HEAD_DIMS = (32, 64)   # head dimensions the HIP attention kernel is built for


@dataclass
class AttentionMatch:
    kernels: list          # the kernels merged, in order
    q: object              # [B, Tq, D]
    k: object              # value whose layout addresses K: [B, D, Tk] (k_transposed) or [B, Tk, D]
    k_transposed: bool
    v: object              # [B, Tk, D]
    mask: object           # additive mask operand or None
    scale_mode: int
    scale: float
    result: object         # value the fused kernel writes
    result_perm: tuple     # result dim i holds per-head output dim result_perm[i]


def _view_perm(v, o):
    """If v is o seen through transposes only, the perm p with v dim i = o dim p[i]."""
    chain = []
    cur = v
    while cur is not o:
        n = cur.node
        if n is None or n.op != "transpose":
            return None
        chain.append(n.attrs["perm"])   # outermost first
        cur = n.inputs[0]
    perm = list(range(o.type.rank))
    for p in reversed(chain):           # transpose: out dim i = in dim p[i]
        perm = [perm[i] for i in p]
    return tuple(perm)


def find_attention(graph: Graph):
    """All attention patterns in a fused, buffer-assigned graph that the HIP
    kernel can run (head dim, unit head-dim stride, 16-byte aligned rows)."""
    users = graph.users()
    results = set(graph.results)
    owner = {n: k for k in graph.kernels for n in k.nodes}
    lay = compute_layouts(graph)
    found = []
    for r in graph.kernels:
        m = _match(graph, r, users, results, owner)
        if m is not None and operand_strides(m, lay) is not None:
            found.append(m)
    return found


def match_kernel(graph: Graph, k: Kernel):
    """The AttentionMatch of a merged ``attention`` kernel (its nodes are split
    back into the five pattern kernels by position)."""
    nodes = list(k.nodes)
    ops_ = [n.op for n in nodes]
    if "reduce_max" not in ops_:
        return None
    j = ops_.index("reduce_max")
    i = 1 if ops_[:2] == ["copy", "matmul"] else 0
    groups = ([nodes[:i]] if i else []) + [nodes[i:j], nodes[j:j + 5], nodes[j + 5:j + 6]]
    if j + 6 < len(nodes):
        groups.append(nodes[j + 6:])
    parts = [Kernel(f"{k.name}.{n}", kind, g) for n, (kind, g) in enumerate(
        zip((["copy"] if i else []) + ["matmul", "reduction", "matmul", "copy"], groups))]
    owner = {n: p for p in parts for n in p.nodes}
    softmax = next(p for p in parts if p.kind == "reduction")
    return _match(graph, softmax, graph.users(), set(graph.results), owner)


def operand_strides(m: AttentionMatch, lay):
    """(q, k, v, out) as (element offset within the buffer, strides over
    (b, t, d)) from the layouts, or None if the kernel cannot address them."""
    out = []
    for v, perm in ((m.q, (0, 1, 2)), (m.k, (0, 2, 1) if m.k_transposed else (0, 1, 2)), (m.v, (0, 1, 2)),
                    (m.result, None)):
        l = lay.get(v)
        if l is None:
            return None
        if perm is None:           # result dim i holds per-head output dim result_perm[i]
            st = [0, 0, 0]
            for i, p in enumerate(m.result_perm):
                st[p] = l.strides[i]
        else:
            st = [l.strides[p] for p in perm]
        if st[2] != 1 or l.offset % 4 or st[0] % 4 or st[1] % 4:
            return None
        out.append((l.offset, tuple(st)))
    return out


def _only_users(users, v, allowed):
    us = users.get(v, [])
    return bool(us) and all(u in allowed for u in us)


def _match(g, r, users, results, owner):
    if r.kind != "reduction" or [n.op for n in r.nodes] != ["reduce_max", "sub", "exp", "reduce_sum", "div"]:
        return None
    mx, sub, ex, sm, dv = r.nodes
    x = mx.inputs[0]
    if x.type.rank != 3:
        return None
    last = [x.type.rank - 1]
    for red in (mx, sm):
        if [d % x.type.rank for d in red.attrs.get("dims", [])] != last or red.out.shape != x.shape[:-1] + (1,):
            return None
    if not (sub.inputs == [x, mx.out] and ex.inputs == [sub.out] and sm.inputs == [ex.out]
            and dv.inputs == [ex.out, sm.out]):
        return None
    prob = dv.out
    if x in results or prob in results or kernel_outputs(g, r, users) != [prob]:
        return None
    if not _only_users(users, x, {mx, sub}):
        return None

    # scores producer: matmul [scale] [mask]
    s = owner.get(x.node)
    if s is None or s.kind != "matmul" or s.nodes[0].op != "matmul":
        return None
    mm = s.nodes[0]
    cur, scale_mode, scale, mask = mm.out, kl.ATTN_SCALE_NONE, 1.0, None
    rest = list(s.nodes[1:])
    if rest and rest[0].op in ("mul", "div") and rest[0].inputs[0] is cur and g.is_scalar_const(rest[0].inputs[1]):
        scale_mode = kl.ATTN_SCALE_MUL if rest[0].op == "mul" else kl.ATTN_SCALE_DIV
        scale = float(g.const_data(rest[0].inputs[1]))
        cur, rest = rest[0].out, rest[1:]
    if rest and rest[0].op == "add" and rest[0].inputs[0] is cur and not g.is_scalar_const(rest[0].inputs[1]):
        mask = rest[0].inputs[1]
        cur, rest = rest[0].out, rest[1:]
    if rest or cur is not x or kernel_outputs(g, s, users) != [x]:
        return None
    if scale_mode == kl.ATTN_SCALE_DIV and scale == 0.0:
        return None
    q, kt = mm.inputs
    if q.type.rank != 3 or kt.type.rank != 3:
        return None
    batch, tq, dh = q.shape
    tk = kt.shape[-1]
    if dh not in HEAD_DIMS or kt.shape[0] != batch or kt.shape[1] != dh or x.shape != (batch, tq, tk):
        return None
    if mask is not None:
        if mask.type.rank > 3 or any(a not in (1, b) for a, b in zip(mask.shape[::-1], (tk, tq, batch))):
            return None

    kernels = [s, r]
    k_src, k_transposed = kt, True
    if kt.node is not None and kt.node.op == "copy":
        c1 = owner.get(kt.node)
        if c1 is None or c1.nodes != [kt.node] or kt in results or not _only_users(users, kt, {mm}):
            return None
        k_src = kt.node.inputs[0]
        kernels.insert(0, c1)

    # probabilities @ v, nothing else in that kernel
    pus = users.get(prob, [])
    if len(pus) != 1 or pus[0].op != "matmul" or pus[0].inputs[0] is not prob:
        return None
    mm2 = pus[0]
    p = owner.get(mm2)
    if p is None or p.nodes != [mm2]:
        return None
    v = mm2.inputs[1]
    if v.type.rank != 3 or v.shape != (batch, tk, dh):
        return None
    o = mm2.out
    kernels.append(p)
    result, perm = o, (0, 1, 2)

    # optional head merge: o -> transpose(s) -> copy, the copy alone in its kernel
    if o not in results:
        chain_users = users.get(o, [])
        if len(chain_users) == 1:
            cur = o
            while len(users.get(cur, [])) == 1 and users[cur][0].op == "transpose":
                cur = users[cur][0].out
            cus = users.get(cur, [])
            if cur is not o and len(cus) == 1 and cus[0].op == "copy":
                c2 = owner.get(cus[0])
                vp = _view_perm(cur, o)
                if c2 is not None and c2.nodes == [cus[0]] and vp is not None:
                    kernels.append(c2)
                    result, perm = cus[0].out, vp
    inside = {n for k in kernels for n in k.nodes}
    for k in kernels:
        for val in kernel_outputs(g, k, users):
            if val is result:
                continue
            # every other value must be consumed only inside the pattern (directly or through views)
            if val in results or not _consumed_inside(users, val, inside):
                return None
    return AttentionMatch(kernels, q, k_src, k_transposed, v, mask, scale_mode, scale, result, perm)


def _consumed_inside(users, v, inside):
    for u in users.get(v, []):
        if u in inside:
            continue
        if ops.kind(u.op) == "view" and _consumed_inside(users, u.out, inside):
            continue
        return False
    return True


class FuseAttention(Pass):
    """Merge each attention pattern into one ``attention`` kernel (see module doc)."""

    name = "fuse-attention"

    def run(self, graph: Graph):
        matches = find_attention(graph)
        for m in matches:
            for k in m.kernels:
                for n in k.nodes:
                    if n.out is not m.result:
                        n.attrs.pop("buffer", None)
            first = graph.kernels.index(m.kernels[0])
            merged = Kernel(m.kernels[0].name, "attention", [n for k in m.kernels for n in k.nodes])
            graph.kernels = [k for k in graph.kernels if all(k is not x for x in m.kernels)]
            graph.kernels.insert(first, merged)
        if not matches:
            return None
        order_kernels(graph)
        lay = compute_layouts(graph)
        for n in graph.nodes:
            if ops.kind(n.op) == "view" and n.out not in lay:
                n.attrs.pop("strides", None)
                n.attrs.pop("offset", None)
        return {"attention": len(matches)}


def causal_or_none(graph: Graph, mask, batch, tq, tk):
    """KH_ATTN_MASK_CAUSAL if the constant mask is 0 on and below the diagonal
    and -inf above it (the frozen ``triu(-inf, 1)`` buffer), else None."""
    if mask is None or not graph.is_const(mask) or mask.type.rank == 0:
        return None
    data = np.asarray(graph.const_data(mask), dtype=np.float32)
    full = np.broadcast_to(data.reshape(mask.shape), (batch, tq, tk) if mask.type.rank == 3 else (tq, tk))
    i = np.arange(tq)[:, None]
    j = np.arange(tk)[None, :]
    above = np.broadcast_to(j > i, (tq, tk))
    ok = np.all(np.isneginf(full[..., above])) and np.all(full[..., ~above] == 0.0)
    return kl.ATTN_MASK_CAUSAL if ok else None
