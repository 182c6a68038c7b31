"""Lower an optimised Kiln graph to kernel-family launch descriptors.

Replaces the reference's Triton code generator (kiln/gpu/codegen.py:145-614).
Instead of writing a kernel's source, each fused Kiln kernel becomes one (or,
for elementwise kernels with outputs of several shapes, a few) ``kh_launch``
descriptors naming a hand-written HIP kernel family:

  matmul kernel           -> GEMM (MFMA) or, for M = 1, GEMV; the fused
                             epilogue becomes a tape over the accumulator
  reduction, innermost    -> ROW; LayerNorm / softmax in the exact form the
                             frontend emits also request the one-wave-per-row
                             fast path
  reduction, other dims   -> RED
  elementwise / copy      -> EW, one launch per distinct output shape
  attention (merged by kiln.hip.attention.FuseAttention)
                          -> ATTN: scores, softmax and (x V) in one launch

Operands are (buffer slot, element offset, element strides over the launch's
iteration space): views never cost a copy, broadcasts are stride 0 - the
same addressing the reference computes in codegen.py:185-219.

Tapes are built over virtual registers, then assigned to the kernels' slots by
linear scan. A tape that fits 8 slots runs with its slots in VGPRs.
"""

from __future__ import annotations

import hashlib
import math
from dataclasses import dataclass, field

from kiln.hip import autotune, bf16
from kiln.hip import lib as kl
from kiln.ir import ops
from kiln.ir.core import Graph, Kernel
from kiln.passes.buffers import Layout, compute_layouts, kernel_inputs, kernel_outputs
from kiln.passes.fusion import is_row_reduction

ROW_SINGLE_CHUNK = 1024   # rows up to this length are held in registers (workgroup x 4)
# rows up to which a LayerNorm runs as the prologue of the small-M GEMM that
# reads it: the prologue's row statistics cost the GEMM time that grows with
# the rows, the LayerNorm launch it saves ~3 us (GPT-2 block, whole call:
# T = 128 0.0470 against 0.0496 ms, T = 256 0.0700 against 0.0713, T = 384
# 0.0947 against 0.0922, T = 512 0.1030 against 0.1020)
LN_PROLOGUE_MAX_ROWS = 256
# queries per workgroup of the blocked attention kernel (kh_launch.cfg[3]):
# 0 lets the library pick (16 for grids that 32-query blocks leave short of
# work); 16 or 32 forces one
ATTN_QUERIES = 0
# the few-query attention kernel's largest query count (kRowsMaxQ in kh_attn.hip)
ATTN_ROWS_MAX_Q = 4
# three-pass plans (allow_tf32) run attention's two products as three-pass
# bf16 on the 32-query kernel where its grid has at least this many
# workgroups (GPT-2 block, 12 heads causal: T = 512 11.9 -> 11.2 us, 1024
# 25.5 -> 20.9, 2048 66.7 -> 52.8); smaller grids keep fp32 products on the
# 16-query kernel, which is faster there (T = 256 6.8 against 7.9 us, T = 128
# 5.2 against 5.8)
ATTN_X3_MIN_GROUPS = 192

_UNARY_OP = {"neg": "neg", "exp": "exp", "tanh": "tanh", "sigmoid": "sigmoid", "relu": "relu",
             "rsqrt": "rsqrt", "sqrt": "sqrt", "erf": "erf", "copy": "mov"}
_BINARY_OP = {"add": "add", "sub": "sub", "mul": "mul", "div": "div", "maximum": "max", "minimum": "min"}


@dataclass
class Launch:
    """One kernel launch of the plan (host-side record + its C descriptor)."""

    name: str
    kernel: str
    family: int
    desc: kl.LaunchDesc
    summary: str
    flops: int = 0
    bytes: int = 0


@dataclass
class Program:
    launches: list = field(default_factory=list)
    consts: list = field(default_factory=list)   # const slot -> constant name
    precision: str = "fp32"
    # constants made at build time from others: name -> (source constant,
    # element offset, strides over (b, k, n), batch, K, N); today the bf16
    # [batch][N][K'] copies of GEMM B operands (kiln/hip/bf16.py)
    derived: dict = field(default_factory=dict)
    # arena buffers: (label, byte offset, bytes, first launch, last launch)
    # - the launches during which the buffer holds a live value (written by
    # the first, read up to the last); the debug runtime poisons a buffer
    # before its first launch and checks the canary after it while it lives
    arena_buffers: list = field(default_factory=list)

    @property
    def source(self) -> str:
        """Human-readable plan listing (the analogue of the reference's
        generated Triton source, codegen.py:601-614)."""
        lines = [f"// Kiln HIP plan: {len(self.launches)} launches, precision {self.precision}"]
        for i, l in enumerate(self.launches):
            lines.append(f"launch {i} {l.name} [{l.kernel}] {kl.FAMILY_NAMES[l.family]}: {l.summary}")
            d = l.desc
            for j in range(d.n_refs):
                r = d.refs[j]
                base = ["input", "output", "const", "arena", "workspace"][r.base]
                lines.append(f"    ref {j}: {base}[{r.index}] +{r.offset} strides {list(r.strides)[:max(d.rank, 3)]}")
            for j in range(d.n_insns):
                ins = d.insns[j]
                lines.append(f"    {j:3d} {kl.OPCODES[ins.op]:<9} dst={ins.dst} a={ins.a} b={ins.b} imm={ins.imm!r}")
        return "\n".join(lines) + "\n"

    def digest(self) -> str:
        return hashlib.sha256(self.source.encode()).hexdigest()[:16]


# ----------------------------------------------------------------------------------
# Tapes over virtual registers.

class _Tape:
    """A straight-line tape over virtual registers, allocated to slots later."""

    def __init__(self):
        self.insns = []          # [op, dst, a, b, imm]; dst/a/b: virtual id, ref index, or None (imm)
        self.n_virt = 0
        self.marks = {}          # virtual -> position it must be live from (row accumulators)

    def virt(self):
        self.n_virt += 1
        return self.n_virt - 1

    def emit(self, op, dst=None, a=None, b=None, imm=0.0):
        self.insns.append([op, dst, a, b, float(imm)])
        return dst

    # operand kinds per opcode
    @staticmethod
    def reads(ins):
        op = ins[0]
        if op == "load":
            return []
        if op == "store":
            return [ins[2]] if ins[2] is not None else []
        if op in ("rsum", "rmax"):
            return [ins[1], ins[2]]
        return [x for x in (ins[2], ins[3]) if x is not None]

    @staticmethod
    def writes(ins):
        return [] if ins[0] == "store" else [ins[1]]


def _allocate(tape: _Tape, loops, limit=kl.NREGS):
    """Linear-scan slot assignment. ``loops`` lists (begin, end) insn ranges
    that execute repeatedly: a value live into a loop stays live through it."""
    first, last = {}, {}
    for i, ins in enumerate(tape.insns):
        for v in tape.writes(ins) + tape.reads(ins):
            first.setdefault(v, i)
            last[v] = i
    for v, pos in tape.marks.items():
        first[v] = min(first.get(v, pos), pos)
        last.setdefault(v, pos)
    for b, e in loops:
        for v in list(first):
            if first[v] < b <= last[v] < e:
                last[v] = e - 1       # defined before the loop, read inside: live to its end
    order = sorted(first, key=lambda v: (first[v], last[v]))
    slot, active, free = {}, [], list(range(limit))
    for v in order:
        start = first[v]
        for u in list(active):
            if last[u] < start:
                active.remove(u)
                free.append(slot[u])
        if not free:
            return None
        free.sort()
        slot[v] = free.pop(0)
        active.append(v)
    return slot


def _encode(tape: _Tape, slot, desc: kl.LaunchDesc, ref_offset=0):
    if len(tape.insns) > kl.MAX_INSNS:
        raise NotImplementedError(f"HIP backend: tape of {len(tape.insns)} instructions exceeds {kl.MAX_INSNS}")
    for i, (op, dst, a, b, imm) in enumerate(tape.insns):
        ins = desc.insns[i]
        ins.op = kl.OP[op]
        ins.imm = imm
        if op == "load":
            ins.dst, ins.a, ins.b = slot[dst], a + ref_offset, 0
        elif op == "store":
            ins.dst, ins.a, ins.b = dst + ref_offset, slot[a], 0
        else:
            ins.dst = slot[dst]
            ins.a = kl.SRC_IMM if a is None else slot[a]
            ins.b = kl.SRC_IMM if b is None else slot[b]
    desc.n_insns = len(tape.insns)
    return max(slot.values(), default=-1) + 1


# ----------------------------------------------------------------------------------

class _Lowerer:
    def __init__(self, graph: Graph, precision: str, matmul_config, gemv_chains: bool = False):
        self.g = graph
        self.gemv_chains = gemv_chains
        self.layouts = compute_layouts(graph)
        self.users = graph.users()
        self.bf16_buffers = set()   # arena buffers held as bf16 (plan_bf16_storage)
        self.pair_buffers = set()   # arena buffers held as pair words (plan_pair_storage)
        self.precision = precision
        self.matmul_config = matmul_config
        self.program = Program(precision=precision)
        self.const_slot = {}
        self._cfg = {}
        self.prologue = {}   # matmul kernel -> (x, gamma, beta, fparams, x as [rows, K]) of a fused LayerNorm
        self.attn_prologue = {}  # GEMV kernel -> (attention match, strides, mask mode, (heads, tk, dh))

    # operands ---------------------------------------------------------------------

    def slot_of(self, base):
        kind = base[0]
        if kind == "input":
            return kl.BASE_INPUT, base[1]
        if kind == "output":
            return kl.BASE_OUTPUT, base[1]
        if kind == "const":
            name = base[1]
            if name not in self.const_slot:
                self.const_slot[name] = len(self.program.consts)
                self.program.consts.append(name)
            return kl.BASE_CONST, self.const_slot[name]
        return kl.BASE_ARENA, 0

    def element_offset(self, v):
        lay = self.layouts[v]
        if lay.base[0] == "arena":
            byte_offset = lay.base[1].node.attrs.get("offset", 0)
            assert byte_offset % 4 == 0
            return byte_offset // 4 + lay.offset
        return lay.offset

    def stored_bf16(self, v) -> bool:
        """Is v's storage an arena buffer held as bf16 (see plan_bf16_storage)?"""
        lay = self.layouts.get(v)
        return lay is not None and lay.base[0] == "arena" and lay.base[1] in self.bf16_buffers

    def stored_pairs(self, v) -> bool:
        """Is v's storage an arena buffer held as pair words (see plan_pair_storage)?"""
        lay = self.layouts.get(v)
        return lay is not None and lay.base[0] == "arena" and lay.base[1] in self.pair_buffers

    def as_bf16(self, r, v):
        """Ref r of v re-expressed over v's bf16 storage: the offset in bf16
        elements (the buffer's byte offset / 2 + v's view offset); strides
        count elements either way."""
        lay = self.layouts[v]
        r.offset = lay.base[1].node.attrs.get("offset", 0) // 2 + lay.offset
        return r

    def plan_bf16_storage(self):
        """bf16 plans: arena buffers that are the A operand of exactly one
        bf16 product on the 64-deep configurations (which read A as bf16) and
        are written by a launch that can round its output to bf16 - the
        one-wave LayerNorm, the blocked attention kernel, or another such
        product with a bias [+ GELU / ReLU] epilogue - are stored as bf16: the
        producer rounds once (to nearest even, as the product would at each
        fragment read), the product copies half the bytes and rounds nothing.
        Results are the same bits as with fp32 storage."""
        out = set()
        if self.precision != "bf16":
            return out
        for k in self.g.kernels:
            if k.kind == "attention":
                buf = self.qkv16_buffer(k)
                if buf is not None:
                    out.add(buf)
                continue
            if k.kind != "matmul" or self.is_gemv(k) or k in self.prologue:
                continue
            cfg, prec = self.matmul_choice(k)
            if prec != "bf16" or int(cfg.get("tile", -1)) not in autotune.BF16_A:
                continue
            buf = self.a16_buffer(k)
            if buf is not None:
                out.add(buf)
        return out

    def plan_pair_storage(self):
        """Three-pass plans: arena buffers whose only reader splits every value
        into bf16 hi and lo halves - the A operand of a three-pass product, or
        the q, k and v of an attention with three-pass products - and whose
        producer can write those halves itself (the one-wave LayerNorm, the
        blocked attention kernel, a three-pass product with a bias [+ GELU /
        ReLU] epilogue and no split-K) are stored as pair words (bf16(x) low,
        bf16(x - bf16(x)) high): the producer splits each value once, the
        reader only regroups halves. Results are the same bits as with fp32
        storage."""
        out = set()
        if self.precision != "bf16x3":
            return out
        for k in self.g.kernels:
            if k.kind == "attention":
                buf = self.qkv_pair_buffer(k)
            elif k.kind == "matmul" and not self.is_gemv(k) and k not in self.prologue:
                buf = self.a_pair_buffer(k)
            else:
                buf = None
            if buf is not None:
                out.add(buf)
        return out

    def a_pair_buffer(self, k, check_choice=True):
        """The arena buffer of three-pass matmul kernel k's A operand if it can
        be stored as pair words: A is the whole buffer with unit K stride, read
        by k alone, not a graph result, and written by a launch that can store
        pair words. Otherwise None. (check_choice=False: before k's
        configuration is chosen, for the tuner's keying, asking only that the
        plan is three-pass.)"""
        if self.precision != "bf16x3" or k in self.prologue:
            return None
        if check_choice and (self.is_gemv(k) or self.matmul_choice(k)[1] != "bf16x3"):
            return None
        mm = next(n for n in k.nodes if n.op == "matmul")
        a, b = mm.inputs
        if a.shape[-2] == 1 or self.layouts[b].base[0] != "const":
            return None
        lay = self.layouts.get(a)
        if lay is None or lay.base[0] != "arena" or lay.offset != 0 or lay.strides[-1] != 1:
            return None
        buf = lay.base[1]
        if self._arena_readers().get(buf) != {k} or buf in self.g.results:
            return None
        producer = self.g.kernel_of(buf.node)
        return buf if producer is not None and self._writes_pairs(producer, buf) else None

    def qkv_pair_buffer(self, k):
        """The arena buffer holding attention kernel k's q, k and v if it can
        be stored as pair words: the attention runs three-pass products, q, k
        and v are views of that one buffer, k reads it alone, and its producer
        can store pair words. Otherwise None."""
        from kiln.hip.attention import match_kernel, operand_strides

        m = match_kernel(self.g, k)
        strides = operand_strides(m, self.layouts) if m is not None else None
        if strides is None or not self.x3_attention(m):
            return None
        bufs = set()
        for v in (m.q, m.k, m.v):
            lay = self.layouts.get(v)
            if lay is None or lay.base[0] != "arena":
                return None
            bufs.add(lay.base[1])
        if len(bufs) != 1:
            return None
        buf = bufs.pop()
        if self._arena_readers().get(buf) != {k} or buf in self.g.results:
            return None
        producer = self.g.kernel_of(buf.node)
        return buf if producer is not None and producer.kind == "matmul" and self._writes_pairs(producer, buf) else None

    def x3_attention(self, m) -> bool:
        """Does the attention matched as m run three-pass products (three-pass
        plans, more than a few queries, a grid of at least ATTN_X3_MIN_GROUPS
        32-query blocks)?"""
        batch, tq, _ = m.q.shape
        return (self.precision == "bf16x3" and tq > ATTN_ROWS_MAX_Q and ATTN_QUERIES != 16
                and batch * -(-tq // 32) >= ATTN_X3_MIN_GROUPS)

    def _writes_pairs(self, k, buf) -> bool:
        """Can kernel k write its output `buf` as pair words?"""
        if k.kind == "attention" or k.kind == "reduction":
            # the blocked attention kernel and the one-wave LayerNorm: the
            # same kernels that can store bf16
            return self._rounds_to_bf16(k, buf, precision="bf16x3")
        if k.kind != "matmul" or self.is_gemv(k) or k in self.prologue:
            return False
        if kernel_outputs(self.g, k, self.users) != [buf]:
            return False
        cfg, prec = self.matmul_choice(k)
        tile = int(cfg.get("tile", -1))
        if prec != "bf16x3" or (tile not in autotune.K_CONTIGUOUS | autotune.SMALL_M and int(cfg.get("splitk", 1)) > 1):
            return False
        return self._bias_act_epilogue(k, buf)

    def _bias_act_epilogue(self, k, buf) -> bool:
        """Is matmul kernel k's tape out = act(acc + bias), act none, GELU or
        ReLU, with out = buf (the library's direct epilogue)?"""
        mm = next(n for n in k.nodes if n.op == "matmul")
        rest = [n for n in k.nodes if n is not mm]
        ops_ = [n.op for n in rest]
        if ops_ not in (["add"], ["add", "gelu"], ["add", "relu"]):
            return False
        bias = rest[0].inputs[1] if rest[0].inputs[0] is mm.out else rest[0].inputs[0]
        chain_ok = rest[0].inputs[0] is mm.out or rest[0].inputs[1] is mm.out
        if len(rest) == 2:
            chain_ok = chain_ok and rest[1].inputs[0] is rest[0].out
        n_cols = mm.out.shape[-1]
        return (chain_ok and rest[-1].out is buf and bias.type.rank >= 1 and bias.shape[-1] == n_cols
                and all(s == 1 for s in bias.shape[:-1]) and n_cols % 4 == 0)

    def _arena_readers(self):
        """arena buffer -> the kernels that read it"""
        if not hasattr(self, "_readers"):
            self._readers = {}
            for k in self.g.kernels:
                members = set(k.nodes)
                for n in k.nodes:
                    for v in n.inputs:
                        lay = self.layouts.get(v)
                        if lay is not None and lay.base[0] == "arena" and v.node not in members:
                            self._readers.setdefault(lay.base[1], set()).add(k)
        return self._readers

    def a16_buffer(self, k):
        """The arena buffer of matmul kernel k's A operand if it can be stored
        as bf16 for a product that reads A that way: A is the whole buffer,
        K-contiguous with 16-byte aligned rows, read by k alone, not a graph
        result, and written by a launch that can round its output to bf16.
        Otherwise None. (Whether k reads A as bf16 depends on its tile; this
        does not ask.)"""
        if self.precision != "bf16" or k.kind != "matmul" or k in self.prologue:
            return None
        mm = next(n for n in k.nodes if n.op == "matmul")
        a, b = mm.inputs
        if a.shape[-2] == 1 or self.layouts[b].base[0] != "const":
            return None
        lay = self.layouts.get(a)
        if lay is None or lay.base[0] != "arena" or lay.offset != 0 or lay.strides[-1] != 1:
            return None
        buf = lay.base[1]
        if a.shape[-1] % 8 or any(st % 8 for st, ext in zip(lay.strides[:-1], lay.shape[:-1]) if ext > 1):
            return None
        if self._arena_readers().get(buf) != {k} or buf in self.g.results:
            return None
        producer = self.g.kernel_of(buf.node)
        return buf if producer is not None and self._rounds_to_bf16(producer, buf) else None

    def qkv16_buffer(self, k):
        """The arena buffer holding attention kernel k's q, k and v if it can
        be stored as bf16: the attention runs bf16 products on the 32-query
        kernel (more than a few queries, not forced to 16 per workgroup), q, k
        and v are views of that one buffer with unit head-dim stride and
        16-byte aligned rows in bf16, k reads it alone, and its producer can
        round its output to bf16 (the rounding the products do when they form
        their operands, so the bits do not change). Otherwise None."""
        from kiln.hip.attention import match_kernel, operand_strides

        m = match_kernel(self.g, k)
        strides = operand_strides(m, self.layouts) if m is not None else None
        if strides is None or m.q.shape[1] <= ATTN_ROWS_MAX_Q or ATTN_QUERIES == 16:
            return None
        bufs = set()
        for v, (_, st) in zip((m.q, m.k, m.v), strides):
            lay = self.layouts.get(v)
            if lay is None or lay.base[0] != "arena" or st[2] != 1 or st[0] % 8 or st[1] % 8 or lay.offset % 8:
                return None
            bufs.add(lay.base[1])
        if len(bufs) != 1:
            return None
        buf = bufs.pop()
        if self._arena_readers().get(buf) != {k} or buf in self.g.results:
            return None
        producer = self.g.kernel_of(buf.node)
        return buf if producer is not None and producer.kind == "matmul" and self._rounds_to_bf16(producer, buf) else None

    def _rounds_to_bf16(self, k, buf, precision="bf16") -> bool:
        """Can kernel k write its output `buf` as bf16? (With precision
        "bf16x3", only its LayerNorm and attention cases are asked, for pair
        words, which the same kernels write.)"""
        outs = kernel_outputs(self.g, k, self.users)
        if k.kind == "attention":
            from kiln.hip.attention import match_kernel

            m = match_kernel(self.g, k)
            return (m is not None and self.layouts[m.result].base == ("arena", buf) and m.q.shape[1] > 4
                    and all(st % 4 == 0 for st in self.layouts[m.result].strides[:-1]))
        if outs != [buf]:
            return False
        if k.kind == "reduction":
            reds = [n for n in k.nodes if n.op.startswith("reduce_")]
            if not reds or not all(is_row_reduction(n) for n in reds):
                return False
            members = set(k.nodes)
            externals = []
            for n in k.nodes:
                for v in n.inputs:
                    if (v.node not in members or v.node is None) and not self.is_imm(v) and v not in externals:
                        externals.append(v)
            variant = self._row_pattern(k, reds, outs, externals)[0]
            inner = buf.shape[-1]
            return variant == kl.ROW_LAYERNORM and inner % 4 == 0 and inner <= 4096
        if k.kind == "matmul" and not self.is_gemv(k) and k not in self.prologue and precision == "bf16":
            cfg, prec = self.matmul_choice(k)
            if prec != "bf16" or int(cfg.get("tile", -1)) not in autotune.BF16_A:
                return False
            return self._bias_act_epilogue(k, buf)
        return False

    def ref(self, v, space):
        """kh_ref for value v read over iteration space `space` (right-aligned
        broadcasting: size-1 dims of v get stride 0)."""
        if v not in self.layouts:
            raise NotImplementedError(f"HIP backend: value {v} has no storage")
        lay = self.layouts[v]
        r = kl.Ref()
        r.base, r.index = self.slot_of(lay.base)
        r.offset = self.element_offset(v)
        rank = len(space)
        lead = rank - len(lay.shape)
        if lead < 0:
            raise NotImplementedError(f"HIP backend: operand {v} has higher rank than its kernel")
        for i, (s, st) in enumerate(zip(lay.shape, lay.strides)):
            r.strides[lead + i] = 0 if s == 1 else st
        return r

    def new_desc(self, family, name, kernel, space):
        d = kl.LaunchDesc()
        d.family = family
        d.rank = len(space)
        if d.rank > kl.MAX_RANK:
            raise NotImplementedError(f"HIP backend: rank {d.rank} > {kl.MAX_RANK}")
        for i, s in enumerate(space):
            d.shape[i] = s
        d.name = f"{kernel.name}_{name}".encode()[:31]
        return d

    def add(self, d, kernel, summary, flops=0, nbytes=0):
        self.program.launches.append(Launch(d.name.decode(), kernel.name, d.family, d, summary, flops, nbytes))

    def is_imm(self, v):
        return self.g.is_scalar_const(v)

    def imm(self, v):
        return float(self.g.const_data(v))

    # elementwise ---------------------------------------------------------------------------

    def lower_elementwise(self, k: Kernel):
        outs = kernel_outputs(self.g, k, self.users)
        by_shape = {}
        for v in outs:
            by_shape.setdefault(tuple(v.shape), []).append(v)
        members = set(k.nodes)
        for i, (shape, group) in enumerate(by_shape.items()):
            d = self.new_desc(kl.FAM_EW, f"ew{i}", k, shape)
            refs, ref_of = [], {}
            needed = self._needed(group, members)
            externals = []
            for n in k.nodes:
                if n.out in needed:
                    for v in n.inputs:
                        if (v.node not in members or v.node is None) and not self.is_imm(v) and v not in externals:
                            externals.append(v)
            for v in externals:
                ref_of[v] = len(refs)
                refs.append(self.ref(v, shape))
            out_ref = {}
            for v in group:
                out_ref[v] = len(refs)
                refs.append(self.ref(v, shape))
            self._check_refs(refs)
            for j, r in enumerate(refs):
                d.refs[j] = r
            d.n_refs = len(refs)

            def build(eager_loads):
                t = _Tape()
                env = {}
                if eager_loads:
                    for v in externals:
                        env[v] = t.emit("load", t.virt(), ref_of[v])
                self._emit_dag(t, env, group, members, k.nodes, ref_of)
                for v in group:
                    t.emit("store", out_ref[v], env[v])
                return t

            self._finish_tape(d, build, loops=[])
            nbytes = 4 * (sum(math.prod(v.shape) for v in externals) + len(group) * math.prod(shape))
            ops_list = " ".join(n.op for n in k.nodes if n.out in needed)
            self.add(d, k, f"shape {list(shape)}: {ops_list}", nbytes=nbytes)

    @staticmethod
    def _needed(wanted, members, stop=()):
        """Member values `wanted` depends on, not looking past values in `stop`."""
        need, todo = set(), list(wanted)
        while todo:
            v = todo.pop()
            if v in need or v.node not in members or v in stop:
                continue
            need.add(v)
            todo.extend(v.node.inputs)
        return need

    def _emit_dag(self, t, env, wanted, members, order, ref_of, node_ok=None):
        """Emit the members needed for `wanted` (program order), loading
        externals on first use when not already in env."""
        need = self._needed(wanted, members, stop=env)

        def operand(v):
            if v in env:
                return env[v]
            if self.is_imm(v):
                return None
            if v.node in members and v.node is not None:
                raise AssertionError(f"value {v} used before it is computed")
            env[v] = t.emit("load", t.virt(), ref_of[v])
            return env[v]

        for n in order:
            if n.out not in need or n.out in env:
                continue
            if node_ok is not None and not node_ok(n):
                continue
            self._emit_node(t, env, n, operand)

    def _emit_node(self, t, env, n, operand):
        op = n.op
        if op in _BINARY_OP:
            a, b = n.inputs
            ra, rb = operand(a), operand(b)
            if ra is None and rb is None:       # both scalar constants: materialise one
                ra = t.emit("mov", t.virt(), None, None, self.imm(a))
            imm = self.imm(a) if ra is None else (self.imm(b) if rb is None else 0.0)
            env[n.out] = t.emit(_BINARY_OP[op], t.virt(), ra, rb, imm)
        elif op == "gelu":
            ra = operand(n.inputs[0])
            opname = "gelu_tanh" if n.attrs.get("approximate", "none") == "tanh" else "gelu_erf"
            imm = self.imm(n.inputs[0]) if ra is None else 0.0
            env[n.out] = t.emit(opname, t.virt(), ra, None, imm)
        elif op in _UNARY_OP:
            ra = operand(n.inputs[0])
            imm = self.imm(n.inputs[0]) if ra is None else 0.0
            env[n.out] = t.emit(_UNARY_OP[op], t.virt(), ra, None, imm)
        else:
            raise NotImplementedError(f"GPU backend: no lowering for '{op}'")

    def _finish_tape(self, d, build, loops, limit=kl.NREGS, ref_offset=0, preset=None):
        """Build the tape (loads first, else loads on demand), allocate, encode.
        Returns the slot count."""
        best = None
        for eager in (True, False):
            t = build(eager)
            lp = loops(t) if callable(loops) else loops
            slot = _allocate(t, lp, limit)
            if preset is not None and slot is not None:
                slot = self._pin(t, slot, preset, lp, limit)
            if slot is None:
                continue
            used = max(slot.values(), default=-1) + 1
            if best is None or used < best[0] or (used <= kl.FAST_SLOTS and eager):
                best = (used, t, slot)
            if used <= kl.FAST_SLOTS:
                break
        if best is None:
            raise NotImplementedError(f"HIP backend: fused kernel needs more than {limit} registers")
        return _encode(best[1], best[2], d, ref_offset)

    @staticmethod
    def _pin(t, slot, preset, loops, limit):
        """Re-run allocation with virtual `preset[0]` forced into slot preset[1]."""
        v0, s0 = preset
        if slot.get(v0) == s0:
            return slot
        # swap slots s0 and slot[v0] globally (valid: a permutation of slots)
        other = slot.get(v0)
        out = {}
        for v, s in slot.items():
            out[v] = other if s == s0 else (s0 if s == other else s)
        return out

    @staticmethod
    def _check_refs(refs):
        if len(refs) > kl.MAX_REFS:
            raise NotImplementedError(f"HIP backend: kernel has {len(refs)} operands (max {kl.MAX_REFS})")

    # row kernels ------------------------------------------------------------------------------

    def lower_reduction(self, k: Kernel):
        reds = [n for n in k.nodes if n.op.startswith("reduce_")]
        if all(is_row_reduction(n) for n in reds):
            return self.lower_row(k, reds)
        if len(k.nodes) != 1:
            raise NotImplementedError("GPU backend: a non-innermost reduction must be alone in its kernel")
        return self.lower_red(k, reds[0])

    def lower_red(self, k, n):
        x, out = n.inputs[0], n.out
        space = tuple(x.shape)
        d = self.new_desc(kl.FAM_RED, "reduce", k, space)
        outs = kernel_outputs(self.g, k, self.users)
        if outs != [out]:
            raise NotImplementedError("GPU backend: reduction kernel with extra outputs")
        d.refs[0] = self.ref(x, space)
        lay = self.layouts[out]
        r = kl.Ref()
        r.base, r.index = self.slot_of(lay.base)
        r.offset = self.element_offset(out)
        for i, (s, st) in enumerate(zip(lay.shape, lay.strides)):
            r.strides[i] = 0 if s == 1 else st
        d.refs[1] = r
        d.n_refs = 2
        dims = {dd % x.type.rank for dd in n.attrs["dims"]}
        d.cfg[0] = sum(1 << dd for dd in dims)
        d.cfg[1] = 1 if n.op == "reduce_max" else 0
        nbytes = 4 * (math.prod(x.shape) + math.prod(out.shape))
        self.add(d, k, f"{n.op} dims {sorted(dims)} of {list(x.shape)}", nbytes=nbytes)

    def lower_row(self, k, reds):
        shape = tuple(reds[0].inputs[0].shape)
        rows, inner = shape[:-1], shape[-1]
        members = set(k.nodes)
        outs = kernel_outputs(self.g, k, self.users)
        single = inner <= ROW_SINGLE_CHUNK

        def is_vec(v):
            return v.type.rank > 0 and v.shape[-1] == inner

        # levels: reductions completed before a value is available
        level = {}
        for n in k.nodes:
            lv = max([level[v] for v in n.inputs if v in level], default=0)
            level[n.out] = lv + (1 if n.op.startswith("reduce_") else 0)
        depth = max(level[n.out] for n in reds)

        externals = []
        for n in k.nodes:
            for v in n.inputs:
                if (v.node not in members or v.node is None) and not self.is_imm(v) and v not in externals:
                    externals.append(v)
        variant, fparams, cfg45, ordered = self._row_pattern(k, reds, outs, externals)
        if ordered is not None:
            externals = ordered
        refs, ref_of = [], {}
        for v in externals:
            ref_of[v] = len(refs)
            refs.append(self.ref(v, shape))
        out_ref = {}
        bf16_mask = 0
        for v in outs:
            out_ref[v] = len(refs)
            r = self.ref(v, shape)
            if self.stored_bf16(v):
                r = self.as_bf16(r, v)
                bf16_mask |= 1 << out_ref[v]
            if self.stored_pairs(v):
                bf16_mask |= 1 << (16 + out_ref[v])
            refs.append(r)
        self._check_refs(refs)

        d = self.new_desc(kl.FAM_ROW, "row", k, shape)
        d.cfg[7] = bf16_mask
        for j, r in enumerate(refs):
            d.refs[j] = r
        d.n_refs = len(refs)
        d.variant = variant
        for i, f in enumerate(fparams):
            d.fparams[i] = f
        d.cfg[4], d.cfg[5] = cfg45

        def build(_eager):
            t = _Tape()
            persist = {}      # values whose slots stay valid for the rest of the row
            segments = []     # per pass: (vec_begin, vec_end, post_begin, post_end, accs, maxs)
            for p in range(depth + 1):
                final = p == depth
                seg_reds = [n for n in reds if level[n.out] == p + 1]
                # accumulators live from the pass start
                accs = {}
                for n in seg_reds:
                    v = t.virt()
                    t.marks[v] = len(t.insns)
                    accs[n.out] = v
                vb = len(t.insns)
                env = dict(persist)
                # leading loads: externals this segment reads directly
                wanted = [n.inputs[0] for n in seg_reds]
                if final:
                    wanted = [v for v in outs if is_vec(v)]

                def vec_ok(n):
                    return is_vec(n.out) or level[n.out] == 0

                need = self._needed(wanted, members, stop=env)
                for v in wanted:
                    if v not in env and (v.node not in members or v.node is None):
                        env[v] = t.emit("load", t.virt(), ref_of[v])
                for n in k.nodes:
                    if n.out in need and vec_ok(n):
                        for v in n.inputs:
                            if v not in env and not self.is_imm(v) and (v.node not in members or v.node is None):
                                env[v] = t.emit("load", t.virt(), ref_of[v])
                self._emit_dag(t, env, wanted, members, k.nodes, ref_of, node_ok=vec_ok)
                for n in seg_reds:
                    t.emit("rsum" if n.op == "reduce_sum" else "rmax", accs[n.out], env[n.inputs[0]])
                if final:
                    for v in outs:
                        if is_vec(v):
                            t.emit("store", out_ref[v], env[v])
                ve = len(t.insns)
                if single:
                    persist.update(env)
                for n in seg_reds:
                    persist[n.out] = accs[n.out]
                # post segment: per-row scalars at the next level (and scalar outputs at the end)
                pb = len(t.insns)
                penv = dict(persist)
                if final:
                    scalars = [v for v in outs if not is_vec(v)]
                else:
                    scalars = [n.out for n in k.nodes if level[n.out] == p + 1 and not is_vec(n.out)
                               and not n.op.startswith("reduce_")]
                self._emit_dag(t, penv, scalars, members, k.nodes, ref_of,
                               node_ok=lambda n: not is_vec(n.out))
                if final:
                    for v in outs:
                        if not is_vec(v):
                            t.emit("store", out_ref[v], penv[v])
                pe = len(t.insns)
                for v in scalars:
                    persist[v] = penv[v]
                for v, r in penv.items():
                    if v.node is not None and v.node in members and not is_vec(v):
                        persist.setdefault(v, r)
                acc_list = [accs[n.out] for n in seg_reds]
                max_list = [accs[n.out] for n in seg_reds if n.op == "reduce_max"]
                segments.append((vb, ve, pb, pe, acc_list, max_list))
            t.segments = segments
            return t

        def loops(t):
            return [] if single else [(s[0], s[1]) for s in t.segments]

        # loads are placed at the start of the segment that reads them
        t = build(True)
        slot = _allocate(t, loops(t), kl.NREGS)
        if slot is None:
            raise NotImplementedError("HIP backend: row kernel needs more than 16 registers")
        _encode(t, slot, d)
        if len(t.segments) > kl.MAX_PASSES:
            raise NotImplementedError(f"HIP backend: row kernel with {len(t.segments)} passes")
        for i, (vb, ve, pb, pe, accs, maxs) in enumerate(t.segments):
            P = d.passes[i]
            P.vec_begin, P.vec_end, P.post_begin, P.post_end = vb, ve, pb, pe
            P.acc_mask = sum(1 << slot[v] for v in accs)
            P.max_mask = sum(1 << slot[v] for v in maxs)
            P.single_chunk = 1 if single else 0
        d.n_passes = len(t.segments)
        nbytes = 4 * (sum(math.prod(v.shape) for v in externals) + sum(math.prod(v.shape) for v in outs))
        kind = {kl.ROW_LAYERNORM: "layernorm", kl.ROW_SOFTMAX: "softmax"}.get(variant, "generic")
        if bf16_mask & 0xFFFF:
            kind += " out:bf16"
            nbytes -= 2 * sum(math.prod(v.shape) for v in outs)
        if bf16_mask >> 16:
            kind += " out:pairs"
        self.add(d, k, f"{kind} rows {list(rows)} x {inner}, {len(t.segments)} passes"
                       f"{'' if single else ' (chunked)'}: {' '.join(n.op for n in k.nodes)}", nbytes=nbytes)

    def _row_pattern(self, k, reds, outs, externals):
        """Recognise the frontend's LayerNorm / softmax decompositions
        (kiln/frontend/fx_import.py:212-230). Returns (variant, fparams,
        (cfg4, cfg5), ordered externals or None)."""
        nodes = k.nodes
        none = (kl.ROW_GENERIC, [], (0, 0), None)
        if len(outs) != 1 or outs[0].node not in set(nodes):
            return none
        out = outs[0]
        imm = lambda v: self.imm(v) if self.is_imm(v) else None
        ops_ = [n.op for n in nodes]
        # softmax: [pre] reduce_max, sub, exp, reduce_sum, div
        if ops_[-5:] == ["reduce_max", "sub", "exp", "reduce_sum", "div"] and len(nodes) in (5, 6):
            mx, sub, ex, sm, dv = nodes[-5:]
            pre, pre_scale, x = 0, 0.0, mx.inputs[0]
            if len(nodes) == 6:
                p = nodes[0]
                if p.op not in ("mul", "div") or p.out is not x or imm(p.inputs[1]) is None:
                    return none
                pre, pre_scale, x = (1 if p.op == "mul" else 2), imm(p.inputs[1]), p.inputs[0]
            ok = (sub.inputs == [mx.inputs[0], mx.out] and ex.inputs == [sub.out] and sm.inputs == [ex.out]
                  and dv.inputs == [ex.out, sm.out] and dv.out is out and x not in set(n.out for n in nodes))
            if ok and externals == [x]:
                return kl.ROW_SOFTMAX, [pre_scale], (pre, 0), [x]
            return none
        # layernorm: reduce_sum, mul c, sub, mul, reduce_sum, mul c, add eps, rsqrt, mul, [mul g], [add b]
        if len(nodes) >= 9 and ops_[:9] == ["reduce_sum", "mul", "sub", "mul", "reduce_sum", "mul", "add",
                                            "rsqrt", "mul"]:
            s1, m1, xc, sq, s2, m2, ad, rs, y = nodes[:9]
            x = s1.inputs[0]
            c1, c2, eps = imm(m1.inputs[1]), imm(m2.inputs[1]), imm(ad.inputs[1])
            ok = (None not in (c1, c2, eps) and m1.inputs[0] is s1.out and xc.inputs == [x, m1.out]
                  and sq.inputs == [xc.out, xc.out] and s2.inputs == [sq.out] and m2.inputs[0] is s2.out
                  and ad.inputs[0] is m2.out and rs.inputs == [ad.out] and y.inputs == [xc.out, rs.out])
            if not ok:
                return none
            rest, cur, gamma, beta = nodes[9:], y.out, None, None
            if rest and rest[0].op == "mul" and rest[0].inputs[0] is cur and not self.is_imm(rest[0].inputs[1]):
                gamma, cur, rest = rest[0].inputs[1], rest[0].out, rest[1:]
            if rest and rest[0].op == "add" and rest[0].inputs[0] is cur and not self.is_imm(rest[0].inputs[1]):
                beta, cur, rest = rest[0].inputs[1], rest[0].out, rest[1:]
            if rest or cur is not out:
                return none
            inner = x.shape[-1]
            for p in (gamma, beta):
                if p is not None and (p.type.rank < 1 or p.shape[-1] != inner
                                      or any(s != 1 for s in p.shape[:-1])):
                    return none
            ordered = [x] + [p for p in (gamma, beta) if p is not None]
            if sorted(map(id, ordered)) != sorted(map(id, externals)) or len(set(map(id, ordered))) != len(ordered):
                return none
            return kl.ROW_LAYERNORM, [c1, c2, eps], (int(gamma is not None), int(beta is not None)), ordered
        return none

    # matmul -----------------------------------------------------------------------------------

    def lower_matmul(self, k: Kernel):
        mm = next(n for n in k.nodes if n.op == "matmul")
        a, b = mm.inputs
        out_shape = tuple(mm.out.shape)
        batch = math.prod(a.shape[:-2]) if a.type.rank == 3 else 1
        m, kk, n = a.shape[-2], a.shape[-1], b.shape[-1]
        members = set(k.nodes)
        outs = kernel_outputs(self.g, k, self.users)
        space3 = (batch, m, n)

        def ref3(v, dims, register=True, lay=None):
            """Strides of v over a 3-d space named by `dims` (v's own dims
            right-aligned; `lay`: v's storage seen with other dims, the same
            base and offset). register=False describes a constant that is only
            read through a derived copy, so it gets no slot (and is not
            uploaded)."""
            lay = lay or self.layouts[v]
            r = kl.Ref()
            r.base, r.index = self.slot_of(lay.base) if register else (kl.BASE_CONST, -1)
            r.offset = self.element_offset(v)
            lead = 3 - len(lay.shape)
            for i, (s, st) in enumerate(zip(lay.shape, lay.strides)):
                r.strides[lead + i] = 0 if s == 1 and dims[lead + i] != 1 else st
            return r

        if a not in self.layouts or b not in self.layouts:
            raise NotImplementedError("HIP backend: matmul operand has no storage")
        cfg, prec = self.matmul_choice(k)
        gemv = self.is_gemv(k)
        pro = self.prologue.get(k)
        a_src = pro[0] if pro else a   # the LayerNorm's input when the product runs it as its prologue
        d = self.new_desc(kl.FAM_GEMV if gemv else kl.FAM_GEMM, "gemv" if gemv else "matmul", k, space3)
        if gemv and self.gemv_chains:
            d.variant = kl.GEMV_CHAIN   # the library may run it in a persistent chain with its GEMV neighbours
        d.gemm[0], d.gemm[1], d.gemm[2], d.gemm[3] = batch, m, n, kk
        d.refs[0] = ref3(a_src, (batch, m, kk), lay=pro[4] if pro else None)
        if not pro and self.stored_bf16(a):
            d.refs[0] = self.as_bf16(d.refs[0], a)
            d.cfg[7] |= 1
        if not pro and not gemv and self.stored_pairs(a):
            d.cfg[7] |= 1 << 16
        k_major = not gemv and int(cfg.get("tile", -1)) in autotune.NK_B
        nk = (gemv and self.layouts[b].base[0] == "const" and kk % 4 == 0) or k_major
        derived_b = prec in ("bf16", "bf16x3") or nk
        d.refs[1] = b_ref = ref3(b, (batch, kk, n), register=not derived_b)
        if prec in ("bf16", "bf16x3"):
            d.refs[1] = self.bf16_weight(b, d.refs[1], batch, kk, n, split=prec == "bf16x3")
        elif nk:
            d.refs[1] = self.nk_weight(b, b_ref, batch, kk, n, scale=pro[1] if pro and not gemv else None)
        externals = []
        for nd in k.nodes:
            if nd is mm:
                continue
            for v in nd.inputs:
                if v is not mm.out and (v.node not in members or v.node is None) and not self.is_imm(v) \
                        and v not in externals:
                    externals.append(v)
        refs, ref_of = [], {}
        for v in externals:
            ref_of[v] = len(refs)
            refs.append(ref3(v, space3))
        out_ref = {}
        for v in outs:
            out_ref[v] = len(refs)
            r = ref3(v, space3)
            if self.stored_bf16(v):
                r = self.as_bf16(r, v)
                d.cfg[7] |= 1 << (2 + out_ref[v])
            if self.stored_pairs(v):
                d.cfg[7] |= 1 << (16 + 2 + out_ref[v])
            refs.append(r)
        pro_refs = []
        attn_work = None
        if gemv and k in self.attn_prologue:
            pro_refs, *attn_work = self.attn_prologue_refs(d, k, 2 + len(refs))
        if pro:
            x, gamma, beta, fparams, _ = pro
            d.cfg[4], d.cfg[5], d.cfg[6] = 1, -1, -1
            if gemv:
                for w, p in ((5, gamma), (6, beta)):
                    if p is not None:
                        d.cfg[w] = 2 + len(refs) + len(pro_refs)
                        pro_refs.append(ref3(p, (batch, m, kk)))
            else:
                # gamma rides in the weight copy; that copy's column sums and
                # beta . W are column constants
                d.cfg[5] = 2 + len(refs) + len(pro_refs)
                pro_refs.append(self.ln_column(b, b_ref, batch, kk, n, gamma, "lng"))
                if beta is not None:
                    d.cfg[6] = 2 + len(refs) + len(pro_refs)
                    pro_refs.append(self.ln_column(b, b_ref, batch, kk, n, beta, "lnc"))
            for i, f in enumerate(fparams):
                d.fparams[i] = f
        self._check_refs(refs + pro_refs + [None, None])
        for j, r in enumerate(refs + pro_refs):
            d.refs[2 + j] = r
        d.n_refs = 2 + len(refs) + len(pro_refs)

        def build(eager):
            t = _Tape()
            acc = t.virt()
            t.marks[acc] = 0
            env = {mm.out: acc}
            if eager:
                for v in externals:
                    env[v] = t.emit("load", t.virt(), ref_of[v])
            self._emit_dag(t, env, outs, members, k.nodes, ref_of)
            for v in outs:
                t.emit("store", out_ref[v], env[v])
            t.acc = acc
            return t

        # slot 0 must hold the accumulator on entry
        best = None
        for eager in (True, False):
            t = build(eager)
            slot = _allocate(t, [], kl.FAST_SLOTS)
            if slot is None:
                continue
            slot = self._pin(t, slot, (t.acc, 0), [], kl.FAST_SLOTS)
            best = (t, slot)
            break
        if best is None:
            raise NotImplementedError("HIP backend: matmul epilogue needs more than 8 registers")
        _encode(best[0], best[1], d, ref_offset=2)
        if gemv:
            # GEMV family: "tile" picks the workgroup variant of the [K][N]
            # kernel (0 = from the shape, 1-5), split-K 0 = from the shape
            cfg = {"tile": int(cfg.get("tile", 0)) if 0 <= int(cfg.get("tile", 0)) <= 5 else 0,
                   "splitk": int(cfg.get("gemv_splitk", cfg.get("splitk", 0))),
                   "precision": cfg.get("precision", self.precision)}
        d.cfg[1] = int(cfg.get("tile", 0))
        d.cfg[2] = int(cfg.get("splitk", 1))
        d.cfg[3] = {"fp32": kl.PREC_FP32, "bf16": kl.PREC_BF16, "bf16x3": kl.PREC_BF16X3}[prec]
        flops = 2 * batch * m * n * kk
        nbytes = 4 * (math.prod(a.shape) + math.prod(b.shape) + sum(math.prod(v.shape) for v in externals)
                      + len(outs) * math.prod(out_shape))
        epi = " ".join(nd.op for nd in k.nodes if nd is not mm)
        summary = f"{batch}x{m}x{n}x{kk}"
        summary += f" tile {d.cfg[1]} splitk {d.cfg[2]}"
        if prec != "fp32":
            summary += f" {prec}"
        if prec == "bf16":   # B read as its bf16 copy (the three-pass copy holds 2 bf16 per weight)
            nbytes -= 2 * math.prod(b.shape)
        if not gemv and d.cfg[7] & 1:   # (a GEMV's cfg[7] is its attention prologue's key count)
            summary += " A:bf16"
            nbytes -= 2 * math.prod(a.shape)
        if any(self.stored_bf16(v) for v in outs):
            summary += " out:bf16"
            nbytes -= 2 * math.prod(out_shape)
        if not gemv and d.cfg[7] >> 16 & 1:
            summary += " A:pairs"
        if any(self.stored_pairs(v) for v in outs):
            summary += " out:pairs"
        if pro:
            summary += " prologue: layernorm"
            nbytes += 4 * kk * len(pro_refs)
        if attn_work:
            summary += " prologue: attention"
            flops += attn_work[0]
            nbytes += attn_work[1] - 4 * kk
        if epi:
            summary += f" epilogue: {epi}"
        self.add(d, k, summary, flops=flops, nbytes=nbytes)

    def is_gemv(self, k: Kernel) -> bool:
        """A one-row matmul runs on the GEMV family: in fp32 always, in bf16
        when B is a constant (read as its bf16 [batch][N][K] copy) and K is a
        multiple of 8 (whole 16-byte weight chunks); other bf16 / bf16x3
        one-row products run on the GEMM tiles."""
        mm = next(n for n in k.nodes if n.op == "matmul")
        return self._gemv_at(mm, self.matmul_choice(k)[1])

    def _gemv_at(self, mm, prec) -> bool:
        a, b = mm.inputs
        if a.shape[-2] != 1:
            return False
        if prec == "fp32":
            return True
        return prec == "bf16" and self.layouts[b].base[0] == "const" and a.shape[-1] % 8 == 0

    def matmul_choice(self, k: Kernel):
        """(configuration, precision) of matmul kernel k, asked once per kernel."""
        if k not in self._cfg:
            mm = next(n for n in k.nodes if n.op == "matmul")
            if getattr(self.matmul_config, "accepts_a16", False) and (
                    self.a16_buffer(k) is not None or self.a_pair_buffer(k, check_choice=False) is not None):
                # the tuner times this product reading A as bf16 / pair words, as the plan can store it
                cfg = dict(self.matmul_config(self.g, k, a16=True))
            else:
                cfg = dict(self.matmul_config(self.g, k))
            prec = cfg.get("precision", self.precision)
            if prec in ("bf16", "bf16x3") and self.layouts[mm.inputs[1]].base[0] != "const":
                # bf16 inputs need B as a build-time bf16 copy of a constant; a
                # matmul on two activations stays on the fp32 path (more exact)
                prec = "fp32"
            a, b = mm.inputs
            batch = math.prod(a.shape[:-2]) if a.type.rank == 3 else 1
            m, n, kk = a.shape[-2], b.shape[-1], a.shape[-1]
            tile = int(cfg.get("tile", -1))
            if not self._gemv_at(mm, prec) and autotune.PRECISION.get(tile) != prec:
                # a configuration of another precision (e.g. the fp32 fallback
                # above): the default of this one, [N][K] configurations only
                # when B can be copied that way
                cfg = {**cfg, **autotune.default_config_for(batch, m, n, kk, precision=prec,
                                                            skinny=self.skinny_ok(mm))}
                tile = int(cfg.get("tile", -1))
            if tile in autotune.NK_B and not (self.skinny_ok(mm) and autotune.k_major_fits(m, kk, tile)):
                cfg = autotune.default_config_for(batch, m, n, kk, precision=prec, skinny=False)
            self._cfg[k] = (cfg, prec)
        return self._cfg[k]

    def skinny_ok(self, mm) -> bool:
        """The skinny-M and K-contiguous GEMMs read B as a build-time
        [batch][N][K] copy of a constant and A as 16-byte pieces along K (unit
        K stride)."""
        a, b = mm.inputs
        la, lb = self.layouts.get(a), self.layouts.get(b)
        return (la is not None and lb is not None and lb.base[0] == "const" and a.shape[-1] % 4 == 0
                and la.strides[-1] == 1 and la.offset % 4 == 0
                and all(st % 4 == 0 for st, ext in zip(la.strides[:-1], la.shape[:-1]) if ext > 1))

    def _arena_range(self, v):
        """Byte range [lo, hi) of v's storage in the arena, or None."""
        lay = self.layouts.get(v)
        if lay is None or lay.base[0] != "arena":
            return None
        buf = lay.base[1]
        lo = buf.node.attrs.get("offset", 0)
        return lo, lo + buf.type.nbytes

    def find_ln_prologues(self):
        """LayerNorm row kernels whose only consumer is the A operand of a
        1-row fp32 matmul (decode: ln_1 -> qkv, ln_2 -> fc) or of a product on
        an fp32 small-M configuration (short prefill: the same pairs at a few
        hundred tokens): the GEMV / GEMM runs the LayerNorm as its prologue and
        the row kernel is not launched (for the GEMM, gamma is folded into the
        weight copy and beta . W into a per-column constant). A reshape that
        merges the LayerNorm's leading dims into the product's rows may sit
        between them ([B, T, K] -> [B*T, K]); x must then merge the same way
        (one row stride). The LayerNorm's
        input must stay intact until the product, so no buffer that a kernel
        from the LayerNorm up to the product writes may overlap it."""
        kernels = self.g.kernels
        owner = {n: k for k in kernels for n in k.nodes}
        results = set(self.g.results)
        skip = set()
        for i, k in enumerate(kernels):
            if k.kind != "reduction":
                continue
            reds = [n for n in k.nodes if n.op.startswith("reduce_")]
            if not reds or not all(is_row_reduction(n) for n in reds):
                continue
            members = set(k.nodes)
            outs = kernel_outputs(self.g, k, self.users)
            externals = []
            for n in k.nodes:
                for v in n.inputs:
                    if (v.node not in members or v.node is None) and not self.is_imm(v) and v not in externals:
                        externals.append(v)
            variant, fparams, (has_g, has_b), ordered = self._row_pattern(k, reds, outs, externals)
            if variant != kl.ROW_LAYERNORM or ordered is None:
                continue
            y, x = outs[0], ordered[0]
            users = self.users.get(y, [])
            if y in results or len(users) != 1 or tuple(x.shape) != tuple(y.shape):
                continue
            a_val = y
            if users[0].op == "reshape" and y.type.rank > 2:
                a_val = users[0].out
                users = self.users.get(a_val, [])
                if a_val in results or len(users) != 1:
                    continue
            if users[0].op != "matmul" or a_val.type.rank != 2:
                continue
            mm = users[0]
            km = owner.get(mm)
            if km is None or km.kind != "matmul" or mm.inputs[0] is not a_val or mm.inputs[1] is a_val:
                continue
            if self._arena_range(y) is None and y not in self.layouts:
                continue
            x_lay = self._rows_layout(x, a_val.shape)
            if x_lay is None:
                continue
            gamma = ordered[1] if has_g else None
            beta = ordered[1 + has_g] if has_b else None
            if not (self.is_gemv(km) if a_val.shape[0] == 1 else self._ln_gemm_ok(km, x_lay, gamma, beta)):
                continue
            j = kernels.index(km)
            xr = self._arena_range(x)
            if xr is not None:
                clash = False
                for kk in kernels[i:j + 1]:
                    for v in kernel_outputs(self.g, kk, self.users):
                        r = self._arena_range(v)
                        if v is not y and r is not None and r[0] < xr[1] and xr[0] < r[1]:
                            clash = True
                if clash:
                    continue
            self.prologue[km] = (x, gamma, beta, list(fparams), x_lay)
            skip.add(k)
        return skip

    def _rows_layout(self, x, shape):
        """x's storage seen as the [rows, K] operand `shape` of a product: x
        itself when it is 2-d, else its leading dims merged into one row
        stride; None when x has no storage or its leading dims do not merge."""
        lay = self.layouts.get(x)
        if lay is None or len(shape) != 2 or tuple(shape) != (math.prod(x.shape[:-1]), x.shape[-1]):
            return None
        if len(lay.shape) == 2:
            return lay
        row, inner = None, None
        for ext, st in reversed(list(zip(lay.shape[:-1], lay.strides[:-1]))):
            if ext == 1:
                continue
            if inner is not None and st != inner[0] * inner[1]:
                return None
            row = st if row is None else row
            inner = (ext, st)
        return Layout(lay.base, lay.offset, tuple(shape), (lay.shape[-1] if row is None else row, lay.strides[-1]))

    def _ln_gemm_ok(self, km, lay, gamma, beta) -> bool:
        """Whether matmul kernel km can run a LayerNorm of x (gamma, beta:
        its parameters or None) as its prologue: an fp32 small-M configuration
        (B the [N][K] copy of a constant, A read with unit K stride) holding at
        most 4 rows per wave, K <= 1024, at most LN_PROLOGUE_MAX_ROWS rows, x laid out like the A operand it
        replaces (`lay`: x's storage as [rows, K]), and gamma / beta constants
        (folded into build-time copies)."""
        cfg, prec = self.matmul_choice(km)
        tile = int(cfg.get("tile", -1))
        if prec != "fp32" or tile not in autotune.SMALL_M or autotune.PRECISION.get(tile) != "fp32":
            return False
        bm, wk = autotune.TILES[tile][0], autotune.TILES[tile][5]
        mm = next(n for n in km.nodes if n.op == "matmul")
        m, kk = mm.inputs[0].shape[-2], mm.inputs[0].shape[-1]
        if bm % wk or bm > 4 * wk or kk > 1024 or m > LN_PROLOGUE_MAX_ROWS:
            return False
        if not (self.skinny_ok(mm) and autotune.k_major_fits(m, kk, tile)):
            return False
        for p in (gamma, beta):
            if p is not None and (p not in self.layouts or self.layouts[p].base[0] != "const"
                                  or math.prod(p.shape) != kk):
                return False
        return (lay.strides[-1] == 1 and lay.offset % 4 == 0
                and all(st % 4 == 0 for st, ext in zip(lay.strides[:-1], lay.shape[:-1]) if ext > 1))

    def _vector_spec(self, v):
        """(constant name, element offset, element stride) of a constant
        vector's values, for a derived-constant recipe."""
        lay = self.layouts[v]
        return (lay.base[1], int(lay.offset), int(lay.strides[-1]))

    def ln_column(self, b, ref, batch, kk, n, vec, kind):
        """Ref of a per-column constant over (b, m, n) (strides 0 over M) of a
        small-M GEMM's LayerNorm prologue, `ref` being W's fp32 ref over (b,
        k, n): kind "lnc" = beta . W (vec = beta), "lng" = the column sums of
        the gamma-scaled weight copy (vec = gamma, or None: of W); registered
        as a derived constant."""
        src = self.layouts[b].base[1]
        strides = (int(ref.strides[0]), int(ref.strides[1]), int(ref.strides[2]))
        spec = self._vector_spec(vec) if vec is not None else ("", 0, 0)
        name = (f"{src}@{kind}:{int(ref.offset)}:{strides[0]},{strides[1]},{strides[2]}:{batch}x{kk}x{n}:"
                f"{spec[0]}:{spec[1]}:{spec[2]}")
        self.program.derived[name] = (src, int(ref.offset), strides, batch, kk, n, spec)
        r = kl.Ref()
        r.base, r.index = self.slot_of(("const", name))
        r.offset = 0
        r.strides[0], r.strides[1], r.strides[2] = (n if batch > 1 else 0), 0, 1
        return r

    def nk_weight(self, b, ref, batch, kk, n, scale=None):
        """Ref of an fp32 [batch][N][K] copy of constant view `b` (fp32 ref
        `ref` over (b, k, n)) for the GEMV family and the skinny-M and
        K-contiguous GEMMs: each
        output column's weights become one contiguous row, which the
        K-contiguous GEMV kernel
        reads 1 KiB per wave load. Registered as a derived constant, made when
        the executable is built."""
        src = self.layouts[b].base[1]
        strides = (int(ref.strides[0]), int(ref.strides[1]), int(ref.strides[2]))
        name = f"{src}@nk:{int(ref.offset)}:{strides[0]},{strides[1]},{strides[2]}:{batch}x{kk}x{n}"
        if scale is None:
            self.program.derived[name] = (src, int(ref.offset), strides, batch, kk, n)
        else:
            # each row scaled by the vector `scale` over K (a LayerNorm's
            # gamma folded into the product that follows it)
            spec = self._vector_spec(scale)
            name = name.replace("@nk:", "@nkg:") + f":{spec[0]}:{spec[1]}:{spec[2]}"
            self.program.derived[name] = (src, int(ref.offset), strides, batch, kk, n, spec)
        r = kl.Ref()
        r.base, r.index = self.slot_of(("const", name))
        r.offset = 0
        r.strides[0], r.strides[1], r.strides[2] = (n * kk if batch > 1 else 0), 1, kk
        return r

    def find_attn_prologues(self):
        """Decode-shaped attention (one query over at most 64 keys, head dim
        32 or 64) whose head-merged output is only the A operand of the next
        kernel, a GEMV (decode: attention -> c_proj): the GEMV computes each
        head's attention output for the K values it loads and the attention
        kernel is not launched. The GEMV's outputs must not overlap q, k, v or
        the mask (its workgroups write while others still read them)."""
        from kiln.hip.attention import causal_or_none, match_kernel, operand_strides

        kernels = self.g.kernels
        results = set(self.g.results)
        skip = set()
        for i, k in enumerate(kernels[:-1]):
            km = kernels[i + 1]
            if k.kind != "attention" or km.kind != "matmul" or km in self.prologue or not self.is_gemv(km):
                continue
            m = match_kernel(self.g, k)
            strides = operand_strides(m, self.layouts) if m is not None else None
            if strides is None:
                continue
            heads, tq, dh = m.q.shape
            tk = m.v.shape[1]
            mm = next(n for n in km.nodes if n.op == "matmul")
            a, b = mm.inputs
            kk = a.shape[-1]
            if tq != 1 or tk > 64 or dh not in (32, 64) or a.shape[-2] != 1 or kk != heads * dh:
                continue
            if self.layouts[b].base[0] != "const" or kk % (8 if self.matmul_choice(km)[1] == "bf16" else 4):
                continue
            # the attention's values feed only the GEMV kernel, directly or
            # through views (no graph result)
            members = set(k.nodes) | set(km.nodes)

            def feeds_only_gemv(v, depth=0):
                if v in results or depth > 8:
                    return False
                return all(u in members or (ops.kind(u.op) == "view" and feeds_only_gemv(u.out, depth + 1))
                           for u in self.users.get(v, []))

            if not all(feeds_only_gemv(n.out) for n in k.nodes):
                continue
            # A is the head-merged attention output: same storage, k = head * dh + d
            la, lr = self.layouts.get(a), self.layouts.get(m.result)
            if la is None or lr is None or la.base != lr.base or self.element_offset(a) != self.element_offset(m.result):
                continue
            if la.strides[-1] != 1 or tuple(strides[3][1][i] for i in (0, 2)) != (dh, 1):
                continue
            mode = kl.ATTN_MASK_NONE
            if m.mask is not None:
                mode = causal_or_none(self.g, m.mask, heads, tq, tk)
                if mode is None:
                    mode = kl.ATTN_MASK_ADD
            reads = [m.q, m.k, m.v] + ([m.mask] if mode == kl.ATTN_MASK_ADD else [])
            outs = kernel_outputs(self.g, km, self.users)
            clash = False
            for v in outs:
                r = self._arena_range(v)
                for w in reads:
                    rw = self._arena_range(w)
                    if r is not None and rw is not None and r[0] < rw[1] and rw[0] < r[1]:
                        clash = True
            if clash:
                continue
            self.attn_prologue[km] = (m, strides, mode, (heads, tk, dh))
            skip.add(k)
        return skip

    def attn_prologue_refs(self, d, km, first_ref):
        """Fill GEMV descriptor `d` for the attention prologue of `km`; its q,
        k, v (and mask) refs start at descriptor ref `first_ref`. Returns the
        refs and (flops, bytes) of the attention."""
        m, strides, mode, (heads, tk, dh) = self.attn_prologue[km]
        refs = []
        for v, (_, st) in zip((m.q, m.k, m.v), strides[:3]):
            r = kl.Ref()
            r.base, r.index = self.slot_of(self.layouts[v].base)
            r.offset = self.element_offset(v)
            for i in range(3):
                r.strides[i] = st[i]
            refs.append(r)
        if mode == kl.ATTN_MASK_ADD:
            refs.append(self.ref(m.mask, (heads, 1, tk)))
        d.cfg[0], d.cfg[4], d.cfg[5] = dh, kl.GEMV_PRO_ATTN, first_ref
        d.cfg[6], d.cfg[7] = mode + 4 * m.scale_mode, tk
        d.fparams[0] = m.scale
        pairs = 1 if mode == kl.ATTN_MASK_CAUSAL else tk
        return refs, 4 * heads * pairs * dh, 4 * heads * dh * (2 + 2 * tk)

    def bf16_weight(self, b, ref, batch, kk, n, split=False):
        """Ref of the bf16 [batch][N][K'] copy of constant view `b` (whose fp32
        ref over (b, k, n) is `ref`), or with `split` the three-pass
        [batch][N][2K'] hi/lo copy; the copy is registered as a derived
        constant and made when the executable is built."""
        src = self.layouts[b].base[1]
        strides = (int(ref.strides[0]), int(ref.strides[1]), int(ref.strides[2]))
        kind = "bf16x3" if split else "bf16"
        name = f"{src}@{kind}:{int(ref.offset)}:{strides[0]},{strides[1]},{strides[2]}:{batch}x{kk}x{n}"
        self.program.derived[name] = (src, int(ref.offset), strides, batch, kk, n)
        row = bf16.padded_k(kk) * (2 if split else 1)
        r = kl.Ref()
        r.base, r.index = self.slot_of(("const", name))
        r.offset = 0
        r.strides[0], r.strides[1], r.strides[2] = (n * row if batch > 1 else 0), 1, row
        return r

    # attention --------------------------------------------------------------------------------

    def lower_attention(self, k: Kernel):
        from kiln.hip.attention import causal_or_none, match_kernel, operand_strides

        m = match_kernel(self.g, k)
        strides = operand_strides(m, self.layouts) if m is not None else None
        if strides is None:
            raise NotImplementedError(f"HIP backend: attention kernel {k.name} does not have the fused form")
        batch, tq, dh = m.q.shape
        tk = m.v.shape[1]
        d = self.new_desc(kl.FAM_ATTN, "attn", k, (batch, tq, tk))
        d.gemm[0], d.gemm[1], d.gemm[2], d.gemm[3] = batch, tq, tk, dh
        for j, (v, (_, st)) in enumerate(zip((m.q, m.k, m.v, m.result), strides)):
            r = kl.Ref()
            r.base, r.index = self.slot_of(self.layouts[v].base)
            r.offset = self.element_offset(v)
            for i in range(3):
                r.strides[i] = st[i]
            if self.stored_bf16(v):   # the output, or (all three) q, k, v
                r = self.as_bf16(r, v)
                d.cfg[7] |= 1 << j
            if self.stored_pairs(v):  # (pair words: addressed as fp32)
                d.cfg[7] |= 1 << (16 + j)
            d.refs[j] = r
        d.n_refs = 4
        mode = kl.ATTN_MASK_NONE
        if m.mask is not None:
            mode = causal_or_none(self.g, m.mask, batch, tq, tk)
            if mode is None:
                mode = kl.ATTN_MASK_ADD
                d.refs[4] = self.ref(m.mask, (batch, tq, tk))
                d.n_refs = 5
        d.cfg[0], d.cfg[1] = mode, m.scale_mode
        d.cfg[3] = ATTN_QUERIES
        # bf16 plans run the two products of attention on bf16 inputs too
        # (fp32 accumulation and softmax), three-pass plans on three-pass bf16
        # where the grid is large enough; decode shapes keep the few-query
        # kernel's fp32 products
        bf_products = self.precision == "bf16" and tq > ATTN_ROWS_MAX_Q
        x3_products = self.x3_attention(m)
        if bf_products:
            d.cfg[5] = 1
        if x3_products:
            d.cfg[5] = 2
        d.fparams[0] = m.scale
        causal = mode == kl.ATTN_MASK_CAUSAL
        pairs = sum(min(tk, i + 1) for i in range(tq)) if causal else tq * tk
        flops = 4 * batch * pairs * dh
        nbytes = 4 * batch * dh * (2 * tq + 2 * tk) + (4 * batch * tq * tk if mode == kl.ATTN_MASK_ADD else 0)
        what = {kl.ATTN_MASK_NONE: "no mask", kl.ATTN_MASK_CAUSAL: "causal", kl.ATTN_MASK_ADD: "additive mask"}[mode]
        scale = {kl.ATTN_SCALE_NONE: "", kl.ATTN_SCALE_MUL: f", scores * {m.scale:g}",
                 kl.ATTN_SCALE_DIV: f", scores / {m.scale:g}"}[m.scale_mode]
        if bf_products:
            scale += ", products:bf16"
        if x3_products:
            scale += ", products:bf16x3"
        if d.cfg[7] & 7:
            scale += ", qkv:bf16"
            nbytes -= 2 * batch * dh * (tq + 2 * tk)
        if d.cfg[7] & 8:
            scale += ", out:bf16"
            nbytes -= 2 * batch * dh * tq
        if d.cfg[7] >> 16 & 7:
            scale += ", qkv:pairs"
        if d.cfg[7] >> 16 & 8:
            scale += ", out:pairs"
        self.add(d, k, f"{batch} heads x {tq} queries x {tk} keys, head dim {dh}, {what}{scale}",
                 flops=flops, nbytes=nbytes)

    # driver --------------------------------------------------------------------------------------

    def run(self) -> Program:
        for k in self.g.kernels:
            for n in k.nodes:
                if ops.kind(n.op) not in ("elementwise", "reduction", "matmul") and k.kind != "attention":
                    raise NotImplementedError(f"GPU backend: unexpected op '{n.op}' in a kernel")
        fused = self.find_ln_prologues() | self.find_attn_prologues()
        self.bf16_buffers = self.plan_bf16_storage()
        self.pair_buffers = self.plan_pair_storage()
        for k in self.g.kernels:
            if k in fused:
                continue
            if k.kind == "attention":
                self.lower_attention(k)
            elif k.kind == "matmul":
                self.lower_matmul(k)
            elif k.kind == "reduction":
                self.lower_reduction(k)
            else:
                self.lower_elementwise(k)
        from kiln.passes.memory_plan import live_ranges

        kernel_index = {k.name: i for i, k in enumerate(self.g.kernels)}
        launch_kernel = [kernel_index.get(launch.kernel, -1) for launch in self.program.launches]
        for v, (kf, kl_) in live_ranges(self.g).items():
            live = [i for i, ki in enumerate(launch_kernel) if kf <= ki <= kl_]
            if live:
                label = f"{self.g.kernels[kf].name} {v.node.op} {list(v.shape)}"
                self.program.arena_buffers.append((label, int(v.node.attrs.get("offset", 0)), int(v.type.nbytes),
                                                   live[0], live[-1]))
        self.program.arena_buffers.sort(key=lambda b: b[1])
        return self.program


def lower_graph(graph: Graph, precision: str = "fp32", matmul_config=None, gemv_chains: bool = False) -> Program:
    """Fused, buffer-assigned, memory-planned graph -> Program (launch list).
    gemv_chains: mark one-row matmuls KH_GEMV_CHAIN, so the library may run
    consecutive ones as one persistent launch."""
    from kiln.hip.autotune import default_matmul_config

    return _Lowerer(graph, precision, matmul_config or default_matmul_config, gemv_chains).run()
