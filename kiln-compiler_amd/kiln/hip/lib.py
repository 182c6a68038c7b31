"""ctypes binding of libkiln_hip.so (include/kiln_hip.h).

The structures below mirror the C ABI field by field; ``load`` checks their
sizes against the compiled library (kh_abi_sizes). Status
codes become the reference's exception types (ValueError, NotImplementedError,
RuntimeError, MemoryError; see kiln/gpu/runtime.py:39-90 and codegen.py:248).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

ABI_VERSION = 1
MAX_RANK = 6
MAX_REFS = 12
MAX_INSNS = 96
NREGS = 16
FAST_SLOTS = 8
MAX_PASSES = 8

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP, ERR_NO_DEVICE, ERR_CAPACITY = range(6)
BASE_INPUT, BASE_OUTPUT, BASE_CONST, BASE_ARENA, BASE_WORKSPACE = range(5)
FAM_EW, FAM_ROW, FAM_GEMM, FAM_GEMV, FAM_RED, FAM_ATTN = 1, 2, 3, 4, 5, 6
ATTN_MASK_NONE, ATTN_MASK_CAUSAL, ATTN_MASK_ADD = 0, 1, 2
GEMV_PRO_NONE, GEMV_PRO_LAYERNORM, GEMV_PRO_ATTN = 0, 1, 2
GEMV_CHAIN = 1   # KH_GEMV_CHAIN: kh_launch.variant flag of a GEMV launch
ATTN_SCALE_NONE, ATTN_SCALE_MUL, ATTN_SCALE_DIV = 0, 1, 2
ROW_GENERIC, ROW_LAYERNORM, ROW_SOFTMAX = 0, 1, 2
PREC_FP32, PREC_BF16, PREC_BF16X3 = 0, 1, 2
NOALLOC_WORKSPACE_BYTES = 16 << 20   # KH_NOALLOC_WORKSPACE_BYTES: kh_plan_run_noalloc's device array

OPCODES = ["mov", "add", "sub", "mul", "div", "max", "min", "neg", "relu", "exp", "tanh", "sigmoid",
           "erf", "gelu_tanh", "gelu_erf", "rsqrt", "sqrt", "rsum", "rmax", "load", "store"]
OP = {name: i for i, name in enumerate(OPCODES)}
SRC_IMM = 0xFF

FAMILY_NAMES = {FAM_EW: "elementwise", FAM_ROW: "row", FAM_GEMM: "gemm", FAM_GEMV: "gemv", FAM_RED: "reduce",
                FAM_ATTN: "attention"}


class Ref(ctypes.Structure):
    _fields_ = [("base", ctypes.c_int32), ("index", ctypes.c_int32), ("offset", ctypes.c_int64),
                ("strides", ctypes.c_int64 * MAX_RANK)]


class Insn(ctypes.Structure):
    _fields_ = [("op", ctypes.c_uint8), ("dst", ctypes.c_uint8), ("a", ctypes.c_uint8), ("b", ctypes.c_uint8),
                ("imm", ctypes.c_float)]


class PassDesc(ctypes.Structure):
    _fields_ = [("vec_begin", ctypes.c_int16), ("vec_end", ctypes.c_int16), ("post_begin", ctypes.c_int16),
                ("post_end", ctypes.c_int16), ("acc_mask", ctypes.c_uint16), ("max_mask", ctypes.c_uint16),
                ("single_chunk", ctypes.c_int16), ("pad", ctypes.c_int16)]


class LaunchDesc(ctypes.Structure):
    _fields_ = [("family", ctypes.c_int32), ("variant", ctypes.c_int32), ("rank", ctypes.c_int32),
                ("n_refs", ctypes.c_int32), ("n_insns", ctypes.c_int32), ("n_passes", ctypes.c_int32),
                ("cfg", ctypes.c_int32 * 8), ("fparams", ctypes.c_float * 4), ("shape", ctypes.c_int64 * MAX_RANK),
                ("gemm", ctypes.c_int64 * 4), ("refs", Ref * MAX_REFS), ("insns", Insn * MAX_INSNS),
                ("passes", PassDesc * MAX_PASSES), ("name", ctypes.c_char * 32)]


def library_path() -> Path:
    env = os.environ.get("KILN_HIP_LIB")
    return Path(env) if env else Path(__file__).resolve().parent / "libkiln_hip.so"


class KilnHipError(RuntimeError):
    pass


_lib = None


def load():
    """Load the in-tree library once. Raises a clear error if it is missing:
    the HIP backend has no fallback path."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise RuntimeError(f"Kiln's HIP backend library is not built ({path}); run "
                           f"`python kiln-compiler_amd/build.py` (or __graft_entry__.build())")
    lib = ctypes.CDLL(str(path))
    vp, ip, i32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int32
    sig = {
        "kh_version": (ip, []),
        "kh_build_id": (ctypes.c_char_p, []),
        "kh_abi_sizes": (ip, [ctypes.POINTER(ctypes.c_size_t)]),
        "kh_last_error": (ctypes.c_char_p, []),
        "kh_init": (ip, [ip]),
        "kh_device_info": (ip, [ctypes.POINTER(ip), ctypes.POINTER(ip), ctypes.c_char_p, ip]),
        "kh_gemm_config_count": (ip, []),
        "kh_gemm_config": (ip, [ip, ctypes.POINTER(i32)]),
        "kh_plan_create": (ip, [ctypes.POINTER(LaunchDesc), ip, ctypes.POINTER(vp)]),
        "kh_plan_workspace_bytes": (ip, [vp, ctypes.POINTER(ctypes.c_size_t)]),
        "kh_plan_bind": (ip, [vp, ctypes.POINTER(vp), ip, vp, vp, ctypes.c_size_t]),
        "kh_plan_run": (ip, [vp, ctypes.POINTER(vp), ip, ctypes.POINTER(vp), ip, vp]),
        "kh_plan_run_noalloc": (ip, [vp, ctypes.POINTER(vp), ip, ctypes.POINTER(vp), ip, vp]),
        "kh_plan_run_host": (ip, [vp, ctypes.POINTER(vp), ip, ctypes.POINTER(vp), ip]),
        "kh_plan_run_one": (ip, [vp, ip, ctypes.POINTER(vp), ip, ctypes.POINTER(vp), ip, vp]),
        "kh_plan_capture": (ip, [vp, ctypes.POINTER(vp), ip, ctypes.POINTER(vp), ip]),
        "kh_plan_replay": (ip, [vp, vp]),
        "kh_plan_time": (ip, [vp, ip, ctypes.POINTER(vp), ip, ctypes.POINTER(vp), ip, ip, ip, vp,
                              ctypes.POINTER(ctypes.c_double)]),
        "kh_plan_chains": (ip, [vp, ctypes.POINTER(ctypes.c_int32), ip, ctypes.POINTER(ip)]),
        "kh_plan_chain_timeouts": (ip, [vp, ctypes.POINTER(ctypes.c_uint64)]),
        "kh_plan_chain_spin": (ip, [vp, ctypes.c_int64]),
        "kh_plan_destroy": (ip, [vp]),
        "kh_probe_attn_timeline": (ip, [vp, vp, vp, vp, ip, ip, ip, ctypes.POINTER(ctypes.c_int64), ip,
                                        ctypes.c_float, vp, vp]),
        "kh_probe_mfma_valu": (ip, [ip, ip, ip, ip, ctypes.POINTER(ctypes.c_double)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    if lib.kh_version() != ABI_VERSION:
        raise RuntimeError(f"libkiln_hip ABI {lib.kh_version()} != binding ABI {ABI_VERSION}; rebuild")
    sizes = (ctypes.c_size_t * 4)()
    lib.kh_abi_sizes(sizes)
    mine = (ctypes.sizeof(LaunchDesc), ctypes.sizeof(Ref), ctypes.sizeof(Insn), ctypes.sizeof(PassDesc))
    if tuple(sizes) != mine:
        raise RuntimeError(f"libkiln_hip struct sizes {tuple(sizes)} != binding {mine}; rebuild")
    _lib = lib
    return lib


EXPORTED = ("kh_version", "kh_build_id", "kh_abi_sizes", "kh_last_error", "kh_init", "kh_device_info", "kh_gemm_config_count", "kh_gemm_config",
            "kh_plan_create", "kh_plan_workspace_bytes", "kh_plan_bind", "kh_plan_run", "kh_plan_run_noalloc",
            "kh_plan_run_host",
            "kh_plan_run_one",
            "kh_plan_capture", "kh_plan_replay", "kh_plan_time", "kh_plan_chains", "kh_plan_chain_timeouts",
            "kh_plan_chain_spin",
            "kh_plan_destroy", "kh_probe_attn_timeline", "kh_probe_mfma_valu")


def check(rc: int, what: str = ""):
    if rc == OK:
        return
    msg = (_lib.kh_last_error() or b"").decode(errors="replace")
    text = f"{what}: {msg}" if what else msg
    if rc == ERR_INVALID:
        raise ValueError(text)
    if rc == ERR_UNSUPPORTED:
        raise NotImplementedError(f"HIP backend: {text}")
    if rc == ERR_CAPACITY:
        raise MemoryError(text)
    raise KilnHipError(text)


def gemm_configs() -> list:
    """[(BM, BN, BK, WM, WN, WK, MFMA, precision)] compiled into the library."""
    lib = load()
    out = []
    buf = (ctypes.c_int32 * 8)()
    for i in range(lib.kh_gemm_config_count()):
        check(lib.kh_gemm_config(i, buf), "kh_gemm_config")
        out.append(tuple(buf))
    return out


def build_id() -> str:
    """Digest of the sources the loaded library was built from."""
    return load().kh_build_id().decode()


def device_info():
    lib = load()
    cus, lds = ctypes.c_int(), ctypes.c_int()
    arch = ctypes.create_string_buffer(64)
    check(lib.kh_device_info(ctypes.byref(cus), ctypes.byref(lds), arch, 64))
    return {"cus": cus.value, "lds_bytes": lds.value, "arch": arch.value.decode()}


def pointer_array(ptrs):
    arr = (ctypes.c_void_p * max(1, len(ptrs)))()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr


class Plan:
    """Owns one kh_plan handle (a compiled graph's launch list)."""

    def __init__(self, launches):
        self.lib = load()
        n = len(launches)
        self._descs = (LaunchDesc * max(1, n))(*launches)
        handle = ctypes.c_void_p()
        check(self.lib.kh_plan_create(self._descs, n, ctypes.byref(handle)), "kh_plan_create")
        self.handle = handle
        self.n_launches = n
        size = ctypes.c_size_t()
        check(self.lib.kh_plan_workspace_bytes(handle, ctypes.byref(size)), "kh_plan_workspace_bytes")
        self.workspace_bytes = size.value
        self._keep = []

    def bind(self, const_ptrs, arena_ptr, workspace_ptr, workspace_bytes):
        arr = pointer_array(const_ptrs)
        self._keep = [arr]
        check(self.lib.kh_plan_bind(self.handle, arr, len(const_ptrs), arena_ptr, workspace_ptr, workspace_bytes),
              "kh_plan_bind")

    def run(self, in_ptrs, out_ptrs, stream):
        ins, outs = pointer_array(in_ptrs), pointer_array(out_ptrs)
        check(self.lib.kh_plan_run(self.handle, ins, len(in_ptrs), outs, len(out_ptrs), stream), "kh_plan_run")

    def run_host(self, in_ptrs, out_ptrs):
        """The plan executed on the CPU over host buffers (kh_plan_run_host)."""
        ins, outs = pointer_array(in_ptrs), pointer_array(out_ptrs)
        check(self.lib.kh_plan_run_host(self.handle, ins, len(in_ptrs), outs, len(out_ptrs)), "kh_plan_run_host")

    def run_one(self, index, in_ptrs, out_ptrs, stream):
        ins, outs = pointer_array(in_ptrs), pointer_array(out_ptrs)
        check(self.lib.kh_plan_run_one(self.handle, index, ins, len(in_ptrs), outs, len(out_ptrs), stream),
              "kh_plan_run_one")

    def capture(self, in_ptrs, out_ptrs):
        ins, outs = pointer_array(in_ptrs), pointer_array(out_ptrs)
        check(self.lib.kh_plan_capture(self.handle, ins, len(in_ptrs), outs, len(out_ptrs)), "kh_plan_capture")

    def replay(self, stream):
        check(self.lib.kh_plan_replay(self.handle, stream), "kh_plan_replay")

    def time(self, in_ptrs, out_ptrs, stream, index=-1, repeats=20, rounds=5) -> float:
        """GPU seconds per execution of one launch (or of all: index -1)."""
        ins, outs = pointer_array(in_ptrs), pointer_array(out_ptrs)
        sec = ctypes.c_double()
        check(self.lib.kh_plan_time(self.handle, index, ins, len(in_ptrs), outs, len(out_ptrs), repeats, rounds,
                                    stream, ctypes.byref(sec)), "kh_plan_time")
        return sec.value

    def chains(self):
        """[(first launch, launches, active)] of the plan's persistent GEMV chains."""
        n = ctypes.c_int()
        check(self.lib.kh_plan_chains(self.handle, None, 0, ctypes.byref(n)), "kh_plan_chains")
        buf = (ctypes.c_int32 * max(1, 3 * n.value))()
        check(self.lib.kh_plan_chains(self.handle, buf, n.value, ctypes.byref(n)), "kh_plan_chains")
        return [tuple(buf[3 * i:3 * i + 3]) for i in range(n.value)]

    def chain_timeouts(self) -> int:
        """Waits inside the plan's chains that gave up, over the plan's life
        (none expected); synchronises the device."""
        n = ctypes.c_uint64()
        check(self.lib.kh_plan_chain_timeouts(self.handle, ctypes.byref(n)), "kh_plan_chain_timeouts")
        return n.value

    def set_chain_spin(self, ticks: int):
        """Bound on each chain wait in 100 MHz ticks (default 2,000,000 = 20 ms);
        negative: every wait gives up at once (tests drive the give-up path)."""
        check(self.lib.kh_plan_chain_spin(self.handle, int(ticks)), "kh_plan_chain_spin")

    def __del__(self):
        h = getattr(self, "handle", None)
        if h and getattr(self, "lib", None) is not None:
            self.lib.kh_plan_destroy(h)
            self.handle = None
