"""GEMM tile configurations: a default heuristic and a measured autotuner.

Replaces the reference's Triton config heuristic and tuner
(kiln/gpu/codegen.py:552-598, kiln/gpu/autotune.py:40-193). The knobs are
the MI355X GEMM family's: the compiled tile configurations (macro-tile
BM x BN x BK, waves along M / N / K, MFMA shape; ``kh_gemm_config``) and the
split-K factor. The tuning contract is Kiln's: a candidate that gives a
wrong result is never chosen, the default stays unless measurement clearly
beats it, and results are cached on disk by device and shape. How it is met
here:

  * candidates are the compiled configurations that fit the problem (no tile
    far larger than it) times the split-K factors that leave at least 64 K
    values per split;
  * each candidate is built as a one-matmul plan (an nn.Linear: activations x
    constant weight + bias epilogue) and checked against float64 (error
    relative to the output's largest magnitude <= 1e-4 for fp32, 2e-2 for
    the bf16 inputs);
  * timing is successive halving on the library's own timer
    (``kh_plan_time``: the plan captured 10 or 20 times into a hipGraph,
    replays timed with hipEvents): every survivor gets a short measurement,
    the fastest quarter (at least FINALISTS, plus the default) a longer one in
    two interleaved passes, and the default is replaced only by a candidate
    more than KEEP_DEFAULT_MARGIN faster;
  * results are cached by device, CU count, precision and shape in
    $KILN_CACHE_DIR/hip_autotune.json (an unreadable cache counts as empty);
  * before measuring, the tuner looks the key up in the table shipped with
    the package (tuned_configs.json, made by kiln.hip.tune_shipped on an
    MI355X for the GPT-2 shapes): a hit is used as-is (source "shipped"), so
    the same model compiles to the same plan on every MI355X.
"""

from __future__ import annotations

import json
import math
import os
import time
import warnings
from pathlib import Path

KEEP_DEFAULT_MARGIN = 1.03
FINALISTS = 3
SPLITS = (1, 2, 3, 4, 6, 8)
# M = 1 (GEMV family): "tile" = workgroup variant (0 = from the shape; 1-3 =
# 32/16/8 columns x 256 threads, 4-5 = 32/16 columns x 1024 threads), split-K
# 0 = from the shape
GEMV_CANDIDATES = [(v, 0) for v in range(6)] + [(0, s) for s in (2, 4)]

# (BM, BN, BK, WM, WN, WK, MFMA) of the compiled configurations, by id; must
# match the table in csrc/kh_gemm.hip (tests check it against kh_gemm_config).
# Ids 0-7, 21-25, 32-33 and 46 are the LDS-copy pipeline (21-25 with 64 K
# values per stage, 32-33 with 128), 8-14 the register-staged kernel, 15-20 and 34-41
# the bf16-input pipeline (34-41 with 64 or 128 K values per stage), 26-31 and
# 42-45 the three-pass bf16 pipeline.
TILES = {
    0: (64, 128, 32, 2, 2, 1, 16),
    1: (128, 64, 32, 2, 2, 1, 16),
    2: (64, 64, 32, 2, 2, 1, 16),
    3: (32, 128, 32, 1, 4, 1, 16),
    4: (32, 64, 32, 2, 2, 1, 16),
    5: (64, 96, 32, 2, 2, 1, 16),
    6: (128, 192, 32, 2, 4, 1, 16),
    7: (128, 128, 32, 2, 4, 1, 16),
    8: (64, 64, 32, 2, 2, 1, 32),
    9: (32, 64, 32, 1, 2, 2, 32),
    10: (32, 32, 32, 1, 1, 4, 32),
    11: (32, 32, 32, 2, 2, 1, 16),
    12: (16, 64, 32, 1, 4, 1, 16),
    13: (64, 32, 32, 2, 2, 1, 16),
    14: (64, 64, 64, 2, 2, 1, 32),
    15: (128, 128, 32, 2, 2, 1, 16),
    16: (64, 128, 32, 2, 2, 1, 16),
    17: (128, 64, 32, 2, 2, 1, 16),
    18: (64, 64, 32, 2, 2, 1, 16),
    19: (32, 64, 32, 2, 2, 1, 16),
    20: (128, 256, 32, 2, 4, 1, 16),
    21: (64, 64, 64, 2, 2, 1, 16),
    22: (64, 128, 64, 2, 2, 1, 16),
    23: (32, 64, 64, 2, 2, 1, 16),
    24: (128, 192, 64, 2, 4, 1, 16),
    25: (64, 96, 64, 2, 2, 1, 16),
    26: (128, 128, 32, 2, 2, 1, 16),
    27: (64, 128, 32, 2, 2, 1, 16),
    28: (128, 64, 32, 2, 2, 1, 16),
    29: (64, 64, 32, 2, 2, 1, 16),
    30: (32, 64, 32, 2, 2, 1, 16),
    31: (128, 256, 32, 2, 4, 1, 16),
    32: (32, 64, 128, 2, 2, 1, 16),
    33: (32, 64, 128, 2, 2, 1, 16),
    34: (128, 128, 64, 2, 2, 1, 16),
    35: (64, 128, 64, 2, 2, 1, 16),
    36: (128, 64, 64, 2, 2, 1, 16),
    37: (64, 64, 64, 2, 2, 1, 16),
    38: (32, 64, 64, 2, 2, 1, 16),
    39: (128, 256, 64, 2, 4, 1, 16),
    40: (32, 64, 128, 2, 2, 1, 16),
    41: (64, 64, 128, 2, 2, 1, 16),
    42: (128, 128, 64, 2, 2, 1, 16),
    43: (64, 128, 64, 2, 2, 1, 16),
    44: (64, 64, 64, 2, 2, 1, 16),
    45: (32, 64, 64, 2, 2, 1, 16),
    46: (32, 96, 32, 2, 2, 1, 16),
    # skinny-M direct loads (BM x BN, WK waves splitting K, B as [N][K])
    47: (16, 32, 16, 1, 1, 8, 16),
    48: (16, 32, 16, 1, 1, 16, 16),
    49: (32, 32, 16, 1, 1, 8, 16),
    50: (16, 64, 16, 1, 1, 8, 16),
    51: (32, 32, 16, 1, 1, 16, 16),
    52: (16, 16, 16, 1, 1, 8, 16),
    53: (32, 64, 16, 1, 1, 8, 16),
    54: (16, 32, 16, 1, 1, 4, 16),
    # one workgroup per CU (persistent), A and B both K-contiguous (B as [N][K])
    55: (128, 192, 32, 2, 2, 1, 16),
    56: (64, 288, 32, 2, 2, 1, 16),
    57: (64, 96, 32, 2, 2, 1, 16),
    58: (128, 96, 32, 2, 2, 1, 16),
    59: (128, 128, 32, 2, 4, 1, 16),
    60: (64, 192, 32, 2, 4, 1, 16),
    61: (128, 192, 32, 2, 4, 1, 16),
    62: (64, 128, 32, 2, 4, 1, 16),
    63: (32, 96, 32, 2, 2, 1, 16),
    64: (64, 64, 32, 2, 2, 1, 16),
    # small tiles, WK waves splitting K, each with a private LDS ring (B as [N][K])
    65: (16, 32, 32, 1, 1, 4, 16),
    66: (16, 32, 32, 1, 1, 4, 16),
    67: (16, 16, 32, 1, 1, 4, 16),
    68: (16, 64, 32, 1, 1, 4, 16),
    69: (32, 32, 32, 1, 1, 4, 16),
    70: (16, 32, 32, 1, 1, 8, 16),
    71: (16, 16, 32, 1, 1, 8, 16),
    72: (32, 64, 32, 1, 1, 4, 16),
    73: (32, 32, 32, 1, 1, 8, 16),
    74: (16, 16, 32, 1, 1, 4, 16),
    # the same kernel over the bf16 (75-79, 84-85) and three-pass bf16 (80-83, 86) weight copies
    75: (16, 32, 32, 1, 1, 4, 16),
    76: (16, 32, 32, 1, 1, 8, 16),
    77: (32, 32, 32, 1, 1, 4, 16),
    78: (16, 64, 32, 1, 1, 4, 16),
    79: (16, 16, 32, 1, 1, 4, 16),
    80: (16, 32, 32, 1, 1, 4, 16),
    81: (16, 32, 32, 1, 1, 8, 16),
    82: (32, 32, 32, 1, 1, 4, 16),
    83: (16, 16, 32, 1, 1, 4, 16),
    84: (16, 16, 32, 1, 1, 8, 16),
    85: (32, 32, 32, 1, 1, 8, 16),
    86: (16, 16, 32, 1, 1, 8, 16),
    # K-contiguous kernel over the bf16 (87-91) and three-pass bf16 (92-94)
    # weight copies
    87: (128, 256, 32, 2, 4, 1, 16),
    88: (128, 192, 32, 2, 2, 1, 16),
    89: (256, 128, 32, 4, 2, 1, 16),
    90: (128, 128, 32, 2, 4, 1, 16),
    91: (64, 192, 32, 2, 2, 1, 16),
    92: (128, 256, 32, 2, 4, 1, 16),
    93: (128, 192, 32, 2, 2, 1, 16),
    94: (128, 128, 32, 2, 4, 1, 16),
    # the bf16 K-contiguous kernel with 64-deep K steps (K a multiple of 64)
    95: (128, 192, 64, 2, 4, 1, 16),
    96: (64, 192, 64, 2, 4, 1, 16),
    97: (64, 128, 64, 2, 4, 1, 16),
    98: (64, 96, 64, 2, 2, 1, 16),
    99: (64, 64, 64, 2, 2, 1, 16),
    100: (128, 96, 64, 2, 2, 1, 16),
}
# configurations of the skinny-M kernel: A row-major with unit K stride and
# K % 4 == 0, B a constant read through its [batch][N][K] copy, no split-K;
# each wave's ring holds SKINNY_DEPTH[tile] 16-deep chunks and turns at most
# SKINNY_TURNS times, which bounds K
SKINNY = frozenset(range(47, 55))
# configurations of the K-contiguous pipeline: A as for the skinny kernel, B
# the [batch][N][K] copy of a constant, K a multiple of 32, no split-K
K_CONTIGUOUS = frozenset(range(55, 65)) | frozenset(range(87, 101))
# the bf16 configurations with 64-deep K steps (kind 7): they also read A as
# bf16 when its producer stores it that way (kiln/hip/lowering.py,
# plan_bf16_storage)
BF16_A = frozenset(range(95, 101))
# configurations of the small-M kernel: as the K-contiguous pipeline (B the
# [batch][N][K] copy, K a positive multiple of 32, no split-K), for products
# with at most SMALL_M_MAX rows
SMALL_M = frozenset(range(65, 87))
SMALL_M_MAX = 1024
# configurations that read B through its [batch][N][K] copy
NK_B = SKINNY | K_CONTIGUOUS | SMALL_M
SKINNY_DEPTH = {47: 8, 48: 4, 49: 8, 50: 4, 51: 4, 52: 8, 53: 4, 54: 8}
SKINNY_TURNS = 4
# input precision of each configuration: 15-20, 34-41, 75-79, 84-85, 87-91 and 95-100
# bf16 (A rounded in the kernel, B a bf16 copy of a constant), 26-31, 42-45,
# 80-83, 86 and 92-94 three-pass bf16
# (allow_tf32: A and B split into bf16 hi + lo, three products), the others
# fp32
PRECISION = {t: ("bf16" if 15 <= t <= 20 or 34 <= t <= 41 or 75 <= t <= 79 or t in (84, 85) or 87 <= t <= 91
                 or 95 <= t <= 100
                 else "bf16x3" if 26 <= t <= 31 or 42 <= t <= 45 or 80 <= t <= 83 or t == 86 or 92 <= t <= 94
                 else "fp32")
             for t in TILES}
# workgroups of each configuration one CU holds at once (LDS / VGPR bound,
# from the compiler's resource report) and its measured main-loop efficiency
# (fraction of the CU's fp32 MFMA rate), for the default heuristic only
OCCUPANCY = {0: 2, 1: 2, 2: 3, 3: 2, 4: 4, 5: 2, 6: 1, 7: 1, 8: 4, 9: 4, 10: 4, 11: 5, 12: 5, 13: 4, 14: 2,
             15: 2, 16: 2, 17: 1, 18: 3, 19: 4, 20: 1, 21: 2, 22: 1, 23: 2, 24: 1, 25: 2,
             26: 1, 27: 2, 28: 2, 29: 3, 30: 4, 31: 1, 32: 1, 33: 1,
             34: 1, 35: 2, 36: 2, 37: 2, 38: 3, 39: 1, 40: 2, 41: 1, 42: 1, 43: 1, 44: 2, 45: 2, 46: 3,
             47: 2, 48: 1, 49: 2, 50: 2, 51: 1, 52: 2, 53: 2, 54: 4,
             55: 1, 56: 1, 57: 1, 58: 1, 59: 1, 60: 1, 61: 1, 62: 1, 63: 1, 64: 1,
             65: 2, 66: 3, 67: 3, 68: 1, 69: 2, 70: 1, 71: 2, 72: 1, 73: 1, 74: 4,
             75: 4, 76: 2, 77: 3, 78: 3, 79: 4, 80: 3, 81: 2, 82: 2, 83: 4, 84: 2, 85: 1, 86: 2,
             87: 1, 88: 1, 89: 1, 90: 1, 91: 1, 92: 1, 93: 1, 94: 1,
             95: 1, 96: 1, 97: 1, 98: 1, 99: 1, 100: 1}
EFFICIENCY = {0: 0.62, 1: 0.6, 2: 0.62, 3: 0.58, 4: 0.66, 5: 0.62, 6: 0.67, 7: 0.55,
              8: 0.55, 9: 0.55, 10: 0.5, 11: 0.5, 12: 0.45, 13: 0.5, 14: 0.55,
              15: 0.15, 16: 0.15, 17: 0.15, 18: 0.15, 19: 0.15, 20: 0.15,
              21: 0.62, 22: 0.6, 23: 0.62, 24: 0.67, 25: 0.62,
              26: 0.3, 27: 0.3, 28: 0.3, 29: 0.3, 30: 0.3, 31: 0.3, 32: 0.62, 33: 0.62,
              34: 0.2, 35: 0.2, 36: 0.2, 37: 0.2, 38: 0.2, 39: 0.2, 40: 0.2, 41: 0.2,
              42: 0.35, 43: 0.35, 44: 0.35, 45: 0.35, 46: 0.62,
              47: 0.45, 48: 0.45, 49: 0.5, 50: 0.5, 51: 0.5, 52: 0.4, 53: 0.5, 54: 0.45,
              55: 0.7, 56: 0.7, 57: 0.7, 58: 0.7, 59: 0.75, 60: 0.75, 61: 0.78, 62: 0.72, 63: 0.65, 64: 0.68,
              65: 0.5, 66: 0.5, 67: 0.45, 68: 0.5, 69: 0.5, 70: 0.5, 71: 0.45, 72: 0.5, 73: 0.5, 74: 0.45,
              75: 0.12, 76: 0.12, 77: 0.12, 78: 0.12, 79: 0.1, 80: 0.25, 81: 0.25, 82: 0.25, 83: 0.2,
              84: 0.1, 85: 0.12, 86: 0.2,
              87: 0.2, 88: 0.2, 89: 0.2, 90: 0.2, 91: 0.2, 92: 0.35, 93: 0.35, 94: 0.35,
              95: 0.3, 96: 0.28, 97: 0.26, 98: 0.26, 99: 0.25, 100: 0.26}
# MFMA rate of a CU relative to fp32, per precision
RATE = {"fp32": 1.0, "bf16": 16.0, "bf16x3": 16.0 / 3}
CU_MFLOP_PER_US = 0.614          # fp32 MFMA: 256 flop/clk/CU at 2.4 GHz
ROUND_OVERHEAD_US = 8.0          # launch, prologue and epilogue of one round of workgroups
REDUCE_US = 3.0                  # split-K reduce kernel launch
DEFAULT_CUS = 256


def device_cus() -> int:
    try:
        from kiln.hip import lib as kl

        return kl.device_info()["cus"]
    except Exception:  # library not built: the heuristic still works with MI355X's count
        return DEFAULT_CUS


def matmul_shape(kernel):
    mm = next(n for n in kernel.nodes if n.op == "matmul")
    a, b = mm.inputs
    batch = math.prod(a.shape[:-2]) if a.type.rank == 3 else 1
    return batch, a.shape[-2], b.shape[-1], a.shape[-1]


def skinny_fits(m, k, tile=None) -> bool:
    """Shapes the skinny-M kernel is offered for (with ``tile``: that
    configuration's waves can hold their share of K)."""
    if m > 256 or k % 4:
        return False
    if tile is None:
        return True
    share = math.ceil(math.ceil(k / 16) / TILES[tile][5])
    return share <= SKINNY_DEPTH[tile] * SKINNY_TURNS


def k_major_fits(m, k, tile) -> bool:
    """Whether configuration ``tile`` (one reading B as [N][K]) takes a
    product with m rows and depth k."""
    if tile in SKINNY:
        return skinny_fits(m, k, tile)
    if tile in SMALL_M and m > SMALL_M_MAX:
        return False
    return k % TILES[tile][2] == 0 and k > 0


def fits(tile, m, n, k) -> bool:
    bm, bn = TILES[tile][:2]
    p2 = lambda x: 1 << max(0, (x - 1).bit_length())
    return bm <= max(16, p2(m)) and bn <= max(16, p2(n))


def estimate(tile, splitk, batch, m, n, k, cus) -> float:  # noqa: C901
    """Modelled microseconds: rounds of co-resident workgroups x a fixed
    overhead, plus the MFMA time of the busiest CU (its workgroups share the
    CU's matrix cores), plus the split-K reduce (partials through HBM)."""
    bm, bn, bk = TILES[tile][:3]
    units = math.ceil(m / bm) * math.ceil(n / bn) * batch * splitk
    rounds = math.ceil(units / (cus * OCCUPANCY[tile]))
    kper = math.ceil(k / splitk / bk) * bk
    per_cu = (math.ceil(units / cus) * 2 * bm * bn * kper / 1e6 / CU_MFLOP_PER_US / EFFICIENCY[tile]
              / RATE[PRECISION[tile]])
    t = rounds * ROUND_OVERHEAD_US + per_cu
    if splitk > 1:
        t += REDUCE_US + batch * m * n * 4 * (splitk + 1) / 4e6
    return t


def default_matmul_config(graph, kernel, cus=None) -> dict:
    """Tile and split-K for a matmul kernel, without measuring.

    Prefer the largest tile that gives every CU a workgroup; when no tile can
    (M = 128 shapes on 256 CUs), pick the tile / split-K pair with the lowest
    modelled time.
    """
    batch, m, n, k = matmul_shape(kernel)
    return default_config_for(batch, m, n, k, cus)


def default_config_for(batch, m, n, k, cus=None, precision="fp32", skinny=True) -> dict:
    """``skinny=False`` leaves out the configurations that read B as a [N][K]
    copy (for a product whose B is not a constant)."""
    if m == 1 and precision == "fp32":
        return {"tile": 0, "splitk": 0}
    cus = cus or device_cus()
    best = None
    for tile in TILES:
        if tile in SPILLING or PRECISION[tile] != precision or not fits(tile, m, n, k):
            continue
        if tile in NK_B and not (skinny and k_major_fits(m, k, tile)):
            continue
        for s in SPLITS:
            if tile in NK_B and s > 1:
                continue
            if s > 1 and k // s < 128:
                continue
            t = estimate(tile, s, batch, m, n, k, cus)
            if best is None or t < best[0]:
                best = (t, tile, s)
    if best is None:
        return {"tile": {"fp32": 11, "bf16": 19, "bf16x3": 30}[precision], "splitk": 1}
    return {"tile": best[1], "splitk": best[2]}


# configurations the compiler builds with register spills (scratch), never
# worth timing: 22 (64 x 128, 64-deep K steps)
SPILLING = {22}


def candidates(batch, m, n, k, cus=None, precision="fp32") -> list:
    if m == 1 and precision == "fp32":
        return [{"tile": v, "splitk": s} for v, s in GEMV_CANDIDATES if s == 0 or k // s >= 64]
    cus = cus or device_cus()
    out = []
    for tile in TILES:
        if tile in SPILLING or PRECISION[tile] != precision or not fits(tile, m, n, k):
            continue
        if tile in NK_B:
            if k_major_fits(m, k, tile):
                out.append({"tile": tile, "splitk": 1})
            continue
        for s in SPLITS:
            if s > 1 and k // s < 64:
                continue
            units = math.ceil(m / TILES[tile][0]) * math.ceil(n / TILES[tile][1]) * batch * s
            if s > 1 and units > 4 * cus:
                continue
            out.append({"tile": tile, "splitk": s})
    return out


SHIPPED_PATH = Path(__file__).resolve().with_name("tuned_configs.json")


def _read_table(path: Path) -> dict:
    """A JSON object file as a dict; {} when missing, unreadable or not an object."""
    try:
        data = json.loads(path.read_text())
    except (OSError, ValueError):
        return {}
    return data if isinstance(data, dict) else {}


def shipped_configs() -> dict:
    """The shipped table {key: entry} (empty if absent or unreadable)."""
    return _read_table(SHIPPED_PATH)


def cache_path() -> Path:
    base = os.environ.get("KILN_CACHE_DIR") or os.path.join(Path.home(), ".cache", "kiln")
    return Path(base) / "hip_autotune.json"


def _usable(entry) -> bool:
    return isinstance(entry, dict) and isinstance(entry.get("config"), dict)


def _linear_graph(batch, m, n, k, weight, bias, a16=False):
    """What a candidate is timed on: an nn.Linear as the frontend imports and
    freezes it - activations [.., M, K] times a constant [K, N] weight, the
    bias added in the GEMM epilogue. a16: the activations are a LayerNorm's
    output (without affine parameters), which a bf16 plan stores as bf16 for
    the configurations that read A that way - the A operand of every bf16
    product of a transformer block."""
    from kiln.ir import Graph, TensorType

    g = Graph("matmul")
    x = g.add_arg(TensorType(((batch,) if batch > 1 else ()) + (m, k)), "a")
    if a16:
        from kiln.frontend.fx_import import _Builder, expand_layer_norm

        x = expand_layer_norm(_Builder(g), x, 1, None, None, LN_EPS)[0]
    product = g.add_node("matmul", [x, g.constant(weight, "b")])
    g.results = [g.add_node("add", [product, g.constant(bias, "bias")])]
    return g


LN_EPS = 1e-5


class _Trial:
    """One candidate configuration, built and checked, ready to be timed."""

    def __init__(self, config, exe, inputs, output):
        self.config = config
        self.exe = exe
        self.ins = [t.data_ptr() for t in inputs]
        self.outs = [output.data_ptr()]
        self.best = float("inf")
        # the product's own launches (a LayerNorm in front of it is not timed)
        names = [launch.name for launch in exe.program.launches]
        mm = [i for i, name in enumerate(names) if "matmul" in name]
        self.index = mm[0] if len(names) > 1 and len(mm) == 1 else -1

    @property
    def key(self):
        return (self.config["tile"], self.config["splitk"])

    def measure(self, repeats, rounds):
        from kiln.hip.runtime import current_stream_handle

        t = self.exe.plan.time(self.ins, self.outs, current_stream_handle(), index=self.index, repeats=repeats,
                               rounds=rounds)
        self.best = min(self.best, t)
        return t


class GPUAutotuner:
    """Chooses GEMM configurations by measurement, with an on-disk cache."""

    def __init__(self, precision="fp32", use_cache=True, use_shipped=True):
        self.precision = precision
        self.use_cache = use_cache
        self.log = []
        self._cache = _read_table(cache_path()) if use_cache else {}
        self._shipped = shipped_configs() if use_shipped else {}

    @staticmethod
    def device_key():
        from kiln.hip import lib as kl

        info = kl.device_info()
        return f"{info['arch']}|{info['cus']}"

    def _remember(self, key, entry):
        self._cache[key] = entry
        if not self.use_cache:
            return
        path = cache_path()
        try:
            path.parent.mkdir(parents=True, exist_ok=True)
            tmp = path.with_name(f".{path.name}.{os.getpid()}.tmp")
            tmp.write_text(json.dumps(self._cache, indent=1, sort_keys=True))
            os.replace(tmp, path)
        except OSError as err:
            warnings.warn(f"Kiln: couldn't write the GPU autotune cache ({err})")

    def config_for(self, graph, kernel, a16=False):
        """The configuration for ``kernel``'s matmul: cached, shipped, or
        measured now (and cached). Every answer is logged. a16: the plan can
        store the product's A operand as bf16 (bf16: its producer rounds it)
        or as pair words (bf16x3: its producer splits it), so candidates are
        timed that way and keyed apart."""
        batch, m, n, k = matmul_shape(kernel)
        a16 = bool(a16) and self.precision in ("bf16", "bf16x3")
        key = f"{self.device_key()}|{self.precision}{'+a16' if a16 else ''}|{batch}x{m}x{n}x{k}"
        if a16 and self.precision == "bf16x3" and not any(_usable(t.get(key)) for t in (self._cache, self._shipped)):
            # three-pass products reading pair-stored A: timed that way only
            # ahead of time (tune_shipped), else the plain entry
            a16 = False
            key = f"{self.device_key()}|{self.precision}|{batch}x{m}x{n}x{k}"
        for source, table in (("cache", self._cache), ("shipped", self._shipped)):
            if _usable(table.get(key)):
                entry = table[key]
                break
        else:
            source = "tuned"
            entry = self.tune(batch, m, n, k, default_config_for(batch, m, n, k, precision=self.precision), a16=a16)
            if entry["candidates"]:
                self._remember(key, entry)
        self.log.append({"shape": (batch, m, n, k), "source": source, **({"a16": True} if a16 else {}), **entry})
        return dict(entry["config"])

    # the lowering may pass a16 (a user's fn(graph, kernel) gets two arguments)
    config_for.accepts_a16 = True

    def _build(self, config, batch, m, n, k, weight, bias, a16=False):
        from kiln.api import Options, compile_graph

        options = Options(device="cuda", cuda_graphs=False, matmul_precision=self.precision,
                          gpu_matmul_config=lambda *_: dict(config))
        exe, _ = compile_graph(_linear_graph(batch, m, n, k, weight, bias, a16), options)
        return exe

    def _trials(self, batch, m, n, k, configs, a16=False):
        """Build every configuration and keep those whose result matches
        float64; returns (trials, reasons for the rejected ones)."""
        import torch

        from kiln.hip.runtime import device

        gen = torch.Generator().manual_seed(0)
        lead = (batch,) if batch > 1 else ()
        x = torch.randn(*lead, m, k, generator=gen)
        w = torch.randn(*lead, k, n, generator=gen) / math.sqrt(k)
        bias = torch.randn(n, generator=gen) * 0.02
        a = x.double()
        if a16:
            a = (a - a.mean(-1, keepdim=True)) / (a.var(-1, unbiased=False, keepdim=True) + LN_EPS).sqrt()
        exact = a @ w.double() + bias.double()
        scale = float(exact.abs().max()) or 1.0
        tolerance = 1e-4 if self.precision == "fp32" else 2e-2
        x_dev = x.to(device())
        trials, rejected = [], []
        for config in configs:
            try:
                exe = self._build(config, batch, m, n, k, w.numpy(), bias.numpy(), a16)
                (out,) = exe(x_dev)
                err = float((out.double().cpu() - exact).abs().max()) / scale
            except Exception as failure:  # noqa: BLE001 - a candidate that fails is dropped, never fatal
                first = str(failure).splitlines()[0][:80] if str(failure) else ""
                rejected.append(f"{config}: {type(failure).__name__}: {first}")
                continue
            if err <= tolerance:
                trials.append(_Trial(config, exe, [x_dev], out))
            else:
                rejected.append(f"{config}: relative error {err:.1e}")
        return trials, rejected

    def tune(self, batch, m, n, k, default, a16=False):
        started = time.perf_counter()
        configs = [default] + [c for c in candidates(batch, m, n, k, precision=self.precision) if c != default]
        trials, rejected = self._trials(batch, m, n, k, configs, a16)
        if not trials:
            warnings.warn(f"Kiln: no GEMM config passed for {batch}x{m}x{n}x{k}; keeping the default. "
                          + "; ".join(rejected[:3]))
            return {"config": dict(default), "default_config": dict(default), "tflops": None,
                    "default_tflops": None, "candidates": 0, "seconds": round(time.perf_counter() - started, 1)}
        # successive halving: a short measurement of everyone, then a longer
        # one of the fastest quarter (the default always stays in)
        for t in trials:
            t.measure(repeats=10, rounds=2)
        ranked = sorted(trials, key=lambda t: t.best)
        keep = ranked[:max(FINALISTS, len(ranked) // 4)]
        base = next((t for t in trials if t.config == default), None)
        if base is not None and base not in keep:
            keep.append(base)
        for t in keep:
            t.best = float("inf")
        for _ in range(2):           # interleaved, so drifting clocks affect all alike
            for t in keep:
                t.measure(repeats=20, rounds=3)
        winner = min(keep, key=lambda t: t.best)
        if base is not None and base.best <= winner.best * KEEP_DEFAULT_MARGIN:
            winner = base
        flops = 2 * batch * m * n * k
        return {
            "config": dict(winner.config),
            "default_config": dict(default),
            "tflops": round(flops / winner.best / 1e12, 2),
            "default_tflops": round(flops / base.best / 1e12, 2) if base is not None else None,
            "candidates": len(trials),
            "seconds": round(time.perf_counter() - started, 1),
        }
