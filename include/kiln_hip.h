/*
 * kiln_hip.h - C ABI of Kiln's MI355X (gfx950) backend library, libkiln_hip.so.
 *
 * The library replaces the reference's generated-Triton GPU backend:
 *   kiln/gpu/codegen.py   (Triton source per fused kernel, Launch list)
 *   kiln/gpu/runtime.py   (launching, CUDA-graph capture/replay)
 *   kiln/gpu/autotune.py  (timed matmul configs; the host side stays in Python
 *                          and times plans built through this ABI)
 * Every fused Kiln kernel is lowered (in Python, kiln/hip/lowering.py) to one or
 * more kh_launch descriptors that name a hand-written HIP kernel family, its
 * operands as (buffer slot, element offset, element strides) and, for fused
 * elementwise work, an instruction tape. A plan is an ordered array of
 * descriptors; one ctypes call runs a whole compiled graph, and a plan can be
 * captured once into a hipGraph and replayed.
 *
 * Conventions
 *   - Every function returns KH_OK (0) or a KH_ERR_* code; kh_last_error()
 *     returns a thread-local message for the last failure.
 *   - Arena, constants, inputs, outputs and the workspace are device pointers
 *     owned by the caller (torch tensors) and borrowed for the plan's
 *     lifetime. The library's own device memory: a 16 MiB array per GPU for
 *     kh_plan_run_noalloc's split-K partials, and the device state of
 *     persistent GEMV chains, allocated by kh_plan_bind and freed by
 *     kh_plan_destroy.
 *   - Kernels are launched on the hipStream_t the caller passes (torch's
 *     current stream), so ordering with the caller's own work is preserved.
 *   - A plan is not reentrant: calls share one arena and one workspace
 *     (as in the reference, kiln/gpu/runtime.py:136).
 *   - No HIP/torch types appear in signatures: streams are passed as void*.
 */
#ifndef KILN_HIP_H
#define KILN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KH_ABI_VERSION 1

#define KH_MAX_RANK 6     /* iteration-space rank of one launch              */
#define KH_MAX_REFS 12    /* operands (loads and stores) of one launch        */
#define KH_MAX_INSNS 96   /* tape length                                      */
#define KH_NREGS 16       /* tape registers                                   */
#define KH_MAX_PASSES 8   /* row-kernel passes (reduction levels + output)    */

/* status codes */
enum {
  KH_OK = 0,
  KH_ERR_INVALID = 1,     /* malformed descriptor or argument -> ValueError          */
  KH_ERR_UNSUPPORTED = 2, /* no kernel for this descriptor -> NotImplementedError    */
  KH_ERR_HIP = 3,         /* a HIP runtime call failed -> RuntimeError               */
  KH_ERR_NO_DEVICE = 4,   /* no usable gfx950 device -> RuntimeError                 */
  KH_ERR_CAPACITY = 5     /* workspace too small for the plan -> MemoryError         */
};

/* buffer slots an operand can live in (reference Launch.bases, codegen.py:106-117) */
enum { KH_BASE_INPUT = 0, KH_BASE_OUTPUT = 1, KH_BASE_CONST = 2, KH_BASE_ARENA = 3, KH_BASE_WORKSPACE = 4 };

/* kernel families (reference _KernelWriter.write dispatch, codegen.py:532-542) */
enum {
  KH_FAM_EW = 1,   /* elementwise DAG / copy over one output shape            */
  KH_FAM_ROW = 2,  /* innermost-dim reductions + elementwise (LN, softmax...) */
  KH_FAM_GEMM = 3, /* [batched] matmul + epilogue tape, MFMA                  */
  KH_FAM_GEMV = 4, /* M = 1 matmul + epilogue tape                            */
  KH_FAM_RED = 5,  /* reduction over non-innermost dims                       */
  KH_FAM_ATTN = 6  /* fused scores -> softmax -> x V (the lowering's pattern)  */
};

/* attention family: how the scores are scaled and masked before the softmax */
enum { KH_ATTN_MASK_NONE = 0, KH_ATTN_MASK_CAUSAL = 1, KH_ATTN_MASK_ADD = 2 };
enum { KH_ATTN_SCALE_NONE = 0, KH_ATTN_SCALE_MUL = 1, KH_ATTN_SCALE_DIV = 2 };

/* row-family variants chosen by the host pattern matcher */
enum { KH_ROW_GENERIC = 0, KH_ROW_LAYERNORM = 1, KH_ROW_SOFTMAX = 2 };

/* GEMM precisions */
enum { KH_PREC_FP32 = 0, KH_PREC_BF16 = 1, KH_PREC_BF16X3 = 2 };
/* Prologues (kh_launch.cfg[4] of a KH_FAM_GEMV launch; LayerNorm also of a
 * KH_FAM_GEMM launch on an fp32 small-M configuration) */
enum { KH_GEMV_PRO_NONE = 0, KH_GEMV_PRO_LAYERNORM = 1, KH_GEMV_PRO_ATTN = 2 };
/* GEMV launch flag (kh_launch.variant of a KH_FAM_GEMV launch): the launch
 * may run inside a persistent chain with the flagged GEMV launches next to it
 * (kh_plan_chains); no counterpart in the reference. */
enum { KH_GEMV_CHAIN = 1 };

/*
 * Tape: a straight-line program over KH_NREGS slots, each slot holding the
 * values of 4 adjacent elements of the iteration space (a per-row scalar or
 * broadcast value is the same in all 4). Operands a/b are slot numbers or
 * KH_SRC_IMM (the instruction's immediate).
 *   LOAD  dst slot <- operand ref `a` at the current elements
 *   STORE operand ref `dst` <- slot `a`
 *   RSUM / RMAX (row family): slot `dst` accumulates the sum / max of slot `a`
 *         over the valid columns of the current chunk
 *   other ops: dst slot <- op(a, b)
 * Loads at the start of a tape (or of a row pass) are issued together.
 * Tapes that use at most 8 slots run with the slots in VGPRs.
 */
enum {
  KH_OP_MOV = 0,  KH_OP_ADD, KH_OP_SUB, KH_OP_MUL, KH_OP_DIV, KH_OP_MAX, KH_OP_MIN,
  KH_OP_NEG, KH_OP_RELU, KH_OP_EXP, KH_OP_TANH, KH_OP_SIGMOID, KH_OP_ERF,
  KH_OP_GELU_TANH, KH_OP_GELU_ERF, KH_OP_RSQRT, KH_OP_SQRT,
  KH_OP_RSUM, KH_OP_RMAX, KH_OP_LOAD, KH_OP_STORE,
  KH_OP_COUNT
};

#define KH_SRC_IMM 0xFF

typedef struct kh_ref {
  int32_t base;                 /* KH_BASE_*                                    */
  int32_t index;                /* input/output/const slot (0 for arena/ws)     */
  int64_t offset;               /* element offset from the slot's pointer       */
  int64_t strides[KH_MAX_RANK]; /* element stride per iteration dim; 0 = broadcast */
} kh_ref;

typedef struct kh_insn {
  uint8_t op, dst, a, b;
  float imm;
} kh_insn;

typedef struct kh_pass {
  int16_t vec_begin, vec_end;   /* tape range run for every column chunk        */
  int16_t post_begin, post_end; /* tape range run once per row after reductions */
  uint16_t acc_mask;            /* slots that are reduction accumulators        */
  uint16_t max_mask;            /* ... of which these reduce with max           */
  int16_t single_chunk;         /* 1: row fits one chunk, slots persist         */
  int16_t pad;
} kh_pass;

/*
 * One kernel launch. Iteration spaces (rank / shape) and operand meaning:
 *   EW   shape = output shape; refs strides over shape.
 *   ROW  shape = row dims + [inner]; refs strides over that space; a per-row
 *        scalar operand has inner stride 0. passes[] splits the tape.
 *        variant KH_ROW_LAYERNORM / KH_ROW_SOFTMAX asks for the one-wave-per-row
 *        fast path (cfg[4], cfg[5], fparams describe it); the tape must still
 *        be complete, it runs when the fast path does not apply.
 *   GEMM gemm = {batch, M, N, K}. refs[0] = A with strides over (b, m, k),
 *        refs[1] = B over (b, k, n); refs[2..] are the epilogue's operands with
 *        strides over (b, m, n). The tape starts with the accumulator in slot 0.
 *        cfg[1] = tile configuration id, cfg[2] = split-K (0: library picks),
 *        cfg[3] = precision. cfg[4] = 1 (fp32 small-M configurations with at
 *        most 4 rows per wave, K <= 1024): LayerNorm prologue - refs[0] is
 *        the LayerNorm's input x and each row enters the product as (x -
 *        mean) * rstd (mean, var and eps from fparams[0..2] as for the GEMV
 *        below); gamma must already be folded into B; refs[cfg[5]] = the
 *        column sums of that B and refs[cfg[6]] = beta . B (-1: none), both
 *        per-column vectors (strides 0 over M, 1 over N), the second added to
 *        the accumulator before the tape.
 *   GEMV as GEMM with M = 1; cfg[1] = workgroup variant of the [K][N] kernel
 *        (0: library picks from the shape; 1-3: 32/16/8 columns x 256 threads;
 *        4-5: 32/16 columns x 1024 threads), cfg[2] = split-K (0: library
 *        picks). B with unit K stride ([batch][N][K], K a multiple of 4) runs
 *        the K-contiguous kernel; cfg[3] = KH_PREC_BF16 reads B as bf16
 *        [batch][N][K] (K a multiple of 8) and rounds x to bf16. cfg[4] = 1:
 *        LayerNorm prologue - refs[0] is the raw row x and the product uses
 *        (x - mean) * rsqrt(var + eps) [* gamma] [+ beta], mean = sum(x) *
 *        fparams[0], var = sum((x - mean)^2) * fparams[1], eps = fparams[2];
 *        cfg[5] / cfg[6] = ref index (>= 2) of gamma / beta, unit stride over
 *        K and stride 0 over M, or -1. cfg[4] = 2: attention prologue (decode:
 *        the head-merged output of one query's attention is the row x) -
 *        refs[0] is not read; refs[cfg[5]], +1, +2 = Q, K, V over (head,
 *        token, d) as in ATTN (+3: an additive mask over (head, query, key));
 *        cfg[0] = head dim (32 or 64, K = heads * head dim), cfg[7] = keys
 *        (1..64), cfg[6] = mask mode + 4 * scale mode, fparams[0] = scale;
 *        x[h * dh + d] = softmax_j(scaled q_h . k_jh [+ mask]) . v_jh[d].
 *        Needs the K-contiguous weight layout (B unit stride over K).
 *   RED  shape = input shape; refs[0] = input, refs[1] = output, both with
 *        strides over the input shape (the output's reduced dims stride 0);
 *        cfg[0] = bitmask of reduced dims, cfg[1] = 1 for max else sum.
 *   ATTN gemm = {batch, Tq, Tk, head dim (32 or 64)}. refs[0] = Q over
 *        (b, query, d), refs[1] = K over (b, key, d), refs[2] = V over
 *        (b, key, d), refs[3] = output over (b, query, d): unit d stride,
 *        16-byte aligned rows. s = q.k, then (cfg[1]) s * fparams[0] or
 *        s / fparams[0], then (cfg[0]) CAUSAL: -inf where key > query, or
 *        ADD: s + refs[4] (strides over (b, query, key)); out = softmax(s) V.
 *        cfg[2] = waves per workgroup splitting the keys (0: library picks),
 *        cfg[3] = queries per workgroup (0: library picks, 16 or 32),
 *        cfg[5] = products precision: 0 fp32; 1 bf16 inputs (q and k for the
 *        scores, the softmax weights and v for the weighted sum rounded to
 *        bf16, round to nearest even; scores, softmax and accumulation
 *        fp32); 2 three-pass bf16 (each of those inputs split into hi =
 *        bf16(x) and lo = bf16(x - hi), lo 0 for a non-finite hi, a product
 *        taken as lo.hi + hi.lo + hi.hi; fp32 q, k, v and 32 queries per
 *        workgroup).
 * cfg[] holds the family configuration (GEMM: tile id, split-K, precision).
 * bf16 storage (ROW, ATTN, GEMM): bit j of cfg[7] says refs[j] holds bf16
 * values (round to nearest even), its offset and strides counted in bf16
 * elements. Accepted only where a kernel implements it, else
 * KH_ERR_UNSUPPORTED: the output of the one-wave LayerNorm (offset and row
 * stride multiples of 4), the output of the blocked attention kernel (refs[3],
 * 8-element aligned rows) and its q, k, v together (refs[0..2], with bf16
 * products, cfg[5] = 1, and 32 queries per workgroup; 16-byte aligned rows),
 * and on the bf16 configurations 95-100 of a GEMM the
 * A operand (bit 0; unit K stride, rows 8-element aligned) and the output ref
 * of a direct epilogue (its bit; unit N stride, rows 4-element aligned).
 * Pair storage (ROW, ATTN, GEMM): bit 16 + j of cfg[7] says refs[j] holds each
 * value x as one 32-bit word, bf16(x) in the low half and bf16(x - bf16(x))
 * (0 for a non-finite bf16(x)) in the high half - the halves a three-pass
 * product splits x into - addressed like fp32. Accepted for the output of the
 * one-wave LayerNorm, the output of the blocked attention kernels and, with
 * three-pass products (cfg[5] = 2), its q, k, v together, and on the
 * three-pass GEMM configurations the A operand (bit 16) and the output of a
 * direct epilogue without split-K.
 */
typedef struct kh_launch {
  int32_t family;
  int32_t variant;
  int32_t rank;
  int32_t n_refs;
  int32_t n_insns;
  int32_t n_passes;
  int32_t cfg[8];
  float fparams[4];
  int64_t shape[KH_MAX_RANK];
  int64_t gemm[4];
  kh_ref refs[KH_MAX_REFS];
  kh_insn insns[KH_MAX_INSNS];
  kh_pass passes[KH_MAX_PASSES];
  char name[32];
} kh_launch;

typedef struct kh_plan kh_plan;

/* library -------------------------------------------------------------------- */
int kh_version(void);
/* Digest of the sources and flags the library was built from (build.py
 * compiles it in): part of the key under which lowered plans are stored, the
 * counterpart of the reference's content-addressed kernel cache
 * (kiln/gpu/runtime.py:53-79), so no stored plan outlives a rebuild that may
 * read its descriptors differently. */
const char *kh_build_id(void);
/* sizeof(kh_launch), sizeof(kh_ref), sizeof(kh_insn), sizeof(kh_pass): lets a
 * binding check its struct mirrors against the compiled library. */
int kh_abi_sizes(size_t *sizes4);
const char *kh_last_error(void);
/* Select `device`, check it is gfx950, cache CU count. */
int kh_init(int device);
/* Device facts: compute units, LDS bytes per CU, gfx arch string (>= 16 bytes). */
int kh_device_info(int *cus, int *lds_bytes, char *arch, int arch_len);
/* Number of GEMM tile configurations compiled into the library, and their shape:
 * out[0..7] = {BM, BN, BK, WM, WN, WK, MFMA, precision}. */
int kh_gemm_config_count(void);
int kh_gemm_config(int id, int32_t *out8);

/* plans: replace generate() + GPUExecutable (codegen.py:601-614, runtime.py:135-217) */
int kh_plan_create(const kh_launch *launches, int n_launches, kh_plan **out);
/* Workspace bytes the plan needs (dense split-K partials, reused by every
 * launch in turn); the caller allocates it and passes it to kh_plan_bind. Its
 * contents need no initialisation: each split-K launch writes all the partials
 * it reads back. kh_plan_bind accepts workspace = NULL with 0 bytes (no
 * workspace bound): kh_plan_run then fails with KH_ERR_CAPACITY on a plan that
 * needs one, and kh_plan_run_noalloc runs it. */
int kh_plan_workspace_bytes(const kh_plan *plan, size_t *bytes);
int kh_plan_bind(kh_plan *plan, void *const *consts, int n_consts, void *arena, void *workspace,
                 size_t workspace_bytes);
/* Run every launch in order on `stream` (GPUExecutable._run, runtime.py:164-179). */
int kh_plan_run(kh_plan *plan, void *const *inputs, int n_inputs, void *const *outputs, int n_outputs,
                void *stream);
/*
 * kh_plan_run without a caller workspace. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under hipGraph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The split-K
 * partials go to a device array of KH_NOALLOC_WORKSPACE_BYTES that the library
 * holds on each GPU it runs on until the process ends; the call allocates
 * nothing. The plan is bound as for kh_plan_run (constants and arena; its
 * workspace argument may be NULL with 0 bytes). Returns KH_ERR_CAPACITY when
 * kh_plan_workspace_bytes exceeds KH_NOALLOC_WORKSPACE_BYTES. Every call on one
 * GPU shares that GPU's array and the array keeps the last call's contents:
 * calls that overlap on one GPU (other streams, other threads) race.
 */
#define KH_NOALLOC_WORKSPACE_BYTES (16u << 20)
int kh_plan_run_noalloc(kh_plan *plan, void *const *inputs, int n_inputs, void *const *outputs, int n_outputs,
                        void *stream);
/* The plan's meaning executed on the CPU: every launch, in order, element by
 * element, over HOST memory (inputs, outputs, and the constants and arena
 * bound with kh_plan_bind must all be host pointers; no workspace is used).
 * The counterpart of the reference's interpreter switch
 * (kiln/gpu/runtime.py:39-50, Triton's TRITON_INTERPRET): it lets the CPU test
 * suite check the lowering's descriptors, addressing and tapes against the
 * oracle without a GPU. A test instrument: the GPU path never calls it.
 * Products and attention accumulate in double, so results agree with the
 * GPU kernels to rounding, not bit for bit. */
int kh_plan_run_host(kh_plan *plan, void *const *inputs, int n_inputs, void *const *outputs, int n_outputs);
/* Run one launch (per-kernel profiling). */
int kh_plan_run_one(kh_plan *plan, int index, void *const *inputs, int n_inputs, void *const *outputs,
                    int n_outputs, void *stream);
/* Capture the whole plan over fixed input/output buffers into a hipGraph
 * (GPUExecutable._capture, runtime.py:191-204) and replay it on `stream`. */
int kh_plan_capture(kh_plan *plan, void *const *inputs, int n_inputs, void *const *outputs, int n_outputs);
int kh_plan_replay(kh_plan *plan, void *stream);
/* GPU seconds per execution of launch `index` (every launch when index = -1),
 * the reference's kernel_seconds method (kiln/gpu/runtime.py:93-132) done in
 * the library: after two plain launches on `stream`, `repeats` executions are
 * captured into a hipGraph of their own (the plan's replay graph is left
 * alone), replayed once, then `rounds` replays are timed with hipEvents on
 * `stream`; *seconds = the fastest replay / repeats. Synchronises `stream`.
 * The autotuner times candidate plans with it. */
int kh_plan_time(kh_plan *plan, int index, void *const *inputs, int n_inputs, void *const *outputs, int n_outputs,
                 int repeats, int rounds, void *stream, double *seconds);
/*
 * Persistent GEMV chains. No counterpart in the reference, which launches
 * every kernel on its own. Consecutive launches flagged KH_GEMV_CHAIN whose
 * operands allow it (each reads the whole output of the one before: decode's
 * GEMV after GEMV) run as ONE launch in which each stage's weights stream
 * while the previous stage's outputs are handed over. kh_plan_bind sets up a
 * chain's device state (it allocates: descriptors, one 8-byte hand-over word
 * per output column of every stage, an epoch); a chain that could not be
 * bound (no GPU) runs launch by launch. kh_plan_run, kh_plan_run_noalloc,
 * kh_plan_capture and kh_plan_time(index -1) take the one launch;
 * kh_plan_run_one and kh_plan_time of one index run the launch alone.
 * kh_plan_chains: *n_chains = the number of chains; ranges receives up to
 * max_chains triples {first launch, number of launches, active}.
 */
int kh_plan_chains(const kh_plan *plan, int32_t *ranges, int max_chains, int *n_chains);
/* Waits inside the plan's chains that gave up, summed over the plan's life (a
 * bounded wait that ran out; none is expected). The workgroup that gave up
 * stored NaN as every output it still owed and left the kernel, so every
 * value computed from those outputs is NaN. Synchronises the device. */
int kh_plan_chain_timeouts(kh_plan *plan, uint64_t *timeouts);
/* Bound on each wait of the plan's chains, in ticks of the 100 MHz wall clock
 * (kh_plan_bind sets 2,000,000 = 20 ms); ticks < 0 makes every wait give up
 * at once, so tests can drive the give-up path with every kernel exiting
 * normally. No counterpart in the reference. */
int kh_plan_chain_spin(kh_plan *plan, int64_t ticks);
int kh_plan_destroy(kh_plan *plan);

/*
 * Measurement probes. No counterpart in the reference (its kernels are
 * generated and it measures them only by wall time, kiln/gpu/runtime.py
 * 93-132); these measure what bounds the hand-written attention kernel.
 *
 * kh_probe_attn_timeline: one run of the 32-query attention kernel (head
 * dimension 64, causal, scores * scale, `waves` = 4 or 8 key-split waves per
 * workgroup) over q, k, v and out given as in an ATTN launch (strides8 =
 * q, k, v, out {head, row} element strides), built with timestamps: rec
 * receives 8 uint64 per wave of every workgroup (workgroup g, wave w at
 * rec + 8 (g * waves + w)): start, loop end and end on the 100 MHz wall
 * clock, shader clock at start and end, the hardware's HW_ID and XCC_ID
 * words, and the key blocks the wave processed. rec must hold
 * 8 * waves * batch * ceil(tq / 32) words. Launches on `stream`.
 *
 * kh_probe_mfma_valu: shader cycles per 32x32x2 fp32 MFMA per SIMD
 * (out2[0]) and the shader clock in GHz (out2[1]) when each SIMD runs
 * waves_per_simd (1 or 2) waves that issue MFMAs in groups of `group`
 * back-to-back over `chains` independent accumulators, each group followed
 * by `valu` independent fp32 FMAs (timed from the first start to the last end
 * of the waves of one CU). Combinations offered (chains, group,
 * valu): (1,1,0) (2,1,0) (1,1,1) (1,1,2) (1,1,4) (2,1,2) (4,1,2) (8,1,2)
 * (1,4,8) (1,8,16) (2,8,16) (1,32,64). Allocates and synchronises the device.
 */
int kh_probe_attn_timeline(const float *q, const float *k, const float *v, float *out, int batch, int tq, int tk,
                           const int64_t *strides8, int waves, float scale, uint64_t *rec, void *stream);
int kh_probe_mfma_valu(int chains, int group, int valu, int waves_per_simd, double *out2);

#ifdef __cplusplus
}
#endif
#endif /* KILN_HIP_H */
