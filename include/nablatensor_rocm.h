/*
 * nablatensor_rocm.h — C ABI of the MI355X (gfx950) fused forward+adjoint
 * Monte-Carlo tape-replay engine.
 *
 * This is the drop-in boundary behind the reference's `rocm` AadEngine. A Java
 * adapter binds these symbols with java.lang.foreign downcalls exactly where
 * the reference binds libamdhip64/libhiprtc (nablatensor-engine-rocm/src/main/
 * java/com/nablatensor/backend/rocm/HipRuntime.java:79-125); a C++ host (this
 * repository's nablatensor_amd/host) binds them the same way.
 *
 * Conventions: every entry point returns int status, NT_OK (0) on success;
 * negative values are engine errors (NT_E_*), positive values are hipError_t
 * or hiprtcResult codes passed through. nt_last_error() returns the message of
 * the calling thread's last failure. Only plain pointers and sizes cross the
 * boundary; the caller owns every array it passes and the engine keeps none of
 * them past the call. An nt_exec is not thread-safe; use one per thread.
 */
#ifndef NABLATENSOR_ROCM_H
#define NABLATENSOR_ROCM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NT_ABI_VERSION 3

enum {
  NT_OK = 0,
  NT_E_INVALID = -1,      /* bad argument (IllegalArgumentException in the reference) */
  NT_E_UNSUPPORTED = -2,  /* tape the engine declines (UnsupportedOperationException) */
  NT_E_NO_DEVICE = -3,    /* no usable gfx950 device (IllegalStateException) */
  NT_E_COMPILE = -4,      /* hipRTC compile failure; nt_last_error() carries the log */
  NT_E_CLOSED = -5,       /* executable already destroyed (IllegalStateException) */
  NT_E_INTERNAL = -6
};

/* Opcodes: AadOpEnum ordinals (nablatensor-core/.../engine/AadOpEnum.java:19-50). */
enum {
  NT_OP_CONST = 0, NT_OP_INPUT, NT_OP_RANDN, NT_OP_RANDU, NT_OP_ADD, NT_OP_SUB, NT_OP_MUL,
  NT_OP_DIV, NT_OP_NEG, NT_OP_EXP, NT_OP_LOG, NT_OP_SQRT, NT_OP_MAX, NT_OP_MIN, NT_OP_ABS
};

/* A recorded tape as the flat arrays of FlatTape
 * (nablatensor-core/.../engine/FlatTape.java:37-79) plus the random-stream
 * counts of AadTape (AadTape.java:116-196). */
typedef struct nt_tape {
  int32_t n_nodes;
  const int32_t *op;        /* opcode per node */
  const int32_t *arg_a;     /* node index; input index (INPUT); draw ordinal (RANDN/RANDU) */
  const int32_t *arg_b;     /* node index; stream index (RANDN/RANDU); -1 when unused */
  const double *constant;   /* literal for CONST nodes */
  int32_t n_inputs;
  const int32_t *input_node;
  int32_t n_outputs;
  const int32_t *output_node;
  int32_t n_streams;        /* random streams (AadTape.randStreamCount), at least 1; stream 0 is the default */
  int32_t n_uniforms;       /* RANDU draws on the default stream (AadTape.randUniformCount(0)); informational,
                               the lowering reads every draw from its node */
} nt_tape;

enum { NT_FP64 = 0, NT_FP32 = 1 };

/* Reverse-sweep storage policy for a rolled step loop. */
enum {
  NT_CKPT_AUTO = 0,       /* cost model picks one of the below */
  NT_CKPT_RECOMPUTE = 1,  /* carries checkpointed per segment; the reverse recomputes each segment */
  NT_CKPT_STORE_DRAWS = 2,/* draw-derived (inactive) values stored; active values recomputed */
  NT_CKPT_STORE_ALL = 3   /* every value the reverse reads is stored; nothing recomputed (a tape with no rolled
                             loop: not cut into segments, every forward value kept live) */
};

/* How the first-order Greeks are propagated. Both give the same derivatives
 * (the pathwise gradient of the output); they differ in cost and rounding. */
enum {
  NT_MODE_AUTO = 0,       /* cost model picks one of the below per tape */
  NT_MODE_REVERSE = 1,    /* adjoint sweep after the forward pass (ScalarReplay.java:129-183) */
  NT_MODE_TANGENT = 2     /* sparse forward tangents carried with the values, one per input the node depends on */
};

/* Options (AadOptions.java:42-156 precision/adjoints, plus the engine's own
 * knobs that the reference passes as engineOptions). Zero means default. */
typedef struct nt_options {
  int32_t precision;        /* NT_FP64 or NT_FP32 */
  int32_t adjoints;         /* 1: value + every first-order Greek; 0: price only (lowered in the tangent frame with
                               no tangents unless mode is NT_MODE_REVERSE, so nt_exec_replay_many shares draws) */
  int32_t block;            /* threads per block; 0 = 256 */
  int32_t max_blocks;       /* grid cap; 0 = the engine's launch geometry (whole blocks per CU from occupancy,
                               up to 8 resident grids for a long path; nt_exec_grid reports it) */
  int32_t checkpoint;       /* NT_CKPT_* */
  int32_t seg_len;          /* loop iterations per checkpoint segment; 0 = cost model. For a tape with no rolled
                               loop swept in reverse: nodes per checkpointed segment (0: about sqrt(nodes), at
                               least 48, on tapes over 512 nodes, as AadCheckpointPlan.java:95-110) */
  int32_t roll;             /* 1 (default): roll the step loop when one is found; -1: never */
  int32_t contract;         /* FMA contraction of the tape's own products and sums: 0 default (off for fp64, on for
                               fp32, plus the fused exponent of a step's multiplicative carry, whose value is
                               rebuilt from a product of factors anyway, the fp64 tangent loop's sums of products
                               of values with no tangent, such as correlated normals, and a carry's exponent sum
                               taken as N p + r S after the loop), 1 on, -1 off (every product and sum of a node
                               rounded separately). The skeleton's math routines and the tangent rules use
                               explicit fma either way */
  int32_t libm;             /* fp64 Box-Muller: 0 the skeleton's own log/sqrt/sincos, 1 device libm, 2 own log/sqrt + libm sincos */
  int32_t mode;             /* NT_MODE_* */
  int32_t markets;          /* nt_lower / nt_compile_check only: lower the kernel that prices this many input
                               sets from each path's draws (what nt_exec_replay_many compiles); 0 or 1 = one */
  int32_t waves;            /* replay kernel: ask the compiler for at least this many waves per SIMD (a register
                               budget; it may fail to meet it or spill); 0 = the engine's choice */
  int32_t basis;            /* tangent loops: the directions the step loop's tangents run over. 0 = the engine's
                               choice, 1 = the inputs, 2 = the loop's parameters (the loop-invariant values the
                               step reads and the carried values' start values), mapped back to the inputs
                               once per path after the loop */
  int32_t allow_spill;      /* 0 (default): a tape whose replay kernel would spill registers to scratch memory
                               is declined with NT_E_UNSUPPORTED by nt_exec_create and nt_compile_check, as the
                               reference's engines decline a tape in compile() so that engine selection falls back
                               (AadEngine.java:50-59); 1: compile and run it anyway */
  int32_t reserved[2];
} nt_options;

typedef struct nt_exec nt_exec;

/* Static facts about a compiled executable (for tests, reports and profiles). */
typedef struct nt_exec_info {
  int32_t n_nodes, n_active, n_inputs, n_channels;  /* channels = 2 + n_inputs (value, value^2, grads) */
  int32_t loop_start, loop_period, loop_iters;      /* period 0: no rolled loop */
  int32_t loop_carries, seg_len, n_segments;
  int32_t checkpoint;                               /* resolved NT_CKPT_* */
  int32_t tape_slots;                               /* stored values per path per run (fp64/fp32 elements) */
  int32_t vgprs, sgprs, agprs;                      /* from the code object */
  int32_t scratch_bytes;                            /* private segment per lane; 0 means no spill */
  int32_t lds_bytes;
  int32_t block, grid_cap;
  int32_t mode;                                     /* resolved NT_MODE_REVERSE or NT_MODE_TANGENT */
  double compile_seconds;
} nt_exec_info;

/* --- device ------------------------------------------------------------- */

/* Count usable gfx950 devices; never fails for their absence (*count = 0).
 * Replaces HipRuntime.probe / HipCompute.reliable (HipCompute.java:57-71). */
int nt_probe(int32_t *count);

/* Name and arch of device 0 ("AMD Instinct MI355X", "gfx950").
 * Replaces HipCompute.deviceName/arch (HipCompute.java:73-95). */
int nt_device_name(char *name, int32_t name_len, char *arch, int32_t arch_len);

/* --- lowering (no device needed) ----------------------------------------- */

/* Lower a tape to its HIP source text. *len in: buffer size; out: bytes needed
 * including the terminator. Replaces CudaAadCodegen.generate
 * (nablatensor-core/.../engine/CudaAadCodegen.java:42-102). */
int nt_lower(const nt_tape *tape, const nt_options *options, char *source, int64_t *len);

/* Lower and compile for gfx950 with hipRTC, without a device; fills *info with
 * the loop plan and the code object's register/scratch usage. Used by build
 * checks and to prefill the code-object cache. Returns NT_E_UNSUPPORTED (with
 * *info filled) when the kernel spills and options->allow_spill is 0. */
int nt_compile_check(const nt_tape *tape, const nt_options *options, nt_exec_info *info);

/* --- executables ---------------------------------------------------------- */

/* Validate, lower, compile (hipRTC, gfx950) and load a tape. Replaces
 * RocmAadEngine.compile -> DeviceAadExecutable.compile
 * (RocmAadEngine.java:76-86, DeviceAadExecutable.java:107-119). A tape whose
 * kernel would spill to scratch is declined with NT_E_UNSUPPORTED unless
 * options->allow_spill is set (AadEngine.java:50-59). */
int nt_exec_create(const nt_tape *tape, const nt_options *options, nt_exec **out);

/* Bind input values (n == tape n_inputs, input order). Replaces setInput +
 * uploadDoubles (DeviceAadExecutable.java:134-137,148-151). */
int nt_exec_set_inputs(nt_exec *exec, const double *inputs, int32_t n);

/* One dispatch over paths [offset, offset + paths) with Philox seed `seed`.
 * Per output o, at sums[o * (2 + n_inputs)]: the sum of the output, the sum of
 * its square, and the sum of its derivative with respect to each input j (zero
 * when built price-only), the AadTotals fields (AadTotals.java:30-40); n_sums
 * must be n_outputs * (2 + n_inputs). timing (nullable) receives {kernel_ms, wall_ms}: kernel_ms from
 * HIP events around the replay and finishing kernels on the executable's
 * stream, wall_ms from entry to sums on the host. Replaces
 * DeviceAadExecutable.replay (DeviceAadExecutable.java:139-168), returning raw
 * sums instead of means so callers can combine dispatches exactly. */
int nt_exec_replay(nt_exec *exec, uint64_t paths, uint64_t offset, uint64_t seed,
                   double *sums, int32_t n_sums, double *timing);

/* Prices `markets` input sets (row-major [markets][n_inputs]) over the same paths and seed in one
 * dispatch; sums[m * n_sums_one + c] as nt_exec_replay's sums (n_sums_one of them) for set m. In tangent mode each path's
 * draws are generated once and shared by the sets in registers (a kernel is compiled per set count on
 * first use; a price-only executable is in tangent mode unless built with NT_MODE_REVERSE); a
 * reverse-sweep executable replays the sets one after another. Either way the sums are
 * bit-identical to `markets` separate nt_exec_replay calls with those inputs. The executable's bound
 * inputs are left unchanged. Replaces VulkanAadKernel.replayMany (nablatensor-engine-vulkan/.../
 * VulkanAadKernel.java:162-238), the draw-sharing form of ScenarioRunner ladders
 * (nablatensor-core/.../ScenarioRunner.java:36-70). */
int nt_exec_replay_many(nt_exec *exec, const double *input_sets, int32_t markets, uint64_t paths,
                        uint64_t offset, uint64_t seed, double *sums, int32_t n_sums, double *timing);

/* Per-path value and adjoints for paths [offset, offset + paths):
 * values[p * n_outputs + o] and grads[(p * n_outputs + o) * n_inputs + j]
 * (values[p] and grads[p * n_inputs + j] for a one-output tape). A testing aid
 * with no counterpart in the reference; it runs the same lowered sweep with a
 * per-path store. */
int nt_exec_replay_paths(nt_exec *exec, uint64_t paths, uint64_t offset, uint64_t seed,
                         double *values, double *grads);

/* Bytes of the static device array behind nt_exec_replay_noalloc (one copy per device). */
#define NT_NOALLOC_SCRATCH_BYTES (8u << 20)

/* nt_exec_replay without allocation, copies or waiting. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP stream capture, tight serving loops, harnesses that forbid hipMalloc).
 * d_inputs: n_inputs doubles in device memory (may be null when the tape has
 * no inputs); d_sums: n_sums doubles of device (or pinned host) memory that
 * receive the sums laid out as nt_exec_replay's; stream: a hipStream_t, null
 * for the executable's own stream. The call enqueues the replay and finishing
 * kernels and returns; the caller synchronizes before reading d_sums. Sums are
 * bit-identical to nt_exec_replay's for the same inputs, paths, offset and
 * seed. The per-block partials (channels x 16 ceil(grid / 8) doubles: room
 * for the replay and exception kernels' entries), the bitmap of lanes that left paths to the
 * exception kernel (one bit per lane of the grid, in a fixed 512 KiB region of
 * its own, for grids of up to 2^22 lanes) and a reverse sweep's per-lane tape, if the
 * executable keeps one in device memory, live in a static array of
 * NT_NOALLOC_SCRATCH_BYTES per device; a dispatch that needs more is refused
 * with NT_E_INVALID before anything is launched. Calls that overlap in time on
 * one device share that array and race. */
int nt_exec_replay_noalloc(nt_exec *exec, const double *d_inputs, uint64_t paths, uint64_t offset, uint64_t seed,
                           double *d_sums, int32_t n_sums, void *stream);

int nt_exec_info_get(const nt_exec *exec, nt_exec_info *info);

/* Blocks (*grid) of *block threads that a single-set dispatch of `paths`
 * launches (nt_exec_replay, nt_exec_replay_noalloc, and each set count of
 * nt_exec_replay_many). At most info.grid_cap; a long path launches more
 * blocks than the device holds at once. A measurement aid with no counterpart
 * in the reference, whose launch geometry is fixed per dispatch
 * (DeviceAadExecutable.java:196-200). */
int nt_exec_grid(const nt_exec *exec, uint64_t paths, int32_t *grid, int32_t *block);

/* Copy of the generated source (same *len protocol as nt_lower). */
int nt_exec_source(const nt_exec *exec, char *source, int64_t *len);

/* Free device buffers, the module and the stream. Replaces close()
 * (DeviceAadExecutable.java:203-221). Null is a no-op. */
int nt_exec_destroy(nt_exec *exec);

/* Thread-local message of the last failure on this thread ("" if none). */
const char *nt_last_error(void);

int nt_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif
