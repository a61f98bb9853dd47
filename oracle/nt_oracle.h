/*
 * CPU oracle for the fused forward+adjoint Monte-Carlo tape replay.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's
 * scalar `cpu` engine, against which the tests hold the HIP engine. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product path (nablatensor_amd) never links, imports or calls anything here.
 *
 * What each function restates (reference paths are relative to the reference
 * repository root):
 *   nto_philox2x32_10   Random123 philox2x32-10 round function; the loop in
 *                       nablatensor-engine-cpu/.../cpu/Philox.java:63-70
 *   nto_normal          Philox.normal(), Philox.java:45-78 (counter = k>>1,
 *                       cosine leg for even k, sine leg for odd k)
 *   nto_uniform         Philox.uniform(), Philox.java:81-94
 *   nto_mark_active     AadTape.markActive, nablatensor-core/.../AadTape.java:70-81
 *   nto_replay          ScalarReplay.run, nablatensor-engine-cpu/.../ScalarReplay.java:78-183,
 *                       split over threads as HostAadExecutable.runRanges
 *                       (nablatensor-core/.../HostAadExecutable.java:85-117)
 *   nto_replay_paths    the same per-path values and adjoints, one row per path
 *   nto_replay_paths_perturbed
 *                       the same with every transcendental result moved by one
 *                       unit (no reference counterpart: the tests' yardstick
 *                       of each path's sensitivity to libm's last place)
 *   nto_to_result       AadTotals.toResult, nablatensor-core/.../AadTotals.java:68-89
 *
 * Parity pins (tests/test_oracle.py): Random123 KATs for the round function;
 * the reference-held Asian-call aggregates (docs/validation.md:56-63);
 * Black-Scholes closed form; knock-out + knock-in = vanilla; per-path central
 * differences with common random numbers for every reverse rule (European,
 * Asian, Heston, a down-and-in barrier for DIV's second operand, a 16-asset
 * worst-of for MIN, random tapes for ABS, LOG and the rest; tests/pins.py),
 * each rule's planted mistake rejected (NTO_PLANT, tests/test_oracle_plants.py);
 * the reference's barrier adjoint-delta bump test (ExoticsTest.java:81-94) and
 * cash digital closed form (ExoticsTest.java:96-107);
 * per-path hand evaluation of the 1-step European;
 * sums and standard error against the per-path rows (sample standard
 * deviation); the Merton jump tape (uniform draws) against the exact Poisson
 * series within 1.5% (JumpModelsTest.java:46-53), its no-jump limit against
 * Black-Scholes, its adjoint delta against a bump; uniform and named-stream
 * moments as RandomStreamsTest.java:51-103.
 *
 * Parity unpinned: the named-stream key multiplier 0x9E3779B1 of nto_normal
 * and nto_uniform for a stream other than the default (Philox.java:48-50,
 * the same literal in JitPhilox.java:107). No reference file holds a value
 * drawn from a named stream, and independence (what the tests check) holds
 * for any odd multiplier, so the literal is restated from the source text
 * only. The default stream (every workload tape) is pinned as above.
 */
#ifndef NT_ORACLE_H
#define NT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opcodes in AadOpEnum ordinal order (nablatensor-core/.../AadOpEnum.java:19-50). */
enum {
  NTO_CONST = 0, NTO_INPUT, NTO_RANDN, NTO_RANDU, NTO_ADD, NTO_SUB, NTO_MUL, NTO_DIV,
  NTO_NEG, NTO_EXP, NTO_LOG, NTO_SQRT, NTO_MAX, NTO_MIN, NTO_ABS
};

/* A tape as the flat parallel arrays of FlatTape (nablatensor-core/.../FlatTape.java:37-79). */
typedef struct nto_tape {
  int32_t n;                 /* nodes */
  const int32_t *op;         /* opcode per node */
  const int32_t *arg_a;      /* node index, input index for INPUT, draw ordinal for RANDN/RANDU */
  const int32_t *arg_b;      /* node index, stream index for RANDN/RANDU */
  const double *constant;    /* literal for CONST */
  int32_t n_inputs;
  const int32_t *input_node;
  int32_t n_outputs;
  const int32_t *output_node;
  int32_t n_streams;         /* random streams (>= 1) */
} nto_tape;

/* Raw sums per output: value, value^2 and adjoint per input (AadTotals fields). */
typedef struct nto_totals {
  double *value;     /* [n_outputs] */
  double *sumsq;     /* [n_outputs] */
  double *gradient;  /* [n_outputs * n_inputs] */
} nto_totals;

void nto_philox2x32_10(uint32_t ctr0, uint32_t ctr1, uint32_t key, uint32_t out[2]);
double nto_normal(uint64_t path, uint64_t seed, int32_t stream, int32_t k);
double nto_uniform(uint64_t path, uint64_t seed, int32_t stream, int32_t k);
void nto_mark_active(const nto_tape *t, uint8_t *active);

/* Sums over paths [offset, offset+paths). f32 != 0 replays in the reference's
 * FLOAT32 semantics. threads <= 0 means omp_get_max_threads(). Returns 0 on
 * success, negative on a malformed tape. */
int nto_replay(const nto_tape *t, const double *inputs, uint64_t paths, uint64_t offset,
               uint64_t seed, int f32, int adjoints, int threads, nto_totals *out);

/* Per-path rows for every output: values[p * n_outputs + o] and
 * grads[(p * n_outputs + o) * n_inputs + j]. */
int nto_replay_paths(const nto_tape *t, const double *inputs, uint64_t paths, uint64_t offset,
                     uint64_t seed, int f32, int threads, double *values, double *grads);

/* nto_replay_paths in fp64 with every transcendental result moved by one
 * unit, up or down by the fixed pseudo-random pattern `pattern` (nonzero):
 * the log, sqrt and exp results of Box-Muller and of EXP/LOG/SQRT nodes by
 * one ulp, Box-Muller's sin and cos by 2^-53 absolute. No reference
 * counterpart: the difference from nto_replay_paths is each path's
 * sensitivity to last-place differences of libm, the yardstick the tests
 * scale their per-path bound by. */
int nto_replay_paths_perturbed(const nto_tape *t, const double *inputs, uint64_t paths, uint64_t offset,
                               uint64_t seed, int threads, uint64_t pattern, double *values, double *grads);

/* mean, standard error and mean gradient from raw sums (AadTotals.toResult). */
void nto_to_result(const nto_totals *sums, int32_t n_outputs, int32_t n_inputs, uint64_t paths,
                   double *mean, double *stderr_out, double *mean_gradient);

#ifdef __cplusplus
}
#endif
#endif
