/*
 * CPU oracle — TEST INFRASTRUCTURE ONLY (see nt_oracle.h for what may load it
 * and which reference file each function restates).
 *
 * Compiled with -ffp-contract=off and no fast-math: the reference evaluates
 * every node with separately rounded IEEE double operations and java.lang.Math
 * transcendentals; glibc's exp/log/sin/cos stand in for the latter (both are
 * within 1 ulp), so per-path results may differ from the Java engine in the
 * last place, never more.
 */
#include "nt_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define NTO_KEY0 0x1BD11BDAu
#define NTO_WEYL 0x9E3779B9u
#define NTO_MULT 0xD256D193u
#define NTO_UINT_SCALE 2.3283064365386963e-10
#define NTO_UNIFORM_TAG 0x40000000u

/* Philox.java:63-70: ten rounds of (hi,lo) = mulhilo(M, c0); c0 = hi^key^c1; c1 = lo; key += W. */
void nto_philox2x32_10(uint32_t ctr0, uint32_t ctr1, uint32_t key, uint32_t out[2]) {
  uint32_t c0 = ctr0, c1 = ctr1;
  for (int i = 0; i < 10; i++) {
    uint64_t product = (uint64_t)NTO_MULT * (uint64_t)c0;
    c0 = (uint32_t)(product >> 32) ^ key ^ c1;
    c1 = (uint32_t)product;
    key += NTO_WEYL;
  }
  out[0] = c0;
  out[1] = c1;
}

/* ---- sensitivity patterns (no reference counterpart) ------------------------
 * A perturbed replay moves every transcendental result by one unit, up or
 * down by a fixed pseudo-random pattern: log, sqrt, exp by one ulp (nextafter),
 * sin and cos by 2^-53 absolute (their errors are absolute near zero). The
 * difference from the unperturbed replay measures how much a path amplifies
 * last-bit differences of libm, which is what separates two correct engines
 * whose transcendentals differ in the last place. pattern 0 is the oracle. */
static uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

static int nudge_up(uint64_t key, uint64_t pattern) {
  return (int)(splitmix64(key ^ splitmix64(pattern)) >> 63);
}

static double nudge_rel(double x, uint64_t key, uint64_t pattern) {
  if (!pattern || !isfinite(x) || x == 0.0) return x;
  return nextafter(x, nudge_up(key, pattern) ? INFINITY : -INFINITY);
}

static double nudge_abs(double x, uint64_t key, uint64_t pattern) {
  if (!pattern || !isfinite(x)) return x;
  return nudge_up(key, pattern) ? x + 0x1p-53 : x - 0x1p-53;
}

static uint64_t path_key(uint64_t path) { return splitmix64(path * 0x9E3779B97F4A7C15ull + 0x632BE59BD9B4E019ull); }

/* One random stream, the state of a reference Philox instance (Philox.java:34-53). */
typedef struct stream_state {
  uint32_t lo, hi;
  uint32_t counter;
  uint32_t uniform_counter;
  double spare;
  int has;
  uint64_t key, pattern;  /* sensitivity pattern (0: none) and this stream's key for it */
} stream_state;

static void stream_init(stream_state *s, uint64_t path, uint64_t seed, int32_t stream) {
  uint32_t l = (uint32_t)path ^ (uint32_t)seed;
  uint32_t h = (uint32_t)(path >> 32) ^ (uint32_t)(seed >> 32);
  if (stream != 0) {
    h ^= (uint32_t)stream * 0x9E3779B1u;   /* Philox.java:48-50 */
  }
  s->lo = l;
  s->hi = h;
  s->counter = 0;
  s->uniform_counter = 0;
  s->spare = 0.0;
  s->has = 0;
  s->key = path_key(path) ^ ((uint64_t)(uint32_t)stream << 40);
  s->pattern = 0;
}

/* Philox.normal(), Philox.java:55-78. */
static double stream_normal(stream_state *s) {
  if (s->has) {
    s->has = 0;
    return s->spare;
  }
  uint32_t o[2];
  const uint64_t k = s->key ^ ((uint64_t)s->counter << 3);
  nto_philox2x32_10(s->lo, s->hi ^ s->counter++, NTO_KEY0, o);
  double u1 = ((double)o[0] + 0.5) * NTO_UINT_SCALE;
  double u2 = ((double)o[1] + 0.5) * NTO_UINT_SCALE;
  double radius = nudge_rel(sqrt(-2.0 * nudge_rel(log(u1), k ^ 1, s->pattern)), k ^ 2, s->pattern);
  double angle = 6.283185307179586 * u2;
  s->spare = radius * nudge_abs(sin(angle), k ^ 3, s->pattern);
  s->has = 1;
  return radius * nudge_abs(cos(angle), k ^ 4, s->pattern);
}

/* Philox.uniform(), Philox.java:81-94. */
static double stream_uniform(stream_state *s) {
  uint32_t o[2];
  nto_philox2x32_10(s->lo, s->hi ^ (s->uniform_counter++ | NTO_UNIFORM_TAG), NTO_KEY0, o);
  return ((double)o[0] + 0.5) * NTO_UINT_SCALE;
}

double nto_normal(uint64_t path, uint64_t seed, int32_t stream, int32_t k) {
  stream_state s;
  stream_init(&s, path, seed, stream);
  double z = 0.0;
  for (int32_t i = 0; i <= k; i++) {
    z = stream_normal(&s);
  }
  return z;
}

double nto_uniform(uint64_t path, uint64_t seed, int32_t stream, int32_t k) {
  stream_state s;
  stream_init(&s, path, seed, stream);
  s.uniform_counter = (uint32_t)k;
  return stream_uniform(&s);
}

/* AadTape.markActive, AadTape.java:70-81. */
void nto_mark_active(const nto_tape *t, uint8_t *active) {
  for (int32_t i = 0; i < t->n; i++) {
    int32_t a = t->arg_a[i], b = t->arg_b[i];
    switch (t->op[i]) {
      case NTO_INPUT: active[i] = 1; break;
      case NTO_CONST: case NTO_RANDN: case NTO_RANDU: active[i] = 0; break;
      case NTO_NEG: case NTO_EXP: case NTO_LOG: case NTO_SQRT: case NTO_ABS:
        active[i] = active[a];
        break;
      default: active[i] = (uint8_t)(active[a] || active[b]); break;
    }
  }
}

static int validate(const nto_tape *t) {
  if (t->n <= 0 || t->n_outputs <= 0 || t->n_streams <= 0) return -1;
  for (int32_t i = 0; i < t->n; i++) {
    int32_t op = t->op[i], a = t->arg_a[i], b = t->arg_b[i];
    if (op < NTO_CONST || op > NTO_ABS) return -2;
    switch (op) {
      case NTO_CONST: break;
      case NTO_INPUT: if (a < 0 || a >= t->n_inputs) return -3; break;
      case NTO_RANDN: case NTO_RANDU: if (b < 0 || b >= t->n_streams || a < 0) return -4; break;
      case NTO_NEG: case NTO_EXP: case NTO_LOG: case NTO_SQRT: case NTO_ABS:
        if (a < 0 || a >= i) return -5;
        break;
      default:
        if (a < 0 || a >= i || b < 0 || b >= i) return -5;
        break;
    }
  }
  for (int32_t o = 0; o < t->n_outputs; o++) {
    if (t->output_node[o] < 0 || t->output_node[o] >= t->n) return -6;
  }
  for (int32_t j = 0; j < t->n_inputs; j++) {
    if (t->input_node[j] < 0 || t->input_node[j] >= t->n) return -7;
  }
  return 0;
}

/* Planted mistakes: a build with -DNTO_PLANT=n (1..12) gets reverse rule n
 * wrong, in the way listed below; the default build (NTO_PLANT 0) has none.
 * tests/test_oracle_plants.py builds each one and checks that the oracle's
 * pins (central differences, the barrier bump) reject it.
 *   1 ADD: second operand's adjoint subtracted   7 EXP: d * v_a for d * v_i
 *   2 SUB: second operand's adjoint added        8 LOG: d / v_i for d / v_a
 *   3 MUL: d * v_a for d * v_b on a              9 SQRT: d * 0.5 * v_i
 *   4 DIV: first operand's sign flipped         10 ABS: sign of v_a inverted
 *   5 DIV: second operand's sign flipped        11 MAX: the smaller operand
 *   6 NEG: adjoint added, not subtracted        12 MIN: the larger operand */
#ifndef NTO_PLANT
#define NTO_PLANT 0
#endif
#define PLANTED(k) (NTO_PLANT == (k))

/* The adjoint add of ScalarReplay.add, ScalarReplay.java:177-183. */
static inline void adj_add(double *d, int32_t node, double contribution, int f32) {
  if (f32) {
    d[node] = (double)(float)(d[node] + (double)(float)contribution);
  } else {
    d[node] += contribution;
  }
}

/* Per-worker sweep over [from, from+count): ScalarReplay.run, ScalarReplay.java:78-172.
 * When rows != NULL the per-path value and adjoints of every output are written
 * there (row (p - row_base) * n_outputs + o) instead of only being summed. */
static void run_range(const nto_tape *t, const uint8_t *active, const double *in,
                      uint64_t from, uint64_t count, uint64_t seed, int f32, int adjoints,
                      double *value, double *sumsq, double *gradient,
                      double *row_values, double *row_grads, uint64_t row_base, uint64_t pattern) {
  const int32_t n = t->n;
  double *v = (double *)malloc(sizeof(double) * (size_t)n);
  double *d = (double *)malloc(sizeof(double) * (size_t)n);
  stream_state *rng = (stream_state *)malloc(sizeof(stream_state) * (size_t)t->n_streams);
  /* Path indices wrap modulo 2^64, as the reference's long arithmetic does
   * (offset + i); counting by i keeps a range that crosses 2^64 whole. */
  for (uint64_t i = 0; i < count; i++) {
    const uint64_t path = from + i;
    for (int32_t s = 0; s < t->n_streams; s++) {
      stream_init(&rng[s], path, seed, s);
      rng[s].pattern = pattern;
    }
    const uint64_t nkey = path_key(path) ^ 0x5A5A000000000000ull;
    for (int32_t i = 0; i < n; i++) {
      int32_t a = t->arg_a[i], b = t->arg_b[i];
      double x;
      switch (t->op[i]) {
        case NTO_CONST: x = t->constant[i]; break;
        case NTO_INPUT: x = in[a]; break;
        case NTO_RANDN: x = stream_normal(&rng[b]); break;
        case NTO_RANDU: x = stream_uniform(&rng[b]); break;
        case NTO_ADD: x = v[a] + v[b]; break;
        case NTO_SUB: x = v[a] - v[b]; break;
        case NTO_MUL: x = v[a] * v[b]; break;
        case NTO_DIV: x = v[a] / v[b]; break;
        case NTO_NEG: x = -v[a]; break;
        case NTO_EXP: x = nudge_rel(exp(v[a]), nkey ^ ((uint64_t)i << 3), pattern); break;
        case NTO_LOG: x = nudge_rel(log(v[a]), nkey ^ ((uint64_t)i << 3), pattern); break;
        case NTO_SQRT: x = nudge_rel(sqrt(v[a]), nkey ^ ((uint64_t)i << 3), pattern); break;
        case NTO_ABS: x = fabs(v[a]); break;
        /* java.lang.Math.max/min: NaN if either is NaN, and -0.0 < +0.0 */
        case NTO_MAX:
          x = (isnan(v[a]) || isnan(v[b])) ? NAN
              : (v[a] == v[b] ? (signbit(v[a]) ? v[b] : v[a]) : (v[a] > v[b] ? v[a] : v[b]));
          break;
        case NTO_MIN:
          x = (isnan(v[a]) || isnan(v[b])) ? NAN
              : (v[a] == v[b] ? (signbit(v[a]) ? v[a] : v[b]) : (v[a] < v[b] ? v[a] : v[b]));
          break;
        default: x = NAN; break;
      }
      v[i] = f32 ? (double)(float)x : x;
    }
    for (int32_t o = 0; o < t->n_outputs; o++) {
      double y = v[t->output_node[o]];
      value[o] += y;
      sumsq[o] += y * y;
    }
    if (row_values) {
      for (int32_t o = 0; o < t->n_outputs; o++) {
        row_values[(path - row_base) * (uint64_t)t->n_outputs + (uint64_t)o] = v[t->output_node[o]];
      }
    }
    if (!adjoints) {
      continue;
    }
    for (int32_t o = 0; o < t->n_outputs; o++) {
      memset(d, 0, sizeof(double) * (size_t)n);
      d[t->output_node[o]] = 1.0;
      for (int32_t i = n - 1; i >= 0; i--) {
        double adjoint = d[i];
        if (adjoint == 0.0 || !active[i]) {
          continue;
        }
        int32_t a = t->arg_a[i], b = t->arg_b[i];
        switch (t->op[i]) {
          case NTO_ADD: adj_add(d, a, adjoint, f32); adj_add(d, b, PLANTED(1) ? -adjoint : adjoint, f32); break;
          case NTO_SUB: adj_add(d, a, adjoint, f32); adj_add(d, b, PLANTED(2) ? adjoint : -adjoint, f32); break;
          case NTO_MUL:
            adj_add(d, a, adjoint * (PLANTED(3) ? v[a] : v[b]), f32);
            adj_add(d, b, adjoint * v[a], f32);
            break;
          case NTO_DIV:
            adj_add(d, a, PLANTED(4) ? -adjoint / v[b] : adjoint / v[b], f32);
            adj_add(d, b, PLANTED(5) ? adjoint * v[i] / v[b] : -adjoint * v[i] / v[b], f32);
            break;
          case NTO_NEG: adj_add(d, a, PLANTED(6) ? adjoint : -adjoint, f32); break;
          case NTO_EXP: adj_add(d, a, adjoint * (PLANTED(7) ? v[a] : v[i]), f32); break;
          case NTO_LOG: adj_add(d, a, adjoint / (PLANTED(8) ? v[i] : v[a]), f32); break;
          case NTO_SQRT: adj_add(d, a, PLANTED(9) ? adjoint * 0.5 * v[i] : adjoint * 0.5 / v[i], f32); break;
          case NTO_ABS: adj_add(d, a, (v[a] < 0.0) != PLANTED(10) ? -adjoint : adjoint, f32); break;
          case NTO_MAX: adj_add(d, (v[a] >= v[b]) != PLANTED(11) ? a : b, adjoint, f32); break;
          case NTO_MIN: adj_add(d, (v[a] <= v[b]) != PLANTED(12) ? a : b, adjoint, f32); break;
          default: break;
        }
      }
      for (int32_t j = 0; j < t->n_inputs; j++) {
        gradient[(size_t)o * (size_t)t->n_inputs + (size_t)j] += d[t->input_node[j]];
      }
      if (row_grads) {
        for (int32_t j = 0; j < t->n_inputs; j++) {
          row_grads[((path - row_base) * (uint64_t)t->n_outputs + (uint64_t)o) * (uint64_t)t->n_inputs + (uint64_t)j] =
              d[t->input_node[j]];
        }
      }
    }
  }
  free(rng);
  free(d);
  free(v);
}

static int resolve_threads(int threads) {
#ifdef _OPENMP
  return threads > 0 ? threads : omp_get_max_threads();
#else
  (void)threads;
  return 1;
#endif
}

/* HostAadExecutable.runRanges (alignment 1): contiguous ranges, worker t gets
 * units/T (+1 for the first units%T workers); totals are added in worker order. */
static int replay_impl(const nto_tape *t, const double *inputs, uint64_t paths, uint64_t offset,
                       uint64_t seed, int f32, int adjoints, int threads, nto_totals *out,
                       double *row_values, double *row_grads, uint64_t pattern) {
  int rc = validate(t);
  if (rc != 0) return rc;
  uint8_t *active = (uint8_t *)malloc((size_t)t->n);
  nto_mark_active(t, active);
  const int T = resolve_threads(threads);
  const size_t no = (size_t)t->n_outputs, ni = (size_t)t->n_inputs;
  double *val = (double *)calloc((size_t)T * no, sizeof(double));
  double *sq = (double *)calloc((size_t)T * no, sizeof(double));
  double *gr = (double *)calloc((size_t)T * no * (ni ? ni : 1), sizeof(double));
  const uint64_t each = paths / (uint64_t)T, extra = paths % (uint64_t)T;
#ifdef _OPENMP
#pragma omp parallel for num_threads(T) schedule(static, 1)
#endif
  for (int w = 0; w < T; w++) {
    uint64_t from = offset + (uint64_t)w * each + ((uint64_t)w < extra ? (uint64_t)w : extra);
    uint64_t count = each + ((uint64_t)w < extra ? 1u : 0u);
    if (count > 0) {
      run_range(t, active, inputs, from, count, seed, f32, adjoints,
                val + (size_t)w * no, sq + (size_t)w * no, gr + (size_t)w * no * ni,
                row_values, row_grads, offset, pattern);
    }
  }
  if (out) {
    for (size_t o = 0; o < no; o++) {
      out->value[o] = 0.0;
      out->sumsq[o] = 0.0;
      for (size_t j = 0; j < ni; j++) out->gradient[o * ni + j] = 0.0;
    }
    for (int w = 0; w < T; w++) {
      for (size_t o = 0; o < no; o++) {
        out->value[o] += val[(size_t)w * no + o];
        out->sumsq[o] += sq[(size_t)w * no + o];
        for (size_t j = 0; j < ni; j++) out->gradient[o * ni + j] += gr[((size_t)w * no + o) * ni + j];
      }
    }
  }
  free(gr);
  free(sq);
  free(val);
  free(active);
  return 0;
}

int nto_replay(const nto_tape *t, const double *inputs, uint64_t paths, uint64_t offset,
               uint64_t seed, int f32, int adjoints, int threads, nto_totals *out) {
  return replay_impl(t, inputs, paths, offset, seed, f32, adjoints, threads, out, NULL, NULL, 0);
}

int nto_replay_paths(const nto_tape *t, const double *inputs, uint64_t paths, uint64_t offset,
                     uint64_t seed, int f32, int threads, double *values, double *grads) {
  return replay_impl(t, inputs, paths, offset, seed, f32, 1, threads, NULL, values, grads, 0);
}

int nto_replay_paths_perturbed(const nto_tape *t, const double *inputs, uint64_t paths, uint64_t offset,
                               uint64_t seed, int threads, uint64_t pattern, double *values, double *grads) {
  return replay_impl(t, inputs, paths, offset, seed, 0, 1, threads, NULL, values, grads, pattern);
}

/* AadTotals.toResult, AadTotals.java:68-89. */
void nto_to_result(const nto_totals *sums, int32_t n_outputs, int32_t n_inputs, uint64_t paths,
                   double *mean, double *stderr_out, double *mean_gradient) {
  for (int32_t o = 0; o < n_outputs; o++) {
    mean[o] = sums->value[o] / (double)paths;
    if (paths > 1) {
      double variance = (sums->sumsq[o] - (double)paths * mean[o] * mean[o]) / (double)(paths - 1);
      stderr_out[o] = sqrt((variance > 0.0 ? variance : 0.0) / (double)paths);
    } else {
      stderr_out[o] = NAN;
    }
    for (int32_t j = 0; j < n_inputs; j++) {
      mean_gradient[o * n_inputs + j] = sums->gradient[o * n_inputs + j] / (double)paths;
    }
  }
}
