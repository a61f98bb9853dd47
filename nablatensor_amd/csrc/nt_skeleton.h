// Hand-written CDNA4 (gfx950) skeleton of the fused forward+adjoint replay.
//
// The tape lowering (lower.cpp) emits one kernel body per tape and includes
// this header; hipRTC compiles the pair for gfx950. Everything that does not
// depend on the tape lives here:
//   * Philox2x32-10 with the reference's keying, counter and leg selection
//     (nablatensor-engine-cpu/.../cpu/Philox.java:45-78 and the device
//     generator of nablatensor-core/.../engine/CudaAadCodegen.java:480-511):
//     ctr = (lo, hi ^ (k >> 1)), key 0x1BD11BDA bumped by 0x9E3779B9 per round,
//     cosine leg for even k, sine leg for odd k. One block feeds both legs.
//   * Box-Muller in fp64 (the reference formula) and fp32.
//   * Deterministic reductions: wave64 butterfly, then LDS across the waves of
//     a block, one per-block partial per channel (channel-major columns); a
//     second kernel sums each column in block order.
#pragma once

#if !defined(__HIPCC_RTC__) && !defined(NT_HOST_EMU)
#include <hip/hip_runtime.h>  // hipRTC provides these builtins itself
#endif

typedef unsigned int nt_u32;
typedef unsigned long long nt_u64;

#define NT_UINT_SCALE 2.3283064365386963e-10

#if !defined(NT_HOST_EMU)
// a ^ b ^ c in one v_bitop3_b32 (truth table 0x96)
__device__ __forceinline__ nt_u32 nt_xor3(nt_u32 a, nt_u32 b, nt_u32 c) { return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96); }
#endif

// Ten Philox2x32 rounds. The key schedule is a compile-time constant, so a
// round is one 32x32->64 multiply (v_mad_u64_u32) and one three-input xor.
__device__ __forceinline__ void nt_philox(nt_u32 c0, nt_u32 c1, nt_u32& o0, nt_u32& o1) {
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const nt_u32 key = 0x1BD11BDAu + 0x9E3779B9u * static_cast<nt_u32>(i);
    const nt_u64 p = static_cast<nt_u64>(0xD256D193u) * c0;
    c0 = nt_xor3(static_cast<nt_u32>(p >> 32), key, c1);
    c1 = static_cast<nt_u32>(p);
  }
  o0 = c0;
  o1 = c1;
}

#include "nt_math_tables.h"

#if !defined(NT_HOST_EMU)
__device__ __forceinline__ nt_u32 nt_hi(double x) { return static_cast<nt_u32>(__double2hiint(x)); }
__device__ __forceinline__ nt_u32 nt_lo(double x) { return static_cast<nt_u32>(__double2loint(x)); }
__device__ __forceinline__ double nt_mk(nt_u32 hi, nt_u32 lo) {
  return __hiloint2double(static_cast<int>(hi), static_cast<int>(lo));
}
__device__ __forceinline__ double nt_rsq(double x) { return __builtin_amdgcn_rsq(x); }
__device__ __forceinline__ double nt_rcp(double x) { return __builtin_amdgcn_rcp(x); }
// x is -0, +0 or a positive normal number: one v_cmp_class_f64
__device__ __forceinline__ bool nt_zero_or_pos_normal(double x) { return __builtin_amdgcn_class(x, 0x160); }
// x is a positive normal number (finite, not subnormal): one v_cmp_class_f64
__device__ __forceinline__ bool nt_pos_normal(double x) { return __builtin_amdgcn_class(x, 0x100); }
// MAX and MIN nodes as java.lang.Math.max/min evaluate them in the reference's
// scalar engine: NaN when either operand is NaN, and -0 below +0 (IEEE
// 754-2019 maximum/minimum). C's fmax/fmin would return the other operand for
// a NaN and hide a path that the reference prices as NaN. fp64: v_max_f64 and
// a NaN select; fp32: one v_maximum3_f32 / v_minimum3_f32.
__device__ __forceinline__ double nt_max(double a, double b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ double nt_min(double a, double b) { return __builtin_elementwise_minimum(a, b); }
__device__ __forceinline__ float nt_maxf(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float nt_minf(float a, float b) { return __builtin_elementwise_minimum(a, b); }
// The fp64 fast pass: v_max_f64 / v_min_f64 (which order -0 below +0), made
// NaN when an operand is NaN or infinite; such a NaN makes the path's sums
// non-finite and the exception kernel evaluates the path again with nt_max /
// nt_min, which also give Math.max/min's value for an infinite operand. Two
// variable operands: times fma(a + b, 0, 1), exactly 1 for finite ones. One
// literal operand c: plus a * 0, an exact +-0 for a finite a that leaves the
// maximum as it is (-0 + -0 stays -0, +0 + -0 is +0 only where the maximum
// is +0); MIN as -MAX(-a, -c), the negations free source modifiers. No
// register beyond the operands, where nt_max's NaN select costs the reverse
// sweep of the Asian its third wave.
__device__ __forceinline__ double nt_max_fast(double a, double b) { return fmax(a, b) * fma(a + b, 0.0, 1.0); }
__device__ __forceinline__ double nt_min_fast(double a, double b) { return fmin(a, b) * fma(a + b, 0.0, 1.0); }
__device__ __forceinline__ double nt_max_lit(double a, double c) { return fma(a, 0.0, fmax(a, c)); }
__device__ __forceinline__ double nt_min_lit(double a, double c) { return -nt_max_lit(-a, -c); }
// fp32 hardware transcendentals (quarter-rate VALU): exp2, log2, sqrt, and
// sin/cos of 2 pi x (the instructions take their argument in revolutions).
__device__ __forceinline__ float nt_hw_exp2f(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float nt_hw_log2f(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float nt_hw_sqrtf(float x) { return __builtin_amdgcn_sqrtf(x); }
__device__ __forceinline__ float nt_hw_sin2pif(float x) { return __builtin_amdgcn_sinf(x); }
__device__ __forceinline__ float nt_hw_cos2pif(float x) { return __builtin_amdgcn_cosf(x); }
// fp32 reciprocal, one v_rcp_f32 (1 ulp): fp32 replay divides as a * (1/b),
// within 2 ulp of the rounded quotient, where a correctly rounded division
// takes ten instructions.
__device__ __forceinline__ float nt_rcpf(float x) { return __builtin_amdgcn_rcpf(x); }
// Optimisation barriers: x comes back unchanged, but the compiler cannot
// see that it equals the argument, and keeps the barriers in program order.
// nt_opaque holds a per-lane value in a VGPR; nt_opaque_u a wave-uniform one
// in SGPRs, so that it stays uniform (a switch on it is a scalar branch). A
// checkpointed straight line starts each segment from such copies, so its
// work is neither hoisted out of the segment loops nor merged with the
// forward pass.
template <typename T>
__device__ __forceinline__ T nt_opaque(T x) {
  asm volatile("" : "+v"(x));
  return x;
}
template <typename T>
__device__ __forceinline__ T nt_opaque_u(T x) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "a 32- or 64-bit value");
  // readfirstlane makes the value provably uniform (a value the compiler
  // holds in a VGPR, such as a converted input, cannot be copied to SGPRs
  // otherwise); on a value already in SGPRs it costs nothing
  if constexpr (sizeof(T) == 4) {
    int v = __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x));
    asm volatile("" : "+s"(v));
    return __builtin_bit_cast(T, v);
  } else {
    const nt_u64 u = __builtin_bit_cast(nt_u64, x);
    int lo = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<nt_u32>(u)));
    int hi = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<nt_u32>(u >> 32)));
    asm volatile("" : "+s"(lo), "+s"(hi));
    return __builtin_bit_cast(T, (static_cast<nt_u64>(static_cast<nt_u32>(hi)) << 32) | static_cast<nt_u32>(lo));
  }
}
#endif

// Strong-zero numbers for the tangents of the re-evaluation pass: a product
// with an exact zero is zero whatever the other factor is, infinite or NaN
// included. The reverse sweep of the reference skips a node whose adjoint is
// zero (ScalarReplay.java:134-136), so nothing flows back through it however
// large its local derivative; in tangent mode the same happens when a zero
// factor meets an infinite tangent, as in 1 / (1 + e) once e = exp(x) has
// overflowed: the quotient's factor for e is 0 / inf = 0 and e's tangent is
// infinite. Sums and differences stay IEEE. Only the re-evaluation pass of a
// path uses them; the fast pass sends any path whose result is not finite
// there.
#define NT_STRONG_ZERO(T, S, FMA)                                                                              \
  struct S {                                                                                                   \
    T v;                                                                                                       \
    __device__ __forceinline__ constexpr S(T x) : v(x) {}                                                      \
    template <class U>                                                                                         \
    __device__ __forceinline__ explicit operator U() const { return static_cast<U>(v); }                       \
  };                                                                                                           \
  __device__ __forceinline__ S operator*(S a, S b) { return (a.v == T(0) || b.v == T(0)) ? S(T(0)) : S(a.v * b.v); } \
  __device__ __forceinline__ S operator+(S a, S b) { return S(a.v + b.v); }                                    \
  __device__ __forceinline__ S operator-(S a, S b) { return S(a.v - b.v); }                                    \
  __device__ __forceinline__ S operator-(S a) { return S(-a.v); }                                              \
  __device__ __forceinline__ S FMA(S a, S b, S c) {                                                            \
    return (a.v == T(0) || b.v == T(0)) ? c : S(FMA(a.v, b.v, c.v));                                          \
  }
NT_STRONG_ZERO(double, nt_sz, fma)
NT_STRONG_ZERO(float, nt_szf, fmaf)
#undef NT_STRONG_ZERO

// fp32 exp as 2^(x log2 e) on the hardware exp2: the rounding of the product
// adds |x| * 2^-24 relative error, well inside fp32 replay's 1e-5 reconcile
// bar for Monte-Carlo exponents (|x| of order 1).
__device__ __forceinline__ float nt_expf(float x) { return nt_hw_exp2f(x * 1.44269504088896341f); }

#ifndef NT_DEVICE_LIBM
// The sin/cos, exp and log tables live in LDS; every block copies them once
// at kernel start.
__constant__ NtTables nt_tables_c = NT_TABLES_INIT;
__shared__ NtTables nt_tables;

__device__ __forceinline__ void nt_tables_load() {
  const double* src = reinterpret_cast<const double*>(&nt_tables_c);
  double* dst = reinterpret_cast<double*>(&nt_tables);
  constexpr unsigned n = sizeof(NtTables) / sizeof(double);
  for (unsigned i = threadIdx.x; i < n; i += blockDim.x) dst[i] = src[i];
  __syncthreads();
}

// exp(x) by Tang's table-driven method: x = (256 m + j) ln2/256 + r with
// |r| <= ln2/512 (ln2/256 split in a 32-bit head and a tail, so the reduction
// keeps r to one rounding), exp(x) = 2^m (T_j + T_j p(r)) with T_j =
// 2^(j/256) as head + tail and p(r) = exp(r) - 1 through r^4 (truncation
// r^5/120 < 4e-17 relative). Below 1 ulp.
// k = 256 m + j comes out of the low word of x 256/ln2 + 1.5 * 2^52 (rounded
// to an integer by that addition), so no float-to-int conversion is needed.
// The result is exact only for |x| <= 708 (results in the normal range);
// outside it (and for infinities and NaN) it is garbage but harmless (the
// table index stays in range) and `bad` is set, so the caller can evaluate
// the path again with device libm.
__device__ __forceinline__ double nt_exp_core(double x) {
  const double t = fma(x, NT_EXP_INV_L, 0x1.8p52);
  const double kd = t - 0x1.8p52;
  const int k = static_cast<int>(nt_lo(t));
  double r = fma(-kd, NT_EXP_L_HI, x);
  r = fma(-kd, NT_EXP_L_LO, r);
  const int j = k & 255;
  const int m = k >> 8;
  double q = fma(r, NT_EXP_C4, NT_EXP_C3);
  q = fma(r, q, NT_EXP_C2);
  const double p = fma(r * r, q, r);
  const double th = nt_tables.ex.t[2 * j];
  const double tl = nt_tables.ex.t[2 * j + 1];
  return ldexp(th + fma(th, p, tl), m);
}

// The fast path with its range check; a caller that has bounded |x| <= 708
// for the whole path beforehand calls nt_exp_core directly.
__device__ __forceinline__ double nt_exp_fast(double x, bool& bad) {
  bad |= !(fabs(x) <= 708.0);
  return nt_exp_core(x);
}

// exp for any argument: the fast path, device libm where it does not apply.
__device__ __forceinline__ double nt_exp(double x) {
  bool bad = false;
  const double y = nt_exp_fast(x, bad);
  return bad ? exp(x) : y;
}

// -2 ln(u) for a positive normal u, by Tang's table-driven method: u = 2^e x
// with x in [sqrt(1/2), sqrt(2)), F = x rounded to 8 fractional bits of its
// binade (rounding the high word at bit 12 moves F = 2 - 2^-8 up to the next
// binade exactly), ln u = e ln2 + ln F + ln(1 + r), r = (x - F) / F,
// |r| <= 2^-9. x - F is exact and F = 1 near u = 1, so ln u keeps full
// relative accuracy there. Tables and constants carry the factor -2 (exact).
// The exponent comes from u's high word alone, so any biased exponent works
// (the high word may carry into bit 31 for u near the largest double; the
// arithmetic is unsigned).
__device__ __forceinline__ double nt_neg2log(double u) {
  nt_u32 hx = nt_hi(u) + (0x3FF00000u - 0x3FE6A09Eu);
  // e = (hx >> 20) - 1023 as a double: the biased exponent in the low word of
  // 2^52 + (hx >> 20), less 2^52 + 1023 (exact), instead of a conversion
  const double ed = nt_mk(0x43300000u, hx >> 20) - 0x1.00000000003ffp52;
  hx = (hx & 0x000FFFFFu) + 0x3FE6A09Eu;
  const double x = nt_mk(hx, nt_lo(u));
  const nt_u32 fhi = (hx + 0x800u) & 0xFFFFF000u;
  const nt_u32 idx = (fhi - 0x3FE6A000u) >> 12;
  const double r = (x - nt_mk(fhi, 0u)) * nt_tables.lg.inv[idx];  // r' = -2 (x - F) / F
  double q = fma(r, NT_LOGQ_4, NT_LOGQ_3);
  q = fma(r, q, NT_LOGQ_2);
  q = fma(r, q, NT_LOGQ_1);
  q = fma(r, q, NT_LOGQ_0);
  const double p = fma(r * r, q, r);  // -2 ln(1 + (x - F) / F)
  const double hi = fma(ed, NT_M2LN2_HI, nt_tables.lg.hi[idx]);  // exact by the table's layout
  const double lo = fma(ed, NT_M2LN2_LO, nt_tables.lg.lo[idx]) + p;
  return hi + lo;
}

// Box-Muller's -2 ln(u) for u = (c + 0.5) * 2^-32.
__device__ __forceinline__ double nt_neg2log_u32(nt_u32 c) {
  return nt_neg2log(fma(static_cast<double>(c), 0x1p-32, 0x1p-33));
}

// ln(a) of a LOG node: -1/2 times nt_neg2log (an exact scaling). An argument
// that is not a positive normal number (zero, subnormal, negative, infinite,
// NaN) sets `bad`, and the path is evaluated again with device libm.
__device__ __forceinline__ double nt_log_fast(double a, bool& bad) {
  bad |= !nt_pos_normal(a);
  return -0.5 * nt_neg2log(a);
}

// sqrt(a) for a positive normal finite a: reciprocal square root seed and one
// coupled Newton step on (sqrt, 1/(2 sqrt)), then a residual correction.
__device__ __forceinline__ double nt_sqrt_pos(double a) {
  const double y = nt_rsq(a);
  double g = a * y;
  double h = 0.5 * y;
  const double r = fma(-g, h, 0.5);
  g = fma(g, r, g);
  h = fma(h, r, h);
  const double d = fma(-g, g, a);
  return fma(d, h, g);
}

// 1/b for a DIV node whose numerator is the constant 1, in fp64 tangent
// kernels (the value is also the node's tangent factor): the v_rcp_f64 seed
// and two Newton steps give it within an ulp, where a correctly rounded
// division takes eleven instructions. For |b| outside [2^-1022, 2^1022]
// (zero, subnormal, huge, infinite, NaN) `bad` is set and the caller
// evaluates the path again with device libm.
__device__ __forceinline__ double nt_recip(double b, bool& bad) {
  bad |= !(fabs(b) >= 0x1p-1022 && fabs(b) <= 0x1p1022);
  double y = nt_rcp(b);
  double e = fma(-b, y, 1.0);
  y = fma(y, e, y);
  e = fma(-b, y, 1.0);
  return fma(y, e, y);
}

// sin and cos of theta = fl(6.283185307179586 * u) for u = (c + 0.5) * 2^-32.
// The reference rounds its angle once, and so does this (theta is that
// rounded product): the per-path results of the Heston tape move by a few
// 1e-12 when the normals lose that rounding (4.7e-15 at most). The circle is
// cut in 512 sectors: c = j 2^23 + d with d the sign-extended low 23 bits, so
// u = j/512 + f exactly, f = (d + 0.5) 2^-32, |f| <= 2^-10 turns. With
// (S, C) = (sin, cos)(2 pi j/512) from the table, sin(2 pi u) = S cos(2 pi f)
// + C sin(2 pi f) and cos(2 pi u) = C cos(2 pi f) - S sin(2 pi f), the
// small-angle parts being polynomials in f. The rounding of theta, eps =
// theta - 2 pi u, is known exactly (two FMAs) and enters as sin(2 pi f + eps)
// = sin(2 pi f) + eps to first order (the second-order terms are below
// 1e-17).
struct __attribute__((aligned(16))) NtPair {
  double a, b;
};
__device__ __forceinline__ void nt_sincos_2pi_u32(nt_u32 c, double& s, double& co) {
  const int d = static_cast<int>(c << 9) >> 9;
  // c - d = j 2^23, so its shift by 19 is the byte offset 16 j of the
  // sector's (sin, cos) pair: one 16-byte load, no masking
  const nt_u32 off = (c - static_cast<nt_u32>(d)) >> 19;
  const double f = fma(static_cast<double>(d), 0x1p-32, 0x1p-33);
  const double t = f * f;
  double ps = fma(t, NT_SC_S5, NT_SC_S3);
  ps = fma(t, ps, NT_SC_S1);
  const double cq = fma(t, NT_SC_C4, NT_SC_C2);
  const double cm = t * cq;  // cos(2 pi f) - 1
  const double u = fma(static_cast<double>(c), 0x1p-32, 0x1p-33);
  const double theta = NT_TWO_PI_D * u;
  const double eps = fma(NT_TWO_PI_D_ERR, u, -fma(NT_TWO_PI_D, u, -theta));
  const double sn = fma(f, ps, eps);  // sin(2 pi f) + eps
  const NtPair sc = *reinterpret_cast<const NtPair*>(reinterpret_cast<const char*>(nt_tables.sc.t) + off);
  const double S = sc.a;
  const double C = sc.b;
  s = S + fma(C, sn, S * cm);
  co = C + fma(C, cm, -(S * sn));
}

// sqrt(a) and the tangent factor 1/(2 sqrt(a)) of a SQRT node, for a = +-0 or
// a positive normal, where a correctly rounded sqrt and a division take two
// dozen instructions. nt_sqrt_pos's coupled Newton step and residual
// correction give the root s; the factor after that step is low by 1.5 e^2
// (e the seed's relative error, about 2^-24 for v_rsq_f64), the same sign
// every time, so a Newton step for h = 1/(2 s), h + 2 h (1/2 - s h), brings it
// to full precision (its error squares): in a carried tangent (a variance
// process) a one-sided error would compound over the steps. The seed is taken at max(a, 2^-1022), so a = +-0 gives sqrt = a and
// a large finite factor (the derivative is infinite there; a zero tangent
// stays zero, as with the capped factor of the libm path). Any other
// argument (negative, subnormal, infinite, NaN) sets `bad`, and the caller
// evaluates the path again with device libm.
__device__ __forceinline__ double nt_sqrt_q(double a, double& q, bool& bad) {
  bad |= !nt_zero_or_pos_normal(a);
  const double y = nt_rsq(fmax(a, 0x1p-1022));
  double g = a * y;
  double h = 0.5 * y;
  const double r = fma(-g, h, 0.5);
  g = fma(g, r, g);
  h = fma(h, r, h);
  const double s = fma(fma(-g, g, a), h, g);
  q = fma(h + h, fma(-s, h, 0.5), h);
  return s;
}
#else
__device__ __forceinline__ void nt_tables_load() {}
__device__ __forceinline__ double nt_exp(double x) { return exp(x); }
#endif

// The k-th uniform of a stream whose counter words are (lo, hi): the Philox
// block at counter (lo, hi ^ (k | 2^30)) (the tag keeps uniforms and normals
// on disjoint counters), u = (c0 + 0.5) 2^-32 (Philox.java:81-94). fp32 rounds
// the double uniform once, as the fp32 oracle does.
__device__ __forceinline__ double nt_uniform(nt_u32 lo, nt_u32 hi, nt_u32 k) {
  nt_u32 c0, c1;
  nt_philox(lo, hi ^ (k | 0x40000000u), c0, c1);
  return fma(static_cast<double>(c0), 0x1p-32, 0x1p-33);
}
__device__ __forceinline__ float nt_uniformf(nt_u32 lo, nt_u32 hi, nt_u32 k) {
  return static_cast<float>(nt_uniform(lo, hi, k));
}

// Both legs of the Box-Muller pair for Philox counter `ctr` of a path whose
// counter words are (lo, hi): u = (c + 0.5) * 2^-32, r = sqrt(-2 log u1),
// z = r cos(2 pi u2) for even draws and r sin(2 pi u2) for odd ones. With
// NT_DEVICE_LIBM the reference expression is evaluated with device libm.
__device__ __forceinline__ void nt_normal_pair(nt_u32 lo, nt_u32 hi, nt_u32 ctr, double& zc, double& zs) {
  nt_u32 c0, c1;
  nt_philox(lo, hi ^ ctr, c0, c1);
#ifdef NT_DEVICE_LIBM
  const double u1 = (static_cast<double>(c0) + 0.5) * NT_UINT_SCALE;
  const double u2 = (static_cast<double>(c1) + 0.5) * NT_UINT_SCALE;
  const double r = sqrt(-2.0 * log(u1));
  const double theta = 6.283185307179586 * u2;
  double s, c;
  sincos(theta, &s, &c);
#elif defined(NT_LIBM_SINCOS)
  const double r = nt_sqrt_pos(nt_neg2log_u32(c0));
  const double u2 = (static_cast<double>(c1) + 0.5) * NT_UINT_SCALE;
  double s, c;
  sincos(6.283185307179586 * u2, &s, &c);
#else
  const double r = nt_sqrt_pos(nt_neg2log_u32(c0));
  double s, c;
  nt_sincos_2pi_u32(c1, s, c);
#endif
  zc = r * c;
  zs = r * s;
}

// fp32 pair: same counters and the reference's fp32 u; the transcendentals
// are the hardware ones: ln u1 = ln2 * log2(u1), and sin/cos of 2 pi u2 read
// u2 directly as revolutions (no multiplication by 2 pi rounds the angle).
__device__ __forceinline__ void nt_normal_pair(nt_u32 lo, nt_u32 hi, nt_u32 ctr, float& zc, float& zs) {
  nt_u32 c0, c1;
  nt_philox(lo, hi ^ ctr, c0, c1);
  // (float(c) + 0.5f) * 2^-32 in one rounding: the same float for every c
  // (exact below 2^24; above, both round the same tie or sub-half-ulp term).
  const float u1 = fmaf(static_cast<float>(c0), 0x1p-32f, 0x1p-33f);
  const float u2 = fmaf(static_cast<float>(c1), 0x1p-32f, 0x1p-33f);
  const float r = nt_hw_sqrtf(-1.38629436111989061f * nt_hw_log2f(u1));  // -2 ln 2 * log2(u1)
  zc = r * nt_hw_cos2pif(u2);
  zs = r * nt_hw_sin2pif(u2);
}

#ifndef NT_HOST_EMU  // the lowering's CPU tests provide their own reductions

// Sum of a double over the 64 lanes of a wave, identical in every lane. The
// butterfly order is fixed, so the result is reproducible run to run.
__device__ __forceinline__ double nt_wave_sum(double x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    x += __shfl_xor(x, m, 64);
  }
  return x;
}

// Bitmap of the lanes whose paths a replay kernel leaves to the exception
// kernel: bit tid % 64 of word tid / 64, one word per wave of the grid (blocks
// are whole waves). A lane flags all of its paths or none, so one bit per lane
// says it all, and the bitmap's size is the grid's, not the dispatch's. Only a
// wave with a flagged lane stores its word (the ballot, from its lowest active
// lane: no atomics); the words start at zero and the exception kernel, which
// reads them on the same grid, sets every nonzero word back to zero
// (nt_take_lane_flag), so the bitmap is zero again between dispatches.
__device__ __forceinline__ void nt_flag_lanes(nt_u64* __restrict__ flags, nt_u64 tid, bool flagged) {
  const nt_u64 mask = __ballot(flagged);
  const nt_u64 active = __ballot(1);
  if (mask != 0 && __lane_id() == static_cast<unsigned>(__ffsll(static_cast<long long>(active)) - 1)) {
    flags[tid >> 6] = mask;
  }
}

// The exception kernel's read of this lane's bit. The wave's lowest active
// lane then clears a nonzero word; the store depends on the loaded word, so
// it follows the load every lane of the wave made with the same instruction.
__device__ __forceinline__ bool nt_take_lane_flag(nt_u64* __restrict__ flags, nt_u64 tid) {
  const nt_u64 w = flags[tid >> 6];
  const nt_u64 active = __ballot(1);
  if (w != 0 && __lane_id() == static_cast<unsigned>(__ffsll(static_cast<long long>(active)) - 1)) {
    flags[tid >> 6] = 0;
  }
  return ((w >> (tid & 63)) & 1) != 0;
}

// Partials are channel-major, one column per channel, so the finishing pass
// reads a channel with contiguous loads (64 entries per wave load); from a
// row-major [block][channel] layout every wave load touched 64 cache lines,
// and the pass, one block, was bound by its CU's address unit (40 us for 35
// channels of 2,048 blocks). Within a column the entries are grouped by
// b mod 8, the XCD the dispatcher deals block b to: block b sits at
// nt_partial_slot(b, grid) = (b mod 8) G8 + b / 8, G8 = ceil(grid / 8), so
// the entries of a 32-byte write granule come from one XCD's L2 (in block
// order, four XCDs would each write back a part of every granule). A column
// holds nt_partial_column(grid) = 16 G8 entries: the replay kernel's 8 G8
// slots, then the exception kernel's (it runs on the same grid, with
// `partials` advanced by 8 G8). The host allocates nch columns of that length.
__device__ __forceinline__ nt_u32 nt_group8(nt_u32 grid) { return (grid + 7u) >> 3; }
__device__ __forceinline__ nt_u64 nt_partial_column(nt_u32 grid) { return 16ull * nt_group8(grid); }
__device__ __forceinline__ nt_u32 nt_partial_slot(nt_u32 b, nt_u32 grid) { return (b & 7u) * nt_group8(grid) + (b >> 3); }

// Reduce NCH per-lane accumulators over the block and write the block's entry
// of each channel's column. `lds` holds NCH * (blockDim.x / 64) doubles.
template <int NCH>
__device__ __forceinline__ void nt_block_store(const double (&acc)[NCH], double* __restrict__ partials,
                                               double* lds) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const double w = nt_wave_sum(acc[c]);
    if (lane == 0) lds[c * waves + wave] = w;
  }
  __syncthreads();
  for (int c = threadIdx.x; c < NCH; c += blockDim.x) {
    double s = 0.0;
    for (int w = 0; w < waves; ++w) s += lds[c * waves + w];
    partials[static_cast<nt_u64>(c) * nt_partial_column(gridDim.x) + nt_partial_slot(blockIdx.x, gridDim.x)] = s;
  }
}

// Second pass: out[c] = sum over blocks of channel c's entries, launched as
// one block of 64 * min(nch, 16) threads; `blocks` is the dispatch's grid.
// Wave w takes channels w, w + waves, ...; its lanes walk the column's slots
// in a fixed order (region, then batches of 64 kBatch slots per class of
// b mod 8, the eight classes side by side, each lane adding its slots in
// order) and the wave adds its 64 lane sums by the fixed butterfly, with no
// block barrier. All 8 kBatch loads of a batch are issued before its first
// add, so a lane waits about one memory round trip per batch. The order
// depends only on the grid, so a channel's result is bitwise the same whatever
// nch is (a market's sums do not change with the markets priced beside it)
// and run to run. `out` is host memory the caller reads after the stream has
// drained.
// The exception kernel's entries (its region of each column; `slow_blocks`
// is the grid when there is such a kernel, else 0) are added only when
// `count`, the number of lanes that left paths to it, is nonzero (an
// exception kernel that found it zero wrote nothing); the pass then sets
// `count` back to zero for the next dispatch.
// With `deferred` set (host memory), the exception kernel has not run yet:
// the pass writes whether it is needed (count nonzero) there and, if it is,
// returns at once, changing nothing; the caller then runs the exception
// kernel and this pass again without `deferred`. The sums are the same bits
// either way.
extern "C" __global__ __launch_bounds__(1024) void nt_finish(const double* __restrict__ partials, nt_u32 blocks,
                                                           nt_u32 slow_blocks, nt_u32 nch, double* __restrict__ out,
                                                           nt_u64* __restrict__ count, nt_u32* __restrict__ deferred) {
  const nt_u32 lane = threadIdx.x & 63;
  const nt_u32 waves = blockDim.x >> 6;
  if (deferred) {
    const bool flagged = count[0] != 0;  // the same value in every thread
    if (threadIdx.x == 0) deferred[0] = flagged ? 1u : 0u;
    if (flagged) return;
  }
  const nt_u32 g8 = nt_group8(blocks);
  const nt_u64 column = nt_partial_column(blocks);
  const nt_u32 regions = (slow_blocks != 0 && count && count[0] != 0) ? 2u : 1u;
  // slots of class x hold the blocks x, x + 8, ...: n[x] of them
  nt_u32 n[8];
#pragma unroll
  for (nt_u32 x = 0; x < 8; ++x) n[x] = blocks > x ? (blocks - x + 7u) >> 3 : 0u;
  constexpr nt_u32 kBatch = 4;
  for (nt_u32 c = threadIdx.x >> 6; c < nch; c += waves) {
    double s = 0.0;
    for (nt_u32 region = 0; region < regions; ++region) {
      const double* col = partials + c * column + static_cast<nt_u64>(region) * 8u * g8;
      for (nt_u32 jb = 0; jb < g8; jb += 64 * kBatch) {
        double v[8][kBatch];
#pragma unroll
        for (nt_u32 x = 0; x < 8; ++x) {
#pragma unroll
          for (nt_u32 k = 0; k < kBatch; ++k) {
            const nt_u32 j = jb + lane + 64 * k;
            v[x][k] = j < n[x] ? col[static_cast<nt_u64>(x) * g8 + j] : 0.0;
          }
        }
#pragma unroll
        for (nt_u32 x = 0; x < 8; ++x) {
#pragma unroll
          for (nt_u32 k = 0; k < kBatch; ++k) {
            if (jb + lane + 64 * k < n[x]) s += v[x][k];
          }
        }
      }
    }
    s = nt_wave_sum(s);
    if (lane == 0) out[c] = s;
  }
  if (count) {
    __syncthreads();  // every thread has read count
    if (threadIdx.x == 0) count[threadIdx.x] = 0;
  }
}

#endif  // NT_HOST_EMU
