// Host emulation of the HIP builtins a generated replay kernel uses, so the
// lowering's output can be compiled with g++ and run on the CPU by the tests.
// Threads of the emulated grid run one after another; every per-lane scratch
// slot keeps the device indexing (slot * T + tid).
#pragma once
#include <math.h>

#include <cmath>
#include <cstring>
#include <limits>

#define NT_HOST_EMU 1
#define __global__
#define __device__
#define __forceinline__ inline
#define __launch_bounds__(n)
#define __shared__ static
#define __constant__ static
inline void __syncthreads() {}

inline unsigned nt_hi(double x) { unsigned long long u; std::memcpy(&u, &x, 8); return static_cast<unsigned>(u >> 32); }
inline unsigned nt_lo(double x) { unsigned long long u; std::memcpy(&u, &x, 8); return static_cast<unsigned>(u); }
inline double nt_mk(unsigned hi, unsigned lo) {
  unsigned long long u = (static_cast<unsigned long long>(hi) << 32) | lo;
  double x;
  std::memcpy(&x, &u, 8);
  return x;
}
inline unsigned nt_xor3(unsigned a, unsigned b, unsigned c) { return a ^ b ^ c; }
// the device's optimisation barriers; on the host the value itself
template <typename T>
inline T nt_opaque(T x) { return x; }
template <typename T>
inline T nt_opaque_u(T x) { return x; }
inline bool nt_pos_normal(double x) { return std::fpclassify(x) == FP_NORMAL && !std::signbit(x); }
// java.lang.Math.max/min: NaN if either operand is NaN, -0 below +0
template <typename T>
inline T nt_jmax(T a, T b) {
  if (std::isnan(a) || std::isnan(b)) return std::numeric_limits<T>::quiet_NaN();
  if (a == b) return std::signbit(a) ? b : a;
  return a > b ? a : b;
}
template <typename T>
inline T nt_jmin(T a, T b) {
  if (std::isnan(a) || std::isnan(b)) return std::numeric_limits<T>::quiet_NaN();
  if (a == b) return std::signbit(a) ? a : b;
  return a < b ? a : b;
}
inline double nt_max(double a, double b) { return nt_jmax(a, b); }
inline double nt_min(double a, double b) { return nt_jmin(a, b); }
inline float nt_maxf(float a, float b) { return nt_jmax(a, b); }
inline float nt_minf(float a, float b) { return nt_jmin(a, b); }
// the device's fast pass: v_max_f64 / v_min_f64 (-0 below +0), NaN for a NaN
// or infinite operand; with a literal operand, MIN as -MAX(-a, -c)
inline double nt_max_fast(double a, double b) { return nt_jmax(a, b) * std::fma(a + b, 0.0, 1.0); }
inline double nt_min_fast(double a, double b) { return nt_jmin(a, b) * std::fma(a + b, 0.0, 1.0); }
inline double nt_max_lit(double a, double c) { return std::fma(a, 0.0, nt_jmax(a, c)); }
inline double nt_min_lit(double a, double c) { return -nt_max_lit(-a, -c); }
inline bool nt_zero_or_pos_normal(double x) {
  const int c = std::fpclassify(x);
  return c == FP_ZERO || (c == FP_NORMAL && !std::signbit(x));
}
// Stand-ins for the device's seed instructions v_rsq_f64 and v_rcp_f64: the
// correctly rounded value with a relative error of up to 2^-22 (the hardware
// seeds' are near 2^-24), one deterministic pseudo-random error per argument,
// so the host tests see routines that start from an inexact seed as the
// device ones do.
inline double nt_seed_error(double x) {
  unsigned long long u;
  std::memcpy(&u, &x, 8);
  u ^= u >> 33;
  u *= 0xff51afd7ed558ccdull;
  u ^= u >> 33;
  return std::ldexp(static_cast<double>(static_cast<long long>(u >> 11) - (1ll << 52)) / (1ll << 52), -22);
}
inline double nt_rsq(double x) { return (1.0 / std::sqrt(x)) * (1.0 + nt_seed_error(x)); }
inline double nt_rcp(double x) { return (1.0 / x) * (1.0 + nt_seed_error(x)); }

struct nt_emu_dim3 {
  unsigned x = 0, y = 1, z = 1;
};
static nt_emu_dim3 gridDim, blockDim, blockIdx, threadIdx;

// fp32 hardware transcendentals, evaluated in double and rounded once
inline float nt_hw_exp2f(float x) { return static_cast<float>(::exp2(static_cast<double>(x))); }
inline float nt_hw_log2f(float x) { return static_cast<float>(::log2(static_cast<double>(x))); }
inline float nt_hw_sqrtf(float x) { return static_cast<float>(::sqrt(static_cast<double>(x))); }
inline float nt_rcpf(float x) { return 1.0f / x; }
inline float nt_hw_sin2pif(float x) { return static_cast<float>(::sin(2.0 * M_PI * static_cast<double>(x))); }
inline float nt_hw_cos2pif(float x) { return static_cast<float>(::cos(2.0 * M_PI * static_cast<double>(x))); }

inline void sincospif(float x, float* s, float* c) {
  const double a = M_PI * static_cast<double>(x);
  *s = static_cast<float>(::sin(a));
  *c = static_cast<float>(::cos(a));
}

// The emulated threads of a block run one after another: every block is taken
// to hold a flagged lane, and each thread sets, and takes back, its own bit of
// a lane bitmap the driver zeroed (on the device a wave stores and clears a
// whole word; the bits read and the bitmap left behind are the same).
inline int __syncthreads_or(int) { return 1; }
inline unsigned long long atomicAdd(unsigned long long* a, unsigned long long v) {
  const unsigned long long old = *a;
  *a += v;
  return old;
}
inline void nt_flag_lanes(unsigned long long* flags, unsigned long long tid, bool flagged) {
  if (flagged) flags[tid >> 6] |= 1ull << (tid & 63);
}
inline bool nt_take_lane_flag(unsigned long long* flags, unsigned long long tid) {
  const unsigned long long bit = 1ull << (tid & 63);
  const bool set = (flags[tid >> 6] & bit) != 0;
  flags[tid >> 6] &= ~bit;
  return set;
}

// Sequential stand-in for the block reduction: every emulated thread adds its
// accumulators into partials[0 .. NCH).
template <int NCH>
inline void nt_block_store(const double (&acc)[NCH], double* partials, double*) {
  for (int c = 0; c < NCH; ++c) partials[c] += acc[c];
}
