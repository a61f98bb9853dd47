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
//     a block, one row of per-block partials; a second kernel sums the rows in
//     block order.
#pragma once

#if !defined(__HIPCC_RTC__) && !defined(NT_HOST_EMU)
#include <hip/hip_runtime.h>  // hipRTC provides these builtins itself
#endif

typedef unsigned int nt_u32;
typedef unsigned long long nt_u64;

#define NT_UINT_SCALE 2.3283064365386963e-10

// Ten Philox2x32 rounds. The key schedule is a compile-time constant, so a
// round is one 32x32->64 multiply and one three-input xor.
__device__ __forceinline__ void nt_philox(nt_u32 c0, nt_u32 c1, nt_u32& o0, nt_u32& o1) {
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const nt_u32 key = 0x1BD11BDAu + 0x9E3779B9u * static_cast<nt_u32>(i);
    const nt_u64 p = static_cast<nt_u64>(0xD256D193u) * c0;
    c0 = static_cast<nt_u32>(p >> 32) ^ key ^ c1;
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
#endif

#ifndef NT_DEVICE_LIBM
// The log table lives in LDS; every block copies it once at kernel start.
__constant__ NtLogTable nt_log_table_c = NT_LOG_TABLE_INIT;
__shared__ NtLogTable nt_log_table;

__device__ __forceinline__ void nt_tables_load() {
  const double* src = &nt_log_table_c.inv[0];
  double* dst = &nt_log_table.inv[0];
  for (unsigned i = threadIdx.x; i < 3u * 129u; i += blockDim.x) dst[i] = src[i];
  __syncthreads();
}

// -2 ln(u) for u = (c + 0.5) * 2^-32, by Tang's table-driven method: u = 2^e x
// with x in [sqrt(1/2), sqrt(2)), F = x rounded to 7 fractional bits,
// ln u = e ln2 + ln F + ln(1 + r), r = (x - F) / F, |r| <= 2^-8. x - F is
// exact and F = 1 near u = 1, so ln u keeps full relative accuracy there.
__device__ __forceinline__ double nt_neg2log_u32(nt_u32 c) {
  const double u = fma(static_cast<double>(c), 0x1p-32, 0x1p-33);
  nt_u32 hx = nt_hi(u) + (0x3FF00000u - 0x3FE6A09Eu);
  const int e = static_cast<int>(hx >> 20) - 0x3FF;
  hx = (hx & 0x000FFFFFu) + 0x3FE6A09Eu;
  const double x = nt_mk(hx, nt_lo(u));
  const nt_u32 j = (((hx >> 12) & 0xFFu) + 1u) >> 1;
  const nt_u32 fhi = (hx & 0xFFF00000u) + (j << 13);
  const nt_u32 idx = (fhi - 0x3FE6A000u) >> 13;
  const double r = (x - nt_mk(fhi, 0u)) * nt_log_table.inv[idx];
  double q = fma(r, 1.0 / 7.0, -1.0 / 6.0);
  q = fma(r, q, 0.2);
  q = fma(r, q, -0.25);
  q = fma(r, q, 1.0 / 3.0);
  q = fma(r, q, -0.5);
  const double p = fma(r * r, q, r);
  const double ed = static_cast<double>(e);
  const double hi = fma(ed, NT_LN2_HI, nt_log_table.hi[idx]);  // exact by the table's layout
  const double lo = fma(ed, NT_LN2_LO, nt_log_table.lo[idx]) + p;
  return -2.0 * (hi + lo);
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

// sin and cos of theta = fl(6.283185307179586 * u) for u = (c + 0.5) * 2^-32:
// the reference rounds its angle once, and so does this (theta is that rounded
// product). The quarter turn q and the remainder f = u - q/4 in [-1/8, 1/8]
// come exactly from the integer c and the polynomials are in f; the rounding
// of theta, eps = theta - 2 pi u, is known exactly (one FMA) and applied as
// sin(2 pi u + eps) = S + eps C, cos = C - eps S.
__device__ __forceinline__ void nt_sincos_2pi_u32(nt_u32 c, double& s, double& co) {
  const nt_u32 q = (c >> 30) + ((c >> 29) & 1u);
  const int d = static_cast<int>(c - (q << 30));
  const double f = fma(static_cast<double>(d), 0x1p-32, 0x1p-33);
  const double t = f * f;
  double ps = fma(t, NT_SIN2PI_7, NT_SIN2PI_6);
  ps = fma(t, ps, NT_SIN2PI_5);
  ps = fma(t, ps, NT_SIN2PI_4);
  ps = fma(t, ps, NT_SIN2PI_3);
  ps = fma(t, ps, NT_SIN2PI_2);
  ps = fma(t, ps, NT_SIN2PI_1);
  ps = fma(t, ps, NT_SIN2PI_0);
  const double sn = f * ps;
  double pc = fma(t, NT_COS2PI_8, NT_COS2PI_7);
  pc = fma(t, pc, NT_COS2PI_6);
  pc = fma(t, pc, NT_COS2PI_5);
  pc = fma(t, pc, NT_COS2PI_4);
  pc = fma(t, pc, NT_COS2PI_3);
  pc = fma(t, pc, NT_COS2PI_2);
  pc = fma(t, pc, NT_COS2PI_1);
  const double cs = fma(t, pc, NT_COS2PI_0);
  const nt_u32 qq = q & 3u;
  const double sv = (qq & 1u) ? cs : sn;
  const double cv = (qq & 1u) ? sn : cs;
  const double s2 = (qq & 2u) ? -sv : sv;
  const double c2 = ((qq + 1u) & 2u) ? -cv : cv;
  const double u = fma(static_cast<double>(c), 0x1p-32, 0x1p-33);
  const double theta = NT_TWO_PI_D * u;
  const double eps = fma(NT_TWO_PI_D_ERR, u, -fma(NT_TWO_PI_D, u, -theta));
  s = fma(eps, c2, s2);
  co = fma(-eps, s2, c2);
}
#else
__device__ __forceinline__ void nt_tables_load() {}
#endif

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

// fp32 pair: same counters, single-precision transcendentals.
__device__ __forceinline__ void nt_normal_pair(nt_u32 lo, nt_u32 hi, nt_u32 ctr, float& zc, float& zs) {
  nt_u32 c0, c1;
  nt_philox(lo, hi ^ ctr, c0, c1);
  const float u1 = (static_cast<float>(c0) + 0.5f) * 2.3283064365386963e-10f;
  const float u2 = (static_cast<float>(c1) + 0.5f) * 2.3283064365386963e-10f;
  const float r = sqrtf(-2.0f * logf(u1));
  float s, c;
  sincospif(2.0f * u2, &s, &c);
  zc = r * c;
  zs = r * s;
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

// Reduce NCH per-lane accumulators over the block and write one row of
// partials[blockIdx.x * NCH + c]. `lds` holds NCH * (blockDim.x / 64) doubles.
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
  if (threadIdx.x < NCH) {
    const int c = threadIdx.x;
    double s = 0.0;
    for (int w = 0; w < waves; ++w) s += lds[c * waves + w];
    partials[static_cast<nt_u64>(blockIdx.x) * NCH + c] = s;
  }
}

// Second pass: out[c] = sum over blocks of partials[b * nch + c], one block of
// 256 threads, fixed assignment and fixed tree order (deterministic).
extern "C" __global__ __launch_bounds__(256) void nt_finish(const double* __restrict__ partials, nt_u32 blocks,
                                                          nt_u32 nch, double* __restrict__ out) {
  __shared__ double red[256];
  for (nt_u32 c = 0; c < nch; ++c) {
    double s = 0.0;
    for (nt_u32 b = threadIdx.x; b < blocks; b += 256) s += partials[static_cast<nt_u64>(b) * nch + c];
    red[threadIdx.x] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
      if (static_cast<int>(threadIdx.x) < w) red[threadIdx.x] += red[threadIdx.x + w];
      __syncthreads();
    }
    if (threadIdx.x == 0) out[c] = red[0];
    __syncthreads();
  }
}

#endif  // NT_HOST_EMU
