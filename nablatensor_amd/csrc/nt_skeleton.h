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

// Both legs of the Box-Muller pair for Philox counter `ctr` of a path whose
// counter words are (lo, hi). fp64 follows the reference expression order:
// u = (c + 0.5) * 2^-32 (exact), r = sqrt(-2 log u1), theta = 2pi * u2.
__device__ __forceinline__ void nt_normal_pair(nt_u32 lo, nt_u32 hi, nt_u32 ctr, double& zc, double& zs) {
  nt_u32 c0, c1;
  nt_philox(lo, hi ^ ctr, c0, c1);
  const double u1 = (static_cast<double>(c0) + 0.5) * NT_UINT_SCALE;
  const double u2 = (static_cast<double>(c1) + 0.5) * NT_UINT_SCALE;
  const double r = sqrt(-2.0 * log(u1));
  const double theta = 6.283185307179586 * u2;
  double s, c;
  sincos(theta, &s, &c);
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
