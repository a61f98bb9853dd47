// Throughput of the replay kernel's building blocks on the local GPU, in units
// of one fp64 FMA per lane: Philox2x32 rounds, fp64 exp/log/sqrt/div/sincos
// (device libm) and a full Box-Muller pair. Guides which transcendentals the
// kernel skeleton implements itself. Built by nablatensor_amd/build.py
// (build_mathbench) into nablatensor_amd/mathbench; run it on a gfx950 box.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include <cmath>
#define N_ITERS 1024
#define CH 8
typedef unsigned int u32; typedef unsigned long long u64;

__global__ void k_fma(double* out, double a) {
  double x[CH]; for (int c = 0; c < CH; ++c) x[c] = threadIdx.x * 1e-3 + c;
  for (int i = 0; i < N_ITERS; ++i) {
#pragma unroll
    for (int c = 0; c < CH; ++c) x[c] = fma(x[c], a, 0.25);
  }
  double s = 0; for (int c = 0; c < CH; ++c) s += x[c]; out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}
__global__ void k_mad64(double* out, u32 m) {
  u32 x[CH], y[CH]; for (int c = 0; c < CH; ++c) { x[c] = threadIdx.x + c; y[c] = c * 7; }
  for (int i = 0; i < N_ITERS; ++i) {
#pragma unroll
    for (int c = 0; c < CH; ++c) { u64 p = (u64)m * x[c]; x[c] = (u32)(p >> 32) ^ y[c] ^ 0x1234u; y[c] = (u32)p; }
  }
  u32 s = 0; for (int c = 0; c < CH; ++c) s ^= x[c] + y[c]; out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}
#define UNARY(name, expr) \
__global__ void name(double* out, double a) { \
  double x[CH]; for (int c = 0; c < CH; ++c) x[c] = 0.3 + threadIdx.x * 1e-6 + c * 1e-3; \
  for (int i = 0; i < N_ITERS / 8; ++i) { \
    _Pragma("unroll") for (int c = 0; c < CH; ++c) { double v = x[c]; x[c] = expr; } \
  } \
  double s = 0; for (int c = 0; c < CH; ++c) s += x[c]; out[blockIdx.x * blockDim.x + threadIdx.x] = s; }
UNARY(k_exp, exp(v * a) * 0.5)
UNARY(k_log, -log(v) * a + 0.1)
UNARY(k_sqrt, sqrt(v) * a + 0.01)
UNARY(k_sincos, ({ double s_, c_; sincos(v * 6.283185307179586, &s_, &c_); fabs(s_ * c_) * a + 0.1; }))
UNARY(k_sincospi, ({ double s_, c_; sincospi(2.0 * v, &s_, &c_); fabs(s_ * c_) * a + 0.1; }))
UNARY(k_div, 1.0 / (v + a))

__global__ void k_bm(double* out, double a) {
  double acc = 0;
  u32 lo = threadIdx.x * 7919u + blockIdx.x, hi = blockIdx.x;
  for (int i = 0; i < N_ITERS / 8; ++i) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      u32 c0 = lo, c1 = hi ^ (u32)(i * CH + c);
#pragma unroll
      for (int r = 0; r < 10; ++r) { u64 p = (u64)0xD256D193u * c0; c0 = (u32)(p >> 32) ^ (0x1BD11BDAu + 0x9E3779B9u * r) ^ c1; c1 = (u32)p; }
      double u1 = ((double)c0 + 0.5) * 2.3283064365386963e-10, u2 = ((double)c1 + 0.5) * 2.3283064365386963e-10;
      double rr = sqrt(-2.0 * log(u1)); double s, cc; sincos(6.283185307179586 * u2, &s, &cc);
      acc += rr * s + rr * cc;
    }
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = acc * a;
}
__global__ void k_philox(double* out, double a) {
  u32 acc = 0; u32 lo = threadIdx.x * 7919u + blockIdx.x, hi = blockIdx.x;
  for (int i = 0; i < N_ITERS / 8; ++i) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      u32 c0 = lo, c1 = hi ^ (u32)(i * CH + c);
#pragma unroll
      for (int r = 0; r < 10; ++r) { u64 p = (u64)0xD256D193u * c0; c0 = (u32)(p >> 32) ^ (0x1BD11BDAu + 0x9E3779B9u * r) ^ c1; c1 = (u32)p; }
      acc += c0 ^ c1;
    }
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = acc * a;
}

int main() {
  const int blocks = 4096, threads = 256;
  double* out; hipMalloc(&out, sizeof(double) * blocks * threads);
  hipEvent_t e0, e1; hipEventCreate(&e0); hipEventCreate(&e1);
  struct K { const char* name; void (*launch)(double*); double ops_per_lane; };
  auto run = [&](const char* name, auto fn, double ops) {
    fn(); hipDeviceSynchronize();
    hipEventRecord(e0); for (int r = 0; r < 3; ++r) fn(); hipEventRecord(e1); hipEventSynchronize(e1);
    float ms; hipEventElapsedTime(&ms, e0, e1); ms /= 3;
    double lane_ops = (double)blocks * threads * ops;
    printf("%-10s %8.3f ms  %8.3f Glane-ops/s  %8.3f ns/1k-lane-op\n", name, ms, lane_ops / ms / 1e6, ms * 1e6 / (lane_ops / 1e3));
    return ms / ops;
  };
  double base = run("fma", [&] { k_fma<<<blocks, threads>>>(out, 0.999); }, (double)N_ITERS * CH);
  auto rel = [&](const char* n, double t) { printf("   %-10s = %6.1f fma-equivalents\n", n, t / base); };
  rel("mad64+xor", run("mad64", [&] { k_mad64<<<blocks, threads>>>(out, 0xD256D193u); }, (double)N_ITERS * CH));
  rel("exp", run("exp", [&] { k_exp<<<blocks, threads>>>(out, 0.999); }, (double)N_ITERS / 8 * CH));
  rel("log", run("log", [&] { k_log<<<blocks, threads>>>(out, 0.2); }, (double)N_ITERS / 8 * CH));
  rel("sqrt", run("sqrt", [&] { k_sqrt<<<blocks, threads>>>(out, 0.999); }, (double)N_ITERS / 8 * CH));
  rel("div", run("div", [&] { k_div<<<blocks, threads>>>(out, 0.5); }, (double)N_ITERS / 8 * CH));
  rel("sincos", run("sincos", [&] { k_sincos<<<blocks, threads>>>(out, 0.999); }, (double)N_ITERS / 8 * CH));
  rel("sincospi", run("sincospi", [&] { k_sincospi<<<blocks, threads>>>(out, 0.999); }, (double)N_ITERS / 8 * CH));
  rel("philox", run("philox", [&] { k_philox<<<blocks, threads>>>(out, 1.0); }, (double)N_ITERS / 8 * CH));
  rel("bm_pair", run("bm_pair", [&] { k_bm<<<blocks, threads>>>(out, 1.0); }, (double)N_ITERS / 8 * CH));
  hipFree(out);
  return 0;
}
