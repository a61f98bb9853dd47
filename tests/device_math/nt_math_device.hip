// Test driver: the skeleton's own fp64 math routines (nt_skeleton.h) as
// compiled for gfx950, evaluated over device arrays, for the accuracy tests
// in tests/test_gpu_math.py. Built by nablatensor_amd/build.py into
// tests/device_math/libnt_math_device.so; each dm_* entry point copies its
// arguments to the device, runs one kernel (every thread loads the LDS
// tables, then strides over the arguments) and copies the results back.
// Returns 0 or the hipError_t of the first failing call.
#include <hip/hip_runtime.h>

#include "nt_skeleton.h"

namespace {

__global__ void k_neg2log(const nt_u32* __restrict__ c, double* __restrict__ out, long n) {
  nt_tables_load();
  const long T = static_cast<long>(gridDim.x) * blockDim.x;
  for (long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += T) out[i] = nt_neg2log_u32(c[i]);
}

__global__ void k_sincos(const nt_u32* __restrict__ c, double* __restrict__ s, double* __restrict__ co, long n) {
  nt_tables_load();
  const long T = static_cast<long>(gridDim.x) * blockDim.x;
  for (long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += T) {
    nt_sincos_2pi_u32(c[i], s[i], co[i]);
  }
}

__global__ void k_exp(const double* __restrict__ x, double* __restrict__ out, int* __restrict__ bad, long n) {
  nt_tables_load();
  const long T = static_cast<long>(gridDim.x) * blockDim.x;
  for (long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += T) {
    bool b = false;
    out[i] = nt_exp_fast(x[i], b);
    bad[i] = b ? 1 : 0;
  }
}

__global__ void k_log(const double* __restrict__ x, double* __restrict__ out, int* __restrict__ bad, long n) {
  nt_tables_load();
  const long T = static_cast<long>(gridDim.x) * blockDim.x;
  for (long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += T) {
    bool b = false;
    out[i] = nt_log_fast(x[i], b);
    bad[i] = b ? 1 : 0;
  }
}

__global__ void k_sqrt_q(const double* __restrict__ a, double* __restrict__ out, double* __restrict__ q,
                         int* __restrict__ bad, long n) {
  const long T = static_cast<long>(gridDim.x) * blockDim.x;
  for (long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += T) {
    bool b = false;
    double qi = 0.0;
    out[i] = nt_sqrt_q(a[i], qi, b);
    q[i] = qi;
    bad[i] = b ? 1 : 0;
  }
}

__global__ void k_recip(const double* __restrict__ x, double* __restrict__ out, int* __restrict__ bad, long n) {
  const long T = static_cast<long>(gridDim.x) * blockDim.x;
  for (long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += T) {
    bool b = false;
    out[i] = nt_recip(x[i], b);
    bad[i] = b ? 1 : 0;
  }
}

__global__ void k_normal_pair(const nt_u32* __restrict__ lo, const nt_u32* __restrict__ hi,
                              const nt_u32* __restrict__ ctr, double* __restrict__ zc, double* __restrict__ zs, long n) {
  nt_tables_load();
  const long T = static_cast<long>(gridDim.x) * blockDim.x;
  for (long i = static_cast<long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += T) {
    nt_normal_pair(lo[i], hi[i], ctr[i], zc[i], zs[i]);
  }
}

// Device copies of host arrays: `in` are copied in, `out` copied back, all freed at the end.
struct Buffers {
  void* d[5] = {};
  size_t bytes[5] = {};
  int k = 0;
  hipError_t err = hipSuccess;
  void* add(const void* host, size_t n) {
    if (err != hipSuccess) return nullptr;
    err = hipMalloc(&d[k], n > 0 ? n : 1);
    if (err == hipSuccess && host) err = hipMemcpy(d[k], host, n, hipMemcpyHostToDevice);
    bytes[k] = n;
    return d[k++];
  }
  void back(int i, void* host) {
    if (err == hipSuccess) err = hipMemcpy(host, d[i], bytes[i], hipMemcpyDeviceToHost);
  }
  ~Buffers() {
    for (int i = 0; i < k; ++i) {
      if (d[i]) (void)hipFree(d[i]);
    }
  }
};

dim3 grid_for(long n) { return dim3(static_cast<unsigned>(n / 256 + 1 < 4096 ? n / 256 + 1 : 4096)); }

int finish(Buffers& b) {
  if (b.err == hipSuccess) b.err = hipGetLastError();
  if (b.err == hipSuccess) b.err = hipDeviceSynchronize();
  return static_cast<int>(b.err);
}

}  // namespace

extern "C" {

int dm_neg2log(const nt_u32* c, double* out, long n) {
  Buffers b;
  auto* dc = static_cast<nt_u32*>(b.add(c, sizeof(nt_u32) * n));
  auto* dout = static_cast<double*>(b.add(nullptr, sizeof(double) * n));
  if (b.err == hipSuccess) hipLaunchKernelGGL(k_neg2log, grid_for(n), dim3(256), 0, 0, dc, dout, n);
  int rc = finish(b);
  b.back(1, out);
  return rc ? rc : static_cast<int>(b.err);
}

int dm_sincos(const nt_u32* c, double* s, double* co, long n) {
  Buffers b;
  auto* dc = static_cast<nt_u32*>(b.add(c, sizeof(nt_u32) * n));
  auto* ds = static_cast<double*>(b.add(nullptr, sizeof(double) * n));
  auto* dco = static_cast<double*>(b.add(nullptr, sizeof(double) * n));
  if (b.err == hipSuccess) hipLaunchKernelGGL(k_sincos, grid_for(n), dim3(256), 0, 0, dc, ds, dco, n);
  int rc = finish(b);
  b.back(1, s);
  b.back(2, co);
  return rc ? rc : static_cast<int>(b.err);
}

int dm_exp(const double* x, double* out, int* bad, long n) {
  Buffers b;
  auto* dx = static_cast<double*>(b.add(x, sizeof(double) * n));
  auto* dout = static_cast<double*>(b.add(nullptr, sizeof(double) * n));
  auto* dbad = static_cast<int*>(b.add(nullptr, sizeof(int) * n));
  if (b.err == hipSuccess) hipLaunchKernelGGL(k_exp, grid_for(n), dim3(256), 0, 0, dx, dout, dbad, n);
  int rc = finish(b);
  b.back(1, out);
  b.back(2, bad);
  return rc ? rc : static_cast<int>(b.err);
}

int dm_log(const double* x, double* out, int* bad, long n) {
  Buffers b;
  auto* dx = static_cast<double*>(b.add(x, sizeof(double) * n));
  auto* dout = static_cast<double*>(b.add(nullptr, sizeof(double) * n));
  auto* dbad = static_cast<int*>(b.add(nullptr, sizeof(int) * n));
  if (b.err == hipSuccess) hipLaunchKernelGGL(k_log, grid_for(n), dim3(256), 0, 0, dx, dout, dbad, n);
  int rc = finish(b);
  b.back(1, out);
  b.back(2, bad);
  return rc ? rc : static_cast<int>(b.err);
}

int dm_sqrt_q(const double* a, double* out, double* q, int* bad, long n) {
  Buffers b;
  auto* da = static_cast<double*>(b.add(a, sizeof(double) * n));
  auto* dout = static_cast<double*>(b.add(nullptr, sizeof(double) * n));
  auto* dq = static_cast<double*>(b.add(nullptr, sizeof(double) * n));
  auto* dbad = static_cast<int*>(b.add(nullptr, sizeof(int) * n));
  if (b.err == hipSuccess) hipLaunchKernelGGL(k_sqrt_q, grid_for(n), dim3(256), 0, 0, da, dout, dq, dbad, n);
  int rc = finish(b);
  b.back(1, out);
  b.back(2, q);
  b.back(3, bad);
  return rc ? rc : static_cast<int>(b.err);
}

int dm_recip(const double* x, double* out, int* bad, long n) {
  Buffers b;
  auto* dx = static_cast<double*>(b.add(x, sizeof(double) * n));
  auto* dout = static_cast<double*>(b.add(nullptr, sizeof(double) * n));
  auto* dbad = static_cast<int*>(b.add(nullptr, sizeof(int) * n));
  if (b.err == hipSuccess) hipLaunchKernelGGL(k_recip, grid_for(n), dim3(256), 0, 0, dx, dout, dbad, n);
  int rc = finish(b);
  b.back(1, out);
  b.back(2, bad);
  return rc ? rc : static_cast<int>(b.err);
}

int dm_normal_pair(const nt_u32* lo, const nt_u32* hi, const nt_u32* ctr, double* zc, double* zs, long n) {
  Buffers b;
  auto* dlo = static_cast<nt_u32*>(b.add(lo, sizeof(nt_u32) * n));
  auto* dhi = static_cast<nt_u32*>(b.add(hi, sizeof(nt_u32) * n));
  auto* dctr = static_cast<nt_u32*>(b.add(ctr, sizeof(nt_u32) * n));
  auto* dzc = static_cast<double*>(b.add(nullptr, sizeof(double) * n));
  auto* dzs = static_cast<double*>(b.add(nullptr, sizeof(double) * n));
  if (b.err == hipSuccess) hipLaunchKernelGGL(k_normal_pair, grid_for(n), dim3(256), 0, 0, dlo, dhi, dctr, dzc, dzs, n);
  int rc = finish(b);
  b.back(3, zc);
  b.back(4, zs);
  return rc ? rc : static_cast<int>(b.err);
}

}  // extern "C"
