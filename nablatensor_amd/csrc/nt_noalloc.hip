// Allocation-free replay: nt_exec_replay_noalloc (include/nablatensor_rocm.h).
//
// nt_exec_replay keeps the replay kernel's per-block partial sums (and, for a
// reverse-sweep executable that stores its tape in device memory, that
// per-lane tape) in buffers the executable allocated with hipMalloc, and
// copies inputs from, and sums to, host memory. This entry point runs the
// same two kernels (replay, then the finishing pass) with those buffers carved
// out of `scratch`, a static device array of NT_NOALLOC_SCRATCH_BYTES that
// each device holds from the first call until the process ends. The caller
// passes device pointers for the inputs and the sums and a stream; nothing is
// allocated, copied or waited for, so the call can sit in a tight loop or
// under stream capture.
//
// The grid is nt_exec_replay's (ntr::grid_for), so the sums are bit-identical
// to that entry point's for the same paths, offset, seed and inputs. Every
// call on a device shares that device's array: calls that overlap in time on
// one device (on different streams, or from different threads) race on it.
// Nothing in the array has to start at zero: every block writes its own row
// of partials and the finishing pass reads only those rows.
//
// Compiled by hipcc (the array is device code); the rest of libnt_rocm.so is
// host C++ built with g++.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "nt_exec.hpp"

static __device__ __align__(256) unsigned char scratch[NT_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices] = {};  // device address of each device's copy of `scratch`

// The device address of `scratch` on device `dev`, looked up once per device
// with that device current (each device holds its own copy at its own
// address). Host code uses this address, never the array's name.
int scratch_on(int dev, void*& out) {
  if (dev < 0 || dev >= kMaxDevices) return ntr::fail(NT_E_INTERNAL, "device index beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    NT_HIP(hipSetDevice(dev), "hipSetDevice");
    NT_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!p) return ntr::fail(NT_E_INTERNAL, "hipGetSymbolAddress(scratch) returned a null address");
    g_scratch[dev] = p;
  }
  out = g_scratch[dev];
  return NT_OK;
}

size_t round_up_256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

}  // namespace

extern "C" int nt_exec_replay_noalloc(nt_exec* x, const double* d_inputs, uint64_t paths, uint64_t offset,
                                      uint64_t seed, double* d_sums, int32_t n_sums, void* stream) {
  if (!x) return ntr::fail(NT_E_CLOSED, "executable is closed");
  if (paths == 0) return ntr::fail(NT_E_INVALID, "paths must be positive");
  const int nch = x->low.plan.n_channels;
  if (!d_sums || n_sums != nch) return ntr::fail(NT_E_INVALID, "d_sums must hold n_outputs * (2 + n_inputs) doubles");
  if (x->low.ir.n_in > 0 && !d_inputs) return ntr::fail(NT_E_INVALID, "d_inputs is null");
  const int grid = ntr::grid_for(x, paths);
  const size_t partial_bytes = round_up_256(sizeof(double) * static_cast<size_t>(grid) * static_cast<size_t>(nch));
  const size_t tape_bytes =
      ntr::tape_bytes_per_lane(x) * static_cast<size_t>(grid) * static_cast<size_t>(x->low.plan.block);
  if (partial_bytes + tape_bytes > static_cast<size_t>(NT_NOALLOC_SCRATCH_BYTES)) {
    char buf[256];
    std::snprintf(buf, sizeof buf,
                  "this dispatch needs %zu bytes of scratch (%zu of partials, %zu of per-lane tape at %d blocks); "
                  "the allocation-free entry point has %zu",
                  partial_bytes + tape_bytes, partial_bytes, tape_bytes, grid,
                  static_cast<size_t>(NT_NOALLOC_SCRATCH_BYTES));
    return ntr::fail(NT_E_INVALID, buf);
  }
  void* base = nullptr;
  int rc = scratch_on(x->dev, base);
  if (rc != NT_OK) return rc;
  NT_HIP(hipSetDevice(x->dev), "hipSetDevice");
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : x->stream;
  double* partials = static_cast<double*>(base);
  void* tape = tape_bytes ? static_cast<void*>(static_cast<char*>(base) + partial_bytes) : nullptr;
  rc = ntr::launch_kernel_on(x, s, x->fn, d_inputs, partials, tape, paths, offset, seed, nullptr, nullptr, grid);
  if (rc != NT_OK) return rc;
  return ntr::launch_finish_on(s, x->fn_finish, partials, grid, nch, d_sums);
}
