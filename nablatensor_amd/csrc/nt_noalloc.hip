// Allocation-free replay: nt_exec_replay_noalloc (include/nablatensor_rocm.h).
//
// nt_exec_replay keeps the replay kernels' per-block partial sums, the bitmap
// of lanes that left paths to the exception kernel and, for a reverse-sweep executable
// that stores its tape in device memory, that per-lane tape in buffers the
// executable allocated with hipMalloc, and copies inputs from, and sums to,
// host memory. This entry point runs the same kernels (replay, exception,
// finishing pass) with those buffers carved out of `scratch`, a static device
// array of NT_NOALLOC_SCRATCH_BYTES that each device holds from the first
// call until the process ends. The caller
// passes device pointers for the inputs and the sums and a stream; nothing is
// allocated, copied or waited for, so the call can sit in a tight loop or
// under stream capture.
//
// The grid is nt_exec_replay's (ntr::grid_for), so the sums are bit-identical
// to that entry point's for the same paths, offset, seed and inputs. Every
// call on a device shares that device's array: calls that overlap in time on
// one device (on different streams, or from different threads) race on it.
// The array is laid out as the flags (a count of the lanes that left paths to
// the exception kernel, then their bitmap, one bit per lane of the grid) in a
// region of their own of kFlagBytes at the start, then the partials and a
// reverse sweep's tape. The flags must be zero before a dispatch and every
// dispatch leaves them zero (the finishing pass resets the count, the
// exception kernel the bitmap words it read), so their region is never used
// for anything else: one dispatch's partials can never be read as another's
// flags. noalloc_prepare clears it once per device when the first executable
// on that device is created. Every block writes its own entry of each
// channel's partials, and the finishing pass reads only the entries written.
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

constexpr size_t round_up_256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

// The flag region: the count and one bitmap word per 64 lanes (the layout of
// ntr::flags_bytes_for for one input set), for up to kFlagLanes lanes (2^22:
// a resident grid on MI355X holds at most 256 CUs x 2,048 lanes, and a
// dispatch launches at most 8 resident grids).
constexpr uint64_t kFlagLanes = 1ull << 22;
constexpr size_t kFlagBytes = round_up_256((1 + kFlagLanes / 64) * sizeof(uint64_t));

// The device address of `scratch` on device `dev`, looked up once per device
// with that device current (each device holds its own copy at its own
// address); the first lookup also clears the flag region. Host code uses this
// address, never the array's name.
int scratch_on(int dev, void*& out) {
  if (dev < 0 || dev >= kMaxDevices) return ntr::fail(NT_E_INTERNAL, "device index beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    NT_HIP(hipSetDevice(dev), "hipSetDevice");
    NT_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!p) return ntr::fail(NT_E_INTERNAL, "hipGetSymbolAddress(scratch) returned a null address");
    NT_HIP(hipMemsetAsync(p, 0, kFlagBytes, nullptr), "hipMemsetAsync(scratch flags)");
    NT_HIP(hipStreamSynchronize(nullptr), "hipStreamSynchronize");  // before any stream uses the array
    g_scratch[dev] = p;
  }
  out = g_scratch[dev];
  return NT_OK;
}

}  // namespace

namespace ntr {

int noalloc_prepare(int dev) {
  void* p = nullptr;
  return scratch_on(dev, p);
}

}  // namespace ntr

extern "C" int nt_exec_replay_noalloc(nt_exec* x, const double* d_inputs, uint64_t paths, uint64_t offset,
                                      uint64_t seed, double* d_sums, int32_t n_sums, void* stream) {
  if (!x) return ntr::fail(NT_E_CLOSED, "executable is closed");
  if (paths == 0) return ntr::fail(NT_E_INVALID, "paths must be positive");
  const int nch = x->low.plan.n_channels;
  if (!d_sums || n_sums != nch) return ntr::fail(NT_E_INVALID, "d_sums must hold n_outputs * (2 + n_inputs) doubles");
  if (x->low.ir.n_in > 0 && !d_inputs) return ntr::fail(NT_E_INVALID, "d_inputs is null");
  const int grid = ntr::grid_for(x, paths);
  const uint64_t lanes = static_cast<uint64_t>(grid) * static_cast<uint64_t>(x->low.plan.block);
  if (lanes > kFlagLanes) {
    return ntr::fail(NT_E_INVALID, "the dispatch's grid has more lanes than the allocation-free entry point's "
                                   "flags cover (2^22)");
  }
  const int rows = ntr::partial_rows(grid);
  const size_t partial_bytes = round_up_256(sizeof(double) * static_cast<size_t>(rows) * static_cast<size_t>(nch));
  const size_t flag_bytes = kFlagBytes;
  const size_t tape_bytes = ntr::tape_bytes_per_lane(x) * static_cast<size_t>(lanes);
  if (partial_bytes + flag_bytes + tape_bytes > static_cast<size_t>(NT_NOALLOC_SCRATCH_BYTES)) {
    char buf[320];
    std::snprintf(buf, sizeof buf,
                  "this dispatch needs %zu bytes of scratch (%zu of partials, %zu of lane flags, %zu of per-lane "
                  "tape at %d blocks); the allocation-free entry point has %zu",
                  partial_bytes + flag_bytes + tape_bytes, partial_bytes, flag_bytes, tape_bytes, grid,
                  static_cast<size_t>(NT_NOALLOC_SCRATCH_BYTES));
    return ntr::fail(NT_E_INVALID, buf);
  }
  void* base = nullptr;
  int rc = scratch_on(x->dev, base);
  if (rc != NT_OK) return rc;
  NT_HIP(hipSetDevice(x->dev), "hipSetDevice");
  hipStream_t s = stream ? static_cast<hipStream_t>(stream) : x->stream;
  char* at = static_cast<char*>(base);
  uint64_t* flags = reinterpret_cast<uint64_t*>(at);
  double* partials = reinterpret_cast<double*>(at + flag_bytes);
  void* tape = tape_bytes ? static_cast<void*>(at + flag_bytes + partial_bytes) : nullptr;
  rc = ntr::launch_kernel_on(x, s, x->fn, x->fn_slow, d_inputs, partials, nch, tape, flags, paths, offset, seed, nullptr,
                             nullptr, grid);
  if (rc != NT_OK) return rc;
  return ntr::launch_finish_on(s, x->fn_finish, partials, grid, x->fn_slow ? grid : 0, nch, d_sums,
                               x->fn_slow ? flags : nullptr);
}
