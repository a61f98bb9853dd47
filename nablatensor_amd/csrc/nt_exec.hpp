// Internal: the executable behind the C ABI's opaque nt_exec handle, and the
// runtime helpers that more than one source file of libnt_rocm.so uses
// (nt_rocm.cpp: every entry point but one; nt_noalloc.hip: the
// allocation-free replay, which owns a static device array and so is
// compiled by hipcc). Not installed; include/nablatensor_rocm.h is the API.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "lower.hpp"
#include "nablatensor_rocm.h"

namespace ntr {

// Records `msg` as the calling thread's nt_last_error() and returns `code`.
int fail(int code, const std::string& msg);
// The same for a failed HIP call: "<what> failed: <hipGetErrorString> (code N)".
int hip_fail(hipError_t e, const char* what);
// The calling thread's last message.
const char* last_error();

#define NT_HIP(call, what)                                  \
  do {                                                      \
    hipError_t e_ = (call);                                 \
    if (e_ != hipSuccess) return ::ntr::hip_fail(e_, what); \
  } while (0)

struct Lowered {
  ntl::TapeIR ir;
  ntl::Plan plan;
  std::string source;
};

// A kernel that prices several input sets per path (nt_exec_replay_many).
struct MarketVariant {
  int vgprs = 0, scratch = 0;
  hipModule_t mod = nullptr;
  hipFunction_t fn = nullptr, fn_finish = nullptr;
  double* d_inputs = nullptr;
  double* d_partials = nullptr;
};

}  // namespace ntr

struct nt_exec {
  nt_options opts{};
  ntr::Lowered low;
  nt_exec_info info{};
  std::vector<char> code;
  hipModule_t mod = nullptr, mod_dump = nullptr;
  hipFunction_t fn = nullptr, fn_finish = nullptr, fn_dump = nullptr;
  hipStream_t stream = nullptr;
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  double* d_inputs = nullptr;
  double* d_partials = nullptr;
  double* h_sums = nullptr;  // pinned host rows the finishing kernels write the sums to
  size_t h_cap = 0;          // doubles in h_sums
  void* d_scratch = nullptr;
  size_t scratch_bytes = 0;  // bytes of d_scratch: the reverse sweep's per-lane tape at the resident grid
  int dev = 0;
  int grid_cap = 1;
  std::vector<double> inputs;
  bool dirty = true;
  std::map<int, ntr::MarketVariant> markets;  // by set count
  int market_chunk = 0;                       // input sets per multi-market dispatch, 0 until chosen
  double* d_set_inputs = nullptr;             // one input set at a time (reverse-sweep executables)

  nt_exec() = default;
  nt_exec(const nt_exec&) = delete;
  nt_exec& operator=(const nt_exec&) = delete;
  // Releases whatever was acquired, so a create that fails part way frees it too.
  ~nt_exec();
};

namespace ntr {

// Grid of a dispatch over `paths`: one block per `block` paths up to the
// resident cap. Every kernel of an executable uses it, so a path always lands
// on the same lane and block and the sums agree bit for bit between entry points.
int grid_for(const nt_exec* x, uint64_t paths);

// Bytes per lane of the reverse sweep's tape (checkpoints and stored values).
size_t tape_bytes_per_lane(const nt_exec* x);

// Launches the replay kernel `fn` over `grid` blocks on `stream`.
int launch_kernel_on(nt_exec* x, hipStream_t stream, hipFunction_t fn, const double* d_inputs, double* d_partials,
                     void* d_tape, uint64_t paths, uint64_t offset, uint64_t seed, double* out_v, double* out_g,
                     int grid);

// Finishing pass over the `grid` partial rows of one replay launch on
// `stream`: `nch` sums written to `out` (device or pinned host memory).
int launch_finish_on(hipStream_t stream, hipFunction_t fn, const double* d_partials, int grid, int nch, double* out);

}  // namespace ntr
