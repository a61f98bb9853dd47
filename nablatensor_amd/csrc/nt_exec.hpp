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
  hipFunction_t fn = nullptr, fn_slow = nullptr, fn_finish = nullptr;  // fn_slow: null when the kernel has none
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
  hipFunction_t fn_slow = nullptr, fn_dump_slow = nullptr;  // exception kernels, null when the tape needs none
  hipStream_t stream = nullptr;
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  double* d_inputs = nullptr;
  double* d_partials = nullptr;
  double* h_sums = nullptr;  // pinned host rows the finishing kernels write the sums to
  uint32_t* h_deferred = nullptr;  // pinned host word: the finishing pass found flagged lanes (nt_exec_replay)
  size_t h_cap = 0;          // doubles in h_sums
  void* d_scratch = nullptr;
  size_t scratch_bytes = 0;  // bytes of d_scratch: the reverse sweep's per-lane tape at the resident grid
  uint64_t* d_flags = nullptr;  // count of lanes that left paths to the exception kernel, then their bitmap
                                //   (grown with the dispatch; the count is zero between dispatches)
  size_t flags_bytes = 0;
  int dev = 0;
  int grid_cap = 1;     // most blocks a dispatch launches (partials, flags and tape are sized for it)
  int resident = 1;     // blocks the device holds at once (occupancy x compute units)
  int cus = 0;          // compute units of the device
  bool fixed_grid = false;  // the caller capped the grid (nt_options.max_blocks)
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

// Bytes of the flags of a dispatch on `lanes` threads (grid x block) pricing
// `markets` input sets: a 64-bit count, then one bit per lane and set in
// 64-bit words (one word per wave). The words must be zero before the first
// dispatch; every dispatch leaves them zero.
size_t flags_bytes_for(uint64_t lanes, int markets);

// Looks up, once per device and with that device current, the address of
// the allocation-free entry point's static array on device `dev`, and clears
// its flag region there (nt_noalloc.hip). Called when an executable is
// created, so that entry point itself never has to.
int noalloc_prepare(int dev);

// Length of each channel's column of partials in a dispatch over `grid`
// blocks (the skeleton's nt_partial_column): the replay kernel's region of
// 8 ceil(grid / 8) slots, then the exception kernel's. A dispatch of `nch`
// channels needs nch such columns, channel-major.
int partial_rows(int grid);

// Offset of the exception kernel's region within each column.
int partial_slow_offset(int grid);

// Launches the replay kernel `fn` over `grid` blocks on `stream` and, when
// `fn_slow` is set, the exception kernel after it, which writes the second
// region of every channel's column (partial_slow_offset).
// `between`, when set, is recorded after the replay kernel (it times that kernel alone).
int launch_kernel_on(nt_exec* x, hipStream_t stream, hipFunction_t fn, hipFunction_t fn_slow, const double* d_inputs,
                     double* d_partials, int nch, void* d_tape, uint64_t* d_flags, uint64_t paths, uint64_t offset,
                     uint64_t seed, double* out_v, double* out_g, int grid, hipEvent_t between = nullptr);

// The exception kernel alone, as launch_kernel_on launches it after the replay kernel.
int launch_slow_on(nt_exec* x, hipStream_t stream, hipFunction_t fn_slow, const double* d_inputs, double* d_partials,
                   int nch, void* d_tape, uint64_t* d_flags, uint64_t paths, uint64_t offset, uint64_t seed,
                   double* out_v, double* out_g, int grid);

// Finishing pass on `stream` over the `grid` rows of the replay kernel and,
// when the count at `d_flags` (null: none) is nonzero, the `slow_grid` rows of
// the exception kernel after them: `nch` sums written to `out` (device or
// pinned host memory); the count is reset to zero. With `deferred` (pinned
// host memory) set, the exception kernel has not run: when the count is
// nonzero the pass only writes 1 there and changes nothing else (else 0 and
// the sums as above).
int launch_finish_on(hipStream_t stream, hipFunction_t fn, const double* d_partials, int grid, int slow_grid, int nch,
                     double* out, uint64_t* d_flags, uint32_t* deferred = nullptr);

}  // namespace ntr
