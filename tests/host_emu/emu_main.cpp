// Driver for an emulated replay kernel; NT_KERNEL_FILE names the generated source.
#include "prelude.h"
#include NT_KERNEL_FILE

#include <cstddef>
#include <vector>

extern "C" int emu_run(nt_u64 n_paths, nt_u64 offset, nt_u64 seed, const double* inputs, double* sums,
                       double* out_v, double* out_g, unsigned grid, unsigned block, unsigned long long slots) {
  gridDim.x = grid;
  // Threads run one after another here, so the block-cooperative table copy is
  // done once, whole, before any of them reads it.
  blockDim.x = 1;
  threadIdx.x = 0;
  nt_tables_load();
  blockDim.x = block;
  std::vector<real> scratch(static_cast<size_t>(grid) * block * (slots ? slots : 1));
  // the count, then one lane bitmap per market (at most 64 markets)
  const size_t lane_words = (static_cast<size_t>(grid) * block + 63) / 64;
  std::vector<nt_u64> flags(1 + lane_words * 64, 0);
  for (unsigned b = 0; b < grid; ++b) {
    for (unsigned t = 0; t < block; ++t) {
      blockIdx.x = b;
      threadIdx.x = t;
      nt_replay(inputs, n_paths, offset, seed, sums, scratch.data(), out_v, out_g, flags.data());
    }
  }
#ifdef NT_HAS_SLOW
  for (unsigned b = 0; b < grid; ++b) {
    for (unsigned t = 0; t < block; ++t) {
      blockIdx.x = b;
      threadIdx.x = t;
      nt_replay_slow(inputs, n_paths, offset, seed, sums, scratch.data(), out_v, out_g, flags.data());
    }
  }
  // the exception kernel leaves the bitmap as it found it before the replay
  for (size_t i = 1; i < flags.size(); ++i) {
    if (flags[i] != 0) return 1;
  }
#endif
  return 0;
}
