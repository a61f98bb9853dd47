// Tape -> HIP lowering for the fused forward+adjoint replay kernel.
//
// Replaces the reference's CudaAadCodegen (nablatensor-core/.../engine/
// CudaAadCodegen.java:42-448) and its opt-in AadCheckpointPlan
// (AadCheckpointPlan.java:95-172). Instead of unrolling every node, the
// lowering finds the per-step loop of a Monte-Carlo tape (the role of the
// cpu-jit engine's detectLoop, nablatensor-engine-cpu/.../jit/
// KernelGenerator.java:549-658) and emits the step body once per segment of
// SEG unrolled iterations:
//   forward:  prologue; NSEG segments (carries checkpointed at each segment
//             start, optionally some body values stored); epilogue
//   reverse:  epilogue adjoints; segments last to first, each recomputing its
//             forward in registers (stored values are reloaded instead) and
//             then sweeping its iterations backwards; prologue adjoints.
// The adjoint accumulation order equals the oracle's node order, so fp64
// paths agree to rounding (FMA contraction aside).
//
// Tangent mode emits no reverse sweep: every active value carries the
// derivatives with respect to the inputs it depends on (a sparse set known at
// lowering time), propagated by the same local derivative rules. A Monte-Carlo
// step body then needs neither checkpoints nor recomputation; the cost model
// in make_plan picks it when those savings exceed the extra tangent work.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "nablatensor_rocm.h"

namespace ntl {

// Validated copy of a tape with activity (AadTape.markActive, AadTape.java:70-81).
struct TapeIR {
  int n = 0, n_in = 0, output = -1;  // output: the first (primary) output node
  std::vector<int> outputs;          // every output node, in output order
  int n_streams = 1;
  bool simple_draws = true;          // one stream and no uniform draws
  std::vector<int32_t> op, a, b;
  std::vector<double> c;
  std::vector<int32_t> input_node;
  std::vector<uint8_t> active;
};

// Operand classes of a body node, relative to its own iteration.
enum { ARG_NONE = 0, ARG_BODY = 1, ARG_CARRY = 2, ARG_INV = 3 };

struct LoopPlan {
  bool found = false;
  int start = 0, period = 0, iters = 0;
  int draws = 0;                      // draw nodes per iteration (normals and uniforms)
  std::vector<int> kind_a, ref_a;     // per body position
  std::vector<int> kind_b, ref_b;
  std::vector<int> rand_base;         // draw ordinal in iteration 0, -1 otherwise
  std::vector<int> rand_step;         // draw ordinal advance per iteration, 0 otherwise
  std::map<int, int> normal_step;     // stream -> normals drawn per iteration
  bool need_even = false;             // some stream draws an odd number of normals per iteration
  std::vector<int> carry_init;        // init node of a carried position, -1 otherwise
  std::vector<uint8_t> is_carry;      // read as carry-in by the next iteration
  std::vector<uint8_t> is_liveout;    // read by the epilogue from the last iteration
  // CONST positions whose literal changes from one iteration to the next (a
  // per-step year fraction): lit_table[j] set, lit_values[j][it] the literal
  // of iteration it. Only a loop detected with literal tables has them.
  std::vector<uint8_t> lit_table;
  std::vector<std::vector<double>> lit_values;
  int end() const { return start + period * iters; }
  bool table_lit(int pos) const { return pos >= 0 && pos < static_cast<int>(lit_table.size()) && lit_table[pos]; }
};

struct Plan {
  int precision = NT_FP64;
  int mode = NT_MODE_REVERSE;             // resolved NT_MODE_REVERSE or NT_MODE_TANGENT
  int markets = 1;                        // input sets per dispatch sharing each path's draws (tangent mode)
  int waves = 0;                          // launch-bound hint: minimum waves per SIMD (0: none)
  int basis = 0;                          // tangent loops: 0 cost model, 1 inputs, 2 loop parameters
  int n_words = 0;                        // 64-bit words per dependency set
  std::vector<uint64_t> deps;             // node -> inputs it depends on (bitset), tangent mode
  std::vector<uint64_t> posdeps;          // loop position -> union over the iterations
  double cost_reverse = 0, cost_tangent = 0;  // estimated extra VALU work per path of each mode
  double cost_forward = 0;                    // estimated VALU work per path of the forward sweep alone
  double path_cost = 0;                   // estimated VALU instructions per path: the forward plus the chosen
                                          // mode's extra work
  int adjoints = 1;
  int block = 256;
  bool contract = false;                  // FMA contraction allowed in the generated code
  bool fuse = true;                       // explicit fma of a tape node's own product and sum allowed where the
                                          // lowering knows it changes nothing the oracle resolves (off: contract -1)
  int libm = 0;                           // Box-Muller: 0 own fp64 math, 1 device libm, 2 own log/sqrt + libm sincos
  LoopPlan loop;
  int seg = 0, nseg_full = 0, tail = 0;   // iterations per segment, full segments, tail iterations
  int ckpt = NT_CKPT_RECOMPUTE;           // resolved policy
  std::vector<uint8_t> taped;             // body value read by the reverse (in-body or as carry-in)
  std::vector<uint8_t> stored;            // body value stored per iteration
  std::vector<int> store_index;           // position -> index among stored, -1 otherwise
  std::vector<int> carries;               // carried positions
  // Reverse sweep of a rolled loop: the positions a segment's recompute
  // produces (the values its rules read and what they are computed from; a
  // stored value is read back instead), and the carries whose value at the
  // segment's start it reads, checkpointed once per segment.
  std::vector<uint8_t> rneed;
  std::vector<int> ck_carries;
  int n_stored = 0;
  int ck_slots = 0, tape_slots = 0;       // per-thread scratch slots: checkpoints; checkpoints + stored values
  // Checkpointed straight line: the reverse sweep of a tape with no rolled
  // loop, cut into segments lbound[s] .. lbound[s + 1] (lbound empty: not
  // cut); lseg[node] is the node's segment. The forward pass runs segment
  // by segment, passing each value a later segment reads in carried slot
  // fslot[node] (kf slots), and stores each value that a later segment's
  // reverse reads once, in tape slot lslot[node]. The reverse, last segment
  // first, recomputes a segment's lneed nodes from lin[s] (stored values
  // read back, constants and inputs re-emitted), then runs its rules; the
  // adjoint of a node that a later segment's rules reach is carried in slot
  // aslot[node] (ka slots) from segment ahi[node], the last such reader,
  // down to its own.
  std::vector<int> lbound, lseg, lslot, fslot, aslot, ahi;
  std::vector<uint8_t> lneed;
  std::vector<std::vector<int>> lin;
  int kf = 0, ka = 0;
  int n_channels = 0;                     // 2 + n_inputs
};

// Returns NT_OK or an NT_E_* code with a message in err.
int build_ir(const nt_tape* tape, TapeIR& ir, std::string& err);
// `lit_tables`: a CONST of the step body may take another literal in each
// iteration (kept as a per-iteration table).
LoopPlan detect_loop(const TapeIR& ir, bool lit_tables = false);
// The same tape with every node that depends on no draw (and is neither an
// INPUT nor an output) moved to just before its first use, operands first;
// draws and the nodes that depend on them keep their order. A step schedule
// recorded up front (the per-step drift and volatility of a non-uniform time
// grid, GbmPath.java:49-66) then sits inside the step it feeds.
TapeIR sink_invariants(const TapeIR& ir);
// May replace `ir` by its sink_invariants form when only that form has a step
// loop covering most of the tape.
int make_plan(TapeIR& ir, const nt_options* opt, Plan& plan, std::string& err);
std::string emit_source(const TapeIR& ir, const Plan& plan);

}  // namespace ntl
