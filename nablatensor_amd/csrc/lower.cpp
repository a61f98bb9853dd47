// Tape -> HIP lowering; see lower.hpp for the structure of the emitted kernel.
#include "lower.hpp"

#include <algorithm>
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <set>
#include <sstream>

namespace ntl {

namespace {

int arity(int op) {
  switch (op) {
    case NT_OP_CONST: case NT_OP_INPUT: case NT_OP_RANDN: case NT_OP_RANDU: return 0;
    case NT_OP_NEG: case NT_OP_EXP: case NT_OP_LOG: case NT_OP_SQRT: case NT_OP_ABS: return 1;
    default: return 2;
  }
}

uint64_t bits(double v) {
  uint64_t u;
  std::memcpy(&u, &v, sizeof u);
  return u;
}

}  // namespace

// ---- validation (AadEngine.requireSupportedTape, AadEngine.java:56-86) ---------

int build_ir(const nt_tape* t, TapeIR& ir, std::string& err) {
  if (!t) { err = "tape is null"; return NT_E_INVALID; }
  if (t->n_nodes <= 0 || !t->op || !t->arg_a || !t->arg_b || !t->constant) {
    err = "tape has no nodes";
    return NT_E_INVALID;
  }
  if (t->n_outputs < 1 || !t->output_node) { err = "no output was recorded"; return NT_E_INVALID; }
  if (t->n_streams < 1) { err = "a tape has at least one random stream"; return NT_E_INVALID; }
  if (t->n_inputs < 0 || (t->n_inputs > 0 && !t->input_node)) { err = "bad input list"; return NT_E_INVALID; }
  const int n = t->n_nodes;
  ir.n = n;
  ir.n_in = t->n_inputs;
  ir.op.assign(t->op, t->op + n);
  ir.a.assign(t->arg_a, t->arg_a + n);
  ir.b.assign(t->arg_b, t->arg_b + n);
  ir.c.assign(t->constant, t->constant + n);
  ir.input_node.assign(t->input_node, t->input_node + t->n_inputs);
  ir.outputs.assign(t->output_node, t->output_node + t->n_outputs);
  ir.output = ir.outputs[0];
  ir.n_streams = t->n_streams;
  ir.simple_draws = t->n_streams == 1;
  for (int i = 0; i < n; ++i) {
    const int op = ir.op[i], a = ir.a[i], b = ir.b[i];
    char buf[160];
    if (op < NT_OP_CONST || op > NT_OP_ABS) {
      std::snprintf(buf, sizeof buf, "node %d has unknown opcode %d", i, op);
      err = buf;
      return NT_E_INVALID;
    }
    if (op == NT_OP_RANDN || op == NT_OP_RANDU) {
      if (a < 0) {
        std::snprintf(buf, sizeof buf, "draw node %d has negative ordinal %d", i, a);
        err = buf;
        return NT_E_INVALID;
      }
      if (b < 0 || b >= t->n_streams) {
        std::snprintf(buf, sizeof buf, "draw node %d names stream %d of %d", i, b, t->n_streams);
        err = buf;
        return NT_E_INVALID;
      }
      if (op == NT_OP_RANDU) ir.simple_draws = false;
    }
    if (op == NT_OP_INPUT && (a < 0 || a >= ir.n_in || ir.input_node[a] != i)) {
      std::snprintf(buf, sizeof buf, "input node %d has bad input index %d", i, a);
      err = buf;
      return NT_E_INVALID;
    }
    const int ar = arity(op);
    if ((ar >= 1 && (a < 0 || a >= i)) || (ar >= 2 && (b < 0 || b >= i))) {
      std::snprintf(buf, sizeof buf, "node %d reads a node that is not before it (%d, %d)", i, a, b);
      err = buf;
      return NT_E_INVALID;
    }
  }
  for (int j = 0; j < ir.n_in; ++j) {
    const int node = ir.input_node[j];
    if (node < 0 || node >= n || ir.op[node] != NT_OP_INPUT || ir.a[node] != j) {
      err = "input list does not match the INPUT nodes";
      return NT_E_INVALID;
    }
  }
  for (int out : ir.outputs) {
    if (out < 0 || out >= n) { err = "output node out of range"; return NT_E_INVALID; }
  }
  ir.active.assign(n, 0);
  for (int i = 0; i < n; ++i) {
    const int op = ir.op[i];
    if (op == NT_OP_INPUT) ir.active[i] = 1;
    else if (op == NT_OP_CONST || op == NT_OP_RANDN || op == NT_OP_RANDU) ir.active[i] = 0;
    else if (arity(op) == 1) ir.active[i] = ir.active[ir.a[i]];
    else ir.active[i] = static_cast<uint8_t>(ir.active[ir.a[i]] || ir.active[ir.b[i]]);
  }
  return NT_OK;
}

// ---- loop detection ----------------------------------------------------------

namespace {

bool is_draw(int op) { return op == NT_OP_RANDN || op == NT_OP_RANDU; }

// A draw k repeating draw i: same kind and stream, ordinal advanced by D (for
// a tape with one stream of normals) or by any positive step (several streams
// or uniforms: verify() then checks that each kind and stream advances evenly).
bool draw_repeats(const TapeIR& t, int i, int k, int D) {
  if (t.b[i] != t.b[k]) return false;
  return t.simple_draws ? t.a[k] - t.a[i] == D : t.a[k] > t.a[i];
}

// Node k = i + P repeats node i: same op and literal (any literal when `lit`),
// draw ordinal advanced, each operand either shifted by P (same iteration /
// carried) or unchanged (invariant).
bool repeats(const TapeIR& t, int i, int k, int P, int D, bool lit) {
  const int op = t.op[i];
  if (op != t.op[k] || op == NT_OP_INPUT) return false;
  if (op == NT_OP_CONST) return lit || bits(t.c[i]) == bits(t.c[k]);
  if (is_draw(op)) return draw_repeats(t, i, k, D);
  const int ar = arity(op);
  if (ar >= 1 && !(t.a[k] == t.a[i] + P || t.a[k] == t.a[i])) return false;
  if (ar >= 2 && !(t.b[k] == t.b[i] + P || t.b[k] == t.b[i])) return false;
  return true;
}

// Iteration [s0, s0+P) followed by [s1 = s0+P, ...): like repeats(), except a
// carried operand of the later iteration may come from any node before s0 (the
// carry's initial value).
bool extends(const TapeIR& t, int s0, int P, int D, bool lit) {
  const int s1 = s0 + P;
  for (int j = 0; j < P; ++j) {
    const int i = s0 + j, k = s1 + j;
    const int op = t.op[i];
    if (op != t.op[k] || op == NT_OP_INPUT) return false;
    if (op == NT_OP_CONST) { if (!lit && bits(t.c[i]) != bits(t.c[k])) return false; continue; }
    if (is_draw(op)) { if (!draw_repeats(t, i, k, D)) return false; continue; }
    const int ar = arity(op);
    for (int slot = 0; slot < ar; ++slot) {
      const int xk = slot == 0 ? t.a[k] : t.b[k];
      const int xi = slot == 0 ? t.a[i] : t.b[i];
      if (xk >= s1) { if (xi != xk - P) return false; }
      else if (xk >= s0) { if (xi >= s0) return false; }
      else if (xi != xk) return false;
    }
  }
  return true;
}

enum { V_OK = 0, V_ITER0 = 1, V_EPI = 2, V_FAIL = 3 };

int verify(const TapeIR& t, int s, int P, int iters, int D, bool lit, LoopPlan& L) {
  const int e = s + P * iters;
  L = LoopPlan();
  L.start = s; L.period = P; L.iters = iters; L.draws = D;
  L.kind_a.assign(P, ARG_NONE); L.ref_a.assign(P, -1);
  L.kind_b.assign(P, ARG_NONE); L.ref_b.assign(P, -1);
  L.rand_base.assign(P, -1);
  L.rand_step.assign(P, 0);
  L.carry_init.assign(P, -1);
  L.is_carry.assign(P, 0);
  L.is_liveout.assign(P, 0);
  // classes from iteration 1
  const int s1 = s + P;
  for (int j = 0; j < P; ++j) {
    const int k = s1 + j;
    const int ar = arity(t.op[k]);
    for (int slot = 0; slot < ar; ++slot) {
      const int x = slot == 0 ? t.a[k] : t.b[k];
      int kind, ref;
      if (x >= s1) { kind = ARG_BODY; ref = x - s1; if (ref >= j) return V_FAIL; }
      else if (x >= s) { kind = ARG_CARRY; ref = x - s; }
      else { kind = ARG_INV; ref = x; }
      (slot == 0 ? L.kind_a : L.kind_b)[j] = kind;
      (slot == 0 ? L.ref_a : L.ref_b)[j] = ref;
      if (kind == ARG_CARRY) L.is_carry[ref] = 1;
    }
    if (is_draw(t.op[s + j])) {
      L.rand_base[j] = t.a[s + j];
      L.rand_step[j] = t.a[s1 + j] - t.a[s + j];
      if (L.rand_base[j] < 0 || L.rand_step[j] <= 0 || t.b[s1 + j] != t.b[s + j]) return V_FAIL;
    }
  }
  // every draw of one kind and stream advances by the same step per iteration
  L.normal_step.clear();
  L.need_even = false;
  std::map<std::pair<int, int>, int> step;
  for (int j = 0; j < P; ++j) {
    if (!is_draw(t.op[s + j])) continue;
    const auto key = std::make_pair(t.op[s + j], t.b[s + j]);
    auto it = step.find(key);
    if (it == step.end()) step[key] = L.rand_step[j];
    else if (it->second != L.rand_step[j]) return V_FAIL;
    if (t.op[s + j] == NT_OP_RANDN) {
      L.normal_step[t.b[s + j]] = L.rand_step[j];
      if (L.rand_step[j] & 1) L.need_even = true;
    }
  }
  for (int it = 0; it < iters; ++it) {
    const int fail = it == 0 ? V_ITER0 : V_FAIL;
    for (int j = 0; j < P; ++j) {
      const int i = s + it * P + j;
      const int op = t.op[i];
      if (op != t.op[s1 + j]) return fail;
      if (op == NT_OP_CONST && !lit && bits(t.c[i]) != bits(t.c[s + j])) return fail;
      if (op == NT_OP_INPUT) return fail;
      if (is_draw(op) && (t.b[i] != t.b[s + j] || t.a[i] != L.rand_base[j] + it * L.rand_step[j])) return fail;
      // one body serves every iteration, so activity must not change along the loop
      if (t.active[i] != t.active[s1 + j]) return fail;
      const int ar = arity(op);
      for (int slot = 0; slot < ar; ++slot) {
        const int x = slot == 0 ? t.a[i] : t.b[i];
        const int kind = (slot == 0 ? L.kind_a : L.kind_b)[j];
        const int ref = (slot == 0 ? L.ref_a : L.ref_b)[j];
        if (kind == ARG_BODY) {
          if (x != s + it * P + ref) return fail;
        } else if (kind == ARG_CARRY) {
          if (it > 0) {
            if (x != s + (it - 1) * P + ref) return fail;
          } else {
            if (x >= s) return V_ITER0;
            if (L.carry_init[ref] == -1) L.carry_init[ref] = x;
            else if (L.carry_init[ref] != x) return V_ITER0;
          }
        } else if (x != ref) {
          return fail;
        }
      }
    }
  }
  const int last = s + (iters - 1) * P;
  for (int i = e; i < t.n; ++i) {
    const int ar = arity(t.op[i]);
    for (int slot = 0; slot < ar; ++slot) {
      const int x = slot == 0 ? t.a[i] : t.b[i];
      if (x >= s && x < e) {
        if (x < last) return V_EPI;
        L.is_liveout[x - last] = 1;
      }
    }
  }
  for (int out : t.outputs) {
    if (out >= s && out < e) {
      if (out < last) return V_EPI;
      L.is_liveout[out - last] = 1;
    }
  }
  if (lit) {
    L.lit_table.assign(P, 0);
    L.lit_values.assign(P, {});
    for (int j = 0; j < P; ++j) {
      if (t.op[s + j] != NT_OP_CONST) continue;
      bool same = true;
      for (int it = 1; it < iters && same; ++it) same = bits(t.c[s + it * P + j]) == bits(t.c[s + j]);
      if (same) continue;
      L.lit_table[j] = 1;
      for (int it = 0; it < iters; ++it) L.lit_values[j].push_back(t.c[s + it * P + j]);
    }
  }
  L.found = true;
  return V_OK;
}

}  // namespace

LoopPlan detect_loop(const TapeIR& t, bool lit) {
  std::vector<int> rp;
  for (int i = 0; i < t.n; ++i) {
    if (is_draw(t.op[i])) rp.push_back(i);
  }
  LoopPlan none;
  if (rp.size() < 8) return none;
  const int mid = static_cast<int>(rp.size()) / 2;
  std::vector<std::pair<int, int>> cands;  // (P, D)
  for (int m = 1; m <= 256 && mid + m < static_cast<int>(rp.size()); ++m) {
    const int P = rp[mid + m] - rp[mid];
    if (P * 4 > t.n) break;
    bool seen = false;
    for (auto& c : cands) seen |= c.first == P;
    if (!seen) cands.push_back({P, m});
  }
  int bestX = -1, bestY = -1, bestP = 0, bestD = 0;
  long bestCover = 0;
  for (auto& cd : cands) {
    const int P = cd.first, D = cd.second;
    int runStart = -1;
    for (int i = 0; i + P <= t.n; ++i) {
      const bool ok = i + P < t.n && repeats(t, i, i + P, P, D, lit);
      if (ok && runStart < 0) runStart = i;
      if (!ok && runStart >= 0) {
        const int x = runStart, y = i;
        const long cover = static_cast<long>((y + P - x) / P) * P;
        if (cover > bestCover) { bestCover = cover; bestX = x; bestY = y; bestP = P; bestD = D; }
        runStart = -1;
      }
    }
  }
  if (bestP == 0) return none;
  const int P = bestP, D = bestD;
  int s = bestX;
  for (int j = 0; j < P && bestX + j < t.n; ++j) {
    if (is_draw(t.op[bestX + j])) { s = bestX + j; break; }
  }
  int iters = (bestY + P - s) / P;
  while (s - P >= 0 && extends(t, s - P, P, D, lit)) { s -= P; ++iters; }
  LoopPlan L;
  for (int attempt = 0; attempt < 8 && iters >= 4; ++attempt) {
    const int r = verify(t, s, P, iters, D, lit, L);
    if (r == V_OK) break;
    if (r == V_EPI) { --iters; continue; }
    if (r == V_ITER0) { s += P; --iters; continue; }
    return none;
  }
  if (!L.found || iters < 4 || static_cast<long>(iters) * P < 32) return none;
  return L;
}

TapeIR sink_invariants(const TapeIR& t) {
  const int n = t.n;
  std::vector<uint8_t> drawn(n, 0), output(n, 0);
  for (int out : t.outputs) output[out] = 1;
  for (int i = 0; i < n; ++i) {
    const int op = t.op[i];
    const int ar = arity(op);
    drawn[i] = is_draw(op) || (ar >= 1 && drawn[t.a[i]]) || (ar >= 2 && drawn[t.b[i]]);
  }
  auto deferred = [&](int i) { return !drawn[i] && t.op[i] != NT_OP_INPUT && !output[i]; };
  std::vector<int> order;
  order.reserve(n);
  std::vector<uint8_t> placed(n, 0);
  std::vector<std::pair<int, int>> stack;  // (node, operands visited)
  auto place = [&](int root) {
    if (placed[root]) return;
    stack.push_back({root, 0});
    while (!stack.empty()) {
      auto& top = stack.back();
      const int i = top.first;
      const int ar = arity(t.op[i]);
      if (top.second < ar) {
        const int x = top.second == 0 ? t.a[i] : t.b[i];
        ++top.second;
        if (!placed[x]) stack.push_back({x, 0});
        continue;
      }
      stack.pop_back();
      if (!placed[i]) {
        placed[i] = 1;
        order.push_back(i);
      }
    }
  };
  for (int i = 0; i < n; ++i) {
    if (!deferred(i)) place(i);
  }
  for (int i = 0; i < n; ++i) place(i);  // what nothing else reads
  std::vector<int> at(n);
  for (int k = 0; k < n; ++k) at[order[k]] = k;
  TapeIR r = t;
  for (int k = 0; k < n; ++k) {
    const int i = order[k];
    const int op = t.op[i];
    const int ar = arity(op);
    r.op[k] = op;
    r.c[k] = t.c[i];
    r.a[k] = ar >= 1 ? at[t.a[i]] : t.a[i];
    r.b[k] = ar >= 2 ? at[t.b[i]] : t.b[i];
    r.active[k] = t.active[i];
  }
  for (int j = 0; j < t.n_in; ++j) r.input_node[j] = at[t.input_node[j]];
  for (size_t o = 0; o < t.outputs.size(); ++o) r.outputs[o] = at[t.outputs[o]];
  r.output = r.outputs[0];
  return r;
}

// ---- plan ----------------------------------------------------------------------

namespace {
int plan_reverse_loop(const TapeIR& t, const nt_options& o, Plan& p, std::string& err);
bool wants_line_segments(const TapeIR& t, const nt_options& o, const Plan& p);
void plan_line_segments(const TapeIR& t, const nt_options& o, Plan& p);
void choose_mode(const TapeIR& t, const nt_options& o, Plan& p);
double fwd_cost(int op, bool f32);
double store_cost(bool f32);
}  // namespace

int make_plan(TapeIR& t, const nt_options* opt, Plan& p, std::string& err) {
  nt_options o{};
  if (opt) o = *opt;
  p = Plan();
  p.precision = o.precision == NT_FP32 ? NT_FP32 : NT_FP64;
  if (o.precision != NT_FP32 && o.precision != NT_FP64) { err = "precision must be NT_FP64 or NT_FP32"; return NT_E_INVALID; }
  p.adjoints = o.adjoints != 0;
  // fp64 defaults to no contraction: the oracle rounds every product and sum
  // separately, and over 500-step tapes fused rounding alone moves adjoints by
  // ~5e-12 relative. fp32 is compared at aggregate level and keeps FMAs.
  p.contract = o.contract > 0 || (o.contract == 0 && p.precision == NT_FP32);
  p.fuse = o.contract >= 0;
  p.libm = (o.libm == 1 || o.libm == 2) ? o.libm : 0;
  p.block = o.block > 0 ? o.block : 256;
  if (p.block % 64 != 0 || p.block > 1024) { err = "block must be a multiple of 64, at most 1024"; return NT_E_INVALID; }
  p.n_channels = static_cast<int>(t.outputs.size()) * (2 + t.n_in);
  if (o.checkpoint < NT_CKPT_AUTO || o.checkpoint > NT_CKPT_STORE_ALL) { err = "unknown checkpoint policy"; return NT_E_INVALID; }
  if (o.seg_len < 0) { err = "seg_len must be >= 0"; return NT_E_INVALID; }
  if (o.mode < NT_MODE_AUTO || o.mode > NT_MODE_TANGENT) { err = "unknown derivative mode"; return NT_E_INVALID; }
  if (o.markets < 0 || o.markets > 64) { err = "markets must be between 1 and 64"; return NT_E_INVALID; }
  p.markets = std::max(1, o.markets);
  if (o.waves < 0 || o.waves > 8) { err = "waves must be between 0 and 8"; return NT_E_INVALID; }
  p.waves = o.waves;
  if (o.basis < 0 || o.basis > 2) { err = "basis must be 0, 1 or 2"; return NT_E_INVALID; }
  p.basis = o.basis;
  if (p.markets > 1 && o.mode == NT_MODE_REVERSE) {
    err = "several markets per dispatch share draws in tangent mode only";
    return NT_E_INVALID;
  }
  if (t.outputs.size() > 1 && o.mode == NT_MODE_REVERSE && o.adjoints) {
    err = "the reverse sweep follows one output; a multi-output tape takes tangent mode";
    return NT_E_UNSUPPORTED;
  }
  if (o.roll >= 0) {
    p.loop = detect_loop(t);
    const long cover = p.loop.found ? static_cast<long>(p.loop.period) * p.loop.iters : 0;
    if (2 * cover < t.n) {
      // No exactly repeating step covers most of the tape: the step's schedule
      // (per-step fractions, drifts, volatilities) may have been recorded up
      // front. Moved next to the steps that read it, with per-step literals
      // read from a table, it can make the step repeat.
      TapeIR sunk = sink_invariants(t);
      LoopPlan L = detect_loop(sunk, true);
      if (L.found && static_cast<long>(L.period) * L.iters > cover) {
        t = std::move(sunk);
        p.loop = std::move(L);
      }
    }
  }
  if (p.loop.found) {
    const int rc = plan_reverse_loop(t, o, p, err);
    if (rc != NT_OK) return rc;
  } else if (wants_line_segments(t, o, p)) {
    plan_line_segments(t, o, p);
    if (p.kf + p.ka > 16) {
      // Values that depend on no draw (a step schedule recorded up front)
      // are carried from where they are computed to where they are read;
      // moved next to their readers, they may not cross a boundary at all.
      TapeIR sunk = sink_invariants(t);
      Plan q = p;
      plan_line_segments(sunk, o, q);
      if (q.kf + q.ka < p.kf + p.ka) {
        t = std::move(sunk);
        p = std::move(q);
      }
    }
  }
  choose_mode(t, o, p);
  return NT_OK;
}

namespace {

int plan_reverse_loop(const TapeIR& t, const nt_options& o, Plan& p, std::string& err) {
  LoopPlan& L = p.loop;
  const int P = L.period, s = L.start;
  p.taped.assign(P, 0);
  p.stored.assign(P, 0);
  p.store_index.assign(P, -1);
  auto body_active = [&](int j) { return t.active[s + j] != 0; };
  std::vector<uint8_t> carry_read(P, 0);  // a rule reads the carried value (its checkpoint in a segment's first iteration)
  auto mark = [&](int kind, int ref) {
    if (kind == ARG_BODY || kind == ARG_CARRY) p.taped[ref] = 1;
    if (kind == ARG_CARRY) carry_read[ref] = 1;
  };
  if (p.adjoints) {
    for (int j = 0; j < P; ++j) {
      if (!body_active(j)) continue;
      const int op = t.op[s + j];
      auto opActive = [&](int kind, int ref) {
        if (kind == ARG_INV) return t.active[ref] != 0;
        if (kind == ARG_BODY || kind == ARG_CARRY) return body_active(ref);
        return false;
      };
      const bool aa = opActive(L.kind_a[j], L.ref_a[j]);
      const bool ba = opActive(L.kind_b[j], L.ref_b[j]);
      switch (op) {
        case NT_OP_MUL:
          if (aa) mark(L.kind_b[j], L.ref_b[j]);
          if (ba) mark(L.kind_a[j], L.ref_a[j]);
          break;
        case NT_OP_DIV:
          mark(L.kind_b[j], L.ref_b[j]);
          if (ba) p.taped[j] = 1;
          break;
        case NT_OP_EXP: case NT_OP_SQRT: p.taped[j] = 1; break;
        case NT_OP_LOG: case NT_OP_ABS: mark(L.kind_a[j], L.ref_a[j]); break;
        case NT_OP_MAX: case NT_OP_MIN:
          mark(L.kind_a[j], L.ref_a[j]);
          mark(L.kind_b[j], L.ref_b[j]);
          break;
        default: break;
      }
    }
  }
  for (int j = 0; j < P; ++j) {
    if (L.is_carry[j]) p.carries.push_back(j);
  }
  int ck = o.checkpoint;
  // Inactive values that feed active body nodes (the draw-derived frontier).
  std::vector<uint8_t> frontier(P, 0);
  bool anyFrontier = false;
  for (int j = 0; j < P && p.adjoints; ++j) {
    if (!body_active(j)) continue;
    for (int slot = 0; slot < arity(t.op[s + j]); ++slot) {
      const int kind = slot == 0 ? L.kind_a[j] : L.kind_b[j];
      const int ref = slot == 0 ? L.ref_a[j] : L.ref_b[j];
      if ((kind == ARG_BODY || kind == ARG_CARRY) && !body_active(ref) && t.op[s + ref] != NT_OP_CONST) {
        frontier[ref] = 1;
        anyFrontier = true;
      }
    }
  }
  if (ck == NT_CKPT_AUTO) {
    // Store the frontier only when recomputing the inactive part of a step
    // costs more than writing and re-reading its frontier values through HBM
    // (measured on MI355X: about 48 VALU instructions' worth per 4 bytes at
    // the replay's rate). With the skeleton's own Box-Muller a draw costs ~30
    // (fp64), so GBM steps recompute their normals (C2 fp64: 2.1 ms against
    // 2.7 ms storing them; C5 fp32, 16 correlated normals: 8.5 against 11.6).
    const bool f32 = p.precision == NT_FP32;
    double recompute = 0;
    int nf = 0;
    for (int j = 0; j < P; ++j) {
      if (!body_active(j)) recompute += fwd_cost(t.op[s + j], f32);
      nf += frontier[j];
    }
    ck = anyFrontier && store_cost(f32) * nf < recompute ? NT_CKPT_STORE_DRAWS : NT_CKPT_RECOMPUTE;
  }
  if (!p.adjoints) ck = NT_CKPT_RECOMPUTE;
  p.ckpt = ck;
  if (p.adjoints && ck == NT_CKPT_STORE_DRAWS) {
    p.stored = frontier;
  } else if (p.adjoints && ck == NT_CKPT_STORE_ALL) {
    for (int j = 0; j < P; ++j) p.stored[j] = p.taped[j] && t.op[s + j] != NT_OP_CONST;
  }
  for (int j = 0; j < P; ++j) {
    if (p.stored[j]) p.store_index[j] = p.n_stored++;
  }
  // What a segment's recompute must produce: the values the rules read and,
  // to a fixed point, what those are computed from (a carried operand is the
  // previous iteration's value of its position, or the segment's checkpoint).
  p.rneed = p.taped;
  for (bool changed = true; changed;) {
    changed = false;
    for (int j = P - 1; j >= 0; --j) {
      if (!p.rneed[j] || p.stored[j]) continue;
      for (int slot = 0; slot < arity(t.op[s + j]); ++slot) {
        const int kind = slot == 0 ? L.kind_a[j] : L.kind_b[j];
        const int ref = slot == 0 ? L.ref_a[j] : L.ref_b[j];
        if (kind != ARG_BODY && kind != ARG_CARRY) continue;
        if (kind == ARG_CARRY) carry_read[ref] = 1;
        if (!p.rneed[ref]) {
          p.rneed[ref] = 1;
          changed = true;
        }
      }
    }
  }
  for (int c : p.carries) {
    if (carry_read[c]) p.ck_carries.push_back(c);
  }
  // Iterations per segment: the recompute keeps every taped value of the
  // segment in registers, so size it against a VGPR budget.
  int taped = 0;
  for (int j = 0; j < P; ++j) taped += p.taped[j];
  const int w = p.precision == NT_FP64 ? 2 : 1;
  int seg;
  if (o.seg_len > 0) {
    seg = o.seg_len;
  } else if (!p.adjoints) {
    seg = 4;
  } else {
    seg = std::max(1, 96 / std::max(1, taped * w));
  }
  seg = std::max(1, std::min({seg, L.iters, 64}));
  if (L.need_even && (seg & 1)) seg = seg > 1 ? seg - 1 : 2;
  seg = std::min(seg, L.iters);
  if (o.seg_len <= 0) {
    for (int cand = seg; cand >= std::max(1, seg / 2); --cand) {
      if (L.iters % cand == 0 && (!L.need_even || !(cand & 1))) { seg = cand; break; }
    }
  }
  if (L.need_even && (seg & 1)) {
    err = "an odd seg_len needs an even number of normal draws per iteration in every stream";
    return NT_E_INVALID;
  }
  p.seg = seg;
  p.nseg_full = L.iters / seg;
  p.tail = L.iters % seg;
  const int segments = p.nseg_full + (p.tail ? 1 : 0);
  p.ck_slots = p.adjoints ? segments * static_cast<int>(p.ck_carries.size()) : 0;
  p.tape_slots = p.ck_slots + L.iters * p.n_stored;
  return NT_OK;
}

// Input dependency sets: INPUT j -> {j}; CONST and draws -> {}; otherwise the
// union over the operands. A node is active exactly when its set is non-empty.
void compute_deps(const TapeIR& t, Plan& p) {
  const int W = std::max(1, (t.n_in + 63) / 64);
  p.n_words = W;
  p.deps.assign(static_cast<size_t>(t.n) * W, 0);
  for (int i = 0; i < t.n; ++i) {
    uint64_t* d = &p.deps[static_cast<size_t>(i) * W];
    const int op = t.op[i];
    if (op == NT_OP_INPUT) {
      d[t.a[i] >> 6] |= uint64_t{1} << (t.a[i] & 63);
      continue;
    }
    const int ar = arity(op);
    for (int slot = 0; slot < ar; ++slot) {
      const uint64_t* x = &p.deps[static_cast<size_t>(slot == 0 ? t.a[i] : t.b[i]) * W];
      for (int w = 0; w < W; ++w) d[w] |= x[w];
    }
  }
  p.posdeps.clear();
  if (!p.loop.found) return;
  const LoopPlan& L = p.loop;
  p.posdeps.assign(static_cast<size_t>(L.period) * W, 0);
  for (int it = 0; it < L.iters; ++it) {
    for (int j = 0; j < L.period; ++j) {
      const uint64_t* x = &p.deps[static_cast<size_t>(L.start + it * L.period + j) * W];
      for (int w = 0; w < W; ++w) p.posdeps[static_cast<size_t>(j) * W + w] |= x[w];
    }
  }
}

int popcount(const uint64_t* x, int W) {
  int n = 0;
  for (int w = 0; w < W; ++w) n += __builtin_popcountll(x[w]);
  return n;
}

// Estimated VALU instructions per lane (fp64 weights; fp32 scales them alike,
// except for draws, whose fp32 transcendentals are single instructions).
double fwd_cost(int op, bool f32) {
  switch (op) {
    case NT_OP_ADD: case NT_OP_SUB: case NT_OP_MUL: return 1;
    case NT_OP_MAX: case NT_OP_MIN: return 1;
    case NT_OP_DIV: return 10;
    case NT_OP_EXP: case NT_OP_LOG: return 20;
    case NT_OP_SQRT: return 8;
    case NT_OP_RANDN: return f32 ? 15 : 30;  // half a Box-Muller pair with its Philox block
    case NT_OP_RANDU: return 12;             // one Philox block
    default: return 0;
  }
}

// One value per iteration stored in the forward pass and read back in the
// reverse sweep, in VALU instructions' worth (the HBM round trip dominates).
double store_cost(bool f32) { return f32 ? 48 : 96; }

// ---- checkpointed straight line ----
//
// A tape with no rolled loop is one basic block: its reverse sweep reads
// forward values from the whole tape, so the kernel keeps O(n) of them live
// and spills once they exceed the register file. Cut into segments (the
// reference's segment-checkpoint plan, AadCheckpointPlan.java:95-172: about
// sqrt(n) nodes each, at least 48, for tapes over 512 nodes,
// DeviceAadExecutable.java:92), the forward pass keeps only what the next
// segments read, and the reverse recomputes one segment at a time before its
// rules, so the live set is one segment's plus the values crossing its start.
// Unlike the reference, which saves every value crossing each boundary once
// per boundary, a value is stored once, in its own slot, and read back only
// by the segments whose reverse needs it; constants and inputs are never
// stored (they are re-emitted), and each boundary moves by up to a quarter
// segment to where the fewest values cross it.

constexpr int kLineMinNodes = 512;

int line_seg_len(const TapeIR& t, const nt_options& o) {
  if (o.seg_len > 0) return std::max(4, o.seg_len);
  return std::max(48, static_cast<int>(std::lround(std::sqrt(static_cast<double>(t.n)))));
}

bool rematerialized(const TapeIR& t, int i) { return t.op[i] == NT_OP_CONST || t.op[i] == NT_OP_INPUT; }

// seg_len > 0 asks for segments of that many nodes on any tape of two or more.
bool wants_line_segments(const TapeIR& t, const nt_options& o, const Plan& p) {
  if (p.loop.found || !p.adjoints || p.markets > 1 || t.outputs.size() > 1) return false;
  if (o.checkpoint == NT_CKPT_STORE_ALL || o.mode == NT_MODE_TANGENT || !t.active[t.output]) return false;
  if (o.seg_len <= 0 && t.n <= kLineMinNodes) return false;
  return t.n >= 2 * line_seg_len(t, o);
}

// Operand values the reverse rule of active node i reads (the rules of
// rev_rules): bit 0 operand a, bit 1 operand b, bit 2 the node's own value.
int rule_reads(const TapeIR& t, int i) {
  const int op = t.op[i];
  const int ar = arity(op);
  const bool aa = ar >= 1 && t.active[t.a[i]];
  const bool ba = ar >= 2 && t.active[t.b[i]];
  switch (op) {
    case NT_OP_MUL: return (aa ? 2 : 0) | (ba ? 1 : 0);
    case NT_OP_DIV: return (aa ? 2 : 0) | (ba ? 6 : 0);
    case NT_OP_EXP: case NT_OP_SQRT: return aa ? 4 : 0;
    case NT_OP_LOG: case NT_OP_ABS: return aa ? 1 : 0;
    case NT_OP_MAX: case NT_OP_MIN: return (aa || ba) ? 3 : 0;
    default: return 0;
  }
}

// Slots for values carried across segment boundaries: node x occupies one
// over boundaries lo[x] .. hi[x] (boundary k sits before segment k); nodes
// come in order of lo, so taking the lowest free slot colours the intervals
// with as many slots as the most that overlap. Returns the slot count.
int colour_intervals(const std::vector<int>& lo, const std::vector<int>& hi, std::vector<int>& slot) {
  const int n = static_cast<int>(lo.size());
  slot.assign(n, -1);
  std::vector<int> busy_until;  // per slot: the last boundary its node occupies
  for (int x = 0; x < n; ++x) {
    if (lo[x] > hi[x]) continue;
    int k = 0;
    while (k < static_cast<int>(busy_until.size()) && busy_until[k] >= lo[x]) ++k;
    if (k == static_cast<int>(busy_until.size())) busy_until.push_back(0);
    busy_until[k] = hi[x];
    slot[x] = k;
  }
  return static_cast<int>(busy_until.size());
}

void plan_line_segments(const TapeIR& t, const nt_options& o, Plan& p) {
  const int n = t.n, len = line_seg_len(t, o);
  // cross[b]: values other than constants and inputs defined before b and
  // read at or after b
  std::vector<int> last(n, -1);
  for (int j = 0; j < n; ++j) {
    const int ar = arity(t.op[j]);
    if (ar >= 1) last[t.a[j]] = std::max(last[t.a[j]], j);
    if (ar >= 2) last[t.b[j]] = std::max(last[t.b[j]], j);
  }
  std::vector<int> cross(n + 1, 0);
  for (int i = 0; i < n; ++i) {
    if (rematerialized(t, i) || last[i] <= i) continue;
    cross[i + 1] += 1;
    if (last[i] + 1 <= n) cross[last[i] + 1] -= 1;
  }
  for (int b = 1; b <= n; ++b) cross[b] += cross[b - 1];
  const int S = (n + len - 1) / len;
  std::vector<int> bound{0};
  for (int s = 1; s < S; ++s) {
    const int nominal = s * len;
    const int lo = std::max(bound.back() + 1, nominal - len / 4), hi = std::min(n - 1, nominal + len / 4);
    int best = std::max(lo, std::min(nominal, hi));
    for (int b = lo; b <= hi; ++b) {
      if (cross[b] < cross[best] || (cross[b] == cross[best] && std::abs(b - nominal) < std::abs(best - nominal))) best = b;
    }
    bound.push_back(best);
  }
  bound.push_back(n);
  std::vector<int>& seg_of = p.lseg;
  seg_of.assign(n, 0);
  for (int s = 0; s < S; ++s) {
    for (int i = bound[s]; i < bound[s + 1]; ++i) seg_of[i] = s;
  }
  // forward: a value read by a later segment is carried from its own
  // segment's end to its last reader's start
  std::vector<int> flo(n, 1), fhi(n, 0), alo(n, 1), ahi(n, -1);
  for (int x = 0; x < n; ++x) {
    if (rematerialized(t, x) || last[x] < 0 || seg_of[last[x]] == seg_of[x]) continue;
    flo[x] = seg_of[x] + 1;
    fhi[x] = seg_of[last[x]];
  }
  // reverse: the adjoint of x is carried from its last active reader in a
  // later segment down to its own segment
  for (int i = 0; i < n; ++i) {
    if (!t.active[i]) continue;
    const int ar = arity(t.op[i]);
    for (int k = 0; k < ar; ++k) {
      const int x = k == 0 ? t.a[i] : t.b[i];
      if (t.active[x] && t.op[x] != NT_OP_INPUT && seg_of[i] > seg_of[x]) ahi[x] = std::max(ahi[x], seg_of[i]);
    }
  }
  std::vector<int> ahi_c(n, 0);  // alo > ahi_c: not carried
  for (int x = 0; x < n; ++x) {
    if (ahi[x] >= 0) {
      alo[x] = seg_of[x] + 1;
      ahi_c[x] = ahi[x];
    } else {
      ahi[x] = seg_of[x];
    }
  }
  p.kf = colour_intervals(flo, fhi, p.fslot);
  p.ka = colour_intervals(alo, ahi_c, p.aslot);
  p.ahi = ahi;
  // reverse recompute: what each segment's rules read, and what computing
  // those reads
  p.lneed.assign(n, 0);
  p.lslot.assign(n, -1);
  p.lin.assign(S, {});
  std::vector<uint8_t> stored(n, 0);
  for (int s = 0; s < S; ++s) {
    const int lo = bound[s], hi = bound[s + 1];
    std::vector<uint8_t> in(lo, 0);
    auto need = [&](int x) {
      if (x >= lo) p.lneed[x] = 1;
      else in[x] = 1;
    };
    for (int i = hi - 1; i >= lo; --i) {
      const int ar = arity(t.op[i]);
      if (t.active[i] && ar > 0) {
        const int r = rule_reads(t, i);
        if (r & 1) need(t.a[i]);
        if (r & 2) need(t.b[i]);
        if (r & 4) need(i);
      }
      if (p.lneed[i] && ar >= 1) need(t.a[i]);
      if (p.lneed[i] && ar >= 2) need(t.b[i]);
    }
    for (int x = 0; x < lo; ++x) {
      if (!in[x]) continue;
      p.lin[s].push_back(x);
      if (!rematerialized(t, x)) stored[x] = 1;
    }
  }
  int slots = 0;
  for (int i = 0; i < n; ++i) {
    if (stored[i]) p.lslot[i] = slots++;
  }
  p.lbound = std::move(bound);
  p.seg = len;
  p.nseg_full = S;
  p.tail = 0;
  p.ckpt = NT_CKPT_RECOMPUTE;
  p.ck_slots = p.tape_slots = slots;
}

double rev_cost(int op, bool aa, bool ba) {
  const double A = aa ? 1 : 0, B = ba ? 1 : 0;
  switch (op) {
    case NT_OP_ADD: case NT_OP_SUB: return A + B;
    case NT_OP_MUL: return 2 * (A + B);
    case NT_OP_DIV: return 11 * A + 13 * B;
    case NT_OP_NEG: return A;
    case NT_OP_EXP: return 2 * A;
    case NT_OP_LOG: return 11 * A;
    case NT_OP_SQRT: return 12 * A;
    case NT_OP_ABS: return 3 * A;
    case NT_OP_MAX: case NT_OP_MIN: return 3 * (A + B);
    default: return 0;
  }
}

// Extra work of one active node in tangent mode: per dependency j, the local
// rule; once per node, the factor it shares across j (a reciprocal, a sign, a
// branch condition).
double tan_cost(const TapeIR& t, const Plan& p, int i) {
  const int W = p.n_words;
  const int op = t.op[i];
  const int ar = arity(op);
  if (ar == 0) return 0;
  const uint64_t* da = &p.deps[static_cast<size_t>(t.a[i]) * W];
  const uint64_t* db = ar >= 2 ? &p.deps[static_cast<size_t>(t.b[i]) * W] : nullptr;
  double c = 0;
  for (int w = 0; w < W; ++w) {
    const uint64_t a = da[w], b = db ? db[w] : 0;
    const double both = __builtin_popcountll(a & b), any = __builtin_popcountll(a | b);
    switch (op) {
      case NT_OP_ADD: case NT_OP_SUB: c += both; break;
      case NT_OP_MUL: c += any + both; break;
      case NT_OP_DIV: c += any + both; break;
      case NT_OP_NEG: break;
      case NT_OP_MAX: case NT_OP_MIN: c += 2 * any; break;
      default: c += any; break;
    }
  }
  switch (op) {
    case NT_OP_DIV: c += 11; break;
    case NT_OP_LOG: case NT_OP_SQRT: c += 10; break;
    case NT_OP_ABS: case NT_OP_MAX: case NT_OP_MIN: c += 1; break;
    default: break;
  }
  return c;
}

void choose_mode(const TapeIR& t, const nt_options& o, Plan& p) {
  p.mode = NT_MODE_REVERSE;
  const bool multi = t.outputs.size() > 1;
  double fwd = 0;
  for (int i = 0; i < t.n; ++i) fwd += fwd_cost(t.op[i], p.precision == NT_FP32);
  p.path_cost = fwd;
  p.cost_forward = fwd;
  // Price only: the tangent frame with no tangents, the frame several input
  // sets per dispatch take, so one set and several give the same bits and a
  // price-only executable shares each path's draws across input sets. Forcing
  // the reverse sweep keeps the step-by-step forward of the reverse frame.
  const bool price_only = !p.adjoints;
  if (price_only && o.mode == NT_MODE_REVERSE && p.markets == 1 && !multi) return;
  compute_deps(t, p);
  const LoopPlan& L = p.loop;
  const int le = L.found ? L.end() : 0;
  const bool f32 = p.precision == NT_FP32;
  double rev = 0, tan = 0;
  for (int i = 0; i < t.n; ++i) {
    const int ar = arity(t.op[i]);
    const bool inLoop = L.found && i >= L.start && i < le;
    if (inLoop && p.ckpt == NT_CKPT_RECOMPUTE && !t.active[i]) rev += fwd_cost(t.op[i], f32);
    if (!t.active[i] || ar == 0) continue;
    const bool aa = t.active[t.a[i]] != 0;
    const bool ba = ar >= 2 && t.active[t.b[i]] != 0;
    rev += rev_cost(t.op[i], aa, ba);
    if (inLoop && p.ckpt != NT_CKPT_STORE_ALL) rev += fwd_cost(t.op[i], f32);  // the reverse recomputes it
    tan += tan_cost(t, p, i);
  }
  if (L.found) rev += store_cost(f32) * L.iters * p.n_stored;
  if (!p.lbound.empty()) {
    // the checkpointed straight line recomputes every segment once and
    // stores each crossing value once
    for (int i = 0; i < t.n; ++i) rev += fwd_cost(t.op[i], f32);
    rev += store_cost(f32) * p.tape_slots;
  }
  p.cost_reverse = rev;
  p.cost_tangent = tan;
  // Several markets per dispatch are priced in tangent mode (also price-only:
  // the tangent frame without tangents).
  // Several outputs get their Jacobian rows from one tangent sweep (the
  // reverse sweep here follows one output).
  // Per estimated instruction, a reverse-sweep kernel takes about twice a
  // tangent kernel's time on MI355X: it holds a segment's values, its
  // adjoints and the accumulators at once (more VGPRs, fewer resident waves)
  // and stores and reloads checkpoints. Measured time over (forward +
  // estimate), reverse against tangent: 1.9-2.2 near the modes' crossover on
  // the local-volatility Asian (8 to 16 coefficients), 1.3-1.7 on C2-C4.
  constexpr double kReverseTime = 2.0;
  const bool tangent = o.mode == NT_MODE_TANGENT || p.markets > 1 || multi || price_only ||
                       (p.adjoints && o.mode == NT_MODE_AUTO && fwd + tan < kReverseTime * (fwd + rev));
  p.path_cost = fwd + (price_only ? 0.0 : tangent ? tan : rev);
  if (!tangent) return;
  p.mode = NT_MODE_TANGENT;
  p.ckpt = 0;
  p.stored.assign(p.stored.size(), 0);
  p.store_index.assign(p.store_index.size(), -1);
  p.n_stored = 0;
  p.ck_slots = p.tape_slots = 0;
  p.lbound.clear();
  p.lseg.clear();
  p.lslot.clear();
  p.fslot.clear();
  p.aslot.clear();
  p.ahi.clear();
  p.lneed.clear();
  p.lin.clear();
  p.kf = p.ka = 0;
  if (!L.found) {
    p.seg = p.nseg_full = p.tail = 0;
    return;
  }
  // Iterations per loop trip, by the registers the carried state and its
  // tangents hold (always an even count when a step draws an odd number of
  // normals, so both Box-Muller legs stay in one trip). Longer trips let the
  // scheduler overlap one step's Philox and transcendental latency with its
  // neighbour's arithmetic; shorter ones keep occupancy when the state is
  // large. Measured on MI355X: Asian fp32 (10 registers of state) 2 and 4
  // steps tie and 8 is 7% slower; barrier fp32 2 beat 4 by 2%; Asian fp64
  // (20) 2 beat 4 by 2.5%; barrier fp64 2 beat 4 by 5%; the 16-asset
  // worst-of (65 fp32, 130 fp64) 1 beat 2 by 9% (fp32) and 5% (fp64).
  const int W = p.n_words;
  int live = 0;
  for (int j = 0; j < L.period; ++j) {
    if (L.is_carry[j] || L.is_liveout[j]) live += 1 + popcount(&p.posdeps[static_cast<size_t>(j) * W], W);
  }
  const int w = p.precision == NT_FP64 ? 2 : 1;
  const int regs = live * w * p.markets;
  int seg = o.seg_len > 0 ? o.seg_len : (regs <= 8 ? 4 : regs <= 48 ? 2 : 1);
  if (L.need_even && (seg & 1)) seg += 1;
  seg = std::max(1, std::min(seg, L.iters));
  p.seg = seg;
  p.nseg_full = L.iters / seg;
  p.tail = L.iters % seg;
}

}  // namespace

// ---- emission --------------------------------------------------------------------

namespace {

class Emitter {
 public:
  Emitter(const TapeIR& t, const Plan& p) : t_(t), p_(p), f32_(p.precision == NT_FP32), L_(p.loop) {}

  std::string run();

 private:
  const TapeIR& t_;
  const Plan& p_;
  const bool f32_;
  const LoopPlan& L_;
  std::ostringstream o_;
  // (stream, Philox counter) -> pair variable stem, per straight-line region
  std::map<std::pair<int, int>, std::string> pairs_;

  // Counter high word of a stream: the path's for stream 0, xor s * 0x9E3779B1
  // for stream s (Philox.java:44-52); declared once per path.
  // key_ names the copies of the Philox key that a recomputed segment of a
  // checkpointed straight line draws from ("" elsewhere).
  std::string key_;
  std::string rhi(int stream) const { return (stream == 0 ? std::string("rhi") : "rhi" + std::to_string(stream)) + key_; }
  std::string rlo() const { return "rlo" + key_; }
  std::string uniform_call(int stream, const std::string& ordinal) const {
    return std::string(f32_ ? "nt_uniformf" : "nt_uniform") + "(" + rlo() + ", " + rhi(stream) + ", " + ordinal + ")";
  }

  std::string lit(double v) const {
    char buf[64];
    if (f32_) {
      float f = static_cast<float>(v);
      if (std::isnan(f)) return "__builtin_nanf(\"\")";
      if (std::isinf(f)) return f > 0 ? "__builtin_inff()" : "(-__builtin_inff())";
      std::snprintf(buf, sizeof buf, "%af", static_cast<double>(f));
    } else {
      if (std::isnan(v)) return "__builtin_nan(\"\")";
      if (std::isinf(v)) return v > 0 ? "__builtin_inf()" : "(-__builtin_inf())";
      std::snprintf(buf, sizeof buf, "%a", v);
    }
    return std::string("(") + buf + ")";
  }
  std::string f(const char* name) const { return f32_ ? std::string(name) + "f" : std::string(name); }
  // Type of tangents and of their scale factors: the re-evaluation pass uses
  // strong-zero numbers (a product with an exact zero is zero, whatever the
  // other factor), the tangent-mode image of the oracle skipping nodes whose
  // adjoint is zero; the fast pass plain IEEE.
  std::string treal() const { return slow_ ? (f32_ ? "nt_szf" : "nt_sz") : "real"; }

  // fp64 Box-Muller and exp read LDS tables that each block loads first.
  bool needs_tables() const {
    if (f32_) return false;
    for (int i = 0; i < t_.n; ++i) {
      if (t_.op[i] == NT_OP_RANDN || t_.op[i] == NT_OP_EXP || t_.op[i] == NT_OP_LOG) return true;
    }
    return false;
  }

  // `node`: the tape node (its first iteration, in a step loop), which tells
  // whether an operand of MAX or MIN is a literal.
  std::string expr(int op, const std::string& x, const std::string& y, double c, int a, int node = -1) const {
    switch (op) {
      case NT_OP_CONST: return lit(c);
      case NT_OP_INPUT: return "in" + std::to_string(a) + ms(true) + in_sfx_;
      case NT_OP_ADD: return x + " + " + y;
      case NT_OP_SUB: return x + " - " + y;
      case NT_OP_MUL: return x + " * " + y;
      case NT_OP_DIV: return f32_ ? x + " * nt_rcpf(" + y + ")" : x + " / " + y;
      case NT_OP_NEG: return "-" + x;
      case NT_OP_EXP:
        if (f32_) return "nt_expf(" + x + ")";
        if (p_.libm == 1 || slow_) return "exp(" + x + ")";
        return "nt_exp_fast(" + x + ", nt_slow" + ms(exp_active_) + ")";
      case NT_OP_LOG:
        if (f32_) return "(nt_hw_log2f(" + x + ") * 0.693147180559945309f)";
        if (p_.libm == 1 || slow_) return "log(" + x + ")";
        return "nt_log_fast(" + x + ", nt_slow" + ms(exp_active_) + ")";
      case NT_OP_SQRT: return f32_ ? "nt_hw_sqrtf(" + x + ")" : "sqrt(" + x + ")";
      case NT_OP_ABS: return f("fabs") + "(" + x + ")";
      case NT_OP_MAX:
      case NT_OP_MIN: {
        const char* name = op == NT_OP_MAX ? "nt_max" : "nt_min";
        if (!max_fast(op) || slow_) return f(name) + "(" + x + ", " + y + ")";
        const bool a_lit = node >= 0 && t_.op[t_.a[node]] == NT_OP_CONST;
        const bool b_lit = node >= 0 && t_.op[t_.b[node]] == NT_OP_CONST;
        if (b_lit && !a_lit) return std::string(name) + "_lit(" + x + ", " + y + ")";
        if (a_lit && !b_lit) return std::string(name) + "_lit(" + y + ", " + x + ")";
        return std::string(name) + "_fast(" + x + ", " + y + ")";
      }
      default: return "0";
    }
  }

  // Reverse rule of one active node (CudaAadCodegen.java:386-448, ScalarReplay.java:129-166);
  // Aa / Ab are empty when that operand is inactive.
  // In the re-evaluation pass a node's rules run only when its adjoint is
  // nonzero, as the oracle skips it (ScalarReplay.java:134-136): an infinite
  // or NaN local derivative under a zero adjoint then contributes nothing.
  void rev(const std::string& ind, int op, const std::string& Ai, const std::string& Vi, const std::string& Va,
           const std::string& Vb, const std::string& Aa, const std::string& Ab) {
    const std::string zero = f32_ ? "0.0f" : "0.0";
    if (!slow_ || (Aa.empty() && Ab.empty())) {
      rev_rules(ind, op, Ai, Vi, Va, Vb, Aa, Ab);
      return;
    }
    o_ << ind << "if (" << Ai << " != " << zero << ") {\n";
    rev_rules(ind + "  ", op, Ai, Vi, Va, Vb, Aa, Ab);
    o_ << ind << "}\n";
  }
  void rev_rules(const std::string& ind, int op, const std::string& Ai, const std::string& Vi, const std::string& Va,
                 const std::string& Vb, const std::string& Aa, const std::string& Ab) {
    const std::string half = f32_ ? "0.5f" : "0.5";
    const std::string zero = f32_ ? "0.0f" : "0.0";
    switch (op) {
      case NT_OP_ADD:
        if (!Aa.empty()) o_ << ind << Aa << " += " << Ai << ";\n";
        if (!Ab.empty()) o_ << ind << Ab << " += " << Ai << ";\n";
        break;
      case NT_OP_SUB:
        if (!Aa.empty()) o_ << ind << Aa << " += " << Ai << ";\n";
        if (!Ab.empty()) o_ << ind << Ab << " -= " << Ai << ";\n";
        break;
      case NT_OP_MUL:
        if (!Aa.empty()) o_ << ind << Aa << " += " << Ai << " * " << Vb << ";\n";
        if (!Ab.empty()) o_ << ind << Ab << " += " << Ai << " * " << Va << ";\n";
        break;
      case NT_OP_DIV:
        if (!Aa.empty()) o_ << ind << Aa << " += " << Ai << " / " << Vb << ";\n";
        if (!Ab.empty()) o_ << ind << Ab << " -= " << Ai << " * " << Vi << " / " << Vb << ";\n";
        break;
      case NT_OP_NEG:
        if (!Aa.empty()) o_ << ind << Aa << " -= " << Ai << ";\n";
        break;
      case NT_OP_EXP:
        if (!Aa.empty()) o_ << ind << Aa << " += " << Ai << " * " << Vi << ";\n";
        break;
      case NT_OP_LOG:
        if (!Aa.empty()) o_ << ind << Aa << " += " << Ai << " / " << Va << ";\n";
        break;
      case NT_OP_SQRT:
        if (!Aa.empty()) o_ << ind << Aa << " += " << Ai << " * " << half << " / " << Vi << ";\n";
        break;
      case NT_OP_ABS:
        if (!Aa.empty()) o_ << ind << Aa << " += " << Va << " < " << zero << " ? -" << Ai << " : " << Ai << ";\n";
        break;
      case NT_OP_MAX:
      case NT_OP_MIN: {
        const std::string cmp = op == NT_OP_MAX ? " >= " : " <= ";
        if (!Aa.empty()) o_ << ind << "if (" << Va << cmp << Vb << ") " << Aa << " += " << Ai << ";\n";
        if (!Ab.empty()) o_ << ind << "if (!(" << Va << cmp << Vb << ")) " << Ab << " += " << Ai << ";\n";
        break;
      }
      default: break;
    }
  }

  // ---- straight-line regions ----
  std::string vname(int node) const;        // forward value of a straight-line node or live-out
  std::string dname(int node) const;        // adjoint of an active straight-line node or live-out
  void line_draw(int lo, int i);
  void trip_counters(const std::string& ind);
  std::string body_draw(int u, int j, std::map<std::pair<int, int>, std::string>& pairs, const std::string& ind);
  void line_forward(int lo, int hi);
  void line_node(int lo, int i);
  void line_reverse(int lo, int hi);

  // ---- loop ----
  std::string body_value(int u, int kind, int ref, bool recompute) const;
  void segment(int U, const std::string& sg, bool forward);
  std::string ck_ref(const std::string& sg, int ci) const;
  int draw_partner(int U, int rel, int& pu, int& pj) const;

  // ---- tangent mode ----
  // Tangent names: "" for a structural zero, "#1" for the seed of an INPUT
  // node, otherwise a variable.
  bool has(int node, int j) const {
    return (p_.deps[static_cast<size_t>(node) * p_.n_words + (j >> 6)] >> (j & 63)) & 1;
  }
  bool poshas(int pos, int j) const {
    if (par_on_) {
      const int d = j - t_.n_in;
      return d >= 0 && d < static_cast<int>(par_node_.size()) && par_deps_[pos][d];
    }
    return (p_.posdeps[static_cast<size_t>(pos) * p_.n_words + (j >> 6)] >> (j & 63)) & 1;
  }
  std::vector<int> deplist(int node) const {
    std::vector<int> d;
    for (int j = 0; j < t_.n_in; ++j) if (has(node, j)) d.push_back(j);
    return d;
  }
  std::vector<int> posdeplist(int pos) const {
    std::vector<int> d;
    const int lo = par_on_ ? t_.n_in : 0, hi = par_on_ ? t_.n_in + static_cast<int>(par_node_.size()) : t_.n_in;
    for (int j = lo; j < hi; ++j) if (poshas(pos, j)) d.push_back(j);
    return d;
  }
  std::string tname(int node, int j) const;  // straight-line node or loop live-out
  // Loop parameters (tangent loops). The step body reads a few loop-invariant
  // values (a drift, a volatility per step) and the carried values' start
  // values; each is a function of the inputs. The loop's tangents can run
  // over those parameters instead of over the inputs (the chain rule taken
  // at the loop's boundary): the tangent of a parameter with respect to
  // itself is 1, so the body multiplies by no input tangent, and after the
  // loop each carried tangent returns to the inputs as the sum over
  // parameters of (tangent per parameter) x (the parameter's tangent per
  // input), once per path. Worth it when the body's tangents depend on fewer
  // parameters than inputs: the Asian step's log-return depends on 2
  // parameters (drift, volatility) against 3 inputs (r, sigma, T). Inside
  // the loop, direction n_in + d stands for parameter d.
  bool par_on_ = false;                     // emitting (or planning) the loop over parameters
  bool use_par_ = false;                    // the loop runs over parameters
  std::vector<int> par_node_;               // parameter -> node outside the loop
  std::map<int, int> par_of_;               // node -> parameter
  std::vector<std::vector<char>> par_deps_; // per loop position, per parameter
  void plan_parameters();
  // The tangent of a value from outside the loop, for input (or parameter) j.
  std::string inv_tname(int node, int j) const {
    if (!par_on_) return tname(node, j);
    auto it = par_of_.find(node);
    return it != par_of_.end() && it->second == j - t_.n_in ? "#1" : "";
  }
  // Scaled tangents. A node whose tangent is its operand's tangent times a
  // local factor (EXP, LOG, SQRT, ABS, NEG, a product or quotient with a value
  // that has no tangent, a max/min that follows one operand) keeps, per input,
  // the pair (base, scale): the tangent is base * scale, base a tangent that
  // was formed as a variable and scale a scalar of the node, the same for
  // every input. A chain of such rules multiplies scalars only; the product
  // per input is formed where a consumer needs it, and a sum or a product
  // rule takes it as one fma. lazy_ maps the name (or expression) that stands
  // for a tangent to its pair.
  mutable std::map<std::string, std::pair<std::string, std::string>> lazy_;
  // "(base * scale)", recorded as a scaled tangent
  std::string product(const std::string& scale, const std::string& base) const {
    const std::string e = "(" + base + " * " + scale + ")";
    lazy_[e] = {base, scale};
    return e;
  }
  // Scalar factors of scaled tangents: expression -> variable, for the scope
  // being emitted (a trip's block restores the set it found).
  std::map<std::string, std::string> scal_;
  int nscal_ = 0;
  std::string scalar(const std::string& ind, const std::string& e);
  // One tangent of one input: expr is its value; when base is set, the
  // tangent is base * scale and expr is that product.
  struct Term {
    std::string expr, base, scale;
    bool empty() const { return expr.empty(); }
  };
  Term lazy_term(const std::string& base, const std::string& scale) const {
    if (scale.empty()) return Term{base, "", ""};
    return Term{"(" + base + " * " + scale + ")", base, scale};
  }
  std::string smul(const std::string& ind, const std::string& s1, const std::string& s2);
  Term scaled(const std::string& ind, const std::string& T, const std::string& s, bool unwrap);
  Term sum(const Term& x, const Term& y) const;
  // Multiplicative carries (tangent loops): a carried value updated as
  // c <- c exp(x), the exponential used nowhere else, keeps G = the product of
  // the exp(x) since the loop began and sigma_k = t_k(loop start) + c0 sum tx_k,
  // c0 its value at the loop start; its tangent is G sigma_k (exact: c = c0 G).
  // Per step that is one fma per input and one multiply per carry, instead of
  // an fma and a multiply per input, and a consumer's sum of G sigma_k is one
  // fma. Tangents return to absolute form after the loop.
  std::vector<char> geo_;  // per loop position
  void plan_geo_carries();
  bool geo(int pos) const { return pos >= 0 && pos < static_cast<int>(geo_.size()) && geo_[pos]; }
  // A multiplicative carry that nothing in the body reads but itself (a
  // worst-of basket's spots, read by the payoff only) carries G alone; its
  // value is c0 G after the loop (c0 G, not the product of the roundings of
  // every step: the same value to a few hundred ulps).
  bool geo_free(int pos) const {
    if (!geo(pos)) return false;
    const int own = 1 + (L_.is_liveout[pos] ? 1 : 0);
    return body_uses_[pos] == own || (body_uses_[pos] == own + 1 && gsum_of_[pos] >= 0);
  }
  // A running sum A <- A + c of such a carry (the Asian average's sum of
  // spots), read by nothing but itself, accumulates G instead: A = A0 + c0
  // sum G after the loop. Per step that drops the carry's own multiply and,
  // for an input whose sigma is constant 1 (c's own start value), the sum of
  // tangents is that same sum of G.
  // A carry kept as G alone whose factor is exp(x) (the worst-of basket's
  // spots): G = exp(sum of x) needs no exponential per step. The loop adds
  // the exponents and the exponential is taken once, after the loop (the
  // fast pass; the re-evaluation pass keeps the product). exp of the sum and
  // the product of the exponentials agree to the rounding of the sum (about
  // sqrt(steps) ulps of the exponent), like G itself against the oracle's
  // step-by-step product.
  std::vector<char> geo_log_;  // per loop position
  void plan_geo_logs();
  bool geo_log(int pos) const {
    return !slow_ && pos >= 0 && pos < static_cast<int>(geo_log_.size()) && geo_log_[pos];
  }
  std::string geo_factor_exponent(int u, int j) const;
  // Such a carry whose exponent is p + r s (or p - r s, r s - p, r s), with p
  // and r loop-invariant and s a value with no tangent (a normal, or a
  // correlated normal: a literal row of a Cholesky factor times the step's
  // normals): over N steps the exponents sum to N p + r S, S the sum of s, and
  // their tangents for input k to N tp_k + tr_k S. The loop adds s alone, one
  // add per carry and step in place of the exponent, its sum and a fma per
  // input; N p + r S and the tangents are formed once, after the loop (the
  // fast pass; the sum differs from the step-by-step one in its roundings
  // only, a few ulps of the exponent).
  struct GeoAffine {
    bool on = false;
    int p = -1, r = -1;  // invariant nodes (p = -1: no offset)
    int s_kind = ARG_NONE, s_ref = -1;
    bool neg_p = false, neg_r = false;
  };
  std::vector<GeoAffine> gaff_;  // per loop position (the carry)
  void plan_geo_affine();
  bool gaff(int pos) const { return geo_log(pos) && pos < static_cast<int>(gaff_.size()) && gaff_[pos].on; }
  void geo_affine_finish(int j);
  void l2e_copies();
  void remat_open(int ls);
  std::vector<int> gsum_;     // per loop position: the geo carry a sum accumulates, or -1
  std::vector<int> gsum_of_;  // per loop position: the sum that accumulates this geo carry, or -1
  void plan_geo_sums();
  // Inputs k for which the sum's tangent is its own value: the carry's sigma_k
  // is the constant 1 (k is the carry's start value and no factor depends on
  // it) and the sum starts with no tangent for k.
  bool gsum_self(int a, int k) const {
    const int j = gsum_[a];
    if (j < 0) return false;
    const int ij = L_.carry_init[j], ia = L_.carry_init[a];
    const bool a_row = L_.kind_a[j] == ARG_CARRY && L_.ref_a[j] == j;
    const int e = a_row ? L_.ref_b[j] : L_.ref_a[j];  // the factor's loop position
    return ij >= 0 && inv_tname(ij, k) == "#1" && !poshas(e, k) && (ia < 0 || inv_tname(ia, k).empty());
  }
  std::vector<int> uses_;       // per node: operand references + outputs
  std::vector<int> body_uses_;  // per loop position: references within and across iterations, + live-out
  void count_uses();
  bool single_body_exp(int pos) const {
    return t_.op[L_.start + pos] == NT_OP_EXP && body_uses_[pos] == 1 && !L_.is_liveout[pos] && !L_.is_carry[pos];
  }
  // 1 / b used by nothing else: a multiplicative carry c <- c / b (a survival
  // probability) has the log-derivative -tb / b = -tb m, no division needed
  bool single_body_recip(int pos) const {
    if (t_.op[L_.start + pos] != NT_OP_DIV || body_uses_[pos] != 1 || L_.is_liveout[pos] || L_.is_carry[pos]) return false;
    const int ka = L_.kind_a[pos], ra = L_.ref_a[pos];
    return (ka == ARG_BODY && is_one(L_.start + ra)) || (ka == ARG_INV && is_one(ra));
  }
  // fp32 tangent loops: exp(p + r s), exp(p - r s), exp(r s - p) (or exp(r s))
  // with p and r loop-invariant and the sum (difference) and product used
  // nowhere else becomes exp2(p' + r' s) (signs kept) with
  // p' = p log2(e) and r' = r log2(e) computed once per path, dropping the
  // per-step multiply by log2(e) that the hardware exp2 otherwise needs.
  struct Exp2Fold {
    bool on = false;
    int p = -1, r = -1;          // invariant nodes (p = -1: no sum)
    int s_kind = ARG_NONE, s_ref = -1;
    bool neg_p = false, neg_r = false;  // r s - p, p - r s
    // p' + r' s with the signs, as an fp32 expression
    std::string arg(const std::string& lp, const std::string& lr, const std::string& sv, bool fuse) const {
      const std::string r = (neg_r ? "-" : "") + lr;
      if (p < 0) return r + " * " + sv;
      const std::string q = (neg_p ? "-" : "") + lp;
      return fuse ? "fmaf(" + r + ", " + sv + ", " + q + ")" : r + " * " + sv + " + " + q;
    }
  };
  std::vector<Exp2Fold> fold_;  // per loop position
  void plan_exp2_folds();
  // fp64 loop bodies: an EXP of p + r z, p - r z or r z, with p and r
  // loop-invariant and |z| <= Z_MAX on every step, cannot leave the fast exp's
  // range if |p| + Z_MAX |r| <= 708. z is a normal draw (|z| <= sqrt(66 ln 2)
  // = 6.764 for every Box-Muller draw, u1 >= 2^-33: Z_MAX 6.77) or a value
  // built from draws and literals alone, bounded through its operands. That is
  // checked once per path, before the loop, and the loop's exponentials skip
  // their own check.
  struct ExpBound {
    bool on = false;
    int p = -1, r = -1;  // invariant nodes (p = -1: no offset)
    int sum = -1, mul = -1, draw = -1;  // loop positions of p +- r z, r z and z
    bool p_first = true;                // p - r z (or a sum) rather than r z - p
    double zmax = 6.77;                 // Z_MAX
  };
  std::vector<ExpBound> bound_;  // per loop position
  void plan_exp_bounds();
  void exp_bound_checks();
  // p + r z feeding only such an exponential, itself only a multiplicative
  // carry's factor, is one fma: fused rounding moves the exponent by an ulp
  // at most, which the carry, kept as a product of factors G (its value
  // rebuilt as c0 G or summed as sum G after the loop, not the oracle's
  // step-by-step product anyway), does not resolve.
  std::vector<int> fused_exp_;  // per loop position: the exponential whose argument this sum is, or -1
  void plan_fused_exponents();
  // Step schedules, once per block (tangent loops). A step that reads a
  // schedule recorded up front (per-step literals combined with loop-invariant
  // values: a non-uniform grid's drift (r - s^2/2) T f_i and volatility
  // s sqrt(T f_i), GbmPath.java:58-64) computes the same values for every
  // path. The block computes them once, for every iteration, with their
  // tangents over the inputs and the reference's rules, into LDS, and each
  // path's step reads them: the step's work is then a uniform step's.
  bool sched_on_ = false;
  std::vector<char> sched_;       // per loop position: depends on no draw and no carried value
  std::vector<int> sched_slot_;   // per loop position: its first LDS row (the value, then its tangents), or -1
  int sched_rows_ = 0;
  void plan_schedule();
  void schedule_prologue();
  std::string l2e_name(int node) const { return "v" + std::to_string(node) + "_l2e" + ms(t_.active[node]); }
  void tangent(const std::string& ind, int op, const std::string& tn, const std::string& sfx, const std::vector<int>& D,
               const std::string& Vi, const std::string& Va, const std::string& Vb,
               const std::function<std::string(int)>& ta, const std::function<std::string(int)>& tb);
  void tline(int lo, int hi);
  void tsegment(int U, const std::string& sg);
  int trip_ = 1;  // loop steps per trip of the pass being emitted
  // Trips start at iteration it_base_ + sg * trip_. A stream that draws an
  // odd number of normals per step, from an odd ordinal in the loop's first
  // iteration (its first step was recorded before the loop), would split
  // every Box-Muller pair across two trips, each computing the pair for one
  // leg: the loop then runs its first iteration alone and its trips from
  // iteration 1, where draw_shift_[stream] = 1 moves the trip's counter base
  // (it0 * step + 1, even) and the draws' trip-relative ordinals down by one.
  int it_base_ = 0;
  std::map<int, int> draw_shift_;
  int draw_lead() const;
  void body_tangent_operand(int u, int kind, int ref, std::function<std::string(int)>& fn) const;

  // ---- markets (tangent mode): several input sets share each path's draws ----
  int m_ = 0, mlo_ = 0, mhi_ = 1;  // market being emitted; range of markets in the current body
  bool exp_active_ = true;         // the EXP being emitted depends on the inputs (per-market flag)
  std::string ms(bool active) const {
    return (p_.markets > 1 && active) ? "_m" + std::to_string(m_) : std::string();
  }
  std::string msuf(int m) const { return p_.markets > 1 ? "_m" + std::to_string(m) : std::string(); }

  // ---- kernel frame ----
  bool slow_ = false;  // emitting the device-libm re-evaluation of a flagged path
  bool exp_fallback() const {
    if (f32_) return false;
    for (int i = 0; i < t_.n; ++i) {
      if (max_fast(t_.op[i])) return true;
      if (p_.libm == 1) continue;
      if (t_.op[i] == NT_OP_EXP || t_.op[i] == NT_OP_LOG ||
          ((t_.op[i] == NT_OP_SQRT || t_.op[i] == NT_OP_DIV) && fast_sqrt())) {
        return true;
      }
    }
    return false;
  }
  // fp64 MAX and MIN: v_max_f64 / v_min_f64 in the fast pass, a non-finite
  // operand making the value NaN (nt_max_fast, nt_max_lit when one operand is
  // a literal), so the path's sums are not finite and the exception kernel
  // evaluates it again with nt_max / nt_min.
  bool max_fast(int op) const { return !f32_ && (op == NT_OP_MAX || op == NT_OP_MIN); }
  bool minmax_fallback() const {
    for (int i = 0; i < t_.n; ++i) {
      if (max_fast(t_.op[i])) return true;
    }
    return false;
  }
  // An active EXP, LOG, SQRT or DIV can leave a derivative infinite or NaN
  // where the oracle's is finite: 0 times an infinite local derivative (1 /
  // (1 + exp(x)) once exp(x) has overflowed) is NaN in IEEE arithmetic, while
  // the oracle never multiplies by a zero adjoint. A path whose value or
  // derivatives come out non-finite is evaluated again in the pass that
  // follows the oracle's zero-adjoint rule.
  bool nonfinite_fallback() const {
    if (!p_.adjoints) return false;
    for (int i = 0; i < t_.n; ++i) {
      const int op = t_.op[i];
      if (t_.active[i] && (op == NT_OP_EXP || op == NT_OP_LOG || op == NT_OP_SQRT || op == NT_OP_DIV)) return true;
    }
    return false;
  }
  // fp64 tangent kernels with the skeleton's own math take a SQRT node's value
  // and tangent factor from one nt_sqrt_q (a path whose argument it does not
  // cover is evaluated again with device libm).
  bool fast_sqrt() const { return !f32_ && p_.libm == 0 && p_.mode == NT_MODE_TANGENT; }
  // fp64 tangent loops, fast pass: x + a b, x - a b and a b - x of values
  // with no tangent (draws and literals alone: a correlated normal, a row of
  // a Cholesky factor times the step's normals), the product used nowhere
  // else, are one fma. Such a value moves by an ulp at most, and it feeds the
  // path only through exponents whose own rounding is of that size.
  bool draw_fma() const { return fast_sqrt() && p_.fuse && !slow_; }
  std::string draw_fma_expr(int u, int j, int op) const;
  // Forward value of a SQRT node; `q` names its tangent factor when the
  // tangent rule below should take it from here.
  std::string sqrt_expr(const std::string& x, const std::string& q, bool act) {
    if (f32_) return "nt_hw_sqrtf(" + x + ")";
    if (!fast_sqrt() || slow_) return "sqrt(" + x + ")";
    sqrt_q_ = q;
    return "nt_sqrt_q(" + x + ", " + q + ", nt_slow" + ms(act) + ")";
  }
  std::string sqrt_q_;  // tangent factor of the SQRT just emitted, if nt_sqrt_q made it
  // A DIV whose numerator is the constant 1 takes nt_recip in the same
  // kernels; its value is then its own tangent factor 1/b.
  bool is_one(int node) const {
    if (L_.found && node >= L_.start && node < L_.end() && L_.table_lit((node - L_.start) % L_.period)) return false;
    return t_.op[node] == NT_OP_CONST && t_.c[node] == 1.0;
  }
  // Literal of loop position j in iteration u of the trip: from the position's
  // table when it changes along the loop (a wave-uniform index: one scalar load).
  std::string body_expr(int j, int u, int op, const std::string& x, const std::string& y) const {
    const int i = L_.start + j;
    if (op == NT_OP_CONST && L_.table_lit(j)) return "nt_lit" + std::to_string(j) + "[it0 + " + std::to_string(u) + "u]";
    return expr(op, x, y, t_.c[i], t_.a[i], i);
  }
  bool recip_ = false;  // the DIV just emitted is a nt_recip
  void preamble();
  void kernel_head(bool slow);
  void kernel(bool slow);
  void accumulate(int m, const std::string& skip);
  void dump_rows(int m);
  bool fallback() const { return exp_fallback() || nonfinite_fallback(); }
  void body_tangent();
  void body_reverse();
  void body_reverse_segmented();
  void line_case_head();
  std::string in_sfx_;  // names the opaque copies of the inputs inside a case of a checkpointed straight line
};

std::string Emitter::vname(int node) const {
  if (L_.found && node >= L_.start && node < L_.end()) {
    const int pos = node - (L_.start + (L_.iters - 1) * L_.period);
    return "st" + std::to_string(pos) + ms(t_.active[L_.start + pos]);
  }
  return "v" + std::to_string(node) + ms(t_.active[node]);
}

std::string Emitter::dname(int node) const {
  if (L_.found && node >= L_.start && node < L_.end()) {
    return "gs" + std::to_string(node - (L_.start + (L_.iters - 1) * L_.period));
  }
  return "d" + std::to_string(node);
}

// A draw of a straight-line region; both legs of a Philox block come from one
// nt_normal_pair call (pairs_ is per region, `lo` keeps the names unique).
void Emitter::line_draw(int lo, int i) {
  const int k = t_.a[i];
  const int stream = t_.b[i];
  if (t_.op[i] == NT_OP_RANDU) {
    o_ << "    const real v" << i << " = " << uniform_call(stream, std::to_string(k) + "u") << ";\n";
    return;
  }
  const int ctr = k >> 1;
  auto it = pairs_.find({stream, ctr});
  std::string stem;
  if (it == pairs_.end()) {
    stem = "zl" + std::to_string(lo) + "_" + std::to_string(stream) + "_" + std::to_string(ctr);
    o_ << "    real " << stem << "c, " << stem << "s;\n";
    o_ << "    nt_normal_pair(" << rlo() << ", " << rhi(stream) << ", " << ctr << "u, " << stem << "c, " << stem << "s);\n";
    pairs_[{stream, ctr}] = stem;
  } else {
    stem = it->second;
  }
  o_ << "    const real v" << i << " = " << stem << ((k & 1) ? "s" : "c") << ";\n";
}

// Per-trip draw counters: normals of stream s in this trip start at ordinal
// it0 * step_s (even, since the trip length times an odd step is even).
void Emitter::trip_counters(const std::string& ind) {
  for (const auto& kv : L_.normal_step) {
    auto sh = draw_shift_.find(kv.first);
    o_ << ind << "const nt_u32 kb" << kv.first << " = it0 * " << kv.second << "u"
       << (sh != draw_shift_.end() && sh->second ? " + " + std::to_string(sh->second) + "u" : std::string()) << ";\n";
  }
}

// 1 when every stream that draws an odd number of normals per step starts
// the loop at an odd ordinal (and some does), 0 otherwise.
int Emitter::draw_lead() const {
  std::map<int, int> first;  // stream -> lowest normal ordinal in iteration 0
  for (int j = 0; j < L_.period; ++j) {
    const int i = L_.start + j;
    if (t_.op[i] != NT_OP_RANDN) continue;
    auto it = first.find(t_.b[i]);
    if (it == first.end() || L_.rand_base[j] < it->second) first[t_.b[i]] = L_.rand_base[j];
  }
  bool odd = false;
  for (const auto& kv : L_.normal_step) {
    if (!(kv.second & 1)) continue;
    if (!(first[kv.first] & 1)) return 0;
    odd = true;
  }
  return odd && L_.iters > 1 ? 1 : 0;
}

// Value of loop draw position j in iteration u of a trip: both legs of a
// normal pair come from one nt_normal_pair call (pairs keyed by stream and
// counter within the trip); a uniform is one Philox block.
std::string Emitter::body_draw(int u, int j, std::map<std::pair<int, int>, std::string>& pairs,
                               const std::string& ind) {
  const int i = L_.start + j;
  const int stream = t_.b[i];
  const int step = L_.rand_step[j];
  if (t_.op[i] == NT_OP_RANDU) {
    return uniform_call(stream, "(it0 + " + std::to_string(u) + "u) * " + std::to_string(step) + "u + " +
                                    std::to_string(L_.rand_base[j]) + "u");
  }
  auto sh = draw_shift_.find(stream);
  const int rel = L_.rand_base[j] + u * step - (sh != draw_shift_.end() ? sh->second : 0);
  const int key = rel >> 1;
  auto it = pairs.find({stream, key});
  std::string stem;
  if (it == pairs.end()) {
    stem = "zp" + std::to_string(stream) + "_" + std::to_string(key);
    o_ << ind << "real " << stem << "c, " << stem << "s;\n";
    o_ << ind << "nt_normal_pair(rlo, " << rhi(stream) << ", (kb" << stream << " >> 1) + " << key << "u, " << stem << "c, "
       << stem << "s);\n";
    pairs[{stream, key}] = stem;
  } else {
    stem = it->second;
  }
  return stem + ((rel & 1) ? "s" : "c");
}

void Emitter::line_forward(int lo, int hi) {
  pairs_.clear();
  for (int i = lo; i < hi; ++i) line_node(lo, i);
}

void Emitter::line_node(int lo, int i) {
  const int op = t_.op[i];
  if (op == NT_OP_RANDN || op == NT_OP_RANDU) {
    line_draw(lo, i);
    return;
  }
  const int ar = arity(op);
  const std::string x = ar >= 1 ? vname(t_.a[i]) : "";
  const std::string y = ar >= 2 ? vname(t_.b[i]) : "";
  o_ << "    const real v" << i << " = " << expr(op, x, y, t_.c[i], t_.a[i]) << ";\n";
}

// The reverse sweep of a checkpointed straight line: two loops over the
// segments, each a switch with one case per segment, so that each segment is
// a basic block of its own (the compiler schedules and allocates registers
// within a segment, and its passes stay fast on long tapes). Values cross
// segments only through the carried slots nt_f<k> (forward) and nt_a<k>
// (adjoints), so the live set at any point is one segment's plus the slots.
//
// Forward loop, segment s: read the values it needs from earlier segments
// from their slots (constants and inputs re-emitted), compute its nodes,
// store those a later segment's reverse reads (scratch[slot * T + lane]),
// and leave those later segments read in their slots. Reverse loop, last
// segment first: read back the stored values the segment needs, recompute
// its needed nodes, take the carried adjoints from their slots, run its
// rules, and leave in slots the adjoints that earlier segments continue. The
// contributions reach each adjoint in the same order as in an uncut sweep.
//
// Every case starts from opaque copies (nt_opaque, nt_opaque_u) of the
// segment index, the inputs, the Philox key and the lane index: the compiler
// can see neither which case runs next nor that a case's work is the same on
// every pass of the loop, so it keeps each segment's arithmetic, draws and
// scratch addresses inside its case instead of hoisting them out of the
// loops (where they would stay live for the whole path) or merging the
// recomputation with the forward pass.
void Emitter::line_case_head() {
  o_ << "        const nt_u64 nt_ct = nt_opaque(tid);\n";
  o_ << "        const nt_u32 rlo_o = nt_opaque(rlo);\n";
  for (int st = 0; st < t_.n_streams; ++st) {
    key_.clear();
    const std::string h = rhi(st);
    key_ = "_o";
    o_ << "        const nt_u32 " << rhi(st) << " = nt_opaque(" << h << ");\n";
  }
  key_ = "_o";
  for (int j = 0; j < t_.n_in; ++j) o_ << "        const real in" << j << "_o = nt_opaque_u(in" << j << ");\n";
  in_sfx_ = "_o";
}

void Emitter::body_reverse_segmented() {
  const auto& B = p_.lbound;
  const auto& seg = p_.lseg;
  const int S = static_cast<int>(B.size()) - 1;
  const std::string zero = f32_ ? "0.0f" : "0.0";
  const std::string one = f32_ ? "1.0f" : "1.0";
  auto slotname = [](const char* stem, int k) { return std::string(stem) + std::to_string(k); };
  o_ << "    {\n";
  for (int k = 0; k < p_.kf; ++k) o_ << "    real nt_f" << k << " = " << zero << ";\n";
  o_ << "    for (int nt_s = 0; nt_s < " << S << "; ++nt_s) {\n";
  o_ << "      switch (nt_opaque_u(nt_s)) {\n";
  for (int s = 0; s < S; ++s) {
    const int lo = B[s], hi = B[s + 1];
    o_ << "      case " << s << ": {  // nodes " << lo << " to " << hi - 1 << "\n";
    line_case_head();
    std::set<int> entering;
    for (int i = lo; i < hi; ++i) {
      const int ar = arity(t_.op[i]);
      if (ar >= 1 && t_.a[i] < lo) entering.insert(t_.a[i]);
      if (ar >= 2 && t_.b[i] < lo) entering.insert(t_.b[i]);
    }
    for (int x : entering) {
      if (p_.fslot[x] >= 0) o_ << "    const real v" << x << " = " << slotname("nt_f", p_.fslot[x]) << ";\n";
      else line_node(lo, x);  // a constant or an input
    }
    pairs_.clear();
    for (int i = lo; i < hi; ++i) line_node(lo, i);
    for (int i = lo; i < hi; ++i) {
      if (p_.lslot[i] >= 0) o_ << "    scratch[(nt_u64)" << p_.lslot[i] << "u * T + nt_ct] = v" << i << ";\n";
    }
    if (t_.output >= lo && t_.output < hi) o_ << "    nt_y[0] = (double)" << vname(t_.output) << ";\n";
    for (int i = lo; i < hi; ++i) {
      if (p_.fslot[i] >= 0) o_ << "    " << slotname("nt_f", p_.fslot[i]) << " = v" << i << ";\n";
    }
    o_ << "        break;\n      }\n";
    key_.clear();
    in_sfx_.clear();
  }
  o_ << "      }\n    }\n    }\n";
  for (int j = 0; j < t_.n_in; ++j) {
    const int node = t_.input_node[j];
    if (t_.active[node]) o_ << "    real d" << node << " = " << (node == t_.output ? one : zero) << ";\n";
  }
  for (int k = 0; k < p_.ka; ++k) o_ << "    real nt_a" << k << " = " << zero << ";\n";
  o_ << "    for (int nt_s = " << S - 1 << "; nt_s >= 0; --nt_s) {\n";
  o_ << "      switch (nt_opaque_u(nt_s)) {\n";
  for (int s = S - 1; s >= 0; --s) {
    const int lo = B[s], hi = B[s + 1];
    o_ << "      case " << s << ": {  // nodes " << lo << " to " << hi - 1 << "\n";
    line_case_head();
    for (int x : p_.lin[s]) {
      if (p_.lslot[x] >= 0) o_ << "    const real v" << x << " = scratch[(nt_u64)" << p_.lslot[x] << "u * T + nt_ct];\n";
      else line_node(lo, x);  // a constant or an input
    }
    pairs_.clear();
    for (int i = lo; i < hi; ++i) {
      if (p_.lneed[i]) line_node(lo, i);
    }
    key_.clear();
    in_sfx_.clear();
    for (int x = 0; x < hi; ++x) {
      if (p_.aslot[x] < 0) continue;
      if (seg[x] <= s && s < p_.ahi[x]) {
        o_ << "    real d" << x << " = " << slotname("nt_a", p_.aslot[x]) << ";\n";
      } else if (seg[x] < s && p_.ahi[x] == s) {
        o_ << "    real d" << x << " = " << (x == t_.output ? one : zero) << ";\n";
      }
    }
    for (int i = lo; i < hi; ++i) {
      if (!t_.active[i] || t_.op[i] == NT_OP_INPUT || arity(t_.op[i]) == 0 || p_.aslot[i] >= 0) continue;
      o_ << "    real d" << i << " = " << (i == t_.output ? one : zero) << ";\n";
    }
    line_reverse(lo, hi);
    for (int x = 0; x < lo; ++x) {
      if (p_.aslot[x] >= 0 && seg[x] < s && s <= p_.ahi[x]) {
        o_ << "    " << slotname("nt_a", p_.aslot[x]) << " = d" << x << ";\n";
      }
    }
    o_ << "        break;\n      }\n";
  }
  o_ << "      }\n    }\n";
  for (int j = 0; j < t_.n_in; ++j) {
    const int node = t_.input_node[j];
    o_ << "    nt_g[" << j << "] = " << (t_.active[node] ? "(double)d" + std::to_string(node) : std::string("0.0"))
       << ";\n";
  }
}

void Emitter::line_reverse(int lo, int hi) {
  for (int i = hi - 1; i >= lo; --i) {
    if (!t_.active[i]) continue;
    const int op = t_.op[i];
    const int ar = arity(op);
    if (ar == 0) continue;
    const int a = t_.a[i], b = ar >= 2 ? t_.b[i] : -1;
    const std::string Aa = t_.active[a] ? dname(a) : "";
    const std::string Ab = (b >= 0 && t_.active[b]) ? dname(b) : "";
    rev("    ", op, "d" + std::to_string(i), "v" + std::to_string(i), vname(a), b >= 0 ? vname(b) : "", Aa, Ab);
  }
}

// Value of a body operand in iteration u of the current segment. Carried
// operands of the first iteration come from the segment-start state (st* in
// the forward pass, checkpoint k* in the recompute).
std::string Emitter::body_value(int u, int kind, int ref, bool recompute) const {
  if (kind == ARG_BODY) return "r" + std::to_string(u) + "_" + std::to_string(ref) + ms(t_.active[L_.start + ref]);
  if (kind == ARG_CARRY) {
    const std::string m = ms(t_.active[L_.start + ref]);
    if (u > 0) return "r" + std::to_string(u - 1) + "_" + std::to_string(ref) + m;
    return (recompute ? "k" : "st") + std::to_string(ref) + m;
  }
  return "v" + std::to_string(ref) + ms(t_.active[ref]);
}

// Emits one segment of U iterations. `sg` is the segment index expression;
// the iteration base is it0 = sg * SEG. forward: compute, store, advance the
// state. !forward: recompute (reloading stored values), then reverse.
// Checkpoint ci of segment sg: a slot of the lane's scratch tape. (Held in
// LDS instead, in blocks of 768 threads to keep three waves per SIMD, the C2
// fp64 reverse sweep measured 2.19 ms against 1.98 ms here.)
std::string Emitter::ck_ref(const std::string& sg, int ci) const {
  const std::string NC = std::to_string(p_.ck_carries.size());
  return "scratch[(nt_u64)((" + sg + ") * " + NC + "u + " + std::to_string(ci) + "u) * T + tid]";
}

void Emitter::segment(int U, const std::string& sg, bool forward) {
  const int P = L_.period, s = L_.start;
  const int NC = static_cast<int>(p_.ck_carries.size());
  const std::string ind = "      ";
  o_ << "    {\n";
  o_ << ind << "const nt_u32 it0 = (" << sg << ") * " << p_.seg << "u;\n";
  trip_counters(ind);
  const bool ckpt = p_.adjoints;
  if (forward && ckpt) {
    for (int ci = 0; ci < NC; ++ci) o_ << ind << ck_ref(sg, ci) << " = st" << p_.ck_carries[ci] << ";\n";
  }
  if (!forward) {
    for (int ci = 0; ci < NC; ++ci) o_ << ind << "const real k" << p_.ck_carries[ci] << " = " << ck_ref(sg, ci) << ";\n";
  }
  // draws of this segment by stream and relative counter, for pairing the two legs
  std::map<std::pair<int, int>, std::string> pairs;
  for (int u = 0; u < U; ++u) {
    for (int j = 0; j < P; ++j) {
      const int i = s + j;
      const int op = t_.op[i];
      const std::string name = "r" + std::to_string(u) + "_" + std::to_string(j);
      const std::string slot = "(nt_u64)(" + std::to_string(p_.ck_slots) + "u + (it0 + " + std::to_string(u) + "u) * " +
                               std::to_string(p_.n_stored) + "u + " + std::to_string(p_.store_index[j] < 0 ? 0 : p_.store_index[j]) +
                               "u) * T + tid";
      if (!forward && p_.stored[j]) {
        o_ << ind << "const real " << name << " = scratch[" << slot << "];\n";
        continue;
      }
      if (!forward && !p_.rneed[j]) continue;  // nothing the rules read depends on it
      if (op == NT_OP_RANDN || op == NT_OP_RANDU) {
        const std::string d = body_draw(u, j, pairs, ind);
        o_ << ind << "const real " << name << " = " << d << ";\n";
      } else {
        const int ar = arity(op);
        const std::string x = ar >= 1 ? body_value(u, L_.kind_a[j], L_.ref_a[j], !forward) : "";
        const std::string y = ar >= 2 ? body_value(u, L_.kind_b[j], L_.ref_b[j], !forward) : "";
        o_ << ind << "const real " << name << " = " << body_expr(j, u, op, x, y) << ";\n";
      }
      if (forward && p_.adjoints && p_.stored[j]) {
        o_ << ind << "scratch[" << slot << "] = " << name << ";\n";
      }
    }
  }
  if (forward) {
    for (int j = 0; j < P; ++j) {
      if (L_.is_carry[j] || L_.is_liveout[j]) {
        o_ << ind << "st" << j << " = r" << (U - 1) << "_" << j << ";\n";
      }
    }
    o_ << "    }\n";
    return;
  }
  const std::string zero = f32_ ? "0.0f" : "0.0";
  for (int u = U - 1; u >= 0; --u) {
    o_ << ind << "{\n";
    const std::string in2 = ind + "  ";
    for (int j = 0; j < P; ++j) {
      if (!t_.active[s + j]) continue;
      o_ << in2 << "real a" << j << " = " << ((L_.is_carry[j] || L_.is_liveout[j]) ? "gs" + std::to_string(j) : zero)
         << ";\n";
    }
    for (int c : p_.carries) {
      if (t_.active[s + c]) o_ << in2 << "real q" << c << " = " << zero << ";\n";
    }
    auto adj = [&](int kind, int ref) -> std::string {
      if (kind == ARG_BODY) return t_.active[s + ref] ? "a" + std::to_string(ref) : "";
      if (kind == ARG_CARRY) return t_.active[s + ref] ? "q" + std::to_string(ref) : "";
      if (kind == ARG_INV) return t_.active[ref] ? "d" + std::to_string(ref) : "";
      return "";
    };
    for (int j = P - 1; j >= 0; --j) {
      if (!t_.active[s + j]) continue;
      const int op = t_.op[s + j];
      const int ar = arity(op);
      if (ar == 0) continue;
      const std::string Va = body_value(u, L_.kind_a[j], L_.ref_a[j], true);
      const std::string Vb = ar >= 2 ? body_value(u, L_.kind_b[j], L_.ref_b[j], true) : "";
      rev(in2, op, "a" + std::to_string(j), "r" + std::to_string(u) + "_" + std::to_string(j), Va, Vb,
          adj(L_.kind_a[j], L_.ref_a[j]), ar >= 2 ? adj(L_.kind_b[j], L_.ref_b[j]) : "");
    }
    for (int j = 0; j < P; ++j) {
      if (!(L_.is_carry[j] || L_.is_liveout[j]) || !t_.active[s + j]) continue;
      o_ << in2 << "gs" << j << " = " << (L_.is_carry[j] ? "q" + std::to_string(j) : zero) << ";\n";
    }
    o_ << ind << "}\n";
  }
  o_ << "    }\n";
}

// ---- tangent mode --------------------------------------------------------------

std::string Emitter::tname(int node, int j) const {
  if (L_.found && node >= L_.start && node < L_.end()) {
    const int pos = node - (L_.start + (L_.iters - 1) * L_.period);
    return poshas(pos, j) ? "ts" + std::to_string(pos) + "_" + std::to_string(j) + ms(true) : "";
  }
  if (!has(node, j)) return "";
  if (t_.op[node] == NT_OP_INPUT) return "#1";
  return "t" + std::to_string(node) + "_" + std::to_string(j) + ms(true);
}

std::string Emitter::scalar(const std::string& ind, const std::string& e) {
  auto it = scal_.find(e);
  if (it != scal_.end()) return it->second;
  const std::string name = "ls" + std::to_string(nscal_++);
  o_ << ind << "const " << treal() << " " << name << " = " << e << ";\n";
  scal_[e] = name;
  return name;
}

// s1 * s2 for scale factors ("" stands for 1)
std::string Emitter::smul(const std::string& ind, const std::string& s1, const std::string& s2) {
  if (s1.empty()) return s2;
  if (s2.empty()) return s1;
  if (slow_) return scalar(ind, "(" + treal() + "(" + s1 + ") * " + s2 + ")");
  return scalar(ind, "(" + s1 + " * " + s2 + ")");
}

// The tangent T ("#1" the seed of an input, a variable, or a scaled tangent)
// times the scalar s. A scaled T is taken apart (its scale times s, one
// scalar operation) only when `unwrap` says that scalar is shared; otherwise
// T's own variable is the base.
Emitter::Term Emitter::scaled(const std::string& ind, const std::string& T, const std::string& s, bool unwrap) {
  if (T == "#1") return Term{s.empty() ? std::string(f32_ ? "1.0f" : "1.0") : s, "", ""};
  auto it = lazy_.find(T);
  // T itself, still known as a scaling of its base; its variable is its value
  if (it != lazy_.end() && s.empty()) return Term{T, it->second.first, it->second.second};
  if (it != lazy_.end() && unwrap) return lazy_term(it->second.first, smul(ind, it->second.second, s));
  return lazy_term(T, s);
}

// x + y, with a scaled term taken as one fma and a term scaled by -1 as a
// subtraction.
Emitter::Term Emitter::sum(const Term& x, const Term& y) const {
  if (x.empty()) return y;
  if (y.empty()) return x;
  const std::string mone = f32_ ? "(-1.0f)" : "(-1.0)";
  if (y.scale == mone) return Term{"(" + x.expr + " - " + y.base + ")", "", ""};
  if (x.scale == mone) return Term{"(" + y.expr + " - " + x.base + ")", "", ""};
  if (!y.base.empty()) return Term{f("fma") + "(" + y.base + ", " + y.scale + ", " + x.expr + ")", "", ""};
  if (!x.base.empty()) return Term{f("fma") + "(" + x.base + ", " + x.scale + ", " + y.expr + ")", "", ""};
  return Term{"(" + x.expr + " + " + y.expr + ")", "", ""};
}

// Tangent of one active node for each input j in D, named tn + j, from the
// operand tangents ta(j), tb(j). The local derivatives are those of the
// reverse rules in rev(): d/da and d/db of ADD SUB MUL DIV NEG EXP LOG SQRT
// ABS, and MAX/MIN following operand a when a >= b (a <= b), else b. Every
// rule is A qa + B qb with scalar factors qa, qb (a max/min selects), so a
// node's tangent stays scaled (base * scale) wherever one operand has a
// tangent for that input. A new scalar (a scale times a factor, a selected
// scale, the sum of two scales of one base) is formed only when at least two
// inputs of the node share it: for a single input it costs what the product
// per input costs.
void Emitter::tangent(const std::string& ind, int op, const std::string& tn, const std::string& sfx,
                      const std::vector<int>& D, const std::string& Vi, const std::string& Va, const std::string& Vb,
                      const std::function<std::string(int)>& ta, const std::function<std::string(int)>& tb) {
  if (D.empty()) return;
  const std::string one = f32_ ? "1.0f" : "1.0";
  const std::string zero = f32_ ? "0.0f" : "0.0";
  const std::string mone = f32_ ? "(-1.0f)" : "(-1.0)";
  bool needB = false;
  for (int j : D) needB |= !tb(j).empty();
  const std::string q = tn + "q" + sfx, r = tn + "r" + sfx, c = tn + "c" + sfx;
  const std::string rcp_one = f32_ ? "nt_rcpf(" : "1.0 / (";
  switch (op) {
    case NT_OP_DIV:
      // (1 / b from nt_recip is its own factor)
      o_ << ind << "const real " << q << " = " << (recip_ ? Vi : rcp_one + Vb + ")") << ";\n";
      if (needB) o_ << ind << "const real " << r << " = " << Vi << " * " << q << ";\n";
      break;
    case NT_OP_LOG: o_ << ind << "const real " << q << " = " << rcp_one << Va << ");\n"; break;
    case NT_OP_SQRT:
      // sqrt(0) = 0 has an infinite local derivative. The reverse sweep never
      // multiplies it by a zero adjoint (zero adjoints are skipped), so the
      // factor is capped at a finite 2^(max exponent) here: a zero tangent
      // (e.g. a full-truncation max(v, 0) that chose the constant) stays zero.
      // nt_sqrt_q has set it already where it computed the value.
      // (A NaN root keeps a NaN factor, as the reverse rule's 0.5 / v does.)
      if (sqrt_q_ == q) break;
      o_ << ind << "const real " << q << " = " << Vi << " == " << zero << " ? " << (f32_ ? "0x1p127f" : "0x1p1023")
         << " : " << (f32_ ? "0.5f * nt_rcpf(" + Vi + ")" : "0.5 / " + Vi) << ";\n";
      break;
    case NT_OP_ABS: o_ << ind << "const real " << q << " = " << Va << " < " << zero << " ? -" << one << " : " << one << ";\n"; break;
    case NT_OP_MAX: o_ << ind << "const bool " << c << " = " << Va << " >= " << Vb << ";\n"; break;
    case NT_OP_MIN: o_ << ind << "const bool " << c << " = " << Va << " <= " << Vb << ";\n"; break;
    default: break;
  }
  std::string qa, qb;  // local factors ("" stands for 1)
  switch (op) {
    case NT_OP_SUB: qb = mone; break;
    case NT_OP_MUL: qa = Vb; qb = Va; break;
    case NT_OP_DIV: qa = q; if (needB) qb = "(-" + r + ")"; break;
    case NT_OP_NEG: qa = mone; break;
    case NT_OP_EXP: qa = Vi; break;
    case NT_OP_LOG: case NT_OP_SQRT: case NT_OP_ABS: qa = q; break;
    default: break;
  }
  // How many inputs would share each new scalar.
  auto scale_of = [&](const std::string& T) -> std::string {
    auto it = lazy_.find(T);
    return it == lazy_.end() ? std::string("=") + T : it->second.second;  // "=" marks an unscaled tangent
  };
  std::map<std::string, int> share;
  for (int j : D) {
    const std::string A = ta(j), B = tb(j);
    if (!A.empty() && A != "#1") ++share["a" + scale_of(A)];
    if (!B.empty() && B != "#1") ++share["b" + scale_of(B)];
  }
  auto shared = [&](const std::string& key) { return share[key] >= 2; };
  const size_t nD = D.size();
  std::vector<Term> x(nD), y(nD);
  for (size_t i = 0; i < nD; ++i) {
    const std::string A = ta(D[i]), B = tb(D[i]);
    if (!A.empty()) x[i] = scaled(ind, A, qa, shared("a" + scale_of(A)));
    if (!B.empty()) y[i] = scaled(ind, B, qb, shared("b" + scale_of(B)));
  }
  std::vector<Term> t(nD);
  if (op == NT_OP_MAX || op == NT_OP_MIN) {
    // c ? A : B: with one side, or both sides scalings of one base, the
    // selection moves to the scale when that selection is shared.
    auto base_of = [](const Term& u) { return u.base.empty() ? u.expr : u.base; };
    auto scale_or_one = [&](const Term& u) { return u.scale.empty() ? one : u.scale; };
    std::vector<std::string> key(nD);
    std::map<std::string, int> nsel;
    for (size_t i = 0; i < nD; ++i) {
      const std::string A = ta(D[i]), B = tb(D[i]);
      const bool ax = !x[i].empty() && A != "#1", by = !y[i].empty() && B != "#1";
      if (ax && by && base_of(x[i]) == base_of(y[i])) key[i] = "(" + c + " ? " + scale_or_one(x[i]) + " : " + scale_or_one(y[i]) + ")";
      else if (ax && y[i].empty()) key[i] = "(" + c + " ? " + scale_or_one(x[i]) + " : " + zero + ")";
      else if (by && x[i].empty()) key[i] = "(" + c + " ? " + zero + " : " + scale_or_one(y[i]) + ")";
      if (!key[i].empty()) ++nsel[key[i]];
    }
    for (size_t i = 0; i < nD; ++i) {
      if (!key[i].empty() && (nsel[key[i]] >= 2 || scal_.count(key[i]))) {
        t[i] = lazy_term(base_of(x[i].empty() ? y[i] : x[i]), scalar(ind, key[i]));
      } else if (!x[i].empty() || !y[i].empty()) {
        t[i] = Term{"(" + c + " ? " + (x[i].empty() ? zero : x[i].expr) + " : " + (y[i].empty() ? zero : y[i].expr) + ")", "", ""};
      }
    }
  } else {
    // Two scalings of one base add their scales when that sum is shared.
    std::map<std::string, int> nadd;
    std::vector<std::string> key(nD);
    for (size_t i = 0; i < nD; ++i) {
      if (!x[i].base.empty() && x[i].base == y[i].base) {
        key[i] = "(" + x[i].scale + " + " + y[i].scale + ")";
        ++nadd[key[i]];
      }
    }
    for (size_t i = 0; i < nD; ++i) {
      if (!key[i].empty() && (nadd[key[i]] >= 2 || scal_.count(key[i]))) t[i] = lazy_term(x[i].base, scalar(ind, key[i]));
      else t[i] = sum(x[i], y[i]);
    }
    // a * b with b = exp(x): the tangent of b is tx b, and A b + a tx b is
    // (A + a tx) b, an fma and a multiply per input with no scalar.
    if (op == NT_OP_MUL) {
      for (size_t i = 0; i < nD; ++i) {
        for (int side = 0; side < 2; ++side) {
          const std::string C = side ? ta(D[i]) : tb(D[i]), E = side ? tb(D[i]) : ta(D[i]);
          const std::string& cv = side ? Va : Vb;  // value of the other factor
          const std::string& ev = side ? Vb : Va;  // value of the exponential
          if (C.empty() || E.empty() || C == "#1" || E == "#1" || lazy_.count(C) || lazy_.count(E) == 0) continue;
          const auto& le = lazy_.at(E);
          // (a scaled tx is used as its variable: free outside the loop body)
          if (le.second != ev || (lazy_.count(le.first) && le.first.rfind("tr", 0) == 0)) continue;
          t[i] = Term{"(" + f("fma") + "(" + le.first + ", " + cv + ", " + C + ") * " + ev + ")", "", ""};
          break;
        }
      }
    }
  }
  for (size_t i = 0; i < nD; ++i) {
    const std::string name = tn + std::to_string(D[i]) + sfx;
    if (!t[i].base.empty()) lazy_[name] = {t[i].base, t[i].scale};
    else lazy_.erase(name);
    o_ << ind << "const " << treal() << " " << name << " = " << (t[i].empty() ? zero : t[i].expr) << ";\n";
  }
}

void Emitter::tline(int lo, int hi) {
  pairs_.clear();
  for (int i = lo; i < hi; ++i) {
    const int op = t_.op[i];
    if (op == NT_OP_RANDN || op == NT_OP_RANDU) {
      line_draw(lo, i);  // a draw is never active: one per path, shared by the markets
      continue;
    }
    const int ar = arity(op);
    const bool act = t_.active[i] != 0;
    for (int m = act ? mlo_ : 0; m < (act ? mhi_ : 1); ++m) {
      m_ = m;
      exp_active_ = act;
      const std::string x = ar >= 1 ? vname(t_.a[i]) : "";
      const std::string y = ar >= 2 ? vname(t_.b[i]) : "";
      std::string val = expr(op, x, y, t_.c[i], t_.a[i], i);
      sqrt_q_.clear();
      if (op == NT_OP_SQRT && fast_sqrt() && !slow_) {
        const std::string q = "t" + std::to_string(i) + "_q" + ms(true);
        o_ << "    real " << q << ";\n";
        val = sqrt_expr(x, q, act);
      }
      recip_ = op == NT_OP_DIV && fast_sqrt() && !slow_ && is_one(t_.a[i]);
      if (recip_) val = "nt_recip(" + y + ", nt_slow" + ms(act) + ")";
      o_ << "    const real v" << i << ms(act) << " = " << val << ";\n";
      if (!act || ar == 0 || !p_.adjoints) continue;
      const int a = t_.a[i], b = ar >= 2 ? t_.b[i] : -1;
      tangent("    ", op, "t" + std::to_string(i) + "_", ms(true), deplist(i), "v" + std::to_string(i) + ms(true), x, y,
              [&](int j) { return tname(a, j); }, [&](int j) { return b >= 0 ? tname(b, j) : std::string(); });
      sqrt_q_.clear();
    }
  }
}

void Emitter::body_tangent_operand(int u, int kind, int ref, std::function<std::string(int)>& fn) const {
  const std::string m = ms(true);
  if ((kind == ARG_BODY || kind == ARG_CARRY) && geo(ref)) {
    // a multiplicative carry's tangent is G sigma
    const int v = kind == ARG_BODY ? u : u - 1;  // iteration whose value is read; -1: the state before the trip
    fn = [this, v, ref, m](int j) {
      if (!poshas(ref, j)) return std::string();
      const std::string r = std::to_string(ref), k = std::to_string(j);
      if (v < 0) return product("gs" + r + m, "ts" + r + "_" + k + m);
      const std::string it = std::to_string(v);
      return product("gq" + it + "_" + r + m, "tr" + it + "_" + r + "_" + k + m);
    };
    return;
  }
  if (kind == ARG_BODY) {
    fn = [this, u, ref, m](int j) {
      return poshas(ref, j) ? "tr" + std::to_string(u) + "_" + std::to_string(ref) + "_" + std::to_string(j) + m
                            : std::string();
    };
  } else if (kind == ARG_CARRY) {
    fn = [this, u, ref, m](int j) {
      if (!poshas(ref, j)) return std::string();
      return u > 0 ? "tr" + std::to_string(u - 1) + "_" + std::to_string(ref) + "_" + std::to_string(j) + m
                   : "ts" + std::to_string(ref) + "_" + std::to_string(j) + m;
    };
  } else if (kind == ARG_INV) {
    fn = [this, ref](int j) { return inv_tname(ref, j); };
  } else {
    fn = [](int) { return std::string(); };
  }
}

// One trip of U loop iterations: values and their tangents, then the carried
// state (values and tangents) advances.
void Emitter::tsegment(int U, const std::string& sg) {
  const int P = L_.period, s = L_.start;
  const std::string ind = "      ";
  const auto outer_scalars = scal_;  // scalars declared in this block end with it
  o_ << "    {\n";
  o_ << ind << "const nt_u32 it0 = " << (it_base_ ? std::to_string(it_base_) + "u + " : std::string()) << "(" << sg
     << ") * " << trip_ << "u;\n";
  trip_counters(ind);
  std::map<std::pair<int, int>, std::string> pairs;
  for (int u = 0; u < U; ++u) {
    for (int j = 0; j < P; ++j) {
      const int i = s + j;
      const int op = t_.op[i];
      const std::string name = "r" + std::to_string(u) + "_" + std::to_string(j);
      if (op == NT_OP_RANDN || op == NT_OP_RANDU) {
        const std::string d = body_draw(u, j, pairs, ind);
        o_ << ind << "const real " << name << " = " << d << ";\n";
        continue;
      }
      const int ar = arity(op);
      const bool act = t_.active[i] != 0;
      if (sched_on_ && !slow_ && sched_[j] && op != NT_OP_CONST) {
        // computed once per block (schedule_prologue)
        const int row = sched_slot_[j];
        if (row < 0) continue;  // read only by other schedule values
        const std::string at = "u * " + std::to_string(L_.iters) + "u + it0 + " + std::to_string(u) + "u]";
        o_ << ind << "const real " << name << " = nt_sch[" << row << at << ";\n";
        if (!p_.adjoints) continue;
        int r = row + 1;
        for (int k : posdeplist(j)) {
          const std::string tn = "tr" + std::to_string(u) + "_" + std::to_string(j) + "_" + std::to_string(k);
          lazy_.erase(tn);
          o_ << ind << "const real " << tn << " = nt_sch[" << r++ << at << ";\n";
        }
        continue;
      }
      for (int m = act ? mlo_ : 0; m < (act ? mhi_ : 1); ++m) {
        m_ = m;
        exp_active_ = act;
        const std::string x = ar >= 1 ? body_value(u, L_.kind_a[j], L_.ref_a[j], false) : "";
        const std::string y = ar >= 2 ? body_value(u, L_.kind_b[j], L_.ref_b[j], false) : "";
        std::string val = body_expr(j, u, op, x, y);
        if (!act && draw_fma() && (op == NT_OP_ADD || op == NT_OP_SUB)) {
          const std::string fm = draw_fma_expr(u, j, op);
          if (!fm.empty()) val = fm;
        }
        if (op == NT_OP_EXP && fold_[j].on) {
          const Exp2Fold& f = fold_[j];
          const std::string sv = body_value(u, f.s_kind, f.s_ref, false);
          val = "nt_hw_exp2f(" + f.arg(f.p >= 0 ? l2e_name(f.p) : "", l2e_name(f.r), sv, p_.fuse) + ")";
        }
        sqrt_q_.clear();
        if (op == NT_OP_SQRT && fast_sqrt() && !slow_) {
          const std::string q = "tr" + std::to_string(u) + "_" + std::to_string(j) + "_q" + ms(true);
          o_ << ind << "real " << q << ";\n";
          val = sqrt_expr(x, q, act);
        }
        if (op == NT_OP_EXP && bound_[j].on && !slow_ && !f32_ && p_.libm != 1) val = "nt_exp_core(" + x + ")";
        recip_ = op == NT_OP_DIV && fast_sqrt() && !slow_ &&
                 ((L_.kind_a[j] == ARG_BODY && is_one(s + L_.ref_a[j])) || (L_.kind_a[j] == ARG_INV && is_one(L_.ref_a[j])));
        if (recip_) val = "nt_recip(" + y + ", nt_slow" + ms(act) + ")";
        if (fused_exp_[j] >= 0 && p_.adjoints) {
          const ExpBound& b = bound_[fused_exp_[j]];
          const std::string rv = body_value(u, ARG_INV, b.r, false), pv = body_value(u, ARG_INV, b.p, false);
          const std::string z = body_value(u, ARG_BODY, b.draw, false);
          const bool sub = op == NT_OP_SUB;
          val = f("fma") + "(" + (sub && b.p_first ? "-" + rv : rv) + ", " + z + ", " + (sub && !b.p_first ? "-" + pv : pv) + ")";
        }
        if (gsum_[j] >= 0 && act && p_.adjoints) {
          // sum of G (the spots' sum is A0 + c0 sum G)
          val = body_value(u, ARG_CARRY, j, false) + " + gq" + std::to_string(u) + "_" + std::to_string(gsum_[j]) + ms(true);
        }
        if (!(geo_free(j) && act && p_.adjoints)) o_ << ind << "const real " << name << ms(act) << " = " << val << ";\n";
        if (!act || ar == 0 || !p_.adjoints) continue;
        if (geo(j)) {
          const bool a_self = L_.kind_a[j] == ARG_CARRY && L_.ref_a[j] == j;
          const int e = a_self ? L_.ref_b[j] : L_.ref_a[j];
          const std::string m = ms(true), sj = std::to_string(j), su = std::to_string(u);
          const std::string prev = u > 0 ? std::to_string(u - 1) : "";
          if (gaff(j)) {
            // the sum of s; exponents and tangents follow after the loop
            const GeoAffine& g = gaff_[j];
            o_ << ind << "const real zq" << su << "_" << sj << m << " = "
               << (u > 0 ? "zq" + prev + "_" + sj + m : "zs" + sj + m) << " + "
               << body_value(u, g.s_kind, g.s_ref, false) << ";\n";
            continue;
          }
          if (geo_log(j)) {
            // log G: the sum of the factors' exponents
            o_ << ind << "const real gq" << su << "_" << sj << m << " = "
               << (u > 0 ? "gq" + prev + "_" + sj + m : "gs" + sj + m) << " + " << geo_factor_exponent(u, j) << ";\n";
          } else {
            o_ << ind << "const real gq" << su << "_" << sj << m << " = "
               << (u > 0 ? "gq" + prev + "_" + sj + m : "gs" + sj + m) << " * " << body_value(u, ARG_BODY, e, false)
               << ";\n";
          }
          // the factor's log-derivative per input: tx for exp(x), -tb m for m = 1 / b
          const bool recip = t_.op[s + e] == NT_OP_DIV;
          std::function<std::string(int)> tx;
          body_tangent_operand(u, recip ? L_.kind_b[e] : L_.kind_a[e], recip ? L_.ref_b[e] : L_.ref_a[e], tx);
          const std::vector<int> Dj = posdeplist(j);
          std::string cs = "c0_" + sj + m;  // sigma_k + cs X_k
          if (recip) cs = scalar(ind, "(-(c0_" + sj + m + " * " + body_value(u, ARG_BODY, e, false) + "))");
          // X_k scaled (a base per input times a scale of the node): taken apart
          // when two or more inputs share the scale, one fma per input
          std::map<std::string, int> n;
          for (int k : Dj) {
            auto it = lazy_.find(tx(k));
            if (it != lazy_.end()) ++n[it->second.second];
          }
          bool shared = false;
          for (const auto& kv : n) shared |= kv.second >= 2;
          for (int k : Dj) {
            const std::string sk = std::to_string(k);
            const std::string sp = u > 0 ? "tr" + prev + "_" + sj + "_" + sk + m : "ts" + sj + "_" + sk + m;
            const std::string X = tx(k);
            const std::string name_k = "tr" + su + "_" + sj + "_" + sk + m;
            lazy_.erase(name_k);
            std::string ex;
            if (X.empty()) ex = sp;
            else if (!recip && !lazy_.count(X)) ex = f("fma") + "(" + cs + ", " + (X == "#1" ? (f32_ ? "1.0f" : "1.0") : X) + ", " + sp + ")";
            else ex = sum(Term{sp, "", ""}, scaled(ind, X, cs, shared)).expr;
            o_ << ind << "const " << treal() << " " << name_k << " = " << ex << ";\n";
          }
          continue;
        }
        std::function<std::string(int)> ta, tb;
        body_tangent_operand(u, L_.kind_a[j], L_.ref_a[j], ta);
        body_tangent_operand(u, ar >= 2 ? L_.kind_b[j] : ARG_NONE, ar >= 2 ? L_.ref_b[j] : -1, tb);
        std::vector<int> Dj = posdeplist(j);
        std::vector<int> self;  // a running sum of G: its tangent for these inputs is its value
        if (gsum_[j] >= 0) {
          std::vector<int> rest;
          for (int k : Dj) (gsum_self(j, k) ? self : rest).push_back(k);
          Dj = rest;
        }
        tangent(ind, op, "tr" + std::to_string(u) + "_" + std::to_string(j) + "_", ms(true), Dj, name + ms(true), x, y,
                ta, tb);
        for (int k : self) {
          const std::string tk = "tr" + std::to_string(u) + "_" + std::to_string(j) + "_" + std::to_string(k) + ms(true);
          lazy_.erase(tk);
          o_ << ind << "const " << treal() << " " << tk << " = " << name << ms(true) << ";\n";
        }
        sqrt_q_.clear();
      }
    }
  }
  for (int j = 0; j < P; ++j) {
    if (!(L_.is_carry[j] || L_.is_liveout[j])) continue;
    const bool act = t_.active[s + j] != 0;
    for (int m = act ? mlo_ : 0; m < (act ? mhi_ : 1); ++m) {
      m_ = m;
      const std::string sm = ms(act);
      if (!(geo_free(j) && act && p_.adjoints)) o_ << ind << "st" << j << sm << " = r" << (U - 1) << "_" << j << sm << ";\n";
      if (!act || !p_.adjoints) continue;
      if (gaff(j)) {
        o_ << ind << "zs" << j << sm << " = zq" << (U - 1) << "_" << j << sm << ";\n";
        continue;
      }
      if (geo(j)) o_ << ind << "gs" << j << sm << " = gq" << (U - 1) << "_" << j << sm << ";\n";
      for (int k : posdeplist(j)) {
        o_ << ind << "ts" << j << "_" << k << sm << " = tr" << (U - 1) << "_" << j << "_" << k << sm << ";\n";
      }
    }
  }
  o_ << "    }\n";
  scal_ = outer_scalars;
}

void Emitter::plan_geo_carries() {
  geo_.assign(L_.found ? L_.period : 0, 0);
  if (!L_.found || p_.mode != NT_MODE_TANGENT || !p_.adjoints) return;
  for (int j = 0; j < L_.period; ++j) {
    if (!L_.is_carry[j] || !t_.active[L_.start + j] || t_.op[L_.start + j] != NT_OP_MUL) continue;
    const bool a_self = L_.kind_a[j] == ARG_CARRY && L_.ref_a[j] == j;
    const bool b_self = L_.kind_b[j] == ARG_CARRY && L_.ref_b[j] == j;
    if (a_self == b_self) continue;
    const int ek = a_self ? L_.kind_b[j] : L_.kind_a[j], er = a_self ? L_.ref_b[j] : L_.ref_a[j];
    if (ek != ARG_BODY || !(single_body_exp(er) || single_body_recip(er))) continue;
    // Worth it when the saving (one operation per input of the carry's
    // tangent) beats the multiply for G plus one multiply per input that some
    // consumer needs as an absolute tangent G sigma_k. The tangent G sigma_k
    // is a scaled tangent (base sigma_k, scale G): a unary rule, or a binary
    // one whose other operand has no tangent for input k, scales it further
    // at no cost per input, and a sum or difference takes it as one fma; a
    // product, quotient, max or min with an operand that has a tangent for k
    // as well pays the multiply.
    const std::vector<int> D = posdeplist(j);
    std::vector<char> need(static_cast<size_t>(t_.n_in) + par_node_.size(), 0);  // per input or parameter
    for (int q = 0; q < L_.period; ++q) {
      const int oq = t_.op[L_.start + q];
      const int ar = arity(oq);
      if (ar < 2 || oq == NT_OP_ADD || oq == NT_OP_SUB) continue;
      for (int slot = 0; slot < ar; ++slot) {
        const int kind = slot ? L_.kind_b[q] : L_.kind_a[q], ref = slot ? L_.ref_b[q] : L_.ref_a[q];
        if (!((kind == ARG_BODY || kind == ARG_CARRY) && ref == j) || (q == j && kind == ARG_CARRY)) continue;
        const int okind = slot ? L_.kind_a[q] : L_.kind_b[q], oref = slot ? L_.ref_a[q] : L_.ref_b[q];
        for (int k : D) {
          bool other = false;
          if (okind == ARG_BODY || okind == ARG_CARRY) other = poshas(oref, k);
          else if (okind == ARG_INV) other = !inv_tname(oref, k).empty();
          if (other) need[k] = 1;
        }
      }
    }
    int materialised = 0;
    for (int k : D) materialised += need[k];
    if (static_cast<int>(D.size()) - 1 - materialised > 0) geo_[j] = 1;
  }
}

// The loop's parameters: the values from outside the loop that active body
// positions read, and the start values of active carries (a node read both
// ways is one parameter: its tangent for each input counts once). A loop
// position depends on a parameter it reads, directly, through an earlier
// position or through a carry (whose state starts at its start value).
void Emitter::plan_parameters() {
  use_par_ = false;
  par_on_ = false;
  par_node_.clear();
  par_of_.clear();
  par_deps_.clear();
  // a schedule computed once per block carries its tangents over the inputs
  if (!L_.found || p_.mode != NT_MODE_TANGENT || !p_.adjoints || p_.basis == 1 || sched_on_) return;
  const int P = L_.period, s = L_.start;
  auto add = [&](int node) {
    if (node < 0 || !t_.active[node] || par_of_.count(node)) return;
    par_of_[node] = static_cast<int>(par_node_.size());
    par_node_.push_back(node);
  };
  for (int j = 0; j < P; ++j) {
    if (!t_.active[s + j]) continue;
    const int ar = arity(t_.op[s + j]);
    if (ar >= 1 && L_.kind_a[j] == ARG_INV) add(L_.ref_a[j]);
    if (ar >= 2 && L_.kind_b[j] == ARG_INV) add(L_.ref_b[j]);
    if (L_.is_carry[j]) add(L_.carry_init[j]);
  }
  const int nd = static_cast<int>(par_node_.size());
  par_deps_.assign(static_cast<size_t>(P), std::vector<char>(static_cast<size_t>(nd), 0));
  for (bool changed = true; changed;) {
    changed = false;
    auto mark = [&](std::vector<char>& d, int q) {
      if (!d[q]) d[q] = 1, changed = true;
    };
    for (int j = 0; j < P; ++j) {
      if (!t_.active[s + j]) continue;
      std::vector<char>& d = par_deps_[j];
      if (L_.is_carry[j]) {
        auto it = par_of_.find(L_.carry_init[j]);
        if (it != par_of_.end()) mark(d, it->second);
      }
      const int ar = arity(t_.op[s + j]);
      for (int slot = 0; slot < ar; ++slot) {
        const int kind = slot ? L_.kind_b[j] : L_.kind_a[j], ref = slot ? L_.ref_b[j] : L_.ref_a[j];
        if (kind == ARG_INV) {
          auto it = par_of_.find(ref);
          if (it != par_of_.end()) mark(d, it->second);
        } else if (kind == ARG_BODY || kind == ARG_CARRY) {
          for (int q = 0; q < nd; ++q) {
            if (par_deps_[ref][q]) mark(d, q);
          }
        }
      }
    }
  }
  // Tangents per step: one per (active position, input or parameter) pair;
  // the parameters win when they make fewer. On a tie, fp32 takes them too:
  // a parameter's tangent for itself is 1, so the rules that read it multiply
  // by nothing (the worst-of basket: 128 tangents per step either way, 3 %
  // fewer instructions over parameters; measured 2.4 % faster in fp32 and
  // 3 % slower in fp64, whose kernel runs one wave per SIMD and depends on
  // the schedule's slack more than on the instruction count).
  int by_input = 0, by_par = 0;
  for (int j = 0; j < P; ++j) {
    if (!t_.active[s + j]) continue;
    by_input += popcount(&p_.posdeps[static_cast<size_t>(j) * p_.n_words], p_.n_words);
    for (char c : par_deps_[j]) by_par += c;
  }
  use_par_ = p_.basis == 2 || (by_par > 0 && (by_par < by_input || (by_par == by_input && f32_)));
}

void Emitter::plan_geo_sums() {
  gsum_.assign(L_.found ? L_.period : 0, -1);
  gsum_of_.assign(L_.found ? L_.period : 0, -1);
  if (!L_.found) return;
  for (int a = 0; a < L_.period; ++a) {
    if (!L_.is_carry[a] || !t_.active[L_.start + a] || t_.op[L_.start + a] != NT_OP_ADD) continue;
    if (body_uses_[a] != 1 + (L_.is_liveout[a] ? 1 : 0)) continue;
    const bool a_self = L_.kind_a[a] == ARG_CARRY && L_.ref_a[a] == a;
    const bool b_self = L_.kind_b[a] == ARG_CARRY && L_.ref_b[a] == a;
    if (a_self == b_self) continue;
    const int ok = a_self ? L_.kind_b[a] : L_.kind_a[a], j = a_self ? L_.ref_b[a] : L_.ref_a[a];
    if (ok != ARG_BODY || !geo(j) || gsum_of_[j] >= 0) continue;
    if (body_uses_[j] != 2 + (L_.is_liveout[j] ? 1 : 0)) continue;
    gsum_[a] = j;
    gsum_of_[j] = a;
  }
}

void Emitter::plan_geo_logs() {
  geo_log_.assign(L_.found ? L_.period : 0, 0);
  if (!L_.found) return;
  for (int j = 0; j < L_.period; ++j) {
    if (!geo(j) || !geo_free(j) || gsum_of_[j] >= 0) continue;
    const bool a_self = L_.kind_a[j] == ARG_CARRY && L_.ref_a[j] == j;
    const int e = a_self ? L_.ref_b[j] : L_.ref_a[j];
    // a factor from the block's schedule (a deterministic growth exp(r dt_i))
    // is read from LDS whole: its exponent is not in the step
    if (sched_on_ && sched_[e]) continue;
    if (t_.op[L_.start + e] == NT_OP_EXP && single_body_exp(e)) geo_log_[j] = 1;
  }
}

// Exponent of geo carry j's factor in iteration u of the trip (log2 units
// where the fp32 factor is a folded exp2).
std::string Emitter::geo_factor_exponent(int u, int j) const {
  const bool a_self = L_.kind_a[j] == ARG_CARRY && L_.ref_a[j] == j;
  const int e = a_self ? L_.ref_b[j] : L_.ref_a[j];
  if (fold_[e].on) {
    const Exp2Fold& f = fold_[e];
    const std::string sv = body_value(u, f.s_kind, f.s_ref, false);
    return f.arg(f.p >= 0 ? l2e_name(f.p) : "", l2e_name(f.r), sv, p_.fuse);
  }
  return body_value(u, L_.kind_a[e], L_.ref_a[e], false);
}

std::string Emitter::draw_fma_expr(int u, int j, int op) const {
  for (int side = 1; side >= 0; --side) {
    const int mk = side ? L_.kind_b[j] : L_.kind_a[j], mr = side ? L_.ref_b[j] : L_.ref_a[j];
    if (mk != ARG_BODY || t_.op[L_.start + mr] != NT_OP_MUL || body_uses_[mr] != 1 || t_.active[L_.start + mr] ||
        L_.is_liveout[mr] || L_.is_carry[mr])
      continue;
    const int ok = side ? L_.kind_a[j] : L_.kind_b[j], orf = side ? L_.ref_a[j] : L_.ref_b[j];
    const std::string a = body_value(u, L_.kind_a[mr], L_.ref_a[mr], false);
    const std::string b = body_value(u, L_.kind_b[mr], L_.ref_b[mr], false);
    const std::string o = body_value(u, ok, orf, false);
    if (op == NT_OP_ADD) return "fma(" + a + ", " + b + ", " + o + ")";
    return side ? "fma(-(" + a + "), " + b + ", " + o + ")" : "fma(" + a + ", " + b + ", -(" + o + "))";
  }
  return std::string();
}

void Emitter::plan_geo_affine() {
  gaff_.assign(L_.found ? L_.period : 0, GeoAffine());
  if (!L_.found || !p_.fuse) return;
  for (int j = 0; j < L_.period; ++j) {
    if (!geo_log_[j]) continue;
    const bool a_self = L_.kind_a[j] == ARG_CARRY && L_.ref_a[j] == j;
    const int e = a_self ? L_.ref_b[j] : L_.ref_a[j];
    GeoAffine g;
    if (f32_) {
      const Exp2Fold& f = fold_[e];
      if (!f.on) continue;
      g.p = f.p;
      g.r = f.r;
      g.s_kind = f.s_kind;
      g.s_ref = f.s_ref;
      g.neg_p = f.neg_p;
      g.neg_r = f.neg_r;
    } else {
      const ExpBound& b = bound_[e];
      if (!b.on) continue;
      if (b.sum >= 0 ? fused_exp_[b.sum] != e
                     : !(L_.kind_a[e] == ARG_BODY && L_.ref_a[e] == b.mul && body_uses_[b.mul] == 1))
        continue;
      const bool sub = b.sum >= 0 && t_.op[L_.start + b.sum] == NT_OP_SUB;
      g.p = b.p;
      g.r = b.r;
      g.s_kind = ARG_BODY;
      g.s_ref = b.draw;
      g.neg_r = sub && b.p_first;
      g.neg_p = sub && !b.p_first;
    }
    // s must carry no tangent: only then is the exponent's tangent affine in s
    if (g.s_kind != ARG_BODY || t_.active[L_.start + g.s_ref]) continue;
    g.on = true;
    gaff_[j] = g;
  }
}

// After the loop: geo carry j's exponent sum N p + r S (log2 units where the
// fp32 factor is a folded exp2) and sigma_k += c0 (N tp_k + tr_k S).
void Emitter::geo_affine_finish(int j) {
  const GeoAffine& g = gaff_[j];
  const std::string m = ms(true), sj = std::to_string(j);
  const std::string S = "zs" + sj + m, N = lit(static_cast<double>(L_.iters));
  const bool fold = f32_;  // fp32 factors are folded exp2s: p and r scaled by log2(e)
  const std::string rv = (g.neg_r ? "-" : "") + (fold ? l2e_name(g.r) : vname(g.r));
  std::string e = rv + " * " + S;
  if (g.p >= 0) {
    const std::string pv = (g.neg_p ? "-" : "") + (fold ? l2e_name(g.p) : vname(g.p));
    e = f("fma") + "(" + rv + ", " + S + ", " + N + " * " + pv + ")";
  }
  o_ << "    gs" << sj << m << " = " << e << ";\n";
  for (int k : posdeplist(j)) {
    const std::string tp = g.p >= 0 ? inv_tname(g.p, k) : std::string(), tr = inv_tname(g.r, k);
    std::string x;
    if (!tp.empty()) x = tp == "#1" ? N : N + " * " + tp;
    if (g.neg_p && !x.empty()) x = "-(" + x + ")";
    if (!tr.empty()) {
      const std::string rs = tr == "#1" ? S : tr + " * " + S;
      x = x.empty() ? (g.neg_r ? "-(" + rs + ")" : rs) : x + (g.neg_r ? " - " : " + ") + rs;
    }
    if (x.empty()) continue;
    const std::string ts = "ts" + sj + "_" + std::to_string(k) + m;
    o_ << "    " << ts << " = " << f("fma") << "(c0_" << sj << m << ", " << x << ", " << ts << ");\n";
  }
}

void Emitter::plan_exp2_folds() {
  fold_.assign(L_.found ? L_.period : 0, Exp2Fold());
  if (!f32_ || !L_.found || p_.mode != NT_MODE_TANGENT) return;
  auto body_only = [&](int pos) { return body_uses_[pos] == 1 && !L_.is_liveout[pos] && !L_.is_carry[pos]; };
  for (int j = 0; j < L_.period; ++j) {
    if (t_.op[L_.start + j] != NT_OP_EXP || L_.kind_a[j] != ARG_BODY || !body_only(L_.ref_a[j])) continue;
    const int a = L_.ref_a[j];
    Exp2Fold f;
    int mul = -1;
    if (t_.op[L_.start + a] == NT_OP_ADD || t_.op[L_.start + a] == NT_OP_SUB) {
      const bool sub = t_.op[L_.start + a] == NT_OP_SUB;
      for (int side = 0; side < 2 && mul < 0; ++side) {
        const int ik = side ? L_.kind_b[a] : L_.kind_a[a], ir = side ? L_.ref_b[a] : L_.ref_a[a];
        const int mk = side ? L_.kind_a[a] : L_.kind_b[a], mr = side ? L_.ref_a[a] : L_.ref_b[a];
        if (ik == ARG_INV && mk == ARG_BODY && t_.op[L_.start + mr] == NT_OP_MUL && body_only(mr)) {
          f.p = ir;
          mul = mr;
          f.neg_r = sub && side == 0;  // p - r s
          f.neg_p = sub && side == 1;  // r s - p
        }
      }
    } else if (t_.op[L_.start + a] == NT_OP_MUL) {
      mul = a;
    }
    if (mul < 0) continue;
    for (int side = 0; side < 2 && !f.on; ++side) {
      const int ik = side ? L_.kind_b[mul] : L_.kind_a[mul], ir = side ? L_.ref_b[mul] : L_.ref_a[mul];
      if (ik != ARG_INV) continue;
      f.r = ir;
      f.s_kind = side ? L_.kind_a[mul] : L_.kind_b[mul];
      f.s_ref = side ? L_.ref_a[mul] : L_.ref_b[mul];
      f.on = true;
    }
    if (f.on) fold_[j] = f;
  }
}

void Emitter::plan_exp_bounds() {
  bound_.assign(L_.found ? L_.period : 0, ExpBound());
  if (f32_ || p_.libm == 1 || !L_.found || p_.mode != NT_MODE_TANGENT) return;
  // Largest magnitude a body value built from draws and literals alone can
  // take (a correlated normal: a literal row of a Cholesky factor times the
  // step's normals), or -1: a normal is at most 6.77, a uniform at most 1,
  // sums and products bound by the sums and products of their operands' bounds.
  std::vector<double> zb(L_.period, -2.0);  // -2: not yet known
  std::function<double(int, int)> zbound = [&](int kind, int ref) -> double {
    if (kind == ARG_INV) return t_.op[ref] == NT_OP_CONST ? std::fabs(t_.c[ref]) : -1.0;
    if (kind != ARG_BODY) return -1.0;
    if (zb[ref] > -2.0) return zb[ref];
    double v = -1.0;
    const int op = t_.op[L_.start + ref];
    if (op == NT_OP_RANDN) v = 6.77;
    else if (op == NT_OP_RANDU) v = 1.0;
    else if (op == NT_OP_CONST) {
      v = std::fabs(t_.c[L_.start + ref]);
      if (L_.table_lit(ref)) {
        for (double x : L_.lit_values[ref]) v = std::max(v, std::fabs(x));
      }
    } else if (op == NT_OP_NEG) {
      v = zbound(L_.kind_a[ref], L_.ref_a[ref]);
    } else if (op == NT_OP_ADD || op == NT_OP_SUB || op == NT_OP_MUL) {
      const double a = zbound(L_.kind_a[ref], L_.ref_a[ref]), b = zbound(L_.kind_b[ref], L_.ref_b[ref]);
      if (a >= 0.0 && b >= 0.0) v = op == NT_OP_MUL ? a * b : a + b;
    }
    // the bound of the computed value, not only of the exact one: a margin
    // far above the roundings of a few dozen operations
    if (v >= 0.0 && op != NT_OP_RANDN && op != NT_OP_RANDU && op != NT_OP_CONST) v *= 1.0 + 1e-9;
    if (!(v <= 1e300)) v = -1.0;
    return zb[ref] = v;
  };
  // r z with r invariant and z bounded: the node at loop position m; sets r,
  // z's position and its bound
  int draw = -1;
  double zmax = 0.0;
  auto scaled_draw = [&](int m, int& r) {
    if (t_.op[L_.start + m] != NT_OP_MUL) return false;
    for (int side = 0; side < 2; ++side) {
      const int ik = side ? L_.kind_b[m] : L_.kind_a[m], ir = side ? L_.ref_b[m] : L_.ref_a[m];
      const int dk = side ? L_.kind_a[m] : L_.kind_b[m], dr = side ? L_.ref_a[m] : L_.ref_b[m];
      if (ik != ARG_INV || dk != ARG_BODY) continue;
      const double zm = zbound(dk, dr);
      if (zm < 0.0) continue;
      r = ir;
      draw = dr;
      zmax = zm;
      return true;
    }
    return false;
  };
  for (int j = 0; j < L_.period; ++j) {
    if (t_.op[L_.start + j] != NT_OP_EXP || L_.kind_a[j] != ARG_BODY) continue;
    const int a = L_.ref_a[j];
    ExpBound b;
    if (scaled_draw(a, b.r)) {
      b.on = true;
      b.mul = a;
    } else if (t_.op[L_.start + a] == NT_OP_ADD || t_.op[L_.start + a] == NT_OP_SUB) {
      for (int side = 0; side < 2 && !b.on; ++side) {
        const int ik = side ? L_.kind_b[a] : L_.kind_a[a], ir = side ? L_.ref_b[a] : L_.ref_a[a];
        const int mk = side ? L_.kind_a[a] : L_.kind_b[a], mr = side ? L_.ref_a[a] : L_.ref_b[a];
        if (ik == ARG_INV && mk == ARG_BODY && scaled_draw(mr, b.r)) {
          b.p = ir;
          b.on = true;
          b.sum = a;
          b.mul = mr;
          b.p_first = side == 0 || t_.op[L_.start + a] == NT_OP_ADD;
        }
      }
    }
    if (b.on) {
      b.draw = draw;
      b.zmax = zmax;
      bound_[j] = b;
    }
  }
}

void Emitter::plan_fused_exponents() {
  fused_exp_.assign(L_.found ? L_.period : 0, -1);
  if (!L_.found || !p_.fuse) return;
  for (int c = 0; c < L_.period; ++c) {
    if (!geo(c) || !(geo_free(c) || gsum_of_[c] >= 0)) continue;
    const bool a_self = L_.kind_a[c] == ARG_CARRY && L_.ref_a[c] == c;
    const int e = a_self ? L_.ref_b[c] : L_.ref_a[c];
    if (t_.op[L_.start + e] != NT_OP_EXP || !single_body_exp(e)) continue;
    const ExpBound& b = bound_[e];
    if (!b.on || b.sum < 0 || body_uses_[b.sum] != 1 || body_uses_[b.mul] != 1) continue;
    fused_exp_[b.sum] = e;
  }
}

void Emitter::plan_schedule() {
  sched_on_ = false;
  sched_rows_ = 0;
  sched_.assign(L_.found ? L_.period : 0, 0);
  sched_slot_.assign(L_.found ? L_.period : 0, -1);
  if (!L_.found || p_.mode != NT_MODE_TANGENT || p_.markets > 1) return;
  const int P = L_.period, s = L_.start;
  std::vector<char> drawfree(s, 1);
  for (int i = 0; i < s; ++i) {
    const int op = t_.op[i], ar = arity(op);
    if (op == NT_OP_RANDN || op == NT_OP_RANDU) drawfree[i] = 0;
    if (ar >= 1 && !drawfree[t_.a[i]]) drawfree[i] = 0;
    if (ar >= 2 && !drawfree[t_.b[i]]) drawfree[i] = 0;
  }
  std::vector<char> vary(P, 0);  // reads a per-step literal
  for (int j = 0; j < P; ++j) {
    const int op = t_.op[s + j], ar = arity(op);
    if (op == NT_OP_RANDN || op == NT_OP_RANDU) continue;
    if (op == NT_OP_CONST) {
      sched_[j] = 1;
      vary[j] = L_.table_lit(j);
      continue;
    }
    bool ok = true;
    for (int slot = 0; slot < ar; ++slot) {
      const int kind = slot == 0 ? L_.kind_a[j] : L_.kind_b[j];
      const int ref = slot == 0 ? L_.ref_a[j] : L_.ref_b[j];
      if (kind == ARG_BODY) {
        ok = ok && sched_[ref];
        vary[j] = vary[j] || vary[ref];
      } else if (kind == ARG_INV) {
        ok = ok && drawfree[ref];
      } else {
        ok = false;
      }
    }
    sched_[j] = ok;
  }
  // the schedule values the rest of the step reads
  std::vector<char> out(P, 0);
  for (int k = 0; k < P; ++k) {
    if (sched_[k]) continue;
    const int ar = arity(t_.op[s + k]);
    for (int slot = 0; slot < ar; ++slot) {
      const int kind = slot == 0 ? L_.kind_a[k] : L_.kind_b[k];
      const int ref = slot == 0 ? L_.ref_a[k] : L_.ref_b[k];
      if (kind == ARG_BODY && sched_[ref] && t_.op[s + ref] != NT_OP_CONST) out[ref] = 1;
    }
  }
  int rows = 0;
  bool any = false;
  for (int j = 0; j < P; ++j) {
    if (!sched_[j] || t_.op[s + j] == NT_OP_CONST) continue;
    if (L_.is_carry[j] || L_.is_liveout[j]) return;
    if (!out[j]) continue;
    // its tangents are stored for the inputs its first iteration depends on
    // and read for those the loop position depends on: the same set for a
    // value no carried state reaches
    if (p_.adjoints && deplist(s + j) != posdeplist(j)) return;
    any = any || vary[j];
    sched_slot_[j] = rows;
    rows += 1 + (p_.adjoints ? static_cast<int>(posdeplist(j).size()) : 0);
  }
  const long bytes = static_cast<long>(rows) * L_.iters * (f32_ ? 4 : 8);
  if (!any || bytes > 32 * 1024) {
    sched_slot_.assign(P, -1);
    return;
  }
  sched_on_ = true;
  sched_rows_ = rows;
}

// The block's schedule: the pre-loop values it reads (the same for every
// iteration), then every iteration's schedule values and tangents, threads
// striding over the iterations, stored in LDS rows of nt_sch[row][iteration].
// Values use correctly rounded or device-libm functions, so they are the
// oracle's; tangents follow the reference's local rules (ScalarReplay.java:
// 129-183, taken forward).
void Emitter::schedule_prologue() {
  if (!sched_on_ || slow_) return;
  const int P = L_.period, s = L_.start, I = L_.iters;
  const std::string zero = f32_ ? "0.0f" : "0.0", one = f32_ ? "1.0f" : "1.0", half = f32_ ? "0.5f" : "0.5";
  std::vector<char> cone(s, 0);
  std::function<void(int)> need = [&](int node) {
    if (node < 0 || node >= s || cone[node]) return;
    cone[node] = 1;
    const int ar = arity(t_.op[node]);
    if (ar >= 1) need(t_.a[node]);
    if (ar >= 2) need(t_.b[node]);
  };
  for (int j = 0; j < P; ++j) {
    if (!sched_[j]) continue;
    const int ar = arity(t_.op[s + j]);
    if (ar >= 1 && L_.kind_a[j] == ARG_INV) need(L_.ref_a[j]);
    if (ar >= 2 && L_.kind_b[j] == ARG_INV) need(L_.ref_b[j]);
  }
  // value and tangent names: pre-loop node q<node>, schedule position qs<j>
  auto val = [&](int kind, int ref) { return kind == ARG_BODY ? "qs" + std::to_string(ref) : "q" + std::to_string(ref); };
  auto tan = [&](int kind, int ref, int k) -> std::string {
    const int node = kind == ARG_BODY ? s + ref : ref;
    if (!p_.adjoints || !has(node, k)) return "";
    if (t_.op[node] == NT_OP_INPUT) return one;
    return val(kind, ref) + "_" + std::to_string(k);
  };
  auto plus = [&](const std::string& x, const std::string& y, bool minus) -> std::string {
    if (y.empty()) return x;
    if (x.empty()) return minus ? "(-" + y + ")" : y;
    return "(" + x + (minus ? " - " : " + ") + y + ")";
  };
  auto times = [&](const std::string& t, const std::string& factor) -> std::string {
    return t.empty() ? "" : "(" + t + " * " + factor + ")";
  };
  auto emit = [&](const std::string& ind, int node, int op, const std::string& name, int ka, int ra, int kb, int rb,
                  const std::string& value) {
    o_ << ind << "const real " << name << " = " << value << ";\n";
    if (!p_.adjoints || op == NT_OP_CONST || op == NT_OP_INPUT) return;
    const std::string va = arity(op) >= 1 ? val(ka, ra) : "", vb = arity(op) >= 2 ? val(kb, rb) : "";
    for (int k : deplist(node)) {
      const std::string ta = arity(op) >= 1 ? tan(ka, ra, k) : "", tb = arity(op) >= 2 ? tan(kb, rb, k) : "";
      std::string e;
      switch (op) {
        case NT_OP_ADD: e = plus(ta, tb, false); break;
        case NT_OP_SUB: e = plus(ta, tb, true); break;
        case NT_OP_MUL: e = plus(times(ta, vb), times(tb, va), false); break;
        case NT_OP_DIV: e = plus(ta.empty() ? "" : "(" + ta + " / " + vb + ")",
                                 tb.empty() ? "" : "(" + tb + " * " + name + " / " + vb + ")", true); break;
        case NT_OP_NEG: e = ta.empty() ? "" : "(-" + ta + ")"; break;
        case NT_OP_EXP: e = times(ta, name); break;
        case NT_OP_LOG: e = ta.empty() ? "" : "(" + ta + " / " + va + ")"; break;
        case NT_OP_SQRT: e = ta.empty() ? "" : "(" + ta + " * " + half + " / " + name + ")"; break;
        case NT_OP_ABS: e = ta.empty() ? "" : "(" + va + " < " + zero + " ? -" + ta + " : " + ta + ")"; break;
        case NT_OP_MAX: case NT_OP_MIN: {
          const std::string cmp = op == NT_OP_MAX ? " >= " : " <= ";
          e = "(" + va + cmp + vb + " ? " + (ta.empty() ? zero : ta) + " : " + (tb.empty() ? zero : tb) + ")";
          break;
        }
        default: break;
      }
      o_ << ind << "const real " << name << "_" << k << " = " << (e.empty() ? zero : e) << ";\n";
    }
  };
  auto fn_value = [&](int op, const std::string& x, const std::string& y, const std::string& lit_value, int a) {
    switch (op) {
      case NT_OP_EXP: return std::string(f32_ ? "expf(" : "exp(") + x + ")";
      case NT_OP_LOG: return std::string(f32_ ? "logf(" : "log(") + x + ")";
      case NT_OP_SQRT: return std::string(f32_ ? "sqrtf(" : "sqrt(") + x + ")";
      case NT_OP_DIV: return x + " / " + y;
      case NT_OP_CONST: return lit_value;
      default: return expr(op, x, y, 0.0, a);
    }
  };
  o_ << "  __shared__ real nt_sch[" << sched_rows_ << " * " << I << "];\n";
  o_ << "  {\n";
  for (int i = 0; i < s; ++i) {
    if (!cone[i]) continue;
    const int op = t_.op[i], ar = arity(op);
    const std::string x = ar >= 1 ? val(ARG_INV, t_.a[i]) : "", y = ar >= 2 ? val(ARG_INV, t_.b[i]) : "";
    emit("    ", i, op, "q" + std::to_string(i), ARG_INV, ar >= 1 ? t_.a[i] : -1, ARG_INV, ar >= 2 ? t_.b[i] : -1,
         fn_value(op, x, y, lit(t_.c[i]), t_.a[i]));
  }
  o_ << "#ifdef NT_HOST_EMU\n    for (nt_u32 it = 0; it < " << I << "u; ++it) {\n#else\n";
  o_ << "    for (nt_u32 it = threadIdx.x; it < " << I << "u; it += blockDim.x) {\n#endif\n";
  o_ << "      const nt_u32 it0 = it;\n";
  for (int j = 0; j < P; ++j) {
    if (!sched_[j]) continue;
    const int op = t_.op[s + j], ar = arity(op);
    const std::string x = ar >= 1 ? val(L_.kind_a[j], L_.ref_a[j]) : "";
    const std::string y = ar >= 2 ? val(L_.kind_b[j], L_.ref_b[j]) : "";
    const std::string lv = L_.table_lit(j) ? "nt_lit" + std::to_string(j) + "[it0]" : lit(t_.c[s + j]);
    emit("      ", s + j, op, "qs" + std::to_string(j), L_.kind_a[j], L_.ref_a[j], L_.kind_b[j], L_.ref_b[j],
         fn_value(op, x, y, lv, t_.a[s + j]));
    if (sched_slot_[j] < 0) continue;
    int row = sched_slot_[j];
    o_ << "      nt_sch[" << row++ << "u * " << I << "u + it] = qs" << j << ";\n";
    if (!p_.adjoints) continue;
    for (int k : posdeplist(j)) o_ << "      nt_sch[" << row++ << "u * " << I << "u + it] = qs" << j << "_" << k << ";\n";
  }
  o_ << "    }\n  }\n  __syncthreads();\n";
}

void Emitter::exp_bound_checks() {
  if (slow_) return;
  for (int j = 0; j < static_cast<int>(bound_.size()); ++j) {
    const ExpBound& b = bound_[j];
    if (!b.on) continue;
    const bool act = t_.active[L_.start + j] != 0;
    for (int m = act ? mlo_ : 0; m < (act ? mhi_ : 1); ++m) {
      m_ = m;
      const std::string off = b.p >= 0 ? "fabs(" + vname(b.p) + ") + " : std::string();
      const std::string zm = b.zmax == 6.77 ? std::string("6.77") : lit(b.zmax);
      o_ << "    nt_slow" << ms(act) << " |= !(" << off << zm << " * fabs(" << vname(b.r) << ") <= 708.0);\n";
    }
  }
}

void Emitter::count_uses() {
  uses_.assign(t_.n, 0);
  for (int i = 0; i < t_.n; ++i) {
    const int ar = arity(t_.op[i]);
    if (ar >= 1) ++uses_[t_.a[i]];
    if (ar >= 2) ++uses_[t_.b[i]];
  }
  for (int out : t_.outputs) ++uses_[out];
  body_uses_.clear();
  if (!L_.found) return;
  body_uses_.assign(L_.period, 0);
  for (int j = 0; j < L_.period; ++j) {
    const int ar = arity(t_.op[L_.start + j]);
    for (int slot = 0; slot < ar; ++slot) {
      const int kind = slot == 0 ? L_.kind_a[j] : L_.kind_b[j];
      const int ref = slot == 0 ? L_.ref_a[j] : L_.ref_b[j];
      if (kind == ARG_BODY || kind == ARG_CARRY) ++body_uses_[ref];
    }
    if (L_.is_liveout[j]) ++body_uses_[j];
  }
}

void Emitter::preamble() {
  const int n = t_.n;
  const int nin = t_.n_in;
  const bool loop = L_.found;
  const bool tangent = p_.mode == NT_MODE_TANGENT;
  o_ << "// generated by nablatensor_amd lowering: " << n << " nodes, " << nin << " inputs, "
     << (loop ? "rolled loop" : "straight line") << (tangent ? ", tangent mode" : "") << "\n";
  if (loop && tangent) {
    o_ << "// loop: start " << L_.start << ", period " << L_.period << ", iterations " << L_.iters << ", draws/iter "
       << L_.draws << ", " << p_.seg << " iterations per trip (" << p_.nseg_full << " trips + tail " << p_.tail << ")\n";
  } else if (loop) {
    o_ << "// loop: start " << L_.start << ", period " << L_.period << ", iterations " << L_.iters << ", draws/iter "
       << L_.draws << ", segment " << p_.seg << " (" << p_.nseg_full << " full + tail " << p_.tail
       << "), checkpoint policy " << p_.ckpt << ", stored/iter " << p_.n_stored << "\n";
  } else if (!p_.lbound.empty() && !tangent) {
    o_ << "// checkpointed straight line: " << p_.lbound.size() - 1 << " segments of about " << p_.seg
       << " nodes, " << p_.tape_slots << " values stored per path, " << p_.kf << " values and " << p_.ka
       << " adjoints carried\n";
  }
  if (tangent) {
    o_ << "// nt-plan: tape_slots=0 seg=" << p_.seg << " ckpt=0 mode=tangent basis="
       << (use_par_ ? "params" : "inputs") << " params=" << (use_par_ ? par_node_.size() : 0)
       << " schedule=" << (sched_on_ ? sched_rows_ : 0) << "\n";
    // Polynomial constants held in VGPRs make v_fmac_f64 (accumulator tied to
    // the destination) cost a 64-bit copy per term; the three-source v_fma_f64
    // needs none. (The reverse sweep below asks for the same.)
    if (!f32_) o_ << "// nt-compile: -fmacf64-inst\n";
  } else {
    o_ << "// nt-plan: tape_slots=" << p_.tape_slots << " seg=" << p_.seg << " ckpt=" << p_.ckpt << " mode=reverse\n";
    if (!f32_) o_ << "// nt-compile: -fmacf64-inst\n";
  }
  if (p_.cost_reverse > 0 || p_.cost_tangent > 0) {
    // the cost model's estimates per path (VALU instructions) behind the choice of mode
    o_ << "// nt-cost: forward=" << static_cast<long>(p_.cost_forward + 0.5)
       << " reverse=" << static_cast<long>(p_.cost_reverse + 0.5)
       << " tangent=" << static_cast<long>(p_.cost_tangent + 0.5) << "\n";
  }
  o_ << "#pragma clang fp contract(" << (p_.contract ? "fast" : "off") << ")\n";
  if (p_.libm == 1) o_ << "#define NT_DEVICE_LIBM 1\n";
  if (p_.libm == 2) o_ << "#define NT_LIBM_SINCOS 1\n";
  o_ << "#include \"nt_skeleton.h\"\n";
  o_ << "typedef " << (f32_ ? "float" : "double") << " real;\n";
  if (fallback()) o_ << "#define NT_HAS_SLOW 1\n";
  for (int j = 0; loop && j < L_.period; ++j) {
    if (!L_.table_lit(j)) continue;
    o_ << "__constant__ real nt_lit" << j << "[" << L_.iters << "] = {";
    for (int it = 0; it < L_.iters; ++it) o_ << (it ? ", " : "") << lit(L_.lit_values[j][it]);
    o_ << "};\n";
  }
}

// Signature and prologue of the replay kernel (nt_replay) or of the exception
// kernel (nt_replay_slow), up to the path variables of the grid-stride loop.
// Both take `flags`: word 0 counts the lanes that left paths to the exception
// kernel, then one lane bitmap per market, T / 64 words each (bit tid % 64 of
// word tid / 64; the two kernels run on the same grid). The exception kernel
// returns at once when the count is zero (the finishing pass then skips its
// rows); otherwise each lane takes its bit (clearing the bitmap behind it),
// visits its paths only if the bit is set, and a block with no such lane loads
// no tables and writes zero partials.
void Emitter::kernel_head(bool slow) {
  const int nin = t_.n_in;
  const int M = p_.markets;
  o_ << "\nextern \"C\" __global__ __launch_bounds__(" << p_.block;
  if (p_.waves > 0 && !slow) o_ << ", " << p_.waves;
  o_ << ") void " << (slow ? "nt_replay_slow" : "nt_replay") << "(\n"
     << "    const double* __restrict__ inputs, nt_u64 n_paths, nt_u64 path_offset, nt_u64 seed,\n"
     << "    double* __restrict__ partials, real* __restrict__ scratch,\n"
     << "    double* __restrict__ out_v, double* __restrict__ out_g, nt_u64* __restrict__ flags) {\n";
  o_ << "  const nt_u64 T = (nt_u64)gridDim.x * blockDim.x;\n";
  o_ << "  const nt_u64 tid = (nt_u64)blockIdx.x * blockDim.x + threadIdx.x;\n";
  if (slow) o_ << "  if (flags[0] == 0) return;  // no lane left a path to this kernel\n";
  o_ << "  const nt_u64 nt_words = T >> 6;  // lane bitmap words per market\n";
  o_ << "  nt_u64* __restrict__ nt_bits = flags + 1;\n";
  o_ << "  (void)scratch; (void)out_v; (void)out_g; (void)nt_bits; (void)nt_words;\n";
  const int nacc = p_.n_channels * M;
  o_ << "  double acc[" << nacc << "];\n";
  o_ << "  for (int c = 0; c < " << nacc << "; ++c) acc[c] = 0.0;\n";
  if (slow) {
    for (int m = 0; m < M; ++m) {
      o_ << "  const bool nt_f" << m << " = nt_take_lane_flag(nt_bits + " << m << "u * nt_words, tid);\n";
    }
    o_ << "  const bool nt_any = nt_f0";
    for (int m = 1; m < M; ++m) o_ << " || nt_f" << m;
    o_ << ";\n";
    o_ << "  if (__syncthreads_or(nt_any)) {\n";
  }
  if (needs_tables()) o_ << "  nt_tables_load();\n";
  for (int m = 0; m < M; ++m) {
    for (int j = 0; j < nin; ++j) {
      o_ << "  const real in" << j << msuf(m) << " = (real)inputs[" << m * nin + j << "];\n";
    }
  }
  if (!slow && fallback()) {
    for (int m = 0; m < M; ++m) o_ << "  bool nt_lane_bad" << m << " = false;\n";
  }
  if (!slow) schedule_prologue();
  // a lane of the exception kernel with no flag visits no path
  o_ << "  for (nt_u64 p = " << (slow ? "nt_any ? tid : n_paths" : "tid") << "; p < n_paths; p += T) {\n";
  o_ << "    const nt_u64 path = p + path_offset;\n";
  o_ << "    const nt_u32 rlo = (nt_u32)path ^ (nt_u32)seed;\n";
  o_ << "    const nt_u32 rhi = (nt_u32)(path >> 32) ^ (nt_u32)(seed >> 32);\n";
  for (int st = 1; st < t_.n_streams; ++st) {
    const uint32_t mult = static_cast<uint32_t>(st) * 0x9E3779B1u;
    char buf[96];
    std::snprintf(buf, sizeof buf, "    const nt_u32 rhi%d = rhi ^ 0x%08Xu;\n", st, mult);
    o_ << buf;
  }
}

// Values and tangents of one path; leaves the output in nt_y and its
// derivatives in nt_g.
void Emitter::body_tangent() {
  const int n = t_.n;
  const bool loop = L_.found;
  const int ls = loop ? L_.start : n;
  const int le = loop ? L_.end() : n;
  const std::string zero = f32_ ? "0.0f" : "0.0";
  const std::string one = f32_ ? "1.0f" : "1.0";
  tline(0, ls);
  bool remat = false;
  if (loop) {
    l2e_copies();
    par_on_ = use_par_;
    for (int j = 0; j < L_.period; ++j) {
      if (!(L_.is_carry[j] || L_.is_liveout[j])) continue;
      const int init = L_.is_carry[j] ? L_.carry_init[j] : -1;
      const bool act = t_.active[L_.start + j] != 0;
      for (int m = act ? mlo_ : 0; m < (act ? mhi_ : 1); ++m) {
        m_ = m;
        const bool gsum = gsum_[j] >= 0 && act && p_.adjoints;
        o_ << "    real st" << j << ms(act) << " = " << (init >= 0 && !gsum ? vname(init) : zero) << ";\n";
        if (!act || !p_.adjoints) continue;
        for (int k : posdeplist(j)) {
          const std::string tin = init >= 0 ? inv_tname(init, k) : "";
          o_ << "    " << treal() << " ts" << j << "_" << k << ms(true) << " = "
             << (tin.empty() ? zero : tin == "#1" ? one : tin) << ";\n";
        }
        if (geo(j)) {
          o_ << "    real gs" << j << ms(true) << " = " << (geo_log(j) ? zero : one) << ";\n";
          o_ << "    const real c0_" << j << ms(true) << " = st" << j << ms(true) << ";\n";
          if (gaff(j)) o_ << "    real zs" << j << ms(true) << " = " << zero << ";\n";
        }
      }
    }
    exp_bound_checks();
    // The re-evaluation pass, which runs for a rare path, takes the shortest
    // trip (one step, two when a step draws an odd number of normals) so its
    // register needs stay below the fast pass's: the kernel's register budget
    // is the larger of the two.
    trip_ = slow_ ? (L_.need_even ? 2 : 1) : p_.seg;
    const int lead = trip_ > 1 ? draw_lead() : 0;
    if (lead) tsegment(1, "0");  // the first iteration alone
    it_base_ = lead;
    if (lead) {
      for (const auto& kv : L_.normal_step) draw_shift_[kv.first] = kv.second & 1;
    }
    const int nfull = (L_.iters - lead) / trip_, tail = (L_.iters - lead) % trip_;
    if (nfull > 0) {
      o_ << "    for (nt_u32 sg = 0; sg < " << nfull << "u; ++sg)\n";
      tsegment(trip_, "sg");
    }
    if (tail) tsegment(tail, std::to_string(nfull) + "u");
    it_base_ = 0;
    draw_shift_.clear();
    for (int j = 0; j < L_.period && !slow_; ++j) remat |= gaff(j);
    if (remat) remat_open(ls);
    for (int j = 0; j < L_.period; ++j) {
      if (!geo(j)) continue;
      for (int m = mlo_; m < mhi_; ++m) {
        m_ = m;
        if (gaff(j)) geo_affine_finish(j);
        if (geo_log(j)) {
          const bool a_self = L_.kind_a[j] == ARG_CARRY && L_.ref_a[j] == j;
          const int e = a_self ? L_.ref_b[j] : L_.ref_a[j];
          const std::string g = "gs" + std::to_string(j) + ms(true);
          std::string ex;
          if (f32_) ex = fold_[e].on ? "nt_hw_exp2f(" + g + ")" : "nt_expf(" + g + ")";
          else ex = p_.libm == 1 ? "exp(" + g + ")" : "nt_exp_fast(" + g + ", nt_slow" + ms(true) + ")";
          o_ << "    " << g << " = " << ex << ";\n";
        }
        if (geo_free(j)) o_ << "    st" << j << ms(true) << " = c0_" << j << ms(true) << " * gs" << j << ms(true) << ";\n";
        if (gsum_of_[j] >= 0) {
          const int a = gsum_of_[j];
          const int init = L_.carry_init[a];
          const std::string c = "c0_" + std::to_string(j) + ms(true) + " * st" + std::to_string(a) + ms(true);
          o_ << "    st" << a << ms(true) << " = " << (init >= 0 ? vname(init) + " + " + c : c) << ";\n";
        }
        for (int k : posdeplist(j)) {
          o_ << "    ts" << j << "_" << k << ms(true) << " = gs" << j << ms(true) << " * ts" << j << "_" << k << ms(true)
             << ";\n";
        }
      }
    }
    if (par_on_) {
      // back to the inputs: t_k = sum over parameters d of t_d x (d's tangent for input k)
      par_on_ = false;
      const int nin = t_.n_in;
      for (int j = 0; j < L_.period; ++j) {
        if (!(L_.is_carry[j] || L_.is_liveout[j]) || !t_.active[L_.start + j]) continue;
        for (int m = mlo_; m < mhi_; ++m) {
          m_ = m;
          for (int k : posdeplist(j)) {
            std::string e;
            for (size_t d = 0; d < par_node_.size(); ++d) {
              if (!par_deps_[j][d]) continue;
              const std::string T = tname(par_node_[d], k);
              if (T.empty()) continue;
              const std::string td = "ts" + std::to_string(j) + "_" + std::to_string(nin + static_cast<int>(d)) + ms(true);
              if (T == "#1") e = e.empty() ? td : "(" + e + " + " + td + ")";
              else e = e.empty() ? "(" + td + " * " + T + ")" : f("fma") + "(" + td + ", " + T + ", " + e + ")";
            }
            o_ << "    const " << treal() << " ts" << j << "_" << k << ms(true) << " = " << (e.empty() ? zero : e) << ";\n";
          }
        }
      }
    }
    tline(le, n);
  }
  const int nin = t_.n_in;
  for (int m = mlo_; m < mhi_; ++m) {
    m_ = m;
    for (size_t o = 0; o < t_.outputs.size(); ++o) {
      const int out = t_.outputs[o];
      o_ << "    nt_y" << msuf(m) << "[" << o << "] = (double)" << vname(out) << ";\n";
      if (!p_.adjoints) continue;
      for (int j = 0; j < nin; ++j) {
        const std::string g = tname(out, j);
        o_ << "    nt_g" << msuf(m) << "[" << o * nin + j << "] = "
           << (g.empty() ? std::string("0.0") : g == "#1" ? std::string("1.0") : "(double)" + g) << ";\n";
      }
    }
  }
  if (remat) o_ << "    }\n";
}

// fp32 exp2 folds: p log2(e) and r log2(e) of every folded exponent
void Emitter::l2e_copies() {
  std::set<int> scaled;
  for (const auto& f : fold_) {
    if (!f.on) continue;
    if (f.p >= 0) scaled.insert(f.p);
    scaled.insert(f.r);
  }
  for (int node : scaled) {
    const bool act = t_.active[node] != 0;
    for (int m = act ? mlo_ : 0; m < (act ? mhi_ : 1); ++m) {
      m_ = m;
      o_ << "    const real " << l2e_name(node) << " = " << vname(node) << " * 1.44269504088896341f;\n";
    }
  }
}

// After the step loop: a scope that computes the values before the loop
// again, from opaque copies of the inputs, so the code after the loop reads
// these copies and the compiler keeps nothing of the path's set-up live
// through the loop but what the loop itself reads. The inputs are uniform, so
// the copies stay in SGPRs; the set-up is a few hundred operations per path,
// against the loop's hundreds per step.
void Emitter::remat_open(int ls) {
  const std::string zero = f32_ ? "0.0f" : "0.0";
  const std::string one = f32_ ? "1.0f" : "1.0";
  o_ << "    {\n";
  for (int m = mlo_; m < mhi_; ++m) {
    for (int j = 0; j < t_.n_in; ++j) {
      o_ << "    const real in" << j << msuf(m) << "_r = nt_opaque_u(in" << j << msuf(m) << ");\n";
    }
  }
  const bool par = par_on_;
  par_on_ = false;
  scal_.clear();
  in_sfx_ = "_r";
  tline(0, ls);
  in_sfx_.clear();
  l2e_copies();
  par_on_ = par;
  for (int j = 0; j < L_.period; ++j) {
    if (!geo(j) || !t_.active[L_.start + j] || !p_.adjoints) continue;
    const int init = L_.carry_init[j];
    for (int m = mlo_; m < mhi_; ++m) {
      m_ = m;
      o_ << "    const real c0_" << j << ms(true) << " = " << (init >= 0 ? vname(init) : zero) << ";\n";
      if (!gaff(j)) continue;
      // the loop leaves these tangents at their start values
      for (int k : posdeplist(j)) {
        const std::string tin = init >= 0 ? inv_tname(init, k) : "";
        o_ << "    ts" << j << "_" << k << ms(true) << " = " << (tin.empty() ? zero : tin == "#1" ? one : tin) << ";\n";
      }
    }
  }
}

// Forward pass, then the reverse sweep; leaves the output in nt_y and the
// adjoints of the inputs in nt_g.
void Emitter::body_reverse() {
  if (!p_.lbound.empty()) {
    body_reverse_segmented();
    return;
  }
  const int n = t_.n;
  const bool loop = L_.found;
  const int ls = loop ? L_.start : n;
  const int le = loop ? L_.end() : n;
  line_forward(0, ls);
  if (loop) {
    for (int j = 0; j < L_.period; ++j) {
      if (!(L_.is_carry[j] || L_.is_liveout[j])) continue;
      o_ << "    real st" << j << " = "
         << (L_.is_carry[j] ? "v" + std::to_string(L_.carry_init[j]) : std::string(f32_ ? "0.0f" : "0.0")) << ";\n";
    }
    if (p_.nseg_full > 0) {
      o_ << "    for (nt_u32 sg = 0; sg < " << p_.nseg_full << "u; ++sg)\n";
      segment(p_.seg, "sg", true);
    }
    if (p_.tail) segment(p_.tail, std::to_string(p_.nseg_full) + "u", true);
    line_forward(le, n);
  }
  o_ << "    nt_y[0] = (double)" << vname(t_.output) << ";\n";
  if (!p_.adjoints) return;
  const std::string zero = f32_ ? "0.0f" : "0.0";
  const std::string one = f32_ ? "1.0f" : "1.0";
  for (int i = 0; i < ls; ++i) {
    if (t_.active[i]) o_ << "    real d" << i << " = " << zero << ";\n";
  }
  if (loop) {
    for (int j = 0; j < L_.period; ++j) {
      if ((L_.is_carry[j] || L_.is_liveout[j]) && t_.active[L_.start + j]) o_ << "    real gs" << j << " = " << zero << ";\n";
    }
    for (int i = le; i < n; ++i) {
      if (t_.active[i]) o_ << "    real d" << i << " = " << zero << ";\n";
    }
  }
  if (t_.active[t_.output]) {
    o_ << "    " << dname(t_.output) << " = " << one << ";\n";
    if (loop) line_reverse(le, n);
    if (loop) {
      if (p_.tail) segment(p_.tail, std::to_string(p_.nseg_full) + "u", false);
      if (p_.nseg_full > 0) {
        o_ << "    for (int sgi = " << (p_.nseg_full - 1) << "; sgi >= 0; --sgi)\n";
        segment(p_.seg, "(nt_u32)sgi", false);
      }
      for (int c : p_.carries) {
        const int init = L_.carry_init[c];
        if (t_.active[L_.start + c] && init >= 0 && t_.active[init]) o_ << "    d" << init << " += gs" << c << ";\n";
      }
    }
    line_reverse(0, ls);
  }
  for (int j = 0; j < t_.n_in; ++j) {
    const int node = t_.input_node[j];
    o_ << "    nt_g[" << j << "] = " << (t_.active[t_.output] ? "(double)" + dname(node) : std::string("0.0")) << ";\n";
  }
}

// channels: [market][output][value, value^2, derivative per input]
// `skip` names a flag under which the path adds nothing (its value and
// derivatives are replaced by zeros with a select, no branch).
void Emitter::accumulate(int m, const std::string& skip) {
  const int nin = t_.n_in;
  const int O = static_cast<int>(t_.outputs.size());
  auto keep = [&](const std::string& v) { return skip.empty() ? v : "(" + skip + " ? 0.0 : " + v + ")"; };
  for (int o = 0; o < O; ++o) {
    const int base = m * p_.n_channels + o * (2 + nin);
    const std::string y = keep("nt_y" + msuf(m) + "[" + std::to_string(o) + "]");
    o_ << "    {\n      const double y = " << y << ";\n";
    o_ << "      acc[" << base << "] += y;\n      acc[" << base + 1 << "] += y * y;\n    }\n";
    if (!p_.adjoints) continue;
    for (int j = 0; j < nin; ++j) {
      o_ << "    acc[" << base + 2 + j << "] += " << keep("nt_g" + msuf(m) + "[" + std::to_string(o * nin + j) + "]")
         << ";\n";
    }
  }
}

// Per-path rows [market][path][output], as the oracle's per-path rows.
void Emitter::dump_rows(int m) {
  const int nin = t_.n_in;
  const int M = p_.markets;
  const int O = static_cast<int>(t_.outputs.size());
  const std::string path_row = M > 1 ? "(" + std::to_string(m) + "u * n_paths + p)" : std::string("p");
  for (int o = 0; o < O; ++o) {
    const std::string row = O > 1 ? "(" + path_row + " * " + std::to_string(O) + "u + " + std::to_string(o) + "u)" : path_row;
    o_ << "      out_v[" << row << "] = nt_y" << msuf(m) << "[" << o << "];\n";
    for (int j = 0; j < nin; ++j) {
      o_ << "      out_g[" << row << " * " << nin << "u + " << j << "u] = "
         << (p_.adjoints ? "nt_g" + msuf(m) + "[" + std::to_string(o * nin + j) + "]" : std::string("0.0")) << ";\n";
    }
  }
}

// One kernel. The replay kernel evaluates every path on the fast pass; a path
// whose fast pass is not valid (an own-math routine met an argument outside
// its range, or the value or a derivative came out non-finite) is left out of
// its sums and flagged in the bitmap. The exception kernel evaluates the
// flagged paths again, one market at a time, with device libm and the
// oracle's zero-adjoint rule, into the second half of each channel's column
// of partials. Kept apart, the rare pass costs the replay kernel no registers.
void Emitter::kernel(bool slow) {
  const int nin = t_.n_in;
  const int M = p_.markets;
  const int O = static_cast<int>(t_.outputs.size());
  const bool tangent = p_.mode == NT_MODE_TANGENT;
  const bool fb = fallback();
  slow_ = slow;
  kernel_head(slow);
  for (int m = 0; m < M; ++m) {
    o_ << "    double nt_y" << msuf(m) << "[" << O << "];\n";
    if (p_.adjoints && nin > 0) o_ << "    double nt_g" << msuf(m) << "[" << O * nin << "];\n";
  }
  if (!slow) {
    if (fb) {
      o_ << "    bool nt_slow = false;\n";  // a flag shared by every market (a draw-only exponent)
      for (int m = 0; m < M && M > 1; ++m) o_ << "    bool nt_slow" << msuf(m) << " = false;\n";
    }
    mlo_ = 0;
    mhi_ = M;
    o_ << "    {\n";
    scal_.clear();
    if (tangent) body_tangent(); else body_reverse();
    o_ << "    }\n";
    for (int m = 0; m < M; ++m) {
      if (fb) o_ << "    nt_lane_bad" << m << " |= nt_slow" << (M > 1 ? " || nt_slow" + msuf(m) : std::string()) << ";\n";
      accumulate(m, "");
      o_ << "#ifdef NT_DUMP_PATHS\n    {\n";
      dump_rows(m);
      o_ << "    }\n#endif\n";
    }
  } else {
    // Each market is evaluated again alone, so its result is the one a
    // single-market kernel gives it.
    for (int m = 0; m < M; ++m) {
      o_ << "    if (nt_f" << m << ") {\n";
      mlo_ = m;
      mhi_ = m + 1;
      scal_.clear();
      if (tangent) body_tangent(); else body_reverse();
      accumulate(m, "");
      o_ << "#ifdef NT_DUMP_PATHS\n";
      dump_rows(m);
      o_ << "#endif\n";
      o_ << "    }\n";
    }
  }
  o_ << "  }\n";
  if (slow) o_ << "  }\n";  // the block had a flagged path
  if (!slow && fb) {
    // A lane that flagged a path, or whose sums are not finite (a value or a
    // derivative of one of its paths was not: the oracle's may still be, where
    // it skips a zero adjoint), adds nothing and leaves every one of its paths
    // to the exception kernel: a rare event, and its paths' contributions need
    // not stay live to the end of each path.
    for (int m = 0; m < M; ++m) {
      const std::string bad = "nt_lane_bad" + std::to_string(m);
      const int c0 = m * p_.n_channels, c1 = c0 + p_.n_channels;
      if (nonfinite_fallback() || minmax_fallback()) {
        o_ << "  for (int c = " << c0 << "; c < " << c1 << "; ++c) " << bad << " |= !__builtin_isfinite(acc[c]);\n";
      }
      o_ << "  if (" << bad << ") {\n    for (int c = " << c0 << "; c < " << c1 << "; ++c) acc[c] = 0.0;\n  }\n";
      o_ << "  nt_flag_lanes(nt_bits + " << m << "u * nt_words, tid, " << bad << ");\n";
    }
    o_ << "  if (nt_lane_bad0";
    for (int m = 1; m < M; ++m) o_ << " || nt_lane_bad" << m;
    o_ << ") atomicAdd(flags, 1ull);\n";
  }
  const int nacc = p_.n_channels * M;
  o_ << "  __shared__ double nt_lds[" << nacc << " * (" << p_.block << " / 64)];\n";
  o_ << "  nt_block_store<" << nacc << ">(acc, partials, nt_lds);\n";
  o_ << "}\n";
  slow_ = false;
  mlo_ = 0;
  mhi_ = M;
}

std::string Emitter::run() {
  count_uses();
  plan_schedule();
  plan_exp2_folds();
  plan_exp_bounds();
  plan_parameters();
  par_on_ = use_par_;
  plan_geo_carries();
  plan_geo_sums();
  plan_geo_logs();
  plan_fused_exponents();
  plan_geo_affine();
  par_on_ = false;
  preamble();
  kernel(false);
  if (fallback()) kernel(true);
  return o_.str();
}

}  // namespace

std::string emit_source(const TapeIR& ir, const Plan& plan) {
  Emitter e(ir, plan);
  return e.run();
}

}  // namespace ntl
