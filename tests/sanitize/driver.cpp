// Sanitizer driver: the lowering (tape validation, planning, source emission;
// nablatensor_amd/csrc/lower.cpp) and the CPU oracle (oracle/nt_oracle.c),
// built with AddressSanitizer and UndefinedBehaviorSanitizer by the Makefile
// beside this file and run by tests/test_sanitize.py.
//
// usage: nt_sanitize_driver <manifest>
// Each manifest line is "<tape file> <ok|invalid>", the tape in the wire
// form of nablatensor_amd/rocm.py (TapeArrays.wire_bytes: little-endian
// int32 counts and indices, binary64 constants, in nt_tape field order). An
// "invalid" tape must be refused by build_ir; an "ok" tape must be accepted,
// then planned and emitted under a spread of nt_options (a plan may refuse
// an option set it does not support, with an error), and replayed by the
// oracle on a few paths. Then the null-pointer and empty-tape cases of the C
// ABI's validation. Exits 0 when every expectation holds; a sanitizer
// report aborts the process.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "lower.hpp"
#include "nt_oracle.h"

namespace {

struct WireTape {
  std::vector<int32_t> op, a, b, input_node, output_node;
  std::vector<double> c;
  int32_t n = 0, n_in = 0, n_out = 0, n_streams = 0, n_uniforms = 0;
  nt_tape view() const {
    return nt_tape{n, op.data(), a.data(), b.data(), c.data(), n_in, input_node.data(), n_out, output_node.data(),
                   n_streams, n_uniforms};
  }
};

// Reads the wire form; a count below zero reads no elements but is kept, so
// the validation sees it.
bool read_tape(const std::string& path, WireTape& t) {
  std::ifstream f(path, std::ios::binary);
  std::string bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  size_t at = 0;
  auto take = [&](void* dst, size_t n) {
    if (at + n > bytes.size()) return false;
    std::memcpy(dst, bytes.data() + at, n);
    at += n;
    return true;
  };
  auto i32s = [&](std::vector<int32_t>& v, int32_t n) {
    v.assign(n > 0 ? n : 0, 0);
    return n <= 0 || take(v.data(), sizeof(int32_t) * static_cast<size_t>(n));
  };
  if (!take(&t.n, 4) || !i32s(t.op, t.n) || !i32s(t.a, t.n) || !i32s(t.b, t.n)) return false;
  t.c.assign(t.n > 0 ? t.n : 0, 0.0);
  if (t.n > 0 && !take(t.c.data(), sizeof(double) * static_cast<size_t>(t.n))) return false;
  if (!take(&t.n_in, 4) || !i32s(t.input_node, t.n_in)) return false;
  if (!take(&t.n_out, 4) || !i32s(t.output_node, t.n_out)) return false;
  return take(&t.n_streams, 4) && take(&t.n_uniforms, 4) && at == bytes.size();
}

nt_options opts(int precision, int mode, int ckpt, int roll, int seg, int markets, int basis, int contract, int libm) {
  nt_options o{};
  o.precision = precision;
  o.adjoints = 1;
  o.mode = mode;
  o.checkpoint = ckpt;
  o.roll = roll;
  o.seg_len = seg;
  o.markets = markets;
  o.basis = basis;
  o.contract = contract;
  o.libm = libm;
  return o;
}

int failures = 0;

void expect(bool ok, const std::string& what) {
  if (ok) return;
  std::printf("FAIL %s\n", what.c_str());
  ++failures;
}

void lower_all(const WireTape& w, const std::string& name) {
  const nt_tape t = w.view();
  ntl::TapeIR ir;
  std::string err;
  const int rc = ntl::build_ir(&t, ir, err);
  expect(rc == NT_OK, name + ": build_ir refused a valid tape: " + err);
  if (rc != NT_OK) return;
  // Each option value at least once; a straight line only below 20,000 nodes.
  std::vector<nt_options> all = {
      opts(NT_FP64, 0, 0, 1, 0, 0, 0, 0, 0),  opts(NT_FP32, 0, 0, 1, 0, 0, 0, 0, 0),
      opts(NT_FP64, 1, 1, 1, 0, 0, 0, 0, 0),  opts(NT_FP64, 1, 2, 1, 0, 0, 0, 0, 1),
      opts(NT_FP64, 1, 3, 1, 0, 0, 0, -1, 2), opts(NT_FP32, 1, 1, 1, 5, 0, 0, 1, 0),
      opts(NT_FP64, 2, 0, 1, 0, 0, 1, 0, 0),  opts(NT_FP64, 2, 0, 1, 3, 0, 2, -1, 1),
      opts(NT_FP32, 2, 0, 1, 0, 3, 0, 0, 0),  opts(NT_FP64, 2, 0, 1, 0, 2, 2, 0, 0),
      opts(NT_FP64, 0, 0, 1, 0, 4, 0, 0, 0),
  };
  if (w.n < 20000) {
    for (nt_options o : {opts(NT_FP64, 1, 0, -1, 0, 0, 0, 0, 0), opts(NT_FP32, 1, 0, -1, 7, 0, 0, 0, 1),
                         opts(NT_FP64, 2, 0, -1, 0, 0, 0, 0, 0), opts(NT_FP64, 1, 3, -1, 0, 0, 0, 0, 0),
                         opts(NT_FP64, 1, 1, -1, 13, 0, 0, -1, 2)}) {
      all.push_back(o);
    }
  }
  for (size_t k = 0; k < all.size(); ++k) {
    ntl::TapeIR copy = ir;
    ntl::Plan plan;
    const int prc = ntl::make_plan(copy, &all[k], plan, err);
    if (prc != NT_OK) {
      expect(prc == NT_E_INVALID || prc == NT_E_UNSUPPORTED, name + ": make_plan returned " + std::to_string(prc));
      continue;
    }
    const std::string src = ntl::emit_source(copy, plan);
    expect(src.find("void nt_replay(") != std::string::npos, name + ": no replay kernel in option set " +
                                                               std::to_string(k));
  }
}

void replay_oracle(const WireTape& w, const std::string& name) {
  std::vector<double> inputs(w.n_in);
  for (int j = 0; j < w.n_in; ++j) inputs[j] = w.c[w.input_node[j]];
  nto_tape t{};
  t.n = w.n;
  t.op = w.op.data();
  t.arg_a = w.a.data();
  t.arg_b = w.b.data();
  t.constant = w.c.data();
  t.n_inputs = w.n_in;
  t.input_node = w.input_node.data();
  t.n_outputs = w.n_out;
  t.output_node = w.output_node.data();
  t.n_streams = w.n_streams;
  const uint64_t paths = w.n > 20000 ? 2 : 9;
  std::vector<double> values(paths * w.n_out), grads(paths * w.n_out * (w.n_in > 0 ? w.n_in : 1));
  const int rc = nto_replay_paths(&t, inputs.data(), paths, 0x100000003ull, 42, 0, 1, values.data(), grads.data());
  expect(rc == 0, name + ": oracle replay failed");
}

void null_cases() {
  ntl::TapeIR ir;
  std::string err;
  expect(ntl::build_ir(nullptr, ir, err) == NT_E_INVALID, "null tape accepted");
  const int32_t op[2] = {NT_OP_INPUT, NT_OP_EXP}, a[2] = {0, 0}, b[2] = {-1, -1}, in[1] = {0}, out[1] = {1};
  const double c[2] = {1.0, 0.0};
  nt_tape t{2, op, a, b, c, 1, in, 1, out, 1, 0};
  expect(ntl::build_ir(&t, ir, err) == NT_OK, "the two-node tape refused: " + err);
  nt_tape u = t;
  u.op = nullptr;
  expect(ntl::build_ir(&u, ir, err) == NT_E_INVALID, "null op array accepted");
  u = t;
  u.constant = nullptr;
  expect(ntl::build_ir(&u, ir, err) == NT_E_INVALID, "null constants accepted");
  u = t;
  u.input_node = nullptr;
  expect(ntl::build_ir(&u, ir, err) == NT_E_INVALID, "null input list accepted");
  u = t;
  u.output_node = nullptr;
  expect(ntl::build_ir(&u, ir, err) == NT_E_INVALID, "null output list accepted");
  u = t;
  u.n_nodes = 0;
  expect(ntl::build_ir(&u, ir, err) == NT_E_INVALID, "empty tape accepted");
  nt_options bad{};
  bad.block = 100;
  ntl::Plan plan;
  ntl::TapeIR good;
  expect(ntl::build_ir(&t, good, err) == NT_OK, "rebuild");
  expect(ntl::make_plan(good, &bad, plan, err) == NT_E_INVALID, "block 100 accepted");
  bad = nt_options{};
  bad.markets = 65;
  expect(ntl::make_plan(good, &bad, plan, err) == NT_E_INVALID, "65 markets accepted");
  bad = nt_options{};
  bad.seg_len = -1;
  expect(ntl::make_plan(good, &bad, plan, err) == NT_E_INVALID, "negative seg_len accepted");
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: %s <manifest>\n", argv[0]);
    return 2;
  }
  std::ifstream m(argv[1]);
  std::string line;
  int tapes = 0, refused = 0;
  while (std::getline(m, line)) {
    std::istringstream ls(line);
    std::string path, want;
    if (!(ls >> path >> want)) continue;
    WireTape w;
    if (!read_tape(path, w)) {
      expect(false, path + ": unreadable wire file");
      continue;
    }
    ++tapes;
    if (want == "invalid") {
      ntl::TapeIR ir;
      std::string err;
      const nt_tape t = w.view();
      const int rc = ntl::build_ir(&t, ir, err);
      expect(rc == NT_E_INVALID && !err.empty(), path + ": a malformed tape was accepted");
      refused += rc == NT_E_INVALID;
      continue;
    }
    lower_all(w, path);
    replay_oracle(w, path);
  }
  null_cases();
  std::printf("tapes %d, refused %d, failures %d\n", tapes, refused, failures);
  return failures == 0 ? 0 : 1;
}
