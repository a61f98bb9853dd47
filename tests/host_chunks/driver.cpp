// The host layer's chunked replay (AadExecutable::calibrate / replaySafe,
// nablatensor_amd/host/engine.cpp; the reference's
// AbstractAadExecutable.java:100-159 and AadResultAccumulator.java:52-96) on
// the CPU, with a stand-in executable whose replay sums a fixed function of
// the path index and reports a chosen time per path. Built with AddressSanitizer
// and UndefinedBehaviorSanitizer (tests/host_chunks/Makefile); prints one
// JSON object per case for tests/test_host_chunks.py.
#include <cmath>
#include <cstdio>
#include <string>
#include <vector>

#include "engine.hpp"

using namespace nablatensor;

namespace {

// Per path p: y = 0.5 + (p mod 1000) / 1000 and dy/dx_j = (j + 1) ((p mod 7) + 1),
// summed exactly in long double over the dispatch's range.
class StandIn : public AadExecutable {
 public:
  StandIn(TapePtr tape, double pathsPerSecond, bool rawSums)
      : AadExecutable(std::move(tape), AadOptions::defaults()), rate_(pathsPerSecond), raw_(rawSums) {}
  std::string engineName() const override { return "stand-in"; }
  AadResult replay(long long paths, long long pathOffset, long long) override {
    checkOpen();
    chunks.push_back(paths);
    const size_t ni = tape().inputNames().size();
    long double sy = 0, syy = 0;
    std::vector<long double> g(ni, 0);
    for (long long p = pathOffset; p < pathOffset + paths; ++p) {
      const long double y = 0.5L + static_cast<long double>(p % 1000) / 1000.0L;
      sy += y;
      syy += y * y;
      for (size_t j = 0; j < ni; ++j) g[j] += static_cast<long double>((j + 1) * ((p % 7) + 1));
    }
    std::vector<double> sums{static_cast<double>(sy), static_cast<double>(syy)};
    for (long double v : g) sums.push_back(static_cast<double>(v));
    const double seconds = static_cast<double>(paths) / rate_;
    AadResult full = AadResult::fromSums(sums, tape().outputNames(), tape().inputNames(), paths, seconds, seconds);
    if (raw_) return full;
    // an engine that reports means and a standard error only
    return AadResult(full.value(), full.standardError(), full.gradients(), tape().inputNames(), paths, seconds);
  }
  std::vector<long long> chunks;

 private:
  double rate_;
  bool raw_;
};

void print_case(const char* name, StandIn& x, const AadResult& chunked, const AadResult& whole) {
  std::printf("{\"case\": \"%s\", \"chunks\": %zu, \"first_chunks\": [", name, x.chunks.size());
  for (size_t i = 0; i < x.chunks.size() && i < 6; ++i) std::printf("%s%lld", i ? ", " : "", x.chunks[i]);
  std::printf("], \"rate\": %.17g, \"paths\": %lld", x.measuredPathsPerSecond(), chunked.paths());
  std::printf(", \"value\": [%.17g, %.17g], \"stderr\": [%.17g, %.17g], \"grad0\": [%.17g, %.17g]",
              chunked.value(), whole.value(), chunked.standardError(), whole.standardError(),
              chunked.gradients()[0], whole.gradients()[0]);
  std::printf(", \"raw\": %zu, \"seconds\": %.17g}\n", chunked.rawSums().size(), chunked.seconds());
}

}  // namespace

int main() {
  TapePtr tape = AadRecorder::record([](AadRecorder& rec) {
    ADouble x = rec.input("x", 1.5);
    ADouble y = rec.input("y", 0.5);
    rec.output(x.mul(rec.randn()).add(y).exp());
  });
  const long long total = 3000000;
  {
    // 10^8 paths/s and a 1 ms budget: calibration probes from 65,536 paths,
    // then chunks of 10^5 paths; the raw sums combine exactly
    StandIn x(tape, 1e8, true);
    x.setMaxChunkSeconds(1e-3);
    AadResult chunked = x.replaySafe(total, 42);
    StandIn y(tape, 1e8, true);
    AadResult whole = y.replay(total, 0, 42);
    print_case("raw", x, chunked, whole);
  }
  {
    // the same with means only: the reference's mean * n recombination
    StandIn x(tape, 1e8, false);
    x.setMaxChunkSeconds(1e-3);
    AadResult chunked = x.replaySafe(total, 42);
    StandIn y(tape, 1e8, true);
    AadResult whole = y.replay(total, 0, 42);
    print_case("means", x, chunked, whole);
  }
  {
    // a budget below the minimum chunk: chunks of 4,096 paths
    StandIn x(tape, 1e8, true);
    x.setMaxChunkSeconds(1e-6);
    AadResult chunked = x.replaySafe(100000, 7);
    StandIn y(tape, 1e8, true);
    AadResult whole = y.replay(100000, 0, 7);
    print_case("min_chunk", x, chunked, whole);
  }
  {
    // a closed executable and a bad budget are refused as the reference does
    StandIn x(tape, 1e8, true);
    int refused = 0;
    try { x.setMaxChunkSeconds(0.0); } catch (const std::invalid_argument&) { ++refused; }
    try { (void)x.replaySafe(0, 1); } catch (const std::invalid_argument&) { ++refused; }
    x.close();
    try { (void)x.replay(10, 0, 1); } catch (const std::logic_error&) { ++refused; }
    std::printf("{\"case\": \"refusals\", \"refused\": %d}\n", refused);
  }
  return 0;
}
