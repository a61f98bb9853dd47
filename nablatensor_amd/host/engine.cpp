// Engine SPI, chunked replay and the rocm engine; see engine.hpp for the
// reference each part follows.
#include "engine.hpp"

#include <dlfcn.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <mutex>
#include <sstream>

#include "nablatensor_rocm.h"

namespace nablatensor {

// ---- AadResult (AadResult.java:50-197, AadTotals.java:68-89) ----------------------

AadResult::AadResult(double value, double standardError, std::vector<double> gradients,
                     std::vector<std::string> inputNames, long long paths, double seconds)
    : value_(value), stderr_(standardError), gradients_(std::move(gradients)), input_names_(std::move(inputNames)),
      paths_(paths), seconds_(seconds) {
  output_names_ = {"value"};
  values_ = {value_};
  stderrs_ = {stderr_};
  jacobian_ = {gradients_};
}

int AadResult::outputIndex(const std::string& outputName) const {
  for (size_t o = 0; o < output_names_.size(); ++o) {
    if (output_names_[o] == outputName) return static_cast<int>(o);
  }
  throw std::invalid_argument("unknown output: " + outputName);
}

double AadResult::gradient(const std::string& outputName, const std::string& inputName) const {
  const auto& row = jacobian_.at(outputIndex(outputName));
  for (size_t i = 0; i < input_names_.size(); ++i) {
    if (input_names_[i] == inputName) return row.at(i);
  }
  throw std::invalid_argument("unknown input: " + inputName);
}

double AadResult::gradient(const std::string& inputName) const {
  for (size_t i = 0; i < input_names_.size(); ++i) {
    if (input_names_[i] == inputName) return gradients_.at(i);
  }
  throw std::invalid_argument("unknown input: " + inputName);
}

std::string AadResult::toString() const {
  std::ostringstream s;
  s << "AadResult(value=" << value_ << ", paths=" << paths_ << ")";
  return s.str();
}

// mean, stderr = sqrt(max(0, (sum y^2 - n mean^2) / (n - 1)) / n), mean adjoints.
AadResult AadResult::fromSums(const std::vector<double>& sums, const std::vector<std::string>& outputNames,
                              const std::vector<std::string>& inputNames, long long paths, double seconds,
                              double kernelSeconds) {
  const double n = static_cast<double>(paths);
  const size_t ni = inputNames.size();
  const size_t no = std::max<size_t>(1, outputNames.size());
  std::vector<double> means(no), ses(no);
  std::vector<std::vector<double>> rows(no, std::vector<double>(ni));
  for (size_t o = 0; o < no; ++o) {
    const size_t b = o * (2 + ni);
    means[o] = sums.at(b) / n;
    ses[o] = std::nan("");
    if (paths > 1) {
      const double variance = (sums.at(b + 1) - n * means[o] * means[o]) / (n - 1.0);
      ses[o] = std::sqrt(std::max(0.0, variance) / n);
    }
    for (size_t j = 0; j < ni; ++j) rows[o][j] = sums.at(b + 2 + j) / n;
  }
  AadResult r(means[0], ses[0], rows[0], inputNames, paths, seconds);
  if (!outputNames.empty()) r.output_names_ = outputNames;
  r.values_ = means;
  r.stderrs_ = ses;
  r.jacobian_ = rows;
  r.raw_ = sums;
  r.kernel_seconds_ = kernelSeconds;
  return r;
}

// ---- AadExecutable chunking (AbstractAadExecutable.java:36-165) ---------------------

namespace {
constexpr long long kProbePaths = 65536;
constexpr long long kMinChunkPaths = 4096;
}  // namespace

AadExecutable::AadExecutable(TapePtr tape, const AadOptions& options)
    : tape_(std::move(tape)), options_(options), inputs_(tape_->recordedInputs()) {}

void AadExecutable::setInput(const std::string& name, double value) {
  const int index = tape_->inputIndex(name);
  if (index < 0) throw std::invalid_argument("unknown input: " + name);
  inputs_[index] = value;
}

void AadExecutable::checkOpen() const {
  if (closed_) throw std::logic_error("executable is closed");
}

void AadExecutable::setMaxChunkSeconds(double seconds) {
  if (!(seconds > 0.0)) throw std::invalid_argument("maxChunkSeconds must be positive");
  max_chunk_seconds_ = seconds;
}

void AadExecutable::observe(long long paths, double seconds) {
  if (seconds <= 0.0) return;
  const double sample = paths / seconds;
  paths_per_second_ = paths_per_second_ <= 0.0 ? sample : 0.5 * (paths_per_second_ + sample);
}

long long AadExecutable::budgetedChunk() const {
  if (paths_per_second_ <= 0.0) return kProbePaths;
  return std::max(kMinChunkPaths, static_cast<long long>(paths_per_second_ * max_chunk_seconds_));
}

double AadExecutable::calibrate(long long seed) {
  long long paths = kProbePaths;
  for (int attempt = 0; attempt < 12; ++attempt) {
    AadResult probe = replay(paths, 0, seed);
    observe(paths, probe.seconds());
    if (probe.seconds() >= max_chunk_seconds_ * 0.2) break;
    const long long next = budgetedChunk();
    if (next <= paths) break;
    paths = std::min(next, paths * 8);
  }
  return paths_per_second_;
}

// Chunks of rate * budget paths. Dispatches that carry raw sums are combined
// exactly; otherwise the reference's mean * n recombination
// (AadResultAccumulator.java:52-96) is used.
std::vector<AadResult> AadExecutable::replayMany(const std::vector<std::vector<double>>& inputSets, long long paths,
                                                long long pathOffset, long long seed) {
  checkOpen();
  if (inputSets.empty()) throw std::invalid_argument("at least one input set is required");
  const std::vector<double> saved = inputs_;
  const auto& names = tape().inputNames();
  std::vector<AadResult> out;
  for (size_t m = 0; m < inputSets.size(); ++m) {
    if (inputSets[m].size() != names.size()) {
      throw std::invalid_argument("input set " + std::to_string(m) + " has " + std::to_string(inputSets[m].size()) +
                                  " values; the tape has " + std::to_string(names.size()) + " inputs");
    }
    for (size_t j = 0; j < names.size(); ++j) setInput(names[j], inputSets[m][j]);
    out.push_back(replay(paths, pathOffset, seed));
  }
  for (size_t j = 0; j < names.size(); ++j) setInput(names[j], saved[j]);
  return out;
}

AadResult AadExecutable::replaySafe(long long totalPaths, long long seed) {
  if (totalPaths <= 0) throw std::invalid_argument("paths must be positive");
  if (paths_per_second_ <= 0.0) calibrate(seed);
  const size_t ni = tape_->inputNames().size();
  const size_t no = static_cast<size_t>(tape_->outputCount());
  std::vector<double> sums(no * (2 + ni), 0.0);
  bool exact = true;
  double seconds = 0.0, kernel = 0.0;
  long long done = 0;
  while (done < totalPaths) {
    const long long chunk = std::min(budgetedChunk(), totalPaths - done);
    AadResult part = replay(chunk, done, seed);
    seconds += part.seconds();
    kernel += part.kernelSeconds();
    if (exact && part.rawSums().size() == sums.size()) {
      for (size_t c = 0; c < sums.size(); ++c) sums[c] += part.rawSums()[c];
    } else {
      // AadResultAccumulator's mean * n reconstruction (AadResultAccumulator.java:52-96)
      exact = false;
      const double n = static_cast<double>(chunk);
      const auto& names = part.outputNames();
      for (size_t o = 0; o < no && o < names.size(); ++o) {
        const size_t b = o * (2 + ni);
        const double v = part.value(names[o]);
        sums[b] += v * n;
        const double se = part.standardError(names[o]);
        const double variance = se * se * n;
        const double denom = chunk > 1 ? n - 1.0 : n;
        sums[b + 1] += std::isnan(se) ? std::nan("") : denom * variance + n * v * v;
        for (size_t j = 0; j < ni; ++j) sums[b + 2 + j] += part.gradients(names[o])[j] * n;
      }
    }
    observe(chunk, part.seconds());
    done += chunk;
  }
  return AadResult::fromSums(sums, tape_->outputNames(), tape_->inputNames(), totalPaths, seconds, kernel);
}

// ---- engine selection (AadEngine.java:56-86, AadEngines.java:41-110) ----------------

void AadEngine::requireSupportedTape(const AadTape& tape) const {
  if (tape.hasExtendedRandom()) {
    throw UnsupportedOperation("engine '" + name() +
                               "' does not yet support rec.randu() or named random streams; use cpu-jit or cpu for this tape");
  }
  if (tape.outputCount() > 1) {
    throw UnsupportedOperation("engine '" + name() + "' does not yet support multi-output tapes; use cpu-jit or cpu for this tape");
  }
}

namespace {

std::mutex& registry_mutex() {
  static std::mutex m;
  return m;
}

std::vector<std::shared_ptr<AadEngine>>& registry() {
  static std::vector<std::shared_ptr<AadEngine>> engines{std::make_shared<RocmAadEngine>()};
  return engines;
}

bool usable(const AadEngine& e, const AadOptions& o) {
  try {
    return e.isAvailable() && e.supports(o);
  } catch (...) {
    return false;
  }
}

std::string names(const std::vector<std::shared_ptr<AadEngine>>& engines) {
  if (engines.empty()) return "(none)";
  std::string s;
  for (size_t i = 0; i < engines.size(); ++i) s += (i ? ", " : "") + engines[i]->name();
  return s;
}

}  // namespace

void AadEngines::registerEngine(std::shared_ptr<AadEngine> engine) {
  std::lock_guard<std::mutex> lock(registry_mutex());
  registry().push_back(std::move(engine));
}

std::vector<std::shared_ptr<AadEngine>> AadEngines::discovered() {
  std::vector<std::shared_ptr<AadEngine>> all;
  {
    std::lock_guard<std::mutex> lock(registry_mutex());
    all = registry();
  }
  std::stable_sort(all.begin(), all.end(), [](const auto& a, const auto& b) { return a->priority() > b->priority(); });
  return all;
}

std::vector<std::shared_ptr<AadEngine>> AadEngines::available(const AadOptions& options) {
  std::vector<std::shared_ptr<AadEngine>> out;
  for (auto& e : discovered()) {
    if (usable(*e, options)) out.push_back(e);
  }
  return out;
}

std::shared_ptr<AadEngine> AadEngines::find(const std::string& name, const AadOptions& options) {
  for (auto& e : discovered()) {
    std::string a = e->name(), b = name;
    std::transform(a.begin(), a.end(), a.begin(), ::tolower);
    std::transform(b.begin(), b.end(), b.begin(), ::tolower);
    if (a == b && usable(*e, options)) return e;
  }
  return nullptr;
}

std::shared_ptr<AadEngine> AadEngines::require(const std::string& name, const AadOptions& options) {
  auto e = find(name, options);
  if (!e) {
    throw std::logic_error("AAD engine '" + name + "' is not usable here; available: " + names(available(options)));
  }
  return e;
}

std::shared_ptr<AadEngine> AadEngines::select(const AadOptions& options) {
  const char* requested = std::getenv("NABLATENSOR_ENGINE");
  if (requested && *requested) return require(requested, options);
  auto usableEngines = available(options);
  if (usableEngines.empty()) {
    throw std::logic_error("no usable AAD engine; discovered: " + names(discovered()));
  }
  return usableEngines.front();
}

// ---- the rocm engine over the C ABI ----------------------------------------------------

namespace {

// The C-ABI entry points, resolved once (the FFM downcall handles of the Java adapter).
struct RocmAbi {
  bool loaded = false;
  std::string error;
  decltype(&nt_probe) probe = nullptr;
  decltype(&nt_device_name) device_name = nullptr;
  decltype(&nt_exec_create) create = nullptr;
  decltype(&nt_exec_set_inputs) set_inputs = nullptr;
  decltype(&nt_exec_replay) replay = nullptr;
  decltype(&nt_exec_replay_many) replay_many = nullptr;
  decltype(&nt_exec_info_get) info = nullptr;
  decltype(&nt_exec_source) source = nullptr;
  decltype(&nt_exec_destroy) destroy = nullptr;
  decltype(&nt_last_error) last_error = nullptr;
};

std::string library_path() {
  const char* env = std::getenv("NABLATENSOR_ROCM_LIB");
  if (env && *env) return env;
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&library_path), &info) && info.dli_fname) {
    std::string p(info.dli_fname);
    size_t slash = p.rfind('/');
    if (slash != std::string::npos) return p.substr(0, slash) + "/libnt_rocm.so";
  }
  return "libnt_rocm.so";
}

const RocmAbi& abi() {
  static RocmAbi a;
  static std::once_flag once;
  std::call_once(once, [] {
    const std::string path = library_path();
    void* h = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
    if (!h) {
      a.error = std::string("cannot load ") + path + ": " + dlerror();
      return;
    }
    bool ok = true;
    auto sym = [&](const char* name) {
      void* p = dlsym(h, name);
      if (!p) ok = false;
      return p;
    };
    a.probe = reinterpret_cast<decltype(a.probe)>(sym("nt_probe"));
    a.device_name = reinterpret_cast<decltype(a.device_name)>(sym("nt_device_name"));
    a.create = reinterpret_cast<decltype(a.create)>(sym("nt_exec_create"));
    a.set_inputs = reinterpret_cast<decltype(a.set_inputs)>(sym("nt_exec_set_inputs"));
    a.replay = reinterpret_cast<decltype(a.replay)>(sym("nt_exec_replay"));
    a.replay_many = reinterpret_cast<decltype(a.replay_many)>(sym("nt_exec_replay_many"));
    a.info = reinterpret_cast<decltype(a.info)>(sym("nt_exec_info_get"));
    a.source = reinterpret_cast<decltype(a.source)>(sym("nt_exec_source"));
    a.destroy = reinterpret_cast<decltype(a.destroy)>(sym("nt_exec_destroy"));
    a.last_error = reinterpret_cast<decltype(a.last_error)>(sym("nt_last_error"));
    auto version = reinterpret_cast<decltype(&nt_abi_version)>(sym("nt_abi_version"));
    a.loaded = ok && version() == NT_ABI_VERSION;
    if (!ok) a.error = path + " lacks an nt_* entry point";
    else if (!a.loaded) a.error = path + " has ABI version " + std::to_string(version()) + ", this host expects " +
                                  std::to_string(NT_ABI_VERSION);
  });
  return a;
}

[[noreturn]] void raise(int status, const char* what) {
  const std::string msg = std::string(what) + ": " + abi().last_error();
  switch (status) {
    case NT_E_INVALID: throw std::invalid_argument(msg);
    case NT_E_UNSUPPORTED: throw UnsupportedOperation(msg);
    case NT_E_NO_DEVICE:
    case NT_E_CLOSED: throw std::logic_error(msg);
    default: throw std::runtime_error(msg);
  }
}

int optionInt(const AadOptions& o, const char* key, int fallback) {
  auto opts = o.engineOptions("rocm");
  auto it = opts.find(key);
  return it == opts.end() ? fallback : std::atoi(it->second.c_str());
}

class RocmAadExecutable : public AadExecutable {
 public:
  RocmAadExecutable(TapePtr tape, const AadOptions& options, nt_exec* exec, double compileSeconds)
      : AadExecutable(std::move(tape), options), exec_(exec), compile_seconds_(compileSeconds) {
    setMaxChunkSeconds(RocmAadEngine::maxLaunchSeconds());
  }
  ~RocmAadExecutable() override { close(); }
  std::string engineName() const override { return "rocm"; }
  double compileSeconds() const override { return compile_seconds_; }
  void setInput(const std::string& name, double value) override {
    AadExecutable::setInput(name, value);
    dirty_ = true;
  }
  AadResult replay(long long paths, long long pathOffset, long long seed) override {
    checkOpen();
    if (paths <= 0) throw std::invalid_argument("paths must be positive");
    const RocmAbi& a = abi();
    if (dirty_) {
      int rc = a.set_inputs(exec_, inputs_.data(), static_cast<int32_t>(inputs_.size()));
      if (rc != NT_OK) raise(rc, "nt_exec_set_inputs");
      dirty_ = false;
    }
    std::vector<double> sums(static_cast<size_t>(tape().outputCount()) * (2 + inputs_.size()));
    double timing[3] = {0, 0, 0};
    int rc = a.replay(exec_, static_cast<uint64_t>(paths), static_cast<uint64_t>(pathOffset),
                      static_cast<uint64_t>(seed), sums.data(), static_cast<int32_t>(sums.size()), timing);
    if (rc != NT_OK) raise(rc, "nt_exec_replay");
    return AadResult::fromSums(sums, tape().outputNames(), tape().inputNames(), paths, timing[1] / 1e3,
                               timing[0] / 1e3);
  }
  std::vector<AadResult> replayMany(const std::vector<std::vector<double>>& inputSets, long long paths,
                                    long long pathOffset, long long seed) override {
    checkOpen();
    if (paths <= 0) throw std::invalid_argument("paths must be positive");
    if (inputSets.empty()) throw std::invalid_argument("at least one input set is required");
    const size_t nin = inputs_.size();
    std::vector<double> flat;
    flat.reserve(inputSets.size() * nin);
    for (size_t m = 0; m < inputSets.size(); ++m) {
      if (inputSets[m].size() != nin) {
        throw std::invalid_argument("input set " + std::to_string(m) + " has " + std::to_string(inputSets[m].size()) +
                                    " values; the tape has " + std::to_string(nin) + " inputs");
      }
      flat.insert(flat.end(), inputSets[m].begin(), inputSets[m].end());
    }
    const int32_t markets = static_cast<int32_t>(inputSets.size());
    const size_t one = static_cast<size_t>(tape().outputCount()) * (2 + nin);
    std::vector<double> sums(one * inputSets.size());
    double timing[3] = {0, 0, 0};
    int rc = abi().replay_many(exec_, flat.data(), markets, static_cast<uint64_t>(paths),
                               static_cast<uint64_t>(pathOffset), static_cast<uint64_t>(seed), sums.data(),
                               static_cast<int32_t>(sums.size()), timing);
    if (rc != NT_OK) raise(rc, "nt_exec_replay_many");
    std::vector<AadResult> out;
    for (int32_t m = 0; m < markets; ++m) {
      std::vector<double> part(sums.begin() + m * one, sums.begin() + (m + 1) * one);
      out.push_back(AadResult::fromSums(part, tape().outputNames(), tape().inputNames(), paths, timing[1] / 1e3,
                                        timing[0] / 1e3));
    }
    return out;
  }
  void close() override {
    if (exec_) {
      abi().destroy(exec_);
      exec_ = nullptr;
    }
    AadExecutable::close();
  }
  nt_exec* handle() const { return exec_; }
 private:
  nt_exec* exec_;
  double compile_seconds_;
  bool dirty_ = true;
};

}  // namespace

double RocmAadEngine::maxLaunchSeconds() {
  const char* env = std::getenv("NABLATENSOR_MAX_LAUNCH_SECONDS");
  return env && *env ? std::atof(env) : 0.5;
}

bool RocmAadEngine::isAvailable() const {
  try {
    const RocmAbi& a = abi();
    if (!a.loaded) return false;
    int32_t n = 0;
    return a.probe(&n) == NT_OK && n > 0;
  } catch (...) {
    return false;
  }
}

std::string RocmAadEngine::describe() const {
  try {
    const RocmAbi& a = abi();
    char name[256] = {0}, arch[64] = {0};
    if (a.loaded && a.device_name(name, sizeof name, arch, sizeof arch) == NT_OK) {
      return std::string("ROCm/HIP · ") + name + " · " + arch + " · hipRTC";
    }
  } catch (...) {
  }
  return "ROCm/HIP · no device";
}

std::unique_ptr<AadExecutable> RocmAadEngine::compile(TapePtr tape, const AadOptions& options) const {
  // Multi-output tapes, uniforms and named streams lower natively here (the
  // reference's device engines decline them with requireSupportedTape).
  const RocmAbi& a = abi();
  if (!a.loaded) throw std::logic_error("no ROCm/HIP device available for the AAD replay kernel (" + a.error + ")");
  const AadTape& t = *tape;
  nt_tape ct{};
  ct.n_nodes = t.size();
  ct.op = t.ops().data();
  ct.arg_a = t.argsA().data();
  ct.arg_b = t.argsB().data();
  ct.constant = t.constants().data();
  ct.n_inputs = t.inputCount();
  ct.input_node = t.inputNodes().data();
  ct.n_outputs = t.outputCount();
  ct.output_node = t.outputNodes().data();
  ct.n_streams = t.randStreamCount();
  ct.n_uniforms = t.randUniformCount(0);
  nt_options o{};
  o.precision = options.precision() == AadOptions::PrecisionEnum::FLOAT32 ? NT_FP32 : NT_FP64;
  o.adjoints = options.adjoints() ? 1 : 0;
  o.block = optionInt(options, "block", 0);
  o.max_blocks = optionInt(options, "maxBlocks", 0);
  o.checkpoint = optionInt(options, "checkpoint", 0);
  o.seg_len = optionInt(options, "segLen", 0);
  o.roll = optionInt(options, "roll", 1);
  o.contract = optionInt(options, "contract", 0);
  o.libm = optionInt(options, "libm", 0);
  o.mode = optionInt(options, "mode", 0);
  o.waves = optionInt(options, "waves", 0);
  o.basis = optionInt(options, "basis", 0);
  o.allow_spill = optionInt(options, "allowSpill", 0);
  const auto t0 = std::chrono::steady_clock::now();
  nt_exec* exec = nullptr;
  int rc = a.create(&ct, &o, &exec);
  if (rc != NT_OK) raise(rc, "nt_exec_create");
  const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  return std::unique_ptr<AadExecutable>(new RocmAadExecutable(tape, options, exec, secs));
}

std::map<std::string, double> rocmExecutableInfo(const AadExecutable& exe) {
  auto* r = dynamic_cast<const RocmAadExecutable*>(&exe);
  if (!r || !r->handle()) throw std::invalid_argument("not an open rocm executable");
  nt_exec_info i{};
  int rc = abi().info(r->handle(), &i);
  if (rc != NT_OK) raise(rc, "nt_exec_info_get");
  return {{"n_nodes", i.n_nodes}, {"n_active", i.n_active}, {"n_inputs", i.n_inputs}, {"n_channels", i.n_channels},
          {"loop_start", i.loop_start}, {"loop_period", i.loop_period}, {"loop_iters", i.loop_iters},
          {"loop_carries", i.loop_carries}, {"seg_len", i.seg_len}, {"n_segments", i.n_segments},
          {"checkpoint", i.checkpoint}, {"tape_slots", i.tape_slots}, {"vgprs", i.vgprs}, {"sgprs", i.sgprs},
          {"agprs", i.agprs}, {"scratch_bytes", i.scratch_bytes}, {"lds_bytes", i.lds_bytes}, {"block", i.block},
          {"grid_cap", i.grid_cap}, {"compile_seconds", i.compile_seconds}};
}

std::string rocmExecutableSource(const AadExecutable& exe) {
  auto* r = dynamic_cast<const RocmAadExecutable*>(&exe);
  if (!r || !r->handle()) throw std::invalid_argument("not an open rocm executable");
  int64_t len = 0;
  abi().source(r->handle(), nullptr, &len);
  std::string s(static_cast<size_t>(len), '\0');
  int rc = abi().source(r->handle(), &s[0], &len);
  if (rc != NT_OK) raise(rc, "nt_exec_source");
  s.resize(static_cast<size_t>(len > 0 ? len - 1 : 0));
  return s;
}

}  // namespace nablatensor
