// Engine SPI, selection, chunked replay, results and the typed facade.
//
// Mirrors the reference interfaces a caller of the `rocm` engine touches:
//   AadOptions            nablatensor-core/.../engine/AadOptions.java:42-156
//   AadResult             AadResult.java:38-197
//   AadResultAccumulator  AadResultAccumulator.java:30-97
//   AadExecutable         AadExecutable.java:37-78 and the chunking of
//                         AbstractAadExecutable.java:100-159
//   AadEngine / AadEngines AadEngine.java:28-87, AadEngines.java:33-111
//   RocmAadEngine         nablatensor-engine-rocm/.../engine/rocm/RocmAadEngine.java:40-87
//   Nabla / MonteCarlo    Nabla.java:159-575, nablatensor-quant/.../quant/MonteCarlo.java:49-207
// RocmAadEngine binds libnt_rocm.so (include/nablatensor_rocm.h) with dlopen /
// dlsym, the C++ counterpart of the Java FFM downcalls. Errors map to the
// reference's exception types: std::invalid_argument for
// IllegalArgumentException, std::logic_error for IllegalStateException,
// UnsupportedOperation for UnsupportedOperationException, std::runtime_error
// for a failed device call.
#pragma once

#include <chrono>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "aad.hpp"
#include "quant.hpp"

namespace nablatensor {

struct UnsupportedOperation : std::logic_error {
  using std::logic_error::logic_error;
};

class AadOptions {
 public:
  enum class PrecisionEnum { FLOAT32, FLOAT64 };
  static AadOptions defaults() { return AadOptions(); }  // FLOAT32, adjoints, threads 0 (AadOptions.java:110-112)
  PrecisionEnum precision() const { return precision_; }
  bool adjoints() const { return adjoints_; }
  int threads() const { return threads_; }
  AadOptions withPrecision(PrecisionEnum p) const { AadOptions o = *this; o.precision_ = p; return o; }
  AadOptions withAdjoints(bool a) const { AadOptions o = *this; o.adjoints_ = a; return o; }
  AadOptions withThreads(int t) const { AadOptions o = *this; o.threads_ = t; return o; }
  AadOptions withEngineOption(const std::string& engine, const std::string& key, const std::string& value) const {
    AadOptions o = *this;
    o.engine_options_[engine][key] = value;
    return o;
  }
  std::map<std::string, std::string> engineOptions(const std::string& engine) const {
    auto it = engine_options_.find(engine);
    return it == engine_options_.end() ? std::map<std::string, std::string>{} : it->second;
  }
 private:
  PrecisionEnum precision_ = PrecisionEnum::FLOAT32;
  bool adjoints_ = true;
  int threads_ = 0;
  std::map<std::string, std::map<std::string, std::string>> engine_options_;
};

// Single-output replay result. Besides the means it keeps the raw sums of the
// dispatch, so chunked results combine exactly.
class AadResult {
 public:
  AadResult(double value, double standardError, std::vector<double> gradients, std::vector<std::string> inputNames,
            long long paths, double seconds);
  double value() const { return value_; }
  double standardError() const { return stderr_; }
  const std::vector<double>& gradients() const { return gradients_; }
  double gradient(const std::string& inputName) const;
  const std::vector<std::string>& inputNames() const { return input_names_; }
  // Every recorded output (AadResult.java:88-151); output 0 is the one the
  // accessors above report.
  const std::vector<std::string>& outputNames() const { return output_names_; }
  int outputCount() const { return static_cast<int>(output_names_.size()); }
  double value(const std::string& outputName) const { return values_.at(outputIndex(outputName)); }
  double standardError(const std::string& outputName) const { return stderrs_.at(outputIndex(outputName)); }
  double gradient(const std::string& outputName, const std::string& inputName) const;
  const std::vector<double>& gradients(const std::string& outputName) const {
    return jacobian_.at(outputIndex(outputName));
  }
  long long paths() const { return paths_; }
  double seconds() const { return seconds_; }
  double pathsPerSecond() const { return paths_ / seconds_; }
  std::string toString() const;
  // raw sums (sum y, sum y^2, sum adjoint_j); empty when built from means only
  const std::vector<double>& rawSums() const { return raw_; }
  double kernelSeconds() const { return kernel_seconds_; }
  // sums: per output, [sum y, sum y^2, sum dy/dx_j] (AadTotals.toResult, AadTotals.java:68-89)
  static AadResult fromSums(const std::vector<double>& sums, const std::vector<std::string>& outputNames,
                            const std::vector<std::string>& inputNames, long long paths, double seconds,
                            double kernelSeconds);
 private:
  int outputIndex(const std::string& outputName) const;
  double value_, stderr_;
  std::vector<std::string> output_names_;
  std::vector<double> values_, stderrs_;
  std::vector<std::vector<double>> jacobian_;
  std::vector<double> gradients_;
  std::vector<std::string> input_names_;
  long long paths_;
  double seconds_;
  std::vector<double> raw_;
  double kernel_seconds_ = 0.0;
};

class AadExecutable {
 public:
  explicit AadExecutable(TapePtr tape, const AadOptions& options);
  virtual ~AadExecutable() = default;
  virtual std::string engineName() const = 0;
  const AadTape& tape() const { return *tape_; }
  TapePtr tapePtr() const { return tape_; }
  virtual void setInput(const std::string& name, double value);
  virtual AadResult replay(long long paths, long long pathOffset, long long seed) = 0;
  // Prices every input set (each in tape().inputNames() order) over the same
  // paths and seed; results equal one replay per set with those inputs. The
  // bound inputs are left unchanged. Engines that can share each path's draws
  // across the sets override it (VulkanAadKernel.replayMany,
  // nablatensor-engine-vulkan/.../VulkanAadKernel.java:162-238).
  virtual std::vector<AadResult> replayMany(const std::vector<std::vector<double>>& inputSets, long long paths,
                                            long long pathOffset, long long seed);
  virtual void close() { closed_ = true; }
  virtual double compileSeconds() const { return 0.0; }
  AadResult replaySafe(long long totalPaths, long long seed);
  double calibrate(long long seed);
  double measuredPathsPerSecond() const { return paths_per_second_; }
  double maxChunkSeconds() const { return max_chunk_seconds_; }
  void setMaxChunkSeconds(double seconds);
 protected:
  void checkOpen() const;
  TapePtr tape_;
  AadOptions options_;
  std::vector<double> inputs_;
 private:
  void observe(long long paths, double seconds);
  long long budgetedChunk() const;
  double paths_per_second_ = 0.0;
  double max_chunk_seconds_ = 2.0;
  bool closed_ = false;
};

class AadEngine {
 public:
  virtual ~AadEngine() = default;
  virtual std::string name() const = 0;
  virtual int priority() const = 0;
  virtual bool isAvailable() const = 0;  // must never throw
  virtual bool supports(const AadOptions& options) const = 0;
  virtual std::string describe() const = 0;
  virtual std::unique_ptr<AadExecutable> compile(TapePtr tape, const AadOptions& options) const = 0;
  // AadEngine.requireSupportedTape, AadEngine.java:56-86
  void requireSupportedTape(const AadTape& tape) const;
};

struct AadEngines {
  static void registerEngine(std::shared_ptr<AadEngine> engine);
  static std::vector<std::shared_ptr<AadEngine>> discovered();
  static std::vector<std::shared_ptr<AadEngine>> available(const AadOptions& options);
  static std::shared_ptr<AadEngine> find(const std::string& name, const AadOptions& options);
  static std::shared_ptr<AadEngine> require(const std::string& name, const AadOptions& options);
  // NABLATENSOR_ENGINE plays the role of -Dnablatensor.engine (AadEngines.java:35,83-94).
  static std::shared_ptr<AadEngine> select(const AadOptions& options);
};

// The `rocm` engine over libnt_rocm.so. Priority 55, as the reference's.
class RocmAadEngine : public AadEngine {
 public:
  std::string name() const override { return "rocm"; }
  int priority() const override { return 55; }
  bool isAvailable() const override;
  bool supports(const AadOptions&) const override { return true; }
  std::string describe() const override;
  std::unique_ptr<AadExecutable> compile(TapePtr tape, const AadOptions& options) const override;
  // 0.5 s per dispatch, RocmAadEngine.java:85 (NABLATENSOR_MAX_LAUNCH_SECONDS overrides)
  static double maxLaunchSeconds();
};

// Executable statistics of a rocm executable (nt_exec_info as a map).
std::map<std::string, double> rocmExecutableInfo(const AadExecutable& exe);
std::string rocmExecutableSource(const AadExecutable& exe);

// ---- typed facade (Nabla.java:159-575) -------------------------------------------

template <class M>
class TypedValuation {
 public:
  TypedValuation(AadResult result, M shapeDefaults) : result_(std::move(result)), shape_(std::move(shapeDefaults)) {}
  double price() const { return result_.value(); }
  double standardError() const { return result_.standardError(); }
  M greeks() const { return M(result_.gradients()); }
  double greek(double (M::*accessor)() const) const { return (greeks().*accessor)(); }
  double greek(const std::string& name) const { return result_.gradient(name); }
  long long scenarios() const { return result_.paths(); }
  double seconds() const { return result_.seconds(); }
  double scenariosPerSecond() const { return result_.pathsPerSecond(); }
  const AadResult& result() const { return result_; }
 private:
  AadResult result_;
  M shape_;
};

template <class M>
class TypedPricer {
 public:
  TypedPricer(std::unique_ptr<AadExecutable> exe, M defaults, double recordSeconds, double buildSeconds)
      : exe_(std::move(exe)), defaults_(std::move(defaults)), record_(recordSeconds), build_(buildSeconds) {}
  // TypedRequest.with(market).scenarios(n).seed(s).run() in one call.
  TypedValuation<M> run(const M& state, long long scenarios, long long seed) {
    for (int i = 0; i < state.size(); ++i) exe_->setInput(state.names()[i], state.values()[i]);
    return TypedValuation<M>(exe_->replaySafe(scenarios, seed), defaults_);
  }
  std::string engine() const { return exe_->engineName(); }
  int nodes() const { return exe_->tape().size(); }
  double recordSeconds() const { return record_; }
  double buildSeconds() const { return build_; }
  AadExecutable& executable() { return *exe_; }
  void close() { exe_->close(); }
 private:
  std::unique_ptr<AadExecutable> exe_;
  M defaults_;
  double record_, build_;
};

template <class M>
class TypedModel {
 public:
  TypedModel(TapePtr tape, M defaults, double recordSeconds)
      : tape_(std::move(tape)), defaults_(std::move(defaults)), record_(recordSeconds) {}
  TypedModel& fp32() { options_ = options_.withPrecision(AadOptions::PrecisionEnum::FLOAT32); return *this; }
  TypedModel& fp64() { options_ = options_.withPrecision(AadOptions::PrecisionEnum::FLOAT64); return *this; }
  TypedModel& greeks() { options_ = options_.withAdjoints(true); return *this; }
  TypedModel& priceOnly() { options_ = options_.withAdjoints(false); return *this; }
  TypedModel& threads(int n) { options_ = options_.withThreads(n); return *this; }
  TypedModel& on(const std::string& engine) { engine_ = engine; return *this; }
  TypedModel& fastest() { engine_.clear(); return *this; }
  TypedModel& tune(const std::string& engine, const std::string& key, const std::string& value) {
    options_ = options_.withEngineOption(engine, key, value);
    return *this;
  }
  TapePtr tape() const { return tape_; }
  const AadOptions& options() const { return options_; }
  std::unique_ptr<TypedPricer<M>> build() const {
    const auto t0 = std::chrono::steady_clock::now();
    auto engine = engine_.empty() ? AadEngines::select(options_) : AadEngines::require(engine_, options_);
    auto exe = engine->compile(tape_, options_);
    const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    return std::unique_ptr<TypedPricer<M>>(new TypedPricer<M>(std::move(exe), defaults_, record_, secs));
  }
 private:
  TapePtr tape_;
  M defaults_;
  double record_;
  AadOptions options_;
  std::string engine_;
};

struct Nabla {
  template <class M>
  static TypedModel<M> model(const M& defaults, const std::function<void(AadRecorder&, Inputs<M>&)>& valuation) {
    const auto t0 = std::chrono::steady_clock::now();
    TapePtr tape = AadRecorder::record([&](AadRecorder& rec) {
      Inputs<M> in(rec, defaults);
      valuation(rec, in);
    });
    const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    return TypedModel<M>(tape, defaults, secs);
  }
};

// MonteCarlo.of(product).market(m).steps(n).greeks().fp64().on("rocm").build() (MonteCarlo.java:107-205).
template <class M>
class MonteCarlo {
 public:
  class Builder {
   public:
    explicit Builder(Product<M> product) : product_(std::move(product)) {}
    Builder& market(const M& m) { market_.reset(new M(m)); return *this; }
    Builder& steps(int n) { grid_ = TimeGrid::uniform(n); return *this; }
    Builder& timeGrid(const TimeGrid& g) { grid_ = g; return *this; }
    Builder& greeks() { greeks_ = true; return *this; }
    Builder& priceOnly() { greeks_ = false; return *this; }
    Builder& fp32() { fp32_ = true; return *this; }
    Builder& fp64() { fp32_ = false; return *this; }
    Builder& threads(int n) { threads_ = n; return *this; }
    Builder& on(const std::string& engine) { engine_ = engine; return *this; }
    Builder& fastest() { engine_.clear(); return *this; }
    Builder& tune(const std::string& key, const std::string& value) { tune_[key] = value; return *this; }
    std::unique_ptr<MonteCarlo<M>> build() const {
      if (!market_) throw std::logic_error("MonteCarlo.Builder needs .market(...) before .build()");
      market_->validated();
      const Product<M> p = product_;
      const TimeGrid g = grid_;
      TypedModel<M> model = Nabla::model<M>(*market_, [&](AadRecorder& rec, Inputs<M>& in) { p.record(rec, in, g); });
      if (fp32_) model.fp32(); else model.fp64();
      if (greeks_) model.greeks(); else model.priceOnly();
      if (threads_ > 0) model.threads(threads_);
      for (auto& kv : tune_) model.tune("rocm", kv.first, kv.second);
      if (engine_.empty()) model.fastest(); else model.on(engine_);
      return std::unique_ptr<MonteCarlo<M>>(new MonteCarlo<M>(model.build(), *market_, greeks_, model.tape()));
    }
   private:
    Product<M> product_;
    std::unique_ptr<M> market_;
    TimeGrid grid_ = TimeGrid::uniform(252);
    bool greeks_ = true;
    bool fp32_ = false;  // MonteCarlo defaults to fp64 (MonteCarlo.java:113)
    int threads_ = 0;
    std::string engine_;
    std::map<std::string, std::string> tune_;
  };
  static Builder of(const Product<M>& product) { return Builder(product); }
  const M& market() const { return market_; }
  bool hasGreeks() const { return greeks_; }
  std::string engine() const { return pricer_->engine(); }
  int nodes() const { return pricer_->nodes(); }
  double recordSeconds() const { return pricer_->recordSeconds(); }
  double buildSeconds() const { return pricer_->buildSeconds(); }
  TypedValuation<M> run(long long scenarios, long long seed) { return run(market_, scenarios, seed); }
  TypedValuation<M> run(const M& state, long long scenarios, long long seed) { return pricer_->run(state, scenarios, seed); }
  TapePtr tape() const { return tape_; }
  AadExecutable& executable() { return pricer_->executable(); }
  void close() { pricer_->close(); }
 private:
  MonteCarlo(std::unique_ptr<TypedPricer<M>> pricer, M market, bool greeks, TapePtr tape)
      : pricer_(std::move(pricer)), market_(std::move(market)), greeks_(greeks), tape_(std::move(tape)) {}
  std::unique_ptr<TypedPricer<M>> pricer_;
  M market_;
  bool greeks_;
  TapePtr tape_;
};

}  // namespace nablatensor
