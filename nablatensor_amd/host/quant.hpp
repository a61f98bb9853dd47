// Market records, model steps and payoffs that record the replayed tapes.
//
// Each follows the reference recording order node for node:
//   EquityMarket       nablatensor-quant/.../quant/EquityMarket.java:35-118 (field order = input order)
//   HestonMarket       nablatensor-quant/.../quant/HestonMarket.java:34-117
//   TimeGrid           nablatensor-quant/.../quant/TimeGrid.java:32-114
//   GbmPath            nablatensor-quant/.../quant/GbmPath.java:38-92
//   Smooth             nablatensor-ops/.../ops/Smooth.java:44-68
//   Products           nablatensor-quant/.../quant/Products.java:32-174
//   ExoticProducts     nablatensor-quant/.../quant/ExoticProducts.java:30-317
//   HestonModel        nablatensor-quant/.../quant/HestonModel.java:41-120
//   CorrelatedNormals  nablatensor-quant/.../quant/CorrelatedNormals.java:27-94
//   Inputs/MarketShape nablatensor-core/.../engine/Nabla.java:201-214, MarketShape.java:33-139
// HestonModel::asian and WorstOfBasket have no ready-made counterpart in the
// reference; they are recorded from the building blocks above.
#pragma once

#include <functional>
#include <string>
#include <vector>

#include "aad.hpp"

namespace nablatensor {

enum class OptionTypeEnum { CALL, PUT };

// n equally spaced steps or explicit fixing times (TimeGrid.java:43-78).
class TimeGrid {
 public:
  static TimeGrid uniform(int n);
  static TimeGrid of(const std::vector<double>& times);
  int steps() const { return static_cast<int>(fraction_.size()); }
  double fraction(int i) const { return fraction_.at(i); }
  double cumulative(int i) const;
  bool isUniform() const { return uniform_; }
 private:
  std::vector<double> fraction_;
  bool uniform_ = true;
};

// A market record: named doubles in declaration order. Typed markets derive
// from it and add accessors; the accessor of a component resolves to its index
// through a probe instance holding index + 0.25 (MarketShape.java:97-107).
class MarketRecord {
 public:
  MarketRecord() = default;
  MarketRecord(std::vector<std::string> names, std::vector<double> values);
  const std::vector<std::string>& names() const { return names_; }
  const std::vector<double>& values() const { return values_; }
  int size() const { return static_cast<int>(names_.size()); }
  int indexOf(const std::string& name) const;
  double get(const std::string& name) const { return values_.at(indexOf(name)); }
 protected:
  std::vector<std::string> names_;
  std::vector<double> values_;
};

class EquityMarket : public MarketRecord {
 public:
  class Builder {
   public:
    Builder& spot(double v) { v_[0] = v; return *this; }
    Builder& strike(double v) { v_[1] = v; return *this; }
    Builder& vol(double v) { v_[2] = v; return *this; }
    Builder& rate(double v) { v_[3] = v; return *this; }
    Builder& maturity(double v) { v_[4] = v; return *this; }
    EquityMarket build() const { return EquityMarket(v_); }
   private:
    std::vector<double> v_ = std::vector<double>(5, 0.0);
  };
  explicit EquityMarket(const std::vector<double>& values);
  static Builder of() { return Builder(); }
  static EquityMarket atmOneYear();
  static EquityMarket probe();
  double spot() const { return values_[0]; }
  double strike() const { return values_[1]; }
  double vol() const { return values_[2]; }
  double rate() const { return values_[3]; }
  double maturity() const { return values_[4]; }
  const EquityMarket& validated() const;  // EquityMarket.java:84-92
  EquityMarket withSpot(double v) const;
  EquityMarket withStrike(double v) const;
  EquityMarket withVol(double v) const;
  EquityMarket withRate(double v) const;
  EquityMarket withMaturity(double v) const;
};

class HestonMarket : public MarketRecord {
 public:
  class Builder {
   public:
    Builder& spot(double v) { v_[0] = v; return *this; }
    Builder& strike(double v) { v_[1] = v; return *this; }
    Builder& rate(double v) { v_[2] = v; return *this; }
    Builder& v0(double v) { v_[3] = v; return *this; }
    Builder& kappa(double v) { v_[4] = v; return *this; }
    Builder& theta(double v) { v_[5] = v; return *this; }
    Builder& xi(double v) { v_[6] = v; return *this; }
    Builder& rho(double v) { v_[7] = v; return *this; }
    HestonMarket build() const { return HestonMarket(v_); }
   private:
    std::vector<double> v_ = std::vector<double>(8, 0.0);
  };
  explicit HestonMarket(const std::vector<double>& values);
  static Builder of() { return Builder(); }
  static HestonMarket probe();
  double spot() const { return values_[0]; }
  double strike() const { return values_[1]; }
  double rate() const { return values_[2]; }
  double v0() const { return values_[3]; }
  double kappa() const { return values_[4]; }
  double theta() const { return values_[5]; }
  double xi() const { return values_[6]; }
  double rho() const { return values_[7]; }
  const HestonMarket& validated() const;  // HestonMarket.java:86-92
};

// One INPUT node per market component, recorded in declaration order
// (Nabla.java:201-207); of() reads an input, recording nothing.
template <class M>
class Inputs {
 public:
  Inputs(AadRecorder& rec, const MarketRecord& defaults) {
    for (int i = 0; i < defaults.size(); ++i) {
      inputs_.push_back(rec.input(defaults.names()[i], defaults.values()[i]));
    }
    names_ = defaults.names();
  }
  ADouble of(double (M::*accessor)() const) const {
    double probed = (M::probe().*accessor)() - 0.25;
    int index = static_cast<int>(probed);
    if (index != probed || index < 0 || index >= static_cast<int>(inputs_.size())) {
      throw std::invalid_argument("expected a plain component accessor");
    }
    return inputs_[index];
  }
  ADouble of(const std::string& name) const {
    for (size_t i = 0; i < names_.size(); ++i) {
      if (names_[i] == name) return inputs_[i];
    }
    throw std::invalid_argument("unknown market component: " + name);
  }
 private:
  std::vector<ADouble> inputs_;
  std::vector<std::string> names_;
};

template <class M>
struct Product {
  std::string label;
  std::function<void(AadRecorder&, Inputs<M>&, const TimeGrid&)> record;
};

// GBM log-Euler step block (GbmPath.java:38-92).
class GbmPath {
 public:
  static GbmPath of(AadRecorder& rec, const ADouble& rate, const ADouble& vol, const TimeGrid& grid,
                    const ADouble& maturity);
  ADouble step(const ADouble& spot, const ADouble& z, int i) const;
 private:
  std::vector<ADouble> drift_, diffusion_;
};

// Smoothed indicators (Smooth.java:44-68).
struct Smooth {
  static ADouble step(AadRecorder& rec, const ADouble& x, double width);
  static ADouble gt(AadRecorder& rec, const ADouble& a, const ADouble& b, double width);
  static ADouble gt(AadRecorder& rec, const ADouble& a, double level, double width);
  static ADouble lt(AadRecorder& rec, const ADouble& a, double level, double width);
  static ADouble lt(AadRecorder& rec, const ADouble& a, const ADouble& b, double width);
};

struct Products {
  static Product<EquityMarket> european(OptionTypeEnum type);
  static Product<EquityMarket> asian(OptionTypeEnum type);
  static Product<EquityMarket> lookback(OptionTypeEnum type);
  static Product<EquityMarket> europeanCall() { return european(OptionTypeEnum::CALL); }
  static Product<EquityMarket> europeanPut() { return european(OptionTypeEnum::PUT); }
  static Product<EquityMarket> asianCall() { return asian(OptionTypeEnum::CALL); }
  static Product<EquityMarket> asianPut() { return asian(OptionTypeEnum::PUT); }
  static Product<EquityMarket> lookbackCall() { return lookback(OptionTypeEnum::CALL); }
  static Product<EquityMarket> lookbackPut() { return lookback(OptionTypeEnum::PUT); }
};

struct ExoticProducts {
  enum class BarrierEnum { UP_OUT, UP_IN, DOWN_OUT, DOWN_IN };
  static Product<EquityMarket> barrier(OptionTypeEnum type, BarrierEnum kind, double barrier, double width);
  static Product<EquityMarket> digitalCash(OptionTypeEnum type, double cash, double width);
};

// Heston full-truncation Euler step block (HestonModel.java:41-102).
class HestonModel {
 public:
  struct State { ADouble spot, variance; };
  static HestonModel of(const Inputs<HestonMarket>& in, double maturity, int steps);
  State start(const Inputs<HestonMarket>& in) const;
  State step(AadRecorder& rec, const State& s, const ADouble& z1, const ADouble& zv) const;
  // HestonModel.european, HestonModel.java:104-119.
  static std::function<void(AadRecorder&, Inputs<HestonMarket>&)> european(OptionTypeEnum type,
                                                                            double maturity, int steps);
  // Arithmetic-average Asian on the Heston path: same step block, a running sum
  // as in Products.asian (Products.java:82-94), discount as in european.
  static std::function<void(AadRecorder&, Inputs<HestonMarket>&)> asian(OptionTypeEnum type,
                                                                         double maturity, int steps);
 private:
  ADouble rate_, kappa_, theta_, xi_, rho_, rhoBar_;
  double dt_ = 0.0, sqrtDt_ = 0.0;
};

// Fixed Cholesky mixing of independent draws (CorrelatedNormals.java:27-94).
class CorrelatedNormals {
 public:
  static CorrelatedNormals of(const std::vector<std::vector<double>>& corr);
  int size() const { return static_cast<int>(lower_.size()); }
  const std::vector<std::vector<double>>& lower() const { return lower_; }
  std::vector<ADouble> mix(AadRecorder& rec, const std::vector<ADouble>& independent) const;
  std::vector<ADouble> draw(AadRecorder& rec) const;
 private:
  std::vector<std::vector<double>> lower_;
};

// Worst-of call on n correlated GBM assets: inputs spot0..n-1, vol0..n-1, rate;
// maturity and strike are recorded as constants. Per step: draw() of the
// correlated normals, then one GbmPath step per asset; payoff
// max(min_i S_i(T) - strike, 0) e^{-rT}.
struct WorstOfBasket {
  static MarketRecord market(const std::vector<double>& spots, const std::vector<double>& vols, double rate);
  static std::function<void(AadRecorder&, Inputs<MarketRecord>&)> call(
      const std::vector<std::vector<double>>& corr, double strike, double maturity, int steps);
};

}  // namespace nablatensor
