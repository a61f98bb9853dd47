// Market records, model steps and payoffs; see quant.hpp for the reference
// file each one follows. Statements are split wherever a Java expression
// records nodes from more than one operand, so the order stays left to right.
#include "quant.hpp"

#include <cmath>
#include <sstream>

namespace nablatensor {

// ---- TimeGrid (TimeGrid.java:43-78) ------------------------------------------

TimeGrid TimeGrid::uniform(int n) {
  if (n < 1) throw std::invalid_argument("steps must be >= 1, got " + std::to_string(n));
  TimeGrid g;
  g.fraction_.assign(n, 1.0 / n);
  g.uniform_ = true;
  return g;
}

TimeGrid TimeGrid::of(const std::vector<double>& times) {
  if (times.empty()) throw std::invalid_argument("need at least one fixing time");
  double total = times.back();
  if (!(total > 0.0)) throw std::invalid_argument("the last fixing time must be positive");
  TimeGrid g;
  double prev = 0.0;
  for (double t : times) {
    double gap = t - prev;
    if (!(gap > 0.0)) throw std::invalid_argument("fixing times must be strictly ascending and positive");
    g.fraction_.push_back(gap / total);
    prev = t;
  }
  g.uniform_ = true;
  for (double v : g.fraction_) {
    if (std::fabs(v - g.fraction_[0]) > 1e-12) {
      g.uniform_ = false;
      break;
    }
  }
  return g;
}

double TimeGrid::cumulative(int i) const {
  double c = 0.0;
  for (int k = 0; k <= i; ++k) c += fraction_.at(k);
  return c;
}

// ---- market records ------------------------------------------------------------

MarketRecord::MarketRecord(std::vector<std::string> names, std::vector<double> values)
    : names_(std::move(names)), values_(std::move(values)) {
  if (names_.size() != values_.size()) throw std::invalid_argument("market names and values differ in length");
  if (names_.empty()) throw std::invalid_argument("a market needs at least one component");
}

int MarketRecord::indexOf(const std::string& name) const {
  for (size_t i = 0; i < names_.size(); ++i) {
    if (names_[i] == name) return static_cast<int>(i);
  }
  throw std::invalid_argument("unknown market component: " + name);
}

static std::vector<double> probe_values(int n) {
  std::vector<double> v(n);
  for (int i = 0; i < n; ++i) v[i] = i + 0.25;
  return v;
}

EquityMarket::EquityMarket(const std::vector<double>& values)
    : MarketRecord({"spot", "strike", "vol", "rate", "maturity"}, values) {}

EquityMarket EquityMarket::atmOneYear() {
  return of().spot(100.0).strike(100.0).vol(0.20).rate(0.03).maturity(1.0).build();
}
EquityMarket EquityMarket::probe() { return EquityMarket(probe_values(5)); }

const EquityMarket& EquityMarket::validated() const {
  if (!(vol() >= 0.0) || !(maturity() >= 0.0) || !(spot() > 0.0) || !(strike() > 0.0)) {
    std::ostringstream s;
    s << "need spot>0, strike>0, vol>=0, maturity>=0; got " << spot() << "/" << strike() << "/" << vol()
      << "/" << maturity();
    throw std::invalid_argument(s.str());
  }
  return *this;
}

EquityMarket EquityMarket::withSpot(double v) const { auto x = values_; x[0] = v; return EquityMarket(x); }
EquityMarket EquityMarket::withStrike(double v) const { auto x = values_; x[1] = v; return EquityMarket(x); }
EquityMarket EquityMarket::withVol(double v) const { auto x = values_; x[2] = v; return EquityMarket(x); }
EquityMarket EquityMarket::withRate(double v) const { auto x = values_; x[3] = v; return EquityMarket(x); }
EquityMarket EquityMarket::withMaturity(double v) const { auto x = values_; x[4] = v; return EquityMarket(x); }

HestonMarket::HestonMarket(const std::vector<double>& values)
    : MarketRecord({"spot", "strike", "rate", "v0", "kappa", "theta", "xi", "rho"}, values) {}

HestonMarket HestonMarket::probe() { return HestonMarket(probe_values(8)); }

const HestonMarket& HestonMarket::validated() const {
  if (!(spot() > 0 && strike() > 0 && v0() >= 0 && kappa() >= 0 && theta() >= 0 && xi() >= 0 && rho() > -1.0 &&
        rho() < 1.0)) {
    throw std::invalid_argument("invalid Heston market");
  }
  return *this;
}

// ---- GbmPath (GbmPath.java:48-91) ----------------------------------------------

GbmPath GbmPath::of(AadRecorder& rec, const ADouble& rate, const ADouble& vol, const TimeGrid& grid,
                    const ADouble& maturity) {
  (void)rec;
  GbmPath p;
  const int n = grid.steps();
  ADouble var = vol.mul(vol);
  ADouble halfVarTerm = var.mul(0.5);
  ADouble halfVar = rate.sub(halfVarTerm);
  if (grid.isUniform()) {
    ADouble dt = maturity.mul(grid.fraction(0));
    ADouble d = halfVar.mul(dt);
    ADouble sq = dt.sqrt();
    ADouble s = vol.mul(sq);
    p.drift_.assign(n, d);
    p.diffusion_.assign(n, s);
  } else {
    for (int i = 0; i < n; ++i) {
      ADouble dt = maturity.mul(grid.fraction(i));
      p.drift_.push_back(halfVar.mul(dt));
      ADouble sq = dt.sqrt();
      p.diffusion_.push_back(vol.mul(sq));
    }
  }
  return p;
}

// spot * exp(drift_i + diffusion_i * z): MUL, ADD, EXP, MUL.
ADouble GbmPath::step(const ADouble& spot, const ADouble& z, int i) const {
  ADouble m = diffusion_.at(i).mul(z);
  ADouble a = drift_.at(i).add(m);
  ADouble e = a.exp();
  return spot.mul(e);
}

// ---- Smooth (Smooth.java:44-68) ------------------------------------------------

ADouble Smooth::step(AadRecorder& rec, const ADouble& x, double width) {
  if (!(width > 0.0) || !std::isfinite(width)) throw std::invalid_argument("width must be positive and finite");
  ADouble e = x.div(width).neg().exp();  // exp(-x/width)
  ADouble one = rec.constant(1.0);       // the receiver is recorded before the argument
  ADouble den = e.add(1.0);
  return one.div(den);
}
ADouble Smooth::gt(AadRecorder& rec, const ADouble& a, const ADouble& b, double width) {
  return step(rec, a.sub(b), width);
}
ADouble Smooth::gt(AadRecorder& rec, const ADouble& a, double level, double width) {
  return step(rec, a.sub(level), width);
}
ADouble Smooth::lt(AadRecorder& rec, const ADouble& a, double level, double width) {
  return step(rec, a.neg().add(level), width);
}
ADouble Smooth::lt(AadRecorder& rec, const ADouble& a, const ADouble& b, double width) {
  return step(rec, b.sub(a), width);
}

// ---- Products (Products.java:70-173) -------------------------------------------

namespace {

struct Sim {
  ADouble spot, strike, rate, maturity;
  GbmPath model;
  Sim(AadRecorder& rec, Inputs<EquityMarket>& in, const TimeGrid& grid)
      : spot(in.of(&EquityMarket::spot)),
        strike(in.of(&EquityMarket::strike)),
        rate(in.of(&EquityMarket::rate)),
        maturity(in.of(&EquityMarket::maturity)),
        model(GbmPath::of(rec, rate, in.of(&EquityMarket::vol), grid, maturity)) {}
  // payoff * exp(-rate * maturity): NEG, MUL, EXP, MUL.
  ADouble discount(const ADouble& payoff) const { return payoff.mul(rate.neg().mul(maturity).exp()); }
};

ADouble intrinsic(OptionTypeEnum type, const ADouble& underlying, const ADouble& strike) {
  ADouble diff = type == OptionTypeEnum::CALL ? underlying.sub(strike) : strike.sub(underlying);
  return diff.max(0.0);
}

const char* type_name(OptionTypeEnum t) { return t == OptionTypeEnum::CALL ? "CALL" : "PUT"; }

}  // namespace

Product<EquityMarket> Products::european(OptionTypeEnum type) {
  return {std::string("European ") + type_name(type),
          [type](AadRecorder& rec, Inputs<EquityMarket>& in, const TimeGrid& grid) {
            Sim sim(rec, in, grid);
            ADouble terminal = sim.spot;
            for (int t = 0; t < grid.steps(); ++t) {
              ADouble z = rec.randn();
              terminal = sim.model.step(terminal, z, t);
            }
            rec.output(sim.discount(intrinsic(type, terminal, sim.strike)));
          }};
}

Product<EquityMarket> Products::asian(OptionTypeEnum type) {
  return {std::string("Asian ") + type_name(type),
          [type](AadRecorder& rec, Inputs<EquityMarket>& in, const TimeGrid& grid) {
            Sim sim(rec, in, grid);
            ADouble path = sim.spot;
            ADouble sum = rec.constant(0.0);
            for (int t = 0; t < grid.steps(); ++t) {
              ADouble z = rec.randn();
              path = sim.model.step(path, z, t);
              sum = sum.add(path);
            }
            ADouble average = sum.div(static_cast<double>(grid.steps()));
            rec.output(sim.discount(intrinsic(type, average, sim.strike)));
          }};
}

Product<EquityMarket> Products::lookback(OptionTypeEnum type) {
  return {std::string("Lookback ") + type_name(type),
          [type](AadRecorder& rec, Inputs<EquityMarket>& in, const TimeGrid& grid) {
            Sim sim(rec, in, grid);
            ADouble path = sim.spot;
            ADouble extremum = sim.spot;
            for (int t = 0; t < grid.steps(); ++t) {
              ADouble z = rec.randn();
              path = sim.model.step(path, z, t);
              extremum = type == OptionTypeEnum::CALL ? extremum.max(path) : extremum.min(path);
            }
            ADouble value = type == OptionTypeEnum::CALL ? extremum.sub(sim.strike).max(0.0)
                                                         : sim.strike.sub(extremum).max(0.0);
            rec.output(sim.discount(value));
          }};
}

// ---- ExoticProducts (ExoticProducts.java:55-93) ----------------------------------

Product<EquityMarket> ExoticProducts::barrier(OptionTypeEnum type, BarrierEnum kind, double level, double width) {
  static const char* kinds[] = {"UP_OUT", "UP_IN", "DOWN_OUT", "DOWN_IN"};
  return {std::string("BarrierEnum ") + kinds[static_cast<int>(kind)] + " " + type_name(type),
          [=](AadRecorder& rec, Inputs<EquityMarket>& in, const TimeGrid& grid) {
            Sim sim(rec, in, grid);
            ADouble path = sim.spot;
            ADouble survival = rec.constant(1.0);
            const bool up = kind == BarrierEnum::UP_OUT || kind == BarrierEnum::UP_IN;
            for (int t = 0; t < grid.steps(); ++t) {
              ADouble z = rec.randn();
              path = sim.model.step(path, z, t);
              ADouble notBreached = up ? Smooth::lt(rec, path, level, width) : Smooth::gt(rec, path, level, width);
              survival = survival.mul(notBreached);
            }
            ADouble vanilla = type == OptionTypeEnum::CALL ? path.sub(sim.strike).max(0.0)
                                                           : sim.strike.sub(path).max(0.0);
            const bool knockOut = kind == BarrierEnum::UP_OUT || kind == BarrierEnum::DOWN_OUT;
            ADouble alive = survival;
            if (!knockOut) {
              ADouble one = rec.constant(1.0);
              alive = one.sub(survival);
            }
            rec.output(sim.discount(vanilla.mul(alive)));
          }};
}

Product<EquityMarket> ExoticProducts::digitalCash(OptionTypeEnum type, double cash, double width) {
  return {std::string("Digital cash ") + type_name(type),
          [=](AadRecorder& rec, Inputs<EquityMarket>& in, const TimeGrid& grid) {
            Sim sim(rec, in, grid);
            ADouble s = sim.spot;
            for (int t = 0; t < grid.steps(); ++t) {
              ADouble z = rec.randn();
              s = sim.model.step(s, z, t);
            }
            ADouble itm = type == OptionTypeEnum::CALL ? Smooth::gt(rec, s, sim.strike, width)
                                                       : Smooth::lt(rec, s, sim.strike, width);
            rec.output(sim.discount(itm.mul(cash)));
          }};
}

// ---- HestonModel (HestonModel.java:59-119) ---------------------------------------

HestonModel HestonModel::of(const Inputs<HestonMarket>& in, double maturity, int steps) {
  HestonModel m;
  m.rate_ = in.of(&HestonMarket::rate);
  m.kappa_ = in.of(&HestonMarket::kappa);
  m.theta_ = in.of(&HestonMarket::theta);
  m.xi_ = in.of(&HestonMarket::xi);
  m.rho_ = in.of(&HestonMarket::rho);
  m.rhoBar_ = m.rho_.mul(m.rho_).neg().add(1.0).sqrt();
  m.dt_ = maturity / steps;
  m.sqrtDt_ = std::sqrt(m.dt_);
  return m;
}

HestonModel::State HestonModel::start(const Inputs<HestonMarket>& in) const {
  return {in.of(&HestonMarket::spot), in.of(&HestonMarket::v0)};
}

HestonModel::State HestonModel::step(AadRecorder& rec, const State& s, const ADouble& z1, const ADouble& zv) const {
  (void)rec;
  ADouble rz1 = rho_.mul(z1);
  ADouble rbzv = rhoBar_.mul(zv);
  ADouble z2 = rz1.add(rbzv);  // corr(z1, z2) = rho

  ADouble vPlus = s.variance.max(0.0);
  ADouble sqrtV = vPlus.sqrt();

  ADouble meanRev = kappa_.mul(theta_.sub(vPlus)).mul(dt_);
  ADouble vDrifted = s.variance.add(meanRev);
  ADouble volOfVol = xi_.mul(sqrtV).mul(sqrtDt_).mul(z2);
  ADouble vNext = vDrifted.add(volOfVol);

  ADouble halfV = vPlus.mul(0.5);
  ADouble logDrift = rate_.sub(halfV).mul(dt_);
  ADouble shock = sqrtV.mul(sqrtDt_).mul(z1);
  ADouble growth = logDrift.add(shock).exp();
  ADouble sNext = s.spot.mul(growth);
  return {sNext, vNext};
}

std::function<void(AadRecorder&, Inputs<HestonMarket>&)> HestonModel::european(OptionTypeEnum type,
                                                                                double maturity, int steps) {
  return [=](AadRecorder& rec, Inputs<HestonMarket>& in) {
    HestonModel m = HestonModel::of(in, maturity, steps);
    State s = m.start(in);
    for (int t = 0; t < steps; ++t) {
      ADouble z1 = rec.randn();
      ADouble zv = rec.randn();
      s = m.step(rec, s, z1, zv);
    }
    ADouble strike = in.of(&HestonMarket::strike);
    ADouble value = type == OptionTypeEnum::CALL ? s.spot.sub(strike).max(0.0) : strike.sub(s.spot).max(0.0);
    ADouble discount = in.of(&HestonMarket::rate).neg().mul(maturity).exp();
    rec.output(value.mul(discount));
  };
}

std::function<void(AadRecorder&, Inputs<HestonMarket>&)> HestonModel::asian(OptionTypeEnum type, double maturity,
                                                                             int steps) {
  return [=](AadRecorder& rec, Inputs<HestonMarket>& in) {
    HestonModel m = HestonModel::of(in, maturity, steps);
    State s = m.start(in);
    ADouble sum = rec.constant(0.0);
    for (int t = 0; t < steps; ++t) {
      ADouble z1 = rec.randn();
      ADouble zv = rec.randn();
      s = m.step(rec, s, z1, zv);
      sum = sum.add(s.spot);
    }
    ADouble average = sum.div(static_cast<double>(steps));
    ADouble strike = in.of(&HestonMarket::strike);
    ADouble value = type == OptionTypeEnum::CALL ? average.sub(strike).max(0.0) : strike.sub(average).max(0.0);
    ADouble discount = in.of(&HestonMarket::rate).neg().mul(maturity).exp();
    rec.output(value.mul(discount));
  };
}

// ---- CorrelatedNormals (CorrelatedNormals.java:36-93) -----------------------------

CorrelatedNormals CorrelatedNormals::of(const std::vector<std::vector<double>>& corr) {
  const size_t n = corr.size();
  std::vector<std::vector<double>> l(n, std::vector<double>(n, 0.0));
  for (size_t i = 0; i < n; ++i) {
    if (corr[i].size() != n) throw std::invalid_argument("correlation matrix must be square");
    for (size_t j = 0; j <= i; ++j) {
      double sum = corr[i][j];
      for (size_t k = 0; k < j; ++k) sum -= l[i][k] * l[j][k];
      if (i == j) {
        if (sum <= 0.0) {
          throw std::invalid_argument("correlation matrix is not positive definite at index " + std::to_string(i));
        }
        l[i][j] = std::sqrt(sum);
      } else {
        l[i][j] = sum / l[j][j];
      }
    }
  }
  CorrelatedNormals c;
  c.lower_ = l;
  return c;
}

std::vector<ADouble> CorrelatedNormals::mix(AadRecorder& rec, const std::vector<ADouble>& independent) const {
  if (independent.size() != lower_.size()) throw std::invalid_argument("draw count differs from the factor size");
  std::vector<ADouble> y;
  for (size_t i = 0; i < lower_.size(); ++i) {
    ADouble acc = rec.constant(0.0);
    for (size_t j = 0; j <= i; ++j) {
      ADouble term = independent[j].mul(lower_[i][j]);
      acc = acc.add(term);
    }
    y.push_back(acc);
  }
  return y;
}

std::vector<ADouble> CorrelatedNormals::draw(AadRecorder& rec) const {
  std::vector<ADouble> z;
  for (size_t i = 0; i < lower_.size(); ++i) z.push_back(rec.randn());
  return mix(rec, z);
}

// ---- WorstOfBasket ------------------------------------------------------------------

MarketRecord WorstOfBasket::market(const std::vector<double>& spots, const std::vector<double>& vols, double rate) {
  if (spots.size() != vols.size() || spots.empty()) throw std::invalid_argument("need one vol per spot");
  std::vector<std::string> names;
  std::vector<double> values;
  for (size_t i = 0; i < spots.size(); ++i) {
    names.push_back("spot" + std::to_string(i));
    values.push_back(spots[i]);
  }
  for (size_t i = 0; i < vols.size(); ++i) {
    names.push_back("vol" + std::to_string(i));
    values.push_back(vols[i]);
  }
  names.push_back("rate");
  values.push_back(rate);
  return MarketRecord(names, values);
}

std::function<void(AadRecorder&, Inputs<MarketRecord>&)> WorstOfBasket::call(
    const std::vector<std::vector<double>>& corr, double strike, double maturity, int steps) {
  CorrelatedNormals mixer = CorrelatedNormals::of(corr);
  return [=](AadRecorder& rec, Inputs<MarketRecord>& in) {
    const int n = mixer.size();
    const TimeGrid grid = TimeGrid::uniform(steps);
    ADouble rate = in.of("rate");
    ADouble tenor = rec.constant(maturity);
    std::vector<GbmPath> models;
    std::vector<ADouble> spot;
    for (int i = 0; i < n; ++i) {
      models.push_back(GbmPath::of(rec, rate, in.of("vol" + std::to_string(i)), grid, tenor));
      spot.push_back(in.of("spot" + std::to_string(i)));
    }
    for (int t = 0; t < steps; ++t) {
      std::vector<ADouble> y = mixer.draw(rec);
      for (int i = 0; i < n; ++i) spot[i] = models[i].step(spot[i], y[i], t);
    }
    ADouble worst = spot[0];
    for (int i = 1; i < n; ++i) worst = worst.min(spot[i]);
    ADouble payoff = worst.sub(strike).max(0.0);
    ADouble discount = rate.neg().mul(tenor).exp();
    rec.output(payoff.mul(discount));
  };
}

}  // namespace nablatensor
