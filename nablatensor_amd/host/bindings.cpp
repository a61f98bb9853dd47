// pybind11 module nablatensor_amd._host: the C++ host layer under the
// reference's own names (camelCase kept), so Python callers and tests read like
// the reference's Java: MonteCarlo.of(Products.asianCall()).market(...)
// .steps(252).greeks().fp64().on("rocm").build().run(n, seed).
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include "aad.hpp"
#include "engine.hpp"
#include "quant.hpp"

namespace py = pybind11;
using namespace nablatensor;

namespace {

template <class T>
py::array_t<T> to_array(const std::vector<T>& v) {
  py::array_t<T> a(v.size());
  std::copy(v.begin(), v.end(), a.mutable_data());
  return a;
}

py::dict flat(const AadTape& t) {
  py::dict d;
  d["op"] = to_array(t.ops());
  d["arg_a"] = to_array(t.argsA());
  d["arg_b"] = to_array(t.argsB());
  d["constant"] = to_array(t.constants());
  d["input_node"] = to_array(t.inputNodes());
  d["output_node"] = to_array(t.outputNodes());
  d["active"] = to_array(t.active());
  d["n_streams"] = t.randStreamCount();
  d["n_uniforms"] = t.randUniformCount(0);
  d["input_names"] = t.inputNames();
  d["recorded_inputs"] = t.recordedInputs();
  return d;
}

// Recorded valuations cross into Python as opaque handles.
struct HestonValuation {
  std::function<void(AadRecorder&, Inputs<HestonMarket>&)> f;
};
struct RecordValuation {
  std::function<void(AadRecorder&, Inputs<MarketRecord>&)> f;
};

template <class M>
void bind_typed(py::module_& m, const char* suffix) {
  using TV = TypedValuation<M>;
  py::class_<TV>(m, (std::string("TypedValuation") + suffix).c_str())
      .def("price", &TV::price)
      .def("standardError", &TV::standardError)
      .def("greek", py::overload_cast<const std::string&>(&TV::greek, py::const_))
      .def("gradients", [](const TV& v) { return v.result().gradients(); })
      .def("inputNames", [](const TV& v) { return v.result().inputNames(); })
      .def("scenarios", &TV::scenarios)
      .def("seconds", &TV::seconds)
      .def("kernelSeconds", [](const TV& v) { return v.result().kernelSeconds(); })
      .def("scenariosPerSecond", &TV::scenariosPerSecond)
      .def("rawSums", [](const TV& v) { return v.result().rawSums(); });
  using TP = TypedPricer<M>;
  py::class_<TP>(m, (std::string("TypedPricer") + suffix).c_str())
      .def("run", &TP::run)
      .def("engine", &TP::engine)
      .def("nodes", &TP::nodes)
      .def("recordSeconds", &TP::recordSeconds)
      .def("buildSeconds", &TP::buildSeconds)
      .def("executable", &TP::executable, py::return_value_policy::reference_internal)
      .def("close", &TP::close);
  using TM = TypedModel<M>;
  py::class_<TM>(m, (std::string("TypedModel") + suffix).c_str())
      .def("fp32", &TM::fp32, py::return_value_policy::reference_internal)
      .def("fp64", &TM::fp64, py::return_value_policy::reference_internal)
      .def("greeks", &TM::greeks, py::return_value_policy::reference_internal)
      .def("priceOnly", &TM::priceOnly, py::return_value_policy::reference_internal)
      .def("threads", &TM::threads, py::return_value_policy::reference_internal)
      .def("on", &TM::on, py::return_value_policy::reference_internal)
      .def("fastest", &TM::fastest, py::return_value_policy::reference_internal)
      .def("tune", &TM::tune, py::return_value_policy::reference_internal)
      .def("tape", &TM::tape)
      .def("build", &TM::build);
}

}  // namespace

PYBIND11_MODULE(_host, m) {
  m.doc() = "nablatensor_amd host layer: recording, products, engine SPI and the rocm engine";

  py::enum_<AadOpEnum>(m, "AadOpEnum")
      .value("CONST", AadOpEnum::CONST).value("INPUT", AadOpEnum::INPUT).value("RANDN", AadOpEnum::RANDN)
      .value("RANDU", AadOpEnum::RANDU).value("ADD", AadOpEnum::ADD).value("SUB", AadOpEnum::SUB)
      .value("MUL", AadOpEnum::MUL).value("DIV", AadOpEnum::DIV).value("NEG", AadOpEnum::NEG)
      .value("EXP", AadOpEnum::EXP).value("LOG", AadOpEnum::LOG).value("SQRT", AadOpEnum::SQRT)
      .value("MAX", AadOpEnum::MAX).value("MIN", AadOpEnum::MIN).value("ABS", AadOpEnum::ABS);

  py::class_<AadTape, std::shared_ptr<AadTape>>(m, "AadTape")
      .def("size", &AadTape::size)
      .def("op", &AadTape::op)
      .def("argA", &AadTape::argA)
      .def("argB", &AadTape::argB)
      .def("constant", &AadTape::constant)
      .def("isActive", &AadTape::isActive)
      .def("inputCount", &AadTape::inputCount)
      .def("inputNode", &AadTape::inputNode)
      .def("inputNames", &AadTape::inputNames)
      .def("recordedInputs", &AadTape::recordedInputs)
      .def("randCount", &AadTape::randCount)
      .def("randStreamCount", &AadTape::randStreamCount)
      .def("randUniformCount", &AadTape::randUniformCount)
      .def("hasExtendedRandom", &AadTape::hasExtendedRandom)
      .def("outputCount", &AadTape::outputCount)
      .def("outputNode", py::overload_cast<>(&AadTape::outputNode, py::const_))
      .def("outputNames", &AadTape::outputNames)
      .def("flat", &flat)
      .def("__repr__", &AadTape::toString);

  py::class_<ADouble>(m, "ADouble")
      .def("add", py::overload_cast<const ADouble&>(&ADouble::add, py::const_))
      .def("add", py::overload_cast<double>(&ADouble::add, py::const_))
      .def("sub", py::overload_cast<const ADouble&>(&ADouble::sub, py::const_))
      .def("sub", py::overload_cast<double>(&ADouble::sub, py::const_))
      .def("mul", py::overload_cast<const ADouble&>(&ADouble::mul, py::const_))
      .def("mul", py::overload_cast<double>(&ADouble::mul, py::const_))
      .def("div", py::overload_cast<const ADouble&>(&ADouble::div, py::const_))
      .def("div", py::overload_cast<double>(&ADouble::div, py::const_))
      .def("max", py::overload_cast<const ADouble&>(&ADouble::max, py::const_))
      .def("max", py::overload_cast<double>(&ADouble::max, py::const_))
      .def("min", py::overload_cast<const ADouble&>(&ADouble::min, py::const_))
      .def("min", py::overload_cast<double>(&ADouble::min, py::const_))
      .def("neg", &ADouble::neg)
      .def("exp", &ADouble::exp)
      .def("log", &ADouble::log)
      .def("sqrt", &ADouble::sqrt)
      .def("abs", &ADouble::abs)
      .def("node", &ADouble::node);

  py::class_<AadRecorder::RandomStream>(m, "RandomStream")
      .def("randn", &AadRecorder::RandomStream::randn)
      .def("randu", &AadRecorder::RandomStream::randu);

  py::class_<AadRecorder, std::unique_ptr<AadRecorder, py::nodelete>>(m, "AadRecorder")
      .def_static("record",
                  [](py::function body) {
                    return std::const_pointer_cast<AadTape>(
                        AadRecorder::record([&](AadRecorder& r) { body(py::cast(&r, py::return_value_policy::reference)); }));
                  })
      .def("input", &AadRecorder::input)
      .def("constant", &AadRecorder::constant)
      .def("randn", &AadRecorder::randn)
      .def("randu", &AadRecorder::randu)
      .def("stream", &AadRecorder::stream)
      .def("output", py::overload_cast<const ADouble&>(&AadRecorder::output))
      .def("output", py::overload_cast<const std::string&, const ADouble&>(&AadRecorder::output));

  py::enum_<OptionTypeEnum>(m, "OptionTypeEnum").value("CALL", OptionTypeEnum::CALL).value("PUT", OptionTypeEnum::PUT);

  py::class_<TimeGrid>(m, "TimeGrid")
      .def_static("uniform", &TimeGrid::uniform)
      .def_static("of", &TimeGrid::of)
      .def("steps", &TimeGrid::steps)
      .def("fraction", &TimeGrid::fraction)
      .def("cumulative", &TimeGrid::cumulative)
      .def("isUniform", &TimeGrid::isUniform);

  py::class_<MarketRecord>(m, "MarketRecord")
      .def(py::init<std::vector<std::string>, std::vector<double>>())
      .def("names", &MarketRecord::names)
      .def("values", &MarketRecord::values)
      .def("get", &MarketRecord::get);

  py::class_<EquityMarket, MarketRecord>(m, "EquityMarket")
      .def(py::init<const std::vector<double>&>())
      .def_static("create", [](double spot, double strike, double vol, double rate, double maturity) {
        return EquityMarket::of().spot(spot).strike(strike).vol(vol).rate(rate).maturity(maturity).build();
      }, py::arg("spot"), py::arg("strike"), py::arg("vol"), py::arg("rate"), py::arg("maturity"))
      .def_static("atmOneYear", &EquityMarket::atmOneYear)
      .def("spot", &EquityMarket::spot)
      .def("strike", &EquityMarket::strike)
      .def("vol", &EquityMarket::vol)
      .def("rate", &EquityMarket::rate)
      .def("maturity", &EquityMarket::maturity)
      .def("validated", &EquityMarket::validated)
      .def("withSpot", &EquityMarket::withSpot)
      .def("withStrike", &EquityMarket::withStrike)
      .def("withVol", &EquityMarket::withVol)
      .def("withRate", &EquityMarket::withRate)
      .def("withMaturity", &EquityMarket::withMaturity);

  py::class_<HestonMarket, MarketRecord>(m, "HestonMarket")
      .def(py::init<const std::vector<double>&>())
      .def_static("create", [](double spot, double strike, double rate, double v0, double kappa, double theta,
                               double xi, double rho) {
        return HestonMarket::of().spot(spot).strike(strike).rate(rate).v0(v0).kappa(kappa).theta(theta).xi(xi)
            .rho(rho).build();
      }, py::arg("spot"), py::arg("strike"), py::arg("rate"), py::arg("v0"), py::arg("kappa"), py::arg("theta"),
         py::arg("xi"), py::arg("rho"))
      .def("spot", &HestonMarket::spot)
      .def("strike", &HestonMarket::strike)
      .def("rate", &HestonMarket::rate)
      .def("v0", &HestonMarket::v0)
      .def("kappa", &HestonMarket::kappa)
      .def("theta", &HestonMarket::theta)
      .def("xi", &HestonMarket::xi)
      .def("rho", &HestonMarket::rho)
      .def("validated", &HestonMarket::validated);

  py::class_<Product<EquityMarket>>(m, "Product")
      .def_readonly("label", &Product<EquityMarket>::label)
      .def("__repr__", [](const Product<EquityMarket>& p) { return p.label; });

  py::class_<Products>(m, "Products")
      .def_static("european", &Products::european)
      .def_static("asian", &Products::asian)
      .def_static("lookback", &Products::lookback)
      .def_static("europeanCall", &Products::europeanCall)
      .def_static("europeanPut", &Products::europeanPut)
      .def_static("asianCall", &Products::asianCall)
      .def_static("asianPut", &Products::asianPut)
      .def_static("lookbackCall", &Products::lookbackCall)
      .def_static("lookbackPut", &Products::lookbackPut);

  py::class_<ExoticProducts> exotic(m, "ExoticProducts");
  py::enum_<ExoticProducts::BarrierEnum>(exotic, "BarrierEnum")
      .value("UP_OUT", ExoticProducts::BarrierEnum::UP_OUT).value("UP_IN", ExoticProducts::BarrierEnum::UP_IN)
      .value("DOWN_OUT", ExoticProducts::BarrierEnum::DOWN_OUT).value("DOWN_IN", ExoticProducts::BarrierEnum::DOWN_IN);
  exotic.def_static("barrier", &ExoticProducts::barrier, py::arg("type"), py::arg("kind"), py::arg("barrier"),
                    py::arg("width"))
      .def_static("digitalCash", &ExoticProducts::digitalCash, py::arg("type"), py::arg("cash"), py::arg("width"));

  py::class_<HestonValuation>(m, "HestonValuation");
  py::class_<RecordValuation>(m, "RecordValuation");
  py::class_<HestonModel>(m, "HestonModel")
      .def_static("european", [](OptionTypeEnum t, double maturity, int steps) {
        return HestonValuation{HestonModel::european(t, maturity, steps)};
      })
      .def_static("asian", [](OptionTypeEnum t, double maturity, int steps) {
        return HestonValuation{HestonModel::asian(t, maturity, steps)};
      });

  py::class_<CorrelatedNormals>(m, "CorrelatedNormals")
      .def_static("of", &CorrelatedNormals::of)
      .def("size", &CorrelatedNormals::size)
      .def("lower", &CorrelatedNormals::lower);

  py::class_<WorstOfBasket>(m, "WorstOfBasket")
      .def_static("market", &WorstOfBasket::market)
      .def_static("call", [](const std::vector<std::vector<double>>& corr, double strike, double maturity, int steps) {
        return RecordValuation{WorstOfBasket::call(corr, strike, maturity, steps)};
      }, py::arg("corr"), py::arg("strike"), py::arg("maturity"), py::arg("steps"));

  // Record a product / valuation against a market into a tape (Nabla.model's recording step).
  m.def("record", [](const Product<EquityMarket>& p, const EquityMarket& market, const TimeGrid& grid) {
    return std::const_pointer_cast<AadTape>(
        Nabla::model<EquityMarket>(market, [&](AadRecorder& rec, Inputs<EquityMarket>& in) { p.record(rec, in, grid); })
            .tape());
  });
  m.def("record", [](const HestonValuation& v, const HestonMarket& market) {
    return std::const_pointer_cast<AadTape>(Nabla::model<HestonMarket>(market, v.f).tape());
  });
  m.def("record", [](const RecordValuation& v, const MarketRecord& market) {
    return std::const_pointer_cast<AadTape>(Nabla::model<MarketRecord>(market, v.f).tape());
  });

  // ---- engine layer ----
  py::class_<AadOptions> opts(m, "AadOptions");
  py::enum_<AadOptions::PrecisionEnum>(opts, "PrecisionEnum")
      .value("FLOAT32", AadOptions::PrecisionEnum::FLOAT32)
      .value("FLOAT64", AadOptions::PrecisionEnum::FLOAT64);
  opts.def_static("defaults", &AadOptions::defaults)
      .def("precision", &AadOptions::precision)
      .def("adjoints", &AadOptions::adjoints)
      .def("threads", &AadOptions::threads)
      .def("withPrecision", &AadOptions::withPrecision)
      .def("withAdjoints", &AadOptions::withAdjoints)
      .def("withThreads", &AadOptions::withThreads)
      .def("withEngineOption", &AadOptions::withEngineOption)
      .def("engineOptions", &AadOptions::engineOptions);

  py::class_<AadResult>(m, "AadResult")
      .def("value", py::overload_cast<>(&AadResult::value, py::const_))
      .def("standardError", py::overload_cast<>(&AadResult::standardError, py::const_))
      .def("gradients", py::overload_cast<>(&AadResult::gradients, py::const_))
      .def("gradients", py::overload_cast<const std::string&>(&AadResult::gradients, py::const_))
      .def("gradient", py::overload_cast<const std::string&>(&AadResult::gradient, py::const_))
      .def("gradient", py::overload_cast<const std::string&, const std::string&>(&AadResult::gradient, py::const_))
      .def("outputNames", &AadResult::outputNames)
      .def("outputCount", &AadResult::outputCount)
      .def("valueOf", py::overload_cast<const std::string&>(&AadResult::value, py::const_))
      .def("standardErrorOf", py::overload_cast<const std::string&>(&AadResult::standardError, py::const_))
      .def("inputNames", &AadResult::inputNames)
      .def("paths", &AadResult::paths)
      .def("seconds", &AadResult::seconds)
      .def("kernelSeconds", &AadResult::kernelSeconds)
      .def("pathsPerSecond", &AadResult::pathsPerSecond)
      .def("rawSums", &AadResult::rawSums)
      .def("__repr__", &AadResult::toString);

  py::class_<AadExecutable>(m, "AadExecutable")
      .def("engineName", &AadExecutable::engineName)
      .def("tape", &AadExecutable::tapePtr)
      .def("setInput", &AadExecutable::setInput)
      .def("replay", &AadExecutable::replay, py::arg("paths"), py::arg("pathOffset"), py::arg("seed"),
           py::call_guard<py::gil_scoped_release>())
      .def("replayMany", &AadExecutable::replayMany, py::arg("inputSets"), py::arg("paths"), py::arg("pathOffset"),
           py::arg("seed"), py::call_guard<py::gil_scoped_release>())
      .def("replaySafe", &AadExecutable::replaySafe, py::call_guard<py::gil_scoped_release>())
      .def("calibrate", &AadExecutable::calibrate, py::call_guard<py::gil_scoped_release>())
      .def("measuredPathsPerSecond", &AadExecutable::measuredPathsPerSecond)
      .def("maxChunkSeconds", &AadExecutable::maxChunkSeconds)
      .def("setMaxChunkSeconds", &AadExecutable::setMaxChunkSeconds)
      .def("compileSeconds", &AadExecutable::compileSeconds)
      .def("info", [](const AadExecutable& e) { return rocmExecutableInfo(e); })
      .def("source", [](const AadExecutable& e) { return rocmExecutableSource(e); })
      .def("close", &AadExecutable::close);

  py::class_<AadEngine, std::shared_ptr<AadEngine>>(m, "AadEngine")
      .def("name", &AadEngine::name)
      .def("priority", &AadEngine::priority)
      .def("isAvailable", &AadEngine::isAvailable)
      .def("supports", &AadEngine::supports)
      .def("describe", &AadEngine::describe)
      .def("compile", [](const AadEngine& e, std::shared_ptr<AadTape> t, const AadOptions& o) {
        return e.compile(t, o);
      });
  py::class_<RocmAadEngine, AadEngine, std::shared_ptr<RocmAadEngine>>(m, "RocmAadEngine")
      .def(py::init<>())
      .def_static("maxLaunchSeconds", &RocmAadEngine::maxLaunchSeconds);

  py::class_<AadEngines>(m, "AadEngines")
      .def_static("discovered", &AadEngines::discovered)
      .def_static("available", &AadEngines::available)
      .def_static("find", &AadEngines::find)
      .def_static("require", &AadEngines::require)
      .def_static("select", &AadEngines::select);

  py::register_exception<UnsupportedOperation>(m, "UnsupportedOperationException", PyExc_NotImplementedError);

  bind_typed<EquityMarket>(m, "Equity");
  bind_typed<HestonMarket>(m, "Heston");
  bind_typed<MarketRecord>(m, "Record");

  using MC = MonteCarlo<EquityMarket>;
  py::class_<MC::Builder>(m, "MonteCarloBuilder")
      .def("market", &MC::Builder::market, py::return_value_policy::reference_internal)
      .def("steps", &MC::Builder::steps, py::return_value_policy::reference_internal)
      .def("timeGrid", &MC::Builder::timeGrid, py::return_value_policy::reference_internal)
      .def("greeks", &MC::Builder::greeks, py::return_value_policy::reference_internal)
      .def("priceOnly", &MC::Builder::priceOnly, py::return_value_policy::reference_internal)
      .def("fp32", &MC::Builder::fp32, py::return_value_policy::reference_internal)
      .def("fp64", &MC::Builder::fp64, py::return_value_policy::reference_internal)
      .def("threads", &MC::Builder::threads, py::return_value_policy::reference_internal)
      .def("on", &MC::Builder::on, py::return_value_policy::reference_internal)
      .def("fastest", &MC::Builder::fastest, py::return_value_policy::reference_internal)
      .def("tune", &MC::Builder::tune, py::return_value_policy::reference_internal)
      .def("build", &MC::Builder::build);
  py::class_<MC>(m, "MonteCarlo")
      .def_static("of", &MC::of)
      .def("market", &MC::market)
      .def("hasGreeks", &MC::hasGreeks)
      .def("engine", &MC::engine)
      .def("nodes", &MC::nodes)
      .def("recordSeconds", &MC::recordSeconds)
      .def("buildSeconds", &MC::buildSeconds)
      .def("tape", [](const MC& mc) { return std::const_pointer_cast<AadTape>(mc.tape()); })
      .def("executable", &MC::executable, py::return_value_policy::reference_internal)
      .def("run", py::overload_cast<long long, long long>(&MC::run), py::call_guard<py::gil_scoped_release>())
      .def("run", py::overload_cast<const EquityMarket&, long long, long long>(&MC::run),
           py::call_guard<py::gil_scoped_release>())
      .def("close", &MC::close);

  m.def("modelHeston", [](const HestonMarket& market, const HestonValuation& v) { return Nabla::model<HestonMarket>(market, v.f); });
  m.def("modelRecord", [](const MarketRecord& market, const RecordValuation& v) { return Nabla::model<MarketRecord>(market, v.f); });
  m.def("modelEquity", [](const EquityMarket& market, const Product<EquityMarket>& p, const TimeGrid& grid) {
    return Nabla::model<EquityMarket>(market, [p, grid](AadRecorder& rec, Inputs<EquityMarket>& in) { p.record(rec, in, grid); });
  });
}
