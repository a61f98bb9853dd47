// Tape recording; see aad.hpp for the reference each class follows.
#include "aad.hpp"

#include <sstream>

namespace nablatensor {

const char* op_name(AadOpEnum op) {
  static const char* names[] = {"CONST", "INPUT", "RANDN", "RANDU", "ADD", "SUB", "MUL", "DIV",
                                "NEG",   "EXP",   "LOG",   "SQRT",  "MAX", "MIN", "ABS"};
  int i = static_cast<int>(op);
  return (i >= 0 && i < 15) ? names[i] : "?";
}

int AadTape::inputIndex(const std::string& name) const {
  for (size_t i = 0; i < input_name_.size(); ++i) {
    if (input_name_[i] == name) return static_cast<int>(i);
  }
  return -1;
}

bool AadTape::hasExtendedRandom() const {
  return rand_stream_name_.size() > 1 || rand_uniform_.at(0) > 0;
}

std::string AadTape::toString() const {
  std::ostringstream s;
  s << "AadTape(nodes=" << size() << ", inputs=[";
  for (size_t i = 0; i < input_name_.size(); ++i) s << (i ? ", " : "") << input_name_[i];
  s << "], randoms=" << randCount() << ")";
  return s.str();
}

// Active = depends on at least one INPUT (AadTape.java:70-81).
void AadTape::markActive() {
  const int n = size();
  active_.assign(n, 0);
  for (int i = 0; i < n; ++i) {
    switch (op(i)) {
      case AadOpEnum::INPUT: active_[i] = 1; break;
      case AadOpEnum::CONST:
      case AadOpEnum::RANDN:
      case AadOpEnum::RANDU: active_[i] = 0; break;
      case AadOpEnum::NEG:
      case AadOpEnum::EXP:
      case AadOpEnum::LOG:
      case AadOpEnum::SQRT:
      case AadOpEnum::ABS: active_[i] = active_[arg_a_[i]]; break;
      default: active_[i] = static_cast<uint8_t>(active_[arg_a_[i]] || active_[arg_b_[i]]); break;
    }
  }
}

// ---- ADouble ----------------------------------------------------------------

ADouble ADouble::binary(AadOpEnum op, const ADouble& o) const {
  if (o.rec_ != rec_) throw std::invalid_argument("operands come from different recordings");
  return rec_->node(op, node_, o.node_);
}
ADouble ADouble::unary(AadOpEnum op) const { return rec_->node(op, node_, -1); }

ADouble ADouble::add(const ADouble& o) const { return binary(AadOpEnum::ADD, o); }
ADouble ADouble::sub(const ADouble& o) const { return binary(AadOpEnum::SUB, o); }
ADouble ADouble::mul(const ADouble& o) const { return binary(AadOpEnum::MUL, o); }
ADouble ADouble::div(const ADouble& o) const { return binary(AadOpEnum::DIV, o); }
ADouble ADouble::add(double v) const { ADouble c = rec_->constant(v); return add(c); }
ADouble ADouble::sub(double v) const { ADouble c = rec_->constant(v); return sub(c); }
ADouble ADouble::mul(double v) const { ADouble c = rec_->constant(v); return mul(c); }
ADouble ADouble::div(double v) const { ADouble c = rec_->constant(v); return div(c); }
ADouble ADouble::neg() const { return unary(AadOpEnum::NEG); }
ADouble ADouble::exp() const { return unary(AadOpEnum::EXP); }
ADouble ADouble::log() const { return unary(AadOpEnum::LOG); }
ADouble ADouble::sqrt() const { return unary(AadOpEnum::SQRT); }
ADouble ADouble::abs() const { return unary(AadOpEnum::ABS); }
ADouble ADouble::max(const ADouble& o) const { return binary(AadOpEnum::MAX, o); }
ADouble ADouble::min(const ADouble& o) const { return binary(AadOpEnum::MIN, o); }
ADouble ADouble::max(double v) const { ADouble c = rec_->constant(v); return max(c); }
ADouble ADouble::min(double v) const { ADouble c = rec_->constant(v); return min(c); }

// ---- AadRecorder ------------------------------------------------------------

TapePtr AadRecorder::record(const std::function<void(AadRecorder&)>& body) {
  AadRecorder rec;
  body(rec);
  if (rec.tape_->output_node_.empty()) throw std::logic_error("no output was recorded");
  rec.tape_->markActive();
  return rec.tape_;
}

int AadRecorder::add(AadOpEnum op, int a, int b, double value) {
  AadTape& t = *tape_;
  t.op_.push_back(static_cast<int32_t>(op));
  t.arg_a_.push_back(a);
  t.arg_b_.push_back(b);
  t.constant_.push_back(value);
  return t.size() - 1;
}

ADouble AadRecorder::node(AadOpEnum op, int a, int b) { return ADouble(this, add(op, a, b, 0.0)); }

ADouble AadRecorder::input(const std::string& name, double value) {
  AadTape& t = *tape_;
  int node = add(AadOpEnum::INPUT, static_cast<int>(t.input_node_.size()), -1, value);
  t.input_node_.push_back(node);
  t.input_name_.push_back(name);
  t.recorded_input_.push_back(value);
  return ADouble(this, node);
}

ADouble AadRecorder::constant(double value) { return ADouble(this, add(AadOpEnum::CONST, -1, -1, value)); }

int AadRecorder::streamIndex(const std::string& name) {
  AadTape& t = *tape_;
  for (size_t i = 0; i < t.rand_stream_name_.size(); ++i) {
    if (t.rand_stream_name_[i] == name) return static_cast<int>(i);
  }
  t.rand_stream_name_.push_back(name);
  t.rand_normal_.push_back(0);
  t.rand_uniform_.push_back(0);
  return static_cast<int>(t.rand_stream_name_.size()) - 1;
}

// RANDN: argA = ordinal within (stream, normal), argB = stream (AadTape.java:281-289).
int AadRecorder::addRandn(const std::string& stream) {
  int si = streamIndex(stream);
  return add(AadOpEnum::RANDN, tape_->rand_normal_[si]++, si, 0.0);
}

int AadRecorder::addRandu(const std::string& stream) {
  int si = streamIndex(stream);
  return add(AadOpEnum::RANDU, tape_->rand_uniform_[si]++, si, 0.0);
}

ADouble AadRecorder::randn() { return ADouble(this, addRandn("default")); }
ADouble AadRecorder::randu() { return ADouble(this, addRandu("default")); }

AadRecorder::RandomStream AadRecorder::stream(const std::string& name) {
  if (name.find_first_not_of(" \t\n") == std::string::npos) {
    throw std::invalid_argument("stream name must be non-blank");
  }
  return RandomStream(this, name);
}

ADouble AadRecorder::RandomStream::randn() { return ADouble(rec_, rec_->addRandn(name_)); }
ADouble AadRecorder::RandomStream::randu() { return ADouble(rec_, rec_->addRandu(name_)); }

void AadRecorder::output(const ADouble& value) { output("value", value); }

void AadRecorder::output(const std::string& name, const ADouble& value) {
  AadTape& t = *tape_;
  for (const auto& n : t.output_name_) {
    if (n == name) throw std::invalid_argument("output '" + name + "' recorded twice");
  }
  t.output_name_.push_back(name);
  t.output_node_.push_back(value.node());
}

}  // namespace nablatensor
