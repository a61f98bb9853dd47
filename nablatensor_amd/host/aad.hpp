// Tape recording: the host half of the fused forward+adjoint replay path.
//
// Mirrors the reference's recording API so a valuation written against it
// records the same nodes in the same order:
//   AadOpEnum   nablatensor-core/src/main/java/com/nablatensor/engine/AadOpEnum.java:19-50
//   AadTape     nablatensor-core/src/main/java/com/nablatensor/engine/AadTape.java:30-329
//   AadRecorder nablatensor-core/src/main/java/com/nablatensor/engine/AadRecorder.java:34-123
//   ADouble     nablatensor-core/src/main/java/com/nablatensor/engine/ADouble.java:23-111
// A node-creating C++ expression with two node-creating operands must be split
// into statements: C++ leaves argument evaluation order unspecified, Java fixes
// it left to right, and the tape order is part of the result (draw ordinals).
#pragma once

#include <cstdint>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace nablatensor {

enum class AadOpEnum : int32_t {
  CONST = 0, INPUT, RANDN, RANDU, ADD, SUB, MUL, DIV, NEG, EXP, LOG, SQRT, MAX, MIN, ABS
};

const char* op_name(AadOpEnum op);

class AadRecorder;

// A recorded scalar computation graph in evaluation order (AadTape.java:30-48).
class AadTape {
 public:
  int size() const { return static_cast<int>(op_.size()); }
  AadOpEnum op(int node) const { return static_cast<AadOpEnum>(op_.at(node)); }
  int argA(int node) const { return arg_a_.at(node); }
  int argB(int node) const { return arg_b_.at(node); }
  double constant(int node) const { return constant_.at(node); }
  bool isActive(int node) const { return active_.at(node) != 0; }
  int inputCount() const { return static_cast<int>(input_node_.size()); }
  int inputNode(int index) const { return input_node_.at(index); }
  const std::string& inputName(int index) const { return input_name_.at(index); }
  const std::vector<std::string>& inputNames() const { return input_name_; }
  int inputIndex(const std::string& name) const;  // -1 when absent
  std::vector<double> recordedInputs() const { return recorded_input_; }
  int randCount() const { return rand_normal_.at(0); }
  int randStreamCount() const { return static_cast<int>(rand_stream_name_.size()); }
  const std::string& randStreamName(int s) const { return rand_stream_name_.at(s); }
  int randNormalCount(int s) const { return rand_normal_.at(s); }
  int randUniformCount(int s) const { return rand_uniform_.at(s); }
  bool hasExtendedRandom() const;  // AadTape.java:190-196
  int outputNode() const { return output_node_.at(0); }
  int outputCount() const { return static_cast<int>(output_node_.size()); }
  int outputNode(int i) const { return output_node_.at(i); }
  const std::string& outputName(int i) const { return output_name_.at(i); }
  const std::vector<std::string>& outputNames() const { return output_name_; }
  std::string toString() const;

  // Flat views (FlatTape.java:37-79): the arrays the C-ABI takes.
  const std::vector<int32_t>& ops() const { return op_; }
  const std::vector<int32_t>& argsA() const { return arg_a_; }
  const std::vector<int32_t>& argsB() const { return arg_b_; }
  const std::vector<double>& constants() const { return constant_; }
  const std::vector<int32_t>& inputNodes() const { return input_node_; }
  const std::vector<int32_t>& outputNodes() const { return output_node_; }
  const std::vector<uint8_t>& active() const { return active_; }

 private:
  friend class AadRecorder;
  void markActive();  // AadTape.java:70-81

  std::vector<int32_t> op_, arg_a_, arg_b_;
  std::vector<double> constant_;
  std::vector<int32_t> input_node_;
  std::vector<std::string> input_name_;
  std::vector<double> recorded_input_;
  std::vector<std::string> rand_stream_name_{"default"};
  std::vector<int32_t> rand_normal_{0};
  std::vector<int32_t> rand_uniform_{0};
  std::vector<int32_t> output_node_;
  std::vector<std::string> output_name_;
  std::vector<uint8_t> active_;
};

using TapePtr = std::shared_ptr<const AadTape>;

// An active scalar: every operation appends one node (ADouble.java:23-111).
class ADouble {
 public:
  ADouble() = default;
  ADouble add(const ADouble& o) const;
  ADouble sub(const ADouble& o) const;
  ADouble mul(const ADouble& o) const;
  ADouble div(const ADouble& o) const;
  ADouble add(double v) const;  // CONST node, then ADD (ADouble.java:60-62)
  ADouble sub(double v) const;
  ADouble mul(double v) const;
  ADouble div(double v) const;
  ADouble neg() const;
  ADouble exp() const;
  ADouble log() const;
  ADouble sqrt() const;
  ADouble abs() const;
  ADouble max(const ADouble& o) const;
  ADouble min(const ADouble& o) const;
  ADouble max(double v) const;
  ADouble min(double v) const;
  int node() const { return node_; }
  AadRecorder* recorder() const { return rec_; }

 private:
  friend class AadRecorder;
  ADouble(AadRecorder* rec, int node) : rec_(rec), node_(node) {}
  ADouble binary(AadOpEnum op, const ADouble& o) const;
  ADouble unary(AadOpEnum op) const;
  AadRecorder* rec_ = nullptr;
  int node_ = -1;
};

// Records one pass of a valuation (AadRecorder.java:34-123).
class AadRecorder {
 public:
  class RandomStream {
   public:
    ADouble randn();
    ADouble randu();
   private:
    friend class AadRecorder;
    RandomStream(AadRecorder* rec, std::string name) : rec_(rec), name_(std::move(name)) {}
    AadRecorder* rec_;
    std::string name_;
  };

  static TapePtr record(const std::function<void(AadRecorder&)>& body);

  ADouble input(const std::string& name, double value);
  ADouble constant(double value);
  ADouble randn();
  ADouble randu();
  RandomStream stream(const std::string& name);
  void output(const ADouble& value);
  void output(const std::string& name, const ADouble& value);

  ADouble node(AadOpEnum op, int a, int b);

 private:
  AadRecorder() : tape_(std::make_shared<AadTape>()) {}
  int add(AadOpEnum op, int a, int b, double value);
  int streamIndex(const std::string& name);
  int addRandn(const std::string& stream);
  int addRandu(const std::string& stream);
  std::shared_ptr<AadTape> tape_;
};

}  // namespace nablatensor
