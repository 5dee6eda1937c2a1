// Compute-graph topology (Pattern), its order-insensitive key, the matcher
// that maps a user Pattern onto a supported one (Ops), and per-call argument
// slots (Args).
//
// Contract follows the reference:
//   PatternBuilder/Pattern/PatternKey   src/include/flash_train/pattern.hpp:83-180,
//                                       src/pattern.cpp:140-295
//   Ops/Args                            src/include/flash_train/ops_args.hpp:25-112,
//                                       src/ops_args.cpp:559-670
// The algorithms here are this library's own: the key is a colour-refinement
// invariant and the matcher is a port-driven backtracking search (see
// pattern.cpp).
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>
#include <vector>

#include "ft/values.hpp"

namespace ftrain {

struct OpNode {
    OperationKind kind;
    std::vector<uint64_t> inputs;   // operand indices in port order
    std::vector<uint64_t> outputs;  // operand indices in port order
};

// Order-insensitive structural fingerprint; equal for Patterns that differ
// only in the order operands and operations were added.
class PatternKey {
  public:
    PatternKey() = default;
    explicit PatternKey(std::vector<uint64_t> tokens);

    bool operator==(const PatternKey& o) const noexcept { return hash_ == o.hash_ && tokens_ == o.tokens_; }
    bool operator!=(const PatternKey& o) const noexcept { return !(*this == o); }
    std::size_t hash() const noexcept { return hash_; }

  private:
    std::vector<uint64_t> tokens_;
    std::size_t hash_ = 0;
};

struct PatternKeyHash {
    std::size_t operator()(const PatternKey& k) const noexcept { return k.hash(); }
};

struct PortRef {
    uint64_t op;
    uint64_t port;
};

// A validated Pattern: operand kinds, operation nodes, the derived reverse
// topology, final refinement colours and the key.  Never refers back to its
// builder.
class Pattern {
  public:
    const PatternKey& key() const noexcept { return key_; }
    std::size_t numOperands() const noexcept { return operand_kinds_.size(); }
    std::size_t numOps() const noexcept { return ops_.size(); }
    OperandKind operandKind(std::size_t i) const { return operand_kinds_.at(i); }
    const OpNode& op(std::size_t i) const { return ops_.at(i); }
    bool isIsolated(std::size_t operand) const { return !producer_[operand] && consumers_[operand].empty(); }
    uint64_t operandColor(std::size_t i) const { return operand_color_[i]; }
    uint64_t opColor(std::size_t i) const { return op_color_[i]; }

  private:
    friend class PatternBuilder;
    std::vector<OperandKind> operand_kinds_;
    std::vector<OpNode> ops_;
    std::vector<std::optional<PortRef>> producer_;
    std::vector<std::vector<PortRef>> consumers_;
    std::vector<uint64_t> operand_color_;
    std::vector<uint64_t> op_color_;
    PatternKey key_;
};

// Mutable graph under construction.  Appends never validate; build() does.
class PatternBuilder {
  public:
    uint64_t addOperand(OperandKind kind) {
        operand_kinds_.push_back(kind);
        return operand_kinds_.size() - 1;
    }
    uint64_t addOperation(OpNode node) {
        ops_.push_back(std::move(node));
        return ops_.size() - 1;
    }

    // Validates (operand ids in range; no operand repeated across an op's
    // inputs or outputs; no output that is also an input; one producer per
    // operand; no dependency cycle) and returns the Pattern.  Violations
    // throw INVALID_ARGUMENT naming the operation and port.
    Pattern build() const;

  private:
    std::vector<OperandKind> operand_kinds_;
    std::vector<OpNode> ops_;
};

class Args;

// Immutable result of matching a user Pattern to a supported one.
class Ops {
  public:
    // Throws UNSUPPORTED when the two Patterns are not isomorphic (same
    // operand kinds, same operation kinds, same port wiring; insertion order
    // ignored).
    Ops(const Pattern& user, const Pattern& supported);

    const PatternKey& key() const noexcept { return key_; }
    Args makeArgs() const;

  private:
    PatternKey key_;
    std::vector<uint64_t> operand_map_;  // user operand -> supported operand
    std::vector<uint64_t> op_map_;       // user op -> supported op
    std::vector<OperandKind> operand_kinds_;
    std::vector<OperationKind> op_kinds_;
};

// One call's concrete values, stored at supported-role slots and set
// through user-role ids.
class Args {
  public:
    const PatternKey& key() const noexcept { return key_; }
    bool isComplete() const noexcept;

    // Supported-role accessors; out-of-range ids throw INVALID_ARGUMENT.
    const std::optional<OperandValue>& operand(uint64_t supported_id) const;
    const std::optional<OperationAttributes>& operation(uint64_t supported_id) const;

    // User-role setters.  INVALID_ARGUMENT when the id is out of range or
    // names a slot of another storage family / operation kind; the Args is
    // unchanged then.
    void setOperand(uint64_t user_id, OperandValue value);
    void setOperation(uint64_t user_id, OperationAttributes attributes);

  private:
    friend class Ops;
    Args() = default;
    PatternKey key_;
    std::vector<uint64_t> operand_map_;
    std::vector<uint64_t> op_map_;
    std::vector<OperandKind> operand_kinds_;
    std::vector<OperationKind> op_kinds_;
    std::vector<std::optional<OperandValue>> operands_;
    std::vector<std::optional<OperationAttributes>> operations_;
};

}  // namespace ftrain
