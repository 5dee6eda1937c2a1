// Pattern validation, colour-refinement key, matcher, Ops and Args.
//
// Validation order and messages follow the reference's
// PatternBuilder::buildPattern (src/pattern.cpp:140-245).  The key is the
// sorted multiset of stable colours from 1-dimensional Weisfeiler-Leman
// refinement over the operand/operation bipartite graph (a textbook graph
// invariant); the matcher is an exact backtracking search over operation
// pairings that derives operand pairings from port positions.
#include "ft/pattern.hpp"

#include <algorithm>
#include <unordered_set>

#include "ft/error.hpp"

namespace ftrain {

namespace {

// splitmix64 finaliser: a well-distributed 64-bit mixer.
inline uint64_t mix64(uint64_t x) noexcept {
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

inline void absorb(uint64_t& h, uint64_t v) noexcept { h = mix64(h ^ mix64(v)); }

std::size_t countClasses(const std::vector<uint64_t>& a, const std::vector<uint64_t>& b) {
    std::vector<uint64_t> all(a);
    all.insert(all.end(), b.begin(), b.end());
    std::sort(all.begin(), all.end());
    return static_cast<std::size_t>(std::unique(all.begin(), all.end()) - all.begin());
}

}  // namespace

PatternKey::PatternKey(std::vector<uint64_t> tokens) : tokens_(std::move(tokens)) {
    uint64_t h = 0x6A09E667F3BCC908ULL;
    for (uint64_t t : tokens_) absorb(h, t);
    hash_ = static_cast<std::size_t>(h);
}

Pattern PatternBuilder::build() const {
    const std::size_t n_operands = operand_kinds_.size();
    Pattern p;
    p.operand_kinds_ = operand_kinds_;
    p.ops_           = ops_;
    p.producer_.assign(n_operands, std::nullopt);
    p.consumers_.assign(n_operands, {});

    for (std::size_t o = 0; o < ops_.size(); ++o) {
        const OpNode& node = ops_[o];
        for (std::size_t port = 0; port < node.inputs.size(); ++port) {
            const uint64_t id = node.inputs[port];
            if (id >= n_operands)
                raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                                "Operation %zu input port %zu references out-of-range operand %llu for %zu operands", o,
                                port, static_cast<unsigned long long>(id), n_operands);
            for (std::size_t q = 0; q < port; ++q)
                if (node.inputs[q] == id)
                    raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                                    "Operation %zu repeats operand %llu across input ports", o,
                                    static_cast<unsigned long long>(id));
            p.consumers_[id].push_back(PortRef{o, port});
        }
        for (std::size_t port = 0; port < node.outputs.size(); ++port) {
            const uint64_t id = node.outputs[port];
            if (id >= n_operands)
                raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                                "Operation %zu output port %zu references out-of-range operand %llu for %zu operands",
                                o, port, static_cast<unsigned long long>(id), n_operands);
            if (std::find(node.inputs.begin(), node.inputs.end(), id) != node.inputs.end())
                raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                                "Operation %zu output port %zu reuses operand %llu from an input port", o, port,
                                static_cast<unsigned long long>(id));
            for (std::size_t q = 0; q < port; ++q)
                if (node.outputs[q] == id)
                    raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                                    "Operation %zu repeats operand %llu across output ports", o,
                                    static_cast<unsigned long long>(id));
            if (p.producer_[id])
                raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                                "Operation %zu output port %zu reuses operand %llu that already has a producer", o,
                                port, static_cast<unsigned long long>(id));
            p.producer_[id] = PortRef{o, port};
        }
    }

    // Dependency cycles: op X precedes op Y when Y consumes an operand X
    // produces.  Peel ops with no unresolved predecessor (Kahn); anything
    // left over lies on or behind a cycle.
    const std::size_t n_ops = ops_.size();
    std::vector<std::vector<std::size_t>> successors(n_ops);
    std::vector<std::size_t> indegree(n_ops, 0);
    for (std::size_t id = 0; id < n_operands; ++id) {
        if (!p.producer_[id]) continue;
        for (const PortRef& c : p.consumers_[id]) {
            successors[p.producer_[id]->op].push_back(c.op);
            ++indegree[c.op];
        }
    }
    std::vector<std::size_t> ready;
    for (std::size_t o = 0; o < n_ops; ++o)
        if (indegree[o] == 0) ready.push_back(o);
    std::size_t peeled = 0;
    while (!ready.empty()) {
        const std::size_t o = ready.back();
        ready.pop_back();
        ++peeled;
        for (std::size_t s : successors[o])
            if (--indegree[s] == 0) ready.push_back(s);
    }
    if (peeled != n_ops) {
        for (std::size_t o = 0; o < n_ops; ++o) {
            if (indegree[o] == 0) continue;
            for (uint64_t in : ops_[o].inputs) {
                const auto& prod = p.producer_[in];
                if (prod && indegree[prod->op] != 0)
                    raise(FTRAIN_STATUS_INVALID_ARGUMENT,
                                    "Operation %zu input port participates in a dependency cycle through operand %llu",
                                    o, static_cast<unsigned long long>(in));
            }
        }
        raise(FTRAIN_STATUS_INTERNAL_ERROR, "cycle check peeled %zu of %zu operations but found no edge",
                        peeled, n_ops);
    }

    // Colour refinement until the number of colour classes stops growing.
    std::vector<uint64_t> oc(n_operands), pc(n_ops);
    for (std::size_t i = 0; i < n_operands; ++i) oc[i] = mix64(0x100 + static_cast<uint64_t>(operand_kinds_[i]));
    for (std::size_t i = 0; i < n_ops; ++i) pc[i] = mix64(0x200 + static_cast<uint64_t>(ops_[i].kind));
    std::size_t classes = countClasses(oc, pc);
    for (std::size_t round = 0; round <= n_operands + n_ops; ++round) {
        std::vector<uint64_t> noc(n_operands), npc(n_ops);
        for (std::size_t i = 0; i < n_operands; ++i) {
            uint64_t h = oc[i];
            absorb(h, p.producer_[i] ? 1 : 0);
            if (p.producer_[i]) {
                absorb(h, p.producer_[i]->port);
                absorb(h, pc[p.producer_[i]->op]);
            }
            std::vector<std::pair<uint64_t, uint64_t>> cons;
            for (const PortRef& c : p.consumers_[i]) cons.emplace_back(c.port, pc[c.op]);
            std::sort(cons.begin(), cons.end());
            absorb(h, cons.size());
            for (const auto& c : cons) {
                absorb(h, c.first);
                absorb(h, c.second);
            }
            noc[i] = h;
        }
        for (std::size_t i = 0; i < n_ops; ++i) {
            uint64_t h = pc[i];
            absorb(h, ops_[i].inputs.size());
            for (uint64_t in : ops_[i].inputs) absorb(h, oc[in]);
            absorb(h, ops_[i].outputs.size());
            for (uint64_t out : ops_[i].outputs) absorb(h, oc[out]);
            npc[i] = h;
        }
        oc.swap(noc);
        pc.swap(npc);
        const std::size_t refined = countClasses(oc, pc);
        if (refined == classes) break;
        classes = refined;
    }
    p.operand_color_ = oc;
    p.op_color_      = pc;

    std::vector<uint64_t> tokens{n_operands, n_ops};
    std::vector<uint64_t> sorted_oc(oc), sorted_pc(pc);
    std::sort(sorted_oc.begin(), sorted_oc.end());
    std::sort(sorted_pc.begin(), sorted_pc.end());
    tokens.insert(tokens.end(), sorted_oc.begin(), sorted_oc.end());
    tokens.insert(tokens.end(), sorted_pc.begin(), sorted_pc.end());
    p.key_ = PatternKey(std::move(tokens));
    return p;
}

// ------------------------------------------------------------------ matcher

namespace {

constexpr uint64_t kUnset = ~uint64_t{0};

class Matcher {
  public:
    Matcher(const Pattern& user, const Pattern& sup)
        : u_(user), s_(sup), u2s_(user.numOperands(), kUnset), s2u_(sup.numOperands(), kUnset),
          op_u2s_(user.numOps(), kUnset), s_op_used_(sup.numOps(), false) {}

    bool run() {
        if (u_.numOperands() != s_.numOperands() || u_.numOps() != s_.numOps()) return false;
        if (!matchOp(0)) return false;
        return pairIsolated();
    }

    std::vector<uint64_t> operandMap() const { return u2s_; }
    std::vector<uint64_t> opMap() const { return op_u2s_; }

  private:
    bool bindPorts(const std::vector<uint64_t>& uports, const std::vector<uint64_t>& sports,
                   std::vector<uint64_t>& bound) {
        if (uports.size() != sports.size()) return false;
        for (std::size_t i = 0; i < uports.size(); ++i) {
            const uint64_t u = uports[i], s = sports[i];
            if (u_.operandKind(u) != s_.operandKind(s)) return false;
            if (u2s_[u] == kUnset && s2u_[s] == kUnset) {
                u2s_[u] = s;
                s2u_[s] = u;
                bound.push_back(u);
            } else if (u2s_[u] != s || s2u_[s] != u) {
                return false;
            }
        }
        return true;
    }

    void unbind(const std::vector<uint64_t>& bound) {
        for (uint64_t u : bound) {
            s2u_[u2s_[u]] = kUnset;
            u2s_[u]       = kUnset;
        }
    }

    bool matchOp(std::size_t uo) {
        if (uo == u_.numOps()) return true;
        const OpNode& un = u_.op(uo);
        for (std::size_t so = 0; so < s_.numOps(); ++so) {
            if (s_op_used_[so] || s_.op(so).kind != un.kind || s_.opColor(so) != u_.opColor(uo)) continue;
            std::vector<uint64_t> bound;
            if (bindPorts(un.inputs, s_.op(so).inputs, bound) && bindPorts(un.outputs, s_.op(so).outputs, bound)) {
                s_op_used_[so] = true;
                op_u2s_[uo]    = so;
                if (matchOp(uo + 1)) return true;
                s_op_used_[so] = false;
                op_u2s_[uo]    = kUnset;
            }
            unbind(bound);
        }
        return false;
    }

    // Operands no operation touches can pair with any free operand of the
    // same storage family.
    bool pairIsolated() {
        for (std::size_t u = 0; u < u_.numOperands(); ++u) {
            if (u2s_[u] != kUnset) continue;
            if (!u_.isIsolated(u)) return false;
            bool paired = false;
            for (std::size_t s = 0; s < s_.numOperands() && !paired; ++s) {
                if (s2u_[s] == kUnset && s_.isIsolated(s) && s_.operandKind(s) == u_.operandKind(u)) {
                    u2s_[u] = s;
                    s2u_[s] = u;
                    paired  = true;
                }
            }
            if (!paired) return false;
        }
        return true;
    }

    const Pattern& u_;
    const Pattern& s_;
    std::vector<uint64_t> u2s_, s2u_, op_u2s_;
    std::vector<bool> s_op_used_;
};

}  // namespace

Ops::Ops(const Pattern& user, const Pattern& supported) : key_(user.key()) {
    if (user.key() != supported.key())
        raise(FTRAIN_STATUS_UNSUPPORTED, "Ops: user Pattern does not match the supported Pattern");
    Matcher m(user, supported);
    if (!m.run()) raise(FTRAIN_STATUS_UNSUPPORTED, "Ops: user Pattern does not match the supported Pattern");
    operand_map_ = m.operandMap();
    op_map_      = m.opMap();
    for (std::size_t i = 0; i < supported.numOperands(); ++i) operand_kinds_.push_back(supported.operandKind(i));
    for (std::size_t i = 0; i < supported.numOps(); ++i) op_kinds_.push_back(supported.op(i).kind);
}

Args Ops::makeArgs() const {
    Args a;
    a.key_           = key_;
    a.operand_map_   = operand_map_;
    a.op_map_        = op_map_;
    a.operand_kinds_ = operand_kinds_;
    a.op_kinds_      = op_kinds_;
    a.operands_.resize(operand_kinds_.size());
    a.operations_.resize(op_kinds_.size());
    return a;
}

bool Args::isComplete() const noexcept {
    for (const auto& v : operands_)
        if (!v) return false;
    for (const auto& v : operations_)
        if (!v) return false;
    return true;
}

const std::optional<OperandValue>& Args::operand(uint64_t id) const {
    if (id >= operands_.size())
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Supported operand role index %llu is out of range [0, %zu)",
                        static_cast<unsigned long long>(id), operands_.size());
    return operands_[id];
}

const std::optional<OperationAttributes>& Args::operation(uint64_t id) const {
    if (id >= operations_.size())
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Supported op role index %llu is out of range [0, %zu)",
                        static_cast<unsigned long long>(id), operations_.size());
    return operations_[id];
}

void Args::setOperand(uint64_t user_id, OperandValue value) {
    if (user_id >= operand_map_.size())
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "User operand role index %llu is out of range [0, %zu)",
                        static_cast<unsigned long long>(user_id), operand_map_.size());
    const uint64_t slot = operand_map_[user_id];
    if (static_cast<std::size_t>(operand_kinds_[slot]) != value.index())
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "User operand role %llu has a different storage family",
                        static_cast<unsigned long long>(user_id));
    operands_[slot] = std::move(value);
}

void Args::setOperation(uint64_t user_id, OperationAttributes attributes) {
    if (user_id >= op_map_.size())
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "User op role index %llu is out of range [0, %zu)",
                        static_cast<unsigned long long>(user_id), op_map_.size());
    const uint64_t slot = op_map_[user_id];
    if (op_kinds_[slot] != attributes.kind)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "User op role %llu has a different operation kind",
                        static_cast<unsigned long long>(user_id));
    operations_[slot] = attributes;
}

}  // namespace ftrain
