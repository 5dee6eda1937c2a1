// Operator-family engines and the process-wide engine registry.
//
// Contract follows the reference's OpsEngine and Handle
// (src/include/flash_train/engine.hpp:97-250, src/engine.cpp:17-27,
// src/include/flash_train/handle.hpp:19-38, src/handle.cpp:18-61):
//   createPrimitives = validate Args -> build Problem -> cache lookup on
//   (constraints, problem) -> on a miss ask the Finders in order (the first
//   Finder that yields an applicable candidate defines the whole ranked
//   selection), else every applicable record in registration order ->
//   publish -> clone + configure.  UNSUPPORTED names every rejection.
#pragma once

#include <algorithm>

#include <memory>
#include <shared_mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "ft/cache.hpp"
#include "ft/pattern.hpp"
#include "ft/primitive.hpp"

namespace ftrain {

class OpsEngineBase {
  public:
    virtual ~OpsEngineBase() = default;
    const Pattern& pattern() const noexcept { return pattern_; }

    virtual std::vector<std::unique_ptr<PrimitiveBase>> createPrimitives(const Args& args,
                                                                         const Constraints& constraints) const = 0;

    // Selection on the calling thread's current device; the Plan is bound
    // to that device.
    Plan createPlan(const Args& args) const {
        const FTrainDeviceId device = getCurrentDeviceId();
        return Plan(createPrimitives(args, Constraints(device)), device);
    }

  protected:
    explicit OpsEngineBase(Pattern pattern) : pattern_(std::move(pattern)) {}

  private:
    Pattern pattern_;
};

template <typename Family, typename... Finders>
class OpsEngine final : public OpsEngineBase {
  public:
    using Problem = typename Family::Problem;
    using Record  = std::shared_ptr<const Primitive<Problem>>;

    OpsEngine() : OpsEngineBase(Family::makePattern()), records_(Family::makeRecords()) {
        for (std::size_t i = 0; i < records_.size(); ++i) {
            if (!records_[i]) raise(FTRAIN_STATUS_INVALID_ARGUMENT, "OpsEngine Primitive %zu must not be null", i);
            const char* n = records_[i]->name();
            if (n == nullptr)
                raise(FTRAIN_STATUS_INVALID_ARGUMENT, "OpsEngine Primitive %zu must not return a null name", i);
            if (!by_name_.emplace(n, i).second)
                raise(FTRAIN_STATUS_INVALID_ARGUMENT, "OpsEngine Primitive %zu repeats the name %s", i, n);
        }
    }

    std::vector<std::unique_ptr<PrimitiveBase>> createPrimitives(const Args& args,
                                                                 const Constraints& constraints) const override {
        if (args.key() != pattern().key())
            raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Args PatternKey does not match this OpsEngine");
        if (!args.isComplete())
            raise(FTRAIN_STATUS_INVALID_ARGUMENT, "Args has one or more unset Operand or Op parameters");
        const Problem problem = Family::makeProblem(args);
        const CacheKey key(constraints.key(), problem.key());
        if (!selectionCacheDisabled()) {
            if (auto hit = cache_.find(key)) return configure(*hit, problem);
        }
        return configure(select(problem, constraints, key), problem);
    }

    // Selection without configuring or caching: the ranked record names.
    // Used by tests and tools to inspect Finder decisions.
    std::vector<std::string> rank(const Problem& problem, const Constraints& constraints) const {
        std::vector<std::string> names;
        Walk w;
        for (std::size_t i : selectInto(problem, constraints, w)) names.push_back(records_[i]->name());
        return names;
    }

  private:
    struct Walk {
        std::vector<std::size_t> chosen;
        std::unordered_set<std::size_t> seen;
        // Rejections grouped by reason, in order of first appearance, so a
        // family of variants that fail for one reason costs one clause of
        // the 2047-character message: "A, B: reason; C: other reason".
        std::vector<std::pair<std::string, std::string>> rejections;  // (reason, names)

        std::string joined() const {
            std::string out;
            for (const auto& [reason, names] : rejections) {
                if (!out.empty()) out += "; ";
                out += names + ": " + reason;
            }
            return out;
        }
    };

    bool offer(std::size_t i, const Problem& problem, const Constraints& constraints, Walk& w) const {
        if (!w.seen.insert(i).second) return false;
        const Record& r = records_[i];
        if (!primitiveAllowed(r->name())) return false;
        const Result ok = r->isApplicable(problem, constraints);
        if (!ok.isSuccess()) {
            const std::string reason = ok.getMessage();
            auto group = std::find_if(w.rejections.begin(), w.rejections.end(),
                                      [&](const auto& g) { return g.first == reason; });
            if (group == w.rejections.end())
                w.rejections.emplace_back(reason, r->name());
            else
                group->second += std::string(", ") + r->name();
            return false;
        }
        w.chosen.push_back(i);
        return true;
    }

    template <typename Finder>
    bool askFinder(const Problem& problem, const Constraints& constraints, Walk& w) const {
        if (disabledFinders().count(Finder::name())) return false;
        bool any = false;
        for (const std::string& candidate : Finder::candidates(problem, constraints)) {
            auto it = by_name_.find(candidate);
            if (it == by_name_.end()) continue;
            any = offer(it->second, problem, constraints, w) || any;
        }
        return any;
    }

    const std::vector<std::size_t>& selectInto(const Problem& problem, const Constraints& constraints, Walk& w) const {
        const bool found = (askFinder<Finders>(problem, constraints, w) || ...);
        if (!found)
            for (std::size_t i = 0; i < records_.size(); ++i) offer(i, problem, constraints, w);
        if (w.chosen.empty())
            raise(FTRAIN_STATUS_UNSUPPORTED, "No Primitive supports the supplied Args and runtime constraints (%s)",
                  w.joined().c_str());
        return w.chosen;
    }

    std::vector<std::size_t> select(const Problem& problem, const Constraints& constraints, const CacheKey& key) const {
        Walk w;
        std::vector<std::size_t> chosen = selectInto(problem, constraints, w);
        cache_.publish(key, chosen);
        return chosen;
    }

    std::vector<std::unique_ptr<PrimitiveBase>> configure(const std::vector<std::size_t>& positions,
                                                          const Problem& problem) const {
        std::vector<std::unique_ptr<PrimitiveBase>> out;
        out.reserve(positions.size());
        for (std::size_t i : positions) {
            std::unique_ptr<PrimitiveBase> p = records_[i]->clone();
            if (!p) raise(FTRAIN_STATUS_INTERNAL_ERROR, "Applicable Primitive returned a null clone");
            static_cast<Primitive<Problem>&>(*p).configure(problem);
            out.push_back(std::move(p));
        }
        return out;
    }

    std::vector<Record> records_;
    std::unordered_map<std::string, std::size_t> by_name_;
    mutable SelectionCache cache_;
};

// Process-wide PatternKey -> engine registry; entries live for the process.
class Handle {
  public:
    // INVALID_ARGUMENT for a null engine or an already registered key.
    void add(std::shared_ptr<OpsEngineBase> engine);
    std::shared_ptr<const OpsEngineBase> find(const PatternKey& key) const;
    std::size_t size() const;

  private:
    mutable std::shared_mutex mutex_;
    std::unordered_map<PatternKey, std::shared_ptr<const OpsEngineBase>, PatternKeyHash> engines_;
};

// The registry holding every built-in engine; built on first use.
Handle& globalHandle();

// The built-in engine catalog (one engine per operator family).
std::vector<std::shared_ptr<OpsEngineBase>> builtinEngines();

}  // namespace ftrain
