#include <mutex>

#include "ft/engine.hpp"

namespace ftrain {

void Handle::add(std::shared_ptr<OpsEngineBase> engine) {
    if (!engine) raise(FTRAIN_STATUS_INVALID_ARGUMENT, "engine registry: cannot register a null engine");
    std::unique_lock lock(mutex_);
    const PatternKey key = engine->pattern().key();
    if (!engines_.emplace(key, std::move(engine)).second)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "engine registry: this Pattern already has an engine");
}

std::shared_ptr<const OpsEngineBase> Handle::find(const PatternKey& key) const {
    std::shared_lock lock(mutex_);
    auto it = engines_.find(key);
    return it == engines_.end() ? nullptr : it->second;
}

std::size_t Handle::size() const {
    std::shared_lock lock(mutex_);
    return engines_.size();
}

Handle& globalHandle() {
    static Handle* const handle = [] {
        auto* h = new Handle();
        for (auto& e : builtinEngines()) h->add(std::move(e));
        return h;
    }();
    return *handle;
}

}  // namespace ftrain
