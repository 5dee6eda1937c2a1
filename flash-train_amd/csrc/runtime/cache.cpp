#include "ft/cache.hpp"

#include <algorithm>
#include <cstdlib>
#include <iterator>
#include <mutex>

#include <flash_train/env.h>

#include "ft/error.hpp"

namespace ftrain {

namespace {

// Lane 1: xor-multiply over the splitmix64 finaliser of each token.
inline uint64_t fmix(uint64_t x) noexcept {
    x ^= x >> 33;
    x *= 0xFF51AFD7ED558CCDULL;
    x ^= x >> 33;
    x *= 0xC4CEB9FE1A85EC53ULL;
    x ^= x >> 33;
    return x;
}

// Lane 2: rotate-multiply accumulation with a different odd constant, so a
// collision in one lane is independent of the other.
inline uint64_t rotl(uint64_t x, int r) noexcept { return (x << r) | (x >> (64 - r)); }

struct TwoLane {
    uint64_t a = 0x243F6A8885A308D3ULL;
    uint64_t b = 0x13198A2E03707344ULL;
    void add(uint64_t t) noexcept {
        a = fmix(a ^ (t + 0x9E3779B97F4A7C15ULL));
        b = rotl(b + t * 0xA0761D6478BD642FULL, 29) * 0xE7037ED1A0B428DBULL;
    }
};

}  // namespace

CacheKey::CacheKey(const std::vector<uint64_t>& constraint_tokens, const std::vector<uint64_t>& problem_tokens) noexcept {
    TwoLane h;
    h.add(constraint_tokens.size());
    for (uint64_t t : constraint_tokens) h.add(t);
    h.add(problem_tokens.size());
    for (uint64_t t : problem_tokens) h.add(t);
    lo_ = h.a;
    hi_ = fmix(h.b ^ h.a);
}

SelectionCache::SelectionCache(std::size_t max_entries, std::size_t shards) {
    if (max_entries == 0 || shards == 0)
        raise(FTRAIN_STATUS_INVALID_ARGUMENT, "selection cache: max_entries=%zu and shards=%zu must both be non-zero",
              max_entries, shards);
    // Each shard holds its even share of the limit, rounded up.
    const std::size_t share = max_entries / shards + (max_entries % shards != 0);
    shards_.resize(shards);
    for (auto& s : shards_) {
        s = std::make_unique<Shard>();
        s->limit = share;
    }
}

std::optional<std::vector<std::size_t>> SelectionCache::find(const CacheKey& key) const {
    Shard& s = shardFor(key);
    std::shared_lock lock(s.mutex);
    const auto it = s.map.find(key);
    if (it == s.map.end()) return std::nullopt;
    it->second.hits.fetch_add(1, std::memory_order_relaxed);
    return it->second.positions;
}

void SelectionCache::publish(const CacheKey& key, std::vector<std::size_t> positions) {
    if (positions.empty()) raise(FTRAIN_STATUS_INVALID_ARGUMENT, "selection cache: a selection must list a Primitive");
    Shard& s = shardFor(key);
    std::unique_lock lock(s.mutex);
    // First publisher wins; a racing second publisher of the same key keeps it.
    if (s.map.find(key) != s.map.end()) return;
    if (s.map.size() >= s.limit) evictBatch(s);
    s.map.emplace(key, Entry(std::move(positions)));
}

// Drops one eighth of a full shard (at least one entry), the entries with the
// fewest hits first.  Two passes: the batch's largest hit count is found by
// selection over the counts alone, then every entry below it goes, and
// entries equal to it go until the batch is complete.
void SelectionCache::evictBatch(Shard& shard) {
    const std::size_t batch = std::max<std::size_t>(1, shard.map.size() / 8);
    std::vector<uint64_t> counts;
    counts.reserve(shard.map.size());
    for (const auto& kv : shard.map) counts.push_back(kv.second.hits.load(std::memory_order_relaxed));
    std::nth_element(counts.begin(), counts.begin() + (batch - 1), counts.end());
    const uint64_t cut = counts[batch - 1];
    std::size_t below = 0;
    for (uint64_t c : counts) below += c < cut;
    std::size_t ties = batch - below;
    for (auto it = shard.map.begin(); it != shard.map.end();) {
        const uint64_t h = it->second.hits.load(std::memory_order_relaxed);
        const bool drop = h < cut || (h == cut && ties > 0);
        if (drop && h == cut) --ties;
        it = drop ? shard.map.erase(it) : std::next(it);
    }
}

std::size_t SelectionCache::size() const {
    std::size_t n = 0;
    for (const auto& s : shards_) {
        std::shared_lock lock(s->mutex);
        n += s->map.size();
    }
    return n;
}

namespace {
std::string trim(const std::string& s) {
    const auto first = s.find_first_not_of(" \t");
    if (first == std::string::npos) return {};
    const auto last = s.find_last_not_of(" \t");
    return s.substr(first, last - first + 1);
}
}  // namespace

std::unordered_set<std::string> parseNameList(const char* value) {
    std::unordered_set<std::string> names;
    if (value == nullptr) return names;
    const std::string text(value);
    std::size_t begin = 0;
    while (true) {
        const std::size_t comma = text.find(',', begin);
        const std::string item  = trim(text.substr(begin, comma == std::string::npos ? std::string::npos : comma - begin));
        if (!item.empty()) names.insert(item);
        if (comma == std::string::npos) break;
        begin = comma + 1;
    }
    return names;
}

bool parseSwitch(const char* value) {
    if (value == nullptr) return false;
    const std::string t = trim(value);
    return !t.empty() && t != "0";
}

const std::unordered_set<std::string>& enabledPrimitives() {
    static const auto v = parseNameList(std::getenv(FTRAIN_ENABLED_PRIMITIVES));
    return v;
}
const std::unordered_set<std::string>& disabledPrimitives() {
    static const auto v = parseNameList(std::getenv(FTRAIN_DISABLED_PRIMITIVES));
    return v;
}
const std::unordered_set<std::string>& disabledFinders() {
    static const auto v = parseNameList(std::getenv(FTRAIN_DISABLED_FINDERS));
    return v;
}
bool selectionCacheDisabled() {
    static const bool v = parseSwitch(std::getenv(FTRAIN_DISABLE_CACHE));
    return v;
}

}  // namespace ftrain
