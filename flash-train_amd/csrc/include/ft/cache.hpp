// Selection cache and environment filters.
//
// Contract follows the reference (src/include/flash_train/cache.hpp:27-170,
// src/cache.cpp:99-194): a 128-bit key summarising (constraint tokens,
// problem tokens); sharded maps under shared mutexes; publish keeps the
// first selection for a key; a full shard evicts a batch (1/8) of its
// least-hit entries; default limit 30,000,000 entries over 256 shards.
// The two hash lanes here are this library's own mixers.
#pragma once

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <shared_mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace ftrain {

class CacheKey {
  public:
    CacheKey(const std::vector<uint64_t>& constraint_tokens, const std::vector<uint64_t>& problem_tokens) noexcept;
    bool operator==(const CacheKey& o) const noexcept { return lo_ == o.lo_ && hi_ == o.hi_; }
    bool operator!=(const CacheKey& o) const noexcept { return !(*this == o); }
    std::size_t hash() const noexcept { return static_cast<std::size_t>(lo_); }

  private:
    uint64_t lo_, hi_;
};

struct CacheKeyHash {
    std::size_t operator()(const CacheKey& k) const noexcept { return k.hash(); }
};

class SelectionCache {
  public:
    static constexpr std::size_t kDefaultEntries = 30000000;
    static constexpr std::size_t kDefaultShards  = 256;

    // INVALID_ARGUMENT for a zero limit or zero shard count.
    explicit SelectionCache(std::size_t max_entries = kDefaultEntries, std::size_t shards = kDefaultShards);

    // Published positions for `key` (counting one hit), or nullopt.
    std::optional<std::vector<std::size_t>> find(const CacheKey& key) const;
    // Stores `positions` unless `key` is present; INVALID_ARGUMENT when empty.
    void publish(const CacheKey& key, std::vector<std::size_t> positions);
    std::size_t size() const;

  private:
    struct Entry {
        std::vector<std::size_t> positions;
        mutable std::atomic<uint64_t> hits{0};
        explicit Entry(std::vector<std::size_t> p) : positions(std::move(p)) {}
        Entry(Entry&& o) noexcept : positions(std::move(o.positions)), hits(o.hits.load()) {}
    };
    struct Shard {
        mutable std::shared_mutex mutex;
        std::unordered_map<CacheKey, Entry, CacheKeyHash> map;
        std::size_t limit = 1;
    };
    Shard& shardFor(const CacheKey& k) const { return *shards_[k.hash() % shards_.size()]; }
    static void evictBatch(Shard& shard);

    std::vector<std::unique_ptr<Shard>> shards_;
};

// Parsed once per process (reference src/cache.cpp:144-194).
const std::unordered_set<std::string>& enabledPrimitives();
const std::unordered_set<std::string>& disabledPrimitives();
const std::unordered_set<std::string>& disabledFinders();
bool selectionCacheDisabled();

// Exposed for unit tests: the parsing rules behind the functions above.
std::unordered_set<std::string> parseNameList(const char* value);
bool parseSwitch(const char* value);

inline bool primitiveAllowed(const std::string& name) {
    const auto& on  = enabledPrimitives();
    const auto& off = disabledPrimitives();
    if (!on.empty() && on.count(name) == 0) return false;
    return off.count(name) == 0;
}

}  // namespace ftrain
