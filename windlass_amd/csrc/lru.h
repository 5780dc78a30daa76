// lru.h — least-recently-used map from (layer, expert) keys to the slots of
// an HBM expert pool. Host-only bookkeeping (no device calls), shared by the
// cache path of moe_host.cpp and the wl_lru_replay test hook.
//
// Semantics follow the reference's ExpertCache (src/glm_expert_cache.cuh:
// 198-308,356-368): a hit moves the key to the most-recent end; a miss takes a
// free slot (the most recently freed first; initially the highest index) or,
// when none is left, evicts the least-recent key and reuses its slot, then
// inserts the new key at the most-recent end. Keys of one request batch are
// deduplicated by the caller.
#pragma once
#include <stdint.h>

#include <list>
#include <unordered_map>
#include <vector>

namespace wl {

class SlotLru {
public:
    explicit SlotLru(uint32_t capacity) : capacity_(capacity), iter_(capacity) {
        free_.reserve(capacity);
        for (uint32_t i = 0; i < capacity; i++) free_.push_back(i);
    }

    struct Result {
        uint32_t slot;
        bool hit;
        bool evicted;
        uint32_t evicted_key;
    };

    // One request. count = false leaves hits/misses untouched (speculative
    // requests are counted by the caller); evictions are always counted.
    Result request(uint32_t key, bool count = true) {
        Result r{0u, false, false, 0u};
        auto it = slot_of_.find(key);
        if (it != slot_of_.end()) {
            r.slot = it->second;
            r.hit = true;
            order_.splice(order_.begin(), order_, iter_[r.slot]);
            iter_[r.slot] = order_.begin();
            if (count) hits_++;
            return r;
        }
        if (!free_.empty()) {
            r.slot = free_.back();
            free_.pop_back();
        } else {
            r.evicted_key = order_.back();
            r.evicted = true;
            r.slot = slot_of_[r.evicted_key];
            slot_of_.erase(r.evicted_key);
            order_.pop_back();
            evictions_++;
        }
        slot_of_[key] = r.slot;
        order_.push_front(key);
        iter_[r.slot] = order_.begin();
        if (count) misses_++;
        return r;
    }

    // Drops a key (its slot becomes free), e.g. when filling it failed.
    void forget(uint32_t key) {
        auto it = slot_of_.find(key);
        if (it == slot_of_.end()) return;
        const uint32_t slot = it->second;
        order_.erase(iter_[slot]);
        slot_of_.erase(it);
        free_.push_back(slot);
    }

    bool contains(uint32_t key) const { return slot_of_.count(key) != 0; }
    uint32_t used() const { return (uint32_t)slot_of_.size(); }
    uint32_t capacity() const { return capacity_; }
    uint64_t hits() const { return hits_; }
    uint64_t misses() const { return misses_; }
    uint64_t evictions() const { return evictions_; }
    void reset_stats() { hits_ = misses_ = evictions_ = 0; }

private:
    uint32_t capacity_;
    std::unordered_map<uint32_t, uint32_t> slot_of_;
    std::list<uint32_t> order_;  // front = most recent
    std::vector<std::list<uint32_t>::iterator> iter_;
    std::vector<uint32_t> free_;
    uint64_t hits_ = 0, misses_ = 0, evictions_ = 0;
};

}  // namespace wl
