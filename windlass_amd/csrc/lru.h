// lru.h — the map from (layer, expert) keys to the slots of an HBM expert
// pool, under a replacement / admission policy. Host-only bookkeeping (no
// device calls), shared by the cache path of moe_host.cpp and the
// wl_policy_replay / wl_lru_replay test hooks.
//
// WL_POLICY_LRU is the reference's ExpertCache (src/glm_expert_cache.cuh:
// 198-308,356-368): a hit moves the key to the most-recent end; a miss takes a
// free slot (the most recently freed first; initially the highest index) or,
// when none is left, evicts the least-recent key and reuses its slot, then
// inserts the new key at the most-recent end. Keys of one request batch are
// deduplicated by the caller. The other policies (no reference counterpart):
//   LFU      evict the key requested least often so far (ties: least recent)
//   SLRU     segmented LRU: misses enter a probationary segment, a hit there
//            promotes to a protected segment of protected_frac x capacity
//            (its least recent key demoted back); victims come from the
//            probationary end first
//   2Q       admission on a second miss: a key missing for the first time
//            (not in the ghost list of the last `ghost` first misses) is not
//            retained
//   TINYLFU  frequency admission: a missing key is retained only if it has
//            been requested more often than the victim it would replace
//            (exact counts)
// Victims are never keys of the current batch, nor pinned keys; a pinned key
// is always admitted. A miss that is not retained (not admitted, or no
// evictable key) is served from one of the pool's transient slots
// [capacity, capacity + transient), used round robin and never looked up
// again.
#pragma once
#include <stdint.h>

#include <list>
#include <set>
#include <unordered_map>
#include <unordered_set>
#include <utility>
#include <vector>

namespace wl {

enum Policy : int32_t { kLru = 0, kLfu = 1, kSlru = 2, k2Q = 3, kTinyLfu = 4, kBelady = 5, kBeladyBypass = 6 };

class SlotLru {
public:
    SlotLru(uint32_t capacity, int32_t policy = kLru, float protected_frac = 0.5f, uint32_t ghost = 0,
            uint32_t transient = 0)
        : capacity_(capacity), policy_(policy), transient_(transient), iter_(capacity), seg_(capacity, 0),
          batch_of_(capacity, 0) {
        free_.reserve(capacity);
        for (uint32_t i = 0; i < capacity; i++) free_.push_back(i);
        prot_cap_ = (uint32_t)(protected_frac * (float)capacity);
        ghost_cap_ = ghost ? ghost : capacity;
    }

    struct Result {
        uint32_t slot;
        bool hit;
        bool evicted;
        uint32_t evicted_key;
        bool transient;  // served from a transient slot, not retained
    };

    // A new request batch: its keys are not evicted by requests of the batch.
    void begin_batch() { batch_++; }

    // One request. count = false leaves hits/misses untouched (speculative
    // requests are counted by the caller); evictions are always counted.
    Result request(uint32_t key, bool count = true) {
        Result r{0u, false, false, 0u, false};
        freq_[key]++;
        auto it = slot_of_.find(key);
        if (it != slot_of_.end()) {
            r.slot = it->second;
            r.hit = true;
            touch(r.slot, key);
            batch_of_[r.slot] = batch_;
            if (count) hits_++;
            return r;
        }
        if (count) misses_++;
        if (!free_.empty()) {
            r.slot = free_.back();
            free_.pop_back();
            insert(r.slot, key);
            return r;
        }
        uint32_t vslot = 0;
        const bool have = victim(vslot);
        bool admit = have;
        const bool pin = pinned_.count(key) != 0;  // a pinned key is always admitted
        if (have && !pin && policy_ == kTinyLfu) admit = freq_[key] > freq_[order_key(vslot)];
        if (policy_ == k2Q && !pin) {
            auto g = ghost_pos_.find(key);
            if (g == ghost_pos_.end()) {  // first miss: remember, do not retain
                ghost_.push_front(key);
                ghost_pos_[key] = ghost_.begin();
                if (ghost_.size() > ghost_cap_) {
                    ghost_pos_.erase(ghost_.back());
                    ghost_.pop_back();
                }
                admit = false;
            } else {
                ghost_.erase(g->second);
                ghost_pos_.erase(g);
            }
        }
        if (!admit || !have) {
            r.transient = true;
            r.slot = transient_ ? capacity_ + (next_transient_++ % transient_) : 0u;
            return r;
        }
        r.evicted_key = order_key(vslot);
        r.evicted = true;
        erase(vslot);
        evictions_++;
        r.slot = vslot;
        insert(vslot, key);
        return r;
    }

    // Drops a key (its slot becomes free), e.g. when filling it failed.
    void forget(uint32_t key) {
        auto it = slot_of_.find(key);
        if (it == slot_of_.end()) return;
        const uint32_t slot = it->second;
        erase(slot);
        free_.push_back(slot);
    }

    void pin(uint32_t key, bool on) {
        if (on) pinned_.insert(key);
        else pinned_.erase(key);
    }
    uint32_t pinned() const { return (uint32_t)pinned_.size(); }

    bool contains(uint32_t key) const { return slot_of_.count(key) != 0; }
    uint32_t used() const { return (uint32_t)slot_of_.size(); }
    uint32_t capacity() const { return capacity_; }
    uint64_t hits() const { return hits_; }
    uint64_t misses() const { return misses_; }
    uint64_t evictions() const { return evictions_; }
    void reset_stats() { hits_ = misses_ = evictions_ = 0; }

private:
    // Segment 0: main / probationary list, 1: protected list (SLRU).
    std::list<uint32_t>& list_of(uint32_t slot) { return seg_[slot] ? prot_ : order_; }
    uint32_t order_key(uint32_t slot) { return *iter_[slot]; }
    void insert(uint32_t slot, uint32_t key) {
        slot_of_[key] = slot;
        order_.push_front(key);
        iter_[slot] = order_.begin();
        seg_[slot] = 0;
        batch_of_[slot] = batch_;
    }
    void erase(uint32_t slot) {
        const uint32_t key = *iter_[slot];
        list_of(slot).erase(iter_[slot]);
        slot_of_.erase(key);
    }
    void touch(uint32_t slot, uint32_t key) {
        if (policy_ == kSlru) {
            if (seg_[slot] == 0) {  // probation -> protected (most recent)
                order_.erase(iter_[slot]);
                prot_.push_front(key);
                iter_[slot] = prot_.begin();
                seg_[slot] = 1;
                if (prot_.size() > prot_cap_) {  // demote the least recent protected key
                    const uint32_t dk = prot_.back();
                    const uint32_t ds = slot_of_[dk];
                    prot_.pop_back();
                    order_.push_front(dk);
                    iter_[ds] = order_.begin();
                    seg_[ds] = 0;
                }
            } else {
                prot_.splice(prot_.begin(), prot_, iter_[slot]);
                iter_[slot] = prot_.begin();
            }
            return;
        }
        order_.splice(order_.begin(), order_, iter_[slot]);
        iter_[slot] = order_.begin();
    }
    bool evictable(uint32_t key) {
        const uint32_t slot = slot_of_[key];
        return batch_of_[slot] != batch_ && !pinned_.count(key);
    }
    // The victim's slot: the least recent evictable key (LRU / 2Q / TinyLFU),
    // of the probationary segment first (SLRU), or the least requested one,
    // ties to the least recent (LFU).
    bool victim(uint32_t& slot) {
        if (policy_ == kLfu) {
            bool found = false;
            uint64_t best = 0;
            for (auto it = order_.rbegin(); it != order_.rend(); ++it) {  // least recent first
                if (!evictable(*it)) continue;
                const uint64_t f = freq_[*it];
                if (!found || f < best) {
                    found = true;
                    best = f;
                    slot = slot_of_[*it];
                }
            }
            return found;
        }
        for (std::list<uint32_t>* l : {&order_, &prot_})
            for (auto it = l->rbegin(); it != l->rend(); ++it)
                if (evictable(*it)) {
                    slot = slot_of_[*it];
                    return true;
                }
        return false;
    }

    uint32_t capacity_;
    int32_t policy_;
    uint32_t transient_, next_transient_ = 0;
    uint32_t prot_cap_ = 0, ghost_cap_ = 0;
    uint64_t batch_ = 1;
    std::unordered_map<uint32_t, uint32_t> slot_of_;
    std::list<uint32_t> order_;  // front = most recent (probationary segment under SLRU)
    std::list<uint32_t> prot_;   // SLRU protected segment, front = most recent
    std::vector<std::list<uint32_t>::iterator> iter_;
    std::vector<uint8_t> seg_;
    std::vector<uint64_t> batch_of_;  // the batch that last requested the slot's key
    std::vector<uint32_t> free_;
    std::unordered_map<uint32_t, uint64_t> freq_;
    std::list<uint32_t> ghost_;
    std::unordered_map<uint32_t, std::list<uint32_t>::iterator> ghost_pos_;
    std::unordered_set<uint32_t> pinned_;
    uint64_t hits_ = 0, misses_ = 0, evictions_ = 0;
};

// Belady's offline bound over a whole request sequence (replay only: it
// needs every future request; no reference counterpart, the reference's
// results discuss LRU only, docs/RESULTS.md:113,123). Keys repeated within a
// batch are skipped (marked 2), as in SlotLru. The bound drops the one
// constraint SlotLru adds to plain paging, that a key the current batch has
// requested is not evicted by the batch's later misses; without it the
// problem is classic paging, where MIN is the optimum, and the relaxed
// optimum bounds every policy under the constraint (and with pinned keys)
// from above. A miss takes a free slot while one is left; otherwise the
// resident key whose next request comes last (never requested again first)
// is evicted. With bypass, a missing key whose own next request comes after
// that victim's is not retained (marked 3), the optimum of a cache that may
// decline a key (the model of the admission policies); without bypass, of
// one that retains every miss (LRU, LFU, SLRU). Ties (keys never requested
// again) go to the smaller key. hit_out[i]: 1 hit, 0 retained miss, 3 miss
// not retained, 2 duplicate within its batch.
inline void belady_replay(uint32_t capacity, const uint32_t* keys, uint32_t n, uint32_t batch, bool bypass,
                          uint8_t* hit_out, uint64_t* hits, uint64_t* misses, uint64_t* evictions) {
    const uint64_t kNever = ~0ull;
    std::vector<uint8_t> dup(n, 0);
    for (uint32_t b0 = 0; b0 < n; b0 += batch) {
        const uint32_t b1 = b0 + batch < n ? b0 + batch : n;
        for (uint32_t i = b0; i < b1; i++)
            for (uint32_t j = b0; j < i && !dup[i]; j++) dup[i] = keys[j] == keys[i];
    }
    // next[i]: the position of the next request of keys[i] (duplicates skipped)
    std::vector<uint64_t> next(n, kNever);
    {
        std::unordered_map<uint32_t, uint64_t> seen;
        for (uint32_t i = n; i-- > 0;) {
            if (dup[i]) continue;
            auto it = seen.find(keys[i]);
            next[i] = it == seen.end() ? kNever : it->second;
            seen[keys[i]] = i;
        }
    }
    std::unordered_map<uint32_t, uint64_t> due;  // resident key -> its next request
    // (next request, key): the victim is the last element, so among keys
    // never requested again the smallest is stored as the largest
    std::set<std::pair<uint64_t, uint32_t>> by_due;
    auto order_key = [](uint32_t k) { return ~k; };
    uint64_t h = 0, m = 0, ev = 0;
    for (uint32_t i = 0; i < n; i++) {
        if (dup[i]) {
            if (hit_out) hit_out[i] = 2;
            continue;
        }
        const uint32_t k = keys[i];
        auto it = due.find(k);
        if (it != due.end()) {
            by_due.erase({it->second, order_key(k)});
            it->second = next[i];
            by_due.insert({next[i], order_key(k)});
            h++;
            if (hit_out) hit_out[i] = 1;
            continue;
        }
        m++;
        uint8_t code = 0;
        if (due.size() >= capacity) {
            const auto v = std::prev(by_due.end());
            if (bypass && !(next[i] < v->first)) {
                code = 3;
            } else {
                due.erase(~v->second);
                by_due.erase(v);
                ev++;
            }
        }
        if (code == 0) {
            due[k] = next[i];
            by_due.insert({next[i], order_key(k)});
        }
        if (hit_out) hit_out[i] = code;
    }
    if (hits) *hits = h;
    if (misses) *misses = m;
    if (evictions) *evictions = ev;
}

}  // namespace wl
