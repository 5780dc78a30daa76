"""CPU restatement of the reference's expert-cache LRU — parity oracle.

TEST INFRASTRUCTURE ONLY (imported by tests/ as the checker).

Follows glm::ExpertCache (src/glm_expert_cache.cuh:198-308,356-368): a hit
moves the key to the most-recent end; a miss takes a free slot (the last of
the free list, initially the highest index) or evicts the least-recent key,
then inserts the key at the most-recent end; keys repeated inside one
prefetch batch are skipped (:186-196). Pinned by the reference's behavioural
cases (src/test_glm_expert_cache.cu:46-181: case 1 cold miss then hit, case 3
LRU order, case 4 batch pattern) in tests/test_cache_lru.py, where case 4's
counts (115 hits, 77 misses, 61 evictions) are also derived by hand-checkable
brute force.
"""
from collections import OrderedDict


class Lru:
    def __init__(self, capacity):
        self.capacity = capacity
        self.order = OrderedDict()  # key -> slot, last = most recent
        self.free = list(range(capacity))
        self.hits = self.misses = self.evictions = 0

    def request(self, key):
        if key in self.order:
            self.order.move_to_end(key)
            self.hits += 1
            return self.order[key], True
        if self.free:
            slot = self.free.pop()
        else:
            _, slot = self.order.popitem(last=False)
            self.evictions += 1
        self.order[key] = slot
        self.misses += 1
        return slot, False


def replay(capacity, keys, batch):
    """Per-key outcome (1 hit, 0 miss, 2 duplicate in its batch) and counters."""
    lru = Lru(capacity)
    out = []
    for b0 in range(0, len(keys), batch):
        seen = set()
        for k in keys[b0:b0 + batch]:
            if k in seen:
                out.append(2)
                continue
            seen.add(k)
            out.append(1 if lru.request(k)[1] else 0)
    return out, lru.hits, lru.misses, lru.evictions
