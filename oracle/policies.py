"""CPU restatement of the expert cache's replacement and admission policies —
parity oracle.

TEST INFRASTRUCTURE ONLY (imported by tests/ as the checker of the library's
policy engine through wl_policy_replay, and of bench.py's policy study).

LRU is the reference's ExpertCache (src/glm_expert_cache.cuh:198-308,
356-368; also oracle/lru.py). The others have no reference counterpart; they
restate the definitions the library documents (include/windlass_moe.h):
  lfu      evict the least requested key (ties: least recent)
  slru     probationary + protected segment (protected_frac of the slots)
  2q       a first miss is remembered in a ghost list and not retained; a
           miss found in the ghost list is retained
  tinylfu  a miss is retained only if its request count exceeds its victim's
Common rules: keys repeated inside a batch are skipped; a victim is never a
key the current batch has already requested (as in the reference, whose LRU
victim is the least recent key: the batch's own keys are the most recent)
nor a pinned key, and a pinned key is always admitted; while a slot is free a miss takes
it (no admission test); a miss that is not retained (not admitted, or no
evictable key) is a miss that leaves the cache unchanged.
Written with ordered dictionaries (most recent last), independently of the
library's linked lists.
"""
from collections import Counter, OrderedDict


class PolicyCache:
    def __init__(self, kind, capacity, protected_frac=0.5, ghost=0, pinned=()):
        self.kind, self.cap = kind, capacity
        self.prot_cap = int(protected_frac * capacity)
        self.ghost_cap = ghost or capacity
        self.main = OrderedDict()  # probationary segment under slru; oldest first
        self.prot = OrderedDict()
        self.ghost = OrderedDict()
        self.freq = Counter()
        self.pinned = set(pinned)
        self.hits = self.misses = self.evictions = 0

    def _size(self):
        return len(self.main) + len(self.prot)

    def _victim(self, batch):
        ok = [k for k in list(self.main) + list(self.prot) if k not in batch and k not in self.pinned]
        if not ok:
            return None
        if self.kind == "lfu":
            # least requested, ties to the least recent (main is oldest first)
            return min(ok, key=lambda k: self.freq[k])
        return ok[0]  # oldest of main first, then of prot

    def request(self, key, batch):
        """1 hit, 0 retained miss, 3 miss not retained."""
        self.freq[key] += 1
        if key in self.prot:
            self.prot.move_to_end(key)
            self.hits += 1
            return 1
        if key in self.main:
            self.hits += 1
            if self.kind == "slru":
                del self.main[key]
                self.prot[key] = True
                if len(self.prot) > self.prot_cap:
                    old, _ = self.prot.popitem(last=False)
                    self.main[old] = True
            else:
                self.main.move_to_end(key)
            return 1
        self.misses += 1
        if self._size() < self.cap:
            self.main[key] = True
            return 0
        v = self._victim(batch)
        admit = v is not None
        pin = key in self.pinned  # pinned keys are always admitted
        if admit and not pin and self.kind == "tinylfu":
            admit = self.freq[key] > self.freq[v]
        if self.kind == "2q" and not pin:
            if key in self.ghost:
                del self.ghost[key]
            else:
                self.ghost[key] = True
                if len(self.ghost) > self.ghost_cap:
                    self.ghost.popitem(last=False)
                admit = False
        if not admit or v is None:
            return 3
        if v in self.main:
            del self.main[v]
        else:
            del self.prot[v]
        self.evictions += 1
        self.main[key] = True
        return 0


def replay(kind, capacity, keys, batch, protected_frac=0.5, ghost=0, pinned=()):
    """(per-key 1 / 0 / 3 / 2-duplicate, hits, misses, evictions) in batches."""
    c = PolicyCache(kind, capacity, protected_frac, ghost, pinned)
    out = []
    for b0 in range(0, len(keys), batch):
        b = keys[b0:b0 + batch]
        seen = set()
        for k in b:
            if k in seen:
                out.append(2)
                continue
            out.append(c.request(k, seen))
            seen.add(k)
    return out, c.hits, c.misses, c.evictions


def belady(capacity, keys, batch, bypass=False):
    """Belady's offline bound (no reference counterpart; the library's
    WL_POLICY_BELADY / WL_POLICY_BELADY_BYPASS replay kinds): keys repeated
    within a batch are skipped; with every future request known, a miss
    evicts the resident key whose next request comes last (keys never
    requested again first, the smaller key of those first); with bypass, a
    miss whose own next request comes after that victim's is not retained.
    Unlike replay(), a batch's miss may evict a key the batch has already
    requested: the bound is plain paging, where this rule is the optimum.
    Returns (per-key codes, hits, misses, evictions) like replay(). Written
    as a forward scan for each next request, independently of the library's
    precomputed next-use table."""
    never = float("inf")

    def next_use(k, i):
        for j in range(i + 1, len(keys)):
            b0 = j - j % batch
            if keys[j] == k and k not in keys[b0:j]:
                return j
        return never

    cache = set()
    out = []
    hits = misses = evictions = 0
    for i, k in enumerate(keys):
        b0 = i - i % batch
        if k in keys[b0:i]:
            out.append(2)
            continue
        if k in cache:
            hits += 1
            out.append(1)
            continue
        misses += 1
        if len(cache) >= capacity:
            victim = max(cache, key=lambda c: (next_use(c, i), -c))
            if bypass and not next_use(k, i) < next_use(victim, i):
                out.append(3)
                continue
            cache.remove(victim)
            evictions += 1
        cache.add(k)
        out.append(0)
    return out, hits, misses, evictions
