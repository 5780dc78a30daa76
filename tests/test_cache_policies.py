"""The cache's replacement and admission policies (CPU): the library's engine
(wl_policy_replay, windlass_amd/csrc/lru.h) against the oracle's independent
restatement (oracle/policies.py) request by request on Zipf-skewed batched
key streams, with and without pinned keys, plus small sequences whose
outcome is worked out by hand for each policy."""
import numpy as np
import pytest

from oracle import lru as OL
from oracle import policies as OP
from windlass_amd import moe


def zipf_batches(n_batches, batch, n_keys, s, seed):
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, n_keys + 1) ** s
    p /= p.sum()
    perm = rng.permutation(n_keys)
    keys = []
    for _ in range(n_batches):
        keys += [int(perm[i]) for i in rng.choice(n_keys, size=batch, replace=False, p=p)]
    return keys


@pytest.mark.parametrize("kind", ["lru", "lfu", "slru", "2q", "tinylfu"])
@pytest.mark.parametrize("seed", [0, 1])
def test_engine_matches_oracle(kind, seed):
    keys = zipf_batches(400, 8, 300, 1.1, seed)
    for cap, ghost, frac in [(40, 0, 0.5), (64, 100, 0.3), (16, 0, 0.8)]:
        got = moe.policy_replay(moe.make_policy(kind, frac, ghost), cap, keys, 8)
        want = OP.replay(kind, cap, keys, 8, frac, ghost)
        assert list(got[0]) == want[0], (kind, cap)
        assert got[1:] == want[1:], (kind, cap, got[1:], want[1:])


@pytest.mark.parametrize("kind", ["lru", "lfu", "slru", "2q", "tinylfu"])
def test_engine_matches_oracle_with_pins(kind):
    keys = zipf_batches(300, 8, 200, 1.1, 7)
    pinned = [keys[3], keys[17], keys[40], 199]
    got = moe.policy_replay(kind, 32, keys, 8, pinned=pinned)
    want = OP.replay(kind, 32, keys, 8, pinned=pinned)
    assert list(got[0]) == want[0] and got[1:] == want[1:]
    # a pinned key, once in, is never a miss again
    for pk in pinned:
        idx = [i for i, k in enumerate(keys) if k == pk]
        if idx:
            assert all(got[0][i] in (1, 2) for i in idx[1:]), pk


def test_lru_policy_is_the_reference_lru():
    keys = zipf_batches(300, 8, 120, 1.1, 3)
    assert moe.policy_replay("lru", 24, keys, 8)[1:] == OL.replay(24, keys, 8)[1:]
    assert moe.lru_replay(24, keys, 8)[1:] == OL.replay(24, keys, 8)[1:]


# Hand-worked sequences, batches of one key, capacity 2 (the state after each
# request written out, most recent first).
SEQ = [1, 2, 1, 3, 1, 3, 2]


def test_hand_lru():
    # [1] [2 1] [1 2]h [3 1]e2 [1 3]h [3 1]h [2 3]e1
    out, h, m, e = moe.policy_replay("lru", 2, SEQ, 1)
    assert list(out) == [0, 0, 1, 0, 1, 1, 0] and (h, m, e) == (3, 4, 2)


def test_hand_lfu():
    # counts: 1:1 [1]; 2:1 [2 1]; 1:2 h; 3: victim = least count among {1:2, 2:1} -> 2, [3 1];
    # 1:3 h; 3:2 h; 2: victim least count {1:3, 3:2} -> 3, [2 1]
    out, h, m, e = moe.policy_replay("lfu", 2, SEQ, 1)
    assert list(out) == [0, 0, 1, 0, 1, 1, 0] and (h, m, e) == (3, 4, 2)


def test_hand_2q():
    # 1, 2 fill the free slots; 1 hit; 3 first miss: ghost {3}, not retained;
    # 1 hit; 3 second miss: retained, evicts LRU 2 (cache [3 1]); 2 first miss
    # after its eviction: ghost {2}, not retained
    out, h, m, e = moe.policy_replay("2q", 2, SEQ, 1)
    assert list(out) == [0, 0, 1, 3, 1, 0, 3] and (h, m, e) == (2, 5, 1)


def test_hand_tinylfu():
    # 3 (count 1) vs victim 2 (count 1): not retained; 1 hit (count 3); 3 (count 2)
    # vs victim 2 (count 1): retained, evicts 2; 2 (count 2) vs victim 1 (count 3): not retained
    out, h, m, e = moe.policy_replay("tinylfu", 2, SEQ, 1)
    assert list(out) == [0, 0, 1, 3, 1, 0, 3] and (h, m, e) == (2, 5, 1)


def test_hand_slru():
    # capacity 2, protected 1: 1 -> prob[1]; 2 -> prob[2 1]; 1 hit -> prot[1] prob[2];
    # 3 miss: victim prob's oldest 2 -> prob[3]; 1 hit in prot; 3 hit in prob ->
    # prot[3], 1 demoted to prob[1]; 2 miss: victim prob's oldest 1 -> prob[2]
    out, h, m, e = moe.policy_replay("slru", 2, SEQ, 1)
    assert list(out) == [0, 0, 1, 0, 1, 1, 0] and (h, m, e) == (3, 4, 2)
    assert OP.replay("slru", 2, SEQ, 1)[1:] == (3, 4, 2)


# The hand answers above, and one sequence that separates LFU from LRU:
# capacity 2, [1 1 2 3 1]: LRU evicts 1 (least recent) for 3, so the last 1
# misses; LFU evicts 2 (count 1 < 2), so it hits.
HAND = {"lru": ([0, 0, 1, 0, 1, 1, 0], (3, 4, 2)), "lfu": ([0, 0, 1, 0, 1, 1, 0], (3, 4, 2)),
        "slru": ([0, 0, 1, 0, 1, 1, 0], (3, 4, 2)), "2q": ([0, 0, 1, 3, 1, 0, 3], (2, 5, 1)),
        "tinylfu": ([0, 0, 1, 3, 1, 0, 3], (2, 5, 1))}
SEQ2 = [1, 1, 2, 3, 1]
HAND2 = {"lru": ([0, 1, 0, 0, 0], (1, 4, 2)), "lfu": ([0, 1, 0, 0, 1], (2, 3, 1))}


def _replay_with(cls, kind, cap, keys):
    c = cls(kind, cap)
    out = [c.request(k, {k}) for k in keys]
    return out, (c.hits, c.misses, c.evictions)


@pytest.mark.parametrize("kind", sorted(HAND))
def test_oracle_hand_cases(kind):
    """The oracle itself against the hand answers (the engine is checked
    against the oracle on random streams)."""
    out, h, m, e = OP.replay(kind, 2, SEQ, 1)
    assert (out, (h, m, e)) == HAND[kind]
    if kind in HAND2:
        out, h, m, e = OP.replay(kind, 2, SEQ2, 1)
        assert (out, (h, m, e)) == HAND2[kind]
        got = moe.policy_replay(kind, 2, SEQ2, 1)
        assert (list(got[0]), got[1:]) == HAND2[kind]


def test_planted_mistakes_fail_the_hand_cases():
    """Mistakes planted in a copy of the oracle: each changes a hand answer."""

    class MostRecentVictim(OP.PolicyCache):  # evicts the newest key instead of the oldest
        def _victim(self, batch):
            ok = [k for k in list(self.main) + list(self.prot) if k not in batch and k not in self.pinned]
            return ok[-1] if ok else None

    class AdmitOnTie(OP.PolicyCache):  # TinyLFU admission with >= instead of >
        def request(self, key, batch):
            self.freq[key] += 1  # compared one higher: count + 1 > victim's  <=>  count >= victim's
            r = super().request(key, batch)
            self.freq[key] -= 1
            return r

    class LfuTiesToNewest(OP.PolicyCache):  # LFU ties broken toward the most recent key
        def _victim(self, batch):
            ok = [k for k in list(self.main) + list(self.prot) if k not in batch and k not in self.pinned]
            return min(reversed(ok), key=lambda k: self.freq[k]) if ok else None

    assert _replay_with(OP.PolicyCache, "lru", 2, SEQ) == HAND["lru"]
    assert _replay_with(MostRecentVictim, "lru", 2, SEQ) != HAND["lru"]
    assert _replay_with(OP.PolicyCache, "tinylfu", 2, SEQ) == HAND["tinylfu"]
    assert _replay_with(AdmitOnTie, "tinylfu", 2, SEQ) != HAND["tinylfu"]
    assert _replay_with(OP.PolicyCache, "lfu", 2, [1, 2, 3, 1]) != _replay_with(LfuTiesToNewest, "lfu", 2,
                                                                                 [1, 2, 3, 1])


# ---- Belady's offline bound ------------------------------------------------

def _optimum(capacity, keys, batch, bypass, protect_batch):
    """The most hits any eviction schedule reaches (exhaustive search over
    every victim choice at every miss, and every decline when bypass is
    allowed). protect_batch: a miss may not evict a key its batch has already
    requested (the library's online rule); without it, plain paging."""
    from functools import lru_cache
    n = len(keys)

    @lru_cache(maxsize=None)
    def best(i, cache):
        if i == n:
            return 0
        k = keys[i]
        b0 = i - i % batch
        if k in keys[b0:i]:
            return best(i + 1, cache)
        if k in cache:
            return 1 + best(i + 1, cache)
        if len(cache) < capacity:
            return best(i + 1, cache | {k})
        held = set(keys[b0:i]) if protect_batch else set()
        opts = [best(i + 1, (cache - {v}) | {k}) for v in cache if v not in held]
        if bypass or not opts:
            opts.append(best(i + 1, cache))
        return max(opts)

    return best(0, frozenset())


def test_belady_hand_case():
    # capacity 2, SEQ = 1 2 1 3 1 3 2: 3 misses with {1 (next at 4), 2 (next
    # at 6)} resident and evicts 2; the last 2 finds {1, 3}, both never
    # requested again: without bypass it evicts 1 (the smaller key), with
    # bypass it is not retained (its own next request, never, is not earlier)
    for got in (moe.policy_replay("belady", 2, SEQ, 1), OP.belady(2, SEQ, 1)):
        assert (list(got[0]), tuple(got[1:])) == ([0, 0, 1, 0, 1, 1, 0], (3, 4, 2))
    for got in (moe.policy_replay("belady_bypass", 2, SEQ, 1), OP.belady(2, SEQ, 1, bypass=True)):
        assert (list(got[0]), tuple(got[1:])) == ([0, 0, 1, 0, 1, 1, 3], (3, 4, 1))


@pytest.mark.parametrize("bypass", [False, True])
def test_belady_is_the_optimum_on_small_sequences(bypass):
    """Exhaustive search pins the bound: on random small batched sequences
    Belady's hits equal the most any eviction schedule reaches in plain
    paging, and are at least the most under the online batch rule."""
    rng = np.random.default_rng(11 + bypass)
    for case in range(150):
        batch = int(rng.integers(1, 3))
        cap = int(rng.integers(batch + 1, 4))
        keys = []
        for _ in range(int(rng.integers(4, 9))):
            keys += [int(x) for x in rng.integers(0, 6, size=batch)]
        want = _optimum(cap, tuple(keys), batch, bypass, False)
        kind = "belady_bypass" if bypass else "belady"
        assert moe.policy_replay(kind, cap, keys, batch)[1] == want, (case, cap, batch, keys)
        assert OP.belady(cap, keys, batch, bypass)[1] == want, (case, cap, batch, keys)
        assert _optimum(cap, tuple(keys), batch, bypass, True) <= want


@pytest.mark.parametrize("seed", [0, 1])
def test_belady_engine_matches_oracle_and_bounds_every_policy(seed):
    keys = zipf_batches(300, 8, 200, 1.1, seed)
    pinned = [keys[5], keys[60]]
    for cap in (24, 48):
        for bypass in (False, True):
            got = moe.policy_replay("belady_bypass" if bypass else "belady", cap, keys, 8)
            want = OP.belady(cap, keys, 8, bypass)
            assert list(got[0]) == want[0] and got[1:] == want[1:], (cap, bypass)
        bound = moe.policy_replay("belady", cap, keys, 8)[1]
        bound_bypass = moe.policy_replay("belady_bypass", cap, keys, 8)[1]
        assert bound <= bound_bypass
        for kind in ("lru", "lfu", "slru"):
            assert moe.policy_replay(kind, cap, keys, 8)[1] <= bound, (kind, cap)
            assert moe.policy_replay(kind, cap, keys, 8, pinned=pinned)[1] <= bound, (kind, cap)
        for kind in ("2q", "tinylfu"):
            assert moe.policy_replay(kind, cap, keys, 8)[1] <= bound_bypass, (kind, cap)
    with pytest.raises(moe.WindlassError):  # the bound takes no pinned keys
        moe.policy_replay("belady", 24, keys, 8, pinned=pinned)


def test_planted_mistake_fails_the_belady_hand_case():
    """Evicting the key whose next request comes FIRST (a planted sign
    mistake, in a copy of the oracle's rule) changes the hand answer."""
    never = float("inf")

    def nearest_victim(capacity, keys):
        cache, hits = [], 0
        for i, k in enumerate(keys):
            if k in cache:
                hits += 1
                continue
            if len(cache) >= capacity:
                nxt = {c: next((j for j in range(i + 1, len(keys)) if keys[j] == c), never) for c in cache}
                cache.remove(min(cache, key=lambda c: nxt[c]))
            cache.append(k)
        return hits

    assert nearest_victim(2, SEQ) != OP.belady(2, SEQ, 1)[1]
    assert moe.policy_replay("belady", 2, [1, 2, 3, 1, 2], 1)[1] == 1
    assert moe.policy_replay("lru", 2, [1, 2, 3, 1, 2], 1)[1] == 0
