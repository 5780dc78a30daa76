"""The expert cache's LRU bookkeeping (CPU): the C++ SlotLru (through the
wl_lru_replay test hook) against the reference's behavioural cases
(src/test_glm_expert_cache.cu:46-181) and the Python restatement in
oracle/lru.py."""
import numpy as np
import pytest

from oracle import lru as OL
from windlass_amd import moe


def _both(capacity, keys, batch):
    got = moe.lru_replay(capacity, keys, batch)
    ref = OL.replay(capacity, list(keys), batch)
    assert list(got[0]) == ref[0]
    assert got[1:] == ref[1:]
    return got


def test_case1_cold_miss_then_hit():
    out, h, m, e = _both(8, [0, 0], 1)
    assert (h, m, e) == (1, 1, 0) and list(out) == [0, 1]


def test_case3_eviction_is_lru():
    # fill 4 slots, bump 0, then 4 evicts the true tail (1): 0 hits, 1 misses
    out, h, m, e = _both(4, [0, 1, 2, 3, 0, 4, 0, 1], 1)
    assert list(out) == [0, 0, 0, 0, 1, 0, 1, 0]
    assert (h, m, e) == (2, 6, 2)


def test_case4_batch_pattern_counts():
    # 24 batches of 8 drawn from a 20-expert pool against 16 slots
    keys = [(b * 3 + k) % 20 for b in range(24) for k in range(8)]
    out, h, m, e = _both(16, keys, 8)
    assert h + m == 24 * 8 and h > 0 and m > 0
    assert (h, m, e) == (115, 77, 61)


def test_case4_counts_by_hand():
    """The same counts from first principles: batch b holds experts
    3b..3b+7 (mod 20); with 16 slots and 8-wide batches, an expert is still
    resident iff it was requested in one of the last two batches or the slots
    never filled. Counted directly, without any LRU structure."""
    hits = misses = 0
    last = {}  # expert -> last batch
    resident = set()
    order = []
    for b in range(24):
        ids = [(b * 3 + k) % 20 for k in range(8)]
        for x in ids:
            if x in resident:
                hits += 1
                order.remove(x)
            else:
                misses += 1
                if len(resident) == 16:
                    resident.discard(order.pop(0))
                resident.add(x)
            order.append(x)
            last[x] = b
    assert (hits, misses) == (115, 77)
    assert misses - 16 == 61  # every miss after the pool filled evicted one key


def test_duplicates_in_a_batch_are_skipped():
    out, h, m, e = _both(4, [5, 5, 6, 5, 7, 7], 3)
    assert list(out) == [0, 2, 0, 1, 0, 2]
    assert (h, m, e) == (1, 3, 0)


@pytest.mark.parametrize("capacity,batch,seed", [(16, 8, 0), (37, 8, 1), (64, 6, 2), (3, 1, 3)])
def test_random_sequences_match_oracle(capacity, batch, seed):
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, 201) ** 1.1  # Zipf-like popularity
    keys = rng.choice(200, size=3000, p=p / p.sum()).astype(np.uint32)
    _both(capacity, keys, batch)
