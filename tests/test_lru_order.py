"""The device-side acquire's algorithm (localstack_amd/csrc/tier.hip, lru_resolve_kernel) restated on the
CPU and held against the pool's LRU semantics (ExpertStore::acquire + release_all,
src/expert_store.cpp:232-295, as a plain ordered dictionary): same slots, hits and misses for every
call of random request streams - several layers sharing one shard, repeated experts within a call,
calls as large as the shard.

The kernel keeps a shard's slots as an array in eviction order and resolves one call in request order:
a resident expert is a hit (its slot marked used), otherwise the first unmarked entry is taken - and
only the first 2n entries are staged, since each request moves past at most two. The new order is the
unmarked entries in order, then the used slots by their last request. No GPU.
"""
import collections

import numpy as np
import pytest


def kernel_call(order, owner, slot_of, layer, experts):
    """One lru_resolve_kernel call. order: slot ids, oldest first (all idle); owner: slot -> (layer,
    expert) or None; slot_of: {(layer, expert): slot}. Returns (slots, misses, new order)."""
    ns, n = len(order), len(experts)
    reach = min(ns, 2 * n)
    used = set()
    got, misses, p = [], [], 0
    for e in experts:
        s = slot_of.get((layer, e), -1)
        if s >= 0:
            used.add(s)
            got.append(s)
            continue
        while p < reach and order[p] in used:
            p += 1
        assert p < reach, "the staged entries ran out"
        s = order[p]
        p += 1
        if owner[s] is not None:
            del slot_of[owner[s]]
        owner[s] = (layer, e)
        slot_of[(layer, e)] = s
        used.add(s)
        got.append(s)
        misses.append((s, e))
    last = {s: i for i, s in enumerate(got)}
    released = [s for i, s in enumerate(got) if last[s] == i]
    new_order = [s for s in order if s not in used] + released
    assert sorted(new_order) == list(range(ns))
    return got, misses, new_order


class DictLru:
    """Acquire (hit: pin; miss: evict the least recently released idle slot) then release_all (a slot
    whose pin count returns to 0 becomes the most recent), as the reference's linked list does."""

    def __init__(self, ns):
        self.idle = collections.OrderedDict((s, None) for s in range(ns))
        self.owner = [None] * ns
        self.slot_of = {}

    def call(self, layer, experts):
        pins, got, misses = collections.Counter(), [], []
        for e in experts:
            s = self.slot_of.get((layer, e), -1)
            if s < 0:
                s = next(iter(self.idle))
                if self.owner[s] is not None:
                    del self.slot_of[self.owner[s]]
                self.owner[s] = (layer, e)
                self.slot_of[(layer, e)] = s
                misses.append((s, e))
            if pins[s] == 0:
                self.idle.pop(s)
            pins[s] += 1
            got.append(s)
        for s in got:
            pins[s] -= 1
            if pins[s] == 0:
                self.idle[s] = None
        return got, misses


@pytest.mark.parametrize("ns,n_layer,E,k,tokens", [(24, 3, 16, 4, 1), (18, 2, 32, 8, 1), (64, 4, 128, 8, 1),
                                                   (40, 2, 64, 8, 4), (16, 1, 64, 8, 2), (9, 1, 12, 9, 1)])
def test_order_array_equals_lru(ns, n_layer, E, k, tokens):
    rng = np.random.default_rng(ns * 1000 + E)
    ref = DictLru(ns)
    order, owner, slot_of = list(range(ns)), [None] * ns, {}
    hits = 0
    for step in range(400):
        layer = step % n_layer
        # Zipf-skewed ids, each token's k distinct; tokens of one call may repeat experts
        experts = []
        for _ in range(tokens):
            p = 1.0 / np.arange(1, E + 1) ** 1.1
            experts += list(rng.choice(E, k, replace=False, p=p / p.sum()))
        experts = experts[:ns]
        want, want_miss = ref.call(layer, experts)
        got, miss, order = kernel_call(order, owner, slot_of, layer, experts)
        assert got == want and miss == want_miss, step
        assert order == list(ref.idle), step
        hits += len(experts) - len(miss)
    assert hits > 0


def test_misses_pass_the_hits_at_the_front():
    # hits on the three oldest entries, then a miss: it passes them and takes the fourth entry
    ns = 8
    order, owner, slot_of = list(range(ns)), [None] * ns, {}
    _, _, order = kernel_call(order, owner, slot_of, 0, [0, 1, 2, 3])  # slots 0..3 hold experts 0..3
    assert order == [4, 5, 6, 7, 0, 1, 2, 3]
    got, miss, order = kernel_call(order, owner, slot_of, 0, [4, 5, 6, 7])  # slots 4..7: experts 4..7
    got, miss, order = kernel_call(order, owner, slot_of, 0, [0, 1, 2, 9])
    assert got == [0, 1, 2, 3] and miss == [(3, 9)]
    assert order == [4, 5, 6, 7, 0, 1, 2, 3]
