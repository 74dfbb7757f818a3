"""ExpertStore slot bookkeeping (src/expert_store.cpp:106-295): the oracle restatement and the
product pool (bookkeeping-only "dry" mode, no GPU) against known answers from the reference's logs
and against each other."""
import numpy as np
import pytest

Q4_K, Q8_0 = 12, 8
SLAB_30B_Q4K = (884736, 884736, 884736)  # per-expert up/gate/down bytes at 2048 x 768


def engine_step_ids(rng, L, E, k, n):
    """Routing ids of one Engine::step_streaming (src/engine.cpp:326-399): layers 0..L-2 acquire all
    n rows, the last layer only the last row (src/engine.cpp:366-368)."""
    out = []
    for l in range(L):
        rows = n if l < L - 1 else 1
        out.append((l, np.stack([rng.choice(E, k, replace=False) for _ in range(rows)]).astype(np.int32)))
    return out


def replay(pool, steps, L=48, E=128, k=8, seed=0):
    """Runs the segment acquire pattern; returns the number of acquire() calls (= segments with experts)."""
    rng = np.random.default_rng(seed)
    calls = 0
    for n in steps:
        for l, ids in engine_step_ids(rng, L, E, k, n):
            pool.acquire(l, ids.ravel())
            pool.release_all()
            calls += 1
    return calls


def oracle_pool(orc, L=48, E=128, pool_bytes=1 << 30, min_slots=128, types=(Q4_K,) * 3, strides=SLAB_30B_Q4K):
    return orc.Pool(L, E, np.tile(types, (L, 1)), np.tile(strides, (L, 1)), pool_bytes, min_slots)


def product_pool(lstk, L=48, E=128, pool_bytes=1 << 30, min_slots=128, types=(Q4_K,) * 3, h=2048, f=768, k=8):
    layers = [(types, None, None, None)] * L
    return lstk.ExpertStore(L, h, f, E, k, 512, layers, pool_bytes=pool_bytes, min_slots=min_slots, streaming=True,
                            dry=True)


# Known answers: "experts: N loads" lines of docs/runs/Qwen3-30B-A3B-UD-Q2_K_XL.md (:12, :50, :30); a
# load is a hit or a miss (src/main.cpp:611-613), so N = sum of acquired ids.
KNOWN = [
    ([18] + [1] * 24, 15992),                    # 18-token prompt, 24 decode steps
    ([32, 1, 64] + [1] * 48, 54928),             # --bench 64 48 (src/main.cpp:343-364)
    ([18] + [1] * 200, 83576),                   # routing-trace run, 200 sampled tokens
]


@pytest.mark.parametrize("steps,loads", KNOWN)
def test_known_answer_load_counts_oracle(orc, steps, loads):
    p = oracle_pool(orc)
    replay(p, steps)
    st = p.stats()
    assert st["hits"] + st["misses"] == loads
    assert st["acquires"] == 48 * len(steps)


@pytest.mark.parametrize("steps,loads", KNOWN)
def test_known_answer_load_counts_product(lstk, steps, loads):
    p = product_pool(lstk)
    replay(p, steps)
    st = p.stats()
    assert st["hits"] + st["misses"] == loads
    assert st["bytes_read"] == st["misses"] * sum(SLAB_30B_Q4K)


def test_repeat_within_call_is_a_hit(orc, lstk):
    # a miss maps its slot at once, so the same expert again in the same call is a hit
    for p in (oracle_pool(orc, L=2, E=8, pool_bytes=0, min_slots=8), product_pool(lstk, L=2, E=8, pool_bytes=0, min_slots=8, k=2)):
        s = p.acquire(0, [3, 5, 3, 3])
        assert s[0] == s[2] == s[3] and s[0] != s[1]
        st = p.stats()
        assert (st["hits"], st["misses"]) == (2, 2)


def test_lru_order_known_sequence(orc, lstk):
    # 4 slots, all start free in the LRU with slot 0 at the head
    for p in (oracle_pool(orc, L=1, E=16, pool_bytes=0, min_slots=4), product_pool(lstk, L=1, E=16, pool_bytes=0, min_slots=4, k=2)):
        assert list(p.acquire(0, [10, 11])) == [0, 1]
        p.release_all()                                   # LRU: 2 3 0 1
        assert list(p.acquire(0, [12])) == [2]
        p.release_all()                                   # LRU: 3 0 1 2
        assert list(p.acquire(0, [10, 13])) == [0, 3]     # 10 hits slot 0; 13 takes the head (3)
        p.release_all()                                   # LRU: 1 2 0 3
        assert list(p.acquire(0, [14])) == [1]            # evicts expert 11
        p.release_all()
        assert list(p.acquire(0, [11])) == [2]            # 11 was evicted: a miss into the head (2)


def test_exhaustion(orc, lstk):
    for p in (oracle_pool(orc, L=1, E=16, pool_bytes=0, min_slots=4), product_pool(lstk, L=1, E=16, pool_bytes=0, min_slots=4, k=2)):
        with pytest.raises(RuntimeError, match="exhausted"):
            p.acquire(0, [0, 1, 2, 3, 4])
        p.release_all()
        assert len(p.acquire(0, [5, 6, 7, 8])) == 4


def test_min_slots_limit(orc, lstk):
    with pytest.raises(ValueError, match="1024"):
        oracle_pool(orc, min_slots=1025)
    with pytest.raises(lstk.LstkError, match="1024"):
        product_pool(lstk, min_slots=1025)


def test_shard_split_235b_known_answer(orc, lstk):
    # 94 Q4_K layers, slab 3 x 3,538,944 B, 32 GiB: want 3236 slots -> 4 shards of ceil(94/4) = 24
    # layers; each shard gets 32 GiB * layers / 94 / slab slots (src/expert_store.cpp:130-149)
    L, slab = 94, 3 * 3538944
    p = orc.Pool(L, 128, np.tile((Q4_K,) * 3, (L, 1)), np.tile((3538944,) * 3, (L, 1)), 32 << 30, 128)
    assert p.n_shards == 4
    assert [p.shard_slots(i) for i in range(4)] == [826, 826, 826, 757]
    assert [p.shard_of_layer(l) for l in (0, 23, 24, 71, 72, 93)] == [0, 0, 1, 2, 3, 3]
    q = lstk.ExpertStore(L, 4096, 1536, 128, 8, 1, [((Q4_K,) * 3, None, None, None)] * L, pool_bytes=32 << 30,
                         min_slots=128, streaming=True, dry=True)
    assert [q.layer_slots(l) for l in (0, 24, 48, 72)] == [826, 826, 826, 757]
    assert q.total_slots() == 826 * 3 + 757
    assert q.total_bytes() == (826 * 3 + 757) * slab
    assert "4 shards" not in q.describe() and q.describe().count("pool q4_K/q4_K/q4_K: 24 layers, 826 slots") == 3


def test_type_classes_split_pools(orc, lstk):
    # layers with different (up, gate, down) types never share a shard; classes in ascending order
    L = 6
    types = [(Q8_0,) * 3 if l % 2 else (Q4_K,) * 3 for l in range(L)]
    strides = [(1671168,) * 3 if l % 2 else (884736,) * 3 for l in range(L)]
    p = orc.Pool(L, 128, np.array(types), np.array(strides), 1 << 30, 128)
    assert p.n_shards == 2
    assert [p.shard_of_layer(l) for l in range(L)] == [1, 0, 1, 0, 1, 0]  # Q8_0 (8) sorts before Q4_K (12)
    q = lstk.ExpertStore(L, 2048, 768, 128, 8, 1, [(t, None, None, None) for t in types], pool_bytes=1 << 30,
                         min_slots=128, streaming=True, dry=True)
    d = q.describe().splitlines()
    assert d[0].strip().startswith("pool q8_0/q8_0/q8_0: 3 layers") and d[1].strip().startswith("pool q4_K/q4_K/q4_K: 3 layers")


def test_product_matches_oracle_random_traces(orc, lstk):
    rng = np.random.default_rng(40)
    L, E, k = 4, 32, 4
    for trial in range(5):
        pool_bytes = int(rng.integers(0, 3)) * 40 * sum(SLAB_30B_Q4K)
        a = oracle_pool(orc, L=L, E=E, pool_bytes=pool_bytes, min_slots=10)
        b = product_pool(lstk, L=L, E=E, pool_bytes=pool_bytes, min_slots=10, k=k)
        for step in range(60):
            layer = int(rng.integers(0, L))
            n = int(rng.integers(1, 4)) * k
            ids = rng.integers(0, E, n).astype(np.int32)
            ra = rb = None
            try:
                ra = a.acquire(layer, ids)
            except RuntimeError as e:
                ra = str(e)
            try:
                rb = b.acquire(layer, ids)
            except lstk.LstkError as e:
                rb = str(e)
            if isinstance(ra, str):
                assert isinstance(rb, str) and "exhausted" in rb
            else:
                assert np.array_equal(ra, rb)
            if rng.random() < 0.7:
                a.release_all()
                b.release_all()
        sa, sb = a.stats(), b.stats()
        assert (sa["hits"], sa["misses"], sa["bytes_read"], sa["acquires"]) == \
               (sb["hits"], sb["misses"], sb["bytes_read"], sb["acquires"])


def test_failed_copy_unmaps_slot(lstk):
    p = product_pool(lstk, L=1, E=16, pool_bytes=0, min_slots=4, k=2)
    p.debug_fail_copies(1)
    with pytest.raises(lstk.LstkError) as ei:
        p.acquire(0, [7])
    assert ei.value.code == lstk.E_IO
    p.release_all()
    st = p.stats()
    p.acquire(0, [7])  # not served from the slot that holds garbage: a fresh miss
    assert p.stats()["misses"] == st["misses"] + 1


def test_resident_acquire_is_identity(lstk):
    p = lstk.ExpertStore(2, 256, 512, 8, 2, 4, [((Q8_0,) * 3, None, None, None)] * 2, dry=True)
    assert list(p.acquire(1, [7, 0, 3])) == [7, 0, 3]
    assert p.layer_slots(0) == 8
    with pytest.raises(lstk.LstkError):
        p.acquire(1, [8])


def test_default_pool_bytes_hbm_budget(lstk):
    """Engine::init's pool budget (src/engine.cpp:84-117) restated for HBM, with injected device figures."""
    G = 1 << 30
    f = lstk.default_pool_bytes
    # a 235B-A22B-shaped Q4_K table fits whole on a 288 GB device: the pool holds the whole table
    table = 94 * 128 * 3 * 3538944
    assert f(table, 3 * G, 1 * G, 288 * 10**9, 280 * 10**9) == table
    # a table larger than the device: total - weights - kv - 1.5 GiB bounds it
    assert f(200 * G, 10 * G, 2 * G, 96 * G, 90 * G) == 96 * G - 10 * G - 2 * G - G - G // 2
    # little free memory right now: free - 3 GiB bounds it
    assert f(200 * G, 10 * G, 2 * G, 96 * G, 20 * G) == 17 * G
    # nothing left: the 16 KiB floor (ExpertStore::init then raises each shard to its minimum slots)
    assert f(200 * G, 90 * G, 10 * G, 96 * G, 2 * G) == 16 << 10
    assert f(0, 0, 0, 96 * G, 96 * G) == 16 << 10


def test_auto_size_needs_a_device_pool(lstk):
    with pytest.raises(lstk.LstkError, match="AUTO_SIZE"):
        lstk.ExpertStore(2, 256, 512, 8, 2, 4, [((8,) * 3, None, None, None)] * 2, pool_bytes=0, min_slots=8,
                         streaming=True, dry=True, auto_size=True)
