"""The streaming pool sized from the device's own memory, on a device: Engine::init's budget
(src/engine.cpp:84-117) restated for HBM as lstk_pool_default_bytes, fed by hipMemGetInfo inside
lstk_pool_create (LSTK_POOL_AUTO_SIZE) and by torch.cuda.mem_get_info in load_qwen3_gguf(streaming=True).

The slot counts a budget gives are taken from a dry pool (bookkeeping only, the same plan_streaming)
created with that budget, so each test checks that the device path read the device's figures and fed them
to the budget, not the budget's arithmetic (tests/test_pool.py pins that with known answers)."""
import numpy as np
import pytest

from localstack_amd import synth

pytestmark = pytest.mark.gpu

GIB = 1 << 30
H, F, K = 256, 512, 2


def _layers(lstk, E, n_layer=2, seed=7):
    rng = np.random.default_rng(seed)
    t = (lstk.TYPE_Q8_0,) * 3
    return [(t, synth.experts(rng, 8, E, F, H), synth.experts(rng, 8, E, F, H), synth.experts(rng, 8, E, H, F))
            for _ in range(n_layer)]


def _table(lstk, E, n_layer=2):
    q = lstk.TYPE_Q8_0
    return n_layer * E * (2 * lstk.matrix_bytes(q, F, H) + lstk.matrix_bytes(q, H, F))


def _dry_slots(lstk, E, budget, min_slots, n_layer=2):
    dry = lstk.ExpertStore(n_layer, H, F, E, K, 4, [((8,) * 3, None, None, None)] * n_layer, pool_bytes=budget,
                           min_slots=min_slots, streaming=True, dry=True)
    n = dry.total_slots()
    dry.close()
    return n


def test_auto_size_holds_the_whole_table_when_it_fits(lstk, dev):
    """On a 288 GB device a small table fits: the budget is the table and every expert gets a slot."""
    import torch
    E = 64
    layers = _layers(lstk, E)
    free_now, total = torch.cuda.mem_get_info(dev)
    store = lstk.ExpertStore(2, H, F, E, K, 4, layers, min_slots=E, streaming=True, auto_size=True)
    budget = lstk.default_pool_bytes(_table(lstk, E), 0, 0, total, free_now)
    print(f"[auto size] free {free_now / GIB:.1f} GiB of {total / GIB:.1f}: budget {budget} B, "
          f"{store.total_slots()} slots", flush=True)
    assert budget == _table(lstk, E)
    assert store.total_slots() == _dry_slots(lstk, E, budget, E) == 2 * E
    store.close()


def test_auto_size_follows_free_memory(lstk, dev):
    """With all but 3 GiB + about 96 slabs of the device taken by other allocations, the free-memory term
    (free - 3 GiB) binds: the pool gets fewer slots than the table has experts and more than its floor,
    exactly as many as the budget from the figures read just before creation gives. Then the pool still
    serves acquires (misses copied from the host tier)."""
    import torch
    E = 64
    layers = _layers(lstk, E)
    slab = _table(lstk, E) // (2 * E)
    torch.cuda.empty_cache()
    filler = []
    for _ in range(16):  # the rest of the device in pieces of at most 32 GiB, until free - 3 GiB is near 96 slabs
        free_now, total = torch.cuda.mem_get_info(dev)
        take = free_now - 3 * GIB - 96 * slab
        if take < 8 * slab:
            break
        filler.append(torch.empty(min(take, 32 * GIB), dtype=torch.uint8, device=dev))
    try:
        free_now, total = torch.cuda.mem_get_info(dev)
        store = lstk.ExpertStore(2, H, F, E, K, 4, layers, min_slots=E, streaming=True, auto_size=True)
        budget = lstk.default_pool_bytes(_table(lstk, E), 0, 0, total, free_now)
        want = _dry_slots(lstk, E, budget, E)
        print(f"[auto size, device nearly full] free {free_now / GIB:.3f} GiB: budget {budget} B "
              f"({budget / slab:.1f} slabs), {store.total_slots()} slots (dry pool: {want})", flush=True)
        assert budget == free_now - 3 * GIB
        assert E < store.total_slots() == want < 2 * E
    finally:
        del filler
        torch.cuda.empty_cache()
    ids = np.arange(0, 2 * K * 4, dtype=np.int32) % E
    for layer in (0, 1):
        slots = store.acquire(layer, ids)
        assert len(set(slots.tolist())) == len(set(ids.tolist()))
        store.release_all()
    s = store.stats()
    assert s["misses"] > 0 and s["acquires"] == 2
    store.close()


def test_load_gguf_streaming_budget_from_device(lstk, dev, tmp_path):
    """load_qwen3_gguf(streaming=True) without pool_bytes sizes the pool from torch.cuda.mem_get_info, the
    dense weights and the KV cache; the table fits, so the streaming model holds every expert and decodes
    exactly like the resident one."""
    import torch
    hp = dict(n_layer=2, n_embd=H, n_head=4, n_head_kv=2, head_dim=64, n_vocab=1024, n_expert=8, n_expert_used=K,
              n_ff_exp=F, n_ctx_train=1024, rms_eps=1e-6, rope_freq_base=10000.0)
    w = synth.qwen3_weights(np.random.default_rng(1234), hp, wtype=8)
    path = tmp_path / "tiny.gguf"
    synth.write_qwen3_gguf(path, hp, w)
    _, rstore, rm, g1 = lstk.load_qwen3_gguf(path, n_batch=16, kv_size=256, device=dev)
    _, sstore, sm, g2 = lstk.load_qwen3_gguf(path, n_batch=16, kv_size=256, device=dev, streaming=True)
    assert sstore.total_slots() == 2 * hp["n_expert"]
    feed = np.random.default_rng(3).integers(0, hp["n_vocab"], 8).astype(np.int32)
    for _ in range(4):
        a = rm.decode(0, feed).cpu().numpy().copy()
        b = sm.decode(0, feed).cpu().numpy().copy()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(a, b)
        feed = np.array([np.argmax(a)], np.int32)
    for x in (rm, sm, rstore, sstore):
        x.close()
