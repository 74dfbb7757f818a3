"""Device-side acquire (LSTK_POOL_DEVICE_LRU): the LRU resolved on the GPU and the misses copied from the
pinned host tier by a kernel.

Bars: the same slots, hits, misses and bytes as the host bookkeeping (ExpertStore::acquire + release_all,
src/expert_store.cpp:232-295) call for call on the reference's recorded routing trace; expert outputs
identical bit for bit to the resident pool's (the copies must move exactly the expert bytes).
"""
import os

import numpy as np
import pytest

from localstack_amd import synth

pytestmark = pytest.mark.gpu

Q8_0, Q4_K = 8, 12
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "routing_trace_30b_a3b_ud_q2_k_xl.npz")


def recorded_steps():
    z = np.load(GOLDEN)
    n_layer, n_expert, k = (int(v) for v in z["header"])
    ids = z["ids"].astype(np.int32)
    steps, off = [], 0
    for n in z["steps"]:
        m = n_layer * int(n) * k
        steps.append(ids[off:off + m].reshape(n_layer, int(n), k))
        off += m
    return n_expert, k, steps


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("n_batch,slots_per_layer", [(1, 16), (8, 12)])
def test_device_lru_equals_host_lru_on_recorded_trace(lstk, dev, n_batch, slots_per_layer):
    """Six layers of the recorded Qwen3-30B-A3B trace in two type classes (two shards, each shared by
    three layers, so evictions cross layers), replayed call by call through the host bookkeeping (a dry
    pool) and the device one: every call's slots and the final counters agree."""
    import torch
    import localstack_amd as L
    E, k, steps = recorded_steps()
    pick = [0, 9, 17, 30, 40, 47]
    h = f = 256
    types = [(Q8_0,) * 3 if i % 2 == 0 else (Q4_K,) * 3 for i in range(len(pick))]
    rng = np.random.default_rng(500)
    layers = []
    for t in types:
        layers.append((t, synth.experts(rng, t[0], E, f, h), synth.experts(rng, t[1], E, f, h),
                       synth.experts(rng, t[2], E, h, f)))
    slab8 = 3 * 256 * 8 * 34
    n_slots = max(min(n_batch * k, E), slots_per_layer * 3)
    # each class gets pool_bytes * 3 / 6 bytes; size it so the Q8_0 class gets n_slots slots
    pool_bytes = 2 * n_slots * slab8
    host = L.ExpertStore(len(pick), h, f, E, k, n_batch, [(t, None, None, None) for t in types], pool_bytes=pool_bytes,
                         min_slots=min(n_batch * k, E), streaming=True, dry=True)
    devp = L.ExpertStore(len(pick), h, f, E, k, n_batch, layers, pool_bytes=pool_bytes,
                         min_slots=min(n_batch * k, E), streaming=True, device_lru=True)
    assert [host.layer_slots(l) for l in range(len(pick))] == [devp.layer_slots(l) for l in range(len(pick))]
    assert devp.layer_slots(0) == n_slots and devp.layer_slots(1) > n_slots  # Q4_K slabs are smaller
    d_ids = torch.zeros(n_batch * k, dtype=torch.int32, device=dev)
    d_slots = torch.zeros(n_batch * k, dtype=torch.int32, device=dev)
    calls = 0
    for ids in steps:
        T = ids.shape[1]
        for t0 in range(0, T, n_batch):
            for l, src in enumerate(pick):
                rows = ids[src, t0:t0 + n_batch]
                rows = rows[rows[:, 0] >= 0]
                if len(rows) == 0:
                    continue
                want = host.acquire(l, rows)
                host.release_all()
                n = rows.size
                d_ids[:n].copy_(torch.from_numpy(rows.ravel()))
                devp.acquire_device(l, d_ids, d_slots, n=n)
                got = d_slots[:n].cpu().numpy().reshape(rows.shape)
                np.testing.assert_array_equal(got, want, err_msg=f"call {calls} layer {l}")
                calls += 1
    devp.check()
    hs, ds = host.stats(), devp.stats()
    print(f"[device lru n_batch {n_batch}] {calls} calls, host {hs}, device {ds}", flush=True)
    for key in ("hits", "misses", "bytes_read", "acquires"):
        assert hs[key] == ds[key], key
    assert hs["misses"] > 0 and hs["hits"] > 0


@pytest.mark.parametrize("types,h,f,E,k,T", [((Q8_0,) * 3, 256, 512, 8, 2, 8), ((Q4_K, Q4_K, Q8_0), 256, 768, 16, 4, 8),
                                             ((Q4_K,) * 3, 4096, 1536, 16, 8, 8), ((Q4_K,) * 3, 1024, 512, 32, 4, 64)])
def test_device_acquire_ffn_equals_resident(orc, lstk, dev, types, h, f, E, k, T):
    """route -> acquire_device -> ffn on a pool that evicts constantly gives exactly the resident block's
    output (the copy kernel moves whole expert matrices, Q8_0 / Q4_K and partial 16 KiB chunks; at 64
    tokens the grouped matrix-core path runs on the slots)."""
    import torch
    import localstack_amd as L
    n_layer = 2
    rng = np.random.default_rng(510 + h + E)
    layers = [(types, synth.experts(rng, types[0], E, f, h), synth.experts(rng, types[1], E, f, h),
               synth.experts(rng, types[2], E, h, f)) for _ in range(n_layer)]
    routers = [to_dev(synth.router_f16(rng, E, h), dev) for _ in range(n_layer)]
    res = L.ExpertStore(n_layer, h, f, E, k, T, layers)
    need = min(T * k, E)
    st = L.ExpertStore(n_layer, h, f, E, k, T, layers, pool_bytes=1, min_slots=need, streaming=True, device_lru=True)
    assert st.layer_slots(0) == need
    ids_r = torch.zeros((T, k), dtype=torch.int32, device=dev)
    w_r = torch.zeros((T, k), dtype=torch.float32, device=dev)
    ids_s, w_s = torch.zeros_like(ids_r), torch.zeros_like(w_r)
    slots = torch.zeros((T, k), dtype=torch.int32, device=dev)
    for step in range(4):
        for l in range(n_layer):
            n = 1 if step % 2 else T
            x = to_dev(synth.activations(rng, T, h), dev)
            resid = to_dev(synth.activations(rng, T, h), dev)
            a = resid.clone()
            res.block(l, x, routers[l], 1, a, a, ids_r, w_r, n_tokens=n)
            b = resid.clone()
            st.route(l, x, routers[l], 1, ids_s, w_s, n_tokens=n)
            st.acquire_device(l, ids_s, slots, n=n * k)
            st.ffn(l, x, slots, w_s, b, b, n_tokens=n)
            torch.cuda.synchronize()
            assert torch.equal(ids_s[:n], ids_r[:n]), (step, l)
            assert torch.equal(a[:n], b[:n]), (step, l)
    st.check()
    s = st.stats()
    print(f"[device acquire {types} h {h}] {s}", flush=True)
    assert s["misses"] > need and s["acquires"] == 4 * n_layer


def test_device_lru_errors(lstk, dev):
    import torch
    import localstack_amd as L
    h, f, E, k, T = 256, 512, 8, 2, 4
    rng = np.random.default_rng(520)
    t = (Q8_0,) * 3
    layers = [(t, synth.experts(rng, 8, E, f, h), synth.experts(rng, 8, E, f, h), synth.experts(rng, 8, E, h, f))]
    with pytest.raises(L.LstkError):  # resident pools keep no LRU
        L.ExpertStore(1, h, f, E, k, T, layers, device_lru=True)
    with pytest.raises(L.LstkError):  # fewer slots than one call can pin
        L.ExpertStore(1, h, f, E, k, T, layers, pool_bytes=1, min_slots=E - 1, streaming=True, device_lru=True)
    st = L.ExpertStore(1, h, f, E, k, T, layers, pool_bytes=1, min_slots=E, streaming=True, device_lru=True)
    host = L.ExpertStore(1, h, f, E, k, T, layers, pool_bytes=1, min_slots=E, streaming=True)
    with pytest.raises(L.LstkError):
        st.acquire(0, [1, 2])
    with pytest.raises(L.LstkError):
        st.debug_fail_copies(1)
    ids = torch.tensor([3, 5, 9, -2], dtype=torch.int32, device=dev)
    slots = torch.zeros(4, dtype=torch.int32, device=dev)
    with pytest.raises(L.LstkError):
        host.acquire_device(0, ids, slots)
    with pytest.raises(L.LstkError):
        st.acquire_device(0, ids, slots, n=T * k + 1)
    with pytest.raises(L.LstkError):
        st.acquire_device(1, ids, slots)
    st.acquire_device(0, ids, slots)  # ids 9 and -2 are out of range: clamped, then reported
    with pytest.raises(L.LstkError):
        st.check()
    got = slots.cpu().numpy()
    assert ((got >= 0) & (got < E)).all()
    st.check()  # the flag was cleared
    ok = torch.tensor([1, 2, 1, 7], dtype=torch.int32, device=dev)
    st.acquire_device(0, ok, slots)
    st.check()
    got = slots.cpu().numpy()
    assert got[0] == got[2] and len(set(got[[0, 1, 3]])) == 3


def test_captured_device_acquire_follows_inputs(lstk, dev):
    """route -> acquire_device -> ffn of several layers captured once and replayed with new hnorm rows
    copied into the graph's inputs: every replay equals the eager run of a twin pool (ids, outputs and
    counters), so the captured acquire resolves what each replay routes."""
    import torch
    import localstack_amd as L
    h, f, E, k, n_layer = 256, 512, 32, 4, 3
    t = (Q8_0,) * 3
    rng = np.random.default_rng(530)
    layers = [(t, synth.experts(rng, 8, E, f, h), synth.experts(rng, 8, E, f, h), synth.experts(rng, 8, E, h, f))
              for _ in range(n_layer)]
    routers = [to_dev(synth.router_f16(rng, E, h), dev) for _ in range(n_layer)]
    mk = lambda: L.ExpertStore(n_layer, h, f, E, k, 1, layers, pool_bytes=1, min_slots=2 * k, streaming=True,
                               device_lru=True)
    pe, pg = mk(), mk()
    assert pe.layer_slots(0) == 2 * k  # three layers share 8 slots: most tokens miss

    def bufs():
        return ([torch.zeros((1, h), dtype=torch.float32, device=dev) for _ in range(n_layer)],
                torch.zeros((n_layer, k), dtype=torch.int32, device=dev),
                torch.zeros((n_layer, k), dtype=torch.float32, device=dev),
                torch.zeros((n_layer, k), dtype=torch.int32, device=dev),
                torch.zeros((n_layer, h), dtype=torch.float32, device=dev))

    def token(p, xs, ids, w, slots, out):
        for l in range(n_layer):
            p.route(l, xs[l], routers[l], 1, ids[l:l + 1], w[l:l + 1])
            p.acquire_device(l, ids[l:l + 1], slots[l:l + 1])
            p.ffn(l, xs[l], slots[l:l + 1], w[l:l + 1], out[l:l + 1], out[l:l + 1])

    be, bg = bufs(), bufs()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            token(pg, *bg)
    torch.cuda.synchronize()
    for step in range(8):
        xs = [to_dev(synth.activations(rng, 1, h), dev) for _ in range(n_layer)]
        for l in range(n_layer):
            be[0][l].copy_(xs[l])
            bg[0][l].copy_(xs[l])
        token(pe, *be)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(be[1], bg[1]), step
        assert torch.equal(be[4], bg[4]), step
    se, sg = pe.stats(), pg.stats()
    print(f"[captured acquire] eager {se} graph {sg}", flush=True)
    for key in ("hits", "misses", "bytes_read", "acquires"):
        assert se[key] == sg[key], key
    assert sg["misses"] > 2 * k
