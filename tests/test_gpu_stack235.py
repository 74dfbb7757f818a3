"""The Qwen3-235B-A22B-shaped MoE stack on MI355X at full size: 94 layers, h 4096, 128 experts top-8 with
f 1536, Q4_K experts (10,616,832 bytes each), Zipf(1.1)-biased F16 routers, batch-1 decode.

One layer's expert table (1.36 GB) is generated and passed for every layer: the resident pool still holds
94 copies (127.7 GB of HBM) and the streaming pools give every layer its own slots and LRU entries (their
pinned host tier holds the one copy). Every layer has its own router and hnorm rows; the residual stream
runs through the stack (layer l's output is layer l + 1's residual input).

1. One layer with all 128 experts against the oracle (the reference's router and moe_apply restated with
   ggml CPU semantics): router ids bit-exact, weights within 1e-6, output within 2e-3 of the largest
   |out - resid|.
2. Three tokens through the 94 layers: the resident pool, the pool capped at 32 GiB with the host acquire
   (ids to the host, ExpertStore::acquire semantics, copies on side streams) and with the device acquire,
   give bit-identical outputs and routing at every layer (the identity of tools/test_streaming.sh:22-36).
"""
import numpy as np
import pytest

import oracle
from localstack_amd import synth

pytestmark = pytest.mark.gpu

H, F, E, K, N_LAYER = 4096, 1536, 128, 8, 94
Q4_K = 12
TOKENS = 3
POOL_GIB = 32


@pytest.fixture(scope="module")
def stack235():
    rng = np.random.default_rng(2350)
    up, gate, down = (synth.experts(rng, Q4_K, E, F, H), synth.experts(rng, Q4_K, E, F, H),
                      synth.experts(rng, Q4_K, E, H, F))
    routers = [synth.zipf_router_f16(rng, E, H) for _ in range(N_LAYER)]
    xs = rng.standard_normal((TOKENS, N_LAYER, H), dtype=np.float32)
    xs[:, :, 0] = 1.0  # the Zipf bias column
    resid0 = rng.standard_normal((TOKENS, H), dtype=np.float32)
    return dict(up=up, gate=gate, down=down, routers=routers, xs=xs, resid0=resid0)


def test_one_235b_layer_with_all_experts_matches_oracle(lstk, dev, stack235):
    import torch
    s = stack235
    store = lstk.ExpertStore(1, H, F, E, K, 1, [((Q4_K,) * 3, s["up"], s["gate"], s["down"])])
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    x, resid, router = s["xs"][0, 0:1], s["resid0"][0:1], s["routers"][0]
    out = torch.zeros((1, H), dtype=torch.float32, device=dev)
    ids = torch.zeros((1, K), dtype=torch.int32, device=dev)
    w = torch.zeros((1, K), dtype=torch.float32, device=dev)
    store.block(0, d(x), d(router), 1, d(resid), out, ids, w)
    store.check()
    rids, rw, _, _ = oracle.router(x, router, oracle.TYPE_F16, K)
    ref = oracle.moe_ffn(x, rids, rw, resid, s["up"].reshape(E, -1), s["gate"].reshape(E, -1), s["down"].reshape(E, -1),
                         (Q4_K,) * 3, F)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    assert np.max(np.abs(w.cpu().numpy() - rw)) <= 1e-6
    got = out.cpu().numpy()
    err = np.abs(got - ref).max() / np.abs(ref - resid).max()
    print(f"[235b layer] ids {rids.ravel().tolist()} rel max err {err:.2e}", flush=True)
    assert err <= 2e-3
    store.close()


def _through_stack(torch, dev, s, run_layer):
    """The TOKENS tokens through the 94 layers with run_layer(l, x, resid, out, ids, w); returns the final
    outputs [TOKENS][H] and the routing [TOKENS][N_LAYER][K]."""
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    outs, trace = [], np.zeros((TOKENS, N_LAYER, K), np.int32)
    bufs = [torch.zeros((1, H), dtype=torch.float32, device=dev) for _ in range(2)]
    ids = torch.zeros((1, K), dtype=torch.int32, device=dev)
    w = torch.zeros((1, K), dtype=torch.float32, device=dev)
    for t in range(TOKENS):
        bufs[0].copy_(d(s["resid0"][t:t + 1]))
        xt = d(s["xs"][t])
        for l in range(N_LAYER):
            run_layer(l, xt[l:l + 1], bufs[l % 2], bufs[(l + 1) % 2], ids, w)
            trace[t, l] = ids.cpu().numpy()[0]
        outs.append(bufs[N_LAYER % 2].cpu().numpy()[0].copy())
    return np.array(outs), trace


def test_235b_stack_streaming_pool_matches_resident(lstk, dev, stack235):
    import torch
    s = stack235
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    routers = [d(r) for r in s["routers"]]
    layers = [((Q4_K,) * 3, s["up"], s["gate"], s["down"])] * N_LAYER

    resident = lstk.ExpertStore(N_LAYER, H, F, E, K, 1, layers)
    assert resident.total_bytes() == N_LAYER * E * 3 * 3538944
    ref_out, ref_trace = _through_stack(
        torch, dev, s, lambda l, x, r, o, ids, w: resident.block(l, x, routers[l], 1, r, o, ids, w))
    resident.check()
    resident.close()
    torch.cuda.synchronize()
    print(f"[235b stack] resident: {TOKENS} tokens through {N_LAYER} layers, "
          f"{len(np.unique(ref_trace[:, 10]))} distinct experts at layer 10", flush=True)

    host = lstk.ExpertStore(N_LAYER, H, F, E, K, 1, layers, pool_bytes=POOL_GIB << 30, min_slots=2 * K + 2,
                            streaming=True)
    slots_d = torch.zeros((1, K), dtype=torch.int32, device=dev)

    def host_layer(l, x, r, o, ids, w):
        host.route(l, x, routers[l], 1, ids, w)
        slots = host.acquire(l, ids.cpu().numpy()[0])  # the router's choice to the host, as the reference does
        slots_d.copy_(torch.from_numpy(np.ascontiguousarray(slots.reshape(1, K))))
        host.ffn(l, x, slots_d, w, r, o)
        host.release_all()

    h_out, h_trace = _through_stack(torch, dev, s, host_layer)
    host.check()
    st = host.stats()
    print(f"[235b stack] 32 GiB pool, host acquire: {host.total_slots()} slots, hits {st['hits']} misses "
          f"{st['misses']}", flush=True)
    assert st["misses"] > 0 and st["hits"] > 0
    host.close()
    np.testing.assert_array_equal(h_trace, ref_trace)
    np.testing.assert_array_equal(h_out, ref_out)

    dpool = lstk.ExpertStore(N_LAYER, H, F, E, K, 1, layers, pool_bytes=POOL_GIB << 30, min_slots=2 * K + 2,
                             streaming=True, device_lru=True)

    def dev_layer(l, x, r, o, ids, w):
        dpool.route(l, x, routers[l], 1, ids, w)
        dpool.acquire_device(l, ids, slots_d)
        dpool.ffn(l, x, slots_d, w, r, o)

    d_out, d_trace = _through_stack(torch, dev, s, dev_layer)
    dpool.check()
    dst = dpool.stats()
    print(f"[235b stack] 32 GiB pool, device acquire: hits {dst['hits']} misses {dst['misses']}", flush=True)
    assert (dst["hits"], dst["misses"]) == (st["hits"], st["misses"])
    dpool.close()
    np.testing.assert_array_equal(d_trace, ref_trace)
    np.testing.assert_array_equal(d_out, ref_out)
