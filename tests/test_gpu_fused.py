"""The fused single-token path (one launch per MoE block, stages handing over inside the kernel;
opt-in with LSTK_FUSED_DECODE=1 at pool creation) against the multi-kernel path, through the C ABI.

Bar: bit-identical outputs, ids and weights (both paths run the same quantizers, dot products and
reduction orders), across routed and given-slot calls, every weight-type combination, an F32
router, consecutive layers and repeated HIP graph replays; and within the oracle tolerance.
"""
import os

import numpy as np
import pytest

from localstack_amd import synth

pytestmark = pytest.mark.gpu

Q8_0, Q4_K = 8, 12
FFN_TOL = 2e-3
SHAPES = {
    "30b_q8": dict(h=2048, f=768, E=128, k=8, types=(Q8_0,) * 3),
    "30b_q4": dict(h=2048, f=768, E=128, k=8, types=(Q4_K,) * 3),
    "tiny": dict(h=256, f=512, E=8, k=2, types=(Q8_0,) * 3),
    "mixed": dict(h=256, f=768, E=16, k=4, types=(Q4_K, Q4_K, Q8_0)),
    "q8_gate_q4_down": dict(h=1024, f=512, E=64, k=6, types=(Q8_0, Q8_0, Q4_K)),
}
_cache = {}


def pools(name, n_layer=2):
    """(cfg, layers, routers, fused pool, multi-kernel pool) over the same expert bytes."""
    if name in _cache:
        return _cache[name]
    import localstack_amd as L
    cfg = SHAPES[name]
    rng = np.random.default_rng(sum(map(ord, name)) + 99)
    t = cfg["types"]
    layers = [(t, synth.experts(rng, t[0], cfg["E"], cfg["f"], cfg["h"]), synth.experts(rng, t[1], cfg["E"], cfg["f"], cfg["h"]),
               synth.experts(rng, t[2], cfg["E"], cfg["h"], cfg["f"])) for _ in range(n_layer)]
    routers = [synth.router_f16(rng, cfg["E"], cfg["h"]) for _ in range(n_layer)]
    args = (n_layer, cfg["h"], cfg["f"], cfg["E"], cfg["k"], 8, layers)
    multi = L.ExpertStore(*args)
    os.environ["LSTK_FUSED_DECODE"] = "1"
    try:
        fused = L.ExpertStore(*args)
    finally:
        del os.environ["LSTK_FUSED_DECODE"]
    _cache[name] = (cfg, layers, routers, fused, multi)
    return _cache[name]


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def run_block(store, layer, x, gate, gate_type, resid, dev):
    import torch
    T, k = x.shape[0], store.dims.n_expert_used
    ids = torch.full((T, k), -1, dtype=torch.int32, device=dev)
    w = torch.zeros((T, k), dtype=torch.float32, device=dev)
    out = torch.zeros((T, x.shape[1]), dtype=torch.float32, device=dev)
    store.block(layer, x, gate, gate_type, resid, out, ids, w)
    store.check()
    return out.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()


@pytest.mark.parametrize("name", list(SHAPES))
def test_fused_block_bit_identical(orc, lstk, dev, name):
    cfg, layers, routers, fused, multi = pools(name)
    rng = np.random.default_rng(7)
    for rep in range(6):
        layer = rep % 2
        x = synth.activations(rng, 1, cfg["h"])
        resid = synth.activations(rng, 1, cfg["h"])
        gate, gt = routers[layer], 1
        if rep == 5:  # F32 router weights
            gate, gt = routers[layer].astype(np.float32) * np.float32(1.01), 0
        xd, rd, gd = to_dev(x, dev), to_dev(resid, dev), to_dev(gate, dev)
        a = run_block(fused, layer, xd, gd, gt, rd, dev)
        b = run_block(multi, layer, xd, gd, gt, rd, dev)
        for u, v in zip(a, b):
            assert np.array_equal(u, v), (name, rep)
        rids, rw, _, _ = orc.router(x, gate, gt, cfg["k"])
        assert np.array_equal(a[1], rids)
        E = cfg["E"]
        ref = orc.moe_ffn(x, rids, rw, resid, layers[layer][1].reshape(E, -1), layers[layer][2].reshape(E, -1),
                          layers[layer][3].reshape(E, -1), cfg["types"], cfg["f"])
        err = np.abs(a[0] - ref).max() / np.abs(ref - resid).max()
        assert err <= FFN_TOL, (name, rep, err)
    print(f"[fused {name}] bit-identical to the multi-kernel path over 6 tokens", flush=True)


@pytest.mark.parametrize("name", ["30b_q8", "mixed"])
def test_fused_ffn_given_slots_bit_identical(orc, lstk, dev, name):
    import torch
    cfg, layers, routers, fused, multi = pools(name)
    rng = np.random.default_rng(11)
    for rep in range(4):
        x = synth.activations(rng, 1, cfg["h"])
        resid = synth.activations(rng, 1, cfg["h"])
        slots = rng.choice(cfg["E"], cfg["k"], replace=False).astype(np.int32)[None]
        w = rng.uniform(0.05, 0.3, (1, cfg["k"])).astype(np.float32)
        outs = []
        for st in (fused, multi):
            o = torch.zeros((1, cfg["h"]), dtype=torch.float32, device=dev)
            st.ffn(rep % 2, to_dev(x, dev), to_dev(slots, dev), to_dev(w, dev), to_dev(resid, dev), o)
            st.check()
            outs.append(o.cpu().numpy())
        assert np.array_equal(outs[0], outs[1])


def test_fused_graph_replays(orc, lstk, dev):
    """Launch counters and flags carry over graph replays: every replay of a captured two-layer step,
    with new inputs copied in between, equals the multi-kernel result of the same inputs."""
    import torch
    cfg, layers, routers, fused, multi = pools("30b_q8")
    h = cfg["h"]
    x = [torch.zeros((1, h), device=dev) for _ in range(2)]
    resid = [torch.zeros((1, h), device=dev) for _ in range(2)]
    out = [torch.zeros((1, h), device=dev) for _ in range(2)]
    ids = [torch.zeros((1, 8), dtype=torch.int32, device=dev) for _ in range(2)]
    w = [torch.zeros((1, 8), device=dev) for _ in range(2)]
    gates = [to_dev(r, dev) for r in routers]

    def step():
        for l in range(2):
            fused.block(l, x[l], gates[l], 1, resid[l], out[l], ids[l], w[l])

    step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    rng = np.random.default_rng(5)
    for rep in range(5):
        xs = [synth.activations(rng, 1, h) for _ in range(2)]
        rs = [synth.activations(rng, 1, h) for _ in range(2)]
        for l in range(2):
            x[l].copy_(to_dev(xs[l], dev))
            resid[l].copy_(to_dev(rs[l], dev))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        fused.check()
        for l in range(2):
            ref = run_block(multi, l, to_dev(xs[l], dev), gates[l], 1, to_dev(rs[l], dev), dev)
            assert np.array_equal(out[l].cpu().numpy(), ref[0]), (rep, l)
            assert np.array_equal(ids[l].cpu().numpy(), ref[1]), (rep, l)


def test_fused_streaming_single_token_matches_resident(orc, lstk, dev):
    """Decode through a streaming pool that evicts on every step: acquire, fused ffn, release."""
    import torch
    import localstack_amd as L
    cfg, layers, routers, fused, multi = pools("tiny")
    os.environ["LSTK_FUSED_DECODE"] = "1"
    try:
        st = L.ExpertStore(2, cfg["h"], cfg["f"], cfg["E"], cfg["k"], 1, layers, pool_bytes=1,
                           min_slots=2 * cfg["k"] + 2, streaming=True)
    finally:
        del os.environ["LSTK_FUSED_DECODE"]
    rng = np.random.default_rng(3)
    for rep in range(8):
        l = rep % 2
        x = synth.activations(rng, 1, cfg["h"])
        resid = synth.activations(rng, 1, cfg["h"])
        rids, rw, _, _ = orc.router(x, routers[l], 1, cfg["k"])
        slots = st.acquire(l, rids)
        o = torch.zeros((1, cfg["h"]), device=dev)
        st.ffn(l, to_dev(x, dev), to_dev(slots, dev), to_dev(rw, dev), to_dev(resid, dev), o)
        st.release_all()
        st.check()
        ref = run_block(multi, l, to_dev(x, dev), to_dev(routers[l], dev), 1, to_dev(resid, dev), dev)
        assert np.array_equal(o.cpu().numpy(), ref[0]), rep
    assert st.stats()["misses"] > 0
