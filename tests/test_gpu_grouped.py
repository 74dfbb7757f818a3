"""GPU parity of the grouped (prefill) path through the C ABI: the permutation kernel against the
oracle's stable counting sort (bit-exact), and the MFMA expert products against the oracle's ggml
semantics (Q4_K weights x Q8_K activations, integer block sums exact on both sides).

Bar: permutation counts / offsets / order bit-exact; MoE output within FFN_TOL of the oracle relative
to the largest |out - resid| (only f32 summation order and expf differ); repeated calls bit-identical.
"""
import numpy as np
import pytest

from localstack_amd import synth

pytestmark = pytest.mark.gpu

Q8_0, Q4_K = 8, 12
FFN_TOL = 2e-3
_cache = {}


def model(name):
    if name in _cache:
        return _cache[name]
    import localstack_amd as L
    cfg = {
        # Qwen3-30B-A3B MoE layer, Q4_K experts (the 512-token prefill config)
        "30b_q4": dict(h=2048, f=768, E=128, k=8, types=(Q4_K,) * 3, n_batch=512),
        # small Q4_K layer: 16 experts, top-4, 256 x 512
        "small_q4": dict(h=256, f=512, E=16, k=4, types=(Q4_K,) * 3, n_batch=256),
        # Qwen3-235B-A22B expert shape (h 4096, f 1536, top-8; 16 experts): gate/up over 16 super-blocks,
        # down over 6, 24 and 32 row blocks per item
        "235b_q4": dict(h=4096, f=1536, E=16, k=8, types=(Q4_K,) * 3, n_batch=128),
        # top-64 of 64 experts: the largest k the kernels take
        "k64": dict(h=256, f=256, E=64, k=64, types=(Q8_0,) * 3, n_batch=64),
    }[name]
    rng = np.random.default_rng(sum(map(ord, name)) + 7)
    t = cfg["types"]
    lb = (synth.experts(rng, t[0], cfg["E"], cfg["f"], cfg["h"]), synth.experts(rng, t[1], cfg["E"], cfg["f"], cfg["h"]),
          synth.experts(rng, t[2], cfg["E"], cfg["h"], cfg["f"]))
    router = synth.zipf_router_f16(rng, cfg["E"], cfg["h"])
    store = L.ExpertStore(1, cfg["h"], cfg["f"], cfg["E"], cfg["k"], cfg["n_batch"], [(t,) + lb])
    _cache[name] = (cfg, lb, router, store)
    return _cache[name]


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def gpu_permute(store, bins, nb, dev):
    import torch
    T, k = bins.shape
    counts = torch.full((nb,), -1, dtype=torch.int32, device=dev)
    offsets = torch.full((nb + 1,), -1, dtype=torch.int32, device=dev)
    perm = torch.full((T * k,), -1, dtype=torch.int32, device=dev)
    store.permute(to_dev(bins, dev), nb, counts, offsets, perm)
    store.check()
    return counts.cpu().numpy(), offsets.cpu().numpy(), perm.cpu().numpy()


def distinct_rows(rng, T, k, nb):
    return np.stack([rng.choice(nb, k, replace=False) for _ in range(T)]).astype(np.int32)


@pytest.mark.parametrize("name,T,nb", [("30b_q4", 1, 128), ("30b_q4", 7, 128), ("30b_q4", 64, 128), ("30b_q4", 333, 1024),
                                       ("30b_q4", 512, 128), ("small_q4", 256, 16), ("small_q4", 100, 1000),
                                       ("k64", 64, 64), ("k64", 3, 1024)])
def test_permute_bit_exact(orc, lstk, dev, name, T, nb):
    cfg, _, _, store = model(name)
    rng = np.random.default_rng(T * 31 + nb)
    bins = distinct_rows(rng, T, cfg["k"], nb)
    counts, offsets, perm = gpu_permute(store, bins, nb, dev)
    rc, ro, rp, _ = orc.permute(bins, nb)
    print(f"[permute {name} T={T} nb={nb}] max count {rc.max()}", flush=True)
    assert np.array_equal(counts, rc)
    assert np.array_equal(offsets, ro)
    assert np.array_equal(perm, rp)


def test_permute_zipf_routing_and_edge_bins(orc, lstk, dev):
    import torch
    cfg, _, router, store = model("30b_q4")
    rng = np.random.default_rng(3)
    x = synth.activations(rng, 512, cfg["h"], bias_unit=True)
    ids, _, _, _ = orc.router(x, router, 1, 8)
    for bins, nb in ((ids, 128), (np.zeros((512, 8), np.int32), 1), (np.full((40, 8), 1023, np.int32), 1024),
                     (rng.integers(0, 3, (300, 8)).astype(np.int32), 3)):  # repeats within a token too
        counts, offsets, perm = gpu_permute(store, bins, nb, dev)
        rc, ro, rp, _ = orc.permute(bins, nb)
        assert np.array_equal(counts, rc) and np.array_equal(offsets, ro) and np.array_equal(perm, rp)
    # a bin out of range is clamped and reported, not followed out of bounds
    bad = distinct_rows(rng, 4, 8, 128)
    bad[1, 3] = 500
    c = torch.zeros(128, dtype=torch.int32, device=dev)
    o = torch.zeros(129, dtype=torch.int32, device=dev)
    p = torch.zeros(32, dtype=torch.int32, device=dev)
    store.permute(to_dev(bad, dev), 128, c, o, p)
    with pytest.raises(lstk.LstkError) as ei:
        store.check()
    assert ei.value.code == lstk.E_BADID


def oracle_ffn(orc, cfg, lb, x, ids, w, resid):
    E = cfg["E"]
    return orc.moe_ffn(x, ids, w, resid, lb[0].reshape(E, -1), lb[1].reshape(E, -1), lb[2].reshape(E, -1), cfg["types"],
                       cfg["f"])


def ffn_err(got, ref, resid):
    return np.abs(got - ref).max() / max(np.abs(ref - resid).max(), 1e-12)


@pytest.mark.parametrize("name,T", [("30b_q4", 64), ("30b_q4", 100), ("30b_q4", 512), ("small_q4", 256), ("small_q4", 65),
                                    ("235b_q4", 64), ("235b_q4", 128)])
def test_grouped_ffn_matches_oracle(orc, lstk, dev, name, T):
    import torch
    cfg, lb, router, store = model(name)
    rng = np.random.default_rng(500 + T)
    x = synth.activations(rng, T, cfg["h"], bias_unit=True)
    resid = synth.activations(rng, T, cfg["h"])
    ids, w, _, _ = orc.router(x, router, 1, cfg["k"])
    out = torch.zeros((T, cfg["h"]), dtype=torch.float32, device=dev)
    store.ffn(0, to_dev(x, dev), to_dev(ids, dev), to_dev(w, dev), to_dev(resid, dev), out)
    store.check()
    got = out.cpu().numpy()
    ref = oracle_ffn(orc, cfg, lb, x, ids, w, resid)
    err = ffn_err(got, ref, resid)
    counts = np.bincount(ids.ravel(), minlength=cfg["E"])
    print(f"[grouped ffn {name} T={T}] rel max err {err:.3e}; tokens per expert max {counts.max()} "
          f"active {np.count_nonzero(counts)}", flush=True)
    assert np.isfinite(got).all()
    assert err <= FFN_TOL


def test_grouped_block_matches_oracle_and_repeats(orc, lstk, dev):
    import torch
    cfg, lb, router, store = model("30b_q4")
    T = 512
    rng = np.random.default_rng(901)
    x = synth.activations(rng, T, cfg["h"], bias_unit=True)
    resid = synth.activations(rng, T, cfg["h"])
    xd, rd, gd = to_dev(x, dev), to_dev(resid, dev), to_dev(router, dev)
    outs = []
    for _ in range(2):
        ids = torch.zeros((T, 8), dtype=torch.int32, device=dev)
        w = torch.zeros((T, 8), dtype=torch.float32, device=dev)
        out = torch.zeros((T, cfg["h"]), dtype=torch.float32, device=dev)
        store.block(0, xd, gd, 1, rd, out, ids, w)
        store.check()
        outs.append(out.cpu())
    assert torch.equal(outs[0], outs[1])
    rids, rw, _, _ = orc.router(x, router, 1, 8)
    assert np.array_equal(ids.cpu().numpy(), rids)
    ref = oracle_ffn(orc, cfg, lb, x, rids, rw, resid)
    err = ffn_err(outs[0].numpy(), ref, resid)
    print(f"[grouped block 30b_q4 T=512] rel max err {err:.3e}", flush=True)
    assert err <= FFN_TOL
