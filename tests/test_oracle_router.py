"""The oracle's router (src/qwen3.cpp:175-192) and permutation, pinned by float64 brute force,
invariants and special cases (no GPU)."""
import numpy as np
import pytest

from localstack_amd import synth


def make(seed, T, h, E, gate_type=1):
    rng = np.random.default_rng(seed)
    x = synth.activations(rng, T, h)
    w = synth.router_f16(rng, E, h)
    if gate_type == 0:
        w = w.astype(np.float32) + rng.standard_normal(w.shape).astype(np.float32) * np.float32(1e-4)
    return x, w


@pytest.mark.parametrize("gate_type", [1, 0])
@pytest.mark.parametrize("shape", [(7, 256, 8), (5, 2048, 128), (3, 4096, 128)])
def test_logits_match_float64(orc, shape, gate_type):
    T, h, E = shape
    x, w = make(10, T, h, E, gate_type)
    got = orc.router_logits(x, w, gate_type)
    xr = x.astype(np.float16).astype(np.float64) if gate_type == 1 else x.astype(np.float64)
    ref = xr @ w.astype(np.float64).T
    scale = np.abs(xr) @ np.abs(w.astype(np.float64)).T
    assert np.all(np.abs(got - ref) <= 4e-7 * scale + 1e-30)
    if gate_type == 1:
        # F16 weights see fp16-rounded activations (a dropped rounding is caught)
        ref_unrounded = x.astype(np.float64) @ w.astype(np.float64).T
        assert np.abs(got - ref_unrounded).max() > np.abs(got - ref).max()


def brute_router(logits, k):
    l = logits.astype(np.float64)
    p = np.exp(l - l.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ids = np.argsort(-l, axis=1, kind="stable")[:, :k]
    sel = np.take_along_axis(p, ids, axis=1)
    return ids, sel / np.maximum(sel.sum(axis=1, keepdims=True), 6.103515625e-5)


@pytest.mark.parametrize("shape", [(64, 256, 8, 2), (200, 2048, 128, 8), (16, 4096, 128, 8), (9, 256, 8, 8),
                                   (9, 2048, 128, 1), (4, 256, 256, 64)])
def test_router_matches_brute_force(orc, shape):
    T, h, E, k = shape
    x, w = make(11, T, h, E)
    ids, wt, logits, probs = orc.router(x, w, 1, k)
    bids, bw = brute_router(logits, k)
    # where the k-th and (k+1)-th logits are separated, the selection and order are forced
    srt = np.sort(logits, axis=1)[:, ::-1]
    gap = srt[:, k - 1] - (srt[:, k] if k < E else -np.inf)
    clear = gap > 1e-6
    assert np.array_equal(ids[clear], bids[clear])
    assert np.allclose(wt, bw, rtol=1e-5, atol=1e-7)
    assert np.allclose(probs.sum(axis=1), 1.0, atol=1e-5)


def test_router_invariants(orc):
    T, h, E, k = 300, 2048, 128, 8
    x, w = make(12, T, h, E)
    ids, wt, logits, probs = orc.router(x, w, 1, k)
    for t in range(T):
        assert len(set(ids[t])) == k
        sel = logits[t, ids[t]]
        assert np.all(np.diff(sel) <= 0)  # descending
        rest = np.delete(logits[t], ids[t])
        assert sel.min() >= rest.max()
    assert np.allclose(wt.sum(axis=1), 1.0, atol=1e-6)
    # the clamp never binds: the top-k mass is at least k/E
    assert (probs[np.arange(T)[:, None], ids].sum(axis=1) >= k / E * 0.999).all()


def test_router_ties_go_to_lower_id(orc):
    h, E, k = 256, 8, 3
    x = np.ones((1, h), np.float32)
    w = np.zeros((E, h), np.float16)
    w[[1, 4, 6], :] = np.float16(0.01)   # three equal maxima
    w[[2, 5], :] = np.float16(0.005)
    ids, wt, _, _ = orc.router(x, w, 1, k)
    assert list(ids[0]) == [1, 4, 6]
    assert np.allclose(wt[0], 1 / 3, atol=1e-7)
    ids, _, _, _ = orc.router(x, w, 1, 5)
    assert list(ids[0]) == [1, 4, 6, 2, 5]


def test_router_k_equals_E_and_k1(orc):
    x, w = make(13, 6, 256, 8)
    ids, wt, logits, probs = orc.router(x, w, 1, 8)
    assert all(sorted(r) == list(range(8)) for r in ids)
    assert np.allclose(wt, np.take_along_axis(probs, ids, axis=1), rtol=1e-6)
    ids1, wt1, _, _ = orc.router(x, w, 1, 1)
    assert np.array_equal(ids1[:, 0], np.argmax(logits, axis=1)) and np.all(wt1 == 1.0)


def stable_sort_reference(bins, n_bins):
    pairs = sorted(range(bins.size), key=lambda p: (bins.flat[p], p))
    counts = np.bincount(bins.ravel(), minlength=n_bins)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    return counts, offsets, np.array(pairs, np.int32), np.nonzero(counts)[0]


@pytest.mark.parametrize("T,k,nb", [(1, 8, 128), (8, 8, 128), (512, 8, 128), (33, 2, 8), (70, 8, 1024), (5, 64, 256)])
def test_permute_is_stable_counting_sort(orc, T, k, nb):
    rng = np.random.default_rng(T * 1000 + k)
    bins = np.stack([rng.choice(nb, k, replace=False) for _ in range(T)]).astype(np.int32)
    counts, offsets, perm, active = orc.permute(bins, nb)
    c2, o2, p2, a2 = stable_sort_reference(bins, nb)
    assert np.array_equal(counts, c2) and np.array_equal(offsets, o2)
    assert np.array_equal(perm, p2) and np.array_equal(active, a2)
    # a bijection whose bins are contiguous and token-major inside each bin
    assert sorted(perm.tolist()) == list(range(T * k))
    for b in active:
        seg = perm[offsets[b]:offsets[b + 1]]
        assert np.all(bins.ravel()[seg] == b) and np.all(np.diff(seg) > 0)


def test_permute_zipf_skew(orc):
    rng = np.random.default_rng(14)
    w = synth.zipf_router_f16(rng, 128, 2048)
    x = synth.activations(rng, 512, 2048, bias_unit=True)
    ids, _, _, _ = orc.router(x, w, 1, 8)
    counts, offsets, perm, active = orc.permute(ids, 128)
    assert counts.max() > 200 and (counts == 0).sum() > 10  # skewed load
    c2, o2, p2, a2 = stable_sort_reference(ids, 128)
    assert np.array_equal(perm, p2)
