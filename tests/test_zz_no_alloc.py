"""lstk_moe_block_noalloc (the MoE block with its scratch in the library's fixed per-device array)
against lstk_moe_block on the same pool and inputs, through the C ABI: bit-identical ids, weights and
outputs on two calls in a row, the second with fewer tokens (the array keeps the first call's
contents), at the 30B-A3B shape with Q8_0 experts and at a Q4_K shape; and the size limit."""
import numpy as np
import pytest

from localstack_amd import synth

pytestmark = pytest.mark.gpu


def _inputs(torch, dev, rng, T, h):
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return d(synth.activations(rng, T, h)), d(synth.activations(rng, T, h))


def _outs(torch, dev, T, h, k):
    return (torch.full((T, h), np.nan, dtype=torch.float32, device=dev),
            torch.full((T, k), -7, dtype=torch.int32, device=dev),
            torch.full((T, k), np.nan, dtype=torch.float32, device=dev))


@pytest.mark.parametrize("wtype,h,f,E,k,n_batch,calls", [
    (8, 2048, 768, 128, 8, 16, (8, 1)),     # 30B-A3B shape, Q8_0: batch then single token
    (12, 2048, 768, 128, 8, 64, (48, 5)),  # Q4_K experts, batch sizes below the grouped threshold
    (8, 256, 512, 8, 2, 16, (16, 3)),       # tiny qwen3moe shape
])
def test_noalloc_block_matches_block(lstk, dev, wtype, h, f, E, k, n_batch, calls):
    import torch
    rng = np.random.default_rng(97 + h + wtype)
    types = (wtype,) * 3
    up, gate, down = (synth.experts(rng, wtype, E, f, h), synth.experts(rng, wtype, E, f, h),
                      synth.experts(rng, wtype, E, h, f))
    router = torch.from_numpy(synth.router_f16(rng, E, h)).to(dev)
    store = lstk.ExpertStore(2, h, f, E, k, n_batch, [(types, up, gate, down)] * 2)
    L = lstk.lib()
    for i, T in enumerate(calls):
        layer = i % 2
        x, resid = _inputs(torch, dev, rng, T, h)
        out_a, ids_a, w_a = _outs(torch, dev, T, h, k)
        out_b, ids_b, w_b = _outs(torch, dev, T, h, k)
        rc = L.lstk_moe_block(store._h, layer, x.data_ptr(), router.data_ptr(), 1, resid.data_ptr(), out_a.data_ptr(),
                              ids_a.data_ptr(), w_a.data_ptr(), T, None)
        assert rc == 0, L.lstk_last_error()
        rc = L.lstk_moe_block_noalloc(store._h, layer, x.data_ptr(), router.data_ptr(), 1, resid.data_ptr(),
                                      out_b.data_ptr(), ids_b.data_ptr(), w_b.data_ptr(), T, None)
        assert rc == 0, L.lstk_last_error()
        torch.cuda.synchronize()
        store.check()
        print(f"noalloc call {i}: T={T} h={h} type={wtype}", flush=True)
        assert torch.equal(ids_a, ids_b), f"call {i} (T={T}): router ids differ"
        assert torch.equal(w_a, w_b), f"call {i} (T={T}): router weights differ"
        assert torch.isfinite(out_b).all()
        assert torch.equal(out_a, out_b), f"call {i} (T={T}): outputs differ, max {float((out_a - out_b).abs().max())}"
    store.close()


def test_noalloc_rejects_tokens_beyond_the_fixed_scratch(lstk, dev):
    import torch
    h, f, E, k = 2048, 768, 128, 8
    rng = np.random.default_rng(5)
    w = synth.experts(rng, 8, E, f, h)
    wd = synth.experts(rng, 8, E, h, f)
    store = lstk.ExpertStore(1, h, f, E, k, 256, [((8,) * 3, w, w, wd)])
    T = 200  # 200 * 93184 bytes > 16 MiB
    router = torch.from_numpy(synth.router_f16(rng, E, h)).to(dev)
    x = torch.zeros((T, h), dtype=torch.float32, device=dev)
    out = torch.zeros_like(x)
    ids = torch.zeros((T, k), dtype=torch.int32, device=dev)
    wt = torch.zeros((T, k), dtype=torch.float32, device=dev)
    L = lstk.lib()
    rc = L.lstk_moe_block_noalloc(store._h, 0, x.data_ptr(), router.data_ptr(), 1, x.data_ptr(), out.data_ptr(),
                                  ids.data_ptr(), wt.data_ptr(), T, None)
    assert rc == lstk.E_INVALID and b"fixed" in L.lstk_last_error()
    torch.cuda.synchronize()
    store.close()
