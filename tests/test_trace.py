"""Routing-trace format and expert-cache simulation against the reference's recorded trace (CPU only).

The fixture is the LSTKRTE1 trace the reference engine wrote for Qwen3-30B-A3B (18 prompt + 200
sampled tokens, 48 layers, 128 experts, top-8), with the figures the reference published for it
(docs/runs/Qwen3-30B-A3B-UD-Q2_K_XL.md:30-43, made by tests/golden/make_trace_fixture.py). The
simulators must reproduce every published LRU and Belady hit rate and LRU miss count to the printed
precision, and the product's own pool bookkeeping must replay a layer with exactly the LRU's hits.
"""
import os

import numpy as np
import pytest

from localstack_amd import trace

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "routing_trace_30b_a3b_ud_q2_k_xl.npz")


@pytest.fixture(scope="module")
def recorded():
    z = np.load(GOLDEN)
    n_layer, n_expert, k = (int(v) for v in z["header"])
    ids = z["ids"].astype(np.int32)
    steps, off = [], 0
    for n in z["steps"]:
        m = n_layer * int(n) * k
        steps.append(ids[off:off + m].reshape(n_layer, int(n), k))
        off += m
    raw = trace.encode_trace(n_layer, n_expert, k, steps)
    return raw, z


def test_format_round_trip(recorded, tmp_path):
    raw, z = recorded
    n_layer, n_expert, k, steps = trace.parse_trace(raw)
    assert (n_layer, n_expert, k) == (48, 128, 8)
    assert [s.shape[1] for s in steps] == list(z["steps"])
    assert trace.encode_trace(n_layer, n_expert, k, steps) == raw
    # a truncated final step is dropped, earlier steps survive
    assert len(trace.parse_trace(raw[:-5])[3]) == len(steps) - 1
    p = tmp_path / "t.bin"
    p.write_bytes(raw)
    _, _, _, seqs = trace.read_trace(p)
    assert max(len(s) for s in seqs) == int(z["tokens"])
    with pytest.raises(ValueError):
        trace.parse_trace(b"LSTKRTE2" + raw[8:])


def test_published_cache_table(recorded):
    raw, z = recorded
    n_layer, n_expert, k, steps = trace.parse_trace(raw)
    seqs = trace.per_layer_sets(n_layer, steps)
    overlap, hot25, hot50 = trace.locality(n_expert, k, seqs)
    assert (round(overlap, 1), round(hot25, 1), round(hot50, 1)) == (float(z["overlap"]), float(z["hot25"]),
                                                                     float(z["hot50"]))
    rows = trace.cache_table(n_expert, k, seqs)
    assert [r[0] for r in rows] == list(z["slots"])
    assert [round(r[1], 1) for r in rows] == list(z["lru"])
    assert [round(r[2], 1) for r in rows] == list(z["belady"])
    assert [round(r[3], 1) for r in rows] == list(z["lru_misses_per_token"])


@pytest.mark.parametrize("layer,cap", [(0, 16), (17, 32), (47, 48)])
def test_pool_is_the_lru(lstk, recorded, layer, cap):
    raw, _ = recorded
    n_layer, n_expert, k, steps = trace.parse_trace(raw)
    seq = trace.per_layer_sets(n_layer, steps)[layer]
    assert trace.pool_hits(seq, cap, n_expert) == trace.sim_lru(seq, cap)
