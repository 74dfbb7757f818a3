"""Converts the reference's recorded routing trace into tests/golden/routing_trace_30b_a3b_ud_q2_k_xl.npz.

Input: docs/runs/Qwen3-30B-A3B-UD-Q2_K_XL.trace.bin of the reference (a data file: the LSTKRTE1 trace
its engine wrote for 18 prompt + 200 sampled tokens of Qwen3-30B-A3B, src/engine.cpp:26-29), read as
bytes. Output: the header, each step's token count and every expert id (int8: ids are < 128 or -1),
compressed. The expected cache-simulation figures are the reference's published ones for this trace
(docs/runs/Qwen3-30B-A3B-UD-Q2_K_XL.md:30-43), copied as data into EXPECTED below.

    python3 tests/golden/make_trace_fixture.py [/root/reference]
"""
import os
import struct
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "routing_trace_30b_a3b_ud_q2_k_xl.npz")

# docs/runs/Qwen3-30B-A3B-UD-Q2_K_XL.md:30-43: per-layer cache of `slots` experts, hit rates in percent,
# LRU misses per token; tokens 218; consecutive-token overlap and hottest-expert coverage in percent
EXPECTED = {
    "tokens": 218, "overlap": 40.6, "hot25": 71.2, "hot50": 94.5,
    "slots": [16, 32, 48, 64, 80, 96],
    "lru": [53.8, 76.1, 86.5, 91.5, 93.7, 94.5],
    "belady": [72.9, 86.7, 91.9, 94.0, 94.5, 94.6],
    "lru_misses_per_token": [177.5, 91.9, 52.0, 32.5, 24.1, 21.2],
}


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    raw = open(os.path.join(ref, "docs/runs/Qwen3-30B-A3B-UD-Q2_K_XL.trace.bin"), "rb").read()
    assert raw[:8] == b"LSTKRTE1"
    n_layer, n_expert, k = struct.unpack_from("<iii", raw, 8)
    off, steps, ids = 20, [], []
    while off + 4 <= len(raw):
        (n,) = struct.unpack_from("<i", raw, off)
        need = 4 + 4 * n_layer * n * k
        if off + need > len(raw):
            break
        steps.append(n)
        ids.append(np.frombuffer(raw, "<i4", n_layer * n * k, off + 4))
        off += need
    ids = np.concatenate(ids)
    assert ids.min() >= -1 and ids.max() < 128
    np.savez_compressed(OUT, header=np.array([n_layer, n_expert, k], np.int32), steps=np.array(steps, np.int32),
                        ids=ids.astype(np.int8), **{k2: np.array(v) for k2, v in EXPECTED.items()})
    print(OUT, os.path.getsize(OUT), "bytes;", len(steps), "steps")


if __name__ == "__main__":
    main()
