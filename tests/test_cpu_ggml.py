"""The timed CPU baseline (oracle/cpu_ggml.c, a SIMD restatement of ggml's CPU algorithm) against the
oracle on the same inputs: identical routing, outputs within the MoE bar (2e-3 of the largest
|out - resid|; only f32 summation order differs, and with it the rare activation value that rounds to
the other side of a quantization step), for Q8_0 and Q4_K experts, one token and a batch."""
import numpy as np
import pytest

import oracle
from oracle import cpu_ggml
from localstack_amd import synth


@pytest.mark.parametrize("wtype,h,f,E,k,T", [(8, 2048, 768, 128, 8, 1), (8, 2048, 768, 128, 8, 8),
                                               (12, 2048, 768, 128, 8, 1), (12, 2048, 768, 32, 8, 64),
                                               (8, 256, 512, 8, 2, 16)])
def test_cpu_baseline_matches_oracle(orc, wtype, h, f, E, k, T):
    rng = np.random.default_rng(h + f + E + T + wtype)
    up, gate, down = (synth.experts(rng, wtype, E, f, h), synth.experts(rng, wtype, E, f, h),
                      synth.experts(rng, wtype, E, h, f))
    router = synth.router_f16(rng, E, h)
    x = synth.activations(rng, T, h)
    resid = synth.activations(rng, T, h)
    out, ids, w = cpu_ggml.moe_block(x, router, up, gate, down, wtype, resid, E, f, k)
    rids, rw, _, _ = oracle.router(x, router, oracle.TYPE_F16, k)
    np.testing.assert_array_equal(ids, rids)
    assert np.max(np.abs(w - rw)) <= 1e-6
    ref = oracle.moe_ffn(x, rids, rw, resid, up.reshape(E, -1), gate.reshape(E, -1), down.reshape(E, -1), (wtype,) * 3, f)
    err = np.abs(out - ref).max() / np.abs(ref - resid).max()
    print(f"cpu baseline ({cpu_ggml.isa()}) vs oracle: rel max err {err:.2e}")
    assert err <= 2e-3


AVX2_CHECK = """
import sys
import numpy as np
sys.path.insert(0, ROOT)
import oracle
from oracle import cpu_ggml
from localstack_amd import synth
assert cpu_ggml.isa() == "avx2"
for wt in (8, 12):
    rng = np.random.default_rng(wt)
    E, f, h, k, T = 16, 512, 1024, 4, 3
    up, gate, down = synth.experts(rng, wt, E, f, h), synth.experts(rng, wt, E, f, h), synth.experts(rng, wt, E, h, f)
    router, x, r = synth.router_f16(rng, E, h), synth.activations(rng, T, h), synth.activations(rng, T, h)
    out, ids, w = cpu_ggml.moe_block(x, router, up, gate, down, wt, r, E, f, k)
    rids, rw, _, _ = oracle.router(x, router, oracle.TYPE_F16, k)
    assert (ids == rids).all()
    ref = oracle.moe_ffn(x, rids, rw, r, up.reshape(E, -1), gate.reshape(E, -1), down.reshape(E, -1), (wt,) * 3, f)
    assert np.abs(out - ref).max() / np.abs(ref - r).max() <= 2e-3
print("ok")
"""


def test_cpu_baseline_avx2_path_matches_oracle(orc):
    """The AVX2 fallback (hosts without AVX-512 VNNI), run in a child process with LSTK_CPU_ISA=avx2."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, LSTK_CPU_ISA="avx2")
    r = subprocess.run([sys.executable, "-c", AVX2_CHECK.replace("ROOT", repr(root))], env=env, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stderr[-2000:]
