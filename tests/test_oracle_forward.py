"""Pins the oracle's forward pass around the MoE block (oracle.c: or_dot_f16 .. or_qwen3_decode) without a GPU.

Nothing in the reference pins these values (its ggml dependency is absent and it commits no golden
logits), so each piece is held against what the mathematics fixes:
  - the F16 dot / mat-mul against float64 sums of the same fp16 values;
  - RMSNorm against its closed form in float64;
  - RoPE: identity at position 0, pair norms preserved, scores depending only on the position
    difference, and the float64 rotation by pos * base^(-2i/hd);
  - attention against a float64 softmax over the same fp16 cache, and a lone cell returning its V row;
  - the whole model against an independent float64 numpy forward of the same weights (dequantized
    experts, no activation rounding) at the logits tolerance, and prefill in one step against the same
    tokens fed one at a time (bit-identical: every row's arithmetic is independent of the step size).
"""
import numpy as np
import pytest

import oracle
from localstack_amd import synth

TINY = dict(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_vocab=1024, n_expert=8, n_expert_used=2,
            n_ff_exp=512, n_ctx_train=1024, rms_eps=1e-6, rope_freq_base=10000.0)


@pytest.fixture(scope="module")
def tiny():
    return synth.qwen3_weights(np.random.default_rng(1234), TINY, wtype=8)


def test_dot_f16_matches_float64():
    rng = np.random.default_rng(0)
    for n in (32, 256, 1000, 4096):
        w = rng.standard_normal(n).astype(np.float16)
        x = rng.standard_normal(n).astype(np.float16)
        exact = float(np.dot(w.astype(np.float64), x.astype(np.float64)))
        got = oracle.dot_f16(w, x)
        assert abs(got - exact) <= 1e-5 * np.sum(np.abs(w.astype(np.float64) * x.astype(np.float64))), n


def test_matmul_rounds_activations_to_fp16():
    rng = np.random.default_rng(1)
    W = rng.standard_normal((16, 96)).astype(np.float16)
    x = rng.standard_normal((3, 96)).astype(np.float32)
    want = x.astype(np.float16).astype(np.float64) @ W.astype(np.float64).T
    got = oracle.matmul_f16(W, x)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-5)
    # and it is not the f32-activation product
    assert np.max(np.abs(got - x.astype(np.float64) @ W.astype(np.float64).T)) > 1e-5


def test_rms_norm_closed_form():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(2048) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 2048).astype(np.float32)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w
    np.testing.assert_allclose(oracle.rms_norm(x, w, 1e-6), want, rtol=2e-6, atol=0)
    np.testing.assert_allclose(oracle.rms_norm(x, None, 1e-6), want / w, rtol=2e-6, atol=0)


def test_rope_neox_properties():
    rng = np.random.default_rng(3)
    hd, base = 64, 10000.0
    ts = np.float32(base) ** np.float32(-2.0 / hd)
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.standard_normal(hd).astype(np.float32)
    np.testing.assert_array_equal(oracle.rope_neox(q, 0, ts), q)
    for pos in (1, 7, 40):
        y = oracle.rope_neox(q, pos, ts)
        half = hd // 2
        np.testing.assert_allclose(y[:half] ** 2 + y[half:] ** 2, q[:half] ** 2 + q[half:] ** 2, rtol=1e-5, atol=1e-6)
        theta = pos * base ** (-2.0 * np.arange(half) / hd)
        q64 = q.astype(np.float64)
        want = np.concatenate([q64[:half] * np.cos(theta) - q64[half:] * np.sin(theta),
                               q64[:half] * np.sin(theta) + q64[half:] * np.cos(theta)])
        np.testing.assert_allclose(y, want, rtol=0, atol=2e-5 * max(1, pos))
    # scores depend on the position difference only
    s = [float(np.dot(oracle.rope_neox(q, m + d, ts), oracle.rope_neox(k, n + d, ts))) for (m, n, d) in
         ((9, 4, 0), (9, 4, 11), (9, 4, 30))]
    np.testing.assert_allclose(s, s[0], rtol=0, atol=2e-4)


def test_attention_row_matches_float64_softmax():
    rng = np.random.default_rng(4)
    hd, n, ld = 64, 37, 128
    q = rng.standard_normal(hd).astype(np.float32)
    K = rng.standard_normal((n, ld)).astype(np.float16)
    V = rng.standard_normal((n, ld)).astype(np.float16)
    scale = 1.0 / np.sqrt(hd)
    got = oracle.attn_row(q, K, V, scale)
    s = (K[:, :hd].astype(np.float64) @ q.astype(np.float16).astype(np.float64)) * scale
    p = np.exp(s - s.max())
    want = (p / p.sum()) @ V[:, :hd].astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)
    # a lone visible cell returns its V row exactly
    np.testing.assert_array_equal(oracle.attn_row(q, K[:1], V[:1], scale), V[0, :hd].astype(np.float32))


# ---- whole model ---------------------------------------------------------------------------

def _dequant_q8_0(raw, rows, cols):
    b = np.frombuffer(np.ascontiguousarray(raw).tobytes(), dtype=oracle.Q8_0_DTYPE).reshape(rows, cols // 32)
    return (b["d"].view(np.float16).astype(np.float64)[..., None] * b["qs"].astype(np.float64)).reshape(rows, cols)


def _np_forward(hp, w, tokens):
    """float64 restatement of qwen3_build_graph (src/qwen3.cpp:223-259) for one sequence from position 0."""
    h, hd, nh, nkv, E, k, f = (hp[n] for n in ("n_embd", "head_dim", "n_head", "n_head_kv", "n_expert", "n_expert_used",
                                                 "n_ff_exp"))
    eps, base = hp["rms_eps"], hp["rope_freq_base"]
    T = len(tokens)

    def rms(x, g):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * g

    def rope(x, pos):  # x [..., hd]
        half = hd // 2
        th = pos * base ** (-2.0 * np.arange(half) / hd)
        c, s = np.cos(th), np.sin(th)
        return np.concatenate([x[..., :half] * c - x[..., half:] * s, x[..., :half] * s + x[..., half:] * c], -1)

    f64 = lambda a: np.asarray(a).astype(np.float64)
    x = f64(w["tok_embd"])[tokens]
    ids_all = []
    for l, L in enumerate(w["layers"]):
        hn = rms(x, f64(L["attn_norm"]))
        q = (hn @ f64(L["wq"]).T).reshape(T, nh, hd)
        kk = (hn @ f64(L["wk"]).T).reshape(T, nkv, hd)
        v = (hn @ f64(L["wv"]).T).reshape(T, nkv, hd)
        q = rms(q, f64(L["q_norm"]))
        kk = rms(kk, f64(L["k_norm"]))
        pos = np.arange(T)[:, None, None]
        q, kk = rope(q, pos), rope(kk, pos)
        att = np.zeros((T, nh, hd))
        for t in range(T):
            for j in range(nh):
                g = j // (nh // nkv)
                s = kk[: t + 1, g] @ q[t, j] / np.sqrt(hd)
                p = np.exp(s - s.max())
                att[t, j] = (p / p.sum()) @ v[: t + 1, g]
        x = x + att.reshape(T, nh * hd) @ f64(L["wo"]).T
        if l == hp["n_layer"] - 1:
            x = x[-1:]
        hn = rms(x, f64(L["ffn_norm"]))
        logit = hn @ f64(L["gate_inp"]).T
        pr = np.exp(logit - logit.max(-1, keepdims=True))
        pr /= pr.sum(-1, keepdims=True)
        ids = np.argsort(-pr, axis=-1, kind="stable")[:, :k]
        wts = np.take_along_axis(pr, ids, -1)
        wts /= wts.sum(-1, keepdims=True)
        ids_all.append(ids)
        up = _dequant_q8_0(L["up"], E * f, h).reshape(E, f, h)
        gate = _dequant_q8_0(L["gate"], E * f, h).reshape(E, f, h)
        down = _dequant_q8_0(L["down"], E * h, f).reshape(E, h, f)
        out = np.zeros_like(x)
        for t in range(x.shape[0]):
            for j in range(k):
                e = ids[t, j]
                gg, uu = gate[e] @ hn[t], up[e] @ hn[t]
                out[t] += wts[t, j] * (down[e] @ (gg / (1 + np.exp(-gg)) * uu))
        x = x + out
    logits = rms(x[-1], f64(w["output_norm"])) @ f64(w["tok_embd"]).T
    return logits, ids_all


def test_forward_matches_float64_model(tiny):
    tokens = np.random.default_rng(5).integers(0, TINY["n_vocab"], 16)
    m = oracle.Qwen3(TINY, tiny, 64)
    logits, trace = m.decode(tokens, want_trace=True)
    want, ids = _np_forward(TINY, tiny, tokens)
    assert np.max(np.abs(logits - want)) <= 1e-2, np.max(np.abs(logits - want))
    assert int(np.argmax(logits)) == int(np.argmax(want))
    # routing agrees wherever the float64 model's k-th and (k+1)-th probabilities are not near-tied
    for l in range(TINY["n_layer"]):
        rows = trace[l] if l < TINY["n_layer"] - 1 else trace[l][-1:]
        np.testing.assert_array_equal(np.sort(rows, -1), np.sort(ids[l], -1))
    assert np.all(trace[-1][:-1] == -1)


def test_prefill_equals_token_by_token(tiny):
    tokens = np.random.default_rng(6).integers(0, TINY["n_vocab"], 12)
    a = oracle.Qwen3(TINY, tiny, 64)
    la = a.decode(tokens)
    b = oracle.Qwen3(TINY, tiny, 64)
    for t in tokens:
        lb = b.decode([t])
    np.testing.assert_array_equal(la, lb)
    assert len(a) == len(b) == 12
    # truncation rewinds the sequence: re-decoding the dropped tokens reproduces the logits
    a.truncate(7)
    np.testing.assert_array_equal(a.decode(tokens[7:]), la)


def test_context_full_is_an_error(tiny):
    m = oracle.Qwen3(TINY, tiny, 8)
    m.decode(np.arange(8))
    with pytest.raises(RuntimeError):
        m.decode([1])


def test_diff_logits_metric(orc):
    """src/main.cpp:195-207: max |d|, sqrt(sum d^2 / n), and the first argmax of each side."""
    mx, rms, ra, oa = orc.diff_logits(np.array([0.0, 1.0, 2.0, 2.0], np.float32), np.array([0.0, 1.5, 2.0, 3.0], np.float32))
    assert mx == 1.0 and abs(rms - np.sqrt((0.25 + 1.0) / 4)) < 1e-15 and ra == 2 and oa == 3
    assert orc.diff_logits([1.0, 1.0], [1.0, 1.0]) == (0.0, 0.0, 0, 0)


def test_layer_by_layer_equals_decode(orc):
    """run_layer over every layer + head + advance reproduces decode() bit for bit (ids too), so a
    layer-by-layer comparison checks the same oracle the whole-model tests use."""
    hp = dict(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_vocab=1024, n_expert=8, n_expert_used=2,
              n_ff_exp=512, n_ctx_train=1024, rms_eps=1e-6, rope_freq_base=10000.0)
    w = synth.qwen3_weights(np.random.default_rng(8), hp, wtype=8)
    a, b = orc.Qwen3(hp, w, 32), orc.Qwen3(hp, w, 32)
    feed = np.random.default_rng(9).integers(0, 1024, 6).astype(np.int32)
    for _ in range(3):
        la, ta = a.decode(feed, want_trace=True)
        x = w["tok_embd"][feed].astype(np.float32)
        tb = []
        for l in range(hp["n_layer"]):
            x, ids = b.run_layer(l, x)
            tb.append(ids)
        lb = b.head(x[-1])
        b.advance(len(feed))
        assert np.array_equal(la, lb) and np.array_equal(ta, np.array(tb)) and len(a) == len(b)
        feed = np.array([np.argmax(la)], np.int32)
