"""lstk_dequant_f16 (include/lstk_gguf.h) and the dense-tensor loader on the CPU: no GPU call is made.

The reference maps dense tensors of any ggml type into its graph (src/qwen3.cpp:52-89); the forward pass
here multiplies F16 matrices, so quantized dense tensors are expanded to F16 on load. ggml (the unvendored
llama.cpp submodule, commit 23b0202a) is absent and the reference holds no golden vectors for these
formats, so each format is pinned as follows:
- F32 -> F16 rounding: numpy's float16 conversion (round to nearest even) over random values at every
  scale, exact ties, the subnormal range, the overflow boundary, infinities and NaN;
- Q8_0 and Q4_K: the oracle's dequantizers (themselves pinned against the reference's own Q8_0 writer,
  tools/make_tiny_moe.py, and closed forms) rounded once to fp16;
- Q5_K: with every high bit clear it is Q4_K of the same header, scales and nibbles (the oracle again);
  each of its 256 high bits, set alone, moves exactly one value by 16 d sc: value 32 j + l for bit j of
  qh[l] (ggml's block_q5_K layout);
- Q6_K: d = 1 and unit scales give q - 32 exactly, which pins where each value's 4 low and 2 high bits
  sit (every bit probed alone) and the 16-value scale groups; power-of-two d makes the products exact.
"""
import numpy as np
import pytest

import oracle
from localstack_amd import synth

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 8, 12, 13, 14


def f16(lstk, type_, blocks, n):
    return lstk.dequant_f16(type_, np.ascontiguousarray(blocks).view(np.uint8).ravel(), n)


def test_f32_rounding_matches_round_to_nearest_even(lstk):
    rng = np.random.default_rng(1)
    xs = [rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000)]
    # exact halfway points between neighbouring fp16 values (normal and subnormal), and their neighbours
    h = np.arange(0, 0x7c00, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    h2 = np.arange(1, 0x7c01, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    mid = ((h + h2) / 2).astype(np.float32)
    xs += [mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(np.inf))]
    edges = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, 70000.0, 3e38, np.inf, -np.inf, 2.0 ** -24,
                      2.0 ** -25, np.nextafter(np.float32(2.0 ** -25), np.float32(1)), 2.0 ** -26, 2.0 ** -14,
                      np.nextafter(np.float32(2.0 ** -14), np.float32(0)), 1e-45], np.float32)
    xs += [edges, -edges]
    x = np.concatenate(xs).astype(np.float32)
    got = f16(lstk, F32, x, x.size)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16)
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
    nan = f16(lstk, F32, np.array([np.nan], np.float32), 1)
    assert np.isnan(nan[0])


def test_f16_is_copied(lstk):
    x = np.random.default_rng(2).integers(0, 65536, 1000).astype(np.uint16)
    np.testing.assert_array_equal(f16(lstk, F16, x, 1000).view(np.uint16), x)


def test_q8_0_matches_oracle(lstk):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((16, 512)) * 10.0 ** rng.uniform(-6, 2, (16, 1))).astype(np.float32)
    blocks = oracle.quantize_q8_0_ref(x)
    blocks["d"][0, 0] = 0x0001  # a subnormal scale
    blocks["d"][0, 1] = 0x7bff  # the largest finite scale: products overflow fp16
    want = oracle.dequant(blocks, oracle.TYPE_Q8_0)
    with np.errstate(over="ignore"):
        want = want.astype(np.float16)
    got = f16(lstk, Q8_0, blocks, x.size).reshape(16, 512)
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


def q4_k_blocks(rng, nb):
    b = synth.q4_k_random(rng, 1, 256 * nb, d0=rng.uniform(1e-5, 1e-1)).view(oracle.Q4_K_DTYPE).copy()
    return b


def test_q4_k_matches_oracle(lstk):
    rng = np.random.default_rng(4)
    for _ in range(8):
        b = q4_k_blocks(rng, 24)
        want = oracle.dequant(b, oracle.TYPE_Q4_K).astype(np.float16)
        got = f16(lstk, Q4_K, b, 24 * 256)
        np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


def q5_k_from_q4_k(b4, qh):
    """Q5_K blocks with the Q4_K blocks' d, dmin, scales and nibbles and the given high bits qh[nb][32]."""
    raw = b4.view(np.uint8).reshape(-1, 144)
    return np.concatenate([raw[:, :16], qh, raw[:, 16:]], axis=1)


def test_q5_k_without_high_bits_is_q4_k(lstk):
    rng = np.random.default_rng(5)
    b4 = q4_k_blocks(rng, 32)
    b5 = q5_k_from_q4_k(b4, np.zeros((32, 32), np.uint8))
    assert b5.shape == (32, 176)
    want = f16(lstk, Q4_K, b4, 32 * 256)
    np.testing.assert_array_equal(f16(lstk, Q5_K, b5, 32 * 256).view(np.uint16), want.view(np.uint16))


def unit_header(rng):
    """A Q4_K block with d = 1, dmin = 0, random 6-bit scales and zero nibbles, and its 8 scales as the
    oracle decodes them (nibbles of 1 give d sc - dmin m = sc)."""
    b = q4_k_blocks(rng, 1)
    b["d"] = 0x3c00  # 1.0
    b["dmin"] = 0
    b["qs"] = 0x11
    sc = oracle.dequant(b, oracle.TYPE_Q4_K).reshape(8, 32)[:, 0]
    b["qs"] = 0
    return b, sc


def test_q5_k_high_bits_layout(lstk):
    rng = np.random.default_rng(6)
    b4, sc = unit_header(rng)
    assert len(set(sc.tolist())) > 1
    for l in range(32):
        for j in range(8):
            qh = np.zeros((1, 32), np.uint8)
            qh[0, l] = 1 << j
            y = f16(lstk, Q5_K, q5_k_from_q4_k(b4, qh), 256).astype(np.float32)
            want = np.zeros(256, np.float32)
            want[32 * j + l] = 16 * sc[j]
            np.testing.assert_array_equal(y, want, err_msg=f"qh[{l}] bit {j}")
    # all bits at once, random
    qh = rng.integers(0, 256, (1, 32), dtype=np.uint8)
    bits = np.unpackbits(qh[0][:, None], axis=1, bitorder="little")  # [l][j]
    want = (16 * sc[:, None] * bits.T).reshape(256)
    np.testing.assert_array_equal(f16(lstk, Q5_K, q5_k_from_q4_k(b4, qh), 256).astype(np.float32), want)


def q6_k_block(ql, qh, scales, d):
    return np.concatenate([ql.astype(np.uint8), qh.astype(np.uint8), scales.astype(np.int8).view(np.uint8),
                           np.array([d], np.float16).view(np.uint8)])


def q6_k_values(ql, qh):
    """Each value's 6-bit q by ggml's block_q6_K layout: value 128 h + 32 j + l takes the low (j < 2) or
    high (j >= 2) nibble of ql[64 h + 32 (j % 2) + l] and bits 2j, 2j + 1 of qh[32 h + l]."""
    q = np.zeros(256, np.int32)
    for i in range(256):
        h, j, l = i // 128, (i % 128) // 32, i % 32
        lo = (int(ql[64 * h + 32 * (j % 2) + l]) >> (4 * (j // 2))) & 0xF
        hi = (int(qh[32 * h + l]) >> (2 * j)) & 3
        q[i] = lo | hi << 4
    return q


def test_q6_k_bit_layout_by_single_bits(lstk):
    ones = np.ones(16, np.int8)
    base = f16(lstk, Q6_K, q6_k_block(np.zeros(128), np.zeros(64), ones, 1.0), 256).astype(np.float32)
    np.testing.assert_array_equal(base, np.full(256, -32.0, np.float32))
    for byte in range(128):
        for bit in range(8):
            ql = np.zeros(128, np.uint8)
            ql[byte] = 1 << bit
            y = f16(lstk, Q6_K, q6_k_block(ql, np.zeros(64), ones, 1.0), 256).astype(np.float32)
            want = np.full(256, -32.0, np.float32) + q6_k_values(ql, np.zeros(64, np.uint8))
            np.testing.assert_array_equal(y, want, err_msg=f"ql[{byte}] bit {bit}")
            assert np.count_nonzero(y != -32) == 1
    for byte in range(64):
        for bit in range(8):
            qh = np.zeros(64, np.uint8)
            qh[byte] = 1 << bit
            y = f16(lstk, Q6_K, q6_k_block(np.zeros(128), qh, ones, 1.0), 256).astype(np.float32)
            want = np.full(256, -32.0, np.float32) + q6_k_values(np.zeros(128, np.uint8), qh)
            np.testing.assert_array_equal(y, want, err_msg=f"qh[{byte}] bit {bit}")
            assert np.count_nonzero(y != -32) == 1


def test_q6_k_scales_and_products(lstk):
    rng = np.random.default_rng(7)
    for d in (1.0, 2.0 ** -9, 2.0 ** -3):
        ql = rng.integers(0, 256, 128)
        qh = rng.integers(0, 256, 64)
        scales = rng.integers(-128, 128, 16)
        q = q6_k_values(ql.astype(np.uint8), qh.astype(np.uint8))
        # d sc (q - 32) is exact in f32 (|sc (q - 32)| <= 4096, d a power of two), then rounded once to fp16
        want = (d * np.repeat(scales, 16) * (q - 32)).astype(np.float32).astype(np.float16).astype(np.float32)
        got = f16(lstk, Q6_K, q6_k_block(ql, qh, scales, d), 256).astype(np.float32)
        np.testing.assert_array_equal(got, want, err_msg=f"d={d}")
    # several blocks in a row, each with its own d: the same as one block at a time
    blocks = [q6_k_block(rng.integers(0, 256, 128), rng.integers(0, 256, 64), rng.integers(-128, 128, 16),
                         float(rng.uniform(1e-4, 1e-2))) for _ in range(5)]
    whole = f16(lstk, Q6_K, np.concatenate(blocks), 5 * 256)
    parts = np.concatenate([f16(lstk, Q6_K, b, 256) for b in blocks])
    np.testing.assert_array_equal(whole.view(np.uint16), parts.view(np.uint16))


def test_rejects_bad_arguments(lstk):
    with pytest.raises(lstk.LstkError, match="no dequantizer"):
        lstk.dequant_f16(15, np.zeros(292, np.uint8), 256)  # Q8_K is an activation format
    with pytest.raises(lstk.LstkError, match="need"):
        lstk.dequant_f16(Q4_K, np.zeros(144, np.uint8), 512)
    with pytest.raises(lstk.LstkError, match="need"):
        lstk.dequant_f16(Q8_0, np.zeros(68, np.uint8), 48)  # not a multiple of 32
    # the C entry point's own checks
    out = np.zeros(256, np.float16)
    src = np.zeros(210, np.uint8)
    assert lstk.lib().lstk_dequant_f16(Q6_K, src.ctypes.data, 100, out.ctypes.data) == lstk.E_INVALID
    assert b"multiple of the type's block" in lstk.lib().lstk_last_error()
    assert lstk.lib().lstk_dequant_f16(99, src.ctypes.data, 256, out.ctypes.data) == lstk.E_INVALID
    assert b"unsupported type 99" in lstk.lib().lstk_last_error()
    assert lstk.lib().lstk_dequant_f16(Q6_K, None, 256, out.ctypes.data) == lstk.E_INVALID


def test_loader_dequantizes_dense_tensors(lstk, tmp_path):
    """A qwen3moe GGUF whose attention matrices are Q8_0 / Q4_K / Q5_K / Q6_K and whose embedding is Q6_K:
    qwen3_dense_weights returns them as F16 equal to lstk_dequant_f16 of the stored bytes; norms stay F32
    views; a Q4_K norm is rejected by name."""
    rng = np.random.default_rng(8)
    hp = dict(n_layer=2, n_embd=256, n_head=2, n_head_kv=1, head_dim=128, n_vocab=64, n_expert=4, n_expert_used=2,
              n_ff_exp=256, n_ctx_train=512, rms_eps=1e-6, rope_freq_base=1e6)
    w = synth.qwen3_weights(rng, hp, wtype=8)
    nb = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}
    per = {Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
    raw = {}

    def quantized(name, type_, rows, cols):
        b = rng.integers(0, 256, rows * cols // per[type_] * nb[type_], dtype=np.uint8).reshape(-1, nb[type_])
        # finite, modest fp16 scales at the format's offsets
        for off in {Q8_0: (0,), Q4_K: (0, 2), Q5_K: (0, 2), Q6_K: (208,)}[type_]:
            b[:, off:off + 2] = rng.uniform(1e-4, 1e-2, len(b)).astype(np.float16).view(np.uint8).reshape(-1, 2)
        raw[name] = (type_, b.ravel(), rows * cols)
        return b.ravel()

    h, hq, hk = hp["n_embd"], hp["n_head"] * hp["head_dim"], hp["n_head_kv"] * hp["head_dim"]
    mats = {"wq": (Q8_0, hq, h), "wk": (Q4_K, hk, h), "wv": (Q5_K, hk, h), "wo": (Q6_K, h, hq)}
    tensors = {}
    for l in range(hp["n_layer"]):
        for key, (t, r, c) in mats.items():
            tensors[(l, key)] = (t, quantized((l, key), t, r, c), r, c)
    emb = quantized("emb", Q6_K, hp["n_vocab"], h)
    path = tmp_path / "quant_dense.gguf"
    synth.write_qwen3_gguf(path, hp, w, dense_override={"token_embd.weight": (Q6_K, emb), **{
        f"blk.{l}.{ {'wq': 'attn_q', 'wk': 'attn_k', 'wv': 'attn_v', 'wo': 'attn_output'}[key] }.weight": (t, b)
        for (l, key), (t, b, r, c) in tensors.items()}})
    g = lstk.GgufFile(path)
    got = lstk.qwen3_dense_weights(g, g.qwen3_hparams())
    for (l, key), (t, b, r, c) in tensors.items():
        a = got["layers"][l][key]
        assert a.dtype == np.float16 and a.shape == (r, c)
        np.testing.assert_array_equal(a.ravel().view(np.uint16), lstk.dequant_f16(t, b, r * c).view(np.uint16))
    assert got["tok_embd"].shape == (hp["n_vocab"], h)
    np.testing.assert_array_equal(got["tok_embd"].ravel().view(np.uint16), lstk.dequant_f16(Q6_K, emb, emb.size // 210 * 256).view(np.uint16))
    np.testing.assert_array_equal(got["layers"][1]["ffn_norm"], w["layers"][1]["ffn_norm"])
    assert got["layers"][0]["attn_norm"].dtype == np.float32 and got["output"] is None
    np.testing.assert_array_equal(got["layers"][0]["gate_inp"], w["layers"][0]["gate_inp"])
    # a quantized norm is refused by name
    bad = tmp_path / "bad_norm.gguf"
    synth.write_qwen3_gguf(bad, hp, w, dense_override={"blk.1.ffn_norm.weight": (Q4_K, np.zeros(144, np.uint8))})
    g = lstk.GgufFile(bad)
    with pytest.raises(lstk.LstkError, match="blk.1.ffn_norm.weight is Q4_K"):
        lstk.qwen3_dense_weights(g, g.qwen3_hparams())
