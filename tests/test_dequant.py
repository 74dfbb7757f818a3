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
  sit (every bit probed alone) and the 16-value scale groups; power-of-two d makes the products exact;
- Q2_K and Q3_K: every quant bit, high-mask bit and scale-byte bit probed alone at unit scales, and the
  scale / min nibbles of each 16-value group.
The oracle's own k-quant dequantizers and dot products (used by the GPU parity tests of k-quant experts)
are held against the probe-pinned product dequantizer and against float64 dots of dequantized values.
"""
import numpy as np
import pytest

import oracle
from localstack_amd import synth

F32, F16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 0, 1, 8, 10, 11, 12, 13, 14


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


# ---- Q2_K and Q3_K ----------------------------------------------------------------------------------

def q2_k_block(scales, qs, d, dmin):
    return np.concatenate([np.asarray(scales, np.uint8), np.asarray(qs, np.uint8),
                           np.array([d, dmin], np.float16).view(np.uint8)])


def q3_k_block(hmask, qs, scales, d):
    return np.concatenate([np.asarray(hmask, np.uint8), np.asarray(qs, np.uint8), np.asarray(scales, np.uint8),
                           np.array([d], np.float16).view(np.uint8)])


def test_q2_k_bit_layout(lstk):
    # each qs bit alone (unit scales, no mins): value 128 n + 32 j + l takes bits 2j, 2j + 1 of qs[32 n + l]
    ones = np.full(16, 0x01, np.uint8)
    for byte in range(64):
        for bit in range(8):
            qs = np.zeros(64, np.uint8)
            qs[byte] = 1 << bit
            y = f16(lstk, Q2_K, q2_k_block(ones, qs, 1.0, 0.0), 256).astype(np.float32)
            n, l, j = byte // 32, byte % 32, bit // 2
            want = np.zeros(256, np.float32)
            want[128 * n + 32 * j + l] = 1 << (bit % 2)
            np.testing.assert_array_equal(y, want, err_msg=f"qs[{byte}] bit {bit}")
    # every value q = 1: the low nibble of scales[i] is the scale of values 16 i .. 16 i + 15; the high
    # nibble is the min, times dmin
    rng = np.random.default_rng(9)
    sc = rng.integers(0, 16, 16)
    m = rng.integers(0, 16, 16)
    y = f16(lstk, Q2_K, q2_k_block(sc | m << 4, np.full(64, 0x55, np.uint8), 1.0, 0.5), 256).astype(np.float32)
    np.testing.assert_array_equal(y, (np.repeat(sc, 16) - 0.5 * np.repeat(m, 16)).astype(np.float32))


def q3_scale_bytes(scale6):
    """The 12 scale bytes holding 16 6-bit values, built bit by bit from the block_q3_K packing: the low
    4 bits of scale i sit in byte i (i < 8, low nibble) or byte i - 8 (high nibble); its bits 4 and 5 in
    byte 8 + i % 4, at bits 2 (i / 4) and 2 (i / 4) + 1."""
    b = np.zeros(12, np.uint8)
    for i, v in enumerate(scale6):
        if i < 8:
            b[i] |= v & 0xF
        else:
            b[i - 8] |= (v & 0xF) << 4
        b[8 + i % 4] |= ((v >> 4) & 3) << (2 * (i // 4))
    return b


def test_q3_k_bit_layout(lstk):
    unit = q3_scale_bytes([33] * 16)  # every scale 33 - 32 = 1
    # all high bits set, no low bits: q = 0 everywhere
    base = f16(lstk, Q3_K, q3_k_block(np.full(32, 0xFF), np.zeros(64), unit, 1.0), 256).astype(np.float32)
    np.testing.assert_array_equal(base, np.zeros(256, np.float32))
    for byte in range(64):
        for bit in range(8):
            qs = np.zeros(64, np.uint8)
            qs[byte] = 1 << bit
            y = f16(lstk, Q3_K, q3_k_block(np.full(32, 0xFF), qs, unit, 1.0), 256).astype(np.float32)
            n, l, j = byte // 32, byte % 32, bit // 2
            want = np.zeros(256, np.float32)
            want[128 * n + 32 * j + l] = 1 << (bit % 2)
            np.testing.assert_array_equal(y, want, err_msg=f"qs[{byte}] bit {bit}")
    for byte in range(32):
        for bit in range(8):
            hm = np.full(32, 0xFF, np.uint8)
            hm[byte] &= ~np.uint8(1 << bit)
            y = f16(lstk, Q3_K, q3_k_block(hm, np.zeros(64), unit, 1.0), 256).astype(np.float32)
            want = np.zeros(256, np.float32)
            want[128 * (bit // 4) + 32 * (bit % 4) + byte] = -4.0  # a clear high bit subtracts 4
            np.testing.assert_array_equal(y, want, err_msg=f"hmask[{byte}] bit {bit}")
    # each scale byte bit alone, values q = 1: the 16-value group(s) it feeds move by its weight
    for byte in range(12):
        for bit in range(8):
            sb = np.zeros(12, np.uint8)
            sb[byte] = 1 << bit
            y = f16(lstk, Q3_K, q3_k_block(np.full(32, 0xFF), np.full(64, 0x55), sb, 1.0), 256).astype(np.float32)
            scale = np.full(16, -32.0)
            if byte < 8:
                scale[byte if bit < 4 else byte + 8] += 1 << (bit % 4)
            else:
                scale[4 * (bit // 2) + byte - 8] += 1 << (4 + bit % 2)
            np.testing.assert_array_equal(y, np.repeat(scale, 16).astype(np.float32), err_msg=f"scales[{byte}] bit {bit}")
    # the helper's packing agrees with the bit probes above on random scales
    rng = np.random.default_rng(10)
    s6 = rng.integers(0, 64, 16)
    y = f16(lstk, Q3_K, q3_k_block(np.full(32, 0xFF), np.full(64, 0x55), q3_scale_bytes(s6), 2.0 ** -4), 256)
    np.testing.assert_array_equal(y.astype(np.float32), np.repeat((s6 - 32) * 2.0 ** -4, 16).astype(np.float32))


def random_k_blocks(rng, type_, nb):
    """nb random blocks of a k-quant with finite, modest fp16 scales."""
    size = oracle.K_QUANTS[type_]
    b = rng.integers(0, 256, (nb, size), dtype=np.uint8)
    offs = {10: (80, 82), 11: (108,), 13: (0, 2), 14: (208,)}[type_]
    for o in offs:
        b[:, o:o + 2] = rng.uniform(1e-4, 1e-2, nb).astype(np.float16).view(np.uint8).reshape(-1, 2)
    return b.ravel()


@pytest.mark.parametrize("type_", [10, 11, 13, 14])
def test_oracle_k_dequant_matches_product(lstk, type_):
    """The oracle's dequantize_row_* restatement against the product's (pinned by the bit probes above),
    rounded once to fp16."""
    rng = np.random.default_rng(type_)
    raw = random_k_blocks(rng, type_, 40)
    want = oracle.dequant_k(type_, raw, 40 * 256).astype(np.float16)
    np.testing.assert_array_equal(f16(lstk, type_, raw, 40 * 256).view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("type_", [10, 11, 13, 14])
def test_oracle_k_dot_equals_float64_dot_of_dequantized(type_):
    """ggml_vec_dot_<type>_q8_K as the oracle restates it: integers exact, so the result equals the float64
    dot of the dequantized weights and activations to f32 rounding."""
    rng = np.random.default_rng(100 + type_)
    nb = 8
    for _ in range(6):
        raw = random_k_blocks(rng, type_, nb)
        x = rng.standard_normal(nb * 256).astype(np.float32)
        xq = oracle.quantize_q8_K(x)
        got = oracle.vec_dot_k(type_, raw, xq)
        w64 = oracle.dequant_k(type_, raw, nb * 256).astype(np.float64)
        x64 = oracle.dequant(xq, oracle.TYPE_Q8_K).astype(np.float64).ravel()
        ref = float(np.dot(w64, x64))
        scale = float(np.sum(np.abs(w64 * x64)))
        assert abs(got - ref) <= 2e-6 * scale, (type_, got, ref)
