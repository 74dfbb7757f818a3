"""The oracle's block formats, pinned by closed forms, hand-built known-answer blocks, an independent
restatement of the 6-bit scale unpacking, and float64 brute force (no GPU)."""
import struct

import numpy as np
import pytest

from localstack_amd import synth


def f16_bits(x):
    with np.errstate(over="ignore"):
        return int(np.array(x, np.float32).astype(np.float16).view(np.uint16))


def test_fp16_roundtrip_all_halves(orc):
    # every finite half converts to float and back unchanged
    for h in range(0, 0x10000, 7):
        e = (h >> 10) & 0x1F
        if e == 31:
            continue
        f = orc.fp16_to_fp32(h)
        assert f == float(np.array(h, np.uint16).view(np.float16).astype(np.float32)), hex(h)
        assert orc.fp32_to_fp16(f) == h or (h == 0x8000 and orc.fp32_to_fp16(f) == 0x8000)


def test_fp16_rounding_matches_numpy(orc):
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10 ** rng.uniform(-9, 5, 20000).astype(np.float32),
        np.array([65504, 65519.9, 65520, 65536, 1e9, 6.1e-5, 6.0e-8, 2.9802322e-8, 2.9802326e-8, 5.96e-8,
                  1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, -0.0, 0.0], np.float32)])
    for x in xs:
        assert orc.fp32_to_fp16(float(x)) == f16_bits(x), repr(x)


def test_q8_0_act_known_answers(orc):
    # amax = 127 -> id = 1 exactly, so q = round-half-even(x)
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:7] = [2.5, 3.5, -2.5, -3.5, 0.5, 1.5]
    b = orc.quantize_q8_0_act(x)[0]
    assert orc.fp16_to_fp32(int(b["d"])) == np.float32(1.0)
    assert list(b["qs"][:7]) == [127, 2, 4, -2, -4, 0, 2]
    # the reference quantizer rounds half away from zero (roundf)
    r = orc.quantize_q8_0_ref(x)[0]
    assert list(r["qs"][:7]) == [127, 3, 4, -3, -4, 1, 2]
    # all-zero block
    z = orc.quantize_q8_0_act(np.zeros(32, np.float32))[0]
    assert int(z["d"]) == 0 and not z["qs"].any()


def test_q8_0_act_scale_rule(orc):
    # d = amax/127 rounded to fp16; q = rne(x * (127/amax)) with the division done in f32
    rng = np.random.default_rng(2)
    x = rng.standard_normal((64, 32)).astype(np.float32)
    b = orc.quantize_q8_0_act(x.reshape(-1))
    amax = np.abs(x).max(axis=1).astype(np.float32)
    d = (amax / np.float32(127)).astype(np.float16).view(np.uint16)
    assert np.array_equal(b["d"], d)
    q = np.rint(x * (np.float32(127) / amax)[:, None]).astype(np.int8)
    assert np.array_equal(b["qs"], q)


def test_q8_0_ref_matches_numpy_writer(orc):
    # two independent implementations of quantize_row_q8_0_ref: the oracle (C) and the synthetic
    # weight writer (numpy) must produce the same bytes
    rng = np.random.default_rng(3)
    x = rng.standard_normal((40, 8, 32)).astype(np.float32) * np.float32(0.02)
    a = orc.quantize_q8_0_ref(x.reshape(40, 256)).view(np.uint8).reshape(-1)
    b = synth.q8_0_quantize(x)
    assert np.array_equal(a, b)


def test_q8_0_dequant_known_answer(orc):
    blk = np.zeros(1, orc.Q8_0_DTYPE)
    blk["d"] = 0x3C00  # 1.0
    blk["qs"] = np.arange(-16, 16, dtype=np.int8)
    assert np.array_equal(orc.dequant(blk, orc.TYPE_Q8_0), np.arange(-16, 16, dtype=np.float32))
    blk["d"] = 0x3800  # 0.5
    assert np.array_equal(orc.dequant(blk, orc.TYPE_Q8_0), np.arange(-16, 16, dtype=np.float32) * 0.5)


def pack_scales(sc, m):
    """Inverse of get_scale_min_k4: 8 six-bit scales and mins -> the 12 packed bytes."""
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (m[j] & 63) | ((m[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4)
    return bytes(s)


def unpack_scales_bitparallel(scales):
    """ggml_vec_dot_q4_K_q8_K's word-parallel unpacking (kmask1/2/3): a second, independent
    formulation of get_scale_min_k4."""
    u = list(struct.unpack("<3I", bytes(scales)))
    k1, k2, k3 = 0x3F3F3F3F, 0x0F0F0F0F, 0x03030303
    u.append(((u[2] >> 4) & k2) | (((u[1] >> 6) & k3) << 4))
    uaux = u[1] & k1
    u[1] = (u[2] & k2) | (((u[0] >> 6) & k3) << 4)
    u[2] = uaux
    u[0] &= k1
    b = struct.pack("<4I", *u)
    return list(b[0:8]), list(b[8:16])


def test_q4_K_scale_min_two_formulations(orc):
    rng = np.random.default_rng(4)
    for _ in range(300):
        scales = rng.integers(0, 256, 12, dtype=np.uint8)
        sc2, m2 = unpack_scales_bitparallel(scales)
        for j in range(8):
            assert orc.q4_K_scale_min(j, scales) == (sc2[j], m2[j])


def test_q4_K_pack_roundtrip(orc):
    rng = np.random.default_rng(5)
    for _ in range(100):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        scales = np.frombuffer(pack_scales(sc, m), np.uint8)
        for j in range(8):
            assert orc.q4_K_scale_min(j, scales) == (sc[j], m[j])


def test_q4_K_dequant_known_answer(orc):
    sc = [1, 2, 3, 63, 17, 40, 5, 60]
    m = [0, 1, 63, 2, 33, 4, 20, 7]
    blk = np.zeros(1, orc.Q4_K_DTYPE)
    blk["d"] = 0x3C00     # 1.0
    blk["dmin"] = 0x3800  # 0.5
    blk["scales"] = np.frombuffer(pack_scales(sc, m), np.uint8)
    rng = np.random.default_rng(6)
    qs = rng.integers(0, 256, 128, dtype=np.uint8)
    blk["qs"] = qs
    expect = np.zeros(256, np.float32)
    for i in range(256):
        c, w = divmod(i, 64)
        if w < 32:
            q, j = qs[32 * c + w] & 0xF, 2 * c
        else:
            q, j = qs[32 * c + w - 32] >> 4, 2 * c + 1
        d1 = np.float32(1.0) * np.float32(sc[j])
        m1 = np.float32(0.5) * np.float32(m[j])
        expect[i] = d1 * np.float32(q) - m1
    assert np.array_equal(orc.dequant(blk, orc.TYPE_Q4_K), expect)


def test_q8_K_max_sign_and_bsums(orc):
    x = np.zeros(256, np.float32)
    x[5], x[9], x[100] = -3.0, 3.0, 1.5
    b = orc.quantize_q8_K(x)[0]
    # the first element with the largest magnitude is -3: iscale = -127/-3
    assert b["qs"][5] == -127 and b["qs"][9] == 127
    assert b["d"] == np.float32(1.0) / (np.float32(-127.0) / np.float32(-3.0))
    assert b["qs"][100] == int(np.rint(np.float32(1.5) * (np.float32(-127.0) / np.float32(-3.0))))
    assert np.array_equal(b["bsums"], b["qs"].astype(np.int32).reshape(16, 16).sum(axis=1))
    x[5], x[9] = 3.0, -3.0  # now +3 comes first: the scale turns negative
    b = orc.quantize_q8_K(x)[0]
    assert b["d"] < 0 and b["qs"][5] == -127 and b["qs"][9] == 127
    z = orc.quantize_q8_K(np.zeros(256, np.float32))[0]
    assert z["d"] == 0 and not z["qs"].any() and not z["bsums"].any()


def test_q8_K_clamps_to_127(orc):
    # values can reach +127.00x after scaling; min(127, .) keeps them in int8
    rng = np.random.default_rng(7)
    for _ in range(50):
        x = rng.standard_normal(256).astype(np.float32)
        b = orc.quantize_q8_K(x)[0]
        assert b["qs"].max() <= 127 and b["qs"].min() >= -127
        assert np.abs(orc.dequant(b[None], orc.TYPE_Q8_K) - x).max() <= abs(b["d"]) * 0.5 + 1e-7


def test_vec_dot_q8_0_is_dequant_dot(orc):
    rng = np.random.default_rng(8)
    n = 2048
    w = orc.quantize_q8_0_ref(rng.standard_normal(n).astype(np.float32) * 0.02)
    x = orc.quantize_q8_0_act(rng.standard_normal(n).astype(np.float32))
    got = orc.vec_dot(orc.TYPE_Q8_0, w, x, n)
    ref = np.dot(orc.dequant(w, orc.TYPE_Q8_0).astype(np.float64), orc.dequant(x, orc.TYPE_Q8_0).astype(np.float64))
    scale = np.dot(np.abs(orc.dequant(w, orc.TYPE_Q8_0)), np.abs(orc.dequant(x, orc.TYPE_Q8_0)))
    assert abs(got - ref) <= 1e-6 * scale


def test_vec_dot_q4_K_is_dequant_dot(orc):
    rng = np.random.default_rng(9)
    n = 2048
    w = synth.q4_k_random(rng, 1, n).view(orc.Q4_K_DTYPE)
    x = orc.quantize_q8_K(rng.standard_normal(n).astype(np.float32))
    got = orc.vec_dot(orc.TYPE_Q4_K, w, x, n)
    wd = orc.dequant(w, orc.TYPE_Q4_K).astype(np.float64)
    xd = orc.dequant(x, orc.TYPE_Q8_K).astype(np.float64)
    ref = np.dot(wd, xd)
    scale = np.dot(np.abs(wd), np.abs(xd))
    assert abs(got - ref) <= 2e-6 * scale
    # a transposed nibble order (high nibbles first) is caught
    bad = w.copy()
    bad["qs"] = ((w["qs"] >> 4) | (w["qs"] << 4)).astype(np.uint8)
    assert abs(orc.vec_dot(orc.TYPE_Q4_K, bad, x, n) - ref) > 100 * 2e-6 * scale


@pytest.mark.parametrize("wtype", [8, 12])
def test_row_bytes(orc, wtype):
    assert orc.row_bytes(wtype, 2048) == (2048 // 32 * 34 if wtype == 8 else 2048 // 256 * 144)
