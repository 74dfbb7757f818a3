"""Integer arithmetic the grouped MFMA kernels (localstack_amd/csrc/grouped.hip, q4k_superblock) rely on,
checked on the CPU: the quantizer's split of a Q8_K group sum into two exact fp16 values
(split_sum_f16, localstack_amd/csrc/device.h), the exactness of the fp16 min-term product in f32 for
any accumulation order, and the kernel's word-wise decoding of the 6-bit scales and mins against the
oracle's get_scale_min_k4 (ggml-quants.c)."""
import struct

import numpy as np


def split_sum(s):
    """64 floor(s / 64) and s mod 64, the two halves split_sum_f16 packs."""
    return s & ~63, s & 63


def test_split_sum_is_exact_in_fp16():
    # a Q8_K group sum is at most 32 * 127 in magnitude; the whole [-4096, 4096] is checked
    for s in range(-4096, 4097):
        hi, lo = split_sum(s)
        assert hi + lo == s and 0 <= lo < 64 and hi % 64 == 0
        assert float(np.float16(hi)) == hi and float(np.float16(lo)) == lo


def test_min_term_product_is_exact_in_f32():
    """sum_j m_j * s_j as the fp16 MFMA sees it (16 products of fp16 pairs, f32 sums) equals the
    integer for every order of the sums: all products and partial sums are integers below 2^24."""
    rng = np.random.default_rng(7)
    for trial in range(1500):
        m = rng.integers(0, 64, 8)
        s = rng.integers(-4064, 4065, 8)
        if trial < 3:  # extremes: every min 63, every sum at one end, then alternating
            m[:] = 63
            s[:] = (-4064, 4064, 0)[trial] if trial < 2 else np.where(np.arange(8) % 2 == 0, -4064, 4064)
        a, b = [], []
        for j in range(8):
            hi, lo = split_sum(int(s[j]))
            a += [hi, lo]
            b += [int(m[j]), int(m[j])]
        prods = [np.float32(np.float16(x)) * np.float32(np.float16(y)) for x, y in zip(a, b)]
        exact = int(np.dot(m.astype(np.int64), s.astype(np.int64)))
        for order in (list(range(16)), list(range(15, -1, -1)), list(rng.permutation(16))):
            acc = np.float32(0.0)
            for i in order:
                acc = np.float32(acc + prods[i])
            assert int(acc) == exact and float(acc) == float(exact)


def kernel_scales(scales):
    """q4k_superblock's decoding: the eight 6-bit scales from three masks of the first and third
    words, the mins of sub-blocks 0-3 / 4-7 from the second and third, and each scale split into
    8 * sh + sl byte-wise."""
    s0, s1, s2 = struct.unpack("<3I", bytes(scales))
    sc_lo = s0 & 0x3F3F3F3F
    sc_hi = (s2 & 0x0F0F0F0F) | ((s0 >> 2) & 0x30303030)
    mins = (s1 & 0x3F3F3F3F, ((s2 >> 4) & 0x0F0F0F0F) | ((s1 >> 2) & 0x30303030))
    sh = ((sc_lo >> 3) & 0x07070707, (sc_hi >> 3) & 0x07070707)
    sl = (sc_lo & 0x07070707, sc_hi & 0x07070707)

    def byte(w, i):
        return (w >> (8 * i)) & 0xFF

    sc = [byte(sc_lo, j) for j in range(4)] + [byte(sc_hi, j) for j in range(4)]
    m = [byte(mins[j // 4], j % 4) for j in range(8)]
    split = [(byte(sh[j // 4], j % 4), byte(sl[j // 4], j % 4)) for j in range(8)]
    return sc, m, split


def test_kernel_scale_decoding_matches_get_scale_min_k4(orc):
    rng = np.random.default_rng(11)
    cases = [rng.integers(0, 256, 12, dtype=np.uint8) for _ in range(500)]
    cases += [np.full(12, v, np.uint8) for v in (0x00, 0xFF, 0xC0, 0x3F, 0x0F, 0xF0)]
    for scales in cases:
        sc, m, split = kernel_scales(scales)
        for j in range(8):
            assert orc.q4_K_scale_min(j, scales) == (sc[j], m[j]), (scales.tolist(), j)
            sh, sl = split[j]
            assert sh <= 7 and sl <= 7 and 8 * sh + sl == sc[j]
