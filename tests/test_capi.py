"""The C ABI library: it loads, exports every symbol include/*.h declares, validates its
inputs, and its host repacker round-trips GGUF bytes (no GPU: no compute call is made)."""
import ctypes
import os
import re

import numpy as np
import pytest

from localstack_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for hdr in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if hdr.endswith(".h"):
            src = open(os.path.join(ROOT, "include", hdr)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            names |= set(re.findall(r"\b(lstk_[a-z_0-9]+)\s*\(", src))
    return sorted(names)


def test_exports_every_declared_symbol(lstk):
    names = declared_functions()
    assert len(names) >= 20
    raw = ctypes.CDLL(lstk.LIB_PATH)
    for n in names:
        assert hasattr(raw, n), n
    assert set(names) == set(lstk.SIGNATURES), set(names) ^ set(lstk.SIGNATURES)
    assert lstk.lib().lstk_abi_version() == 1


@pytest.mark.parametrize("wtype,rows,cols", [(8, 768, 2048), (8, 2048, 768), (12, 768, 2048), (12, 256, 512), (8, 3, 256),
                                             (12, 40, 512)])
def test_repack_roundtrip_and_layout(lstk, wtype, rows, cols):
    rng = np.random.default_rng(rows + cols + wtype)
    g = synth.experts(rng, wtype, 1, rows, cols)
    assert g.size == lstk.matrix_bytes(wtype, rows, cols)
    p = lstk.repack_matrix(wtype, rows, cols, g)
    assert np.array_equal(lstk.unpack_matrix(wtype, rows, cols, p), g)
    assert not np.array_equal(p, g) or rows == 1
    # chunk (sb, c) of row r sits in row block r // 16 (16 rows, or the rows left over in the last one):
    # at ((r // 16) * 16 * nsb * C + (sb * C + c) * block_rows + r % 16) * 16
    C = 17 if wtype == 8 else 9
    sbb, nsb = C * 16, cols // 256
    for r in sorted({0, 15 % rows, rows // 2, rows - 1}):
        for sb in sorted({0, nsb - 1}):
            row = g[r * nsb * sbb:(r + 1) * nsb * sbb]
            blk = row[sb * sbb:(sb + 1) * sbb]
            rb, rr = r // 16, r % 16
            block_rows = min(16, rows - 16 * rb)
            at = lambda c: p[(rb * 16 * nsb * C + (sb * C + c) * block_rows + rr) * 16:][:16]
            if wtype == 12:
                for c in range(9):
                    assert np.array_equal(at(c), blk[16 * c:16 * c + 16])
            else:
                b = blk.reshape(8, 34)
                assert np.array_equal(at(0), b[:, 0:2].reshape(-1))
                for i in range(8):
                    assert np.array_equal(at(1 + 2 * i), b[i, 2:18]) and np.array_equal(at(2 + 2 * i), b[i, 18:34])


@pytest.mark.parametrize("wtype", [10, 11, 13, 14])
def test_repack_k_quants_to_kq8(lstk, wtype):
    """Q2_K / Q3_K / Q5_K / Q6_K matrices enter the pool unpacked to KQ8 (19 chunks per super-block row:
    {f32 d, f32 dmin}, 16 int8 scales, 16 mins, 16 x 16 int8 quants): the values (d * sc) * q - dmin * m
    read back from the packed chunks equal the oracle's dequantize_row_* bit for bit (f32)."""
    import oracle
    rows, cols = 96, 512
    rng = np.random.default_rng(wtype)
    g = synth.experts(rng, wtype, 1, rows, cols)
    assert g.size == rows * cols // 256 * oracle.K_QUANTS[wtype]
    assert lstk.matrix_bytes(wtype, rows, cols) == rows * (cols // 256) * 19 * 16
    p = lstk.repack_matrix(wtype, rows, cols, g)
    C, nsb = 19, cols // 256
    # [row block][sb][c][16 rows][16 B] (96 rows: six full blocks) -> [sb][c][row][16 B]
    chunks = p.reshape(rows // 16, nsb, C, 16, 16).transpose(1, 2, 0, 3, 4).reshape(nsb, C, rows, 16)
    d = chunks[:, 0, :, 0:4].copy().view(np.float32)[..., 0]    # [sb][row]
    dmin = chunks[:, 0, :, 4:8].copy().view(np.float32)[..., 0]
    sc = chunks[:, 1].view(np.int8).astype(np.float32)           # [sb][row][16]
    m = chunks[:, 2].astype(np.float32)
    q = chunks[:, 3:].view(np.int8).astype(np.float32)           # [sb][16][row][16]
    q = q.transpose(0, 2, 1, 3).reshape(nsb, rows, 256)
    dl = (d[..., None] * sc).astype(np.float32)                  # d * sc per 16 values, in f32
    vals = np.repeat(dl, 16, axis=2) * q
    if wtype in (10, 13):
        vals = vals - np.repeat((dmin[..., None] * m).astype(np.float32), 16, axis=2)
    got = vals.astype(np.float32).transpose(1, 0, 2).reshape(rows, cols)
    want = oracle.dequant_k(wtype, g, rows * cols).reshape(rows, cols)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    with pytest.raises(lstk.LstkError):
        lstk.unpack_matrix(wtype, rows, cols, p)  # the unpacking is one-way


def test_rejects_bad_shapes_and_types(lstk):
    Q8 = (8, 8, 8)
    cases = [
        (dict(n_embd=300), "n_embd"),
        (dict(n_ff_exp=100), "n_ff_exp"),
        (dict(n_embd=8192), "4096"),
        (dict(n_expert=300), "n_expert"),
        (dict(n_expert_used=9), "n_expert_used"),
        (dict(types=(2, 2, 2)), "unsupported expert type"),
        (dict(types=(8, 12, 8)), "share a quant type"),
    ]
    for over, msg in cases:
        a = dict(n_layer=2, n_embd=256, n_ff_exp=512, n_expert=8, n_expert_used=2, n_batch=4, types=Q8)
        a.update(over)
        t = a.pop("types")
        with pytest.raises(lstk.LstkError, match=msg) as ei:
            lstk.ExpertStore(a["n_layer"], a["n_embd"], a["n_ff_exp"], a["n_expert"], a["n_expert_used"], a["n_batch"],
                             [(t, None, None, None)] * a["n_layer"], dry=True)
        assert ei.value.code == lstk.E_INVALID


def test_dry_pool_refuses_compute(lstk):
    p = lstk.ExpertStore(1, 256, 512, 8, 2, 4, [((8, 8, 8), None, None, None)], dry=True)
    with pytest.raises(lstk.LstkError, match="dry pool"):
        p.ffn(0, 16, 16, 16, 16, 16, n_tokens=1, stream=0)
    with pytest.raises(lstk.LstkError, match="dry pool"):
        p.block(0, 16, 16, 1, 16, 16, 16, 16, n_tokens=1, stream=0)
    with pytest.raises(lstk.LstkError, match="dry pool"):
        p.permute(16, 8, 16, 16, 16, n_tokens=1, stream=0)


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    import importlib
    import localstack_amd
    monkeypatch.setattr(localstack_amd, "_lib", None)
    monkeypatch.setattr(localstack_amd, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(ImportError, match="missing"):
        localstack_amd.lib()
