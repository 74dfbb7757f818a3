"""The GGUF reader on a file the reference's own writer produced (tests/golden/tiny_qwen3moe_reference.gguf,
made by tests/golden/make_tiny_gguf_fixture.py with tools/make_tiny_moe.py's defaults). CPU only.

An independent walk of the bytes in this test (GGUF v3: header, metadata, tensor index, 32-byte aligned
data) gives the expected keys, shapes, types and offsets; the reader must agree on every tensor, the
qwen3moe hyperparameters (src/qwen3.cpp:16-45), the expert locator (src/qwen3.cpp:92-109) and the dense
weights. The writer's Q8_0 (tools/make_tiny_moe.py:24-34: d = max|v| / 127 in fp16, q = round(v / d))
leaves +-127 in every non-zero block, which the located expert bytes must show. The oracle's forward pass
runs on the file's weights (finite logits, deterministic greedy tokens). The GPU kernels take n_embd in
multiples of 256 (the Qwen3 MoE models' 2048 and 4096), so the pool refuses this file's n_embd of 64 with
a message that says so.
"""
import os
import struct

import numpy as np
import pytest

import oracle

PATH = os.path.join(os.path.dirname(__file__), "golden", "tiny_qwen3moe_reference.gguf")
GGUF_SIZES = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}


def walk(raw):
    """(kv {key: value}, tensors [(name, ne, type, absolute offset)]) from the file's bytes."""
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from(fmt, raw, pos)
        pos += struct.calcsize(fmt)
        return v if len(v) > 1 else v[0]

    def string():
        nonlocal pos
        n = take("<Q")
        s = raw[pos:pos + n].decode()
        pos += n
        return s

    def value(t):
        if t == 8:
            return string()
        if t == 9:
            et, n = take("<IQ")
            return [value(et) for _ in range(n)]
        fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}[t]
        return take(fmt)

    assert raw[:4] == b"GGUF"
    pos = 4
    version, n_t, n_kv = take("<IQQ")
    assert version == 3
    kv = {}
    for _ in range(n_kv):
        k = string()
        kv[k] = value(take("<I"))
    index = []
    for _ in range(n_t):
        name = string()
        nd = take("<I")
        ne = [take("<Q") for _ in range(nd)]
        t, off = take("<IQ")
        index.append((name, ne, t, off))
    align = kv.get("general.alignment", 32)
    start = (pos + align - 1) // align * align
    return kv, [(n, ne, t, start + off) for n, ne, t, off in index]


@pytest.fixture(scope="module")
def ref_file():
    raw = open(PATH, "rb").read()
    return raw, *walk(raw)


def nbytes(t, ne):
    n = int(np.prod(ne))
    return {0: 4 * n, 1: 2 * n, 8: n // 32 * 34}[t]


def test_reader_agrees_with_the_byte_walk(lstk, ref_file):
    raw, kv, index = ref_file
    g = lstk.GgufFile(PATH)
    assert g.arch == "qwen3moe" and g.version == 3 and g.alignment == 32
    assert g.get_str("general.name") == kv["general.name"] == "tiny-qwen3moe-test"
    for k, v in kv.items():
        if isinstance(v, str):
            assert g.get_str(k) == v
        elif isinstance(v, float):
            assert g.get_float(k) == v
        else:
            assert g.get_int(k) == v, k
    ts = g.tensors()
    assert [t["name"] for t in ts] == [n for n, *_ in index]
    for t, (name, ne, typ, off) in zip(ts, index):
        assert t["ne"] == tuple(ne) and t["type"] == typ and t["offset"] == off, name
        assert t["nbytes"] == nbytes(typ, ne), name
        np.testing.assert_array_equal(g.tensor_bytes(name), np.frombuffer(raw, np.uint8, t["nbytes"], off))
    # the writer's tensor set: 1 embedding + 1 norm + 2 layers of 12; tied head
    assert len(ts) == 2 + 2 * 12 and "output.weight" not in [t["name"] for t in ts]


def test_hparams_and_experts(lstk, ref_file):
    raw, kv, index = ref_file
    g = lstk.GgufFile(PATH)
    hp = g.qwen3_hparams()
    want = dict(n_layer=2, n_embd=64, n_head=2, n_head_kv=1, head_dim=32, n_vocab=256, n_expert=8,
                n_expert_used=2, n_ff_exp=32, n_ctx_train=1024)
    for k, v in want.items():
        assert hp[k] == v, k
    assert hp["rms_eps"] == pytest.approx(1e-6) and hp["rope_freq_base"] == 10000.0
    where = {n: (ne, t, off) for n, ne, t, off in index}
    for l, (types, up, gate, down) in enumerate(g.qwen3_experts(hp)):
        assert types == (8, 8, 8)
        for ptr, which in ((up, "up"), (gate, "gate"), (down, "down")):
            ne, t, off = where[f"blk.{l}.ffn_{which}_exps.weight"]
            size = nbytes(t, ne)
            got = np.ctypeslib.as_array((np.ctypeslib.ctypes.c_uint8 * size).from_address(ptr))
            np.testing.assert_array_equal(got, np.frombuffer(raw, np.uint8, size, off))
            blocks = got.view(oracle.Q8_0_DTYPE)
            amax = np.abs(blocks["qs"].astype(np.int32)).max(axis=1)
            assert np.all((amax == 127) | (blocks["d"] == 0)), (l, which)
            vals = oracle.dequant(blocks, oracle.TYPE_Q8_0)
            assert 0.04 < float(vals.std()) < 0.06  # the writer's N(0, 0.05)


def test_dense_weights_and_oracle_forward(lstk, ref_file):
    g = lstk.GgufFile(PATH)
    hp = g.qwen3_hparams()
    w = lstk.qwen3_dense_weights(g, hp)
    assert w["tok_embd"].dtype == np.float16 and w["tok_embd"].shape == (256, 64)
    L = w["layers"][1]
    assert L["wq"].shape == (64, 64) and L["wk"].shape == (32, 64) and L["wo"].shape == (64, 64)
    assert L["gate_inp"].dtype == np.float16 and L["gate_inp"].shape == (8, 64)
    for name in ("attn_norm", "ffn_norm", "q_norm", "k_norm"):
        np.testing.assert_array_equal(L[name], 1.0)
    np.testing.assert_array_equal(w["output_norm"], 1.0)
    experts = g.qwen3_experts(hp)
    for l, (types, up, gate, down) in enumerate(experts):
        size = {"up": 32 * 64 // 32 * 34 * 8, "down": 64 * 32 // 32 * 34 * 8}
        as_u8 = lambda p, n: np.ctypeslib.as_array((np.ctypeslib.ctypes.c_uint8 * n).from_address(p)).copy()
        w["layers"][l].update(types=types, up=as_u8(up, size["up"]), gate=as_u8(gate, size["up"]),
                              down=as_u8(down, size["down"]))
    runs = []
    for _ in range(2):
        m = oracle.Qwen3(hp, w, 64)
        toks, nxt = [], np.array([1, 2, 3, 4], np.int32)
        for _ in range(6):
            lg = m.decode(nxt)
            assert np.all(np.isfinite(lg)) and lg.shape == (256,)
            nxt = np.array([int(np.argmax(lg))], np.int32)
            toks.append(int(nxt[0]))
        runs.append(toks)
    assert runs[0] == runs[1]


def test_pool_names_the_shape_limit(lstk):
    g = lstk.GgufFile(PATH)
    hp = g.qwen3_hparams()
    with pytest.raises(lstk.LstkError, match="n_embd must be a positive multiple of 256"):
        lstk.ExpertStore(hp["n_layer"], hp["n_embd"], hp["n_ff_exp"], hp["n_expert"], hp["n_expert_used"], 4,
                         g.qwen3_experts(hp), dry=True)
