"""The GGUF reader (include/lstk_gguf.h) on the CPU: no GPU call is made.

GgufModel (src/gguf_model.cpp:14-103) reads files through ggml's gguf library, absent here, so the
reader is held against the published layout: a file assembled byte by byte in this test (not by the
package's writer) for the header / metadata / index / alignment rules, then round trips through
synth.write_gguf for every metadata type, tensor shapes and data, the qwen3moe hyperparameters
(src/qwen3.cpp:16-45) and the expert tensors (src/qwen3.cpp:92-109); malformed files are rejected,
truncated ones at every cut point.
"""
import struct

import numpy as np
import pytest

from localstack_amd import synth

TINY = dict(n_layer=2, n_embd=256, n_head=4, n_head_kv=2, head_dim=64, n_vocab=1024, n_expert=8, n_expert_used=2,
            n_ff_exp=512, n_ctx_train=1024, rms_eps=1e-6, rope_freq_base=10000.0)


def s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def hand_built():
    """GGUF v3, 2 metadata keys, 2 tensors, default alignment 32, assembled from the layout rules."""
    body = b"GGUF" + struct.pack("<IQQ", 3, 2, 2)
    body += s("general.architecture") + struct.pack("<I", 8) + s("toy")
    body += s("toy.count") + struct.pack("<I", 4) + struct.pack("<I", 7)
    body += s("a") + struct.pack("<I", 1) + struct.pack("<Q", 4) + struct.pack("<IQ", 0, 0)        # F32 [4] at 0
    body += s("b") + struct.pack("<I", 2) + struct.pack("<QQ", 2, 3) + struct.pack("<IQ", 1, 32)  # F16 [2, 3] at 32
    pad = (32 - len(body) % 32) % 32
    data_start = len(body) + pad
    body += b"\0" * pad
    body += struct.pack("<4f", 1, 2, 3, 4) + b"\0" * 16
    body += np.arange(6, dtype=np.float16).tobytes()
    return body, data_start


def test_hand_built_file(lstk, tmp_path):
    body, data_start = hand_built()
    p = tmp_path / "toy.gguf"
    p.write_bytes(body)
    g = lstk.GgufFile(p)
    assert g.arch == "toy" and g.version == 3 and g.alignment == 32
    assert g.get_int("toy.count") == 7
    ts = g.tensors()
    assert [t["name"] for t in ts] == ["a", "b"]
    assert ts[0]["offset"] == data_start and ts[1]["offset"] == data_start + 32
    assert ts[0]["nbytes"] == 16 and ts[1]["nbytes"] == 12 and ts[1]["ne"] == (2, 3)
    np.testing.assert_array_equal(g.tensor_array("a"), [1, 2, 3, 4])
    np.testing.assert_array_equal(g.tensor_array("b"), np.arange(6, dtype=np.float16).reshape(3, 2))


def test_metadata_types_round_trip(lstk, tmp_path):
    kv = [("general.architecture", synth.GGUF_STR, "toy"), ("u8", synth.GGUF_U8, 250), ("i8", synth.GGUF_I8, -5),
          ("u16", synth.GGUF_U16, 65000), ("i16", synth.GGUF_I16, -30000), ("u32", synth.GGUF_U32, 4000000000),
          ("i32", synth.GGUF_I32, -2000000000), ("u64", synth.GGUF_U64, 2 ** 40), ("i64", synth.GGUF_I64, -2 ** 40),
          ("f32", synth.GGUF_F32, 1.5), ("f64", synth.GGUF_F64, -2.25), ("yes", synth.GGUF_BOOL, True),
          ("words", synth.GGUF_ARR, (synth.GGUF_STR, ["a", "bc", ""])), ("ids", synth.GGUF_ARR, (synth.GGUF_U32, [1, 2, 3])),
          ("name", synth.GGUF_STR, "héllo")]
    p = tmp_path / "kv.gguf"
    synth.write_gguf(p, kv, [("t", [8], 0, np.zeros(8, np.float32).tobytes())])
    g = lstk.GgufFile(p)
    for k, t, v in kv:
        if t in (synth.GGUF_STR, synth.GGUF_ARR):
            continue
        if t in (synth.GGUF_F32, synth.GGUF_F64):
            assert g.get_float(k) == v
            assert g.get_int(k, -1) == -1  # a float is not an integer
        else:
            assert g.get_int(k) == int(v), k
            assert g.get_float(k) == float(int(v))  # integers read as floats
    assert g.get_str("name") == "héllo"
    assert g.get_str("u32", "none") == "none" and g.get_str("absent", "d") == "d"
    assert g.has("words") and g.has("ids") and not g.has("absent")
    assert g.get_int("absent", 42) == 42 and g.get_float("absent", 0.5) == 0.5
    # the tensor index after the arrays was found
    assert g.tensors()[0]["name"] == "t"


def test_alignment_key(lstk, tmp_path):
    p = tmp_path / "al.gguf"
    data = [np.arange(n, dtype=np.float32).tobytes() for n in (3, 5, 64)]
    synth.write_gguf(p, [("general.architecture", synth.GGUF_STR, "toy"), ("general.alignment", synth.GGUF_U32, 128)],
                     [(f"t{i}", [len(d) // 4], 0, d) for i, d in enumerate(data)], align=128)
    g = lstk.GgufFile(p)
    assert g.alignment == 128
    for i, t in enumerate(g.tensors()):
        assert t["offset"] % 128 == 0
        np.testing.assert_array_equal(g.tensor_array(f"t{i}"), np.frombuffer(data[i], np.float32))


@pytest.fixture(scope="module")
def tiny_file(tmp_path_factory):
    w = synth.qwen3_weights(np.random.default_rng(1234), TINY, wtype=8)
    p = tmp_path_factory.mktemp("g") / "tiny.gguf"
    synth.write_qwen3_gguf(p, TINY, w)
    return p, w


def test_qwen3_hparams_and_experts(lstk, tiny_file):
    p, w = tiny_file
    g = lstk.GgufFile(p)
    hp = g.qwen3_hparams()
    for k, v in TINY.items():
        assert hp[k] == pytest.approx(v), k
    layers = g.qwen3_experts(hp)
    for l, (types, up, gate, down) in enumerate(layers):
        assert types == (8, 8, 8)
        for ptr, ref in ((up, w["layers"][l]["up"]), (gate, w["layers"][l]["gate"]), (down, w["layers"][l]["down"])):
            got = np.ctypeslib.as_array((np.ctypeslib.ctypes.c_uint8 * ref.size).from_address(ptr))
            np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(g.tensor_array("blk.1.attn_q.weight"), w["layers"][1]["wq"])
    np.testing.assert_array_equal(g.tensor_array("token_embd.weight"), w["tok_embd"])
    with pytest.raises(lstk.LstkError, match="missing tensor output.weight"):
        g.tensor_info("output.weight")  # tied head


def test_views_keep_the_mapping_alive(lstk, tiny_file):
    import gc
    p, w = tiny_file
    a = lstk.GgufFile(p).tensor_array("token_embd.weight")  # the file object is dropped at once
    gc.collect()
    np.testing.assert_array_equal(a, w["tok_embd"])


def corrupt(path, fn):
    b = bytearray(path.read_bytes())
    fn(b)
    q = path.with_name("bad.gguf")
    q.write_bytes(bytes(b))
    return q


def test_rejects_malformed_files(lstk, tiny_file):
    p, _ = tiny_file
    cases = {
        "bad magic": lambda b: b.__setitem__(slice(0, 4), b"GGUX"),
        "unsupported GGUF version": lambda b: b.__setitem__(slice(4, 8), struct.pack("<I", 1)),
        "truncated or malformed GGUF header": lambda b: b.__setitem__(slice(8, 16), struct.pack("<Q", 2 ** 62)),
    }
    for msg, fn in cases.items():
        with pytest.raises(lstk.LstkError, match=msg):
            lstk.GgufFile(corrupt(p, fn))
    with pytest.raises(lstk.LstkError) as e:
        lstk.GgufFile(p.with_name("does-not-exist.gguf"))
    assert e.value.code == lstk.E_IO


def test_rejects_every_truncation(lstk, tiny_file, tmp_path):
    body = tiny_file[0].read_bytes()
    rng = np.random.default_rng(0)
    cuts = sorted(set([0, 3, 4, 8, 23, 24, 25, 100, 1000, len(body) - 1] + list(rng.integers(0, len(body), 40))))
    for n in cuts:
        q = tmp_path / f"cut{n}.gguf"
        q.write_bytes(body[:n])
        with pytest.raises(lstk.LstkError):
            lstk.GgufFile(q)


def write_variant(tmp_path, name, hp, mutate):
    w = synth.qwen3_weights(np.random.default_rng(7), hp, wtype=8)
    mutate(w)
    p = tmp_path / name
    synth.write_qwen3_gguf(p, hp, w)
    return p


def test_expert_checks(lstk, tmp_path):
    small = dict(TINY, n_layer=1, n_vocab=64)

    def q6(w):
        w["layers"][0]["types"] = (8, 8, 14)  # Q6_K down: bytes of the right size for the sizing rule
        w["layers"][0]["down"] = np.arange(small["n_expert"] * small["n_embd"] * (small["n_ff_exp"] // 256) * 210).astype(np.uint8)

    def q4_0(w):
        w["layers"][0]["types"] = (8, 8, 2)  # Q4_0 (18 B per 32 values): not a type the pool stores
        w["layers"][0]["down"] = np.zeros(small["n_expert"] * small["n_embd"] * (small["n_ff_exp"] // 32) * 18, np.uint8)

    g = lstk.GgufFile(write_variant(tmp_path, "q6.gguf", small, q6))
    hp = g.qwen3_hparams()
    types, _, _, down = g.qwen3_experts(hp)[0]  # the other k-quants are located like Q8_0 / Q4_K
    assert types == (8, 8, 14)
    nb = small["n_expert"] * small["n_embd"] * (small["n_ff_exp"] // 256) * 210
    np.testing.assert_array_equal(np.ctypeslib.as_array((np.ctypeslib.ctypes.c_uint8 * nb).from_address(down)),
                                  np.arange(nb).astype(np.uint8))
    g = lstk.GgufFile(write_variant(tmp_path, "q4_0.gguf", small, q4_0))
    with pytest.raises(lstk.LstkError, match=r"layer 0: blk.0.ffn_down_exps.weight is Q4_0; the expert pool stores Q8_0, Q2_K"):
        g.qwen3_experts(g.qwen3_hparams())
    g = lstk.GgufFile(write_variant(tmp_path, "ok.gguf", small, lambda w: None))
    hp = g.qwen3_hparams()
    with pytest.raises(lstk.LstkError, match="expert tensor shapes do not match the hyperparameters for layer 0"):
        g.qwen3_experts(dict(hp, n_ff_exp=256))
    with pytest.raises(lstk.LstkError, match="missing expert tensors for layer 1"):
        g.qwen3_experts(dict(hp, n_layer=2))


def test_architecture_and_unknown_types(lstk, tmp_path):
    p = tmp_path / "dense.gguf"
    synth.write_gguf(p, [("general.architecture", synth.GGUF_STR, "qwen3")], [("t", [4], 0, bytes(16))])
    with pytest.raises(lstk.LstkError, match="unsupported architecture: qwen3"):
        lstk.GgufFile(p).qwen3_hparams()
    p = tmp_path / "noarch.gguf"
    synth.write_gguf(p, [("x", synth.GGUF_U32, 1)], [])
    with pytest.raises(lstk.LstkError, match="no general.architecture"):
        lstk.GgufFile(p)
    p = tmp_path / "type99.gguf"
    synth.write_gguf(p, [("general.architecture", synth.GGUF_STR, "toy")], [("t", [4], 99, bytes(16))])
    with pytest.raises(lstk.LstkError, match="unknown type 99"):
        lstk.GgufFile(p)
    p = tmp_path / "past_end.gguf"
    synth.write_gguf(p, [("general.architecture", synth.GGUF_STR, "toy")], [("t", [1024], 0, bytes(16))])
    with pytest.raises(lstk.LstkError, match="lies outside the file"):
        lstk.GgufFile(p)


def test_rejects_dims_whose_product_wraps(lstk, tmp_path):
    """Four dims of 2^32 F32 values each pass the per-dim bound of a 640 MiB file, but their byte count,
    2^130, wraps to 0 in 128-bit arithmetic; the reader must reject the tensor, not map it as 0 bytes.
    The file is sparse: only its header is written."""
    p = tmp_path / "wrap.gguf"
    synth.write_gguf(p, [("general.architecture", synth.GGUF_STR, "toy")], [("t", [2 ** 32] * 4, 0, bytes(16))])
    with open(p, "r+b") as f:
        f.truncate(640 << 20)
    with pytest.raises(lstk.LstkError, match="outside the file"):
        lstk.GgufFile(p)
    # the same file with dims whose product fits is read
    synth.write_gguf(p, [("general.architecture", synth.GGUF_STR, "toy")], [("t", [4, 1, 1, 1], 0, bytes(16))])
    with open(p, "r+b") as f:
        f.truncate(640 << 20)
    assert lstk.GgufFile(p).tensor_info("t")["nbytes"] == 16
