"""Seeded synthetic weights and inputs of the Qwen3-MoE shapes (numpy, host side).

The reference ships a tiny-model writer (tools/make_tiny_moe.py) that draws weights from Python's
Mersenne Twister and quantizes experts to Q8_0; these generators play the same part for the
benchmark and test shapes, using numpy's PCG64 so that every machine draws identical bytes:
  - q8_0_from_normal: N(0, std) values quantized by quantize_row_q8_0_ref's rule
    (d = amax/127 stored as fp16, q = round-half-away(x / d) computed as x * (1/d));
  - q4_k_random: Q4_K blocks with uniform 4-bit values and 6-bit scales/mins, d ~ U(0.5, 1.5) * d0
    and dmin = 7.5 d, so dequantized weights are roughly zero-mean with |w| ~ 1e-2;
  - router weights F16 N(0, 0.02), optionally with a Zipf(s) per-expert logit bias carried by a
    constant activation column (zipf_router_f16);
  - qwen3_weights: a whole Qwen3-MoE model in the tensor set make_tiny_moe.py writes
    (tools/make_tiny_moe.py:122-136): F16 embedding (tied output head) and attention, f32 norms of
    1.0 (as that writer sets them), F16 router, quantized experts;
  - write_gguf / write_qwen3_gguf: a GGUF v3 file of such a model, laid out as the reference's
    writer lays it out (tools/make_tiny_moe.py:37-77: header, metadata, tensor index, 32-byte aligned
    data), with the qwen3moe metadata keys of tools/make_tiny_moe.py:106-120.
"""
import struct

import numpy as np

Q8_0_BLOCK = 34
Q4_K_BLOCK = 144


def q8_0_from_normal(rng, rows, cols, std=0.02):
    """rows x cols values ~ N(0, std) as GGUF Q8_0 bytes (rows * cols/32 * 34 bytes)."""
    x = rng.standard_normal((rows, cols // 32, 32), dtype=np.float32) * np.float32(std)
    return q8_0_quantize(x)


def q8_0_quantize(x):
    """x [..., nb, 32] f32 -> GGUF Q8_0 bytes (quantize_row_q8_0_ref's rule)."""
    x = np.asarray(x, np.float32)
    amax = np.max(np.abs(x), axis=-1, keepdims=True)
    d = amax / np.float32(127.0)
    with np.errstate(divide="ignore"):
        inv = np.where(d > 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    v = x * inv
    q = (np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))).astype(np.int8)
    out = np.empty(x.shape[:-1] + (Q8_0_BLOCK,), np.uint8)
    out[..., 0:2] = d.astype(np.float16).view(np.uint8).reshape(x.shape[:-1] + (2,))
    out[..., 2:] = q.view(np.uint8)
    return out.reshape(-1)


def q4_k_random(rng, rows, cols, d0=1e-4):
    """rows x cols Q4_K blocks with random nibbles and 6-bit scales/mins (rows * cols/256 * 144 bytes)."""
    nb = rows * (cols // 256)
    out = np.empty((nb, Q4_K_BLOCK), np.uint8)
    d = (rng.uniform(0.5, 1.5, nb) * d0).astype(np.float16)
    dmin = (d.astype(np.float32) * np.float32(7.5)).astype(np.float16)
    out[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    out[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    out[:, 4:] = rng.integers(0, 256, (nb, 140), dtype=np.uint8)
    return out.reshape(-1)


def q4_k_centered(rng, rows, cols, std=0.02):
    """Q4_K blocks whose dequantized values are zero-mean with standard deviation about std, as a
    trained model's are: sub-block scales sc in [4, 8], mins m = round(7.5 sc), dmin = d, so that
    w = d (sc q - m) with q uniform in 0..15 (std 4.61) centres each sub-block on zero."""
    nb = rows * (cols // 256)
    sc = rng.integers(4, 9, (nb, 8)).astype(np.uint8)
    m = np.rint(7.5 * sc.astype(np.float64)).astype(np.uint8)
    d = (rng.uniform(0.8, 1.2, nb) * std / (4.61 * 6.0)).astype(np.float16)
    out = np.empty((nb, Q4_K_BLOCK), np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    out[:, 2:4] = d.view(np.uint8).reshape(nb, 2)
    # get_scale_min_k4 packing: bytes 0-3 / 4-7 hold sc / m of sub-blocks 0-3 (6 bits) plus the top two
    # bits of sub-blocks 4-7; bytes 8-11 hold the low nibbles of sc / m of sub-blocks 4-7
    out[:, 4:8] = sc[:, :4] | ((sc[:, 4:] >> 4) << 6)
    out[:, 8:12] = m[:, :4] | ((m[:, 4:] >> 4) << 6)
    out[:, 12:16] = (sc[:, 4:] & 0xF) | ((m[:, 4:] & 0xF) << 4)
    out[:, 16:] = rng.integers(0, 256, (nb, 128), dtype=np.uint8)
    return out.reshape(-1)


# Q2_K, Q3_K, Q5_K, Q6_K: bytes per 256-value block, the fp16 fields' offsets and a d that keeps the
# dequantized values' spread near 0.02 (mins, where the format has them, about centre the values)
K_BLOCKS = {10: (84, (80, 82), 2.5e-3, 1.5), 11: (110, (108,), 5e-4, None), 13: (176, (0, 2), 6e-5, 15.5),
            14: (210, (208,), 1.5e-5, None)}


def k_quant_random(rng, wtype, rows, cols):
    """rows x cols random blocks of Q2_K / Q3_K / Q5_K / Q6_K: random quants and scales, fp16 d drawn
    around the type's scale (dmin = d times the type's centring factor)."""
    size, offs, d0, dmin_f = K_BLOCKS[wtype]
    nb = rows * (cols // 256)
    out = rng.integers(0, 256, (nb, size), dtype=np.uint8)
    d = (rng.uniform(0.5, 1.5, nb) * d0).astype(np.float16)
    out[:, offs[0]:offs[0] + 2] = d.view(np.uint8).reshape(nb, 2)
    if dmin_f is not None:
        dmin = (d.astype(np.float32) * np.float32(dmin_f)).astype(np.float16)
        out[:, offs[1]:offs[1] + 2] = dmin.view(np.uint8).reshape(nb, 2)
    return out.reshape(-1)


def experts(rng, wtype, n_expert, rows, cols, std=0.02, centered=False):
    """Stacked expert tensor [n_expert][rows][cols] as GGUF bytes of wtype (8 = Q8_0, 10 = Q2_K,
    11 = Q3_K, 12 = Q4_K, 13 = Q5_K, 14 = Q6_K). Q4_K is q4_k_random unless centered (q4_k_centered
    with the given std); the other k-quants are k_quant_random."""
    parts = []
    for _ in range(n_expert):
        if wtype == 8:
            parts.append(q8_0_from_normal(rng, rows, cols, std))
        elif wtype == 12:
            parts.append(q4_k_centered(rng, rows, cols, std) if centered else q4_k_random(rng, rows, cols))
        elif wtype in K_BLOCKS:
            parts.append(k_quant_random(rng, wtype, rows, cols))
        else:
            raise ValueError(f"unsupported expert type {wtype}")
    return np.concatenate(parts)


def f16_spread(rng, rows, cols):
    """rows x cols fp16 values drawn straight as bit patterns (fast for full-size models): a random sign, a
    random 10-bit mantissa and a binary exponent in [-10, -6], so |w| lies in [2^-10, 2^-5) (std about
    0.01, zero mean). Stands in for N(0, 0.02) dense weights where generating normals would dominate."""
    r = rng.integers(0, 65536, size=(rows, cols), dtype=np.uint16)
    exp = ((r >> np.uint16(10)) & np.uint16(0x1F)) % np.uint16(5) + np.uint16(5)
    bits = (r & np.uint16(0x83FF)) | (exp << np.uint16(10))
    return bits.view(np.float16)


def router_f16(rng, n_expert, n_embd, std=0.02):
    """ffn_gate_inp [n_expert][n_embd] as fp16."""
    return (rng.standard_normal((n_expert, n_embd), dtype=np.float32) * np.float32(std)).astype(np.float16)


def zipf_router_f16(rng, n_expert, n_embd, s=1.1, std=0.02):
    """Router weights whose logits carry a Zipf(s) per-expert bias: logit_e += ln(p_r(e)).

    p_r ~ r^-s over ranks r = a seeded permutation of 1..n_expert. The bias sits in column 0 of the
    weights and the activations carry a constant 1.0 in column 0 (activations(..., bias_unit=True)),
    so the router's plain matmul adds it; columns 1.. hold the usual N(0, std) weights. Hot experts
    then receive hundreds of the 4096 rows of a 512-token prefill, cold ones a few.
    """
    w = rng.standard_normal((n_expert, n_embd), dtype=np.float32) * np.float32(std)
    ranks = rng.permutation(n_expert) + 1
    p = ranks.astype(np.float64) ** (-s)
    p /= p.sum()
    w[:, 0] = np.log(p).astype(np.float32)
    return w.astype(np.float16)


def activations(rng, n_tokens, n_embd, bias_unit=False):
    """hnorm rows ~ N(0, 1) (the RMS-normalised hidden state); bias_unit sets column 0 to 1.0."""
    x = rng.standard_normal((n_tokens, n_embd), dtype=np.float32)
    if bias_unit:
        x[:, 0] = 1.0
    return x


def qwen3_weights(rng, hp, wtype=8, std=0.02):
    """Seeded Qwen3-MoE weights for hp (dict with n_layer, n_embd, n_head, n_head_kv, head_dim, n_vocab,
    n_expert, n_ff_exp). Dense weights N(0, std) as fp16 [rows][cols]; norms 1.0; experts GGUF bytes of
    wtype (Q4_K centred), stacked [n_expert] per matrix (up, gate: n_ff_exp x n_embd; down: n_embd x
    n_ff_exp)."""
    h, hd, E, f = hp["n_embd"], hp["head_dim"], hp["n_expert"], hp["n_ff_exp"]
    hq, hk = hp["n_head"] * hd, hp["n_head_kv"] * hd

    def f16(rows, cols):
        return (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(std)).astype(np.float16)

    ones = lambda n: np.ones(n, np.float32)
    w = {"tok_embd": f16(hp["n_vocab"], h), "output_norm": ones(h), "output": None, "layers": []}
    for _ in range(hp["n_layer"]):
        w["layers"].append({
            "attn_norm": ones(h), "wq": f16(hq, h), "wk": f16(hk, h), "wv": f16(hk, h), "wo": f16(h, hq),
            "q_norm": ones(hd), "k_norm": ones(hd), "ffn_norm": ones(h), "gate_inp": f16(E, h),
            "types": (wtype, wtype, wtype),
            "up": experts(rng, wtype, E, f, h, std, True), "gate": experts(rng, wtype, E, f, h, std, True),
            "down": experts(rng, wtype, E, h, f, std, True)})
    return w


# GGUF metadata value types
GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32, GGUF_BOOL, GGUF_STR, GGUF_ARR, GGUF_U64, GGUF_I64, \
    GGUF_F64 = range(13)
_SCALAR = {GGUF_U8: "<B", GGUF_I8: "<b", GGUF_U16: "<H", GGUF_I16: "<h", GGUF_U32: "<I", GGUF_I32: "<i", GGUF_F32: "<f",
           GGUF_BOOL: "<?", GGUF_U64: "<Q", GGUF_I64: "<q", GGUF_F64: "<d"}


def _gguf_str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _gguf_value(t, v):
    if t == GGUF_STR:
        return _gguf_str(v)
    if t == GGUF_ARR:
        et, items = v
        body = struct.pack("<IQ", et, len(items))
        return body + b"".join(_gguf_str(x) if et == GGUF_STR else struct.pack(_SCALAR[et], x) for x in items)
    return struct.pack(_SCALAR[t], v)


def write_gguf(path, kv, tensors, align=32, version=3):
    """kv: list of (key, type, value) (arrays: (element type, items)); tensors: list of (name, ne in ggml
    order, ggml type, bytes). Tensor data start at multiples of `align` after the padded index."""
    body = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv)))
    for k, t, v in kv:
        body += _gguf_str(k) + struct.pack("<I", t) + _gguf_value(t, v)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off += (len(data) + align - 1) // align * align
    for (name, ne, gtype, _), o in zip(tensors, offsets):
        body += _gguf_str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        body += struct.pack("<IQ", gtype, o)
    body += b"\0" * ((align - len(body) % align) % align)
    for _, _, _, data in tensors:
        body += bytes(data) + b"\0" * ((align - len(data) % align) % align)
    with open(path, "wb") as f:
        f.write(body)


def write_qwen3_gguf(path, hp, w, extra_kv=(), dense_override=None):
    """The model of qwen3_weights(hp) as a qwen3moe GGUF (tied head: no output.weight). dense_override maps
    a tensor name to (ggml type, bytes) stored in place of that tensor's data (same shape)."""
    a = "qwen3moe."
    kv = [("general.architecture", GGUF_STR, "qwen3moe"), ("general.name", GGUF_STR, "synthetic-qwen3moe"),
          (a + "block_count", GGUF_U32, hp["n_layer"]), (a + "context_length", GGUF_U32, hp.get("n_ctx_train", 1024)),
          (a + "embedding_length", GGUF_U32, hp["n_embd"]),
          (a + "feed_forward_length", GGUF_U32, hp["n_ff_exp"] * hp["n_expert_used"]),
          (a + "attention.head_count", GGUF_U32, hp["n_head"]), (a + "attention.head_count_kv", GGUF_U32, hp["n_head_kv"]),
          (a + "attention.key_length", GGUF_U32, hp["head_dim"]), (a + "attention.value_length", GGUF_U32, hp["head_dim"]),
          (a + "attention.layer_norm_rms_epsilon", GGUF_F32, hp["rms_eps"]),
          (a + "rope.freq_base", GGUF_F32, hp["rope_freq_base"]), (a + "expert_count", GGUF_U32, hp["n_expert"]),
          (a + "expert_used_count", GGUF_U32, hp["n_expert_used"]),
          (a + "expert_feed_forward_length", GGUF_U32, hp["n_ff_exp"])] + list(extra_kv)
    h, E, f, hd = hp["n_embd"], hp["n_expert"], hp["n_ff_exp"], hp["head_dim"]
    b = lambda arr: np.ascontiguousarray(arr).tobytes()
    ts = [("token_embd.weight", [h, hp["n_vocab"]], 1, b(w["tok_embd"])), ("output_norm.weight", [h], 0, b(w["output_norm"]))]
    if w.get("output") is not None:
        ts.append(("output.weight", [h, hp["n_vocab"]], 1, b(w["output"])))
    for l, L in enumerate(w["layers"]):
        p = f"blk.{l}."
        ts += [(p + "attn_norm.weight", [h], 0, b(L["attn_norm"])),
               (p + "attn_q.weight", [h, hp["n_head"] * hd], 1, b(L["wq"])),
               (p + "attn_k.weight", [h, hp["n_head_kv"] * hd], 1, b(L["wk"])),
               (p + "attn_v.weight", [h, hp["n_head_kv"] * hd], 1, b(L["wv"])),
               (p + "attn_output.weight", [hp["n_head"] * hd, h], 1, b(L["wo"])),
               (p + "attn_q_norm.weight", [hd], 0, b(L["q_norm"])), (p + "attn_k_norm.weight", [hd], 0, b(L["k_norm"])),
               (p + "ffn_norm.weight", [h], 0, b(L["ffn_norm"])),
               (p + "ffn_gate_inp.weight", [h, E], 1 if L["gate_inp"].dtype == np.float16 else 0, b(L["gate_inp"])),
               (p + "ffn_up_exps.weight", [h, f, E], L["types"][0], b(L["up"])),
               (p + "ffn_gate_exps.weight", [h, f, E], L["types"][1], b(L["gate"])),
               (p + "ffn_down_exps.weight", [f, h, E], L["types"][2], b(L["down"]))]
    for name, (gtype, data) in (dense_override or {}).items():
        i = next(i for i, t in enumerate(ts) if t[0] == name)
        ts[i] = (name, ts[i][1], gtype, b(data))
    write_gguf(path, kv, ts)
