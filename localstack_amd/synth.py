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
    1.0 (as that writer sets them), F16 router, quantized experts.
"""
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


def experts(rng, wtype, n_expert, rows, cols, std=0.02, centered=False):
    """Stacked expert tensor [n_expert][rows][cols] as GGUF bytes of wtype (8 = Q8_0, 12 = Q4_K).
    Q4_K is q4_k_random unless centered (q4_k_centered with the given std)."""
    parts = []
    for _ in range(n_expert):
        if wtype == 8:
            parts.append(q8_0_from_normal(rng, rows, cols, std))
        elif wtype == 12:
            parts.append(q4_k_centered(rng, rows, cols, std) if centered else q4_k_random(rng, rows, cols))
        else:
            raise ValueError(f"unsupported expert type {wtype}")
    return np.concatenate(parts)


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
