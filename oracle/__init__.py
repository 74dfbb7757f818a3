"""ctypes view of the CPU oracle (oracle/liblstk_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, always as the checker or the timed CPU baseline, never by the product package. The C source
(oracle.c) restates the reference's MoE path with ggml CPU semantics; see lstk_oracle.h.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblstk_oracle.so")

QK8_0 = 32
QK_K = 256
TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q8_K = 0, 1, 8, 12, 15

Q8_0_DTYPE = np.dtype([("d", "<u2"), ("qs", "i1", (32,))])
Q4_K_DTYPE = np.dtype([("d", "<u2"), ("dmin", "<u2"), ("scales", "u1", (12,)), ("qs", "u1", (128,))])
Q8_K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i2", (16,))])
assert Q8_0_DTYPE.itemsize == 34 and Q4_K_DTYPE.itemsize == 144 and Q8_K_DTYPE.itemsize == 292

_lib = None


def build():
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("oracle library not built: run `make -C oracle` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i32, u64, f32 = ctypes.c_int, ctypes.c_uint64, ctypes.c_float
        sz = ctypes.c_size_t
        sig = {
            "or_fp32_to_fp16": (ctypes.c_uint16, [f32]),
            "or_fp16_to_fp32": (f32, [ctypes.c_uint16]),
            "or_row_bytes": (sz, [i32, i32]),
            "or_quantize_q8_0_ref": (None, [P, i32, P]),
            "or_quantize_q8_0_act": (None, [P, i32, P]),
            "or_quantize_q8_K": (None, [P, i32, P]),
            "or_dequant_q8_0": (None, [P, i32, P]),
            "or_dequant_q4_K": (None, [P, i32, P]),
            "or_dequant_q8_K": (None, [P, i32, P]),
            "or_dequant_k": (None, [i32, P, i32, P]),
            "or_vec_dot_k_q8_K": (ctypes.c_float, [i32, i32, P, P]),
            "or_q4_K_scale_min": (None, [i32, P, P, P]),
            "or_vec_dot_q8_0_q8_0": (f32, [i32, P, P]),
            "or_vec_dot_q4_K_q8_K": (f32, [i32, P, P]),
            "or_router_logits": (None, [P, i32, i32, P, i32, i32, P]),
            "or_router": (None, [P, i32, i32, P, i32, i32, i32, P, P, P, P]),
            "or_permute": (i32, [P, i32, i32, i32, P, P, P, P]),
            "or_moe_ffn": (None, [P, i32, i32, i32, i32, P, P, P, P, P, P, sz, sz, sz, i32, i32, i32, P, P, i32]),
            "or_pool_create": (P, [i32, i32, P, P, u64, ctypes.c_uint32, ctypes.c_char_p, sz]),
            "or_pool_destroy": (None, [P]),
            "or_pool_acquire": (i32, [P, i32, P, i32, P, ctypes.c_char_p, sz]),
            "or_pool_release_all": (None, [P]),
            "or_pool_stats": (None, [P, P]),
            "or_pool_n_shards": (i32, [P]),
            "or_pool_shard_of_layer": (i32, [P, i32]),
            "or_pool_shard_slots": (i32, [P, i32]),
            "or_pool_slot_owner": (i32, [P, i32, i32, P, P]),
            "or_pool_lru": (i32, [P, i32, P, i32]),
            "or_dot_f16": (f32, [P, P, i32]),
            "or_set_f16_double": (None, [i32]),
            "or_matmul_f16": (None, [P, i32, i32, P, i32, P]),
            "or_rms_norm": (None, [P, i32, P, f32, P]),
            "or_rope_neox": (None, [P, i32, i32, f32, P]),
            "or_attn_row": (None, [P, P, P, i32, i32, i32, f32, P]),
            "or_qwen3_create": (P, [P, P, P, P, P, i32]),
            "or_qwen3_destroy": (None, [P]),
            "or_qwen3_decode": (i32, [P, P, i32, P, P]),
            "or_qwen3_len": (i32, [P]),
            "or_qwen3_truncate": (None, [P, i32]),
            "or_qwen3_run_layer": (i32, [P, i32, P, i32, P]),
            "or_qwen3_head": (None, [P, P, P]),
            "or_qwen3_advance": (None, [P, i32]),
            "or_qwen3_set_kv": (i32, [P, i32, i32, i32, P, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def set_f16_double(on):
    """Sums every F16 dot product of the oracle in double (True) or in ggml's f32 SIMD order (False, the
    default): the oracle's own sensitivity to a legitimate reordering."""
    lib().or_set_f16_double(1 if on else 0)


def diff_logits(ref, ours):
    """diff_logits of src/main.cpp:195-207: max and RMS of |ref - ours| in double, and both argmaxes
    (first index of the largest value, as std::max_element). Returns (max_abs, rms, ref_arg, our_arg)."""
    r = np.asarray(ref, np.float64).ravel()
    o = np.asarray(ours, np.float64).ravel()
    d = np.abs(r - o)
    return float(d.max()), float(np.sqrt(np.sum(d * d) / d.size)), int(np.argmax(r)), int(np.argmax(o))


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- fp16 / formats -------------------------------------------------------------------------

def fp32_to_fp16(x):
    return lib().or_fp32_to_fp16(float(x))


def fp16_to_fp32(h):
    return lib().or_fp16_to_fp32(int(h))


def row_bytes(type_, n):
    return lib().or_row_bytes(type_, n)


def _quant(fn, x, out_dtype, block):
    x = _c(x, np.float32)
    assert x.shape[-1] % block == 0
    rows = x.reshape(-1, x.shape[-1])
    out = np.zeros((rows.shape[0], rows.shape[1] // block), dtype=out_dtype)
    for i in range(rows.shape[0]):
        fn(_p(rows[i]), rows.shape[1], _p(out[i]))
    return out.reshape(x.shape[:-1] + (x.shape[-1] // block,))


def quantize_q8_0_ref(x):
    return _quant(lib().or_quantize_q8_0_ref, x, Q8_0_DTYPE, QK8_0)


def quantize_q8_0_act(x):
    return _quant(lib().or_quantize_q8_0_act, x, Q8_0_DTYPE, QK8_0)


def quantize_q8_K(x):
    return _quant(lib().or_quantize_q8_K, x, Q8_K_DTYPE, QK_K)


# the other k-quants: ggml type id -> bytes per 256-value block
K_QUANTS = {10: 84, 11: 110, 13: 176, 14: 210}


def dequant_k(type_, raw, n):
    """n values of Q2_K / Q3_K / Q5_K / Q6_K blocks (raw bytes) to f32 (dequantize_row_*)."""
    raw = np.ascontiguousarray(np.frombuffer(raw, np.uint8) if not isinstance(raw, np.ndarray) else raw.view(np.uint8).ravel())
    assert n % QK_K == 0 and raw.nbytes >= n // QK_K * K_QUANTS[type_]
    out = np.zeros(n, np.float32)
    lib().or_dequant_k(type_, _p(raw), n, _p(out))
    return out


def vec_dot_k(type_, raw, xq):
    """ggml_vec_dot_<type>_q8_K of one row: raw k-quant bytes against Q8_K blocks xq."""
    raw = np.ascontiguousarray(raw).view(np.uint8).ravel()
    xq = np.ascontiguousarray(xq)
    n = xq.size * QK_K
    return float(lib().or_vec_dot_k_q8_K(type_, n, _p(raw), _p(xq)))


def dequant(blocks, type_):
    blocks = np.ascontiguousarray(blocks)
    fn, per = {TYPE_Q8_0: (lib().or_dequant_q8_0, QK8_0), TYPE_Q4_K: (lib().or_dequant_q4_K, QK_K),
               TYPE_Q8_K: (lib().or_dequant_q8_K, QK_K)}[type_]
    rows = blocks.reshape(-1, blocks.shape[-1])
    out = np.zeros((rows.shape[0], rows.shape[1] * per), dtype=np.float32)
    for i in range(rows.shape[0]):
        r = np.ascontiguousarray(rows[i])
        fn(_p(r), out.shape[1], _p(out[i]))
    return out.reshape(blocks.shape[:-1] + (blocks.shape[-1] * per,))


def q4_K_scale_min(j, scales):
    s = _c(scales, np.uint8)
    sc = np.zeros(1, np.uint8)
    m = np.zeros(1, np.uint8)
    lib().or_q4_K_scale_min(j, _p(s), _p(sc), _p(m))
    return int(sc[0]), int(m[0])


def vec_dot(wtype, w, x, n):
    w = np.ascontiguousarray(w)
    x = np.ascontiguousarray(x)
    if wtype == TYPE_Q8_0:
        return lib().or_vec_dot_q8_0_q8_0(n, _p(w), _p(x))
    return lib().or_vec_dot_q4_K_q8_K(n, _p(w), _p(x))


# ---- router / permutation / ffn ------------------------------------------------------------

def router_logits(hnorm, gate_inp, gate_type):
    hnorm = _c(hnorm, np.float32)
    T, h = hnorm.shape
    g = np.ascontiguousarray(gate_inp)
    E = g.shape[0]
    out = np.zeros((T, E), np.float32)
    lib().or_router_logits(_p(hnorm), T, h, _p(g), gate_type, E, _p(out))
    return out


def router(hnorm, gate_inp, gate_type, k):
    """Returns (ids [T,k] int32, weights [T,k] f32, logits [T,E], probs [T,E])."""
    hnorm = _c(hnorm, np.float32)
    T, h = hnorm.shape
    g = np.ascontiguousarray(gate_inp)
    E = g.shape[0]
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    logits = np.zeros((T, E), np.float32)
    probs = np.zeros((T, E), np.float32)
    lib().or_router(_p(hnorm), T, h, _p(g), gate_type, E, k, _p(ids), _p(w), _p(logits), _p(probs))
    return ids, w, logits, probs


def permute(bins, n_bins):
    """bins [T,k] -> (counts, offsets, perm, active)."""
    bins = _c(bins, np.int32)
    T, k = bins.shape
    counts = np.zeros(n_bins, np.int32)
    offsets = np.zeros(n_bins + 1, np.int32)
    perm = np.zeros(T * k, np.int32)
    active = np.zeros(max(n_bins, 1), np.int32)
    na = lib().or_permute(_p(bins), T, k, n_bins, _p(counts), _p(offsets), _p(perm), _p(active))
    return counts, offsets, perm, active[:na]


def moe_ffn(hnorm, slots, weights, resid, up, gate, down, types, f, n_threads=None, want_y=False):
    """Expert FFN + combine + residual. up/gate/down: uint8 arrays [n_slots, stride]."""
    hnorm = _c(hnorm, np.float32)
    T, h = hnorm.shape
    slots = _c(slots, np.int32)
    k = slots.shape[1]
    weights = _c(weights, np.float32)
    resid = _c(resid, np.float32)
    up, gate, down = (np.ascontiguousarray(a) for a in (up, gate, down))
    out = np.zeros((T, h), np.float32)
    y = np.zeros((T, k, h), np.float32) if want_y else None
    if n_threads is None:
        n_threads = len(os.sched_getaffinity(0))
    lib().or_moe_ffn(_p(hnorm), T, h, f, k, _p(slots), _p(weights), _p(resid), _p(up), _p(gate), _p(down),
                     up.strides[0], gate.strides[0], down.strides[0], types[0], types[1], types[2], _p(out),
                     _p(y) if want_y else None, n_threads)
    return (out, y) if want_y else out


class Pool:
    """ExpertStore slot bookkeeping restated in C (src/expert_store.cpp:106-295)."""

    def __init__(self, n_layer, n_expert, types, strides, pool_bytes, min_slots):
        t = _c(types, np.int32).reshape(n_layer, 3)
        s = _c(strides, np.uint64).reshape(n_layer, 3)
        err = ctypes.create_string_buffer(512)
        self._h = lib().or_pool_create(n_layer, n_expert, _p(t), _p(s), int(pool_bytes), int(min_slots), err, 512)
        if not self._h:
            raise ValueError(err.value.decode())

    def __del__(self):
        if getattr(self, "_h", None):
            lib().or_pool_destroy(self._h)
            self._h = None

    def acquire(self, layer, experts):
        e = _c(experts, np.int32)
        slots = np.zeros(len(e), np.int32)
        err = ctypes.create_string_buffer(512)
        rc = lib().or_pool_acquire(self._h, layer, _p(e), len(e), _p(slots), err, 512)
        if rc != 0:
            raise RuntimeError(err.value.decode())
        return slots

    def release_all(self):
        lib().or_pool_release_all(self._h)

    def stats(self):
        out = np.zeros(4, np.uint64)
        lib().or_pool_stats(self._h, _p(out))
        return dict(hits=int(out[0]), misses=int(out[1]), bytes_read=int(out[2]), acquires=int(out[3]))

    @property
    def n_shards(self):
        return lib().or_pool_n_shards(self._h)

    def shard_of_layer(self, layer):
        return lib().or_pool_shard_of_layer(self._h, layer)

    def shard_slots(self, shard):
        return lib().or_pool_shard_slots(self._h, shard)

    def slot_owner(self, shard, slot):
        lay = np.zeros(1, np.int32)
        ex = np.zeros(1, np.int32)
        rc = lib().or_pool_slot_owner(self._h, shard, slot, _p(lay), _p(ex))
        return int(lay[0]), int(ex[0]), rc

    def lru(self, shard):
        cap = self.shard_slots(shard)
        out = np.zeros(cap, np.int32)
        n = lib().or_pool_lru(self._h, shard, _p(out), cap)
        return out[:n].tolist()


# ---- forward pass around the MoE block ------------------------------------------------------

def dot_f16(w, x):
    w = _c(w, np.float16)
    x = _c(x, np.float16)
    return lib().or_dot_f16(_p(w), _p(x), w.size)


def matmul_f16(W, x):
    W = _c(W, np.float16)
    x = _c(np.atleast_2d(x), np.float32)
    y = np.zeros((x.shape[0], W.shape[0]), np.float32)
    lib().or_matmul_f16(_p(W), W.shape[0], W.shape[1], _p(x), x.shape[0], _p(y))
    return y


def rms_norm(x, w, eps):
    x = _c(x, np.float32)
    y = np.zeros_like(x)
    wv = None if w is None else _c(w, np.float32)
    lib().or_rms_norm(_p(x), x.size, None if wv is None else _p(wv), eps, _p(y))
    return y


def rope_neox(x, pos, theta_scale):
    x = _c(x, np.float32)
    y = np.zeros_like(x)
    lib().or_rope_neox(_p(x), x.size, int(pos), float(theta_scale), _p(y))
    return y


def attn_row(q, K, V, scale):
    q = _c(q, np.float32)
    K = _c(K, np.float16)
    V = _c(V, np.float16)
    out = np.zeros_like(q)
    lib().or_attn_row(_p(q), _p(K), _p(V), K.shape[0], q.size, K.shape[1], float(scale), _p(out))
    return out


class _HP(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_vocab",
                                              "n_expert", "n_expert_used", "n_ff_exp")] + \
               [("rms_eps", ctypes.c_float), ("rope_freq_base", ctypes.c_float)]


class _Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("attn_norm", "wq", "wk", "wv", "wo", "q_norm", "k_norm", "ffn_norm",
                                               "gate_inp")] + \
               [(n, ctypes.c_int32) for n in ("type_up", "type_gate", "type_down")] + \
               [(n, ctypes.c_void_p) for n in ("up", "gate", "down")]


class Qwen3:
    """The forward pass of one sequence (src/qwen3.cpp:223-259) on the CPU. hp / weights as for
    localstack_amd.Qwen3Model (weights['layers'][l] also holds types, up, gate, down)."""

    def __init__(self, hp, weights, max_ctx):
        self.hp = dict(hp)
        self._keep = []

        def ptr(a, dtype):
            if a is None:
                return None
            a = np.ascontiguousarray(a).view(dtype) if dtype is not None else np.ascontiguousarray(a)
            self._keep.append(a)
            return a.ctypes.data

        f16, f32 = np.uint16, np.float32
        names = ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_vocab", "n_expert", "n_expert_used",
                 "n_ff_exp")
        self._hp = _HP(*(int(self.hp[n]) for n in names), float(self.hp["rms_eps"]), float(self.hp["rope_freq_base"]))
        n_layer = self.hp["n_layer"]
        self._layers = (_Layer * n_layer)()
        for l, L in enumerate(weights["layers"]):
            t = L["types"]
            self._layers[l] = _Layer(ptr(L["attn_norm"], f32), ptr(L["wq"], f16), ptr(L["wk"], f16), ptr(L["wv"], f16),
                                     ptr(L["wo"], f16), ptr(L.get("q_norm"), f32), ptr(L.get("k_norm"), f32),
                                     ptr(L["ffn_norm"], f32), ptr(L["gate_inp"], f16), t[0], t[1], t[2],
                                     ptr(L["up"], None), ptr(L["gate"], None), ptr(L["down"], None))
        self._h = lib().or_qwen3_create(ctypes.byref(self._hp), self._layers, ptr(weights["tok_embd"], f16),
                                        ptr(weights["output_norm"], f32), ptr(weights.get("output"), f16), int(max_ctx))
        if not self._h:
            raise ValueError("unsupported shape")

    def __del__(self):
        if getattr(self, "_h", None):
            lib().or_qwen3_destroy(self._h)
            self._h = None

    def decode(self, tokens, want_trace=False):
        """One step over `tokens`; returns the last token's logits (and the router trace [n_layer][T][k])."""
        tok = _c(np.ravel(tokens), np.int32)
        logits = np.zeros(self.hp["n_vocab"], np.float32)
        trace = np.zeros((self.hp["n_layer"], tok.size, self.hp["n_expert_used"]), np.int32) if want_trace else None
        rc = lib().or_qwen3_decode(self._h, _p(tok), tok.size, _p(logits), _p(trace) if want_trace else None)
        if rc != 0:
            raise RuntimeError("context full")
        return (logits, trace) if want_trace else logits

    def run_layer(self, l, x):
        """Layer l on x [T][n_embd] (f32) at the current positions, K / V written there, position unchanged;
        returns (x after the layer, router ids [T][k], -1 for rows the last layer skips)."""
        xx = np.array(x, dtype=np.float32, order="C", copy=True)
        T = xx.shape[0]
        ids = np.zeros((T, self.hp["n_expert_used"]), np.int32)
        if lib().or_qwen3_run_layer(self._h, int(l), _p(xx), T, _p(ids)) != 0:
            raise RuntimeError("context full or bad layer")
        return xx, ids

    def head(self, x_row):
        """The final RMSNorm and output head of one row: logits [n_vocab]."""
        xr = _c(np.ravel(x_row), np.float32)
        logits = np.zeros(self.hp["n_vocab"], np.float32)
        lib().or_qwen3_head(self._h, _p(xr), _p(logits))
        return logits

    def advance(self, T):
        lib().or_qwen3_advance(self._h, int(T))

    def set_kv(self, l, pos, K, V):
        """Sets the fp16 K / V rows [n][n_head_kv * head_dim] of positions pos .. pos + n - 1 of layer l."""
        K, V = _c(K, np.float16), _c(V, np.float16)
        if lib().or_qwen3_set_kv(self._h, int(l), int(pos), K.shape[0], _p(K), _p(V)) != 0:
            raise ValueError("positions outside the context")

    def __len__(self):
        return lib().or_qwen3_len(self._h)

    def truncate(self, keep):
        lib().or_qwen3_truncate(self._h, int(keep))
