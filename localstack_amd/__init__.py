"""localstack_amd - MI355X (gfx950) Qwen3-MoE expert-FFN path behind a C ABI.

The shared library liblstk_moe.so (built by localstack_amd/build.py from csrc/) holds the HIP
kernels, the HBM expert pool and the C ABI declared in include/lstk_moe.h. This module is a thin
ctypes view of that ABI that mirrors the reference's interface for the path:

  ExpertStore          src/expert_store.h:113-131 (init / acquire / release_all / stats / describe)
  ExpertStore.route    router()    src/qwen3.cpp:175-192
  ExpertStore.ffn      moe_apply() src/qwen3.cpp:197-214 plus the residual add (:250 / :287)
  ExpertStore.block    the resident MoE block of qwen3_build_graph (src/qwen3.cpp:239-250)
  Qwen3Model           the forward pass around it (include/lstk_qwen3.h): Engine::decode
                       (src/engine.cpp:250-278) over qwen3_build_graph (src/qwen3.cpp:223-259)
                       with the KvCache block table (src/kv_cache.cpp:59-150)

Device buffers are torch tensors on a ROCm device (or raw integer device pointers); torch is used
only to own device memory and streams. There is no CPU fallback: every compute call runs the HIP
kernels, and a missing library raises.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# LSTK_LIBRARY names another build of the library (the sanitizer build of the CPU tests)
LIB_PATH = os.environ.get("LSTK_LIBRARY") or os.path.join(HERE, "liblstk_moe.so")

TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_Q4_K = 0, 1, 8, 12
POOL_STREAMING, POOL_DRY, POOL_DEVICE_LRU, POOL_AUTO_SIZE = 1, 2, 4, 8
E_INVALID, E_NOMEM, E_EXHAUSTED, E_DEVICE, E_IO, E_BADID = -1, -2, -3, -4, -5, -6


class LstkError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


class MoeDims(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_int32), ("n_embd", ctypes.c_int32), ("n_ff_exp", ctypes.c_int32),
                ("n_expert", ctypes.c_int32), ("n_expert_used", ctypes.c_int32), ("n_batch", ctypes.c_int32)]


class ExpertLayer(ctypes.Structure):
    _fields_ = [("type_up", ctypes.c_int32), ("type_gate", ctypes.c_int32), ("type_down", ctypes.c_int32),
                ("host_up", ctypes.c_void_p), ("host_gate", ctypes.c_void_p), ("host_down", ctypes.c_void_p)]


class PoolStats(ctypes.Structure):
    _fields_ = [("hits", ctypes.c_uint64), ("misses", ctypes.c_uint64), ("bytes_read", ctypes.c_uint64),
                ("acquires", ctypes.c_uint64), ("wait_ms", ctypes.c_double)]


class GgufTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int32), ("n_dims", ctypes.c_int32),
                ("ne", ctypes.c_int64 * 4), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64),
                ("data", ctypes.c_void_p)]


class Qwen3HParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "n_vocab",
                                              "n_expert", "n_expert_used", "n_ff_exp", "n_ctx_train")] + \
               [("rms_eps", ctypes.c_float), ("rope_freq_base", ctypes.c_float)]


class Qwen3Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("attn_norm", "wq", "wk", "wv", "wo", "q_norm", "k_norm", "ffn_norm",
                                               "gate_inp")] + [("gate_inp_type", ctypes.c_int32)]


class Qwen3Weights(ctypes.Structure):
    _fields_ = [("tok_embd", ctypes.c_void_p), ("output_norm", ctypes.c_void_p), ("output", ctypes.c_void_p),
                ("layers", ctypes.c_void_p)]


# name -> (restype, argtypes); every function declared in include/lstk_moe.h and include/lstk_qwen3.h
_P, _I, _SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
SIGNATURES = {
    "lstk_last_error": (ctypes.c_char_p, []),
    "lstk_abi_version": (_I, []),
    "lstk_pool_create": (_I, [ctypes.POINTER(MoeDims), _P, _SZ, ctypes.c_uint32, ctypes.c_uint32, ctypes.POINTER(_P)]),
    "lstk_pool_destroy": (None, [_P]),
    "lstk_pool_default_bytes": (_SZ, [_SZ, _SZ, _SZ, _SZ, _SZ]),
    "lstk_pool_acquire": (_I, [_P, _I, _P, _I, _P, _P]),
    "lstk_pool_acquire_device": (_I, [_P, _I, _P, _I, _P, _P]),
    "lstk_pool_release_all": (_I, [_P, _P]),
    "lstk_pool_stats": (_I, [_P, ctypes.POINTER(PoolStats)]),
    "lstk_pool_total_bytes": (_SZ, [_P]),
    "lstk_pool_total_slots": (ctypes.c_uint32, [_P]),
    "lstk_pool_layer_slots": (_I, [_P, _I]),
    "lstk_pool_describe": (_I, [_P, ctypes.c_char_p, _SZ]),
    "lstk_moe_route": (_I, [_P, _I, _P, _I, _P, _I, _P, _P, _P]),
    "lstk_moe_ffn": (_I, [_P, _I, _P, _P, _P, _P, _P, _I, _P]),
    "lstk_moe_block": (_I, [_P, _I, _P, _P, _I, _P, _P, _P, _P, _I, _P]),
    "lstk_moe_block_noalloc": (_I, [_P, _I, _P, _P, _I, _P, _P, _P, _P, _I, _P]),
    "lstk_moe_permute": (_I, [_P, _P, _I, _I, _P, _P, _P, _P]),
    "lstk_pool_check": (_I, [_P, _P]),
    "lstk_pool_set_timing": (_I, [_P, _I]),
    "lstk_pool_timing": (_I, [_P, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)]),
    "lstk_matrix_bytes": (_SZ, [_I, _I, _I]),
    "lstk_repack_matrix": (_I, [_I, _I, _I, _P, _P]),
    "lstk_unpack_matrix": (_I, [_I, _I, _I, _P, _P]),
    "lstk_pool_debug_fail_copies": (_I, [_P, _I]),
    "lstk_model_create": (_I, [ctypes.POINTER(Qwen3HParams), ctypes.POINTER(Qwen3Weights), _P, ctypes.c_uint32,
                               ctypes.c_uint32, ctypes.POINTER(_P)]),
    "lstk_model_destroy": (None, [_P]),
    "lstk_model_decode": (_I, [_P, ctypes.c_int32, _P, _I, _P, _P, _P]),
    "lstk_model_prepare": (_I, [_P, ctypes.c_int32, _P, _I, ctypes.POINTER(ctypes.c_int32), _P]),
    "lstk_model_forward": (_I, [_P, ctypes.c_int32, _I, ctypes.c_int32, _P, _P, _P]),
    "lstk_model_fill_context": (_I, [_P, ctypes.c_int32, _I, ctypes.c_uint64, _P]),
    "lstk_model_set_trace": (_I, [_P, ctypes.c_char_p]),
    "lstk_model_debug_capture": (_I, [_P, _P]),
    "lstk_model_debug_capture_moe_in": (_I, [_P, _P]),
    "lstk_model_remove_seq": (_I, [_P, ctypes.c_int32]),
    "lstk_model_truncate_seq": (_I, [_P, ctypes.c_int32, ctypes.c_int32]),
    "lstk_model_seq_len": (ctypes.c_int32, [_P, ctypes.c_int32]),
    "lstk_gguf_open": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "lstk_gguf_close": (None, [_P]),
    "lstk_gguf_arch": (ctypes.c_char_p, [_P]),
    "lstk_gguf_version": (_I, [_P]),
    "lstk_gguf_alignment": (_I, [_P]),
    "lstk_gguf_has": (_I, [_P, ctypes.c_char_p]),
    "lstk_gguf_get_int": (ctypes.c_int64, [_P, ctypes.c_char_p, ctypes.c_int64]),
    "lstk_gguf_get_float": (ctypes.c_double, [_P, ctypes.c_char_p, ctypes.c_double]),
    "lstk_gguf_get_str": (ctypes.c_char_p, [_P, ctypes.c_char_p, ctypes.c_char_p]),
    "lstk_gguf_n_tensors": (_I, [_P]),
    "lstk_gguf_tensor_at": (_I, [_P, _I, ctypes.POINTER(GgufTensor)]),
    "lstk_gguf_find_tensor": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(GgufTensor)]),
    "lstk_gguf_qwen3_hparams": (_I, [_P, ctypes.POINTER(Qwen3HParams)]),
    "lstk_gguf_qwen3_experts": (_I, [_P, ctypes.POINTER(Qwen3HParams), _P]),
    "lstk_dequant_f16": (_I, [_I, _P, ctypes.c_size_t, _P]),
    "lstk_model_set_timing": (_I, [_P, _I]),
    "lstk_debug_attn_plan": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "lstk_model_debug_options": (_I, [_P, _I]),
    "lstk_model_timing": (_I, [_P, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64)]),
}

_lib = None


def lib():
    """Loads liblstk_moe.so; raises if it has not been built (there is no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python localstack_amd/build.py`")
        # torch ships its own HIP runtime (SONAME libamdhip64.so.7). Loading it first makes the
        # library's libamdhip64.so.7 dependency bind to that same runtime, so the library and torch
        # share one device context and torch's streams are valid handles for the library.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(rc):
    if rc != 0:
        raise LstkError(rc, lib().lstk_last_error().decode())
    return rc


def _ptr(x):
    """Device/host pointer of a torch tensor, numpy array or integer."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if hasattr(x, "data_ptr"):
        return x.data_ptr()
    if isinstance(x, np.ndarray):
        return x.ctypes.data
    raise TypeError(f"cannot take the address of {type(x)}")


def _stream(stream):
    if stream is None:
        try:
            import torch
            if torch.cuda.is_available():
                return torch.cuda.current_stream().cuda_stream
        except ImportError:
            pass
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def matrix_bytes(type_, rows, cols):
    return lib().lstk_matrix_bytes(type_, rows, cols)


def default_pool_bytes(table_bytes, weight_bytes, kv_bytes, device_total, device_free):
    """Engine::init's pool budget (src/engine.cpp:84-117) for HBM: min(table, total - weights - kv - 1.5 GiB,
    free - 3 GiB), at least 16 KiB."""
    return lib().lstk_pool_default_bytes(int(table_bytes), int(weight_bytes), int(kv_bytes), int(device_total),
                                         int(device_free))


def attn_plan(n_tokens, n_head, n_kv, head_dim, kv_size, n_cells, cell_begin=0, rope_in=False):
    """The attention launch plan the library takes for a step (host arithmetic, no device call):
    (rows per work-group, row blocks, cells per chunk, chunks, RoPE inside the launch, work-groups)."""
    out = (ctypes.c_int32 * 6)()
    _check(lib().lstk_debug_attn_plan(int(n_tokens), int(n_head), int(n_kv), int(head_dim), int(kv_size), int(n_cells),
                                      int(cell_begin), 1 if rope_in else 0, ctypes.cast(out, ctypes.c_void_p)))
    return out[0], out[1], out[2], out[3], bool(out[4]), out[5]


def repack_matrix(type_, rows, cols, gguf):
    gguf = np.ascontiguousarray(gguf, dtype=np.uint8)
    out = np.empty(matrix_bytes(type_, rows, cols), np.uint8)
    _check(lib().lstk_repack_matrix(type_, rows, cols, gguf.ctypes.data, out.ctypes.data))
    return out


def unpack_matrix(type_, rows, cols, packed):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty(matrix_bytes(type_, rows, cols), np.uint8)
    _check(lib().lstk_unpack_matrix(type_, rows, cols, packed.ctypes.data, out.ctypes.data))
    return out


class ExpertStore:
    """The HBM expert pool (ExpertStore, src/expert_store.h:113-131) and the MoE calls that read it.

    layers: one (types, up, gate, down) per layer; types = (type_up, type_gate, type_down), and
    up/gate/down are the layer's stacked expert tensors as GGUF bytes (numpy uint8, expert-major).
    """

    def __init__(self, n_layer, n_embd, n_ff_exp, n_expert, n_expert_used, n_batch, layers, pool_bytes=0,
                 min_slots=0, streaming=False, dry=False, device_lru=False, auto_size=False):
        self.dims = MoeDims(n_layer, n_embd, n_ff_exp, n_expert, n_expert_used, n_batch)
        arr = (ExpertLayer * n_layer)()
        self._keep = []
        for l, (types, up, gate, down) in enumerate(layers):
            ptrs = []
            for a in (up, gate, down):
                if a is None or isinstance(a, int):
                    ptrs.append(a)
                else:
                    a = np.ascontiguousarray(a)
                    self._keep.append(a)
                    ptrs.append(a.ctypes.data)
            arr[l] = ExpertLayer(types[0], types[1], types[2], *ptrs)
        flags = ((POOL_STREAMING if streaming else 0) | (POOL_DRY if dry else 0) | (POOL_DEVICE_LRU if device_lru else 0) |
                 (POOL_AUTO_SIZE if auto_size else 0))
        h = ctypes.c_void_p()
        _check(lib().lstk_pool_create(ctypes.byref(self.dims), ctypes.cast(arr, ctypes.c_void_p), int(pool_bytes),
                                      int(min_slots), flags, ctypes.byref(h)))
        self._h = h
        self._keep = None  # the pool copied what it needs
        self._destroy = lib().lstk_pool_destroy  # held, so that closing works during interpreter shutdown

    def close(self):
        if getattr(self, "_h", None):
            self._destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    # -- ExpertStore bookkeeping ------------------------------------------------------------
    def acquire(self, layer, experts, stream=None):
        e = np.ascontiguousarray(experts, dtype=np.int32).ravel()
        slots = np.zeros(e.size, np.int32)
        _check(lib().lstk_pool_acquire(self._h, layer, e.ctypes.data, e.size, slots.ctypes.data, _stream(stream)))
        return slots.reshape(np.shape(experts))

    def acquire_device(self, layer, experts, slots, n=None, stream=None):
        """Device-side acquire + release of one segment (pools made with device_lru=True): experts and
        slots are int32 device tensors."""
        n = experts.numel() if n is None else n
        _check(lib().lstk_pool_acquire_device(self._h, layer, _ptr(experts), n, _ptr(slots), _stream(stream)))

    def release_all(self, stream=None):
        _check(lib().lstk_pool_release_all(self._h, _stream(stream)))

    def stats(self):
        s = PoolStats()
        _check(lib().lstk_pool_stats(self._h, ctypes.byref(s)))
        return dict(hits=s.hits, misses=s.misses, bytes_read=s.bytes_read, acquires=s.acquires, wait_ms=s.wait_ms)

    def total_bytes(self):
        return lib().lstk_pool_total_bytes(self._h)

    def total_slots(self):
        return lib().lstk_pool_total_slots(self._h)

    def layer_slots(self, layer):
        n = lib().lstk_pool_layer_slots(self._h, layer)
        if n < 0:
            _check(n)
        return n

    def describe(self):
        buf = ctypes.create_string_buffer(1 << 16)
        _check(lib().lstk_pool_describe(self._h, buf, len(buf)))
        return buf.value.decode()

    def debug_fail_copies(self, n):
        _check(lib().lstk_pool_debug_fail_copies(self._h, n))

    # -- compute ----------------------------------------------------------------------------
    def route(self, layer, hnorm, gate_inp, gate_type, ids, weights, n_tokens=None, stream=None):
        T = hnorm.shape[0] if n_tokens is None else n_tokens
        _check(lib().lstk_moe_route(self._h, layer, _ptr(hnorm), T, _ptr(gate_inp), gate_type, _ptr(ids), _ptr(weights),
                                    _stream(stream)))

    def ffn(self, layer, hnorm, slots, weights, resid, out, n_tokens=None, stream=None):
        T = hnorm.shape[0] if n_tokens is None else n_tokens
        _check(lib().lstk_moe_ffn(self._h, layer, _ptr(hnorm), _ptr(slots), _ptr(weights), _ptr(resid), _ptr(out), T,
                                  _stream(stream)))

    def block(self, layer, hnorm, gate_inp, gate_type, resid, out, ids, weights, n_tokens=None, stream=None):
        T = hnorm.shape[0] if n_tokens is None else n_tokens
        _check(lib().lstk_moe_block(self._h, layer, _ptr(hnorm), _ptr(gate_inp), gate_type, _ptr(resid), _ptr(out),
                                    _ptr(ids), _ptr(weights), T, _stream(stream)))

    def block_noalloc(self, layer, hnorm, gate_inp, gate_type, resid, out, ids, weights, n_tokens=None, stream=None):
        """block() with the call's scratch in the library's fixed per-device array (allocates nothing)."""
        T = hnorm.shape[0] if n_tokens is None else n_tokens
        _check(lib().lstk_moe_block_noalloc(self._h, layer, _ptr(hnorm), _ptr(gate_inp), gate_type, _ptr(resid),
                                            _ptr(out), _ptr(ids), _ptr(weights), T, _stream(stream)))

    def permute(self, bins, n_bins, counts, offsets, perm, n_tokens=None, stream=None):
        """Stable grouping of the (token, slot) pairs by bin, as ggml's CPU mul_mat_id walks them."""
        T = bins.shape[0] if n_tokens is None else n_tokens
        _check(lib().lstk_moe_permute(self._h, _ptr(bins), T, n_bins, _ptr(counts), _ptr(offsets), _ptr(perm),
                                      _stream(stream)))

    def check(self, stream=None):
        _check(lib().lstk_pool_check(self._h, _stream(stream)))

    def set_timing(self, on):
        _check(lib().lstk_pool_set_timing(self._h, 1 if on else 0))

    def timing(self):
        """(ms, launches) per stage: router (+ top-k), gate_up, down, combine."""
        ms = (ctypes.c_double * 4)()
        n = (ctypes.c_int64 * 4)()
        _check(lib().lstk_pool_timing(self._h, ms, n))
        return list(ms), list(n)


class Qwen3Model:
    """The Qwen3-MoE forward pass on the device (include/lstk_qwen3.h), mirroring Engine::decode.

    hp: dict of the lstk_qwen3_hparams fields. weights: dict with numpy arrays tok_embd (fp16
    [n_vocab][n_embd]), output_norm (f32), optional output (fp16), and layers, a list of dicts with
    attn_norm, wq, wk, wv, wo, q_norm, k_norm (or None), ffn_norm and gate_inp (fp16 [n_expert][n_embd]).
    The dense tensors are uploaded to `device` here (torch owns that memory); the experts live in
    `store`, an ExpertStore of matching dims created by the caller (resident or streaming).
    """

    def __init__(self, hp, weights, store, kv_size, n_batch, device="cuda", join_qkv=True):
        import torch
        self.hp = dict(hp)
        self.store = store
        self.device = torch.device(device)
        self._keep = []

        def up(a, dtype):
            if a is None:
                return None
            a = np.ascontiguousarray(a)
            if not a.flags.writeable:  # a view of a read-only file mapping: torch wants a writable source
                a = a.copy()
            t = torch.from_numpy(a.view(dtype)).to(self.device)
            self._keep.append(t)
            return t.data_ptr()

        def up_joined(arrs, dtype):
            """The arrays one after the other in one device buffer (Q, K and V weights, so the model can
            multiply all three in one product); returns each one's device pointer."""
            flat = [np.ascontiguousarray(a).view(dtype).ravel() for a in arrs]
            t = torch.from_numpy(np.concatenate(flat)).to(self.device)
            self._keep.append(t)
            offs = np.cumsum([0] + [a.size for a in flat[:-1]])
            return [t.data_ptr() + int(o) * t.element_size() for o in offs]

        f16, f32 = np.uint16, np.float32
        self._hp = Qwen3HParams(*(int(self.hp[n]) for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim",
                                                             "n_vocab", "n_expert", "n_expert_used", "n_ff_exp")),
                                int(self.hp.get("n_ctx_train", 0)), float(self.hp["rms_eps"]),
                                float(self.hp["rope_freq_base"]))
        n_layer = self.hp["n_layer"]
        self._layers = (Qwen3Layer * n_layer)()
        for l, L in enumerate(weights["layers"]):
            if join_qkv:
                wq, wk, wv = up_joined((L["wq"], L["wk"], L["wv"]), f16)
            else:
                wq, wk, wv = up(L["wq"], f16), up(L["wk"], f16), up(L["wv"], f16)
            self._layers[l] = Qwen3Layer(up(L["attn_norm"], f32), wq, wk, wv,
                                         up(L["wo"], f16), up(L.get("q_norm"), f32), up(L.get("k_norm"), f32),
                                         up(L["ffn_norm"], f32),
                                         up(L["gate_inp"], f32 if L["gate_inp"].dtype == np.float32 else f16),
                                         TYPE_F32 if L["gate_inp"].dtype == np.float32 else TYPE_F16)
        self._w = Qwen3Weights(up(weights["tok_embd"], f16), up(weights["output_norm"], f32),
                               up(weights.get("output"), f16), ctypes.cast(self._layers, ctypes.c_void_p))
        h = ctypes.c_void_p()
        _check(lib().lstk_model_create(ctypes.byref(self._hp), ctypes.byref(self._w), store._h, int(kv_size),
                                       int(n_batch), ctypes.byref(h)))
        self._h = h
        self._destroy = lib().lstk_model_destroy
        self.logits = torch.empty(self.hp["n_vocab"], dtype=torch.float32, device=self.device)

    def close(self):
        if getattr(self, "_h", None):
            self._destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def decode(self, seq, tokens, trace=None, logits=None, stream=None):
        """Appends tokens to sequence seq; returns the device logits [n_vocab] of the last token.

        trace: optional device int32 tensor [n_layer, n_step_tokens, n_expert_used] for the router ids
        of the last step (-1 for rows the last layer skips)."""
        tok = np.ascontiguousarray(tokens, dtype=np.int32).ravel()
        out = self.logits if logits is None else logits
        _check(lib().lstk_model_decode(self._h, int(seq), tok.ctypes.data, tok.size, _ptr(out), _ptr(trace),
                                       _stream(stream)))
        return out

    def prepare(self, seq, tokens, stream=None):
        """First half of a step: KV cells and input upload; returns the attended cell count."""
        tok = np.ascontiguousarray(tokens, dtype=np.int32).ravel()
        n = ctypes.c_int32()
        _check(lib().lstk_model_prepare(self._h, int(seq), tok.ctypes.data, tok.size, ctypes.byref(n), _stream(stream)))
        return n.value

    def forward(self, seq, n_tokens, n_cells, trace=None, logits=None, stream=None):
        """Second half of a step: the kernels (capturable in a HIP graph with a resident pool)."""
        out = self.logits if logits is None else logits
        _check(lib().lstk_model_forward(self._h, int(seq), int(n_tokens), int(n_cells), _ptr(out), _ptr(trace),
                                        _stream(stream)))
        return out

    def fill_context(self, seq, n_cells, seed=0, stream=None):
        """Appends n_cells synthetic positions (seeded random K/V, no tokens run) to sequence seq."""
        _check(lib().lstk_model_fill_context(self._h, int(seq), int(n_cells), int(seed), _stream(stream)))

    def debug_capture(self, states):
        """Test hook: every forward copies the residual stream after each layer into the device tensor
        states ([n_layer][T][n_embd] f32, T the step's tokens); None turns it off."""
        self._capture = states
        _check(lib().lstk_model_debug_capture(self._h, None if states is None else _ptr(states)))

    def debug_capture_moe_in(self, states):
        """Test hook: every forward copies the residual stream entering each layer's MoE block (the router's
        input before ffn_norm) into the device tensor states ([n_layer][T][n_embd] f32); None turns it off."""
        self._capture_moe = states
        _check(lib().lstk_model_debug_capture_moe_in(self._h, None if states is None else _ptr(states)))

    def debug_options(self, rope_apart=False):
        """Test hook: rope_apart runs a single-token step's RoPE in its own launch (multi-pass attention
        chunks) instead of inside the attention launch (one-pass chunks)."""
        _check(lib().lstk_model_debug_options(self._h, 1 if rope_apart else 0))

    def set_trace(self, path):
        """Routing trace to `path` (LSTKRTE1, read by localstack_amd.trace); None closes it."""
        _check(lib().lstk_model_set_trace(self._h, None if path is None else os.fsencode(path)))

    def remove_seq(self, seq):
        _check(lib().lstk_model_remove_seq(self._h, int(seq)))

    def truncate_seq(self, seq, keep):
        _check(lib().lstk_model_truncate_seq(self._h, int(seq), int(keep)))

    def seq_len(self, seq):
        return lib().lstk_model_seq_len(self._h, int(seq))

    def set_timing(self, on):
        _check(lib().lstk_model_set_timing(self._h, 1 if on else 0))

    def timing(self):
        """(ms, launches) per stage: norms, Q/K/V + RoPE, attention, o-proj, output head."""
        ms = (ctypes.c_double * 5)()
        n = (ctypes.c_int64 * 5)()
        _check(lib().lstk_model_timing(self._h, ms, n))
        return list(ms), list(n)


_GGML_NP = {0: np.float32, 1: np.float16}
_GGML_NAME = {0: "F32", 1: "F16", 8: "Q8_0", 10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 15: "Q8_K", 30: "BF16"}
# types lstk_dequant_f16 expands, with (values, bytes) per block
DEQUANT_TYPES = {0: (1, 4), 1: (1, 2), 8: (32, 34), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176),
                 14: (256, 210)}


def dequant_f16(type_, data, n):
    """n values of ggml type type_ (bytes-like or uint8 array) to a float16 numpy array (lstk_dequant_f16)."""
    if type_ not in DEQUANT_TYPES:
        raise LstkError(E_INVALID, f"no dequantizer for {_GGML_NAME.get(type_, type_)}")
    per, nb = DEQUANT_TYPES[type_]
    src = np.ascontiguousarray(np.frombuffer(data, np.uint8) if not isinstance(data, np.ndarray) else data.view(np.uint8).ravel())
    if n % per or src.nbytes < n // per * nb:
        raise LstkError(E_INVALID, f"{n} values of {_GGML_NAME[type_]} need {-(-n // per) * nb} bytes, got {src.nbytes}")
    out = np.empty(n, np.float16)
    _check(lib().lstk_dequant_f16(type_, src.ctypes.data, n, out.ctypes.data))
    return out


class GgufFile:
    """A memory-mapped GGUF file (include/lstk_gguf.h), mirroring GgufModel (src/gguf_model.h:31-60).

    The mapping lives as long as this object or any array view taken from it (tensor_bytes /
    tensor_array keep the object alive), so a view never outlives the memory it reads."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        _check(lib().lstk_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self._h = h
        self._destroy = lib().lstk_gguf_close
        self.path = path

    def __del__(self):
        if getattr(self, "_h", None):
            self._destroy(self._h)
            self._h = None

    @property
    def arch(self):
        return lib().lstk_gguf_arch(self._h).decode()

    @property
    def version(self):
        return lib().lstk_gguf_version(self._h)

    @property
    def alignment(self):
        return lib().lstk_gguf_alignment(self._h)

    def has(self, key):
        return bool(lib().lstk_gguf_has(self._h, key.encode()))

    def get_int(self, key, default=0):
        return lib().lstk_gguf_get_int(self._h, key.encode(), int(default))

    def get_float(self, key, default=0.0):
        return lib().lstk_gguf_get_float(self._h, key.encode(), float(default))

    def get_str(self, key, default=""):
        r = lib().lstk_gguf_get_str(self._h, key.encode(), None)
        return default if r is None else r.decode()

    def _info(self, t):
        return {"name": t.name.decode(), "type": t.type, "ne": tuple(t.ne[:t.n_dims]), "offset": t.offset,
                "nbytes": t.nbytes, "data": t.data}

    def tensors(self):
        out = []
        for i in range(lib().lstk_gguf_n_tensors(self._h)):
            t = GgufTensor()
            _check(lib().lstk_gguf_tensor_at(self._h, i, ctypes.byref(t)))
            out.append(self._info(t))
        return out

    def tensor_info(self, name):
        t = GgufTensor()
        _check(lib().lstk_gguf_find_tensor(self._h, name.encode(), ctypes.byref(t)))
        return self._info(t)

    def tensor_bytes(self, name):
        """A read-only uint8 view of the tensor's bytes in the mapping (valid while the file is open)."""
        info = self.tensor_info(name)
        buf = (ctypes.c_uint8 * info["nbytes"]).from_address(info["data"])
        buf._owner = self  # the view keeps the mapping alive
        a = np.ctypeslib.as_array(buf)
        a.flags.writeable = False
        return a

    def tensor_array(self, name):
        """F32 / F16 tensors as numpy arrays shaped [ne[n-1]]...[ne[0]] (a view of the mapping)."""
        info = self.tensor_info(name)
        if info["type"] not in _GGML_NP:
            raise LstkError(E_INVALID, f"tensor {name} is {_GGML_NAME.get(info['type'], info['type'])}, not F32/F16")
        return self.tensor_bytes(name).view(_GGML_NP[info["type"]]).reshape(tuple(reversed(info["ne"])))

    def tensor_f16(self, name):
        """Any type lstk_dequant_f16 expands (F32, F16, Q8_0, Q2_K .. Q6_K) as a float16 array shaped
        [ne[n-1]]...[ne[0]]; F16 stays a view of the mapping, the others are dequantized copies."""
        info = self.tensor_info(name)
        if info["type"] == 1:
            return self.tensor_array(name)
        n = int(np.prod(info["ne"]))
        return dequant_f16(info["type"], self.tensor_bytes(name), n).reshape(tuple(reversed(info["ne"])))

    def qwen3_hparams(self):
        hp = Qwen3HParams()
        _check(lib().lstk_gguf_qwen3_hparams(self._h, ctypes.byref(hp)))
        return {n: getattr(hp, n) for n, _ in Qwen3HParams._fields_}

    def qwen3_experts(self, hp):
        c = Qwen3HParams(*(hp[n] for n, _ in Qwen3HParams._fields_))
        arr = (ExpertLayer * hp["n_layer"])()
        _check(lib().lstk_gguf_qwen3_experts(self._h, ctypes.byref(c), ctypes.cast(arr, ctypes.c_void_p)))
        return [((L.type_up, L.type_gate, L.type_down), L.host_up, L.host_gate, L.host_down) for L in arr]


def qwen3_dense_weights(g, hp):
    """The non-expert tensors of a qwen3moe GGUF as the forward pass takes them (qwen3_map_weights,
    src/qwen3.cpp:52-89): {"tok_embd", "output_norm", "output" (None when the head is tied), "layers": [...]}.
    Norms must be F32; the router is taken as F16 or F32 as stored; the matrices the forward pass multiplies
    in F16 (embedding, attention, output) are taken as stored when F16 and dequantized to F16 from F32, Q8_0,
    Q2_K, Q3_K, Q4_K, Q5_K or Q6_K (lstk_dequant_f16); other types are rejected with the tensor's name."""
    names = {t["name"] for t in g.tensors()}

    def dense(name, types=tuple(DEQUANT_TYPES), optional=False):
        if optional and name not in names:
            return None
        t = g.tensor_info(name)
        if t["type"] not in types:
            want = "/".join(_GGML_NAME[x] for x in types)
            raise LstkError(E_INVALID, f"tensor {name} is {_GGML_NAME.get(t['type'], t['type'])}; the forward pass takes {want}")
        if types == (0,) or (types == (0, 1) and t["type"] in types):
            return g.tensor_array(name)
        return g.tensor_f16(name)

    w = {"tok_embd": dense("token_embd.weight"), "output_norm": dense("output_norm.weight", (0,)),
         "output": dense("output.weight", optional=True), "layers": []}
    for l in range(hp["n_layer"]):
        p = f"blk.{l}."
        w["layers"].append({
            "attn_norm": dense(p + "attn_norm.weight", (0,)), "wq": dense(p + "attn_q.weight"),
            "wk": dense(p + "attn_k.weight"), "wv": dense(p + "attn_v.weight"), "wo": dense(p + "attn_output.weight"),
            "q_norm": dense(p + "attn_q_norm.weight", (0,), optional=True),
            "k_norm": dense(p + "attn_k_norm.weight", (0,), optional=True),
            "ffn_norm": dense(p + "ffn_norm.weight", (0,)), "gate_inp": dense(p + "ffn_gate_inp.weight", (0, 1))})
    return w


def load_qwen3_gguf(path, n_batch=64, kv_size=4096, device="cuda", pool_bytes=None, min_slots=None, streaming=False,
                    device_lru=False):
    """qwen3_load_hparams + qwen3_map_weights + the expert pool (src/qwen3.cpp:16-109,
    src/engine.cpp:31-173) from a qwen3moe GGUF: returns (hparams, ExpertStore, Qwen3Model, GgufFile).
    The experts go to the pool straight from the mapping; the dense tensors as qwen3_dense_weights takes them."""
    g = GgufFile(path)
    hp = g.qwen3_hparams()
    experts = g.qwen3_experts(hp)
    w = qwen3_dense_weights(g, hp)
    if min_slots is None:
        # a pool class never has fewer slots than one layer's experts (src/engine.cpp:114-116)
        min_slots = max(hp["n_expert"], 2 * hp["n_expert_used"] + 2) if streaming else 0
    if pool_bytes is None:
        pool_bytes = 0
        if streaming:
            # Engine::init's budget (src/engine.cpp:84-117) from this device's memory, the dense weights and
            # the KV cache
            import torch
            free_now, total = torch.cuda.mem_get_info(torch.device(device))
            table = sum((matrix_bytes(t[0], hp["n_ff_exp"], hp["n_embd"]) + matrix_bytes(t[1], hp["n_ff_exp"], hp["n_embd"]) +
                         matrix_bytes(t[2], hp["n_embd"], hp["n_ff_exp"])) * hp["n_expert"] for t, *_ in experts)
            dense_bytes = sum(a.nbytes for a in (w["tok_embd"], w["output_norm"], w["output"]) if a is not None)
            dense_bytes += sum(a.nbytes for lw in w["layers"] for a in lw.values() if a is not None)
            kv = hp["n_layer"] * ((kv_size + 255) // 256 * 256) * hp["n_head_kv"] * hp["head_dim"] * 2 * 2
            pool_bytes = default_pool_bytes(table, dense_bytes, kv, total, free_now)
    store = ExpertStore(hp["n_layer"], hp["n_embd"], hp["n_ff_exp"], hp["n_expert"], hp["n_expert_used"], n_batch,
                        experts, pool_bytes=pool_bytes, min_slots=min_slots, streaming=streaming,
                        device_lru=device_lru)
    model = Qwen3Model(hp, w, store, kv_size, n_batch, device=device)
    return hp, store, model, g
