"""ctypes view of oracle/libcpu_ggml.so: the timed CPU baseline of bench.py, a SIMD restatement of
ggml's CPU algorithm for the MoE block (cpu_ggml.c). Benchmark infrastructure, checked against the oracle
by tests/test_cpu_ggml.py; never part of the product."""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcpu_ggml.so")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("CPU baseline not built: run `make -C oracle` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        P, i32 = ctypes.c_void_p, ctypes.c_int
        L.cg_moe_block.restype = i32
        L.cg_moe_block.argtypes = [P, i32, i32, i32, i32, i32, P, P, P, P, i32, P, P, P, P, i32]
        L.cg_isa.restype = ctypes.c_char_p
        L.cg_isa.argtypes = []
        _lib = L
    return _lib


def isa():
    return lib().cg_isa().decode()


def moe_block(hnorm, gate_inp_f16, up, gate, down, wtype, resid, E, f, k, n_threads=0):
    """router() + moe_apply() + residual on the host: returns (out [T][h], ids [T][k], weights [T][k])."""
    x = np.ascontiguousarray(hnorm, np.float32)
    T, h = x.shape
    g = np.ascontiguousarray(gate_inp_f16).view(np.uint16)
    r = np.ascontiguousarray(resid, np.float32)
    out = np.empty_like(x)
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    u8 = lambda a: np.ascontiguousarray(a, np.uint8)
    up, gate, down = u8(up), u8(gate), u8(down)
    rc = lib().cg_moe_block(x.ctypes.data, T, h, f, E, k, g.ctypes.data, up.ctypes.data, gate.ctypes.data,
                            down.ctypes.data, int(wtype), r.ctypes.data, out.ctypes.data, ids.ctypes.data, w.ctypes.data,
                            int(n_threads))
    if rc != 0:
        raise ValueError("bad arguments")
    return out, ids, w
