"""ctypes binding of the CPU oracle (liboracle.so). TEST INFRASTRUCTURE ONLY.

Importable from tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg; the product
package never imports it. See oracle.c for what each function restates and how it is pinned.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

F32, F16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ3_XXS, IQ2_S, IQ4_XS, BF16 = 0, 1, 8, 10, 11, 12, 13, 14, 16, 18, 22, 23, 30
Q8_1_BYTES = 36
_P = C.c_void_p


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError("oracle not built: run `make -C oracle` (or __graft_entry__.build())")
        L = C.CDLL(path)
        L.or_f16_to_f32.restype = C.c_float
        L.or_f16_to_f32.argtypes = [C.c_uint16]
        L.or_f32_to_f16.restype = C.c_uint16
        L.or_f32_to_f16.argtypes = [C.c_float]
        L.or_block.argtypes = [C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]
        L.or_dequantize.argtypes = [C.c_int, _P, C.c_int64, _P]
        L.or_quantize_q8_1.argtypes = [_P, C.c_int64, _P]
        L.or_dequantize_q8_1.argtypes = [_P, C.c_int64, _P]
        L.or_rng_next.restype = C.c_uint64
        L.or_rng_next.argtypes = [C.POINTER(C.c_uint64)]
        L.or_random_blocks.argtypes = [C.c_int, C.c_int64, C.POINTER(C.c_uint64), _P]
        L.or_gemv.argtypes = [C.c_int, _P, C.c_int64, C.c_int, C.c_int, _P, C.c_int64, C.c_int, C.c_int, _P, C.c_int]
        L.or_swiglu.restype = C.c_double
        L.or_swiglu.argtypes = [C.c_double, C.c_double, C.c_double]
        L.or_moe_ffn.argtypes = [C.c_int, C.c_int, _P, _P, _P, C.c_int64, C.c_int64, C.c_int, C.c_int, C.c_int, _P,
                                 C.c_int, _P, _P, _P, C.c_float, _P, _P, C.c_int, C.c_int]
        for name, ty in [("or_table_ksigns", C.c_uint8), ("or_table_iq2xxs", C.c_uint64), ("or_table_iq2s", C.c_uint64),
                         ("or_table_iq3xxs", C.c_uint32), ("or_table_iq4nl", C.c_int8)]:
            getattr(L, name).restype = C.POINTER(ty)
        _LIB = L
    return _LIB


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def block(ty):
    e, b = C.c_int(), C.c_int()
    if lib().or_block(ty, C.byref(e), C.byref(b)) != 0:
        raise ValueError(f"unknown type {ty}")
    return e.value, b.value


def row_bytes(ty, k):
    e, b = block(ty)
    assert k % e == 0
    return k // e * b


def f16_to_f32(h):
    return lib().or_f16_to_f32(h)


def f32_to_f16(f):
    return lib().or_f32_to_f16(f)


def dequantize(ty, raw, n):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    y = np.empty(n, dtype=np.float32)
    if lib().or_dequantize(ty, _ptr(raw), n, _ptr(y)) != 0:
        raise ValueError("dequantize: bad type or size")
    return y


def quantize_q8_1(x):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size % 32 == 0
    out = np.empty(x.size // 32 * Q8_1_BYTES, dtype=np.uint8)
    lib().or_quantize_q8_1(_ptr(x), x.size, _ptr(out))
    return out


def dequantize_q8_1(q, n):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    y = np.empty(n, dtype=np.float32)
    lib().or_dequantize_q8_1(_ptr(q), n, _ptr(y))
    return y


class Rng:
    """xorshift64* of qtest.rs:27-39."""

    def __init__(self, seed):
        self.state = C.c_uint64(seed)

    def next(self):
        return lib().or_rng_next(C.byref(self.state))

    def random_blocks(self, ty, n_elems):
        e, b = block(ty)
        out = np.empty(n_elems // e * b, dtype=np.uint8)
        if lib().or_random_blocks(ty, n_elems, C.byref(self.state), _ptr(out)) != 0:
            raise ValueError("random_blocks: bad type or size")
        return out


ACT = {"f32": 0, "q8_1": 1, "f16": 2, "f16x": 3, "f16s": 4, "f16sx": 5}


def gemv(ty, W, row_stride, K, rows, x, B=1, x_stride=None, quant_x=True, nthreads=1, act=None):
    """f64 y[B][rows] = deq(W) . deq(q8_1(x[b])) (act "q8_1", the default), deq(W) . x (act "f32" or
    quant_x=False), or f16(deq(W)) . f16(x) (act "f16", the reference's multi-token GEMM)."""
    mode = ACT[act] if act is not None else (1 if quant_x else 0)
    W = np.ascontiguousarray(W, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty((B, rows), dtype=np.float64)
    rc = lib().or_gemv(ty, _ptr(W), row_stride, K, rows, _ptr(x), K if x_stride is None else x_stride, B,
                       mode, _ptr(y), nthreads)
    if rc != 0:
        raise ValueError("or_gemv failed")
    return y


def moe_ffn(ty_gu, ty_down, gate, up, down, gu_row_stride, down_row_stride, n_embd, n_ff, x, pair_tok, pair_exp,
            pair_w, lim=0.0, nthreads=1, want_h=False, act="q8_1"):
    """Routed-expert FFN oracle. gate/up/down: lists of uint8 arrays indexed by expert id.
    act: "q8_1" (fused decode path: q8_1 activations), "f16" (multi-token GEMM path, gemm.cu:
    half activations and half-rounded dequantized weights) or "f16x" (half activations, exact
    dequantized weights)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    n_exp = len(gate)
    keep = [np.ascontiguousarray(a, dtype=np.uint8) for a in list(gate) + list(up) + list(down)]
    ptrs = (C.c_void_p * (3 * n_exp))(*[a.ctypes.data for a in keep])
    base = C.addressof(ptrs)
    ps = C.sizeof(C.c_void_p)
    pt = np.ascontiguousarray(pair_tok, dtype=np.int32)
    pe = np.ascontiguousarray(pair_exp, dtype=np.int32)
    pw = np.ascontiguousarray(pair_w, dtype=np.float32)
    y = np.zeros((T, n_embd), dtype=np.float64)
    h = np.empty((len(pt), n_ff), dtype=np.float32) if want_h else None
    rc = lib().or_moe_ffn(ty_gu, ty_down, C.c_void_p(base), C.c_void_p(base + n_exp * ps),
                          C.c_void_p(base + 2 * n_exp * ps), gu_row_stride, down_row_stride, n_embd, n_ff, T, _ptr(x),
                          len(pt), _ptr(pt), _ptr(pe), _ptr(pw), lim, _ptr(y),
                          _ptr(h) if want_h else None, nthreads, ACT[act])
    if rc != 0:
        raise ValueError("or_moe_ffn failed")
    return (y, h) if want_h else y


def table(name, n):
    p = getattr(lib(), "or_table_" + name)()
    return np.ctypeslib.as_array(p, shape=(n,)).copy()
