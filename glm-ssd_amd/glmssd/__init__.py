"""Python host binding of libglmssd_hip.so (ctypes over the gs_* C ABI in include/glmssd.h).

Mirrors the safe wrappers GLM-SSD's Rust host keeps around the same ABI
(crates/cuda/src/lib.rs:127-443): `check` turns a nonzero return into an exception carrying
gs_error_string (lib.rs:169-175); `Stream`, `Event`, `DeviceBuffer`, `PinnedBuffer` own the
runtime objects (lib.rs:202-366); `ops` holds the quantized ops (lib.rs:127-155); `MoeBatch` is
the repr(C) fused-MoE batch (lib.rs:411-429). Everything computes through the HIP library; there
is no CPU fallback, and loading fails loudly when the library is missing.
"""
import ctypes as C
import os

import numpy as np

from .types import GgmlType, block, row_bytes, TYPE_NAMES  # noqa: F401

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "libglmssd_hip.so")
_LIB = None

MOE_MAX = 16
MOE_NT = 2
_P = C.c_void_p
_I64 = C.c_int64


class GsError(RuntimeError):
    pass


class MoeBatch(C.Structure):
    """#[repr(C)] fused-MoE batch (crates/cuda/src/lib.rs:417-424)."""
    _fields_ = [("gate", C.c_void_p * MOE_MAX), ("up", C.c_void_p * MOE_MAX), ("down", C.c_void_p * MOE_MAX),
                ("w", (C.c_float * MOE_MAX) * MOE_NT), ("n", C.c_int)]


class ExpertPtrs(C.Structure):
    """Device pointers of one routed expert's gate / up / down matrices (GsExpertPtrs; the
    engine's ExpertPtrs, crates/engine/src/experts.rs:133-137)."""
    _fields_ = [("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p)]


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 256), ("cc_major", C.c_int), ("cc_minor", C.c_int), ("sm_count", C.c_int),
                ("total_mem", C.c_uint64), ("free_mem", C.c_uint64), ("pci_bus", C.c_int), ("pci_device", C.c_int),
                ("async_engines", C.c_int), ("can_map_host", C.c_int)]


# signature table: name -> argtypes (all return int unless noted)
SIGNATURES = {
    "gs_device_info": [C.c_int, C.POINTER(DeviceInfo)],
    "gs_malloc": [C.POINTER(C.c_void_p), C.c_size_t],
    "gs_free": [_P],
    "gs_host_alloc": [C.POINTER(C.c_void_p), C.c_size_t],
    "gs_host_free": [_P],
    "gs_host_register": [_P, C.c_size_t],
    "gs_host_unregister": [_P],
    "gs_stream_create": [C.POINTER(C.c_void_p)],
    "gs_stream_destroy": [_P],
    "gs_stream_sync": [_P],
    "gs_device_sync": [],
    "gs_device_reset": [],
    "gs_memcpy_h2d": [_P, _P, C.c_size_t, _P],
    "gs_memcpy_d2h": [_P, _P, C.c_size_t, _P],
    "gs_memcpy_d2d": [_P, _P, C.c_size_t, _P],
    "gs_event_create": [C.POINTER(C.c_void_p)],
    "gs_event_create_timed": [C.POINTER(C.c_void_p)],
    "gs_event_destroy": [_P],
    "gs_event_record": [_P, _P],
    "gs_event_sync": [_P],
    "gs_event_query": [_P],
    "gs_stream_wait_event": [_P, _P],
    "gs_event_elapsed_ms": [C.POINTER(C.c_float), _P, _P],
    "gs_memset": [_P, C.c_int, C.c_size_t, _P],
    "gs_saxpy": [C.c_int, C.c_float, _P, _P, _P],
    "gs_dequant_f32": [C.c_int, _P, _I64, _P, _P],
    "gs_dequant_f16": [C.c_int, _P, _I64, _P, _P],
    "gs_gemv": [C.c_int, _P, _I64, C.c_int, C.c_int, _P, _I64, _P, _I64, C.c_int, C.c_int, _P],
    "gs_gemv_batched": [C.c_int, _P, _I64, C.c_int, C.c_int, _P, _P, C.c_int, _I64, _I64, _I64, _P],
    "gs_moe_gateup": [C.c_int, C.POINTER(MoeBatch), C.c_int, _I64, C.c_int, C.c_int, _P, _P, C.c_float, _P],
    "gs_moe_down": [C.c_int, C.POINTER(MoeBatch), C.c_int, _I64, C.c_int, C.c_int, _P, _P, _P],
    "gs_moe_ffn": [C.c_int, C.c_int, C.POINTER(MoeBatch), C.c_int, _I64, C.c_int, C.c_int, _I64, _P, _P, _P, C.c_float,
                   _P],
    "gs_moe_ffn_tokens": [C.c_int, C.c_int, C.POINTER(MoeBatch), C.c_int, _I64, C.c_int, C.c_int, _I64, _P, _P, _P,
                          C.c_float, _P],
    "gs_swiglu": [_P, _P, _P, _I64, C.c_float, _P],
    "gs_axpy": [_P, _P, C.c_float, _I64, _P],
    "gs_gemm": [C.c_int, _P, _I64, C.c_int, C.c_int, _P, _I64, _P, _I64, C.c_int, C.c_int, C.c_int, _I64, _I64, _I64,
                _P],
    "gs_gemm_workspace": [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_size_t)],
    "gs_gemm_path": [C.c_int, C.c_int, C.c_int, C.c_int, _I64, _I64, C.c_size_t],
    "gs_gemm_ex": [C.c_int, _P, _I64, C.c_int, C.c_int, _P, _I64, _P, _I64, C.c_int, C.c_int, C.c_int, _I64, _I64,
                   _I64, _P, C.c_size_t, _P],
    "gs_wait_status": [_P],
    "gs_debug_wait_limit": [C.c_uint32, C.c_int],
    "gs_gather_rows": [_P, _P, _P, C.c_int, C.c_int, _P],
    "gs_scatter_add_rows": [_P, _P, _P, _P, C.c_int, C.c_int, _P],
    "gs_f32_to_f16": [_P, _P, _I64, _P],
    "gs_quant_q8_1": [_P, _P, _I64, _P],
    "gs_moe_grouped_workspace": [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_size_t)],
    "gs_moe_grouped": [C.c_int, C.c_int, _P, C.c_int, _P, _P, _P, C.c_int, C.c_int, _I64, C.c_int, C.c_int, _I64,
                       _P, _P, C.c_float, _P, C.c_size_t, _P],
    "gs_moe_grouped_scatter": [C.c_int, C.c_int, _P, C.c_int, _P, _P, _P, _P, C.c_int, C.c_int, _I64, C.c_int,
                               C.c_int, _I64, _P, _P, C.c_float, _P, C.c_size_t, _P],
    "gs_moe_grouped_noalloc": [C.c_int, C.c_int, _P, C.c_int, _P, _P, _P, C.c_int, C.c_int, _I64, C.c_int, C.c_int,
                               _I64, _P, _P, C.c_float, _P],
}


def lib():
    """Load libglmssd_hip.so (built in-tree by `make -C glm-ssd_amd` / __graft_entry__.build())."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise GsError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = C.c_int
        L.gs_error_string.argtypes = [C.c_int]
        L.gs_error_string.restype = C.c_char_p
        _LIB = L
    return _LIB


def check(code):
    """Nonzero return -> GsError with the runtime's message (crates/cuda/src/lib.rs:169-175)."""
    if code != 0:
        msg = lib().gs_error_string(code)
        raise GsError(f"HIP error {code}: {msg.decode() if msg else '?'}")


def device_info(dev=0):
    i = DeviceInfo()
    check(lib().gs_device_info(dev, C.byref(i)))
    return i


class Stream:
    def __init__(self):
        self.h = C.c_void_p()
        check(lib().gs_stream_create(C.byref(self.h)))

    def raw(self):
        return self.h

    def sync(self):
        check(lib().gs_stream_sync(self.h))

    def close(self):
        if self.h:
            check(lib().gs_stream_destroy(self.h))
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self, timed=True):
        self.h = C.c_void_p()
        check((lib().gs_event_create_timed if timed else lib().gs_event_create)(C.byref(self.h)))

    def record(self, s):
        check(lib().gs_event_record(self.h, s.raw()))

    def sync(self):
        check(lib().gs_event_sync(self.h))

    def elapsed_ms(self, later):
        ms = C.c_float()
        check(lib().gs_event_elapsed_ms(C.byref(ms), self.h, later.h))
        return ms.value

    def __del__(self):
        try:
            if self.h:
                lib().gs_event_destroy(self.h)
        except Exception:
            pass


class DeviceBuffer:
    """Owned device allocation (crates/cuda/src/lib.rs:290-330)."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.p = C.c_void_p()
        check(lib().gs_malloc(C.byref(self.p), max(1, self.nbytes)))

    @classmethod
    def from_array(cls, a, s=None):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a, s)
        return b

    def ptr(self, offset=0):
        return C.c_void_p(self.p.value + offset)

    def upload(self, a, s=None, offset=0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(lib().gs_memcpy_h2d(self.ptr(offset), a.ctypes.data_as(_P), a.nbytes, s.raw() if s else None))
        if s is None:
            check(lib().gs_device_sync())
        else:
            s.sync()

    def download(self, dtype, count=None, s=None, offset=0):
        dtype = np.dtype(dtype)
        count = (self.nbytes - offset) // dtype.itemsize if count is None else count
        out = np.empty(count, dtype=dtype)
        check(lib().gs_memcpy_d2h(out.ctypes.data_as(_P), self.ptr(offset), out.nbytes, s.raw() if s else None))
        if s is None:
            check(lib().gs_device_sync())
        else:
            s.sync()
        return out

    def zero(self, s=None):
        check(lib().gs_memset(self.p, 0, self.nbytes, s.raw() if s else None))

    def free(self):
        if self.p:
            check(lib().gs_free(self.p))
            self.p = C.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _raw(s):
    return s.raw() if s is not None else None


def _p(x):
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.p
    if isinstance(x, C.c_void_p):
        return x
    return C.c_void_p(int(x))


class ops:
    """Quantized ops; all pointers are device pointers (crates/cuda/src/lib.rs:127-155)."""

    @staticmethod
    def dequant_f32(ty, src, n, dst, s=None):
        check(lib().gs_dequant_f32(ty, _p(src), n, _p(dst), _raw(s)))

    @staticmethod
    def dequant_f16(ty, src, n, dst, s=None):
        check(lib().gs_dequant_f16(ty, _p(src), n, _p(dst), _raw(s)))

    @staticmethod
    def quant_q8_1(x, q, n, s=None):
        check(lib().gs_quant_q8_1(_p(x), _p(q), n, _raw(s)))

    @staticmethod
    def gemv(ty, w, row_stride, k, rows, x, x_stride, y, y_stride, n_vec, accumulate=False, s=None):
        check(lib().gs_gemv(ty, _p(w), row_stride, k, rows, _p(x), x_stride, _p(y), y_stride, n_vec,
                            1 if accumulate else 0, _raw(s)))

    @staticmethod
    def gemv_batched(ty, w, row_stride, k, rows, x, y, n_batch, w_bs, x_bs, y_bs, s=None):
        check(lib().gs_gemv_batched(ty, _p(w), row_stride, k, rows, _p(x), _p(y), n_batch, w_bs, x_bs, y_bs, _raw(s)))

    @staticmethod
    def moe_gateup(ty, batch, nt, row_stride, k, rows, x, h, lim=0.0, s=None):
        check(lib().gs_moe_gateup(ty, C.byref(batch), nt, row_stride, k, rows, _p(x), _p(h), lim, _raw(s)))

    @staticmethod
    def moe_down(ty, batch, nt, row_stride, k, rows, h, y, s=None):
        check(lib().gs_moe_down(ty, C.byref(batch), nt, row_stride, k, rows, _p(h), _p(y), _raw(s)))

    @staticmethod
    def moe_ffn(ty_gu, ty_dn, batch, nt, rs_gu, n_embd, n_ff, rs_dn, x, h, y, lim=0.0, s=None):
        """gs_moe_ffn: moe_gateup then moe_down."""
        check(lib().gs_moe_ffn(ty_gu, ty_dn, C.byref(batch), nt, rs_gu, n_embd, n_ff, rs_dn, _p(x), _p(h), _p(y), lim,
                               _raw(s)))

    @staticmethod
    def moe_ffn_tokens(ty_gu, ty_dn, batches, rs_gu, n_embd, n_ff, rs_dn, x, h, y, lim=0.0, s=None):
        """gs_moe_ffn_tokens: moe_ffn of token t over batches[t] (one token each, equal expert counts),
        x and y [n_tok][n_embd], h [n_tok][n][n_ff], in one gate/up and one down launch."""
        arr = (MoeBatch * len(batches))(*batches)
        check(lib().gs_moe_ffn_tokens(ty_gu, ty_dn, arr, len(batches), rs_gu, n_embd, n_ff, rs_dn, _p(x), _p(h), _p(y),
                                      lim, _raw(s)))


    @staticmethod
    def gemm(ty, w, row_stride, k, rows, x, x_stride, y, y_stride, n, accumulate=False, n_batch=1, w_bs=0, x_bs=0,
             y_bs=0, s=None):
        check(lib().gs_gemm(ty, _p(w), row_stride, k, rows, _p(x), x_stride, _p(y), y_stride, n,
                            1 if accumulate else 0, n_batch, w_bs, x_bs, y_bs, _raw(s)))

    @staticmethod
    def gemm_workspace(k, rows, n, n_batch=1):
        """gs_gemm_workspace: bytes of workspace gs_gemm_ex would use (K-split partials, or the f16
        operands of the library path from N = 256, or above 128 at rows*K >= 2^25; 0: none)."""
        b = C.c_size_t()
        check(lib().gs_gemm_workspace(k, rows, n, n_batch, C.byref(b)))
        return b.value

    @staticmethod
    def gemm_path(ty, k, rows, n, row_stride, y_stride, work_bytes):
        """gs_gemm_path: 0 f16 MFMA tiles, 1 tiles with the K split, 2 f16 dequant + hipBLASLt."""
        r = lib().gs_gemm_path(int(ty), k, rows, n, row_stride, y_stride, work_bytes)
        if r < 0:
            check(-r)
        return r

    @staticmethod
    def gemm_ex(ty, w, row_stride, k, rows, x, x_stride, y, y_stride, n, accumulate=False, n_batch=1, w_bs=0, x_bs=0,
                y_bs=0, work=None, work_bytes=0, s=None):
        """gs_gemm_ex: gs_gemm with a caller workspace (K split of small problems, or the f16
        operands of the dequant + library GEMM path at many tokens; gemm_path says which)."""
        check(lib().gs_gemm_ex(ty, _p(w), row_stride, k, rows, _p(x), x_stride, _p(y), y_stride, n,
                               1 if accumulate else 0, n_batch, w_bs, x_bs, y_bs, _p(work), work_bytes, _raw(s)))

    @staticmethod
    def wait_status(s=None):
        """gs_wait_status: raises GsError if a bounded LDS wait expired since the last query."""
        check(lib().gs_wait_status(_raw(s)))

    @staticmethod
    def debug_wait_limit(polls, force=False):
        """gs_debug_wait_limit: test hook for the bounded LDS waits (poll bound, forced expiry)."""
        check(lib().gs_debug_wait_limit(polls, 1 if force else 0))

    @staticmethod
    def moe_grouped_workspace(n_tok, n_pairs, k, n_ff):
        n = C.c_size_t()
        check(lib().gs_moe_grouped_workspace(n_tok, n_pairs, k, n_ff, C.byref(n)))
        return n.value

    @staticmethod
    def moe_grouped(ty_gu, ty_down, experts, n_exp, offs, idx, w, n_pairs, n_tok, gu_row_stride, k, n_ff,
                    down_row_stride, x, y, lim, work, work_bytes, s=None):
        check(lib().gs_moe_grouped(ty_gu, ty_down, _p(experts), n_exp, _p(offs), _p(idx), _p(w), n_pairs, n_tok,
                                   gu_row_stride, k, n_ff, down_row_stride, _p(x), _p(y), lim, _p(work), work_bytes,
                                   _raw(s)))

    @staticmethod
    def moe_grouped_scatter(ty_gu, ty_down, experts, n_exp, offs, idx, out_idx, w, n_pairs, n_tok, gu_row_stride,
                            k, n_ff, down_row_stride, x, y, lim, work, work_bytes, s=None):
        """gs_moe_grouped_scatter: pair p adds into y[out_idx[p]] (the deterministic slot combine)."""
        check(lib().gs_moe_grouped_scatter(ty_gu, ty_down, _p(experts), n_exp, _p(offs), _p(idx), _p(out_idx),
                                           _p(w), n_pairs, n_tok, gu_row_stride, k, n_ff, down_row_stride, _p(x),
                                           _p(y), lim, _p(work), work_bytes, _raw(s)))

    @staticmethod
    def moe_grouped_noalloc(ty_gu, ty_down, experts, n_exp, offs, idx, w, n_pairs, n_tok, gu_row_stride, k, n_ff,
                            down_row_stride, x, y, lim, s=None):
        """gs_moe_grouped_noalloc: gs_moe_grouped with the library's per-GPU workspace array."""
        check(lib().gs_moe_grouped_noalloc(ty_gu, ty_down, _p(experts), n_exp, _p(offs), _p(idx), _p(w), n_pairs,
                                           n_tok, gu_row_stride, k, n_ff, down_row_stride, _p(x), _p(y), lim,
                                           _raw(s)))

    @staticmethod
    def swiglu(g, u, y, n, lim=0.0, s=None):
        check(lib().gs_swiglu(_p(g), _p(u), _p(y), n, lim, _raw(s)))

    @staticmethod
    def axpy(y, x, a, n, s=None):
        check(lib().gs_axpy(_p(y), _p(x), a, n, _raw(s)))

    @staticmethod
    def gather_rows(x, idx, y, rows, n, s=None):
        check(lib().gs_gather_rows(_p(x), _p(idx), _p(y), rows, n, _raw(s)))

    @staticmethod
    def scatter_add_rows(acc, idx, w, y, rows, n, s=None):
        check(lib().gs_scatter_add_rows(_p(acc), _p(idx), _p(w), _p(y), rows, n, _raw(s)))
