"""Python view of the library's GGUF v3 header reader (include/glmssd_gguf.h), mirroring
GLM-SSD's crates/gguf (src/lib.rs): Gguf.open / open_headers_only / open_shard, tensor infos
with absolute (shard, offset, n_bytes), metadata getters, slice_range for 3-D expert tensors.
Parsing is native (glm-ssd_amd/csrc/gguf.cpp); this module only binds it and reads tensor bytes."""
import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import lib as _lib

NAME_MAX = 256
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)


class GgufError(Exception):
    pass


class _Tensor(C.Structure):
    _fields_ = [("name", C.c_char * NAME_MAX), ("n_dims", C.c_int), ("dims", C.c_uint64 * 4), ("ty", C.c_int),
                ("shard", C.c_int), ("offset", C.c_uint64), ("n_bytes", C.c_uint64), ("row_bytes", C.c_uint64)]


_SIGS = {
    "gs_gguf_open": ([C.c_char_p, C.c_int, C.POINTER(C.c_void_p)], C.c_int),
    "gs_gguf_close": ([C.c_void_p], None),
    "gs_gguf_error": ([], C.c_char_p),
    "gs_gguf_n_shards": ([C.c_void_p], C.c_int),
    "gs_gguf_shard_path": ([C.c_void_p, C.c_int, C.c_char_p, C.c_size_t], C.c_int),
    "gs_gguf_n_tensors": ([C.c_void_p], C.c_int),
    "gs_gguf_tensor": ([C.c_void_p, C.c_int, C.POINTER(_Tensor)], C.c_int),
    "gs_gguf_find": ([C.c_void_p, C.c_char_p], C.c_int),
    "gs_gguf_slice_range": ([C.POINTER(_Tensor), C.c_uint64, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)], C.c_int),
    "gs_gguf_kv_type": ([C.c_void_p, C.c_char_p], C.c_int),
    "gs_gguf_kv_u64": ([C.c_void_p, C.c_char_p, C.POINTER(C.c_uint64)], C.c_int),
    "gs_gguf_kv_f64": ([C.c_void_p, C.c_char_p, C.POINTER(C.c_double)], C.c_int),
    "gs_gguf_kv_str": ([C.c_void_p, C.c_char_p, C.c_char_p, C.c_size_t], C.c_int),
    "gs_gguf_kv_arr": ([C.c_void_p, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_uint64)], C.c_int),
}
_BOUND = None


def _L():
    global _BOUND
    if _BOUND is None:
        L = _lib()
        for name, (args, res) in _SIGS.items():
            f = getattr(L, name)
            f.argtypes, f.restype = args, res
        _BOUND = L
    return _BOUND


def _check(rc):
    if rc < 0:
        raise GgufError(_L().gs_gguf_error().decode(errors="replace"))
    return rc


@dataclass
class TensorInfo:
    """lib.rs:86-112. dims in GGML order (dims[0] contiguous)."""
    name: str
    dims: tuple
    ty: int
    shard: int
    offset: int
    n_bytes: int
    row_bytes: int
    _raw: object = None

    def n_elements(self):
        n = 1
        for d in self.dims:
            n *= d
        return n

    def slice_range(self, e):
        """byte (offset, size) of expert e of a tensor whose last dim counts experts"""
        off, n = C.c_uint64(), C.c_uint64()
        _check(_L().gs_gguf_slice_range(C.byref(self._raw), e, C.byref(off), C.byref(n)))
        return off.value, n.value


class Gguf:
    """A parsed model header (crates/gguf Gguf). mode: "all" (every shard, sizes checked),
    "headers" (no file-length check), "shard" (this one file)."""
    MODES = {"all": 0, "headers": 1, "shard": 2}

    def __init__(self, path, mode="all"):
        h = C.c_void_p()
        _check(_L().gs_gguf_open(str(path).encode(), self.MODES[mode], C.byref(h)))
        self._h = h
        L = _L()
        buf = C.create_string_buffer(4096)
        self.shards = []
        for i in range(_check(L.gs_gguf_n_shards(h))):
            _check(L.gs_gguf_shard_path(h, i, buf, len(buf)))
            self.shards.append(buf.value.decode())
        self.tensors = []
        for i in range(_check(L.gs_gguf_n_tensors(h))):
            t = _Tensor()
            _check(L.gs_gguf_tensor(h, i, C.byref(t)))
            self.tensors.append(TensorInfo(t.name.decode(), tuple(t.dims[:t.n_dims]), t.ty, t.shard, t.offset,
                                           t.n_bytes, t.row_bytes, t))
        self.by_name = {t.name: i for i, t in enumerate(self.tensors)}

    @classmethod
    def open(cls, path):
        return cls(path, "all")

    @classmethod
    def open_headers_only(cls, path):
        return cls(path, "headers")

    @classmethod
    def open_shard(cls, path):
        return cls(path, "shard")

    def close(self):
        if self._h:
            _L().gs_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor(self, name):
        i = self.by_name.get(name)
        return None if i is None else self.tensors[i]

    def kv_type(self, key):
        rc = _L().gs_gguf_kv_type(self._h, key.encode())
        return None if rc < 0 else rc

    def u64(self, key):
        v = C.c_uint64()
        _check(_L().gs_gguf_kv_u64(self._h, key.encode(), C.byref(v)))
        return v.value

    def f64(self, key):
        v = C.c_double()
        _check(_L().gs_gguf_kv_f64(self._h, key.encode(), C.byref(v)))
        return v.value

    def str(self, key):
        buf = C.create_string_buffer(1 << 16)
        _check(_L().gs_gguf_kv_str(self._h, key.encode(), buf, len(buf)))
        return buf.value.decode(errors="replace")

    def arr(self, key):
        et, n = C.c_int(), C.c_uint64()
        _check(_L().gs_gguf_kv_arr(self._h, key.encode(), C.byref(et), C.byref(n)))
        return et.value, n.value

    def arch(self):
        return self.str("general.architecture")

    def read(self, t, offset=0, n_bytes=None):
        """bytes [offset, offset+n_bytes) of tensor t's data (relative to the tensor), as uint8"""
        n = t.n_bytes - offset if n_bytes is None else n_bytes
        if offset < 0 or n < 0 or offset + n > t.n_bytes:
            raise GgufError(f"{t.name}: byte range out of the tensor")
        with open(self.shards[t.shard], "rb") as f:
            f.seek(t.offset + offset)
            b = f.read(n)
        if len(b) != n:
            raise GgufError(f"{t.name}: truncated file")
        return np.frombuffer(b, dtype=np.uint8).copy()
