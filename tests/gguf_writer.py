"""Small GGUF v3 writer for the tests (the shape of the reference's test writer, crates/gguf/src/
lib.rs:402-447: key/values, tensor infos, zero-padded data start). Test infrastructure only."""
import struct


def _s(v):
    b = v.encode() if isinstance(v, str) else v
    return struct.pack("<Q", len(b)) + b


class Writer:
    def __init__(self):
        self.kv = b""
        self.n_kv = 0
        self.ti = b""
        self.n_t = 0

    def kv_u32(self, k, v):
        return self.kv_raw(k, 4, struct.pack("<I", v))

    def kv_str(self, k, v):
        return self.kv_raw(k, 8, _s(v))

    def kv_f32(self, k, v):
        return self.kv_raw(k, 6, struct.pack("<f", v))

    def kv_raw(self, k, ty, body):
        self.kv += _s(k) + struct.pack("<I", ty) + body
        self.n_kv += 1
        return self

    def tensor(self, name, dims, ty, off):
        self.ti += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        self.ti += struct.pack("<IQ", ty, off)
        self.n_t += 1
        return self

    def header(self, n_t=None, n_kv=None):
        return (b"GGUF" + struct.pack("<IQQ", 3, self.n_t if n_t is None else n_t, self.n_kv if n_kv is None else n_kv)
                + self.kv + self.ti)

    def build(self, data=0, n_t=None, n_kv=None, align=32):
        """header, zero padding to the aligned data start, then `data` bytes (an int: zeros)"""
        b = self.header(n_t, n_kv)
        b += b"\0" * ((-len(b)) % align)
        return b + (b"\0" * data if isinstance(data, int) else data)
