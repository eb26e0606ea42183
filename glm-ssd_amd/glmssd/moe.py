"""Host side of the grouped routed-expert FFN: the pair grouping the engine builds before its
multi-token MoE pass (crates/engine/src/forward.rs:1017-1036, :1335-1349), in the CSR form that
gs_moe_grouped takes, and a resident-layer helper that owns the device arrays."""
import ctypes as C

import numpy as np

from . import DeviceBuffer, ExpertPtrs, ops
from .types import GgmlType as T, row_bytes


def group_pairs(routes, n_exp):
    """routes: per token a sequence of (expert, weight). Returns (offs[n_exp+1], idx, w, pair_exp):
    pairs sorted by expert (ascending id), within an expert in token order, as forward.rs
    groups[e].push((ti, w)) then flattens the used experts in id order."""
    groups = [[] for _ in range(n_exp)]
    for ti, r in enumerate(routes):
        for e, wt in r:
            e = int(e)
            if not 0 <= e < n_exp:
                raise ValueError(f"expert id {e} out of range 0..{n_exp - 1}")
            groups[e].append((ti, float(wt)))
    offs = np.zeros(n_exp + 1, dtype=np.int32)
    idx, w, pe = [], [], []
    for e in range(n_exp):
        offs[e] = len(idx)
        for ti, wt in groups[e]:
            idx.append(ti)
            w.append(wt)
            pe.append(e)
    offs[n_exp] = len(idx)
    return (offs, np.asarray(idx, dtype=np.int32), np.asarray(w, dtype=np.float32), np.asarray(pe, dtype=np.int32))


class ResidentMoeLayer:
    """Every routed expert of one MoE layer resident in device memory, plus the GsExpertPtrs
    table gs_moe_grouped reads."""

    def __init__(self, gate, up, down, n_embd, n_ff, ty_gu=T.IQ2_XXS, ty_down=T.IQ2_XXS):
        self.n_exp, self.n_embd, self.n_ff = len(gate), n_embd, n_ff
        self.ty_gu, self.ty_down = ty_gu, ty_down
        self.rs_gu, self.rs_down = row_bytes(ty_gu, n_embd), row_bytes(ty_down, n_ff)
        self.bufs = [DeviceBuffer.from_array(a) for a in list(gate) + list(up) + list(down)]
        n = self.n_exp
        tab = (ExpertPtrs * n)()
        for e in range(n):
            tab[e].gate, tab[e].up, tab[e].down = (self.bufs[e].p.value, self.bufs[n + e].p.value,
                                                   self.bufs[2 * n + e].p.value)
        self.table = DeviceBuffer.from_array(np.frombuffer(bytes(tab), dtype=np.uint8))
        self.work = None

    def upload_routes(self, routes, s=None):
        offs, idx, w, pe = group_pairs(routes, self.n_exp)
        self.n_pairs = int(idx.size)
        self.d_offs = DeviceBuffer.from_array(offs, s)
        self.d_idx = DeviceBuffer.from_array(idx if idx.size else np.zeros(1, np.int32), s)
        self.d_w = DeviceBuffer.from_array(w if w.size else np.zeros(1, np.float32), s)
        return offs, idx, w, pe

    def forward(self, x_dev, y_dev, n_tok, lim=0.0, s=None):
        need = ops.moe_grouped_workspace(n_tok, self.n_pairs, self.n_embd, self.n_ff)
        if self.work is None or self.work.nbytes < need:
            self.work = DeviceBuffer(need)
        ops.moe_grouped(self.ty_gu, self.ty_down, self.table, self.n_exp, self.d_offs, self.d_idx, self.d_w,
                        self.n_pairs, n_tok, self.rs_gu, self.n_embd, self.n_ff, self.rs_down, x_dev, y_dev, lim,
                        self.work, self.work.nbytes, s)
