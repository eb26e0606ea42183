"""Host side of the grouped routed-expert FFN: the pair grouping the engine builds before its
multi-token MoE pass (crates/engine/src/forward.rs:1017-1036, :1335-1349), in the CSR form that
gs_moe_grouped takes, and a resident-layer helper that owns the device arrays."""
import ctypes as C
import os

import numpy as np

from . import DeviceBuffer, ExpertPtrs, ops
from .types import GgmlType as T, row_bytes


def _at(buf, offset):
    """device address buf + offset bytes (buf: DeviceBuffer or c_void_p)"""
    base = buf.p.value if isinstance(buf, DeviceBuffer) else C.c_void_p(buf).value if isinstance(buf, int) else buf.value
    return C.c_void_p(base + offset)


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


def slot_index(routes, idx, pair_exp):
    """Deterministic-combine slot of each pair (forward.rs:1039-1048): (rank of the pair's expert in
    its token's route) * n_tok + token. Every (rank, token) slot is hit by exactly one pair."""
    t = len(routes)
    rank = [{int(e): k for k, (e, _) in enumerate(r)} for r in routes]
    return np.asarray([rank[ti][int(e)] * t + ti for ti, e in zip(idx.tolist(), pair_exp.tolist())], dtype=np.int32)


def deterministic_default():
    """GLMSSD_DETERMINISTIC=1 selects the ordered combine, as the engine reads it (forward.rs:551)."""
    return os.environ.get("GLMSSD_DETERMINISTIC") == "1"


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

    def upload_routes(self, routes, s=None, slots=False):
        """Pairs of `routes` to the device; with `slots`, also each pair's deterministic-combine slot."""
        offs, idx, w, pe = group_pairs(routes, self.n_exp)
        self.n_pairs = int(idx.size)
        self.d_offs = DeviceBuffer.from_array(offs, s)
        self.d_idx = DeviceBuffer.from_array(idx if idx.size else np.zeros(1, np.int32), s)
        self.d_w = DeviceBuffer.from_array(w if w.size else np.zeros(1, np.float32), s)
        self.d_slot = None
        if slots:
            sl = slot_index(routes, idx, pe)
            self.d_slot = DeviceBuffer.from_array(sl if sl.size else np.zeros(1, np.int32), s)
        return offs, idx, w, pe

    def _work(self, n_tok):
        need = ops.moe_grouped_workspace(n_tok, self.n_pairs, self.n_embd, self.n_ff)
        if self.work is None or self.work.nbytes < need:
            self.work = DeviceBuffer(need)
        return self.work

    def forward(self, x_dev, y_dev, n_tok, lim=0.0, s=None):
        """y[token] += every routed expert's weighted FFN output (f32 atomics: run-to-run order varies)"""
        wk = self._work(n_tok)
        ops.moe_grouped(self.ty_gu, self.ty_down, self.table, self.n_exp, self.d_offs, self.d_idx, self.d_w,
                        self.n_pairs, n_tok, self.rs_gu, self.n_embd, self.n_ff, self.rs_down, x_dev, y_dev, lim,
                        wk, wk.nbytes, s)

    def forward_slots(self, x_dev, slots_dev, n_tok, lim=0.0, s=None):
        """slots[rank * n_tok + token] += the pair's weighted FFN output (needs upload_routes(slots=True);
        `slots` zeroed, [k * n_tok][n_embd]): one addition per element, so the result is reproducible."""
        if self.d_slot is None:
            raise ValueError("upload_routes(..., slots=True) first")
        wk = self._work(n_tok)
        ops.moe_grouped_scatter(self.ty_gu, self.ty_down, self.table, self.n_exp, self.d_offs, self.d_idx,
                                self.d_slot, self.d_w, self.n_pairs, n_tok, self.rs_gu, self.n_embd, self.n_ff,
                                self.rs_down, x_dev, slots_dev, lim, wk, wk.nbytes, s)


def route(logits, bias, k, weights_norm=True, weights_scale=1.0):
    """Host routing of forward.rs:964-980 (`Engine::route`): per token, sigmoid scores, the k
    experts with the largest score + bias (descending), weights score / (sum of the chosen
    scores + 1e-20) * scale (the sum is 1 without normalisation). logits: [t][n_expert] f32."""
    logits = np.asarray(logits, dtype=np.float32)
    bias = np.asarray(bias, dtype=np.float32)
    out = []
    for row in logits.reshape(-1, bias.size):
        scores = (1.0 / (1.0 + np.exp(-row.astype(np.float32)))).astype(np.float32)
        sel = scores + bias
        order = sorted(range(bias.size), key=lambda e: -sel[e])[:k]   # stable: ties keep id order
        wsum = np.float32(sum(scores[e] for e in order)) if weights_norm else np.float32(1.0)
        out.append([(e, float(scores[e] / (wsum + np.float32(1e-20)) * np.float32(weights_scale))) for e in order])
    return out


class Mat:
    """A resident weight matrix in GGUF layout: rows of `K` elements of type `ty`."""

    def __init__(self, raw, ty, K, rows, s=None):
        self.ty, self.K, self.rows = ty, K, rows
        self.row_bytes = row_bytes(ty, K)
        self.buf = raw if isinstance(raw, DeviceBuffer) else DeviceBuffer.from_array(np.asarray(raw), s)
        self.offset = 0

    def ptr(self):
        return self.buf.ptr(self.offset)


class MoeLayer:
    """One MoE FFN layer with every expert resident: the work of forward.rs:982-1136
    (`Engine::moe`) without the expert cache. forward(): router logits (F32 GEMV), host routing,
    shared expert SwiGLU FFN into `out`, routed experts into an accumulator (up to 16 tokens: a
    one-token FFN per token over its own experts, in gs_moe_ffn_tokens calls of up to 32 (token,
    expert) pairs, where the engine's decode branch batches up to 16 experts for 1-2 tokens; more
    tokens: the grouped MFMA kernel when every expert matrix is IQ2_XXS or IQ3_XXS, else per-expert
    gather / GEMM / SwiGLU / scatter-add as run_expert_rows), then out += accumulator.

    experts: list of (gate, up, down) host byte arrays; gate/up [n_ff rows x n_embd], down
    [n_embd rows x n_ff].

    deterministic (default: GLMSSD_DETERMINISTIC=1 in the environment, forward.rs:551): the
    engine's ordered combine. One-token FFNs take each token's experts in id order (forward.rs:
    1071-1081); multi-token paths write every (route rank, token) pair into its own slot and sum
    the slots in rank order (forward.rs:1119-1127), so the output is bit-reproducible."""
    MOE_MAX, PER_TOKEN_MAX = 16, 16

    def __init__(self, router, bias, shared, experts, n_embd, n_ff, ty_gu, ty_down, k=8, weights_norm=True,
                 weights_scale=1.0, clamp_exp=0.0, clamp_shexp=0.0, router_ty=T.F32, shared_ty=(T.Q6_K,) * 3,
                 n_ff_shexp=None, s=None, deterministic=None):
        from . import MoeBatch   # noqa: F401  (layout shared with the C ABI)
        self.n_embd, self.n_ff, self.k = n_embd, n_ff, k
        self.deterministic = deterministic_default() if deterministic is None else bool(deterministic)
        self.n_exp = len(experts)
        self.bias = np.asarray(bias, dtype=np.float32)
        self.norm, self.scale, self.lim, self.lim_sh = weights_norm, weights_scale, clamp_exp, clamp_shexp
        self.ty_gu, self.ty_down = ty_gu, ty_down
        self.router = Mat(router, router_ty, n_embd, self.n_exp, s)
        nsh = n_ff if n_ff_shexp is None else n_ff_shexp
        self.sh = [Mat(shared[0], shared_ty[0], n_embd, nsh, s), Mat(shared[1], shared_ty[1], n_embd, nsh, s),
                   Mat(shared[2], shared_ty[2], nsh, n_embd, s)]
        self.n_ff_sh = nsh
        self.gate = [Mat(e[0], ty_gu, n_embd, n_ff, s) for e in experts]
        self.up = [Mat(e[1], ty_gu, n_embd, n_ff, s) for e in experts]
        self.down = [Mat(e[2], ty_down, n_ff, n_embd, s) for e in experts]
        self.grouped = None
        grp = (T.IQ2_XXS, T.IQ3_XXS)
        if ty_gu in grp and ty_down in grp:
            self.grouped = ResidentMoeLayer([e[0] for e in experts], [e[1] for e in experts],
                                            [e[2] for e in experts], n_embd, n_ff, ty_gu, ty_down)
        self._scratch = {}
        self.last_routes = None

    def _buf(self, name, nbytes):
        b = self._scratch.get(name)
        if b is None or b.nbytes < nbytes:
            b = self._scratch[name] = DeviceBuffer(max(nbytes, 4))
        return b

    def _mm(self, m, x, y, t, s, x_stride=None, y_stride=None):
        """forward.rs:700-710 mm_s: GEMV for up to 8 vectors, else GEMM (gs_gemm_ex: small problems
        split K into the layer's workspace; the layer's calls run in order on one stream, so they
        share it)"""
        xs = m.K if x_stride is None else x_stride
        ys = m.rows if y_stride is None else y_stride
        if t <= 8:
            ops.gemv(m.ty, m.ptr(), m.row_bytes, m.K, m.rows, x, xs, y, ys, t, False, s)
        else:
            need = ops.gemm_workspace(m.K, m.rows, t)
            wk = self._buf("gemm_ws", need) if need else None
            ops.gemm_ex(m.ty, m.ptr(), m.row_bytes, m.K, m.rows, x, xs, y, ys, t, False, 1, 0, 0, 0, wk,
                        wk.nbytes if wk else 0, s)

    def forward(self, xn, out, t, s=None):
        """xn: device [t][n_embd] (normalised hidden states); out: device [t][n_embd], overwritten
        with shared-expert FFN + routed-expert FFN. Returns the routes."""
        from . import MoeBatch
        n, ne = self.n_embd, self.n_exp
        logits_d = self._buf("logits", t * ne * 4)
        self._mm(self.router, xn, logits_d, t, s)
        logits = logits_d.download(np.float32, t * ne, s)
        routes = route(logits.reshape(t, ne), self.bias, self.k, self.norm, self.scale)
        self.last_routes = routes
        # shared expert (forward.rs:1108-1110, swiglu_ffn :915-921)
        g, u = self._buf("sh_g", t * self.n_ff_sh * 4), self._buf("sh_u", t * self.n_ff_sh * 4)
        self._mm(self.sh[0], xn, g, t, s)
        self._mm(self.sh[1], xn, u, t, s)
        ops.swiglu(g, u, g, t * self.n_ff_sh, self.lim_sh, s)
        self._mm(self.sh[2], g, out, t, s)
        acc = self._buf("acc", t * n * 4)
        acc.zero(s)
        groups = [[] for _ in range(ne)]
        for ti, r in enumerate(routes):
            for e, w in r:
                groups[e].append((ti, w))
        used = [e for e in range(ne) if groups[e]]
        if t <= self.PER_TOKEN_MAX:
            # decode, MTP and short-batch sizes: a one-token FFN per token over its own experts, the
            # tokens in gs_moe_ffn_tokens calls of up to 32 (token, expert) pairs when their expert
            # counts are equal. On the config-2 experts (top-8 of 288, Zipf routing) 2/4/8/16 tokens
            # take 23/40/88/167 us this way against 70/109/134/202 us through the grouped GEMM.
            routes_d = [sorted(r, key=lambda ew: ew[0]) if self.deterministic else r for r in routes]
            kk = len(routes_d[0])
            if t > 1 and all(len(r) == kk for r in routes_d) and 0 < kk <= self.MOE_MAX:
                per = max(1, 32 // kk)
                h = self._buf("h", min(t, per) * kk * self.n_ff * 4)
                for t0 in range(0, t, per):
                    bs = []
                    for r in routes_d[t0:t0 + per]:
                        b = MoeBatch()
                        b.n = kk
                        for i, (e, w) in enumerate(r):
                            b.gate[i], b.up[i], b.down[i] = (self.gate[e].ptr().value, self.up[e].ptr().value,
                                                             self.down[e].ptr().value)
                            b.w[0][i] = w
                        bs.append(b)
                    ops.moe_ffn_tokens(self.ty_gu, self.ty_down, bs, self.gate[0].row_bytes, n, self.n_ff,
                                       self.down[0].row_bytes, _at(xn, t0 * n * 4), h, acc.ptr(t0 * n * 4),
                                       self.lim, s)
                routes_d = []
            h = self._buf("h", self.MOE_MAX * self.n_ff * 4)
            for ti, r in enumerate(routes_d):
                for b0 in range(0, len(r), self.MOE_MAX):
                    chunk = r[b0:b0 + self.MOE_MAX]
                    b = MoeBatch()
                    b.n = len(chunk)
                    for i, (e, w) in enumerate(chunk):
                        b.gate[i], b.up[i], b.down[i] = (self.gate[e].ptr().value, self.up[e].ptr().value,
                                                         self.down[e].ptr().value)
                        b.w[0][i] = w
                    ops.moe_ffn(self.ty_gu, self.ty_down, b, 1, self.gate[0].row_bytes, n, self.n_ff,
                                self.down[0].row_bytes, _at(xn, ti * n * 4), h, acc.ptr(ti * n * 4), self.lim, s)
        elif self.grouped is not None:
            self.grouped.upload_routes(routes, s, slots=self.deterministic)
            if self.deterministic:
                slots = self._buf("slots", self.k * t * n * 4)
                slots.zero(s)
                self.grouped.forward_slots(xn, slots, t, self.lim, s)
                self._sum_slots(acc, slots, t, s)
            else:
                self.grouped.forward(xn, acc, t, self.lim, s)
        else:
            # run_expert_rows (forward.rs:1399-1413) per used expert
            offs, idx, w, pe = group_pairs(routes, ne)
            d_idx, d_w = DeviceBuffer.from_array(idx, s), DeviceBuffer.from_array(w, s)
            to, slots = d_idx, None
            if self.deterministic:
                to = DeviceBuffer.from_array(slot_index(routes, idx, pe), s)
                slots = self._buf("slots", self.k * t * n * 4)
                slots.zero(s)
            m_max = max(len(groups[e]) for e in used)
            xg = self._buf("xg", m_max * n * 4)
            eg, eu = self._buf("eg", m_max * self.n_ff * 4), self._buf("eu", m_max * self.n_ff * 4)
            ey = self._buf("ey", m_max * n * 4)
            for e in used:
                m, o = len(groups[e]), int(offs[e])
                ops.gather_rows(xn, d_idx.ptr(4 * o), xg, m, n, s)
                self._mm(self.gate[e], xg, eg, m, s)
                self._mm(self.up[e], xg, eu, m, s)
                ops.swiglu(eg, eu, eg, m * self.n_ff, self.lim, s)
                self._mm(self.down[e], eg, ey, m, s)
                ops.scatter_add_rows(acc if slots is None else slots, to.ptr(4 * o), d_w.ptr(4 * o), ey, m, n, s)
            if slots is not None:
                self._sum_slots(acc, slots, t, s)
        ops.axpy(out, acc, 1.0, t * n, s)
        return routes

    def _sum_slots(self, acc, slots, t, s):
        """acc += slots[rank] for rank 0..k-1 in order (forward.rs:1122-1127)"""
        n = self.n_embd
        for r in range(self.k):
            ops.axpy(acc, slots.ptr(4 * r * t * n), 1.0, t * n, s)
