"""HIP graph capture of the matmul calls. A decode-and-verify step made of

  * gs_moe_ffn at config 2's shape (8 IQ2_XXS experts, 4096/1536, one token),
  * gs_gemv: Q4_K one vector (streaming kernel) and Q8_0 four vectors (int8 MFMA pass),
  * gs_moe_grouped_scatter (the deterministic grouped FFN, 20 tokens top-4 of 8 experts),
  * gs_gemm (f16 MFMA tiles, 37 tokens) and gs_gemm_ex on its hipBLASLt path (256 tokens),

is captured once on a stream (global capture mode: the calls may not allocate, synchronize or
touch the device outside the stream) and the graph is replayed. Before each replay fresh inputs
are copied into the captured buffers and the accumulated outputs reset, with an eager call and a
synchronization in between; every replay must equal the same calls run eagerly on those inputs,
bit for bit (every call here is deterministic). The calls record no memset nodes, so replays
after the first see the same operations as the first."""
import ctypes as C
import sys

import numpy as np
import pytest

import glmssd as G
from glmssd import GgmlType as T
from glmssd import moe as M
from glmssd import synth

pytestmark = pytest.mark.gpu

CAPTURE_GLOBAL = 0   # hipStreamCaptureModeGlobal


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _hip():
    """The HIP runtime the library is linked against (already loaded in this process)."""
    G.lib()
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64.so" in line:
                return C.CDLL(line.split()[-1])
    raise RuntimeError("libamdhip64 not loaded")


def _ok(rc, what):
    assert rc == 0, f"{what}: hip error {rc}"


class Step:
    """The buffers and calls of one step; run(s) issues every call on stream s."""

    def __init__(self, s):
        wr = np.random.default_rng(4242)
        self.nrng = np.random.default_rng(4243)
        nr = self.nrng
        # weights with the f16 scale fields drawn as the configs draw them (finite f16 GEMM operands)
        iq2 = lambda n: synth.random_blocks(wr, T.IQ2_XXS, n, 0.02, [0])
        q4k = lambda n: synth.random_blocks(wr, T.Q4_K, n, 0.01, [0, 2])
        q80 = lambda n: synth.random_blocks(wr, T.Q8_0, n, 1.0 / 127, [0])
        # gs_moe_ffn, config 2's shape
        self.n_embd, self.n_ff, self.n = 4096, 1536, 8
        ne, nf, n = self.n_embd, self.n_ff, self.n
        w = [iq2(nf * ne) for _ in range(3 * n)]
        self.ffn_w = [G.DeviceBuffer.from_array(a) for a in w]
        self.batch = G.MoeBatch()
        self.batch.n = n
        for e in range(n):
            self.batch.gate[e], self.batch.up[e], self.batch.down[e] = (
                self.ffn_w[e].p.value, self.ffn_w[n + e].p.value, self.ffn_w[2 * n + e].p.value)
            self.batch.w[0][e] = float(nr.random())
        self.rs_gu, self.rs_dn = G.row_bytes(T.IQ2_XXS, ne), G.row_bytes(T.IQ2_XXS, nf)
        self.ffn_x = G.DeviceBuffer(ne * 4)
        self.ffn_h = G.DeviceBuffer(n * nf * 4)
        self.ffn_y = G.DeviceBuffer(ne * 4)
        # gs_gemv: Q4_K 2048 x 4096 one vector; Q8_0 1024 x 4096 four vectors
        self.q4 = G.DeviceBuffer.from_array(q4k(2048 * 4096))
        self.q8 = G.DeviceBuffer.from_array(q80(1024 * 4096))
        self.gv_x = G.DeviceBuffer(4 * 4096 * 4)
        self.gv_y4 = G.DeviceBuffer(2048 * 4)
        self.gv_y8 = G.DeviceBuffer(4 * 1024 * 4)
        # gs_moe_grouped_scatter: 20 tokens, top-4 of 8 IQ2_XXS experts, 1024/512
        self.g_tok, self.g_k, self.g_embd, self.g_ff = 20, 4, 1024, 512
        gate = [iq2(512 * 1024) for _ in range(8)]
        up = [iq2(512 * 1024) for _ in range(8)]
        down = [iq2(1024 * 512) for _ in range(8)]
        self.layer = M.ResidentMoeLayer(gate, up, down, 1024, 512, T.IQ2_XXS, T.IQ2_XXS)
        routes = [list(zip(e, wt)) for e, wt in synth.zipf_topk(np.random.default_rng(7), 20, 8, 4)]
        self.layer.upload_routes(routes, s, slots=True)
        self.layer._work(20)
        self.g_x = G.DeviceBuffer(20 * 1024 * 4)
        self.g_slots = G.DeviceBuffer(4 * 20 * 1024 * 4)
        # gs_gemm tiles (Q4_K 512 x 2048, 37 tokens) and gs_gemm_ex library path (Q8_0 1024 x 1024,
        # 256 tokens)
        self.m4 = G.DeviceBuffer.from_array(q4k(512 * 2048))
        self.mm_x = G.DeviceBuffer(37 * 2048 * 4)
        self.mm_y = G.DeviceBuffer(37 * 512 * 4)
        self.m8 = G.DeviceBuffer.from_array(q80(1024 * 1024))
        self.lx = G.DeviceBuffer(256 * 1024 * 4)
        self.ly = G.DeviceBuffer(256 * 1024 * 4)
        wb = G.ops.gemm_workspace(1024, 1024, 256)
        assert G.ops.gemm_path(T.Q8_0, 1024, 1024, 256, G.row_bytes(T.Q8_0, 1024), 1024, wb) == 2
        self.work = G.DeviceBuffer(wb)

    def inputs(self, s):
        """Fresh inputs into the (captured) input buffers; accumulated outputs reset."""
        nr = self.nrng
        f = lambda *shape: nr.standard_normal(shape).astype(np.float32)
        self.ffn_x.upload(f(self.n_embd), s)
        self.ffn_y.upload(f(self.n_embd), s)          # gs_moe_ffn adds into y
        self.gv_x.upload(f(4, 4096), s)
        self.g_x.upload(f(20, 1024), s)
        self.g_slots.upload(np.zeros(4 * 20 * 1024, np.float32), s)
        self.mm_x.upload(f(37, 2048) * 0.1, s)
        self.lx.upload(f(256, 1024) * 0.1, s)

    def run(self, s):
        o = G.ops
        o.moe_ffn(T.IQ2_XXS, T.IQ2_XXS, self.batch, 1, self.rs_gu, self.n_embd, self.n_ff, self.rs_dn, self.ffn_x,
                  self.ffn_h, self.ffn_y, 0.0, s)
        o.gemv(T.Q4_K, self.q4, G.row_bytes(T.Q4_K, 4096), 4096, 2048, self.gv_x, 4096, self.gv_y4, 2048, 1, s=s)
        o.gemv(T.Q8_0, self.q8, G.row_bytes(T.Q8_0, 4096), 4096, 1024, self.gv_x, 4096, self.gv_y8, 1024, 4, s=s)
        self.layer.forward_slots(self.g_x, self.g_slots, 20, 0.0, s)
        o.gemm(T.Q4_K, self.m4, G.row_bytes(T.Q4_K, 2048), 2048, 512, self.mm_x, 2048, self.mm_y, 512, 37, s=s)
        o.gemm_ex(T.Q8_0, self.m8, G.row_bytes(T.Q8_0, 1024), 1024, 1024, self.lx, 1024, self.ly, 1024, 256,
                  work=self.work, work_bytes=self.work.nbytes, s=s)

    def outputs(self, s):
        return {"ffn_y": self.ffn_y.download(np.float32, s=s), "ffn_h": self.ffn_h.download(np.float32, s=s),
                "gemv_q4_k": self.gv_y4.download(np.float32, s=s), "gemv_q8_0_x4": self.gv_y8.download(np.float32, s=s),
                "grouped_slots": self.g_slots.download(np.float32, s=s), "gemm": self.mm_y.download(np.float32, s=s),
                "gemm_ex_lib": self.ly.download(np.float32, s=s)}


def test_step_graph_replays_match_eager():
    hip = _hip()
    s = G.Stream()
    st = Step(s)
    state = np.random.default_rng(0).bit_generator.state
    # eager results for three input sets (the first eager pass also does every one-time set-up:
    # code objects, the library handle and its algorithm choice)
    st.nrng.bit_generator.state = state
    eager = []
    for i in range(3):
        st.inputs(s)
        st.run(s)
        s.sync()
        eager.append(st.outputs(s))
        say(f"eager set {i}: " + ", ".join(f"{k} {np.abs(v).max():.3g}" for k, v in eager[-1].items()))
        for k, v in eager[-1].items():
            assert np.all(np.isfinite(v)), k
    # capture
    graph, gexec = C.c_void_p(), C.c_void_p()
    _ok(hip.hipStreamBeginCapture(s.raw(), CAPTURE_GLOBAL), "hipStreamBeginCapture")
    try:
        st.run(s)
    finally:
        _ok(hip.hipStreamEndCapture(s.raw(), C.byref(graph)), "hipStreamEndCapture")
    n_nodes = C.c_size_t()
    _ok(hip.hipGraphGetNodes(graph, None, C.byref(n_nodes)), "hipGraphGetNodes")
    say(f"captured {n_nodes.value} nodes")
    _ok(hip.hipGraphInstantiate(C.byref(gexec), graph, None, None, C.c_size_t(0)), "hipGraphInstantiate")
    try:
        st.nrng.bit_generator.state = state
        scratch = G.DeviceBuffer(2048 * 4)
        for i in range(3):
            st.inputs(s)
            _ok(hip.hipGraphLaunch(gexec, s.raw()), "hipGraphLaunch")
            s.sync()
            got = st.outputs(s)
            # eager work between replays on the same stream
            G.ops.gemv(T.Q4_K, st.q4, G.row_bytes(T.Q4_K, 4096), 4096, 2048, st.gv_x, 4096, scratch, 2048, 1, s=s)
            s.sync()
            for k, v in got.items():
                same = np.array_equal(v.view(np.uint32), eager[i][k].view(np.uint32))
                if not same:
                    say(f"replay {i}: {k} differs, max |diff| {np.abs(v - eager[i][k]).max():.3g}")
                assert same, f"replay {i}: {k}"
            say(f"replay {i}: every output equals the eager call's")
    finally:
        hip.hipGraphExecDestroy(gexec)
        hip.hipGraphDestroy(graph)
