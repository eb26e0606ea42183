"""Real-tensor parity in the style of the reference's `qtest -m` (crates/engine/src/qtest.rs:
172-189): tensors are located through the native GGUF reader and run through the GPU kernels,
against the CPU oracle. No model file ships here, so the test writes a GGUF whose tensors hold
seeded random blocks of every supported type, plus 3-D expert tensors in the target model's
layout (IQ2_XXS ffn_{gate,up}_exps [K, n_ff, n_exp], IQ3_XXS ffn_down_exps [n_ff, K, n_exp]);
the expert FFN goes through gs_moe_ffn on the slices slice_range() gives."""
import sys

import numpy as np
import pytest

import glmssd as G
from glmssd import GgmlType as T
from glmssd.gguf import Gguf
import oracle as O
from gguf_writer import Writer

pytestmark = pytest.mark.gpu
REL_L2 = 1e-3
TYPES = [T.F32, T.F16, T.Q8_0, T.Q2_K, T.Q3_K, T.Q4_K, T.Q5_K, T.Q6_K, T.IQ2_XXS, T.IQ2_S, T.IQ3_XXS, T.IQ4_XS]


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    rng = O.Rng(2024)
    K, R = 2048, 96
    NE, NF = 4, 1024
    tensors = []
    for ty in TYPES:
        tensors.append((f"blk.0.{G.TYPE_NAMES[ty].lower()}.weight", [K, R], ty, rng.random_blocks(ty, K * R)))
    for name, ty, dims in [("blk.1.ffn_gate_exps.weight", T.IQ2_XXS, [K, NF, NE]),
                           ("blk.1.ffn_up_exps.weight", T.IQ2_XXS, [K, NF, NE]),
                           ("blk.1.ffn_down_exps.weight", T.IQ3_XXS, [NF, K, NE])]:
        tensors.append((name, dims, ty, rng.random_blocks(ty, dims[0] * dims[1] * dims[2])))
    w = Writer().kv_str("general.architecture", "glm4moe").kv_u32("general.alignment", 32)
    w.kv_u32("glm4moe.expert_count", NE)
    data, off = b"", 0
    for name, dims, ty, raw in tensors:
        w.tensor(name, dims, int(ty), off)
        b = raw.tobytes()
        b += b"\0" * ((-len(b)) % 32)
        data += b
        off += len(b)
    path = tmp_path_factory.mktemp("gguf") / "synthetic-model.gguf"
    path.write_bytes(w.build(data))
    return Gguf.open(path), {n: raw for n, _, _, raw in tensors}


@pytest.fixture(scope="module")
def stream():
    return G.Stream()


def test_reader_locates_the_written_tensors(model):
    g, raws = model
    assert g.arch() == "glm4moe" and g.u64("glm4moe.expert_count") == 4
    for t in g.tensors:
        assert bytes(g.read(t)) == raws[t.name].tobytes(), t.name


@pytest.mark.parametrize("ty", TYPES)
def test_gemv_on_file_tensor(model, ty, stream):
    g, _ = model
    t = g.tensor(f"blk.0.{G.TYPE_NAMES[ty].lower()}.weight")
    k, rows = t.dims[0], min(t.dims[1], 64)          # qtest.rs:182-185: up to 64 rows of the tensor
    raw = g.read(t, 0, rows * t.row_bytes)
    x = np.random.default_rng(ty).standard_normal(k).astype(np.float32)
    dw, dx, dy = G.DeviceBuffer.from_array(raw), G.DeviceBuffer.from_array(x), G.DeviceBuffer(rows * 4)
    G.ops.gemv(ty, dw, t.row_bytes, k, rows, dx, k, dy, rows, 1, s=stream)
    got = dy.download(np.float32, rows, stream)
    want = O.gemv(ty, raw, t.row_bytes, k, rows, x, act="f32" if ty in (T.F32, T.F16) else "q8_1")[0]
    e = rel_l2(got, want)
    say(f"  {t.name}: rel-L2 {e:.2e}")
    assert e <= REL_L2


def test_expert_ffn_on_file_slices(model, stream):
    g, _ = model
    tg, tu, td = (g.tensor(f"blk.1.ffn_{p}_exps.weight") for p in ("gate", "up", "down"))
    K, NF, NE = tg.dims
    whole = {t.name: G.DeviceBuffer.from_array(g.read(t)) for t in (tg, tu, td)}
    x = np.random.default_rng(5).standard_normal((1, K)).astype(np.float32)
    w = np.array([0.5, 0.25, 0.0, 0.25], np.float32)
    b = G.MoeBatch()
    b.n = NE
    gate, up, down = [], [], []
    for e in range(NE):
        for t, lst, field in ((tg, gate, b.gate), (tu, up, b.up), (td, down, b.down)):
            off, n = t.slice_range(e)
            field[e] = whole[t.name].p.value + (off - t.offset)
            lst.append(g.read(t, off - t.offset, n))
        b.w[0][e] = w[e]
    want = O.moe_ffn(T.IQ2_XXS, T.IQ3_XXS, gate, up, down, tg.row_bytes, td.row_bytes, K, NF, x,
                     [0] * NE, list(range(NE)), list(w), nthreads=8)
    dx, dh, dy = G.DeviceBuffer.from_array(x), G.DeviceBuffer(NE * NF * 4), G.DeviceBuffer(K * 4)
    dy.zero(stream)
    G.ops.moe_ffn(T.IQ2_XXS, T.IQ3_XXS, b, 1, tg.row_bytes, K, NF, td.row_bytes, dx, dh, dy, 0.0, stream)
    e = rel_l2(dy.download(np.float32, K, stream), want[0])
    say(f"  expert FFN from file slices: rel-L2 {e:.2e}")
    assert e <= REL_L2
