"""Frozen fixtures (tests/golden/golden.npz, written by tests/golden/make_golden.py from the
oracle): the oracle must still reproduce them bit for bit (CPU), and the HIP library must match
them through the C ABI (GPU) -- dequantization and q8_1 bit-exact, GEMV / GEMM / expert FFN within
the same tolerances as the oracle parity tests."""
import os
import sys

import numpy as np
import pytest

import oracle as O

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_golden as MG  # noqa: E402

G_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(G_PATH, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


# ---- CPU: the oracle against its frozen results ------------------------------------------------
def test_oracle_dequant_frozen(gold):
    for ty in MG.TYPES:
        raw, want = gold[f"deq_raw_{ty}"], gold[f"deq_out_{ty}"]
        got = O.dequantize(ty, raw, want.size)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), ty


def test_oracle_q8_1_frozen(gold):
    q = O.quantize_q8_1(gold["q81_x"])
    assert np.array_equal(q, gold["q81_q"])
    # the convention the fixture records: block 1 holds the halves -15.5 .. 14.5 and 127, so d = 1
    # and q = round-half-away(x): ties away from zero (0.5 -> 1, -0.5 -> -1, 2.5 -> 3)
    blk = gold["q81_q"][36:72]
    assert blk[:2].view(np.float16)[0] == np.float16(1.0)
    qs = blk[4:].view(np.int8).astype(int)
    x = gold["q81_x"][32:64].astype(np.float64)
    assert np.array_equal(qs, np.sign(x) * np.floor(np.abs(x) + 0.5))
    assert qs[16] == 1 and qs[15] == -1 and qs[18] == 3


def test_oracle_matmuls_frozen(gold):
    K, rows, B = 512, 8, 3
    for ty in MG.HOT:
        y = O.gemv(ty, gold[f"gemv_w_{ty}"], O.row_bytes(ty, K), K, rows, gold["gemv_x"], B=B).astype(np.float32)
        assert np.array_equal(y, gold[f"gemv_y_{ty}"]), ty
    for ty in (8, 12, 16):
        y = O.gemv(ty, gold[f"gemm_w_{ty}"], O.row_bytes(ty, 512), 512, 16, gold["gemm_x"], B=9,
                   act="f16").astype(np.float32)
        assert np.array_equal(y, gold[f"gemm_y_{ty}"]), ty


def test_oracle_ffn_frozen(gold):
    for name, (seed, n_exp, K, n_ff, ty_gu, ty_dn, n_tok, act) in MG.FFN.items():
        gate, up, down = MG.ffn_case(seed, n_exp, K, n_ff, ty_gu, ty_dn)
        tok, exp = gold[f"{name}_pairs"]
        y = O.moe_ffn(ty_gu, ty_dn, gate, up, down, O.row_bytes(ty_gu, K), O.row_bytes(ty_dn, n_ff), K, n_ff,
                      gold[f"{name}_x"], tok, exp, gold[f"{name}_w"], act=act).astype(np.float32)
        assert np.array_equal(y, gold[f"{name}_y"]), name


# ---- GPU: the HIP library against the same fixtures --------------------------------------------
@pytest.mark.gpu
def test_gpu_golden_dequant_and_q8_1(gold):
    import glmssd as G
    s = G.Stream()
    for ty in MG.TYPES:
        raw, want = gold[f"deq_raw_{ty}"], gold[f"deq_out_{ty}"]
        src, dst = G.DeviceBuffer.from_array(raw), G.DeviceBuffer(want.size * 4)
        G.ops.dequant_f32(ty, src, want.size, dst, s)
        got = dst.download(np.float32, want.size, s)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), G.TYPE_NAMES[ty]
    x = gold["q81_x"]
    dx, dq = G.DeviceBuffer.from_array(x), G.DeviceBuffer(gold["q81_q"].size)
    G.ops.quant_q8_1(dx, dq, x.size, s)
    assert np.array_equal(dq.download(np.uint8, gold["q81_q"].size, s), gold["q81_q"])


@pytest.mark.gpu
def test_gpu_golden_gemv_gemm(gold):
    import glmssd as G
    s = G.Stream()
    K, rows, B = 512, 8, 3
    dx = G.DeviceBuffer.from_array(gold["gemv_x"])
    for ty in MG.HOT:
        dw, dy = G.DeviceBuffer.from_array(gold[f"gemv_w_{ty}"]), G.DeviceBuffer(B * rows * 4)
        G.ops.gemv(ty, dw, G.row_bytes(ty, K), K, rows, dx, K, dy, rows, B, False, s)
        e = rel_l2(dy.download(np.float32, B * rows, s), gold[f"gemv_y_{ty}"].reshape(-1))
        assert e <= 1e-5, (G.TYPE_NAMES[ty], e)
    dxm = G.DeviceBuffer.from_array(gold["gemm_x"])
    for ty in (8, 12, 16):
        dw, dy = G.DeviceBuffer.from_array(gold[f"gemm_w_{ty}"]), G.DeviceBuffer(9 * 16 * 4)
        G.ops.gemm(ty, dw, G.row_bytes(ty, 512), 512, 16, dxm, 512, dy, 16, 9, False, 1, 0, 0, 0, s)
        e = rel_l2(dy.download(np.float32, 9 * 16, s), gold[f"gemm_y_{ty}"].reshape(-1))
        assert e <= 1e-5, (G.TYPE_NAMES[ty], e)


@pytest.mark.gpu
def test_gpu_golden_expert_ffn(gold):
    import glmssd as G
    from glmssd.moe import ResidentMoeLayer
    s = G.Stream()
    # one-token decode FFN through gs_moe_ffn (q8_1 activations)
    seed, n_exp, K, n_ff, ty_gu, ty_dn, n_tok, act = MG.FFN["ffn_decode"]
    gate, up, down = MG.ffn_case(seed, n_exp, K, n_ff, ty_gu, ty_dn)
    tok, exp = gold["ffn_decode_pairs"]
    w = gold["ffn_decode_w"]
    bufs = [G.DeviceBuffer.from_array(a) for a in gate + up + down]
    b = G.MoeBatch()
    b.n = n_exp
    for e in range(n_exp):
        b.gate[e], b.up[e], b.down[e] = bufs[e].p.value, bufs[n_exp + e].p.value, bufs[2 * n_exp + e].p.value
        b.w[0][e] = 0.0
    for t, e, wt in zip(tok, exp, w):
        b.w[int(t)][int(e)] = float(wt)
    dx = G.DeviceBuffer.from_array(gold["ffn_decode_x"])
    dh, dy = G.DeviceBuffer(n_exp * n_ff * 4), G.DeviceBuffer.from_array(np.zeros(K, np.float32))
    G.ops.moe_ffn(ty_gu, ty_dn, b, 1, G.row_bytes(ty_gu, K), K, n_ff, G.row_bytes(ty_dn, n_ff), dx, dh, dy, 0.0, s)
    e = rel_l2(dy.download(np.float32, K, s), gold["ffn_decode_y"].reshape(-1))
    assert e <= 1e-5, e
    # multi-token grouped FFN (f16 activations with row scaling, exact weights)
    seed, n_exp, K, n_ff, ty_gu, ty_dn, n_tok, act = MG.FFN["ffn_grouped"]
    gate, up, down = MG.ffn_case(seed, n_exp, K, n_ff, ty_gu, ty_dn)
    tok, exp = gold["ffn_grouped_pairs"]
    w = gold["ffn_grouped_w"]
    routes = [[] for _ in range(n_tok)]
    for t, e, wt in zip(tok, exp, w):
        routes[int(t)].append((int(e), float(wt)))
    layer = ResidentMoeLayer(gate, up, down, K, n_ff, ty_gu, ty_dn)
    layer.upload_routes(routes, s)
    dx = G.DeviceBuffer.from_array(gold["ffn_grouped_x"])
    dy = G.DeviceBuffer.from_array(np.zeros((n_tok, K), np.float32))
    layer.forward(dx, dy, n_tok, 0.0, s)
    e = rel_l2(dy.download(np.float32, n_tok * K, s), gold["ffn_grouped_y"].reshape(-1))
    assert e <= 1e-4, e
