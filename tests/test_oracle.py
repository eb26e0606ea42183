"""Pins of the CPU oracle (oracle/oracle.c) that do not retype its formulas.

- f16<->f32: exhaustive round trip (the reference's own test, crates/quants/src/lib.rs:361-370)
  plus numpy's IEEE float16 casts.
- ggml tables: SHA-256 of the values in the reference's crates/quants/src/tables.rs, closed forms.
- dequantize: bit-exact against the independent per-element numpy decoders in npdecode.py, on the
  reference qtest generator's random blocks (qtest.rs:41-60) and on blocks sweeping every code.
- q8_1: invariants and a numpy re-derivation.
- GEMV / MoE FFN: brute-force f64 matmul of the oracle's own dequantized operands, linearity.
"""
import hashlib
import os
import re

import numpy as np
import pytest

import npdecode as npd
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# SHA-256 over the little-endian values of the ggml tables as the reference holds them
# (crates/quants/src/tables.rs:20, :87, :346, :381), computed once from that file.
TABLE_SHA = {
    "iq2xxs_grid": "05826b5d3e472a3a78f196be62ac78acf81df0f909626e12ab9fa2a5d490dd54",
    "iq2s_grid": "e1aa1473412b0552c2174c30ef22ab4073f6a181b85a17056e8249bd2932fd88",
    "iq3xxs_grid": "46e35f5a997efdee6c99ce57854c8a0d4f0ff8ca57e5e8a60c0793ea580acf5d",
    "kvalues_iq4nl": "61aa47540aa024b5d6ddaa839b84ffe59f3d5a349af5c6c7ffcb5e0474b46163",
}
TABLE_DT = {"iq2xxs_grid": "<u8", "iq2s_grid": "<u8", "iq3xxs_grid": "<u4", "kvalues_iq4nl": "i1"}


def test_f16_roundtrip_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([O.f16_to_f32(int(v)) for v in h], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    back = np.array([O.f32_to_f16(float(v)) for v in got[~nan]], dtype=np.uint16)
    assert np.array_equal(back, h[~nan])


def test_f32_to_f16_rounding_matches_numpy():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=20000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    # ties / subnormal boundary cases
    extra = np.array([65504.0, 65520.0, 65519.99, 6.1035156e-05, 5.9604645e-08, 2.9802322e-08, 2.9802326e-08,
                      1.0 + 2**-11, 1.0 + 3 * 2**-11, -0.0], dtype=np.float32)
    x = np.concatenate([x, extra])
    got = np.array([O.f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    with np.errstate(over="ignore"):   # 65520 and above round to inf, as intended
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def _header_table(path, name, dt):
    text = open(path).read()
    m = re.search(r"%s\[(\d+)\] = \{(.*?)\};" % name, text, re.S)
    vals = [int(v.rstrip("ul"), 0) for v in re.findall(r"-?0x[0-9a-fA-F]+u?l*l*|-?\d+", m.group(2))]
    assert len(vals) == int(m.group(1))
    return np.array(vals, dtype=np.int64).astype(dt)


@pytest.mark.parametrize("name", list(TABLE_SHA))
def test_tables_match_reference_hash(name):
    n = {"iq2xxs_grid": 256, "iq2s_grid": 1024, "iq3xxs_grid": 256, "kvalues_iq4nl": 16}[name]
    short = {"iq2xxs_grid": "iq2xxs", "iq2s_grid": "iq2s", "iq3xxs_grid": "iq3xxs", "kvalues_iq4nl": "iq4nl"}[name]
    t = O.table(short, n).astype(TABLE_DT[name])
    assert hashlib.sha256(t.tobytes()).hexdigest() == TABLE_SHA[name]
    # the product library's own copy must carry the same values
    prod = _header_table(os.path.join(ROOT, "glm-ssd_amd", "csrc", "ggml_grids.h"), name, TABLE_DT[name])
    assert hashlib.sha256(prod.tobytes()).hexdigest() == TABLE_SHA[name]


def test_table_closed_forms():
    ks = O.table("ksigns", 128)
    assert np.array_equal(ks.astype(np.uint64), npd.ksigns_closed(np.arange(128)))
    g = O.table("iq2xxs", 256)
    b = g.view(np.uint8).reshape(256, 8)
    assert set(np.unique(b)) == {0x08, 0x19, 0x2B}
    assert len(np.unique(g)) == 256


HOT = [O.Q8_0, O.Q4_K, O.Q6_K, O.IQ2_XXS]
ALL = [O.Q8_0, O.Q2_K, O.Q3_K, O.Q4_K, O.Q5_K, O.Q6_K, O.IQ2_XXS, O.IQ2_S, O.IQ3_XXS, O.IQ4_XS]


def _np_decode(ty, raw):
    if ty == O.Q8_0: return npd.q8_0(raw)
    if ty == O.Q2_K: return npd.q2_k(raw)
    if ty == O.Q3_K: return npd.q3_k(raw)
    if ty == O.Q4_K: return npd.q4_k(raw)
    if ty == O.Q5_K: return npd.q5_k(raw)
    if ty == O.Q6_K: return npd.q6_k(raw)
    if ty == O.IQ2_XXS: return npd.iq2_xxs(raw, O.table("iq2xxs", 256))
    if ty == O.IQ2_S: return npd.iq2_s(raw, O.table("iq2s", 1024))
    if ty == O.IQ3_XXS: return npd.iq3_xxs(raw, O.table("iq3xxs", 256))
    if ty == O.IQ4_XS: return npd.iq4_xs(raw, O.table("iq4nl", 16))
    raise ValueError


@pytest.mark.parametrize("ty", ALL)
def test_dequant_matches_independent_decoder(ty):
    be, bb = O.block(ty)
    rng = O.Rng(0x9E3779B97F4A7C15)
    raw = rng.random_blocks(ty, 64 * 256)
    got = O.dequantize(ty, raw, 64 * 256)
    want = _np_decode(ty, raw)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.abs(got).max() > 0 and len(np.unique(got)) > 16


@pytest.mark.parametrize("ty", ALL)
def test_dequant_all_byte_values(ty):
    """Every byte value at every non-scale byte position, scales fixed to a few exact f16s."""
    be, bb = O.block(ty)
    nblk = 256
    raw = np.zeros((nblk, bb), dtype=np.uint8)
    for pos in range(bb):
        raw[:, pos] = (np.arange(nblk) * 37 + pos * 11) % 256   # every value once per position
    halves = {O.Q8_0: [0], O.Q2_K: [80, 82], O.Q3_K: [108], O.Q4_K: [0, 2], O.Q5_K: [0, 2], O.Q6_K: [208],
              O.IQ2_XXS: [0], O.IQ2_S: [0], O.IQ3_XXS: [0], O.IQ4_XS: [0]}[ty]
    for i, off in enumerate(halves):
        v = np.float16([0.5, -0.03125, 2.0, 1.5e-3][i % 4] * (1 + i))
        raw[:, off:off + 2] = np.frombuffer(v.tobytes(), dtype=np.uint8)
    raw = raw.reshape(-1)
    got = O.dequantize(ty, raw, nblk * be)
    want = _np_decode(ty, raw)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q8_0_closed_form_all_codes():
    # y = d * q for every int8 q, exactly (no rounding: d has 11 bits, q 8)
    d = np.float16(0.0173)
    blk = np.zeros((8, 34), dtype=np.uint8)
    blk[:, 0:2] = np.frombuffer(d.tobytes(), dtype=np.uint8)
    blk[:, 2:] = np.arange(256, dtype=np.uint8).reshape(8, 32)
    got = O.dequantize(O.Q8_0, blk.reshape(-1), 256)
    want = np.arange(256, dtype=np.uint8).view(np.int8).astype(np.float64) * float(d)
    assert np.array_equal(got.astype(np.float64), want)


def test_iq2_xxs_enumeration_exact():
    """All 256 grid indices x 128 sign indices x 16 scales: value == d*(2s+1)/8 * grid * sign exactly."""
    grid = O.table("iq2xxs", 256).view(np.uint8).reshape(256, 8)
    d = np.float16(0.0213)
    nblk = 256 * 16 // 8 * 8  # each block holds 8 groups x 4 (grid, sign) pairs
    pairs = [(g, s, sc) for sc in range(16) for g in range(256) for s in ((g * 5 + sc * 17) % 128,)]
    pairs += [(g % 256, s, s % 16) for s in range(128) for g in (s * 3, s * 7 + 1)]
    nb = (len(pairs) + 31) // 32
    raw = np.zeros((nb, 66), dtype=np.uint8)
    raw[:, 0:2] = np.frombuffer(d.tobytes(), dtype=np.uint8)
    want = np.zeros((nb, 256))
    for i, (g, s, sc) in enumerate(pairs):
        b, grp = divmod(i, 32)
        ib32, l = divmod(grp, 4)
        a0 = int.from_bytes(raw[b, 2 + 8 * ib32:6 + 8 * ib32].tobytes(), "little")
        a1 = int.from_bytes(raw[b, 6 + 8 * ib32:10 + 8 * ib32].tobytes(), "little")
        a0 |= g << (8 * l)
        a1 = (a1 & ~(0xF << 28)) | (sc << 28) | (s << (7 * l))
        raw[b, 2 + 8 * ib32:6 + 8 * ib32] = np.frombuffer(a0.to_bytes(4, "little"), dtype=np.uint8)
        raw[b, 6 + 8 * ib32:10 + 8 * ib32] = np.frombuffer(a1.to_bytes(4, "little"), dtype=np.uint8)
    # expected from the closed form after all words are final (the 4-bit scale is shared per group of 4)
    for b in range(nb):
        for ib32 in range(8):
            a0 = int.from_bytes(raw[b, 2 + 8 * ib32:6 + 8 * ib32].tobytes(), "little")
            a1 = int.from_bytes(raw[b, 6 + 8 * ib32:10 + 8 * ib32].tobytes(), "little")
            sc = a1 >> 28
            for l in range(4):
                g = (a0 >> (8 * l)) & 255
                s7 = (a1 >> (7 * l)) & 127
                s8 = s7 | ((bin(s7).count("1") & 1) << 7)
                for j in range(8):
                    sign = -1.0 if (s8 >> j) & 1 else 1.0
                    want[b, 32 * ib32 + 8 * l + j] = float(d) * (2 * sc + 1) / 8 * grid[g, j] * sign
    got = O.dequantize(O.IQ2_XXS, raw.reshape(-1), nb * 256)
    assert np.array_equal(got.astype(np.float64), want.reshape(-1))


def _q8_1_numpy(x):
    xb = x.reshape(-1, 32).astype(np.float32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(over="ignore"):
        idv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, np.float32(1)), np.float32(0)).astype(np.float32)
    idv = np.where(np.isfinite(idv), idv, np.float32(0)).astype(np.float32)   # d < 2^-128: q = 0
    v = (xb * idv[:, None]).astype(np.float32).astype(np.float64)
    q = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int64)
    s = (q.sum(axis=1).astype(np.float32) * d).astype(np.float32)
    return d.astype(np.float16), s.astype(np.float16), q


def test_q8_1_invariants_and_rederivation():
    rng = np.random.default_rng(11)
    x = rng.standard_normal(4096 * 8).astype(np.float32)
    x[:32] = 0.0                       # zero block
    x[32:64] = 0.5                     # constant block
    x[64:96] = np.linspace(-3, 3, 32)  # symmetric ramp (ties)
    x[96:128] = np.float32(1e-40) * (np.arange(32) - 16)   # subnormals: 1/d overflows, q = 0
    q8 = O.quantize_q8_1(x).reshape(-1, 36)
    d = q8[:, 0:2].copy().view(np.float16).reshape(-1)
    s = q8[:, 2:4].copy().view(np.float16).reshape(-1)
    q = q8[:, 4:].view(np.int8).astype(np.int64)
    assert np.abs(q).max() <= 127
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    tiny = (amax / np.float32(127)).astype(np.float32) < np.float32(2.0 ** -128)   # 1/d overflows
    nz = (amax > 0) & ~tiny
    assert np.all(np.abs(q[nz]).max(axis=1) == 127)
    assert tiny[3] and np.all(q[tiny] == 0) and np.all(d[tiny] == 0)
    assert np.all(q[0] == 0) and d[0] == 0 and s[0] == 0
    dw, sw, qw = _q8_1_numpy(x)
    assert np.array_equal(q, qw) and np.array_equal(d.view(np.uint16), dw.view(np.uint16))
    assert np.array_equal(s.view(np.uint16), sw.view(np.uint16))
    # reconstruction: |x - (amax/127) q| <= (amax/127)/2 (+ rounding slack)
    dd = np.abs(x.reshape(-1, 32)).max(axis=1) / 127.0
    err = np.abs(x.reshape(-1, 32) - dd[:, None] * q)
    assert np.all(err <= dd[:, None] * 0.5 * (1 + 1e-5) + 1e-12)
    xh = O.dequantize_q8_1(q8.reshape(-1), x.size)
    assert np.array_equal(xh, (d.astype(np.float32)[:, None] * q.astype(np.float32)).reshape(-1))


@pytest.mark.parametrize("ty", HOT)
def test_gemv_bruteforce(ty):
    K, rows, B = 512, 37, 3
    rng = O.Rng(1234 + ty)
    W = rng.random_blocks(ty, rows * K)
    x = np.random.default_rng(ty).standard_normal((B, K)).astype(np.float32)
    y = O.gemv(ty, W, O.row_bytes(ty, K), K, rows, x, B=B)
    Wd = O.dequantize(ty, W, rows * K).reshape(rows, K).astype(np.float64)
    xh = np.stack([O.dequantize_q8_1(O.quantize_q8_1(x[b]), K) for b in range(B)]).astype(np.float64)
    want = xh @ Wd.T
    assert np.allclose(y, want, rtol=1e-12, atol=1e-12)
    # threads split rows only
    y4 = O.gemv(ty, W, O.row_bytes(ty, K), K, rows, x, B=B, nthreads=4)
    assert np.array_equal(y, y4)
    # unquantized variant is linear in x
    y1 = O.gemv(ty, W, O.row_bytes(ty, K), K, rows, x, B=B, quant_x=False)
    y2 = O.gemv(ty, W, O.row_bytes(ty, K), K, rows, 2 * x, B=B, quant_x=False)
    assert np.allclose(y2, 2 * y1, rtol=1e-12, atol=1e-15)


def test_swiglu_special_cases():
    assert O.lib().or_swiglu(0.0, 5.0, 0.0) == 0.0
    assert abs(O.lib().or_swiglu(1.0, 1.0, 0.0) - 1 / (1 + np.exp(-1))) < 1e-15
    assert O.lib().or_swiglu(10.0, 10.0, 2.0) == pytest.approx(2 / (1 + np.exp(-2)) * 2)
    assert O.lib().or_swiglu(1.0, -10.0, 2.0) == pytest.approx(1 / (1 + np.exp(-1)) * -2)


def test_moe_ffn_bruteforce():
    n_embd, n_ff, n_exp, T = 256, 512, 4, 2
    rng = O.Rng(99)
    rb = O.row_bytes(O.IQ2_XXS, n_embd)
    rbd = O.row_bytes(O.IQ2_XXS, n_ff)
    gate = [rng.random_blocks(O.IQ2_XXS, n_ff * n_embd) for _ in range(n_exp)]
    up = [rng.random_blocks(O.IQ2_XXS, n_ff * n_embd) for _ in range(n_exp)]
    down = [rng.random_blocks(O.IQ2_XXS, n_embd * n_ff) for _ in range(n_exp)]
    x = np.random.default_rng(3).standard_normal((T, n_embd)).astype(np.float32)
    pt, pe, pw = [0, 0, 1, 1], [1, 3, 3, 0], [0.6, 0.4, 0.7, 0.0]
    y, h = O.moe_ffn(O.IQ2_XXS, O.IQ2_XXS, gate, up, down, rb, rbd, n_embd, n_ff, x, pt, pe, pw, lim=0.0,
                     want_h=True)
    want = np.zeros((T, n_embd))
    for p, (t, e, w) in enumerate(zip(pt, pe, pw)):
        xh = O.dequantize_q8_1(O.quantize_q8_1(x[t]), n_embd).astype(np.float64)
        G = O.dequantize(O.IQ2_XXS, gate[e], n_ff * n_embd).reshape(n_ff, n_embd) @ xh
        U = O.dequantize(O.IQ2_XXS, up[e], n_ff * n_embd).reshape(n_ff, n_embd) @ xh
        hh = (G / (1 + np.exp(-G)) * U).astype(np.float32)
        assert np.allclose(h[p], hh, rtol=1e-6, atol=1e-9)
        hq = O.dequantize_q8_1(O.quantize_q8_1(h[p]), n_ff).astype(np.float64)
        D = O.dequantize(O.IQ2_XXS, down[e], n_embd * n_ff).reshape(n_embd, n_ff) @ hq
        if w != 0:
            want[t] += np.float64(np.float32(w)) * D
    assert np.allclose(y, want, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("ty", [O.IQ2_XXS, O.Q4_K])
def test_gemv_f16_mode_matches_numpy_half_casts(ty):
    # OR_ACT_F16 = the reference's multi-token GEMM (gemm.cu:57-78): dequantized weights rounded to
    # half, activations converted to half, then an exact-ish dot. numpy's float16 cast is an
    # independent IEEE round-to-nearest-even implementation.
    K, rows, B = 512, 29, 3
    rng = O.Rng(777 + ty)
    W = rng.random_blocks(ty, rows * K)
    x = (np.random.default_rng(ty).standard_normal((B, K)) * 3).astype(np.float32)
    x[0, :8] = [65519.0, -65520.0, 6e-8, -3e-8, 1e-5, 2.0 ** -24, 0.0, -0.0]   # overflow / subnormal edges
    y = O.gemv(ty, W, O.row_bytes(ty, K), K, rows, x, B=B, act="f16")
    Wd = O.dequantize(ty, W, rows * K).reshape(rows, K).astype(np.float16).astype(np.float64)
    with np.errstate(over="ignore"):
        xh = x.astype(np.float16).astype(np.float64)
    want = xh @ Wd.T
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(y), fin)
    assert np.allclose(y[fin], want[fin], rtol=1e-12, atol=1e-9)
    # f16x: half activations, exact weights
    yx = O.gemv(ty, W, O.row_bytes(ty, K), K, rows, x, B=B, act="f16x")
    wantx = xh @ O.dequantize(ty, W, rows * K).reshape(rows, K).astype(np.float64).T
    assert np.allclose(yx[fin], wantx[fin], rtol=1e-12, atol=1e-9)


def test_moe_ffn_f16_mode_bruteforce():
    n_embd, n_ff, n_exp, T = 256, 512, 3, 2
    rng = O.Rng(4242)
    rb, rbd = O.row_bytes(O.IQ2_XXS, n_embd), O.row_bytes(O.IQ2_XXS, n_ff)
    gate = [rng.random_blocks(O.IQ2_XXS, n_ff * n_embd) for _ in range(n_exp)]
    up = [rng.random_blocks(O.IQ2_XXS, n_ff * n_embd) for _ in range(n_exp)]
    down = [rng.random_blocks(O.IQ2_XXS, n_embd * n_ff) for _ in range(n_exp)]
    x = np.random.default_rng(5).standard_normal((T, n_embd)).astype(np.float32)
    pt, pe, pw = [0, 1, 1], [2, 2, 0], [0.5, 0.25, 1.0]
    y, h = O.moe_ffn(O.IQ2_XXS, O.IQ2_XXS, gate, up, down, rb, rbd, n_embd, n_ff, x, pt, pe, pw, lim=3.0,
                     want_h=True, act="f16")
    half = lambda a: np.asarray(a).astype(np.float16).astype(np.float64)
    want = np.zeros((T, n_embd))
    for p, (t, e, w) in enumerate(zip(pt, pe, pw)):
        G = half(O.dequantize(O.IQ2_XXS, gate[e], n_ff * n_embd).reshape(n_ff, n_embd)) @ half(x[t])
        U = half(O.dequantize(O.IQ2_XXS, up[e], n_ff * n_embd).reshape(n_ff, n_embd)) @ half(x[t])
        Gc, Uc = np.minimum(G, 3.0), np.clip(U, -3.0, 3.0)
        hh = (Gc / (1 + np.exp(-Gc)) * Uc).astype(np.float32)
        assert np.allclose(h[p], hh, rtol=1e-6, atol=1e-9)
        D = half(O.dequantize(O.IQ2_XXS, down[e], n_embd * n_ff).reshape(n_embd, n_ff)) @ half(h[p])
        want[t] += np.float64(np.float32(w)) * D
    assert np.allclose(y, want, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("ty", [O.IQ2_XXS, O.Q8_0])
def test_gemv_f16s_modes_scaled_half(ty):
    # OR_ACT_F16S / F16SX: activation rows scaled by a power of two into [2^14, 2^15) before the half
    # rounding. Pinned by (1) equality with F16 / F16X where every activation is a normal half
    # (a power-of-two scale commutes with rounding there), (2) equivariance: scaling x by 2^k
    # scales y by exactly 2^k for any k, far past the half range, (3) a brute-force numpy
    # restatement for one row beyond the half range.
    K, rows = 256, 17
    rng = O.Rng(99 + ty)
    W = rng.random_blocks(ty, rows * K)
    rb = O.row_bytes(ty, K)
    x = (np.random.default_rng(ty).standard_normal((2, K)) * 50).astype(np.float32)
    for a, b in (("f16", "f16s"), ("f16x", "f16sx")):
        assert np.array_equal(O.gemv(ty, W, rb, K, rows, x, B=2, act=a), O.gemv(ty, W, rb, K, rows, x, B=2, act=b))
    for k in (-20, 7, 40, 100):
        xs = (x.astype(np.float64) * 2.0 ** k).astype(np.float32)
        for b in ("f16s", "f16sx"):
            assert np.array_equal(O.gemv(ty, W, rb, K, rows, xs, B=2, act=b),
                                  O.gemv(ty, W, rb, K, rows, x, B=2, act=b) * 2.0 ** k)
    big = x[:1] * np.float32(1e9)
    y = O.gemv(ty, W, rb, K, rows, big, act="f16sx")
    m, e = np.frexp(np.abs(big).max())
    sc = 2.0 ** (int(e) - 15)
    xh = (big / sc).astype(np.float16).astype(np.float64) * sc
    want = xh @ O.dequantize(ty, W, rows * K).reshape(rows, K).astype(np.float64).T
    assert np.all(np.isfinite(y)) and np.allclose(y, want, rtol=1e-12, atol=0)
