"""GPU parity: the HIP library (called through its C ABI) against the CPU oracle on identical
seeded inputs. Integer/byte work (dequantization, q8_1) must be bit-exact; matmul outputs must be
within rel-L2 <= 1e-3 of the oracle's f64 result (per type)."""
import sys

import numpy as np
import pytest

import glmssd as G
from glmssd import GgmlType as T
import oracle as O

pytestmark = pytest.mark.gpu
REL_L2 = 1e-3
ALL = [T.F32, T.F16, T.BF16, T.Q8_0, T.Q2_K, T.Q3_K, T.Q4_K, T.Q5_K, T.Q6_K, T.IQ2_XXS, T.IQ2_S, T.IQ3_XXS, T.IQ4_XS]
HOT = [T.Q8_0, T.Q4_K, T.Q6_K, T.IQ2_XXS]
FLOAT = (T.F32, T.F16, T.BF16)
REL_L2_F32 = 1e-5   # f32 activations on both sides: only the summation order differs


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel_l2(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


@pytest.fixture(scope="module")
def stream():
    return G.Stream()


@pytest.mark.parametrize("ty", ALL)
def test_dequant_bit_exact(ty, stream):
    say("dequant", G.TYPE_NAMES[ty])
    n = 256 * 257
    raw = O.Rng(0x9E3779B97F4A7C15 + ty).random_blocks(ty, n)
    want = O.dequantize(ty, raw, n)
    dw = G.DeviceBuffer.from_array(raw)
    dy = G.DeviceBuffer(n * 4)
    G.ops.dequant_f32(ty, dw, n, dy, stream)
    got = dy.download(np.float32, n, stream)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    dh = G.DeviceBuffer(n * 2)
    G.ops.dequant_f16(ty, dw, n, dh, stream)
    goth = dh.download(np.uint16, n, stream)
    with np.errstate(over="ignore"):
        wh = want.astype(np.float16)
    nan = np.isnan(wh)           # NaN payloads are not specified by the conversion
    assert np.array_equal(np.isnan(goth.view(np.float16)), nan)
    bad = np.nonzero(goth[~nan] != wh.view(np.uint16)[~nan])[0]
    if bad.size:
        i = bad[:5]
        say("  f16 mismatches", bad.size, want[~nan][i], goth[~nan][i], wh.view(np.uint16)[~nan][i])
    assert bad.size == 0


@pytest.mark.parametrize("ty", [T.Q8_0, T.Q4_K, T.Q6_K])
def test_dequant_blocks_ending_the_allocation(ty, stream):
    # the formats decoded with whole-dword reads: the last blocks of an allocation whose size is a
    # multiple of 2 MiB (no slack after it), so a read past the final block would leave the
    # allocation; the decoders read only the block's own bytes
    say("dequant at the allocation's end", G.TYPE_NAMES[ty])
    qk, bb = G.block(ty)
    total = int(np.lcm(bb, 2 << 20))
    nb = 96
    raw = O.Rng(0x5EED + ty).random_blocks(ty, nb * qk)
    buf = G.DeviceBuffer(total)
    buf.upload(raw, stream, total - raw.nbytes)
    n = nb * qk
    want = O.dequantize(ty, raw, n)
    dy, dh = G.DeviceBuffer(n * 4), G.DeviceBuffer(n * 2)
    G.ops.dequant_f32(ty, buf.ptr(total - raw.nbytes), n, dy, stream)
    G.ops.dequant_f16(ty, buf.ptr(total - raw.nbytes), n, dh, stream)
    assert np.array_equal(dy.download(np.float32, n, stream).view(np.uint32), want.view(np.uint32))
    with np.errstate(over="ignore"):
        wh = want.astype(np.float16).view(np.uint16)
    assert np.array_equal(dh.download(np.uint16, n, stream), wh)


def test_quant_q8_1_bit_exact(stream):
    say("quant_q8_1")
    rng = np.random.default_rng(5)
    x = rng.standard_normal(32 * 4099).astype(np.float32)
    x[:32] = 0
    x[32:64] = np.linspace(-3, 3, 32)
    x[64:96] = 1e-30
    x[96:128] = rng.standard_normal(32).astype(np.float32) * 1e4
    want = O.quantize_q8_1(x)
    dx = G.DeviceBuffer.from_array(x)
    dq = G.DeviceBuffer(want.nbytes)
    G.ops.quant_q8_1(dx, dq, x.size, stream)
    got = dq.download(np.uint8, want.size, stream)
    assert np.array_equal(got, want)


def _probe_x(K, seed):
    """activations covering the quantizer's edge cases, unit by unit (32 elements each)"""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(K).astype(np.float32)
    x[:32] = 0                                                        # zero unit: d = 0, id = 0
    x[32:64] = np.linspace(-3, 3, 32)
    x[64:96] = 1e-30                                                  # amax / 127 subnormal
    x[96:128] = rng.standard_normal(32).astype(np.float32) * 3e4      # large (f16 d stays finite)
    x[128:160] = np.arange(32, dtype=np.float32) - 15.5               # halves: ties away from zero
    x[160] = 127.0                                                    # d = 1 exactly ...
    x[161:192] = (np.arange(31, dtype=np.float32) - 15) + 0.5         # ... so every q is a tie
    x[192:224] = -x[160:192]
    x[224:256] = np.float32(2.0 ** -118) * (1 + np.arange(32, dtype=np.float32) / 32)   # fast-path edge
    return x


@pytest.mark.parametrize("B", [1, 3])
def test_staged_q8_1_bit_exact(B, stream):
    # One-hot Q8_0 rows (row r: weight 1 at column r, block scale 1.0) make the GEMV return the
    # kernel's own q8_1 activation f16(d) * q exactly, so the quantization each streaming kernel
    # stages in LDS is compared bit for bit with the oracle's q8_1.
    say("staged q8_1 B", B)
    K = 2048
    rb = G.row_bytes(T.Q8_0, K)
    w = np.zeros((K, K // 32, 34), dtype=np.uint8)
    r = np.arange(K)
    w[r, r // 32, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), dtype=np.uint8)
    w[r, r // 32, 2 + r % 32] = 1
    x = np.concatenate([_probe_x(K, 40 + b) for b in range(B)])
    want = np.concatenate([O.dequantize_q8_1(O.quantize_q8_1(x[b * K:(b + 1) * K]), K) for b in range(B)])
    dw = G.DeviceBuffer.from_array(w.reshape(-1))
    dx = G.DeviceBuffer.from_array(x)
    dy = G.DeviceBuffer(B * K * 4)
    G.ops.gemv(T.Q8_0, dw, rb, K, K, dx, K, dy, K, B, False, stream)
    got = dy.download(np.float32, B * K, stream)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    if bad.size:
        say("  mismatches", bad.size, bad[:5], got[bad[:5]], want[bad[:5]])
    assert bad.size == 0


def _gemv_case(ty, rows, K, B, stream, seed, x_stride=None, accumulate=False, row_stride=None):
    rb = G.row_bytes(ty, K)
    rs = rb if row_stride is None else row_stride
    raw = O.Rng(seed).random_blocks(ty, rows * K)
    if rs != rb:  # spread rows apart
        big = np.zeros(rows * rs, dtype=np.uint8)
        for r in range(rows):
            big[r * rs:r * rs + rb] = raw[r * rb:(r + 1) * rb]
        wbytes = big
    else:
        wbytes = raw
    xs = K if x_stride is None else x_stride
    rng = np.random.default_rng(seed)
    x = np.zeros(B * xs, dtype=np.float32)
    for b in range(B):
        x[b * xs:b * xs + K] = rng.standard_normal(K).astype(np.float32)
    # float matrices take f32 activations (quants.cu:81-96), the quantized formats q8_1 ones
    want = O.gemv(ty, wbytes, rs, K, rows, x, B=B, x_stride=xs, act="f32" if ty in FLOAT else "q8_1")
    # three sentinel vectors after the B outputs: no launch (or vector group) writes past B
    y0 = rng.standard_normal((B + 3) * rows).astype(np.float32)
    dw = G.DeviceBuffer.from_array(wbytes)
    dx = G.DeviceBuffer.from_array(x)
    dy = G.DeviceBuffer.from_array(y0)
    G.ops.gemv(ty, dw, rs, K, rows, dx, xs, dy, rows, B, accumulate, stream)
    full = dy.download(np.float32, (B + 3) * rows, stream)
    assert np.array_equal(full[B * rows:], y0[B * rows:]), "output written past vector B"
    got = full[:B * rows].reshape(B, rows)
    y0 = y0[:B * rows]
    if accumulate:
        got = got.astype(np.float64) - y0.reshape(B, rows)
    e = rel_l2(got, want)
    say(f"  gemv {G.TYPE_NAMES[ty]} rows={rows} K={K} B={B} rs={rs} acc={accumulate}: rel-L2 {e:.2e}")
    return e


# BF16 is left out like in the reference harness (qtest.rs:12-25): its random blocks hold NaN/Inf
@pytest.mark.parametrize("ty", [t for t in ALL if t != T.BF16])
@pytest.mark.parametrize("rows,K", [(101, 4096), (3001, 2048), (257, 1536)])
def test_gemv_matches_oracle(ty, rows, K, stream):
    for B in (1, 3, 8):
        assert _gemv_case(ty, rows, K, B, stream, seed=1000 * ty + rows + B) <= (REL_L2_F32 if ty in FLOAT else REL_L2)


@pytest.mark.parametrize("ty,rows,K", [(T.Q8_0, 37, 256), (T.Q8_0, 200, 1024), (T.Q8_0, 1000, 4096), (T.Q8_0, 45, 96),
                                        (T.Q8_0, 64, 8192), (T.Q4_K, 37, 256), (T.Q4_K, 300, 4096), (T.Q4_K, 61, 12288),
                                        (T.Q6_K, 33, 2048), (T.Q6_K, 200, 4096), (T.Q6_K, 61, 12288), (T.Q6_K, 40, 256),
                                        (T.Q5_K, 77, 4096), (T.Q5_K, 30, 8192),
                                        (T.Q4_K, 4200, 4096), (T.Q6_K, 4111, 2048), (T.Q5_K, 4113, 1024),
                                        (T.Q4_K, 4200, 8192), (T.Q6_K, 4111, 12288),
                                        (T.Q8_0, 4200, 2048), (T.Q5_K, 4113, 2048)])
def test_gemv_vectors_on_mfma(ty, rows, K, stream):
    # Q8_0 (from 3 vectors) and Q4_K / Q5_K / Q6_K (from 5, from 3 with K > 4096) run as one
    # int8-MFMA pass, fewer vectors on the streaming kernels (both checked here; the ~4100-row shapes
    # have more 16-row tiles than CUs, so each workgroup walks several, with K > 4096 over every
    # chunk of the row): 16-row tiles (a
    # tail tile in each shape), the row in chunks of up to 4096 elements (K = 8192 and 12288: two
    # and three chunks; K = 256 gives each of the 8 waves at most one unit). Q8_0 with K = 96 and
    # Q6_K with K = 256 (rows not whole 16-byte pieces) take the streaming kernels, as do rows
    # padded by 2 bytes: every vector count, strided activations, rows padded by 16 bytes and
    # accumulate, against the oracle
    for B in range(2, 9):
        pad = 16 * (B % 2) if B % 4 else 2
        e = _gemv_case(ty, rows, K, B, stream, seed=7 * K + B + 100 * ty, x_stride=K + 4 * (B % 3),
                       accumulate=B % 2 == 1, row_stride=G.row_bytes(ty, K) + pad)
        assert e <= REL_L2


@pytest.mark.parametrize("rows,K,pad,acc", [(8200, 4096, 0, False), (8200, 4096, 2, True), (9000, 2048, 2, False),
                                          (8192, 8192, 2, False), (8192, 8192, 0, True), (600, 4096, 0, True),
                                          (8200, 1056, 0, False)])
def test_gemv_q8_0_aligned_pairs(rows, K, pad, acc, stream):
    # one Q8_0 vector: rows 4-byte aligned (pad 0) read each unit pair as 17 aligned dwords (_w4);
    # other rows (pad 2: rows start alternately at 0 and 2 mod 4), from 4 rows per wave, shift
    # each unit's quants out of an aligned window (_wa, both shifts); an odd number of blocks per
    # row (K = 1056) keeps the plain loads (a pair would cross the row end)
    e = _gemv_case(T.Q8_0, rows, K, 1, stream, seed=rows + K + pad, accumulate=acc,
                   row_stride=G.row_bytes(T.Q8_0, K) + pad)
    assert e <= REL_L2


@pytest.mark.parametrize("rows,K,pad,acc", [(8200, 4096, 0, False), (8200, 4096, 4, True), (8192, 8192, 0, False),
                                          (8300, 2048, 2, False)])
def test_gemv_q6_k_aligned_pairs(rows, K, pad, acc, stream):
    # one Q6_K vector over at least 4 rows per wave with 4-byte aligned rows takes the
    # aligned-pair kernel (_wa: odd super-blocks start 2 bytes past a multiple of 4, so both shifts
    # run); rows 2 bytes apart from a multiple of 4 (pad 2) keep the plain loads
    e = _gemv_case(T.Q6_K, rows, K, 1, stream, seed=rows + K + pad + 1, accumulate=acc,
                   row_stride=G.row_bytes(T.Q6_K, K) + pad)
    assert e <= REL_L2


@pytest.mark.parametrize("rows,K,acc", [(8200, 4096, False), (8192, 8192, True)])
def test_gemv_iq2_xxs_many_rows(rows, K, acc, stream):
    # one IQ2_XXS vector over several row batches per wave (the row ring's refills)
    e = _gemv_case(T.IQ2_XXS, rows, K, 1, stream, seed=rows + K + 7, accumulate=acc)
    assert e <= REL_L2


@pytest.mark.parametrize("pad", [0, 2])
def test_gemv_q8_0_aligned_pairs_ending_the_allocation(pad, stream):
    # the aligned-pair kernel on a matrix whose last row ends at the end of an allocation (a
    # multiple of 2 MiB, minus `pad`): no load reaches past the allocation
    rows, K = 8192, 4096
    rb = G.row_bytes(T.Q8_0, K)
    rs = rb + 2
    raw = O.Rng(5150 + pad).random_blocks(T.Q8_0, rows * K)
    nbytes = (rows - 1) * rs + rb
    big = np.zeros(nbytes, dtype=np.uint8)
    for r in range(rows):
        big[r * rs:r * rs + rb] = raw[r * rb:(r + 1) * rb]
    total = -(-(nbytes + pad) // (2 << 20)) * (2 << 20)
    buf = G.DeviceBuffer(total)
    off = total - pad - nbytes
    buf.upload(big, stream, off)
    x = np.random.default_rng(pad).standard_normal(K).astype(np.float32)
    want = O.gemv(T.Q8_0, big, rs, K, rows, x, B=1)
    dx, dy = G.DeviceBuffer.from_array(x), G.DeviceBuffer(rows * 4)
    G.ops.gemv(T.Q8_0, buf.ptr(off), rs, K, rows, dx, K, dy, rows, 1, False, stream)
    got = dy.download(np.float32, rows, stream)
    assert rel_l2(got[None], want[:1]) <= REL_L2


@pytest.mark.parametrize("ty", [t for t in ALL if t != T.BF16])
@pytest.mark.parametrize("K", [4096, 1536, 2816])
def test_gemv_matrix_ending_the_allocation(ty, K, stream):
    # the matrix's last byte is the last byte of an allocation whose size is a multiple of 2 MiB
    # (no slack after it): the streaming loads of the last row read only its blocks' bytes
    # (48 rows: every type's matrix is then a multiple of 16 bytes, so it starts 16-byte aligned)
    rows = 48
    rb = G.row_bytes(ty, K)
    raw = O.Rng(77 * ty + K).random_blocks(ty, rows * K)
    total = -(-raw.nbytes // (2 << 20)) * (2 << 20)
    buf = G.DeviceBuffer(total)
    off = total - raw.nbytes
    buf.upload(raw, stream, off)
    x = np.random.default_rng(K + ty).standard_normal((3, K)).astype(np.float32)
    want = O.gemv(ty, raw, rb, K, rows, x, B=3, act="f32" if ty in FLOAT else "q8_1")
    dx, dy = G.DeviceBuffer.from_array(x), G.DeviceBuffer(3 * rows * 4)
    for B in (1, 3):
        G.ops.gemv(ty, buf.ptr(off), rb, K, rows, dx, K, dy, rows, B, False, stream)
        got = dy.download(np.float32, B * rows, stream).reshape(B, rows)
        assert rel_l2(got, want[:B]) <= (REL_L2_F32 if ty in FLOAT else REL_L2)


# BF16 with finite blocks: bf16 bit patterns of N(0,1) values (the reference harness skips BF16
# because its random bytes hold NaN/Inf; a real BF16 matrix is finite)
@pytest.mark.parametrize("rows,K", [(101, 4096), (513, 1536)])
def test_gemv_bf16_finite(rows, K, stream):
    ty = T.BF16
    v = np.random.default_rng(rows + K).standard_normal(rows * K).astype(np.float32)
    raw = (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
    x = np.random.default_rng(5).standard_normal((3, K)).astype(np.float32)
    rb = G.row_bytes(ty, K)
    want = O.gemv(ty, raw, rb, K, rows, x, B=3, quant_x=False)
    dw, dx, dy = G.DeviceBuffer.from_array(raw), G.DeviceBuffer.from_array(x), G.DeviceBuffer(3 * rows * 4)
    G.ops.gemv(ty, dw, rb, K, rows, dx, K, dy, rows, 3, False, stream)
    got = dy.download(np.float32, 3 * rows, stream).reshape(3, rows)
    assert rel_l2(got, want) <= REL_L2_F32


# Rows beyond one batch per wave (more than 2 x 2048 rows for one vector): the one-token kernels
# refill their row slots as they go (the row ring), including the last batch's empty refills and
# rows that end inside a batch; config 3's Q4_K shape among them.
@pytest.mark.parametrize("ty,rows,K", [(T.Q4_K, 12288, 4096), (T.Q8_0, 8191, 4096), (T.IQ2_XXS, 10001, 4096),
                                       (T.IQ3_XXS, 9000, 2048), (T.Q6_K, 6000, 12288)])
def test_gemv_many_rows_ring(ty, rows, K, stream):
    assert _gemv_case(ty, rows, K, 1, stream, seed=31 * ty + rows) <= REL_L2
    assert _gemv_case(ty, rows, K, 1, stream, seed=37 * ty + rows, accumulate=True) <= REL_L2


@pytest.mark.parametrize("ty", HOT)
def test_gemv_accumulate_and_strides(ty, stream):
    K = 1024
    assert _gemv_case(ty, 77, K, 2, stream, 7, accumulate=True) <= REL_L2
    assert _gemv_case(ty, 77, K, 2, stream, 8, x_stride=K + 3) <= REL_L2       # unaligned x rows
    assert _gemv_case(ty, 33, K, 1, stream, 9, row_stride=G.row_bytes(ty, K) + 2) <= REL_L2  # sparse rows


@pytest.mark.parametrize("ty", [T.Q6_K, T.Q8_0])
def test_gemv_long_rows_split(ty, stream):
    # K beyond one launch's register-resident activation (K > 16384 at B=1) takes the K-split path;
    # 2..4 vectors whose rows exceed the multi-vector kernels' reach but fit one vector's run as
    # one single-vector slice per vector (strided, accumulating); past 16384 they split K too
    assert _gemv_case(ty, 64, 24576, 1, stream, 11) <= REL_L2
    assert _gemv_case(ty, 64, 12288, 4, stream, 12) <= REL_L2
    assert _gemv_case(ty, 96, 8192, 3, stream, 13, accumulate=True, x_stride=8192 + 4) <= REL_L2
    assert _gemv_case(ty, 64, 24576, 2, stream, 14) <= REL_L2


@pytest.mark.parametrize("ty", [T.Q8_0, T.Q4_K, T.IQ2_XXS])
def test_gemv_5_to_8_vectors_token_groups(ty, stream):
    # more than 4 vectors with K > 2048 run as groups of 4 vectors over the whole K (B = 8: both
    # groups in one launch; B = 5..7: a group of 4 and one of B - 4), with strides and accumulate
    for B in (5, 7, 8):
        assert _gemv_case(ty, 130, 4096, B, stream, 50 + B) <= REL_L2
    assert _gemv_case(ty, 130, 4096, 8, stream, 61, accumulate=True, x_stride=4096 + 4) <= REL_L2
    assert _gemv_case(ty, 130, 4096, 6, stream, 62, accumulate=True) <= REL_L2


@pytest.mark.parametrize("ty", [T.F32, T.F16])
def test_gemv_float_rows_of_8(ty, stream):
    # plain rows whose length is a multiple of 8 but not of 32 (the reference's K % 8 rule,
    # quants.cu:225-229), with strides, accumulate and several vectors
    for B in (1, 3, 8):
        assert _gemv_case(ty, 77, 1000, B, stream, 70 + B) <= REL_L2_F32
    assert _gemv_case(ty, 45, 264, 2, stream, 80, accumulate=True, x_stride=268) <= REL_L2_F32


def test_gemv_batched(stream):
    ty, K, rows, nb = T.Q4_K, 512, 96, 5
    rb = G.row_bytes(ty, K)
    raw = O.Rng(77).random_blocks(ty, nb * rows * K)
    x = np.random.default_rng(1).standard_normal(nb * K).astype(np.float32)
    dw, dx = G.DeviceBuffer.from_array(raw), G.DeviceBuffer.from_array(x)
    dy = G.DeviceBuffer(nb * rows * 4)
    G.ops.gemv_batched(ty, dw, rb, K, rows, dx, dy, nb, rows * rb, K, rows, stream)
    got = dy.download(np.float32, nb * rows, stream).reshape(nb, rows)
    for b in range(nb):
        want = O.gemv(ty, raw[b * rows * rb:(b + 1) * rows * rb], rb, K, rows, x[b * K:(b + 1) * K])
        assert rel_l2(got[b], want[0]) <= REL_L2


def _experts(ty_gu, ty_dn, n_exp, n_embd, n_ff, seed):
    rng = O.Rng(seed)
    gate = [rng.random_blocks(ty_gu, n_ff * n_embd) for _ in range(n_exp)]
    up = [rng.random_blocks(ty_gu, n_ff * n_embd) for _ in range(n_exp)]
    down = [rng.random_blocks(ty_dn, n_embd * n_ff) for _ in range(n_exp)]
    return gate, up, down


@pytest.mark.parametrize("ty,nt,n,lim", [(T.IQ2_XXS, 1, 8, 0.0), (T.IQ2_XXS, 2, 16, 0.0), (T.Q4_K, 2, 5, 7.0),
                                         (T.Q8_0, 1, 3, 0.0), (T.Q6_K, 2, 4, 3.0)])
def test_moe_fused_matches_oracle(ty, nt, n, lim, stream):
    say(f"moe {G.TYPE_NAMES[ty]} nt={nt} n={n} lim={lim}")
    n_embd, n_ff = 2048, 1536 if ty != T.Q8_0 else 1024
    gate, up, down = _experts(ty, ty, n, n_embd, n_ff, 4242 + ty)
    rng = np.random.default_rng(ty)
    x = rng.standard_normal((nt, n_embd)).astype(np.float32)
    w = rng.random((nt, n)).astype(np.float32)
    w[0, 1] = 0.0                                   # token 0 not routed to expert 1
    pt, pe, pw = [], [], []
    for t in range(nt):
        for e in range(n):
            pt.append(t); pe.append(e); pw.append(w[t, e])
    rbg, rbd = G.row_bytes(ty, n_embd), G.row_bytes(ty, n_ff)
    want, hwant = O.moe_ffn(ty, ty, gate, up, down, rbg, rbd, n_embd, n_ff, x, pt, pe, pw, lim=lim, want_h=True,
                            nthreads=8)
    bufs = [G.DeviceBuffer.from_array(a) for a in gate + up + down]
    b = G.MoeBatch()
    b.n = n
    for e in range(n):
        b.gate[e], b.up[e], b.down[e] = bufs[e].p.value, bufs[n + e].p.value, bufs[2 * n + e].p.value
        for t in range(nt):
            b.w[t][e] = w[t, e]
    dx = G.DeviceBuffer.from_array(x)
    dh = G.DeviceBuffer(n * nt * n_ff * 4)
    y0 = rng.standard_normal((nt, n_embd)).astype(np.float32)
    dy = G.DeviceBuffer.from_array(y0)
    G.ops.moe_gateup(ty, b, nt, rbg, n_embd, n_ff, dx, dh, lim, stream)
    G.ops.moe_down(ty, b, nt, rbd, n_ff, n_embd, dh, dy, stream)
    h = dh.download(np.float32, n * nt * n_ff, stream).reshape(n, nt, n_ff)
    hw = hwant.reshape(nt, n, n_ff).transpose(1, 0, 2)
    eh = rel_l2(h, hw)
    got = dy.download(np.float32, nt * n_embd, stream).reshape(nt, n_embd).astype(np.float64) - y0
    ey = rel_l2(got, want)
    say(f"  h rel-L2 {eh:.2e}  y rel-L2 {ey:.2e}")
    assert eh <= REL_L2 and ey <= REL_L2


def test_elementwise_and_rows(stream):
    rng = np.random.default_rng(3)
    n = 10007
    g, u = rng.standard_normal(n).astype(np.float32) * 4, rng.standard_normal(n).astype(np.float32) * 4
    dg, du, dy = G.DeviceBuffer.from_array(g), G.DeviceBuffer.from_array(u), G.DeviceBuffer(n * 4)
    for lim in (0.0, 2.5):
        G.ops.swiglu(dg, du, dy, n, lim, stream)
        want = np.array([O.lib().or_swiglu(float(a), float(b), lim) for a, b in zip(g, u)])
        assert np.allclose(dy.download(np.float32, n, stream), want, rtol=1e-5, atol=1e-6)
    y0 = rng.standard_normal(n).astype(np.float32)
    dy.upload(y0)
    G.ops.axpy(dy, dg, 0.5, n, stream)
    assert np.allclose(dy.download(np.float32, n, stream), y0 + np.float32(0.5) * g, rtol=1e-6, atol=1e-6)
    rows, width = 37, 4096
    x = rng.standard_normal((64, width)).astype(np.float32)
    idx = rng.permutation(64)[:rows].astype(np.int32)
    wv = rng.random(rows).astype(np.float32)
    dx, di, dwv = G.DeviceBuffer.from_array(x), G.DeviceBuffer.from_array(idx), G.DeviceBuffer.from_array(wv)
    dg2 = G.DeviceBuffer(rows * width * 4)
    G.ops.gather_rows(dx, di, dg2, rows, width, stream)
    gathered = dg2.download(np.float32, rows * width, stream).reshape(rows, width)
    assert np.array_equal(gathered, x[idx])
    acc = rng.standard_normal((64, width)).astype(np.float32)
    da = G.DeviceBuffer.from_array(acc)
    G.ops.scatter_add_rows(da, di, dwv, dg2, rows, width, stream)
    want = acc.copy()
    want[idx] += wv[:, None] * x[idx]
    assert np.allclose(da.download(np.float32, 64 * width, stream).reshape(64, width), want, rtol=1e-6, atol=1e-6)


# gs_gemm has the reference's multi-token GEMM semantics (gemm.cu:57-78): weights dequantized and
# rounded to f16, activations rounded to f16, f32 accumulation -- the oracle's act="f16" computes
# the same products exactly, in f64, so only the summation order differs (tight bound below). The
# q8_1 GEMV of the same rows is within the north-star bound of it.
GEMM_REL = 1e-5


def _gemm_case(ty, K, rows, N, stream, seed, accumulate=False, x_stride=None, y_stride=None):
    rb = G.row_bytes(ty, K)
    if ty == T.BF16:
        v = np.random.default_rng(seed).standard_normal(rows * K).astype(np.float32)
        raw = (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)
    else:
        raw = O.Rng(seed).random_blocks(ty, rows * K)
        if ty in (T.F16, T.F32):   # finite values
            v = np.random.default_rng(seed).standard_normal(rows * K)
            raw = v.astype(np.float16 if ty == T.F16 else np.float32).view(np.uint8)
    xs = K if x_stride is None else x_stride
    ys = rows if y_stride is None else y_stride
    X = np.random.default_rng(seed + 1).standard_normal((N, xs)).astype(np.float32)
    want = O.gemv(ty, raw, rb, K, rows, X, B=N, x_stride=xs, act="f16", nthreads=8)
    # prior contents on the scale of the product (accumulate: the f32 sum then keeps its bits)
    y0 = (np.random.default_rng(seed + 2).standard_normal((N, ys)) * np.std(want)).astype(np.float32)
    dw, dx, dy = G.DeviceBuffer.from_array(raw), G.DeviceBuffer.from_array(X), G.DeviceBuffer.from_array(y0)
    G.ops.gemm(ty, dw, rb, K, rows, dx, xs, dy, ys, N, accumulate, 1, 0, 0, 0, stream)
    got = dy.download(np.float32, N * ys, stream).reshape(N, ys)
    assert np.array_equal(got[:, rows:], y0[:, rows:])   # padding columns untouched
    if accumulate:
        got = got.astype(np.float64) - y0
    return rel_l2(got[:, :rows], want)


@pytest.mark.parametrize("ty", [T.IQ2_XXS, T.IQ3_XXS, T.Q4_K, T.Q6_K, T.Q8_0])
@pytest.mark.parametrize("N", [9, 37, 512])
def test_gemm_hot_types(ty, N, stream):
    K, rows = (2048, 300) if N < 512 else (1024, 200)
    e = _gemm_case(ty, K, rows, N, stream, seed=100 * ty + N)
    say(f"gemm {G.TYPE_NAMES[ty]} N={N}: rel-L2 {e:.2e}")
    assert e <= GEMM_REL


@pytest.mark.parametrize("ty", ALL)
def test_gemm_weights_bit_exact(ty, stream):
    # X = the identity (token n one-hot at element n): Y[n][r] is then exactly the f16 rounding of
    # weight (r, n), so the tile decoders (byte-wise and dword-wise) are checked bit for bit
    # against the oracle's dequantization, for every element of two super-blocks of 70 rows
    K, rows = 512, 70
    rb = G.row_bytes(ty, K)
    if ty in FLOAT:
        v = np.random.default_rng(ty).standard_normal(rows * K).astype(np.float32)
        raw = {T.F32: v.view(np.uint8), T.F16: v.astype(np.float16).view(np.uint8),
               T.BF16: (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)}[ty]
    else:
        raw = O.Rng(3 * ty + 1).random_blocks(ty, rows * K)
    with np.errstate(over="ignore", invalid="ignore"):
        w16 = O.dequantize(ty, raw, rows * K).reshape(rows, K).astype(np.float16)
    ok = np.all(np.isfinite(w16), axis=1)   # a non-finite weight makes 0 x w non-finite in its row
    assert ok.mean() > 0.5
    X = np.eye(K, dtype=np.float32)
    dw, dx, dy = G.DeviceBuffer.from_array(raw), G.DeviceBuffer.from_array(X), G.DeviceBuffer(K * rows * 4)
    G.ops.gemm(ty, dw, rb, K, rows, dx, K, dy, rows, K, False, 1, 0, 0, 0, stream)
    got = dy.download(np.float32, K * rows, stream).reshape(K, rows).T
    want = w16.astype(np.float32) + np.float32(0)   # -0 -> +0: a sum of products that starts at +0
    bad = np.count_nonzero(got[ok].view(np.uint32) != want[ok].view(np.uint32))
    say(f"gemm weights {G.TYPE_NAMES[ty]}: {ok.sum()} finite rows, {bad} mismatching elements")
    assert bad == 0


@pytest.mark.parametrize("ty", [t for t in ALL])
def test_gemm_every_type(ty, stream):
    e = _gemm_case(ty, 512, 131, 70, stream, seed=7 * ty)
    say(f"gemm {G.TYPE_NAMES[ty]}: rel-L2 {e:.2e}")
    assert e <= GEMM_REL


def test_gemm_full_grid_and_k_split(stream):
    # 17 row blocks x 8 token blocks = 136 tiles: one launch over the whole K, no workspace needed.
    # Few tiles (12 row blocks, one token block): gs_gemm_ex splits K into 16 slices in the caller's
    # workspace, summed by the reduce pass, reproducible call to call; plain gs_gemm runs the same
    # problem unsplit (it allocates nothing) -- both within the f32 summation-order bound
    e = _gemm_case(T.Q8_0, 512, 2176, 512, stream, 21)
    say(f"gemm Q8_0 2176x512 N=512 (full grid): rel-L2 {e:.2e}")
    assert e <= GEMM_REL
    # a full grid below the library path's token count needs no workspace (204 tiles, 4.5 M
    # weights at 192 tokens); from 256 tokens, or above 128 for matrices of 2^25 weights and
    # more, the workspace holds the f16 operands of the library path
    assert G.ops.gemm_workspace(512, 8704, 192) == 0
    assert G.ops.gemm_workspace(512, 2176, 256) >= 2176 * 512 * 2 + 256 * 512 * 2
    assert G.ops.gemm_workspace(4096, 8192, 136) >= 8192 * 4096 * 2 + 136 * 4096 * 2
    assert G.ops.gemm_path(T.Q4_K, 4096, 8192, 128, G.row_bytes(T.Q4_K, 4096), 8192, 1 << 30) != 2
    ty, K, rows, N = T.IQ2_XXS, 4096, 1536, 64
    rb = G.row_bytes(ty, K)
    raw = O.Rng(22).random_blocks(ty, rows * K)
    X = np.random.default_rng(23).standard_normal((N, K)).astype(np.float32)
    want = O.gemv(ty, raw, rb, K, rows, X, B=N, act="f16", nthreads=8)
    dw, dx = G.DeviceBuffer.from_array(raw), G.DeviceBuffer.from_array(X)
    need = G.ops.gemm_workspace(K, rows, N)
    assert 0 < need <= 256 * 32768
    wk = G.DeviceBuffer(need)
    outs = []
    for _ in range(3):
        dy = G.DeviceBuffer(N * rows * 4)
        G.ops.gemm_ex(ty, dw, rb, K, rows, dx, K, dy, rows, N, False, 1, 0, 0, 0, wk, need, stream)
        outs.append(dy.download(np.float32, N * rows, stream))
    e = rel_l2(outs[0].reshape(N, rows), want)
    say(f"gemm_ex IQ2_XXS 1536x4096 N=64 (K split): rel-L2 {e:.2e}")
    assert e <= GEMM_REL
    assert all(np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)) for o in outs[1:])
    dy = G.DeviceBuffer(N * rows * 4)
    G.ops.gemm(ty, dw, rb, K, rows, dx, K, dy, rows, N, False, 1, 0, 0, 0, stream)
    e = rel_l2(dy.download(np.float32, N * rows, stream).reshape(N, rows), want)
    say(f"gemm IQ2_XXS 1536x4096 N=64 (unsplit): rel-L2 {e:.2e}")
    assert e <= GEMM_REL
    # a workspace smaller than the query's answer is refused before any launch
    with pytest.raises(G.GsError):
        G.ops.gemm_ex(ty, dw, rb, K, rows, dx, K, dy, rows, N, False, 1, 0, 0, 0, wk, need - 4, stream)


def test_gemm_ex_accumulate_and_batches(stream):
    # the K split with accumulate and n_batch = 2: slices summed in order, then added to Y
    ty, K, rows, N, nb = T.Q8_0, 2048, 256, 24, 2
    rb = G.row_bytes(ty, K)
    raw = O.Rng(31).random_blocks(ty, nb * rows * K)
    X = np.random.default_rng(32).standard_normal((nb, N, K)).astype(np.float32)
    wants = [O.gemv(ty, raw[z * rows * rb:(z + 1) * rows * rb], rb, K, rows, X[z], B=N, act="f16", nthreads=8)
             for z in range(nb)]
    # prior contents on the scale of the product, so the f32 sum keeps the product's bits
    y0 = (np.random.default_rng(33).standard_normal((nb, N, rows)) * np.std(wants[0])).astype(np.float32)
    dw, dx, dy = G.DeviceBuffer.from_array(raw), G.DeviceBuffer.from_array(X), G.DeviceBuffer.from_array(y0)
    need = G.ops.gemm_workspace(K, rows, N, nb)
    assert need > 0
    wk = G.DeviceBuffer(need)
    G.ops.gemm_ex(ty, dw, rb, K, rows, dx, K, dy, rows, N, True, nb, rows * rb, N * K, N * rows, wk, need, stream)
    got = dy.download(np.float32, nb * N * rows, stream).reshape(nb, N, rows).astype(np.float64) - y0
    for z in range(nb):
        assert rel_l2(got[z], wants[z]) <= GEMM_REL


@pytest.mark.parametrize("ty", [T.Q4_K, T.Q5_K, T.Q6_K, T.IQ2_XXS, T.F16, T.Q8_0])
def test_gemm_ex_library_path(ty, stream):
    # N = 400 tokens with the workspace gs_gemm_workspace asks for: the weights are dequantized
    # to f16 in the workspace, X converted to f16, and the contraction runs in the GEMM library.
    # Against the oracle's f16-operand product (f32 accumulation order differs) with accumulate,
    # two batches, a strided Y; and two calls give the same bits.
    K, rows, N, nb, ys = 512, 200, 400, 2, 203
    rb = G.row_bytes(ty, K)
    if ty == T.F16:
        raw = np.random.default_rng(ty).standard_normal(nb * rows * K).astype(np.float16).view(np.uint8)
    else:
        raw = O.Rng(7 * ty).random_blocks(ty, nb * rows * K)
    X = np.random.default_rng(ty + 1).standard_normal((nb, N, K)).astype(np.float32)
    wants = [O.gemv(ty, raw[z * rows * rb:(z + 1) * rows * rb], rb, K, rows, X[z], B=N, act="f16", nthreads=8)
             for z in range(nb)]
    y0 = (np.random.default_rng(ty + 2).standard_normal((nb, N, ys)) * np.std(wants[0])).astype(np.float32)
    need = G.ops.gemm_workspace(K, rows, N, nb)
    assert need >= rows * K * 2 + N * K * 2   # holds the f16 operands
    assert G.ops.gemm_path(ty, K, rows, N, rb, ys, need) == 2
    assert G.ops.gemm_path(ty, K, rows, N, rb + 2, ys, need) != 2   # padded rows: the tiles
    assert G.ops.gemm_path(ty, K, rows, N, rb, ys, 0) == 0   # no workspace: plain tiles
    dw, dx, wk = G.DeviceBuffer.from_array(raw), G.DeviceBuffer.from_array(X), G.DeviceBuffer(need)
    outs = []
    for rep in range(2):
        dy = G.DeviceBuffer.from_array(y0)
        G.ops.gemm_ex(ty, dw, rb, K, rows, dx, K, dy, ys, N, True, nb, rows * rb, N * K, N * ys, wk, need, stream)
        outs.append(dy.download(np.float32, nb * N * ys, stream).reshape(nb, N, ys))
    assert np.array_equal(outs[0], outs[1])
    got = outs[0]
    assert np.array_equal(got[:, :, rows:], y0[:, :, rows:])   # padding columns untouched
    for z in range(nb):
        e = rel_l2(got[z, :, :rows].astype(np.float64) - y0[z, :, :rows], wants[z])
        say(f"gemm_ex library path {G.TYPE_NAMES[ty]} batch {z}: rel-L2 {e:.2e}")
        assert e <= GEMM_REL


def test_gemm_ex_library_path_f16_unaligned(stream):
    # F16 weights 2 bytes past a 16-byte boundary: the library path copies them (the dequant
    # pass) instead of handing the library a misaligned operand; same product as aligned
    ty, K, rows, N = T.F16, 512, 96, 320
    rb = G.row_bytes(ty, K)
    raw = np.random.default_rng(41).standard_normal(rows * K).astype(np.float16).view(np.uint8)
    X = np.random.default_rng(42).standard_normal((N, K)).astype(np.float32)
    want = O.gemv(ty, raw, rb, K, rows, X, B=N, act="f16", nthreads=8)
    dw = G.DeviceBuffer(raw.nbytes + 16)
    dw.upload(raw, stream, 2)
    dx, dy = G.DeviceBuffer.from_array(X), G.DeviceBuffer(N * rows * 4)
    need = G.ops.gemm_workspace(K, rows, N, 1)
    assert G.ops.gemm_path(ty, K, rows, N, rb, rows, need) == 2
    wk = G.DeviceBuffer(need)
    G.ops.gemm_ex(ty, dw.ptr(2), rb, K, rows, dx, K, dy, rows, N, False, 1, 0, 0, 0, wk, need, stream)
    got = dy.download(np.float32, N * rows, stream).reshape(N, rows)
    assert rel_l2(got, want) <= GEMM_REL


@pytest.mark.parametrize("ty", [T.Q4_K, T.Q6_K, T.IQ2_XXS, T.Q5_K, T.Q2_K, T.Q3_K, T.IQ4_XS, T.IQ3_XXS, T.IQ2_S,
                                T.Q8_0])
def test_gemm_ex_library_weights_bit_exact(ty, stream):
    # the library path's weights: X = the identity (N = K = 512 tokens), so Y[n][r] is exactly
    # the f16 rounding of weight (r, n), bit for bit against the oracle's dequantization
    K, rows = 512, 70
    rb = G.row_bytes(ty, K)
    raw = O.Rng(3 * ty + 2).random_blocks(ty, rows * K)
    with np.errstate(over="ignore", invalid="ignore"):
        w16 = O.dequantize(ty, raw, rows * K).reshape(rows, K).astype(np.float16)
    ok = np.all(np.isfinite(w16), axis=1)
    assert ok.mean() > 0.5
    X = np.eye(K, dtype=np.float32)
    need = G.ops.gemm_workspace(K, rows, K, 1)
    assert G.ops.gemm_path(ty, K, rows, K, rb, rows, need) == 2
    dw, dx, dy, wk = G.DeviceBuffer.from_array(raw), G.DeviceBuffer.from_array(X), G.DeviceBuffer(K * rows * 4), G.DeviceBuffer(need)
    G.ops.gemm_ex(ty, dw, rb, K, rows, dx, K, dy, rows, K, False, 1, 0, 0, 0, wk, need, stream)
    got = dy.download(np.float32, K * rows, stream).reshape(K, rows).T
    want = w16.astype(np.float32) + np.float32(0)
    bad = np.count_nonzero(got[ok].view(np.uint32) != want[ok].view(np.uint32))
    say(f"gemm_ex library weights {G.TYPE_NAMES[ty]}: {ok.sum()} finite rows, {bad} mismatching elements")
    assert bad == 0


def test_gemm_accumulate_strides_and_partial_superblock(stream):
    # Q8_0 with K = 800 (the last 256-element step is partial), strided X / Y, accumulate
    assert _gemm_case(T.Q8_0, 800, 129, 65, stream, 11, accumulate=True, x_stride=804, y_stride=133) <= GEMM_REL
    assert _gemm_case(T.F32, 96, 40, 3, stream, 12, x_stride=100) <= GEMM_REL


def test_gemm_batched(stream):
    # n_batch = 3 independent problems (per-head matrices), non-zero batch strides
    ty, K, rows, N, nb = T.Q4_K, 512, 144, 20, 3
    rb = G.row_bytes(ty, K)
    raw = O.Rng(5).random_blocks(ty, nb * rows * K)
    X = np.random.default_rng(6).standard_normal((nb, N, K)).astype(np.float32)
    dw, dx, dy = G.DeviceBuffer.from_array(raw), G.DeviceBuffer.from_array(X), G.DeviceBuffer(nb * N * rows * 4)
    G.ops.gemm(ty, dw, rb, K, rows, dx, K, dy, rows, N, False, nb, rows * rb, N * K, N * rows, stream)
    got = dy.download(np.float32, nb * N * rows, stream).reshape(nb, N, rows)
    for z in range(nb):
        want = O.gemv(ty, raw[z * rows * rb:(z + 1) * rows * rb], rb, K, rows, X[z], B=N, act="f16")
        assert rel_l2(got[z], want) <= GEMM_REL


def test_gemm_vs_gemv_semantics(stream):
    # the f16 GEMM and the q8_1 GEMV of the same rows agree within the north-star bound
    ty, K, rows, N = T.IQ2_XXS, 2048, 256, 8
    rb = G.row_bytes(ty, K)
    raw = O.Rng(9).random_blocks(ty, rows * K)
    X = np.random.default_rng(10).standard_normal((N, K)).astype(np.float32)
    dw, dx, dy = G.DeviceBuffer.from_array(raw), G.DeviceBuffer.from_array(X), G.DeviceBuffer(N * rows * 4)
    G.ops.gemm(ty, dw, rb, K, rows, dx, K, dy, rows, N, False, 1, 0, 0, 0, stream)
    got = dy.download(np.float32, N * rows, stream).reshape(N, rows)
    want = O.gemv(ty, raw, rb, K, rows, X, B=N, act="f32")
    assert rel_l2(got, want) <= REL_L2
