"""GPU parity of gs_moe_ffn (the whole routed-expert FFN in one call: gate/up + SwiGLU, then
down + weighted combine): against the CPU oracle (rel-L2 <= 1e-3, as every matmul path), and bit
for bit against gs_moe_gateup + gs_moe_down called separately."""
import sys

import numpy as np
import pytest

import glmssd as G
from glmssd import GgmlType as T
import oracle as O

pytestmark = pytest.mark.gpu
REL_L2 = 1e-3


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


# (gate/up type, down type, tokens, experts, n_embd, n_ff, clamp); nt = 2 takes the two-launch path
CASES = [(T.IQ2_XXS, T.IQ2_XXS, 1, 8, 4096, 1536, 0.0), (T.IQ2_XXS, T.IQ3_XXS, 1, 8, 2048, 1536, 0.0),
         (T.Q4_K, T.Q4_K, 1, 5, 2048, 1024, 7.0), (T.Q8_0, T.Q8_0, 1, 3, 1024, 1024, 0.0),
         (T.Q6_K, T.Q6_K, 1, 4, 2048, 512, 3.0), (T.IQ3_XXS, T.IQ3_XXS, 1, 1, 2048, 768, 0.0),
         (T.IQ2_XXS, T.IQ2_XXS, 2, 6, 2048, 1024, 0.0), (T.Q5_K, T.Q5_K, 1, 2, 1024, 512, 0.0),
         # the target model's routed experts: IQ2_XXS gate/up, IQ3_XXS down, n_ff_exp = 2048
         # (validate.rs:376-386), one decode token and a 2-token MTP step
         (T.IQ2_XXS, T.IQ3_XXS, 1, 8, 4096, 2048, 0.0), (T.IQ2_XXS, T.IQ3_XXS, 2, 8, 4096, 2048, 0.0),
         # down with more rows than one batch per wave (n_embd 8192: the down row ring)
         (T.IQ2_XXS, T.IQ2_XXS, 1, 4, 8192, 512, 0.0),
         # the other streaming formats through gate/up and down (paired units split between gate
         # and up; one and two tokens)
         (T.Q2_K, T.Q3_K, 1, 3, 1024, 512, 0.0), (T.Q3_K, T.Q2_K, 2, 2, 1024, 512, 5.0),
         (T.IQ4_XS, T.IQ2_S, 1, 3, 1024, 768, 0.0), (T.IQ2_S, T.IQ4_XS, 2, 2, 2048, 512, 0.0),
         (T.F16, T.BF16, 1, 2, 1024, 512, 0.0),
         # one token over 12 experts at n_ff 2048: the down pass as two launches (8 + 4 experts)
         (T.IQ2_XXS, T.IQ2_XXS, 1, 12, 2048, 2048, 0.0)]


def _weights(rng, nrng, ty, n_elems):
    """Random blocks of a quantized type; for the float types finite values (random 16-bit words
    hold NaN/Inf), scaled like a trained matrix's."""
    if ty == T.F16:
        return (0.05 * nrng.standard_normal(n_elems)).astype(np.float16).view(np.uint8)
    if ty == T.BF16:
        v = (0.05 * nrng.standard_normal(n_elems)).astype(np.float32).view(np.uint32)
        return (v >> 16).astype(np.uint16).view(np.uint8)
    return rng.random_blocks(ty, n_elems)


@pytest.mark.parametrize("ty_gu,ty_dn,nt,n,n_embd,n_ff,lim", CASES)
def test_moe_ffn(ty_gu, ty_dn, nt, n, n_embd, n_ff, lim, stream):
    say(f"moe_ffn {G.TYPE_NAMES[ty_gu]}/{G.TYPE_NAMES[ty_dn]} nt={nt} n={n} {n_embd}x{n_ff} lim={lim}")
    rng = O.Rng(777 + 31 * ty_gu + ty_dn + n)
    nrng = np.random.default_rng(n_embd + n)
    gate = [_weights(rng, nrng, ty_gu, n_ff * n_embd) for _ in range(n)]
    up = [_weights(rng, nrng, ty_gu, n_ff * n_embd) for _ in range(n)]
    down = [_weights(rng, nrng, ty_dn, n_embd * n_ff) for _ in range(n)]
    x = nrng.standard_normal((nt, n_embd)).astype(np.float32)
    w = nrng.random((nt, n)).astype(np.float32)
    if n > 1:
        w[0, 1] = 0.0                                   # token 0 not routed to expert 1
    pt, pe, pw = [], [], []
    for t in range(nt):
        for e in range(n):
            pt.append(t); pe.append(e); pw.append(w[t, e])
    rbg, rbd = G.row_bytes(ty_gu, n_embd), G.row_bytes(ty_dn, n_ff)
    # the float formats keep f32 activations; the quantized ones quantize them to q8_1
    flt = (T.F32, T.F16, T.BF16)
    assert (ty_gu in flt) == (ty_dn in flt)
    want = O.moe_ffn(ty_gu, ty_dn, gate, up, down, rbg, rbd, n_embd, n_ff, x, pt, pe, pw, lim=lim, nthreads=8,
                     act="f32" if ty_gu in flt else "q8_1")
    bufs = [G.DeviceBuffer.from_array(a) for a in gate + up + down]
    b = G.MoeBatch()
    b.n = n
    for e in range(n):
        b.gate[e], b.up[e], b.down[e] = bufs[e].p.value, bufs[n + e].p.value, bufs[2 * n + e].p.value
        for t in range(nt):
            b.w[t][e] = w[t, e]
    dx = G.DeviceBuffer.from_array(x)
    y0 = nrng.standard_normal((nt, n_embd)).astype(np.float32)
    # reference: the two launches
    dh2 = G.DeviceBuffer(n * nt * n_ff * 4)
    dy2 = G.DeviceBuffer.from_array(y0)
    G.ops.moe_gateup(ty_gu, b, nt, rbg, n_embd, n_ff, dx, dh2, lim, stream)
    G.ops.moe_down(ty_dn, b, nt, rbd, n_ff, n_embd, dh2, dy2, stream)
    y2 = dy2.download(np.float32, nt * n_embd, stream)
    h2 = dh2.download(np.float32, n * nt * n_ff, stream)
    for rep in range(3):
        dh = G.DeviceBuffer(n * nt * n_ff * 4)
        dy = G.DeviceBuffer.from_array(y0)
        G.ops.moe_ffn(ty_gu, ty_dn, b, nt, rbg, n_embd, n_ff, rbd, dx, dh, dy, lim, stream)
        y = dy.download(np.float32, nt * n_embd, stream)
        h = dh.download(np.float32, n * nt * n_ff, stream)
        got = y.reshape(nt, n_embd).astype(np.float64) - y0
        e = rel_l2(got, want)
        say(f"  call {rep}: y rel-L2 vs oracle {e:.2e}; identical to two launches: h {np.array_equal(h, h2)} "
            f"y {np.array_equal(y, y2)}")
        assert e <= REL_L2
        assert np.array_equal(h, h2) and np.array_equal(y, y2)


# (gate/up type, down type, tokens, experts per token, pool of experts, n_embd, n_ff, clamp): the
# tokens draw their experts from a shared pool, so they overlap as MTP verify tokens do
TOKEN_CASES = [(T.IQ2_XXS, T.IQ2_XXS, 4, 8, 12, 4096, 1536, 0.0), (T.IQ2_XXS, T.IQ3_XXS, 3, 8, 10, 4096, 2048, 0.0),
               (T.Q4_K, T.Q4_K, 2, 5, 6, 2048, 1024, 7.0), (T.Q6_K, T.Q6_K, 4, 4, 8, 2048, 512, 3.0),
               (T.IQ2_XXS, T.IQ2_XXS, 2, 16, 20, 8192, 512, 0.0), (T.IQ3_XXS, T.IQ3_XXS, 32, 1, 3, 1024, 512, 0.0)]


@pytest.mark.parametrize("ty_gu,ty_dn,n_tok,n,pool,n_embd,n_ff,lim", TOKEN_CASES)
def test_moe_ffn_tokens(ty_gu, ty_dn, n_tok, n, pool, n_embd, n_ff, lim, stream):
    """gs_moe_ffn_tokens is bit for bit gs_moe_ffn per token (h and y), and within the matmul
    tolerance of the oracle."""
    say(f"moe_ffn_tokens {G.TYPE_NAMES[ty_gu]}/{G.TYPE_NAMES[ty_dn]} n_tok={n_tok} n={n} pool={pool} "
        f"{n_embd}x{n_ff} lim={lim}")
    rng = O.Rng(991 + 17 * ty_gu + ty_dn + n_tok)
    gate = [rng.random_blocks(ty_gu, n_ff * n_embd) for _ in range(pool)]
    up = [rng.random_blocks(ty_gu, n_ff * n_embd) for _ in range(pool)]
    down = [rng.random_blocks(ty_dn, n_embd * n_ff) for _ in range(pool)]
    nrng = np.random.default_rng(n_embd + n_tok)
    x = nrng.standard_normal((n_tok, n_embd)).astype(np.float32)
    experts = [nrng.choice(pool, n, replace=False) for _ in range(n_tok)]
    w = nrng.random((n_tok, n)).astype(np.float32)
    rbg, rbd = G.row_bytes(ty_gu, n_embd), G.row_bytes(ty_dn, n_ff)
    bufs = [G.DeviceBuffer.from_array(a) for a in gate + up + down]
    batches = []
    for t in range(n_tok):
        b = G.MoeBatch()
        b.n = n
        for i, e in enumerate(experts[t]):
            b.gate[i], b.up[i], b.down[i] = bufs[e].p.value, bufs[pool + e].p.value, bufs[2 * pool + e].p.value
            b.w[0][i] = w[t, i]
        batches.append(b)
    dx = G.DeviceBuffer.from_array(x)
    y0 = nrng.standard_normal((n_tok, n_embd)).astype(np.float32)
    dh1 = G.DeviceBuffer(n_tok * n * n_ff * 4)
    dy1 = G.DeviceBuffer.from_array(y0)
    for t in range(n_tok):
        G.ops.moe_ffn(ty_gu, ty_dn, batches[t], 1, rbg, n_embd, n_ff, rbd, dx.p.value + t * n_embd * 4,
                      dh1.p.value + t * n * n_ff * 4, dy1.p.value + t * n_embd * 4, lim, stream)
    y1 = dy1.download(np.float32, n_tok * n_embd, stream)
    h1 = dh1.download(np.float32, n_tok * n * n_ff, stream)
    if n_tok * n <= 12:
        pt = [t for t in range(n_tok) for _ in range(n)]
        pe = [int(e) for t in range(n_tok) for e in experts[t]]
        pw = [float(w[t, i]) for t in range(n_tok) for i in range(n)]
        want = O.moe_ffn(ty_gu, ty_dn, gate, up, down, rbg, rbd, n_embd, n_ff, x, pt, pe, pw, lim=lim, nthreads=8)
        e = rel_l2(y1.reshape(n_tok, n_embd).astype(np.float64) - y0, want)
        say(f"  per-token calls: y rel-L2 vs oracle {e:.2e}")
        assert e <= REL_L2
    for rep in range(2):
        dh = G.DeviceBuffer(n_tok * n * n_ff * 4)
        dy = G.DeviceBuffer.from_array(y0)
        G.ops.moe_ffn_tokens(ty_gu, ty_dn, batches, rbg, n_embd, n_ff, rbd, dx, dh, dy, lim, stream)
        y = dy.download(np.float32, n_tok * n_embd, stream)
        h = dh.download(np.float32, n_tok * n * n_ff, stream)
        say(f"  call {rep}: identical to per-token calls: h {np.array_equal(h, h1)} y {np.array_equal(y, y1)}")
        assert np.array_equal(h, h1) and np.array_equal(y, y1)


def test_moe_ffn_tokens_config4(stream):
    """BASELINE config 4 through the MoE layer's path for up to 16 tokens: 4 tokens, each top-8
    Zipf(1.1) over 288 resident IQ2_XXS experts (4096 / 1536, d ~ |N(0, 0.02)|), as one
    gs_moe_ffn_tokens call; every token's output against the oracle's q8_1 FFN."""
    from glmssd import synth
    n_exp, n_tok, k, n_embd, n_ff = 288, 4, 8, 4096, 1536
    rng = np.random.default_rng(4)
    experts = [synth.iq2_xxs_expert(rng, n_embd, n_ff) for _ in range(n_exp)]
    routes = synth.zipf_topk(rng, n_tok, n_exp, k)
    x = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    bufs = [[G.DeviceBuffer.from_array(m) for m in ex] for ex in experts]
    batches = []
    for ex, wt in routes:
        b = G.MoeBatch()
        b.n = k
        for i, e in enumerate(ex):
            b.gate[i], b.up[i], b.down[i] = (bufs[e][0].p.value, bufs[e][1].p.value, bufs[e][2].p.value)
            b.w[0][i] = wt[i]
        batches.append(b)
    rbg, rbd = G.row_bytes(T.IQ2_XXS, n_embd), G.row_bytes(T.IQ2_XXS, n_ff)
    dx = G.DeviceBuffer.from_array(x)
    dh = G.DeviceBuffer(n_tok * k * n_ff * 4)
    dy = G.DeviceBuffer.from_array(np.zeros((n_tok, n_embd), np.float32))
    G.ops.moe_ffn_tokens(T.IQ2_XXS, T.IQ2_XXS, batches, rbg, n_embd, n_ff, rbd, dx, dh, dy, 0.0, stream)
    got = dy.download(np.float32, n_tok * n_embd, stream).reshape(n_tok, n_embd)
    used = sorted({int(e) for ex, _ in routes for e in ex})
    pos = {e: i for i, e in enumerate(used)}
    pt = [t for t in range(n_tok) for _ in range(k)]
    pe = [pos[int(e)] for ex, _ in routes for e in ex]
    pw = [float(v) for _, wt in routes for v in wt]
    want = O.moe_ffn(T.IQ2_XXS, T.IQ2_XXS, [experts[e][0] for e in used], [experts[e][1] for e in used],
                     [experts[e][2] for e in used], rbg, rbd, n_embd, n_ff, x, pt, pe, pw, nthreads=16, act="q8_1")
    errs = [rel_l2(got[t], want[t]) for t in range(n_tok)]
    say(f"  config 4 (288 experts, {len(used)} used, 4 tokens): per-token rel-L2 " + " ".join(f"{e:.2e}" for e in errs))
    assert max(errs) <= REL_L2


# shapes beyond the streaming kernels' register plan: the reference takes any K % QK == 0
# (quants.cu:378-392); (gate/up type, down type, tokens, experts, n_embd, n_ff)
LONG_K = [(T.IQ2_XXS, T.IQ2_XXS, 1, 3, 12288, 512), (T.Q4_K, T.Q4_K, 2, 2, 8192, 1024),
          (T.IQ2_XXS, T.IQ3_XXS, 1, 2, 1024, 20480), (T.F16, T.F16, 2, 2, 1000, 520)]


@pytest.mark.parametrize("ty_gu,ty_dn,nt,n,n_embd,n_ff", LONG_K)
def test_moe_ffn_any_k(ty_gu, ty_dn, nt, n, n_embd, n_ff, stream):
    """gs_moe_gateup / gs_moe_down at K = 12288 (one token), K = 8192 (two tokens), a down row of
    20480, and float rows of 8-element multiples (K % 32 != 0): within the matmul bound of the
    oracle; gs_moe_ffn_tokens over the same experts equals gs_moe_ffn per token bit for bit."""
    say(f"moe_ffn any K {G.TYPE_NAMES[ty_gu]}/{G.TYPE_NAMES[ty_dn]} nt={nt} n={n} {n_embd}x{n_ff}")
    rng = O.Rng(55 + n_embd + n_ff)
    nrng = np.random.default_rng(n_embd * 3 + n)
    gate = [_weights(rng, nrng, ty_gu, n_ff * n_embd) for _ in range(n)]
    up = [_weights(rng, nrng, ty_gu, n_ff * n_embd) for _ in range(n)]
    down = [_weights(rng, nrng, ty_dn, n_embd * n_ff) for _ in range(n)]
    x = nrng.standard_normal((nt, n_embd)).astype(np.float32)
    w = nrng.random((nt, n)).astype(np.float32)
    pt = [t for t in range(nt) for _ in range(n)]
    pe = [e for _ in range(nt) for e in range(n)]
    pw = [float(w[t, e]) for t in range(nt) for e in range(n)]
    rbg, rbd = G.row_bytes(ty_gu, n_embd), G.row_bytes(ty_dn, n_ff)
    flt = ty_gu in (T.F32, T.F16, T.BF16)
    want = O.moe_ffn(ty_gu, ty_dn, gate, up, down, rbg, rbd, n_embd, n_ff, x, pt, pe, pw, nthreads=16,
                     act="f32" if flt else "q8_1")
    bufs = [G.DeviceBuffer.from_array(a) for a in gate + up + down]
    b = G.MoeBatch()
    b.n = n
    for e in range(n):
        b.gate[e], b.up[e], b.down[e] = bufs[e].p.value, bufs[n + e].p.value, bufs[2 * n + e].p.value
        for t in range(nt):
            b.w[t][e] = w[t, e]
    dx = G.DeviceBuffer.from_array(x)
    dh = G.DeviceBuffer(n * nt * n_ff * 4)
    dy = G.DeviceBuffer.from_array(np.zeros((nt, n_embd), np.float32))
    G.ops.moe_gateup(ty_gu, b, nt, rbg, n_embd, n_ff, dx, dh, 0.0, stream)
    G.ops.moe_down(ty_dn, b, nt, rbd, n_ff, n_embd, dh, dy, stream)
    got = dy.download(np.float32, nt * n_embd, stream).reshape(nt, n_embd)
    e = rel_l2(got, want)
    say(f"  y rel-L2 vs oracle {e:.2e}")
    assert e <= REL_L2
    if nt == 1:
        return
    # the token loop: one-token batches of the same experts
    bs = []
    for t in range(nt):
        bt = G.MoeBatch()
        bt.n = n
        for i in range(n):
            bt.gate[i], bt.up[i], bt.down[i] = b.gate[i], b.up[i], b.down[i]
            bt.w[0][i] = w[t, i]
        bs.append(bt)
    dh1 = G.DeviceBuffer(nt * n * n_ff * 4)
    dy1 = G.DeviceBuffer.from_array(np.zeros((nt, n_embd), np.float32))
    for t in range(nt):
        G.ops.moe_ffn(ty_gu, ty_dn, bs[t], 1, rbg, n_embd, n_ff, rbd, dx.p.value + t * n_embd * 4,
                      dh1.p.value + t * n * n_ff * 4, dy1.p.value + t * n_embd * 4, 0.0, stream)
    dh2 = G.DeviceBuffer(nt * n * n_ff * 4)
    dy2 = G.DeviceBuffer.from_array(np.zeros((nt, n_embd), np.float32))
    G.ops.moe_ffn_tokens(ty_gu, ty_dn, bs, rbg, n_embd, n_ff, rbd, dx, dh2, dy2, 0.0, stream)
    y1 = dy1.download(np.float32, nt * n_embd, stream)
    y2 = dy2.download(np.float32, nt * n_embd, stream)
    assert rel_l2(y1.reshape(nt, n_embd), want) <= REL_L2
    assert np.array_equal(y1, y2)


def test_moe_ffn_tokens_rejects(stream):
    """Unequal expert counts, and more than 32 (token, expert) pairs, are rejected before any launch."""
    b1, b2 = G.MoeBatch(), G.MoeBatch()
    b1.n, b2.n = 4, 3
    with pytest.raises(RuntimeError):
        G.ops.moe_ffn_tokens(T.IQ2_XXS, T.IQ2_XXS, [b1, b2], 66, 256, 512, 66, 0, 0, 0, 0.0, stream)
    bs = [G.MoeBatch() for _ in range(5)]
    for b in bs:
        b.n = 8
    with pytest.raises(RuntimeError):
        G.ops.moe_ffn_tokens(T.IQ2_XXS, T.IQ2_XXS, bs, 66, 256, 512, 66, 0, 0, 0, 0.0, stream)
