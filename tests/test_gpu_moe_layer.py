"""GPU parity of a whole MoE FFN layer (glmssd.moe.MoeLayer, the work of forward.rs:982-1136 with
every expert resident): router GEMV (F32, f32 activations), host routing, shared-expert SwiGLU
FFN (Q6_K), routed experts (the target model's IQ2_XXS gate/up + IQ3_XXS down) through the fused
FFN, one fused one-token FFN per token for up to 4 tokens, the grouped MFMA kernel for more. The oracle restates the same composition on the
CPU; the routes must agree exactly and the output within rel-L2 1e-3."""
import sys

import numpy as np
import pytest
from scipy.special import expit

import glmssd as G
from glmssd import GgmlType as T
from glmssd.moe import MoeLayer, route
from glmssd import synth
import oracle as O

pytestmark = pytest.mark.gpu
REL_L2 = 1e-3


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def _swiglu(g, u, lim):
    if lim > 0:
        g, u = np.minimum(g, lim), np.clip(u, -lim, lim)
    return g * expit(g) * u   # logistic without exp overflow for large negative g


# 1-16 tokens: one-token FFNs (gs_moe_ffn, gs_moe_ffn_tokens); 20: the grouped MFMA kernel
@pytest.mark.parametrize("t,ty_dn", [(1, T.IQ3_XXS), (2, T.IQ3_XXS), (4, T.IQ3_XXS), (5, T.IQ3_XXS), (5, T.IQ2_XXS),
                                     (16, T.IQ2_XXS), (20, T.IQ3_XXS), (20, T.IQ2_XXS)])
def test_moe_layer(t, ty_dn):
    n_embd, n_ff, n_sh, ne, k = 2048, 512, 1024, 32, 8
    lim_e, lim_s = 7.0, 0.0
    nrng = np.random.default_rng(t * 10 + ty_dn)
    # small weight scales (|N(0,1e-4)| Q6_K super-block d, |N(0,0.02)| IQ), so the unclamped shared
    # expert's activations stay within f16 range where its matmuls run as GEMMs (t > 8)
    router = (nrng.standard_normal((ne, n_embd)) * 0.05).astype(np.float32)
    bias = (nrng.standard_normal(ne) * 0.1).astype(np.float32)
    shared = [synth.random_blocks(nrng, T.Q6_K, n_sh * n_embd, 1e-4, [208]),
              synth.random_blocks(nrng, T.Q6_K, n_sh * n_embd, 1e-4, [208]),
              synth.random_blocks(nrng, T.Q6_K, n_embd * n_sh, 1e-4, [208])]
    experts = [(synth.random_blocks(nrng, T.IQ2_XXS, n_ff * n_embd, 0.02, [0]),
                synth.random_blocks(nrng, T.IQ2_XXS, n_ff * n_embd, 0.02, [0]),
                synth.random_blocks(nrng, ty_dn, n_embd * n_ff, 0.02, [0])) for _ in range(ne)]
    s = G.Stream()
    layer = MoeLayer(router.view(np.uint8).reshape(-1), bias, shared, experts, n_embd, n_ff, T.IQ2_XXS, ty_dn, k=k,
                     weights_norm=True, weights_scale=2.5, clamp_exp=lim_e, clamp_shexp=lim_s, n_ff_shexp=n_sh, s=s)
    x = nrng.standard_normal((t, n_embd)).astype(np.float32)
    dx, dout = G.DeviceBuffer.from_array(x, s), G.DeviceBuffer(t * n_embd * 4)
    routes = layer.forward(dx, dout, t, s)
    got = dout.download(np.float32, t * n_embd, s).reshape(t, n_embd)

    # oracle: the same composition on the CPU
    logits = O.gemv(T.F32, router.view(np.uint8).reshape(-1), n_embd * 4, n_embd, ne, x, B=t, act="f32")
    want_routes = route(logits.astype(np.float32), bias, k, True, 2.5)
    assert [[e for e, _ in r] for r in routes] == [[e for e, _ in r] for r in want_routes]
    rb_sh = G.row_bytes(T.Q6_K, n_embd)
    sact = "f16" if t > 8 else "q8_1"   # the shared expert's matmuls: GEMV up to 8 vectors, else GEMM
    g = O.gemv(T.Q6_K, shared[0], rb_sh, n_embd, n_sh, x, B=t, act=sact)
    u = O.gemv(T.Q6_K, shared[1], rb_sh, n_embd, n_sh, x, B=t, act=sact)
    h = _swiglu(g, u, lim_s).astype(np.float32)
    sh = O.gemv(T.Q6_K, shared[2], G.row_bytes(T.Q6_K, n_sh), n_sh, n_embd, h, B=t, act=sact)
    pt, pe, pw = [], [], []
    for ti, r in enumerate(want_routes):
        for e, w in r:
            pt.append(ti); pe.append(e); pw.append(w)
    act = "f16s" if t > MoeLayer.PER_TOKEN_MAX else "q8_1"   # grouped MFMA path: the GEMM semantics
    routed = O.moe_ffn(T.IQ2_XXS, ty_dn, [e[0] for e in experts], [e[1] for e in experts],
                       [e[2] for e in experts], G.row_bytes(T.IQ2_XXS, n_embd), G.row_bytes(ty_dn, n_ff), n_embd,
                       n_ff, x, pt, pe, pw, lim=lim_e, nthreads=8, act=act)
    want = sh + routed
    acc = layer._scratch["acc"].download(np.float32, t * n_embd, s).reshape(t, n_embd)   # routed part alone
    e, er, es = rel_l2(got, want), rel_l2(acc, routed), rel_l2(got - acc, sh)
    say(f"  MoE layer t={t} down={G.TYPE_NAMES[ty_dn]}: rel-L2 {e:.2e}; routed {er:.2e}; shared {es:.2e}")
    assert e <= REL_L2 and er <= REL_L2 and es <= REL_L2


def test_moe_layer_expert_rows_q4_k():
    """Non-IQ routed experts (Q4_K) at t = 20: the per-expert multi-token branch (run_expert_rows,
    forward.rs:1399-1413: gather, gate/up matmuls, SwiGLU, down, weighted scatter-add), where each
    matmul is mm_s (forward.rs:700-710): a q8_1 GEMV for an expert group of up to 8 pairs, the f16
    GEMM above. The oracle follows the same split per expert."""
    t, n_embd, n_ff, n_sh, ne, k = 20, 1024, 512, 512, 24, 8
    lim_e = 7.0
    rrng = np.random.default_rng(4242)
    router = (rrng.standard_normal((ne, n_embd)) * 0.05).astype(np.float32)
    bias = (rrng.standard_normal(ne) * 0.5).astype(np.float32)   # skewed popularity: groups of 1..20 pairs
    x = rrng.standard_normal((t, n_embd)).astype(np.float32)
    nrng = np.random.default_rng(4243)
    shared = [synth.random_blocks(nrng, T.Q6_K, n_sh * n_embd, 1e-4, [208]),
              synth.random_blocks(nrng, T.Q6_K, n_sh * n_embd, 1e-4, [208]),
              synth.random_blocks(nrng, T.Q6_K, n_embd * n_sh, 1e-4, [208])]
    # small Q4_K scales keep h inside the f16 range of the GEMM semantics
    experts = [tuple(synth.random_blocks(nrng, T.Q4_K, n_ff * n_embd, 2e-4, [0, 2]) for _ in range(3))
               for _ in range(ne)]
    s = G.Stream()
    layer = MoeLayer(router.view(np.uint8).reshape(-1), bias, shared, experts, n_embd, n_ff, T.Q4_K, T.Q4_K, k=k,
                     clamp_exp=lim_e, n_ff_shexp=n_sh, s=s)
    assert layer.grouped is None
    dx, dout = G.DeviceBuffer.from_array(x, s), G.DeviceBuffer(t * n_embd * 4)
    routes = layer.forward(dx, dout, t, s)
    acc = layer._scratch["acc"].download(np.float32, t * n_embd, s).reshape(t, n_embd)   # routed part
    groups = {}
    for ti, r in enumerate(routes):
        for e, w in r:
            groups.setdefault(e, []).append((ti, w))
    sizes = sorted(len(v) for v in groups.values())
    assert sizes[0] <= 8 < sizes[-1], sizes   # both matmul branches run
    rb = G.row_bytes(T.Q4_K, n_embd)
    rbd = G.row_bytes(T.Q4_K, n_ff)
    want = np.zeros((t, n_embd))
    for e, prs in groups.items():
        act = "q8_1" if len(prs) <= 8 else "f16"
        want += O.moe_ffn(T.Q4_K, T.Q4_K, [experts[e][0]], [experts[e][1]], [experts[e][2]], rb, rbd, n_embd, n_ff,
                          x, [p[0] for p in prs], [0] * len(prs), [p[1] for p in prs], lim=lim_e, nthreads=8, act=act)
    e = rel_l2(acc, want)
    say(f"  MoE layer t={t} Q4_K experts (group sizes {sizes[0]}..{sizes[-1]}): routed rel-L2 {e:.2e}")
    assert e <= REL_L2
