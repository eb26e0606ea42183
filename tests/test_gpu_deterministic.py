"""The engine's deterministic combine (GLMSSD_DETERMINISTIC, forward.rs:276-278, :1039-1048,
:1119-1127) through MoeLayer(deterministic=True): two runs give bit-identical outputs, the
routed accumulator is exactly the rank-ordered f32 sum of the per-(rank, token) slots, and the
result agrees with the atomic-combine layer (same products, another summation order) and with
the oracle."""
import sys

import numpy as np
import pytest

import glmssd as G
from glmssd import GgmlType as T
from glmssd.moe import MoeLayer
from glmssd import synth
import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def _layer(nrng, ty_gu, ty_dn, n_embd, n_ff, ne, k, det, s):
    router = (nrng.standard_normal((ne, n_embd)) * 0.05).astype(np.float32)
    bias = (nrng.standard_normal(ne) * 0.1).astype(np.float32)
    n_sh = 512
    # shared expert small enough that its f16 GEMM activations (more than 8 tokens) stay finite
    q6 = lambda r, c: synth.random_blocks(nrng, T.Q6_K, r * c, 1e-4, [208])
    shared = [q6(n_sh, n_embd), q6(n_sh, n_embd), q6(n_embd, n_sh)]
    # f16 scale fields per type (sigma, byte offsets): every other byte random
    sc = {T.IQ2_XXS: (0.02, [0]), T.IQ3_XXS: (0.02, [0]), T.Q4_K: (1e-3, [0, 2]), T.Q6_K: (1e-4, [208])}
    blk = lambda ty, n: synth.random_blocks(nrng, ty, n, *sc[ty])
    experts = [(blk(ty_gu, n_ff * n_embd), blk(ty_gu, n_ff * n_embd), blk(ty_dn, n_embd * n_ff))
               for _ in range(ne)]
    mk = lambda d: MoeLayer(router.view(np.uint8).reshape(-1), bias, shared, experts, n_embd, n_ff, ty_gu, ty_dn,
                            k=k, weights_norm=True, weights_scale=2.5, clamp_exp=7.0, n_ff_shexp=n_sh, s=s,
                            deterministic=d)
    return mk(det), mk(not det), experts


@pytest.mark.parametrize("t,ty_gu,ty_dn", [(3, T.IQ2_XXS, T.IQ3_XXS), (9, T.IQ2_XXS, T.IQ3_XXS), (24, T.IQ2_XXS, T.IQ3_XXS),
                                           (24, T.Q4_K, T.Q6_K)])
def test_deterministic_layer(t, ty_gu, ty_dn):
    n_embd, n_ff, ne, k = 1024, 512, 16, 8
    nrng = np.random.default_rng(1000 + t + ty_gu)
    s = G.Stream()
    det, atom, experts = _layer(nrng, ty_gu, ty_dn, n_embd, n_ff, ne, k, True, s)
    x = nrng.standard_normal((t, n_embd)).astype(np.float32)
    dx = G.DeviceBuffer.from_array(x, s)
    outs, accs = [], []
    for _ in range(2):
        dout = G.DeviceBuffer(t * n_embd * 4)
        routes = det.forward(dx, dout, t, s)
        outs.append(dout.download(np.float32, t * n_embd, s))
        accs.append(det._scratch["acc"].download(np.float32, t * n_embd, s))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), "deterministic mode not reproducible"
    if t > MoeLayer.PER_TOKEN_MAX:
        # acc = 0 + slot[0] + slot[1] + ... in rank order, f32 at every step
        sl = det._scratch["slots"].download(np.float32, k * t * n_embd, s).reshape(k, t * n_embd)
        want = np.zeros(t * n_embd, np.float32)
        for r in range(k):
            want = want + sl[r]
        assert np.array_equal(accs[0].view(np.uint32), want.view(np.uint32))
        assert np.all(sl != 0.0, axis=1).mean() > 0.99   # every (rank, token) slot written
    dout = G.DeviceBuffer(t * n_embd * 4)
    routes2 = atom.forward(dx, dout, t, s)
    assert routes == routes2
    other = dout.download(np.float32, t * n_embd, s)
    acc_a = atom._scratch["acc"].download(np.float32, t * n_embd, s)
    e_sum = rel_l2(accs[0], acc_a)
    # one-token FFNs: the same products summed in another expert order; grouped: atomics
    assert e_sum <= 1e-5, e_sum
    assert rel_l2(outs[0], other) <= 1e-5
    if ty_gu == T.IQ2_XXS and t > MoeLayer.PER_TOKEN_MAX:
        pt, pe, pw = [], [], []
        for ti, r in enumerate(routes):
            for e, w in r:
                pt.append(ti); pe.append(e); pw.append(w)
        routed = O.moe_ffn(ty_gu, ty_dn, [e[0] for e in experts], [e[1] for e in experts],
                           [e[2] for e in experts], G.row_bytes(ty_gu, n_embd), G.row_bytes(ty_dn, n_ff), n_embd,
                           n_ff, x, pt, pe, pw, lim=7.0, nthreads=8, act="f16s")
        e_or = rel_l2(accs[0].reshape(t, n_embd), routed)
        say(f"  deterministic t={t}: vs atomic {e_sum:.2e}, vs oracle {e_or:.2e}")
        assert e_or <= 1e-3
    else:
        say(f"  deterministic t={t} {G.TYPE_NAMES[ty_gu]}/{G.TYPE_NAMES[ty_dn]}: vs atomic {e_sum:.2e}")
