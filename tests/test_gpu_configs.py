"""BASELINE configs 1-3 at their own shapes and with their own input generators (glmssd.synth:
the generators bench.py measures), through the C ABI, against the CPU oracle (rel-L2 <= 1e-3, the
north-star bound; activations quantized to q8_1 on both sides).
  1: Q8_0 4096 x 4096 GEMV, q uniform in [-127, 127], d = |N(0,1)| / 127, x ~ N(0,1)
  2: the routed-expert FFN of one token over 8 of 288 IQ2_XXS experts (4096 / 1536), d ~ |N(0, 0.02)|,
     random index/sign/scale words, softmax weights over N(0,1) logits
  3: Q4_K rows 12288 x K 4096 and Q6_K rows 4096 x K 12288, d / dmin ~ |N(0, 0.01)|
(Configs 4 and 5 are in test_gpu_ffn.py and test_gpu_grouped.py.)"""
import sys

import numpy as np
import pytest

import glmssd as G
from glmssd import GgmlType as T
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


@pytest.mark.parametrize("cfg,ty,rows,K,make,seed", [
    (1, T.Q8_0, 4096, 4096, synth.q8_0_matrix, 1),
    (3, T.Q4_K, 12288, 4096, synth.q4_k_matrix, 3),
    (3, T.Q6_K, 4096, 12288, synth.q6_k_matrix, 3)])
def test_config_gemv(cfg, ty, rows, K, make, seed):
    rng = np.random.default_rng(seed)
    raw = make(rng, rows, K)
    x = rng.standard_normal(K).astype(np.float32)
    rb = G.row_bytes(ty, K)
    want = O.gemv(ty, raw, rb, K, rows, x, act="q8_1", nthreads=16)
    s = G.Stream()
    dw, dx, dy = G.DeviceBuffer.from_array(raw), G.DeviceBuffer.from_array(x), G.DeviceBuffer(rows * 4)
    G.ops.gemv(ty, dw, rb, K, rows, dx, K, dy, rows, 1, False, s)
    e = rel_l2(dy.download(np.float32, rows, s), want[0])
    say(f"config {cfg} {G.TYPE_NAMES[ty]} rows={rows} K={K}: rel-L2 {e:.2e}")
    assert e <= REL_L2


def test_config2_routed_ffn():
    n_expert, n_embd, n_ff = 288, 4096, 1536
    rng = np.random.default_rng(2)
    experts = [synth.iq2_xxs_expert(rng, n_embd, n_ff) for _ in range(n_expert)]
    chosen = rng.choice(n_expert, 8, replace=False)
    w = synth.softmax(rng.standard_normal(8))
    x = rng.standard_normal((1, n_embd)).astype(np.float32)
    rbg, rbd = G.row_bytes(T.IQ2_XXS, n_embd), G.row_bytes(T.IQ2_XXS, n_ff)
    want = O.moe_ffn(T.IQ2_XXS, T.IQ2_XXS, [experts[e][0] for e in chosen], [experts[e][1] for e in chosen],
                     [experts[e][2] for e in chosen], rbg, rbd, n_embd, n_ff, x, [0] * 8, list(range(8)), w,
                     nthreads=16, act="q8_1")
    s = G.Stream()
    bufs = {int(e): [G.DeviceBuffer.from_array(m) for m in experts[e]] for e in chosen}
    b = G.MoeBatch()
    b.n = 8
    for i, e in enumerate(chosen):
        g, u, d = bufs[int(e)]
        b.gate[i], b.up[i], b.down[i] = g.p.value, u.p.value, d.p.value
        b.w[0][i] = w[i]
    dx = G.DeviceBuffer.from_array(x)
    dh = G.DeviceBuffer(8 * n_ff * 4)
    dy = G.DeviceBuffer.from_array(np.zeros(n_embd, np.float32))
    G.ops.moe_gateup(T.IQ2_XXS, b, 1, rbg, n_embd, n_ff, dx, dh, 0.0, s)
    G.ops.moe_down(T.IQ2_XXS, b, 1, rbd, n_ff, n_embd, dh, dy, s)
    e = rel_l2(dy.download(np.float32, n_embd, s), want[0])
    say(f"config 2 (experts {sorted(int(c) for c in chosen)}): rel-L2 {e:.2e}")
    assert e <= REL_L2
