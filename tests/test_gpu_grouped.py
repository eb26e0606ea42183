"""GPU parity of the grouped routed-expert FFN (gs_moe_grouped, the MFMA path for prefill and
MTP verify) against the CPU oracle's per-pair FFN:
  * act="f16s"  -- the reference's multi-token GEMM semantics (half activations x and h,
    half-rounded dequantized weights, crates/cuda/kernels/gemm.cu:57-78 under
    forward.rs:1399-1413): rel-L2 <= 1e-3, the north-star bound for FFN outputs;
  * act="f16sx" -- half activations with exact weights, which is what the kernel computes (its
    weights are exact integers times the block scale): rel-L2 <= 1e-4, so the kernel's own error
    (f32 accumulation order) is checked well inside the reference bound.
Where the reference semantics' own weight rounding exceeds 1e-3 against exact weights (random
IQ3_XXS blocks), the first bound becomes that distance + 1e-4 (the triangle inequality with the
second bound)."""
import sys

import numpy as np
import pytest

import glmssd as G
from glmssd import GgmlType as T
from glmssd import moe as M
from glmssd import synth
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


def run_case(n_exp, n_tok, k, n_embd, n_ff, seed, lim=0.0, routes=None, zero_w=False, ty_gu=T.IQ2_XXS,
             ty_down=T.IQ2_XXS):
    say(f"grouped: {G.TYPE_NAMES[ty_gu]}/{G.TYPE_NAMES[ty_down]} n_exp={n_exp} n_tok={n_tok} top{k} K={n_embd} "
        f"n_ff={n_ff} lim={lim} seed={seed}")
    orng = O.Rng(1000 + seed)
    gate = [orng.random_blocks(ty_gu, n_ff * n_embd) for _ in range(n_exp)]
    up = [orng.random_blocks(ty_gu, n_ff * n_embd) for _ in range(n_exp)]
    down = [orng.random_blocks(ty_down, n_embd * n_ff) for _ in range(n_exp)]
    rng = np.random.default_rng(seed)
    if routes is None:
        routes = [list(zip(e, w)) for e, w in synth.zipf_topk(rng, n_tok, n_exp, k)]
    if zero_w:
        routes[0][0] = (routes[0][0][0], 0.0)
    x = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    layer = M.ResidentMoeLayer(gate, up, down, n_embd, n_ff, ty_gu, ty_down)
    offs, idx, w, pe = layer.upload_routes(routes)
    want = O.moe_ffn(ty_gu, ty_down, gate, up, down, layer.rs_gu, layer.rs_down, n_embd, n_ff, x, idx, pe, w, lim=lim,
                     nthreads=8, act="f16s")
    wantx = O.moe_ffn(ty_gu, ty_down, gate, up, down, layer.rs_gu, layer.rs_down, n_embd, n_ff, x, idx, pe, w, lim=lim,
                      nthreads=8, act="f16sx")
    y0 = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    s = G.Stream()
    dx, dy = G.DeviceBuffer.from_array(x), G.DeviceBuffer.from_array(y0)
    layer.forward(dx, dy, n_tok, lim, s)
    got = dy.download(np.float32, n_tok * n_embd, s).reshape(n_tok, n_embd).astype(np.float64) - y0
    err, errx = rel_l2(got, want), rel_l2(got, wantx)
    err_ref = rel_l2(want, wantx)   # the reference semantics' own half-rounding of the weights
    say(f"  pairs={idx.size} max group={np.diff(offs).max()} rel-L2 vs reference GEMM semantics {err:.2e}, "
        f"vs exact weights {errx:.2e} (reference semantics vs exact weights {err_ref:.2e})")
    # Within 1e-3 of the reference's result, unless the reference's own weight rounding already
    # moves it further than that from the exact-weight result (random IQ3_XXS blocks can): then
    # within that distance plus the kernel's own bound below.
    assert err <= max(REL_L2, err_ref + 1e-4)
    assert errx <= 1e-4
    return layer, got


def test_grouped_zipf_prefill_like():
    run_case(n_exp=24, n_tok=48, k=4, n_embd=1024, n_ff=512, seed=5)


def test_grouped_decode_like_mtp():
    run_case(n_exp=64, n_tok=4, k=8, n_embd=2048, n_ff=512, seed=4)


def test_grouped_hot_expert_chunks_and_clamp():
    # expert 3 takes every token (> one 64-token chunk), expert 1 and 5 none; one pair weight 0
    n_tok = 150
    rng = np.random.default_rng(9)
    routes = [[(3, 0.6), (int(rng.choice([0, 2, 4, 6, 7])), 0.4)] for _ in range(n_tok)]
    run_case(n_exp=8, n_tok=n_tok, k=2, n_embd=768, n_ff=512, seed=6, lim=7.0, routes=routes, zero_w=True)


def test_grouped_repeat_is_stable():
    # two calls into fresh outputs agree up to the order of the f32 atomic combine
    layer, a = run_case(n_exp=16, n_tok=20, k=4, n_embd=512, n_ff=768, seed=11)
    x = np.random.default_rng(11).standard_normal((20, 512)).astype(np.float32)
    s = G.Stream()
    dx = G.DeviceBuffer.from_array(x)
    outs = []
    for _ in range(2):
        dy = G.DeviceBuffer.from_array(np.zeros((20, 512), np.float32))
        layer.forward(dx, dy, 20, 0.0, s)
        outs.append(dy.download(np.float32, 20 * 512, s).astype(np.float64))
    d = rel_l2(outs[1], outs[0])
    say(f"  repeat: rel-L2 between two calls {d:.2e}")
    assert np.all(np.isfinite(outs[0]))
    assert d <= 1e-6


def test_grouped_iq3_xxs_down_target_types():
    # the target model's expert types: IQ2_XXS gate/up, IQ3_XXS down (n_ff 2048 shape family)
    run_case(n_exp=16, n_tok=40, k=4, n_embd=1024, n_ff=2048, seed=21, ty_down=T.IQ3_XXS)


def test_grouped_iq3_xxs_everywhere_decode_sized():
    # random IQ3_XXS gate/up blocks drive h past the f16 range of the reference semantics (inf in
    # the oracle); the SwiGLU clamp the model uses keeps it finite
    run_case(n_exp=32, n_tok=4, k=8, n_embd=768, n_ff=512, seed=22, lim=7.0, ty_gu=T.IQ3_XXS, ty_down=T.IQ3_XXS)


def run_layer_sampled(n_tok, seed, n_sample, n_exp=288, k=8, n_embd=4096, n_ff=1536, ty=T.IQ2_XXS):
    """A layer at a benchmark configuration's own shapes (288 resident IQ2_XXS experts, hidden
    4096, intermediate 1536, top-8 Zipf(1.1) routing). The whole batch runs on the GPU; the oracle
    recomputes the output rows of n_sample tokens (every pair of those tokens), always including
    tokens of the most loaded expert."""
    say(f"grouped (benchmark shapes): n_exp={n_exp} n_tok={n_tok} top{k} K={n_embd} n_ff={n_ff} seed={seed} "
        f"sampled tokens={n_sample}")
    # the configuration's own generator: random IQ2_XXS blocks with d ~ |N(0, 0.02)|
    rng = np.random.default_rng(seed)
    gate, up, down = map(list, zip(*[synth.iq2_xxs_expert(rng, n_embd, n_ff) for _ in range(n_exp)]))
    routes = [list(zip(e, w)) for e, w in synth.zipf_topk(rng, n_tok, n_exp, k)]
    x = rng.standard_normal((n_tok, n_embd)).astype(np.float32)
    layer = M.ResidentMoeLayer(gate, up, down, n_embd, n_ff, ty, ty)
    offs, idx, w, pe = layer.upload_routes(routes)
    counts = np.diff(offs)
    hot = int(np.argmax(counts))
    s = G.Stream()
    dx = G.DeviceBuffer.from_array(x)
    dy = G.DeviceBuffer.from_array(np.zeros((n_tok, n_embd), np.float32))
    layer.forward(dx, dy, n_tok, 0.0, s)
    got = dy.download(np.float32, n_tok * n_embd, s).reshape(n_tok, n_embd).astype(np.float64)
    # sampled tokens: half from the hottest expert's pairs, the rest uniformly
    hot_toks = idx[offs[hot]:offs[hot + 1]]
    pick = set(rng.choice(hot_toks, size=min(n_sample // 2, hot_toks.size), replace=False).tolist())
    rest = [t for t in rng.permutation(n_tok).tolist() if t not in pick]
    pick = sorted(pick | set(rest[:n_sample - len(pick)]))
    sel = np.isin(idx, pick)
    remap = {t: i for i, t in enumerate(pick)}
    ptok = np.array([remap[int(t)] for t in idx[sel]], dtype=np.int32)
    xs = x[pick]
    kw = dict(nthreads=16)
    want = O.moe_ffn(ty, ty, gate, up, down, layer.rs_gu, layer.rs_down, n_embd, n_ff, xs, ptok, pe[sel], w[sel],
                     act="f16s", **kw)
    wantx = O.moe_ffn(ty, ty, gate, up, down, layer.rs_gu, layer.rs_down, n_embd, n_ff, xs, ptok, pe[sel], w[sel],
                      act="f16sx", **kw)
    g = got[pick]
    err, errx, err_ref = rel_l2(g, want), rel_l2(g, wantx), rel_l2(want, wantx)
    say(f"  pairs={idx.size} unique experts={int(np.count_nonzero(counts))} max group={counts.max()} "
        f"(expert {hot}); checked {len(pick)} tokens / {int(sel.sum())} pairs: rel-L2 vs reference GEMM semantics "
        f"{err:.2e}, vs exact weights {errx:.2e} (reference semantics vs exact weights {err_ref:.2e})")
    assert np.all(np.isfinite(got))
    assert err <= max(REL_L2, err_ref + 1e-4)
    assert errx <= 1e-4
    # tokens without pairs get nothing; every routed token gets something
    assert np.count_nonzero(np.abs(got).sum(axis=1) == 0) == n_tok - np.unique(idx).size


def test_grouped_config4_mtp_verify_shapes():
    # 4 tokens through one layer of 288 IQ2_XXS experts (4096/1536), top-8 Zipf
    run_layer_sampled(n_tok=4, seed=4, n_sample=4)


def test_grouped_config5_prefill_shapes():
    # 512 tokens (4096 pairs, hot expert groups of hundreds of pairs)
    run_layer_sampled(n_tok=512, seed=5, n_sample=48)
