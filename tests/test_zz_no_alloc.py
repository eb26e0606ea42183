"""gs_moe_grouped_noalloc (the grouped routed-expert FFN with the library's own per-GPU workspace
array, for callers that cannot allocate) against gs_moe_grouped with a caller workspace, through
the C ABI: two calls in a row, the second smaller, each within the atomic-combine noise of the
workspace call (the two compute the same sums; only the f32 atomic order of the combine differs).
Also: a size beyond the array is rejected before any launch."""
import sys

import numpy as np
import pytest

import glmssd as G
from glmssd import GgmlType as T
from glmssd import moe as M
from glmssd import synth

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def _layer(n_exp, n_embd, n_ff, seed):
    rng = np.random.default_rng(seed)
    gate, up, down = map(list, zip(*[synth.iq2_xxs_expert(rng, n_embd, n_ff) for _ in range(n_exp)]))
    return M.ResidentMoeLayer(gate, up, down, n_embd, n_ff, T.IQ2_XXS, T.IQ2_XXS)


def _compare(layer, n_tok, seed, s):
    rng = np.random.default_rng(seed)
    routes = [list(zip(e, w)) for e, w in synth.zipf_topk(rng, n_tok, layer.n_exp, 8)]
    layer.upload_routes(routes, s)
    x = G.DeviceBuffer.from_array(rng.standard_normal((n_tok, layer.n_embd)).astype(np.float32), s)
    y_ws = G.DeviceBuffer.from_array(np.zeros((n_tok, layer.n_embd), np.float32), s)
    y_na = G.DeviceBuffer.from_array(np.zeros((n_tok, layer.n_embd), np.float32), s)
    layer.forward(x, y_ws, n_tok, 0.0, s)
    G.ops.moe_grouped_noalloc(layer.ty_gu, layer.ty_down, layer.table, layer.n_exp, layer.d_offs, layer.d_idx,
                              layer.d_w, layer.n_pairs, n_tok, layer.rs_gu, layer.n_embd, layer.n_ff, layer.rs_down,
                              x, y_na, 0.0, s)
    a = y_ws.download(np.float32, n_tok * layer.n_embd, s)
    b = y_na.download(np.float32, n_tok * layer.n_embd, s)
    e = rel_l2(b, a)
    say(f"noalloc n_tok={n_tok} pairs={layer.n_pairs}: rel-L2 vs workspace call {e:.2e}")
    assert np.all(np.isfinite(b)) and np.abs(b).max() > 0
    assert e <= 1e-6


def test_noalloc_matches_workspace_call():
    s = G.Stream()
    layer = _layer(64, 2048, 1024, 3)
    _compare(layer, 160, 31, s)   # first call on the device: the array is looked up
    _compare(layer, 20, 32, s)    # a second, smaller call reuses it


def test_noalloc_near_the_array_bound():
    # the sizing the header quotes: 512 tokens x top-8 at 4096 / 1536 (4096 pairs, about 42 MB of
    # the 48 MiB array), so the layout's last regions (h16 and its row scales) lie near its end
    s = G.Stream()
    layer = _layer(12, 4096, 1536, 5)
    need = G.ops.moe_grouped_workspace(512, 4096, 4096, 1536)
    assert 40 << 20 < need <= (48 << 20)
    _compare(layer, 512, 51, s)


def test_noalloc_rejects_beyond_scratch():
    s = G.Stream()
    layer = _layer(4, 2048, 1024, 4)
    x = G.DeviceBuffer(8 * 2048 * 4)
    y = G.DeviceBuffer(8 * 2048 * 4)
    # 8 tokens, but a pair count whose workspace exceeds the array: refused before any launch
    n_pairs = 20000
    assert G.ops.moe_grouped_workspace(8, n_pairs, 2048, 1024) > (48 << 20)
    with pytest.raises(G.GsError):
        G.ops.moe_grouped_noalloc(T.IQ2_XXS, T.IQ2_XXS, layer.table, layer.n_exp, x, x, x, n_pairs, 8, layer.rs_gu,
                                  2048, 1024, layer.rs_down, x, y, 0.0, s)
