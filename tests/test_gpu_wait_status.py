"""The bounded LDS waits of the MFMA kernels (gs_gemm's double-buffered steps, gs_moe_grouped's
activation slots and epilogue operands) report an expiry instead of passing silently: the host's
test hook makes every wait run to a tiny poll bound (each kernel still runs to its end), and
gs_wait_status must then return an error once, and clear it. With the default bound the same
calls report nothing and match the oracle."""
import sys

import numpy as np
import pytest

import glmssd as G
from glmssd import GgmlType as T
from glmssd import moe as M
import oracle as O

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _gemm(s):
    ty, K, rows, N = T.Q8_0, 1024, 256, 64   # Q8_0: the double-buffered steps with fill waits
    rb = G.row_bytes(ty, K)
    raw = O.Rng(3).random_blocks(ty, rows * K)
    X = np.random.default_rng(4).standard_normal((N, K)).astype(np.float32)
    dw, dx, dy = G.DeviceBuffer.from_array(raw), G.DeviceBuffer.from_array(X), G.DeviceBuffer(N * rows * 4)
    G.ops.gemm(ty, dw, rb, K, rows, dx, K, dy, rows, N, False, 1, 0, 0, 0, s)
    got = dy.download(np.float32, N * rows, s).reshape(N, rows)
    want = O.gemv(ty, raw, rb, K, rows, X, B=N, act="f16", nthreads=8)
    return float(np.linalg.norm(got - want) / np.linalg.norm(want))


def _grouped(s):
    n_exp, n_tok, k, n_embd, n_ff = 8, 24, 2, 512, 512
    rng = O.Rng(5)
    gate = [rng.random_blocks(T.IQ2_XXS, n_ff * n_embd) for _ in range(n_exp)]
    up = [rng.random_blocks(T.IQ2_XXS, n_ff * n_embd) for _ in range(n_exp)]
    down = [rng.random_blocks(T.IQ2_XXS, n_embd * n_ff) for _ in range(n_exp)]
    nrng = np.random.default_rng(6)
    routes = [[(int(e), 0.5) for e in nrng.choice(n_exp, k, replace=False)] for _ in range(n_tok)]
    layer = M.ResidentMoeLayer(gate, up, down, n_embd, n_ff)
    layer.upload_routes(routes, s)
    x = nrng.standard_normal((n_tok, n_embd)).astype(np.float32)
    dx = G.DeviceBuffer.from_array(x)
    dy = G.DeviceBuffer.from_array(np.zeros((n_tok, n_embd), np.float32))
    layer.forward(dx, dy, n_tok, 0.0, s)
    return dy.download(np.float32, n_tok * n_embd, s)


def test_wait_expiry_is_reported():
    s = G.Stream()
    G.ops.wait_status(s)   # nothing pending from earlier tests
    try:
        for name, run in (("gemm", _gemm), ("grouped", _grouped)):
            say(f"{name}: every LDS wait forced to expire after 4 polls")
            G.ops.debug_wait_limit(4, force=True)
            run(s)
            with pytest.raises(G.GsError):
                G.ops.wait_status(s)
            G.ops.wait_status(s)   # the query cleared the flag
    finally:
        G.ops.debug_wait_limit(1 << 16, force=False)
    say("default bound: no expiry, results as the oracle")
    assert _gemm(s) <= 1e-5
    assert np.all(np.isfinite(_grouped(s)))
    G.ops.wait_status(s)
