"""Seeded synthetic inputs for the benchmark configurations (BASELINE.json `configs`).

Weights are random quantized blocks with sane f16 scales; activations N(0,1). All generation is
numpy on the host; the arrays are uploaded once and stay resident in HBM.
"""
import numpy as np

from .types import GgmlType as T, block, row_bytes


def _set_half(raw, bb, off, vals):
    blk = raw.reshape(-1, bb)
    blk[:, off:off + 2] = np.asarray(vals, dtype=np.float16).view(np.uint8).reshape(-1, 2)


def q8_0_matrix(rng, rows, K):
    """int8 quants uniform in [-127,127], f16 d = |N(0,1)|/127 (config 1)."""
    nb = rows * K // 32
    raw = np.empty((nb, 34), dtype=np.uint8)
    raw[:, 2:] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    _set_half(raw, 34, 0, np.abs(rng.standard_normal(nb)) / 127.0)
    return raw.reshape(-1)


def random_blocks(rng, ty, n_elems, scale_sigma, half_offs):
    """Random bytes with the f16 scale fields at `half_offs` set to |N(0, scale_sigma)|."""
    be, bb = block(ty)
    nb = n_elems // be
    raw = np.frombuffer(rng.bytes(nb * bb), dtype=np.uint8).copy()
    for off in half_offs:
        _set_half(raw, bb, off, np.abs(rng.standard_normal(nb)) * scale_sigma)
    return raw


def iq2_xxs_expert(rng, n_embd=4096, n_ff=1536):
    """gate, up [n_ff rows x n_embd], down [n_embd rows x n_ff]; d ~ |N(0,0.02)| (config 2)."""
    g = random_blocks(rng, T.IQ2_XXS, n_ff * n_embd, 0.02, [0])
    u = random_blocks(rng, T.IQ2_XXS, n_ff * n_embd, 0.02, [0])
    d = random_blocks(rng, T.IQ2_XXS, n_embd * n_ff, 0.02, [0])
    return g, u, d


def q4_k_matrix(rng, rows, K):
    return random_blocks(rng, T.Q4_K, rows * K, 0.01, [0, 2])


def q6_k_matrix(rng, rows, K):
    return random_blocks(rng, T.Q6_K, rows * K, 0.01, [208])


def softmax(v):
    v = np.asarray(v, dtype=np.float64)
    e = np.exp(v - v.max())
    return (e / e.sum()).astype(np.float32)


def zipf_topk(rng, n_tokens, n_expert=288, k=8, s=1.1):
    """Per token k distinct experts drawn Zipf(s) over a seeded permutation of expert ids, with
    softmax weights over N(0,1) logits (configs 4 and 5)."""
    perm = rng.permutation(n_expert)
    p = 1.0 / np.arange(1, n_expert + 1) ** s
    p /= p.sum()
    routes = []
    for _ in range(n_tokens):
        ranks = rng.choice(n_expert, size=k, replace=False, p=p)
        experts = perm[ranks]
        routes.append((experts.astype(np.int32), softmax(rng.standard_normal(k))))
    return routes


def expert_bytes(n_embd=4096, n_ff=1536, ty=T.IQ2_XXS):
    return 2 * n_ff * row_bytes(ty, n_embd) + n_embd * row_bytes(ty, n_ff)
