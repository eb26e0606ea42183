"""Writes tests/golden/golden.npz: small seeded inputs and the oracle's outputs for them, frozen.

The reference holds no golden vectors for this path (its quantized-matmul tests compare against
gguf-py at run time), so these fixtures come from this repository's oracle after its own pins
(tests/test_oracle.py). They freeze its results, the q8_1 rounding convention included: any later
change to the oracle or to the GPU path that moves a result shows up against them.

Inputs are stored as bytes (weights: the reference qtest generator, xorshift64* seeded per case);
the expert FFN cases store their generator seed instead of ~100 KB of expert weights.
Run from the repository root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402

TYPES = [0, 1, 30, 8, 10, 11, 12, 13, 14, 16, 22, 18, 23]   # F32 F16 BF16 Q8_0 Q2_K..Q6_K IQ2_XXS IQ2_S IQ3_XXS IQ4_XS
HOT = [8, 12, 14, 16, 18]                                    # Q8_0 Q4_K Q6_K IQ2_XXS IQ3_XXS


def q81_vector():
    """256 values: ordinary N(0,1) blocks, a block of exact halves with d = 1 (round-half-away ties),
    a zero block, a block of f32 subnormals, a block with one huge value, all-negative values."""
    rng = np.random.default_rng(81)
    x = rng.standard_normal(256).astype(np.float32)
    x[32:64] = (np.arange(32) - 15.5).astype(np.float32)   # ties: -15.5 .. 15.5
    x[63] = 127.0                                           # amax 127: d = 1 exactly
    x[64:96] = 0.0
    x[96:128] = np.float32(1e-40) * (np.arange(32) - 16)
    x[128:160] = rng.standard_normal(32).astype(np.float32)
    x[140] = 3.0e4
    x[160:192] = -np.abs(rng.standard_normal(32)).astype(np.float32)
    return x


def ffn_case(seed, n_exp, K, n_ff, ty_gu, ty_dn):
    rng = O.Rng(seed)
    gate = [rng.random_blocks(ty_gu, n_ff * K) for _ in range(n_exp)]
    up = [rng.random_blocks(ty_gu, n_ff * K) for _ in range(n_exp)]
    down = [rng.random_blocks(ty_dn, K * n_ff) for _ in range(n_exp)]
    return gate, up, down


FFN = {  # name: (seed, n_exp, K, n_ff, ty_gu, ty_dn, tokens, act)
    "ffn_decode": (7001, 4, 512, 256, 16, 16, 1, "q8_1"),
    "ffn_grouped": (7002, 4, 512, 512, 16, 18, 6, "f16sx"),
}


def ffn_routes(n_tok, n_exp):
    rng = np.random.default_rng(n_tok * 100 + n_exp)
    tok, exp, w = [], [], []
    for t in range(n_tok):
        for e in rng.permutation(n_exp)[:2]:
            tok.append(t); exp.append(int(e)); w.append(float(rng.uniform(0.1, 1.0)))
    return np.array(tok, np.int32), np.array(exp, np.int32), np.array(w, np.float32)


def main():
    out = {}
    for ty in TYPES:
        e, b = O.block(ty)
        n = 512 if e == 1 else 2 * e
        raw = O.Rng(100 + ty).random_blocks(ty, n)
        out[f"deq_raw_{ty}"] = raw
        out[f"deq_out_{ty}"] = O.dequantize(ty, raw, n)
    x = q81_vector()
    out["q81_x"] = x
    out["q81_q"] = O.quantize_q8_1(x)
    K, rows, B = 512, 8, 3
    xg = np.random.default_rng(5).standard_normal((B, K)).astype(np.float32)
    out["gemv_x"] = xg
    for ty in HOT:
        raw = O.Rng(200 + ty).random_blocks(ty, rows * K)
        out[f"gemv_w_{ty}"] = raw
        out[f"gemv_y_{ty}"] = O.gemv(ty, raw, O.row_bytes(ty, K), K, rows, xg, B=B).astype(np.float32)
    Kg, rg, N = 512, 16, 9
    xm = np.random.default_rng(6).standard_normal((N, Kg)).astype(np.float32)
    out["gemm_x"] = xm
    for ty in (8, 12, 16):
        raw = O.Rng(300 + ty).random_blocks(ty, rg * Kg)
        out[f"gemm_w_{ty}"] = raw
        out[f"gemm_y_{ty}"] = O.gemv(ty, raw, O.row_bytes(ty, Kg), Kg, rg, xm, B=N, act="f16").astype(np.float32)
    for name, (seed, n_exp, Kf, n_ff, ty_gu, ty_dn, n_tok, act) in FFN.items():
        gate, up, down = ffn_case(seed, n_exp, Kf, n_ff, ty_gu, ty_dn)
        xf = np.random.default_rng(seed).standard_normal((n_tok, Kf)).astype(np.float32)
        tok, exp, w = ffn_routes(n_tok, n_exp)
        y = O.moe_ffn(ty_gu, ty_dn, gate, up, down, O.row_bytes(ty_gu, Kf), O.row_bytes(ty_dn, n_ff), Kf, n_ff, xf,
                      tok, exp, w, act=act)
        out[f"{name}_x"] = xf
        out[f"{name}_pairs"] = np.stack([tok, exp]).astype(np.int32)
        out[f"{name}_w"] = w
        out[f"{name}_y"] = y.astype(np.float32)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
