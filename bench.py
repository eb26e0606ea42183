"""Benchmark of the quantized-matmul hot path on one MI355X.

Headline: routed-expert FFN for one decode token, 8 IQ2_XXS experts of
288 resident in HBM (hidden 4096, intermediate 1536). One step = gs_moe_gateup + gs_moe_down (the
engine's fused decode path) for one token; each step routes to the next 8 experts of a seeded
permutation, so an expert's 4.87 MB come back only after all 288 (1.4 GB) were read: no step is
served from the 256 MB last-level cache. value = algorithmic weight bytes per step / step time.

Also reported (secondary): config 1 (Q8_0 GEMV), config 3 (Q4_K / Q6_K GEMV), weight copies
rotated over > 512 MB. The CPU baseline is the oracle's C port of the reference CPU path
(crates/quants dequantize + f64 dot, crates/engine/src/qtest.rs:77-108) on a bounded sample.

Each timed loop runs its W warm-up steps and then more, untimed, until at least --ramp-ms
(default 100) of GPU time has passed: after the host has spent seconds generating a workload's
data the GPU's clocks need tens of milliseconds of load to come back up (config 2: 17.9 us per step
after 50 warm-up steps, 16.7 us once 85 ms of steps have run). Then exactly K steps are timed,
continuing the weight rotation.

Usage: python bench.py [--gpus 1] [--steps 500] [--warmup 50] [--ramp-ms 100] [--no-cpu] [--calib]
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "glm-ssd_amd"))

METRIC = "quant-GEMV weight GB/s (% HBM peak); MoE grouped-GEMM TFLOP/s at 512 tok"
HBM_PEAK_GBPS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0   # dense f16 MFMA (the grouped GEMM's operand type)


GATEUP_KERNEL = "gs_k_stream_16_1_1_4_w"   # the kernel gs_moe_gateup launches for config 2


def profile_entry(kernel, key):
    """`key` of `kernel` in the committed rocprofv3 counter summary, if it covers them."""
    try:
        with open(os.path.join(ROOT, "profiles", "stream_kernels_traffic.json")) as f:
            return json.load(f)["kernels"][kernel][key]
    except (OSError, KeyError, ValueError):
        return None


def traffic_bytes(kernel):
    """HBM bytes per launch from the committed rocprofv3 counter summary."""
    return profile_entry(kernel, "traffic_bytes")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def bench_lib():
    import glmssd
    glmssd.lib()
    L = C.CDLL(os.path.join(ROOT, "glm-ssd_amd", "libglmssd_bench.so"))
    P, I64 = C.c_void_p, C.c_int64
    L.bn_moe_decode.argtypes = [C.c_int, C.c_int, P, C.c_int, C.c_int, I64, C.c_int, C.c_int, I64, P, P, P, C.c_int,
                                C.c_int, P, C.POINTER(C.c_float), C.POINTER(C.c_float)]
    L.bn_gemv.argtypes = [C.c_int, P, C.c_int, I64, C.c_int, C.c_int, P, P, C.c_int, C.c_int, C.c_int, P,
                          C.POINTER(C.c_float)]
    L.bn_moe_ffn.argtypes = [C.c_int, C.c_int, P, C.c_int, C.c_int, I64, C.c_int, C.c_int, I64, P, P, P, C.c_int,
                             C.c_int, P, C.POINTER(C.c_float)]
    L.bn_moe_ffn_tokens.argtypes = [C.c_int, C.c_int, P, C.c_int, C.c_int, I64, C.c_int, C.c_int, I64, P, P, P,
                                    C.c_int, C.c_int, P, C.POINTER(C.c_float)]
    L.bn_copy.argtypes = [P, P, C.c_size_t, C.c_int, P, C.POINTER(C.c_float)]
    L.bn_read.argtypes = [P, C.c_int, C.c_size_t, C.c_int, C.c_int, P, C.POINTER(C.c_float)]
    L.bn_gemm.argtypes = [C.c_int, P, C.c_int, I64, C.c_int, C.c_int, P, P, C.c_int, C.c_int, C.c_int, P,
                          C.c_size_t, P, C.POINTER(C.c_float)]
    L.bn_set_ramp_ms.argtypes = [C.c_float]
    L.bn_set_ramp_ms.restype = None
    L.bn_moe_grouped.argtypes = [C.c_int, C.c_int, P, C.c_int, C.c_int, P, P, P, P, C.c_int, I64, C.c_int, C.c_int, I64, P, P,
                                 P, C.c_size_t, C.c_int, C.c_int, P, C.POINTER(C.c_float)]
    return L


def run_moe_decode(L, s, steps, warmup, n_expert=288, n_embd=4096, n_ff=1536, seed=2, ty_dn=None, label="config 2"):
    """Decode-step FFN over 8 of n_expert resident experts, a new 8 each step (rotation defeats the
    last-level cache). IQ2_XXS gate/up; down IQ2_XXS (config 2) or ty_dn."""
    import glmssd as G
    from glmssd import synth
    ty = G.GgmlType.IQ2_XXS
    ty_dn = ty if ty_dn is None else ty_dn
    rng = np.random.default_rng(seed)
    rbg, rbd = G.row_bytes(ty, n_embd), G.row_bytes(ty_dn, n_ff)
    mat = n_ff * rbg                       # bytes of one gate (= up) matrix
    mat_dn = n_embd * rbd                  # bytes of one down matrix
    gate = G.DeviceBuffer(n_expert * mat)
    up = G.DeviceBuffer(n_expert * mat)
    down = G.DeviceBuffer(n_expert * mat_dn)
    log(f"{label}: generating {n_expert * (2 * mat + mat_dn) / 1e9:.2f} GB of experts")
    for e in range(n_expert):
        if ty_dn == ty:
            g, u, d = synth.iq2_xxs_expert(rng, n_embd, n_ff)
        else:
            g = synth.random_blocks(rng, ty, n_ff * n_embd, 0.02, [0])
            u = synth.random_blocks(rng, ty, n_ff * n_embd, 0.02, [0])
            d = synth.random_blocks(rng, ty_dn, n_embd * n_ff, 0.02, [0])
        gate.upload(g, s, e * mat)
        up.upload(u, s, e * mat)
        down.upload(d, s, e * mat_dn)
    x = rng.standard_normal(n_embd).astype(np.float32)
    dx = G.DeviceBuffer.from_array(x, s)
    dh = G.DeviceBuffer(8 * n_ff * 4)
    dy = G.DeviceBuffer(n_embd * 4)
    dy.zero(s)
    # n_expert/8 batches = one pass over a permutation of all experts, 8 distinct per step
    perm = rng.permutation(n_expert)
    nb = n_expert // 8
    batches = (G.MoeBatch * nb)()
    for i in range(nb):
        b = batches[i]
        b.n = 8
        w = synth.softmax(rng.standard_normal(8))
        for j in range(8):
            e = int(perm[8 * i + j])
            b.gate[j] = gate.p.value + e * mat
            b.up[j] = up.p.value + e * mat
            b.down[j] = down.p.value + e * mat_dn
            b.w[0][j] = w[j]
    ms, msg = C.c_float(), C.c_float()
    rc = L.bn_moe_decode(ty, ty_dn, C.cast(batches, C.c_void_p), nb, 1, rbg, n_embd, n_ff, rbd, dx.p, dh.p, dy.p,
                         steps, warmup, s.raw(), C.byref(ms), C.byref(msg))
    G.check(rc)
    step_bytes = 8 * (2 * mat + mat_dn)
    gu_bytes = 8 * 2 * mat
    keep = (gate, up, down, dx, dh, dy, batches)
    layer = dict(gate=gate, up=up, down=down, mat=mat, mat_dn=mat_dn, n_expert=n_expert, n_embd=n_embd, n_ff=n_ff,
                 rbg=rbg, rbd=rbd, ty_gu=int(ty), ty_dn=int(ty_dn))
    return dict(ms_step=ms.value, ms_gateup=msg.value, step_bytes=step_bytes, gateup_bytes=gu_bytes,
                flops=8 * 3 * 2 * n_ff * n_embd), keep, layer


def run_moe_grouped(L, s, layer, n_tok, steps, warmup, seed, n_rout=4, k=8):
    """Configs 4 and 5: n_tok tokens through one MoE layer of the 288 resident experts, top-k per token
    drawn Zipf(1.1) over a seeded permutation (a fresh permutation per routing, n_rout routings
    rotated), one gs_moe_grouped call per step."""
    import glmssd as G
    from glmssd import synth
    from glmssd.moe import group_pairs
    n_exp, mat, mat_dn = layer["n_expert"], layer["mat"], layer["mat_dn"]
    tab = (G.ExpertPtrs * n_exp)()
    for e in range(n_exp):
        tab[e].gate = layer["gate"].p.value + e * mat
        tab[e].up = layer["up"].p.value + e * mat
        tab[e].down = layer["down"].p.value + e * mat_dn
    dtab = G.DeviceBuffer.from_array(np.frombuffer(bytes(tab), dtype=np.uint8), s)
    rng = np.random.default_rng(seed)
    keep, offs_p, idx_p, w_p, npairs, uniq, maxg = [dtab], [], [], [], [], [], []
    for _ in range(n_rout):
        routes = [list(zip(e, w)) for e, w in synth.zipf_topk(rng, n_tok, n_exp, k)]
        offs, idx, w, _pe = group_pairs(routes, n_exp)
        bufs = [G.DeviceBuffer.from_array(a, s) for a in (offs, idx, w)]
        keep += bufs
        offs_p.append(bufs[0].p.value); idx_p.append(bufs[1].p.value); w_p.append(bufs[2].p.value)
        npairs.append(int(idx.size))
        uniq.append(int(np.count_nonzero(np.diff(offs))))
        maxg.append(int(np.diff(offs).max()))
    n_embd, n_ff = layer["n_embd"], layer["n_ff"]
    x = G.DeviceBuffer.from_array(rng.standard_normal((n_tok, n_embd)).astype(np.float32), s)
    y = G.DeviceBuffer(n_tok * n_embd * 4)
    y.zero(s)
    wb = max(G.ops.moe_grouped_workspace(n_tok, n, n_embd, n_ff) for n in npairs)
    work = G.DeviceBuffer(wb)
    A = lambda v, t: (t * len(v))(*v)
    ms = C.c_float()
    G.check(L.bn_moe_grouped(layer["ty_gu"], layer["ty_dn"], dtab.p, n_exp, n_rout,
                             C.cast(A(offs_p, C.c_void_p), C.c_void_p),
                             C.cast(A(idx_p, C.c_void_p), C.c_void_p), C.cast(A(w_p, C.c_void_p), C.c_void_p),
                             C.cast(A(npairs, C.c_int), C.c_void_p), n_tok, layer["rbg"], n_embd, n_ff, layer["rbd"],
                             x.p, y.p, work.p, wb, steps, warmup, s.raw(), C.byref(ms)))
    u = float(np.mean(uniq))
    wbytes = u * (2 * mat + mat_dn)
    flops = float(np.mean(npairs)) * 3 * 2 * n_ff * n_embd
    t = ms.value * 1e-3
    return dict(us_per_step=round(ms.value * 1e3, 2), unique_experts=round(u, 1), max_group=max(maxg),
                pairs=int(np.mean(npairs)), weight_bytes=int(wbytes), GBps=round(wbytes / t / 1e9, 1),
                frac_hbm_peak=round(wbytes / t / 1e9 / HBM_PEAK_GBPS, 4), TFLOPs=round(flops / t / 1e12, 2),
                frac_mfma_f16_peak=round(flops / t / 1e12 / MFMA_F16_PEAK_TFLOPS, 4), routings_rotated=n_rout)


def run_moe_per_token(L, s, layer, n_tok, steps, warmup, seed, n_rout=4, k=8):
    """Config 4 as one-token FFNs, each token over its own top-k experts (Zipf(1.1) routings as
    run_moe_grouped draws them, n_rout rotated), timed two ways: n_tok gs_moe_ffn calls per step
    (bn_moe_ffn, us_per_step) and one gs_moe_ffn_tokens call per step, the MoE layer's path
    (bn_moe_ffn_tokens, us_per_step_one_call)."""
    import glmssd as G
    from glmssd import synth
    n_exp, mat, mat_dn = layer["n_expert"], layer["mat"], layer["mat_dn"]
    rng = np.random.default_rng(seed)
    batches = (G.MoeBatch * (n_rout * n_tok))()
    uniq = []
    for r in range(n_rout):
        routes = synth.zipf_topk(rng, n_tok, n_exp, k)
        uniq.append(len({int(e) for ex, _ in routes for e in ex}))
        for t, (ex, w) in enumerate(routes):
            b = batches[r * n_tok + t]
            b.n = len(ex)
            for j, (e, wj) in enumerate(zip(ex, w)):
                e = int(e)
                b.gate[j] = layer["gate"].p.value + e * mat
                b.up[j] = layer["up"].p.value + e * mat
                b.down[j] = layer["down"].p.value + e * mat_dn
                b.w[0][j] = float(wj)
    n_embd, n_ff = layer["n_embd"], layer["n_ff"]
    x = G.DeviceBuffer.from_array(rng.standard_normal(n_embd).astype(np.float32), s)
    h = G.DeviceBuffer(k * n_ff * 4)
    y = G.DeviceBuffer(n_embd * 4)
    y.zero(s)
    ms = C.c_float()
    G.check(L.bn_moe_ffn(layer["ty_gu"], layer["ty_dn"], C.cast(batches, C.c_void_p), n_rout * n_tok, 1,
                         layer["rbg"], n_embd, n_ff, layer["rbd"], x.p, h.p, y.p, steps * n_tok, warmup * n_tok,
                         s.raw(), C.byref(ms)))
    t = ms.value * n_tok * 1e-3
    wbytes = float(np.mean(uniq)) * (2 * mat + mat_dn)
    # the same steps as one gs_moe_ffn_tokens call each (token t in blockIdx.y slice t)
    xs = G.DeviceBuffer.from_array(rng.standard_normal((n_tok, n_embd)).astype(np.float32), s)
    hs = G.DeviceBuffer(n_tok * k * n_ff * 4)
    ys = G.DeviceBuffer(n_tok * n_embd * 4)
    ys.zero(s)
    G.check(L.bn_moe_ffn_tokens(layer["ty_gu"], layer["ty_dn"], C.cast(batches, C.c_void_p), n_rout, n_tok,
                                layer["rbg"], n_embd, n_ff, layer["rbd"], xs.p, hs.p, ys.p, steps, warmup, s.raw(),
                                C.byref(ms)))
    t1 = ms.value * 1e-3
    return dict(us_per_step=round(t * 1e6, 2), us_per_step_one_call=round(t1 * 1e6, 2),
                unique_experts=round(float(np.mean(uniq)), 1), weight_bytes=int(wbytes), GBps=round(wbytes / t / 1e9, 1),
                GBps_one_call=round(wbytes / t1 / 1e9, 1), frac_hbm_peak=round(wbytes / t / 1e9 / HBM_PEAK_GBPS, 4),
                calls_per_step=n_tok, routings_rotated=n_rout)


def run_read_ceiling(L, s, sizes, steps, warmup, ramp_ms, min_pool=768 << 20):
    """Plain HBM read (bench_kernels.hip bn_k_read_*, the best of its read shapes) of each byte count, the start address rotated
    over a pool of at least 768 MB so no call is served from the last-level cache: the achievable
    ceiling the streaming kernels are compared with at the same byte count. The warm-up floor
    applies before the first size only (the sizes follow each other with no idle time between
    them), so every later size is exactly `warmup` + `steps` launches."""
    import glmssd as G
    sizes = [(n + 4095) // 4096 * 4096 for n in sizes]
    pool_bytes = max(min_pool, max(sizes))
    pool = G.DeviceBuffer(pool_bytes)
    out = {}
    for n in sizes:
        nb = max(1, min(64, pool_bytes // n))
        step = (pool_bytes - n) // max(1, nb - 1) // 4096 * 4096 if nb > 1 else 0
        offs = [i * step for i in range(nb)]
        assert all(o + n <= pool_bytes for o in offs)   # every read stays inside the pool
        bases = (C.c_void_p * nb)(*[pool.p.value + o for o in offs])
        ms = C.c_float()
        L.bn_set_ramp_ms(ramp_ms if n == sizes[0] else 0.0)
        G.check(L.bn_read(C.cast(bases, C.c_void_p), nb, n, steps, warmup, s.raw(), C.byref(ms)))
        out[str(n)] = {"bytes": n, "us": round(ms.value * 1e3, 2), "GB/s": round(n / (ms.value * 1e-3) / 1e9, 1),
                       "rotated_bases": nb}
    L.bn_set_ramp_ms(ramp_ms)
    return out


def run_gemv(L, s, ty, rows, K, make, steps, warmup, seed, min_rot_bytes=640 << 20, B=1):
    import glmssd as G
    rng = np.random.default_rng(seed)
    raw = make(rng, rows, K)
    n = max(2, -(-min_rot_bytes // raw.nbytes))
    buf = G.DeviceBuffer(n * raw.nbytes)
    buf.upload(raw, s)
    for i in range(1, n):
        G.check(G.lib().gs_memcpy_d2d(buf.ptr(i * raw.nbytes), buf.p, raw.nbytes, s.raw()))
    s.sync()
    ptrs = (C.c_void_p * n)(*[buf.p.value + i * raw.nbytes for i in range(n)])
    x = G.DeviceBuffer.from_array(rng.standard_normal(B * K).astype(np.float32), s)
    y = G.DeviceBuffer(B * rows * 4)
    ms = C.c_float()
    G.check(L.bn_gemv(ty, C.cast(ptrs, C.c_void_p), n, G.row_bytes(ty, K), K, rows, x.p, y.p, B, steps, warmup,
                      s.raw(), C.byref(ms)))
    return dict(ms=ms.value, bytes=raw.nbytes, gbps=raw.nbytes / (ms.value * 1e-3) / 1e9, copies=n)


def run_gemm(L, s, ty, rows, K, N, make, steps, warmup, seed, min_rot_bytes=640 << 20, use_work=True):
    """gs_gemm_ex of N tokens through a rows x K matrix, weight copies rotated, with the workspace
    gs_gemm_workspace asks for (K split of small problems; from N = 256 the f16 dequant + library
    GEMM path); use_work=False: no workspace, i.e. plain gs_gemm's f16 MFMA tiles."""
    import glmssd as G
    rng = np.random.default_rng(seed)
    raw = make(rng, rows, K)
    n = max(2, -(-min_rot_bytes // raw.nbytes))
    buf = G.DeviceBuffer(n * raw.nbytes)
    buf.upload(raw, s)
    for i in range(1, n):
        G.check(G.lib().gs_memcpy_d2d(buf.ptr(i * raw.nbytes), buf.p, raw.nbytes, s.raw()))
    s.sync()
    ptrs = (C.c_void_p * n)(*[buf.p.value + i * raw.nbytes for i in range(n)])
    x = G.DeviceBuffer.from_array(rng.standard_normal(N * K).astype(np.float32), s)
    y = G.DeviceBuffer(N * rows * 4)
    need = G.ops.gemm_workspace(K, rows, N) if use_work else 0
    wk = G.DeviceBuffer(need) if need else None
    ms = C.c_float()
    G.check(L.bn_gemm(ty, C.cast(ptrs, C.c_void_p), n, G.row_bytes(ty, K), K, rows, x.p, y.p, N, steps, warmup,
                      wk.p if wk else None, need, s.raw(), C.byref(ms)))
    t = ms.value * 1e-3
    flops = 2.0 * N * rows * K
    return {"us_per_call": round(ms.value * 1e3, 2), "TFLOPs": round(flops / t / 1e12, 1), "workspace_bytes": need,
            "frac_mfma_f16_peak": round(flops / t / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
            "weight_GBps": round(raw.nbytes / t / 1e9, 1), "tokens": N, "rotated_copies": n}


GROUPED_KERNELS = ("gs_k_grouped_16_1_2_2_8", "gs_k_grouped_16_2_2_4_8")   # config 5's gate/up and down


def config5_roofline(r):
    """BASELINE's second metric: the 512-token grouped MoE step against the HBM and f16 MFMA peaks."""
    if not r:
        return None
    tr = [traffic_bytes(k) for k in GROUPED_KERNELS]
    ctr = [profile_entry(k, "counters") for k in GROUPED_KERNELS]
    busy = None
    if all(c is not None for c in ctr):
        busy = {"gate_up": ctr[0]["mfma_busy_frac"], "down": ctr[1]["mfma_busy_frac"],
                "valu_active": [c["valu_active_frac"] for c in ctr],
                "source": "profiles/stream_kernels_traffic.json (rocprofv3 SQ_VALU_MFMA_BUSY_CYCLES / 4 / "
                          "SQ_BUSY_CU_CYCLES per kernel, padded token slots included)"}
    return {"bound": "hbm", "achieved": r["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": round(r["GBps"] / HBM_PEAK_GBPS, 4),
            "traffic": sum(tr) if all(t is not None for t in tr) else None,
            "traffic_source": "profiles/stream_kernels_traffic.json (gate/up + down kernels, rocprofv3 FETCH_SIZE + "
                              "WRITE_SIZE, calibrated on a 1 GiB device copy)",
            "algorithmic_bytes_per_step": r["weight_bytes"], "us_per_step": r["us_per_step"],
            "mfma": {"achieved": r["TFLOPs"], "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": r["frac_mfma_f16_peak"], "dtype": "f16 x f16 -> f32 (v_mfma_f32_16x16x32_f16)",
                     "busy": busy}}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(budget_s=10.0, n_embd=4096, n_ff=1536, seed=2):
    """Oracle (C port of crates/quants dequantize + f64 dot, the reference CPU path of
    crates/engine/src/qtest.rs:77-108) on the config-2 FFN: one thread, as the reference runs it,
    then every host core."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    from glmssd import synth
    import glmssd as G
    ty = G.GgmlType.IQ2_XXS
    rng = np.random.default_rng(seed)
    experts = [synth.iq2_xxs_expert(rng, n_embd, n_ff) for _ in range(8)]
    gate, up, down = [e[0] for e in experts], [e[1] for e in experts], [e[2] for e in experts]
    x = rng.standard_normal((1, n_embd)).astype(np.float32)
    w = synth.softmax(rng.standard_normal(8))
    rbg, rbd = G.row_bytes(ty, n_embd), G.row_bytes(ty, n_ff)
    step_bytes = 8 * 3 * n_ff * rbg

    def timed(threads, budget):
        t0 = time.perf_counter()
        steps = 0
        while True:
            O.moe_ffn(ty, ty, gate, up, down, rbg, rbd, n_embd, n_ff, x, [0] * 8, list(range(8)), w, nthreads=threads)
            steps += 1
            el = time.perf_counter() - t0
            if el >= budget or steps >= 200:
                return steps, el

    n1, t1 = timed(1, budget_s)
    host = os.cpu_count() or 1
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else host
    cores = min(16, avail)   # a GPU box's CPU share is 16 threads whatever the host has
    na, ta = timed(cores, budget_s / 2)
    model = cpu_model()
    return {"value": round(step_bytes * n1 / t1 / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{n1} config-2 steps (8 IQ2_XXS experts, 1 token) in {t1:.1f} s, oracle C port "
                      f"(dequantize + f64 dot), 1 thread as the reference CPU path runs",
            "ms_per_step": round(t1 / n1 * 1e3, 2), "cpu_model": model, "host_cores": host,
            "cores_available": avail,
            "all_cores": {"value": round(step_bytes * na / ta / 1e9, 4), "unit": "GB/s", "cores": cores,
                          "ms_per_step": round(ta / na * 1e3, 2),
                          "sample": f"{na} config-2 steps in {ta:.1f} s, {cores} threads (rows split)"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--ramp-ms", type=float, default=100.0,
                    help="minimum GPU time of each timed loop's warm-up (the W steps, then more until this much "
                         "GPU time has passed): the clocks come back up from idle over tens of milliseconds")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--calib", action="store_true", help="also run a 1 GiB d2d copy (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU (the hot path has no multi-GPU part); --gpus {args.gpus} "
              "is not supported", file=sys.stderr)
        sys.exit(2)
    import glmssd as G
    L = bench_lib()
    L.bn_set_ramp_ms(args.ramp_ms)
    s = G.Stream()
    info = G.device_info(0)
    log(f"device: {info.name.decode()} CUs={info.sm_count}")

    res, keep, layer = run_moe_decode(L, s, args.steps, args.warmup)
    value = res["step_bytes"] / (res["ms_step"] * 1e-3) / 1e9
    gu_gbps = res["gateup_bytes"] / (res["ms_gateup"] * 1e-3) / 1e9
    log(f"config 2: {res['ms_step'] * 1e3:.2f} us/step, {value:.1f} GB/s; gate/up kernel {res['ms_gateup'] * 1e3:.2f} us "
        f"= {gu_gbps:.1f} GB/s")

    secondary = {}
    if not args.no_secondary:
        gsteps, gwarm = max(10, args.steps // 10), max(3, args.warmup // 10)
        for name, n_tok, seed in [("config4_mtp_verify_4tok_grouped", 4, 4), ("config5_prefill_512tok_grouped", 512, 5)]:
            r = run_moe_grouped(L, s, layer, n_tok, gsteps, gwarm, seed)
            secondary[name] = r
            log(f"{name}: {r}")
        r = run_moe_per_token(L, s, layer, 4, gsteps, gwarm, 4)
        secondary["config4_mtp_verify_4tok_per_token_ffn"] = r
        log(f"config4_mtp_verify_4tok_per_token_ffn: {r}")
    del keep, layer
    if not args.no_secondary:
        # the target model's routed experts: IQ2_XXS gate/up, IQ3_XXS down, n_ff_exp = 2048
        rr, keep2, layer2 = run_moe_decode(L, s, args.steps, args.warmup, n_expert=96, n_ff=2048, seed=6,
                                           ty_dn=G.GgmlType.IQ3_XXS, label="target-model decode FFN")
        secondary["decode_ffn_iq2xxs_gateup_iq3xxs_down_nff2048"] = {
            "us_per_step": round(rr["ms_step"] * 1e3, 2), "GB/s": round(rr["step_bytes"] / rr["ms_step"] / 1e6, 1),
            "weight_bytes": rr["step_bytes"],
            "experts_resident": 96}
        log(f"target-model decode FFN: {secondary['decode_ffn_iq2xxs_gateup_iq3xxs_down_nff2048']}")
        # config 5's 512-token prefill on the target model's expert types and shapes
        r = run_moe_grouped(L, s, layer2, 512, gsteps, gwarm, 7)
        secondary["prefill_512tok_grouped_iq2xxs_gateup_iq3xxs_down_nff2048"] = r
        log(f"target-model prefill: {r}")
        del keep2, layer2
        from glmssd import synth
        r1 = run_gemv(L, s, G.GgmlType.Q8_0, 4096, 4096, synth.q8_0_matrix, args.steps, args.warmup, 1)
        r3a = run_gemv(L, s, G.GgmlType.Q4_K, 12288, 4096, synth.q4_k_matrix, args.steps, args.warmup, 3)
        r3b = run_gemv(L, s, G.GgmlType.Q6_K, 4096, 12288, synth.q6_k_matrix, args.steps, args.warmup, 4)
        for B in (2, 4, 8):
            rb = run_gemv(L, s, G.GgmlType.Q8_0, 4096, 4096, synth.q8_0_matrix, args.steps, args.warmup, 1, B=B)
            secondary[f"config1_q8_0_gemv_4096x4096_B{B}"] = {
                "GB/s": round(rb["gbps"], 1), "us_per_call": round(rb["ms"] * 1e3, 2),
                "frac_hbm_peak": round(rb["gbps"] / HBM_PEAK_GBPS, 4), "weight_bytes": rb["bytes"], "vectors": B}
            log(f"config1 B={B}: {rb['ms'] * 1e3:.2f} us, {rb['gbps']:.1f} GB/s")
        # config 3's matrices with several vectors (multi-token decode: MTP verify)
        for name, ty, rows, K, mk in (("config3_q4_k_gemv_k4096_rows12288", G.GgmlType.Q4_K, 12288, 4096, synth.q4_k_matrix),
                                      ("config3_q6_k_gemv_k12288_rows4096", G.GgmlType.Q6_K, 4096, 12288, synth.q6_k_matrix)):
            for B in (4, 8):
                rb = run_gemv(L, s, ty, rows, K, mk, args.steps, args.warmup, 3, B=B)
                secondary[f"{name}_B{B}"] = {
                    "GB/s": round(rb["gbps"], 1), "us_per_call": round(rb["ms"] * 1e3, 2),
                    "frac_hbm_peak": round(rb["gbps"] / HBM_PEAK_GBPS, 4), "weight_bytes": rb["bytes"], "vectors": B}
                log(f"{name} B={B}: {rb['ms'] * 1e3:.2f} us")
        from glmssd import synth as S
        iq = lambda rng, rows, K: S.random_blocks(rng, G.GgmlType.IQ2_XXS, rows * K, 0.02, [0])
        # sustained rate: one vector through a matrix of 262144 x 4096 (0.3-0.9 GB, an LM-head-sized
        # GEMV), two rotated copies, where launch ramp and drain no longer dominate
        q80 = lambda rng, rows, K: S.random_blocks(rng, G.GgmlType.Q8_0, rows * K, 1 / 127, [0])
        for name, ty, mk in (("q4_k", G.GgmlType.Q4_K, S.q4_k_matrix), ("q8_0", G.GgmlType.Q8_0, q80),
                             ("q6_k", G.GgmlType.Q6_K, S.q6_k_matrix), ("iq2_xxs", G.GgmlType.IQ2_XXS, iq)):
            rb = run_gemv(L, s, ty, 262144, 4096, mk, max(10, args.steps // 20), max(3, args.warmup // 10), 5,
                          min_rot_bytes=1 << 30)
            secondary[f"sustained_gemv_{name}_262144x4096"] = {
                "GB/s": round(rb["gbps"], 1), "us_per_call": round(rb["ms"] * 1e3, 2),
                "frac_hbm_peak": round(rb["gbps"] / HBM_PEAK_GBPS, 4), "weight_bytes": rb["bytes"],
                "rotated_copies": rb["copies"]}
            log(f"sustained {name}: {rb['ms'] * 1e3:.1f} us, {rb['gbps']:.1f} GB/s")
        q6 = lambda rng, rows, K: S.q6_k_matrix(rng, rows, K)
        for name, ty, rows, K, N, mk, uw in [
                ("gemm_q4_k_k4096_rows12288_N512", G.GgmlType.Q4_K, 12288, 4096, 512, S.q4_k_matrix, True),
                ("gemm_q4_k_k4096_rows12288_N512_tiles", G.GgmlType.Q4_K, 12288, 4096, 512, S.q4_k_matrix, False),
                ("gemm_q4_k_k4096_rows12288_N192", G.GgmlType.Q4_K, 12288, 4096, 192, S.q4_k_matrix, True),
                ("gemm_q4_k_k4096_rows12288_N192_tiles", G.GgmlType.Q4_K, 12288, 4096, 192, S.q4_k_matrix, False),
                ("gemm_q6_k_k12288_rows4096_N512", G.GgmlType.Q6_K, 4096, 12288, 512, q6, True),
                ("gemm_q8_0_k4096_rows4096_N512", G.GgmlType.Q8_0, 4096, 4096, 512, S.q8_0_matrix, True),
                ("gemm_iq2_xxs_k4096_rows1536_N64", G.GgmlType.IQ2_XXS, 1536, 4096, 64, iq, True)]:
            r = run_gemm(L, s, ty, rows, K, N, mk, max(20, args.steps // 5), max(5, args.warmup // 5), 9, use_work=uw)
            r["path"] = ["f16 MFMA tiles", "f16 MFMA tiles (K split)", "f16 dequant + hipBLASLt"][
                G.ops.gemm_path(ty, K, rows, N, G.row_bytes(ty, K), rows, r["workspace_bytes"])]
            secondary[name] = r
            log(f"{name}: {r}")
        rc = run_read_ceiling(L, s, [17825792, 25952256, 28311552, 38928384, 41287680, 1 << 30], args.steps,
                              args.warmup, args.ramp_ms)
        secondary["plain_read_ceiling"] = rc
        log(f"plain-read ceiling: {rc}")
        for name, r in [("config1_q8_0_gemv_4096x4096", r1), ("config3_q4_k_gemv_k4096_rows12288", r3a),
                        ("config3_q6_k_gemv_k12288_rows4096", r3b)]:
            secondary[name] = {"GB/s": round(r["gbps"], 1), "us_per_call": round(r["ms"] * 1e3, 2),
                               "frac_hbm_peak": round(r["gbps"] / HBM_PEAK_GBPS, 4), "weight_bytes": r["bytes"],
                               "rotated_copies": r["copies"]}
            # against a plain read of the same byte count (launch, ramp-up and drain included in both)
            near = min(rc.values(), key=lambda v: abs(v["bytes"] - r["bytes"]))
            secondary[name]["frac_of_plain_read_at_same_bytes"] = round(r["gbps"] / near["GB/s"], 3)
            log(f"{name}: {r['ms'] * 1e3:.2f} us, {r['gbps']:.1f} GB/s")
    if args.calib:
        src, dst = G.DeviceBuffer(1 << 30), G.DeviceBuffer(1 << 30)
        ms = C.c_float()
        G.check(L.bn_copy(dst.p, src.p, 1 << 30, 5, s.raw(), C.byref(ms)))
        log(f"calib: 1 GiB d2d copy {ms.value:.3f} ms")

    cpu = None if args.no_cpu else cpu_baseline()
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_min_gpu_ms": args.ramp_ms,
        "ms_per_step": round(res["ms_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "dtype_detail": "IQ2_XXS weights x q8_1 activations: int8 dot4 products, f32 accumulation",
        "data": "synthetic (seeded random IQ2_XXS blocks, d~|N(0,0.02)|; x~N(0,1))",
        "config": {"workload": "config 2: routed-expert FFN, 1 decode token, 8 of 288 resident IQ2_XXS experts "
                               "(hidden 4096, intermediate 1536), gate/up+SwiGLU then down+weighted combine",
                   "weight_bytes_per_step": res["step_bytes"], "frac_hbm_peak": round(value / HBM_PEAK_GBPS, 4),
                   "frac_of_plain_read_at_same_bytes": (round(value / secondary["plain_read_ceiling"]["38928384"]["GB/s"], 3)
                                                        if "plain_read_ceiling" in secondary else None),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": "gs_moe_gateup (gs_k_stream_16_1_1_4_w)",
                     "achieved": round(gu_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gu_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic_bytes(GATEUP_KERNEL),
                     "traffic_source": "profiles/stream_kernels_traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE, "
                                       "calibrated on a 1 GiB device copy)",
                     "algorithmic_bytes_per_launch": res["gateup_bytes"],
                     "avg_launch_us": round(res["ms_gateup"] * 1e3, 3)},
        "cpu_baseline": cpu,
        "roofline_config5": config5_roofline(secondary.get("config5_prefill_512tok_grouped")),
        "secondary": secondary,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
