// gfx950 kernels of the quantized-matmul hot path. Compiled to one code object
// (hipcc --genco --offload-arch=gfx950) that host.cpp loads with hipModuleLoadData; every
// kernel is extern "C" with a fixed name and takes one argument block from kargs.h by value.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "kargs.h"
#include "formats.h"

// =============================================================================================
// q8_1 activation quantization of one 32-element unit, in registers.
//   d = amax/127 (correctly rounded), id = d ? 1/d : 0, q = roundf(x*id) (half away from zero),
//   stored scale D = f16(d) read back as f32; s = f16(d * sum q) for the ggml block layout.
// =============================================================================================
struct Q81 {
    uint32_t q[8];
    float d;       // unrounded f32 scale
    int slo, shi;
};

__device__ __forceinline__ Q81 quant_unit(const float (&v)[32]) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(v[i]));
    Q81 r;
    r.d = amax / 127.0f;
    const float id = r.d != 0.f ? 1.0f / r.d : 0.f;
    r.slo = r.shi = 0;
#pragma unroll
    for (int w = 0; w < 8; w++) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const float p = v[4 * w + b] * id;
            const int q = (int)__builtin_roundf(p);
            word |= ((uint32_t)q & 0xffu) << (8 * b);
            if (w < 4) r.slo += q; else r.shi += q;
        }
        r.q[w] = word;
    }
    return r;
}

__device__ __forceinline__ void load32(const float *src_, bool aligned, float (&v)[32]) {
    const GS_GLOBAL float *src = (const GS_GLOBAL float *)src_;
    if (aligned) {
        const GS_GLOBAL float4 *p = (const GS_GLOBAL float4 *)src;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 f = p[i];
            v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = src[i];
    }
}

// =============================================================================================
// Cross-lane sum over groups of 16/32/64 lanes with DPP; the group's last lane ends with the total.
// =============================================================================================
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_plus(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWMASK, 0xF, false));
}
__device__ __forceinline__ float group_sum(float v, int lpr) {
    v = dpp_plus<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v = dpp_plus<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v = dpp_plus<0x141, 0xF>(v);  // row_half_mirror
    v = dpp_plus<0x140, 0xF>(v);  // row_mirror: every lane of a 16-lane row holds the row sum
    if (lpr >= 32) v = dpp_plus<0x142, 0xA>(v);  // row_bcast:15 -> rows 1, 3
    if (lpr >= 64) v = dpp_plus<0x143, 0xC>(v);  // row_bcast:31 -> rows 2, 3
    return v;
}

__device__ __forceinline__ float swiglu(float g, float u, float lim) { // ops.cu:101-115
    if (lim > 0.f) {
        g = fminf(g, lim);
        u = fminf(fmaxf(u, -lim), lim);
    }
    return g / (1.f + expf(-g)) * u;
}

// =============================================================================================
// Streaming matrix-vector kernel (GEMV / fused MoE gate-up / fused MoE down).
//
// Lanes form groups of `lpr` (16, 32 or 64) lanes; a group computes one output row at a time and
// every lane owns the same `upl` 32-element units of every row it visits, so the lane's q8_1
// activation units are quantized once (workgroup prologue, through LDS) and then stay in VGPRs.
// Weight bytes go straight from HBM to VGPRs with unaligned 8/16-byte loads; rows are software-
// pipelined PF deep (the loads of row i+PF are issued before row i is decoded). Row partials are
// summed across the group with DPP. A "row" spans several matrices for the fused MoE kernels:
//   kind 0 GEMV:    units of one matrix row
//   kind 1 GATEUP:  units of gate_e[r] then up_e[r] (two sums, SwiGLU epilogue)
//   kind 2 DOWN:    units of down_e[r] for every expert e of the batch (one weighted sum)
// =============================================================================================
// Rows in flight per lane group: as many as ~64 VGPRs of raw weight bytes hold (at most 8), so a
// group's whole share of a decode-sized matrix is requested before the first row is decoded.
#ifndef GS_PF_REGS
#define GS_PF_REGS 48
#endif
template <class F, int UMAX>
__device__ __forceinline__ constexpr int pf_depth() {
    constexpr int n = GS_PF_REGS / (F::RAW * UMAX);
    return n < 1 ? 1 : (n > 8 ? 8 : n);
}

// Load activation unit (vector v, unit up) from the LDS q8_1 staging area; `scale` multiplies D
// (routing weight and the format's constant factor); a zero scale or padding unit yields zeros.
template <class F, bool XNEG>
__device__ __forceinline__ XU load_xu(const uint8_t *xq, const uint32_t *xm, int K, int nu, int v, int up, float scale,
                                      bool valid) {
    XU z;
    const bool live = valid && scale != 0.f;
    const int mi = v * nu + up;
    const uint4 *src = (const uint4 *)(xq + (size_t)v * K + 32 * (live ? up : 0));
    const uint4 lo = src[0], hi = src[1];
    const uint32_t dbits = xm[live ? 2 * mi : 0], ss = xm[live ? 2 * mi + 1 : 1];
    z.q[0] = live ? lo.x : 0u; z.q[1] = live ? lo.y : 0u; z.q[2] = live ? lo.z : 0u; z.q[3] = live ? lo.w : 0u;
    z.q[4] = live ? hi.x : 0u; z.q[5] = live ? hi.y : 0u; z.q[6] = live ? hi.z : 0u; z.q[7] = live ? hi.w : 0u;
    z.D = live ? __builtin_bit_cast(float, dbits) * scale * XScale<F>::value : 0.f;
    z.slo = live ? (int)(int16_t)(ss & 0xffff) : 0;
    z.shi = live ? (int)(int16_t)(ss >> 16) : 0;
    if (XNEG) {
#pragma unroll
        for (int i = 0; i < 8; i++) {   // bytewise -q (|q| <= 127, no overflow)
            uint32_t n = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) n |= ((uint32_t)(-(int)(int8_t)(z.q[i] >> (8 * b))) & 0xffu) << (8 * b);
            z.nq[i] = n;
        }
    }
    return z;
}

// UMAX = weight units per lane per row. GEMV / DOWN: units j of the (concatenated) row.
// GATEUP: j < UMAX/2 are units of the gate row, j >= UMAX/2 the same units of the up row, so
// the lane holds UMAX/2 activation units.
//
// Rows are processed in batches of PF rows per lane group: every load of a batch is issued
// unconditionally (rows past the end are clamped to a valid row and their results dropped), so
// the waits before each row are exact in-order counts and decoding row 0 overlaps the arrival of
// rows 1..PF-1. Results are stored after the batch.
#ifdef GS_STREAM_TS
// profiling build only: per-wave phase timestamps (100 MHz s_memrealtime)
__device__ unsigned long long gs_stream_ts[1 << 16];
#define GS_TS(i, extra)                                                                          \
    if ((threadIdx.x & 63) == 0)                                                                \
        gs_stream_ts[((size_t)blockIdx.x * (GS_WG / 64) + (threadIdx.x >> 6)) * 8 + (i)] =       \
            __builtin_amdgcn_s_memrealtime() + (extra);
#else
#define GS_TS(i, extra)
#endif

template <class F, int KIND, int NV, int UMAX>
__device__ __forceinline__ void stream_body(const StreamArgs &a) {
    constexpr int PF = pf_depth<F, UMAX>();
    constexpr int UX = KIND == 1 ? UMAX / 2 : UMAX;       // activation units per lane
    constexpr bool XNEG = NegX<F>::value && UX * NV <= 4;  // -q in registers only while it is cheap
    static_assert(KIND != 1 || UMAX % 2 == 0, "gate/up needs an even unit count");
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x;
    GS_TS(0, 0)
    uint8_t *tab = smem;
    uint8_t *xq = smem + ((F::TAB + 15) & ~15);

    const uint8_t *wb = a.w0[0];
    const float *x = a.x;
    float *y = a.y;
    if (KIND == 0) {
        wb += (int64_t)blockIdx.y * a.w_bs;
        x += (int64_t)blockIdx.y * a.x_bs;
        y += (int64_t)blockIdx.y * a.y_bs;
    }
    const int K = a.K, nu = a.nu, nv = a.nvec, rows = a.rows;
    const int lpr = a.lpr, lane = tid & (lpr - 1);
    const int tot = KIND == 2 ? a.nseg * nu : nu;          // units along the (concatenated) row
    // Lane groups: GATEUP pins each wave to one expert (its pointers are wave-uniform) and the
    // wave's groups stride over that expert's rows; other kinds stride over all rows.
    const int gpw = 64 / lpr;                                   // groups per wave
    const int wave_all = blockIdx.x * (GS_WG / 64) + (tid >> 6);
    const int nwaves_all = gridDim.x * (GS_WG / 64);
    const int gin = (tid & 63) / lpr;                           // group within the wave
    int ge = 0, ngroups, gid, nrow;
    if (KIND == 1) {
        ge = __builtin_amdgcn_readfirstlane(wave_all % a.nseg);
        const int wpe = nwaves_all / a.nseg;                    // waves per expert
        ngroups = wpe * gpw;
        gid = (wave_all / a.nseg) * gpw + gin;
        nrow = wave_all >= wpe * a.nseg ? 0 : rows;             // leftover waves idle
    } else {
        ngroups = nwaves_all * gpw;
        gid = wave_all * gpw + gin;
        nrow = rows;
    }
    const int64_t rs = a.row_stride;
    // expert pointer tables: one vector load (lane i <- entry i), then readlane / bpermute, so no
    // weight address waits on a second, dependent kernel-argument fetch
    const int L64 = tid & 63;
    const uint64_t tw0 = KIND != 0 && L64 < GS_SEG_MAX ? (uint64_t)a.w0[L64] : 0;
    const uint64_t tw1 = KIND == 1 && L64 < GS_SEG_MAX ? (uint64_t)a.w1[L64] : 0;
    auto lane_u64 = [](uint64_t v, int src) -> uint64_t {   // v of lane `src` (per-lane src)
        const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)(uint32_t)v);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)(uint32_t)(v >> 32));
        return (uint64_t)lo | ((uint64_t)hi << 32);
    };
    const uint8_t *wg = nullptr, *wu = nullptr;
    if (KIND == 1) {
        wg = (const uint8_t *)(((uint64_t)__builtin_amdgcn_readlane((int)(uint32_t)(tw0 >> 32), ge) << 32) |
                               (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)tw0, ge));
        wu = (const uint8_t *)(((uint64_t)__builtin_amdgcn_readlane((int)(uint32_t)(tw1 >> 32), ge) << 32) |
                               (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)tw1, ge));
    }

    // per-unit geometry; padding units re-read the lane's first unit (their activation is 0)
    int uspan[UX], usub[UX];
    uint32_t uoff[UX];
    bool uval[UX];
#pragma unroll
    for (int j = 0; j < UX; j++) {
        const int u0 = lane + lpr * j;
        const bool valid = j < a.upl && u0 < tot;
        const int u = valid ? u0 : (lane < tot ? lane : 0);
        const int s = KIND == 2 ? u / nu : 0;
        const int up = u - s * nu;
        uval[j] = valid;
        uspan[j] = s;
        uoff[j] = F::off(up);
        usub[j] = F::sub(up);
    }
    const uint8_t *ubase[UX];
#pragma unroll
    for (int j = 0; j < UX; j++)
        ubase[j] = (KIND == 2 ? (const uint8_t *)lane_u64(tw0, uspan[j]) : (KIND == 1 ? nullptr : wb)) + uoff[j];

    // ---- prologue loads first: activation units and lookup tables are requested before the
    // weight loads, so waiting for them (vmcnt counts in issue order) never waits on weights
    constexpr int XQ = 2;                                       // activation units per thread in flight
    const int nxv = KIND == 2 ? a.nseg * nv : nv;
    const int nxu = nxv * nu;
    float xf[XQ][32];
#pragma unroll
    for (int k = 0; k < XQ; k++) {
        const int i = min(tid + GS_WG * k, nxu - 1);            // clamped: the loads are unconditional
        const int v = i / nu, u = i - v * nu;
        const float *src = (KIND == 2 ? x + (int64_t)v * K : x + (int64_t)v * a.x_stride) + 32 * u;
        load32(src, a.x_aligned != 0, xf[k]);
    }
    typename F::TabReg treg;
    F::tab_load(tid, treg);

    // ---- weight batches ------------------------------------------------------------------------
    typename F::Raw R[PF][UMAX];
    const int last = nrow > 0 ? nrow - 1 : 0;
    auto load_batch = [&](int base) {
#pragma unroll
        for (int p = 0; p < PF; p++) {
            const int r = min(base + p * ngroups, last);
            const int64_t roff = (int64_t)r * rs;
            if (KIND == 1) {
#pragma unroll
                for (int j = 0; j < UX; j++) {
                    F::load(wg + roff + uoff[j], usub[j], R[p][j]);
                    F::load(wu + roff + uoff[j], usub[j], R[p][UX + j]);
                }
            } else {
#pragma unroll
                for (int j = 0; j < UX; j++) F::load(ubase[j] + roff, usub[j], R[p][j]);
            }
        }
    };
    GS_TS(1, 0)
    load_batch(gid);
    GS_TS(2, 0)

    // ---- prologue compute: tables + q8_1 quantization of every activation vector into LDS ----
    F::tab_store(tid, treg);
    uint32_t *xm = (uint32_t *)(xq + (size_t)nxv * K);
    auto quant_store = [&](int i, const float (&f)[32]) {
        const int v = i / nu, u = i - v * nu;
        const Q81 q = quant_unit(f);
        uint4 *dst = (uint4 *)(xq + (size_t)v * K + 32 * u);
        dst[0] = make_uint4(q.q[0], q.q[1], q.q[2], q.q[3]);
        dst[1] = make_uint4(q.q[4], q.q[5], q.q[6], q.q[7]);
        xm[2 * i] = __builtin_bit_cast(uint32_t, h2f(f2h(q.d)));
        xm[2 * i + 1] = ((uint32_t)q.slo & 0xffffu) | ((uint32_t)q.shi << 16);
    };
#pragma unroll
    for (int k = 0; k < XQ; k++)
        if (tid + GS_WG * k < nxu) quant_store(tid + GS_WG * k, xf[k]);
    for (int i = tid + GS_WG * XQ; i < nxu; i += GS_WG) {   // large activation sets: the rest
        const int v = i / nu, u = i - v * nu;
        float f[32];
        load32((KIND == 2 ? x + (int64_t)v * K : x + (int64_t)v * a.x_stride) + 32 * u, a.x_aligned != 0, f);
        quant_store(i, f);
    }
    __syncthreads();
    GS_TS(3, 0)
    XU xr[UX][NV];
#pragma unroll
    for (int j = 0; j < UX; j++) {
        const int up = lane + lpr * j - uspan[j] * nu;
#pragma unroll
        for (int t = 0; t < NV; t++) {
            const int v = KIND == 2 ? uspan[j] * nv + t : t;
            const float w = KIND == 2 ? a.wt[t][uspan[j]] : 1.f;   // routing weight folded into D
            xr[j][t] = load_xu<F, XNEG>(xq, xm, K, nu, v, up, w, uval[j] && t < nv);
        }
    }

    // ---- batches of PF rows per group ----------------------------------------------------------
    for (int base = gid; base < nrow; base += PF * ngroups) {
        if (base != gid) load_batch(base);
        float res0[PF][NV], res1[PF][NV];
#pragma unroll
        for (int p = 0; p < PF; p++) {
            float acc0[NV], acc1[NV];
#pragma unroll
            for (int t = 0; t < NV; t++) acc0[t] = acc1[t] = 0.f;
#ifdef GS_STREAM_TS
            if (base == gid && p == 0) {
                uint32_t h = 0;
#pragma unroll
                for (int j = 0; j < UMAX; j++) h ^= ((const uint32_t *)&R[0][j])[0];
                GS_TS(4, h == 0x9e3779b9u)
            }
#endif
            if (base + p * ngroups < nrow) {   // no loads inside: the waits stay exact
#pragma unroll
                for (int j = 0; j < UX; j++) {
                    F::template dot<NV, XNEG>(R[p][j], usub[j], tab, xr[j], nv, acc0);
                    if (KIND == 1) F::template dot<NV, XNEG>(R[p][UX + j], usub[j], tab, xr[j], nv, acc1);
                }
            }
#pragma unroll
            for (int t = 0; t < NV; t++) {
                res0[p][t] = group_sum(acc0[t], lpr);
                if (KIND == 1) res1[p][t] = group_sum(acc1[t], lpr);
            }
        }
        if (lane == lpr - 1) {
#pragma unroll
            for (int p = 0; p < PF; p++) {
                const int rr = base + p * ngroups;
                if (rr < nrow) {
#pragma unroll
                    for (int t = 0; t < NV; t++) {
                        if (t < nv) {
                            if (KIND == 0) {
                                float *dst = y + (int64_t)t * a.y_stride + rr;
                                *dst = a.accumulate ? *dst + res0[p][t] : res0[p][t];
                            } else if (KIND == 1) {
                                y[((int64_t)ge * nv + t) * rows + rr] = swiglu(res0[p][t], res1[p][t], a.lim);
                            } else {
                                y[(int64_t)t * a.y_stride + rr] += res0[p][t];
                            }
                        }
                    }
                }
            }
        }
    }
    GS_TS(5, 0)
}

// waves per SIMD the streaming kernels are register-allocated for (HBM latency hiding)
#ifndef GS_WPE
#define GS_WPE 1
#endif
#define GS_STREAM_KERNEL(F, NAME, KIND, NV, UM)                                                  \
    extern "C" __global__ void __launch_bounds__(GS_WG) __attribute__((amdgpu_waves_per_eu(GS_WPE))) \
        gs_k_stream_##NAME##_##KIND##_##NV##_##UM(StreamArgs a) {                                \
        stream_body<F, KIND, NV, UM>(a);                                                        \
    }
// instantiated (activation vectors, weight units per lane) pairs; host.cpp keeps the same table
#define GS_STREAM_MV(F, NAME, KIND)                                                             \
    GS_STREAM_KERNEL(F, NAME, KIND, 1, 2) GS_STREAM_KERNEL(F, NAME, KIND, 1, 4)                 \
    GS_STREAM_KERNEL(F, NAME, KIND, 1, 6) GS_STREAM_KERNEL(F, NAME, KIND, 1, 8)                 \
    GS_STREAM_KERNEL(F, NAME, KIND, 2, 2)                                                       \
    GS_STREAM_KERNEL(F, NAME, KIND, 2, 4) GS_STREAM_KERNEL(F, NAME, KIND, 4, 1)                 \
    GS_STREAM_KERNEL(F, NAME, KIND, 4, 2) GS_STREAM_KERNEL(F, NAME, KIND, 8, 1)
#define GS_STREAM_GU(F, NAME)                                                                   \
    GS_STREAM_KERNEL(F, NAME, 1, 1, 2) GS_STREAM_KERNEL(F, NAME, 1, 1, 4)                       \
    GS_STREAM_KERNEL(F, NAME, 1, 1, 8) GS_STREAM_KERNEL(F, NAME, 1, 2, 2)                       \
    GS_STREAM_KERNEL(F, NAME, 1, 2, 4) GS_STREAM_KERNEL(F, NAME, 1, 4, 2)                       \
    GS_STREAM_KERNEL(F, NAME, 1, 4, 4) GS_STREAM_KERNEL(F, NAME, 1, 8, 2)
#define GS_STREAM_ALL(F, NAME) GS_STREAM_MV(F, NAME, 0) GS_STREAM_GU(F, NAME) GS_STREAM_MV(F, NAME, 2)

// One code object per format keeps the build parallel: the Makefile compiles this file once
// per GS_STREAM_TYPE (F-struct, type id) and once with GS_COMMON for the kernels below.
#if defined(GS_STREAM_F)
GS_STREAM_ALL(GS_STREAM_F, GS_STREAM_ID)
#endif

#if defined(GS_COMMON)

// =============================================================================================
// Whole-tensor dequantization (gs_dequant_f32 / gs_dequant_f16): one thread per 8 elements.
// =============================================================================================
#define GS_DEQ_KERNEL(TY, QK, BB, DEQ)                                                           \
    extern "C" __global__ void __launch_bounds__(256) gs_k_dequant_f32_##TY(DequantArgs a) {    \
        const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;                        \
        if (g >= a.n_groups) return;                                                            \
        constexpr int GPB = QK / 8;                                                             \
        float v[8];                                                                             \
        DEQ(a.src + (g / GPB) * BB, (int)(g % GPB), v);                                         \
        float4 *d = (float4 *)((float *)a.dst + g * 8);                                         \
        d[0] = make_float4(v[0], v[1], v[2], v[3]);                                             \
        d[1] = make_float4(v[4], v[5], v[6], v[7]);                                             \
    }                                                                                           \
    extern "C" __global__ void __launch_bounds__(256) gs_k_dequant_f16_##TY(DequantArgs a) {    \
        const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;                        \
        if (g >= a.n_groups) return;                                                            \
        constexpr int GPB = QK / 8;                                                             \
        float v[8];                                                                             \
        DEQ(a.src + (g / GPB) * BB, (int)(g % GPB), v);                                         \
        /* opaque to the optimizer: keeps the f32 value (and the sign of a zero) intact before  \
           the single f32 -> f16 rounding */                                                   \
        for (int i = 0; i < 8; i++) asm volatile("" : "+v"(v[i]));                              \
        uint4 o;                                                                                \
        o.x = f2h(v[0]) | (f2h(v[1]) << 16);                                                    \
        o.y = f2h(v[2]) | (f2h(v[3]) << 16);                                                    \
        o.z = f2h(v[4]) | (f2h(v[5]) << 16);                                                    \
        o.w = f2h(v[6]) | (f2h(v[7]) << 16);                                                    \
        *(uint4 *)((uint16_t *)a.dst + g * 8) = o;                                              \
    }
GS_TYPE_LIST(GS_DEQ_KERNEL)

// =============================================================================================
// q8_1 quantization to the ggml block layout {f16 d; f16 s; int8 qs[32]} (gs_quant_q8_1)
// =============================================================================================
extern "C" __global__ void __launch_bounds__(256) gs_k_quant_q8_1(QuantArgs a) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= a.n_blocks) return;
    float v[32];
    load32(a.x + 32 * b, false, v);
    const Q81 q = quant_unit(v);
    uint8_t *o = a.out + 36 * b;
    const uint32_t hd = f2h(q.d), hs = f2h((float)(q.slo + q.shi) * q.d);
    uint32_t *ow = (uint32_t *)o;   // 36-byte blocks are 4-byte aligned
    ow[0] = hd | (hs << 16);
#pragma unroll
    for (int i = 0; i < 8; i++) ow[1 + i] = q.q[i];
}

// =============================================================================================
// Element-wise and row kernels of the MoE glue (ops.cu:101-125, gemm.cu:125-163)
// =============================================================================================
extern "C" __global__ void __launch_bounds__(256) gs_k_swiglu(EltArgs a) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.n) a.y[i] = swiglu(a.a[i], a.b[i], a.s);
}
extern "C" __global__ void __launch_bounds__(256) gs_k_axpy(EltArgs a) {   // y += s * x
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.n) a.y[i] += a.s * a.a[i];
}
extern "C" __global__ void __launch_bounds__(256) gs_k_f32_to_f16(EltArgs a) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.n) ((uint16_t *)a.y)[i] = (uint16_t)f2h(a.a[i]);
}
extern "C" __global__ void __launch_bounds__(256) gs_k_saxpy(EltArgs a) {  // y = s*x + y
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.n) a.y[i] = a.s * a.a[i] + a.y[i];
}
// y[i][:] = x[idx[i]][:]
extern "C" __global__ void __launch_bounds__(256) gs_k_gather_rows(RowsArgs a) {
    const int i = blockIdx.y;
    const float *src = a.x + (int64_t)a.idx[i] * a.n;
    float *dst = a.y + (int64_t)i * a.n;
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < a.n; c += gridDim.x * blockDim.x) dst[c] = src[c];
}
// acc[idx[i]][:] += w[i] * y[i][:]  (idx unique within one call); acc passed as .y, rows as .x
extern "C" __global__ void __launch_bounds__(256) gs_k_scatter_add_rows(RowsArgs a) {
    const int i = blockIdx.y;
    float *dst = a.y + (int64_t)a.idx[i] * a.n;
    const float *src = a.x + (int64_t)i * a.n;
    const float s = a.w[i];
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < a.n; c += gridDim.x * blockDim.x) dst[c] += s * src[c];
}
#endif  // GS_COMMON
