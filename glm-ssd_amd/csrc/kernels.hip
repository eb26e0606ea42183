// gfx950 kernels of the quantized-matmul hot path. Compiled (hipcc --genco --offload-arch=gfx950)
// into one code object per weight format (GS_STREAM_F / GS_STREAM_ID select that format's
// streaming kernels) and one with the format-independent kernels (GS_COMMON: quantization,
// dequantization, gather/scatter, SwiGLU, axpy, f16 conversion); host.cpp loads them all with
// hipModuleLoadData. Every kernel is extern "C" with a fixed name and takes one argument block
// from kargs.h by value.
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
    // 1/d overflows for d < 2^-128 (a block of tiny subnormals): q = 0 (its f16 d is 0 anyway)
    float id = r.d != 0.f ? 1.0f / r.d : 0.f;
    id = id <= 3.40282347e38f ? id : 0.f;
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

__device__ __forceinline__ void load8(const float *src_, bool aligned, float (&v)[8]) {
    const GS_GLOBAL float *src = (const GS_GLOBAL float *)src_;
    if (aligned) {
        const GS_GLOBAL float4 *p = (const GS_GLOBAL float4 *)src;
        const float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = src[i];
    }
}

// value of another lane of the same quad (DPP quad_perm CTRL)
template <int CTRL>
__device__ __forceinline__ float quad_swap(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// q8_1 quantizer arithmetic in fewer operations, bit-identical to the IEEE forms (checked for
// every input of the ranges below by tests/arith/q8_arith_check.c):
//   amax / 127: product with RN(1/127) and one fma correction of its residual (Markstein), for
//     finite amax >= 2^-118 (a normal quotient); other values take the IEEE division;
//   roundf(v) (half away from zero) as a truncating conversion of v + copysign(0.49999997, v),
//     for |v| <= 2^23 (the quantizer's |v| <= 127.x).
__device__ __forceinline__ float q8_div127(float amax) {
    if (__builtin_expect(!(amax >= 0x1p-118f && amax <= 0x1.fffffep127f), 0)) return amax / 127.0f;
    const float c = 1.0f / 127.0f;
    const float q = amax * c;
    return __builtin_fmaf(__builtin_fmaf(-q, 127.0f, amax), c, q);
}
// roundf(x * id) with the product rounded first (no fma contraction, as the check assumes)
__device__ __forceinline__ int q8_round_mul(float x, float id) {
#pragma clang fp contract(off)
    const float v = x * id;
    return (int)(v + __builtin_copysignf(0.49999997f, v));
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
// The same with the hardware exp2 and reciprocal (about 1 ulp each instead of the correctly
// rounded library sequences): the fused gate/up epilogue, where h then goes through q8_1.
__device__ __forceinline__ float swiglu_fast(float g, float u, float lim) {
    if (lim > 0.f) {
        g = fminf(g, lim);
        u = fminf(fmaxf(u, -lim), lim);
    }
    return g * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f)) * u;
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
// Rows in flight per lane group: as many as GS_PF_REGS VGPRs of raw weight bytes hold (1..8).
// Gate/up rows carry twice the units (gate and up), so their budget is smaller: 3 ring slots
// (config 2 gate/up: 9.9 -> 9.4 us against 2; 4 were slower), while the down and GEMV passes
// keep deeper batches. The MoE ring kernels request only their first slot before the activation
// staging and the others right after it: a smaller first request arrives sooner (config 2 down
// 9.35 -> 9.0 us; all slots at once, the first batch grows and comes later). The GEMVs request
// all at once (Q4_K's three batches per wave: 8.8 us against 8.97 with the split).
#ifndef GS_PF_REGS
#define GS_PF_REGS 48
#endif
#ifndef GS_PF_REGS_GU
#define GS_PF_REGS_GU 36
#endif
// ring slots requested before the activation staging (the others right after it)
#ifndef GS_RING_EARLY
#define GS_RING_EARLY 1
#endif
// Formats whose paired units share their bytes (JOINT: load2 fills the pair's registers once,
// dot_pair decodes both, RAW2 registers per unit; their unit numbering within a block is a
// permutation, so the activation unit of weight unit up is F::xunit(up)).
template <class F, class = void> struct Joint { static constexpr bool value = false; static constexpr int raw2 = F::RAW; };
template <class F> struct Joint<F, decltype((void)F::JOINT, void())> {
    static constexpr bool value = F::JOINT;
    static constexpr int raw2 = F::RAW2;
};
template <class F, class = void> struct Paired { static constexpr bool value = false; };
template <class F> struct Paired<F, decltype((void)F::PAIR, void())> { static constexpr bool value = F::PAIR; };
template <class F, int UMAX, int KIND = 0>
__device__ __forceinline__ constexpr int pf_depth() {
    constexpr int ux = KIND == 1 ? UMAX / 2 : UMAX;
    constexpr bool joint = Joint<F>::value && Paired<F>::value && ux % 2 == 0;
    constexpr int n = (KIND == 1 ? GS_PF_REGS_GU : GS_PF_REGS) / ((joint ? Joint<F>::raw2 : F::RAW) * UMAX);
    // joint formats keep two rows in flight however many units a lane holds: a wave's second row
    // then streams while the first is decoded (Q6_K K = 12288: 6 units per lane)
    constexpr int lo = joint ? 2 : 1;
    return n < lo ? lo : (n > 8 ? 8 : n);
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
    if (F32Act<F>::value) {   // f32 activations: staged as floats, read by the unit's dot
        z.xs = (const float *)xq + (size_t)v * K + 32 * (live ? up : 0);
        z.D = live ? scale : 0.f;
    }
    z.slo = live ? (int)(int16_t)(ss & 0xffff) : 0;
    z.shi = live ? (int)(int16_t)(ss >> 16) : 0;
    if (XNEG) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            // bytewise -q in four operations: per byte, 0x80 - (q & 0x7f) is ~q's low seven bits
            // plus one (no borrow leaves the byte), and the sign bit is then flipped unless q's
            // was set. |q| <= 127, so -q never overflows.
            const uint32_t q = z.q[i];
            z.nq[i] = (0x80808080u - (q & 0x7f7f7f7fu)) ^ (q & 0x80808080u) ^ 0x80808080u;
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

// Unit decode in two phases where the format has them (LDS table reads, then arithmetic), so
// the row loop can issue unit i+1's reads before unit i's arithmetic; one phase otherwise.
template <class F, class = void>
struct TwoPhase {
    struct Dec {};
    __device__ static __forceinline__ void fetch(const typename F::Raw &, Dec &) {}
    template <int NV, bool XNEG>
    __device__ static __forceinline__ void dot(const typename F::Raw &w, const Dec &, int j, const uint8_t *tab,
                                               const XU (&x)[NV], int nv, float (&r)[NV]) {
        F::template dot<NV, XNEG>(w, j, tab, x, nv, r);
    }
};
template <class F>
struct TwoPhase<F, decltype((void)sizeof(typename F::Dec), void())> {
    using Dec = typename F::Dec;
    __device__ static __forceinline__ void fetch(const typename F::Raw &w, Dec &e) { F::fetch(w, e); }
    template <int NV, bool XNEG>
    __device__ static __forceinline__ void dot(const typename F::Raw &w, const Dec &e, int, const uint8_t *,
                                               const XU (&x)[NV], int nv, float (&r)[NV]) {
        F::template dot2<NV, XNEG>(w, e, x, nv, r);
    }
};

// h (gate/up output) stores at device scope: written through past this XCD's L2, so the down
// launch that follows (on every XCD) finds h without this launch's end-of-kernel L2 write-back
// in its way (config 2: ~0.2 us per step against plain stores).
__device__ __forceinline__ void store_h(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Exact u / d for 0 <= u < 2^21 through the rounded reciprocal rd = 1/d (two VALU operations
// instead of a ~20-instruction integer division): (u + 0.5) / d lies at least 0.5/d from an
// integer, and the two roundings move it by at most 3 * 2^-24 * (u + 0.5) / d, less than that.
__device__ __forceinline__ int udiv_small(int u, float rd) { return (int)(((float)u + 0.5f) * rd); }

// Formats that load two consecutive units of a block with one wide access (load2): d once and
// one 16-byte read for both units' indices, half the vector-memory instructions of two loads
// (Paired, declared with pf_depth above).


template <bool B> struct BoolC { static constexpr bool value = B; };

// LP: 0 = lane-group width from the arguments; 64 = fixed 64 (whole rows per wave, so the row
// index and every row address are wave-uniform scalars)
template <class F, int KIND, int NV, int UMAX, int LP = 0>
struct StreamPass {
    static constexpr int PF = pf_depth<F, UMAX, KIND>();
    // (one slot gains nothing from the ring: measured slower on Q6_K's two rows per wave)
    static constexpr bool RING = LP == 64 && PF >= 2;
    static constexpr int UX = KIND == 1 ? UMAX / 2 : UMAX;       // activation units per lane
    // -q in registers only while it is cheap (down's 6 units per lane measured no faster with it)
    static constexpr bool XNEG = NegX<F>::value && UX * NV <= 4;
    // activation prologue: 4 threads per 32-element unit (8 floats each), XP passes of GS_WG/4
    // units in flight before the weight loads (a decode-sized x is one pass: 2 loads per thread)
    static constexpr int XT = 4, XPU = GS_WG / XT;
    // (down: a row's units, at most 64 * UX for the whole activation set, need UX / 2 passes; a
    // GEMV's NV vectors of up to 64 * UX units each, NV * UX / 2: passes loaded inside the staging
    // would queue behind the weight loads and wait for them, as vector loads return in order)
    static constexpr int XPG = (NV * UX + 1) / 2;
    static constexpr int XP = KIND == 2 ? (UX / 2 < 1 ? 1 : (UX / 2 > 4 ? 4 : UX / 2))
                                        : KIND == 0 ? (XPG < NV ? NV : (XPG > 4 ? 4 : XPG)) : (NV < 4 ? NV : 4);
    // paired units: the lane's units j, j+1 (j even) are consecutive units of one block
    static constexpr bool PAIRS = Paired<F>::value && UX % 2 == 0;
    static constexpr bool JOINT = Joint<F>::value && PAIRS;
    __device__ __forceinline__ int unit_of(int j) const {
        return PAIRS ? 2 * (lane + lpr * (j >> 1)) + (j & 1) : lane + lpr * j;
    }
    static_assert(KIND != 1 || UMAX % 2 == 0, "gate/up needs an even unit count");

    const StreamArgs &a;
    int tid;
    uint8_t *tab, *xq;
    const float *x;
    float *y;
    int K, nu, nv, rows, lpr, lane, tot, ngroups, gid, nrow, ge, nxv, nxu;
    int sy;   // GATEUP/DOWN: first pointer-table entry of this blockIdx.y slice (one token each)
    float rnu;   // 1/nu
    int64_t rs;
    const uint8_t *wg, *wu, *wb0;   // GATEUP gate / up, GEMV matrix (wave-uniform)
    uint64_t tw0, tw1;              // expert pointer tables (lane i: expert i), until bind()
    int uspan[UX], usub[UX];
    uint32_t uoff[UX];
    bool uval[UX];
    const uint8_t *ubase[UX];
    float xf[XP][8];
    typename F::TabReg treg;
    typename F::Raw R[PF][UMAX];
    float wtl[NV];   // DOWN: lane i holds vector t's combine weight for expert i

    // geometry of this pass; issues no memory access except the pointer-table load (DOWN/GATEUP)
    __device__ __forceinline__ StreamPass(const StreamArgs &a_, uint8_t *smem) : a(a_) {
        tid = threadIdx.x;
        tab = smem;
        xq = smem + ((F::TAB + 15) & ~15);
        const uint8_t *wb = a.w0[0];
        x = a.x;
        y = a.y;
        // blockIdx.y slices: GEMV batches (own matrix); GATEUP/DOWN tokens, slice y owning table
        // entries [y * nseg, (y + 1) * nseg) and its own activations and outputs
        if (KIND == 0) wb += (int64_t)blockIdx.y * a.w_bs;
        x += (int64_t)blockIdx.y * a.x_bs;
        y += (int64_t)blockIdx.y * a.y_bs;
        sy = KIND != 0 ? (int)blockIdx.y * a.nseg : 0;
        K = a.K, nu = a.nu, nv = a.nvec, rows = a.rows;
        if (KIND == 0 && a.nv_tail && blockIdx.y == gridDim.y - 1) nv = a.nv_tail;
        lpr = LP ? LP : a.lpr, lane = tid & (lpr - 1);
        tot = KIND == 2 ? a.nseg * nu : nu;          // units along the (concatenated) row
        // Lane groups: GATEUP pins each wave to one expert (its pointers are wave-uniform) and the
        // wave's groups stride over that expert's rows; other kinds stride over all rows.
        const int lsh = __builtin_ctz(lpr);                         // lpr is a power of two
        const int gpw = 64 >> lsh;                                  // groups per wave
        // wave-uniform (SGPR) wave index: the expert/row split below stays on the scalar unit
        const int wave_all = blockIdx.x * (GS_WG / 64) + __builtin_amdgcn_readfirstlane(tid >> 6);
        const int nwaves_all = gridDim.x * (GS_WG / 64);
        const int gin = (tid & 63) >> lsh;                          // group within the wave
        rnu = 1.0f / (float)nu;
        ge = 0;
        if (KIND == 1) {
            // each expert owns a block of consecutive waves, so its adjacent rows (which share a
            // 128-byte line when rows are not line multiples) go to waves of one workgroup and
            // one XCD's L2 rather than to two XCDs that would both fetch the shared line
            const int wpe = nwaves_all / a.nseg;                    // waves per expert
            const int wq = wave_all / wpe;
            ge = __builtin_amdgcn_readfirstlane(wq < a.nseg ? wq : a.nseg - 1);
            ngroups = wpe * gpw;
            gid = (wave_all - wq * wpe) * gpw + gin;
            nrow = wq >= a.nseg ? 0 : rows;                         // leftover waves idle
        } else {
            ngroups = nwaves_all * gpw;
            gid = wave_all * gpw + gin;
            nrow = rows;
        }
        rs = a.row_stride;
        // expert pointer tables: one vector load (lane i <- entry i), then readlane / bpermute, so no
        // weight address waits on a second, dependent kernel-argument fetch
        const int L64 = tid & 63;
        tw0 = KIND != 0 && L64 < GS_SEG_MAX ? (uint64_t)a.w0[L64] : 0;
        tw1 = KIND == 1 && L64 < GS_SEG_MAX ? (uint64_t)a.w1[L64] : 0;
        // combine weights likewise (lane i <- expert i), requested before the weight loads so the
        // activation setup does not wait for them
#pragma unroll
        for (int t = 0; t < NV; t++) wtl[t] = KIND == 2 && L64 < GS_SEG_MAX && t < nv ? a.wt[t][L64] : 0.f;
        wg = wu = nullptr;
        wb0 = wb;
        // per-unit geometry; padding units re-read the lane's first unit (their activation is 0)
#pragma unroll
        for (int j = 0; j < UX; j++) {
            const int u0 = unit_of(j);
            const bool valid = (PAIRS || j < a.upl) && u0 < tot;
            const int u = valid ? u0 : (unit_of(0) < tot ? unit_of(0) : 0);
            const int s = KIND == 2 ? udiv_small(u, rnu) : 0;
            const int up = u - s * nu;
            uval[j] = valid;
            uspan[j] = s;
            uoff[j] = F::off(up);
            usub[j] = F::sub(up);
        }
#pragma unroll
        for (int j = 0; j < UX; j++) ubase[j] = KIND == 0 ? wb : nullptr;
        nxv = KIND == 2 ? a.nseg * nv : nv;
        nxu = nxv * nu;
    }

    // Expert addresses from the pointer tables the constructor requested. Called after issue_x
    // and issue_tab: waiting for the tables (in issue order) then leaves the activation loads in
    // flight instead of holding them back behind the tables.
    __device__ __forceinline__ void bind() {
        auto lane_u64 = [](uint64_t v, int src) -> uint64_t {   // v of lane `src` (per-lane src)
            const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)(uint32_t)v);
            const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(src << 2, (int)(uint32_t)(v >> 32));
            return (uint64_t)lo | ((uint64_t)hi << 32);
        };
        if (KIND == 1) {
            const int se = ge + sy;
            wg = (const uint8_t *)(((uint64_t)__builtin_amdgcn_readlane((int)(uint32_t)(tw0 >> 32), se) << 32) |
                                   (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)tw0, se));
            wu = (const uint8_t *)(((uint64_t)__builtin_amdgcn_readlane((int)(uint32_t)(tw1 >> 32), se) << 32) |
                                   (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)tw1, se));
        }
        if (KIND == 2) {
#pragma unroll
            for (int j = 0; j < UX; j++) {
                ubase[j] = (const uint8_t *)lane_u64(tw0, uspan[j] + sy);
                if (LP == 64) uoff[j] += (uint32_t)(ubase[j] - a.wlo);
            }
        }
    }

    __device__ __forceinline__ const float *xsrc(int v, int u) const {
        return (KIND == 2 ? x + (int64_t)v * K : x + (int64_t)v * a.x_stride) + 32 * u;
    }

    // activation pieces (8 floats of one unit per thread, first XP passes) and the lookup-table
    // words: requested before the weight loads, so waiting for them (vmcnt counts in issue
    // order) never waits on weights
    __device__ __forceinline__ void issue_x() {
        const int sub = tid & (XT - 1);
#pragma unroll
        for (int k = 0; k < XP; k++) {
            const int i = min((tid / XT) + XPU * k, nxu - 1);      // clamped: the loads are unconditional
            const int v = udiv_small(i, rnu), u = i - v * nu;
            load8(xsrc(v, u) + 8 * sub, a.x_aligned != 0, xf[k]);
        }
    }
    __device__ __forceinline__ void issue_tab() { F::tab_load(tid, treg); }

    // unit j of the row through accessor m into Rp[base + j]; paired formats load units j and
    // j+1 together at the even j and skip the odd one (its registers are already filled)
    template <class M>
    __device__ __forceinline__ void load_unit(const M &m, int j, typename F::Raw (&Rp)[UMAX], int base) {
        if constexpr (PAIRS) {
            if ((j & 1) == 0) F::load2(m, uoff[j], usub[j], Rp[base + j], Rp[base + j + 1]);
        } else {
            F::load(m, uoff[j], usub[j], Rp[base + j]);
        }
    }

    // one row per lane group into slot p. Rows past the end are clamped to a valid row and their
    // results dropped; with 64-lane groups their loads go through an empty buffer resource
    // instead (issued, so wait counts stay exact, but no memory is read).
    __device__ __forceinline__ void load_row(int p, int row) {
        const int last = nrow > 0 ? nrow - 1 : 0;
        const uint32_t nrec = __builtin_amdgcn_readfirstlane(row < nrow ? 0xffffffffu : 0u);   // SGPR
        // A 64-lane group covers whole rows, so its row index is wave-uniform: the row address is
        // then scalar arithmetic and every load goes through a buffer resource on that address
        // with a 32-bit lane offset (no per-load 64-bit vector adds).
        if (KIND == 2 && LP == 64) {   // experts within 4 GiB of a.wlo: lane offsets + row offset
            const int r = __builtin_amdgcn_readfirstlane(min(row, last));
            const BufferAt m(a.wlo, (uint32_t)((int64_t)r * rs), nrec);
#pragma unroll
            for (int j = 0; j < UX; j++) load_unit(m, j, R[p], 0);
            return;
        }
        if (KIND != 2 && LP == 64) {
            const uint8_t *bg = KIND == 1 ? wg : wb0;
            const int r = __builtin_amdgcn_readfirstlane(min(row, last));
            const BufferAt mg(bg + (int64_t)r * rs, 0, nrec);
            const BufferAt mu(KIND == 1 ? wu + (int64_t)r * rs : bg, 0, nrec);
#pragma unroll
            for (int j = 0; j < UX; j++) {
                load_unit(mg, j, R[p], 0);
                if (KIND == 1) load_unit(mu, j, R[p], UX);
            }
            return;
        }
        const int64_t roff = (int64_t)min(row, last) * rs;
        if (KIND == 1) {
#pragma unroll
            for (int j = 0; j < UX; j++) {
                load_unit(GlobalAt{wg + roff}, j, R[p], 0);
                load_unit(GlobalAt{wu + roff}, j, R[p], UX);
            }
        } else {
#pragma unroll
            for (int j = 0; j < UX; j++) load_unit(GlobalAt{ubase[j] + roff}, j, R[p], 0);
        }
    }
    // the first PF rows of the lane group (later rows are requested by run_rows as slots free up);
    // slots [p0, p1) only
    __device__ __forceinline__ void load_batch(int base, int p0 = 0, int p1 = PF) {
#pragma unroll
        for (int p = 0; p < PF; p++)
            if (p >= p0 && p < p1) load_row(p, base + p * ngroups);
    }

    // tables + q8_1 quantization of every activation vector into LDS (the caller then syncs).
    // The 4 threads of a unit share its amax and its two half sums through quad DPP; the
    // arithmetic per element is quant_unit's, so the result is the same bit for bit.
    __device__ __forceinline__ void stage_x() {
        F::tab_store(tid, treg);
        uint32_t *xm = (uint32_t *)(xq + (size_t)nxv * K);
        const int sub = tid & (XT - 1);
        if (F32Act<F>::value) {   // f32 activations: the floats themselves
            auto store_f = [&](int i, const float (&f)[8]) {
                const int v = udiv_small(i, rnu), u = i - v * nu;
                float4 *dst = (float4 *)((float *)xq + (size_t)v * K + 32 * u + 8 * sub);
                dst[0] = make_float4(f[0], f[1], f[2], f[3]);
                dst[1] = make_float4(f[4], f[5], f[6], f[7]);
            };
#pragma unroll
            for (int k = 0; k < XP; k++)
                if ((tid / XT) + XPU * k < nxu) store_f((tid / XT) + XPU * k, xf[k]);
            for (int i0 = XPU * XP; i0 < nxu; i0 += XPU) {
                const int i = i0 + tid / XT;
                if (i < nxu) {
                    const int v = udiv_small(i, rnu), u = i - v * nu;
                    float f[8];
                    load8(xsrc(v, u) + 8 * sub, a.x_aligned != 0, f);
                    store_f(i, f);
                }
            }
            return;
        }
        auto quant_store = [&](int i, const float (&f)[8]) {
            const int v = udiv_small(i, rnu), u = i - v * nu;
            float amax = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(f[e]));
            // quad max on the bit patterns (non-negative floats order as unsigned integers)
            uint32_t ab = __builtin_bit_cast(uint32_t, amax);
            ab = max(ab, __builtin_bit_cast(uint32_t, quad_swap<0xB1>(__builtin_bit_cast(float, ab))));   // [1,0,3,2]
            ab = max(ab, __builtin_bit_cast(uint32_t, quad_swap<0x4E>(__builtin_bit_cast(float, ab))));   // [2,3,0,1]
            amax = __builtin_bit_cast(float, ab);
            const float d = q8_div127(amax);
            float id = d != 0.f ? 1.0f / d : 0.f;
            id = id <= 3.40282347e38f ? id : 0.f;   // d < 2^-128: q = 0, as quant_unit
            uint32_t w[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                int q[4];
#pragma unroll
                for (int b = 0; b < 4; b++) q[b] = q8_round_mul(f[4 * h + b], id);
                w[h] = __builtin_amdgcn_perm((uint32_t)q[1], (uint32_t)q[0], 0x0c0c0400u) |
                       __builtin_amdgcn_perm((uint32_t)q[3], (uint32_t)q[2], 0x04000c0cu);
            }
            const int sum = __builtin_amdgcn_sdot4((int)w[1], 0x01010101, __builtin_amdgcn_sdot4((int)w[0], 0x01010101, 0, false), false);
            *(uint2 *)(xq + (size_t)v * K + 32 * u + 8 * sub) = make_uint2(w[0], w[1]);
            const int half = sum + __builtin_bit_cast(int, quad_swap<0xB1>(__builtin_bit_cast(float, sum)));
            const int shi = __builtin_bit_cast(int, quad_swap<0x4E>(__builtin_bit_cast(float, half)));
            if (sub == 0) {   // elements 0..15 sum in this lane, 16..31 in lane 2 of the quad
                xm[2 * i] = __builtin_bit_cast(uint32_t, h2f(f2h(d)));
                xm[2 * i + 1] = ((uint32_t)half & 0xffffu) | ((uint32_t)shi << 16);
            }
        };
#pragma unroll
        for (int k = 0; k < XP; k++)
            if ((tid / XT) + XPU * k < nxu) quant_store((tid / XT) + XPU * k, xf[k]);
        for (int i0 = XPU * XP; i0 < nxu; i0 += XPU) {   // large activation sets: the rest
            const int i = i0 + tid / XT;
            if (i < nxu) {   // whole quads are in or out together
                const int v = udiv_small(i, rnu), u = i - v * nu;
                float f[8];
                load8(xsrc(v, u) + 8 * sub, a.x_aligned != 0, f);
                quant_store(i, f);
            }
        }
    }

    // whether this wave's rows fit one batch
    __device__ __forceinline__ bool single_batch() const {
        return __builtin_amdgcn_readfirstlane(gid) + PF * ngroups >= nrow;
    }

    // activation units from LDS into registers, then every batch of rows (the first batch is
    // already loaded) with the results stored.
    __device__ __forceinline__ void run_rows() {
        const uint32_t *xm = (const uint32_t *)(xq + (size_t)nxv * K);
        XU xr[UX][NV];
#pragma unroll
        for (int j = 0; j < UX; j++) {
            const int up = unit_of(j) - uspan[j] * nu;
#pragma unroll
            for (int t = 0; t < NV; t++) {
                const int v = KIND == 2 ? uspan[j] * nv + t : t;
                const float w = KIND == 2 ? __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(
                                                (uspan[j] + sy) << 2, __builtin_bit_cast(int, wtl[t])))
                                          : 1.f;   // routing weight folded into D
                int xu = up;
                if constexpr (Joint<F>::value) xu = F::xunit(up);
                xr[j][t] = load_xu<F, XNEG>(xq, xm, K, nu, v, xu, w, uval[j] && t < nv);
            }
        }
        // Row results are gathered into lanes (lane p*NV + t of the group holds row p, vector t)
        // and finished in parallel: one SwiGLU / store sequence per batch instead of one per row.
        // Groups narrower than PF*NV results keep one store per row from the group's last lane.
        const bool gather = PF * NV <= lpr;
        const int bsrc = ((tid & 63) | (lpr - 1)) << 2;    // byte address of the group's last lane
        using TP = TwoPhase<F>;
        // Row ring (64-lane groups): slot p is refilled with the same slot's row of the next batch
        // as soon as its units are decoded, so PF rows stay in flight across batches. The refill is
        // unconditional inside the loop, also in the last batch (past the end it reads nothing):
        // a branch around it, or a last batch peeled off the loop, makes the compiler copy the
        // slots and wait for every load at the loop head. Waves with a single batch skip the
        // refills. Other widths load each batch at its start.
        auto batch = [&](const int base, auto issue_c) {
            constexpr bool ISSUE = decltype(issue_c)::value;
            float res0[PF][NV], res1[PF][NV];
            float out0 = 0.f, out1 = 0.f;
            // ring kernels (one vector, gather lanes): the output a GEMV / down store adds to, read
            // before this batch's refills so its wait does not cover them (clamped, always issued)
            float yold = 0.f;
            if (RING && KIND != 1) yold = y[min(base + min(lane, PF - 1) * ngroups, nrow - 1)];
            // units of the batch in order (row p, unit j), each one's table reads issued one unit
            // ahead (reads of rows past the end fetch valid table entries and are unused)
            typename TP::Dec dec[2];
            TP::fetch(R[0][0], dec[0]);
#pragma unroll
            for (int p = 0; p < PF; p++) {
                float acc0[NV], acc1[NV];
#pragma unroll
                for (int t = 0; t < NV; t++) acc0[t] = acc1[t] = 0.f;
                if (base + p * ngroups < nrow) {   // no loads inside: the waits stay exact
#pragma unroll
                    for (int j = 0; j < UMAX; j++) {
                        const int i = p * UMAX + j;
                        if (i + 1 < PF * UMAX) TP::fetch(R[(i + 1) / UMAX][(i + 1) % UMAX], dec[(i + 1) & 1]);
                        if (KIND != 1 && j >= UX) continue;
                        const int jx = j % UX;
                        if constexpr (JOINT) {   // the pair (j, j + 1) at even j
                            if (j & 1) continue;
                            if (KIND == 1 && j >= UX)
                                F::template dot_pair<NV>(R[p][j], R[p][j + 1], usub[jx], xr[jx], xr[jx + 1], nv, acc1);
                            else
                                F::template dot_pair<NV>(R[p][j], R[p][j + 1], usub[jx], xr[jx], xr[jx + 1], nv, acc0);
                            continue;
                        }
                        if (KIND == 1 && j >= UX)
                            TP::template dot<NV, XNEG>(R[p][j], dec[i & 1], usub[jx], tab, xr[jx], nv, acc1);
                        else
                            TP::template dot<NV, XNEG>(R[p][j], dec[i & 1], usub[jx], tab, xr[jx], nv, acc0);
                    }
                } else if (p + 1 < PF) {
                    TP::fetch(R[p + 1][0], dec[((p + 1) * UMAX) & 1]);
                }
                if (ISSUE) {   // kept after the slot's last use: hoisted above it, the loads would
                               // need fresh registers and a full wait at the loop head
                    __builtin_amdgcn_sched_barrier(0);
                    load_row(p, base + (PF + p) * ngroups);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int t = 0; t < NV; t++) {
                    res0[p][t] = group_sum(acc0[t], lpr);
                    if (KIND == 1) res1[p][t] = group_sum(acc1[t], lpr);
                    if (gather) {
                        const float v0 = __builtin_bit_cast(
                            float, __builtin_amdgcn_ds_bpermute(bsrc, __builtin_bit_cast(int, res0[p][t])));
                        out0 = lane == p * NV + t ? v0 : out0;
                        if (KIND == 1) {
                            const float v1 = __builtin_bit_cast(
                                float, __builtin_amdgcn_ds_bpermute(bsrc, __builtin_bit_cast(int, res1[p][t])));
                            out1 = lane == p * NV + t ? v1 : out1;
                        }
                    }
                }
            }
            if (gather) {
                const int p = lane / NV, t = lane % NV;   // NV is a power of two
                const int rr = base + p * ngroups;
                if (lane < PF * NV && t < nv && rr < nrow) {
                    if (KIND == 0) {
                        float *dst = y + (int64_t)t * a.y_stride + rr;
                        *dst = a.accumulate ? (RING ? yold : *dst) + out0 : out0;
                    } else if (KIND == 1) {
                        store_h(&y[((int64_t)ge * nv + t) * rows + rr], swiglu_fast(out0, out1, a.lim));
                    } else {
                        y[(int64_t)t * a.y_stride + rr] = (RING ? yold : y[(int64_t)t * a.y_stride + rr]) + out0;
                    }
                }
            } else if (lane == lpr - 1) {
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
                                    store_h(&y[((int64_t)ge * nv + t) * rows + rr], swiglu_fast(res0[p][t], res1[p][t], a.lim));
                                } else {
                                    y[(int64_t)t * a.y_stride + rr] += res0[p][t];
                                }
                            }
                        }
                    }
                }
            }
        };
        if (RING && single_batch()) {   // one batch: no refills
            if (gid < nrow) batch(gid, BoolC<false>{});
            return;
        }
        for (int base = gid; base < nrow; base += PF * ngroups) {
            if (!RING && base != gid) load_batch(base);
            batch(base, BoolC<RING>{});
        }
    }
};

template <class F, int KIND, int NV, int UMAX, int LP = 0>
__device__ __forceinline__ void stream_body(const StreamArgs &a) {
    extern __shared__ __align__(16) uint8_t smem[];
    StreamPass<F, KIND, NV, UMAX, LP> P(a, smem);
    P.issue_x();
    P.issue_tab();
    // GEMV: the activation loads stay ahead of the weight loads (vector loads return in order, so
    // the staging below then waits for the activations only, not for the weights the compiler
    // would otherwise hoist above them): Q8_0 6.9 -> 6.2 us, Q4_K 8.8 -> 8.2, Q6_K 16.4 -> 14.8.
    // (The MoE passes order their own requests around the staging; the barrier gained them nothing.)
    if constexpr (KIND == 0) __builtin_amdgcn_sched_barrier(0);
    P.bind();
    // ring kernels: only the first GS_RING_EARLY slots before the activation staging (a smaller
    // first request arrives sooner), the rest after it. For a GEMV the activations themselves
    // queue behind the chip-wide burst of first weight requests, so long rows (4+ units per lane)
    // split too: Q6_K K = 12288 14.7 -> 12.9 us; at 2 units per lane (K = 4096) all slots at once
    // (Q8_0 6.2 against 6.35 us, Q4_K even).
    constexpr int E = P.RING && (KIND != 0 || UMAX >= 4) && GS_RING_EARLY < P.PF ? GS_RING_EARLY : P.PF;
    P.load_batch(P.gid, 0, E);
    P.stage_x();
    __syncthreads();
    P.load_batch(P.gid, E, P.PF);
    P.run_rows();
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
// one-token GEMV, gate/up and down with 64-lane groups fixed at compile time (suffix _w; for down
// the host also guarantees a.wlo)
#define GS_STREAM_KERNEL_W(F, NAME, KIND, UM)                                                    \
    extern "C" __global__ void __launch_bounds__(GS_WG) __attribute__((amdgpu_waves_per_eu(GS_WPE))) \
        gs_k_stream_##NAME##_##KIND##_1_##UM##_w(StreamArgs a) {                                  \
        stream_body<F, KIND, 1, UM, 64>(a);                                                     \
    }
#define GS_STREAM_W(F, NAME)                                                                    \
    GS_STREAM_KERNEL_W(F, NAME, 0, 2) GS_STREAM_KERNEL_W(F, NAME, 0, 4)                         \
    GS_STREAM_KERNEL_W(F, NAME, 0, 6) GS_STREAM_KERNEL_W(F, NAME, 0, 8)                         \
    GS_STREAM_KERNEL_W(F, NAME, 1, 2) GS_STREAM_KERNEL_W(F, NAME, 1, 4) GS_STREAM_KERNEL_W(F, NAME, 1, 8) \
    GS_STREAM_KERNEL_W(F, NAME, 2, 2) GS_STREAM_KERNEL_W(F, NAME, 2, 4)                         \
    GS_STREAM_KERNEL_W(F, NAME, 2, 6) GS_STREAM_KERNEL_W(F, NAME, 2, 8)
#define GS_STREAM_ALL(F, NAME) GS_STREAM_MV(F, NAME, 0) GS_STREAM_GU(F, NAME) GS_STREAM_MV(F, NAME, 2) GS_STREAM_W(F, NAME)

// One code object per format keeps the build parallel: the Makefile compiles this file once
// per format (GS_STREAM_F: the F-struct, GS_STREAM_ID: its type id) and once with GS_COMMON for
// the kernels below.
#if defined(GS_STREAM_F)
GS_STREAM_ALL(GS_STREAM_F, GS_STREAM_ID)
// one-vector GEMV variants with aligned loads: _w4 (Q8_0, rows 4-byte aligned: FQ8_0A4) and _wa
// (Q8_0 other rows: FQ8_0A; Q6_K: FQ6_KA)
#if GS_STREAM_ID == 8
extern "C" __global__ void __launch_bounds__(GS_WG) __attribute__((amdgpu_waves_per_eu(GS_WPE)))
gs_k_stream_8_0_1_2_wa(StreamArgs a) { stream_body<FQ8_0A, 0, 1, 2, 64>(a); }
extern "C" __global__ void __launch_bounds__(GS_WG) __attribute__((amdgpu_waves_per_eu(GS_WPE)))
gs_k_stream_8_0_1_4_wa(StreamArgs a) { stream_body<FQ8_0A, 0, 1, 4, 64>(a); }
extern "C" __global__ void __launch_bounds__(GS_WG) __attribute__((amdgpu_waves_per_eu(GS_WPE)))
gs_k_stream_8_0_1_2_w4(StreamArgs a) { stream_body<FQ8_0A4, 0, 1, 2, 64>(a); }
extern "C" __global__ void __launch_bounds__(GS_WG) __attribute__((amdgpu_waves_per_eu(GS_WPE)))
gs_k_stream_8_0_1_4_w4(StreamArgs a) { stream_body<FQ8_0A4, 0, 1, 4, 64>(a); }
#endif
#if GS_STREAM_ID == 14
extern "C" __global__ void __launch_bounds__(GS_WG) __attribute__((amdgpu_waves_per_eu(GS_WPE)))
gs_k_stream_14_0_1_2_wa(StreamArgs a) { stream_body<FQ6_KA, 0, 1, 2, 64>(a); }
extern "C" __global__ void __launch_bounds__(GS_WG) __attribute__((amdgpu_waves_per_eu(GS_WPE)))
gs_k_stream_14_0_1_4_wa(StreamArgs a) { stream_body<FQ6_KA, 0, 1, 4, 64>(a); }
#endif
#endif

#if defined(GS_COMMON)

// =============================================================================================
// Whole-tensor dequantization (gs_dequant_f32 / gs_dequant_f16): one thread per 32-element unit
// (exact.h), stored as 8 (f32) or 4 (f16) 16-byte writes when the destination allows it.
// =============================================================================================
// Decode unit u of a tensor of n elements into v; returns the number of valid elements (32,
// except a plain-type tensor's last unit, which is decoded from a zero-padded copy so no byte
// past the tensor is read).
template <int QKB, int BB, void (*DEC)(const uint8_t *, int, float (&)[32])>
__device__ __forceinline__ int dequant_unit(const uint8_t *src, int64_t u, int64_t n, float (&v)[32]) {
    if (QKB >= 32) {
        constexpr int UPB = QKB / 32;
        const uint8_t *blk = src + (u / UPB) * BB;
        // whole-dword reads (unaligned global loads) where a dword decoder exists: the same values,
        // and no byte past the block is read (the last block may end the allocation)
        if constexpr (DEC == &exact::q8_0) exact::al::q8_0_block(blk, v);
        else if constexpr (DEC == &exact::q4_k) exact::al::q4_k(blk, (int)(u % UPB), v);
        else if constexpr (DEC == &exact::q6_k) exact::al::q6_k(blk, (int)(u % UPB), v);
        else DEC(blk, (int)(u % UPB), v);
        return 32;
    }
    const uint8_t *base = src + u * 32 * BB;
    const int cnt = (int)(n - 32 * u < 32 ? n - 32 * u : 32);
    if (cnt == 32) {
        DEC(base, 0, v);
    } else {
        uint8_t tmp[32 * BB];
        for (int i = 0; i < 32 * BB; i++) tmp[i] = i < cnt * BB ? base[i] : 0;
        DEC(tmp, 0, v);
    }
    return cnt;
}
// piece i (4 values) of the f32 -> f16 row conversion: one 16-byte load, one 8-byte store, so the
// lanes of a wave read 1 KB and write 512 bytes back to back (rows 16-byte aligned, K % 4 == 0)
__device__ __forceinline__ void rows_to_f16(const float *x, uint16_t *y, int64_t x_stride, int K, int N, int64_t i) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const int64_t per = K / 4;
    if (i >= per * N) return;
    const int64_t n = i / per, c = i - n * per;
    const f4v f = *(const f4v *)(x + n * x_stride + 4 * c);
    *(h4 *)(y + n * K + 4 * c) = __builtin_convertvector(f, h4);
}
#define GS_DEQ_KERNEL(TY, QKB, BB, DEC)                                                          \
    extern "C" __global__ void __launch_bounds__(256) gs_k_dequant_f32_##TY(DequantArgs a) {    \
        const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;                        \
        if (u >= a.n_units) return;                                                             \
        float v[32];                                                                            \
        const int cnt = dequant_unit<QKB, BB, DEC>(a.src, u, a.n, v);                           \
        float *d = (float *)a.dst + 32 * u;                                                     \
        if (cnt == 32 && a.aligned) {                                                           \
            for (int i = 0; i < 8; i++)                                                         \
                ((float4 *)d)[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]); \
        } else {                                                                                \
            for (int i = 0; i < cnt; i++) d[i] = v[i];                                          \
        }                                                                                       \
    }                                                                                           \
    extern "C" __global__ void __launch_bounds__(256) gs_k_dequant_f16_##TY(DequantArgs a) {    \
        __shared__ uint4 tr[256 * 4];   /* per wave 64 units x 64 bytes: the store transpose */    \
        if (a.cvt_n && (int)blockIdx.x >= a.w_blocks) {   /* the activation blocks */            \
            rows_to_f16(a.cvt_x, a.cvt_y, a.cvt_x_stride, a.cvt_K, a.cvt_n,                      \
                        (int64_t)(blockIdx.x - a.w_blocks) * blockDim.x + threadIdx.x);          \
            return;                                                                             \
        }                                                                                       \
        const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;                        \
        const int lane = threadIdx.x & 63;                                                       \
        const int64_t u0 = u - lane;   /* the wave's first unit */                               \
        float v[32];                                                                            \
        const int cnt = u < a.n_units ? dequant_unit<QKB, BB, DEC>(a.src, u, a.n, v) : 0;       \
        /* opaque to the optimizer: the f32 value (and the sign of a zero) reaches the single   \
           f32 -> f16 rounding unchanged */                                                     \
        for (int i = 0; i < 32; i++) asm volatile("" : "+v"(v[i]));                             \
        uint4 h[4];                                                                             \
        for (int i = 0; i < 4; i++)                                                             \
            h[i] = make_uint4(f2h(v[8 * i]) | (f2h(v[8 * i + 1]) << 16), f2h(v[8 * i + 2]) | (f2h(v[8 * i + 3]) << 16), \
                              f2h(v[8 * i + 4]) | (f2h(v[8 * i + 5]) << 16), f2h(v[8 * i + 6]) | (f2h(v[8 * i + 7]) << 16)); \
        if (a.aligned && u0 + 64 <= a.n_units && (QKB >= 32 || 32 * (u0 + 64) <= a.n)) {        \
            /* whole wave of full units: each lane's 64 bytes through LDS, then 16-byte pieces    \
               in address order, so every store instruction writes 1 KB back to back */           \
            uint4 *w = tr + (threadIdx.x >> 6) * 256;                                            \
            for (int i = 0; i < 4; i++) w[4 * lane + ((i + lane) & 3)] = h[i];                  \
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");                      \
            __builtin_amdgcn_wave_barrier();                                                    \
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");                      \
            uint4 *d = (uint4 *)((uint16_t *)a.dst + 32 * u0);                                   \
            for (int j = 0; j < 4; j++) {                                                       \
                const int c = 64 * j + lane, src_lane = c >> 2, piece = c & 3;                   \
                d[c] = w[4 * src_lane + ((piece + src_lane) & 3)];                              \
            }                                                                                   \
            return;                                                                             \
        }                                                                                       \
        if (cnt == 0) return;                                                                   \
        uint16_t *d = (uint16_t *)a.dst + 32 * u;                                               \
        if (cnt == 32 && a.aligned) {                                                           \
            for (int i = 0; i < 4; i++) ((uint4 *)d)[i] = h[i];                                   \
        } else {                                                                                \
            for (int i = 0; i < cnt; i++) d[i] = (uint16_t)f2h(v[i]);                           \
        }                                                                                       \
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
// Quantized GEMV of 2..8 vectors on int8 MFMA (quants.cu:53-256 semantics: y[t][r] (+)= W[r] . x[t])
//
// A 32-element unit is one v_mfma_i32_16x16x32_i8 step: the format's integer weights (Q8_0 int8,
// Q4_K nibbles, Q5_K 5-bit values, Q6_K 6-bit values - 32) against the vectors' q8_1 int8 values (quantized in the
// workgroup with the streaming kernels' arithmetic: the same int8 values, f16-rounded scales and
// sums). The MFMA gives the exact int32 dot of every (vector, row) pair of the unit for 16 rows at
// once; the unit's scales then take it into the f32 sum, as the streaming kernels do per unit:
//   Q8_0  d * d_x * dot;   Q4_K, Q5_K  (d*sc) * d_x * dot - (dmin*m) * s_x  (s_x = d_x * sum q_x);
//   Q6_K  the unit's two 16-element halves have their own scales: two MFMAs, each with the other
//         half's weight bytes zero, (d*sc_h) * d_x * dot_h summed.
// So each weight is read once for all vectors, where the streaming kernels hold at most 4 vectors'
// activations in registers (5..8: the matrix read twice) and, for rows beyond that register plan
// (Q6_K K = 12288), run one vector per slice.
// Workgroup: 16 rows, the row walked in chunks of 4096 elements. Per chunk the 16 rows' bytes go
// to LDS with 16-byte loads (1 KB per wave load; fragment-shaped loads touched 16 rows' lines per
// instruction), rows 16 bytes apart beyond their length so a fragment's 16 rows sit in different
// banks; the vectors' q8_1 units in LDS unit-major ([unit][vector][32 B]: a lane's 8 bytes for one
// MFMA are one conflict-free read). The next chunk's loads are issued before this chunk's
// contraction. 8 waves split a chunk's units; their partial sums are added in wave order.
// =============================================================================================
typedef int mv_v4i __attribute__((ext_vector_type(4)));
typedef uint32_t mv_u4 __attribute__((ext_vector_type(4)));   // a native vector: the chunk array stays in VGPRs

// 8 bytes at a 2-byte aligned LDS offset: three aligned dwords, shifted into place
__device__ __forceinline__ uint64_t mv_ld8(const uint8_t *r, uint32_t o) {
    const uint32_t oa = o & ~3u, sh = o & 3u;
    const uint32_t w0 = *(const uint32_t *)(r + oa), w1 = *(const uint32_t *)(r + oa + 4), w2 = *(const uint32_t *)(r + oa + 8);
    return (uint64_t)__builtin_amdgcn_alignbyte(w1, w0, sh) | ((uint64_t)__builtin_amdgcn_alignbyte(w2, w1, sh) << 32);
}
// unit u of a chunk row in LDS, lane quarter q (elements 8q .. 8q+7): the weights as int8 (b0; b1
// the second half for HALVES formats, each with the other half zero) and the scales
struct MvUnit {
    uint64_t b0, b1;
    float s0, s1, mn;
};
struct MvQ8_0 {
    static constexpr int TY = GS_Q8_0, QK = 32, BB = 34;
    static constexpr bool MIN = false, HALVES = false;
    __device__ static __forceinline__ void unit(const uint8_t *r, int u, int q, MvUnit &m) {
        const uint32_t blk = 34u * (uint32_t)u;
        m.b0 = mv_ld8(r, blk + 2u + 8u * (uint32_t)q);
        m.s0 = h2f(*(const uint16_t *)(r + blk));
    }
};
struct MvQ4_K {   // lib.rs:204-218 with scale_min_k4 (lib.rs:87-93)
    static constexpr int TY = GS_Q4_K, QK = 256, BB = 144;
    static constexpr bool MIN = true, HALVES = false;
    __device__ static __forceinline__ void unit(const uint8_t *r, int u, int q, MvUnit &m) {
        const uint32_t b = (uint32_t)u >> 3, uu = (uint32_t)u & 7u, blk = 144u * b;
        const uint64_t raw = *(const uint64_t *)(r + blk + 16u + 32u * (uu >> 1) + 8u * (uint32_t)q);
        m.b0 = (raw >> (4u * (uu & 1u))) & 0x0f0f0f0f0f0f0f0full;
        const uint32_t dd = *(const uint32_t *)(r + blk), sh = 8u * (uu & 3u);
        const uint32_t b1 = (*(const uint32_t *)(r + blk + 4) >> sh) & 0xffu, b2 = (*(const uint32_t *)(r + blk + 8) >> sh) & 0xffu,
                       b3 = (*(const uint32_t *)(r + blk + 12) >> sh) & 0xffu;
        const uint32_t sc = uu < 4 ? (b1 & 63u) : ((b3 & 0xfu) | ((b1 >> 6) << 4));
        const uint32_t mi = uu < 4 ? (b2 & 63u) : ((b3 >> 4) | ((b2 >> 6) << 4));
        m.s0 = h2f(dd & 0xffffu) * (float)sc;
        m.mn = h2f(dd >> 16) * (float)mi;
    }
};
struct MvQ5_K {   // lib.rs:221-240: Q4_K's nibbles and scales, bit u of qh[l] as the fifth bit
    static constexpr int TY = GS_Q5_K, QK = 256, BB = 176;
    static constexpr bool MIN = true, HALVES = false;
    __device__ static __forceinline__ void unit(const uint8_t *r, int u, int q, MvUnit &m) {
        const uint32_t b = (uint32_t)u >> 3, uu = (uint32_t)u & 7u, blk = 176u * b;
        const uint64_t raw = *(const uint64_t *)(r + blk + 48u + 32u * (uu >> 1) + 8u * (uint32_t)q);
        const uint64_t qh = *(const uint64_t *)(r + blk + 16u + 8u * (uint32_t)q);
        m.b0 = ((raw >> (4u * (uu & 1u))) & 0x0f0f0f0f0f0f0f0full) | (((qh >> uu) & 0x0101010101010101ull) << 4);
        const uint32_t dd = *(const uint32_t *)(r + blk), sh = 8u * (uu & 3u);
        const uint32_t b1 = (*(const uint32_t *)(r + blk + 4) >> sh) & 0xffu, b2 = (*(const uint32_t *)(r + blk + 8) >> sh) & 0xffu,
                       b3 = (*(const uint32_t *)(r + blk + 12) >> sh) & 0xffu;
        const uint32_t sc = uu < 4 ? (b1 & 63u) : ((b3 & 0xfu) | ((b1 >> 6) << 4));
        const uint32_t mi = uu < 4 ? (b2 & 63u) : ((b3 >> 4) | ((b2 >> 6) << 4));
        m.s0 = h2f(dd & 0xffffu) * (float)sc;
        m.mn = h2f(dd >> 16) * (float)mi;
    }
};
struct MvQ6_K {   // lib.rs:243-262
    static constexpr int TY = GS_Q6_K, QK = 256, BB = 210;
    static constexpr bool MIN = false, HALVES = true;
    __device__ static __forceinline__ void unit(const uint8_t *r, int u, int q, MvUnit &m) {
        const uint32_t b = (uint32_t)u >> 3, uu = (uint32_t)u & 7u, n = uu >> 2, g = uu & 3u, blk = 210u * b;
        const uint64_t ql = mv_ld8(r, blk + 64u * n + 32u * (g & 1u) + 8u * (uint32_t)q);
        const uint64_t qh = mv_ld8(r, blk + 128u + 32u * n + 8u * (uint32_t)q);
        uint64_t v = ((ql >> (4u * (g >> 1))) & 0x0f0f0f0f0f0f0f0full) | (((qh >> (2u * g)) & 0x0303030303030303ull) << 4);
        // v - 32 per byte without borrows between bytes (values 0..63)
        v = ((v | 0x8080808080808080ull) - 0x2020202020202020ull) ^ 0x8080808080808080ull;
        m.b0 = q < 2 ? v : 0ull;
        m.b1 = q < 2 ? 0ull : v;
        const float d = h2f(*(const uint16_t *)(r + blk + 208));
        const uint32_t scw = *(const uint16_t *)(r + blk + 192u + 8u * n + 2u * g);   // the two halves' int8 scales
        m.s0 = d * (float)(int)(int8_t)(scw & 0xffu);
        m.s1 = d * (float)(int)(int8_t)(scw >> 8);
    }
};

template <class F, bool MULTI>
__device__ __forceinline__ void mv_body(const MvArgs &a) {
    extern __shared__ __align__(16) uint8_t mv_lds[];
    constexpr int CK = 4096;                                    // elements per chunk (at most)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ck = a.K < CK ? a.K : CK, nch = a.K / ck;         // the host checks a.K % ck == 0
    const int U = ck / 32, nv = a.nv;                           // units per chunk
    const int rbytes = ck / F::QK * F::BB, RS = rbytes + 16;    // chunk row bytes (16-byte multiple), LDS pitch
    uint8_t *wl = mv_lds;                                       // [16][RS] raw rows of the chunk
    uint8_t *xq = mv_lds + 16 * (size_t)RS;                     // [U][8][32] int8
    float *xd = (float *)(xq + 256 * (size_t)U);                // [U][8] f16-rounded scales
    float *xs = xd + 8 * (size_t)U;                             // [U][8] scale * sum of q (MIN formats)
    float *red = xs + 8 * (size_t)U;                            // [8 waves][64 lanes][4]
    const int r0 = blockIdx.x * 16;
    const int ntask = nv * U * 4;                               // 8 floats per task, 4 tasks per unit
    const int cpr = rbytes / 16, nchunk = 16 * cpr;             // 16-byte pieces per row, per tile
    constexpr int XC = 8, WC = 9;                               // per thread: tasks, pieces (<= 4352 B rows)

    float f[XC][8];
    mv_u4 wc[WC];
    int wdst[WC];   // LDS byte offset of the piece (-1: none)
    // divisions by U and cpr through their reciprocals (exact below 2^21), and a scheduling
    // barrier after each load: the loads then go out as their addresses are ready, instead of
    // after every address of the step (which the compiler otherwise computes first: ~1 us later)
    const float rU = 1.0f / (float)U, rcpr = 1.0f / (float)cpr;
    auto issue_x = [&](int c) __attribute__((always_inline)) {
        const int k0 = c * ck;
#pragma unroll
        for (int i = 0; i < XC; i++) {
            // passes past the last task re-read a valid piece (uniform; no early exit, so the array
            // stays in registers)
            const int t = min(512 * i + tid, ntask - 1);
            const int sub = t & 3, vu = t >> 2, v = udiv_small(vu, rU), u = vu - v * U;
            const float4 *src = (const float4 *)(a.x + (int64_t)v * a.x_stride + k0 + 32 * u + 8 * sub);
            const float4 p0 = src[0], p1 = src[1];
            f[i][0] = p0.x; f[i][1] = p0.y; f[i][2] = p0.z; f[i][3] = p0.w;
            f[i][4] = p1.x; f[i][5] = p1.y; f[i][6] = p1.z; f[i][7] = p1.w;
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto issue_w = [&](int tile, int c) __attribute__((always_inline)) {
        const int64_t wk0 = (int64_t)(c * ck / F::QK) * F::BB;
#pragma unroll
        for (int i = 0; i < WC; i++) {
            const int z = min(512 * i + tid, nchunk - 1), rr = udiv_small(z, rcpr), cc = z - rr * cpr;
            const uint8_t *row = a.w + (int64_t)min(16 * tile + rr, a.rows - 1) * a.row_stride + wk0;   // tail rows: clamped, dropped
            wc[i] = *(const mv_u4 *)(row + 16 * cc);
            wdst[i] = 512 * i + tid < nchunk ? rr * RS + 16 * cc : -1;
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto stage_x = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < XC; i++) {
            if (512 * i >= ntask) continue;                      // uniform; quads are in or out together
            const int t = 512 * i + tid;
            float amax = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(f[i][e]));
            uint32_t ab = __builtin_bit_cast(uint32_t, amax);
            ab = max(ab, __builtin_bit_cast(uint32_t, quad_swap<0xB1>(__builtin_bit_cast(float, ab))));
            ab = max(ab, __builtin_bit_cast(uint32_t, quad_swap<0x4E>(__builtin_bit_cast(float, ab))));
            amax = __builtin_bit_cast(float, ab);
            const float d = q8_div127(amax);
            float id = d != 0.f ? 1.0f / d : 0.f;
            id = id <= 3.40282347e38f ? id : 0.f;   // d < 2^-128: q = 0, as quant_unit
            uint32_t w[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                int qv[4];
#pragma unroll
                for (int b = 0; b < 4; b++) qv[b] = q8_round_mul(f[i][4 * h + b], id);
                w[h] = __builtin_amdgcn_perm((uint32_t)qv[1], (uint32_t)qv[0], 0x0c0c0400u) |
                       __builtin_amdgcn_perm((uint32_t)qv[3], (uint32_t)qv[2], 0x04000c0cu);
            }
            int sum = 0;
            if (F::MIN) {   // the unit's sum of q: this thread's 8, then the quad's
                sum = __builtin_amdgcn_sdot4((int)w[1], 0x01010101, __builtin_amdgcn_sdot4((int)w[0], 0x01010101, 0, false), false);
                sum += __builtin_bit_cast(int, quad_swap<0xB1>(__builtin_bit_cast(float, sum)));
                sum += __builtin_bit_cast(int, quad_swap<0x4E>(__builtin_bit_cast(float, sum)));
            }
            if (t < ntask) {
                const int sub = t & 3, vu = t >> 2, v = udiv_small(vu, rU), u = vu - v * U;
                *(uint2 *)(xq + 256 * (size_t)u + 32 * v + 8 * sub) = make_uint2(w[0], w[1]);
                if (sub == 0) {
                    const float dh = h2f(f2h(d));
                    xd[8 * u + v] = dh;
                    if (F::MIN) xs[8 * u + v] = dh * (float)sum;
                }
            }
        }
    };

    const int j = lane & 15, q = lane >> 4;
    const int ta = j & 7;                 // the lane's A row (vector); rows 8..15 repeat 0..7, dropped
    const int tq = 4 * (q & 1);           // first vector of the lane's four D rows (q >= 2: dropped)
    const uint8_t *wrow = wl + (size_t)j * RS;
    const int upw = (U + 7) / 8, u0 = wave * upw, u1 = min(U, u0 + upw);
    // the workgroup's (chunk, tile) steps, chunk-major over its tiles blockIdx.x, blockIdx.x +
    // gridDim.x, ...: the activations of a chunk are staged once for all the workgroup's tiles, and
    // with several tiles each step adds its chunk's partial sums into y (chunk 0 stores them), in
    // chunk order; a single tile keeps them in registers until its last chunk
    // (MULTI = false: the host launched one step per workgroup, so no load is issued during a
    // contraction and the load registers are free there)
    const int ntile = (a.rows + 15) / 16;
    const int ntw = MULTI ? (ntile - 1 - (int)blockIdx.x) / (int)gridDim.x + 1 : 1;   // tiles of this workgroup
    const int nstep = MULTI ? ntw * nch : 1;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    issue_x(0);
    issue_w(blockIdx.x, 0);
    for (int k = 0; k < nstep; k++) {
        const int c = k / ntw, ti = k - c * ntw, tile = blockIdx.x + ti * gridDim.x;
        __builtin_amdgcn_sched_barrier(0);
        if (ti == 0) stage_x();
#pragma unroll
        for (int i = 0; i < WC; i++)
            if (wdst[i] >= 0) *(mv_u4 *)(wl + wdst[i]) = wc[i];
        __syncthreads();
        if (MULTI && k + 1 < nstep) {   // in flight during this step's contraction
            const int k1 = k + 1, c1 = k1 / ntw, t1 = k1 - c1 * ntw;
            if (t1 == 0) issue_x(c1);
            issue_w(blockIdx.x + t1 * gridDim.x, c1);
        }
        // four units per step: their LDS reads and MFMAs overlap
        constexpr int US = 4;
        for (int ub = u0; ub < u1; ub += US) {
            MvUnit m[US];
            uint64_t xa[US];
            float4 dx[US], sx[US];
#pragma unroll
            for (int i = 0; i < US; i++) {
                const int u = min(ub + i, u1 - 1);   // past the wave's last unit: re-read it, dropped below
                F::unit(wrow, u, q, m[i]);
                xa[i] = *(const uint64_t *)(xq + 256 * (size_t)u + 32 * ta + 8 * q);
                dx[i] = *(const float4 *)(xd + 8 * u + tq);
                if (F::MIN) sx[i] = *(const float4 *)(xs + 8 * u + tq);
            }
            mv_v4i dot0[US], dot1[US];
#pragma unroll
            for (int i = 0; i < US; i++) {
                dot0[i] = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)xa[i], (long)m[i].b0, mv_v4i{0, 0, 0, 0}, 0, 0, 0);
                if (F::HALVES)
                    dot1[i] = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)xa[i], (long)m[i].b1, mv_v4i{0, 0, 0, 0}, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < US; i++) {
                if (ub + i >= u1) continue;   // uniform
                const float e[4] = {dx[i].x, dx[i].y, dx[i].z, dx[i].w};
#pragma unroll
                for (int kk = 0; kk < 4; kk++) {
                    if (F::HALVES) acc[kk] += ((float)dot0[i][kk] * m[i].s0 + (float)dot1[i][kk] * m[i].s1) * e[kk];
                    else acc[kk] += (float)dot0[i][kk] * (m[i].s0 * e[kk]);
                }
                if (F::MIN) {
                    acc[0] -= m[i].mn * sx[i].x;
                    acc[1] -= m[i].mn * sx[i].y;
                    acc[2] -= m[i].mn * sx[i].z;
                    acc[3] -= m[i].mn * sx[i].w;
                }
            }
        }
        if (ntw > 1 || c == nch - 1) {   // the waves' partial sums, in wave order
            *(float4 *)(red + 4 * (64 * wave + lane)) = make_float4(acc[0], acc[1], acc[2], acc[3]);
            acc[0] = acc[1] = acc[2] = acc[3] = 0.f;
            __syncthreads();
            if (tid < 16 * 8) {
                const int t = tid >> 4, jj = tid & 15, r = 16 * tile + jj;
                const int src = 16 * (t >> 2) + jj, i = t & 3;   // the lane that holds D[t][jj]
                float sum = 0.f;
#pragma unroll
                for (int w = 0; w < 8; w++) sum += red[4 * (64 * w + src) + i];
                if (t < nv && r < a.rows) {
                    float *dst = a.y + (int64_t)t * a.y_stride + r;
                    *dst = a.accumulate || (ntw > 1 && c > 0) ? *dst + sum : sum;
                }
            }
        }
        __syncthreads();   // every wave is done with this step's LDS before the next is stored
    }
}
// _0: one (chunk, tile) step per workgroup; _1: a walk over several (chunk-major over its tiles)
#define GS_MV_KERNELS(TY, F)                                                                     \
    extern "C" __global__ void __launch_bounds__(512) gs_k_mv_##TY##_0(MvArgs a) { mv_body<F, false>(a); } \
    extern "C" __global__ void __launch_bounds__(512) gs_k_mv_##TY##_1(MvArgs a) { mv_body<F, true>(a); }
GS_MV_KERNELS(8, MvQ8_0)
GS_MV_KERNELS(12, MvQ4_K)
GS_MV_KERNELS(13, MvQ5_K)
GS_MV_KERNELS(14, MvQ6_K)

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
extern "C" __global__ void __launch_bounds__(256) gs_k_rows_to_f16(CvtArgs a) {
    rows_to_f16(a.x, a.y, a.x_stride, a.K, a.N, (int64_t)blockIdx.x * blockDim.x + threadIdx.x);
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

// =============================================================================================
// Row-length-independent matrix-vector kernels: the shapes the streaming kernels' register plan
// does not hold (gate/up rows longer than 64 lanes x 4 units per token, a down expert longer than
// 64 x 8 units) and plain-type rows whose length is a multiple of 8 but not of 32. The reference
// takes any K % 8 == 0 and K % QK == 0 (quants.cu:225-229, 380-381, 396-397); so do these.
// One wave per output row; lane l walks units l, l + 64, ... of the row, decodes each with the
// exact unit decoder and quantizes the matching activation unit to q8_1 on the fly (quant_unit,
// the same values the streaming kernels stage), so the result is the q8_1 product of the fast
// path up to f32 summation order. Plain types (F32, F16, BF16) take the f32 activations as they
// are, as the streaming kernels do.
//   kind 0 GEMV:   y[z][b][r] (+)= W[z][r] . x[z][b]              blockIdx.y = batch z
//   kind 1 GATEUP: h[e][t][r] = swiglu(gate_e[r] . x[t], up_e[r] . x[t])   blockIdx.y = expert e
//   kind 2 DOWN:   y[t][r] += sum_e w[t][e] (down_e[r] . h[e][t])
// Not a hot path: every row re-quantizes its activation units (they come from L2).
// =============================================================================================
template <int QKB, int BB, void (*DEC)(const uint8_t *, int, float (&)[32])>
__device__ __forceinline__ void any_unit_w(const uint8_t *row, int u, int K, float (&v)[32]) {
    if (QKB == 256) {
        DEC(row + (u >> 3) * BB, u & 7, v);
    } else if (QKB == 32) {
        DEC(row + u * BB, 0, v);
    } else {   // plain: the last unit of a row may be partial (K % 32 != 0): zero-padded copy
        const uint8_t *p = row + (int64_t)u * 32 * BB;
        const int cnt = min(32, K - 32 * u);
        if (cnt == 32) {
            DEC(p, 0, v);
        } else {
            uint8_t tmp[32 * BB];
            for (int i = 0; i < 32 * BB; i++) tmp[i] = i < cnt * BB ? p[i] : 0;
            DEC(tmp, 0, v);
        }
    }
}
// dot of 32 decoded weights with activation unit u of the row at xr
template <bool PLAIN>
__device__ __forceinline__ float any_unit_dot(const float (&w)[32], const float *xr, int u, int K) {
    float v[32];
    const int cnt = min(32, K - 32 * u);
#pragma unroll
    for (int i = 0; i < 32; i++) v[i] = i < cnt ? xr[32 * u + i] : 0.f;
    if (PLAIN) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) s += w[i] * v[i];
        return s;
    }
    const Q81 q = quant_unit(v);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) s += w[i] * (float)(int8_t)(q.q[i >> 2] >> (8 * (i & 3)));
    return h2f(f2h(q.d)) * s;
}
__device__ __forceinline__ float any_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
template <int KIND, int QKB, int BB, void (*DEC)(const uint8_t *, int, float (&)[32])>
__device__ __forceinline__ void any_body(const StreamArgs &a) {
    constexpr bool PLAIN = QKB == 1;
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6), nwave = gridDim.x * (blockDim.x >> 6);
    const int K = a.K, nu = (K + 31) / 32, nv = a.nvec;
    const int64_t rs = a.row_stride;
    for (int r = wave; r < a.rows; r += nwave) {
        float acc[GS_NT_MAX], acc2[GS_NT_MAX];
#pragma unroll
        for (int t = 0; t < GS_NT_MAX; t++) acc[t] = acc2[t] = 0.f;
        if (KIND == 0) {
            const int z = blockIdx.y;
            const uint8_t *row = a.w0[0] + (int64_t)z * a.w_bs + (int64_t)r * rs;
            const float *x = a.x + (int64_t)z * a.x_bs;
            for (int u = lane; u < nu; u += 64) {
                float w[32];
                any_unit_w<QKB, BB, DEC>(row, u, K, w);
#pragma unroll
                for (int t = 0; t < GS_NT_MAX; t++)
                    if (t < nv) acc[t] += any_unit_dot<PLAIN>(w, x + (int64_t)t * a.x_stride, u, K);
            }
        } else if (KIND == 1) {
            const int e = blockIdx.y;
            const uint8_t *rg = a.w0[e] + (int64_t)r * rs, *ru = a.w1[e] + (int64_t)r * rs;
            for (int u = lane; u < nu; u += 64) {
                float wg[32], wu[32];
                any_unit_w<QKB, BB, DEC>(rg, u, K, wg);
                any_unit_w<QKB, BB, DEC>(ru, u, K, wu);
#pragma unroll
                for (int t = 0; t < GS_NT_MAX; t++)
                    if (t < nv) {
                        acc[t] += any_unit_dot<PLAIN>(wg, a.x + (int64_t)t * a.x_stride, u, K);
                        acc2[t] += any_unit_dot<PLAIN>(wu, a.x + (int64_t)t * a.x_stride, u, K);
                    }
            }
        } else {
            for (int e = 0; e < a.nseg; e++) {
                const uint8_t *row = a.w0[e] + (int64_t)r * rs;
                float pe[GS_NT_MAX];
#pragma unroll
                for (int t = 0; t < GS_NT_MAX; t++) pe[t] = 0.f;
                for (int u = lane; u < nu; u += 64) {
                    float w[32];
                    any_unit_w<QKB, BB, DEC>(row, u, K, w);
#pragma unroll
                    for (int t = 0; t < GS_NT_MAX; t++)
                        if (t < nv && a.wt[t][e] != 0.f) pe[t] += any_unit_dot<PLAIN>(w, a.x + ((int64_t)e * nv + t) * K, u, K);
                }
#pragma unroll
                for (int t = 0; t < GS_NT_MAX; t++)
                    if (t < nv && a.wt[t][e] != 0.f) acc[t] += a.wt[t][e] * pe[t];
            }
        }
#pragma unroll
        for (int t = 0; t < GS_NT_MAX; t++) {
            if (t >= nv) continue;
            const float s = any_wave_sum(acc[t]);
            if (KIND == 1) {
                const float s2 = any_wave_sum(acc2[t]);
                if (lane == 0) a.y[((int64_t)blockIdx.y * nv + t) * a.rows + r] = swiglu(s, s2, a.lim);
            } else if (lane == 0) {
                float *dst = KIND == 0 ? a.y + (int64_t)blockIdx.y * a.y_bs + (int64_t)t * a.y_stride + r
                                       : a.y + (int64_t)t * a.y_stride + r;
                *dst = (KIND == 2 || a.accumulate) ? *dst + s : s;
            }
        }
    }
}
#define GS_ANY_KERNEL(TY, QKB, BB, DEC)                                                          \
    extern "C" __global__ void __launch_bounds__(256) gs_k_any_0_##TY(StreamArgs a) { any_body<0, QKB, BB, DEC>(a); } \
    extern "C" __global__ void __launch_bounds__(256) gs_k_any_1_##TY(StreamArgs a) { any_body<1, QKB, BB, DEC>(a); } \
    extern "C" __global__ void __launch_bounds__(256) gs_k_any_2_##TY(StreamArgs a) { any_body<2, QKB, BB, DEC>(a); }
GS_TYPE_LIST(GS_ANY_KERNEL)
#endif  // GS_COMMON
