// gfx950 grouped MoE GEMM for the multi-token routed-expert FFN (prefill, MTP verify).
//
// The (token, expert) pairs arrive sorted by expert (CSR offsets, as the engine's grouping in
// crates/engine/src/forward.rs:1017-1036 builds them). One launch covers every expert of the
// layer: a persistent grid walks a tile list (expert, row block, token chunk) that each workgroup
// derives from the offsets, so no host round trip and no per-expert launch.
//
// Contraction on MFMA (v_mfma_f32_16x16x32_f16), weights as the B operand:
//   * IQ2_XXS super-block (256 weights of one row) -> f16 B fragments that hold the exact integers
//     grid * sign * (2s+1) (|v| <= 43*31 = 1333, exact in f16); the remaining factor d/8 of the
//     super-block is applied to the f32 accumulator once per super-block. A lane owns one row
//     (the D column it accumulates), so that factor is one scalar per lane.
//   * activations (A operand) are the q8_1 values D*q of each row after a power-of-two row scale
//     (restored in the epilogue). D*q has up to 19 significant bits, so for gate/up it is carried
//     exactly as two f16 halves (hi + lo, two MFMAs per fragment): a rounded x would perturb
//     gate/up by ~1e-4 relative, enough to flip q8_1 rounding decisions when h is re-quantized
//     (rel-L2 ~2e-3 at the output). h enters the down projection as one rounded f16 (~2e-4).
//   * the K order inside a super-block is permuted so that a lane decodes whole 32-element units:
//     lane quarter Q (lane >> 4) owns units 2Q and 2Q+1, MFMA m (0..7) takes group m&3 of unit
//     2Q + (m>>2). A and B use the same permutation, so the dot product is unchanged.
// Epilogues: kind 1 (gate/up) writes h = swiglu(gate.x, up.x) per pair; kind 2 (down) adds the
// routing-weighted result into y[token] with f32 atomics (the combine of quants.cu:324-363).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "kargs.h"
#include "formats.h"

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// grid values as f16 (8 per entry) and the f16 sign masks of ksigns(i) (bit 15 per negative lane)
__shared__ uint4 gs_grp_grid16[256];
__shared__ uint4 gs_grp_sgn16[128];
__shared__ int gs_grp_pre[GS_GRP_EXP_MAX + 1];

__device__ __forceinline__ void grp_tables(int tid) {
    if (tid < 256) {
        const uint64_t g = iq2xxs_grid[tid];
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lo = f2h((float)((g >> (16 * i)) & 0xff));
            const uint32_t hi = f2h((float)((g >> (16 * i + 8)) & 0xff));
            w[i] = lo | (hi << 16);
        }
        gs_grp_grid16[tid] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    if (tid < 128) {
        const uint32_t k = ksigns((uint32_t)tid);
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; i++) w[i] = (((k >> (2 * i)) & 1u) << 15) | (((k >> (2 * i + 1)) & 1u) << 31);
        gs_grp_sgn16[tid] = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// B fragment: group G (0..3) of the unit with words (a0 = grid indices, a1 = signs | s << 28),
// times c = 2s+1, as 8 f16 integers
template <int G>
__device__ __forceinline__ h8 iq2_frag(uint32_t a0, uint32_t a1, _Float16 c) {
    const uint4 g = gs_grp_grid16[(a0 >> (8 * G)) & 0xff];
    const uint4 s = gs_grp_sgn16[(a1 >> (7 * G)) & 127];
    const uint4 v = make_uint4(g.x ^ s.x, g.y ^ s.y, g.z ^ s.z, g.w ^ s.w);
    return __builtin_bit_cast(h8, v) * c;
}

__device__ __forceinline__ float grp_swiglu(float g, float u, float lim) {   // ops.cu:101-115
    if (lim > 0.f) {
        g = fminf(g, lim);
        u = fminf(fmaxf(u, -lim), lim);
    }
    return g / (1.f + expf(-g)) * u;
}

// Tile list: expert e owns ceil(m_e / MT) * nrb consecutive tiles (row block fastest, so the
// workgroups that share a token chunk run side by side and share its activations in L2).
__device__ __forceinline__ void grp_prefix(const GroupedArgs &a, int MT, int nrb) {
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid < 64) {
        int carry = 0;
        for (int e0 = 0; e0 < a.n_exp; e0 += 64) {
            const int e = e0 + lane;
            int cnt = 0;
            if (e < a.n_exp) {
                const int m = a.offs[e + 1] - a.offs[e];
                cnt = m > 0 ? (m + MT - 1) / MT * nrb : 0;
            }
            int v = cnt;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int u = __shfl_up(v, o);
                if (lane >= o) v += u;
            }
            if (e < a.n_exp) gs_grp_pre[e + 1] = carry + v;
            carry += __shfl(v, 63);
        }
        if (lane == 0) gs_grp_pre[0] = 0;
    }
}

// KIND 1: gate/up + SwiGLU -> h[pair][rows] (f32).  KIND 2: down, y[token][rows] += w * result.
// NT token sub-tiles of 16, NR row sub-tiles of 16 per wave, 4 waves per workgroup.
template <int KIND, int NT, int NR>
__device__ __forceinline__ void grouped_body(const GroupedArgs &a) {
    constexpr int MATS = KIND == 1 ? 2 : 1;
    constexpr int HL = KIND == 1 ? 2 : 1;   // activation halves (hi, lo)
    constexpr int MT = 16 * NT;
    constexpr int RB = GS_GRP_WAVES * 16 * NR;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, q = lane >> 4;
    const int K = a.K, rows = a.rows, nsb = K / 256;
    const int nrb = (rows + RB - 1) / RB;
    grp_tables(tid);
    grp_prefix(a, MT, nrb);
    __syncthreads();
    const int total = gs_grp_pre[a.n_exp];

    for (int t = blockIdx.x; t < total; t += gridDim.x) {
        int lo = 0, hi = a.n_exp;   // largest e with pre[e] <= t
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (gs_grp_pre[mid] <= t) lo = mid; else hi = mid;
        }
        const int e = __builtin_amdgcn_readfirstlane(lo);
        const int local = t - gs_grp_pre[e];
        const int chunk = local / nrb, rb = local - chunk * nrb;
        const int p_beg = a.offs[e] + chunk * MT;
        const int p_end = min(p_beg + MT, a.offs[e + 1]);
        const int n_here = p_end - p_beg;
        const int row0 = rb * RB + wave * 16 * NR;

        // weights: lane row row0 + 16n + j (clamped; results of clamped rows are dropped)
        const uint8_t *wrow[NR][MATS];
#pragma unroll
        for (int n = 0; n < NR; n++) {
            const int r = min(row0 + 16 * n + j, rows - 1);
#pragma unroll
            for (int mt = 0; mt < MATS; mt++) {
                const uint8_t *base = a.experts[3 * e + (KIND == 2 ? 2 : mt)];
                wrow[n][mt] = base + (int64_t)r * a.row_stride + 2 + 16 * q;
            }
        }
        // activations: lane row = slot 16t + j of the chunk (clamped to the last pair)
        int64_t arow[NT];
#pragma unroll
        for (int tt = 0; tt < NT; tt++) {
            const int p = p_beg + min(16 * tt + j, n_here - 1);
            const int r = KIND == 1 ? a.idx[p] : p;
            arow[tt] = (int64_t)r * K + 64 * q;
        }

        f4 acc[NT][NR][MATS];
#pragma unroll
        for (int tt = 0; tt < NT; tt++)
#pragma unroll
            for (int n = 0; n < NR; n++)
#pragma unroll
                for (int mt = 0; mt < MATS; mt++) acc[tt][n][mt] = f4{0.f, 0.f, 0.f, 0.f};

        // raw weight words of the next super-block, prefetched one super-block ahead
        uint4 wq[NR][MATS];
        uint32_t wd[NR][MATS];
#pragma unroll
        for (int n = 0; n < NR; n++)
#pragma unroll
            for (int mt = 0; mt < MATS; mt++) {
                wq[n][mt] = ldg16(wrow[n][mt]);
                wd[n][mt] = ldg2(wrow[n][mt] - 2 - 16 * q);
            }

        for (int b = 0; b < nsb; b++) {
            uint4 cq[NR][MATS];
            float cd[NR][MATS];
#pragma unroll
            for (int n = 0; n < NR; n++)
#pragma unroll
                for (int mt = 0; mt < MATS; mt++) {
                    cq[n][mt] = wq[n][mt];
                    cd[n][mt] = h2f(wd[n][mt]) * 0.125f;
                }
            if (b + 1 < nsb) {
#pragma unroll
                for (int n = 0; n < NR; n++)
#pragma unroll
                    for (int mt = 0; mt < MATS; mt++) {
                        const uint8_t *p = wrow[n][mt] + (int64_t)(b + 1) * 66;
                        wq[n][mt] = ldg16(p);
                        wd[n][mt] = ldg2(p - 2 - 16 * q);
                    }
            }
            h8 av[HL][NT][8];
#pragma unroll
            for (int hl = 0; hl < HL; hl++)
#pragma unroll
                for (int tt = 0; tt < NT; tt++)
                    if (tt == 0 || 16 * tt < n_here) {
                        const uint4 *src = (const uint4 *)((hl ? a.act_lo : a.act) + arow[tt] + 256 * b);
#pragma unroll
                        for (int m = 0; m < 8; m++) av[hl][tt][m] = __builtin_bit_cast(h8, src[m]);
                    }
            f4 sb[NT][NR][MATS];
#pragma unroll
            for (int tt = 0; tt < NT; tt++)
#pragma unroll
                for (int n = 0; n < NR; n++)
#pragma unroll
                    for (int mt = 0; mt < MATS; mt++) sb[tt][n][mt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int hu = 0; hu < 2; hu++) {    // unit 2q + hu
                _Float16 c[NR][MATS];
#pragma unroll
                for (int n = 0; n < NR; n++)
#pragma unroll
                    for (int mt = 0; mt < MATS; mt++) {
                        const uint32_t a1 = hu ? cq[n][mt].w : cq[n][mt].y;
                        c[n][mt] = (_Float16)(int)(2 * (a1 >> 28) + 1);
                    }
#define GS_GRP_STEP(G)                                                                             \
    {                                                                                              \
        h8 bf[NR][MATS];                                                                           \
        _Pragma("unroll") for (int n = 0; n < NR; n++)                                             \
        _Pragma("unroll") for (int mt = 0; mt < MATS; mt++)                                        \
            bf[n][mt] = iq2_frag<G>(hu ? cq[n][mt].z : cq[n][mt].x, hu ? cq[n][mt].w : cq[n][mt].y, c[n][mt]); \
        _Pragma("unroll") for (int tt = 0; tt < NT; tt++)                                          \
            if (tt == 0 || 16 * tt < n_here) {                                                     \
                _Pragma("unroll") for (int hl = 0; hl < HL; hl++)                                  \
                _Pragma("unroll") for (int n = 0; n < NR; n++)                                     \
                _Pragma("unroll") for (int mt = 0; mt < MATS; mt++)                                \
                    sb[tt][n][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[hl][tt][4 * hu + G],  \
                                                                           bf[n][mt], sb[tt][n][mt], 0, 0, 0); \
            }                                                                                      \
    }
                GS_GRP_STEP(0) GS_GRP_STEP(1) GS_GRP_STEP(2) GS_GRP_STEP(3)
#undef GS_GRP_STEP
            }
#pragma unroll
            for (int tt = 0; tt < NT; tt++)
#pragma unroll
                for (int n = 0; n < NR; n++)
#pragma unroll
                    for (int mt = 0; mt < MATS; mt++) acc[tt][n][mt] += cd[n][mt] * sb[tt][n][mt];
        }

        // epilogue: lane holds tokens 16t + 4q + i (i < 4) of row row0 + 16n + j
#pragma unroll
        for (int tt = 0; tt < NT; tt++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int slot = 16 * tt + 4 * q + i;
                if (slot >= n_here) continue;
                const int p = p_beg + slot;
                const int tok = a.idx[p];
                const float sc = a.ascale[KIND == 1 ? tok : p];
                const float wt = KIND == 2 ? a.w[p] : 1.f;
                if (KIND == 2 && wt == 0.f) continue;
#pragma unroll
                for (int n = 0; n < NR; n++) {
                    const int r = row0 + 16 * n + j;
                    if (r >= rows) continue;
                    if (KIND == 1) {
                        a.out[(int64_t)p * rows + r] = grp_swiglu(acc[tt][n][0][i] * sc, acc[tt][n][1][i] * sc, a.lim);
                    } else {
                        unsafeAtomicAdd(a.out + (int64_t)tok * rows + r, wt * (acc[tt][n][0][i] * sc));
                    }
                }
            }
        }
    }
}

#define GS_GRP_KERNEL(KIND, NT, NR)                                                              \
    extern "C" __global__ void __launch_bounds__(64 * GS_GRP_WAVES)                             \
        gs_k_grouped_16_##KIND##_##NT##_##NR(GroupedArgs a) {                                   \
        grouped_body<KIND, NT, NR>(a);                                                          \
    }
GS_GRP_KERNEL(1, 1, 1)
GS_GRP_KERNEL(1, 2, 1)
GS_GRP_KERNEL(1, 4, 1)
GS_GRP_KERNEL(2, 1, 2)
GS_GRP_KERNEL(2, 2, 2)
GS_GRP_KERNEL(2, 4, 2)

// ---------------------------------------------------------------------------------------------
// Activation rows -> f16 MFMA operands. Each 32-element unit is q8_1-quantized exactly as the
// streaming kernels do (d = amax/127, q = round(x/d), D = f16(d)); the f16 operand is
// D*q*2^-E with 2^E >= 2 * row amax, so no value overflows f16 and the relative rounding error
// stays below 2^-11. scale[row] = 2^E restores the magnitude in the GEMM epilogue.
// One wave per row, 4 rows per workgroup.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

extern "C" __global__ void __launch_bounds__(256) gs_k_rows_q8f16(RowsQArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.nrows) return;
    const int nu = a.K / 32;
    const float *src = a.x + (int64_t)row * a.x_stride;
    float amax = 0.f;
    for (int u = lane; u < nu; u += 64) {
        const float4 *p = (const float4 *)(src + 32 * u);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 f = p[i];
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(f.x), fabsf(f.y)), fmaxf(fabsf(f.z), fabsf(f.w))));
        }
    }
    amax = wave_max(amax);
    int E = 0;
    if (amax > 0.f) (void)frexpf(amax, &E);   // amax < 2^E
    E -= 14;                                     // values * 2^-E < 2^14 (D rounding stays below 2^15)
    const float down = ldexpf(1.f, -E);
    if (lane == 0) a.scale[row] = ldexpf(1.f, E);
    uint16_t *dst = a.out + (int64_t)row * a.K;
    for (int u = lane; u < nu; u += 64) {
        float v[32];
        const float4 *p = (const float4 *)(src + 32 * u);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 f = p[i];
            v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
        }
        float m = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) m = fmaxf(m, fabsf(v[i]));
        const float d = m / 127.0f;
        const float id = d != 0.f ? 1.0f / d : 0.f;
        const float D = h2f(f2h(d)) * down;
        uint32_t o[16], ol[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float v0 = D * __builtin_roundf(v[2 * i] * id), v1 = D * __builtin_roundf(v[2 * i + 1] * id);
            const uint32_t h0 = f2h(v0), h1 = f2h(v1);
            o[i] = h0 | (h1 << 16);
            ol[i] = f2h(v0 - h2f(h0)) | (f2h(v1 - h2f(h1)) << 16);   // exact remainders
        }
        uint4 *d4 = (uint4 *)(dst + 32 * u);
#pragma unroll
        for (int i = 0; i < 4; i++) d4[i] = make_uint4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
        if (a.out_lo) {
            uint4 *l4 = (uint4 *)(a.out_lo + (int64_t)row * a.K + 32 * u);
#pragma unroll
            for (int i = 0; i < 4; i++) l4[i] = make_uint4(ol[4 * i], ol[4 * i + 1], ol[4 * i + 2], ol[4 * i + 3]);
        }
    }
}
