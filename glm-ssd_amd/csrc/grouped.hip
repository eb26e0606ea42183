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
typedef uint32_t u4 __attribute__((ext_vector_type(4)));   // staging chunk (a native vector, so it stays in VGPRs)

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
#ifdef GS_GRP_PROBE_NODECODE   // profiling variant: no table lookups
    return __builtin_bit_cast(h8, make_uint4(a0, a1, a0 ^ a1, a0 + a1));
#endif
    const uint4 g = gs_grp_grid16[(a0 >> (8 * G)) & 0xff];
    const uint4 s = gs_grp_sgn16[(a1 >> (7 * G)) & 127];
    const uint4 v = make_uint4(g.x ^ s.x, g.y ^ s.y, g.z ^ s.z, g.w ^ s.w);
    return __builtin_bit_cast(h8, v) * c;
}

// profiling variants replace single components of the contraction
#ifdef GS_GRP_PROBE_NOLDSA
#define GS_GRP_AV(p) __builtin_bit_cast(h8, make_uint4(cc, j, hl, tt))
#else
#define GS_GRP_AV(p) __builtin_bit_cast(h8, *(const uint4 *)(p))
#endif
#ifdef GS_GRP_PROBE_NOMFMA
#define GS_GRP_MFMA(A, B, C) ((C) + __builtin_bit_cast(f4, (A) + (B)))
#else
#define GS_GRP_MFMA(A, B, C) __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, C, 0, 0, 0)
#endif

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
//
// Software pipeline over the workgroup's flat sequence of (tile, super-block) positions, across
// tile boundaries: weight words are loaded two positions ahead, the activations one position
// ahead (into registers, stored to the other LDS buffer after the current position is
// contracted; one barrier per position). A tile's descriptor (expert, pair range, activation
// rows) is fetched at the start of the previous tile and its epilogue operands (token ids,
// scales, combine weights) during the tile, so no load is waited on right after it is issued.
// A token row of one super-block is 512 B in LDS (32 chunks of 16 B); chunk c of slot i sits at
// chunk position c ^ (i & 15), so the 16 lanes that read one chunk column hit 16 bank groups.
template <int KIND, int NT, int NR>
__device__ __forceinline__ void grouped_body(const GroupedArgs &a) {
    constexpr int MATS = KIND == 1 ? 2 : 1;
    constexpr int HL = KIND == 1 ? 2 : 1;            // activation halves (hi, lo)
    constexpr int MT = 16 * NT;
    constexpr int RB = GS_GRP_WAVES * 16 * NR;
    constexpr int NTH = 64 * GS_GRP_WAVES;
    constexpr int SLAB = HL * MT * 512;              // bytes of one staged super-block
    constexpr int NLD = SLAB / 16 / NTH;             // 16-byte chunks per thread per super-block
    static_assert(SLAB % (16 * NTH) == 0, "staging split");
    extern __shared__ __align__(16) uint8_t gs_grp_dyn[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, q = lane >> 4;
    const int K = a.K, rows = a.rows, nsb = K / 256;
    const int nrb = (rows + RB - 1) / RB;
    const uint32_t rs = (uint32_t)a.row_stride;
    grp_tables(tid);
    grp_prefix(a, MT, nrb);
    __syncthreads();
    const int total = gs_grp_pre[a.n_exp];
    int t = blockIdx.x;
    if (t >= total) return;

    // staging chunks of this thread: chunk z = tid + NTH*k -> half, slot, chunk column
    int dst[NLD];
#pragma unroll
    for (int k = 0; k < NLD; k++) {
        const int z = tid + NTH * k;
        const int i = (z >> 5) % MT, c = z & 31;
        dst[k] = (z >> 5) / MT * MT * 512 + i * 512 + ((c ^ (i & 15)) << 4);
    }

    // ---- tile descriptors ---------------------------------------------------------------------
    struct Desc {
        int p_beg, n_here, row0;
        const uint8_t *wb[MATS];   // expert matrix bases (uniform)
    };
    auto describe = [&](int tt_, Desc &d) {
        int lo = 0, hi = a.n_exp;   // largest e with pre[e] <= t
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (gs_grp_pre[mid] <= tt_) lo = mid; else hi = mid;
        }
        const int e = __builtin_amdgcn_readfirstlane(lo);
        const int local = tt_ - gs_grp_pre[e];
        const int chunk = local / nrb, rb = local - chunk * nrb;
        const int o0 = a.offs[e], o1 = a.offs[e + 1];
        d.p_beg = o0 + chunk * MT;
        d.n_here = min(MT, o1 - d.p_beg);
        d.row0 = rb * RB + wave * 16 * NR;
#pragma unroll
        for (int mt = 0; mt < MATS; mt++) d.wb[mt] = a.experts[3 * e + (KIND == 2 ? 2 : mt)];
    };
    // per-lane weight offsets of a tile (row of sub-tile n, this lane's 16 bytes of each block)
    auto woffs = [&](const Desc &d, uint32_t (&wo)[NR]) {
#pragma unroll
        for (int n = 0; n < NR; n++) wo[n] = (uint32_t)min(d.row0 + 16 * n + j, rows - 1) * rs + 2 + 16 * q;
    };
    // activation source rows of the staging chunks (raw: pair index or token id)
    auto arows_raw = [&](const Desc &d, int (&ar)[NLD]) {
#pragma unroll
        for (int k = 0; k < NLD; k++) {
            const int i = ((tid + NTH * k) >> 5) % MT;
            const int p = d.p_beg + min(i, d.n_here - 1);
            ar[k] = KIND == 1 ? a.idx[p] : p;
        }
    };

    Desc cur, nxt;
    describe(t, cur);
    const int tstep = gridDim.x;
    bool has_nxt = t + tstep < total;
    if (has_nxt) describe(t + tstep, nxt);
    uint32_t wo_cur[NR], wo_nxt[NR];
    woffs(cur, wo_cur);
    if (has_nxt) woffs(nxt, wo_nxt);
    int ar_cur[NLD], ar_nxt[NLD];
    arows_raw(cur, ar_cur);
    if (has_nxt) arows_raw(nxt, ar_nxt);

    auto load_w = [&](const Desc &d, const uint32_t (&wo)[NR], int b, uint4 (&wq)[NR][MATS], uint32_t (&wd)[NR][MATS]) {
#pragma unroll
        for (int n = 0; n < NR; n++)
#pragma unroll
            for (int mt = 0; mt < MATS; mt++) {
#ifdef GS_GRP_PROBE_NOWLOAD   // profiling variant: every position re-reads super-block 0 (cache hits)
                const uint8_t *p = d.wb[mt] + wo[n];
#else
                const uint8_t *p = d.wb[mt] + (wo[n] + 66u * b);
#endif
                wq[n][mt] = ldg16(p);
                wd[n][mt] = ldg2(p - 2 - 16 * q);
            }
    };
    auto load_a = [&](const int (&ar)[NLD], int b, u4 (&stg)[NLD]) {
#pragma unroll
        for (int k = 0; k < NLD; k++) {
            const int z = tid + NTH * k;
            const uint16_t *base = (z >> 5) / MT ? a.act_lo : a.act;
#ifdef GS_GRP_PROBE_NOSTG   // profiling variant: no activation staging loads
            stg[k] = u4{(uint32_t)ar[k], (uint32_t)b, (uint32_t)z, 0u};
            (void)base;
#else
            stg[k] = *(const GS_GLOBAL u4 *)(const GS_GLOBAL uint16_t *)(base + ((uint32_t)ar[k] * (uint32_t)K + 256u * b + 8u * (z & 31)));
#endif
        }
    };

    // prologue: weights of positions 0 and 1, activations of position 0
    uint4 w0q[NR][MATS], w1q[NR][MATS];
    uint32_t w0d[NR][MATS], w1d[NR][MATS];
    {
        u4 stg0[NLD];
        load_a(ar_cur, 0, stg0);
        load_w(cur, wo_cur, 0, w0q, w0d);
        load_w(cur, wo_cur, 1, w1q, w1d);
#pragma unroll
        for (int k = 0; k < NLD; k++) *(u4 *)(gs_grp_dyn + dst[k]) = stg0[k];
    }
    __syncthreads();

    // epilogue operands of the current tile, requested early
    int ep_tok[NT][4];
    float ep_sc[NT][4], ep_w[NT][4];
    auto ep_load = [&](const Desc &d) {
#pragma unroll
        for (int tt = 0; tt < NT; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int p = d.p_beg + min(16 * tt + 4 * q + i, d.n_here - 1);
                ep_tok[tt][i] = a.idx[p];
                ep_w[tt][i] = KIND == 2 ? a.w[p] : 1.f;
                if (KIND == 2) ep_sc[tt][i] = a.ascale[p];
            }
    };
    ep_load(cur);

    f4 acc[NT][NR][MATS];
#pragma unroll
    for (int tt = 0; tt < NT; tt++)
#pragma unroll
        for (int n = 0; n < NR; n++)
#pragma unroll
            for (int mt = 0; mt < MATS; mt++) acc[tt][n][mt] = f4{0.f, 0.f, 0.f, 0.f};

    int b = 0, buf = 0;
    for (;;) {
        // ---- issue: activations of position +1, weights of position +2 -------------------
        const bool last_sb = b == nsb - 1;
        const bool have1 = !last_sb || has_nxt;
        u4 stg[NLD];
        if (have1) {   // one load site: select the tile element-wise (no array aliasing)
            int ar[NLD];
#pragma unroll
            for (int k = 0; k < NLD; k++) ar[k] = last_sb ? ar_nxt[k] : ar_cur[k];
            load_a(ar, last_sb ? 0 : b + 1, stg);
        }
        uint4 w2q[NR][MATS];
        uint32_t w2d[NR][MATS];
        {
            const bool in_cur = b + 2 < nsb;
            if (in_cur || has_nxt) {
                Desc d;
                uint32_t wo[NR];
#pragma unroll
                for (int mt = 0; mt < MATS; mt++) d.wb[mt] = in_cur ? cur.wb[mt] : nxt.wb[mt];
#pragma unroll
                for (int n = 0; n < NR; n++) wo[n] = in_cur ? wo_cur[n] : wo_nxt[n];
                load_w(d, wo, in_cur ? b + 2 : b + 2 - nsb, w2q, w2d);
            }
        }
        if (KIND == 1 && b == nsb / 2) {   // gate/up row scales by token id
#pragma unroll
            for (int tt = 0; tt < NT; tt++)
#pragma unroll
                for (int i = 0; i < 4; i++) ep_sc[tt][i] = a.ascale[ep_tok[tt][i]];
        }

        // ---- contract position (cur, b) ------------------------------------------------------
        {
            const uint8_t *slab = gs_grp_dyn + buf * SLAB;
            const int n_here = cur.n_here;
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
                        const uint32_t a1 = hu ? w0q[n][mt].w : w0q[n][mt].y;
                        c[n][mt] = (_Float16)(int)(2 * (a1 >> 28) + 1);
                    }
#define GS_GRP_STEP(G)                                                                             \
    {                                                                                              \
        h8 bf[NR][MATS];                                                                           \
        _Pragma("unroll") for (int n = 0; n < NR; n++)                                             \
        _Pragma("unroll") for (int mt = 0; mt < MATS; mt++)                                        \
            bf[n][mt] = iq2_frag<G>(hu ? w0q[n][mt].z : w0q[n][mt].x, hu ? w0q[n][mt].w : w0q[n][mt].y, c[n][mt]); \
        const int cc = 8 * q + 4 * hu + G;                                                         \
        _Pragma("unroll") for (int tt = 0; tt < NT; tt++)                                          \
            if (tt == 0 || 16 * tt < n_here) {                                                     \
                _Pragma("unroll") for (int hl = 0; hl < HL; hl++) {                                \
                    const h8 av = GS_GRP_AV(slab + (hl * MT + 16 * tt + j) * 512 + ((cc ^ j) << 4)); \
                    _Pragma("unroll") for (int n = 0; n < NR; n++)                                 \
                    _Pragma("unroll") for (int mt = 0; mt < MATS; mt++)                            \
                        sb[tt][n][mt] = GS_GRP_MFMA(av, bf[n][mt], sb[tt][n][mt]);                 \
                }                                                                                  \
            }                                                                                      \
    }
                GS_GRP_STEP(0) GS_GRP_STEP(1) GS_GRP_STEP(2) GS_GRP_STEP(3)
#undef GS_GRP_STEP
            }
#pragma unroll
            for (int n = 0; n < NR; n++)
#pragma unroll
                for (int mt = 0; mt < MATS; mt++) {
                    const float cd = h2f(w0d[n][mt]) * 0.125f;
#pragma unroll
                    for (int tt = 0; tt < NT; tt++) acc[tt][n][mt] += cd * sb[tt][n][mt];
                }
        }

        // ---- tile epilogue: lane holds tokens 16t + 4q + i (i < 4) of row row0 + 16n + j ----
        if (last_sb) {
#pragma unroll
            for (int tt = 0; tt < NT; tt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int slot = 16 * tt + 4 * q + i;
                    const float sc = ep_sc[tt][i], wt = ep_w[tt][i];
                    if (slot < cur.n_here && (KIND == 1 || wt != 0.f)) {
                        const int p = cur.p_beg + slot;
#pragma unroll
                        for (int n = 0; n < NR; n++) {
                            const int r = cur.row0 + 16 * n + j;
                            if (r < rows) {
                                if (KIND == 1)
                                    a.out[(int64_t)p * rows + r] =
                                        grp_swiglu(acc[tt][n][0][i] * sc, acc[tt][n][1][i] * sc, a.lim);
                                else
                                    unsafeAtomicAdd(a.out + (int64_t)ep_tok[tt][i] * rows + r, wt * (acc[tt][n][0][i] * sc));
                            }
                        }
                    }
                }
#pragma unroll
            for (int tt = 0; tt < NT; tt++)
#pragma unroll
                for (int n = 0; n < NR; n++)
#pragma unroll
                    for (int mt = 0; mt < MATS; mt++) acc[tt][n][mt] = f4{0.f, 0.f, 0.f, 0.f};
        }
        if (!have1) break;

        // ---- advance: stage position +1, rotate the weight registers -------------------------
#pragma unroll
        for (int k = 0; k < NLD; k++) *(u4 *)(gs_grp_dyn + (buf ^ 1) * SLAB + dst[k]) = stg[k];
#pragma unroll
        for (int n = 0; n < NR; n++)
#pragma unroll
            for (int mt = 0; mt < MATS; mt++) {
                w0q[n][mt] = w1q[n][mt]; w0d[n][mt] = w1d[n][mt];
                w1q[n][mt] = w2q[n][mt]; w1d[n][mt] = w2d[n][mt];
            }
        buf ^= 1;
        if (last_sb) {   // enter the next tile; fetch the one after it
            b = 0;
            t += tstep;
            cur = nxt;
#pragma unroll
            for (int n = 0; n < NR; n++) wo_cur[n] = wo_nxt[n];
#pragma unroll
            for (int k = 0; k < NLD; k++) ar_cur[k] = ar_nxt[k];
            ep_load(cur);
            has_nxt = t + tstep < total;
            if (has_nxt) {
                describe(t + tstep, nxt);
                woffs(nxt, wo_nxt);
                arows_raw(nxt, ar_nxt);
            }
        } else {
            b++;
        }
        __syncthreads();
    }
}

#define GS_GRP_KERNEL(KIND, NT, NR)                                                              \
    extern "C" __global__ void __launch_bounds__(64 * GS_GRP_WAVES)                             \
        gs_k_grouped_16_##KIND##_##NT##_##NR(GroupedArgs a) {                                   \
        grouped_body<KIND, NT, NR>(a);                                                          \
    }
GS_GRP_KERNEL(1, 1, 1)
GS_GRP_KERNEL(1, 1, 2)
GS_GRP_KERNEL(1, 2, 1)
GS_GRP_KERNEL(1, 2, 2)
GS_GRP_KERNEL(1, 2, 4)
GS_GRP_KERNEL(2, 1, 1)
GS_GRP_KERNEL(2, 1, 2)
GS_GRP_KERNEL(2, 2, 2)
GS_GRP_KERNEL(2, 2, 4)
GS_GRP_KERNEL(2, 4, 4)

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
