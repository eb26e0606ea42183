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
//     (the D column it accumulates), so that factor is one scalar per lane. Weights are therefore
//     exact, where the reference's GEMM rounds dequantized weights to half (gemm.cu:57-66).
//   * IQ3_XXS (98-byte super-blocks) the same way: grid * sign * (2s+1) (|v| <= 62*31 = 1922),
//     remaining factor d/4; a unit's 8 index bytes give two 4-value table entries per group.
//   * activations (A operand) are f16, as in the reference's multi-token GEMM (gemm.cu:69-78),
//     after a power-of-two row scale that keeps the row's largest value in the f16 normal range
//     (restored exactly in the epilogue); h enters the down projection the same way.
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

// Decode tables in LDS, built by every workgroup at start:
//   signs (16 KB, at byte 0): for a 7-bit sign index i, the 8 elements' sign bits of ksigns(i) as
//     two words P (elements 0..3) and Q (4..7), 8 bytes: P holds element 0 at bit 15, 1 at bit 31,
//     2 at bit 14 and 3 at bit 30, so P & 0x80008000 and (P << 1) & 0x80008000 are the f16 sign
//     masks of element pairs (0, 1) and (2, 3); Q likewise for 4..7. Replicated 16 times: lane j
//     reads its copy at 128 i + 8 (j & 15), so the 16 lanes reading at once never share a bank;
//   grid (64 KB, at byte GS_GRP_GRID_OFF): for grid index g and unit scale s (0..15), the 8
//     (IQ2_XXS) or 4 (IQ3_XXS) grid values times 2s+1 as f16 at 256 g + 16 s -- the address is one
//     v_perm of the index byte and the scale nibble (grid * (2s+1) <= 43 * 31 = 1333 for IQ2_XXS,
//     62 * 31 = 1922 for IQ3_XXS: exact in f16).
// A B fragment (8 weights) is one 16-byte grid read, one 8-byte sign read, 2 shifts and 4
// mask-and-XORs (one v_bitop3 each).
#define GS_GRP_GRID_OFF 16384
#define GS_GRP_TAB_BYTES (16384 + 65536)
// Workgroup bookkeeping, in the dynamic LDS after the tables and the activation slots (the kernels
// declare no static LDS, so the dynamic LDS starts at address 0 and every table address is a
// compile-time offset from 0: no base-address add per lookup).
struct GrpMeta {
    int pre[GS_GRP_EXP_MAX + 1];   // tile prefix over the experts
    // epilogue operands of a tile's token slots, by tile parity (waves drift up to one position apart)
    int ep_tok[2][64];
    float ep_w[2][64], ep_sc[2][64];
    // fills of the four activation slots (slot s has been stored by cnt[s] waves so far) and, per
    // tile parity, the sequence number of the tile whose epilogue operands are in ep_*
    uint32_t cnt[4];
    uint32_t ep_seq[2];
};
static_assert(sizeof(GrpMeta) <= GS_GRP_META_BYTES, "bookkeeping fits its LDS share");

// Sticky expiry flag of this code object's bounded LDS waits (host.cpp gs_wait_status reads and
// clears it): nonzero once any wait gave up before its count arrived, i.e. some output of a
// launch since the last clear may be wrong.
__device__ uint32_t gs_wait_expired;

template <int TY, int NTH>
__device__ __forceinline__ void grp_tables(uint8_t *tab, int tid) {
    // thread -> (grid index g, 8 of the 16 scales): one table read per thread, issued up front
    constexpr int PER = 4096 / NTH;   // entries per thread (8 with 512 threads)
    static_assert(PER >= 1 && 16 % PER == 0, "threads per workgroup");
    const int e0 = tid * PER, g = e0 >> 4;
    const uint64_t grid = TY == GS_IQ2_XXS ? iq2xxs_grid[g] : (uint64_t)iq3xxs_grid[g];
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int e = e0 + k, sc = e & 15;
        const float m = (float)(2 * sc + 1);
        uint32_t w[4];
        if (TY == GS_IQ2_XXS) {
#pragma unroll
            for (int i = 0; i < 4; i++)
                w[i] = f2h(m * (float)((grid >> (16 * i)) & 0xff)) | (f2h(m * (float)((grid >> (16 * i + 8)) & 0xff)) << 16);
        } else {   // IQ3_XXS: 4 grid values per entry, the upper 8 bytes of the slot unused
#pragma unroll
            for (int i = 0; i < 2; i++)
                w[i] = f2h(m * (float)((grid >> (16 * i)) & 0xff)) | (f2h(m * (float)((grid >> (16 * i + 8)) & 0xff)) << 16);
            w[2] = w[3] = 0;
        }
        *(uint4 *)(tab + GS_GRP_GRID_OFF + (e << 4)) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    for (int e = tid; e < 128 * 16; e += NTH) {
        const uint32_t k = ksigns((uint32_t)(e >> 4));
        uint32_t w[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint32_t b = k >> (4 * h);
            w[h] = ((b & 1u) << 15) | (((b >> 1) & 1u) << 31) | (((b >> 2) & 1u) << 14) | (((b >> 3) & 1u) << 30);
        }
        *(uint2 *)(tab + (e << 3)) = make_uint2(w[0], w[1]);
    }
}

// B fragment of group G (0..3) of one unit: 8 f16 integers grid * sign * (2s+1). Two phases, so
// a decode step issues the table reads of all its fragments before it waits for any of them:
//   IQ2_XXS: a0 = the unit's 4 grid-index bytes, a1 = signs | s << 28; one 16-byte grid read;
//   IQ3_XXS: g0, g1 = its 8 index bytes, a1 as above; two 8-byte reads of 4-value entries
//     (lib.rs:312-328);
// both: one 8-byte sign read (r16 = 8 (j & 15), the lane's replica); finish expands it to the
// four f16 sign masks and applies them with XOR.
struct FragRaw {
    uint4 g;
    uint2 sm;
    uint2 g2;   // IQ3_XXS: the second 4-value entry
};
template <int G>
__device__ __forceinline__ uint32_t sign_off(uint32_t a1, uint32_t r16) {
    return (__builtin_amdgcn_ubfe(a1, 7 * G, 7) << 7) | r16;
}
template <int G>
__device__ __forceinline__ void iq2_frag_fetch(const uint8_t *tab, uint32_t a0, uint32_t a1, uint32_t r16, FragRaw &r) {
    const uint32_t ga = __builtin_amdgcn_perm(a0, a1 & 0xF0000000u, 0x0c0c0403u + (G << 8));
    r.g = *(const uint4 *)(tab + GS_GRP_GRID_OFF + ga);
    r.sm = *(const uint2 *)(tab + sign_off<G>(a1, r16));
}
template <int G>
__device__ __forceinline__ void iq3_frag_fetch(const uint8_t *tab, uint32_t g0, uint32_t g1, uint32_t a1, uint32_t r16,
                                               FragRaw &r) {
    const uint32_t gw = G < 2 ? g0 : g1;
    constexpr uint32_t b0 = (2 * G) & 3;
    const uint32_t hs = a1 & 0xF0000000u;
    const uint2 lo = *(const uint2 *)(tab + GS_GRP_GRID_OFF + __builtin_amdgcn_perm(gw, hs, 0x0c0c0403u + (b0 << 8)));
    r.g2 = *(const uint2 *)(tab + GS_GRP_GRID_OFF + __builtin_amdgcn_perm(gw, hs, 0x0c0c0403u + ((b0 + 1) << 8)));
    r.g = make_uint4(lo.x, lo.y, 0u, 0u);
    r.sm = *(const uint2 *)(tab + sign_off<G>(a1, r16));
}
// Load of a wave-uniform address in data no kernel of this launch writes (the CSR offsets and the
// expert table), through the constant address space: a scalar load, waited on by its own counter
// instead of the in-order vector-memory counter that the weight stream keeps busy.
template <class T>
__device__ __forceinline__ T ld_scalar(const T *p) {
    return *(const __attribute__((address_space(4))) T *)(const __attribute__((address_space(4))) void *)p;
}
template <bool IQ3>
__device__ __forceinline__ h8 frag_finish(const FragRaw &r) {
    const uint4 g = IQ3 ? make_uint4(r.g.x, r.g.y, r.g2.x, r.g2.y) : r.g;
    constexpr uint32_t M = 0x80008000u;
    return __builtin_bit_cast(h8, make_uint4(g.x ^ (r.sm.x & M), g.y ^ ((r.sm.x << 1) & M), g.z ^ (r.sm.y & M),
                                             g.w ^ ((r.sm.y << 1) & M)));
}

#define GS_GRP_AV_LOAD(tt, cc) __builtin_bit_cast(h8, *(const uint4 *)(slab + (16 * (tt) + j) * 512 + ((((cc) ^ j)) << 4)))

__device__ __forceinline__ float grp_swiglu(float g, float u, float lim) {   // ops.cu:101-115
    if (lim > 0.f) {
        g = fminf(g, lim);
        u = fminf(fmaxf(u, -lim), lim);
    }
    return g / (1.f + expf(-g)) * u;
}

// Tile list, experts in id order. Expert e owns ceil(m_e / MT) * nrb consecutive tiles, the token
// chunks of one row block adjacent (chunk fastest), so the chunks that read the same weights run
// side by side. (Scheduling experts by pair count, largest first, made no difference at 512
// tokens: every tile streams the same K, so tiles cost about the same; the count ranking itself,
// done by every workgroup, took 10 us of a 4-token call.)
// m_tmp: n_exp ints of scratch (the staging area, free during the prologue).
template <int NTH>
__device__ __forceinline__ void grp_prefix(const GroupedArgs &a, int MT, int nrb, int *m_tmp, int *pre) {
    const int tid = threadIdx.x, lane = tid & 63;
    for (int e = tid; e < a.n_exp; e += NTH) m_tmp[e] = a.offs[e + 1] - a.offs[e];
    __syncthreads();
    if (tid < 64) {
        int carry = 0;
        for (int r0 = 0; r0 < a.n_exp; r0 += 64) {
            const int r = r0 + lane;
            int cnt = 0;
            if (r < a.n_exp) {
                const int m = m_tmp[r];
                cnt = m > 0 ? (m + MT - 1) / MT * nrb : 0;
            }
            int v = cnt;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int u = __shfl_up(v, o);
                if (lane >= o) v += u;
            }
            if (r < a.n_exp) pre[r + 1] = carry + v;
            carry += __shfl(v, 63);
        }
        if (lane == 0) pre[0] = 0;
    }
}

// KIND 1: gate/up + SwiGLU -> h[pair][rows] (f32).  KIND 2: down, y[token][rows] += w * result.
// NT token sub-tiles of 16, NR row sub-tiles of 16 per wave, WV waves per workgroup.
//
// Software pipeline over the workgroup's flat sequence of (tile, super-block) positions, across
// tile boundaries: weight words are loaded two positions ahead, the activations one position
// ahead (into registers, stored to the other LDS buffer after the current position is
// contracted; one barrier per position). A tile's descriptor (expert, pair range, activation
// rows) is fetched at the start of the previous tile and its epilogue operands (token ids,
// scales, combine weights) during the tile, so no load is waited on right after it is issued.
// A token row of one super-block is 512 B in LDS (32 chunks of 16 B); chunk c of slot i sits at
// chunk position c ^ (i & 15), so the 16 lanes that read one chunk column hit 16 bank groups.
template <int TY, int KIND, int NT, int NR, int WV>
__device__ __forceinline__ void grouped_body(const GroupedArgs &a) {
    static_assert(TY == GS_IQ2_XXS || TY == GS_IQ3_XXS, "grouped formats: IQ2_XXS, IQ3_XXS");
    constexpr bool IQ3 = TY == GS_IQ3_XXS;
    constexpr uint32_t BB = IQ3 ? 98 : 66;                  // bytes per super-block
    constexpr float XS = IQ3 ? 0.25f : 0.125f;             // d factor left after the (2s+1) integers
    constexpr int MATS = KIND == 1 ? 2 : 1;
    constexpr int MT = 16 * NT;
    constexpr int RB = WV * 16 * NR;
    constexpr int NTH = 64 * WV;
    constexpr int SLAB = MT * 512;                   // bytes of one staged super-block
    constexpr int NCH = SLAB / 16;                   // 16-byte chunks per staged super-block
    constexpr int NLD = (NCH + NTH - 1) / NTH;       // per thread (the last one may be partial)
    // The launch's dynamic LDS is the kernel's only LDS, so it starts at LDS address 0; spelling
    // that address as a constant (rather than through an extern __shared__ symbol, whose address
    // is left to the linker) lets every table address fold into the load's offset field.
    uint8_t *const gs_grp_dyn =
        (uint8_t *)__builtin_bit_cast(__attribute__((address_space(3))) uint8_t *, (uint32_t)0);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, q = lane >> 4;
    const uint32_t r16 = (uint32_t)j << 3;   // the lane's sign-table replica
    const int K = a.K, rows = a.rows, nsb = K / 256;
    const int nrb = (rows + RB - 1) / RB;
    const uint32_t rs = (uint32_t)a.row_stride;
    uint8_t *const tab = gs_grp_dyn;
    uint8_t *const stage = gs_grp_dyn + GS_GRP_TAB_BYTES;
    grp_tables<TY, NTH>(tab, tid);
    GrpMeta &M = *(GrpMeta *)(gs_grp_dyn + GS_GRP_TAB_BYTES + 4 * SLAB);
    grp_prefix<NTH>(a, MT, nrb, (int *)stage, M.pre);
    __syncthreads();
    const int total = M.pre[a.n_exp];
    // Workgroup w runs on XCD w % 8 (round-robin dispatch). With a grid that is a multiple of 8,
    // round k of workgroup w takes tile k*G + (w % 8) * G/8 + w / 8, so consecutive tiles of the
    // list (the chunks of one row block) run at the same time on one XCD and share its L2.
    const int G8 = gridDim.x >> 3;
    int t = (gridDim.x & 7) == 0 ? (int)(blockIdx.x & 7) * G8 + (int)(blockIdx.x >> 3) : (int)blockIdx.x;
    if (t >= total) return;

    // staging chunks of this thread: chunk z = tid + NTH*k -> slot z >> 5, chunk column z & 31
    int dst[NLD];
#pragma unroll
    for (int k = 0; k < NLD; k++) {
        const int z = tid + NTH * k;
        const int i = min(z >> 5, MT - 1), c = z & 31;
        dst[k] = i * 512 + ((c ^ (i & 15)) << 4);
    }

    // ---- tile descriptors ---------------------------------------------------------------------
    struct Desc {
        int p_beg, n_here, row0;
        const uint8_t *wb[MATS];   // expert matrix bases (uniform)
    };
    auto describe = [&](int tt_, Desc &d) {
        int lo = 0, hi = a.n_exp;   // largest expert e with pre[e] <= t (the owner of tile t)
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (M.pre[mid] <= tt_) lo = mid; else hi = mid;
        }
        const int e = __builtin_amdgcn_readfirstlane(lo);
        const int local = tt_ - M.pre[e];
        const int o0 = ld_scalar(a.offs + e), o1 = ld_scalar(a.offs + e + 1);
        const int nch = (o1 - o0 + MT - 1) / MT;
        const int rb = local / nch, chunk = local - rb * nch;
        d.p_beg = o0 + chunk * MT;
        d.n_here = min(MT, o1 - d.p_beg);
        d.row0 = rb * RB + wave * 16 * NR;
#pragma unroll
        for (int mt = 0; mt < MATS; mt++) d.wb[mt] = ld_scalar(a.experts + 3 * e + (KIND == 2 ? 2 : mt));
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
            const int i = min((tid + NTH * k) >> 5, MT - 1);
            const int p = d.p_beg + min(i, d.n_here - 1);
            ar[k] = KIND == 1 ? a.idx[p] : p;
        }
    };

    // nxt repeats cur when there is no next tile (its loads are issued and dropped)
    Desc cur, nxt;
    describe(t, cur);
    const int tstep = gridDim.x;
    bool has_nxt = t + tstep < total;
    describe(has_nxt ? t + tstep : t, nxt);
    uint32_t wo_cur[NR], wo_nxt[NR];
    woffs(cur, wo_cur);
    woffs(nxt, wo_nxt);
    int ar_cur[NLD], ar_nxt[NLD];
    arows_raw(cur, ar_cur);
    arows_raw(nxt, ar_nxt);

    static_assert(NR * MATS <= 4, "one block-scale load per lane quarter");
    struct WRegs {   // one position's raw weight words: 16 bytes (units 2q, 2q+1) + f16 d per row
        uint4 q[NR][MATS];
        uint2 sg[NR][MATS];   // IQ3_XXS: the two units' sign/scale words
        uint32_t dq;          // f16 block scale of row sub-tile (n, mt) = (q / MATS, q % MATS), row j
    };
    auto load_w = [&](const Desc &d, const uint32_t (&wo)[NR], int b, WRegs &w) {
#pragma unroll
        for (int n = 0; n < NR; n++)
#pragma unroll
            for (int mt = 0; mt < MATS; mt++) {
                const uint8_t *p = d.wb[mt] + (wo[n] + BB * b);
                w.q[n][mt] = ldg16(p);
                if (IQ3) w.sg[n][mt] = ldg8(p + 64 - 8 * q);   // block + 66 + 8q
            }
        // one 2-byte load per lane for all NR x MATS row sub-tiles' block scales (lane quarter q
        // takes sub-tile q), instead of one load instruction per sub-tile
        {
            const int sq = q < NR * MATS ? q : 0, sn = sq / MATS, smt = sq % MATS;
            const uint8_t *wbq = d.wb[0];
#pragma unroll
            for (int mt = 1; mt < MATS; mt++) wbq = smt == mt ? d.wb[mt] : wbq;
            uint32_t won = wo[0];
#pragma unroll
            for (int n = 1; n < NR; n++) won = sn == n ? wo[n] : won;
            w.dq = ldg2(wbq + (won + BB * b) - 2 - 16 * q);
        }
    };
    auto load_a = [&](const int (&ar)[NLD], int b, u4 (&stg)[NLD]) {
#pragma unroll
        for (int k = 0; k < NLD; k++) {
            const int z = tid + NTH * k;
            if (NCH % NTH != 0 && z >= NCH) continue;
            stg[k] = *(const GS_GLOBAL u4 *)(const GS_GLOBAL uint16_t *)(a.act + ((uint32_t)ar[k] * (uint32_t)K + 256u * b + 8u * (z & 31)));
        }
    };

    // prologue: weights and activations of positions 0 and 1 (nsb >= 2: both in the first tile).
    // Three weight register sets rotate by role (the loop body is instantiated three times), so a
    // set loaded for position p + 2 is not touched until position p + 2: no register copies.
    WRegs W0, W1, W2;
    {
        u4 stg0[NLD], stg1[NLD];
        load_a(ar_cur, 0, stg0);
        load_a(ar_cur, 1, stg1);
        load_w(cur, wo_cur, 0, W0);
        load_w(cur, wo_cur, 1, W1);
#pragma unroll
        for (int k = 0; k < NLD; k++)
            if (NCH % NTH == 0 || tid + NTH * k < NCH) {
                *(u4 *)(stage + dst[k]) = stg0[k];
                *(u4 *)(stage + SLAB + dst[k]) = stg1[k];
            }
    }
    if (tid < 4) M.cnt[tid] = tid < 2 ? NTH / 64 : 0u;   // slots 0, 1: positions 0, 1, stored by every wave
    if (tid < 2) M.ep_seq[tid] = 0xffffffffu;
    // token slots hold a valid token id (0) before the first publication, so an epilogue that
    // ran past an expired wait still addresses rows of y
    if (tid < 128) (&M.ep_tok[0][0])[tid] = 0;
    __syncthreads();

    // Epilogue operands of the current tile (per token slot: token id, combine weight, activation
    // row scale): thread `tid` < MT loads slot tid's at tile entry and stores them to LDS at
    // position nsb-2, so the epilogue at nsb-1 reads them from LDS after a barrier (three
    // registers instead of NT x 12 per lane).
    int ep_tok = 0;
    float ep_w = 1.f, ep_sc = 1.f;
    auto ep_load = [&](const Desc &d) {
        if (tid < MT) {
            const int p = d.p_beg + min(tid, d.n_here - 1);
            ep_tok = a.idx[p];
            if (KIND == 2) {
                ep_w = a.w[p];
                ep_sc = a.ascale[p];
            } else {
                ep_sc = a.ascale[ep_tok];   // waits for the token id here, once per tile
            }
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

    // Positions run through four activation slots without a workgroup barrier: each wave stores
    // its share of position P + 2 at the end of position P and then counts the fill; position Q is
    // read from slot Q % 4 once every wave has stored its share (the slot's count reaches
    // 8 (Q / 4 + 1)). A wave reading Q thus knows every wave has finished Q - 2, so waves drift at
    // most two positions apart, and the slot a wave overwrites at the end of P (last read at
    // P - 2) is no longer read by anyone. The epilogue operands of tile T are published with T's
    // sequence number (per tile parity) and awaited before the epilogue. Every wait is bounded:
    // it gives up after a.wait_limit polls (2^16 by default; no configuration comes near; it
    // keeps a lost fill from hanging the GPU) and then sets gs_wait_expired.
    int b = 0, buf = 0, tpar = 0;
    uint32_t pos = 0, tseq = 0;
    // The count (or sequence number) is read relaxed and followed by an acquire fence on LDS at
    // workgroup scope; the writer's release fence on LDS precedes its increment (store), so a
    // wave that sees the count also sees the stores it counts. a.wait_force (set only by the
    // host's test hook) makes the target unreachable, so every wait runs to its limit.
    const uint32_t wlim = a.wait_limit, wadd = a.wait_force ? 0x40000000u : 0u;
    bool waited = false;   // the last wait found its count short (this wave was ahead)
    auto wait_lds = [&](const uint32_t *c, uint32_t want, bool eq) __attribute__((always_inline)) {
        want += wadd;
        waited = false;
        for (uint32_t spin = 0;; spin++) {
            const uint32_t v = __hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (eq ? v == want : v >= want) break;
            waited = true;
            if (spin >= wlim) {   // expired: recorded, and the wave goes on (never hangs)
                if (lane == 0) __hip_atomic_fetch_or(&gs_wait_expired, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };
    auto wait_count = [&](const uint32_t *c, uint32_t want) __attribute__((always_inline)) { wait_lds(c, want, false); };
    auto wait_seq = [&](const uint32_t *c, uint32_t want) __attribute__((always_inline)) { wait_lds(c, want, true); };
    auto wait_slot = [&]() __attribute__((always_inline)) {
        if (pos > 1) wait_count(&M.cnt[buf], (uint32_t)(NTH / 64) * (pos / 4u + 1u));
    };
    auto step = [&](WRegs &wu, WRegs &wl) __attribute__((always_inline)) -> bool {
        wait_slot();
        // Issue priority follows the lag: every wave stores its share of each slot, so the
        // workgroup runs at the pace of its slowest wave. A wave that found its slot already
        // filled is that wave (the others were waiting on it) and takes a higher priority for this
        // position; one that had to wait drops to the lowest. Without this the waves that issue
        // their loads later on each SIMD lost the vector-memory arbitration position after
        // position (phase clocks: 4 of the 8 waves spent 3.6x as long issuing loads, the other 4
        // waited on them): config 5 783 -> 728 us.
        if (waited) __builtin_amdgcn_s_setprio(0);
        else __builtin_amdgcn_s_setprio(2);
        // ---- issue: activations of position +1, weights of position +2 -------------------
        const bool last_sb = b == nsb - 1;
        const bool have1 = !last_sb || has_nxt;
        const bool have2 = b + 2 < nsb || has_nxt;   // position +2 exists (nsb >= 2)
        // Both requests are issued unconditionally (at the end of the tile list they re-read valid
        // data of the current tile and are dropped), so every wait on them is an exact count.
        u4 stg[NLD];
        {
            const bool a_nxt = b + 2 >= nsb;
            int ar[NLD];
#pragma unroll
            for (int k = 0; k < NLD; k++) ar[k] = a_nxt ? ar_nxt[k] : ar_cur[k];
            load_a(ar, a_nxt ? b + 2 - nsb : b + 2, stg);
        }
        {
            const bool in_cur = b + 2 < nsb;
            const bool w_nxt = !in_cur;
            Desc d;
            uint32_t wo[NR];
#pragma unroll
            for (int mt = 0; mt < MATS; mt++) d.wb[mt] = w_nxt ? nxt.wb[mt] : cur.wb[mt];
#pragma unroll
            for (int n = 0; n < NR; n++) wo[n] = w_nxt ? wo_nxt[n] : wo_cur[n];
            load_w(d, wo, in_cur ? b + 2 : b + 2 - nsb, wl);
        }

        // ---- contract position (cur, b) ------------------------------------------------------
        {
            const uint8_t *slab = stage + buf * SLAB;
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
#define GS_GRP_FRAGS(G)                                                                            \
        FragRaw fr[NR][MATS];                                                                      \
        _Pragma("unroll") for (int n = 0; n < NR; n++)                                             \
        _Pragma("unroll") for (int mt = 0; mt < MATS; mt++) {                                      \
            if (IQ3) iq3_frag_fetch<G>(tab, hu ? wu.q[n][mt].z : wu.q[n][mt].x, hu ? wu.q[n][mt].w : wu.q[n][mt].y, \
                                       hu ? wu.sg[n][mt].y : wu.sg[n][mt].x, r16, fr[n][mt]);       \
            else iq2_frag_fetch<G>(tab, hu ? wu.q[n][mt].z : wu.q[n][mt].x, hu ? wu.q[n][mt].w : wu.q[n][mt].y, r16, fr[n][mt]); \
        }                                                                                          \
        _Pragma("unroll") for (int n = 0; n < NR; n++)                                             \
        _Pragma("unroll") for (int mt = 0; mt < MATS; mt++) bf[n][mt] = frag_finish<IQ3>(fr[n][mt]);
#define GS_GRP_STEP(G)                                                                             \
    {                                                                                              \
        h8 bf[NR][MATS];                                                                           \
        GS_GRP_FRAGS(G)                                                                            \
        const int cc = 8 * q + 4 * hu + G;                                                         \
        _Pragma("unroll") for (int tt = 0; tt < NT; tt++)                                          \
            if (tt == 0 || 16 * tt < n_here) {                                                     \
                const h8 av = GS_GRP_AV_LOAD(tt, cc);                                              \
                _Pragma("unroll") for (int n = 0; n < NR; n++)                                     \
                _Pragma("unroll") for (int mt = 0; mt < MATS; mt++)                                \
                    sb[tt][n][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bf[n][mt], sb[tt][n][mt], 0, 0, 0);                     \
            }                                                                                      \
    }
                GS_GRP_STEP(0) GS_GRP_STEP(1) GS_GRP_STEP(2) GS_GRP_STEP(3)
#undef GS_GRP_STEP
            }
#pragma unroll
            for (int n = 0; n < NR; n++)
#pragma unroll
                for (int mt = 0; mt < MATS; mt++) {
                    const float cd = h2f((uint32_t)__builtin_amdgcn_ds_bpermute((j + 16 * (n * MATS + mt)) << 2, (int)wu.dq)) * XS;
#pragma unroll
                    for (int tt = 0; tt < NT; tt++)
                        if (tt == 0 || 16 * tt < n_here) acc[tt][n][mt] += cd * sb[tt][n][mt];
                }
        }

        // ---- tile epilogue: lane holds tokens 16t + 4q + i (i < 4) of row row0 + 16n + j ----
        if (last_sb) {
            wait_seq(&M.ep_seq[tpar], tseq);
#pragma unroll
            for (int tt = 0; tt < NT; tt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int slot = 16 * tt + 4 * q + i;
                    const float sc = M.ep_sc[tpar][slot], wt = M.ep_w[tpar][slot];
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
                                    unsafeAtomicAdd(a.out + (int64_t)M.ep_tok[tpar][slot] * rows + r, wt * (acc[tt][n][0][i] * sc));
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
        if (b == nsb - 2 && tid < MT) {   // read by the epilogue of position nsb-1, after the barrier
            M.ep_tok[tpar][tid] = ep_tok;
            M.ep_w[tpar][tid] = ep_w;
            M.ep_sc[tpar][tid] = ep_sc;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");   // wave 0's stores, then the sequence number
            if (tid == 0) __hip_atomic_store(&M.ep_seq[tpar], tseq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        if (!have1) return false;

        // ---- advance: stage position +2, rotate the weight registers -------------------------
        if (have2) {
            const int sbuf = (buf + 2) & 3;
#pragma unroll
            for (int k = 0; k < NLD; k++)
                if (NCH % NTH == 0 || tid + NTH * k < NCH) *(u4 *)(stage + sbuf * SLAB + dst[k]) = stg[k];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");   // this wave's stores, then the count
            if (lane == 0) __hip_atomic_fetch_add(&M.cnt[sbuf], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        buf = (buf + 1) & 3;
        pos++;
        if (last_sb) {   // enter the next tile; fetch the one after it
            b = 0;
            t += tstep;
            tpar ^= 1;
            tseq++;
            cur = nxt;
#pragma unroll
            for (int n = 0; n < NR; n++) wo_cur[n] = wo_nxt[n];
#pragma unroll
            for (int k = 0; k < NLD; k++) ar_cur[k] = ar_nxt[k];
            has_nxt = t + tstep < total;
            describe(has_nxt ? t + tstep : t, nxt);
            woffs(nxt, wo_nxt);
            arows_raw(nxt, ar_nxt);
            ep_load(cur);
            // (no explicit wait for every outstanding load here: the compiler's own waits for the
            // values fetched here measured 1.4 % faster than draining the weight prefetch per tile)
        } else {
            b++;
        }
        return true;
    };
    for (;;) {
        if (!step(W0, W2)) break;
        if (!step(W1, W0)) break;
        if (!step(W2, W1)) break;
    }
}

#define GS_GRP_KERNEL1(TY, KIND, NT, NR, WV)                                                     \
    extern "C" __global__ void __launch_bounds__(64 * WV)                                       \
        gs_k_grouped_##TY##_##KIND##_##NT##_##NR##_##WV(GroupedArgs a) {                        \
        grouped_body<TY, KIND, NT, NR, WV>(a);                                                  \
    }
#define GS_GRP_KERNEL(KIND, NT, NR, WV) GS_GRP_KERNEL1(16, KIND, NT, NR, WV) GS_GRP_KERNEL1(18, KIND, NT, NR, WV)
// instantiated (kind, NT, NR, waves) tile shapes for IQ2_XXS (16) and IQ3_XXS (18); host.cpp
// grouped_launch keeps the same list
GS_GRP_KERNEL(1, 1, 1, 8)
GS_GRP_KERNEL(1, 1, 2, 8)
GS_GRP_KERNEL(1, 2, 1, 8)
GS_GRP_KERNEL(1, 2, 2, 8)
GS_GRP_KERNEL(1, 1, 1, 16)
GS_GRP_KERNEL(2, 1, 1, 8)
GS_GRP_KERNEL(2, 1, 2, 8)
GS_GRP_KERNEL(2, 1, 4, 8)
GS_GRP_KERNEL(2, 2, 1, 8)
GS_GRP_KERNEL(2, 2, 2, 8)
GS_GRP_KERNEL(2, 2, 4, 8)
GS_GRP_KERNEL(2, 1, 1, 16)
GS_GRP_KERNEL(2, 1, 2, 16)
GS_GRP_KERNEL(2, 2, 1, 16)

// ---------------------------------------------------------------------------------------------
// Activation rows -> f16 MFMA operands: out = f16(x * 2^-E), scale[row] = 2^E, with 2^E the
// power of two that puts the row's largest magnitude in [2^14, 2^15). Where f16(x) is normal this
// is exactly f16(x) (scaling by a power of two commutes with rounding); rows with values beyond
// the f16 range stay finite, and small rows keep full precision. One wave per row, 4 per block.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

extern "C" __global__ void __launch_bounds__(256) gs_k_rows_f16(RowsQArgs a) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.nrows) return;
    const int n8 = a.K / 8;
    const float4 *src = (const float4 *)(a.x + (int64_t)row * a.x_stride);
    uint4 *dst = (uint4 *)(a.out + (int64_t)row * a.K);
    // rows of up to 64 x RQ 8-value pieces (K <= 4096) stay in registers between the max and the
    // conversion, every load issued before the first is needed; longer rows are read twice
    constexpr int RQ = 8;
    float4 r0[RQ], r1[RQ];
    float amax = 0.f;
    const bool held = n8 <= 64 * RQ;
    if (held) {
#pragma unroll
        for (int i = 0; i < RQ; i++) {
            const int u = min(lane + 64 * i, n8 - 1);   // clamped: re-reads a valid piece
            r0[i] = src[2 * u];
            r1[i] = src[2 * u + 1];
        }
#pragma unroll
        for (int i = 0; i < RQ; i++)
            amax = fmaxf(amax, fmaxf(fmaxf(fmaxf(fabsf(r0[i].x), fabsf(r0[i].y)), fmaxf(fabsf(r0[i].z), fabsf(r0[i].w))),
                                     fmaxf(fmaxf(fabsf(r1[i].x), fabsf(r1[i].y)), fmaxf(fabsf(r1[i].z), fabsf(r1[i].w)))));
    } else {
        for (int u = lane; u < n8; u += 64) {
            const float4 f0 = src[2 * u], f1 = src[2 * u + 1];
            amax = fmaxf(amax, fmaxf(fmaxf(fmaxf(fabsf(f0.x), fabsf(f0.y)), fmaxf(fabsf(f0.z), fabsf(f0.w))),
                                     fmaxf(fmaxf(fabsf(f1.x), fabsf(f1.y)), fmaxf(fabsf(f1.z), fabsf(f1.w)))));
        }
    }
    amax = wave_max(amax);
    int E = 0;
    if (amax > 0.f && amax <= 3.4e38f) (void)frexpf(amax, &E);   // amax < 2^E
    E -= 15;
    const float down = ldexpf(1.f, -E);
    if (lane == 0) a.scale[row] = ldexpf(1.f, E);
    auto put = [&](int u, const float4 &f0, const float4 &f1) {
        dst[u] = make_uint4(f2h(f0.x * down) | (f2h(f0.y * down) << 16), f2h(f0.z * down) | (f2h(f0.w * down) << 16),
                            f2h(f1.x * down) | (f2h(f1.y * down) << 16), f2h(f1.z * down) | (f2h(f1.w * down) << 16));
    };
    if (held) {
#pragma unroll
        for (int i = 0; i < RQ; i++)
            if (lane + 64 * i < n8) put(lane + 64 * i, r0[i], r1[i]);
    } else {
        for (int u = lane; u < n8; u += 64) put(u, src[2 * u], src[2 * u + 1]);
    }
}

// The same conversion with one 256-thread workgroup per row, for few long rows (the prompt's
// tokens: 512 rows of 4096 gave 128 four-row blocks, half the CUs and 16 loads in a row per lane).
// The row's largest magnitude is a max, so the result is the one-wave kernel's bit for bit.
extern "C" __global__ void __launch_bounds__(256) gs_k_rows_f16_wg(RowsQArgs a) {
    __shared__ float wmax[4];
    const int t = threadIdx.x, row = blockIdx.x;
    const int n8 = a.K / 8;
    const float4 *src = (const float4 *)(a.x + (int64_t)row * a.x_stride);
    uint4 *dst = (uint4 *)(a.out + (int64_t)row * a.K);
    constexpr int RQ = 4;   // rows of up to 256 x RQ 8-value pieces (K <= 8192) stay in registers
    float4 r0[RQ], r1[RQ];
    float amax = 0.f;
    const bool held = n8 <= 256 * RQ;
    if (held) {
#pragma unroll
        for (int i = 0; i < RQ; i++) {
            const int u = min(t + 256 * i, n8 - 1);   // clamped: re-reads a valid piece
            r0[i] = src[2 * u];
            r1[i] = src[2 * u + 1];
        }
#pragma unroll
        for (int i = 0; i < RQ; i++)
            amax = fmaxf(amax, fmaxf(fmaxf(fmaxf(fabsf(r0[i].x), fabsf(r0[i].y)), fmaxf(fabsf(r0[i].z), fabsf(r0[i].w))),
                                     fmaxf(fmaxf(fabsf(r1[i].x), fabsf(r1[i].y)), fmaxf(fabsf(r1[i].z), fabsf(r1[i].w)))));
    } else {
        for (int u = t; u < n8; u += 256) {
            const float4 f0 = src[2 * u], f1 = src[2 * u + 1];
            amax = fmaxf(amax, fmaxf(fmaxf(fmaxf(fabsf(f0.x), fabsf(f0.y)), fmaxf(fabsf(f0.z), fabsf(f0.w))),
                                     fmaxf(fmaxf(fabsf(f1.x), fabsf(f1.y)), fmaxf(fabsf(f1.z), fabsf(f1.w)))));
        }
    }
    amax = wave_max(amax);
    if ((t & 63) == 0) wmax[t >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int E = 0;
    if (amax > 0.f && amax <= 3.4e38f) (void)frexpf(amax, &E);   // amax < 2^E
    E -= 15;
    const float down = ldexpf(1.f, -E);
    if (t == 0) a.scale[row] = ldexpf(1.f, E);
    auto put = [&](int u, const float4 &f0, const float4 &f1) {
        dst[u] = make_uint4(f2h(f0.x * down) | (f2h(f0.y * down) << 16), f2h(f0.z * down) | (f2h(f0.w * down) << 16),
                            f2h(f1.x * down) | (f2h(f1.y * down) << 16), f2h(f1.z * down) | (f2h(f1.w * down) << 16));
    };
    if (held) {
#pragma unroll
        for (int i = 0; i < RQ; i++)
            if (t + 256 * i < n8) put(t + 256 * i, r0[i], r1[i]);
    } else {
        for (int u = t; u < n8; u += 256) put(u, src[2 * u], src[2 * u + 1]);
    }
}
