// gfx950 quantized GEMM for token batches (gs_gemm: prefill projections, MoE expert groups run
// one expert at a time, MTP verification) -- crates/cuda/kernels/gemm.cu:13-123 semantics:
//
//   Y[n][r] (+)= sum_k f16(deq(W[r][k])) * f16(X[n][k])     f32 accumulation
//
// Dequantized weights and activations are rounded to f16 exactly as the reference's tiles are
// (round to nearest even); the products run on v_mfma_f32_16x16x32_f16.
//
// Tile: 128 weight rows x 64 tokens per workgroup of 8 waves; a wave owns 16 rows (one MFMA
// column block) and all 64 tokens (four 16-token row blocks): 4 accumulators, each B fragment
// (weights) feeds 4 MFMAs. The K loop steps one 256-element super-block at a time:
//   * raw weight bytes of the tile's rows (one super-block each) are copied into LDS with 16-byte
//     loads (one buffer resource per tile, so the tail of the last row reads zeros, never past
//     the matrix) and shifted to a 4-byte aligned slot; each lane then decodes its own two
//     32-element units of its row from LDS with the exact unit decoders (exact.h) and rounds them
//     to f16;
//   * X rows are converted to f16 into LDS, 512 bytes per token row, 16-byte
//     chunk c of token i at chunk position c ^ (i & 15) so the 16 lanes reading one chunk column
//     hit distinct banks;
//   * the K order inside a super-block is permuted so a lane's B fragments come from whole units:
//     lane quarter q (lane >> 4) owns units 2q and 2q+1, MFMA m (0..7) takes 8-element group m&3
//     of unit 2q + (m>>2); the A fragments use the same permutation, so each dot product is
//     unchanged.
// Plain formats (F32, F16, BF16) skip the LDS copy: a lane reads its units straight from memory.
// Workgroup order: the token blocks of one row block run back to back on one XCD (workgroup w
// is dispatched to XCD w % 8), so the row block's weights come from that XCD's L2 after the first.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "kargs.h"
#include "formats.h"

typedef _Float16 gh8 __attribute__((ext_vector_type(8)));
typedef float gf4 __attribute__((ext_vector_type(4)));

#define GM_NR 1     // 16-row MFMA column blocks per wave
#define GM_RB 128   // weight rows per workgroup (GM_WV waves x GM_NR x 16)
#define GM_WV (GM_RB / (16 * GM_NR))
#define GM_NTH (64 * GM_WV)
static_assert(GM_NTH == GS_GEMM_THREADS, "host launch width");
#define GM_TN 64    // tokens per workgroup (4 x 16)

template <bool B> struct BoolC { static constexpr bool value = B; };

// fills of the two LDS buffers of the double-buffered steps: buffer s has been stored by
// gm_fill[s] waves so far
__shared__ uint32_t gm_fill[2];

// Sticky expiry flag of this code object's bounded LDS waits (host.cpp gs_wait_status reads and
// clears it): nonzero once any wait gave up before its count arrived.
__device__ uint32_t gs_wait_expired;

// 8 floats -> 8 halves (round to nearest even, as __floats2half2_rn)
// (a vector conversion: v_cvt_pk_f16_f32, two values per instruction, round to nearest even)
typedef float gf8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ gh8 to_h8(const float *v) {
    const gf8 f = {v[0], v[1], v[2], v[3], v[4], v[5], v[6], v[7]};
    return __builtin_convertvector(f, gh8);
}

template <int QKB, int BB, void (*DEC)(const uint8_t *, int, float (&)[32])>
struct GemmFmt {
    static constexpr bool PLAIN = QKB == 1;
    // bytes of one 256-element super-block of a row
    static constexpr int SB = QKB == 1 ? 256 * BB : 256 / QKB * BB;
    // LDS slot: the super-block realigned to the slot start (the copy reads from the 4-byte
    // boundary at or below the block and shifts the bytes into place), so every decoder sees a
    // 4-byte aligned block and its byte reads merge into dword reads. An odd number of dwords:
    // the 16 rows a wave decodes side by side then start in 16 different banks (a multiple of 16
    // bytes put rows 4 apart in one bank, and the lane quarters' units 32 bytes apart on top of
    // them: 16-way conflicts on every read)
    static constexpr int SBP = 4 * (((SB + 3) / 4) | 1);
    // exact decode of 32-element unit u (0..7) of a super-block starting at p
    __device__ static __forceinline__ void unit(const uint8_t *p, int u, float (&v)[32]) {
        if (QKB == 256) DEC(p, u, v);
        else if (QKB == 32) DEC(p + u * BB, 0, v);
        else DEC(p + 32 * u * BB, 0, v);
    }
    // the same from the dword-aligned LDS slot: the dword decoders where the format has one
    __device__ static __forceinline__ void slot_unit(const uint8_t *p, int u, float (&v)[32]) {
        if constexpr (DEC == &exact::q8_0) exact::al::q8_0(p, u, v);
        else if constexpr (DEC == &exact::q4_k) exact::al::q4_k(p, u, v);
        else if constexpr (DEC == &exact::q6_k) exact::al::q6_k(p, u, v);
        else unit(p, u, v);
    }
};

template <int QKB, int BB, void (*DEC)(const uint8_t *, int, float (&)[32]), int GM_NBUF>
__device__ __forceinline__ void gemm_body(const GemmArgs &a) {
    using F = GemmFmt<QKB, BB, DEC>;
    constexpr int CPR = F::PLAIN ? 1 : (F::SBP + 15) / 16;          // raw 16-byte chunks per row
    constexpr int NRAW = F::PLAIN ? 1 : (GM_RB * CPR + GM_NTH - 1) / GM_NTH;
    constexpr int RAWB = F::PLAIN ? 16 : GM_RB * F::SBP;            // one raw buffer
    constexpr int ASLAB = GM_TN * 512;                              // one f16 activation buffer
    constexpr int NXA = GM_TN * 32 / GM_NTH;                        // 16-byte A chunks per thread (8)
    extern __shared__ __align__(16) uint8_t gm_lds[];
    uint8_t *const rawbuf = gm_lds;
    uint8_t *const abuf = gm_lds + GM_NBUF * RAWB;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, q = lane >> 4;
    // workgroup -> (row block, token block): row block r on XCD r % 8, its token blocks in a row
    const int L = blockIdx.x, xcd = L & 7, k8 = L >> 3;
    const int rblk = xcd + 8 * (k8 / a.n_tb), tblk = k8 % a.n_tb;
    if (rblk >= a.n_rb) return;
    const int z = blockIdx.y;
    const uint8_t *W = a.W + (int64_t)z * a.w_bs;
    const float *X = a.X + (int64_t)z * a.x_bs;
    float *Y = a.Y + (int64_t)z * a.y_bs;
    const int K = a.K, rows = a.rows, N = a.N, nsb = K / 256 + (K % 256 != 0);
    // K slice (blockIdx.z): super-blocks [kb0, kb1)
    const int ks = blockIdx.z, kb0 = ks * a.ksb, kb1 = min(nsb, kb0 + a.ksb);
    const int r0 = rblk * GM_RB, n0 = tblk * GM_TN;
    const int nrows = min(GM_RB, rows - r0), ntok = min(GM_TN, N - n0);
    const int64_t rs = a.row_stride;

    // raw copy: chunk z = tid + GM_NTH*i -> tile row z / CPR, chunk z % CPR, read from the row's
    // super-block start rounded down to 4 bytes; one buffer resource per tile bounded at the tile's
    // last valid byte
    const int64_t row_bytes = (int64_t)(K / QKB) * BB;
    // the resource starts at the 4-byte boundary at or below the tile's first row (d0 bytes
    // before it) and ends at the 4-byte boundary at or above its last byte: every read is
    // dword-aligned and the range check passes every dword that holds a byte of the tile
    const uint8_t *tile = W + (int64_t)r0 * rs;
    const uint32_t d0 = (uint32_t)((uintptr_t)tile & 3u);
    const BufferAt wt(tile - d0, 0,
                      F::PLAIN ? 0u : (uint32_t)((d0 + (int64_t)(nrows - 1) * rs + row_bytes + 3) & ~(int64_t)3));
    uint32_t roff[NRAW];
    int rdst[NRAW], rcap[NRAW];
#pragma unroll
    for (int i = 0; i < NRAW; i++) {
        const int zc = tid + GM_NTH * i, rr = min(zc / CPR, nrows - 1), c = zc % CPR;
        roff[i] = d0 + (uint32_t)((int64_t)rr * rs) + 16u * c;
        rdst[i] = zc < GM_RB * CPR ? (zc / CPR) * F::SBP + 16 * c : -1;
        rcap[i] = F::SBP - 16 * c;   // bytes of the slot from this chunk on
    }
    // chunk i of super-block b: 20 bytes from the dword boundary at or below its first byte
    auto raw_load = [&](int b, uint4 (&rv)[NRAW], uint32_t (&rx)[NRAW]) {
        if constexpr (!F::PLAIN) {
#pragma unroll
            for (int i = 0; i < NRAW; i++) {
                const uint32_t o = (roff[i] + (uint32_t)(F::SB * b)) & ~3u;
                rv[i] = wt.u128(o);
                rx[i] = wt.u32(o + 16);
            }
        }
    };
    // the chunk shifted by the block's misalignment (v_alignbyte), as dword stores (slots are
    // 4-byte aligned), none past the slot
    auto raw_store = [&](int buf, int b, const uint4 (&rv)[NRAW], const uint32_t (&rx)[NRAW]) {
        if constexpr (!F::PLAIN) {
#pragma unroll
            for (int i = 0; i < NRAW; i++)
                if (rdst[i] >= 0) {
                    const uint32_t lead = (roff[i] + (uint32_t)(F::SB * b)) & 3u;
                    uint32_t *d = (uint32_t *)(rawbuf + buf * RAWB + rdst[i]);
                    const int room = rcap[i];
                    d[0] = __builtin_amdgcn_alignbyte(rv[i].y, rv[i].x, lead);
                    if (room > 4) d[1] = __builtin_amdgcn_alignbyte(rv[i].z, rv[i].y, lead);
                    if (room > 8) d[2] = __builtin_amdgcn_alignbyte(rv[i].w, rv[i].z, lead);
                    if (room > 12) d[3] = __builtin_amdgcn_alignbyte(rx[i], rv[i].w, lead);
                }
        }
    };
    // activations: A chunk y = tid + GM_NTH*i -> token row y >> 5, 8-element chunk y & 31
    // unconditional loads (a clamped address past the tokens or the row; zeroed at the store), so
    // the compiler's waits for them stay exact counts instead of draining at a branch
    auto x_load = [&](int b, float4 (&xv)[NXA][2]) {
#pragma unroll
        for (int i = 0; i < NXA; i++) {
            const int y = tid + GM_NTH * i, t = y >> 5, c = y & 31;
            const int kk = min(256 * b + 8 * c, K - 8);
            const float4 *p = (const float4 *)(X + (int64_t)(n0 + min(t, ntok - 1)) * a.x_stride + kk);
            xv[i][0] = p[0];
            xv[i][1] = p[1];
        }
    };
    auto x_store = [&](int buf, int b, const float4 (&xv)[NXA][2]) {
        auto put = [&](auto masked) {
#pragma unroll
            for (int i = 0; i < NXA; i++) {
                const int y = tid + GM_NTH * i, t = y >> 5, c = y & 31;
                const bool ok = !decltype(masked)::value || (t < ntok && 256 * b + 8 * c < K);
                const float f[8] = {ok ? xv[i][0].x : 0.f, ok ? xv[i][0].y : 0.f, ok ? xv[i][0].z : 0.f,
                                    ok ? xv[i][0].w : 0.f, ok ? xv[i][1].x : 0.f, ok ? xv[i][1].y : 0.f,
                                    ok ? xv[i][1].z : 0.f, ok ? xv[i][1].w : 0.f};
                *(gh8 *)(abuf + buf * ASLAB + t * 512 + ((c ^ (t & 15)) << 4)) = to_h8(f);
            }
        };
        // masking only where the tile has missing tokens or the row ends inside the step (a
        // workgroup-uniform branch)
        if (ntok < GM_TN || 256 * (b + 1) > K) put(BoolC<true>{});
        else put(BoolC<false>{});
    };

    gf4 acc[4][GM_NR];
#pragma unroll
    for (int tt = 0; tt < 4; tt++)
#pragma unroll
        for (int n = 0; n < GM_NR; n++) acc[tt][n] = gf4{0.f, 0.f, 0.f, 0.f};

    if (GM_NBUF == 2) {   // prologue: super-block 0
        uint4 rv[NRAW];
        uint32_t rx[NRAW];
        float4 xv[NXA][2];
        raw_load(kb0, rv, rx);
        x_load(kb0, xv);
        raw_store(0, kb0, rv, rx);
        x_store(0, kb0, xv);
        if (tid < 2) gm_fill[tid] = tid == 0 ? GM_WV : 0u;   // buffer 0: step 0, stored by every wave
        __syncthreads();
    }
    // Double-buffered steps without a workgroup barrier: step b is read from buffer b & 1 once
    // every wave has stored its share of it (the buffer's fill count reaches GM_WV (b / 2 + 1));
    // each wave stores step b + 1 at the end of step b and then counts the fill. A wave reading
    // step b thus knows every wave has finished computing step b - 1, the last reader of the
    // buffer it overwrites next. The count is read relaxed and followed by an acquire fence on
    // LDS at workgroup scope (the storing wave's release fence precedes its increment). The wait
    // is bounded (a.wait_limit polls, 2^16 by default; it keeps a lost fill from hanging the GPU)
    // and an expiry sets gs_wait_expired; a.wait_force (the host's test hook) makes the count
    // unreachable so the wait runs to its limit.
    auto wait_fill = [&](int b) __attribute__((always_inline)) {
        const uint32_t want = (uint32_t)GM_WV * (uint32_t)(b / 2 + 1) + (a.wait_force ? 0x40000000u : 0u);
        for (uint32_t spin = 0;; spin++) {
            if (__hip_atomic_load(&gm_fill[b & 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= want) break;
            if (spin >= a.wait_limit) {
                if (lane == 0) __hip_atomic_fetch_or(&gs_wait_expired, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };

    const int ntt = (ntok + 15) >> 4;   // token row blocks with any token (wave-uniform)
    for (int b = kb0; b < kb1; b++) {
        const int bl = b - kb0;   // step within the slice (buffer parity, fill counts)
        const int buf = GM_NBUF == 2 ? bl & 1 : 0;
        const bool more = GM_NBUF == 2 && b + 1 < kb1;
        uint4 rv[NRAW];
        uint32_t rx[NRAW];
        float4 xv[NXA][2];
        if (GM_NBUF == 1) {
            // one buffer: the other workgroup on the CU computes while this one loads
            if (bl > 0) __syncthreads();   // every wave is done with step b-1
            raw_load(b, rv, rx);
            x_load(b, xv);
            raw_store(0, b, rv, rx);
            x_store(0, b, xv);
            __syncthreads();
        } else {
            // next super-block in flight while this one is decoded and contracted (issued on the
            // last step too, re-reading that step's data, so every wait on them is an exact count)
            raw_load(more ? b + 1 : b, rv, rx);
            x_load(more ? b + 1 : b, xv);
            if (bl > 0) wait_fill(bl);
        }
        // B fragments: units 2q, 2q+1 of this lane's two rows, rounded to f16
        // (the step that ends past the row, K % 256 != 0, is a workgroup-uniform second path, so
        // the others carry no masking)
        // Per unit hu: decode (B fragments of unit 2q + hu, rounded to f16), then the four MFMAs of
        // each token block that take it (MFMA m takes group m & 3 of unit 2q + (m >> 2)). Each
        // (full tile, step inside the row) combination is one straight-line block, so the matrix
        // core runs unit 0's products while the VALU decodes unit 1. A partial tile guards each
        // token block (a per-MFMA branch serializes each fragment read with its MFMA, so full
        // tiles have none); the step that ends past the row (K % 256 != 0) zeroes those units.
        const uint8_t *slab = abuf + buf * ASLAB;
        auto compute = [&](auto full, auto tail) __attribute__((always_inline)) {
#pragma unroll
            for (int hu = 0; hu < 2; hu++) {
                gh8 bf[GM_NR][4];
#pragma unroll
                for (int n = 0; n < GM_NR; n++) {
                    const int rr = min(wave * 16 * GM_NR + 16 * n + j, nrows - 1);
                    const bool past = decltype(tail)::value && 256 * b + 32 * (2 * q + hu) >= K;
                    float v[32];
                    if constexpr (F::PLAIN) {   // straight from memory: nothing is read past the row
                        if (past) {
#pragma unroll
                            for (int e = 0; e < 32; e++) v[e] = 0.f;
                        } else {
                            F::unit(W + (int64_t)(r0 + rr) * rs + (int64_t)256 * b * BB, 2 * q + hu, v);
                        }
                    } else {   // the LDS slot is always readable: decode, then zero what is past the row
                        F::slot_unit((const uint8_t *)__builtin_assume_aligned(rawbuf + buf * RAWB + rr * F::SBP, 4), 2 * q + hu, v);
                    }
#pragma unroll
                    for (int g = 0; g < 4; g++) bf[n][g] = past ? gh8{} : to_h8(v + 8 * g);
                }
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    const int cc = 8 * q + 4 * hu + g;
                    gh8 av[4];
#pragma unroll
                    for (int tt = 0; tt < 4; tt++)
                        if (decltype(full)::value || tt < ntt) av[tt] = *(const gh8 *)(slab + (16 * tt + j) * 512 + ((cc ^ j) << 4));
#pragma unroll
                    for (int tt = 0; tt < 4; tt++)
                        if (decltype(full)::value || tt < ntt)
#pragma unroll
                            for (int n = 0; n < GM_NR; n++)
                                acc[tt][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[tt], bf[n][g], acc[tt][n], 0, 0, 0);
                }
            }
        };
        const bool tail = 256 * (b + 1) > K;   // workgroup-uniform
        if (ntt == 4 && !tail) compute(BoolC<true>{}, BoolC<false>{});
        else if (!tail) compute(BoolC<false>{}, BoolC<false>{});
        else compute(BoolC<false>{}, BoolC<true>{});
        if (more) {
            raw_store(buf ^ 1, b + 1, rv, rx);
            x_store(buf ^ 1, b + 1, xv);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");   // this wave's stores, then the count
            if (lane == 0) __hip_atomic_fetch_add(&gm_fill[buf ^ 1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }

    // lane holds tokens 16tt + 4q + i of row 32 wave + 16n + j
#pragma unroll
    for (int tt = 0; tt < 4; tt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 16 * tt + 4 * q + i;
            if (t < ntok) {
#pragma unroll
                for (int n = 0; n < GM_NR; n++) {
                    const int rr = wave * 16 * GM_NR + 16 * n + j;
                    if (rr < nrows) {
                        if (a.part) {   // K slice: its partial, summed in slice order by gs_k_gemm_reduce
                            a.part[((int64_t)(ks * gridDim.y + z) * N + n0 + t) * rows + r0 + rr] = acc[tt][n][i];
                        } else {
                            float *dst = Y + (int64_t)(n0 + t) * a.y_stride + r0 + rr;
                            *dst = a.accumulate ? *dst + acc[tt][n][i] : acc[tt][n][i];
                        }
                    }
                }
            }
        }
}

#define GS_GEMM_KERNEL(TY, QKB, BB, DEC)                                                          \
    extern "C" __global__ void __launch_bounds__(GM_NTH, 3 - gs_gemm_nbuf(TY)) gs_k_gemm_##TY(GemmArgs a) {    \
        gemm_body<QKB, BB, DEC, gs_gemm_nbuf(TY)>(a);                                            \
    }
GS_TYPE_LIST(GS_GEMM_KERNEL)

// Y[z][n][r] (+)= sum over K slices s = 0, 1, ... of part[s][z][n][r], in slice order (a fixed
// order: the result does not depend on which slice finished first)
extern "C" __global__ void __launch_bounds__(256) gs_k_gemm_reduce(GemmReduceArgs a) {
    const int64_t per = (int64_t)a.N * a.rows, total = per * a.n_batch;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
        float v[GS_GEMM_KS_MAX];   // every slice's load issued before the first add
#pragma unroll
        for (int s = 0; s < GS_GEMM_KS_MAX; s++) v[s] = s < a.nks ? a.part[(int64_t)s * total + i] : 0.f;
        float sum = v[0];
#pragma unroll
        for (int s = 1; s < GS_GEMM_KS_MAX; s++)
            if (s < a.nks) sum += v[s];
        const int64_t z = i / per, rem = i - z * per, n = rem / a.rows, r = rem - n * a.rows;
        float *dst = a.Y + z * a.y_bs + n * a.y_stride + r;
        *dst = a.accumulate ? *dst + sum : sum;
    }
}
