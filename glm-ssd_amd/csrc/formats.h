// gfx950 device-side decoders of the ggml block formats.
//
// Two families:
//   * exact::* (exact.h): exact dequantization of one 32-element unit, bit-identical to the CPU
//               reference (crates/quants/src/lib.rs:131-343). Used by gs_dequant_* and by
//               gs_gemm's tiles.
//   * F*::load/dot : the streaming kernels' paths, one per format (F32, F16, BF16, Q8_0, Q2_K,
//               Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ2_S, IQ3_XXS, IQ4_XS). load() fetches one
//               32-element "unit" of a weight row straight from HBM into registers; dot() decodes it
//               and dots it with up to NV activation units held in registers (q8_1 with
//               v_dot4_i32_i8 for the quantized formats, f32 for the plain ones), applying the
//               block scales in f32.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "kargs.h"

// ---- small helpers --------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint32_t h) {
    _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
    return (float)v;
}
__device__ __forceinline__ uint32_t f2h(float f) { // round to nearest even (v_cvt_f16_f32)
    _Float16 v = (_Float16)f;
    return (uint32_t)__builtin_bit_cast(uint16_t, v);
}
// byte-wise little-endian reads through any pointer (global or LDS), no alignment needed
__device__ __forceinline__ uint32_t rb8(const uint8_t *p, int i) { return p[i]; }
__device__ __forceinline__ uint32_t rb16(const uint8_t *p, int i) { return (uint32_t)p[i] | ((uint32_t)p[i + 1] << 8); }
__device__ __forceinline__ uint32_t rb32(const uint8_t *p, int i) {
    return (uint32_t)p[i] | ((uint32_t)p[i + 1] << 8) | ((uint32_t)p[i + 2] << 16) | ((uint32_t)p[i + 3] << 24);
}

// ggml tables live in the code object's read-only data
#include "ggml_grids.h"

// ksigns_iq2xs[i] == i | parity(i) << 7  (closed form of crates/quants/src/tables.rs:9-18)
__device__ __forceinline__ uint32_t ksigns(uint32_t i) { return i | ((__builtin_popcount(i) & 1u) << 7); }

__device__ __forceinline__ uint32_t ksigns_of(uint32_t i) { return ksigns(i); }
#include "exact.h"

// =============================================================================================
// Fast unit dot products against q8_1 activations
// =============================================================================================
// One q8_1 activation unit (32 elements) in registers.
struct XU {
    uint32_t q[8];   // int8 x 32
    uint32_t nq[8];  // -q per byte (only formats with NEG_X read it)
    float D;         // f16-rounded scale (x the routing weight for MoE down, x the format's XSCALE);
                     // formats with f32 activations: the routing weight alone
    int slo, shi;    // sum of q over elements 0..15 / 16..31
    const float *xs; // formats with f32 activations: the unit's 32 floats in LDS
};
// Traits defaults: formats opt in to negated activations / a folded constant scale.
template <class F, class = void> struct NegX { static constexpr bool value = false; };
template <class F> struct NegX<F, decltype((void)F::NEG_X, void())> { static constexpr bool value = F::NEG_X; };
template <class F, class = void> struct F32Act { static constexpr bool value = false; };
template <class F> struct F32Act<F, decltype((void)F::F32X, void())> { static constexpr bool value = F::F32X; };
template <class F, class = void> struct XScale { static constexpr float value = 1.0f; };
template <class F> struct XScale<F, decltype((void)F::XSCALE, void())> { static constexpr float value = F::XSCALE; };

// Formats without lookup tables: empty table hooks.
struct NoTable {
    struct TabReg {};
    __device__ static __forceinline__ void tab_load(int, TabReg &) {}
    __device__ static __forceinline__ void tab_store(int, const TabReg &) {}
};

// Per-format geometry of a unit (32 elements) within a row: byte offset of its block and the
// unit index inside that block.
template <int QK, int BB>
struct UnitGeom {
    static constexpr int UPB = QK >= 32 ? QK / 32 : 1;   // units per block
    __device__ static __forceinline__ uint32_t off(int u) {
        return QK >= 32 ? (uint32_t)(u / UPB) * BB : (uint32_t)u * (32 / QK) * BB;
    }
    __device__ static __forceinline__ int sub(int u) { return QK >= 32 ? u % UPB : 0; }
};

__device__ __forceinline__ int dot8(const uint32_t (&w)[8], const uint32_t (&q)[8]) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) s = __builtin_amdgcn_sdot4((int)w[i], (int)q[i], s, false);
    return s;
}

// Unaligned loads straight from HBM: every block field is 2-byte aligned and gfx950 serves
// unaligned global loads (the driver runs the GPU in unaligned-access mode), so a lane reads its
// unit's bytes with one 8- or 16-byte load whatever the block size.
// The weights are always in global memory: the address-space cast makes these global_load
// (not flat_load, which would also count against the LDS wait counter and defeat exact waits).
#define GS_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ T ldg(const uint8_t *p) { return *(const GS_GLOBAL T *)(const GS_GLOBAL uint8_t *)p; }
// Wide unaligned loads are written as dword loads that the backend merges into one
// global_load_dwordx2/x4; a direct 8/16-byte load at 2-byte alignment is lowered to flat_load.
__device__ __forceinline__ uint32_t ldg4(const uint8_t *p) { return ldg<uint32_t>(p); }
__device__ __forceinline__ uint2 ldg8(const uint8_t *p) { return make_uint2(ldg4(p), ldg4(p + 4)); }
__device__ __forceinline__ uint4 ldg16(const uint8_t *p) { return make_uint4(ldg4(p), ldg4(p + 4), ldg4(p + 8), ldg4(p + 12)); }
__device__ __forceinline__ uint32_t ldg2(const uint8_t *p) { return ldg<uint16_t>(p); }

// Weight byte accessors for the formats' load(): GlobalAt reads base + offset with global loads;
// BufferAt reads through a buffer resource built from a wave-uniform base, so every load is
// SGPR resource + 32-bit lane offset (no per-load 64-bit address arithmetic). Offsets are bytes,
// 2-byte aligned; both serve unaligned 4/8/16-byte reads.
struct GlobalAt {
    const uint8_t *b;
    __device__ __forceinline__ uint32_t u16(uint32_t o) const { return ldg2(b + o); }
    __device__ __forceinline__ uint32_t u32(uint32_t o) const { return ldg4(b + o); }
    __device__ __forceinline__ uint2 u64(uint32_t o) const { return ldg8(b + o); }
    __device__ __forceinline__ uint4 u128(uint32_t o) const { return ldg16(b + o); }
    __device__ __forceinline__ const uint8_t *ptr(uint32_t o) const { return b + o; }
};
struct BufferAt {
    __amdgpu_buffer_rsrc_t r;
    const uint8_t *b;
    uint32_t so;   // wave-uniform offset added to every access (the scalar offset operand)
    // nrec: the resource's size in bytes; 0 makes every access out of range, so a load is
    // issued (and counted) but reads no memory and returns zeros
    __device__ __forceinline__ explicit BufferAt(const uint8_t *base, uint32_t soff = 0, uint32_t nrec = 0xffffffffu)
        : r(__builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)nrec, 0x00020000)), b(base), so(soff) {}
    __device__ __forceinline__ uint32_t u16(uint32_t o) const { return __builtin_amdgcn_raw_buffer_load_b16(r, o, so, 0); }
    __device__ __forceinline__ uint32_t u32(uint32_t o) const { return __builtin_amdgcn_raw_buffer_load_b32(r, o, so, 0); }
    __device__ __forceinline__ uint2 u64(uint32_t o) const {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, o, so, 0);
        return make_uint2(v[0], v[1]);
    }
    __device__ __forceinline__ uint4 u128(uint32_t o) const {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, o, so, 0);
        return make_uint4(v[0], v[1], v[2], v[3]);
    }
    __device__ __forceinline__ const uint8_t *ptr(uint32_t o) const { return b + so + o; }
};

// Each format: Raw = the registers one unit needs from memory; load() issues the loads for unit
// `j` of the block at byte offset o of an accessor (GlobalAt / BufferAt); dot() decodes Raw and accumulates r[t] += W_unit . x_t for t < nv.
struct FQ8_0 : UnitGeom<32, 34>, NoTable {
    static constexpr int TYPE = GS_Q8_0, QK = 32, BB = 34, TAB = 0, RAW = 9;
    struct Raw { uint4 lo, hi; uint32_t d; };
    template <class M>
    __device__ static __forceinline__ void load(const M &m, uint32_t o, int, Raw &w) {
        w.d = m.u16(o);
        w.lo = m.u128(o + 2);
        w.hi = m.u128(o + 18);
    }
    template <int NV, bool XNEG = false>
    __device__ static __forceinline__ void dot(const Raw &w, int, const uint8_t *, const XU (&x)[NV], int nv,
                                               float (&r)[NV]) {
        const float d = h2f(w.d);
        const uint32_t q[8] = {w.lo.x, w.lo.y, w.lo.z, w.lo.w, w.hi.x, w.hi.y, w.hi.z, w.hi.w};
#pragma unroll
        for (int t = 0; t < NV; t++)
            if (NV == 1 || t < nv) r[t] += (d * x[t].D) * (float)dot8(q, x[t].q);
    }
};

// Q8_0 with aligned loads (FQ8_0A: the one-vector GEMV over many rows). The 34-byte blocks put
// every other block's quants at a 2-byte aligned address, and 16-byte loads there stream about a
// third slower than 4-byte aligned ones (measured: 4.9 against 6.5 TB/s over 1 GiB). A lane's unit
// pair (two consecutive blocks) therefore reads each unit's 32 quant bytes as the 36-byte
// dword-aligned window around them (two 16-byte loads and one 4-byte load) and shifts them into
// place (v_alignbyte); the shift (0 or 2 bytes) rides in the high half of the scale word. That
// costs 8 more VALU per unit and 8 load instructions per pair instead of 6, so a GEMV with few
// rows per wave (4096 x 4096) stays on FQ8_0. Nothing past the pair's 68 bytes is read but the
// rest of the dword holding its last two bytes (4-byte aligned, so never on another page); a
// window whose last dword is not needed (no shift) repeats the one before it instead.
struct FQ8_0A : UnitGeom<32, 34>, NoTable {
    static constexpr int TYPE = GS_Q8_0, QK = 32, BB = 34, TAB = 0, RAW = 10;
    struct Raw { uint4 lo, hi; uint32_t x8, d; };   // d: f16 scale | byte shift << 16
    template <class M>
    __device__ static __forceinline__ void load(const M &m, uint32_t o, int, Raw &w) {
        w.d = m.u16(o);
        w.lo = m.u128(o + 2);
        w.hi = m.u128(o + 18);
        w.x8 = 0;
    }
    static constexpr bool PAIR = true;
    template <class M>
    __device__ static __forceinline__ void load2(const M &m, uint32_t o, int, Raw &w0, Raw &w1) {
        const uint32_t a = (uint32_t)(uintptr_t)m.ptr(o) & 3u;   // 0 or 2: rows are 2-byte aligned
        const uint32_t s0 = (a + 2u) & 3u, s1 = a;                 // shifts of the quants at o+2, o+36
        const uint32_t o0 = o + 2u - s0, o1 = o + 36u - s1;        // their 4-byte aligned windows
        w0.d = m.u16(o) | (s0 << 16);
        w1.d = m.u16(o + 34u) | (s1 << 16);
        w0.lo = m.u128(o0);
        w0.hi = m.u128(o0 + 16u);
        w0.x8 = m.u32(o0 + (s0 ? 32u : 28u));
        w1.lo = m.u128(o1);
        w1.hi = m.u128(o1 + 16u);
        w1.x8 = m.u32(o1 + (s1 ? 32u : 28u));
    }
    template <int NV, bool XNEG = false>
    __device__ static __forceinline__ void dot(const Raw &w, int, const uint8_t *, const XU (&x)[NV], int nv,
                                               float (&r)[NV]) {
        const float d = h2f(w.d & 0xffffu);
        const uint32_t sh = w.d >> 16;
        const uint32_t dw[9] = {w.lo.x, w.lo.y, w.lo.z, w.lo.w, w.hi.x, w.hi.y, w.hi.z, w.hi.w, w.x8};
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = __builtin_amdgcn_alignbyte(dw[i + 1], dw[i], sh);
#pragma unroll
        for (int t = 0; t < NV; t++)
            if (NV == 1 || t < nv) r[t] += (d * x[t].D) * (float)dot8(q, x[t].q);
    }
};

// Q8_0 over rows that start 4-byte aligned (FQ8_0A4): a lane's unit pair then always starts
// aligned (68 bytes per pair), so the pair is read as 17 aligned dwords (four 16-byte loads and
// one 4-byte load, where FQ8_0 issues six loads, four of them 2-byte aligned): unit 0 (sub 0)
// keeps dwords 0..8 (its scale in the low half of dword 0, its quants 2 bytes in, shifted into
// place with v_alignbyte), unit 1 dwords 9..16 (its quants aligned) and dword 8 (its scale in the
// high half). No byte outside the pair is read.
struct FQ8_0A4 : UnitGeom<32, 34>, NoTable {
    static constexpr int TYPE = GS_Q8_0, QK = 32, BB = 34, TAB = 0, RAW = 9;
    struct Raw { uint4 lo, hi; uint32_t x8; };
    __device__ static __forceinline__ int sub(int u) { return u & 1; }   // the unit's place in its pair
    template <class M>
    __device__ static __forceinline__ void load(const M &m, uint32_t o, int s, Raw &w) {
        if (s == 0) {   // o 4-byte aligned
            w.lo = m.u128(o);
            w.hi = m.u128(o + 16);
            w.x8 = m.u32(o + 32);
        } else {        // o 2 bytes past a multiple of 4: quants at o+2 aligned, scale to the high half
            w.lo = m.u128(o + 2);
            w.hi = m.u128(o + 18);
            w.x8 = m.u16(o) << 16;
        }
    }
    static constexpr bool PAIR = true;
    template <class M>
    __device__ static __forceinline__ void load2(const M &m, uint32_t o, int, Raw &w0, Raw &w1) {
        w0.lo = m.u128(o);
        w0.hi = m.u128(o + 16);
        const uint4 c = m.u128(o + 32);
        w1.hi = m.u128(o + 48);
        const uint32_t e = m.u32(o + 64);
        w0.x8 = c.x;
        w1.x8 = c.x;
        w1.lo = make_uint4(c.y, c.z, c.w, w1.hi.x);
        w1.hi = make_uint4(w1.hi.y, w1.hi.z, w1.hi.w, e);
    }
    template <int NV, bool XNEG = false>
    __device__ static __forceinline__ void dot(const Raw &w, int s, const uint8_t *, const XU (&x)[NV], int nv,
                                               float (&r)[NV]) {
        const uint32_t dw[9] = {w.lo.x, w.lo.y, w.lo.z, w.lo.w, w.hi.x, w.hi.y, w.hi.z, w.hi.w, w.x8};
        uint32_t q[8];
        float d;
        if (s == 0) {
            d = h2f(w.lo.x & 0xffffu);
#pragma unroll
            for (int i = 0; i < 8; i++) q[i] = __builtin_amdgcn_alignbyte(dw[i + 1], dw[i], 2);
        } else {
            d = h2f(w.x8 >> 16);
#pragma unroll
            for (int i = 0; i < 8; i++) q[i] = dw[i];
        }
#pragma unroll
        for (int t = 0; t < NV; t++)
            if (NV == 1 || t < nv) r[t] += (d * x[t].D) * (float)dot8(q, x[t].q);
    }
};

struct FQ4_K : UnitGeom<256, 144>, NoTable {
    static constexpr int TYPE = GS_Q4_K, QK = 256, BB = 144, TAB = 0, RAW = 12;
    struct Raw { uint4 hd, lo, hi; };   // bytes 0..15 (d, dmin, scales[12]); 32 quant bytes
    template <class M>
    __device__ static __forceinline__ void load(const M &m, uint32_t o, int j, Raw &w) {
        w.hd = m.u128(o);
        w.lo = m.u128(o + 16 + 32 * (uint32_t)(j >> 1));
        w.hi = m.u128(o + 32 + 32 * (uint32_t)(j >> 1));
    }
    template <int NV, bool XNEG = false>
    __device__ static __forceinline__ void dot(const Raw &w, int j, const uint8_t *, const XU (&x)[NV], int nv,
                                               float (&r)[NV]) {
        const float d = h2f(w.hd.x & 0xffff), dmin = h2f(w.hd.x >> 16);
        const uint32_t hs[3] = {w.hd.y, w.hd.z, w.hd.w};
        // byte k of scales[] (crates/quants/src/lib.rs:87-93 scale_min_k4)
        auto sb = [&](int k) -> uint32_t { return (hs[k >> 2] >> (8 * (k & 3))) & 0xff; };
        uint32_t sc, mn;
        if (j < 4) {
            sc = sb(j) & 63;
            mn = sb(j + 4) & 63;
        } else {
            sc = (sb(j + 4) & 0xF) | ((sb(j - 4) >> 6) << 4);
            mn = (sb(j + 4) >> 4) | ((sb(j) >> 6) << 4);
        }
        const int sh = (j & 1) * 4;
        const uint32_t q0[8] = {w.lo.x, w.lo.y, w.lo.z, w.lo.w, w.hi.x, w.hi.y, w.hi.z, w.hi.w};
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = (q0[i] >> sh) & 0x0F0F0F0Fu;
        const float ds = d * (float)sc, dm = dmin * (float)mn;
#pragma unroll
        for (int t = 0; t < NV; t++)
            if (NV == 1 || t < nv) r[t] += x[t].D * (ds * (float)dot8(q, x[t].q) - dm * (float)(x[t].slo + x[t].shi));
    }
};

// Q5_K (lib.rs:221-240): Q4_K's header (d, dmin, 12 bytes of 6-bit scales/mins) and nibbles,
// plus a fifth bit per element: unit j takes nibble j & 1 of the 32 qs bytes at 48 + 32 (j >> 1)
// and bit j of the 32 qh bytes at 16. Units 2i and 2i + 1 read the same 64 bytes, so a lane's
// pair loads them once (load2: 10 registers per unit instead of 20).
struct FQ5_K : UnitGeom<256, 176>, NoTable {
    static constexpr int TYPE = GS_Q5_K, QK = 256, BB = 176, TAB = 0, RAW = 20, RAW2 = 10;
    static constexpr bool PAIR = true, JOINT = true;
    // single unit: a = qs bytes, b = qh bytes, h = header. Pair: w0.a = qs, w0.h = header, w1.a = qh.
    struct Raw { uint4 a0, a1, b0, b1, h; };
    __device__ static __forceinline__ int xunit(int up) { return up; }
    template <class M>
    __device__ static __forceinline__ void load(const M &m, uint32_t o, int j, Raw &w) {
        const uint32_t qs = o + 48 + 32 * ((uint32_t)j >> 1);
        w.h = m.u128(o);
        w.a0 = m.u128(qs);
        w.a1 = m.u128(qs + 16);
        w.b0 = m.u128(o + 16);
        w.b1 = m.u128(o + 32);
    }
    template <class M>
    __device__ static __forceinline__ void load2(const M &m, uint32_t o, int j, Raw &w0, Raw &w1) {
        const uint32_t qs = o + 48 + 32 * ((uint32_t)j >> 1);
        w0.h = m.u128(o);
        w0.a0 = m.u128(qs);
        w0.a1 = m.u128(qs + 16);
        w1.a0 = m.u128(o + 16);
        w1.a1 = m.u128(o + 32);
    }
    // unit j: 5-bit values from nibble j & 1 and qh bit j, scale and min from scale_min_k4 (as
    // Q4_K); sum (d sc q - dmin m) x = d sc sum q x - dmin m sum x
    template <int NV>
    __device__ static __forceinline__ void dot_q(const uint4 &hd, const uint32_t (&ql)[8], const uint32_t (&qh)[8], int j,
                                                 const XU (&x)[NV], int nv, float (&r)[NV]) {
        const float d = h2f(hd.x & 0xffff), dmin = h2f(hd.x >> 16);
        const uint32_t hs[3] = {hd.y, hd.z, hd.w};
        auto sb = [&](int k) -> uint32_t { return (hs[k >> 2] >> (8 * (k & 3))) & 0xff; };
        uint32_t sc, mn;
        if (j < 4) {
            sc = sb(j) & 63;
            mn = sb(j + 4) & 63;
        } else {
            sc = (sb(j + 4) & 0xF) | ((sb(j - 4) >> 6) << 4);
            mn = (sb(j + 4) >> 4) | ((sb(j) >> 6) << 4);
        }
        const int sh = (j & 1) * 4;
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = ((ql[i] >> sh) & 0x0F0F0F0Fu) | (((qh[i] >> j) & 0x01010101u) << 4);
        const float ds = d * (float)sc, dm = dmin * (float)mn;
#pragma unroll
        for (int t = 0; t < NV; t++)
            if (NV == 1 || t < nv) r[t] += x[t].D * (ds * (float)dot8(q, x[t].q) - dm * (float)(x[t].slo + x[t].shi));
    }
    template <int NV, bool XNEG = false>
    __device__ static __forceinline__ void dot(const Raw &w, int j, const uint8_t *, const XU (&x)[NV], int nv,
                                               float (&r)[NV]) {
        const uint32_t ql[8] = {w.a0.x, w.a0.y, w.a0.z, w.a0.w, w.a1.x, w.a1.y, w.a1.z, w.a1.w};
        const uint32_t qh[8] = {w.b0.x, w.b0.y, w.b0.z, w.b0.w, w.b1.x, w.b1.y, w.b1.z, w.b1.w};
        dot_q<NV>(w.h, ql, qh, j, x, nv, r);
    }
    // the pair (j even, j + 1) loaded by load2, unit j then unit j + 1 (the order of two dot calls)
    template <int NV>
    __device__ static __forceinline__ void dot_pair(const Raw &w0, const Raw &w1, int j, const XU (&x0)[NV],
                                                    const XU (&x1)[NV], int nv, float (&r)[NV]) {
        const uint32_t ql[8] = {w0.a0.x, w0.a0.y, w0.a0.z, w0.a0.w, w0.a1.x, w0.a1.y, w0.a1.z, w0.a1.w};
        const uint32_t qh[8] = {w1.a0.x, w1.a0.y, w1.a0.z, w1.a0.w, w1.a1.x, w1.a1.y, w1.a1.z, w1.a1.w};
        dot_q<NV>(w0.h, ql, qh, j, x0, nv, r);
        dot_q<NV>(w0.h, ql, qh, j + 1, x1, nv, r);
    }
};

// IQ4_XS (lib.rs:331-343): per 32-element unit ib, 16 qs bytes at 8 + 16 ib whose low nibbles are
// elements 0..15 and high nibbles elements 16..31, each an index into the 16 int8 values of
// kvalues_iq4nl; the unit's 6-bit scale ls (4 bits from scales_l, 2 from scales_h) gives
// d (ls - 32). The lookup runs in registers: two v_perm_b32 over the table's halves (entries
// 0..7 and 8..15, selector = index & 7) and a bytewise select on index bit 3, four values per
// three operations; the unit's sum of kvalue * q is one integer dot.
struct FIQ4_XS : UnitGeom<256, 136>, NoTable {
    static constexpr int TYPE = GS_IQ4_XS, QK = 256, BB = 136, TAB = 0, RAW = 6;
    struct Raw { uint4 q; uint2 h; };   // the unit's 16 qs bytes; block bytes 0..7 (d, scales_h, scales_l)
    template <class M>
    __device__ static __forceinline__ void load(const M &m, uint32_t o, int j, Raw &w) {
        w.h = m.u64(o);
        w.q = m.u128(o + 8 + 16 * (uint32_t)j);
    }
    // units j, j+1 of one block (j even): the header once, their 32 qs bytes together
    static constexpr bool PAIR = true;
    template <class M>
    __device__ static __forceinline__ void load2(const M &m, uint32_t o, int j, Raw &w0, Raw &w1) {
        w0.h = w1.h = m.u64(o);
        w0.q = m.u128(o + 8 + 16 * (uint32_t)j);
        w1.q = m.u128(o + 24 + 16 * (uint32_t)j);
    }
    __device__ static __forceinline__ uint32_t kv4(int i) {   // table entries 4i..4i+3 as bytes
        return (uint32_t)(uint8_t)kvalues_iq4nl[4 * i] | ((uint32_t)(uint8_t)kvalues_iq4nl[4 * i + 1] << 8) |
               ((uint32_t)(uint8_t)kvalues_iq4nl[4 * i + 2] << 16) | ((uint32_t)(uint8_t)kvalues_iq4nl[4 * i + 3] << 24);
    }
    // four nibble indices (one per byte, 0..15) -> their four int8 table values
    __device__ static __forceinline__ uint32_t lut4(uint32_t n, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
        const uint32_t sel = n & 0x07070707u;
        const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);   // entries 0..7
        const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);   // entries 8..15
        const uint32_t m = ((n >> 3) & 0x01010101u) * 0xffu;      // 0xff in the bytes with index bit 3
        return (hi & m) | (lo & ~m);
    }
    template <int NV, bool XNEG = false>
    __device__ static __forceinline__ void dot(const Raw &w, int j, const uint8_t *, const XU (&x)[NV], int nv,
                                               float (&r)[NV]) {
        const uint32_t t0 = kv4(0), t1 = kv4(1), t2 = kv4(2), t3 = kv4(3);
        const uint32_t qw[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        uint32_t v[8];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            v[k] = lut4(qw[k] & 0x0F0F0F0Fu, t0, t1, t2, t3);
            v[k + 4] = lut4((qw[k] >> 4) & 0x0F0F0F0Fu, t0, t1, t2, t3);
        }
        const uint32_t sh = w.h.x >> 16, sl = w.h.y;
        const int ls = (int)((sl >> (4 * j)) & 0xfu) | (int)(((sh >> (2 * j)) & 3u) << 4);
        const float dl = h2f(w.h.x & 0xffff) * (float)(ls - 32);
#pragma unroll
        for (int t = 0; t < NV; t++)
            if (NV == 1 || t < nv) r[t] += (dl * x[t].D) * (float)dot8(v, x[t].q);
    }
};

// Q2_K (lib.rs:139-160) and Q3_K (lib.rs:163-201): unit u = quarter j = u & 3 of the 128-element
// half n = u >> 2 takes the 2-bit fields 2j of the 32 qs bytes of its half (Q2_K at 16 + 32 n,
// Q3_K at 32 + 32 n); Q3_K adds bit 4n + j of the 32 hmask bytes (set: +0, clear: -4). Each
// 16-element half of a unit has its own scale (Q2_K: a byte of 4-bit scale and min; Q3_K: a
// 6-bit scale unpacked from 12 bytes). Units j and j + 1 of a half read the same bytes, so a
// lane's pair loads them once. Sums: Q2_K d sc sum q x - dmin m sum x; Q3_K with
// v = (q | h << 2) - 4: sum v x = sum (q | h << 2) x - 4 sum x.
struct FQ2_K : UnitGeom<256, 84>, NoTable {
    static constexpr int TYPE = GS_Q2_K, QK = 256, BB = 84, TAB = 0, RAW = 10, RAW2 = 5;
    static constexpr bool PAIR = true, JOINT = true;
    // a = the half's 32 qs bytes, s = scale bytes from 8n + 2j (the unit's two, or the pair's
    // four), dd = d | dmin << 16
    struct Raw { uint4 a0, a1; uint32_t s, dd; };
    __device__ static __forceinline__ int xunit(int up) { return up; }
    template <class M>
    __device__ static __forceinline__ void load(const M &m, uint32_t o, int u, Raw &w) {
        const uint32_t n = (uint32_t)u >> 2, j = (uint32_t)u & 3;
        w.a0 = m.u128(o + 16 + 32 * n);
        w.a1 = m.u128(o + 32 + 32 * n);
        w.s = m.u16(o + 8 * n + 2 * j);
        w.dd = m.u32(o + 80);
    }
    template <class M>
    __device__ static __forceinline__ void load2(const M &m, uint32_t o, int u, Raw &w0, Raw &) {
        const uint32_t n = (uint32_t)u >> 2, j = (uint32_t)u & 3;
        w0.a0 = m.u128(o + 16 + 32 * n);
        w0.a1 = m.u128(o + 32 + 32 * n);
        w0.s = m.u32(o + 8 * n + 2 * j);
        w0.dd = m.u32(o + 80);
    }
    template <int NV>
    __device__ static __forceinline__ void dot_q(const Raw &w, int j, uint32_t sc2, const XU (&x)[NV], int nv,
                                                 float (&r)[NV]) {
        const uint32_t qw[8] = {w.a0.x, w.a0.y, w.a0.z, w.a0.w, w.a1.x, w.a1.y, w.a1.z, w.a1.w};
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = (qw[i] >> (2 * j)) & 0x03030303u;
        const float d = h2f(w.dd & 0xffff), dmin = h2f(w.dd >> 16);
        const int s0 = (int)(sc2 & 0xf), m0 = (int)((sc2 >> 4) & 0xf), s1 = (int)((sc2 >> 8) & 0xf), m1 = (int)((sc2 >> 12) & 0xf);
#pragma unroll
        for (int t = 0; t < NV; t++) {
            if (NV == 1 || t < nv) {
                int lo = 0, hi = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) lo = __builtin_amdgcn_sdot4((int)q[i], (int)x[t].q[i], lo, false);
#pragma unroll
                for (int i = 4; i < 8; i++) hi = __builtin_amdgcn_sdot4((int)q[i], (int)x[t].q[i], hi, false);
                r[t] += x[t].D * (d * (float)(s0 * lo + s1 * hi) - dmin * (float)(m0 * x[t].slo + m1 * x[t].shi));
            }
        }
    }
    template <int NV, bool XNEG = false>
    __device__ static __forceinline__ void dot(const Raw &w, int u, const uint8_t *, const XU (&x)[NV], int nv,
                                               float (&r)[NV]) {
        dot_q<NV>(w, u & 3, w.s, x, nv, r);
    }
    template <int NV>
    __device__ static __forceinline__ void dot_pair(const Raw &w0, const Raw &, int u, const XU (&x0)[NV],
                                                    const XU (&x1)[NV], int nv, float (&r)[NV]) {
        dot_q<NV>(w0, u & 3, w0.s & 0xffff, x0, nv, r);
        dot_q<NV>(w0, (u & 3) + 1, w0.s >> 16, x1, nv, r);
    }
};

struct FQ3_K : UnitGeom<256, 110>, NoTable {
    static constexpr int TYPE = GS_Q3_K, QK = 256, BB = 110, TAB = 0, RAW = 20, RAW2 = 10;
    static constexpr bool PAIR = true, JOINT = true;
    // single unit: a = the half's 32 qs bytes, b = the 32 hmask bytes, sc = the 12 scale bytes,
    // dd = d. Pair: w0.a = qs, w0.sc, w0.dd; w1.a = hmask.
    struct Raw { uint4 a0, a1, b0, b1; uint32_t sc0, sc1, sc2, dd; };
    __device__ static __forceinline__ int xunit(int up) { return up; }
    template <class M>
    __device__ static __forceinline__ void load_common(const M &m, uint32_t o, int u, Raw &w) {
        const uint32_t n = (uint32_t)u >> 2;
        w.a0 = m.u128(o + 32 + 32 * n);
        w.a1 = m.u128(o + 48 + 32 * n);
        const uint2 s01 = m.u64(o + 96);
        w.sc0 = s01.x;
        w.sc1 = s01.y;
        w.sc2 = m.u32(o + 104);
        w.dd = m.u16(o + 108);
    }
    template <class M>
    __device__ static __forceinline__ void load(const M &m, uint32_t o, int u, Raw &w) {
        load_common(m, o, u, w);
        w.b0 = m.u128(o);
        w.b1 = m.u128(o + 16);
    }
    template <class M>
    __device__ static __forceinline__ void load2(const M &m, uint32_t o, int u, Raw &w0, Raw &w1) {
        load_common(m, o, u, w0);
        w1.a0 = m.u128(o);
        w1.a1 = m.u128(o + 16);
    }
    // 6-bit scale is (0..15) from the 12 raw bytes (lib.rs:166-179): low nibble of raw byte is & 7
    // (the high nibble for is >= 8), bits 2 (is >> 2) of raw byte 8 + (is & 3) on top
    // (selects, not a runtime array index: that would put the words in scratch memory)
    __device__ static __forceinline__ int scale6(const Raw &w, int is) {
        const int b = is & 7;
        const uint32_t word = b >= 4 ? w.sc1 : w.sc0;
        const uint32_t lo = (word >> (8 * (b & 3) + (is >= 8 ? 4 : 0))) & 0xfu;
        const uint32_t hi = (w.sc2 >> (8 * (is & 3) + 2 * (is >> 2))) & 3u;
        return (int)(lo | (hi << 4)) - 32;
    }
    template <int NV>
    __device__ static __forceinline__ void dot_q(const uint32_t (&qw)[8], const uint32_t (&hw)[8], const Raw &ws, int u,
                                                 const XU (&x)[NV], int nv, float (&r)[NV]) {
        const int n = u >> 2, j = u & 3;
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            q[i] = ((qw[i] >> (2 * j)) & 0x03030303u) | (((hw[i] >> (4 * n + j)) & 0x01010101u) << 2);
        const float d = h2f(ws.dd);
        const int s0 = scale6(ws, 8 * n + 2 * j), s1 = scale6(ws, 8 * n + 2 * j + 1);
#pragma unroll
        for (int t = 0; t < NV; t++) {
            if (NV == 1 || t < nv) {
                int lo = 0, hi = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) lo = __builtin_amdgcn_sdot4((int)q[i], (int)x[t].q[i], lo, false);
#pragma unroll
                for (int i = 4; i < 8; i++) hi = __builtin_amdgcn_sdot4((int)q[i], (int)x[t].q[i], hi, false);
                r[t] += (d * x[t].D) * (float)(s0 * (lo - 4 * x[t].slo) + s1 * (hi - 4 * x[t].shi));
            }
        }
    }
    template <int NV, bool XNEG = false>
    __device__ static __forceinline__ void dot(const Raw &w, int u, const uint8_t *, const XU (&x)[NV], int nv,
                                               float (&r)[NV]) {
        const uint32_t qw[8] = {w.a0.x, w.a0.y, w.a0.z, w.a0.w, w.a1.x, w.a1.y, w.a1.z, w.a1.w};
        const uint32_t hw[8] = {w.b0.x, w.b0.y, w.b0.z, w.b0.w, w.b1.x, w.b1.y, w.b1.z, w.b1.w};
        dot_q<NV>(qw, hw, w, u, x, nv, r);
    }
    template <int NV>
    __device__ static __forceinline__ void dot_pair(const Raw &w0, const Raw &w1, int u, const XU (&x0)[NV],
                                                    const XU (&x1)[NV], int nv, float (&r)[NV]) {
        const uint32_t qw[8] = {w0.a0.x, w0.a0.y, w0.a0.z, w0.a0.w, w0.a1.x, w0.a1.y, w0.a1.z, w0.a1.w};
        const uint32_t hw[8] = {w1.a0.x, w1.a0.y, w1.a0.z, w1.a0.w, w1.a1.x, w1.a1.y, w1.a1.z, w1.a1.w};
        dot_q<NV>(qw, hw, w0, u, x0, nv, r);
        dot_q<NV>(qw, hw, w0, u + 1, x1, nv, r);
    }
};

// Q6_K (lib.rs:243-262). A super-block's 32-element unit of quarter q in half h takes the low
// (q < 2) or high (q >= 2) nibbles of the 32 ql bytes at 64h + 32(q & 1) and 2-bit fields 2q of
// the 32 qh bytes at 128 + 32h, so quarters q and q + 2 of a half read the same 64 bytes. The
// streaming kernels number a super-block's units in pair order -- v = 0..7 is quarter
// qp + 2(v & 1) of half v >> 2 with qp = (v >> 1) & 1 -- so the two units of a lane's pair (v even,
// v + 1) share their bytes and load them once (load2: 9 registers per unit instead of 18) and
// the activation unit of v is the natural unit nat(v) (xunit).
struct FQ6_K : UnitGeom<256, 210>, NoTable {
    static constexpr int TYPE = GS_Q6_K, QK = 256, BB = 210, TAB = 0, RAW = 18, RAW2 = 9;
    static constexpr bool PAIR = true, JOINT = true;
    // single unit: a = ql, b = qh, e0 = its two int8 scales, e1 = d. Pair (load2): w0.a = ql,
    // w0.e0 = both units' scales, w1.a = qh, w1.e0 = d.
    struct Raw { uint4 a0, a1, b0, b1; uint32_t e0, e1; };
    __device__ static __forceinline__ int nat(int v) { return (v & 4) | ((v >> 1) & 1) | ((v & 1) << 1); }
    __device__ static __forceinline__ int xunit(int up) { return (up & ~7) | nat(up & 7); }
    template <class M>
    __device__ static __forceinline__ void load(const M &m, uint32_t o, int v, Raw &w) {
        const uint32_t n = (uint32_t)nat(v), half = n >> 2, quarter = n & 3;
        const uint32_t ql = o + 64 * half + 32 * (quarter & 1), qh = o + 128 + 32 * half;
        w.a0 = m.u128(ql);
        w.a1 = m.u128(ql + 16);
        w.b0 = m.u128(qh);
        w.b1 = m.u128(qh + 16);
        w.e0 = m.u16(o + 192 + 8 * half + 2 * quarter);
        w.e1 = m.u16(o + 208);
    }
    template <class M>
    __device__ static __forceinline__ void load2(const M &m, uint32_t o, int v, Raw &w0, Raw &w1) {
        const uint32_t half = (uint32_t)v >> 2, qp = ((uint32_t)v >> 1) & 1;
        const uint32_t ql = o + 64 * half + 32 * qp, qh = o + 128 + 32 * half, sc = o + 192 + 8 * half + 2 * qp;
        w0.a0 = m.u128(ql);
        w0.a1 = m.u128(ql + 16);
        w1.a0 = m.u128(qh);
        w1.a1 = m.u128(qh + 16);
        w0.e0 = m.u16(sc) | (m.u16(sc + 4) << 16);
        w1.e0 = m.u16(o + 208);
    }
    // one unit: 6-bit values from nibble shift nsh of ql and field hsh of qh, dotted per 16-element
    // half with its int8 scale (sum (q-32) x = sum q x - 32 sum x)
    template <int NV>
    __device__ static __forceinline__ void dot_q(const uint32_t (&ql)[8], const uint32_t (&qh)[8], int nsh, int hsh,
                                                 uint32_t sc, float d, const XU (&x)[NV], int nv, float (&r)[NV]) {
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = ((ql[i] >> nsh) & 0x0F0F0F0Fu) | (((qh[i] >> hsh) & 0x03030303u) << 4);
        const int sc0 = (int8_t)(sc & 0xff), sc1 = (int8_t)((sc >> 8) & 0xff);
#pragma unroll
        for (int t = 0; t < NV; t++) {
            if (t < nv) {
                int lo = 0, hi = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) lo = __builtin_amdgcn_sdot4((int)q[i], (int)x[t].q[i], lo, false);
#pragma unroll
                for (int i = 4; i < 8; i++) hi = __builtin_amdgcn_sdot4((int)q[i], (int)x[t].q[i], hi, false);
                r[t] += (d * x[t].D) * (float)(sc0 * (lo - 32 * x[t].slo) + sc1 * (hi - 32 * x[t].shi));
            }
        }
    }
    template <int NV, bool XNEG = false>
    __device__ static __forceinline__ void dot(const Raw &w, int v, const uint8_t *, const XU (&x)[NV], int nv,
                                               float (&r)[NV]) {
        const int quarter = nat(v) & 3;
        const uint32_t ql[8] = {w.a0.x, w.a0.y, w.a0.z, w.a0.w, w.a1.x, w.a1.y, w.a1.z, w.a1.w};
        const uint32_t qh[8] = {w.b0.x, w.b0.y, w.b0.z, w.b0.w, w.b1.x, w.b1.y, w.b1.z, w.b1.w};
        dot_q<NV>(ql, qh, quarter >= 2 ? 4 : 0, 2 * quarter, w.e0, h2f(w.e1), x, nv, r);
    }
    // the pair (v even, v + 1) loaded by load2, unit v then unit v + 1 (the order of two dot calls)
    template <int NV>
    __device__ static __forceinline__ void dot_pair(const Raw &w0, const Raw &w1, int v, const XU (&x0)[NV],
                                                    const XU (&x1)[NV], int nv, float (&r)[NV]) {
        const int qp = (v >> 1) & 1;
        const uint32_t ql[8] = {w0.a0.x, w0.a0.y, w0.a0.z, w0.a0.w, w0.a1.x, w0.a1.y, w0.a1.z, w0.a1.w};
        const uint32_t qh[8] = {w1.a0.x, w1.a0.y, w1.a0.z, w1.a0.w, w1.a1.x, w1.a1.y, w1.a1.z, w1.a1.w};
        const float d = h2f(w1.e0);
        dot_q<NV>(ql, qh, 0, 2 * qp, w0.e0 & 0xffffu, d, x0, nv, r);
        dot_q<NV>(ql, qh, 4, 2 * qp + 4, w0.e0 >> 16, d, x1, nv, r);
    }
};

// Q6_K with aligned loads (FQ6_KA: the one-vector GEMV over many rows whose rows start 4-byte
// aligned). Odd super-blocks start 2 bytes past a multiple of 4, and their 16-byte ql / qh loads
// stream far slower than aligned ones (262144 x 4096: 187 us against 146 with aligned addresses).
// A pair reads each of its 32-byte ql and qh stretches as the 36-byte dword-aligned window around
// it and shifts it into place (v_alignbyte, 8 per unit); the shift rides in the high half of the
// d word. The windows stay inside the super-block (ql and qh are followed by more of its bytes;
// with the row 4-byte aligned, a window starting 2 bytes early belongs to an odd block, so the
// bytes before it are the previous block's); where no shift is needed the ninth dword repeats
// the eighth.
struct FQ6_KA : FQ6_K {
    static constexpr int RAW2 = 10;
    template <class M>
    __device__ static __forceinline__ void load2(const M &m, uint32_t o, int v, Raw &w0, Raw &w1) {
        const uint32_t half = (uint32_t)v >> 2, qp = ((uint32_t)v >> 1) & 1;
        const uint32_t sh = (uint32_t)(uintptr_t)m.ptr(o) & 3u;   // 0 or 2
        const uint32_t ql = o + 64 * half + 32 * qp - sh, qh = o + 128 + 32 * half - sh, sc = o + 192 + 8 * half + 2 * qp;
        w0.a0 = m.u128(ql);
        w0.a1 = m.u128(ql + 16);
        w0.b0.x = m.u32(ql + (sh ? 32u : 28u));
        w1.a0 = m.u128(qh);
        w1.a1 = m.u128(qh + 16);
        w1.b0.x = m.u32(qh + (sh ? 32u : 28u));
        w0.e0 = m.u16(sc) | (m.u16(sc + 4) << 16);
        w1.e0 = m.u16(o + 208) | (sh << 16);
    }
    template <int NV>
    __device__ static __forceinline__ void dot_pair(const Raw &w0, const Raw &w1, int v, const XU (&x0)[NV],
                                                    const XU (&x1)[NV], int nv, float (&r)[NV]) {
        const int qp = (v >> 1) & 1;
        const uint32_t sh = w1.e0 >> 16;
        const uint32_t dl[9] = {w0.a0.x, w0.a0.y, w0.a0.z, w0.a0.w, w0.a1.x, w0.a1.y, w0.a1.z, w0.a1.w, w0.b0.x};
        const uint32_t dh[9] = {w1.a0.x, w1.a0.y, w1.a0.z, w1.a0.w, w1.a1.x, w1.a1.y, w1.a1.z, w1.a1.w, w1.b0.x};
        uint32_t ql[8], qh[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            ql[i] = __builtin_amdgcn_alignbyte(dl[i + 1], dl[i], sh);
            qh[i] = __builtin_amdgcn_alignbyte(dh[i + 1], dh[i], sh);
        }
        const float d = h2f(w1.e0 & 0xffffu);
        dot_q<NV>(ql, qh, 0, 2 * qp, w0.e0 & 0xffffu, d, x0, nv, r);
        dot_q<NV>(ql, qh, 4, 2 * qp + 4, w0.e0 >> 16, d, x1, nv, r);
    }
};

// IQ2_XXS: the 256-entry grid (2 KiB) and a table of v_perm_b32 selectors (2 KiB: 128 sign
// indices, each stored twice so an 8-bit index with a stray top bit needs no mask) live in LDS at fixed addresses (folded into the ds_read offsets). The signs are applied to the
// activations, not the weights: a selector picks, per byte, q (sel = i) or -q (sel = i+4) from
// the pair {-q, q}, and -q is computed once per activation unit (XU::nq), so a group of 8
// elements costs 2 table reads, 2 v_perm_b32 and 2 v_dot4_i32_i8.
__shared__ uint2 gs_iq2xxs_grid_lds[256];
__shared__ uint2 gs_iq2xxs_sel_lds[256];   // entry i = selectors of sign index i & 127

// v_perm_b32 selectors for sign index i (two words, elements 0-3 and 4-7): byte e selects q
// (selector e) or -q (selector e + 4) from the pair {-q, q} by bit e of ksigns(i).
__device__ __forceinline__ uint2 sign_sel(int i) {
    const uint32_t k = ksigns((uint32_t)i);
    uint32_t lo = 0x03020100u, hi = 0x03020100u;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        lo += ((k >> b) & 1u) << (8 * b + 2);
        hi += ((k >> (b + 4)) & 1u) << (8 * b + 2);
    }
    return make_uint2(lo, hi);
}

// byte L of a, times 8: one SDWA shift (byte select on the source operand) instead of a
// shift-and-mask pair; it is the byte offset of a 256-entry table of 8-byte rows.
template <int L>
__device__ __forceinline__ uint32_t grid_off(uint32_t a) {
    uint32_t r;
    if (L == 0) asm("v_lshlrev_b32_sdwa %0, 3, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0" : "=v"(r) : "v"(a));
    if (L == 1) asm("v_lshlrev_b32_sdwa %0, 3, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1" : "=v"(r) : "v"(a));
    if (L == 2) asm("v_lshlrev_b32_sdwa %0, 3, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2" : "=v"(r) : "v"(a));
    if (L == 3) asm("v_lshlrev_b32_sdwa %0, 3, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3" : "=v"(r) : "v"(a));
    return r;
}

// Byte offset of the selector row of sign field L (7 bits at bit 7L of a): byte L of a << L holds
// the field in its low 7 bits (the 8th bit is the next field's, which the doubled table ignores).
template <int L>
__device__ __forceinline__ uint32_t sel_off(uint32_t a) {
    return grid_off<L>(L ? a << L : a);
}

// sum of 4 int8 products, with a zero accumulator (the VOP3 form: no register to clear first)
__device__ __forceinline__ int sdot4_0(uint32_t a, uint32_t b) {
    int r;
    asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// r[t] += dh * x[t].D * m * sum over 4 groups of 8: grid bytes g[l] . (signs s[l] applied) q. XNEG: the
// activation units carry -q and the v_perm_b32 selectors pick q or -q per byte (2 operations per
// 8 elements); otherwise the signs go on the grid bytes (every grid byte is nonzero, so
// 0x01010100 - g negates bytewise; one more operation per 4 elements).
// The unit scale is dh * m with m = 2s+1 an odd integer up to 31, applied to the integer sum
// (|sum| < 2^18, so the 24-bit multiply is exact) before the one float conversion.
template <int NV, bool XNEG>
__device__ __forceinline__ void signed_dot8x4(const uint2 (&g_)[4], const uint2 (&s)[4], float dh, int m,
                                              const XU (&x)[NV], int nv, float (&r)[NV]) {
    uint2 g[4] = {g_[0], g_[1], g_[2], g_[3]};
    if (!XNEG) {
#pragma unroll
        for (int l = 0; l < 4; l++) {
            g[l].x = __builtin_amdgcn_perm(0x01010100u - g[l].x, g[l].x, s[l].x);
            g[l].y = __builtin_amdgcn_perm(0x01010100u - g[l].y, g[l].y, s[l].y);
        }
    }
#pragma unroll
    for (int t = 0; t < NV; t++) {
        if (NV == 1 || t < nv) {
            int acc = 0;
#pragma unroll
            for (int l = 0; l < 4; l++) {
                const uint32_t q0 = XNEG ? __builtin_amdgcn_perm(x[t].nq[2 * l], x[t].q[2 * l], s[l].x) : x[t].q[2 * l];
                const uint32_t q1 =
                    XNEG ? __builtin_amdgcn_perm(x[t].nq[2 * l + 1], x[t].q[2 * l + 1], s[l].y) : x[t].q[2 * l + 1];
                acc = l == 0 ? sdot4_0(g[l].x, q0) : __builtin_amdgcn_sdot4((int)g[l].x, (int)q0, acc, false);
                acc = __builtin_amdgcn_sdot4((int)g[l].y, (int)q1, acc, false);
            }
            r[t] += (dh * x[t].D) * (float)__mul24(acc, m);
        }
    }
}

struct FIQ2_XXS : UnitGeom<256, 66> {
    static constexpr int TYPE = GS_IQ2_XXS, QK = 256, BB = 66, TAB = 0, RAW = 3;
    static constexpr bool NEG_X = true;
    static constexpr float XSCALE = 0.125f;   // the format's /4 and the 1/2 of (2s+1)/2, in the activation scale
    struct Raw { uint2 a; uint32_t d; };
    // table setup split in two so the global read can be issued before the weight prefetch
    struct TabReg { uint64_t g; };
    __device__ static __forceinline__ void tab_load(int tid, TabReg &r) { r.g = tid < 256 ? iq2xxs_grid[tid] : 0; }
    __device__ static __forceinline__ void tab_store(int tid, const TabReg &r) {
        if (tid < 256) gs_iq2xxs_grid_lds[tid] = make_uint2((uint32_t)r.g, (uint32_t)(r.g >> 32));
        if (tid < 256) gs_iq2xxs_sel_lds[tid] = sign_sel(tid & 127);
    }
    template <class M>
    __device__ static __forceinline__ void load(const M &m, uint32_t o, int j, Raw &w) {
        w.d = m.u16(o);
        w.a = m.u64(o + 2 + 8 * (uint32_t)j);
    }
    // units j, j+1 of one block (j even): one scale read, one 16-byte read
    static constexpr bool PAIR = true;
    template <class M>
    __device__ static __forceinline__ void load2(const M &m, uint32_t o, int j, Raw &w0, Raw &w1) {
        w0.d = w1.d = m.u16(o);
        const uint4 a = m.u128(o + 2 + 8 * (uint32_t)j);
        w0.a = make_uint2(a.x, a.y);
        w1.a = make_uint2(a.z, a.w);
    }
    // XNEG: the activation units carry -q (signs applied on the activation side, 2 ops per 8
    // elements); otherwise the signs are applied to the grid bytes (one more op per 4 elements,
    // 8 fewer registers per activation unit).
    // Two phases so the row loop can issue the next unit's table reads before this unit's
    // arithmetic: fetch() reads the grid rows and sign selectors from LDS, dot2() consumes them.
    struct Dec { uint2 g[4], s[4]; };
    __device__ static __forceinline__ void fetch(const Raw &w, Dec &e) {
        const uint32_t gofs[4] = {grid_off<0>(w.a.x), grid_off<1>(w.a.x), grid_off<2>(w.a.x), grid_off<3>(w.a.x)};
        const uint32_t sofs[4] = {sel_off<0>(w.a.y), sel_off<1>(w.a.y), sel_off<2>(w.a.y), sel_off<3>(w.a.y)};
#pragma unroll
        for (int l = 0; l < 4; l++) {
            e.g[l] = *(const uint2 *)((const uint8_t *)gs_iq2xxs_grid_lds + gofs[l]);
        }
#pragma unroll
        for (int l = 0; l < 4; l++) e.s[l] = *(const uint2 *)((const uint8_t *)gs_iq2xxs_sel_lds + sofs[l]);
    }
    template <int NV, bool XNEG = true>
    __device__ static __forceinline__ void dot2(const Raw &w, const Dec &e, const XU (&x)[NV], int nv, float (&r)[NV]) {
        // db = d * (0.5 + s) * 0.25 = d * (2s+1) * 0.125 (lib.rs:279); the 0.125 is in x.D, and
        // (a >> 27) | 1 = 2s+1 whatever bit 27 (a sign bit) is
        signed_dot8x4<NV, XNEG>(e.g, e.s, h2f(w.d), (int)((w.a.y >> 27) | 1u), x, nv, r);
    }
    template <int NV, bool XNEG = true>
    __device__ static __forceinline__ void dot(const Raw &w, int, const uint8_t *, const XU (&x)[NV], int nv,
                                               float (&r)[NV]) {
        Dec e;
        fetch(w, e);
        dot2<NV, XNEG>(w, e, x, nv, r);
    }
};

// IQ2_S (lib.rs:291-309): unit u has 4 groups of 8; group l's grid index is qs byte 2 + 4u + l
// plus bits 2l..2l+1 of qh byte 66 + u as bits 8..9 (1024-entry grid, 8 KiB in LDS), its signs
// are the raw byte 34 + 4u + l (no parity bit), and the unit's scale byte 74 + u holds one 4-bit
// scale per 16 elements: db = d (0.5 + s) / 4 = d (2s+1) / 8, the 1/8 folded into the activation
// scale. The signs go on the activation side through v_perm_b32 selectors (a 256-entry table
// indexed by the sign byte itself), as for IQ2_XXS.
__shared__ uint2 gs_iq2s_grid_lds[1024];
__shared__ uint2 gs_iq2s_sel_lds[256];

// v_perm_b32 selectors for the 8 sign bits s: byte e selects q (e) or -q (e + 4)
__device__ __forceinline__ uint2 sign_sel_raw(uint32_t s) {
    uint32_t lo = 0x03020100u, hi = 0x03020100u;
#pragma unroll
    for (int b = 0; b < 4; b++) {
        lo += ((s >> b) & 1u) << (8 * b + 2);
        hi += ((s >> (b + 4)) & 1u) << (8 * b + 2);
    }
    return make_uint2(lo, hi);
}

struct FIQ2_S : UnitGeom<256, 82> {
    static constexpr int TYPE = GS_IQ2_S, QK = 256, BB = 82, TAB = 0, RAW = 5;
    static constexpr bool NEG_X = true;
    static constexpr float XSCALE = 0.125f;
    struct Raw { uint32_t a, sg, qh, sc, d; };   // index bytes, sign bytes, qh byte, scale byte, d
    struct TabReg { uint64_t g0, g1; };
    __device__ static __forceinline__ void tab_load(int tid, TabReg &r) {
        r.g0 = tid < 1024 ? iq2s_grid[tid] : 0;
        r.g1 = tid + 512 < 1024 ? iq2s_grid[tid + 512] : 0;
    }
    __device__ static __forceinline__ void tab_store(int tid, const TabReg &r) {
        if (tid < 1024) gs_iq2s_grid_lds[tid] = make_uint2((uint32_t)r.g0, (uint32_t)(r.g0 >> 32));
        if (tid + 512 < 1024) gs_iq2s_grid_lds[tid + 512] = make_uint2((uint32_t)r.g1, (uint32_t)(r.g1 >> 32));
        if (tid < 256) gs_iq2s_sel_lds[tid] = sign_sel_raw((uint32_t)tid);
    }
    template <class M>
    __device__ static __forceinline__ void load(const M &m, uint32_t o, int j, Raw &w) {
        w.d = m.u16(o);
        w.a = m.u32(o + 2 + 4 * (uint32_t)j);
        w.sg = m.u32(o + 34 + 4 * (uint32_t)j);
        w.qh = m.u16(o + 66 + (uint32_t)j);
        // the scale byte 74 + j as the high byte of the u16 before it: unit 7's u16 at 74 + j would
        // end past the 82-byte block (the last block of an allocation)
        w.sc = m.u16(o + 73 + (uint32_t)j) >> 8;
    }
    // units j, j+1 of one block (j even): d once, both units' bytes in 8-byte and 2-byte reads
    static constexpr bool PAIR = true;
    template <class M>
    __device__ static __forceinline__ void load2(const M &m, uint32_t o, int j, Raw &w0, Raw &w1) {
        w0.d = w1.d = m.u16(o);
        const uint2 a = m.u64(o + 2 + 4 * (uint32_t)j), sg = m.u64(o + 34 + 4 * (uint32_t)j);
        const uint32_t qh = m.u16(o + 66 + (uint32_t)j), sc = m.u16(o + 74 + (uint32_t)j);
        w0.a = a.x, w1.a = a.y;
        w0.sg = sg.x, w1.sg = sg.y;
        w0.qh = qh, w1.qh = qh >> 8;   // the low byte is the unit's (only bits 0..7 are read)
        w0.sc = sc, w1.sc = sc >> 8;
    }
    struct Dec { uint2 g[4], s[4]; };
    template <int L>
    __device__ static __forceinline__ uint32_t gofs(const Raw &w) {   // byte offset of group L's grid row
        return grid_off<L>(w.a) | (((w.qh >> (2 * L)) & 3u) << 11);
    }
    __device__ static __forceinline__ void fetch(const Raw &w, Dec &e) {
        const uint32_t go[4] = {gofs<0>(w), gofs<1>(w), gofs<2>(w), gofs<3>(w)};
        const uint32_t so[4] = {grid_off<0>(w.sg), grid_off<1>(w.sg), grid_off<2>(w.sg), grid_off<3>(w.sg)};
#pragma unroll
        for (int l = 0; l < 4; l++) e.g[l] = *(const uint2 *)((const uint8_t *)gs_iq2s_grid_lds + go[l]);
#pragma unroll
        for (int l = 0; l < 4; l++) e.s[l] = *(const uint2 *)((const uint8_t *)gs_iq2s_sel_lds + so[l]);
    }
    template <int NV, bool XNEG = true>
    __device__ static __forceinline__ void dot2(const Raw &w, const Dec &e, const XU (&x)[NV], int nv, float (&r)[NV]) {
        uint2 g[4] = {e.g[0], e.g[1], e.g[2], e.g[3]};
        if (!XNEG) {   // signs on the grid bytes (every grid byte is nonzero: 0x01010100 - g negates)
#pragma unroll
            for (int l = 0; l < 4; l++) {
                g[l].x = __builtin_amdgcn_perm(0x01010100u - g[l].x, g[l].x, e.s[l].x);
                g[l].y = __builtin_amdgcn_perm(0x01010100u - g[l].y, g[l].y, e.s[l].y);
            }
        }
        const int m0 = 2 * (int)(w.sc & 0xfu) + 1, m1 = 2 * (int)((w.sc >> 4) & 0xfu) + 1;
        const float dh = h2f(w.d);
#pragma unroll
        for (int t = 0; t < NV; t++) {
            if (NV == 1 || t < nv) {
                int acc[2] = {0, 0};
#pragma unroll
                for (int l = 0; l < 4; l++) {
                    const uint32_t q0 = XNEG ? __builtin_amdgcn_perm(x[t].nq[2 * l], x[t].q[2 * l], e.s[l].x) : x[t].q[2 * l];
                    const uint32_t q1 =
                        XNEG ? __builtin_amdgcn_perm(x[t].nq[2 * l + 1], x[t].q[2 * l + 1], e.s[l].y) : x[t].q[2 * l + 1];
                    acc[l >> 1] = __builtin_amdgcn_sdot4((int)g[l].x, (int)q0, acc[l >> 1], false);
                    acc[l >> 1] = __builtin_amdgcn_sdot4((int)g[l].y, (int)q1, acc[l >> 1], false);
                }
                r[t] += (dh * x[t].D) * (float)(acc[0] * m0 + acc[1] * m1);
            }
        }
    }
    template <int NV, bool XNEG = true>
    __device__ static __forceinline__ void dot(const Raw &w, int, const uint8_t *, const XU (&x)[NV], int nv,
                                               float (&r)[NV]) {
        Dec e;
        fetch(w, e);
        dot2<NV, XNEG>(w, e, x, nv, r);
    }
};

// IQ3_XXS: a unit is 8 grid indices (one byte each, 4 values per entry) and one 32-bit word of
// four 7-bit sign indices plus the 4-bit scale (lib.rs:312-328). The 256-entry grid (1 KiB) sits
// in LDS next to the IQ2_XXS sign selectors (shared: both formats use ksigns), and the signs go on
// the activation side exactly as for IQ2_XXS.
__shared__ uint32_t gs_iq3xxs_grid_lds[256];

// byte L of a, times 4 (byte offset into a table of 4-byte rows), one SDWA shift.
template <int L>
__device__ __forceinline__ uint32_t grid_off4(uint32_t a) {
    uint32_t r;
    if (L == 0) asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0" : "=v"(r) : "v"(a));
    if (L == 1) asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1" : "=v"(r) : "v"(a));
    if (L == 2) asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2" : "=v"(r) : "v"(a));
    if (L == 3) asm("v_lshlrev_b32_sdwa %0, 2, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3" : "=v"(r) : "v"(a));
    return r;
}

struct FIQ3_XXS : UnitGeom<256, 98> {
    static constexpr int TYPE = GS_IQ3_XXS, QK = 256, BB = 98, TAB = 0, RAW = 4;
    static constexpr bool NEG_X = true;
    static constexpr float XSCALE = 0.25f;   // the format's *0.5 and the 1/2 of (2s+1)/2, in the activation scale
    struct Raw { uint2 a; uint32_t s; uint32_t d; };
    struct TabReg { uint32_t g; };
    __device__ static __forceinline__ void tab_load(int tid, TabReg &r) { r.g = tid < 256 ? iq3xxs_grid[tid] : 0; }
    __device__ static __forceinline__ void tab_store(int tid, const TabReg &r) {
        if (tid < 256) gs_iq3xxs_grid_lds[tid] = r.g;
        if (tid < 256) gs_iq2xxs_sel_lds[tid] = sign_sel(tid & 127);
    }
    template <class M>
    __device__ static __forceinline__ void load(const M &m, uint32_t o, int j, Raw &w) {
        w.d = m.u16(o);
        w.a = m.u64(o + 2 + 8 * (uint32_t)j);
        w.s = m.u32(o + 66 + 4 * (uint32_t)j);
    }
    static constexpr bool PAIR = true;
    template <class M>
    __device__ static __forceinline__ void load2(const M &m, uint32_t o, int j, Raw &w0, Raw &w1) {
        w0.d = w1.d = m.u16(o);
        const uint4 a = m.u128(o + 2 + 8 * (uint32_t)j);
        const uint2 sg = m.u64(o + 66 + 4 * (uint32_t)j);
        w0.a = make_uint2(a.x, a.y);
        w1.a = make_uint2(a.z, a.w);
        w0.s = sg.x;
        w1.s = sg.y;
    }
    struct Dec { uint2 g[4], s[4]; };
    __device__ static __forceinline__ void fetch(const Raw &w, Dec &e) {
        const uint8_t *gt = (const uint8_t *)gs_iq3xxs_grid_lds;
        e.g[0] = make_uint2(*(const uint32_t *)(gt + grid_off4<0>(w.a.x)), *(const uint32_t *)(gt + grid_off4<1>(w.a.x)));
        e.g[1] = make_uint2(*(const uint32_t *)(gt + grid_off4<2>(w.a.x)), *(const uint32_t *)(gt + grid_off4<3>(w.a.x)));
        e.g[2] = make_uint2(*(const uint32_t *)(gt + grid_off4<0>(w.a.y)), *(const uint32_t *)(gt + grid_off4<1>(w.a.y)));
        e.g[3] = make_uint2(*(const uint32_t *)(gt + grid_off4<2>(w.a.y)), *(const uint32_t *)(gt + grid_off4<3>(w.a.y)));
        const uint32_t sofs[4] = {sel_off<0>(w.s), sel_off<1>(w.s), sel_off<2>(w.s), sel_off<3>(w.s)};
#pragma unroll
        for (int l = 0; l < 4; l++) e.s[l] = *(const uint2 *)((const uint8_t *)gs_iq2xxs_sel_lds + sofs[l]);
    }
    template <int NV, bool XNEG = true>
    __device__ static __forceinline__ void dot2(const Raw &w, const Dec &e, const XU (&x)[NV], int nv, float (&r)[NV]) {
        // db = d * (0.5 + s) * 0.5 = d * (2s+1) * 0.25 (lib.rs:318); the 0.25 is in x.D
        signed_dot8x4<NV, XNEG>(e.g, e.s, h2f(w.d), (int)((w.s >> 27) | 1u), x, nv, r);
    }
    template <int NV, bool XNEG = true>
    __device__ static __forceinline__ void dot(const Raw &w, int, const uint8_t *, const XU (&x)[NV], int nv,
                                               float (&r)[NV]) {
        Dec e;
        fetch(w, e);
        dot2<NV, XNEG>(w, e, x, nv, r);
    }
};

// Plain float matrices (F32, F16, BF16: the router and other unquantized weights) with f32
// activations (quants.cu:81-96). A unit's 32 weights are loaded into registers with the row's
// other units (128 or 64 bytes, so they stream ahead of use like the quantized formats), widened
// to f32 exactly, and dotted with the staged f32 activations read as float4 from LDS, in four
// partial sums.
template <int T, int BB_>
struct FPlain : UnitGeom<8, BB_>, NoTable {
    static constexpr int TYPE = T, QK = 8, BB = BB_, TAB = 0;
    static constexpr bool F32X = true;
    static constexpr int NW = T == GS_F32 ? 8 : 4;   // 16-byte words per unit
    static constexpr int RAW = 4 * NW;
    struct Raw { uint4 d[NW]; };
    template <class M>
    __device__ static __forceinline__ void load(const M &m, uint32_t o, int, Raw &w) {
#pragma unroll
        for (int k = 0; k < NW; k++) w.d[k] = m.u128(o + 16 * k);
    }
    __device__ static __forceinline__ float wf(const Raw &w, int i) {
        const uint32_t word = (&w.d[0].x)[T == GS_F32 ? i : i >> 1];
        if (T == GS_F32) return __builtin_bit_cast(float, word);
        const uint32_t h = (i & 1) ? word >> 16 : word & 0xffffu;
        return T == GS_BF16 ? __builtin_bit_cast(float, h << 16) : (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    }
    template <int NV, bool XNEG = false>
    __device__ static __forceinline__ void dot(const Raw &w, int, const uint8_t *, const XU (&x)[NV], int nv,
                                               float (&r)[NV]) {
        float v[32];
#pragma unroll
        for (int i = 0; i < 32; i++) v[i] = wf(w, i);
#pragma unroll
        for (int t = 0; t < NV; t++) {
            if (t < nv) {
                const float4 *xs = (const float4 *)x[t].xs;
                float s4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float4 xv = xs[i];
                    s4[0] += v[4 * i] * xv.x;
                    s4[1] += v[4 * i + 1] * xv.y;
                    s4[2] += v[4 * i + 2] * xv.z;
                    s4[3] += v[4 * i + 3] * xv.w;
                }
                r[t] += x[t].D * ((s4[0] + s4[1]) + (s4[2] + s4[3]));
            }
        }
    }
};
using FF32 = FPlain<GS_F32, 32>;
using FF16 = FPlain<GS_F16, 16>;
using FBF16 = FPlain<GS_BF16, 16>;
