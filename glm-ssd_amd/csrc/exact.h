// Exact dequantization of one 32-element unit of a ggml block, bit-identical to the CPU
// reference's per-block decoders (crates/quants/src/lib.rs:131-343).
//
// A unit is the natural 32-element slice of each format: one Q8_0 block, one of the eight
// 32-element sub-blocks of a K-quant / IQ super-block (unit u covers elements 32u .. 32u+31), or
// 32 consecutive plain values. Each decoder evaluates lib.rs's expression for those 32 elements
// with lib.rs's f32 operation order; FP contraction is off for the whole file, so no multiply and
// add are fused (Q2_K / Q4_K / Q5_K subtract the min after the scaled product, as lib.rs does).
//
// Used by gs_dequant_f32 / gs_dequant_f16 (one thread per unit) and by gs_gemm's tiles (each
// lane decodes its own units from the raw super-blocks staged in LDS, then rounds them to f16).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#pragma clang fp contract(off)

namespace exact {

__device__ __forceinline__ float half_at(const uint8_t *b, int off) {
    const uint16_t h = (uint16_t)(b[off] | (b[off + 1] << 8));
    return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint32_t le32(const uint8_t *b, int off) {
    return (uint32_t)b[off] | ((uint32_t)b[off + 1] << 8) | ((uint32_t)b[off + 2] << 16) | ((uint32_t)b[off + 3] << 24);
}
// ggml get_scale_min_k4 (lib.rs:87-93): 6-bit scale and min of sub-block j from the 12 packed bytes
// dl * q - ml of the K-quants with mins (Q2_K, Q4_K, Q5_K) as one fused multiply-add: dl is an f16
// times a scale of at most 6 bits (at most 17 significant bits) and q has at most 5, so dl * q is
// exact in f32 and the single rounding of the fma equals lib.rs's rounding of the subtraction
__device__ __forceinline__ float dq_min(float dl, float q, float ml) { return __builtin_fmaf(dl, q, -ml); }

__device__ __forceinline__ void k4_scale_min(int j, const uint8_t *q, float &sc, float &mn) {
    uint32_t s, m;
    if (j < 4) {
        s = q[j] & 63u;
        m = q[j + 4] & 63u;
    } else {
        s = (q[j + 4] & 0xFu) | ((uint32_t)(q[j - 4] >> 6) << 4);
        m = (uint32_t)(q[j + 4] >> 4) | ((uint32_t)(q[j] >> 6) << 4);
    }
    sc = (float)s;
    mn = (float)m;
}
// sign of element j of a ksigns byte (lib.rs:265-271), applied as a multiplication by +-1
__device__ __forceinline__ float sgn(uint32_t signs, int j) { return (signs >> j) & 1u ? -1.0f : 1.0f; }

// ---- plain values: u is unused, b points at the unit's first element ------------------------
__device__ __forceinline__ void f32(const uint8_t *b, int, float (&y)[32]) {
    for (int i = 0; i < 32; i++) y[i] = __builtin_bit_cast(float, le32(b, 4 * i));
}
__device__ __forceinline__ void f16(const uint8_t *b, int, float (&y)[32]) {
    for (int i = 0; i < 32; i++) y[i] = half_at(b, 2 * i);
}
__device__ __forceinline__ void bf16(const uint8_t *b, int, float (&y)[32]) {
    for (int i = 0; i < 32; i++) y[i] = __builtin_bit_cast(float, (uint32_t)(b[2 * i] | (b[2 * i + 1] << 8)) << 16);
}

// ---- block_q8_0 { half d; i8 qs[32] } (lib.rs:131-136) ---------------------------------------
__device__ __forceinline__ void q8_0(const uint8_t *b, int, float (&y)[32]) {
    const float d = half_at(b, 0);
    for (int i = 0; i < 32; i++) y[i] = (float)(int8_t)b[2 + i] * d;
}

// ---- block_q2_K { u8 scales[16]; u8 qs[64]; half d; half dmin } (lib.rs:139-160) ------------
// lib.rs walks two 128-element halves n, four 2-bit planes (shift 2j) and two 16-element
// sub-blocks per plane, advancing the scale index is = 8n + 2j + half; unit u is plane j = u % 4
// of half n = u / 4.
__device__ __forceinline__ void q2_k(const uint8_t *b, int u, float (&y)[32]) {
    const int n = u >> 2, shift = 2 * (u & 3);
    const float d = half_at(b, 80), mn = half_at(b, 82);
    const uint8_t *q = b + 16 + 32 * n;
    for (int half = 0; half < 2; half++) {
        const uint32_t sc = b[8 * n + 2 * (u & 3) + half];
        const float dl = d * (float)(sc & 0xFu), ml = mn * (float)(sc >> 4);
        for (int l = 0; l < 16; l++) y[16 * half + l] = dq_min(dl, (float)((q[l + 16 * half] >> shift) & 3), ml);
    }
}

// ---- block_q3_K { u8 hmask[32]; u8 qs[64]; u8 scales[12]; half d } (lib.rs:163-201) --------
// The sixteen 6-bit scales are unpacked from the 12 raw bytes through lib.rs's four aux words;
// the walk over halves, planes and sub-blocks is Q2_K's, with hmask bit 4n + j as the high bit.
__device__ __forceinline__ void q3_k(const uint8_t *b, int u, float (&y)[32]) {
    const uint32_t K1 = 0x03030303u, K2 = 0x0f0f0f0fu;
    const uint32_t r0 = le32(b, 96), r1 = le32(b, 100), r2 = le32(b, 104);
    const uint32_t aux[4] = {(r0 & K2) | ((r2 & K1) << 4), (r1 & K2) | (((r2 >> 2) & K1) << 4),
                             ((r0 >> 4) & K2) | (((r2 >> 4) & K1) << 4), ((r1 >> 4) & K2) | (((r2 >> 6) & K1) << 4)};
    const int n = u >> 2, j = u & 3, shift = 2 * j;
    const float d = half_at(b, 108);
    const uint32_t m = 1u << (4 * n + j);
    const uint8_t *q = b + 32 + 32 * n;
    for (int half = 0; half < 2; half++) {
        const int is = 8 * n + 2 * j + half;
        const int sc = (int)(int8_t)((aux[is >> 2] >> (8 * (is & 3))) & 0xffu);
        const float dl = d * (float)(sc - 32);
        for (int l = 0; l < 16; l++) {
            const int qv = (q[l + 16 * half] >> shift) & 3;
            const int hv = (b[l + 16 * half] & m) ? 0 : 4;
            y[16 * half + l] = dl * (float)(qv - hv);
        }
    }
}

// ---- block_q4_K { half d; half dmin; u8 scales[12]; u8 qs[128] } (lib.rs:204-218) ----------
// 32-byte chunk jb of qs holds sub-block 2jb in its low nibbles and 2jb+1 in its high ones.
__device__ __forceinline__ void q4_k(const uint8_t *b, int u, float (&y)[32]) {
    const int jb = u >> 1, nib = 4 * (u & 1);
    float sc, mn;
    k4_scale_min(u, b + 4, sc, mn);
    const float dl = half_at(b, 0) * sc, ml = half_at(b, 2) * mn;
    const uint8_t *q = b + 16 + 32 * jb;
    for (int l = 0; l < 32; l++) y[l] = dq_min(dl, (float)((q[l] >> nib) & 0xF), ml);
}

// ---- block_q5_K { half d; half dmin; u8 scales[12]; u8 qh[32]; u8 qs[128] } (lib.rs:221-240)
// as Q4_K, plus bit u of qh[l] as the fifth bit (lib.rs's u1 = 1 << 2jb, u2 = 2 << 2jb)
__device__ __forceinline__ void q5_k(const uint8_t *b, int u, float (&y)[32]) {
    const int jb = u >> 1, nib = 4 * (u & 1);
    float sc, mn;
    k4_scale_min(u, b + 4, sc, mn);
    const float dl = half_at(b, 0) * sc, ml = half_at(b, 2) * mn;
    const uint8_t *q = b + 48 + 32 * jb;
    for (int l = 0; l < 32; l++) {
        const uint32_t v = ((q[l] >> nib) & 0xFu) + ((b[16 + l] >> u) & 1u) * 16u;
        y[l] = dq_min(dl, (float)v, ml);
    }
}

// ---- block_q6_K { u8 ql[128]; u8 qh[64]; i8 scales[16]; half d } (lib.rs:243-262) ----------
// Half n = u / 4 holds four 32-element quarters k = u % 4: low nibbles of ql[l] (k = 0) and
// ql[l+32] (k = 1), high nibbles of the same (k = 2, 3), 2-bit planes 2k of qh[l]; element l
// takes scale l / 16 + 2k. lib.rs's product order: (d * scale) * (q - 32).
__device__ __forceinline__ void q6_k(const uint8_t *b, int u, float (&y)[32]) {
    const int n = u >> 2, k = u & 3;
    const float d = half_at(b, 208);
    const uint8_t *ql = b + 64 * n + 32 * (k & 1), *qh = b + 128 + 32 * n;
    const int8_t *sc = (const int8_t *)(b + 192 + 8 * n);
    for (int l = 0; l < 32; l++) {
        const int q = (int)(((ql[l] >> (4 * (k >> 1))) & 0xF) | (((qh[l] >> (2 * k)) & 3) << 4)) - 32;
        y[l] = d * (float)sc[l / 16 + 2 * k] * (float)q;
    }
}

// ---- block_iq2_xxs { half d; u16 qs[32] } (lib.rs:274-288) ----------------------------------
__device__ __forceinline__ void iq2_xxs(const uint8_t *b, int u, float (&y)[32]) {
    const uint32_t a0 = le32(b, 2 + 8 * u), a1 = le32(b, 6 + 8 * u);
    const float db = half_at(b, 0) * (0.5f + (float)(a1 >> 28)) * 0.25f;
    for (int l = 0; l < 4; l++) {
        const uint64_t grid = iq2xxs_grid[(a0 >> (8 * l)) & 0xff];
        const uint32_t signs = ksigns_of((a1 >> (7 * l)) & 127);
        for (int j = 0; j < 8; j++) y[8 * l + j] = db * (float)((grid >> (8 * j)) & 0xff) * sgn(signs, j);
    }
}

// ---- block_iq2_s { half d; u8 qs[32]; u8 signs[32]; u8 qh[8]; u8 scales[8] } (lib.rs:291-310)
__device__ __forceinline__ void iq2_s(const uint8_t *b, int u, float (&y)[32]) {
    const float d = half_at(b, 0);
    const uint32_t sc = b[74 + u];
    const float db[2] = {d * (0.5f + (float)(sc & 0xf)) * 0.25f, d * (0.5f + (float)(sc >> 4)) * 0.25f};
    for (int l = 0; l < 4; l++) {
        const uint32_t idx = b[2 + 4 * u + l] | (((uint32_t)b[66 + u] << (8 - 2 * l)) & 0x300u);
        const uint64_t grid = iq2s_grid[idx];
        const uint32_t s = b[34 + 4 * u + l];
        for (int j = 0; j < 8; j++) y[8 * l + j] = db[l >> 1] * (float)((grid >> (8 * j)) & 0xff) * sgn(s, j);
    }
}

// ---- block_iq3_xxs { half d; u8 qs[64]; u8 scales_and_signs[32] } (lib.rs:312-328) ----------
__device__ __forceinline__ void iq3_xxs(const uint8_t *b, int u, float (&y)[32]) {
    const uint32_t aux = le32(b, 66 + 4 * u);
    const float db = half_at(b, 0) * (0.5f + (float)(aux >> 28)) * 0.5f;
    for (int l = 0; l < 4; l++) {
        const uint32_t signs = ksigns_of((aux >> (7 * l)) & 127);
        const uint32_t g1 = iq3xxs_grid[b[2 + 8 * u + 2 * l]], g2 = iq3xxs_grid[b[3 + 8 * u + 2 * l]];
        for (int j = 0; j < 4; j++) {
            y[8 * l + j] = db * (float)((g1 >> (8 * j)) & 0xff) * sgn(signs, j);
            y[8 * l + j + 4] = db * (float)((g2 >> (8 * j)) & 0xff) * sgn(signs, j + 4);
        }
    }
}

// ---- block_iq4_xs { half d; u16 scales_h; u8 scales_l[4]; u8 qs[128] } (lib.rs:331-343) -----
__device__ __forceinline__ void iq4_xs(const uint8_t *b, int u, float (&y)[32]) {
    const uint32_t sh = (uint32_t)(b[2] | (b[3] << 8));
    const int ls = (int)(((uint32_t)b[4 + u / 2] >> (4 * (u % 2))) & 0xfu) | (int)(((sh >> (2 * u)) & 3u) << 4);
    const float dl = half_at(b, 0) * (float)(ls - 32);
    const uint8_t *q = b + 8 + 16 * u;
    for (int j = 0; j < 16; j++) {
        y[j] = dl * (float)kvalues_iq4nl[q[j] & 0xf];
        y[j + 16] = dl * (float)kvalues_iq4nl[q[j] >> 4];
    }
}

// ---- the same decoders over a 4-byte aligned copy of a 256-element group in LDS ---------------
// (gs_gemm stages each row's super-block into an LDS slot that starts on a dword.) They read whole
// dwords and convert bytes with shifts and masks, where the byte-wise decoders above compile to
// one LDS read per byte, and evaluate the same f32 expressions in the same order, so their output
// is bit-identical.
namespace al {
__device__ __forceinline__ uint32_t w32(const uint8_t *p, int off) { return *(const uint32_t *)(p + off); }
__device__ __forceinline__ float h16(uint32_t w, int hi) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(hi ? w >> 16 : w)); }
// the f16 at byte `off` (2-byte aligned) by itself: no byte past it is read
__device__ __forceinline__ float h16_at(const uint8_t *p, int off) {
    return (float)__builtin_bit_cast(_Float16, *(const uint16_t *)(p + off));
}
__device__ __forceinline__ float sbyte(uint32_t w, int i) { return (float)(int)(int8_t)(w >> (8 * i)); }
__device__ __forceinline__ float ubyte(uint32_t w, int i) { return (float)((w >> (8 * i)) & 0xffu); }
// a value whose bits the compiler must not track: byte i of it then converts with one
// v_cvt_f32_ubyte<i> instead of a bit-field extract of the known nibble plus a conversion
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm("" : "+v"(v));
    return v;
}

// Q8_0: unit u = block u of the group (34-byte blocks, so block u starts 2 (u & 1) bytes past a dword)
__device__ __forceinline__ void q8_0(const uint8_t *p, int u, float (&y)[32]) {
    const int o = 34 * u, base = o & ~3, sh = o & 3;
    uint32_t w[10];
    for (int i = 0; i < 10; i++) w[i] = w32(p, base + 4 * i);
    const float d = h16(w[0], sh);
    for (int k = 0; k < 8; k++) {
        const uint32_t q = sh ? w[k + 1] : __builtin_amdgcn_alignbyte(w[k + 1], w[k], 2);
        for (int i = 0; i < 4; i++) y[4 * k + i] = sbyte(q, i) * d;
    }
}

// Q4_K: d and dmin in dword 0, the 12 scale bytes in dwords 1..3, unit u's nibbles in the 32 qs
// bytes at 16 + 32 (u >> 1)
__device__ __forceinline__ void q4_k(const uint8_t *p, int u, float (&y)[32]) {
    const uint32_t dd = w32(p, 0);
    // scale_min_k4 (lib.rs:87-93) on byte j & 3 of the three scale dwords
    const uint32_t sh = 8u * (uint32_t)(u & 3);
    const uint32_t b1 = (w32(p, 4) >> sh) & 0xffu, b2 = (w32(p, 8) >> sh) & 0xffu, b3 = (w32(p, 12) >> sh) & 0xffu;
    // both forms computed and one selected (u varies across the lanes: no divergent branch)
    const uint32_t sc_lo = b1 & 63u, sc_hi = (b3 & 0xfu) | ((b1 >> 6) << 4);
    const uint32_t mn_lo = b2 & 63u, mn_hi = (b3 >> 4) | ((b2 >> 6) << 4);
    const uint32_t sci = u < 4 ? sc_lo : sc_hi, mni = u < 4 ? mn_lo : mn_hi;
    const float dl = h16(dd, 0) * (float)sci, ml = h16(dd, 1) * (float)mni;
    const int nib = 4 * (u & 1);
    for (int k = 0; k < 8; k++) {
        const uint32_t q = opaque((w32(p, 16 + 32 * (u >> 1) + 4 * k) >> nib) & 0x0f0f0f0fu);
        for (int i = 0; i < 4; i++) y[4 * k + i] = dq_min(dl, ubyte(q, i), ml);
    }
}

// Q8_0 block in global memory (34 bytes, 2-byte aligned): d as 16 bits, the 32 quants as the 8
// dwords at bytes 2..33 (unaligned loads). Reads no byte past the block, so the last block of an
// allocation is safe where q8_0 above, made for a dword-aligned LDS group, reads on to byte 35.
__device__ __forceinline__ void q8_0_block(const uint8_t *b, float (&y)[32]) {
    const float d = h16_at(b, 0);
    for (int k = 0; k < 8; k++) {
        const uint32_t q = w32(b, 2 + 4 * k);
        for (int i = 0; i < 4; i++) y[4 * k + i] = sbyte(q, i) * d;
    }
}

// Q6_K: unit u = quarter k = u % 4 of half n = u / 4; ql, qh and the int8 scales start on dwords;
// d (bytes 208-209, the block's last) is read as 16 bits, so nothing past the 210-byte block is
// read (the decoder also runs on blocks in global memory)
__device__ __forceinline__ void q6_k(const uint8_t *p, int u, float (&y)[32]) {
    const int n = u >> 2, k = u & 3;
    const float d = h16_at(p, 208);
    // scale bytes 2k and 2k + 1 of the half (elements 0..15, 16..31), in the dword at 4 (k >> 1)
    const uint32_t scw = w32(p, 192 + 8 * n + 4 * (k >> 1));
    const float s0 = d * sbyte(scw, 2 * (k & 1)), s1 = d * sbyte(scw, 2 * (k & 1) + 1);
    for (int m = 0; m < 8; m++) {
        const uint32_t lo = (w32(p, 64 * n + 32 * (k & 1) + 4 * m) >> (4 * (k >> 1))) & 0x0f0f0f0fu;
        const uint32_t hi = ((w32(p, 128 + 32 * n + 4 * m) >> (2 * k)) & 0x03030303u) << 4;
        const uint32_t q = opaque(lo | hi);
        for (int i = 0; i < 4; i++) y[4 * m + i] = (m < 4 ? s0 : s1) * (ubyte(q, i) - 32.f);
    }
}
}  // namespace al

}  // namespace exact

#pragma clang fp contract(fast)

// X(type id, elements per ggml block, bytes per ggml block, unit decoder)
#define GS_TYPE_LIST(X)                                                                          \
    X(0, 1, 4, exact::f32) X(1, 1, 2, exact::f16) X(30, 1, 2, exact::bf16)                        \
    X(8, 32, 34, exact::q8_0) X(10, 256, 84, exact::q2_k) X(11, 256, 110, exact::q3_k)           \
    X(12, 256, 144, exact::q4_k) X(13, 256, 176, exact::q5_k) X(14, 256, 210, exact::q6_k)       \
    X(16, 256, 66, exact::iq2_xxs) X(22, 256, 82, exact::iq2_s)                                  \
    X(18, 256, 98, exact::iq3_xxs) X(23, 256, 136, exact::iq4_xs)
