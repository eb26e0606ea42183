/* CPU oracle for the quantized-matmul hot path. TEST INFRASTRUCTURE ONLY: loaded by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the product library.
 *
 * Restates, in C, the reference's CPU path:
 *   - f16 <-> f32                 crates/quants/src/lib.rs:15-74
 *   - block geometry              crates/gguf/src/types.rs:85-122
 *   - dequantize (all 13 types)   crates/quants/src/lib.rs:96-343
 *   - qtest data generator        crates/engine/src/qtest.rs:27-60
 *   - f64 GEMV oracle             crates/engine/src/qtest.rs:101-108
 *   - SwiGLU clamp / MoE combine  crates/cuda/kernels/ops.cu:101-115, quants.cu:279-363
 * plus the q8_1 activation quantizer, which the reference does not have (it keeps activations in
 * f32). It is defined here after ggml's quantize_row_q8_1_ref convention.
 *
 * Parity pins (tests/test_oracle.py), each independent of the formula it checks:
 *   f16<->f32     exhaustive 65,536-pattern round trip (lib.rs:361-370) + numpy float16 casts.
 *   tables        SHA-256 of each ggml table vs the values in the reference's tables.rs;
 *                 closed forms ksigns[i] = i | parity(i)<<7, kmask[j] = 1<<j.
 *   Q8_0 / Q4_K / Q5_K / Q6_K / Q2_K / Q3_K / IQ4_XS
 *                 per-element closed forms from the struct layout, computed by an independent
 *                 numpy decoder over all code values (tests/test_oracle.py).
 *   IQ2_XXS / IQ2_S / IQ3_XXS
 *                 enumeration of grid index x sign index x scale against an independent
 *                 numpy decoder, exact products.
 *   q8_1          invariants (|q|<=127, max|q|==127, zero block, s == f16(d*sum q)),
 *                 reconstruction bound |x - d q| <= d/2, and numpy re-derivation.
 *   GEMV / FFN    brute force f64 numpy matmul of the oracle's own dequantized operands on small
 *                 shapes, and linearity in x.
 * Build with -ffp-contract=off: the reference's dequant arithmetic is unfused (d1*q - m1).
 */
#include "oracle.h"
#include "ggml_tables.h"
#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- f16 <-> f32 (crates/quants/src/lib.rs:15-74) ----------------------------------------- */
static float bits_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            uint32_t e = 113, m = man;
            while ((m & 0x400) == 0) { m <<= 1; e -= 1; }
            bits = sign | (e << 23) | ((m & 0x3ff) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    return bits_f32(bits);
}

uint16_t or_f32_to_f16(float f) { /* round to nearest even */
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    int32_t exp = (int32_t)((x >> 23) & 0xff);
    uint32_t man = x & 0x7fffff;
    if (exp == 0xff) return sign | 0x7c00 | (man ? 0x200 : 0);
    int32_t e = exp - 127 + 15;
    if (e >= 31) return sign | 0x7c00;
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = man | 0x800000;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half = 1u << (shift - 1);
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t r = m >> shift;
        if (rem > half || (rem == half && (r & 1))) r += 1;
        return sign | (uint16_t)r;
    }
    uint32_t rem = man & 0x1fff;
    uint32_t r = ((uint32_t)e << 10) | (man >> 13);
    if (rem > 0x1000 || (rem == 0x1000 && (r & 1))) r += 1;
    return sign | (uint16_t)r;
}

/* ---- block geometry (crates/gguf/src/types.rs:85-113) ------------------------------------- */
int or_block(int ty, int *elems, int *bytes) {
    int e, b;
    switch (ty) {
        case OR_F32: e = 1; b = 4; break;
        case OR_F16: case OR_BF16: e = 1; b = 2; break;
        case OR_Q8_0: e = 32; b = 34; break;
        case OR_Q2_K: e = 256; b = 84; break;
        case OR_Q3_K: e = 256; b = 110; break;
        case OR_Q4_K: e = 256; b = 144; break;
        case OR_Q5_K: e = 256; b = 176; break;
        case OR_Q6_K: e = 256; b = 210; break;
        case OR_IQ2_XXS: e = 256; b = 66; break;
        case OR_IQ2_S: e = 256; b = 82; break;
        case OR_IQ3_XXS: e = 256; b = 98; break;
        case OR_IQ4_XS: e = 256; b = 136; break;
        default: return -1;
    }
    if (elems) *elems = e;
    if (bytes) *bytes = b;
    return 0;
}

static float hf(const uint8_t *b, int off) { return or_f16_to_f32((uint16_t)(b[off] | (b[off + 1] << 8))); }
static uint32_t u32le(const uint8_t *b, int off) {
    return (uint32_t)b[off] | ((uint32_t)b[off + 1] << 8) | ((uint32_t)b[off + 2] << 16) | ((uint32_t)b[off + 3] << 24);
}
/* KSIGNS_IQ2XS / KMASK_IQ2XS as data (crates/quants/src/tables.rs:5-18) */
static uint8_t ksigns_tab[128];
static const uint8_t kmask_tab[8] = {1, 2, 4, 8, 16, 32, 64, 128};
static const uint8_t ksigns_data[128] = {
    0, 129, 130, 3, 132, 5, 6, 135, 136, 9, 10, 139, 12, 141, 142, 15,
    144, 17, 18, 147, 20, 149, 150, 23, 24, 153, 154, 27, 156, 29, 30, 159,
    160, 33, 34, 163, 36, 165, 166, 39, 40, 169, 170, 43, 172, 45, 46, 175,
    48, 177, 178, 51, 180, 53, 54, 183, 184, 57, 58, 187, 60, 189, 190, 63,
    192, 65, 66, 195, 68, 197, 198, 71, 72, 201, 202, 75, 204, 77, 78, 207,
    80, 209, 210, 83, 212, 85, 86, 215, 216, 89, 90, 219, 92, 221, 222, 95,
    96, 225, 226, 99, 228, 101, 102, 231, 232, 105, 106, 235, 108, 237, 238, 111,
    240, 113, 114, 243, 116, 245, 246, 119, 120, 249, 250, 123, 252, 125, 126, 255,
};
static float sgn(uint8_t signs, int j) { return (signs & kmask_tab[j]) ? -1.0f : 1.0f; } /* lib.rs:265-271 */

/* exported for the table-pinning tests */
const uint8_t *or_table_ksigns(void) { memcpy(ksigns_tab, ksigns_data, 128); return ksigns_tab; }
const uint64_t *or_table_iq2xxs(void) { return iq2xxs_grid; }
const uint64_t *or_table_iq2s(void) { return iq2s_grid; }
const uint32_t *or_table_iq3xxs(void) { return iq3xxs_grid; }
const int8_t *or_table_iq4nl(void) { return kvalues_iq4nl; }

/* scale_min_k4 (lib.rs:87-93) */
static void scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ---- per-block decoders (crates/quants/src/lib.rs:131-343) -------------------------------- */
static void dq_q8_0(const uint8_t *b, float *y) { /* lib.rs:131-136 */
    float d = hf(b, 0);
    for (int j = 0; j < 32; j++) y[j] = (float)(int8_t)b[2 + j] * d;
}

static void dq_q2_k(const uint8_t *b, float *y) { /* lib.rs:139-160 */
    const uint8_t *scales = b, *qs = b + 16;
    float d = hf(b, 80), mn = hf(b, 82);
    int yi = 0, is = 0;
    for (int n = 0; n < 256; n += 128) {
        const uint8_t *q = qs + n / 4;
        int shift = 0;
        for (int j = 0; j < 4; j++) {
            for (int half = 0; half < 2; half++) {
                uint8_t sc = scales[is++];
                float dl = d * (float)(sc & 0xF), ml = mn * (float)(sc >> 4);
                for (int l = 0; l < 16; l++) y[yi++] = dl * (float)((q[l + 16 * half] >> shift) & 3) - ml;
            }
            shift += 2;
        }
    }
}

static void dq_q3_k(const uint8_t *b, float *y) { /* lib.rs:163-201 */
    const uint8_t *hm = b, *qs = b + 32, *raw = b + 96;
    float d_all = hf(b, 108);
    const uint32_t KM1 = 0x03030303u, KM2 = 0x0f0f0f0fu;
    uint32_t aux[4] = {u32le(raw, 0), u32le(raw, 4), u32le(raw, 8), 0};
    uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & KM2) | (((tmp >> 4) & KM1) << 4);
    aux[3] = ((aux[1] >> 4) & KM2) | (((tmp >> 6) & KM1) << 4);
    aux[0] = (aux[0] & KM2) | ((tmp & KM1) << 4);
    aux[1] = (aux[1] & KM2) | (((tmp >> 2) & KM1) << 4);
    int8_t scales[16];
    for (int i = 0; i < 4; i++)
        for (int k = 0; k < 4; k++) scales[4 * i + k] = (int8_t)(uint8_t)(aux[i] >> (8 * k));
    int yi = 0, is = 0;
    uint8_t m = 1;
    for (int n = 0; n < 256; n += 128) {
        const uint8_t *q = qs + n / 4;
        int shift = 0;
        for (int j = 0; j < 4; j++) {
            for (int half = 0; half < 2; half++) {
                float dl = d_all * (float)((int)scales[is] - 32);
                is++;
                for (int l = 0; l < 16; l++) {
                    int qv = (q[l + 16 * half] >> shift) & 3;
                    int hv = (hm[l + 16 * half] & m) ? 0 : 4;
                    y[yi++] = dl * (float)(qv - hv);
                }
            }
            shift += 2;
            m = (uint8_t)(m << 1);
        }
    }
}

static void dq_q4_k(const uint8_t *b, float *y) { /* lib.rs:204-218 */
    float d = hf(b, 0), mn = hf(b, 2);
    const uint8_t *scales = b + 4, *qs = b + 16;
    int yi = 0;
    for (int jb = 0; jb < 4; jb++) {
        const uint8_t *q = qs + 32 * jb;
        uint8_t sc1, m1, sc2, m2;
        scale_min_k4(2 * jb, scales, &sc1, &m1);
        scale_min_k4(2 * jb + 1, scales, &sc2, &m2);
        float d1 = d * (float)sc1, fm1 = mn * (float)m1, d2 = d * (float)sc2, fm2 = mn * (float)m2;
        for (int l = 0; l < 32; l++) {
            y[yi + l] = d1 * (float)(q[l] & 0xF) - fm1;
            y[yi + 32 + l] = d2 * (float)(q[l] >> 4) - fm2;
        }
        yi += 64;
    }
}

static void dq_q5_k(const uint8_t *b, float *y) { /* lib.rs:221-240 */
    float d = hf(b, 0), mn = hf(b, 2);
    const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
    int yi = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int jb = 0; jb < 4; jb++) {
        const uint8_t *ql = qs + 32 * jb;
        uint8_t sc1, m1, sc2, m2;
        scale_min_k4(2 * jb, scales, &sc1, &m1);
        scale_min_k4(2 * jb + 1, scales, &sc2, &m2);
        float d1 = d * (float)sc1, fm1 = mn * (float)m1, d2 = d * (float)sc2, fm2 = mn * (float)m2;
        for (int l = 0; l < 32; l++) {
            int hi1 = (qh[l] & u1) ? 16 : 0, hi2 = (qh[l] & u2) ? 16 : 0;
            y[yi + l] = d1 * (float)((ql[l] & 0xF) + hi1) - fm1;
            y[yi + 32 + l] = d2 * (float)((ql[l] >> 4) + hi2) - fm2;
        }
        yi += 64;
        u1 = (uint8_t)(u1 << 2);
        u2 = (uint8_t)(u2 << 2);
    }
}

static void dq_q6_k(const uint8_t *b, float *y) { /* lib.rs:243-262 */
    float d = hf(b, 208);
    for (int n = 0; n < 2; n++) {
        const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n, *sc = b + 192 + 8 * n;
        float *yo = y + 128 * n;
        for (int l = 0; l < 32; l++) {
            int is = l / 16;
            int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
            int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            yo[l] = d * (float)(int8_t)sc[is] * (float)q1;
            yo[l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
            yo[l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
            yo[l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
        }
    }
}

static void dq_iq2_xxs(const uint8_t *b, float *y) { /* lib.rs:274-288 */
    float d = hf(b, 0);
    for (int ib32 = 0; ib32 < 8; ib32++) {
        uint32_t a0 = u32le(b, 2 + 8 * ib32), a1 = u32le(b, 2 + 8 * ib32 + 4);
        float db = d * (0.5f + (float)(a1 >> 28)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            uint64_t grid = iq2xxs_grid[(a0 >> (8 * l)) & 0xff];
            uint8_t signs = ksigns_data[(a1 >> (7 * l)) & 127];
            for (int j = 0; j < 8; j++)
                y[32 * ib32 + 8 * l + j] = db * (float)(uint8_t)(grid >> (8 * j)) * sgn(signs, j);
        }
    }
}

static void dq_iq2_s(const uint8_t *b, float *y) { /* lib.rs:291-310 */
    float d = hf(b, 0);
    const uint8_t *qs = b + 2, *signs = b + 34, *qh = b + 66, *scales = b + 74;
    for (int ib32 = 0; ib32 < 8; ib32++) {
        float db[2] = {d * (0.5f + (float)(scales[ib32] & 0xf)) * 0.25f, d * (0.5f + (float)(scales[ib32] >> 4)) * 0.25f};
        for (int l = 0; l < 4; l++) {
            float dl = db[l / 2];
            int idx = qs[4 * ib32 + l] | (((int)qh[ib32] << (8 - 2 * l)) & 0x300);
            uint64_t grid = iq2s_grid[idx];
            uint8_t s = signs[4 * ib32 + l];
            for (int j = 0; j < 8; j++) y[32 * ib32 + 8 * l + j] = dl * (float)(uint8_t)(grid >> (8 * j)) * sgn(s, j);
        }
    }
}

static void dq_iq3_xxs(const uint8_t *b, float *y) { /* lib.rs:313-328 */
    float d = hf(b, 0);
    const uint8_t *qs = b + 2;
    for (int ib32 = 0; ib32 < 8; ib32++) {
        uint32_t aux = u32le(b, 66 + 4 * ib32);
        float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
        for (int l = 0; l < 4; l++) {
            uint8_t signs = ksigns_data[(aux >> (7 * l)) & 127];
            uint32_t g1 = iq3xxs_grid[qs[8 * ib32 + 2 * l]], g2 = iq3xxs_grid[qs[8 * ib32 + 2 * l + 1]];
            for (int j = 0; j < 4; j++) {
                y[32 * ib32 + 8 * l + j] = db * (float)(uint8_t)(g1 >> (8 * j)) * sgn(signs, j);
                y[32 * ib32 + 8 * l + j + 4] = db * (float)(uint8_t)(g2 >> (8 * j)) * sgn(signs, j + 4);
            }
        }
    }
}

static void dq_iq4_xs(const uint8_t *b, float *y) { /* lib.rs:331-343 */
    float d = hf(b, 0);
    uint16_t scales_h = (uint16_t)(b[2] | (b[3] << 8));
    const uint8_t *scales_l = b + 4, *qs = b + 8;
    for (int ib = 0; ib < 8; ib++) {
        int ls = ((scales_l[ib / 2] >> (4 * (ib % 2))) & 0xf) | (((scales_h >> (2 * ib)) & 3) << 4);
        float dl = d * (float)(ls - 32);
        for (int j = 0; j < 16; j++) {
            y[32 * ib + j] = dl * (float)kvalues_iq4nl[qs[16 * ib + j] & 0xf];
            y[32 * ib + j + 16] = dl * (float)kvalues_iq4nl[qs[16 * ib + j] >> 4];
        }
    }
}

/* dequantize (lib.rs:96-123): n elements, a whole number of blocks */
int or_dequantize(int ty, const uint8_t *src, int64_t n, float *y) {
    int be, bb;
    if (or_block(ty, &be, &bb) != 0 || n % be != 0) return -1;
    int64_t nb = n / be;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t *blk = src + i * bb;
        float *out = y + i * be;
        switch (ty) {
            case OR_F32: memcpy(out, blk, 4); break;
            case OR_F16: out[0] = hf(blk, 0); break;
            case OR_BF16: out[0] = bits_f32((uint32_t)(blk[0] | (blk[1] << 8)) << 16); break;
            case OR_Q8_0: dq_q8_0(blk, out); break;
            case OR_Q2_K: dq_q2_k(blk, out); break;
            case OR_Q3_K: dq_q3_k(blk, out); break;
            case OR_Q4_K: dq_q4_k(blk, out); break;
            case OR_Q5_K: dq_q5_k(blk, out); break;
            case OR_Q6_K: dq_q6_k(blk, out); break;
            case OR_IQ2_XXS: dq_iq2_xxs(blk, out); break;
            case OR_IQ2_S: dq_iq2_s(blk, out); break;
            case OR_IQ3_XXS: dq_iq3_xxs(blk, out); break;
            case OR_IQ4_XS: dq_iq4_xs(blk, out); break;
            default: return -1;
        }
    }
    return 0;
}

/* ---- q8_1 activation quantizer (build-defined; no counterpart in the reference) -----------
 * After ggml's quantize_row_q8_1_ref: per block of 32, d = amax/127, id = d ? 1/d : 0,
 * q = roundf(x*id) (round half away from zero), stored d = f16(d), s = f16(d * sum q)
 * (d here is the unrounded f32 d). Dequantized value: f16->f32(stored d) * q. */
void or_quantize_q8_1(const float *x, int64_t n, uint8_t *out) {
    for (int64_t ib = 0; ib < n / 32; ib++) {
        const float *xb = x + 32 * ib;
        uint8_t *ob = out + OR_Q8_1_BYTES * ib;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            float a = fabsf(xb[j]);
            if (a > amax) amax = a;
        }
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        /* 1/d overflows for d < 2^-128 (a block of tiny subnormals): q = 0, as the stored f16 d is
           0 for such a block anyway (the int conversion of an infinite product is undefined) */
        if (!(id <= FLT_MAX)) id = 0.0f;
        int sum = 0;
        for (int j = 0; j < 32; j++) {
            float v = xb[j] * id;
            int q = (int)roundf(v);
            ob[4 + j] = (uint8_t)(int8_t)q;
            sum += q;
        }
        uint16_t dh = or_f32_to_f16(d), sh = or_f32_to_f16((float)sum * d);
        ob[0] = (uint8_t)dh; ob[1] = (uint8_t)(dh >> 8);
        ob[2] = (uint8_t)sh; ob[3] = (uint8_t)(sh >> 8);
    }
}

void or_dequantize_q8_1(const uint8_t *q, int64_t n, float *y) {
    for (int64_t ib = 0; ib < n / 32; ib++) {
        const uint8_t *b = q + OR_Q8_1_BYTES * ib;
        float d = hf(b, 0);
        for (int j = 0; j < 32; j++) y[32 * ib + j] = d * (float)(int8_t)b[4 + j];
    }
}

/* ---- qtest.rs test-data generator (qtest.rs:27-60) ---------------------------------------- */
uint64_t or_rng_next(uint64_t *s) { /* xorshift64* */
    *s ^= *s >> 12;
    *s ^= *s << 25;
    *s ^= *s >> 27;
    return *s * 0x2545f4914f6cdd1dull;
}
float or_rng_f32(uint64_t *s) { return (float)(or_rng_next(s) >> 40) / (float)(1u << 24); }

static int half_offsets(int ty, int *offs) { /* lib.rs:346-356 */
    switch (ty) {
        case OR_Q8_0: case OR_IQ2_XXS: case OR_IQ2_S: case OR_IQ3_XXS: case OR_IQ4_XS: offs[0] = 0; return 1;
        case OR_Q2_K: offs[0] = 80; offs[1] = 82; return 2;
        case OR_Q3_K: offs[0] = 108; return 1;
        case OR_Q4_K: case OR_Q5_K: offs[0] = 0; offs[1] = 2; return 2;
        case OR_Q6_K: offs[0] = 208; return 1;
        default: return 0;
    }
}

int or_random_blocks(int ty, int64_t n_elems, uint64_t *s, uint8_t *v) {
    int be, bb;
    if (or_block(ty, &be, &bb) != 0 || n_elems % be != 0) return -1;
    int64_t nblk = n_elems / be;
    for (int64_t i = 0; i < nblk * bb; i++) v[i] = (uint8_t)or_rng_next(s);
    int offs[2];
    int nh = half_offsets(ty, offs);
    for (int64_t i = 0; i < nblk; i++) {
        uint8_t *blk = v + i * bb;
        if (ty == OR_F32) {
            float f = or_rng_f32(s) * 2.0f - 1.0f;
            memcpy(blk, &f, 4);
        } else if (ty == OR_F16) {
            uint16_t h = or_f32_to_f16(or_rng_f32(s) * 2.0f - 1.0f);
            blk[0] = (uint8_t)h; blk[1] = (uint8_t)(h >> 8);
        } else {
            for (int k = 0; k < nh; k++) {
                float mag = 1e-3f + or_rng_f32(s) * 5e-2f;
                float val = (or_rng_next(s) & 1) == 0 ? mag : -mag;
                uint16_t h = or_f32_to_f16(val);
                blk[offs[k]] = (uint8_t)h; blk[offs[k] + 1] = (uint8_t)(h >> 8);
            }
        }
    }
    return 0;
}

/* ---- f64 GEMV (qtest.rs:101-108, with q8_1 activations) ----------------------------------- */
typedef struct {
    int ty, K, rows, B, r0, r1;
    const uint8_t *W;
    int64_t row_stride;
    const float *xh; /* [B][K] dequantized activations */
    double *y;
    int mode;        /* OR_ACT_*: OR_ACT_F16 also rounds the dequantized weights to half */
} gemv_job;

static void *gemv_worker(void *p) {
    gemv_job *j = (gemv_job *)p;
    float *w = (float *)malloc(sizeof(float) * (size_t)j->K);
    for (int r = j->r0; r < j->r1; r++) {
        or_dequantize(j->ty, j->W + (int64_t)r * j->row_stride, j->K, w);
        if (j->mode == OR_ACT_F16 || j->mode == OR_ACT_F16S)
            for (int k = 0; k < j->K; k++) w[k] = or_f16_to_f32(or_f32_to_f16(w[k]));
        for (int b = 0; b < j->B; b++) {
            const float *xv = j->xh + (int64_t)b * j->K;
            double acc = 0.0;
            for (int k = 0; k < j->K; k++) acc += (double)w[k] * (double)xv[k];
            j->y[(int64_t)b * j->rows + r] = acc;
        }
    }
    free(w);
    return NULL;
}

static void quant_dequant_row(const float *x, int K, float *xh, int mode) {
    if (mode == OR_ACT_F32) { memcpy(xh, x, sizeof(float) * (size_t)K); return; }
    if (mode == OR_ACT_F16 || mode == OR_ACT_F16X) {
        for (int k = 0; k < K; k++) xh[k] = or_f16_to_f32(or_f32_to_f16(x[k]));
        return;
    }
    if (mode == OR_ACT_F16S || mode == OR_ACT_F16SX) {
        float amax = 0.0f;
        for (int k = 0; k < K; k++) amax = fmaxf(amax, fabsf(x[k]));
        int E = 0;
        if (amax > 0.0f && amax <= 3.4e38f) (void)frexpf(amax, &E);   /* amax < 2^E */
        E -= 15;
        for (int k = 0; k < K; k++) xh[k] = ldexpf(or_f16_to_f32(or_f32_to_f16(ldexpf(x[k], -E))), E);
        return;
    }
    uint8_t *q = (uint8_t *)malloc((size_t)(K / 32) * OR_Q8_1_BYTES);
    or_quantize_q8_1(x, K, q);
    or_dequantize_q8_1(q, K, xh);
    free(q);
}

int or_gemv(int ty, const uint8_t *W, int64_t row_stride, int K, int rows, const float *x, int64_t x_stride,
            int B, int quant_x, double *y, int nthreads) {
    int be, bb;
    if (or_block(ty, &be, &bb) != 0 || K % be != 0 || B < 1 || quant_x < 0 || quant_x > 5) return -1;
    if (quant_x == OR_ACT_Q8_1 ? K % 32 != 0 : K % 8 != 0) return -1;   /* q8_1 units of 32; plain rows of 8 */
    float *xh = (float *)malloc(sizeof(float) * (size_t)K * B);
    for (int b = 0; b < B; b++) quant_dequant_row(x + (int64_t)b * x_stride, K, xh + (int64_t)b * K, quant_x);
    if (nthreads < 1) nthreads = 1;
    if (nthreads > rows) nthreads = rows;
    gemv_job *jobs = (gemv_job *)calloc((size_t)nthreads, sizeof(gemv_job));
    pthread_t *th = (pthread_t *)calloc((size_t)nthreads, sizeof(pthread_t));
    for (int t = 0; t < nthreads; t++) {
        gemv_job j = {ty, K, rows, B, (int)((int64_t)rows * t / nthreads), (int)((int64_t)rows * (t + 1) / nthreads),
                      W, row_stride, xh, y, quant_x};
        jobs[t] = j;
        if (nthreads == 1) gemv_worker(&jobs[t]);
        else pthread_create(&th[t], NULL, gemv_worker, &jobs[t]);
    }
    if (nthreads > 1)
        for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    free(jobs); free(th); free(xh);
    return 0;
}

/* ---- SwiGLU with clamp (ops.cu:101-115): silu(min(g, L)) * clamp(u, -L, L); L <= 0: none ---- */
double or_swiglu(double g, double u, double lim) {
    if (lim > 0.0) {
        if (g > lim) g = lim;
        if (u > lim) u = lim;
        if (u < -lim) u = -lim;
    }
    return g / (1.0 + exp(-g)) * u;
}

/* ---- routed-expert FFN (quants.cu:279-363 semantics; q8_1 on x and h) --------------------- */
int or_moe_ffn(int ty_gu, int ty_down, const uint8_t *const *gate, const uint8_t *const *up,
               const uint8_t *const *down, int64_t gu_row_stride, int64_t down_row_stride, int n_embd, int n_ff,
               int T, const float *x, int n_pairs, const int *pair_tok, const int *pair_exp, const float *pair_w,
               float lim, double *y, float *h_out, int nthreads, int act_mode) {
    double *g = (double *)malloc(sizeof(double) * (size_t)n_ff);
    double *u = (double *)malloc(sizeof(double) * (size_t)n_ff);
    double *o = (double *)malloc(sizeof(double) * (size_t)n_embd);
    float *h = (float *)malloc(sizeof(float) * (size_t)n_ff);
    int rc = 0;
    for (int p = 0; p < n_pairs && rc == 0; p++) {
        int t = pair_tok[p], e = pair_exp[p];
        if (t < 0 || t >= T) { rc = -1; break; }
        const float *xt = x + (int64_t)t * n_embd;
        rc |= or_gemv(ty_gu, gate[e], gu_row_stride, n_embd, n_ff, xt, n_embd, 1, act_mode, g, nthreads);
        rc |= or_gemv(ty_gu, up[e], gu_row_stride, n_embd, n_ff, xt, n_embd, 1, act_mode, u, nthreads);
        for (int r = 0; r < n_ff; r++) h[r] = (float)or_swiglu(g[r], u[r], lim);
        if (h_out) memcpy(h_out + (int64_t)p * n_ff, h, sizeof(float) * (size_t)n_ff);
        rc |= or_gemv(ty_down, down[e], down_row_stride, n_ff, n_embd, h, n_ff, 1, act_mode, o, nthreads);
        if (pair_w[p] != 0.0f)
            for (int r = 0; r < n_embd; r++) y[(int64_t)t * n_embd + r] += (double)pair_w[p] * o[r];
    }
    free(g); free(u); free(o); free(h);
    return rc;
}
