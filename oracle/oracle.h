/* CPU oracle for the quantized-matmul hot path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library, and only as the checker (or as the timed CPU baseline). The product library
 * (libglmssd_hip.so) never links or calls it.
 *
 * Every function restates the reference's CPU path (GLM-SSD crates/quants, qtest.rs,
 * quants.cu / ops.cu semantics) in plain C; each definition cites the reference line it
 * follows. Parity pins (what checks each function independently of its own formula) are
 * listed in oracle.c's header comment.
 */
#ifndef GLMSSD_ORACLE_H
#define GLMSSD_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (crates/gguf/src/types.rs:74-82) */
enum {
    OR_F32 = 0, OR_F16 = 1, OR_Q8_0 = 8, OR_Q2_K = 10, OR_Q3_K = 11, OR_Q4_K = 12, OR_Q5_K = 13,
    OR_Q6_K = 14, OR_IQ2_XXS = 16, OR_IQ3_XXS = 18, OR_IQ2_S = 22, OR_IQ4_XS = 23, OR_BF16 = 30,
};

/* q8_1 activation block: { f16 d; f16 s; int8 qs[32] } = 36 bytes */
#define OR_Q8_1_BYTES 36

float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
int or_block(int ty, int *elems, int *bytes);
int or_dequantize(int ty, const uint8_t *src, int64_t n, float *y);
void or_quantize_q8_1(const float *x, int64_t n, uint8_t *out);
void or_dequantize_q8_1(const uint8_t *q, int64_t n, float *y);

/* qtest.rs test-data generator (xorshift64* + random_blocks) */
uint64_t or_rng_next(uint64_t *state);
float or_rng_f32(uint64_t *state);
int or_random_blocks(int ty, int64_t n_elems, uint64_t *state, uint8_t *out);

/* y[b*rows + r] = sum_k what[r][k] * xhat[b][k] in f64. Activation modes (quant_x):
 *   OR_ACT_F32  (0): xhat = x, what = deq(W)
 *   OR_ACT_Q8_1 (1): xhat = deq(q8_1(x)), what = deq(W)          (this build's GEMV / fused decode)
 *   OR_ACT_F16  (2): xhat = f16(x), what = f16(deq(W))            (the reference's multi-token GEMM,
 *                    crates/cuda/kernels/gemm.cu:57-78: weights dequantized then rounded to half,
 *                    activations converted to half, f32 accumulation)
 *   OR_ACT_F16X (3): xhat = f16(x), what = deq(W)                 (half activations, exact weights:
 *                    what this build's grouped MFMA GEMM computes)
 *   OR_ACT_F16S (4), OR_ACT_F16SX (5): as F16 / F16X, with each activation row first scaled by the
 *                    power of two 2^-E that puts its largest magnitude in [2^14, 2^15) and scaled
 *                    back after the half rounding (equal to F16 / F16X wherever those stay finite;
 *                    rows beyond the half range do not overflow)
 * nthreads > 1 splits rows over pthreads. */
#define OR_ACT_F32 0
#define OR_ACT_Q8_1 1
#define OR_ACT_F16 2
#define OR_ACT_F16X 3
#define OR_ACT_F16S 4
#define OR_ACT_F16SX 5
int or_gemv(int ty, const uint8_t *W, int64_t row_stride, int K, int rows, const float *x, int64_t x_stride,
            int B, int quant_x, double *y, int nthreads);

/* SwiGLU with clamp (ops.cu:101-115), in f64 */
double or_swiglu(double g, double u, double lim);

/* Routed-expert FFN for T tokens over n_pairs (token, expert, weight) pairs:
 *   g = gate_e·x̂; u = up_e·x̂; h = swiglu(g,u,lim) (rounded to f32); y[t] += w * down_e·ĥ,
 * with x̂, ĥ and the weights as or_gemv's act_mode says (OR_ACT_Q8_1: the fused decode path,
 * quants.cu:279-363; OR_ACT_F16: the multi-token path, forward.rs:1399-1413 over gemm.cu).
 * f64 throughout; y is added to, not cleared. experts: pointer arrays indexed by expert id.
 * h_out (optional) gets h per pair [n_pairs][n_ff]. */
int or_moe_ffn(int ty_gu, int ty_down, const uint8_t *const *gate, const uint8_t *const *up,
               const uint8_t *const *down, int64_t gu_row_stride, int64_t down_row_stride, int n_embd, int n_ff,
               int T, const float *x, int n_pairs, const int *pair_tok, const int *pair_exp, const float *pair_w,
               float lim, double *y, float *h_out, int nthreads, int act_mode);

#ifdef __cplusplus
}
#endif
#endif
