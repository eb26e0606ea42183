/* glmssd.h — C ABI of libglmssd_hip.so, the MI355X (gfx950) drop-in for GLM-SSD's quantized
 * matmul hot path.
 *
 * Every symbol below keeps the name, signature, argument meaning and error behaviour of the
 * entry point the GLM-SSD engine binds in crates/cuda/src/lib.rs (the `extern "C"` block at
 * lib.rs:24-124); each declaration cites it. Return value: 0 on success, else a HIP error code
 * (hipErrorInvalidValue == 1 for bad arguments, as cudaErrorInvalidValue is in the reference;
 * crates/cuda/kernels/common.cuh:6-14). Pointers are device pointers unless noted; `stream` is a
 * hipStream_t (NULL = default stream). Calls are asynchronous on `stream`.
 *
 * Activations entering a quantized matmul are quantized to q8_1 inside the kernels (blocks of
 * 32: f16 scale d = amax/127, int8 q = round(x/d)); the f32 activation ABI is unchanged.
 * Constraints beyond the reference's: weight rows 2-byte aligned (every ggml tensor is). Row
 * lengths are the reference's (K % 8 == 0 and a whole number of blocks; gs_gemm K % 32 == 0).
 */
#ifndef GLMSSD_H
#define GLMSSD_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (crates/gguf/src/types.rs:74-82) */
enum {
    GS_TYPE_F32 = 0, GS_TYPE_F16 = 1, GS_TYPE_Q8_0 = 8, GS_TYPE_Q2_K = 10, GS_TYPE_Q3_K = 11, GS_TYPE_Q4_K = 12,
    GS_TYPE_Q5_K = 13, GS_TYPE_Q6_K = 14, GS_TYPE_IQ2_XXS = 16, GS_TYPE_IQ3_XXS = 18, GS_TYPE_IQ2_S = 22,
    GS_TYPE_IQ4_XS = 23, GS_TYPE_BF16 = 30,
};

#define GS_MOE_MAX 16 /* experts per fused batch  (crates/cuda/src/lib.rs:411) */
#define GS_MOE_NT 2   /* tokens per fused batch   (crates/cuda/src/lib.rs:413) */

/* Fused-MoE batch, passed by pointer and copied by value into the kernel arguments
 * (crates/cuda/src/lib.rs:417-429 == crates/cuda/kernels/quants.cu:265-273). w[t][e] == 0 marks
 * token t as not routed to expert e. 516 bytes. */
typedef struct GsMoeBatch {
    const uint8_t *gate[GS_MOE_MAX];
    const uint8_t *up[GS_MOE_MAX];
    const uint8_t *down[GS_MOE_MAX];
    float w[GS_MOE_NT][GS_MOE_MAX];
    int n;
} GsMoeBatch;

/* crates/cuda/src/lib.rs:11-22 (runtime.cu:6-14) */
typedef struct GsDeviceInfo {
    char name[256];
    int cc_major, cc_minor;
    int sm_count; /* compute units */
    uint64_t total_mem, free_mem;
    int pci_bus, pci_device;
    int async_engines;
    int can_map_host;
} GsDeviceInfo;

/* ---- runtime (crates/cuda/src/lib.rs:25-51; crates/cuda/kernels/runtime.cu:16-91) ---------- */
int gs_device_info(int dev, GsDeviceInfo *out);              /* lib.rs:25 */
const char *gs_error_string(int e);                          /* lib.rs:26 */
int gs_malloc(void **p, size_t n);                           /* lib.rs:27 */
int gs_free(void *p);                                        /* lib.rs:28 */
int gs_host_alloc(void **p, size_t n);                       /* lib.rs:29 */
int gs_host_free(void *p);                                   /* lib.rs:30 */
int gs_host_register(void *p, size_t n);                     /* lib.rs:31 */
int gs_host_unregister(void *p);                             /* lib.rs:32 */
int gs_stream_create(void **s);                              /* lib.rs:33 */
int gs_stream_destroy(void *s);                              /* lib.rs:34 */
int gs_stream_sync(void *s);                                 /* lib.rs:35 */
int gs_device_sync(void);                                    /* lib.rs:36 */
int gs_device_reset(void);                                   /* lib.rs:37 */
int gs_memcpy_h2d(void *dst, const void *src, size_t n, void *s); /* lib.rs:38 */
int gs_memcpy_d2h(void *dst, const void *src, size_t n, void *s); /* lib.rs:39 */
int gs_memcpy_d2d(void *dst, const void *src, size_t n, void *s); /* lib.rs:40 */
int gs_event_create(void **e);                               /* lib.rs:41 */
int gs_event_create_timed(void **e);                         /* lib.rs:42 */
int gs_event_destroy(void *e);                               /* lib.rs:43 */
int gs_event_record(void *e, void *s);                       /* lib.rs:44 */
int gs_event_sync(void *e);                                  /* lib.rs:45 */
int gs_event_query(void *e);                                 /* lib.rs:46 */
int gs_stream_wait_event(void *s, void *e);                  /* lib.rs:47 */
int gs_event_elapsed_ms(float *ms, void *a, void *b);        /* lib.rs:48 */
int gs_memset(void *p, int v, size_t n, void *s);            /* lib.rs:49 */
int gs_saxpy(int n, float a, const float *x, float *y, void *s); /* lib.rs:50 */

/* ---- quantized ops (crates/cuda/src/lib.rs:52-69; kernels/quants.cu) ---------------------- */
/* dequantize n elements (a whole number of blocks) to f32 / f16, bit-exact with crates/quants
 * (lib.rs:52; quants.cu:21-47) */
int gs_dequant_f32(int ty, const void *src, int64_t n, float *dst, void *s);
int gs_dequant_f16(int ty, const void *src, int64_t n, void *dst, void *s); /* lib.rs:53 */

/* y[b*y_stride + r] (+)= W[r] . x[b*x_stride + :], b < B (1..8); W: rows rows of K elements,
 * row_stride bytes apart (lib.rs:54-57; quants.cu:223-243). Quantized formats take q8_1
 * activations, as in every matrix-vector path here. Several vectors of Q8_0 (from 3), Q4_K, Q5_K
 * and Q6_K (from 5, from 3 when K > 4096) contract in one int8-MFMA pass when rows are whole 4096-element
 * chunks (or one shorter chunk) of whole 16-byte pieces and rows and x are 16-byte aligned: the
 * same int8 operands and per-unit scales, only the f32 summation order differs. */
int gs_gemv(int ty, const void *W, int64_t row_stride, int K, int rows, const float *x, int64_t x_stride, float *y,
            int64_t y_stride, int B, int accumulate, void *s);

/* n_batch independent GEMVs: matrix b at W + b*w_bs bytes, x + b*x_bs, y + b*y_bs floats
 * (lib.rs:58-61; quants.cu:246-256) */
int gs_gemv_batched(int ty, const void *W, int64_t row_stride, int K, int rows, const float *x, float *y, int n_batch,
                    int64_t w_bs, int64_t x_bs, int64_t y_bs, void *s);

/* fused routed-expert gate/up + SwiGLU: h[e][t][r] = swiglu(gate_e[r].x[t], up_e[r].x[t]);
 * x [nt][K], h [b->n][nt][rows] (lib.rs:62-65; quants.cu:378-393). Any K the reference takes;
 * rows longer than the fast kernels' per-lane register plan (K > 8192 for one token, K > 4096
 * for two) run on a slower one-wave-per-row kernel with the same q8_1 arithmetic. */
int gs_moe_gateup(int ty, const GsMoeBatch *b, int nt, int64_t row_stride, int K, int rows, const float *x, float *h,
                  float lim, void *s);

/* fused routed-expert down + weighted combine: y[t][r] += sum_e w[t][e] * down_e[r].h[e][t]
 * (always accumulates; lib.rs:66-69; quants.cu:394-409) */
int gs_moe_down(int ty, const GsMoeBatch *b, int nt, int64_t row_stride, int K, int rows, const float *h, float *y,
                void *s);

/* Additive (no counterpart in the reference): the whole routed-expert FFN of one layer, exactly
 * gs_moe_gateup(ty_gu, b, nt, rs_gu, n_embd, n_ff, x, h, lim) followed by
 * gs_moe_down(ty_dn, b, nt, rs_dn, n_ff, n_embd, h, y) (two launches on s); replaces the pair the
 * decode path calls per expert batch (crates/engine/src/forward.rs:1067-1107). */
int gs_moe_ffn(int ty_gu, int ty_dn, const GsMoeBatch *b, int nt, int64_t rs_gu, int n_embd, int n_ff, int64_t rs_dn,
               const float *x, float *h, float *y, float lim, void *s);

/* Additive (no counterpart in the reference): the routed-expert FFN of n_tok tokens, token t over
 * its own one-token batch b[t] (every b[t].n equal, n_tok * n <= 32): exactly
 * gs_moe_ffn(ty_gu, ty_dn, &b[t], 1, ..., x + t*n_embd, h + t*n*n_ff, y + t*n_embd, lim) for each
 * t, as one gate/up and one down launch; replaces the per-token loop of the engine's MTP verify
 * step through the MoE layer (crates/engine/src/forward.rs:1067-1107). */
int gs_moe_ffn_tokens(int ty_gu, int ty_dn, const GsMoeBatch *b, int n_tok, int64_t rs_gu, int n_embd, int n_ff,
                      int64_t rs_dn, const float *x, float *h, float *y, float lim, void *s);

/* ---- GEMM and MoE glue (crates/cuda/src/lib.rs:71-74,115-122; kernels/gemm.cu, ops.cu) ---- */
/* SwiGLU with clamp: y = silu(min(g,L)) * clamp(u,-L,L); L <= 0: no clamp (lib.rs:76; ops.cu:101-115) */
int gs_swiglu(const float *g, const float *u, float *y, int64_t n, float lim, void *s);
/* y += a*x (lib.rs:77; ops.cu:117-125) */
int gs_axpy(float *y, const float *x, float a, int64_t n, void *s);
/* Y[n*y_stride + m] (+)= W[m] . X[n*x_stride + :], n < N tokens; z-batched (lib.rs:115-118; gemm.cu:107-123).
 * Like the reference, allocates nothing and never synchronizes. */
int gs_gemm(int ty, const void *W, int64_t row_stride, int K, int rows, const float *X, int64_t x_stride, float *Y,
            int64_t y_stride, int N, int accumulate, int n_batch, int64_t w_bs, int64_t x_bs, int64_t y_bs, void *s);
/* Additive (no counterpart in the reference): gs_gemm with a caller-owned workspace, used two ways.
 * (1) Problems with few 128-row x 64-token tiles (small N, few rows) split K across workgroups:
 * each slice writes its f32 partial tile into `work` and the slices are added in a fixed order.
 * (2) From N = 256 tokens (N > 128 for matrices of rows*K >= 2^25 weights), for every weight
 * type but F32 and BF16 and rows stored back to back (row_stride = bytes of a row), the weights are dequantized into `work` as f16 (F16 weights
 * are used in place), X is converted to f16 there too, and the product runs as an f16 x f16 -> f32
 * GEMM in hipBLASLt (the heuristic's first algorithm for the shape, so a shape always takes the
 * same one). Both round the operands to f16 exactly as gs_gemm does and accumulate in f32; results
 * repeat call to call and differ from gs_gemm only in f32 summation order. gs_gemm_workspace gives
 * the bytes a problem needs on the current device (0: `work` unused; for (2) rows*K*2 + N*K*2
 * rounded up to 256 each, plus 32 MiB of library workspace).
 * work: 16-byte aligned, >= that many bytes, not used by another call in flight; work == NULL
 * (or a smaller workspace) runs as gs_gemm. Never synchronizes; allocates nothing itself (the first
 * call of kind (2) on a device creates that device's hipBLASLt handle, kept until the process
 * ends). */
int gs_gemm_workspace(int K, int rows, int N, int n_batch, size_t *bytes);
/* Additive (no counterpart in the reference): the path gs_gemm_ex takes for a problem (one batch)
 * on the current device with a workspace of work_bytes: 0 the f16 MFMA tiles, 1 the tiles with the
 * K split, 2 the f16 dequant + hipBLASLt path (the library opens and has an algorithm for the
 * shape); a negative HIP error code if the device cannot run the library at all. */
int gs_gemm_path(int ty, int K, int rows, int N, int64_t row_stride, int64_t y_stride, size_t work_bytes);
int gs_gemm_ex(int ty, const void *W, int64_t row_stride, int K, int rows, const float *X, int64_t x_stride, float *Y,
               int64_t y_stride, int N, int accumulate, int n_batch, int64_t w_bs, int64_t x_bs, int64_t y_bs,
               void *work, size_t work_bytes, void *s);
/* y[i][:] = x[idx[i]][:] (lib.rs:119; gemm.cu:125-138) */
int gs_gather_rows(const float *x, const int *idx, float *y, int rows, int n, void *s);
/* acc[idx[i]][:] += w[i] * y[i][:], idx unique within a call (lib.rs:120-122; gemm.cu:139-152) */
int gs_scatter_add_rows(float *acc, const int *idx, const float *w, const float *y, int rows, int n, void *s);
/* f32 -> f16 (lib.rs:123; gemm.cu:155-163) */
int gs_f32_to_f16(const float *x, void *y, int64_t n, void *s);

/* ---- additive entry points (no counterpart in the reference) ------------------------------ */
/* q8_1 quantization of n f32 values (n % 32 == 0) to ggml block_q8_1 {f16 d; f16 s; int8 qs[32]}
 * (36 bytes per 32). The same quantizer the matmul kernels apply to their activations; exposed
 * for bit-exact testing. */
int gs_quant_q8_1(const float *x, void *q, int64_t n, void *s);

/* Grouped routed-expert FFN over every expert of one MoE layer in one call (prefill, MTP verify;
 * the multi-token path crates/engine/src/forward.rs:1335-1368 + run_expert_rows :1399-1413 runs
 * as gs_gather_rows, gs_gemm x3, gs_swiglu, gs_scatter_add_rows per expert). The pairs are the
 * engine's grouping (forward.rs:1017-1036): pair p = (token idx[p], weight w[p]), sorted by
 * expert, expert e owning pairs offs[e] .. offs[e+1]-1 (offs has n_exp+1 entries; empty experts
 * allowed). experts[e] holds the device pointers of expert e's gate/up ([K] x n_ff rows,
 * gu_row_stride bytes apart) and down ([n_ff] x K rows, down_row_stride apart).
 *   y[idx[p]][:] += w[p] * down_e . swiglu(gate_e . x[idx[p]], up_e . x[idx[p]])   (always adds)
 * x [n_tok][K], y [n_tok][K] f32. Numerics are the reference's multi-token GEMM's (gemm.cu:57-78):
 * x and h enter the contractions as f16 (after a power-of-two row scale that keeps each row in
 * the f16 normal range), accumulation is f32; the weights are exact (the reference rounds the
 * dequantized weights to f16). The experts' outputs are combined into y with f32 atomics, so the
 * summation order (and the last bits of y) can differ between runs (gs_moe_grouped_scatter below
 * gives the reference's bit-reproducible mode).
 * Supported: ty_gu, ty_down each IQ2_XXS or IQ3_XXS, K and n_ff multiples of 256 and >= 512,
 * n_exp <= 1024, x 16-byte aligned. `work` (256-byte aligned, >= gs_moe_grouped_workspace bytes) is caller-owned scratch.
 * All of offs/idx/w/experts are device arrays; the call launches without a host sync. */
typedef struct GsExpertPtrs {
    const uint8_t *gate;
    const uint8_t *up;
    const uint8_t *down;
} GsExpertPtrs;
int gs_moe_grouped_workspace(int n_tok, int n_pairs, int K, int n_ff, size_t *bytes);
int gs_moe_grouped(int ty_gu, int ty_down, const GsExpertPtrs *experts, int n_exp, const int *offs, const int *idx,
                   const float *w, int n_pairs, int n_tok, int64_t gu_row_stride, int K, int n_ff,
                   int64_t down_row_stride, const float *x, float *y, float lim, void *work, size_t work_bytes, void *s);

/* gs_moe_grouped with the output row of each pair given separately: pair p reads x[idx[p]] and
 * adds w[p] * FFN_e(x[idx[p]]) into y[out_idx[p]][:]. The reference's deterministic combine
 * (GLMSSD_DETERMINISTIC, crates/engine/src/forward.rs:276-278, :1039-1048, :1119-1127) scatters
 * every (route rank r, token t) pair into its own slot r * n_tok + t and sums the slots in rank
 * order with gs_axpy; with distinct out_idx into a zeroed y each element receives exactly one
 * addition, so the result is bit-reproducible. Arguments and limits otherwise as gs_moe_grouped
 * (out_idx a device array of n_pairs entries; y holds as many rows as out_idx addresses). */
int gs_moe_grouped_scatter(int ty_gu, int ty_down, const GsExpertPtrs *experts, int n_exp, const int *offs,
                           const int *idx, const int *out_idx, const float *w, int n_pairs, int n_tok,
                           int64_t gu_row_stride, int K, int n_ff, int64_t down_row_stride, const float *x, float *y,
                           float lim, void *work, size_t work_bytes, void *s);

/* No counterpart in the reference; for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): gs_moe_grouped with
 * its workspace in a device array of the library (GS_MOE_GROUPED_SCRATCH_MAX bytes, one per GPU,
 * held until the process ends) instead of a caller buffer. Allocates nothing: the first call on
 * a device looks up that device's array (and, like any first gs_* call, loads the library's
 * code objects), later calls only launch. Returns hipErrorInvalidValue when
 * gs_moe_grouped_workspace(n_tok, n_pairs, K, n_ff) exceeds GS_MOE_GROUPED_SCRATCH_MAX (e.g.
 * 512 tokens x top-8 at 4096 / 1536 needs about 42 MB). Every call on one GPU shares its array:
 * calls that overlap in time on one GPU (other streams, other threads) race and must not be
 * issued. */
#define GS_MOE_GROUPED_SCRATCH_MAX (48u << 20)
/* (The array is reserved on every GPU on which the library is used, whether or not this entry
 * point is called.) */
int gs_moe_grouped_noalloc(int ty_gu, int ty_down, const GsExpertPtrs *experts, int n_exp, const int *offs,
                           const int *idx, const float *w, int n_pairs, int n_tok, int64_t gu_row_stride, int K,
                           int n_ff, int64_t down_row_stride, const float *x, float *y, float lim, void *s);

/* No counterpart in the reference. The MFMA kernels of gs_gemm(_ex) and gs_moe_grouped* pass work
 * between the waves of a workgroup through LDS fill counters (release / acquire at workgroup
 * scope). Each wait for a count is bounded (2^16 polls, far beyond any legitimate wait) so that a
 * lost fill can never hang the GPU; a wait that runs out sets a sticky per-device flag, and the
 * output of that launch is then unreliable. gs_wait_status synchronizes `stream`, returns
 * hipErrorLaunchFailure if any wait has expired on the current device since the last query (and
 * clears the flag), else 0. */
int gs_wait_status(void *stream);
/* Test hook (no counterpart in the reference): sets the poll bound of those waits for later
 * launches (default 2^16); force != 0 makes every wait run to the bound and expire, so the
 * expiry path can be exercised without a fault. Outputs of such launches are meaningless. */
int gs_debug_wait_limit(uint32_t polls, int force);

#ifdef __cplusplus
}
#endif
#endif
