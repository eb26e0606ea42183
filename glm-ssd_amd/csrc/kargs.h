// Kernel argument blocks shared by the host launcher (host.cpp) and the gfx950 kernels
// (kernels.hip). Plain C layout: each kernel takes exactly one of these by value, so the
// host packs it once and hands its address to hipModuleLaunchKernel.
#pragma once
#include <stdint.h>

// ggml type ids (crates/gguf/src/types.rs:74-82)
enum GsType {
    GS_F32 = 0, GS_F16 = 1, GS_Q8_0 = 8, GS_Q2_K = 10, GS_Q3_K = 11, GS_Q4_K = 12, GS_Q5_K = 13,
    GS_Q6_K = 14, GS_IQ2_XXS = 16, GS_IQ3_XXS = 18, GS_IQ2_S = 22, GS_IQ4_XS = 23, GS_BF16 = 30,
};

#ifndef GS_WG
#define GS_WG 512          // threads per workgroup of the streaming kernels (8 wave64)
#endif
#define GS_SEG_MAX 32      // weight matrices (experts) per fused-MoE launch
#define GS_NT_MAX 8        // activation vectors (tokens) per launch

// Matrix-vector work description ("stream" kernels). One launch streams the rows of one or
// more quantized matrices ("segments") from HBM.
//   kind 0 (GEMV):   y[b][r] (+)= W[r] . xq[b]                      seg = 1 (blockIdx.y batches)
//   kind 1 (GATEUP): h[e][t][r] = swiglu(gate_e[r] . xq[t], up_e[r] . xq[t])
//   kind 2 (DOWN):   y[t][r] += sum_e w[t][e] * (down_e[r] . hq[e][t])
struct StreamArgs {
    const uint8_t *w0[GS_SEG_MAX];   // GEMV: w0[0]; GATEUP: gate; DOWN: down
    const uint8_t *w1[GS_SEG_MAX];   // GATEUP: up
    float wt[GS_NT_MAX][GS_SEG_MAX]; // DOWN: combine weights (0 = token not routed)
    const float *x;                  // activations (f32; quantized to q8_1 in the prologue)
    float *y;                        // output
    int64_t row_stride;              // bytes between rows
    int64_t x_stride;                // floats between activation vectors
    int64_t y_stride;                // floats between output vectors
    int64_t w_bs, x_bs, y_bs;        // per blockIdx.y slice: GEMV batch (bytes / floats / floats); MoE token (x, y)
    int K;                           // row length (elements)
    int rows;                        // rows per matrix
    int nvec;                        // activation vectors (B or tokens)
    int nv_tail;                     // GEMV: vectors of the last blockIdx.y slice (0: nvec)
    int nseg;                        // segments (experts) in this launch
    int accumulate;                  // GEMV only: y += result
    float lim;                       // SwiGLU clamp (<= 0: none)
    int row_bytes;                   // bytes of one row's data
    int nu;                          // q8_1 units (32 elements) per row = K/32
    int lpr;                         // lanes per row group (16, 32 or 64)
    int upl;                         // units per lane = ceil(segments*nu/lpr)
    int x_aligned;                   // x and x_stride allow 16-byte loads
    const uint8_t *wlo;              // DOWN, 64-lane kernels: lowest expert pointer; every expert's
                                     // rows lie within 4 GiB above it (32-bit offsets)
};

// Whole-tensor dequantization
struct CvtArgs;
struct DequantArgs {
    const uint8_t *src;
    void *dst;
    int64_t n;          // elements
    int64_t n_units;    // 32-element units (the last one may be partial for plain types)
    int aligned;        // dst is 16-byte aligned (vector stores)
    // f16 only: blocks from w_blocks on convert f32 rows to f16 instead (the GEMM library path's
    // activations, cvt_*: as CvtArgs); cvt_n == 0: none
    int w_blocks;
    const float *cvt_x;
    uint16_t *cvt_y;
    int64_t cvt_x_stride;
    int cvt_K, cvt_n;
};

// q8_1 quantization of f32 rows: out = n/32 blocks of {f16 d; f16 s; int8 qs[32]}
struct QuantArgs {
    const float *x;
    uint8_t *out;
    int64_t n_blocks;
};

// multi-vector Q8_0 GEMV on int8 MFMA (gs_gemv with 2..8 vectors): y[t][r] (+)= W[r] . q8_1(x[t])
struct MvArgs {
    const uint8_t *w;
    int64_t row_stride;   // bytes
    const float *x;
    int64_t x_stride;     // floats
    float *y;
    int64_t y_stride;     // floats
    int K, rows, nv, accumulate;
};

// f32 rows -> compact f16 rows (round to nearest even): N rows of K values, source row stride
// x_stride (elements), destination rows K apart (the GEMM library path's activations)
struct CvtArgs {
    const float *x;
    uint16_t *y;
    int64_t x_stride;
    int K;    // a multiple of 4
    int N;
};

struct EltArgs {
    const float *a;
    const float *b;
    float *y;
    int64_t n;
    float s;       // lim (swiglu) or alpha (axpy)
};

struct RowsArgs {
    const float *x;
    const int *idx;
    const float *w;
    float *y;
    int rows;
    int n;
};

// Grouped MoE GEMM (grouped.hip): pairs sorted by expert, offs = CSR offsets per expert.
#define GS_GRP_EXP_MAX 1024   // experts per layer the device-side tile list holds
#define GS_GRP_META_BYTES 6144   // grouped kernels' per-workgroup bookkeeping in LDS (tile prefix, epilogue operands, fill counters)
struct GroupedArgs {
    const uint8_t *const *experts;   // [n_exp][3] device pointers: gate, up, down
    const int *offs;                 // [n_exp + 1] pair offsets
    const int *idx;                  // [n_pairs] token of each pair
    const float *w;                  // [n_pairs] combine weights (kind 2)
    const uint16_t *act;             // f16 activation rows (x16 [n_tok][K] or h16 [n_pairs][K])
    const float *ascale;             // per activation row: power-of-two scale of act
    float *out;                      // kind 1: h [n_pairs][rows]; kind 2: y [n_tok][rows] (+=)
    int64_t row_stride;              // bytes between weight rows
    int K;                           // row length (multiple of 256)
    int rows;                        // rows per expert matrix
    int n_exp;
    float lim;                       // SwiGLU clamp (<= 0: none)
    uint32_t wait_limit;             // polls before an LDS fill wait gives up (and flags it)
    uint32_t wait_force;             // test hook: nonzero makes every such wait run to its limit
};

// f32 rows -> f16 with a power-of-two row scale (grouped GEMM operands)
struct RowsQArgs {
    const float *x;
    int64_t x_stride;   // floats between rows
    uint16_t *out;      // [nrows][K]
    float *scale;       // [nrows]
    int K;
    int nrows;
};

// Quantized GEMM (gemm.hip): Y[z][n][r] (+)= sum_k f16(deq(W[z][r][k])) * f16(X[z][n][k])
// threads per gs_k_gemm_* workgroup (gemm.hip: 8 waves, 16 weight rows each)
#define GS_GEMM_THREADS 512
// LDS buffers per gs_k_gemm_* workgroup: 2 = the next super-block prefetched through registers
// (one workgroup per CU); 1 = single-buffered steps, two workgroups per CU taking turns (Q4_K
// 12288 x 4096 x 512 measured 173 against 212 us that way until the contraction lost its
// per-MFMA branches; since then both take about 165 us and every format is double-buffered)
static inline constexpr int gs_gemm_nbuf(int) { return 2; }
struct GemmArgs {
    const uint8_t *W;
    const float *X;
    float *Y;
    int64_t row_stride;   // bytes between weight rows
    int64_t x_stride;     // floats between X rows
    int64_t y_stride;     // floats between Y rows
    int64_t w_bs, x_bs, y_bs;   // per blockIdx.y (z) batch strides: bytes / floats / floats
    int K, rows, N, accumulate;
    int n_rb, n_tb;       // row blocks and token blocks of one problem
    int ksb;              // super-blocks per K slice (blockIdx.z); every super-block when not split
    float *part;          // K split: slice partials [slice][batch][N][rows] (null: write Y)
    uint32_t wait_limit;  // polls before an LDS fill wait gives up (and flags it)
    uint32_t wait_force;  // test hook: nonzero makes every such wait run to its limit
};
#define GS_GEMM_KS_MAX 16   // K slices of one gs_gemm call at most
// sum of the K slices' partials in slice order into Y (+= when accumulate)
struct GemmReduceArgs {
    const float *part;
    float *Y;
    int64_t y_stride, y_bs;
    int rows, N, n_batch, nks, accumulate;
};
