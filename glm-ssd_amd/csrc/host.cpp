// Host side of libglmssd_hip.so: the gs_* C ABI (include/glmssd.h) over the HIP module API.
//
// The gfx950 code objects are embedded in the library (blobs.S) and loaded per device with
// hipModuleLoadData on first use; kernels are looked up by name and launched with
// hipModuleLaunchKernel, each with a single by-value argument block (kargs.h). Argument
// validation mirrors the reference's (crates/cuda/kernels/quants.cu:223-256,378-409,
// gemm.cu:107-152) and returns hipErrorInvalidValue without launching on bad input.
#include <dlfcn.h>
#include <hip/hip_runtime_api.h>
#include <hipblaslt/hipblaslt.h>   // types only: the library is opened at run time (gemm_lib)

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/glmssd.h"
#include "kargs.h"


#define GS_EXPORT extern "C" __attribute__((visibility("default")))

// ---- embedded code objects --------------------------------------------------------------------
#define GS_BLOB(NAME)                                 \
    extern "C" const unsigned char gs_blob_##NAME##_start[]; \
    extern "C" const unsigned char gs_blob_##NAME##_end[];
#define GS_BLOB_LIST(X) X(common) X(grouped) X(gemm) X(t0) X(t1) X(t8) X(t10) X(t11) X(t12) X(t13) X(t14) X(t16) X(t18) X(t22) X(t23) X(t30)
GS_BLOB_LIST(GS_BLOB)

namespace {

struct Blob {
    const unsigned char *p;
    size_t n;
};
std::vector<Blob> blobs() {
    std::vector<Blob> v;
#define GS_BLOB_ITEM(NAME) v.push_back({gs_blob_##NAME##_start, (size_t)(gs_blob_##NAME##_end - gs_blob_##NAME##_start)});
    GS_BLOB_LIST(GS_BLOB_ITEM)
#undef GS_BLOB_ITEM
    return v;
}

struct DeviceCtx {
    std::vector<hipModule_t> mods;
    std::map<std::string, hipFunction_t> fns;
    int cu_count = 0;
    size_t max_lds = 0;
    hipError_t init_err = hipSuccess;
    std::map<std::pair<std::string, int>, int> occ;  // (kernel, lds) -> blocks per CU
    std::vector<void *> wait_flags;   // gs_wait_expired of each code object that has one
    // GEMM library path (gs_gemm_ex with many tokens): the device's hipBLASLt handle,
    // created on first use, and one plan per problem shape
    std::mutex lt_mu;
    hipblasLtHandle_t lt = nullptr;
    bool lt_failed = false;
    struct LtPlan {
        hipblasLtMatmulDesc_t desc;
        hipblasLtMatrixLayout_t la, lb, lc;
        hipblasLtMatmulAlgo_t algo;
    };
    std::map<std::vector<int64_t>, LtPlan> lt_plans;
};

std::mutex g_mu;
std::map<int, DeviceCtx *> g_ctx;
// poll bound of the MFMA kernels' LDS fill waits, and the test hook that makes them expire
std::atomic<uint32_t> g_wait_limit{1u << 16};
std::atomic<uint32_t> g_wait_force{0};

DeviceCtx *ctx(hipError_t *err) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        *err = e;
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_ctx.find(dev);
    if (it != g_ctx.end()) {
        *err = it->second->init_err;
        return it->second->init_err == hipSuccess ? it->second : nullptr;
    }
    DeviceCtx *c = new DeviceCtx();
    g_ctx[dev] = c;
    hipDeviceProp_t p;
    e = hipGetDeviceProperties(&p, dev);
    if (e == hipSuccess) {
        c->cu_count = p.multiProcessorCount;
        c->max_lds = p.sharedMemPerBlock;
        if (!strstr(p.gcnArchName, "gfx950")) {
            fprintf(stderr, "glmssd: device %d is %s; this library carries gfx950 code only\n", dev, p.gcnArchName);
            e = hipErrorNoBinaryForGpu;
        }
    }
    if (e == hipSuccess) {
        for (const Blob &b : blobs()) {
            hipModule_t m;
            e = hipModuleLoadData(&m, (const void *)b.p);
            if (e != hipSuccess) break;
            c->mods.push_back(m);
            hipDeviceptr_t fp = nullptr;
            size_t fsz = 0;
            if (hipModuleGetGlobal(&fp, &fsz, m, "gs_wait_expired") == hipSuccess && fsz == 4)
                c->wait_flags.push_back((void *)fp);
            else
                (void)hipGetLastError();   // code objects without bounded waits
        }
    }
    c->init_err = e;
    *err = e;
    return e == hipSuccess ? c : nullptr;
}

hipError_t get_fn(DeviceCtx *c, const std::string &name, hipFunction_t *f) {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = c->fns.find(name);
    if (it != c->fns.end()) {
        *f = it->second;
        return hipSuccess;
    }
    for (hipModule_t m : c->mods) {
        if (hipModuleGetFunction(f, m, name.c_str()) == hipSuccess) {
            c->fns[name] = *f;
            return hipSuccess;
        }
    }
    (void)hipGetLastError();  // clear the lookup misses
    fprintf(stderr, "glmssd: kernel %s not found in the embedded code objects\n", name.c_str());
    return hipErrorNotFound;
}

template <class A>
hipError_t launch(const std::string &name, dim3 grid, dim3 block, size_t lds, hipStream_t s, const A &args) {
    hipError_t e;
    DeviceCtx *c = ctx(&e);
    if (!c) return e;
    hipFunction_t f;
    if ((e = get_fn(c, name, &f)) != hipSuccess) return e;
    if (lds > c->max_lds) return hipErrorInvalidValue;
    size_t sz = sizeof(A);
    void *cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, (void *)&args, HIP_LAUNCH_PARAM_BUFFER_SIZE, &sz,
                   HIP_LAUNCH_PARAM_END};
    return hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, (unsigned)lds, s, nullptr, cfg);
}

// ---- ggml geometry (crates/gguf/src/types.rs:85-113); plain types use 8-element "blocks" ------
bool geometry(int ty, int &qk, int &bb) {
    switch (ty) {
        case GS_F32: qk = 8; bb = 32; return true;
        case GS_F16: case GS_BF16: qk = 8; bb = 16; return true;
        case GS_Q8_0: qk = 32; bb = 34; return true;
        case GS_Q2_K: qk = 256; bb = 84; return true;
        case GS_Q3_K: qk = 256; bb = 110; return true;
        case GS_Q4_K: qk = 256; bb = 144; return true;
        case GS_Q5_K: qk = 256; bb = 176; return true;
        case GS_Q6_K: qk = 256; bb = 210; return true;
        case GS_IQ2_XXS: qk = 256; bb = 66; return true;
        case GS_IQ2_S: qk = 256; bb = 82; return true;
        case GS_IQ3_XXS: qk = 256; bb = 98; return true;
        case GS_IQ4_XS: qk = 256; bb = 136; return true;
        default: return false;
    }
}
int ggml_block_elems(int ty) {  // elements per ggml block (1 for plain types)
    return ty == GS_F32 || ty == GS_F16 || ty == GS_BF16 ? 1 : (ty == GS_Q8_0 ? 32 : 256);
}
int table_bytes(int) { return 0; }  // lookup tables are static LDS arrays of their kernels

// Plan of one streaming pass: lanes per row group and unit budget (into `a`), the kernel's
// weight-unit budget and its dynamic LDS bytes.
struct StreamPlan {
    int um = 0;
    size_t lds = 0;
};
hipError_t plan_stream(DeviceCtx *c, int kind, int ty, StreamArgs &a, StreamPlan &P) {
    int qk, bb;
    if (!geometry(ty, qk, bb)) return hipErrorInvalidValue;
    const int NVt = a.nvec <= 1 ? 1 : a.nvec <= 2 ? 2 : a.nvec <= 4 ? 4 : 8;
    a.row_bytes = (int)((int64_t)a.K / qk * bb);
    a.nu = a.K / 32;
    // units one lane must cover per row: GEMV one row, GATEUP the same units of gate and up
    // (two per activation unit), DOWN the concatenated rows of every expert in the batch
    const int tot = kind == 2 ? a.nseg * a.nu : a.nu;
    const int mult = kind == 1 ? 2 : 1;
    // instantiated weight-unit budgets per lane (kernels.hip GS_STREAM_MV / GS_STREAM_GU)
    std::vector<int> umaxes;
    if (kind == 1) umaxes = NVt == 1 ? std::vector<int>{2, 4, 8} : NVt == 2 ? std::vector<int>{2, 4}
                          : NVt == 4 ? std::vector<int>{2, 4} : std::vector<int>{2};
    else umaxes = NVt == 1 ? std::vector<int>{2, 4, 6, 8} : NVt == 2 ? std::vector<int>{2, 4}
                : NVt == 4 ? std::vector<int>{1, 2} : std::vector<int>{1};
    int best_lpr = -1, best_um = 0;
    double best_eff = -1.0;
    for (int lpr : {64, 32, 16}) {
        const int upl = (tot + lpr - 1) / lpr;
        int um = 0;
        for (int u : umaxes)
            if (u >= upl * mult) { um = u; break; }
        if (!um) continue;
        const double eff = (double)tot * mult / ((double)lpr * um);
        if (eff > best_eff + 1e-9) {
            best_eff = eff;
            best_lpr = lpr;
            best_um = um;
        }
    }
    if (best_lpr < 0) return hipErrorInvalidValue;
    a.lpr = best_lpr;
    a.upl = (tot + best_lpr - 1) / best_lpr;
    const int tab = (table_bytes(ty) + 15) & ~15;
    // staged activations per vector: q8_1 bytes + scale/sum words, or the f32 values themselves
    // for the float formats (F32, F16, BF16 take f32 activations, like the reference)
    const bool f32x = ty == GS_F32 || ty == GS_F16 || ty == GS_BF16;
    P.lds = (size_t)tab + (size_t)(kind == 2 ? a.nseg * a.nvec : a.nvec) * (f32x ? (size_t)a.K * 4 : a.K + a.nu * 8);
    if (P.lds > std::min<size_t>(c->max_lds, 160 * 1024)) return hipErrorInvalidValue;
    P.um = best_um;
    return hipSuccess;
}

// Plan and launch one streaming kernel (kind 0 GEMV, 1 MoE gate/up, 2 MoE down).
hipError_t stream(int kind, int ty, StreamArgs &a, hipStream_t s, int n_batch = 1) {
    hipError_t e;
    DeviceCtx *c = ctx(&e);
    if (!c) return e;
    StreamPlan P;
    if ((e = plan_stream(c, kind, ty, a, P)) != hipSuccess) return e;
    const int NVt = a.nvec <= 1 ? 1 : a.nvec <= 2 ? 2 : a.nvec <= 4 ? 4 : 8;
    // one token with 64-lane groups: the variant with the group width fixed at compile time
    const bool w64 = a.lpr == 64 && NVt == 1 && (kind != 2 || a.wlo != nullptr);
    // One-vector GEMV variants with aligned loads (formats.h). Q8_0 rows of an even number of
    // blocks up to 8192 elements (a lane's unit pair never crosses the row end): rows that start
    // 4-byte aligned read each pair as 17 aligned dwords (_w4, FQ8_0A4; measured 4096 x 4096
    // 6.2-7.7 -> 6.3-6.6 us across processes, 12288 x 4096 11.6 -> 11.0, 16384 x 8192 31.7 ->
    // 24.4); other rows, from 4 rows per wave, shift each unit's quants out of an aligned window
    // (_wa, FQ8_0A; 262144 x 4096 245 -> 196 us; with fewer rows the plain loads stay faster).
    // Q6_K from 4 rows per wave, rows 4-byte aligned (its windows start 2 bytes before odd
    // blocks), up to 8192 elements (the K = 12288 variant spills): _wa, FQ6_KA (12288 x 4096
    // 11.6 -> 10.7 us, 16384 x 8192 25.9 -> 24.7, 262144 x 4096 186 -> 159).
    const bool one_vec = w64 && kind == 0 && n_batch == 1 && P.um <= 4;
    const bool many_rows = (int64_t)a.rows >= 4 * (int64_t)c->cu_count * (GS_WG / 64);
    const bool rows4 = a.row_stride % 4 == 0 && ((uintptr_t)a.w0[0] & 3) == 0;
    const bool q8_pairs = one_vec && ty == GS_Q8_0 && a.K % 64 == 0;
    const bool w4 = q8_pairs && rows4;
    const bool wa = one_vec && many_rows && ((q8_pairs && !rows4) || (ty == GS_Q6_K && rows4));
    const std::string name = "gs_k_stream_" + std::to_string(ty) + "_" + std::to_string(kind) + "_" +
                             std::to_string(NVt) + "_" + std::to_string(P.um) +
                             (w64 ? (w4 ? "_w4" : wa ? "_wa" : "_w") : "");
    hipFunction_t f;
    if ((e = get_fn(c, name, &f)) != hipSuccess) return e;
    const int G = GS_WG / a.lpr;
    const int nrow = kind == 1 ? a.nseg * a.rows : a.rows;
    // one workgroup per CU by default: each workgroup pays the activation prologue once, and the
    // row pipeline inside it supplies the memory parallelism
    int grid = std::max(1, std::min((nrow + G - 1) / G, c->cu_count));
    // blockIdx.y slices (GEMV batches or vector groups, MoE tokens): the CUs split between the
    // slices, so every slice runs at once and each workgroup pays its prologue once. A full grid
    // per slice runs the slices one after another (one workgroup per CU): 8-vector Q8_0 GEMV
    // 15.5 -> 12.7 us, IQ2_XXS 22.4 -> 13.5 us; MoE tokens measured best against 1/2, 3/4, 3/2
    // and 2x this split.
    if (n_batch > 1) grid = std::max(1, grid / n_batch);
    if (kind == 1) {   // waves are pinned to experts: at least one per expert, a whole number each
        const int wpw = GS_WG / 64;
        const int waves = std::max(grid * wpw, a.nseg) / a.nseg * a.nseg;
        grid = (waves + wpw - 1) / wpw;
    }
    return launch(name, dim3(grid, n_batch, 1), dim3(GS_WG, 1, 1), P.lds, s, a);
}

// Row-length-independent kernels (kernels.hip gs_k_any_<kind>_<type>): one wave per row, for the
// shapes the streaming kernels' register plan does not hold; blockIdx.y = GEMV batch or expert.
hipError_t stream_any(int kind, int ty, const StreamArgs &a, int ny, hipStream_t s) {
    hipError_t e;
    DeviceCtx *c = ctx(&e);
    if (!c) return e;
    const int grid = std::max(1, std::min((a.rows + 3) / 4, 8 * c->cu_count / std::max(1, ny)));
    return launch("gs_k_any_" + std::to_string(kind) + "_" + std::to_string(ty), dim3(grid, ny, 1), dim3(256, 1, 1), 0, s, a);
}

// whether one streaming launch can hold the plan for these arguments (kind 1 or 2)
bool stream_fits(int kind, int ty, StreamArgs a) {
    hipError_t e;
    DeviceCtx *c = ctx(&e);
    if (!c) return true;   // the launch itself reports the error
    StreamPlan P;
    return plan_stream(c, kind, ty, a, P) == hipSuccess;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

int check_w(const void *W, int64_t row_stride) { return ((uintptr_t)W & 1) == 0 && (row_stride & 1) == 0; }

}  // namespace

// =============================================================================================
// runtime (crates/cuda/kernels/runtime.cu:16-91)
// =============================================================================================
GS_EXPORT int gs_device_info(int dev, GsDeviceInfo *out) {
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, dev);
    if (e != hipSuccess) return e;
    if ((e = hipSetDevice(dev)) != hipSuccess) return e;
    size_t fr = 0, tot = 0;
    if ((e = hipMemGetInfo(&fr, &tot)) != hipSuccess) return e;
    memset(out, 0, sizeof(*out));
    {
        const char *nm = p.name[0] ? p.name : p.gcnArchName;
        memcpy(out->name, nm, std::min(strlen(nm), sizeof(out->name) - 1));
    }
    out->cc_major = p.major;
    out->cc_minor = p.minor;
    out->sm_count = p.multiProcessorCount;
    out->total_mem = tot;
    out->free_mem = fr;
    out->pci_bus = p.pciBusID;
    out->pci_device = p.pciDeviceID;
    out->async_engines = p.asyncEngineCount;
    out->can_map_host = p.canMapHostMemory;
    return 0;
}
GS_EXPORT const char *gs_error_string(int e) { return hipGetErrorString((hipError_t)e); }
GS_EXPORT int gs_malloc(void **p, size_t n) { return hipMalloc(p, n); }
GS_EXPORT int gs_free(void *p) { return hipFree(p); }
GS_EXPORT int gs_host_alloc(void **p, size_t n) { return hipHostMalloc(p, n, hipHostMallocDefault); }
GS_EXPORT int gs_host_free(void *p) { return hipHostFree(p); }
GS_EXPORT int gs_host_register(void *p, size_t n) { return hipHostRegister(p, n, hipHostRegisterDefault); }
GS_EXPORT int gs_host_unregister(void *p) { return hipHostUnregister(p); }
GS_EXPORT int gs_stream_create(void **s) { return hipStreamCreateWithFlags((hipStream_t *)s, hipStreamNonBlocking); }
GS_EXPORT int gs_stream_destroy(void *s) { return hipStreamDestroy((hipStream_t)s); }
GS_EXPORT int gs_stream_sync(void *s) { return hipStreamSynchronize((hipStream_t)s); }
GS_EXPORT int gs_device_sync(void) { return hipDeviceSynchronize(); }
GS_EXPORT int gs_device_reset(void) {
    {
        std::lock_guard<std::mutex> lk(g_mu);
        int dev = 0;
        if (hipGetDevice(&dev) == hipSuccess) {
            auto it = g_ctx.find(dev);
            if (it != g_ctx.end()) {   // modules die with the context; forget them
                delete it->second;
                g_ctx.erase(it);
            }
        }
    }
    return hipDeviceReset();
}
GS_EXPORT int gs_memcpy_h2d(void *dst, const void *src, size_t n, void *s) {
    return hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, (hipStream_t)s);
}
GS_EXPORT int gs_memcpy_d2h(void *dst, const void *src, size_t n, void *s) {
    return hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, (hipStream_t)s);
}
GS_EXPORT int gs_memcpy_d2d(void *dst, const void *src, size_t n, void *s) {
    return hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, (hipStream_t)s);
}
GS_EXPORT int gs_event_create(void **e) { return hipEventCreateWithFlags((hipEvent_t *)e, hipEventDisableTiming); }
GS_EXPORT int gs_event_create_timed(void **e) { return hipEventCreate((hipEvent_t *)e); }
GS_EXPORT int gs_event_destroy(void *e) { return hipEventDestroy((hipEvent_t)e); }
GS_EXPORT int gs_event_record(void *e, void *s) { return hipEventRecord((hipEvent_t)e, (hipStream_t)s); }
GS_EXPORT int gs_event_sync(void *e) { return hipEventSynchronize((hipEvent_t)e); }
GS_EXPORT int gs_event_query(void *e) { return hipEventQuery((hipEvent_t)e); }
GS_EXPORT int gs_stream_wait_event(void *s, void *e) { return hipStreamWaitEvent((hipStream_t)s, (hipEvent_t)e, 0); }
GS_EXPORT int gs_event_elapsed_ms(float *ms, void *a, void *b) {
    return hipEventElapsedTime(ms, (hipEvent_t)a, (hipEvent_t)b);
}
GS_EXPORT int gs_memset(void *p, int v, size_t n, void *s) { return hipMemsetAsync(p, v, n, (hipStream_t)s); }
GS_EXPORT int gs_saxpy(int n, float a, const float *x, float *y, void *s) {
    if (n <= 0) return 0;
    EltArgs g{x, nullptr, y, n, a};
    return launch("gs_k_saxpy", dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)s, g);
}

// =============================================================================================
// dequantization (quants.cu:21-47)
// =============================================================================================
static int dequant(int ty, const void *src, int64_t n, void *dst, void *s, const char *suffix) {
    int qk, bb;
    if (n <= 0 || n % 8 != 0 || !geometry(ty, qk, bb) || n % ggml_block_elems(ty) != 0) return hipErrorInvalidValue;
    DequantArgs a{(const uint8_t *)src, dst, n, (n + 31) / 32, aligned16(dst), 0, nullptr, nullptr, 0, 0, 0};
    const std::string name = std::string("gs_k_dequant_") + suffix + "_" + std::to_string(ty);
    return launch(name, dim3((unsigned)((a.n_units + 255) / 256)), dim3(256), 0, (hipStream_t)s, a);
}
GS_EXPORT int gs_dequant_f32(int ty, const void *src, int64_t n, float *dst, void *s) {
    return dequant(ty, src, n, dst, s, "f32");
}
GS_EXPORT int gs_dequant_f16(int ty, const void *src, int64_t n, void *dst, void *s) {
    return dequant(ty, src, n, dst, s, "f16");
}

GS_EXPORT int gs_quant_q8_1(const float *x, void *q, int64_t n, void *s) {
    if (n <= 0 || n % 32 != 0) return hipErrorInvalidValue;
    QuantArgs a{x, (uint8_t *)q, n / 32};
    return launch("gs_k_quant_q8_1", dim3((unsigned)((a.n_blocks + 255) / 256)), dim3(256), 0, (hipStream_t)s, a);
}

// =============================================================================================
// GEMV (quants.cu:223-256)
// =============================================================================================
// nv_tail: vectors of the last blockIdx.y slice when it differs from B (the second group of a
// 5..7-vector call)
static int gemv_impl(int ty, const void *W, int64_t row_stride, int K, int rows, const float *x, int64_t x_stride,
                     float *y, int64_t y_stride, int B, int accumulate, int n_batch, int64_t w_bs, int64_t x_bs,
                     int64_t y_bs, void *s, int nv_tail = 0) {
    int qk, bb;
    if (!geometry(ty, qk, bb)) return hipErrorInvalidValue;
    if (K <= 0 || K % 8 != 0 || K % ggml_block_elems(ty) != 0) return hipErrorInvalidValue;
    if (B < 1 || B > 8 || rows < 0 || n_batch < 1 || n_batch > 65535) return hipErrorInvalidValue;
    if (!check_w(W, row_stride) || (n_batch > 1 && (w_bs & 1))) return hipErrorInvalidValue;
    if (rows == 0) return 0;
    if (K % 32 != 0) {   // plain types only (quantized blocks are multiples of 32): 8-element rows
        StreamArgs a;
        memset(&a, 0, sizeof(a));
        a.w0[0] = (const uint8_t *)W;
        a.x = x;
        a.y = y;
        a.row_stride = row_stride;
        a.x_stride = x_stride;
        a.y_stride = y_stride;
        a.w_bs = w_bs;
        a.x_bs = x_bs;
        a.y_bs = y_bs;
        a.K = K;
        a.rows = rows;
        a.nvec = B;
        a.nseg = 1;
        a.accumulate = accumulate;
        return stream_any(0, ty, a, n_batch, (hipStream_t)s);
    }
    // Vectors of Q8_0 / Q4_K / Q5_K / Q6_K in one pass on int8 MFMA, every weight read once for all
    // vectors (gs_k_mv_<ty>_<0|1>: 16 rows per workgroup, the row in chunks of up to 4096 elements
    // in LDS with the vectors' q8_1 units). Rows: whole chunks of whole 16-byte pieces, 16-byte
    // aligned rows and activations. Taken where it beats the streaming kernels (measured, one
    // MI355X, 4096 x 4096, 12288 x 4096, 4096 x 12288): from 5 vectors, where they read the
    // matrix twice (Q4_K 12288 x 4096 x 8 vectors: 20.2 against 24.5 us, Q8_0 19.6 against 25.2),
    // from 3 when rows are longer than their register plan (K > 4096: one vector per slice; Q6_K
    // 4096 x 12288 x 4 vectors: 26.4 against 30.3 us), and for Q8_0 from 3 (4096 x 4096: 7.8 against
    // 8.5 us at 3 vectors, 7.9 against 9.2 at 4); below that they stay faster (they overlap the dot
    // products with the weight stream, where this kernel waits for a tile's bytes).
    const int mv_min = ty == GS_Q8_0 || K > 4096 ? 3 : 5;
    if ((ty == GS_Q8_0 || ty == GS_Q4_K || ty == GS_Q5_K || ty == GS_Q6_K) && B >= mv_min && n_batch == 1 && nv_tail == 0 &&
        aligned16(x) && x_stride % 4 == 0 && aligned16(W) && row_stride % 16 == 0) {
        const int ck = std::min(K, 4096);
        const int64_t rbytes = (int64_t)(ck / qk) * bb;
        if (K % ck == 0 && ck % qk == 0 && rbytes % 16 == 0 && rbytes <= 4352) {
            MvArgs m{(const uint8_t *)W, row_stride, x, x_stride, y, y_stride, K, rows, B, accumulate};
            const size_t U = ck / 32, lds = 16 * ((size_t)rbytes + 16) + 320 * U + 8 * 64 * 16;
            // one workgroup per CU at most (its LDS), each walking tiles of 16 rows
            hipError_t e;
            DeviceCtx *c = ctx(&e);
            if (!c) return e;
            const int ntile = (rows + 15) / 16, grid = std::min(ntile, c->cu_count);
            const bool multi = ntile > grid || K > ck;
            return launch("gs_k_mv_" + std::to_string(ty) + (multi ? "_1" : "_0"), dim3((unsigned)grid), dim3(512), lds,
                          (hipStream_t)s, m);
        }
    }
    // more than 4 vectors whose units do not fit 8-vector registers (K > 2048): groups of 4 vectors
    // over the whole K instead of K slices of 8 vectors (8 x 4096 Q8_0: 14 us against 28 us), both
    // groups in one launch (blockIdx.y; the second holds B - 4 vectors), reading the same weights
    // at the same time.
    if (B > 4 && n_batch == 1 && K > 64 * 32)
        return gemv_impl(ty, W, row_stride, K, rows, x, x_stride, y, y_stride, 4, accumulate, 2, 0, 4 * x_stride,
                         4 * y_stride, s, B == 8 ? 0 : B - 4);
    // split K so one lane's q8_1 activation units fit in registers: K <= 64 lanes x (8/NV) units x 32
    const int NVt = B <= 1 ? 1 : B <= 2 ? 2 : B <= 4 ? 4 : 8;
    const int kmax_units = 64 * (8 / NVt);
    // 2..4 vectors whose rows exceed that but fit one vector's units (K <= 16384): one slice per
    // vector in one launch (blockIdx.y, the CUs split between them) instead of K slices launched
    // one after another; a weight row's second and later reads come from the last-level cache
    // (Q6_K 512 x 12288, 4 vectors: 25.8 -> 17.5 us)
    if (B > 1 && B <= 4 && n_batch == 1 && nv_tail == 0 && K > kmax_units * 32 && K <= 64 * 8 * 32)
        return gemv_impl(ty, W, row_stride, K, rows, x, x_stride, y, y_stride, 1, accumulate, B, 0, x_stride, y_stride,
                         s);
    const int step = std::max(qk, 32);
    int kc = std::min(K, kmax_units * 32);
    kc -= kc % step;
    if (kc <= 0) return hipErrorInvalidValue;
    const bool xal = aligned16(x) && (x_stride % 4 == 0) && (x_bs % 4 == 0);
    for (int k0 = 0; k0 < K; k0 += kc) {
        const int kk = std::min(kc, K - k0);
        StreamArgs a;
        memset(&a, 0, sizeof(a));
        a.w0[0] = (const uint8_t *)W + (int64_t)k0 / qk * bb;
        a.x = x + k0;
        a.y = y;
        a.row_stride = row_stride;
        a.x_stride = x_stride;
        a.y_stride = y_stride;
        a.w_bs = w_bs;
        a.x_bs = x_bs;
        a.y_bs = y_bs;
        a.K = kk;
        a.rows = rows;
        a.nvec = B;
        a.nv_tail = nv_tail;
        a.nseg = 1;
        a.accumulate = (k0 > 0) ? 1 : accumulate;
        a.x_aligned = xal && ((k0 * 4) % 16 == 0);
        hipError_t e = stream(0, ty, a, (hipStream_t)s, n_batch);
        if (e != hipSuccess) return e;
    }
    return 0;
}

GS_EXPORT int gs_gemv(int ty, const void *W, int64_t row_stride, int K, int rows, const float *x, int64_t x_stride,
                      float *y, int64_t y_stride, int B, int accumulate, void *s) {
    return gemv_impl(ty, W, row_stride, K, rows, x, x_stride, y, y_stride, B, accumulate, 1, 0, 0, 0, s);
}

GS_EXPORT int gs_gemv_batched(int ty, const void *W, int64_t row_stride, int K, int rows, const float *x, float *y,
                              int n_batch, int64_t w_bs, int64_t x_bs, int64_t y_bs, void *s) {
    return gemv_impl(ty, W, row_stride, K, rows, x, 0, y, 0, 1, 0, n_batch, w_bs, x_bs, y_bs, s);
}

// =============================================================================================
// fused routed-expert FFN (quants.cu:378-409)
// =============================================================================================
static int moe_check(int ty, const GsMoeBatch *b, int nt, int K, int rows, int64_t row_stride) {
    int qk, bb;
    if (!b || b->n <= 0 || b->n > GS_MOE_MAX || nt < 1 || nt > GS_MOE_NT) return hipErrorInvalidValue;
    if (K <= 0 || rows <= 0 || K % 8 != 0) return hipErrorInvalidValue;
    if (!geometry(ty, qk, bb) || K % ggml_block_elems(ty) != 0 || (row_stride & 1)) return hipErrorInvalidValue;
    return 0;
}

static int gateup_args(StreamArgs &a, const GsMoeBatch *b, int nt, int64_t row_stride, int K, int rows,
                       const float *x, float *h, float lim) {
    memset(&a, 0, sizeof(a));
    for (int e = 0; e < b->n; e++) {
        if (((uintptr_t)b->gate[e] | (uintptr_t)b->up[e]) & 1) return hipErrorInvalidValue;
        a.w0[e] = b->gate[e];
        a.w1[e] = b->up[e];
    }
    a.x = x;
    a.y = h;
    a.row_stride = row_stride;
    a.x_stride = K;
    a.K = K;
    a.rows = rows;
    a.nvec = nt;
    a.nseg = b->n;
    a.lim = lim;
    a.x_aligned = aligned16(x) && K % 4 == 0;
    return 0;
}

// experts e0 .. e0+n-1 of the batch
static int down_args(StreamArgs &a, const GsMoeBatch *b, int e0, int n, int nt, int64_t row_stride, int K, int rows,
                     const float *h, float *y) {
    memset(&a, 0, sizeof(a));
    for (int e = 0; e < n; e++) {
        if ((uintptr_t)b->down[e0 + e] & 1) return hipErrorInvalidValue;
        a.w0[e] = b->down[e0 + e];
        for (int t = 0; t < nt; t++) a.wt[t][e] = b->w[t][e0 + e];
    }
    a.x = h + (int64_t)e0 * nt * K;
    a.y = y;
    a.row_stride = row_stride;
    a.y_stride = rows;
    // 32-bit addressing for the 64-lane kernels when every expert's rows lie within 4 GiB of the
    // lowest expert pointer (one buffer resource for all of them); wlo stays null otherwise
    uintptr_t lo = UINTPTR_MAX, hi = 0;
    for (int e = 0; e < n; e++) {
        lo = std::min(lo, (uintptr_t)b->down[e0 + e]);
        hi = std::max(hi, (uintptr_t)b->down[e0 + e] + (uintptr_t)rows * (uintptr_t)row_stride);
    }
    if (n > 0 && hi - lo < (uintptr_t)0xffffffffu) a.wlo = (const uint8_t *)lo;
    a.K = K;
    a.rows = rows;
    a.nvec = nt;
    a.nseg = n;
    a.x_aligned = aligned16(a.x) && K % 4 == 0;
    return 0;
}

// experts one down launch covers: as many as fit one lane's register budget (64 lanes x 8/NV units)
static int down_per_launch(int nt, int K) {
    const int NVt = nt <= 1 ? 1 : 2;
    return std::max(1, 64 * (8 / NVt) / (K / 32));
}

GS_EXPORT int gs_moe_gateup(int ty, const GsMoeBatch *b, int nt, int64_t row_stride, int K, int rows, const float *x,
                            float *h, float lim, void *s) {
    int rc = moe_check(ty, b, nt, K, rows, row_stride);
    if (rc) return rc;
    StreamArgs a;
    if ((rc = gateup_args(a, b, nt, row_stride, K, rows, x, h, lim))) return rc;
    // rows longer than the lanes' register plan holds, or plain rows of 8-element multiples: the
    // row-length-independent kernel, one blockIdx.y slice per expert
    if (K % 32 != 0 || !stream_fits(1, ty, a)) return stream_any(1, ty, a, b->n, (hipStream_t)s);
    return stream(1, ty, a, (hipStream_t)s);
}

GS_EXPORT int gs_moe_down(int ty, const GsMoeBatch *b, int nt, int64_t row_stride, int K, int rows, const float *h,
                          float *y, void *s) {
    int rc = moe_check(ty, b, nt, K, rows, row_stride);
    if (rc) return rc;
    const int per = down_per_launch(nt, K);
    StreamArgs a1;
    if ((rc = down_args(a1, b, 0, 1, nt, row_stride, K, rows, h, y))) return rc;
    if (K % 32 != 0 || !stream_fits(2, ty, a1)) {   // one expert's row exceeds the register plan
        StreamArgs a;
        if ((rc = down_args(a, b, 0, b->n, nt, row_stride, K, rows, h, y))) return rc;
        return stream_any(2, ty, a, 1, (hipStream_t)s);
    }
    for (int e0 = 0; e0 < b->n; e0 += per) {
        const int n = std::min(per, b->n - e0);
        StreamArgs a;
        if ((rc = down_args(a, b, e0, n, nt, row_stride, K, rows, h, y))) return rc;
        hipError_t e = stream(2, ty, a, (hipStream_t)s);
        if (e != hipSuccess) return e;
    }
    return 0;
}

// Routed-expert FFN of one layer: exactly gs_moe_gateup followed by gs_moe_down (h is written
// too), as two launches. (A one-launch variant with a grid-wide barrier between the two passes was
// measured slower once the barrier carries the agent-scope release/acquire fences its cross-XCD
// hand-over of h needs: 27 us against 18 us for config 2.)
GS_EXPORT int gs_moe_ffn(int ty_gu, int ty_dn, const GsMoeBatch *b, int nt, int64_t rs_gu, int n_embd, int n_ff,
                         int64_t rs_dn, const float *x, float *h, float *y, float lim, void *s) {
    int rc = moe_check(ty_gu, b, nt, n_embd, n_ff, rs_gu);
    if (rc) return rc;
    if ((rc = moe_check(ty_dn, b, nt, n_ff, n_embd, rs_dn))) return rc;
    if ((rc = gs_moe_gateup(ty_gu, b, nt, rs_gu, n_embd, n_ff, x, h, lim, s))) return rc;
    return gs_moe_down(ty_dn, b, nt, rs_dn, n_ff, n_embd, h, y, s);
}

// lowest table pointer when every matrix's rows lie within 4 GiB above it, else null
static const uint8_t *table_base(const StreamArgs &a, int n, int rows) {
    uintptr_t lo = UINTPTR_MAX, hi = 0;
    for (int i = 0; i < n; i++) {
        lo = std::min(lo, (uintptr_t)a.w0[i]);
        hi = std::max(hi, (uintptr_t)a.w0[i] + (uintptr_t)rows * (uintptr_t)a.row_stride);
    }
    return n > 0 && hi - lo < (uintptr_t)0xffffffffu ? (const uint8_t *)lo : nullptr;
}

// Routed-expert FFN of n_tok tokens, each over its own batch b[t] (one token, b[t].n experts, the
// same n for every token): exactly gs_moe_ffn(ty_gu, ty_dn, &b[t], 1, ...) per token on
// x + t*n_embd, h + t*n*n_ff, y + t*n_embd, as one gate/up and one down launch whose blockIdx.y
// slice t runs token t with pointer-table entries [t*n, (t+1)*n).
GS_EXPORT int gs_moe_ffn_tokens(int ty_gu, int ty_dn, const GsMoeBatch *b, int n_tok, int64_t rs_gu, int n_embd,
                                int n_ff, int64_t rs_dn, const float *x, float *h, float *y, float lim, void *s) {
    if (!b || n_tok < 1 || n_tok > GS_SEG_MAX) return hipErrorInvalidValue;
    const int n = b[0].n;
    for (int t = 0; t < n_tok; t++) {
        int rc = moe_check(ty_gu, &b[t], 1, n_embd, n_ff, rs_gu);
        if (rc) return rc;
        if ((rc = moe_check(ty_dn, &b[t], 1, n_ff, n_embd, rs_dn))) return rc;
        if (b[t].n != n) return hipErrorInvalidValue;
    }
    if (n_tok * n > GS_SEG_MAX) return hipErrorInvalidValue;
    StreamArgs a, at;
    int rc;
    {   // shapes outside the streaming plan: the per-token FFN (the same arithmetic)
        StreamArgs g, d;
        if ((rc = gateup_args(g, &b[0], 1, rs_gu, n_embd, n_ff, x, h, lim))) return rc;
        if ((rc = down_args(d, &b[0], 0, 1, 1, rs_dn, n_ff, n_embd, h, y))) return rc;
        if (n_embd % 32 != 0 || n_ff % 32 != 0 || !stream_fits(1, ty_gu, g) || !stream_fits(2, ty_dn, d)) {
            for (int t = 0; t < n_tok; t++)
                if ((rc = gs_moe_ffn(ty_gu, ty_dn, &b[t], 1, rs_gu, n_embd, n_ff, rs_dn, x + (int64_t)t * n_embd,
                                     h + (int64_t)t * n * n_ff, y + (int64_t)t * n_embd, lim, s)))
                    return rc;
            return 0;
        }
    }
    for (int t = 0; t < n_tok; t++) {
        if ((rc = gateup_args(at, &b[t], 1, rs_gu, n_embd, n_ff, x, h, lim))) return rc;
        if (t == 0) a = at;
        for (int e = 0; e < n; e++) a.w0[t * n + e] = at.w0[e], a.w1[t * n + e] = at.w1[e];
    }
    a.x_bs = n_embd;
    a.y_bs = (int64_t)n * n_ff;
    hipError_t e = stream(1, ty_gu, a, (hipStream_t)s, n_tok);
    if (e != hipSuccess) return e;
    const int per = down_per_launch(1, n_ff);
    for (int e0 = 0; e0 < n; e0 += per) {
        const int m = std::min(per, n - e0);
        for (int t = 0; t < n_tok; t++) {
            if ((rc = down_args(at, &b[t], e0, m, 1, rs_dn, n_ff, n_embd, h, y))) return rc;
            if (t == 0) a = at;
            for (int i = 0; i < m; i++) a.w0[t * m + i] = at.w0[i], a.wt[0][t * m + i] = at.wt[0][i];
        }
        a.wlo = table_base(a, n_tok * m, n_embd);
        a.x_bs = (int64_t)n * n_ff;
        a.y_bs = n_embd;
        if ((e = stream(2, ty_dn, a, (hipStream_t)s, n_tok)) != hipSuccess) return e;
    }
    return 0;
}

// =============================================================================================
// GEMM (gemm.cu:107-123): MFMA tiles of 128 weight rows x 64 tokens (gemm.hip)
// =============================================================================================
namespace {
// K slices of a gs_gemm problem: small grids (at most half as many 128 x 64 tiles as CUs) split K
// over blockIdx.z so the slices fill the idle CUs; 1 = no split.
int gemm_slices(DeviceCtx *c, int K, int rows, int N, int n_batch, int *ksb) {
    const int nsb = (K + 255) / 256;
    const int64_t tiles = (int64_t)((rows + 127) / 128) * ((N + 63) / 64) * n_batch;
    *ksb = nsb;
    if (!(2 * tiles <= c->cu_count && nsb >= 2)) return 1;
    // one super-block per slice where the CUs allow (IQ2_XXS 1536 x 4096, N = 64: 75 -> 16 us;
    // two per slice: 19 us)
    int nks = (int)std::min<int64_t>(std::min(nsb, GS_GEMM_KS_MAX), c->cu_count / tiles);
    *ksb = (nsb + nks - 1) / nks;
    return (nsb + *ksb - 1) / *ksb;
}
size_t gemm_part_bytes(int nks, int rows, int N, int n_batch) {
    return nks > 1 ? (size_t)nks * n_batch * N * rows * sizeof(float) : 0;
}

// ---- library path: dequantize to f16, convert X to f16, contract on hipBLASLt -----------------
// With enough tokens (gemm_lib_tokens) and a workspace, gs_gemm_ex writes the weights once as f16
// (the same f16(dequant) values the tile kernel rounds to), converts X to f16 (same rounding) and
// runs the contraction as a plain f16 x f16 -> f32 GEMM (f32 accumulation) in hipBLASLt: Q4_K
// 12288 x 4096 x 512 tokens 126 us in the tile kernel against about 82 us this way (dequant
// pass ~24 us, conversion ~3 us, library GEMM ~55 us). The algorithm is the library heuristic's
// first choice for the shape (fixed per shape, so results repeat call to call).
// Token counts where the library path wins (measured, one MI355X): above 128 tokens for matrices
// of 2^25 weights and more (Q4_K 12288 x 4096: 58 against 84 us at N = 136, where the tiles pass
// 256 CUs and need a second round, 44 against 62 us the other way at N = 128; Q6_K 4096 x 12288:
// 59 against 77 us at 136, 75 against 131 us at 320), from 256 tokens otherwise (Q4_K 4096 x 4096:
// even at 256, 38 against 43 us at 320); below that the fixed dequant pass costs more than the
// tiles lose.
bool gemm_lib_tokens(int K, int rows, int N) {
    return N >= 256 || (N > 128 && (int64_t)rows * K >= ((int64_t)1 << 25));
}
// hipBLASLt entry points, from libhipblaslt opened on first use (no link-time dependency: without
// the library the tiles run every problem)
struct LtApi {
    decltype(&hipblasLtCreate) create = nullptr;
    decltype(&hipblasLtMatmulDescCreate) desc_create = nullptr;
    decltype(&hipblasLtMatmulDescSetAttribute) desc_set = nullptr;
    decltype(&hipblasLtMatrixLayoutCreate) layout_create = nullptr;
    decltype(&hipblasLtMatmulPreferenceCreate) pref_create = nullptr;
    decltype(&hipblasLtMatmulPreferenceSetAttribute) pref_set = nullptr;
    decltype(&hipblasLtMatmulPreferenceDestroy) pref_destroy = nullptr;
    decltype(&hipblasLtMatmulAlgoGetHeuristic) heuristic = nullptr;
    decltype(&hipblasLtMatmul) matmul = nullptr;
};
const LtApi *lt_api() {
    static LtApi api;
    static std::once_flag once;
    static bool ok = false;
    std::call_once(once, [] {
        void *h = dlopen("libhipblaslt.so.1", RTLD_NOW | RTLD_LOCAL);
        if (!h) h = dlopen("libhipblaslt.so", RTLD_NOW | RTLD_LOCAL);
        if (!h) return;
#define GS_LT_SYM(field, name) api.field = (decltype(api.field))dlsym(h, #name)
        GS_LT_SYM(create, hipblasLtCreate);
        GS_LT_SYM(desc_create, hipblasLtMatmulDescCreate);
        GS_LT_SYM(desc_set, hipblasLtMatmulDescSetAttribute);
        GS_LT_SYM(layout_create, hipblasLtMatrixLayoutCreate);
        GS_LT_SYM(pref_create, hipblasLtMatmulPreferenceCreate);
        GS_LT_SYM(pref_set, hipblasLtMatmulPreferenceSetAttribute);
        GS_LT_SYM(pref_destroy, hipblasLtMatmulPreferenceDestroy);
        GS_LT_SYM(heuristic, hipblasLtMatmulAlgoGetHeuristic);
        GS_LT_SYM(matmul, hipblasLtMatmul);
#undef GS_LT_SYM
        ok = api.create && api.desc_create && api.desc_set && api.layout_create && api.pref_create && api.pref_set &&
             api.pref_destroy && api.heuristic && api.matmul;
    });
    return ok ? &api : nullptr;
}
constexpr size_t GS_GEMM_LT_WS = (size_t)32 << 20;
size_t a256(size_t n) { return (n + 255) & ~(size_t)255; }
size_t gemm_lib_bytes(int K, int rows, int N) {
    return a256((size_t)rows * K * 2) + a256((size_t)N * K * 2) + GS_GEMM_LT_WS;
}
// the plan for this shape; nullptr if the library is unavailable (the caller then runs the tiles)
DeviceCtx::LtPlan *lt_plan(DeviceCtx *c, int K, int rows, int N, int64_t y_stride) {
    const LtApi *L = lt_api();
    if (!L) return nullptr;
    std::lock_guard<std::mutex> lk(c->lt_mu);
    if (c->lt_failed) return nullptr;
    if (!c->lt && L->create(&c->lt) != HIPBLAS_STATUS_SUCCESS) {
        c->lt = nullptr;
        c->lt_failed = true;
        return nullptr;
    }
    const std::vector<int64_t> key{K, rows, N, y_stride};
    auto it = c->lt_plans.find(key);
    if (it != c->lt_plans.end()) return &it->second;
    // column-major view: Y (rows x N, ld y_stride) = W16^T (W16: K x rows, ld K) * X16 (K x N, ld K)
    DeviceCtx::LtPlan P;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    const hipblasStatus_t S = HIPBLAS_STATUS_SUCCESS;
    bool ok = L->desc_create(&P.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == S;
    ok = ok && L->desc_set(P.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) == S;
    ok = ok && L->desc_set(P.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) == S;
    ok = ok && L->layout_create(&P.la, HIP_R_16F, K, rows, K) == S;
    ok = ok && L->layout_create(&P.lb, HIP_R_16F, K, N, K) == S;
    ok = ok && L->layout_create(&P.lc, HIP_R_32F, rows, N, y_stride) == S;
    hipblasLtMatmulPreference_t pref = nullptr;
    size_t ws = GS_GEMM_LT_WS;
    ok = ok && L->pref_create(&pref) == S;
    ok = ok && L->pref_set(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)) == S;
    hipblasLtMatmulHeuristicResult_t r;
    int nr = 0;
    ok = ok && L->heuristic(c->lt, P.desc, P.la, P.lb, P.lc, P.lc, pref, 1, &r, &nr) == S && nr > 0;
    if (pref) L->pref_destroy(pref);
    (void)hipGetLastError();
    if (!ok) return nullptr;   // no algorithm for this shape: the tiles run it
    P.algo = r.algo;
    return &(c->lt_plans[key] = P);
}
// the library path's conditions (gs_gemm_ex; gs_gemm_path reports them)
bool gemm_lib_eligible(int ty, int K, int rows, int N, int64_t row_stride, int64_t y_stride, size_t work_bytes) {
    int qk, bb;
    if (!geometry(ty, qk, bb)) return false;
    const bool lib_ty = ty != GS_F32 && ty != GS_BF16;   // float weights: not measured this way
    return lib_ty && rows > 0 && gemm_lib_tokens(K, rows, N) && row_stride == (int64_t)(K / qk) * bb && y_stride >= rows &&
           work_bytes >= gemm_lib_bytes(K, rows, N);
}
// -1: not taken (the tile kernel runs the problem); otherwise the HIP status of the launches
int gemm_lib(DeviceCtx *c, int ty, const uint8_t *W, int K, int rows, const float *X, int64_t x_stride, float *Y,
             int64_t y_stride, int N, int accumulate, int n_batch, int64_t w_bs, int64_t x_bs, int64_t y_bs, void *work,
             hipStream_t s) {
    DeviceCtx::LtPlan *P = lt_plan(c, K, rows, N, y_stride);
    if (!P) return -1;
    uint8_t *w16 = (uint8_t *)work;
    uint16_t *x16 = (uint16_t *)(w16 + a256((size_t)rows * K * 2));
    void *lws = (uint8_t *)x16 + a256((size_t)N * K * 2);
    const float alpha = 1.f, beta = accumulate ? 1.f : 0.f;
    for (int z = 0; z < n_batch; z++) {
        const void *a16 = w16;
        const int64_t xthr = (int64_t)N * (K / 4);   // activation pieces of 4 values
        int e;
        if (ty == GS_F16 && aligned16(W + z * w_bs)) {   // already f16, contiguous and 16-byte aligned: in place
            a16 = W + z * w_bs;
            CvtArgs cv{X + z * x_bs, x16, x_stride, K, N};
            e = launch("gs_k_rows_to_f16", dim3((unsigned)((xthr + 255) / 256)), dim3(256), 0, s, cv);
        } else {
            // one launch: the weight units' blocks, then the activation conversion's blocks
            const int64_t n = (int64_t)rows * K;
            DequantArgs d{W + z * w_bs, w16, n, (n + 31) / 32, 1, 0, X + z * x_bs, x16, x_stride, K, N};
            d.w_blocks = (int)((d.n_units + 255) / 256);
            const std::string name = "gs_k_dequant_f16_" + std::to_string(ty);
            e = launch(name, dim3((unsigned)(d.w_blocks + (xthr + 255) / 256)), dim3(256), 0, s, d);
        }
        if (e != hipSuccess) return e;
        float *y = Y + z * y_bs;
        if (lt_api()->matmul(c->lt, P->desc, &alpha, a16, P->la, x16, P->lb, &beta, y, P->lc, y, P->lc, &P->algo, lws,
                            GS_GEMM_LT_WS, s) != HIPBLAS_STATUS_SUCCESS)
            return hipErrorLaunchFailure;
    }
    return hipSuccess;
}

int gemm_impl(int ty, const void *W, int64_t row_stride, int K, int rows, const float *X, int64_t x_stride, float *Y,
              int64_t y_stride, int N, int accumulate, int n_batch, int64_t w_bs, int64_t x_bs, int64_t y_bs,
              void *work, size_t work_bytes, void *s) {
    if (K <= 0 || K % 32 != 0 || N < 1 || n_batch < 1 || x_stride % 4 != 0 || rows < 0) return hipErrorInvalidValue;
    int qk, bb;
    if (!geometry(ty, qk, bb) || K % ggml_block_elems(ty) != 0) return hipErrorInvalidValue;
    // X rows are read as float4 (the reference's contract: 16-byte aligned rows)
    if (!aligned16(X) || (n_batch > 1 && x_bs % 4 != 0)) return hipErrorInvalidValue;
    if (!check_w(W, row_stride) || (n_batch > 1 && (w_bs & 1))) return hipErrorInvalidValue;
    if (rows == 0) return 0;
    // bytes of one 256-element super-block of a row and its LDS slot (gemm.hip GemmFmt::SB, SBP:
    // rounded up to an odd number of dwords)
    const int eb = ggml_block_elems(ty);
    const int sb = eb == 1 ? 256 * (bb / qk) : 256 / eb * bb;
    const int sbp = 4 * (((sb + 3) / 4) | 1);
    const bool plain = eb == 1;
    const size_t lds = gs_gemm_nbuf(ty) * ((plain ? 16 : (size_t)128 * sbp) + (size_t)64 * 512);
    GemmArgs a;
    memset(&a, 0, sizeof(a));
    a.W = (const uint8_t *)W;
    a.X = X;
    a.Y = Y;
    a.row_stride = row_stride;
    a.x_stride = x_stride;
    a.y_stride = y_stride;
    a.w_bs = w_bs;
    a.x_bs = x_bs;
    a.y_bs = y_bs;
    a.K = K;
    a.rows = rows;
    a.N = N;
    a.accumulate = accumulate;
    a.wait_limit = g_wait_limit.load();
    a.wait_force = g_wait_force.load();
    a.n_rb = (rows + 127) / 128;
    a.n_tb = (N + 63) / 64;
    // row block r runs on XCD r % 8 (workgroup w -> XCD w % 8): 8 x ceil(n_rb / 8) x n_tb workgroups
    const int64_t nwg = (int64_t)8 * ((a.n_rb + 7) / 8) * a.n_tb;
    if (nwg > 0x7fffffff || n_batch > 65535) return hipErrorInvalidValue;
    a.ksb = (K + 255) / 256;
    hipError_t e;
    DeviceCtx *c = ctx(&e);
    if (!c) return e;
    // many tokens and a workspace for the f16 operands: dequantize + library GEMM (contiguous rows;
    // every block format, and F16 weights as they are: Q8_0 too, whose tile decode is the cheapest,
    // 42 against 50 us at 4096 x 4096 x 512 and 82 against 137 us at 12288 x 4096 x 512)
    if (work && aligned16(work) && gemm_lib_eligible(ty, K, rows, N, row_stride, y_stride, work_bytes)) {
        const int r = gemm_lib(c, ty, (const uint8_t *)W, K, rows, X, x_stride, Y, y_stride, N, accumulate, n_batch, w_bs,
                               x_bs, y_bs, work, (hipStream_t)s);
        if (r >= 0) return r;
    }
    const std::string name = "gs_k_gemm_" + std::to_string(ty);
    // K split only into the caller's workspace: each slice writes its f32 partial tile there and
    // gs_k_gemm_reduce sums the slices in slice order into Y (a fixed order, so the result is
    // reproducible). Without a workspace the whole K runs in one tile pass.
    int ksb = 0;
    const int nks = work ? gemm_slices(c, K, rows, N, n_batch, &ksb) : 1;
    if (nks == 1)
        return launch(name, dim3((unsigned)nwg, n_batch, 1), dim3(GS_GEMM_THREADS, 1, 1), lds, (hipStream_t)s, a);
    if (work_bytes < gemm_part_bytes(nks, rows, N, n_batch) || !aligned16(work)) return hipErrorInvalidValue;
    a.ksb = ksb;
    a.part = (float *)work;
    e = launch(name, dim3((unsigned)nwg, n_batch, nks), dim3(GS_GEMM_THREADS, 1, 1), lds, (hipStream_t)s, a);
    if (e == hipSuccess) {
        GemmReduceArgs r{a.part, Y, y_stride, y_bs, rows, N, n_batch, nks, accumulate};
        const int64_t total = (int64_t)n_batch * N * rows;
        const unsigned g = (unsigned)std::min<int64_t>((total + 255) / 256, 4 * (int64_t)c->cu_count);
        e = launch("gs_k_gemm_reduce", dim3(g), dim3(256), 0, (hipStream_t)s, r);
    }
    return e;
}
}  // namespace

GS_EXPORT int gs_gemm(int ty, const void *W, int64_t row_stride, int K, int rows, const float *X, int64_t x_stride,
                      float *Y, int64_t y_stride, int N, int accumulate, int n_batch, int64_t w_bs, int64_t x_bs,
                      int64_t y_bs, void *s) {
    return gemm_impl(ty, W, row_stride, K, rows, X, x_stride, Y, y_stride, N, accumulate, n_batch, w_bs, x_bs, y_bs,
                     nullptr, 0, s);
}

GS_EXPORT int gs_gemm_workspace(int K, int rows, int N, int n_batch, size_t *bytes) {
    if (!bytes || K <= 0 || rows < 0 || N < 1 || n_batch < 1) return hipErrorInvalidValue;
    hipError_t e;
    DeviceCtx *c = ctx(&e);
    if (!c) return e;
    int ksb = 0;
    *bytes = rows == 0 ? 0 : gemm_part_bytes(gemm_slices(c, K, rows, N, n_batch, &ksb), rows, N, n_batch);
    if (rows > 0 && gemm_lib_tokens(K, rows, N)) *bytes = std::max(*bytes, gemm_lib_bytes(K, rows, N));
    return 0;
}

GS_EXPORT int gs_gemm_path(int ty, int K, int rows, int N, int64_t row_stride, int64_t y_stride, size_t work_bytes) {
    hipError_t e;
    DeviceCtx *c = ctx(&e);
    if (!c) return -(int)e;
    if (gemm_lib_eligible(ty, K, rows, N, row_stride, y_stride, work_bytes) && lt_plan(c, K, rows, N, y_stride))
        return 2;
    int ksb = 0;
    return work_bytes > 0 && gemm_slices(c, K, rows, N, 1, &ksb) > 1 &&
                   work_bytes >= gemm_part_bytes(gemm_slices(c, K, rows, N, 1, &ksb), rows, N, 1)
               ? 1
               : 0;
}

GS_EXPORT int gs_gemm_ex(int ty, const void *W, int64_t row_stride, int K, int rows, const float *X, int64_t x_stride,
                         float *Y, int64_t y_stride, int N, int accumulate, int n_batch, int64_t w_bs, int64_t x_bs,
                         int64_t y_bs, void *work, size_t work_bytes, void *s) {
    return gemm_impl(ty, W, row_stride, K, rows, X, x_stride, Y, y_stride, N, accumulate, n_batch, w_bs, x_bs, y_bs,
                     work, work_bytes, s);
}

// =============================================================================================
// element-wise / row glue (ops.cu:101-125; gemm.cu:125-163)
// =============================================================================================
GS_EXPORT int gs_swiglu(const float *g, const float *u, float *y, int64_t n, float lim, void *s) {
    if (n <= 0) return 0;
    EltArgs a{g, u, y, n, lim};
    return launch("gs_k_swiglu", dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)s, a);
}
GS_EXPORT int gs_axpy(float *y, const float *x, float alpha, int64_t n, void *s) {
    if (n <= 0) return 0;
    EltArgs a{x, nullptr, y, n, alpha};
    return launch("gs_k_axpy", dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)s, a);
}
GS_EXPORT int gs_f32_to_f16(const float *x, void *y, int64_t n, void *s) {
    if (n <= 0) return 0;
    EltArgs a{x, nullptr, (float *)y, n, 0.f};
    return launch("gs_k_f32_to_f16", dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)s, a);
}
GS_EXPORT int gs_gather_rows(const float *x, const int *idx, float *y, int rows, int n, void *s) {
    if (rows <= 0) return 0;
    if (n <= 0) return hipErrorInvalidValue;
    RowsArgs a{x, idx, nullptr, y, rows, n};
    return launch("gs_k_gather_rows", dim3((n + 255) / 256, rows), dim3(256), 0, (hipStream_t)s, a);
}
GS_EXPORT int gs_scatter_add_rows(float *acc, const int *idx, const float *w, const float *y, int rows, int n, void *s) {
    if (rows <= 0) return 0;
    if (n <= 0) return hipErrorInvalidValue;
    RowsArgs a{y, idx, w, acc, rows, n};
    return launch("gs_k_scatter_add_rows", dim3((n + 255) / 256, rows), dim3(256), 0, (hipStream_t)s, a);
}


// =============================================================================================
// grouped routed-expert FFN (no single reference kernel: it fuses what forward.rs:1399-1413
// run_expert_rows does per expert -- gather, gate/up GEMM, SwiGLU, down GEMM, weighted
// scatter-add -- for every expert of a layer at once)
// =============================================================================================
namespace {
size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
struct GroupedWork {
    size_t x16, xs, h, h16, hs, total;
};
GroupedWork grouped_layout(int n_tok, int n_pairs, int K, int n_ff) {
    GroupedWork w;
    size_t o = 0;
    w.x16 = o; o += align256((size_t)n_tok * K * 2);
    w.xs = o;  o += align256((size_t)n_tok * 4);
    w.h = o;   o += align256((size_t)n_pairs * n_ff * 4);
    w.h16 = o; o += align256((size_t)n_pairs * n_ff * 2);
    w.hs = o;  o += align256((size_t)n_pairs * 4);
    w.total = o;
    return w;
}

hipError_t rows_f16(const float *x, int64_t x_stride, int K, int nrows, uint16_t *out, float *scale, hipStream_t s) {
    if (nrows <= 0) return hipSuccess;
    RowsQArgs a{x, x_stride, out, scale, K, nrows};
    // one wave per row while that fills the chip (four rows per block); fewer, long rows take a
    // workgroup each (same result)
    hipError_t e;
    DeviceCtx *c = ctx(&e);
    if (!c) return e;
    if (K >= 2048 && nrows < 4 * c->cu_count)
        return launch("gs_k_rows_f16_wg", dim3(nrows), dim3(256), 0, s, a);
    return launch("gs_k_rows_f16", dim3((nrows + 3) / 4), dim3(256), 0, s, a);
}

// kind 1 (gate/up) or 2 (down) over every tile of the layer; the grid is persistent.
// Tile shape: NT token sub-tiles of 16 (the chunk of one expert's pairs a workgroup takes), NR row
// sub-tiles of 16 per wave, WV waves per workgroup (one workgroup per CU shares the 65 KB decode
// table; WV = 16 doubles the waves available to hide latency where registers allow). Larger
// tiles stage fewer activation bytes per weight byte, but the tile count must still fill the
// chip: take the first preferred shape whose (upper-bound) tile count is at least two per CU.
// Instantiated shapes: grouped.hip GS_GRP_KERNEL.
struct GrpShape {
    int nt, nr, wv;
};
hipError_t grouped_launch(int kind, int ty, GroupedArgs &a, int n_pairs, hipStream_t s) {
    hipError_t e;
    DeviceCtx *c = ctx(&e);
    if (!c) return e;
    static const std::vector<GrpShape> all1 = {{1, 1, 8}, {1, 2, 8}, {2, 1, 8}, {2, 2, 8}, {1, 1, 16}};
    static const std::vector<GrpShape> all2 = {{1, 1, 8}, {1, 2, 8}, {1, 4, 8}, {2, 1, 8}, {2, 2, 8}, {2, 4, 8},
                                               {1, 1, 16}, {1, 2, 16}, {2, 1, 16}};
    // preference order (largest useful tile first), per token-chunk size
    static const std::vector<GrpShape> pref1 = {{2, 2, 8}, {2, 1, 8}, {1, 2, 8}, {1, 1, 16}, {1, 1, 8}};
    static const std::vector<GrpShape> pref2 = {{2, 4, 8}, {2, 2, 8}, {1, 4, 8}, {1, 2, 8}, {2, 1, 8}, {1, 1, 8}};
    const int groups = std::min(a.n_exp, n_pairs);
    auto tiles = [&](const GrpShape &sh) {
        const int64_t rbk = (int64_t)sh.wv * 16 * sh.nr;
        return (a.rows + rbk - 1) / rbk * (groups + (n_pairs + 16 * sh.nt - 1) / (16 * sh.nt));
    };
    GrpShape sh{0, 0, 0};
    for (const GrpShape &p : kind == 1 ? pref1 : pref2) {
        if ((n_pairs <= 64) != (p.nt == 1)) continue;    // decode-sized batches: one token sub-tile
        sh = p;
        if (tiles(p) >= 2 * (int64_t)c->cu_count) break;
    }
    const auto &all = kind == 1 ? all1 : all2;
    if (std::none_of(all.begin(), all.end(),
                     [&](const GrpShape &p) { return p.nt == sh.nt && p.nr == sh.nr && p.wv == sh.wv; }))
        return hipErrorInvalidValue;
    const std::string name = "gs_k_grouped_" + std::to_string(ty) + "_" + std::to_string(kind) + "_" + std::to_string(sh.nt) + "_" +
                             std::to_string(sh.nr) + "_" + std::to_string(sh.wv);
    hipFunction_t f;
    if ((e = get_fn(c, name, &f)) != hipSuccess) return e;
    const int threads = 64 * sh.wv;
    // decode tables (80 KB, grouped.hip GS_GRP_TAB_BYTES) + four staged activation super-blocks +
    // the workgroup's bookkeeping
    const size_t lds = 16384 + 65536 + 4 * (size_t)16 * sh.nt * 512 + GS_GRP_META_BYTES;
    int per_cu = 1;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto key = std::make_pair(name, (int)lds);
        auto it = c->occ.find(key);
        if (it != c->occ.end()) {
            per_cu = it->second;
        } else {
            int nb = 0;
            if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&nb, f, threads, lds) != hipSuccess || nb < 1) nb = 1;
            c->occ[key] = per_cu = nb;
        }
    }
    const int grid = (int)std::max<int64_t>(1, std::min<int64_t>(tiles(sh), (int64_t)c->cu_count * per_cu));
    return launch(name, dim3(grid), dim3(threads), lds, s, a);
}
}  // namespace

GS_EXPORT int gs_moe_grouped_workspace(int n_tok, int n_pairs, int K, int n_ff, size_t *bytes) {
    if (!bytes || n_tok < 0 || n_pairs < 0 || K <= 0 || n_ff <= 0) return hipErrorInvalidValue;
    *bytes = grouped_layout(n_tok, n_pairs, K, n_ff).total;
    return 0;
}

namespace {
// Both grouped entry points: pair p reads x[idx[p]] and adds into y[out_idx[p]].
int grouped_ffn(int ty_gu, int ty_down, const GsExpertPtrs *experts, int n_exp, const int *offs, const int *idx,
                const int *out_idx, const float *w, int n_pairs, int n_tok, int64_t gu_row_stride, int K, int n_ff,
                int64_t down_row_stride, const float *x, float *y, float lim, void *work, size_t work_bytes, void *s) {
    auto grp_type = [](int t) { return t == GS_IQ2_XXS || t == GS_IQ3_XXS; };
    if (!grp_type(ty_gu) || !grp_type(ty_down)) return hipErrorInvalidValue;
    if (n_exp < 1 || n_exp > GS_GRP_EXP_MAX || n_pairs < 0 || n_tok < 1) return hipErrorInvalidValue;
    // whole super-blocks, at least two per row (the kernel's load pipeline runs two ahead)
    if (K < 512 || n_ff < 512 || K % 256 != 0 || n_ff % 256 != 0) return hipErrorInvalidValue;
    if (!experts || !offs || !x || !y || (gu_row_stride & 1) || (down_row_stride & 1)) return hipErrorInvalidValue;
    auto sb_bytes = [](int t) { return t == GS_IQ3_XXS ? 98 : 66; };
    if (gu_row_stride < (int64_t)K / 256 * sb_bytes(ty_gu) || down_row_stride < (int64_t)n_ff / 256 * sb_bytes(ty_down))
        return hipErrorInvalidValue;
    if (n_pairs == 0) return 0;
    if (!idx || !out_idx || !w || !aligned16(x) || ((uintptr_t)work & 255)) return hipErrorInvalidValue;
    const GroupedWork L = grouped_layout(n_tok, n_pairs, K, n_ff);
    if (!work || work_bytes < L.total) return hipErrorInvalidValue;
    uint8_t *wb = (uint8_t *)work;
    uint16_t *x16 = (uint16_t *)(wb + L.x16), *h16 = (uint16_t *)(wb + L.h16);
    float *xs = (float *)(wb + L.xs), *h = (float *)(wb + L.h), *hs = (float *)(wb + L.hs);
    hipStream_t st = (hipStream_t)s;
    hipError_t e = rows_f16(x, K, K, n_tok, x16, xs, st);
    if (e != hipSuccess) return e;
    GroupedArgs a;
    memset(&a, 0, sizeof(a));
    a.experts = (const uint8_t *const *)experts;
    a.offs = offs;
    a.idx = idx;
    a.w = w;
    a.act = x16;
    a.ascale = xs;
    a.out = h;
    a.row_stride = gu_row_stride;
    a.K = K;
    a.rows = n_ff;
    a.n_exp = n_exp;
    a.lim = lim;
    a.wait_limit = g_wait_limit.load();
    a.wait_force = g_wait_force.load();
    if ((e = grouped_launch(1, ty_gu, a, n_pairs, st)) != hipSuccess) return e;
    if ((e = rows_f16(h, n_ff, n_ff, n_pairs, h16, hs, st)) != hipSuccess) return e;
    a.act = h16;
    a.ascale = hs;
    a.out = y;
    a.idx = out_idx;   // the down pass reads h per pair; idx only addresses its output rows
    a.row_stride = down_row_stride;
    a.K = n_ff;
    a.rows = K;
    return grouped_launch(2, ty_down, a, n_pairs, st);
}
}  // namespace

GS_EXPORT int gs_moe_grouped(int ty_gu, int ty_down, const GsExpertPtrs *experts, int n_exp, const int *offs,
                             const int *idx, const float *w, int n_pairs, int n_tok, int64_t gu_row_stride, int K,
                             int n_ff, int64_t down_row_stride, const float *x, float *y, float lim, void *work,
                             size_t work_bytes, void *s) {
    return grouped_ffn(ty_gu, ty_down, experts, n_exp, offs, idx, idx, w, n_pairs, n_tok, gu_row_stride, K, n_ff,
                       down_row_stride, x, y, lim, work, work_bytes, s);
}

GS_EXPORT int gs_moe_grouped_scatter(int ty_gu, int ty_down, const GsExpertPtrs *experts, int n_exp, const int *offs,
                                     const int *idx, const int *out_idx, const float *w, int n_pairs, int n_tok,
                                     int64_t gu_row_stride, int K, int n_ff, int64_t down_row_stride, const float *x,
                                     float *y, float lim, void *work, size_t work_bytes, void *s) {
    return grouped_ffn(ty_gu, ty_down, experts, n_exp, offs, idx, out_idx, w, n_pairs, n_tok, gu_row_stride, K, n_ff,
                       down_row_stride, x, y, lim, work, work_bytes, s);
}



// =============================================================================================
// bounded-wait status (no counterpart in the reference)
// =============================================================================================
GS_EXPORT int gs_wait_status(void *s) {
    hipError_t e;
    DeviceCtx *c = ctx(&e);
    if (!c) return e;
    if ((e = hipStreamSynchronize((hipStream_t)s)) != hipSuccess) return e;
    bool expired = false;
    for (void *f : c->wait_flags) {
        uint32_t v = 0;
        if ((e = hipMemcpy(&v, f, 4, hipMemcpyDeviceToHost)) != hipSuccess) return e;
        if (v) {
            expired = true;
            const uint32_t zero = 0;
            if ((e = hipMemcpy(f, &zero, 4, hipMemcpyHostToDevice)) != hipSuccess) return e;
        }
    }
    return expired ? hipErrorLaunchFailure : hipSuccess;
}

GS_EXPORT int gs_debug_wait_limit(uint32_t polls, int force) {
    g_wait_limit.store(polls);
    g_wait_force.store(force ? 1u : 0u);
    return 0;
}
