// Native timing loops for bench.py. Each loop drives the gs_* C ABI exactly as the engine's
// decode path does (crates/engine/src/forward.rs:1067-1107: one gs_moe_gateup + one gs_moe_down
// per expert batch) and brackets the timed launches with HIP events on the launch stream, so the
// host-side Python loop adds no gaps between kernels.
#include <stdint.h>
#include "../../include/glmssd.h"

#define BN_EXPORT extern "C" __attribute__((visibility("default")))
#define CK(x)                  \
    do {                       \
        int _e = (x);          \
        if (_e) return _e;     \
    } while (0)

namespace {
struct Timer {
    void *a = nullptr, *b = nullptr;
    int init() {
        CK(gs_event_create_timed(&a));
        return gs_event_create_timed(&b);
    }
    ~Timer() {
        if (a) gs_event_destroy(a);
        if (b) gs_event_destroy(b);
    }
};

// Minimum GPU time of warm-up before a timed loop (bn_set_ramp_ms). After an idle stretch (the host
// generating a workload's data) the GPU's clocks need tens of milliseconds of load to come back
// up, far longer than a few dozen warm-up steps of a few microseconds: config 2 times 17.9 us per
// step after 50 warm-up steps against 16.7 us once 85 ms of steps have run.
float g_ramp_ms = 100.0f;

// The `warmup` steps step(0 .. warmup-1), then more (in chunks, with a GPU-time check between
// chunks) until at least g_ramp_ms of GPU time has passed; *done = steps run, so the timed steps
// continue the rotation and none of them re-reads data a warm-up step just left in the caches.
// step(0) runs and completes before the ramp's clock starts: a first call's one-time host work
// (the GEMM library path opens hipBLASLt and picks its algorithm: 0.75 s) would otherwise sit
// inside the first interval as idle GPU time, end the ramp at once and leave the timed loop on
// idle clocks (Q4_K 12288 x 4096 x 512: 86 against 73 us).
template <class F>
int warm(F &&step, int warmup, void *s, int *done) {
    Timer t;
    CK(t.init());
    CK(step(0));
    CK(gs_stream_sync(s));
    CK(gs_event_record(t.a, s));
    int i = 1;
    for (; i < warmup; i++) CK(step(i));
    while (g_ramp_ms > 0.0f) {
        CK(gs_event_record(t.b, s));
        CK(gs_event_sync(t.b));
        float ms = 0.0f;
        CK(gs_event_elapsed_ms(&ms, t.a, t.b));
        if (ms >= g_ramp_ms) break;
        for (int j = 0; j < 32; j++, i++) CK(step(i));
    }
    *done = i;
    return gs_stream_sync(s);
}
}  // namespace

BN_EXPORT void bn_set_ramp_ms(float ms) { g_ramp_ms = ms; }

// Decode step = gs_moe_gateup + gs_moe_down over batch (i % nb). ms_step: mean per step;
// ms_gateup: mean of a separate loop of gs_moe_gateup alone (dominant kernel).
BN_EXPORT int bn_moe_decode(int ty_gu, int ty_dn, const GsMoeBatch *batches, int nb, int nt, int64_t rs_gu, int n_embd,
                            int n_ff, int64_t rs_dn, const float *x, float *h, float *y, int steps, int warmup,
                            void *s, float *ms_step, float *ms_gateup) {
    Timer t;
    CK(t.init());
    auto step = [&](int i) {
        const GsMoeBatch *b = &batches[i % nb];
        CK(gs_moe_gateup(ty_gu, b, nt, rs_gu, n_embd, n_ff, x, h, 0.0f, s));
        return gs_moe_down(ty_dn, b, nt, rs_dn, n_ff, n_embd, h, y, s);
    };
    int w0 = 0;
    CK(warm(step, warmup, s, &w0));
    CK(gs_event_record(t.a, s));
    for (int i = 0; i < steps; i++) {
        const GsMoeBatch *b = &batches[(w0 + i) % nb];
        CK(gs_moe_gateup(ty_gu, b, nt, rs_gu, n_embd, n_ff, x, h, 0.0f, s));
        CK(gs_moe_down(ty_dn, b, nt, rs_dn, n_ff, n_embd, h, y, s));
    }
    CK(gs_event_record(t.b, s));
    CK(gs_event_sync(t.b));
    CK(gs_event_elapsed_ms(ms_step, t.a, t.b));
    *ms_step /= steps;
    CK(gs_stream_sync(s));
    CK(gs_event_record(t.a, s));
    for (int i = 0; i < steps; i++) {
        const GsMoeBatch *b = &batches[(w0 + steps + i) % nb];
        CK(gs_moe_gateup(ty_gu, b, nt, rs_gu, n_embd, n_ff, x, h, 0.0f, s));
    }
    CK(gs_event_record(t.b, s));
    CK(gs_event_sync(t.b));
    CK(gs_event_elapsed_ms(ms_gateup, t.a, t.b));
    *ms_gateup /= steps;
    return 0;
}

// Decode step through gs_moe_ffn (gate/up then down in one call) over batch (i % nb); mean ms.
BN_EXPORT int bn_moe_ffn(int ty_gu, int ty_dn, const GsMoeBatch *batches, int nb, int nt, int64_t rs_gu, int n_embd,
                         int n_ff, int64_t rs_dn, const float *x, float *h, float *y, int steps, int warmup, void *s,
                         float *ms_step) {
    Timer t;
    CK(t.init());
    auto step = [&](int i) {
        return gs_moe_ffn(ty_gu, ty_dn, &batches[i % nb], nt, rs_gu, n_embd, n_ff, rs_dn, x, h, y, 0.0f, s);
    };
    int w0 = 0;
    CK(warm(step, warmup, s, &w0));
    CK(gs_event_record(t.a, s));
    for (int i = 0; i < steps; i++) CK(step(w0 + i));
    CK(gs_event_record(t.b, s));
    CK(gs_event_sync(t.b));
    CK(gs_event_elapsed_ms(ms_step, t.a, t.b));
    *ms_step /= steps;
    return 0;
}

// Token-sliced routed-expert FFN: step i is one gs_moe_ffn_tokens call over the n_tok batches at
// batches[(i % nr) * n_tok]; mean ms per step.
BN_EXPORT int bn_moe_ffn_tokens(int ty_gu, int ty_dn, const GsMoeBatch *batches, int nr, int n_tok, int64_t rs_gu,
                                int n_embd, int n_ff, int64_t rs_dn, const float *x, float *h, float *y, int steps,
                                int warmup, void *s, float *ms_step) {
    Timer t;
    CK(t.init());
    auto step = [&](int i) {
        return gs_moe_ffn_tokens(ty_gu, ty_dn, &batches[(i % nr) * n_tok], n_tok, rs_gu, n_embd, n_ff, rs_dn, x, h, y,
                                 0.0f, s);
    };
    int w0 = 0;
    CK(warm(step, warmup, s, &w0));
    CK(gs_event_record(t.a, s));
    for (int i = 0; i < steps; i++) CK(step(w0 + i));
    CK(gs_event_record(t.b, s));
    CK(gs_event_sync(t.b));
    CK(gs_event_elapsed_ms(ms_step, t.a, t.b));
    *ms_step /= steps;
    return 0;
}

// GEMV over rotating weight copies Ws[i % nw] (defeats the last-level cache); mean ms per call.
BN_EXPORT int bn_gemv(int ty, const void *const *Ws, int nw, int64_t rs, int K, int rows, const float *x, float *y,
                      int B, int steps, int warmup, void *s, float *ms) {
    Timer t;
    CK(t.init());
    auto step = [&](int i) { return gs_gemv(ty, Ws[i % nw], rs, K, rows, x, K, y, rows, B, 0, s); };
    int w0 = 0;
    CK(warm(step, warmup, s, &w0));
    CK(gs_event_record(t.a, s));
    for (int i = 0; i < steps; i++) CK(step(w0 + i));
    CK(gs_event_record(t.b, s));
    CK(gs_event_sync(t.b));
    CK(gs_event_elapsed_ms(ms, t.a, t.b));
    *ms /= steps;
    return 0;
}

// Grouped MoE FFN (prefill / MTP verify): one gs_moe_grouped call per step over routing
// (i % nr); offs/idx/w hold nr device pointers each. y accumulates across steps (the values are
// not checked here). Mean ms per step.
BN_EXPORT int bn_moe_grouped(int ty_gu, int ty_dn, const GsExpertPtrs *experts, int n_exp, int nr, const int *const *offs,
                             const int *const *idx, const float *const *w, const int *n_pairs, int n_tok, int64_t rs_gu,
                             int n_embd, int n_ff, int64_t rs_dn, const float *x, float *y, void *work,
                             size_t work_bytes, int steps, int warmup, void *s, float *ms) {
    Timer t;
    CK(t.init());
    auto call = [&](int i) {
        const int r = i % nr;
        return gs_moe_grouped(ty_gu, ty_dn, experts, n_exp, offs[r], idx[r], w[r], n_pairs[r], n_tok, rs_gu, n_embd, n_ff,
                              rs_dn, x, y, 0.0f, work, work_bytes, s);
    };
    int w0 = 0;
    CK(warm(call, warmup, s, &w0));
    CK(gs_event_record(t.a, s));
    for (int i = 0; i < steps; i++) CK(call(w0 + i));
    CK(gs_event_record(t.b, s));
    CK(gs_event_sync(t.b));
    CK(gs_event_elapsed_ms(ms, t.a, t.b));
    *ms /= steps;
    return 0;
}

// Device-to-device copy of n bytes, reps times: the known-size reference for HBM byte counters.
BN_EXPORT int bn_copy(void *dst, const void *src, size_t n, int reps, void *s, float *ms) {
    Timer t;
    CK(t.init());
    CK(gs_memcpy_d2d(dst, src, n, s));
    CK(gs_stream_sync(s));
    CK(gs_event_record(t.a, s));
    for (int i = 0; i < reps; i++) CK(gs_memcpy_d2d(dst, src, n, s));
    CK(gs_event_record(t.b, s));
    CK(gs_event_sync(t.b));
    CK(gs_event_elapsed_ms(ms, t.a, t.b));
    *ms /= reps;
    return 0;
}

// ---- plain-read ceiling ------------------------------------------------------------------------
#include <hip/hip_runtime_api.h>
extern "C" const unsigned char bn_blob_start[];

// Read `bytes` (a multiple of 16) starting at bases[i % nb] per call (the rotation keeps the reads
// out of the last-level cache), `steps` calls after `warmup`, for each read shape of
// bench_kernels.hip; *ms: the best shape's mean ms per call.
BN_EXPORT int bn_read(const void *const *bases, int nb, size_t bytes, int steps, int warmup, void *s, float *ms) {
    struct Shape {
        const char *name;
        int threads, loads, grid_per_cu;
        hipFunction_t fn;
    };
    static Shape shapes[] = {{"bn_k_read_512_4", 512, 4, 4, nullptr}, {"bn_k_read_512_4", 512, 4, 8, nullptr},
                             {"bn_k_read_512_8", 512, 8, 1, nullptr}, {"bn_k_read_256_1", 256, 1, 32, nullptr},
                             {"bn_k_read_256_2", 256, 2, 16, nullptr}};
    static hipModule_t mod = nullptr;
    static uint32_t *sink = nullptr;
    if (!mod) {
        CK(hipModuleLoadData(&mod, bn_blob_start));
        for (Shape &sh : shapes) CK(hipModuleGetFunction(&sh.fn, mod, sh.name));
        CK(hipMalloc((void **)&sink, 256));
    }
    int cus = 0;
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    const int64_t n16 = (int64_t)(bytes / 16);
    struct {
        const void *p;
        int64_t n16;
        uint32_t *sink;
    } args;
    size_t sz = sizeof(args);
    float best = 0.0f;
    int done = 0;   // rotation position carried across shapes
    for (const Shape &sh : shapes) {
        const int64_t want = (n16 + (int64_t)sh.threads * sh.loads - 1) / ((int64_t)sh.threads * sh.loads);
        const int64_t cap = (int64_t)sh.grid_per_cu * cus;
        const unsigned grid = (unsigned)(want < 1 ? 1 : (want > cap ? cap : want));
        auto call = [&](int i) {
            args = {bases[i % nb], n16, sink};
            void *cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, &args, HIP_LAUNCH_PARAM_BUFFER_SIZE, &sz, HIP_LAUNCH_PARAM_END};
            return (int)hipModuleLaunchKernel(sh.fn, grid, 1, 1, sh.threads, 1, 1, 0, (hipStream_t)s, nullptr, cfg);
        };
        Timer t;
        CK(t.init());
        int w0 = 0;
        CK(warm([&](int i) { return call(done + i); }, warmup, s, &w0));
        done += w0;
        CK(gs_event_record(t.a, s));
        for (int i = 0; i < steps; i++) CK(call(done + i));
        done += steps;
        CK(gs_event_record(t.b, s));
        CK(gs_event_sync(t.b));
        float m = 0.0f;
        CK(gs_event_elapsed_ms(&m, t.a, t.b));
        m /= steps;
        if (best == 0.0f || m < best) best = m;
    }
    *ms = best;
    return 0;
}

// gs_gemm over rotating weight copies Ws[i % nw]: Y[N][rows] = X[N][K] . W^T; mean ms per call.
// gs_gemm_ex with the caller's workspace (work = NULL: plain gs_gemm)
BN_EXPORT int bn_gemm(int ty, const void *const *Ws, int nw, int64_t rs, int K, int rows, const float *X, float *Y,
                      int N, int steps, int warmup, void *work, size_t work_bytes, void *s, float *ms) {
    Timer t;
    CK(t.init());
    auto step = [&](int i) {
        return gs_gemm_ex(ty, Ws[i % nw], rs, K, rows, X, K, Y, rows, N, 0, 1, 0, 0, 0, work, work_bytes, s);
    };
    int w0 = 0;
    CK(warm(step, warmup, s, &w0));
    CK(gs_event_record(t.a, s));
    for (int i = 0; i < steps; i++) CK(step(w0 + i));
    CK(gs_event_record(t.b, s));
    CK(gs_event_sync(t.b));
    CK(gs_event_elapsed_ms(ms, t.a, t.b));
    *ms /= steps;
    return 0;
}
