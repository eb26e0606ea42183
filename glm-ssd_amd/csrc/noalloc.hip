// gs_moe_grouped_noalloc: gs_moe_grouped with its workspace in a device array of the library
// instead of a caller buffer, for callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc). Compiled as HIP (not as a code
// object for hipModuleLoadData) so the array is registered with the runtime and its per-device
// address can be looked up.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

#include "../../include/glmssd.h"

// The workspace: one copy per GPU, held until the process ends. Host code must never use the
// name itself as a device address (on the host it only names the symbol): the address comes from
// hipGetSymbolAddress, once per device.
static __device__ __align__(256) unsigned char scratch[GS_MOE_GROUPED_SCRATCH_MAX];

namespace {
std::mutex g_mu;
std::map<int, void *> g_ptr;   // device -> address of that device's scratch

// address of the current device's scratch (looked up on the device's first call)
hipError_t scratch_ptr(void **p) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_ptr.find(dev);
    if (it != g_ptr.end()) {
        *p = it->second;
        return hipSuccess;
    }
    void *q = nullptr;
    if ((e = hipGetSymbolAddress(&q, HIP_SYMBOL(scratch))) != hipSuccess) return e;
    g_ptr[dev] = q;
    *p = q;
    return hipSuccess;
}
}  // namespace

extern "C" __attribute__((visibility("default"))) int gs_moe_grouped_noalloc(
    int ty_gu, int ty_down, const GsExpertPtrs *experts, int n_exp, const int *offs, const int *idx, const float *w,
    int n_pairs, int n_tok, int64_t gu_row_stride, int K, int n_ff, int64_t down_row_stride, const float *x, float *y,
    float lim, void *s) {
    size_t need = 0;
    int rc = gs_moe_grouped_workspace(n_tok, n_pairs, K, n_ff, &need);
    if (rc) return rc;
    if (need > (size_t)GS_MOE_GROUPED_SCRATCH_MAX) return hipErrorInvalidValue;   // beyond the array
    void *work = nullptr;
    if ((rc = scratch_ptr(&work)) != hipSuccess) return rc;
    rc = gs_moe_grouped(ty_gu, ty_down, experts, n_exp, offs, idx, w, n_pairs, n_tok, gu_row_stride, K, n_ff,
                        down_row_stride, x, y, lim, work, (size_t)GS_MOE_GROUPED_SCRATCH_MAX, s);
    if (rc != hipSuccess && rc != hipErrorInvalidValue) {
        // a runtime failure (e.g. after a device reset): look the address up again next time
        int dev = 0;
        if (hipGetDevice(&dev) == hipSuccess) {
            std::lock_guard<std::mutex> lk(g_mu);
            g_ptr.erase(dev);
        }
    }
    return rc;
}
