// Measurement kernels of the benchmark library (not part of libglmssd_hip.so): a plain HBM read
// at a given byte count, the achievable-bandwidth ceiling the streaming kernels are compared with.
#include <hip/hip_runtime.h>
#include <stdint.h>

// Every thread reads 16-byte words with a grid stride, U loads in flight; the XOR of everything
// read is stored only if it equals a value no input here produces, so the loads stay live. The
// ceiling is the best of several shapes (threads per workgroup, loads in flight, grid size): no
// single one is fastest at every byte count (measured 17.8 MB to 1 GiB).
template <int NT, int U>
__device__ __forceinline__ void read_body(const uint4 *p, int64_t n16, uint32_t *sink) {
    const int64_t stride = (int64_t)gridDim.x * NT;
    int64_t i = (int64_t)blockIdx.x * NT + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = p[i + u * stride];
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const uint4 a = p[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}
#define BN_READ(NT, U)                                                                             \
    extern "C" __global__ void __launch_bounds__(NT) bn_k_read_##NT##_##U(const uint4 *p, int64_t n16, uint32_t *sink) { \
        read_body<NT, U>(p, n16, sink);                                                           \
    }
BN_READ(512, 4)
BN_READ(512, 8)
BN_READ(256, 1)
BN_READ(256, 2)
