// Measurement kernels of the benchmark library (not part of libglmssd_hip.so): a plain HBM read
// at a given byte count, the achievable-bandwidth ceiling the streaming kernels are compared with.
#include <hip/hip_runtime.h>
#include <stdint.h>

// Every thread reads 16-byte words with a grid stride, 4 in flight; the XOR of everything read
// is stored only if it equals a value no input here produces, so the loads stay live.
extern "C" __global__ void __launch_bounds__(512) bn_k_read(const uint4 *p, int64_t n16, uint32_t *sink) {
    const int64_t stride = (int64_t)gridDim.x * 512;
    int64_t i = (int64_t)blockIdx.x * 512 + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n16; i += stride) {
        const uint4 a = p[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}
