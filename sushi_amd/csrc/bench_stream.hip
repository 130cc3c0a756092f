// Measurement kernels for bench.py (not part of the hot path's ABI): a streaming read, the practical HBM read
// ceiling that the decode GEMV's traffic is compared with.
//
// stream_read_kernel reads `n16` 16-byte words, four loads in flight per thread before any use, and folds them into
// one XOR per thread.  The fold's value is only stored when it equals a constant the data never produces, so the
// reads cannot be dropped and the kernel writes (almost) nothing: its traffic is the read alone.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int SR_THREADS = 256;
constexpr uint32_t SR_NEVER = 0x5EEDF00Du;

__global__ __launch_bounds__(SR_THREADS) void stream_read_kernel(const uint4 *__restrict__ p, size_t n16,
                                                                 uint32_t *__restrict__ sink) {
    const size_t stride = (size_t)gridDim.x * SR_THREADS;
    size_t i = (size_t)blockIdx.x * SR_THREADS + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n16; i += stride) {
        const uint4 a = p[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == SR_NEVER) sink[0] = acc;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16, 16-byte aligned) of device memory at p with `blocks` workgroups of 256 threads
// on `stream`.  `sink` is a device word the kernel writes only in a case zero-filled data rules out.
// Returns 0, or the HIP error code of the launch.
int32_t sb_stream_read(const void *p, size_t bytes, int32_t blocks, uint32_t *sink, hipStream_t stream) {
    if (!p || bytes % 16 || blocks <= 0) return (int32_t)hipErrorInvalidValue;
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(SR_THREADS), 0, stream,
                       static_cast<const uint4 *>(p), bytes / 16, sink);
    return (int32_t)hipGetLastError();
}

}  // extern "C"
