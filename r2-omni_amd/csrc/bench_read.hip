// Streaming-read probe for bench.py (not part of the decode library): reads a device buffer once with
// 16-byte loads, several in flight per lane, and writes nothing unless the running XOR of the data
// hits a fixed value, so the measured time is HBM read traffic alone.  It gives the box's read-only
// bandwidth, next to the copy rate, as the practical ceiling of read-dominated kernels.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kUnroll = 4;

template <bool NT>
__device__ __forceinline__ u4 load16(const u4* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}

template <bool NT>
__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u4* __restrict__ src, int64_t n16,
                                                               uint32_t* __restrict__ sink) {
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
        u4 v[kUnroll];
#pragma unroll
        for (int k = 0; k < kUnroll; ++k) v[k] = load16<NT>(src + i + k * stride);
#pragma unroll
        for (int k = 0; k < kUnroll; ++k) acc ^= v[k][0] ^ v[k][1] ^ v[k][2] ^ v[k][3];
    }
    for (; i < n16; i += stride) {
        const u4 v = load16<NT>(src + i);
        acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
    if (acc == 0x5EED5EEDu) sink[blockIdx.x] = acc;  // keeps the loads; practically never stores
}

}  // namespace

// Reads nbytes (a multiple of 16, 16-byte aligned) at src with `blocks` workgroups of 256 threads;
// sink holds at least `blocks` words.  Returns 0, 1 for a bad argument, 2 for a launch error.
extern "C" int r2o_bench_stream_read(const void* src, int64_t nbytes, uint32_t* sink, int64_t blocks,
                                     int nontemporal, void* stream) {
    if (!src || !sink || nbytes <= 0 || nbytes % 16 || reinterpret_cast<uintptr_t>(src) % 16 || blocks <= 0 ||
        blocks > (1 << 20))
        return 1;
    const dim3 grid((unsigned)blocks), block(kThreads);
    if (nontemporal)
        hipLaunchKernelGGL(stream_read_kernel<true>, grid, block, 0, (hipStream_t)stream,
                           static_cast<const u4*>(src), nbytes / 16, sink);
    else
        hipLaunchKernelGGL(stream_read_kernel<false>, grid, block, 0, (hipStream_t)stream,
                           static_cast<const u4*>(src), nbytes / 16, sink);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}
