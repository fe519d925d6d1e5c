// Read probes for bench.py (not part of the decode library).  Both read a device buffer once and write
// nothing unless the running XOR of the data hits a fixed value, so the measured time is HBM read
// traffic alone:
//  - stream_read_kernel: 16-byte loads, several in flight per lane, over a large buffer: the box's
//    read-only bandwidth, next to the copy rate, the ceiling of read-dominated kernels;
//  - dma_tile_read_kernel: the partial decode kernel's launch shape and DMA pattern without its compute,
//    run on the call's byte count: the floor of moving those bytes that way (start-up and tail included).
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

// The partial decode kernel's memory pattern with no compute: 256-thread blocks of 4 waves, two
// resident per CU; wave w streams its own contiguous run of KB-kilobyte tiles by global->LDS DMA
// (16-byte chunks, nontemporal), one tile in flight, waiting for each before re-arming its stage.
// Its time on a byte count is what moving those bytes costs at that launch shape.
template <int KB>
__global__ __launch_bounds__(kThreads, 2) void dma_tile_read_kernel(const unsigned char* __restrict__ src,
                                                                   int64_t ntiles, uint32_t* __restrict__ sink) {
    __shared__ __align__(16) unsigned char stage[4][KB * 1024];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t waves = (int64_t)gridDim.x * 4;
    const int64_t per = (ntiles + waves - 1) / waves;
    const int64_t t0 = ((int64_t)blockIdx.x * 4 + wave) * per;
    const int64_t n = t0 < ntiles ? (per < ntiles - t0 ? per : ntiles - t0) : 0;
    unsigned char* ring = stage[wave];
    uint32_t acc = 0;
    for (int64_t i = 0; i < n; ++i) {
        const unsigned char* g = src + (t0 + i) * (KB * 1024) + lane * 16;
#pragma unroll
        for (int j = 0; j < KB; ++j)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(g + j * 1024),
                                             (__attribute__((address_space(3))) void*)(ring + j * 1024), 16, 0, 2);
        __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8));  // vmcnt(0): the tile has landed
        __builtin_amdgcn_wave_barrier();
        acc ^= *reinterpret_cast<const uint32_t*>(ring + lane * 16);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): read before the stage is re-armed
        __builtin_amdgcn_wave_barrier();
    }
    if (acc == 0x5EED5EEDu) sink[blockIdx.x] = acc;
}

}  // namespace

// Reads the first ntiles * tile_kb KiB at src (16-byte aligned) with dma_tile_read_kernel: `blocks`
// workgroups, tiles of tile_kb = 4 or 8 KiB; sink holds at least `blocks` words.  Returns 0, 1 for a
// bad argument, 2 for a launch error.
extern "C" int r2o_bench_dma_read(const void* src, int64_t nbytes, uint32_t* sink, int64_t blocks, int tile_kb,
                                  void* stream) {
    if (!src || !sink || nbytes <= 0 || reinterpret_cast<uintptr_t>(src) % 16 || blocks <= 0 || blocks > (1 << 20) ||
        !(tile_kb == 4 || tile_kb == 8))
        return 1;
    const int64_t ntiles = nbytes / (tile_kb * 1024);
    if (ntiles < 1) return 1;
    const dim3 grid((unsigned)blocks), block(kThreads);
    const unsigned char* s = static_cast<const unsigned char*>(src);
    if (tile_kb == 4)
        hipLaunchKernelGGL(dma_tile_read_kernel<4>, grid, block, 0, (hipStream_t)stream, s, ntiles, sink);
    else
        hipLaunchKernelGGL(dma_tile_read_kernel<8>, grid, block, 0, (hipStream_t)stream, s, ntiles, sink);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}

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
