// HBM read-bandwidth ceiling probe (a measurement kernel with no counterpart
// in the reference).  Every thread streams 16-byte loads of a buffer, `depth`
// of them in flight, over a grid-stride walk of the whole buffer (all waves
// sweep one address window together, the friendliest pattern for the DRAM
// pages), and writes one folded word so no load is dropped.  Plain or
// non-temporal loads; the grid is `waves_per_cu` resident waves per CU.

#include "common.hpp"

namespace slimkv {

template <int DEPTH, bool NT>
__global__ void __launch_bounds__(256) stream_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                          uint32_t* __restrict__ sink) {
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    for (int64_t base = tid; base < n16; base += stride * DEPTH) {
        u32x4 v[DEPTH];
#pragma unroll
        for (int u = 0; u < DEPTH; ++u) {
            const int64_t i = base + u * stride;
            const u32x4* p = src + (i < n16 ? i : 0);
            v[u] = NT ? __builtin_nontemporal_load(p) : *p;
        }
#pragma unroll
        for (int u = 0; u < DEPTH; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    sink[tid] = acc;
}

template <int DEPTH>
hipError_t launch_stream_read(const u32x4* src, int64_t n16, uint32_t* sink, int grid, bool nt, hipStream_t st) {
    if (nt) hipLaunchKernelGGL((stream_read_kernel<DEPTH, true>), dim3(grid), dim3(256), 0, st, src, n16, sink);
    else hipLaunchKernelGGL((stream_read_kernel<DEPTH, false>), dim3(grid), dim3(256), 0, st, src, n16, sink);
    return hipGetLastError();
}

}  // namespace slimkv

using namespace slimkv;

extern "C" int slimkv_probe_stream_read(const void* src, int64_t bytes, uint32_t* sink, int64_t sink_words,
                                        int32_t waves_per_cu, int32_t depth, int32_t non_temporal, void* stream) {
    if (!src || !sink || bytes < 16 || (bytes & 15) || (reinterpret_cast<uintptr_t>(src) & 15))
        return fail(SLIMKV_EINVAL, "probe needs a 16-byte aligned buffer of a multiple of 16 bytes");
    if (waves_per_cu < 4 || waves_per_cu % 4 || waves_per_cu > 64)
        return fail(SLIMKV_EINVAL, "waves_per_cu must be a multiple of 4 in [4, 64]");
    const int grid = device_cu_count() * waves_per_cu / 4;
    if (sink_words < (int64_t)grid * 256) return fail(SLIMKV_EINVAL, "sink too small (grid * 256 words)");
    const int64_t n16 = bytes / 16;
    const u32x4* s = static_cast<const u32x4*>(src);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const bool nt = non_temporal != 0;
    hipError_t e;
    switch (depth) {
        case 1: e = launch_stream_read<1>(s, n16, sink, grid, nt, st); break;
        case 2: e = launch_stream_read<2>(s, n16, sink, grid, nt, st); break;
        case 4: e = launch_stream_read<4>(s, n16, sink, grid, nt, st); break;
        case 8: e = launch_stream_read<8>(s, n16, sink, grid, nt, st); break;
        default: return fail(SLIMKV_EINVAL, "depth must be 1, 2, 4 or 8");
    }
    return check_hip(e, "stream read probe launch");
}
