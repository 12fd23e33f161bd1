// Measurement probes, built as libslimkv_probe.so beside the serving library
// (no counterpart in the reference; nothing on the attention path calls
// them).  Each reports a hardware ceiling the kernels' measured rates are read
// against:
//
// * slimkv_probe_stream_read: the HBM read rate.  Every thread streams
//   16-byte loads of a buffer, `depth` of them in flight, over a grid-stride
//   walk of the whole buffer (all waves sweep one address window together,
//   the friendliest pattern for the DRAM pages), and writes one folded word so
//   no load is dropped.  Plain or non-temporal loads; the grid is
//   `waves_per_cu` resident waves per CU.
// * slimkv_probe_lds_read: the LDS read rate of a CU.  Workgroups of four
//   waves fill 64 KB of LDS, then every lane reads `width` bytes a read
//   (ds_read_b64 / ds_read_b128) at consecutive addresses -- a wave reads a
//   contiguous 512 B or 1 KB, bank-conflict free, as the prefill kernel's
//   operand reads are laid out -- `iters` passes of 16 reads, and folds the
//   words into one per lane.  Bytes read = grid threads x iters x 16 x width.
// * slimkv_probe_gather_read: the HBM read rate of scattered chunks at table
//   offsets (a chunk a page, as a paged decode reads its rows): the chunks'
//   16-byte pieces dealt grid-stride, four in flight a thread, each piece's
//   chunk id looked up first (as a decode looks up its page ids).
// * slimkv_probe_touch: the per-launch floor.  One wave a workgroup, one store
//   a wave; captured back to back in a graph, a launch costs its dispatch and
//   hand-off and nothing else, the floor every kernel of a decode layer pays.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/slimkv_probe.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

thread_local std::string g_probe_error;

int probe_fail(const char* msg) {
    g_probe_error = msg;
    return -1;
}

int probe_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return 0;
    g_probe_error = std::string(what) + ": " + hipGetErrorString(e);
    return -4;
}

int cu_count() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                hipSuccess)
        return 0;
    return cus;
}

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

constexpr int kLdsWords = 16384;                       // 64 KB of 32-bit words

// Every read address stays inside the 64 KB buffer (the index is masked).
template <int WIDTH>
__global__ void __launch_bounds__(256) lds_read_kernel(int iters, uint32_t* __restrict__ sink) {
    __shared__ __attribute__((aligned(16))) uint32_t buf[kLdsWords];
    for (int i = threadIdx.x; i < kLdsWords; i += blockDim.x) buf[i] = i * 2654435761u;
    __syncthreads();
    constexpr int W = WIDTH / 4;                       // words a read
    constexpr int kReads = kLdsWords / W;              // reads a pass of the buffer holds
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t acc = 0;
    int r = (wave * 16 * 64 + lane) % kReads;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int idx = ((r + 64 * u) % kReads) * W;
            if constexpr (WIDTH == 16) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(buf + idx);
                acc ^= v.x ^ v.y ^ v.z ^ v.w;
            } else {
                const u32x2 v = *reinterpret_cast<const u32x2*>(buf + idx);
                acc ^= v.x ^ v.y;
            }
        }
        r = (r + 64 * 16) % kReads;
    }
    sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

__global__ void __launch_bounds__(256) gather_read_kernel(const uint8_t* __restrict__ src, int64_t bytes,
                                                          const int64_t* __restrict__ ids, int64_t pieces,
                                                          int64_t per_chunk, int64_t stride, int64_t offset,
                                                          int64_t chunk, uint32_t* __restrict__ sink) {
    constexpr int DEPTH = 4;
    const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    for (int64_t base = tid; base < pieces; base += step * DEPTH) {
        int64_t at[DEPTH];
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            const int64_t p = base + d * step;
            const int64_t c = (p < pieces ? p : 0) / per_chunk;
            int64_t start = ids[c] * stride + offset;
            if (start < 0 || start + chunk > bytes) start = offset;          // out of the buffer: chunk 0
            at[d] = p < pieces ? start + (p % per_chunk) * 16 : -1;
        }
        u32x4 v[DEPTH];
#pragma unroll
        for (int d = 0; d < DEPTH; ++d)
            v[d] = *reinterpret_cast<const u32x4*>(src + (at[d] >= 0 ? at[d] : offset));
#pragma unroll
        for (int d = 0; d < DEPTH; ++d)
            if (at[d] >= 0) acc ^= v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
    }
    sink[tid] = acc;
}

__global__ void __launch_bounds__(64) touch_kernel(uint32_t* __restrict__ sink) {
    if (threadIdx.x == 0) sink[blockIdx.x] = blockIdx.x;
}

}  // namespace

extern "C" const char* slimkv_probe_last_error(void) { return g_probe_error.c_str(); }

extern "C" int slimkv_probe_gather_read(const void* src, int64_t bytes, const int64_t* ids, int64_t count,
                                        int64_t stride_bytes, int64_t offset_bytes, int32_t chunk_bytes,
                                        uint32_t* sink, int64_t sink_words, int32_t waves_per_cu, void* stream) {
    if (!src || !ids || !sink || (reinterpret_cast<uintptr_t>(src) & 15) || count <= 0)
        return probe_fail("gather probe needs a 16-byte aligned buffer and chunk ids");
    if (chunk_bytes < 16 || chunk_bytes > 16384 || (chunk_bytes & 15) || (stride_bytes & 15) || (offset_bytes & 15) ||
        offset_bytes < 0 || offset_bytes + chunk_bytes > bytes)
        return probe_fail("gather probe: chunk, stride and offset multiples of 16, chunk 16..16384 inside the buffer");
    if (waves_per_cu < 4 || waves_per_cu % 4 || waves_per_cu > 64)
        return probe_fail("waves_per_cu must be a multiple of 4 in [4, 64]");
    const int grid = cu_count() * waves_per_cu / 4;
    if (grid <= 0) return probe_fail("no device");
    if (sink_words < (int64_t)grid * 256) return probe_fail("sink too small (grid * 256 words)");
    const int64_t per_chunk = chunk_bytes / 16;
    hipLaunchKernelGGL(gather_read_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint8_t*>(src), bytes, ids, count * per_chunk, per_chunk, stride_bytes,
                       offset_bytes, (int64_t)chunk_bytes, sink);
    return probe_hip(hipGetLastError(), "gather read probe launch");
}

extern "C" int slimkv_probe_stream_read(const void* src, int64_t bytes, uint32_t* sink, int64_t sink_words,
                                        int32_t waves_per_cu, int32_t depth, int32_t non_temporal, void* stream) {
    if (!src || !sink || bytes < 16 || (bytes & 15) || (reinterpret_cast<uintptr_t>(src) & 15))
        return probe_fail("probe needs a 16-byte aligned buffer of a multiple of 16 bytes");
    if (waves_per_cu < 4 || waves_per_cu % 4 || waves_per_cu > 64)
        return probe_fail("waves_per_cu must be a multiple of 4 in [4, 64]");
    const int grid = cu_count() * waves_per_cu / 4;
    if (grid <= 0) return probe_fail("no device");
    if (sink_words < (int64_t)grid * 256) return probe_fail("sink too small (grid * 256 words)");
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
        default: return probe_fail("depth must be 1, 2, 4 or 8");
    }
    return probe_hip(e, "stream read probe launch");
}

extern "C" int slimkv_probe_lds_read(uint32_t* sink, int64_t sink_words, int32_t workgroups_per_cu, int32_t iters,
                                     int32_t width, void* stream) {
    if (!sink || workgroups_per_cu < 1 || workgroups_per_cu > 2 || iters < 1 || (width != 8 && width != 16))
        return probe_fail("lds probe: 1 or 2 workgroups per CU, iters >= 1, width 8 or 16");
    const int grid = cu_count() * workgroups_per_cu;
    if (grid <= 0) return probe_fail("no device");
    if (sink_words < (int64_t)grid * 256) return probe_fail("sink too small (grid * 256 words)");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (width == 16) hipLaunchKernelGGL(lds_read_kernel<16>, dim3(grid), dim3(256), 0, st, iters, sink);
    else hipLaunchKernelGGL(lds_read_kernel<8>, dim3(grid), dim3(256), 0, st, iters, sink);
    return probe_hip(hipGetLastError(), "lds read probe launch");
}

extern "C" int slimkv_probe_touch(uint32_t* sink, int64_t sink_words, int32_t workgroups, void* stream) {
    if (!sink || workgroups < 1 || workgroups > 65536 || sink_words < workgroups)
        return probe_fail("touch probe: 1..65536 workgroups, a sink word each");
    hipLaunchKernelGGL(touch_kernel, dim3(workgroups), dim3(64), 0, static_cast<hipStream_t>(stream), sink);
    return probe_hip(hipGetLastError(), "touch probe launch");
}
