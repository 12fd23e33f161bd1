// Paged KV-cache I/O in the reference page formats; every copy is bit-exact.
//
// Beacon pages (slimkv/vllm_plugin/paged_cache.py:11-99): a physical page is
// `page_stride` bf16 elements; logical beacon i of a request lives in page
// table[i / slots] at columns sink_elements + (i % slots) * width + [0, width),
// K latent (key_rank) first, then V latent (value_rank).
// Raw pages (paged_cache.py:102-127): [blocks, block_size, 2, Hkv, D]; token t
// lives in block table[t / block_size] at row t % block_size.  Table entries
// follow torch's indexing rules; an index error moves nothing and is reported.
// An optional per-request `starts` offsets each request's first row (a batch
// of requests at different positions, such as one decode step's appends).
//
// These copies are HBM-bound byte moves: one thread moves one 16-byte piece
// (VEC = 8 bf16) whenever every row start and width allows it, else one
// element.  blockIdx.y is the request, so a request's rows are contiguous in
// the grid and neighbouring threads touch neighbouring bytes of a row; a raw
// token is one workgroup (its block looked up once, 32-bit index math).

#include "common.hpp"

#include <algorithm>

namespace slimkv {

template <int VEC>
__device__ __forceinline__ void copy_piece(uint16_t* dst, const uint16_t* src) {
    if constexpr (VEC == 8) *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src);
    else *dst = *src;
}

template <int VEC>
__global__ void __launch_bounds__(256)
beacon_pages_kernel(slimkv_beacon_pages_args a) {
    const int64_t b = blockIdx.y;
    const int64_t width = a.key_rank + a.value_rank;
    const int64_t per_row = width / VEC;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= a.count * per_row) return;
    const int64_t r = gid / per_row;
    const int64_t c = (gid % per_row) * VEC;           // column inside [K | V]
    const int64_t logical = a.start + (a.starts ? a.starts[b] : 0) + r;
    if (a.lengths && logical >= a.lengths[b]) return;
    const int64_t col = logical >= 0 ? logical / a.slots : -1;     // a negative position is an index error
    const int64_t page = col >= 0 && col < a.t_cols ? table_page(a.table[b * a.t_sb + col], a.num_pages) : -1;
    if (page < 0) {
        report_bad_page(a.status);
        return;
    }
    uint16_t* pg = static_cast<uint16_t*>(a.pages) + page * a.page_stride + a.sink_elements +
                   (logical % a.slots) * width + c;
    const bool is_k = c < a.key_rank;
    uint16_t* dn = is_k ? static_cast<uint16_t*>(a.dense_k) + b * a.dk_sb + r * a.dk_sn + c
                        : static_cast<uint16_t*>(a.dense_v) + b * a.dv_sb + r * a.dv_sn + (c - a.key_rank);
    if (a.to_pages) copy_piece<VEC>(pg, dn);
    else copy_piece<VEC>(dn, pg);
}

// One workgroup per (token, request): the token's block is looked up once and
// the 2 * Hkv * D elements of its K and V rows are moved with 32-bit index math.
template <int VEC>
__global__ void __launch_bounds__(256)
raw_pages_kernel(slimkv_raw_pages_args a) {
    const int64_t b = blockIdx.y;
    const int64_t r = blockIdx.x;
    const int64_t t = a.start + (a.starts ? a.starts[b] : 0) + r;
    if (a.lengths && t >= a.lengths[b]) return;
    const int64_t col = t >= 0 ? t / a.block_size : -1;             // a negative position is an index error
    const int64_t block = col >= 0 && col < a.t_cols ? table_page(a.table[b * a.t_sb + col], a.num_blocks) : -1;
    if (block < 0) {
        if (threadIdx.x == 0) report_bad_page(a.status);
        return;
    }
    const int dv = (int)a.head_dim / VEC, hd = (int)a.kv_heads * dv;
    uint16_t* pg = static_cast<uint16_t*>(a.pages) + block * a.p_sblk + (t % a.block_size) * a.p_stok;
    for (int i = threadIdx.x; i < 2 * hd; i += blockDim.x) {
        const int kind = i >= hd;
        const int rem = i - kind * hd;
        const int h = rem / dv;
        const int d = (rem - h * dv) * VEC;
        uint16_t* pe = pg + kind * a.p_skind + h * a.p_sh + d;
        uint16_t* dn = kind ? static_cast<uint16_t*>(a.dense_v) + b * a.dv_sb + h * a.dv_sh + r * a.dv_sn + d
                            : static_cast<uint16_t*>(a.dense_k) + b * a.dk_sb + h * a.dk_sh + r * a.dk_sn + d;
        if (a.to_pages) copy_piece<VEC>(pe, dn);
        else copy_piece<VEC>(dn, pe);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

bool all_multiple_of_8(std::initializer_list<int64_t> xs) {
    for (int64_t x : xs)
        if (x % 8) return false;
    return true;
}

dim3 io_grid(int64_t items, int64_t batch) {
    return dim3((unsigned)((items + 255) / 256), (unsigned)batch);
}

}  // namespace slimkv

using namespace slimkv;

extern "C" int slimkv_beacon_pages(const slimkv_beacon_pages_args* a, void* stream) {
    if (!a || !a->pages || !a->table || (a->count > 0 && (!a->dense_k || !a->dense_v)))
        return fail(SLIMKV_EINVAL, "null pointer");
    if (a->slots <= 0 || a->key_rank <= 0 || a->value_rank <= 0 || a->sink_elements < 0 || a->start < 0 ||
        a->count < 0 || a->batch < 0 || a->num_pages < 0 || a->batch > 65535 || a->t_cols <= 0 || a->t_sb < a->t_cols ||
        a->page_stride < a->sink_elements + a->slots * (a->key_rank + a->value_rank))
        return fail(SLIMKV_EINVAL, "invalid beacon page layout");
    if (a->count == 0 || a->batch == 0) return SLIMKV_OK;
    const int64_t width = a->key_rank + a->value_rank;
    const bool vec = all_multiple_of_8({a->key_rank, a->value_rank, a->page_stride, a->sink_elements, a->dk_sb,
                                        a->dk_sn, a->dv_sb, a->dv_sn}) &&
                     aligned16(a->pages) && aligned16(a->dense_k) && aligned16(a->dense_v);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (vec) hipLaunchKernelGGL(beacon_pages_kernel<8>, io_grid(a->count * width / 8, a->batch), dim3(256), 0, st, *a);
    else hipLaunchKernelGGL(beacon_pages_kernel<1>, io_grid(a->count * width, a->batch), dim3(256), 0, st, *a);
    return check_hip(hipGetLastError(), "beacon page kernel launch");
}

extern "C" int slimkv_raw_pages(const slimkv_raw_pages_args* a, void* stream) {
    if (!a || !a->pages || !a->table || (a->count > 0 && (!a->dense_k || !a->dense_v)))
        return fail(SLIMKV_EINVAL, "null pointer");
    if (a->block_size <= 0 || a->kv_heads <= 0 || a->head_dim <= 0 || a->start < 0 || a->count < 0 ||
        a->batch < 0 || a->batch > 65535 || a->num_blocks < 0 || a->t_cols <= 0 || a->t_sb < a->t_cols)
        return fail(SLIMKV_EINVAL, "invalid raw page layout");
    if (a->count == 0 || a->batch == 0) return SLIMKV_OK;
    if (a->count > ((int64_t)1 << 31) - 1 || a->kv_heads * a->head_dim > (1 << 20))
        return fail(SLIMKV_EINVAL, "raw copy too large");
    const bool vec = all_multiple_of_8({a->head_dim, a->p_sblk, a->p_stok, a->p_skind, a->p_sh, a->dk_sb, a->dk_sh,
                                        a->dk_sn, a->dv_sb, a->dv_sh, a->dv_sn}) &&
                     aligned16(a->pages) && aligned16(a->dense_k) && aligned16(a->dense_v);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)a->count, (unsigned)a->batch);
    if (vec) hipLaunchKernelGGL(raw_pages_kernel<8>, grid, dim3(256), 0, st, *a);
    else hipLaunchKernelGGL(raw_pages_kernel<1>, grid, dim3(256), 0, st, *a);
    return check_hip(hipGetLastError(), "raw page kernel launch");
}
