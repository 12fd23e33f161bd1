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

// Rows of a decode step (slimkv_paged_step_rows): 16 lanes a (request, row,
// KV head), 8 features a lane; the rotate-half partner (d +- 64) from lane
// l ^ 8 of the same 16-lane row by a DPP rotation.  A row whose page entry is
// bad still loads (a valid fallback row) so the rotation sees whole rows, and
// stores nothing.
__device__ __forceinline__ uint32_t step_ror8(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xf, 0xf, true);
}

__global__ void __launch_bounds__(256)
paged_step_rows_kernel(slimkv_paged_step_rows_args a) {
    constexpr int D = 128;
    const int64_t b = blockIdx.y;
    const int lane16 = threadIdx.x & 15;
    const int dd = lane16 * 8;
    const int64_t item = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;
    const int64_t H = a.kv_heads;
    const int64_t rc = a.raw_count[b];
    const int64_t len = a.sink + rc + 1;
    const int64_t r_item = item / H, h = item % H;
    // a raw set longer than the dense buffer's rows would lose its new token's
    // row (and the flush write): report it as a slot outside the buffer
    if (item == 0 && lane16 == 0 && len > a.rows && a.status) *a.status = SLIMKV_STATUS_BAD_SLOT;
    // a 16-lane row group past the request's raw set has nothing to do; the
    // rotation's DPP reads only lanes of its own group, so it may leave
    if (r_item >= len || r_item >= a.rows) return;
    bool live = true;
    const int64_t r = r_item;
    const uint16_t* ksrc;
    const uint16_t* vsrc;
    uint16_t* page_row = nullptr;            // raw page row of the new token (flush), or null
    uint16_t* sink_row = nullptr;            // root page of a sink row (flush)
    const uint16_t* fallback = static_cast<const uint16_t*>(a.new_k) + b * a.nk_sb + h * D;
    if (r < a.sink) {
        const int64_t page = table_page(a.beacon_table[b * a.bt_sb], a.num_pages);
        if (page < 0) {
            if (live && lane16 == 0) report_bad_page(a.status);
            live = false;
            ksrc = vsrc = fallback;
        } else {
            uint16_t* root = static_cast<uint16_t*>(a.beacon_pages) + page * a.page_stride;
            ksrc = root + h * D;
            vsrc = root + H * D + h * D;
            sink_row = root;
        }
    } else if (r < a.sink + rc) {
        const int64_t pos = a.window_start[b] + (r - a.sink);
        const int64_t col = pos >= 0 ? pos / a.block_size : -1;
        const int64_t blk = col >= 0 && col < a.rt_cols ? table_page(a.raw_table[b * a.rt_sb + col], a.num_blocks) : -1;
        if (blk < 0) {
            if (live && lane16 == 0) report_bad_page(a.status);
            live = false;
            ksrc = vsrc = fallback;
        } else {
            const uint16_t* row = static_cast<const uint16_t*>(a.raw_pages) + blk * a.p_sblk + (pos % a.block_size) * a.p_stok;
            ksrc = row + h * a.p_sh;
            vsrc = row + a.p_skind + h * a.p_sh;
        }
    } else {
        ksrc = fallback;
        vsrc = static_cast<const uint16_t*>(a.new_v) + b * a.nv_sb + h * D;
        const int64_t pos = a.window_start[b] + rc;
        if (a.flush && pos < a.raw_write_end[b]) {
            const int64_t col = pos >= 0 ? pos / a.block_size : -1;
            const int64_t blk = col >= 0 && col < a.rt_cols ? table_page(a.raw_table[b * a.rt_sb + col], a.num_blocks)
                                                             : -1;
            if (blk < 0) {
                if (live && lane16 == 0) report_bad_page(a.status);
            } else {
                page_row = static_cast<uint16_t*>(a.raw_pages) + blk * a.p_sblk + (pos % a.block_size) * a.p_stok;
            }
        }
    }
    const u32x4 xk = *reinterpret_cast<const u32x4*>(ksrc + dd);
    const u32x4 xv = *reinterpret_cast<const u32x4*>(vsrc + dd);
    const int64_t prow = clamp_i64(a.positions[b * a.pos_sb + r], 0, a.rope_rows - 1) * D + dd;
    const float4 c0 = *reinterpret_cast<const float4*>(a.cos + prow), c1 = *reinterpret_cast<const float4*>(a.cos + prow + 4);
    const float4 s0 = *reinterpret_cast<const float4*>(a.sin + prow), s1 = *reinterpret_cast<const float4*>(a.sin + prow + 4);
    const float c8[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    const float s8[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const uint32_t xs[4] = {xk.x, xk.y, xk.z, xk.w};
    const uint32_t pr[4] = {step_ror8(xk.x), step_ror8(xk.y), step_ror8(xk.z), step_ror8(xk.w)};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float sum[2];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            const float v = hb ? hi_bf16(xs[e]) : lo_bf16(xs[e]);
            float pt = hb ? hi_bf16(pr[e]) : lo_bf16(pr[e]);
            if (lane16 < 8) pt = -pt;
            sum[hb] = round_bf16_hw(v * round_bf16_hw(c8[2 * e + hb])) + round_bf16_hw(pt * round_bf16_hw(s8[2 * e + hb]));
        }
        o[e] = pack_bf16(sum[0], sum[1]);
    }
    if (!live) return;
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(a.out_k) + b * a.ok_sb + r * a.ok_sn + h * D + dd) =
        u32x4{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(a.out_v) + b * a.ov_sb + r * a.ov_sn + h * D + dd) = xv;
    if (!a.flush) return;
    if (page_row) {                              // the new token into its raw page, K before RoPE
        *reinterpret_cast<u32x4*>(page_row + h * a.p_sh + dd) = xk;
        *reinterpret_cast<u32x4*>(page_row + a.p_skind + h * a.p_sh + dd) = xv;
    }
    if (sink_row && a.sink_update[b]) {          // the new token becomes the sink (read above)
        const uint16_t* nk = static_cast<const uint16_t*>(a.new_k) + b * a.nk_sb + h * D + dd;
        const uint16_t* nv = static_cast<const uint16_t*>(a.new_v) + b * a.nv_sb + h * D + dd;
        *reinterpret_cast<u32x4*>(sink_row + h * D + dd) = *reinterpret_cast<const u32x4*>(nk);
        *reinterpret_cast<u32x4*>(sink_row + H * D + h * D + dd) = *reinterpret_cast<const u32x4*>(nv);
    }
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

extern "C" int slimkv_paged_step_rows(const slimkv_paged_step_rows_args* a, void* stream) {
    if (!a || !a->raw_pages || !a->raw_table || !a->new_k || !a->new_v || !a->window_start || !a->raw_count ||
        !a->positions || !a->cos || !a->sin || !a->out_k || !a->out_v || (a->sink && (!a->beacon_pages || !a->beacon_table)) ||
        (a->flush && (!a->raw_write_end || (a->sink && !a->sink_update))))
        return fail(SLIMKV_EINVAL, "null pointer");
    if (a->head_dim != 128) return fail(SLIMKV_EUNSUP, "paged step rows support head_dim 128");
    if (a->batch < 0 || a->batch > 65535 || a->rows <= 0 || a->kv_heads <= 0 || a->sink < 0 || a->sink > 1 ||
        a->block_size <= 0 || a->num_blocks <= 0 || a->rt_cols <= 0 || a->rt_sb < a->rt_cols || a->rope_rows <= 0 ||
        (a->sink && (a->num_pages <= 0 || a->page_stride < 2 * a->kv_heads * 128)) ||
        a->rows * a->kv_heads > ((int64_t)1 << 26))
        return fail(SLIMKV_EINVAL, "invalid paged step rows sizes");
    if (!all_multiple_of_8({a->p_sblk, a->p_stok, a->p_skind, a->p_sh, a->page_stride, a->nk_sb, a->nv_sb, a->ok_sb,
                            a->ok_sn, a->ov_sb, a->ov_sn}) ||
        !aligned16(a->raw_pages) || !aligned16(a->new_k) || !aligned16(a->new_v) || !aligned16(a->out_k) ||
        !aligned16(a->out_v) || !aligned16(a->cos) || !aligned16(a->sin) || (a->sink && !aligned16(a->beacon_pages)))
        return fail(SLIMKV_EINVAL, "paged step rows need 16-byte aligned rows (strides multiples of 8 elements)");
    if (a->batch == 0) return SLIMKV_OK;
    const int64_t threads = a->rows * a->kv_heads * 16;
    hipLaunchKernelGGL(paged_step_rows_kernel, dim3((unsigned)((threads + 255) / 256), (unsigned)a->batch), dim3(256),
                       0, static_cast<hipStream_t>(stream), *a);
    return check_hip(hipGetLastError(), "paged step rows launch");
}
