// Beacon down-projection on the 16x16x32 bf16 MFMA: the latents of the
// selected (beacon) rows of a window,
//
//   out[b, i, :] = bf16(x[b, rows[i], :] @ W^T),   W [N, K] (nn.Linear weight)
//
// as in _project_beacon_key/_project_beacon_value followed by the role
// selection of _incremental_cache (slimkv/llama3/modeling_llama.py:383-390,
// 444-451, 1347-1367); only the selected rows are projected.  A block-diagonal
// W (per-KV-head bases, `blocks` diagonal blocks) contracts each output block
// over its own K block only.
//
// One wavefront computes C^T[n, m] = W[n, :] . x[m, :] for 16 outputs x 64
// rows: A = W rows and B = x rows are both contiguous along the contraction,
// and a lane ends with 4 consecutive outputs of one row (8-byte stores).  Long
// contractions are split over workgroups into fp32 partials summed in a fixed
// order by a second kernel, so results do not depend on scheduling.

#include "common.hpp"

#include <algorithm>

namespace slimkv {

namespace {

struct DownParams {
    const uint16_t* x; int64_t x_sb, x_sl;
    const int64_t* rows; int64_t length;
    const uint16_t* w;
    uint16_t* out; int64_t o_sb, o_sn;
    float* part;                 // [splits, M, N] when splits > 1
    int B, n, N, K, blocks, splits, kchunk;
    // Page destination (table != null): row i of request b is beacon start + i,
    // written at out + page * page_stride + ((start + i) % slots) * slot_width
    // with page = table[b * t_sb + (start + i) / slots] under torch's indexing
    // rules; a row whose table column lies past t_cols or whose entry lies
    // outside [-num_pages, num_pages) is not written and is reported in status.
    const int64_t* table; int64_t t_sb, t_cols, slots, page_stride, num_pages, slot_width, start;
    int32_t* status;
};

__device__ __forceinline__ uint16_t* dst_row(const DownParams& p, int b, int i) {
    if (!p.table) return p.out + (int64_t)b * p.o_sb + (int64_t)i * p.o_sn;
    const int64_t beacon = p.start + i;
    const int64_t idx = beacon / p.slots;
    const int64_t page = idx < p.t_cols ? table_page(p.table[(int64_t)b * p.t_sb + idx], p.num_pages) : -1;
    if (page < 0) {
        report_bad_page(p.status);
        return nullptr;
    }
    return p.out + page * p.page_stride + (beacon % p.slots) * p.slot_width;
}

constexpr int kMFrags = 4;       // 64 rows per wave

__device__ __forceinline__ u32x4 zero_if_not(bool ok, u32x4 v) {
    return u32x4{ok ? v.x : 0u, ok ? v.y : 0u, ok ? v.z : 0u, ok ? v.w : 0u};
}

__device__ __forceinline__ void down_body(const DownParams& p, int block) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int ngroups = (p.N + 63) / 64;
    const int M = p.B * p.n;
    const int mtiles = (M + 16 * kMFrags - 1) / (16 * kMFrags);
    const int s = block % p.splits;
    const int rest = block / p.splits;
    const int ng = rest % ngroups;
    const int mt = rest / ngroups;
    if (mt >= mtiles) return;
    const int n0 = ng * 64 + wave * 16;
    if (n0 >= p.N) return;

    const int kb = p.K / p.blocks;
    const int head = n0 / (p.N / p.blocks);
    int k_lo = p.blocks > 1 ? head * kb : 0;
    int k_hi = p.blocks > 1 ? k_lo + kb : p.K;
    k_lo += s * p.kchunk;
    k_hi = min(k_hi, k_lo + p.kchunk);

    const uint16_t* wrow = p.w + (int64_t)(n0 + col) * p.K + 8 * grp;
    const uint16_t* xrow[kMFrags];
    bool mok[kMFrags], rok[kMFrags];
#pragma unroll
    for (int f = 0; f < kMFrags; ++f) {
        const int m = mt * 16 * kMFrags + 16 * f + col;
        mok[f] = m < M;
        const int mm = mok[f] ? m : 0;
        const int b = mm / p.n, i = mm % p.n;
        const int64_t r = p.rows ? p.rows[i] : i;
        rok[f] = r >= 0 && r < p.length;            // a row outside x projects to zeros
        xrow[f] = p.x + (int64_t)b * p.x_sb + (rok[f] ? r : 0) * p.x_sl + 8 * grp;
    }
    v4f acc[kMFrags];
#pragma unroll
    for (int f = 0; f < kMFrags; ++f) acc[f] = v4f{0.f, 0.f, 0.f, 0.f};
    // Four 32-wide steps per pass: every operand load of the pass is issued
    // before its first MFMA (steps past k_hi read column k_lo and are zeroed),
    // so a pass costs one memory round trip; the accumulation order over k is
    // unchanged.
    for (int k0 = k_lo; k0 < k_hi; k0 += 128) {
        u32x4 a[4], xv[4][kMFrags];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const bool kin = k0 + 32 * u < k_hi;
            const int kk = kin ? k0 + 32 * u : k_lo;
            a[u] = zero_if_not(kin, *reinterpret_cast<const u32x4*>(wrow + kk));
#pragma unroll
            for (int f = 0; f < kMFrags; ++f) xv[u][f] = zero_if_not(kin, *reinterpret_cast<const u32x4*>(xrow[f] + kk));
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int f = 0; f < kMFrags; ++f) acc[f] = mfma32(a[u], xv[u][f], acc[f]);
    }
    const int M_ = M;
#pragma unroll
    for (int f = 0; f < kMFrags; ++f) {
        if (!mok[f]) continue;
        if (!rok[f]) acc[f] = v4f{0.f, 0.f, 0.f, 0.f};
        const int m = mt * 16 * kMFrags + 16 * f + col;
        const int nn = n0 + 4 * grp;
        if (p.splits == 1) {
            const int b = m / p.n, i = m % p.n;
            u32x2 w;
            w.x = pack_bf16(acc[f][0], acc[f][1]);
            w.y = pack_bf16(acc[f][2], acc[f][3]);
            uint16_t* dst = dst_row(p, b, i);
            if (dst) *reinterpret_cast<u32x2*>(dst + nn) = w;
        } else {
            *reinterpret_cast<v4f*>(p.part + ((int64_t)s * M_ + m) * p.N + nn) = acc[f];
        }
    }
}

__global__ void __launch_bounds__(256) down_kernel(DownParams p) { down_body(p, blockIdx.x); }

// Two down-projections without split partials in one launch (the K and V
// latents of a window's beacon rows): the first `blocks0` workgroups run the
// first, the rest the second, each as the single kernel's workgroup.
__global__ void __launch_bounds__(256) down_pair_kernel(DownParams p0, DownParams p1, int blocks0) {
    if ((int)blockIdx.x < blocks0) down_body(p0, blockIdx.x);
    else down_body(p1, blockIdx.x - blocks0);
}

// Sum the split partials in split order and round once to bf16.
__global__ void __launch_bounds__(256) down_reduce_kernel(DownParams p) {
    const int64_t M = (int64_t)p.B * p.n;
    const int64_t quads = M * (p.N / 4);
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= quads) return;
    const int64_t m = id / (p.N / 4);
    const int nn = (int)(id % (p.N / 4)) * 4;
    v4f sum = *reinterpret_cast<const v4f*>(p.part + m * p.N + nn);
    for (int s = 1; s < p.splits; ++s) sum += *reinterpret_cast<const v4f*>(p.part + ((int64_t)s * M + m) * p.N + nn);
    const int b = (int)(m / p.n), i = (int)(m % p.n);
    u32x2 w;
    w.x = pack_bf16(sum[0], sum[1]);
    w.y = pack_bf16(sum[2], sum[3]);
    uint16_t* dst = dst_row(p, b, i);
    if (dst) *reinterpret_cast<u32x2*>(dst + nn) = w;
}

bool al16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

struct DownPlan {
    int splits, kchunk;
    size_t bytes;
};

int plan_down(const slimkv_down_project_args* a, DownPlan* plan) {
    if (!a || !a->x || !a->weight || !a->out) return fail(SLIMKV_EINVAL, "null pointer");
    if (a->batch < 0 || a->row_count < 0 || a->length < 0 || (!a->rows && a->row_count > a->length) ||
        a->in_features <= 0 || a->out_features <= 0 || a->blocks <= 0 || a->batch > (1 << 20) ||
        a->row_count > (1 << 24) || a->batch * a->row_count > (1 << 30))
        return fail(SLIMKV_EINVAL, "invalid down-projection sizes");
    if (a->out_features % (16 * a->blocks) || a->in_features % (32 * a->blocks))
        return fail(SLIMKV_EUNSUP, "down-projection needs out_features/blocks % 16 == 0 and in_features/blocks % 32 == 0");
    if (a->x_sb % 8 || a->x_sl % 8 || a->o_sb % 4 || a->o_sn % 4 || !al16(a->x) || !al16(a->weight) ||
        (reinterpret_cast<uintptr_t>(a->out) & 7))
        return fail(SLIMKV_EINVAL, "x rows must be 16-byte aligned and out rows 8-byte aligned");
    const int64_t M = a->batch * a->row_count;
    const int64_t kb = a->in_features / a->blocks;
    const int64_t base = (a->out_features + 63) / 64 * ((M + 63) / 64);
    int splits = 1;
    if (base > 0 && base < 512) splits = (int)std::min<int64_t>((512 + base - 1) / base, kb / 256);
    splits = std::max(splits, 1);
    int64_t kchunk = (kb + splits - 1) / splits;
    kchunk = (kchunk + 31) / 32 * 32;
    splits = (int)((kb + kchunk - 1) / kchunk);
    plan->splits = splits;
    plan->kchunk = (int)kchunk;
    plan->bytes = splits > 1 ? (size_t)splits * M * a->out_features * sizeof(float) : 0;
    return SLIMKV_OK;
}

}  // namespace

}  // namespace slimkv

using namespace slimkv;

extern "C" size_t slimkv_down_project_workspace(const slimkv_down_project_args* a) {
    DownPlan plan{};
    if (plan_down(a, &plan) != SLIMKV_OK) return 0;
    return std::max<size_t>(plan.bytes, 1);
}

namespace {

DownParams down_params(const slimkv_down_project_args* a, const slimkv_page_rows* pg, const DownPlan& plan,
                       void* workspace) {
    DownParams p{};
    p.x = static_cast<const uint16_t*>(a->x); p.x_sb = a->x_sb; p.x_sl = a->x_sl;
    p.rows = a->rows; p.length = a->length;
    p.w = static_cast<const uint16_t*>(a->weight);
    p.out = static_cast<uint16_t*>(a->out); p.o_sb = a->o_sb; p.o_sn = a->o_sn;
    p.part = static_cast<float*>(workspace);
    p.B = (int)a->batch; p.n = (int)a->row_count; p.N = (int)a->out_features; p.K = (int)a->in_features;
    p.blocks = (int)a->blocks; p.splits = plan.splits; p.kchunk = plan.kchunk;
    if (pg) {
        p.out = static_cast<uint16_t*>(pg->pages) + pg->sink_elements + pg->column;
        p.table = pg->table; p.t_sb = pg->t_sb; p.t_cols = pg->t_cols; p.slots = pg->slots;
        p.page_stride = pg->page_stride; p.num_pages = pg->num_pages; p.slot_width = pg->slot_width;
        p.start = pg->start;
        p.status = pg->status;
    }
    return p;
}

int64_t down_grid(const DownParams& p) {
    const int64_t M = (int64_t)p.B * p.n;
    return (p.N + 63) / 64 * ((M + 63) / 64) * p.splits;
}

int down_run(const slimkv_down_project_args* a, const slimkv_page_rows* pg, void* workspace, size_t workspace_bytes,
             void* stream) {
    DownPlan plan{};
    int rc = plan_down(a, &plan);
    if (rc != SLIMKV_OK) return rc;
    if (plan.bytes && (!workspace || workspace_bytes < plan.bytes))
        return fail(SLIMKV_EWORKSPACE, "workspace too small");
    const int64_t M = a->batch * a->row_count;
    if (M == 0) return SLIMKV_OK;
    const DownParams p = down_params(a, pg, plan, workspace);
    const int64_t grid = down_grid(p);
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(down_kernel, dim3((unsigned)grid), dim3(256), 0, st, p);
    rc = check_hip(hipGetLastError(), "down-projection launch");
    if (rc != SLIMKV_OK || p.splits == 1) return rc;
    const int64_t quads = M * (p.N / 4);
    hipLaunchKernelGGL(down_reduce_kernel, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, st, p);
    return check_hip(hipGetLastError(), "down-projection reduce launch");
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace

extern "C" int slimkv_down_project(const slimkv_down_project_args* a, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    return down_run(a, nullptr, workspace, workspace_bytes, stream);
}

extern "C" size_t slimkv_down_project_pair_workspace(const slimkv_down_project_args* a,
                                                     const slimkv_down_project_args* b) {
    DownPlan pa{}, pb{};
    if (plan_down(a, &pa) != SLIMKV_OK || plan_down(b, &pb) != SLIMKV_OK) return 0;
    return std::max<size_t>(align256(pa.bytes) + pb.bytes, 1);
}

extern "C" int slimkv_down_project_pair(const slimkv_down_project_args* a, const slimkv_down_project_args* b,
                                        void* workspace, size_t workspace_bytes, void* stream) {
    DownPlan pa{}, pb{};
    int rc = plan_down(a, &pa);
    if (rc != SLIMKV_OK) return rc;
    rc = plan_down(b, &pb);
    if (rc != SLIMKV_OK) return rc;
    const size_t need = align256(pa.bytes) + pb.bytes;
    if (need && (!workspace || workspace_bytes < need)) return fail(SLIMKV_EWORKSPACE, "workspace too small");
    char* ws = static_cast<char*>(workspace);
    const int64_t Ma = a->batch * a->row_count, Mb = b->batch * b->row_count;
    if (pa.splits > 1 || pb.splits > 1 || Ma == 0 || Mb == 0) {
        // split partials (a reduce launch each) or an empty problem: one at a time
        rc = down_run(a, nullptr, ws, align256(pa.bytes), stream);
        if (rc != SLIMKV_OK) return rc;
        return down_run(b, nullptr, ws ? ws + align256(pa.bytes) : nullptr, pb.bytes, stream);
    }
    const DownParams p0 = down_params(a, nullptr, pa, nullptr);
    const DownParams p1 = down_params(b, nullptr, pb, nullptr);
    const int64_t g0 = down_grid(p0), g1 = down_grid(p1);
    if (g0 + g1 > 0x7fffffff) return fail(SLIMKV_EINVAL, "down-projection grid too large");
    hipLaunchKernelGGL(down_pair_kernel, dim3((unsigned)(g0 + g1)), dim3(256), 0, static_cast<hipStream_t>(stream), p0,
                       p1, (int)g0);
    return check_hip(hipGetLastError(), "down-projection pair launch");
}

extern "C" int slimkv_down_project_to_pages(const slimkv_down_project_args* a, const slimkv_page_rows* dst,
                                            void* workspace, size_t workspace_bytes, void* stream) {
    if (!a || !dst || !dst->pages || !dst->table) return fail(SLIMKV_EINVAL, "null pointer");
    if (dst->num_pages < 0 || dst->slots <= 0 || dst->t_cols <= 0 || dst->t_sb < dst->t_cols || dst->start < 0 ||
        dst->sink_elements < 0 || dst->column < 0 || dst->column + a->out_features > dst->slot_width ||
        dst->page_stride < dst->sink_elements + dst->slots * dst->slot_width)
        return fail(SLIMKV_EINVAL, "invalid page destination");
    if ((dst->page_stride | dst->sink_elements | dst->column | dst->slot_width) % 4 ||
        (reinterpret_cast<uintptr_t>(dst->pages) & 7))
        return fail(SLIMKV_EINVAL, "page rows must be 8-byte aligned");
    slimkv_down_project_args b = *a;
    b.out = dst->pages; b.o_sb = 0; b.o_sn = 0;
    return down_run(&b, dst, workspace, workspace_bytes, stream);
}
