// Projections of a decode step's rows on gfx950: the new token's q/k/v
// projection with its key RoPE and raw-cache appends in the epilogue
// (slimkv_decode_qkv), and plain few-row projections such as o_proj
// (slimkv_linear_rows).
//
// A decode step multiplies a handful of rows (one token per sequence) by
// weights of tens of MB, so the work is a weight stream: every weight byte is
// read once, with 16-byte non-temporal loads, and fp32 dot products of bf16
// pairs (v_dot2_f32_bf16) against the rows.  A wavefront owns the output
// rows n and n + 64 of a 128-row block -- the rotate-half partners of a head
// -- so the key RoPE finds both halves of each pair in one wavefront; lane l
// reads 16-byte pieces l, l + 64, ... of both weight rows.
#include "common.hpp"

#include <algorithm>

namespace slimkv {
namespace {

constexpr int kProjMaxRows = 4;
constexpr int kProjUnroll = 8;      // 16-byte pieces per lane and row per pass: K = 4096 in one pass

struct ProjParams {
    const uint16_t* x; int64_t x_sm;
    const uint16_t* w; const uint16_t* bias;
    int64_t n, k;
    uint16_t* out; int64_t o_sm;                       // plain rows
    int64_t nq, nkv;                                   // q rows, k rows (= v rows) of the fused projection
    uint16_t* q; int64_t q_sm;
    uint16_t* raw_k; uint16_t* plain_k; uint16_t* raw_v; int64_t c_sm, c_sn;
    const int64_t* slot; int64_t capacity; int32_t* status;
    const float* cos; const float* sin; int64_t rope_rows;
    const int64_t* pos; int64_t pos_sm;
};

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Eight bf16 products summed into c in fp32 (four v_dot2_f32_bf16).  The
// pairs come from one cast of the whole vector: with this compiler a
// __builtin_bit_cast of a vector element (v.y) reads element 0 instead.
__device__ __forceinline__ float dot8(u32x4 a, u32x4 b, float c) {
    const bf16x8 x = __builtin_bit_cast(bf16x8, a), y = __builtin_bit_cast(bf16x8, b);
    c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 0, 1), __builtin_shufflevector(y, y, 0, 1), c,
                                        false);
    c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 2, 3), __builtin_shufflevector(y, y, 2, 3), c,
                                        false);
    c = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 4, 5), __builtin_shufflevector(y, y, 4, 5), c,
                                        false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(x, x, 6, 7), __builtin_shufflevector(y, y, 6, 7),
                                           c, false);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) v += shfl_xor_f(v, o);
    return rows_sum(v);
}

__device__ __forceinline__ uint16_t bf16_bits(float v) { return (uint16_t)pack_bf16(v, 0.f); }

template <int M, bool QKV>
__global__ void __launch_bounds__(256) project_rows_kernel(ProjParams p) {
    const int lane = threadIdx.x & 63;
    const int64_t pair = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (pair >= p.n / 2) return;
    const int64_t n0 = 128 * (pair / 64) + pair % 64, n1 = n0 + 64;
    const int64_t pieces = p.k / 8;
    const uint16_t* w0 = p.w + n0 * p.k;
    const uint16_t* w1 = p.w + n1 * p.k;
    float acc0[M], acc1[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc0[m] = acc1[m] = 0.f;
    for (int64_t base = 0; base < pieces; base += 64 * kProjUnroll) {
        u32x4 a[kProjUnroll], b[kProjUnroll], xv[M][kProjUnroll];
#pragma unroll
        for (int u = 0; u < kProjUnroll; ++u) {
            const int64_t c = base + 64 * u + lane;
            const int64_t cc = c < pieces ? c : 0;           // pieces past K read piece 0, unused
            a[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w0 + 8 * cc));
            b[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(w1 + 8 * cc));
#pragma unroll
            for (int m = 0; m < M; ++m) xv[m][u] = *reinterpret_cast<const u32x4*>(p.x + m * p.x_sm + 8 * cc);
        }
#pragma unroll
        for (int u = 0; u < kProjUnroll; ++u) {
            if (base + 64 * u + lane >= pieces) continue;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                acc0[m] = dot8(a[u], xv[m][u], acc0[m]);
                acc1[m] = dot8(b[u], xv[m][u], acc1[m]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
        acc0[m] = wave_sum(acc0[m]);
        acc1[m] = wave_sum(acc1[m]);
    }
    if (lane >= M) return;
    // lane m writes row m (every lane holds every sum)
    float y0 = acc0[0], y1 = acc1[0];
#pragma unroll
    for (int m = 1; m < M; ++m)
        if (lane == m) { y0 = acc0[m]; y1 = acc1[m]; }
    if (p.bias) {
        y0 += bf16_to_f32(p.bias[n0]);
        y1 += bf16_to_f32(p.bias[n1]);
    }
    const int m = lane;
    if constexpr (!QKV) {
        p.out[m * p.o_sm + n0] = bf16_bits(y0);
        p.out[m * p.o_sm + n1] = bf16_bits(y1);
    } else {
        if (n0 < p.nq) {
            p.q[m * p.q_sm + n0] = bf16_bits(y0);
            p.q[m * p.q_sm + n1] = bf16_bits(y1);
            return;
        }
        const bool is_k = n0 < p.nq + p.nkv;
        const int64_t r = n0 - p.nq - (is_k ? 0 : p.nkv);   // within the k (or v) rows
        const int64_t slot = *p.slot;
        if (slot < 0 || slot >= p.capacity) {               // no cache row is written
            if (p.status) *p.status = SLIMKV_STATUS_BAD_SLOT;
            return;
        }
        const int64_t off = m * p.c_sm + slot * p.c_sn + r;  // head r / 128, element r % 128 (< 64)
        const float x0 = round_bf16_hw(y0), x1 = round_bf16_hw(y1);
        if (!is_k) {
            p.raw_v[off] = bf16_bits(x0);
            p.raw_v[off + 64] = bf16_bits(x1);
            return;
        }
        if (p.plain_k) {
            p.plain_k[off] = bf16_bits(x0);
            p.plain_k[off + 64] = bf16_bits(x1);
        }
        // y[d] = bf16(bf16(x[d] c[d]) + bf16(-x[d+64] s[d])),
        // y[d+64] = bf16(bf16(x[d+64] c[d+64]) + bf16(x[d] s[d+64])), bf16 tables
        const int64_t row = clamp_i64(p.pos[m * p.pos_sm], 0, p.rope_rows - 1) * 128 + r % 128;
        const float c0 = round_bf16_hw(p.cos[row]), s0 = round_bf16_hw(p.sin[row]);
        const float c1 = round_bf16_hw(p.cos[row + 64]), s1 = round_bf16_hw(p.sin[row + 64]);
        p.raw_k[off] = bf16_bits(round_bf16_hw(x0 * c0) + round_bf16_hw(-x1 * s0));
        p.raw_k[off + 64] = bf16_bits(round_bf16_hw(x1 * c1) + round_bf16_hw(x0 * s1));
    }
}

bool al8(int64_t v) { return (v & 7) == 0; }
bool pal16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

template <bool QKV>
int launch_project(const ProjParams& p, int64_t m, hipStream_t st) {
    const dim3 grid((unsigned)((p.n / 2 + 3) / 4)), block(256);
    switch (m) {
        case 1: hipLaunchKernelGGL((project_rows_kernel<1, QKV>), grid, block, 0, st, p); break;
        case 2: hipLaunchKernelGGL((project_rows_kernel<2, QKV>), grid, block, 0, st, p); break;
        case 3: hipLaunchKernelGGL((project_rows_kernel<3, QKV>), grid, block, 0, st, p); break;
        default: hipLaunchKernelGGL((project_rows_kernel<4, QKV>), grid, block, 0, st, p); break;
    }
    return check_hip(hipGetLastError(), "projection kernel launch");
}

int check_rows(const void* x, int64_t x_sm, const void* w, int64_t m, int64_t n, int64_t k) {
    if (m < 1 || m > kProjMaxRows) return fail(SLIMKV_EUNSUP, "decode projections take 1 to 4 rows");
    if (n <= 0 || n % 128 || k <= 0 || k % 8) return fail(SLIMKV_EINVAL, "N must be a multiple of 128, K of 8");
    if ((m > 1 && (x_sm < k || !al8(x_sm))) || !pal16(x) || !pal16(w))
        return fail(SLIMKV_EINVAL, "x rows and W must be 16-byte aligned, rows at least K apart");
    return SLIMKV_OK;
}

}  // namespace
}  // namespace slimkv

using namespace slimkv;

extern "C" int slimkv_linear_rows(const slimkv_linear_rows_args* a, void* stream) {
    if (!a || !a->x || !a->weight || !a->out) return fail(SLIMKV_EINVAL, "null pointer");
    int rc = check_rows(a->x, a->x_sm, a->weight, a->m, a->n, a->k);
    if (rc != SLIMKV_OK) return rc;
    if (a->m > 1 && a->o_sm < a->n) return fail(SLIMKV_EINVAL, "output rows overlap");
    ProjParams p{};
    p.x = static_cast<const uint16_t*>(a->x); p.x_sm = a->x_sm;
    p.w = static_cast<const uint16_t*>(a->weight); p.bias = static_cast<const uint16_t*>(a->bias);
    p.n = a->n; p.k = a->k;
    p.out = static_cast<uint16_t*>(a->out); p.o_sm = a->o_sm;
    return launch_project<false>(p, a->m, static_cast<hipStream_t>(stream));
}

extern "C" int slimkv_decode_qkv(const slimkv_decode_qkv_args* a, void* stream) {
    if (!a || !a->x || !a->weight || !a->q || !a->raw_k || !a->raw_v || !a->slot_index || !a->cos || !a->sin ||
        !a->positions)
        return fail(SLIMKV_EINVAL, "null pointer");
    if (a->head_dim != 128) return fail(SLIMKV_EUNSUP, "decode projection is built for head_dim 128");
    if (a->heads <= 0 || a->kv_heads <= 0 || a->rope_rows <= 0) return fail(SLIMKV_EINVAL, "invalid sizes");
    const int64_t nq = a->heads * 128, nkv = a->kv_heads * 128;
    int rc = check_rows(a->x, a->x_sm, a->weight, a->m, nq + 2 * nkv, a->k);
    if (rc != SLIMKV_OK) return rc;
    if (a->m > 1 && (a->q_sm < nq || a->c_sm < nkv || a->pos_sm < 1))
        return fail(SLIMKV_EINVAL, "output rows overlap");
    if (a->c_sn < nkv) return fail(SLIMKV_EINVAL, "cache slots overlap");
    if (a->capacity <= 0) return fail(SLIMKV_EINVAL, "cache capacity must be positive");
    ProjParams p{};
    p.x = static_cast<const uint16_t*>(a->x); p.x_sm = a->x_sm;
    p.w = static_cast<const uint16_t*>(a->weight); p.bias = static_cast<const uint16_t*>(a->bias);
    p.n = nq + 2 * nkv; p.k = a->k;
    p.nq = nq; p.nkv = nkv;
    p.q = static_cast<uint16_t*>(a->q); p.q_sm = a->q_sm;
    p.raw_k = static_cast<uint16_t*>(a->raw_k); p.plain_k = static_cast<uint16_t*>(a->plain_k);
    p.raw_v = static_cast<uint16_t*>(a->raw_v); p.c_sm = a->c_sm; p.c_sn = a->c_sn;
    p.slot = a->slot_index; p.capacity = a->capacity; p.status = a->status;
    p.cos = a->cos; p.sin = a->sin; p.rope_rows = a->rope_rows;
    p.pos = a->positions; p.pos_sm = a->pos_sm;
    return launch_project<true>(p, a->m, static_cast<hipStream_t>(stream));
}
