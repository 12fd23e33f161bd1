// Elementwise decode/prefill RoPE (bf16-exact operation boundaries) and the
// two-branch LSE merge.  Each thread handles 8 consecutive features of one row
// with 128-bit loads/stores; the rotate-half partner is read from the same row.

#include "common.hpp"

#include <algorithm>

namespace slimkv {

struct RopeRow {
    const uint16_t* src;
    uint16_t* dst;
    int64_t pos;        // table row, or -1 to copy unchanged
};

// out = bf16(bf16(x*bf16(cos)) + bf16(rotate_half(x)*bf16(sin))) for 8 lanes of a row.
__device__ __forceinline__ void rope8(const uint16_t* src, uint16_t* dst, int dd, int D,
                                      const float* cos, const float* sin, int64_t pos) {
    const u32x4 xv = *reinterpret_cast<const u32x4*>(src + dd);
    if (pos < 0) {
        *reinterpret_cast<u32x4*>(dst + dd) = xv;
        return;
    }
    const int half = D / 2;
    const int pd = dd < half ? dd + half : dd - half;
    const u32x4 pv = *reinterpret_cast<const u32x4*>(src + pd);
    const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
    const uint32_t ps[4] = {pv.x, pv.y, pv.z, pv.w};
    const float* cr = cos + pos * D + dd;
    const float* sr = sin + pos * D + dd;
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float sum[2];
#pragma unroll
        for (int hbit = 0; hbit < 2; ++hbit) {
            const int idx = 2 * e + hbit;
            const float x = bf16_to_f32(hbit ? (xs[e] >> 16) : (xs[e] & 0xffffu));
            float pt = bf16_to_f32(hbit ? (ps[e] >> 16) : (ps[e] & 0xffffu));
            if (dd < half) pt = -pt;
            const float c = round_bf16_hw(cr[idx]);
            const float s = round_bf16_hw(sr[idx]);
            sum[hbit] = round_bf16_hw(x * c) + round_bf16_hw(pt * s);
        }
        o[e] = pack_bf16(sum[0], sum[1]);
    }
    *reinterpret_cast<u32x4*>(dst + dd) = u32x4{o[0], o[1], o[2], o[3]};
}

struct RopeDecodeParams {
    slimkv_rope_decode_args a;
    int64_t q_rows, k_rows;     // rows of q and k (B*H*L)
};

__global__ void __launch_bounds__(256)
rope_decode_kernel(RopeDecodeParams p) {
    const slimkv_rope_decode_args& a = p.a;
    const int per_row = (int)(a.dim / 8);
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t qitems = p.q_rows * per_row;
    const int64_t kitems = p.k_rows * per_row;
    if (gid >= qitems + kitems) return;
    const int D = (int)a.dim;
    if (gid < qitems) {
        const int64_t row = gid / per_row;
        const int dd = (int)(gid % per_row) * 8;
        const int64_t s = row % a.queries;
        const int64_t hh = (row / a.queries) % a.heads;
        const int64_t b = row / (a.queries * a.heads);
        const uint16_t* src = static_cast<const uint16_t*>(a.q) + b * a.q_sb + hh * a.q_sh + s * a.q_ss;
        uint16_t* dst = static_cast<uint16_t*>(a.out_q) + row * D;
        const int64_t pos = clamp_i64(a.q_positions[b * a.pos_sb + s], 0, a.rope_rows - 1);
        rope8(src, dst, dd, D, a.cos, a.sin, pos);
    } else {
        const int64_t kg = gid - qitems;
        const int64_t row = kg / per_row;
        const int dd = (int)(kg % per_row) * 8;
        const int64_t s = row % a.keys;
        const int64_t hh = (row / a.keys) % a.kv_heads;
        const int64_t b = row / (a.keys * a.kv_heads);
        const uint16_t* src = static_cast<const uint16_t*>(a.k) + b * a.k_sb + hh * a.k_sh + s * a.k_ss;
        uint16_t* dst = static_cast<uint16_t*>(a.out_k) + row * D;
        int64_t pos;
        if (s < a.sink) {
            pos = s;
        } else if (s == a.keys - 1) {
            pos = a.q_positions[b * a.pos_sb];
        } else {
            const int64_t ri = clamp_i64(s - a.sink, 0, a.raw_index_count - 1);
            pos = a.raw_indices[ri] + a.sink + a.history;
        }
        pos = clamp_i64(pos, 0, a.rope_rows - 1);
        rope8(src, dst, dd, D, a.cos, a.sin, pos);
    }
}

struct PrefillRopeParams {
    slimkv_prefill_rope_args a;
    int64_t q_rows, k_rows;
};

__global__ void __launch_bounds__(256)
prefill_rope_kernel(PrefillRopeParams p) {
    const slimkv_prefill_rope_args& a = p.a;
    const int per_row = (int)(a.dim / 8);
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t qitems = p.q_rows * per_row;
    const int64_t kitems = p.k_rows * per_row;
    if (gid >= qitems + kitems) return;
    const int D = (int)a.dim;
    if (gid < qitems) {
        const int64_t row = gid / per_row;
        const int dd = (int)(gid % per_row) * 8;
        const int64_t s = row % a.queries;
        const int64_t hh = (row / a.queries) % a.heads;
        const int64_t b = row / (a.queries * a.heads);
        const uint16_t* src = static_cast<const uint16_t*>(a.q) + b * a.q_sb + hh * a.q_sh + s * a.q_ss;
        uint16_t* dst = static_cast<uint16_t*>(a.out_q) + b * a.oq_sb + hh * a.oq_sh + s * a.oq_ss;
        const int64_t pos = clamp_i64(a.positions[b * a.pos_sb + a.keys - a.queries + s], 0, a.rope_rows - 1);
        rope8(src, dst, dd, D, a.cos, a.sin, pos);
    } else {
        const int64_t kg = gid - qitems;
        const int64_t row = kg / per_row;
        const int dd = (int)(kg % per_row) * 8;
        const int64_t s = row % a.keys;
        const int64_t hh = (row / a.keys) % a.kv_heads;
        const int64_t b = row / (a.keys * a.kv_heads);
        const uint16_t* src = static_cast<const uint16_t*>(a.k) + b * a.k_sb + hh * a.k_sh + s * a.k_ss;
        uint16_t* dst = static_cast<uint16_t*>(a.out_k) + b * a.ok_sb + hh * a.ok_sh + s * a.ok_ss;
        const int64_t prefix = a.keys - a.role_len;
        bool beacon = s < prefix && s >= a.sink;
        if (s >= prefix) {
            const int64_t role = a.roles[s - prefix];
            beacon = beacon || role == 1 || role == 2;
        }
        const int64_t pos = beacon ? -1 : clamp_i64(a.positions[b * a.pos_sb + s], 0, a.rope_rows - 1);
        rope8(src, dst, dd, D, a.cos, a.sin, pos);
        if (a.v) {
            const uint16_t* vs = static_cast<const uint16_t*>(a.v) + b * a.v_sb + hh * a.v_sh + s * a.v_ss;
            uint16_t* vd = static_cast<uint16_t*>(a.out_v) + b * a.ov_sb + hh * a.ov_sh + s * a.ov_ss;
            *reinterpret_cast<u32x4*>(vd + dd) = *reinterpret_cast<const u32x4*>(vs + dd);
        }
    }
}

// head_dim 128: 16 lanes a row (8 features a lane, one 16-byte load), the
// rotate-half partner (features d +- 64) taken from lane l ^ 8 of the same
// 16-lane row by a DPP rotation instead of a second load, 32-bit index math,
// and kRopeRows rows a lane group with all their loads issued before any use.
constexpr int kRopeRows = 4;

__device__ __forceinline__ uint32_t ror8(uint32_t v) {        // row_ror:8 inside each 16-lane row
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xf, 0xf, true);
}

__global__ void __launch_bounds__(256)
prefill_rope_rows_kernel(PrefillRopeParams p) {
    const slimkv_prefill_rope_args& a = p.a;
    const uint32_t lane16 = threadIdx.x & 15;
    const uint32_t group = (blockIdx.x * 256u + threadIdx.x) >> 4;
    const uint32_t Q = (uint32_t)p.q_rows, total = (uint32_t)(p.q_rows + p.k_rows);
    const uint32_t queries = (uint32_t)a.queries, keys = (uint32_t)a.keys;
    const uint32_t heads = (uint32_t)a.heads, kv_heads = (uint32_t)a.kv_heads;
    const int dd = (int)lane16 * 8;
    const int64_t prefix = a.keys - a.role_len;
    const uint16_t* src[kRopeRows];
    uint16_t* dst[kRopeRows];
    int64_t pos[kRopeRows];
    bool live[kRopeRows], beacon[kRopeRows];
    u32x4 x[kRopeRows];
    // value rows copied beside the key rows (a.v set): source and destination
    // of row i, null for query rows
    const uint16_t* vsrc[kRopeRows];
    uint16_t* vdst[kRopeRows];
#pragma unroll
    for (int i = 0; i < kRopeRows; ++i) {
        const uint32_t r = group * kRopeRows + i;
        live[i] = r < total;
        const uint32_t rr = live[i] ? r : total - 1;          // dead rows read a live one, store nothing
        if (rr < Q) {
            const uint32_t s = rr % queries, t = rr / queries, hh = t % heads, b = t / heads;
            src[i] = static_cast<const uint16_t*>(a.q) + (int64_t)b * a.q_sb + (int64_t)hh * a.q_sh + (int64_t)s * a.q_ss;
            dst[i] = static_cast<uint16_t*>(a.out_q) + (int64_t)b * a.oq_sb + (int64_t)hh * a.oq_sh + (int64_t)s * a.oq_ss;
            pos[i] = a.positions[(int64_t)b * a.pos_sb + a.keys - a.queries + s];
            beacon[i] = false;
            vsrc[i] = nullptr;
            vdst[i] = nullptr;
        } else {
            const uint32_t kr = rr - Q;
            const uint32_t s = kr % keys, t = kr / keys, hh = t % kv_heads, b = t / kv_heads;
            src[i] = static_cast<const uint16_t*>(a.k) + (int64_t)b * a.k_sb + (int64_t)hh * a.k_sh + (int64_t)s * a.k_ss;
            dst[i] = static_cast<uint16_t*>(a.out_k) + (int64_t)b * a.ok_sb + (int64_t)hh * a.ok_sh + (int64_t)s * a.ok_ss;
            pos[i] = a.positions[(int64_t)b * a.pos_sb + s];
            const bool in_window = (int64_t)s >= prefix;
            const int64_t role = in_window ? a.roles[(int64_t)s - prefix] : 0;
            beacon[i] = in_window ? (role == 1 || role == 2) : ((int64_t)s >= a.sink);
            vsrc[i] = a.v ? static_cast<const uint16_t*>(a.v) + (int64_t)b * a.v_sb + (int64_t)hh * a.v_sh +
                                (int64_t)s * a.v_ss
                          : nullptr;
            vdst[i] = a.v ? static_cast<uint16_t*>(a.out_v) + (int64_t)b * a.ov_sb + (int64_t)hh * a.ov_sh +
                                (int64_t)s * a.ov_ss
                          : nullptr;
        }
        x[i] = *reinterpret_cast<const u32x4*>(src[i] + dd);
    }
    // the value rows go out with the key rows' loads and are stored as they are
#pragma unroll
    for (int i = 0; i < kRopeRows; ++i)
        if (live[i] && vsrc[i]) *reinterpret_cast<u32x4*>(vdst[i] + dd) = *reinterpret_cast<const u32x4*>(vsrc[i] + dd);
    float4 cv[kRopeRows][2], sv[kRopeRows][2];
#pragma unroll
    for (int i = 0; i < kRopeRows; ++i) {
        const int64_t row = clamp_i64(pos[i], 0, a.rope_rows - 1) * a.dim + dd;
        cv[i][0] = *reinterpret_cast<const float4*>(a.cos + row);
        cv[i][1] = *reinterpret_cast<const float4*>(a.cos + row + 4);
        sv[i][0] = *reinterpret_cast<const float4*>(a.sin + row);
        sv[i][1] = *reinterpret_cast<const float4*>(a.sin + row + 4);
    }
#pragma unroll
    for (int i = 0; i < kRopeRows; ++i) {
        const uint32_t pr[4] = {ror8(x[i].x), ror8(x[i].y), ror8(x[i].z), ror8(x[i].w)};
        const uint32_t xs[4] = {x[i].x, x[i].y, x[i].z, x[i].w};
        const float c8[8] = {cv[i][0].x, cv[i][0].y, cv[i][0].z, cv[i][0].w, cv[i][1].x, cv[i][1].y, cv[i][1].z, cv[i][1].w};
        const float s8[8] = {sv[i][0].x, sv[i][0].y, sv[i][0].z, sv[i][0].w, sv[i][1].x, sv[i][1].y, sv[i][1].z, sv[i][1].w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float sum[2];
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                const float v = hb ? hi_bf16(xs[e]) : lo_bf16(xs[e]);
                float pt = hb ? hi_bf16(pr[e]) : lo_bf16(pr[e]);
                if (lane16 < 8) pt = -pt;
                sum[hb] = round_bf16_hw(v * round_bf16_hw(c8[2 * e + hb])) +
                          round_bf16_hw(pt * round_bf16_hw(s8[2 * e + hb]));
            }
            o[e] = pack_bf16(sum[0], sum[1]);
        }
        const u32x4 out = beacon[i] ? x[i] : u32x4{o[0], o[1], o[2], o[3]};
        if (live[i]) *reinterpret_cast<u32x4*>(dst[i] + dd) = out;
    }
}

__global__ void __launch_bounds__(256)
merge_kernel(slimkv_merge_args a) {
    const int per_row = (int)(a.dim / 8);
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t rows = a.batch * a.heads * a.length;
    if (gid >= rows * per_row) return;
    const int64_t row = gid / per_row;
    const int dd = (int)(gid % per_row) * 8;
    const int64_t q = row % a.length;
    const int64_t hh = (row / a.length) % a.heads;
    const int64_t b = row / (a.length * a.heads);
    const float r = a.raw_lse[b * a.rl_sb + hh * a.rl_sh + q * a.rl_sl];
    const float l = a.latent_lse[b * a.ll_sb + hh * a.ll_sh + q * a.ll_sl];
    const float m = fmaxf(r, l);
    const float total = m + log1pf(expf(-fabsf(r - l)));
    const float rw = expf(r - total);
    const float lw = expf(l - total);
    const u32x4 rv = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.raw) + b * a.r_sb + hh * a.r_sh + q * a.r_sl + dd);
    const u32x4 lv = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.latent) + b * a.l_sb + hh * a.l_sh + q * a.l_sl + dd);
    const uint32_t rs[4] = {rv.x, rv.y, rv.z, rv.w};
    const uint32_t ls[4] = {lv.x, lv.y, lv.z, lv.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float r0 = bf16_to_f32(rs[e] & 0xffffu), r1 = bf16_to_f32(rs[e] >> 16);
        const float l0 = bf16_to_f32(ls[e] & 0xffffu), l1 = bf16_to_f32(ls[e] >> 16);
        o[e] = pack_bf16(rw * r0 + lw * l0, rw * r1 + lw * l1);
    }
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(a.out) + row * a.dim + dd) = u32x4{o[0], o[1], o[2], o[3]};
}

namespace {
bool al8(int64_t x) { return (x & 7) == 0; }
bool pal16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
}  // namespace

}  // namespace slimkv

using namespace slimkv;

extern "C" int slimkv_rope_decode(const slimkv_rope_decode_args* a, void* stream) {
    if (!a || !a->q || !a->k || !a->out_q || !a->out_k || !a->cos || !a->sin || !a->q_positions)
        return fail(SLIMKV_EINVAL, "null pointer");
    if (a->dim <= 0 || a->dim % 16 || a->batch <= 0 || a->heads <= 0 || a->kv_heads <= 0 || a->queries <= 0 ||
        a->keys < 0 || a->rope_rows <= 0 || a->sink < 0 || a->history < 0)
        return fail(SLIMKV_EINVAL, "invalid RoPE sizes (dim must be a multiple of 16)");
    const int64_t strides[] = {a->q_sb, a->q_sh, a->q_ss, a->k_sb, a->k_sh, a->k_ss};
    for (int64_t st : strides)
        if (!al8(st)) return fail(SLIMKV_EINVAL, "strides must be multiples of 8 elements");
    if (!pal16(a->q) || !pal16(a->k) || !pal16(a->out_q) || !pal16(a->out_k))
        return fail(SLIMKV_EINVAL, "tensors must be 16-byte aligned");
    const int64_t middle = a->keys > 0 ? std::max<int64_t>(0, a->keys - 1 - a->sink) : 0;
    if (middle > 0 && (!a->raw_indices || a->raw_index_count < middle))
        return fail(SLIMKV_EINVAL, "raw indices must cover every tail slot");
    RopeDecodeParams p{};
    p.a = *a;
    if (p.a.raw_index_count <= 0) p.a.raw_index_count = 1;
    p.q_rows = a->batch * a->heads * a->queries;
    p.k_rows = a->batch * a->kv_heads * a->keys;
    const int64_t items = (p.q_rows + p.k_rows) * (a->dim / 8);
    if (items == 0) return SLIMKV_OK;
    const int64_t blocks = (items + 255) / 256;
    hipLaunchKernelGGL(rope_decode_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), p);
    return check_hip(hipGetLastError(), "rope kernel launch");
}

extern "C" int slimkv_prefill_rope(const slimkv_prefill_rope_args* a, void* stream) {
    if (!a || (a->queries && (!a->q || !a->out_q)) || !a->k || !a->out_k || !a->cos || !a->sin || !a->positions ||
        !a->roles)
        return fail(SLIMKV_EINVAL, "null pointer");
    if (a->dim <= 0 || a->dim % 16 || a->batch <= 0 || a->heads <= 0 || a->kv_heads <= 0 || a->queries < 0 ||
        a->keys < a->queries || a->role_len < 0 || a->role_len > a->keys || a->rope_rows <= 0 || a->sink < 0)
        return fail(SLIMKV_EINVAL, "invalid prefill RoPE sizes");
    const int64_t strides[] = {a->q_sb, a->q_sh, a->q_ss, a->k_sb, a->k_sh, a->k_ss,
                               a->oq_sb, a->oq_sh, a->oq_ss, a->ok_sb, a->ok_sh, a->ok_ss};
    for (int64_t st : strides)
        if (!al8(st)) return fail(SLIMKV_EINVAL, "strides must be multiples of 8 elements");
    if (!pal16(a->q) || !pal16(a->k) || !pal16(a->out_q) || !pal16(a->out_k))
        return fail(SLIMKV_EINVAL, "tensors must be 16-byte aligned");
    if (a->v) {
        if (!a->out_v) return fail(SLIMKV_EINVAL, "null pointer");
        const int64_t vstrides[] = {a->v_sb, a->v_sh, a->v_ss, a->ov_sb, a->ov_sh, a->ov_ss};
        for (int64_t st : vstrides)
            if (!al8(st)) return fail(SLIMKV_EINVAL, "strides must be multiples of 8 elements");
        if (!pal16(a->v) || !pal16(a->out_v)) return fail(SLIMKV_EINVAL, "tensors must be 16-byte aligned");
    }
    PrefillRopeParams p{};
    p.a = *a;
    p.q_rows = a->batch * a->heads * a->queries;
    p.k_rows = a->batch * a->kv_heads * a->keys;
    const int64_t items = (p.q_rows + p.k_rows) * (a->dim / 8);
    if (items == 0) return SLIMKV_OK;
    if (a->dim == 128 && p.q_rows + p.k_rows < ((int64_t)1 << 31) - kRopeRows * 4096 && a->queries < (1 << 30) &&
        a->keys < (1 << 30) && pal16(a->cos) && pal16(a->sin)) {
        const int64_t groups = (p.q_rows + p.k_rows + kRopeRows - 1) / kRopeRows;
        hipLaunchKernelGGL(prefill_rope_rows_kernel, dim3((unsigned)((groups * 16 + 255) / 256)), dim3(256), 0,
                           static_cast<hipStream_t>(stream), p);
        return check_hip(hipGetLastError(), "prefill rope kernel launch");
    }
    const int64_t blocks = (items + 255) / 256;
    hipLaunchKernelGGL(prefill_rope_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), p);
    return check_hip(hipGetLastError(), "prefill rope kernel launch");
}

extern "C" int slimkv_merge(const slimkv_merge_args* a, void* stream) {
    if (!a || !a->raw || !a->latent || !a->raw_lse || !a->latent_lse || !a->out)
        return fail(SLIMKV_EINVAL, "null pointer");
    if (a->batch <= 0 || a->heads <= 0 || a->length <= 0 || a->dim <= 0 || a->dim % 8)
        return fail(SLIMKV_EINVAL, "invalid merge sizes (dim must be a multiple of 8)");
    const int64_t strides[] = {a->r_sb, a->r_sh, a->r_sl, a->l_sb, a->l_sh, a->l_sl};
    for (int64_t st : strides)
        if (!al8(st)) return fail(SLIMKV_EINVAL, "strides must be multiples of 8 elements");
    if (!pal16(a->raw) || !pal16(a->latent) || !pal16(a->out))
        return fail(SLIMKV_EINVAL, "tensors must be 16-byte aligned");
    const int64_t items = a->batch * a->heads * a->length * (a->dim / 8);
    const int64_t blocks = (items + 255) / 256;
    hipLaunchKernelGGL(merge_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream), *a);
    return check_hip(hipGetLastError(), "merge kernel launch");
}
