// Prefill attention for gfx950: causal (bottom-right aligned) GQA flash
// attention over a whole window, head_dim 128, bf16 operands on the
// 16x16x32 bf16 MFMA with fp32 accumulation and an fp32 online softmax.
//
// Semantics: flash_attn_func(q, k, v, causal=True) as called by
// LlamaFlashAttention2._flash_attention_forward (slimkv/llama3/modeling_llama.py:1752-1809).
//
// Work split.  A workgroup is 4 waves and owns 128 query rows of one head;
// each wave owns 32 rows (two 16-column MFMA tiles).  Keys stream through LDS
// in tiles of 64: K row-major ([key][d]) and V transposed ([d][key]), double
// buffered so one barrier per tile separates writing tile t+1 from reading
// tile t, and prefetched into registers two tiles ahead so global latency
// hides under the MFMAs.  Tiles that every query of the wave sees in full
// skip the mask.
//
// Layouts (lane l, col = l % 16, grp = l / 16; the 16x16x32 MFMA takes
// A[col][8*grp + j], B[8*grp + j][col] and returns D[4*grp + i][col]):
//   S^T = K . Q^T   A = K rows from LDS (8 contiguous d), B = Q rows held in
//                   registers for the whole loop; lane owns query column col.
//   O^T = V^T . P^T P^T comes straight from S^T's accumulator layout with the
//                   contraction order of the 32 keys of a step permuted to
//                   (4*grp + j | 16 + 4*grp + j); V^T is read from LDS in the
//                   same order (one 16-byte read).  The query stays in the
//                   lane, so softmax statistics never cross lanes except for
//                   the two-step max/sum over grp.
//   l  = 1 . P^T    The row sums come from the matrix cores too: one more
//                   MFMA per P^T operand with an A whose row 0 is all ones, so
//                   the denominator sums the same bf16 P the numerator uses
//                   (32 fewer dependent VALU adds a tile: C3 step 1.879 ->
//                   1.833 ms, same box).
//
// Scheduling.  Workgroups sharing a KV head (the g query heads of one group
// for one query block) are placed on the same XCD so the group's K/V tiles
// are fetched into that XCD's L2 once; groups are issued longest-first (the
// last query block sees the most keys under the causal mask).

#include "common.hpp"

namespace slimkv {

namespace {

constexpr int kD = 128;                  // head dim
constexpr int kQRows = 128;              // query rows per workgroup
constexpr int kKeys = 64;                // keys per tile
// Row paddings of 16 elements: 2 % faster than 8 (fewer LDS bank-conflict
// cycles), and two workgroups' buffers (2 x 77,824 B) still fit a CU's LDS.
constexpr int kKStride = kD + 16;        // K tile row (bf16), 288 B
constexpr int kVStride = kKeys + 16;     // V^T tile row (bf16), 160 B: 16-byte aligned reads
constexpr int kXcds = 8;

struct PrefillParams {
    const uint16_t* q; int64_t q_sb, q_sl, q_sh;
    const uint16_t* k; int64_t k_sb, k_sn, k_sh;
    const uint16_t* v; int64_t v_sb, v_sn, v_sh;
    uint16_t* out; int64_t o_sb, o_sl, o_sh;
    float* lse;
    const int32_t* seqlens;
    int B, Lq, Hq, Hk, Nk, causal;
    int qblocks;
    float scale_log2;
    const uint32_t* pairs; int64_t rope_rows; int repeats;    // query RoPE when pairs != nullptr
    const int64_t* q_pos; int64_t qpos_sb;
};

__device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_bf16(lo, hi); }

// Query RoPE in the operand registers: lane pieces kk and kk + 2 hold d and
// d + 64 (d = 32 kk + 8 grp + e), rotate_half's partners.  The reference's bf16
// steps, element by element: bf16(bf16(x * bf16(c)) + bf16(r * bf16(s))) with
// r = -x[d + 64] below the half and x[d - 64] above it; (bf16 c | bf16 s)
// pairs from the table prepared once (slimkv_prepare_rope_pairs), the upper
// half read from the lower one where every row repeats its first half.
struct QPairs {
    u32x4 p[4][2];          // pairs of piece kk: d = 32 kk + 8 grp .. + 7
};

__device__ __forceinline__ void load_q_pairs(QPairs& t, const uint32_t* row, int grp, int repeats) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const int d = 32 * kk + 8 * grp;
        const int c = (kk >= 2 && repeats) ? d - 64 : d;
        t.p[kk][0] = *reinterpret_cast<const u32x4*>(row + c);
        t.p[kk][1] = *reinterpret_cast<const u32x4*>(row + c + 4);
    }
}

__device__ __forceinline__ void rope_q_operand(u32x4 (&x)[4], const QPairs& t) {
    u32x4 y[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
        const u32x4& own = x[kk];
        const u32x4& partner = x[kk ^ 2];
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float sum[2];
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                const uint32_t cs = t.p[kk][e >> 1][2 * (e & 1) + hb];
                const float v = hb ? hi_bf16(own[e]) : lo_bf16(own[e]);
                float r = hb ? hi_bf16(partner[e]) : lo_bf16(partner[e]);
                if (kk < 2) r = -r;
                sum[hb] = round_bf16_hw(v * lo_bf16(cs)) + round_bf16_hw(r * hi_bf16(cs));
            }
            o[e] = pack_bf16(sum[0], sum[1]);
        }
        y[kk] = u32x4{o[0], o[1], o[2], o[3]};
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) x[kk] = y[kk];
}

// V^T keeps, per 32-key step, the keys a lane group reads together side by
// side: key 16h + 4g + j of the step sits at 8g + 4h + j, so the eight keys of
// lane group g (4g + j and 16 + 4g + j, the P^T contraction order) are one
// 16-byte read.
__device__ __forceinline__ int vt_pos(int kq) {       // kq: group of 4 keys in the 64-key tile
    return 32 * (kq >> 3) + 8 * (kq & 3) + 4 * ((kq >> 2) & 1);
}

// bf16 element e of a and of b side by side: (a_e | b_e << 16), one byte
// permute (selector bytes 0-3 pick from a, 4-7 from b).
__device__ __forceinline__ uint32_t pair_of(const u32x4& a, const u32x4& b, int e) {
    return __builtin_amdgcn_perm(b[e >> 1], a[e >> 1], (e & 1) ? 0x07060302u : 0x05040100u);
}

struct TileRegs {
    u32x4 k[4];     // 4 x 16 B of K: pieces threadIdx.x + 256 r -> (row p/16, d-piece p%16)
    u32x4 v[4];     // 4 keys (4*kq + r) x 8 d (d-piece cp) of V
};

// Tile loads go through a buffer resource built per tile on the scalar unit:
// base = the tile's first key row, range = its rows below n.  Each lane's byte
// offset into the tile is loop-invariant (no per-tile address arithmetic), and
// rows past n read as zero -- their scores are masked and their P is zero.
struct TileOffsets {
    uint32_t k[4], v[4];    // bytes from the tile's first key row
};

__device__ __forceinline__ TileOffsets tile_offsets(int64_t k_sn, int64_t v_sn) {
    TileOffsets o;
    const int tid = threadIdx.x;
#pragma unroll
    for (int r = 0; r < 4; ++r) {   // K pieces tid + 256 r -> (row p / 16, d-piece p % 16)
        const int p = tid + 256 * r;
        o.k[r] = (uint32_t)(2 * ((p >> 4) * k_sn + 8 * (p & 15)));
    }
    const int kq = tid & 15, cp = tid >> 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) o.v[r] = (uint32_t)(2 * ((4 * kq + r) * v_sn + 8 * cp));   // keys 4kq + r, d-piece cp
    return o;
}

constexpr int kBufferWord3 = 0x00020000;   // raw buffer, 32-bit data format

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_resource(const uint16_t* base, int64_t sn, int k0, int n) {
    const int rows = min(n - k0, kKeys);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(base + (int64_t)k0 * sn), 0, rows * (int)(2 * sn),
                                             kBufferWord3);
}

__device__ __forceinline__ void load_tile(TileRegs& t, const uint16_t* kb, const uint16_t* vb, int64_t k_sn,
                                          int64_t v_sn, int k0, int n, const TileOffsets& o) {
    const __amdgpu_buffer_rsrc_t rk = tile_resource(kb, k_sn, k0, n);
    const __amdgpu_buffer_rsrc_t rv = tile_resource(vb, v_sn, k0, n);
#pragma unroll
    for (int r = 0; r < 4; ++r) t.k[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, o.k[r], 0, 0));
#pragma unroll
    for (int r = 0; r < 4; ++r) t.v[r] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, o.v[r], 0, 0));
}

__device__ __forceinline__ void store_tile(const TileRegs& t, uint16_t* ks, uint16_t* vts) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int p = tid + 256 * r;
        *reinterpret_cast<u32x4*>(ks + (p >> 4) * kKStride + 8 * (p & 15)) = t.k[r];
    }
    const int kq = tid & 15, cp = tid >> 4;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        u32x2 w;
        w.x = pair_of(t.v[0], t.v[1], e);
        w.y = pair_of(t.v[2], t.v[3], e);
        *reinterpret_cast<u32x2*>(vts + (8 * cp + e) * kVStride + vt_pos(kq)) = w;
    }
}

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
prefill_kernel(PrefillParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t ks_buf[2][kKeys * kKStride];
    __shared__ __attribute__((aligned(16))) uint16_t vts_buf[2][kD * kVStride];

    const int g = p.Hq / p.Hk;
    const int xcd = blockIdx.x % kXcds;
    const int slot = blockIdx.x / kXcds;
    const int group = (slot / g) * kXcds + xcd;
    const int ngroups = p.qblocks * p.B * p.Hk;
    if (group >= ngroups) return;
    const int qb = p.qblocks - 1 - group / (p.B * p.Hk);
    const int rem = group % (p.B * p.Hk);
    const int b = rem / p.Hk, kvh = rem % p.Hk;
    const int h = kvh * g + slot % g;
    const int n = p.seqlens ? max(0, min(p.seqlens[b], p.Nk)) : p.Nk;

    // the wave index in a scalar register: the full-tile test below is then a
    // scalar branch, and the masked path's index arithmetic stays inside it
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, grp = lane >> 4;
    const int q0 = qb * kQRows + wave * 32;
    const int shift = n - p.Lq;
    int k_end = n;
    if (p.causal) k_end = min(n, min(qb * kQRows + kQRows, p.Lq) + shift);
    const int ntiles = k_end > 0 ? (k_end + kKeys - 1) / kKeys : 0;

    // Query RoPE: the rows' positions first, their table pairs once the
    // first K/V tile's loads are issued, the rotation before the tile loop.
    int64_t qpos[2] = {0, 0};
    if (p.pairs) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
            qpos[nt] = clamp_i64(p.q_pos[(int64_t)b * p.qpos_sb + min(q0 + 16 * nt + col, p.Lq - 1)], 0,
                                 p.rope_rows - 1);
    }

    // Q operand: rows q0 + 16 nt + col, d = 32 ks + 8 grp .. +7
    u32x4 qr[2][4];
    {
        const uint16_t* qbase = p.q + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const int row = q0 + 16 * nt + col;
            const bool ok = row < p.Lq;
            const uint16_t* src = qbase + (int64_t)min(row, p.Lq - 1) * p.q_sl + 8 * grp;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const u32x4 x = *reinterpret_cast<const u32x4*>(src + 32 * kk);
                qr[nt][kk] = u32x4{ok ? x.x : 0u, ok ? x.y : 0u, ok ? x.z : 0u, ok ? x.w : 0u};
            }
        }
    }

    v4f o[8][2];
#pragma unroll
    for (int md = 0; md < 8; ++md)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) o[md][nt] = v4f{0.f, 0.f, 0.f, 0.f};
    float m[2] = {kNegInf, kNegInf};
    // row sums of P on the matrix cores: A row 0 all ones, so row 0 of the
    // accumulator (lanes of lane group 0, element 0) is the sum over keys
    v4f lacc[2] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
    const uint32_t one2 = col == 0 ? 0x3f803f80u : 0u;
    const u32x4 ones = u32x4{one2, one2, one2, one2};

    const uint16_t* kb = p.k + (int64_t)b * p.k_sb + (int64_t)kvh * p.k_sh;
    const uint16_t* vb = p.v + (int64_t)b * p.v_sb + (int64_t)kvh * p.v_sh;
    const TileOffsets toff = tile_offsets(p.k_sn, p.v_sn);
    TileRegs tr;
    if (ntiles > 0) load_tile(tr, kb, vb, p.k_sn, p.v_sn, 0, n, toff);
    if (p.pairs) {
        QPairs qp[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) load_q_pairs(qp[nt], p.pairs + qpos[nt] * kD, grp, p.repeats);
        if (ntiles > 0) {
            store_tile(tr, ks_buf[0], vts_buf[0]);
            if (ntiles > 1) load_tile(tr, kb, vb, p.k_sn, p.v_sn, kKeys, n, toff);
        }
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) rope_q_operand(qr[nt], qp[nt]);
    } else if (ntiles > 0) {
        store_tile(tr, ks_buf[0], vts_buf[0]);
        if (ntiles > 1) load_tile(tr, kb, vb, p.k_sn, p.v_sn, kKeys, n, toff);
    }
    if (ntiles > 0) __syncthreads();
    // the wave's earliest query sees keys up to q0 + shift
    const int wave_last = p.causal ? q0 + shift : n - 1;

    for (int t = 0; t < ntiles; ++t) {
        const int k0 = t * kKeys;
        const uint16_t* ks = ks_buf[t & 1];
        const uint16_t* vts = vts_buf[t & 1];
        const bool full = k0 + kKeys - 1 <= min(wave_last, n - 1);

        // S^T = K . Q^T for 64 keys x 32 queries
        v4f s[4][2];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) s[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const u32x4 a = *reinterpret_cast<const u32x4*>(ks + (16 * mt + col) * kKStride + 32 * kk + 8 * grp);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) s[mt][nt] = mfma32(a, qr[nt][kk], s[mt][nt]);
            }
        }

        // masked, scaled scores and the online softmax (per query column)
        u32x4 pb[2][2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            float mx = kNegInf;
            // raw scores: the scale (> 0) is applied inside the exponent's FMA
            if (full) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[mt][nt][i]);
            } else {
                // key k0 + 16 mt + 4 grp + i is visible while 16 mt + i <= lim
                const int qi = q0 + 16 * nt + col;
                const int lim = (p.causal ? min(qi + shift, n - 1) : n - 1) - k0 - 4 * grp;
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float x = 16 * mt + i <= lim ? s[mt][nt][i] : kNegInf;
                        s[mt][nt][i] = x;
                        mx = fmaxf(mx, x);
                    }
            }
            mx = rows_max(mx);
            const float m_new = fmaxf(m[nt], mx * p.scale_log2);
            const float base = m_new == kNegInf ? 0.f : m_new;
            const float alpha = fast_exp2(m[nt] - base);
            m[nt] = m_new;
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[mt][nt][i] = fast_exp2(__builtin_fmaf(s[mt][nt][i], p.scale_log2, -base));
            // once the running maxima settle (most tiles of a long window) no
            // column's alpha moves off 1, and the wave skips the rescale
            if (__ballot(alpha != 1.f)) {
#pragma unroll
                for (int md = 0; md < 8; ++md) o[md][nt] *= alpha;
                lacc[nt] *= alpha;
            }
#pragma unroll
            for (int ss = 0; ss < 2; ++ss)
                pb[ss][nt] = u32x4{pack2(s[2 * ss][nt][0], s[2 * ss][nt][1]), pack2(s[2 * ss][nt][2], s[2 * ss][nt][3]),
                                   pack2(s[2 * ss + 1][nt][0], s[2 * ss + 1][nt][1]),
                                   pack2(s[2 * ss + 1][nt][2], s[2 * ss + 1][nt][3])};
        }

        // O^T += V^T . P^T
#pragma unroll
        for (int ss = 0; ss < 2; ++ss) {
#pragma unroll
            for (int md = 0; md < 8; ++md) {
                const u32x4 a = *reinterpret_cast<const u32x4*>(vts + (16 * md + col) * kVStride + 32 * ss + 8 * grp);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) o[md][nt] = mfma32(a, pb[ss][nt], o[md][nt]);
            }
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) lacc[nt] = mfma32(ones, pb[ss][nt], lacc[nt]);
        }
        // tile t + 1 (in registers) into the other buffer, then fetch tile t + 2;
        // the barrier orders this write after every wave's reads of tile t - 1
        // and before every wave's reads of tile t + 1
        if (t + 1 < ntiles) {
            store_tile(tr, ks_buf[(t + 1) & 1], vts_buf[(t + 1) & 1]);
            if (t + 2 < ntiles) load_tile(tr, kb, vb, p.k_sn, p.v_sn, k0 + 2 * kKeys, n, toff);
        }
        __syncthreads();
    }

#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const float tot = rows_sum(lacc[nt][0]);
        const float inv = tot > 0.f ? 1.f / tot : 0.f;
        const int qi = q0 + 16 * nt + col;
        if (qi >= p.Lq) continue;
        uint16_t* dst = p.out + (int64_t)b * p.o_sb + (int64_t)qi * p.o_sl + (int64_t)h * p.o_sh + 4 * grp;
#pragma unroll
        for (int md = 0; md < 8; ++md) {
            u32x2 w;
            w.x = pack2(o[md][nt][0] * inv, o[md][nt][1] * inv);
            w.y = pack2(o[md][nt][2] * inv, o[md][nt][3] * inv);
            *reinterpret_cast<u32x2*>(dst + 16 * md) = w;
        }
        if (p.lse && grp == 0)
            p.lse[((int64_t)b * p.Hq + h) * p.Lq + qi] = tot > 0.f ? (m[nt] + __log2f(tot)) * kLn2 : kNegInf;
    }
}

bool al16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace

}  // namespace slimkv

using namespace slimkv;

extern "C" int slimkv_prefill_attention(const slimkv_prefill_attention_args* a, void* stream) {
    if (!a || !a->q || !a->k || !a->v || !a->out) return fail(SLIMKV_EINVAL, "null pointer");
    if (a->head_dim != kD) return fail(SLIMKV_EUNSUP, "prefill attention supports head_dim 128");
    if (a->batch < 0 || a->queries < 0 || a->keys < 0 || a->heads <= 0 || a->kv_heads <= 0 ||
        a->heads % a->kv_heads || a->batch > 65535 || a->queries > (1 << 24) || a->keys > (1 << 30))
        return fail(SLIMKV_EINVAL, "invalid prefill attention sizes");
    for (int64_t s : {a->q_sb, a->q_sl, a->q_sh, a->k_sb, a->k_sn, a->k_sh, a->v_sb, a->v_sn, a->v_sh, a->o_sb,
                      a->o_sl, a->o_sh})
        if (s % 8) return fail(SLIMKV_EINVAL, "strides must be multiples of 8 elements");
    if (!al16(a->q) || !al16(a->k) || !al16(a->v) || !al16(a->out))
        return fail(SLIMKV_EINVAL, "tensors must be 16-byte aligned");
    if (!(a->scale > 0.0)) return fail(SLIMKV_EINVAL, "the softmax scale must be positive");
    // tile loads hold a tile's byte offsets and range in 32 bits; a key row
    // holds at least its own head's 128 elements
    if (a->k_sn < kD || a->v_sn < kD || a->k_sn >= (1 << 23) || a->v_sn >= (1 << 23))
        return fail(SLIMKV_EUNSUP, "K/V key strides must be in [128, 2^23) elements");
    if (a->batch == 0 || a->queries == 0) return SLIMKV_OK;
    PrefillParams p{};
    p.q = static_cast<const uint16_t*>(a->q); p.q_sb = a->q_sb; p.q_sl = a->q_sl; p.q_sh = a->q_sh;
    p.k = static_cast<const uint16_t*>(a->k); p.k_sb = a->k_sb; p.k_sn = a->k_sn; p.k_sh = a->k_sh;
    p.v = static_cast<const uint16_t*>(a->v); p.v_sb = a->v_sb; p.v_sn = a->v_sn; p.v_sh = a->v_sh;
    p.out = static_cast<uint16_t*>(a->out); p.o_sb = a->o_sb; p.o_sl = a->o_sl; p.o_sh = a->o_sh;
    p.lse = a->lse;
    p.seqlens = a->seqlens_k;
    p.B = (int)a->batch; p.Lq = (int)a->queries; p.Hq = (int)a->heads; p.Hk = (int)a->kv_heads;
    p.Nk = (int)a->keys; p.causal = a->causal ? 1 : 0;
    p.qblocks = (p.Lq + kQRows - 1) / kQRows;
    p.scale_log2 = (float)(a->scale * 1.4426950408889634);
    if (a->rope_pairs) {
        // positions [batch, >= queries] with row stride qpos_sb (0: one row for every batch entry)
        if (!a->q_positions || a->rope_rows <= 0 || a->qpos_sb < 0 || (a->qpos_sb > 0 && a->qpos_sb < a->queries))
            return fail(SLIMKV_EINVAL, "query RoPE needs rope pairs, rope_rows > 0 and [batch, >= queries] positions");
        if (!al16(a->rope_pairs)) return fail(SLIMKV_EINVAL, "RoPE pairs must be 16-byte aligned");
        p.pairs = a->rope_pairs; p.rope_rows = a->rope_rows; p.repeats = a->rope_repeats ? 1 : 0;
        p.q_pos = a->q_positions; p.qpos_sb = a->qpos_sb;
    }
    const int64_t groups = (int64_t)p.qblocks * p.B * p.Hk;
    const int64_t grid = (groups + kXcds - 1) / kXcds * kXcds * (p.Hq / p.Hk);
    if (grid > 0x7fffffff) return fail(SLIMKV_EINVAL, "prefill grid too large");
    hipLaunchKernelGGL(prefill_kernel, dim3((unsigned)grid), dim3(256), 0, static_cast<hipStream_t>(stream), p);
    return check_hip(hipGetLastError(), "prefill attention launch");
}
