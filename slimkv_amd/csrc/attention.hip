// Split-K decode attention on gfx950 MFMA tiles, plus the fused latent beacon
// decode built from it.
//
// One kernel family, `split_kernel`, computes flash-decode partials for up to
// two key segments in a single launch (the raw full-dim segment and the latent
// beacon segment of the fused decode, or the only segment of plain attention).
// A workgroup owns (batch b, KV head h, column tile t, key split s):
//   * a column tile is up to 16 packed query rows p = jj*Lq + l of one KV head
//     (jj = query head within the GQA group, l = query index), the MFMA N side;
//   * 4 wavefronts walk 16-key row tiles of the split in lockstep, each keeping
//     its own online-softmax state for the 16 columns;
//   * scores S^T[key, col] = K_tile (A, straight from HBM, 128-bit loads) x
//     Qop^T (B, registers) on v_mfma_f32_16x16x16_bf16, so each lane owns one
//     column and four keys -- the softmax max needs two cross-lane shuffles;
//   * P^T stays in the score registers and is the B operand of
//     O^T[v, col] += V_tile^T (A, transposed out of LDS) x P^T.
// Latent K rows are shared by every query head (MQA-like after absorption);
// when the up-projections are block diagonal a column tile only reads the
// latent slices of the heads it holds, so each latent byte is read once.
//
// The combine kernels merge the split partials of both segments in fp32, lift
// the latent accumulator through U_V once per (b, head), fold both biases and
// write bf16 output plus the natural-log LSE.

#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <vector>

namespace slimkv {

// ---------------------------------------------------------------------------
// split kernel
// ---------------------------------------------------------------------------

struct Seg {
    const uint16_t* q; int64_t q_sb, q_sl, q_sh;   // query operand rows
    const uint16_t* k; int64_t k_sb, k_sn, k_sh;
    const uint16_t* v; int64_t v_sb, v_sn, v_sh;
    const int32_t* seqlens;                          // per-batch key counts or null
    int n;                                           // keys (upper bound)
    int hk;                                          // KV heads of this segment
    int g;                                           // query heads per KV head
    int wk, wv;                                      // K / V row widths
    int causal;
    int tiles, cols, splits, rows_per_split;            // cols: packed query rows per tile (<= 16)
    int blk_heads, blk_k, blk_v;                     // block-diagonal layout (0 = full rows)
    int q_compact;                                   // q operand holds only the own block slice
    float* part_ml;                                  // [B][Hq*Lq][splits][2]
    float* part_acc;                                 // [B][Hq*Lq][splits][wown]
    int wown;
    int nwg;
    // Paged rows (PAGED instances): row i of batch b starts at
    // k / v + page(table[b][i / slots]) * page_stride + (i % slots) * k_sn,
    // page() with torch's indexing rules; an entry outside the pool is
    // reported in *status (the row then reads page 0, inside the pool).
    const int64_t* table; int64_t t_sb, page_stride, num_pages;
    int slots, slots_shift;                          // slots_shift = log2(slots) or -1
    int32_t* status;
    // Compact schedule: workgroup items enumerate only the non-empty splits of
    // each batch entry (needs seqlens); items past the last one exit at once.
    int compact;
};

// Second row segment of the bulk segment (SEG2 instances): rows [0, n1) of a
// sequence at Seg::k / v, rows [n1, n) here, row i at index i - n1.  Kept at
// the end of SplitParams so that the other instances read their arguments at
// the same offsets as without it.
struct SegRows2 {
    const uint16_t* k2; int64_t k2_sb, k2_sn;
    const uint16_t* v2; int64_t v2_sb, v2_sn;
    int n1;
};

// Raw rows read through raw pages (RAWPG instances, the raw segment of the
// paged decode): row r of sequence b is token r % block of block
// table[b][r / block] in pages [blocks, block, 2, Hkv, D] (Seg::k / v point
// at the pool's K and V halves, Seg::k_sn is the token stride).  Block ids
// follow torch's indexing; an entry outside the pool that a row needs is
// reported in Seg::status and read as block 0.
struct RawPagesArg {
    const int64_t* table; int64_t t_sb;
    int64_t blk_stride, num_blocks;
    int block_shift;                                 // block = 1 << block_shift tokens
};

// Query rows rotated where the split kernel reads them (the fused
// reconstruction decode, which needs no other query preparation): q as given,
// the RoPE tables and the query positions (null: the tables hold one row per
// query, row b * Lq + l).  cos null: q is used as given.
struct QRope {
    const uint16_t* q; int64_t q_sb, q_sl, q_sh;
    const int64_t* pos; int64_t pos_sb;
    const float* cos; const float* sin; int64_t rope_rows;
};

__device__ __forceinline__ int64_t qrope_row(const QRope& r, int b, int l, int Lq) {
    if (!r.pos) return (int64_t)b * Lq + l;
    return clamp_i64(r.pos[(int64_t)b * r.pos_sb + l], 0, r.rope_rows - 1);
}

// Latent query operands made inside the split kernel (the fused decode with
// per-KV-head bases): each latent wave rotates its query rows from
// SplitParams::qrope and absorbs them into its heads' U_K on the MFMA, and the
// raw waves rotate theirs, so no prologue launch precedes the split kernel.
struct QAbsorb {
    const uint16_t* ut;                              // per-head U_K^T [Hkv][wq][128], null: Seg::q holds operands
    int wq;                                          // per-head K rank
};

// K bias of the latent rows when the split kernel makes the query operands:
// the raw waves of split 0 write each query row's LSE shift (q . b_k of its KV
// head, times the natural-log scale) for the combine, as the prologue does
// when it runs.  bias null: no K bias.
struct QShift {
    const uint16_t* bias;                            // up_k_bias [Hkv * 128]
    float* shift;                                    // [B][Hq*Lq]
    float scale;
};

struct SplitParams {
    Seg seg[2];
    int nseg;
    int B, Lq, Hq;
    float scale_log2;
    SegRows2 two;
    RawPagesArg rawp;
    QRope qrope;                                     // q null: seg[].q holds rotated rows
    QAbsorb absorb;
    QShift kshift;
};

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;

template <int KS>
struct SplitLds {
    static constexpr int RS = 16 * KS + 8;                       // padded V row (bf16)
    static constexpr int bytes = kWaves * 2 * 16 * RS * 2;      // per-wave double-buffered V tiles
};

// Order LDS accesses of one wavefront: a wave's LDS instructions execute in
// issue order, so only compiler reordering has to be prevented.
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One 16-key tile held in registers: the K tile already in MFMA A-operand
// order, the V tile as coalesced 16-byte pieces on their way to LDS.
template <int KS>
struct TileRegs {
    u32x4 k[KS / 2];
    u32x4 v[KS / 2];
};

// Loads are branch-free: an invalid piece reads a clamped in-bounds address.
// Pieces that must read as zero are zeroed by a select where they are used,
// never where they are loaded: a select at the load site would make the
// compiler wait for the load there (vmcnt) and empty the software pipeline.
__device__ __forceinline__ u32x4 zero_unless(bool ok, u32x4 v) {
    return u32x4{ok ? v.x : 0u, ok ? v.y : 0u, ok ? v.z : 0u, ok ? v.w : 0u};
}

// Key/value rows are read once per decode step.  Dense tiles of KS k-steps
// read them with non-temporal loads (gfx950 `nt`) where that measured faster:
// the 64-column latent tiles (rank-32 layer 30.6 against 32.5 us, B16 32K)
// and the 96-column ones (rank 48: 38.1 against 40.9 us).  The 128-column
// tiles -- the raw rows, head_dim 128 -- ran slower with them (rank-16 layer
// 18.0 against 17.4 us; the paged decode's raw segment 148.2 against 146.7 us
// a step), and the paged row policies keep plain loads.
template <int KS>
struct StreamLoads {
    static constexpr bool value = KS == 4 || KS == 6;
};

template <bool NT>
__device__ __forceinline__ u32x4 tile_load(const uint16_t* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    else return *reinterpret_cast<const u32x4*>(p);
}


// The RoPE table values one lane needs for a head_dim-128 query row held as
// MFMA operand pieces (elements 32c + 8*grp + [0, 8), c = 0..3).
struct RopeRow {
    float4 c[4][2], s[4][2];
};

__device__ __forceinline__ void load_rope_row(RopeRow& t, const float* cs, const float* sn, int grp) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int d0 = 32 * c + 8 * grp;
        t.c[c][0] = *reinterpret_cast<const float4*>(cs + d0);
        t.c[c][1] = *reinterpret_cast<const float4*>(cs + d0 + 4);
        t.s[c][0] = *reinterpret_cast<const float4*>(sn + d0);
        t.s[c][1] = *reinterpret_cast<const float4*>(sn + d0 + 4);
    }
}

// Rotate one head_dim-128 query row held as MFMA operand pieces: x[c] holds
// elements 32c + 8*grp + [0, 8); the rotate-half partner of piece c is c ^ 2.
// out = bf16(bf16(x * bf16(cos)) + bf16(rotate_half(x) * bf16(sin))), the
// reference's bf16 operation order (decode_kernels.py:7-51), each rounding one
// packed conversion (round to nearest even).
__device__ __forceinline__ void rope_operand(u32x4 (&x)[4], const RopeRow& t) {
    float v[4][8];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[c][2 * e] = bf16_to_f32(x[c][e] & 0xffffu);
            v[c][2 * e + 1] = bf16_to_f32(x[c][e] >> 16);
        }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const float4 c0 = t.c[c][0], c1 = t.c[c][1], s0 = t.s[c][0], s1 = t.s[c][1];
        const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            float o[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const float partner = c < 2 ? -v[c ^ 2][i + u] : v[c ^ 2][i + u];
                o[u] = round_bf16_hw(v[c][i + u] * round_bf16_hw(cv[i + u])) +
                       round_bf16_hw(partner * round_bf16_hw(sv[i + u]));
            }
            w[i / 2] = pack_bf16(o[0], o[1]);       // the sum's rounding
        }
        x[c] = u32x4{w[0], w[1], w[2], w[3]};
    }
}

// Row addresses of dense rows: one tensor, or two tensors split at row n1
// (a sequence's history and its current window, each read where it lies).
struct OneRows {
    const uint16_t* base; int64_t sn;
    __device__ __forceinline__ const uint16_t* row(int r) const { return base + (int64_t)r * sn; }
};
struct TwoRows {
    const uint16_t* base; int64_t sn;
    const uint16_t* base2; int64_t sn2;
    int n1;
    __device__ __forceinline__ const uint16_t* row(int r) const {
        return r < n1 ? base + (int64_t)r * sn : base2 + (int64_t)(r - n1) * sn2;
    }
};

struct RawPageRows {
    const uint16_t* base;                            // the pool's K or V half, head offset included
    const int64_t* tab;                              // the sequence's block table row
    int64_t blk_stride, tok_stride, num_blocks;
    int shift, last_valid;
    bool* bad;
    __device__ __forceinline__ const uint16_t* row(int r) const {
        const int rc = min(r, last_valid);
        const int64_t blk = table_page(tab[rc >> shift], num_blocks);
        *bad |= blk < 0;
        return base + (blk < 0 ? 0 : blk) * blk_stride + (int64_t)(rc & ((1 << shift) - 1)) * tok_stride;
    }
};

template <int KS, class Rows>
__device__ __forceinline__ void load_tile(TileRegs<KS>& t, const Rows& krows, const Rows& vrows, int r0, int last_row,
                                          int span_k, int span_v, int col, int grp, int lane) {
    constexpr int VT = KS;
    // K: lane (row = col, group grp) takes elements [32c + 8*grp, +8) of the
    // tile's k range for c < KS/2 -- a row's four groups read 64 contiguous bytes.
    {
        const uint16_t* src = krows.row(min(r0 + col, last_row));
#pragma unroll
        for (int c = 0; c < KS / 2; ++c) {
            const int kk = 32 * c + 8 * grp;
            t.k[c] = tile_load<StreamLoads<KS>::value>(src + (kk + 8 <= span_k ? kk : 0));
        }
    }
    // V: 16 rows x 2*VT pieces of 16 bytes; piece p = 64c + lane is row
    // p / (2VT), column piece p % (2VT) -- consecutive lanes, consecutive bytes.
#pragma unroll
    for (int c = 0; c < VT / 2; ++c) {
        const int p = 64 * c + lane;
        const int row = r0 + p / (2 * VT);
        const int pc = p % (2 * VT);
        const uint16_t* src = vrows.row(min(row, last_row)) + (8 * pc + 8 <= span_v ? 8 * pc : 0);
        t.v[c] = tile_load<StreamLoads<KS>::value>(src);
    }
}

// Compact schedule: item -> (b, s) over the non-empty splits of every batch
// entry, splits of b = ceil(len_b / rps).  Wave-uniform; false past the end.
__device__ __forceinline__ bool locate_split(int item, const int32_t* lens, int B, int n, int rps, int& b, int& s) {
    const int lane = threadIdx.x & 63;
    int base = 0;
    for (int b0 = 0; b0 < B; b0 += 64) {
        const int bi = b0 + lane;
        int len = bi < B ? lens[bi] : 0;
        len = len < 0 ? 0 : (len > n ? n : len);
        const int cnt = (len + rps - 1) / rps;
        int inc = cnt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(inc, o, 64);
            if (lane >= o) inc += y;
        }
        const int tot = __shfl(inc, 63, 64);
        if (item < base + tot) {
            const unsigned long long m = __ballot(base + inc > item);
            const int first = __ffsll(m) - 1;
            const int excl = __shfl(inc - cnt, first, 64);
            b = b0 + first;
            s = item - base - excl;
            return true;
        }
        base += tot;
    }
    return false;
}

// Page ids of one tile's rows for the lanes' K row and V pieces (PAGED),
// already resolved into [0, num_pages) (the host limits pools to 2^31 pages).
template <int KS>
struct TilePages {
    int32_t k;
    int32_t v[KS / 2];
};

// When a page holds at least 16 rows a 16-row tile touches at most two pages:
// the wave reads their ids once per tile (p0 for the page of the tile's first
// row, p1 for the next one), and each lane places its row from the first row's
// slot with one compare instead of a division per row.  r0c is the tile's
// first row clamped to the sequence's last row, as every row is.
struct TilePair {
    int32_t p0, p1;
    int r0c, slot0;
};

// Paged variant of load_tile: the same lane/piece mapping, each row's base
// taken from its resolved page id, so every address is inside the pool
// whatever the table holds.
template <int KS>
__device__ __forceinline__ void load_tile_paged(TileRegs<KS>& t, const TilePages<KS>& pg, const Seg& sg,
                                                const uint16_t* kpage, const uint16_t* vpage, int r0,
                                                int last_valid, int span_k, int span_v, int col, int grp, int lane) {
    constexpr int VT = KS;
    auto row_base = [&](int32_t pid, int row) -> int64_t {
        const int r = min(row, last_valid);
        const int slot = sg.slots_shift >= 0 ? (r & (sg.slots - 1)) : r % sg.slots;
        return pid * sg.page_stride + (int64_t)slot * sg.k_sn;
    };
    {
        const uint16_t* src = kpage + row_base(pg.k, r0 + col);
#pragma unroll
        for (int c = 0; c < KS / 2; ++c) {
            const int kk = 32 * c + 8 * grp;
            t.k[c] = tile_load<false>(src + (kk + 8 <= span_k ? kk : 0));
        }
    }
#pragma unroll
    for (int c = 0; c < VT / 2; ++c) {
        const int p = 64 * c + lane;
        const int row = r0 + p / (2 * VT);
        const int pc = p % (2 * VT);
        const uint16_t* src = vpage + row_base(pg.v[c], row) + (8 * pc + 8 <= span_v ? 8 * pc : 0);
        t.v[c] = tile_load<false>(src);
    }
}

// load_tile_paged with the tile's two pages: the same lane/piece mapping and
// clamping (a lane's clamped row is at most 15 rows past r0c).
template <int KS>
__device__ __forceinline__ void load_tile_pair(TileRegs<KS>& t, const TilePair& tp, const Seg& sg,
                                               const uint16_t* kpage, const uint16_t* vpage, int r0,
                                               int last_valid, int span_k, int span_v, int col, int grp, int lane) {
    constexpr int VT = KS;
    auto row_base = [&](int row) -> int64_t {
        int slot = tp.slot0 + (min(row, last_valid) - tp.r0c);
        const bool next = slot >= sg.slots;
        slot = next ? slot - sg.slots : slot;
        return (int64_t)(next ? tp.p1 : tp.p0) * sg.page_stride + (int64_t)slot * sg.k_sn;
    };
    {
        const uint16_t* src = kpage + row_base(r0 + col);
#pragma unroll
        for (int c = 0; c < KS / 2; ++c) {
            const int kk = 32 * c + 8 * grp;
            t.k[c] = tile_load<false>(src + (kk + 8 <= span_k ? kk : 0));
        }
    }
#pragma unroll
    for (int c = 0; c < VT / 2; ++c) {
        const int p = 64 * c + lane;
        const int row = r0 + p / (2 * VT);
        const int pc = p % (2 * VT);
        const uint16_t* src = vpage + row_base(row) + (8 * pc + 8 <= span_v ? 8 * pc : 0);
        t.v[c] = tile_load<false>(src);
    }
}

// Fused query operands (FQ instances): the RoPE table rows of a wave's query
// positions pass through the wave's own LDS (its V-tile buffer, idle until the
// first tile is consumed), so a lane holds one 16-byte piece of them instead
// of the 64 table values its rotation reads.  Lane l loads elements
// 4 (l % 32) + [0, 4) of the cos (l < 32) or sin (l >= 32) row of query slot
// lq' < Lq <= 2; the wave's LDS holds row lq' at [256 lq', 256 lq' + 256)
// floats, cos then sin.
struct RopeStage {
    u32x4 v[2];                                      // table bits (ext vector: kept in registers)
};

// Both slots are loaded and stored whatever Lq is (slot 1 repeats slot 0 when
// Lq is 1), and without tables (a query given rotated) the loads read the
// query's first 16 bytes, unused: a load under a run-time condition would be
// kept in scratch memory.
__device__ __forceinline__ void rope_stage_load(RopeStage& st, const QRope& qr, int b, int Lq, int lane) {
    const bool tables = qr.cos != nullptr;
    const float* tab = !tables ? reinterpret_cast<const float*>(qr.q) : ((lane >> 5) ? qr.sin : qr.cos);
    const int e = tables ? 4 * (lane & 31) : 0;
#pragma unroll
    for (int l = 0; l < 2; ++l) {
        const int64_t row = tables ? qrope_row(qr, b, l < Lq ? l : 0, Lq) : 0;
        st.v[l] = *reinterpret_cast<const u32x4*>(tab + row * 128 + e);
    }
}

__device__ __forceinline__ void rope_stage_store(const RopeStage& st, float* rows, int lane) {
#pragma unroll
    for (int l = 0; l < 2; ++l)
        *reinterpret_cast<u32x4*>(rows + 256 * l + 128 * (lane >> 5) + 4 * (lane & 31)) = st.v[l];
}

// rope_operand with the table row read from LDS (cos at row[0, 128), sin at
// row[128, 256)): the same values and the same bf16 operation order, one
// rotate-half pair of pieces (c, c + 2) at a time so that a lane holds 32 of
// the table values at once instead of 64.
__device__ __forceinline__ void rope_operand_lds(u32x4 (&x)[4], const float* row, int grp) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        float v[2][8];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[h][2 * e] = bf16_to_f32(x[c + 2 * h][e] & 0xffffu);
                v[h][2 * e + 1] = bf16_to_f32(x[c + 2 * h][e] >> 16);
            }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int d0 = 32 * (c + 2 * h) + 8 * grp;
            const float4 c0 = *reinterpret_cast<const float4*>(row + d0);
            const float4 c1 = *reinterpret_cast<const float4*>(row + d0 + 4);
            const float4 s0 = *reinterpret_cast<const float4*>(row + 128 + d0);
            const float4 s1 = *reinterpret_cast<const float4*>(row + 128 + d0 + 4);
            const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
            uint32_t w[4];
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                float o[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const float partner = h == 0 ? -v[1][i + u] : v[0][i + u];
                    o[u] = round_bf16_hw(v[h][i + u] * round_bf16_hw(cv[i + u])) +
                           round_bf16_hw(partner * round_bf16_hw(sv[i + u]));
                }
                w[i / 2] = pack_bf16(o[0], o[1]);
            }
            x[c + 2 * h] = u32x4{w[0], w[1], w[2], w[3]};
        }
    }
}

// The absorption of a latent wave's rotated query rows into its heads' U_K
// (what the prologue writes to the workspace, bit for bit, made in place):
// chunk c of the operand (tile columns 32c + [0, 32)) comes from two MFMA
// blocks t, and block t's row 4g + e is tile column 32c + 8g + 4t + e, so lane
// (col, grp) receives exactly the eight columns 32c + 8grp + [0, 8) it feeds
// the score MFMA.  A row's head and latent dimension follow from its tile
// column (per-head blocks of blk_k columns from the wave's first block); rows
// past the span read row 0 of the first block and meet a zero select.  Each
// U_K^T row is read as the prologue reads it (k-steps of 32 in order), so each
// output element is the same MFMA dot product.  The rows are loaded first
// (absorb_load) and used once the query is rotated (absorb_apply), so that
// the caller can issue other loads in between.
template <int KS>
struct AbsorbRows {
    u32x4 a[KS / 2][2][4];
};

template <int KS>
__device__ __forceinline__ void absorb_load(AbsorbRows<KS>& u, const QAbsorb& qa, int col, int grp, int first_blk,
                                            int blk_k, int span_k) {
#pragma unroll
    for (int c = 0; c < KS / 2; ++c)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int xcol = 32 * c + 8 * (col >> 2) + 4 * t + (col & 3);
            const bool in = xcol < span_k;
            const int head = first_blk + (in ? xcol / blk_k : 0);
            const int dim = in ? xcol % blk_k : 0;
            const uint16_t* urow = qa.ut + ((int64_t)head * qa.wq + dim) * 128 + 8 * grp;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) u.a[c][t][kk] = *reinterpret_cast<const u32x4*>(urow + 32 * kk);
        }
}

template <int KS>
__device__ __forceinline__ void absorb_apply(u32x4 (&qv)[KS / 2], const AbsorbRows<KS>& u, const u32x4 (&x)[4],
                                             int col, int span_k) {
#pragma unroll
    for (int c = 0; c < KS / 2; ++c) {
        v4f acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const bool in = 32 * c + 8 * (col >> 2) + 4 * t + (col & 3) < span_k;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) acc[t] = mfma32(zero_unless(in, u.a[c][t][kk]), x[kk], acc[t]);
        }
        qv[c] = u32x4{pack_bf16(acc[0][0], acc[0][1]), pack_bf16(acc[0][2], acc[0][3]),
                      pack_bf16(acc[1][0], acc[1][1]), pack_bf16(acc[1][2], acc[1][3])};
    }
}

// q . b_k of one query row: lane (col, grp) holds elements 32c + 8grp + [0, 8)
// of the rotated row and of its KV head's bias; the lane groups' sums meet by
// two swaps.  The prologue and the split kernel's raw waves both take the
// shift from here, so it is the same bits whichever of them runs.
__device__ __forceinline__ float kbias_dot(const u32x4 (&q)[4], const u32x4 (&bk)[4]) {
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            dot += bf16_to_f32(q[c][e] & 0xffffu) * bf16_to_f32(bk[c][e] & 0xffffu);
            dot += bf16_to_f32(q[c][e] >> 16) * bf16_to_f32(bk[c][e] >> 16);
        }
    dot += shfl_xor_f(dot, 16);
    dot += shfl_xor_f(dot, 32);
    return dot;
}

// A workgroup owns (batch b, group of 4 tile slots, key split s); a slot is a
// (KV head, column tile) pair and each wave takes one slot.  The four waves
// therefore stream the same keys' rows at the same time (whole DRAM pages),
// never exchange data, and write their own partials.
// PAGED: 0 dense rows, 1 rows through per-lane page ids, 2 rows through the
// tile's two pages (pages of at least 16 rows).
template <int KS, int DEPTH, int PAGED = 0, int SEG2 = 0, int RAWPG = 0, int FQ = 0>
__device__ __forceinline__ void split_segment(const Seg& sg, int w, int B, int Lq, int Hq,
                                              float scale_log2, char* lds, const SegRows2* two = nullptr,
                                              const RawPagesArg* rawp = nullptr, const QRope* qr = nullptr,
                                              const QAbsorb* qa = nullptr, const QShift* qs = nullptr) {
    static_assert(!FQ || KS <= 8, "fused query operands are built for tiles up to 128 columns");
    constexpr int VT = KS;                   // V tiles of 16 (same width budget as K)
    constexpr int RS = SplitLds<KS>::RS;
    const int lane = threadIdx.x & 63;
    // Everything derived from the wave index is wave-uniform: scalar registers,
    // and scalar branches for the tile loop (a lane-divergent exit would let
    // the last tile's prefetch reach the loop header and force a full wait
    // for outstanding loads at the top of every iteration).
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15;
    const int grp = lane >> 4;

    // Wave items: (batch, split, slot) with the slot fastest, kWaves per
    // workgroup -- the waves of a workgroup read the same key rows (different
    // heads) of one split, or of consecutive splits when a split has fewer
    // slots than the workgroup has waves.
    const int slots = sg.hk * sg.tiles;
    const int64_t item = (int64_t)w * kWaves + wave;
    const int slot = (int)(item % slots);
    const int64_t split_item = item / slots;
    int s, b;
    if (sg.compact) {
        // wave-uniform: every lane of the wave has the same split_item
        if (!locate_split((int)split_item, sg.seqlens, B, sg.n, sg.rows_per_split, b, s)) return;
        b = __builtin_amdgcn_readfirstlane(b);
        s = __builtin_amdgcn_readfirstlane(s);
    } else {
        s = (int)(split_item % sg.splits);
        b = (int)(split_item / sg.splits);
        if (b >= B) return;                  // waves never synchronise, so an idle one may leave
    }
    const int h = slot / sg.tiles;
    const int t = slot % sg.tiles;

    const int P = Lq * sg.g;
    const int p0 = t * sg.cols;
    const int pl = p0 + col;
    const bool colv = col < sg.cols && pl < P;
    const int jj = colv ? pl / Lq : 0;
    const int lq = colv ? pl % Lq : 0;
    const int j = h * sg.g + jj;

    int k_off = 0, v_off = 0, first_blk = 0;
    int span_k = sg.wk, span_v = sg.wv;
    int own_k_lo = 0, own_k_w = sg.wk, own_v_lo = 0;
    if (sg.blk_heads) {
        const int pend = (P < p0 + sg.cols ? P : p0 + sg.cols) - 1;
        first_blk = (p0 / Lq) / sg.blk_heads;
        const int last_blk = (pend / Lq) / sg.blk_heads;
        k_off = first_blk * sg.blk_k;
        v_off = first_blk * sg.blk_v;
        span_k = (last_blk - first_blk + 1) * sg.blk_k;
        span_v = (last_blk - first_blk + 1) * sg.blk_v;
        own_k_lo = (jj / sg.blk_heads) * sg.blk_k - k_off;
        own_k_w = sg.blk_k;
        own_v_lo = (jj / sg.blk_heads) * sg.blk_v - v_off;
    }
    if (k_off + span_k > sg.wk) span_k = sg.wk - k_off;
    if (v_off + span_v > sg.wv) span_v = sg.wv - v_off;

    int Nb = sg.n;
    if (sg.seqlens) {
        const int sl = sg.seqlens[b];
        Nb = sl < 0 ? 0 : (sl < sg.n ? sl : sg.n);
    }
    const int lim = !colv ? 0 : (sg.causal ? Nb - Lq + lq + 1 : Nb);
    // Striped splits: the sequence's 16-row tiles are dealt round-robin over
    // its ceil(Nb / rows_per_split) non-empty splits, so split s takes tiles
    // s, s + S, s + 2S, ...  The workgroups resident at one time then read one
    // contiguous window of each sequence's rows instead of a separate stream
    // per split (far fewer DRAM rows open per channel); a split still owns a
    // fixed tile set, so results do not depend on scheduling.
    const int S = max(1, (Nb + sg.rows_per_split - 1) / sg.rows_per_split);
    const int tiles_b = (Nb + 15) / 16;
    const int ntile = s < S ? (tiles_b - s + S - 1) / S : 0;   // S <= tiles_b; splits past S are empty
    const int r_begin = 16 * s;               // first row of the split's first tile
    const int r_step = 16 * S;
    const int r_end = Nb;
    const int vis = min(lim, r_end);
    const int last_row = sg.n - 1;
    // The splits of sequence b start their walk over their tiles at tile
    // b * ntile / B and wrap, so the B sequences' concurrent reads sit at
    // staggered offsets of their rows instead of advancing in step (measured
    // 1-1.5 us faster a rank-32 layer at one workgroup a CU).
    const int phase = ntile > 0 ? (int)(((int64_t)b * ntile) / B) : 0;
    auto tile_row = [&](int it) {
        const int k = it + phase;
        return r_begin + (k >= ntile ? k - ntile : k) * r_step;
    };

    const uint16_t* kbase = sg.k + (int64_t)b * sg.k_sb + (int64_t)h * sg.k_sh + k_off;
    const uint16_t* vbase = sg.v + (int64_t)b * sg.v_sb + (int64_t)h * sg.v_sh + v_off;

    bool bad = false;
    auto fetch = [&](TileRegs<KS>& tr, int it) {
        const int r0 = it < ntile ? tile_row(it) : r_begin;
        if constexpr (RAWPG) {
            const int64_t* tb = rawp->table + (int64_t)b * rawp->t_sb;
            const int lv = Nb > 0 ? Nb - 1 : 0;
            load_tile<KS>(tr, RawPageRows{kbase, tb, rawp->blk_stride, sg.k_sn, rawp->num_blocks, rawp->block_shift, lv, &bad},
                          RawPageRows{vbase, tb, rawp->blk_stride, sg.v_sn, rawp->num_blocks, rawp->block_shift, lv, &bad},
                          r0, last_row, span_k, span_v, col, grp, lane);
        } else if constexpr (SEG2) {
            const uint16_t* k2 = two->k2 + (int64_t)b * two->k2_sb + (int64_t)h * sg.k_sh + k_off;
            const uint16_t* v2 = two->v2 + (int64_t)b * two->v2_sb + (int64_t)h * sg.v_sh + v_off;
            load_tile<KS>(tr, TwoRows{kbase, sg.k_sn, k2, two->k2_sn, two->n1},
                          TwoRows{vbase, sg.v_sn, v2, two->v2_sn, two->n1}, r0, last_row, span_k, span_v, col, grp,
                          lane);
        } else {
            load_tile<KS>(tr, OneRows{kbase, sg.k_sn}, OneRows{vbase, sg.v_sn}, r0, last_row, span_k, span_v, col,
                          grp, lane);
        }
    };
    // Paged rows: the page ids of a tile are loaded two tiles ahead of its
    // data.  An entry outside the pool that a row of the sequence needs sets
    // `bad` (reported once the split is done) and is read as page 0.
    const int64_t* tab = PAGED ? sg.table + (int64_t)b * sg.t_sb : nullptr;
    const int last_valid = Nb > 0 ? Nb - 1 : 0;
    auto page_of = [&](int row, bool used) -> int32_t {
        const int r = min(row, last_valid);
        const int64_t p = table_page(tab[sg.slots_shift >= 0 ? (r >> sg.slots_shift) : r / sg.slots], sg.num_pages);
        bad |= used && p < 0;
        return p < 0 ? 0 : (int32_t)p;
    };
    const int last_page = PAGED == 2 ? last_valid / sg.slots : 0;
    auto load_pages = [&](auto& pg, int it) {
        const bool act = it < ntile;
        const int r0 = act ? tile_row(it) : r_begin;
        if constexpr (PAGED == 2) {
            const int r0c = __builtin_amdgcn_readfirstlane(min(r0, last_valid));
            const int pi = __builtin_amdgcn_readfirstlane(r0c / sg.slots);
            const int64_t a = table_page(tab[pi], sg.num_pages);
            const int64_t c = table_page(tab[min(pi + 1, last_page)], sg.num_pages);
            pg.r0c = r0c;
            pg.slot0 = r0c - pi * sg.slots;
            // the tile's valid rows reach the next page when its last one does
            const bool crosses = min(r0 + 15, last_valid) - r0c + pg.slot0 >= sg.slots;
            bad |= act && (a < 0 || (crosses && c < 0));
            pg.p0 = a < 0 ? 0 : (int32_t)a;
            pg.p1 = c < 0 ? 0 : (int32_t)c;
        } else {
            pg.k = page_of(r0 + col, act && r0 + col < r_end);
#pragma unroll
            for (int c = 0; c < VT / 2; ++c) {
                const int row = r0 + (64 * c + lane) / (2 * VT);
                pg.v[c] = page_of(row, act && row < r_end);
            }
        }
    };
    auto fetch_paged = [&](TileRegs<KS>& tr, const auto& pg, int it) {
        const int r0 = it < ntile ? tile_row(it) : r_begin;
        if constexpr (PAGED == 2)
            load_tile_pair<KS>(tr, pg, sg, kbase, vbase, r0, last_valid, span_k, span_v, col, grp, lane);
        else
            load_tile_paged<KS>(tr, pg, sg, kbase, vbase, r0, last_valid, span_k, span_v, col, grp, lane);
    };
    using PageIds = std::conditional_t<PAGED == 2, TilePair, TilePages<KS>>;
    PageIds pcur, poth;
    uint16_t* vbuf = reinterpret_cast<uint16_t*>(lds) + wave * 2 * 16 * RS;
    // FQ: the query rows and their RoPE table rows go out first, so that
    // waiting for them does not wait for the first tile (loads complete in
    // issue order); the first tile follows at once and is in flight while the
    // rotation runs.  qa null: the raw segment.
    const bool fq_rot = FQ && qr->cos;
    RopeStage rst;
    u32x4 fx[4];
    if constexpr (FQ) {
        rope_stage_load(rst, *qr, b, Lq, lane);
        const uint16_t* q0 = qr->q + (int64_t)b * qr->q_sb + (int64_t)lq * qr->q_sl + (int64_t)j * qr->q_sh + 8 * grp;
#pragma unroll
        for (int c = 0; c < 4; ++c) fx[c] = *reinterpret_cast<const u32x4*>(q0 + 32 * c);
    }
    // First tile in flight before the query operand is fetched.
    TileRegs<KS> cur;
    if constexpr (PAGED) {
        load_pages(pcur, 0);
        load_pages(poth, 1);
        fetch_paged(cur, pcur, 0);
        load_pages(pcur, 2);
    } else {
        fetch(cur, 0);
    }

    // Query operand (B of the score MFMA), same k permutation as the K tile:
    // step 2c+e holds elements 32c + 8*grp + 4e + [0,4).
    // A query given as is (QRope::q set) is rotated here; a null QRope::q, or
    // no QRope, means the segment's q holds prepared operands.  The pointers
    // are never selected at run time (that would put the kernel arguments in
    // scratch memory), only the fields they point at are tested.
    const bool rot = !FQ && qr && qr->q;
    const bool absorb = rot && qa && qa->ut;
    u32x4 qv[KS / 2];
    if constexpr (FQ) {
        float* rows = reinterpret_cast<float*>(vbuf);
        rope_stage_store(rst, rows, lane);
        if (fq_rot) {
            wave_lds_fence();
#pragma unroll
            for (int c = 0; c < 4; ++c) fx[c] = zero_unless(colv, fx[c]);
            rope_operand_lds(fx, rows + 256 * lq, grp);
            wave_lds_fence();
        }
        if (qa) {
            // U_K^T rows once the query is rotated (few registers are live
            // then); the absorption waits for them and, loads completing in
            // issue order, for the first tile.  The second tile goes out after
            // the absorption: issued before it, the second tile or the U_K^T
            // rows left too few registers for the other (spills) or made the
            // absorption wait for both tiles (C1 ranks 16/32/48: 18.7 / 27.1 /
            // 41.7 us a launch this way; 18.9 / 28.1 / 43.2 with the second
            // tile before the U_K^T rows; 23-26 / 34-37 / 57 with the rows
            // first, spilling).
            AbsorbRows<KS> u;
            absorb_load<KS>(u, *qa, col, grp, first_blk, sg.blk_k, span_k);
            absorb_apply<KS>(qv, u, fx, col, span_k);
#pragma unroll
            for (int c = 0; c < KS / 2; ++c) {
                const int kk = 32 * c + 8 * grp;
                const bool in = colv && kk >= own_k_lo && kk + 8 <= own_k_lo + own_k_w && kk + 8 <= span_k;
                qv[c] = zero_unless(in, qv[c]);
            }
        } else {
#pragma unroll
            for (int c = 0; c < KS / 2; ++c) qv[c] = zero_unless(colv, fx[c]);
        }
    } else if constexpr (KS == 8) {
        if (rot && !absorb) {
            // Rotated here from the query as given: the four pieces hold the
            // head's 128 elements, piece c's rotate-half partner is piece c ^ 2.
            const uint16_t* q0 = qr->q + (int64_t)b * qr->q_sb + (int64_t)lq * qr->q_sl + (int64_t)j * qr->q_sh;
#pragma unroll
            for (int c = 0; c < 4; ++c) qv[c] = *reinterpret_cast<const u32x4*>(q0 + 32 * c + 8 * grp);
            if (qr->cos) {
                RopeRow rr;
                const int64_t row = qrope_row(*qr, b, lq, Lq);
                load_rope_row(rr, qr->cos + row * 128, qr->sin + row * 128, grp);
                rope_operand(qv, rr);
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) qv[c] = zero_unless(colv, qv[c]);
        }
    }
    if (FQ) {
        // the operand is made above
    } else if (!(KS == 8 && rot)) {
        const uint16_t* qrow = sg.q + (int64_t)b * sg.q_sb + (int64_t)lq * sg.q_sl + (int64_t)j * sg.q_sh;
#pragma unroll
        for (int c = 0; c < KS / 2; ++c) {
            const int kk = 32 * c + 8 * grp;
            const bool in = colv && kk >= own_k_lo && kk + 8 <= own_k_lo + own_k_w && kk + 8 <= span_k;
            const int idx = in ? (sg.q_compact ? (kk - own_k_lo) : (k_off + kk)) : 0;
            qv[c] = zero_unless(in, *reinterpret_cast<const u32x4*>(qrow + idx));
        }
    }

    float m = kNegInf, lsum = 0.f;
    v4f acc[VT];
#pragma unroll
    for (int i = 0; i < VT; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};

    // One 16-key tile: V to LDS, scores, online softmax, P^T V^T.  The tile's
    // rows past the sequence were read from a clamped row: their scores are
    // masked below, and their V pieces are zeroed here so that a non-finite
    // value there cannot reach the product (0 * inf).  K pieces outside the
    // span meet zero query elements.
    auto consume = [&](const TileRegs<KS>& tile, int it) {
        const int r0 = tile_row(it);
        uint16_t* vb = vbuf + (it & 1) * 16 * RS;
#pragma unroll
        for (int c = 0; c < VT / 2; ++c) {
            const int p = 64 * c + lane;
            *reinterpret_cast<u32x4*>(vb + (p / (2 * VT)) * RS + 8 * (p % (2 * VT))) =
                zero_unless(r0 + p / (2 * VT) < r_end, tile.v[c]);
        }
        // Two independent accumulation chains halve the MFMA dependency latency.
        v4f sc0 = {0.f, 0.f, 0.f, 0.f}, sc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < KS / 2; ++c) {
            sc0 = mfma16(as_v4s(tile.k[c].x, tile.k[c].y), as_v4s(qv[c].x, qv[c].y), sc0);
            sc1 = mfma16(as_v4s(tile.k[c].z, tile.k[c].w), as_v4s(qv[c].z, qv[c].w), sc1);
        }
        const v4f sc = sc0 + sc1;
        // raw scores (the scale is positive: it is applied to the maximum
        // and inside the exponent's FMA)
        float sv[4];
        float tmax = kNegInf;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = r0 + 4 * grp + i;
            const float x = n < vis ? sc[i] : kNegInf;
            sv[i] = x;
            tmax = fmaxf(tmax, x);
        }
        tmax = rows_max(tmax) * scale_log2;
        const float mnew = fmaxf(m, tmax);
        const float mref = mnew == kNegInf ? 0.f : mnew;
        const float alpha = fast_exp2(m - mref);
        float p[4];
        float psum = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            p[i] = fast_exp2(fmaf(sv[i], scale_log2, -mref));
            psum += p[i];
        }
        lsum = lsum * alpha + psum;
        m = mnew;
#pragma unroll
        for (int i = 0; i < VT; ++i) acc[i] *= alpha;
        const v4s pb = as_v4s(pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3]));
        wave_lds_fence();
#pragma unroll
        for (int u = 0; u < VT / 2; ++u) {
            uint32_t w4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                w4[i] = *reinterpret_cast<const uint32_t*>(vb + (4 * grp + i) * RS + 32 * u + 2 * col);
            const v4s lo = as_v4s((w4[0] & 0xffffu) | (w4[1] << 16), (w4[2] & 0xffffu) | (w4[3] << 16));
            const v4s hi = as_v4s((w4[0] >> 16) | (w4[1] & 0xffff0000u), (w4[2] >> 16) | (w4[3] & 0xffff0000u));
            acc[2 * u] = mfma16(lo, pb, acc[2 * u]);
            acc[2 * u + 1] = mfma16(hi, pb, acc[2 * u + 1]);
        }
        wave_lds_fence();
    };

    // The tile loops run whole rounds of the register ring with no exit inside
    // a round, then finish the last tiles outside the loop: an exit between
    // two tiles of a round would reach the loop header with that round's
    // prefetch outstanding and force a full wait for loads there.  No tile
    // past the split's last one is fetched.
    if constexpr (PAGED) {
        TileRegs<KS> other;
        int it = 0;
        for (; it + 2 < ntile; it += 2) {
            fetch_paged(other, poth, it + 1);
            load_pages(poth, it + 3);
            consume(cur, it);
            fetch_paged(cur, pcur, it + 2);
            load_pages(pcur, it + 4);
            consume(other, it + 1);
        }
        if (it < ntile) {
            if (it + 1 < ntile) fetch_paged(other, poth, it + 1);
            consume(cur, it);
            if (it + 1 < ntile) consume(other, it + 1);
        }
    } else if constexpr (DEPTH > 1) {
        // A ring of DEPTH register tiles: the loads of the next DEPTH - 1
        // tiles stay in flight while a tile is consumed (the ring index is
        // static in the unrolled body, so no register copies).  At the top of
        // a round ring[d] holds tile it + d for d < DEPTH - 1.
        TileRegs<KS> ring[DEPTH];
        ring[0] = cur;
#pragma unroll
        for (int d = 1; d < DEPTH - 1; ++d) fetch(ring[d], d);
        int it = 0;
        for (; it + 2 * DEPTH - 2 < ntile; it += DEPTH) {
#pragma unroll
            for (int d = 0; d < DEPTH; ++d) {
                fetch(ring[(d + DEPTH - 1) % DEPTH], it + d + DEPTH - 1);
                consume(ring[d], it + d);
            }
        }
        // at most 2 * DEPTH - 2 tiles are left
#pragma unroll
        for (int d = 0; d < 2 * DEPTH - 2; ++d) {
            if (it + d >= ntile) break;
            if (it + d + DEPTH - 1 < ntile) fetch(ring[(d + DEPTH - 1) % DEPTH], it + d + DEPTH - 1);
            consume(ring[d % DEPTH], it + d);
        }
    } else {
        for (int it = 0; it < ntile; ++it) {
            if (it) fetch(cur, it);
            consume(cur, it);
        }
    }

    if constexpr (PAGED || RAWPG) {
        if (bad) report_bad_page(sg.status);
    }
    // Column sums: every lane group holds a quarter of the keys.
    lsum = rows_sum(lsum);
    if constexpr (FQ && KS == 8) {
        // Raw waves of split 0 with a latent K bias: the row's LSE shift, from
        // the operand rotated above.  Loaded after the tiles, when the raw
        // wave's registers are free; raw work drains long before the latent.
        if (qs && qs->bias && s == 0) {
            const uint16_t* bk = qs->bias + (int64_t)h * 128 + 8 * grp;
            u32x4 kb[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) kb[c] = *reinterpret_cast<const u32x4*>(bk + 32 * c);
            const float dot = kbias_dot(qv, kb);
            if (colv && grp == 0) qs->shift[(int64_t)b * Hq * Lq + j * Lq + lq] = dot * qs->scale;
        }
    }
    if (!colv) return;
    const int pr = j * Lq + lq;
    const int64_t slot_out = ((int64_t)b * Hq * Lq + pr) * sg.splits + s;
    if (grp == 0) {
        sg.part_ml[slot_out * 2] = m;
        sg.part_ml[slot_out * 2 + 1] = lsum;
    }
    // Lane holds v = 32u + 8*grp + 2i + e in acc[2u+e][i]: eight consecutive
    // values per u, all inside or all outside the column's own V slice.
    float* dst = sg.part_acc + slot_out * sg.wown;
#pragma unroll
    for (int u = 0; u < VT / 2; ++u) {
        const int v0 = 32 * u + 8 * grp;
        const int o = v0 - own_v_lo;
        if (o >= 0 && o + 8 <= sg.wown && v0 + 8 <= span_v) {
            float4* d4 = reinterpret_cast<float4*>(dst + o);
            d4[0] = make_float4(acc[2 * u][0], acc[2 * u + 1][0], acc[2 * u][1], acc[2 * u + 1][1]);
            d4[1] = make_float4(acc[2 * u][2], acc[2 * u + 1][2], acc[2 * u][3], acc[2 * u + 1][3]);
        }
    }
    (void)first_blk;
}

// Segment 0 (KA, pipelined) is the bulk segment.  The optional segment 1 (KB,
// single register set) is short work -- the raw rows of the fused decode in
// 32-key splits -- and is placed first in the grid so it drains while the bulk
// workgroups stream (last in the grid for paged rows, see split_kernel).
template <int KA>
struct SplitWaves {
    static constexpr int value = KA <= 4 ? 4 : (KA <= 6 ? 3 : (KA <= 12 ? 2 : 1));
};

// Register tiles in flight per latent wave (2 = ping-pong).
template <int KA>
struct SplitDepth {
    static constexpr int value = 2;
};

// FQ: the query operands are made here (QRope and QAbsorb of SplitParams),
// no prologue launch precedes the kernel.
template <int KA, int KB, int PAGED = 0, int SEG2 = 0, int RAWPG = 0, int FQ = 0>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(SplitWaves<KA>::value)))
split_kernel(SplitParams prm) {
    constexpr int LA = SplitLds<KA>::bytes;
    constexpr int LB = KB > 0 ? SplitLds<(KB > 0 ? KB : 2)>::bytes : 0;
    __shared__ __attribute__((aligned(16))) char lds[LA > LB ? LA : LB];
    int w = blockIdx.x;
    if constexpr (KB > 0 && PAGED) {
        // Paged rows: the beacon workgroups come first, so every compact item
        // starts at launch and the short raw workgroups fill the slots left
        // over and those of the grid's empty items (64 sequences of U[1K,
        // 128K] tokens: 134.6 against 145.7 us with the raw workgroups first,
        // which held half the beacon items back until they drained).
        if (w >= prm.seg[0].nwg) {
            split_segment<KB, 1, 0, 0, RAWPG, FQ>(prm.seg[1], w - prm.seg[0].nwg, prm.B, prm.Lq, prm.Hq,
                                                  prm.scale_log2, lds, nullptr, &prm.rawp, FQ ? &prm.qrope : nullptr,
                                                  nullptr, FQ ? &prm.kshift : nullptr);
            return;
        }
    } else if constexpr (KB > 0) {
        if (w < prm.seg[1].nwg) {
            split_segment<KB, 1, 0, 0, RAWPG, FQ>(prm.seg[1], w, prm.B, prm.Lq, prm.Hq, prm.scale_log2, lds, nullptr,
                                                  &prm.rawp, FQ ? &prm.qrope : nullptr, nullptr,
                                                  FQ ? &prm.kshift : nullptr);
            return;
        }
        w -= prm.seg[1].nwg;
    }
    split_segment<KA, SplitDepth<KA>::value, PAGED, SEG2, 0, FQ>(prm.seg[0], w, prm.B, prm.Lq, prm.Hq, prm.scale_log2,
                                                                 lds, &prm.two, nullptr, FQ ? &prm.qrope : nullptr,
                                                                 FQ ? &prm.absorb : nullptr);
}

// ---------------------------------------------------------------------------
// fused reconstruction decode: beacon K rebuilt and rotated per 16-key tile
// ---------------------------------------------------------------------------

// Beacon segment of the reconstruction decode with block-diagonal bases.  A
// wavefront owns (b, KV head h, key split) with the head's g*Lq query rows as
// MFMA columns.  Per 16-key tile it rebuilds K^T[d, n] = U_K[h*128 + d, :] .
// l_k[n, h-slice] on the MFMA with U_K's tile held in registers (lane (n, grp)
// ends with d = 16t + 4grp + i, so d and d + 64 share a lane), adds the bias,
// rounds to bf16 and rotates at the beacon's position with the reference's
// bf16 steps -- the same bits the up-projection kernel writes -- and feeds the
// result straight in as the A operand of the score MFMA (ROPE = 1).  ROPE = 2
// adds the bias and rotates in fp32 and rounds once into the operand: about a
// third of the per-tile VALU work, keys within one bf16 rounding of the exact
// rotation (the reference's steps round five times).  V stays latent: the
// P.V MFMA accumulates the rv-wide latent sum that the combine lifts through
// W_V.  RoPE reads (bf16 cos | bf16 sin << 16) pairs prepared once per table,
// only the first half of each row: the fused route is taken for rotate-half
// tables whose rows repeat their first half (cos[d] = cos[d + 64]), which the
// caller checks once per table.
struct ReconSeg {
    const uint16_t* q; int64_t q_sb, q_sl, q_sh;        // rotated queries [B, Lq, Hq, 128]
    const uint16_t* lk; int64_t lk_sb, lk_sn;           // latent K rows, head h at [h*rk, (h+1)*rk)
    const uint16_t* lv; int64_t lv_sb, lv_sn;           // latent V rows, head h at [h*rv, (h+1)*rv)
    const uint16_t* w; const uint16_t* bias; int64_t w_ld;   // U_K [Hkv*128, Rk] (nn.Linear), bias or null
    const uint32_t* pairs; int64_t rope_rows;           // [rope_rows][128] or null (no beacon RoPE)
    const int64_t* pos; int64_t pos_sb;                 // beacon positions [B, Nl]
    const int32_t* seqlens;
    int n, hk, g, causal;
    int splits, rows_per_split, nwg;
    float* part_ml; float* part_acc;                    // partials, rv wide
    QRope qr;                                           // q null: q above holds rotated rows
};

// One 16-key tile of latent rows in registers, with the key position of the
// lane's row (its RoPE pairs are fetched two tiles before the tile is used).
template <int KSR, int VL>
struct ReconTile {
    // latent K pieces of the lane's key (B operand of the rebuild): 32 latent
    // dims a 16x16x32 MFMA, then 16 a 16x16x16 one when KSR is odd
    u32x4 kq[KSR / 2 > 0 ? KSR / 2 : 1];
    u32x2 kr;
    u32x4 v[VL];          // latent V pieces on their way to LDS
    int64_t pos;
};

// Tiles in flight per wavefront: the rebuild's arithmetic is long enough that
// two tiles do not cover the memory latency at two waves per SIMD.
constexpr int kReconRing = 4;

// Instances whose two tiles in flight (the software pipeline of recon_segment)
// fit the register budget without spilling; the others run each tile's two
// phases back to back.
template <int KSR, int VL>
struct ReconPipeline {
    static constexpr bool value = (KSR <= 2 && VL == 1) || (KSR == 1 && VL == 2);
};

template <int KSR, int VL, int ROPE>
__device__ __forceinline__ void recon_segment(const ReconSeg& sg, int w, int Lq, int Hq, float scale_log2,
                                              char* lds) {
    constexpr int D = 128;
    constexpr int RV = 32 * VL;
    constexpr int RSV = RV + 8;
    constexpr int PPR = RV / 8;                        // 16-byte V pieces per row
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int groups = (sg.hk + kWaves - 1) / kWaves;
    const int s = w % sg.splits;
    const int rem = w / sg.splits;
    const int b = rem / groups;
    const int h = (rem % groups) * kWaves + wave;
    if (h >= sg.hk) return;
    const int P = Lq * sg.g;
    const bool colv = col < P;
    const int jj = colv ? col / Lq : 0, lq = colv ? col % Lq : 0;
    const int j = h * sg.g + jj;
    const int rk = 16 * KSR;

    int Nb = sg.n;
    if (sg.seqlens) {
        const int sl = sg.seqlens[b];
        Nb = sl < 0 ? 0 : (sl < sg.n ? sl : sg.n);
    }
    const int lim = !colv ? 0 : (sg.causal ? Nb - Lq + lq + 1 : Nb);
    // Striped splits: the sequence's 16-row tiles are dealt round-robin over
    // its ceil(Nb / rows_per_split) non-empty splits, so split s takes tiles
    // s, s + S, s + 2S, ...  The workgroups resident at one time then read one
    // contiguous window of each sequence's rows instead of a separate stream
    // per split (far fewer DRAM rows open per channel); a split still owns a
    // fixed tile set, so results do not depend on scheduling.
    const int S = max(1, (Nb + sg.rows_per_split - 1) / sg.rows_per_split);
    const int tiles_b = (Nb + 15) / 16;
    const int ntile = s < S ? (tiles_b - s + S - 1) / S : 0;   // S <= tiles_b; splits past S are empty
    const int r_begin = 16 * s;               // first row of the split's first tile
    const int r_step = 16 * S;
    const int r_end = Nb;
    const int vis = min(lim, r_end);
    const int last_row = sg.n - 1;

    constexpr int KP = KSR / 2, KO = KSR & 1;         // 32-deep rebuild steps, then a 16-deep one
    const uint16_t* kbase = sg.lk + (int64_t)b * sg.lk_sb + (int64_t)h * rk;
    const uint16_t* vbase = sg.lv + (int64_t)b * sg.lv_sb + (int64_t)h * RV;
    const int64_t* pbase = ROPE ? sg.pos + (int64_t)b * sg.pos_sb : nullptr;

    // Raw loads only (clamped in-bounds addresses, no selects on the data), so
    // nothing waits for them before the tile is consumed: keys outside the
    // split are masked in the scores and their V rows are zeroed on the way
    // to LDS, where the tile is used.
    auto fetch = [&](ReconTile<KSR, VL>& t, int it) {
        const int r0 = it < ntile ? r_begin + it * r_step : r_begin;
        const uint16_t* src = kbase + (int64_t)min(r0 + col, last_row) * sg.lk_sn;
#pragma unroll
        for (int m = 0; m < KP; ++m) t.kq[m] = *reinterpret_cast<const u32x4*>(src + 32 * m + 8 * grp);
        if constexpr (KO) t.kr = *reinterpret_cast<const u32x2*>(src + 32 * KP + 4 * grp);
#pragma unroll
        for (int c = 0; c < VL; ++c) {
            const int p = 64 * c + lane;
            t.v[c] = *reinterpret_cast<const u32x4*>(vbase + (int64_t)min(r0 + p / PPR, last_row) * sg.lv_sn +
                                                     8 * (p % PPR));
        }
        if constexpr (ROPE) t.pos = pbase[min(r0 + col, last_row)];
    };
    // RoPE pairs of the lane's key for d = 16t + 4grp + [0, 4), t < 4 (rows
    // repeat their first half, so d + 64 uses the same pair).
    auto fetch_pairs = [&](u32x4 (&cs)[4], int64_t pos) {
        const uint32_t* src = sg.pairs + clamp_i64(pos, 0, sg.rope_rows - 1) * D + 4 * grp;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) cs[tt] = *reinterpret_cast<const u32x4*>(src + 16 * tt);
    };

    // U_K tile of this head (A operand of the rebuild) and the bias, once:
    // lane (col, grp) holds row 16tt + col at the latent dims its latent
    // pieces hold (32m + 8grp + [0, 8), then 32KP + 4grp + [0, 4)).
    u32x4 wq[8][KP > 0 ? KP : 1];
    u32x2 wr[8];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
        const uint16_t* wrow = sg.w + ((int64_t)h * D + 16 * tt + col) * sg.w_ld + h * rk;
#pragma unroll
        for (int m = 0; m < KP; ++m) wq[tt][m] = *reinterpret_cast<const u32x4*>(wrow + 32 * m + 8 * grp);
        if constexpr (KO) wr[tt] = *reinterpret_cast<const u32x2*>(wrow + 32 * KP + 4 * grp);
    }
    uint32_t bias2[8][2];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
        const u32x2 bb = sg.bias ? *reinterpret_cast<const u32x2*>(sg.bias + (int64_t)h * D + 16 * tt + 4 * grp)
                                 : u32x2{0u, 0u};
        bias2[tt][0] = bb.x;
        bias2[tt][1] = bb.y;
    }
    // ROPE == 2: the bias is the rebuild's initial accumulator (fp32), so no
    // per-tile bias arithmetic.
    v4f kinit[8];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt)
        kinit[tt] = ROPE == 2 ? v4f{lo_bf16(bias2[tt][0]), hi_bf16(bias2[tt][0]), lo_bf16(bias2[tt][1]),
                                    hi_bf16(bias2[tt][1])}
                              : v4f{0.f, 0.f, 0.f, 0.f};
    // Rotated query of the column (B operand of the scores): d = 16t + 4grp + [0, 4).
    u32x2 qop[8];
    if (sg.qr.q) {
        // Rotated here from the query as given, with the reference's bf16
        // steps (as rope_operand): element 16t + 4grp + e has its rotate-half
        // partner at t ^ 4 in the same lane.
        const uint16_t* qrow = sg.qr.q + (int64_t)b * sg.qr.q_sb + (int64_t)lq * sg.qr.q_sl + (int64_t)j * sg.qr.q_sh +
                               4 * grp;
        u32x2 x[8];
#pragma unroll
        for (int tt = 0; tt < 8; ++tt) x[tt] = *reinterpret_cast<const u32x2*>(qrow + 16 * tt);
        if (sg.qr.cos) {
            const int64_t row = qrope_row(sg.qr, b, lq, Lq);
            float4 cs[8], sn[8];
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) {
                cs[tt] = *reinterpret_cast<const float4*>(sg.qr.cos + row * 128 + 16 * tt + 4 * grp);
                sn[tt] = *reinterpret_cast<const float4*>(sg.qr.sin + row * 128 + 16 * tt + 4 * grp);
            }
            float v[8][4];
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) {
                v[tt][0] = lo_bf16(x[tt].x); v[tt][1] = hi_bf16(x[tt].x);
                v[tt][2] = lo_bf16(x[tt].y); v[tt][3] = hi_bf16(x[tt].y);
            }
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) {
                const float cv[4] = {cs[tt].x, cs[tt].y, cs[tt].z, cs[tt].w};
                const float sv[4] = {sn[tt].x, sn[tt].y, sn[tt].z, sn[tt].w};
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float partner = tt < 4 ? -v[tt ^ 4][e] : v[tt ^ 4][e];
                    o[e] = round_bf16_hw(v[tt][e] * round_bf16_hw(cv[e])) + round_bf16_hw(partner * round_bf16_hw(sv[e]));
                }
                x[tt] = u32x2{pack_bf16(o[0], o[1]), pack_bf16(o[2], o[3])};
            }
        }
#pragma unroll
        for (int tt = 0; tt < 8; ++tt) qop[tt] = u32x2{colv ? x[tt].x : 0u, colv ? x[tt].y : 0u};
    } else {
        const uint16_t* qrow = sg.q + (int64_t)b * sg.q_sb + (int64_t)lq * sg.q_sl + (int64_t)j * sg.q_sh + 4 * grp;
#pragma unroll
        for (int tt = 0; tt < 8; ++tt) {
            const u32x2 x = *reinterpret_cast<const u32x2*>(qrow + 16 * tt);
            qop[tt] = u32x2{colv ? x.x : 0u, colv ? x.y : 0u};
        }
    }

    ReconTile<KSR, VL> ring[kReconRing];
    u32x4 pairs[2][4];
#pragma unroll
    for (int u = 0; u < kReconRing; ++u) fetch(ring[u], u);
    if constexpr (ROPE) {
        fetch_pairs(pairs[0], ring[0].pos);
        fetch_pairs(pairs[1], ring[1].pos);
    }
    __builtin_amdgcn_sched_barrier(0);

    float m = kNegInf, lsum = 0.f;
    v4f acc[2 * VL];
#pragma unroll
    for (int i = 0; i < 2 * VL; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
    uint16_t* vbuf = reinterpret_cast<uint16_t*>(lds) + wave * 2 * 16 * RSV;

    // Phase A of tile it: its V rows into LDS buffer it & 1, its K rebuilt,
    // biased and rotated into the score MFMA's operand kop.
    auto phase_a = [&](const ReconTile<KSR, VL>& t, const u32x4 (&cs)[4], int it, u32x2 (&kop)[8]) {
        const int r0 = r_begin + it * r_step;
        const int re = it < ntile ? r_end : r_begin;
        uint16_t* vb = vbuf + (it & 1) * 16 * RSV;
#pragma unroll
        for (int c = 0; c < VL; ++c) {
            const int p = 64 * c + lane;
            *reinterpret_cast<u32x4*>(vb + (p / PPR) * RSV + 8 * (p % PPR)) = zero_unless(r0 + p / PPR < re, t.v[c]);
        }
        // rebuild the K tile
        v4f kc[8];
#pragma unroll
        for (int tt = 0; tt < 8; ++tt) kc[tt] = kinit[tt];
#pragma unroll
        for (int m = 0; m < KP; ++m)
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) kc[tt] = mfma32(wq[tt][m], t.kq[m], kc[tt]);
        if constexpr (KO) {
            const v4s bop = as_v4s(t.kr.x, t.kr.y);
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) kc[tt] = mfma16(as_v4s(wr[tt].x, wr[tt].y), bop, kc[tt]);
        }
        if constexpr (ROPE == 2) {
            // x = acc + bias (the bias was the accumulator's start), y[d] =
            // x[d] c - x[d + 64] s, y[d + 64] = x[d + 64] c + x[d] s, in fp32
            // with the table's bf16 (c, s); one rounding when packed.
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                const uint32_t cw[4] = {cs[tt].x, cs[tt].y, cs[tt].z, cs[tt].w};
                float ya[4], yb[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float c = lo_bf16(cw[i]), sn = hi_bf16(cw[i]);
                    const float xa = kc[tt][i], xz = kc[tt + 4][i];
                    ya[i] = fmaf(xa, c, -xz * sn);
                    yb[i] = fmaf(xz, c, xa * sn);
                }
                kop[tt] = u32x2{pack_bf16(ya[0], ya[1]), pack_bf16(ya[2], ya[3])};
                kop[tt + 4] = u32x2{pack_bf16(yb[0], yb[1]), pack_bf16(yb[2], yb[3])};
            }
        } else if constexpr (ROPE == 1) {
            // x = bf16(acc + bias) as floats (a missing bias is held as +0: x + 0
            // is x except that -0 becomes +0).  rotate_half pairs d with d + 64
            // (t with t + 4) under the same (c, s):
            //   y[d]      = bf16(bf16(x[d] * c) + bf16(-x[d + 64] * s))
            //   y[d + 64] = bf16(bf16(x[d + 64] * c) + bf16(x[d] * s))
            float x[8][4];
#pragma unroll
            for (int tt = 0; tt < 8; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t bw = bias2[tt][i >> 1];
                    x[tt][i] = round_bf16_hw(kc[tt][i] + ((i & 1) ? hi_bf16(bw) : lo_bf16(bw)));
                }
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                const uint32_t cw[4] = {cs[tt].x, cs[tt].y, cs[tt].z, cs[tt].w};
                float ya[4], yb[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float c = lo_bf16(cw[i]), sn = hi_bf16(cw[i]);
                    const float xa = x[tt][i], xz = x[tt + 4][i];
                    ya[i] = round_bf16_hw(xa * c) + round_bf16_hw(-xz * sn);
                    yb[i] = round_bf16_hw(xz * c) + round_bf16_hw(xa * sn);
                }
                kop[tt] = u32x2{pack_bf16(ya[0], ya[1]), pack_bf16(ya[2], ya[3])};
                kop[tt + 4] = u32x2{pack_bf16(yb[0], yb[1]), pack_bf16(yb[2], yb[3])};
            }
        } else {
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) {
                uint32_t w2[2];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
                    w2[hh] = pack_bf16(kc[tt][2 * hh] + lo_bf16(bias2[tt][hh]), kc[tt][2 * hh + 1] + hi_bf16(bias2[tt][hh]));
                kop[tt] = u32x2{w2[0], w2[1]};
            }
        }
    };
    // Phase B of tile it: scores, online softmax, P V from LDS buffer it & 1.
    auto phase_b = [&](const u32x2 (&kop)[8], int it) {
        const int r0 = r_begin + it * r_step;
        uint16_t* vb = vbuf + (it & 1) * 16 * RSV;
        // scores S^T[key, col] on 16x16x32 MFMAs: a lane's eight k values are
        // dims 32p + 4grp + [0, 4) and 32p + 16 + 4grp + [0, 4) of both the
        // rotated key (kop) and the query (qop), so the contraction covers
        // each dim once
        v4f sc0 = {0.f, 0.f, 0.f, 0.f}, sc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int tt = 0; tt < 8; tt += 4) {
            sc0 = mfma32(u32x4{kop[tt].x, kop[tt].y, kop[tt + 1].x, kop[tt + 1].y},
                         u32x4{qop[tt].x, qop[tt].y, qop[tt + 1].x, qop[tt + 1].y}, sc0);
            sc1 = mfma32(u32x4{kop[tt + 2].x, kop[tt + 2].y, kop[tt + 3].x, kop[tt + 3].y},
                         u32x4{qop[tt + 2].x, qop[tt + 2].y, qop[tt + 3].x, qop[tt + 3].y}, sc1);
        }
        const v4f sc = sc0 + sc1;
        // raw scores (the scale is positive: it is applied to the maximum
        // and inside the exponent's FMA)
        float sv[4];
        float tmax = kNegInf;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int nn = r0 + 4 * grp + i;
            const float xv = nn < vis ? sc[i] : kNegInf;
            sv[i] = xv;
            tmax = fmaxf(tmax, xv);
        }
        tmax = rows_max(tmax) * scale_log2;
        const float mnew = fmaxf(m, tmax);
        const float mref = mnew == kNegInf ? 0.f : mnew;
        const float alpha = fast_exp2(m - mref);
        float pr[4];
        float psum = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pr[i] = fast_exp2(fmaf(sv[i], scale_log2, -mref));
            psum += pr[i];
        }
        lsum = lsum * alpha + psum;
        m = mnew;
#pragma unroll
        for (int i = 0; i < 2 * VL; ++i) acc[i] *= alpha;
        const v4s pb = as_v4s(pack_bf16(pr[0], pr[1]), pack_bf16(pr[2], pr[3]));
        wave_lds_fence();
#pragma unroll
        for (int u = 0; u < VL; ++u) {
            uint32_t w4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                w4[i] = *reinterpret_cast<const uint32_t*>(vb + (4 * grp + i) * RSV + 32 * u + 2 * col);
            const v4s lo = as_v4s((w4[0] & 0xffffu) | (w4[1] << 16), (w4[2] & 0xffffu) | (w4[3] << 16));
            const v4s hi = as_v4s((w4[0] >> 16) | (w4[1] & 0xffff0000u), (w4[2] >> 16) | (w4[3] & 0xffff0000u));
            acc[2 * u] = mfma16(lo, pb, acc[2 * u]);
            acc[2 * u + 1] = mfma16(hi, pb, acc[2 * u + 1]);
        }
        wave_lds_fence();
    };

    // Whole rounds of the ring, branch-free: tiles past the split's end are
    // loaded clamped and zeroed and every key in them is masked, so they leave
    // the running softmax unchanged.
    u32x2 kop[2][8];
    if constexpr (ReconPipeline<KSR, VL>::value) {
        // Software pipeline: phase A of tile t + 1 (rebuild MFMAs, rotation) is
        // issued beside phase B of tile t (score MFMAs, softmax, P V), so the
        // one wavefront of a SIMD keeps the matrix cores and the VALU busy
        // together (C2 layer: 36.0 -> 35.1 us).  The last round's phase A of
        // the tile after it is unused.
        phase_a(ring[0], pairs[0], 0, kop[0]);
        fetch(ring[0], kReconRing);
        if constexpr (ROPE) fetch_pairs(pairs[0], ring[2].pos);
        for (int it = 0; it < ntile; it += kReconRing) {
#pragma unroll
            for (int u = 0; u < kReconRing; ++u) {
                phase_a(ring[(u + 1) % kReconRing], pairs[(u + 1) & 1], it + u + 1, kop[(u + 1) & 1]);
                fetch(ring[(u + 1) % kReconRing], it + u + 1 + kReconRing);
                if constexpr (ROPE) fetch_pairs(pairs[(u + 1) & 1], ring[(u + 3) % kReconRing].pos);
                phase_b(kop[u & 1], it + u);
            }
        }
    } else {
        for (int it = 0; it < ntile; it += kReconRing) {
#pragma unroll
            for (int u = 0; u < kReconRing; ++u) {
                phase_a(ring[u], pairs[u & 1], it + u, kop[0]);
                phase_b(kop[0], it + u);
                fetch(ring[u], it + u + kReconRing);
                if constexpr (ROPE) fetch_pairs(pairs[u & 1], ring[(u + 2) % kReconRing].pos);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    lsum = rows_sum(lsum);
    if (!colv) return;
    const int prow = j * Lq + lq;
    const int64_t slot_out = ((int64_t)b * Hq * Lq + prow) * sg.splits + s;
    if (grp == 0) {
        sg.part_ml[slot_out * 2] = m;
        sg.part_ml[slot_out * 2 + 1] = lsum;
    }
    float* dst = sg.part_acc + slot_out * RV;
#pragma unroll
    for (int u = 0; u < VL; ++u) {
        float4* d4 = reinterpret_cast<float4*>(dst + 32 * u + 8 * grp);
        d4[0] = make_float4(acc[2 * u][0], acc[2 * u + 1][0], acc[2 * u][1], acc[2 * u + 1][1]);
        d4[1] = make_float4(acc[2 * u][2], acc[2 * u + 1][2], acc[2 * u][3], acc[2 * u + 1][3]);
    }
}

// Raw rows (split_segment, head_dim 128) first in the grid, then the beacon splits.
template <int KSR, int VL, int ROPE>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
recon_split_kernel(SplitParams prm, ReconSeg rs) {
    constexpr int LA = kWaves * 2 * 16 * (32 * VL + 8) * 2;
    constexpr int LB = SplitLds<8>::bytes;
    __shared__ __attribute__((aligned(16))) char lds[LA > LB ? LA : LB];
    int w = blockIdx.x;
    if (w < prm.seg[0].nwg) {
        split_segment<8, 1>(prm.seg[0], w, prm.B, prm.Lq, prm.Hq, prm.scale_log2, lds, nullptr, nullptr,
                            prm.qrope.q ? &prm.qrope : nullptr);
        return;
    }
    w -= prm.seg[0].nwg;
    recon_segment<KSR, VL, ROPE>(rs, w, prm.Lq, prm.Hq, prm.scale_log2, lds);
}

// ---------------------------------------------------------------------------
// combine kernel
// ---------------------------------------------------------------------------

struct CombineParams {
    const float* a_ml; const float* a_acc; int a_splits, a_w;
    const float* b_ml; const float* b_acc; int b_splits, b_w;   // b_splits = 0: no latent segment
    const uint16_t* up_v; int64_t up_v_ld; const uint16_t* up_v_bias;
    int blockdiag;                                               // latent acc holds the own block slice
    const float* b_shift;                                        // [B][Hq*Lq] natural-log units or null
    const int32_t* b_len; int b_rps, b_n;                        // compact latent schedule: splits of b =
                                                                 // ceil(min(len_b, b_n) / b_rps); null = all
    int B, Lq, Hq, Hkv, D;                                       // D = output width
    uint16_t* out; int64_t o_sb, o_sl, o_sh;
    float* lse;                                                  // [B, Hq, Lq] or null
};

constexpr int kMaxSplits = 256;
constexpr int kMaxLatW = 1024;
constexpr int kCombineThreads = 128;

__device__ __forceinline__ float block_max128(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, shfl_xor_f(v, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = fmaxf(red[0], red[1]);
    __syncthreads();
    return v;
}

__device__ __forceinline__ float block_sum128(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += shfl_xor_f(v, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    v = red[0] + red[1];
    __syncthreads();
    return v;
}

// Latent splits written for batch entry b (all of them unless the schedule was compact).
__device__ __forceinline__ int live_b_splits(const CombineParams& cp, int b) {
    if (!cp.b_len || !cp.b_splits) return cp.b_splits;
    int len = cp.b_len[b];
    len = len < 0 ? 0 : (len > cp.b_n ? cp.b_n : len);
    return min(cp.b_splits, (len + cp.b_rps - 1) / cp.b_rps);
}

// One workgroup per (b, query head, query): LSE-merge the split partials of
// both segments, lift the latent accumulator through U_V, fold the biases.
__global__ void __launch_bounds__(kCombineThreads)
combine_kernel(CombineParams cp) {
    __shared__ float wts[2 * kMaxSplits];
    __shared__ float accb[kMaxLatW];
    __shared__ float red[2];
    const int HL = cp.Hq * cp.Lq;
    const int pr = blockIdx.x % HL;
    const int b = blockIdx.x / HL;
    const int j = pr / cp.Lq;
    const int lq = pr % cp.Lq;
    const int h = j / (cp.Hq / cp.Hkv);
    const int64_t row = (int64_t)b * HL + pr;
    const float* aml = cp.a_ml + row * cp.a_splits * 2;
    const float* bml = cp.b_splits ? cp.b_ml + row * cp.b_splits * 2 : nullptr;
    const float shift = (cp.b_splits && cp.b_shift) ? cp.b_shift[row] * kLog2e : 0.f;
    const int bsp = live_b_splits(cp, b);
    const int total = cp.a_splits + bsp;

    // Split maxima and masses, one split per thread.
    float mloc = kNegInf;
    for (int s = threadIdx.x; s < total; s += kCombineThreads) {
        float mv = s < cp.a_splits ? aml[2 * s] : bml[2 * (s - cp.a_splits)];
        if (s >= cp.a_splits && mv != kNegInf) mv += shift;
        wts[s] = mv;
        mloc = fmaxf(mloc, mv);
    }
    const float M = block_max128(mloc, red);
    const float Mref = M == kNegInf ? 0.f : M;
    float la = 0.f, lb = 0.f;
    for (int s = threadIdx.x; s < total; s += kCombineThreads) {
        const float wgt = wts[s] == kNegInf ? 0.f : fast_exp2(wts[s] - Mref);
        wts[s] = wgt;
        if (s < cp.a_splits) la += aml[2 * s + 1] * wgt;
        else lb += bml[2 * (s - cp.a_splits) + 1] * wgt;
    }
    const float LA = block_sum128(la, red);
    const float LB = block_sum128(lb, red);
    const float L = LA + LB;

    if (cp.b_splits) {
        // Weighted latent accumulator: threads split (k, split group).
        const float* bacc = cp.b_acc + row * cp.b_splits * cp.b_w;
        const float* wb = wts + cp.a_splits;
        if (cp.b_w <= kCombineThreads / 2) {
            const int groups = kCombineThreads / cp.b_w;
            const int k = threadIdx.x % cp.b_w, gsel = threadIdx.x / cp.b_w;
            float sum = 0.f;
            if (gsel < groups)
                for (int s = gsel; s < bsp; s += groups) sum += bacc[(int64_t)s * cp.b_w + k] * wb[s];
            __shared__ float part[kCombineThreads];
            part[threadIdx.x] = sum;
            __syncthreads();
            if (threadIdx.x < cp.b_w) {
                float t = 0.f;
                for (int g2 = 0; g2 < groups; ++g2) t += part[g2 * cp.b_w + threadIdx.x];
                accb[threadIdx.x] = t;
            }
        } else {
            for (int k = threadIdx.x; k < cp.b_w; k += kCombineThreads) {
                float sum = 0.f;
                for (int s = 0; s < bsp; ++s) sum += bacc[(int64_t)s * cp.b_w + k] * wb[s];
                accb[k] = sum;
            }
        }
        __syncthreads();
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const float* aacc = cp.a_acc + row * cp.a_splits * cp.a_w;
    uint16_t* orow = cp.out + (int64_t)b * cp.o_sb + (int64_t)lq * cp.o_sl + (int64_t)j * cp.o_sh;
    for (int dd = threadIdx.x; dd < cp.D; dd += kCombineThreads) {
        float sum = 0.f;
        for (int s = 0; s < cp.a_splits; ++s) sum += aacc[(int64_t)s * cp.a_w + dd] * wts[s];
        if (cp.b_splits && !cp.up_v) {
            sum += accb[dd];          // full-dim second segment: no lift
        } else if (cp.b_splits) {
            const int64_t wrow = (int64_t)h * cp.D + dd;
            const uint16_t* wr = cp.up_v + wrow * cp.up_v_ld + (cp.blockdiag ? h * cp.b_w : 0);
            float lift = 0.f;
            for (int k = 0; k < cp.b_w; k += 8) {
                const u32x4 wv = *reinterpret_cast<const u32x4*>(wr + k);
                const uint32_t ws[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    lift += bf16_to_f32(ws[e] & 0xffffu) * accb[k + 2 * e];
                    lift += bf16_to_f32(ws[e] >> 16) * accb[k + 2 * e + 1];
                }
            }
            sum += lift;
            if (cp.up_v_bias) sum += bf16_to_f32(cp.up_v_bias[wrow]) * LB;
        }
        orow[dd] = (uint16_t)pack_bf16(sum * inv, 0.f);
    }
    if (cp.lse && threadIdx.x == 0) {
        cp.lse[((int64_t)b * cp.Hq + j) * cp.Lq + lq] = L > 0.f ? (M + __log2f(L)) * kLn2 : kNegInf;
    }
}

// Raw buffer resource over `bytes` bytes at p (a null p with 0 bytes: every
// load returns zeros).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Fast path for the fused decode's shapes (D <= 128 output features, few raw
// splits, narrow latent slices): every global load is issued before the first
// reduction, so the whole combine costs one memory round trip.
constexpr int kFastRawSplits = 32;
constexpr int kFastRawPer = 8;      // 16-byte raw partial loads (4 columns) per thread
constexpr int kFastLatW = 64;
constexpr int kFastLatPer = 8;      // 16-byte latent partial loads (4 columns) per thread

// Latent splits the fast combine with T threads takes at latent width b_w (a
// multiple of 8): each thread loads kFastLatPer quads of one column group.
constexpr int fast_lat_splits(int b_w, int T) { return kFastLatPer * (T / (b_w / 4)); }

// T = 128 or 256 threads: one split's (m, l) per thread, so a_splits +
// b_splits <= T, and the raw and latent partials as 4-column quads: thread t
// takes quad t % (w / 4) of splits t / (w / 4) + i * (T / (w / 4)) of a
// segment of width w; the groups of splits meet in LDS.
template <int T>
__global__ void __launch_bounds__(T)
combine_fast_kernel(CombineParams cp) {
    __shared__ float wts[2 * kMaxSplits];
    __shared__ float4 part[T];
    __shared__ float4 partr[T];
    __shared__ float accb[kFastLatW];
    __shared__ float red[3 * (T / 64)];      // per-wave maximum, then the two sums
    const int t = threadIdx.x;
    const int HL = cp.Hq * cp.Lq;
    const int pr = blockIdx.x % HL;
    const int b = blockIdx.x / HL;
    const int j = pr / cp.Lq;
    const int lq = pr % cp.Lq;
    const int h = j / (cp.Hq / cp.Hkv);
    const int64_t row = (int64_t)b * HL + pr;
    const int bsp = live_b_splits(cp, b);
    const int total = cp.a_splits + bsp;
    const float* aml = cp.a_ml + row * cp.a_splits * 2;
    const float* bml = cp.b_splits ? cp.b_ml + row * cp.b_splits * 2 : nullptr;

    // -- issue every load --  All through buffer resources: a lane with
    // nothing to read uses an offset past the resource's range and receives
    // zeros, and an absent optional operand is a resource of zero bytes, so the
    // loads form one straight block with no branch around any of them and the
    // split statistics, issued first, are waited on alone -- the weight
    // reductions run while the partials are still arriving.
    constexpr uint32_t kPast = 0x7ffffff0u;          // beyond every resource below
    const bool live = t < total;
    const bool in_a = t < cp.a_splits;
    const auto r_aml = buffer_of(aml, (uint32_t)cp.a_splits * 8u);
    const auto r_bml = buffer_of(bml, cp.b_splits ? (uint32_t)cp.b_splits * 8u : 0u);
    const auto mla = __builtin_amdgcn_raw_buffer_load_b64(r_aml, in_a ? 8u * t : kPast, 0, 0);
    const auto mlb = __builtin_amdgcn_raw_buffer_load_b64(r_bml, (!in_a && live) ? 8u * (t - cp.a_splits) : kPast, 0, 0);
    float mv = live ? __uint_as_float(in_a ? mla[0] : mlb[0]) : kNegInf;
    const float lv = __uint_as_float(in_a ? mla[1] : mlb[1]);     // zero past the live splits
    const auto r_shift = buffer_of(cp.b_shift ? cp.b_shift + row : nullptr, (cp.b_splits && cp.b_shift) ? 4u : 0u);
    const float shift = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r_shift, 0u, 0, 0)) * kLog2e;
    const int dd = t;
    const bool has_dd = dd < cp.D;
    const int rq = cp.a_w / 4;
    const int rkq = t % rq, r0 = t / rq, rstep = T / rq;
    float4 ra[kFastRawPer];
    const float* aacc = cp.a_acc + row * cp.a_splits * cp.a_w;
    const auto r_aacc = buffer_of(aacc, (uint32_t)(cp.a_splits * cp.a_w) * 4u);
#pragma unroll
    for (int i = 0; i < kFastRawPer; ++i) {
        const int s = r0 + i * rstep;
        const bool ok = s < cp.a_splits && r0 < rstep;
        ra[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                    r_aacc, ok ? (uint32_t)(s * cp.a_w + 4 * rkq) * 4u : kPast, 0, 0));
    }
    float4 lb[kFastLatPer];
    const int quads = cp.b_w / 4;
    const int kq = quads ? t % quads : 0;
    const int sstep = quads ? T / quads : 1;
    const int s0 = quads ? t / quads : 0;
    const float* bacc = cp.b_splits ? cp.b_acc + row * cp.b_splits * cp.b_w : nullptr;
    const auto r_bacc = buffer_of(bacc, (uint32_t)(cp.b_splits * cp.b_w) * 4u);
#pragma unroll
    for (int i = 0; i < kFastLatPer; ++i) {
        const int s = s0 + i * sstep;
        const bool ok = s < bsp && s0 < sstep;
        lb[i] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                    r_bacc, ok ? (uint32_t)(s * cp.b_w + 4 * kq) * 4u : kPast, 0, 0));
    }
    // V lift rows: W_V row h*D + dd, the head's b_w columns (own block when
    // block-diagonal); rows past D read zeros.
    const uint32_t w_bytes = cp.b_splits ? (uint32_t)((int64_t)cp.Hkv * cp.D * cp.up_v_ld * 2) : 0u;
    const auto r_wv = buffer_of(cp.up_v, w_bytes);
    const uint32_t w_off = (uint32_t)((((int64_t)h * cp.D + dd) * cp.up_v_ld + (cp.blockdiag ? h * cp.b_w : 0)) * 2);
    u32x4 wv[kFastLatW / 8];
#pragma unroll
    for (int c = 0; c < kFastLatW / 8; ++c)
        wv[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                    r_wv, (has_dd && 8 * c < cp.b_w) ? w_off + 16u * c : kPast, 0, 0));
    const auto r_bias = buffer_of(cp.up_v_bias, (cp.b_splits && cp.up_v_bias) ? (uint32_t)(cp.Hkv * cp.D * 2) : 0u);
    const float bias_v = bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(
        r_bias, has_dd ? (uint32_t)(((int64_t)h * cp.D + dd) * 2) : kPast, 0, 0));

    // -- split weights --
    if (t >= cp.a_splits && t < total && mv != kNegInf) mv += shift;
    // One barrier for the maximum, one for both sums (each reduction has its own
    // slots in red[], so no barrier guards their reuse).
    constexpr int NW = T / 64;
    const int wave = t >> 6;
    float M = mv;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, shfl_xor_f(M, o));
    if ((t & 63) == 0) red[wave] = M;
    __syncthreads();
    M = red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, red[w]);
    const float Mref = M == kNegInf ? 0.f : M;
    const float wgt = (t < total && mv != kNegInf) ? fast_exp2(mv - Mref) : 0.f;
    if (t < total) wts[t] = wgt;
    float LA = t < cp.a_splits ? lv * wgt : 0.f;
    float LB = t >= cp.a_splits && t < total ? lv * wgt : 0.f;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        LA += shfl_xor_f(LA, o);
        LB += shfl_xor_f(LB, o);
    }
    if ((t & 63) == 0) {
        red[NW + 2 * wave] = LA;
        red[NW + 2 * wave + 1] = LB;
    }
    __syncthreads();            // also makes wts[] visible
    LA = red[NW];
    LB = red[NW + 1];
#pragma unroll
    for (int w = 1; w < NW; ++w) {
        LA += red[NW + 2 * w];
        LB += red[NW + 2 * w + 1];
    }
    const float L = LA + LB;

    // -- weighted partial sums of both segments, one barrier --
    {
        float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < kFastRawPer; ++i) {
            const int s = r0 + i * rstep;
            if (s < cp.a_splits && r0 < rstep) {
                const float w = wts[s];
                sum.x += ra[i].x * w; sum.y += ra[i].y * w; sum.z += ra[i].z * w; sum.w += ra[i].w * w;
            }
        }
        partr[t] = sum;
    }
    if (cp.b_splits) {
        float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < kFastLatPer; ++i) {
            const int s = s0 + i * sstep;
            if (s < bsp && s0 < sstep) {
                const float w = wts[cp.a_splits + s];
                sum.x += lb[i].x * w; sum.y += lb[i].y * w; sum.z += lb[i].z * w; sum.w += lb[i].w * w;
            }
        }
        part[t] = sum;
    }
    __syncthreads();
    // -- latent accumulator --
    if (cp.b_splits) {
        if (t < cp.b_w) {
            const float* pf = reinterpret_cast<const float*>(part);
            float acc = 0.f;
            for (int g2 = 0; g2 < sstep; ++g2) acc += pf[4 * (g2 * quads + t / 4) + t % 4];
            accb[t] = acc;
        }
        __syncthreads();
    }
    // -- output --
    if (has_dd) {
        const float* pr4 = reinterpret_cast<const float*>(partr);
        float sum = 0.f;
        for (int g2 = 0; g2 < rstep; ++g2) sum += pr4[4 * (g2 * rq + dd / 4) + dd % 4];
        if (cp.b_splits) {
            float lift = 0.f;
#pragma unroll
            for (int c = 0; c < kFastLatW / 8; ++c) {
                if (8 * c >= cp.b_w) break;
                const uint32_t w4[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    lift += bf16_to_f32(w4[e] & 0xffffu) * accb[8 * c + 2 * e];
                    lift += bf16_to_f32(w4[e] >> 16) * accb[8 * c + 2 * e + 1];
                }
            }
            sum += lift + bias_v * LB;
        }
        const float inv = L > 0.f ? 1.f / L : 0.f;
        cp.out[(int64_t)b * cp.o_sb + (int64_t)lq * cp.o_sl + (int64_t)j * cp.o_sh + dd] = (uint16_t)pack_bf16(sum * inv, 0.f);
    }
    if (cp.lse && t == 0)
        cp.lse[((int64_t)b * cp.Hq + j) * cp.Lq + lq] = L > 0.f ? (M + __log2f(L)) * kLn2 : kNegInf;
}

// Whether the fast combine with T threads takes these partials.  Latent widths
// that do not divide the block (48) leave the threads past (T / b_w) * b_w
// idle in the weighted sum.
bool combine_fast_ok(const CombineParams& cp, int T) {
    if (cp.b_splits && !cp.up_v) return false;
    return cp.D <= T && cp.a_w >= cp.D && cp.a_w % 4 == 0 && cp.a_w <= 4 * T && cp.a_splits <= kFastRawSplits &&
           cp.a_splits <= kFastRawPer * (T / (cp.a_w / 4)) && cp.a_splits + cp.b_splits <= T && cp.b_w <= kFastLatW &&
           (cp.b_splits == 0 || (cp.b_w % 8 == 0 && cp.b_splits <= fast_lat_splits(cp.b_w, T)));
}

// One wave per (b, query head, query): the merge of combine_fast_kernel with
// no barrier -- split statistics on lanes (raw splits, then latent), row
// reductions over the wave with DPP row rotations and row swaps, split
// weights broadcast with readlane, the latent lane groups meeting in the
// wave's own LDS; a lane owns output columns 2 * lane and 2 * lane + 1.
constexpr int kWaveRaw = 8;         // raw splits
constexpr int kWaveLat = 4;         // latent partial quads per lane

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(v), CTRL, 0xf, 0xf, true));
}
// Over all 64 lanes: row_ror 1, 2, 4, 8 inside each 16-lane row, then the
// row swaps.  Each lane's sum associates in its own rotation order, so lanes
// may hold sums an fp32 ulp apart (deterministic for given inputs); callers
// that need one value on every lane take lane 0's (wave_first).
__device__ __forceinline__ float wave_max64(float v) {
    v = fmaxf(v, dpp_f<0x121>(v));
    v = fmaxf(v, dpp_f<0x122>(v));
    v = fmaxf(v, dpp_f<0x124>(v));
    v = fmaxf(v, dpp_f<0x128>(v));
    return rows_max(v);
}
__device__ __forceinline__ float wave_sum64(float v) {
    v += dpp_f<0x121>(v);
    v += dpp_f<0x122>(v);
    v += dpp_f<0x124>(v);
    v += dpp_f<0x128>(v);
    return rows_sum(v);
}

// Lane 0's value on every lane (a scalar register).
__device__ __forceinline__ float wave_first(float v) {
    return __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(v)));
}

template <int LW>   // latent width bound (own block), a multiple of 8
__global__ void __launch_bounds__(64)
combine_wave_kernel(CombineParams cp) {
    __shared__ float4 red4[64 + LW / 4];
    float* red = reinterpret_cast<float*>(red4);
    const int lane = threadIdx.x;
    const int HL = cp.Hq * cp.Lq;
    const int pr = blockIdx.x % HL;
    const int b = blockIdx.x / HL;
    const int j = pr / cp.Lq;
    const int lq = pr % cp.Lq;
    const int h = j / (cp.Hq / cp.Hkv);
    const int64_t row = (int64_t)b * HL + pr;
    const int Sa = cp.a_splits, Sb = cp.b_splits, bsp = live_b_splits(cp, b);
    const int bw = cp.b_w;
    const int dd = 2 * lane;
    constexpr uint32_t kPast = 0x7ffffff0u;

    // -- every load at once --
    const bool in_a = lane < Sa, in_b = lane >= Sa && lane < Sa + bsp;
    const auto r_aml = buffer_of(cp.a_ml + row * Sa * 2, (uint32_t)Sa * 8u);
    const auto r_bml = buffer_of(Sb ? cp.b_ml + row * Sb * 2 : nullptr, Sb ? (uint32_t)Sb * 8u : 0u);
    const auto mla = __builtin_amdgcn_raw_buffer_load_b64(r_aml, in_a ? 8u * lane : kPast, 0, 0);
    const auto mlb = __builtin_amdgcn_raw_buffer_load_b64(r_bml, in_b ? 8u * (lane - Sa) : kPast, 0, 0);
    const auto r_shift = buffer_of(cp.b_shift ? cp.b_shift + row : nullptr, (Sb && cp.b_shift) ? 4u : 0u);
    const float shift = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r_shift, 0u, 0, 0)) * kLog2e;
    const auto r_aacc = buffer_of(cp.a_acc + row * Sa * cp.a_w, (uint32_t)(Sa * cp.a_w) * 4u);
    u32x2 ra[kWaveRaw];
#pragma unroll
    for (int s = 0; s < kWaveRaw; ++s)
        ra[s] = __builtin_amdgcn_raw_buffer_load_b64(r_aacc, s < Sa ? (uint32_t)(s * cp.a_w + dd) * 4u : kPast, 0, 0);
    const int quads = bw / 4;
    const int ngr = quads ? 64 / quads : 1;
    const int cq = quads ? lane % quads : 0, lg = quads ? lane / quads : 0;
    const auto r_bacc = buffer_of(Sb ? cp.b_acc + row * Sb * bw : nullptr, (uint32_t)(Sb * bw) * 4u);
    u32x4 lb[kWaveLat];
#pragma unroll
    for (int k = 0; k < kWaveLat; ++k) {
        const int s = lg + k * ngr;
        const bool ok = lg < ngr && s < bsp;
        lb[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                    r_bacc, ok ? (uint32_t)(s * bw + 4 * cq) * 4u : kPast, 0, 0));
    }
    const uint32_t w_bytes = Sb ? (uint32_t)((int64_t)cp.Hkv * cp.D * cp.up_v_ld * 2) : 0u;
    const auto r_wv = buffer_of(cp.up_v, w_bytes);
    const uint32_t w0 = (uint32_t)((((int64_t)h * cp.D + dd) * cp.up_v_ld + (cp.blockdiag ? h * bw : 0)) * 2);
    const uint32_t w1 = w0 + (uint32_t)(cp.up_v_ld * 2);
    u32x4 wa[LW / 8], wb[LW / 8];
#pragma unroll
    for (int c = 0; c < LW / 8; ++c) {
        wa[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r_wv, 8 * c < bw ? w0 + 16u * c : kPast, 0, 0));
        wb[c] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r_wv, 8 * c < bw ? w1 + 16u * c : kPast, 0, 0));
    }
    const auto r_bias = buffer_of(cp.up_v_bias, (Sb && cp.up_v_bias) ? (uint32_t)(cp.Hkv * cp.D * 2) : 0u);
    const uint32_t bias2 = __builtin_amdgcn_raw_buffer_load_b32(r_bias, (uint32_t)((h * cp.D + dd) * 2), 0, 0);

    // -- split weights --
    float mv = in_a ? __uint_as_float(mla[0]) : (in_b ? __uint_as_float(mlb[0]) : kNegInf);
    const float lv = in_a ? __uint_as_float(mla[1]) : __uint_as_float(mlb[1]);
    if (in_b && mv != kNegInf) mv += shift;
    // one maximum and one pair of sums for the whole row: every lane scales
    // its two columns by the same 1 / L, lane 0 writes the LSE from that L
    const float M = wave_first(wave_max64(mv));
    const float Mref = M == kNegInf ? 0.f : M;
    const float w = mv != kNegInf ? fast_exp2(mv - Mref) : 0.f;
    const float LA = wave_first(wave_sum64(in_a ? lv * w : 0.f));
    const float LB = wave_first(wave_sum64(in_b ? lv * w : 0.f));
    const float L = LA + LB;

    // -- raw rows --
    float o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int s = 0; s < kWaveRaw; ++s) {
        if (s >= Sa) break;
        const float ws = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(w), s));
        o0 += ws * __uint_as_float(ra[s][0]);
        o1 += ws * __uint_as_float(ra[s][1]);
    }
    // -- latent accumulator: lane groups meet in LDS, then every lane reads it --
    if (Sb) {
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int k = 0; k < kWaveLat; ++k) {
            const int s = lg + k * ngr;
            const float ws = __shfl(w, Sa + s < 64 ? Sa + s : 63, 64);
            if (lg < ngr && s < bsp) {
                q.x += ws * __uint_as_float(lb[k].x);
                q.y += ws * __uint_as_float(lb[k].y);
                q.z += ws * __uint_as_float(lb[k].z);
                q.w += ws * __uint_as_float(lb[k].w);
            }
        }
        if (lg < ngr) red4[lane] = q;
        wave_lds_fence();
        if (lane < bw) {
            float a = 0.f;
            for (int g = 0; g < ngr; ++g) a += red[g * bw + lane];
            red[256 + lane] = a;
        }
        wave_lds_fence();
        float l0 = 0.f, l1 = 0.f;
#pragma unroll
        for (int c = 0; c < LW / 8; ++c) {
            if (8 * c >= bw) break;
            const float4 x0 = red4[64 + 2 * c], x1 = red4[65 + 2 * c];
            const float av[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            const uint32_t pa[4] = {wa[c].x, wa[c].y, wa[c].z, wa[c].w};
            const uint32_t pb[4] = {wb[c].x, wb[c].y, wb[c].z, wb[c].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                l0 += lo_bf16(pa[e]) * av[2 * e] + hi_bf16(pa[e]) * av[2 * e + 1];
                l1 += lo_bf16(pb[e]) * av[2 * e] + hi_bf16(pb[e]) * av[2 * e + 1];
            }
        }
        o0 += l0 + lo_bf16(bias2) * LB;
        o1 += l1 + hi_bf16(bias2) * LB;
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    *reinterpret_cast<uint32_t*>(cp.out + (int64_t)b * cp.o_sb + (int64_t)lq * cp.o_sl + (int64_t)j * cp.o_sh + dd) =
        pack_bf16(o0 * inv, o1 * inv);
    if (cp.lse && lane == 0)
        cp.lse[((int64_t)b * cp.Hq + j) * cp.Lq + lq] = L > 0.f ? (M + __log2f(L)) * kLn2 : kNegInf;
}

// Whether the one-wave combine takes these partials.
bool combine_wave_ok(const CombineParams& cp) {
    if (cp.D != 128 || cp.a_w != 128 || cp.a_splits > kWaveRaw || cp.a_splits + cp.b_splits > 64) return false;
    if ((reinterpret_cast<uintptr_t>(cp.out) & 3) || cp.o_sb % 2 || cp.o_sl % 2 || cp.o_sh % 2) return false;
    if (!cp.b_splits) return true;
    if (!cp.up_v || cp.b_w % 8 || cp.b_w > 64) return false;
    const int ngr = 64 / (cp.b_w / 4);
    return (cp.b_splits + ngr - 1) / ngr <= kWaveLat;
}

// The one-wave combine takes the shapes it fits (the batch-16 32K decode
// sweep: 1.180 -> 1.138 ms; the 64-sequence paged step: 0.151 -> 0.147 ms
// against combine_fast_kernel<128>); more splits or wider latents keep the
// workgroup kernels.
void launch_combine(const CombineParams& cp, int rows, hipStream_t st) {
    if (combine_wave_ok(cp)) {
        if (!cp.b_splits || cp.b_w <= 16) hipLaunchKernelGGL(combine_wave_kernel<16>, dim3(rows), dim3(64), 0, st, cp);
        else if (cp.b_w <= 32) hipLaunchKernelGGL(combine_wave_kernel<32>, dim3(rows), dim3(64), 0, st, cp);
        else if (cp.b_w <= 48) hipLaunchKernelGGL(combine_wave_kernel<48>, dim3(rows), dim3(64), 0, st, cp);
        else hipLaunchKernelGGL(combine_wave_kernel<64>, dim3(rows), dim3(64), 0, st, cp);
        return;
    }
    if (combine_fast_ok(cp, 128))
        hipLaunchKernelGGL(combine_fast_kernel<128>, dim3(rows), dim3(128), 0, st, cp);
    else if (combine_fast_ok(cp, 256))
        hipLaunchKernelGGL(combine_fast_kernel<256>, dim3(rows), dim3(256), 0, st, cp);
    else
        hipLaunchKernelGGL(combine_kernel, dim3(rows), dim3(kCombineThreads), 0, st, cp);
}

// ---------------------------------------------------------------------------
// prologue: query RoPE + absorption into U_K + K-bias shift
// ---------------------------------------------------------------------------

struct PrologueParams {
    const uint16_t* q; int64_t q_sb, q_sl, q_sh;
    const int64_t* pos; int64_t pos_sb;
    const float* cos; const float* sin; int64_t rope_rows;
    uint16_t* q_rot;                       // [B][Lq][Hq][D]
    const uint16_t* up_k; const uint16_t* up_k_bias;   // [Hkv*D][Rk]
    int blockdiag; int wq;                 // q_lat width (own block or Rk)
    uint16_t* q_lat;                       // [B][Lq][Hq][wq]
    float* shift;                          // [B][Hq*Lq] or null
    int B, Lq, Hq, Hkv, D, Rk, parts;      // parts: power of two <= 16 dividing D
    float scale;
    const uint16_t* ut;                    // [Hkv][wq][D] per-head U_K^T (MFMA prologue) or null
};

constexpr int kMaxRows = 16;
constexpr int kMaxD = 256;

// RoPE table row of query (b, l): its position, or -- without positions --
// row b * Lq + l of tables already taken at the query positions (one gather
// per decode step serves every layer).
__device__ __forceinline__ int64_t query_rope_row(const PrologueParams& pp, int b, int l) {
    if (!pp.pos) return (int64_t)b * pp.Lq + l;
    return clamp_i64(pp.pos[(int64_t)b * pp.pos_sb + l], 0, pp.rope_rows - 1);
}

// One workgroup per (b, KV head).  Rows r = jj*Lq + l of the head's query group
// are rotated into LDS; thread (k8, part) then forms 8 consecutive q_lat
// columns over a D/parts slice with 16-byte weight loads, and the parts are
// reduced with lane shuffles (they are adjacent lanes).
__global__ void __launch_bounds__(256)
prologue_kernel(PrologueParams pp) {
    __shared__ float qs[kMaxRows * kMaxD];
    const int h = blockIdx.x % pp.Hkv;
    const int b = blockIdx.x / pp.Hkv;
    const int g = pp.Hq / pp.Hkv;
    const int rows = g * pp.Lq;
    const int D = pp.D;
    const int pieces = D / 8;
    for (int e = threadIdx.x; e < rows * pieces; e += blockDim.x) {
        const int r = e / pieces, dd = (e % pieces) * 8;
        const int jj = r / pp.Lq, l = r % pp.Lq;
        const int jh = h * g + jj;
        const uint16_t* qrow = pp.q + (int64_t)b * pp.q_sb + (int64_t)l * pp.q_sl + (int64_t)jh * pp.q_sh;
        const u32x4 xv = *reinterpret_cast<const u32x4*>(qrow + dd);
        uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
        float x[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = bf16_to_f32(xs[i] & 0xffffu);
            x[2 * i + 1] = bf16_to_f32(xs[i] >> 16);
        }
        if (pp.cos) {
            const int half = D / 2;
            const int pd = dd < half ? dd + half : dd - half;
            const u32x4 pv = *reinterpret_cast<const u32x4*>(qrow + pd);
            const uint32_t ps[4] = {pv.x, pv.y, pv.z, pv.w};
            const int64_t pos = query_rope_row(pp, b, l);
            const float4* c4 = reinterpret_cast<const float4*>(pp.cos + pos * D + dd);
            const float4* s4 = reinterpret_cast<const float4*>(pp.sin + pos * D + dd);
            const float4 ca = c4[0], cb = c4[1], sa = s4[0], sb = s4[1];
            const float cs[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
            const float ss[8] = {sa.x, sa.y, sa.z, sa.w, sb.x, sb.y, sb.z, sb.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float pt = bf16_to_f32(i & 1 ? (ps[i / 2] >> 16) : (ps[i / 2] & 0xffffu));
                if (dd < half) pt = -pt;
                x[i] = round_bf16_hw(round_bf16_hw(x[i] * round_bf16_hw(cs[i])) +
                                     round_bf16_hw(pt * round_bf16_hw(ss[i])));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) xs[i] = pack_bf16(x[2 * i], x[2 * i + 1]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) qs[r * D + dd + i] = x[i];
        *reinterpret_cast<u32x4*>(pp.q_rot + (((int64_t)b * pp.Lq + l) * pp.Hq + jh) * D + dd) =
            u32x4{xs[0], xs[1], xs[2], xs[3]};
    }
    __syncthreads();
    if (pp.shift && threadIdx.x < rows) {
        const int r = threadIdx.x;
        const int jj = r / pp.Lq, l = r % pp.Lq;
        float sum = 0.f;
        for (int dd = 0; dd < D; ++dd)
            sum += qs[r * D + dd] * bf16_to_f32(pp.up_k_bias[(int64_t)h * D + dd]);
        pp.shift[(int64_t)b * pp.Hq * pp.Lq + (h * g + jj) * pp.Lq + l] = sum * pp.scale;
    }
    if (pp.wq == 0) return;
    // Absorption: thread (row r, 8-column group k8, part) sums D/parts terms for
    // 8 consecutive q_lat columns; partial sums meet in LDS.
    __shared__ float red[256 * 8];
    const int parts = pp.parts;
    const int per = D / parts;
    const int k8n = pp.wq / 8;
    for (int base = 0; base < rows * k8n * parts; base += 256) {
        const int task = base + threadIdx.x;
        const bool active = task < rows * k8n * parts;
        const int part = task % parts;
        const int rk = task / parts;            // r * k8n + k8
        const int r = rk / k8n, k8 = rk % k8n;
        float acc8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (active) {
            const int kg = (pp.blockdiag ? h * pp.wq : 0) + 8 * k8;
            const uint16_t* wbase = pp.up_k + ((int64_t)h * D + part * per) * pp.Rk + kg;
            const float* qr = qs + r * D + part * per;
            for (int d0 = 0; d0 < per; d0 += 8) {
                u32x4 wv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) wv[i] = *reinterpret_cast<const u32x4*>(wbase + (int64_t)(d0 + i) * pp.Rk);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float qv = qr[d0 + i];
                    const uint32_t w4[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        acc8[2 * e] += qv * bf16_to_f32(w4[e] & 0xffffu);
                        acc8[2 * e + 1] += qv * bf16_to_f32(w4[e] >> 16);
                    }
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) red[threadIdx.x * 8 + e] = acc8[e];
        __syncthreads();
        if (active && part == 0) {
            float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            for (int q = 0; q < parts; ++q)
#pragma unroll
                for (int e = 0; e < 8; ++e) sum[e] += red[(threadIdx.x + q) * 8 + e];
            const int jj = r / pp.Lq, l = r % pp.Lq;
            uint32_t o4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o4[e] = pack_bf16(sum[2 * e], sum[2 * e + 1]);
            *reinterpret_cast<u32x4*>(pp.q_lat + (((int64_t)b * pp.Lq + l) * pp.Hq + h * g + jj) * pp.wq + 8 * k8) =
                u32x4{o4[0], o4[1], o4[2], o4[3]};
        }
        __syncthreads();
    }
}

// MFMA prologue for block-diagonal bases, one wavefront per (b, KV head): the
// g*Lq query rows of the head are the MFMA columns (lane col), rotated in
// registers, and q_lat^T[c][p] = U_K^T[c][:] . q_rot[p][:] comes from NCT
// 16-row tiles of the prepared per-head U_K^T.  Every load is issued before any
// result is needed: q, U_K^T and the RoPE table rows in one memory round trip
// (given positions, the rows follow the position load they depend on).
template <int NCT>
__global__ void __launch_bounds__(64)
prologue_mfma_kernel(PrologueParams pp) {
    const int h = blockIdx.x % pp.Hkv;
    const int b = blockIdx.x / pp.Hkv;
    const int g = pp.Hq / pp.Hkv;
    const int rows = g * pp.Lq;
    const int lane = threadIdx.x, col = lane & 15, grp = lane >> 4;
    const bool valid = col < rows;
    const int p = valid ? col : 0;
    const int jj = p / pp.Lq, l = p % pp.Lq;
    const int j = h * g + jj;
    constexpr int D = 128;
    u32x4 ua[NCT][4];
    const uint16_t* ub = pp.ut + ((int64_t)h * pp.wq + col) * D + 8 * grp;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int c = 0; c < 4; ++c) ua[ct][c] = *reinterpret_cast<const u32x4*>(ub + (int64_t)16 * ct * D + 32 * c);
    u32x4 qr[4];
    const uint16_t* qrow = pp.q + (int64_t)b * pp.q_sb + (int64_t)l * pp.q_sl + (int64_t)j * pp.q_sh + 8 * grp;
#pragma unroll
    for (int c = 0; c < 4; ++c) qr[c] = *reinterpret_cast<const u32x4*>(qrow + 32 * c);
    // The table rows go out with the query and basis loads (with positions,
    // after the position load they depend on).
    RopeRow rr;
    if (pp.cos) {
        const int64_t pos = query_rope_row(pp, b, l);
        load_rope_row(rr, pp.cos + pos * D, pp.sin + pos * D, grp);
    }
    u32x4 kb[4];
    if (pp.shift) {
        const uint16_t* bk = pp.up_k_bias + (int64_t)h * D + 8 * grp;
#pragma unroll
        for (int c = 0; c < 4; ++c) kb[c] = *reinterpret_cast<const u32x4*>(bk + 32 * c);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) qr[c] = valid ? qr[c] : u32x4{0u, 0u, 0u, 0u};
    if (pp.cos) rope_operand(qr, rr);
    const int64_t prow = ((int64_t)b * pp.Lq + l) * pp.Hq + j;
    if (valid) {
#pragma unroll
        for (int c = 0; c < 4; ++c) *reinterpret_cast<u32x4*>(pp.q_rot + prow * D + 32 * c + 8 * grp) = qr[c];
    }
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
        v4f t4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c) t4 = mfma32(ua[ct][c], qr[c], t4);
        if (valid)
            *reinterpret_cast<u32x2*>(pp.q_lat + prow * pp.wq + 16 * ct + 4 * grp) =
                u32x2{pack_bf16(t4[0], t4[1]), pack_bf16(t4[2], t4[3])};
    }
    if (pp.shift) {
        const float dot = kbias_dot(qr, kb);
        if (valid && grp == 0) pp.shift[(int64_t)b * pp.Hq * pp.Lq + j * pp.Lq + l] = dot * pp.scale;
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

namespace {

thread_local std::string g_error;

hipError_t dispatch_split(int ka, int kb, const struct SplitParams& prm, int grid, hipStream_t st);
hipError_t dispatch_split_seg2(int ka, const struct SplitParams& prm, int grid, hipStream_t st);
template <int MODE, int RAWPG>
hipError_t launch_split_paged(int ka, const SplitParams& prm, int grid, hipStream_t st) {
    switch (ka) {
        case 2: hipLaunchKernelGGL((split_kernel<2, 8, MODE, 0, RAWPG>), dim3(grid), dim3(kThreads), 0, st, prm); break;
        case 4: hipLaunchKernelGGL((split_kernel<4, 8, MODE, 0, RAWPG>), dim3(grid), dim3(kThreads), 0, st, prm); break;
        case 6: hipLaunchKernelGGL((split_kernel<6, 8, MODE, 0, RAWPG>), dim3(grid), dim3(kThreads), 0, st, prm); break;
        case 8: hipLaunchKernelGGL((split_kernel<8, 8, MODE, 0, RAWPG>), dim3(grid), dim3(kThreads), 0, st, prm); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Pages of at least 16 rows take the two-pages-per-tile addressing; raw rows
// come from dense tensors or through raw pages.
hipError_t dispatch_split_paged(int ka, const SplitParams& prm, int grid, hipStream_t st) {
    const bool raw_pages = prm.rawp.table != nullptr;
    if (prm.seg[0].slots >= 16)
        return raw_pages ? launch_split_paged<2, 1>(ka, prm, grid, st) : launch_split_paged<2, 0>(ka, prm, grid, st);
    return raw_pages ? launch_split_paged<1, 1>(ka, prm, grid, st) : launch_split_paged<1, 0>(ka, prm, grid, st);
}

hipError_t launch_split_any(int ka, int kb, const SplitParams& prm, int grid, hipStream_t st, bool paged = false,
                            bool seg2 = false) {
    if (paged) return dispatch_split_paged(ka, prm, grid, st);
    return seg2 ? dispatch_split_seg2(ka, prm, grid, st) : dispatch_split(ka, kb, prm, grid, st);
}

// Instances that make their query operands (FQ): latent tiles up to 128
// columns beside the head_dim-128 raw rows -- dense rows in one or two
// segments, and rows through pages of at least 16 slots with the raw rows
// dense or through raw pages.
template <int PAGED, int SEG2, int RAWPG>
hipError_t launch_split_fq(int ka, const SplitParams& prm, int grid, hipStream_t st) {
    switch (ka) {
        case 2: hipLaunchKernelGGL((split_kernel<2, 8, PAGED, SEG2, RAWPG, 1>), dim3(grid), dim3(kThreads), 0, st, prm); break;
        case 4: hipLaunchKernelGGL((split_kernel<4, 8, PAGED, SEG2, RAWPG, 1>), dim3(grid), dim3(kThreads), 0, st, prm); break;
        case 6: hipLaunchKernelGGL((split_kernel<6, 8, PAGED, SEG2, RAWPG, 1>), dim3(grid), dim3(kThreads), 0, st, prm); break;
        case 8: hipLaunchKernelGGL((split_kernel<8, 8, PAGED, SEG2, RAWPG, 1>), dim3(grid), dim3(kThreads), 0, st, prm); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

bool split_fq_ok(int ka, bool paged, int slots) {
    return (ka == 2 || ka == 4 || ka == 6 || ka == 8) && (!paged || slots >= 16);
}

hipError_t launch_split_fused(int ka, const SplitParams& prm, int grid, hipStream_t st, bool paged, bool seg2) {
    if (paged) return prm.rawp.table ? launch_split_fq<2, 0, 1>(ka, prm, grid, st) : launch_split_fq<2, 0, 0>(ka, prm, grid, st);
    return seg2 ? launch_split_fq<0, 1, 0>(ka, prm, grid, st) : launch_split_fq<0, 0, 0>(ka, prm, grid, st);
}

int round_even_tile(int width) {
    // MFMA k-steps of 16 needed for `width`, rounded to the instantiated set.
    const int ks = (width + 15) / 16;
    const int set[] = {2, 4, 6, 8, 12, 16, 24};
    for (int v : set)
        if (ks <= v) return v;
    return -1;
}

bool aligned8(int64_t x) { return (x & 7) == 0; }
bool ptr_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct SegPlan {
    int tiles, cols, splits, rows_per_split, nwg, wown, ks;
};

// Workgroups covering B * splits * slots wave items, kWaves per workgroup.
int wave_item_groups(int B, int splits, int slots) {
    const int64_t items = (int64_t)B * splits * slots;
    return (int)((items + kWaves - 1) / kWaves);
}

// Split the key range so the launch holds a few workgroups per CU.
SegPlan plan_segment(int B, int hk, int P, int cols, int n, int span_k, int wown, int req_splits,
                     int target_wg) {
    SegPlan sp{};
    sp.cols = std::min(cols, 16);
    sp.tiles = (P + sp.cols - 1) / sp.cols;
    sp.ks = round_even_tile(span_k);
    sp.wown = wown;
    // workgroups per split index: kWaves wave items (slots) per workgroup
    const int64_t slot_items = (int64_t)B * hk * sp.tiles;
    int splits = req_splits;
    if (splits <= 0) {
        const int max_by_rows = std::max(1, (n + 15) / 16);
        const int64_t fit = ((int64_t)target_wg * kWaves + slot_items - 1) / slot_items;
        splits = (int)std::max<int64_t>(1, std::min<int64_t>(max_by_rows, fit));
        splits = std::min(splits, kMaxSplits);
    }
    splits = std::min(splits, kMaxSplits);
    int rps = (n + splits - 1) / splits;
    rps = std::max(16, (rps + 15) / 16 * 16);
    splits = std::max(1, (n + rps - 1) / rps);
    sp.splits = splits;
    sp.rows_per_split = rps;
    sp.nwg = wave_item_groups(B, splits, hk * sp.tiles);
    return sp;
}

template <int KA, int KB, int SEG2 = 0>
hipError_t launch_split(const SplitParams& prm, int grid, hipStream_t st) {
    hipLaunchKernelGGL((split_kernel<KA, KB, 0, SEG2>), dim3(grid), dim3(kThreads), 0, st, prm);
    return hipGetLastError();
}

// Latent rows in two tensors (the fused decode's dense rows only).
hipError_t dispatch_split_seg2(int ka, const SplitParams& prm, int grid, hipStream_t st) {
    switch (ka) {
        case 2: return launch_split<2, 8, 1>(prm, grid, st);
        case 4: return launch_split<4, 8, 1>(prm, grid, st);
        case 6: return launch_split<6, 8, 1>(prm, grid, st);
        case 8: return launch_split<8, 8, 1>(prm, grid, st);
        case 12: return launch_split<12, 8, 1>(prm, grid, st);
        case 16: return launch_split<16, 8, 1>(prm, grid, st);
        case 24: return launch_split<24, 8, 1>(prm, grid, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t dispatch_split(int ka, int kb, const SplitParams& prm, int grid, hipStream_t st) {
    if (kb == 0) {
        switch (ka) {
            case 2: return launch_split<2, 0>(prm, grid, st);
            case 4: return launch_split<4, 0>(prm, grid, st);
            case 6: return launch_split<6, 0>(prm, grid, st);
            case 8: return launch_split<8, 0>(prm, grid, st);
            case 12: return launch_split<12, 0>(prm, grid, st);
            case 16: return launch_split<16, 0>(prm, grid, st);
            case 24: return launch_split<24, 0>(prm, grid, st);
            default: return hipErrorInvalidValue;
        }
    }
    if (kb != 8) return hipErrorInvalidValue;   // the raw segment is head_dim 128
    switch (ka) {
        case 2: return launch_split<2, 8>(prm, grid, st);
        case 4: return launch_split<4, 8>(prm, grid, st);
        case 6: return launch_split<6, 8>(prm, grid, st);
        case 8: return launch_split<8, 8>(prm, grid, st);
        case 12: return launch_split<12, 8>(prm, grid, st);
        case 16: return launch_split<16, 8>(prm, grid, st);
        case 24: return launch_split<24, 8>(prm, grid, st);
        default: return hipErrorInvalidValue;
    }
}

// Resident workgroups per CU of a split-kernel instance (cached per device).
int split_occupancy(int ka, int kb) {
    static std::mutex mu;
    static std::vector<std::pair<int, int>> keys;
    static std::vector<int> vals;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const int key = (dev << 16) | (ka << 8) | kb;
    std::lock_guard<std::mutex> lock(mu);
    for (size_t i = 0; i < keys.size(); ++i)
        if (keys[i].first == key) return vals[i];
    const void* fn = nullptr;
#define SLIMKV_FN(A, B) if (ka == A && kb == B) fn = reinterpret_cast<const void*>(&split_kernel<A, B>);
    SLIMKV_FN(2, 0) SLIMKV_FN(2, 8) SLIMKV_FN(4, 0) SLIMKV_FN(6, 0) SLIMKV_FN(8, 0) SLIMKV_FN(12, 0) SLIMKV_FN(16, 0) SLIMKV_FN(24, 0)
    SLIMKV_FN(4, 8) SLIMKV_FN(6, 8) SLIMKV_FN(8, 8) SLIMKV_FN(12, 8) SLIMKV_FN(16, 8) SLIMKV_FN(24, 8)
#undef SLIMKV_FN
    int blocks = 0;
    if (!fn || hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, fn, kThreads, 0) != hipSuccess || blocks < 1)
        blocks = 1;
    keys.push_back({key, 0});
    vals.push_back(blocks);
    return blocks;
}

struct AttnPlan {
    SegPlan sp;
    size_t ml_off, acc_off, total;
};

int plan_attention(const slimkv_attention_args* a, AttnPlan* plan) {
    if (!a || !a->q || !a->k || !a->v || !a->out) return fail(SLIMKV_EINVAL, "null tensor pointer");
    const int64_t B = a->batch, Lq = a->queries, Hq = a->heads, Hk = a->kv_heads, N = a->keys;
    if (B <= 0 || Lq <= 0 || Hq <= 0 || Hk <= 0 || N <= 0 || Hq % Hk)
        return fail(SLIMKV_EINVAL, "invalid attention sizes or GQA head counts");
    if (a->width_k <= 0 || a->width_v <= 0 || !aligned8(a->width_k) || !aligned8(a->width_v))
        return fail(SLIMKV_EINVAL, "K/V widths must be positive multiples of 8");
    if (a->width_k > 384 || a->width_v > 384) return fail(SLIMKV_EUNSUP, "K/V widths above 384 are not supported");
    const int64_t strides[] = {a->q_sb, a->q_sl, a->q_sh, a->k_sb, a->k_sn, a->k_sh, a->v_sb, a->v_sn, a->v_sh};
    for (int64_t st : strides)
        if (!aligned8(st)) return fail(SLIMKV_EINVAL, "strides must be multiples of 8 elements");
    if (!ptr_aligned16(a->q) || !ptr_aligned16(a->k) || !ptr_aligned16(a->v))
        return fail(SLIMKV_EINVAL, "q/k/v must be 16-byte aligned");
    if (N > (int64_t)1 << 30 || B * Hq * Lq > (int64_t)1 << 30) return fail(SLIMKV_EINVAL, "sizes too large");
    const int g = (int)(Hq / Hk);
    const int P = (int)Lq * g;
    const int span = (int)std::max(a->width_k, a->width_v);
    const int ks = round_even_tile(span);
    if (ks < 0) return fail(SLIMKV_EUNSUP, "width not supported");
    const int target = device_cu_count() * split_occupancy(ks, 0);
    plan->sp = plan_segment((int)B, (int)Hk, P, 16, (int)N, span, (int)a->width_v, a->splits, target);
    if (a->splits > kMaxSplits) return fail(SLIMKV_EINVAL, "too many splits");
    const size_t rows = (size_t)B * Hq * Lq * plan->sp.splits;
    plan->ml_off = 0;
    plan->acc_off = align256(rows * 2 * sizeof(float));
    plan->total = plan->acc_off + align256(rows * (size_t)a->width_v * sizeof(float));
    return SLIMKV_OK;
}

}  // namespace

void set_error(const std::string& msg) { g_error = msg; }

int fail(int code, const std::string& msg) {
    g_error = msg;
    return code;
}

int check_hip(hipError_t err, const char* what) {
    if (err == hipSuccess) return SLIMKV_OK;
    return fail(SLIMKV_EHIP, std::string(what) + ": " + hipGetErrorString(err));
}

int device_cu_count() {
    static std::mutex mu;
    static std::vector<int> counts;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if ((int)counts.size() <= dev) counts.resize(dev + 1, 0);
    if (!counts[dev]) {
        int cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0) cu = 256;
        counts[dev] = cu;
    }
    return counts[dev];
}

}  // namespace slimkv

using namespace slimkv;

extern "C" const char* slimkv_last_error(void) { return g_error.c_str(); }

extern "C" int slimkv_abi_version(void) { return 15; }

extern "C" size_t slimkv_attention_workspace(const slimkv_attention_args* a) {
    AttnPlan plan{};
    if (plan_attention(a, &plan) != SLIMKV_OK) return 0;
    return plan.total;
}

extern "C" int slimkv_attention_forward(const slimkv_attention_args* a, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    AttnPlan plan{};
    int rc = plan_attention(a, &plan);
    if (rc != SLIMKV_OK) return rc;
    if (!workspace || workspace_bytes < plan.total) return fail(SLIMKV_EWORKSPACE, "workspace too small");
    char* ws = static_cast<char*>(workspace);
    const int Hq = (int)a->heads, Lq = (int)a->queries, Hk = (int)a->kv_heads;
    SplitParams prm{};
    prm.nseg = 1;
    prm.B = (int)a->batch;
    prm.Lq = Lq;
    prm.Hq = Hq;
    prm.scale_log2 = (float)(a->scale * 1.4426950408889634);
    Seg& sg = prm.seg[0];
    sg.q = static_cast<const uint16_t*>(a->q); sg.q_sb = a->q_sb; sg.q_sl = a->q_sl; sg.q_sh = a->q_sh;
    sg.k = static_cast<const uint16_t*>(a->k); sg.k_sb = a->k_sb; sg.k_sn = a->k_sn; sg.k_sh = a->k_sh;
    sg.v = static_cast<const uint16_t*>(a->v); sg.v_sb = a->v_sb; sg.v_sn = a->v_sn; sg.v_sh = a->v_sh;
    sg.seqlens = a->seqlens;
    sg.n = (int)a->keys;
    sg.hk = Hk;
    sg.g = Hq / Hk;
    sg.wk = (int)a->width_k;
    sg.wv = (int)a->width_v;
    sg.causal = a->causal ? 1 : 0;
    sg.tiles = plan.sp.tiles;
    sg.cols = plan.sp.cols;
    sg.splits = plan.sp.splits;
    sg.rows_per_split = plan.sp.rows_per_split;
    sg.part_ml = reinterpret_cast<float*>(ws + plan.ml_off);
    sg.part_acc = reinterpret_cast<float*>(ws + plan.acc_off);
    sg.wown = (int)a->width_v;
    sg.nwg = plan.sp.nwg;
    hipStream_t st = static_cast<hipStream_t>(stream);
    rc = check_hip(launch_split_any(plan.sp.ks, 0, prm, sg.nwg, st), "split kernel launch");
    if (rc != SLIMKV_OK) return rc;
    CombineParams cp{};
    cp.a_ml = sg.part_ml; cp.a_acc = sg.part_acc; cp.a_splits = sg.splits; cp.a_w = sg.wown;
    cp.b_splits = 0;
    cp.B = prm.B; cp.Lq = Lq; cp.Hq = Hq; cp.Hkv = Hk; cp.D = (int)a->width_v;
    cp.out = static_cast<uint16_t*>(a->out); cp.o_sb = a->o_sb; cp.o_sl = a->o_sl; cp.o_sh = a->o_sh;
    cp.lse = a->lse;
    launch_combine(cp, prm.B * Hq * Lq, st);
    return check_hip(hipGetLastError(), "combine kernel launch");
}

// ---------------------------------------------------------------------------
// fused latent decode
// ---------------------------------------------------------------------------

namespace {

struct LatentPlan {
    SegPlan raw, lat;
    int wq;               // q_lat width per head
    int parts;
    size_t qrot_off, qlat_off, shift_off, rml_off, racc_off, lml_off, lacc_off, total;
    size_t prologue_lds;
};

// Beacon rows read straight out of pages (slimkv_paged_latent_decode).
struct PagedRows {
    const uint16_t* pages; int64_t num_pages, page_stride;
    const int64_t* table; int64_t t_sb, t_cols;
    int64_t slots, sink, rows_total;
    int32_t* status;
    // raw rows through raw pages (raw_pages null: dense base.raw_k / raw_v)
    const uint16_t* raw_pages; int64_t raw_blocks, raw_block;
    int64_t raw_blk_stride, raw_tok_stride, raw_kind_stride, raw_head_stride;
    const int64_t* raw_table; int64_t raw_t_sb, raw_t_cols;
};

int check_paged(const slimkv_latent_decode_args* a, const PagedRows* pg) {
    if (!pg->pages || !pg->table || !a->lat_lengths) return fail(SLIMKV_EINVAL, "paged decode needs pages, table and lengths");
    if (pg->num_pages <= 0 || pg->slots <= 0 || pg->sink < 0 || pg->t_cols <= 0 || pg->t_sb < pg->t_cols)
        return fail(SLIMKV_EINVAL, "invalid page geometry or block-table shape");
    if (pg->num_pages >= ((int64_t)1 << 31) || pg->num_pages > ((int64_t)1 << 40) / std::max<int64_t>(pg->page_stride, 1))
        return fail(SLIMKV_EINVAL, "page pool too large");
    if (!aligned8(pg->page_stride) || !aligned8(pg->sink) || !ptr_aligned16(pg->pages))
        return fail(SLIMKV_EINVAL, "page stride and sink must be multiples of 8 elements, pages 16-byte aligned");
    if (pg->sink + pg->slots * (a->rank_k + a->rank_v) > pg->page_stride)
        return fail(SLIMKV_EINVAL, "beacon slots do not fit in a page");
    if (a->lat_keys > 0 && (a->lat_keys + pg->slots - 1) / pg->slots > pg->t_cols)
        return fail(SLIMKV_EINVAL, "block table narrower than the beacon count");
    if (pg->slots > (1 << 20) || pg->rows_total < 0) return fail(SLIMKV_EINVAL, "invalid page geometry");
    if (pg->raw_pages) {
        const int64_t blk = pg->raw_block;
        if (!pg->raw_table || !a->raw_lengths) return fail(SLIMKV_EINVAL, "raw pages need a raw table and raw lengths");
        if (a->lat_keys <= 0) return fail(SLIMKV_EUNSUP, "raw pages are read beside beacon rows (lat_keys > 0)");
        if (blk < 16 || blk > (1 << 20) || (blk & (blk - 1)) || pg->raw_blocks <= 0 || pg->raw_blocks >= ((int64_t)1 << 31) ||
            pg->raw_t_cols <= 0 || pg->raw_t_sb < pg->raw_t_cols)
            return fail(SLIMKV_EINVAL, "invalid raw page geometry (block size a power of two >= 16)");
        if ((a->raw_keys + blk - 1) / blk > pg->raw_t_cols)
            return fail(SLIMKV_EINVAL, "raw block table narrower than the raw row count");
        if (!aligned8(pg->raw_blk_stride) || !aligned8(pg->raw_tok_stride) || !aligned8(pg->raw_kind_stride) ||
            !aligned8(pg->raw_head_stride) || !ptr_aligned16(pg->raw_pages))
            return fail(SLIMKV_EINVAL, "raw page strides must be multiples of 8 elements, pages 16-byte aligned");
        if (pg->raw_blocks > ((int64_t)1 << 40) / std::max<int64_t>(pg->raw_blk_stride, 1))
            return fail(SLIMKV_EINVAL, "raw page pool too large");
    }
    return SLIMKV_OK;
}

int plan_latent(const slimkv_latent_decode_args* a, LatentPlan* p, const PagedRows* pg = nullptr) {
    if (!a || !a->q || !a->out || !a->up_k || !a->up_v || ((!a->raw_k || !a->raw_v) && !(pg && pg->raw_pages)))
        return fail(SLIMKV_EINVAL, "null tensor pointer");
    if (pg) {
        const int rc = check_paged(a, pg);
        if (rc != SLIMKV_OK) return rc;
    }
    const int64_t B = a->batch, Lq = a->queries, Hq = a->heads, Hkv = a->kv_heads, D = a->head_dim;
    const int64_t Rk = a->rank_k, Rv = a->rank_v;
    if (B <= 0 || Lq <= 0 || Lq > 2 || Hq <= 0 || Hkv <= 0 || Hq % Hkv)
        return fail(SLIMKV_EINVAL, "invalid batch, query count (1 or 2) or GQA head counts");
    if (D != 128) return fail(SLIMKV_EUNSUP, "fused latent decode is built for head_dim 128");
    if (Rk <= 0 || Rv <= 0 || !aligned8(Rk) || !aligned8(Rv) || Rk > 384 || Rv > kMaxLatW)
        return fail(SLIMKV_EINVAL, "latent ranks must be positive multiples of 8, K rank <= 384");
    const int g = (int)(Hq / Hkv);
    if (g * Lq > kMaxRows) return fail(SLIMKV_EUNSUP, "more than 16 query rows per KV head");
    if (a->raw_keys < 0 || a->lat_keys < 0 || a->raw_keys + a->lat_keys <= 0)
        return fail(SLIMKV_EINVAL, "invalid key counts");
    if (a->raw_keys <= 0) return fail(SLIMKV_EINVAL, "the raw branch always holds the current token");
    if (!pg && a->lat_keys > 0 && (!a->lat_k || !a->lat_v)) return fail(SLIMKV_EINVAL, "null latent pointer");
    if (a->lat_k2 || a->lat_v2) {
        if (pg) return fail(SLIMKV_EINVAL, "paged rows take no second latent segment");
        if (!a->lat_k2 || !a->lat_v2 || a->lat_split <= 0 || a->lat_split >= a->lat_keys)
            return fail(SLIMKV_EINVAL, "a second latent segment needs both tensors and 0 < lat_split < lat_keys");
        if (!aligned8(a->lk2_sb) || !aligned8(a->lk2_sn) || !aligned8(a->lv2_sb) || !aligned8(a->lv2_sn) ||
            !ptr_aligned16(a->lat_k2) || !ptr_aligned16(a->lat_v2))
            return fail(SLIMKV_EINVAL, "second latent segment: strides must be multiples of 8 elements, 16-byte aligned");
        if (a->lat_keys >= ((int64_t)1 << 31)) return fail(SLIMKV_EINVAL, "too many latent rows");
    }
    if (a->cos && (!a->sin || a->rope_rows <= 0)) return fail(SLIMKV_EINVAL, "RoPE needs sin and a table size");
    if (a->cos && !a->q_positions && a->rope_rows < B * Lq)
        return fail(SLIMKV_EINVAL, "without query positions the RoPE tables hold one row per query");
    const int64_t strides[] = {a->q_sb, a->q_sl, a->q_sh, a->rk_sb, a->rk_sn, a->rk_sh, a->rv_sb, a->rv_sn,
                               a->rv_sh, a->lk_sb, a->lk_sn, a->lv_sb, a->lv_sn};
    for (int64_t st : strides)
        if (!aligned8(st)) return fail(SLIMKV_EINVAL, "strides must be multiples of 8 elements");
    if (!ptr_aligned16(a->raw_k) || !ptr_aligned16(a->raw_v) || !ptr_aligned16(a->lat_k) ||
        !ptr_aligned16(a->lat_v) || !ptr_aligned16(a->up_v))
        return fail(SLIMKV_EINVAL, "tensors must be 16-byte aligned");
    const bool bd = a->block_diagonal != 0;
    if (bd && (Rk % Hkv || Rv % Hkv || !aligned8(Rk / Hkv) || !aligned8(Rv / Hkv)))
        return fail(SLIMKV_EINVAL, "block-diagonal ranks must split into per-head multiples of 8");
    const int rk = (int)(bd ? Rk / Hkv : Rk);
    const int rv = (int)(bd ? Rv / Hkv : Rv);
    const int cu = device_cu_count();
    // Latent: every query head against shared rows.  With block-diagonal bases a
    // tile spans only its own heads' latent slices; narrow tiles (8 packed rows)
    // keep the slice span -- and the register footprint -- small.
    const int P = (int)(Lq * Hq);
    auto span_of = [&](int cols) {
        if (!bd) return (int)std::max(Rk, Rv);
        int worst = 0;
        for (int t = 0; t * cols < P; ++t) {
            const int p0 = t * cols, pend = std::min(P, p0 + cols) - 1;
            const int blocks = (pend / (int)Lq) / g - (p0 / (int)Lq) / g + 1;
            worst = std::max(worst, blocks * std::max(rk, rv));
        }
        return worst;
    };
    // Whole KV heads a wave with per-head bases: four at ranks up to 16, else
    // two -- a 64-column tile at ranks 16 and 32, 96 at rank 48 -- as many as
    // fit the MFMA's sixteen query rows and divide the KV heads, so no tile
    // spans a head it shares with the next tile and a sequence's waves split
    // each latent row evenly (B16 32K layers, GQA group of four: rank 16 with
    // four heads a wave 24.4 us against 27.7 with two; rank 48 with two heads
    // against four faster).  Eight rows for every group before: a group of
    // five got tiles of two or three KV heads and read every latent row 1.5
    // times (rank 32: 51.1 against 34.1 us); a group of eight, or four with
    // two queries, one head a tile (ranks 32 / 48: 40.0 / 68.4 against 34.9 /
    // 51.6 us); a group of two, four heads a tile (ranks 16 / 32 / 48: 26.9 /
    // 36.9 / 55.6 against 22.7 / 32.9 / 48.3 us).  General bases: eight query
    // rows a tile, every tile reads whole rows.
    int cols = 8;
    if (bd) {
        int heads = std::max(1, std::min(std::max(rk, rv) <= 16 ? 4 : 2, kMaxRows / (g * (int)Lq)));
        while (Hkv % heads) --heads;
        cols = heads * g * (int)Lq;
    }
    const int span = span_of(cols);
    const int lat_ks = round_even_tile(span);
    if (lat_ks < 0) return fail(SLIMKV_EUNSUP, "latent width not supported");
    const int64_t nl = std::max<int64_t>(a->lat_keys, 1);
    const int has_lat = a->lat_keys > 0;
    // Raw rows: splits of two 16-row tiles (four beside paged rows, whose
    // many short sequences would otherwise launch a raw workgroup per 32 rows
    // of every sequence: 64 sequences, 138 against 144 us a step).
    const int raw_rows = pg ? 64 : 32;
    const int raw_req0 =
        a->raw_splits > 0 ? a->raw_splits : (int)std::max<int64_t>(1, (a->raw_keys + raw_rows - 1) / raw_rows);
    // Dense rows: a whole number of latent workgroups per CU.  Each CU streams
    // its workgroups' rows at about the same rate, so a launch whose
    // workgroups do not spread evenly over the CUs lasts as long as its most
    // loaded CU (rank-32 layer, B16: 16 splits = 256 workgroups, one a CU,
    // 25.4 us; 18 splits 34.4 us; 43 splits filling the resident slots
    // 30.6 us).  Tiles of 64 latent columns and wider take one workgroup a CU,
    // narrower ones two.
    int lat_target = cu * (lat_ks <= 2 ? 2 : 1);
    // Paged rows (compact schedule): 3.5 split items per CU.  The page reads
    // (2 KiB chunks through the table) want more workgroups in flight than the
    // dense rows do; 64 sequences of U[1K, 128K] tokens ran a step in 0.151 ms
    // at 3.5 per CU, 0.160 at 2.5, 0.164 at 3 and 0.168 at 4 (beacon
    // workgroups first in the grid).
    int fill_target = cu * 7 / 2;
    // Keep the latent split count within the fast combine's reach (one latent
    // partial register pass, and one split per combine thread with the raw
    // ones): at small batches the slots would otherwise fill with ever shorter
    // splits whose partials the generic combine reads serially.
    const int wown = bd ? rv : (int)Rv;
    int fast_cap = kMaxSplits;
    if (wown % 8 == 0 && wown <= kFastLatW)
        fast_cap = std::max(1, std::min(fast_lat_splits(wown, 256), 256 - raw_req0));
    // workgroups per latent split index (a wave per column tile)
    const int64_t lat_tiles = (int64_t)B * ((P + cols - 1) / cols);
    if (a->lat_splits <= 0) {
        lat_target = (int)std::min<int64_t>(lat_target, (lat_tiles * fast_cap + kWaves - 1) / kWaves);
        fill_target = (int)std::min<int64_t>(fill_target, (lat_tiles * fast_cap + kWaves - 1) / kWaves);
    }
    // Whole workgroups per CU: round the split count down, never up.
    int lat_req = a->lat_splits;
    if (lat_req <= 0 && !pg)
        lat_req = (int)std::max<int64_t>(1, std::min<int64_t>(kMaxSplits, (int64_t)lat_target * kWaves / lat_tiles));
    p->lat = plan_segment((int)B, 1, P, cols, (int)nl, span, rv, lat_req, lat_target);
    if (pg && a->lat_splits <= 0) {
        // Compact schedule: size the splits from the total row count so the
        // non-empty splits of all sequences make about fill_target items.
        const int64_t total = pg->rows_total > 0 ? pg->rows_total : B * nl;
        int64_t rps = (total + fill_target - 1) / fill_target;
        rps = std::max<int64_t>(rps, (nl + std::min(kMaxSplits, fast_cap) - 1) / std::min(kMaxSplits, fast_cap));
        rps = std::max<int64_t>(16, (rps + 15) / 16 * 16);
        p->lat.rows_per_split = (int)rps;
        p->lat.splits = (int)((nl + rps - 1) / rps);
        p->lat.nwg = wave_item_groups((int)B, p->lat.splits, p->lat.tiles);
    }
    // Raw: one column tile per KV head over the full head width (the raw set
    // is sinks + tail + current token).  Splits of two tiles measured 2-4 us
    // faster a layer than one split per tile (and 1-2 us faster than three):
    // fewer raw partials and workgroups, with the raw rows still read long
    // before the latent ones.
    p->raw = plan_segment((int)B, (int)Hkv, (int)Lq * g, 16, (int)a->raw_keys, (int)D, (int)D, raw_req0, 0);
    if (p->raw.tiles != 1 || p->raw.ks != 8) return fail(SLIMKV_EUNSUP, "raw tile shape");
    p->wq = rk;
    int parts = 1;
    while (parts < 16 && g * (int)Lq * (p->wq / 8) * parts * 2 <= 256) parts *= 2;
    p->parts = parts;
    p->prologue_lds = 0;
    size_t off = 0;
    p->qrot_off = off; off = align256(off + (size_t)B * Lq * Hq * D * 2);
    p->qlat_off = off; off = align256(off + (size_t)B * Lq * Hq * p->wq * 2);
    p->shift_off = off; off = align256(off + (size_t)B * Hq * Lq * 4);
    const size_t rr = (size_t)B * Hq * Lq * p->raw.splits;
    p->rml_off = off; off = align256(off + rr * 8);
    p->racc_off = off; off = align256(off + rr * D * 4);
    const size_t lr = (size_t)B * Hq * Lq * p->lat.splits;
    p->lml_off = off; off = align256(off + lr * 8);
    p->lacc_off = off; off = align256(off + lr * (size_t)rv * 4);
    p->total = off;
    return SLIMKV_OK;
}

}  // namespace

extern "C" size_t slimkv_latent_decode_workspace(const slimkv_latent_decode_args* a) {
    LatentPlan p{};
    if (plan_latent(a, &p) != SLIMKV_OK) return 0;
    return p.total;
}

namespace {

int check_stages(int stages) {
    if (stages <= 0 || stages > SLIMKV_STAGE_ALL) return fail(SLIMKV_EINVAL, "stages must be a nonempty mask of SLIMKV_STAGE_*");
    return SLIMKV_OK;
}

// Prologue (query RoPE + absorption into the workspace), split-K attention
// (partials into the workspace), combine (merge + V lift into the output):
// the stages in `stages` run in that order and hand over through the workspace.
int latent_decode_run(const slimkv_latent_decode_args* a, const PagedRows* pg, void* workspace,
                      size_t workspace_bytes, void* stream, int stages = SLIMKV_STAGE_ALL) {
    int rc = check_stages(stages);
    if (rc != SLIMKV_OK) return rc;
    LatentPlan p{};
    rc = plan_latent(a, &p, pg);
    if (rc != SLIMKV_OK) return rc;
    if (!workspace || workspace_bytes < p.total) return fail(SLIMKV_EWORKSPACE, "workspace too small");
    char* ws = static_cast<char*>(workspace);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int B = (int)a->batch, Lq = (int)a->queries, Hq = (int)a->heads, Hkv = (int)a->kv_heads;
    const int D = (int)a->head_dim, Rk = (int)a->rank_k, Rv = (int)a->rank_v;
    const int g = Hq / Hkv;
    const bool bd = a->block_diagonal != 0;
    const bool has_lat = a->lat_keys > 0;

    uint16_t* q_rot = reinterpret_cast<uint16_t*>(ws + p.qrot_off);
    uint16_t* q_lat = reinterpret_cast<uint16_t*>(ws + p.qlat_off);
    float* shift = reinterpret_cast<float*>(ws + p.shift_off);

    PrologueParams pp{};
    pp.q = static_cast<const uint16_t*>(a->q); pp.q_sb = a->q_sb; pp.q_sl = a->q_sl; pp.q_sh = a->q_sh;
    pp.pos = a->q_positions; pp.pos_sb = a->pos_sb;
    pp.cos = a->cos; pp.sin = a->sin; pp.rope_rows = a->rope_rows;
    pp.q_rot = q_rot;
    pp.up_k = static_cast<const uint16_t*>(a->up_k);
    pp.up_k_bias = static_cast<const uint16_t*>(a->up_k_bias);
    pp.blockdiag = bd ? 1 : 0;
    pp.wq = has_lat ? p.wq : 0;
    pp.q_lat = q_lat;
    pp.shift = (has_lat && a->up_k_bias) ? shift : nullptr;
    pp.B = B; pp.Lq = Lq; pp.Hq = Hq; pp.Hkv = Hkv; pp.D = D; pp.Rk = Rk; pp.parts = p.parts;
    pp.scale = (float)a->scale;
    pp.ut = static_cast<const uint16_t*>(a->up_k_t);
    const int nct = pp.wq / 16;
    const bool mfma_prologue = has_lat && bd && pp.ut && pp.wq % 16 == 0 && nct >= 1 && nct <= 3 &&
                               g * Lq <= 16 && ptr_aligned16(pp.ut) && ptr_aligned16(a->q) &&
                               (!a->up_k_bias || ptr_aligned16(a->up_k_bias));
    // With per-head bases, a call that runs the prologue and the attend stage
    // together makes the query operands inside the split kernel (its raw waves
    // rotate their rows and, with a K bias, write the rows' LSE shifts; its
    // latent waves rotate and absorb theirs): two launches a layer instead of
    // three, the same bits.
    const bool fused = mfma_prologue && (stages & SLIMKV_STAGE_PROLOGUE) && (stages & SLIMKV_STAGE_ATTEND) &&
                       split_fq_ok(p.lat.ks, pg != nullptr, pg ? (int)pg->slots : 0);
    if (fused || !(stages & SLIMKV_STAGE_PROLOGUE)) {
        // the query operands of an earlier prologue stage are in the workspace
    } else if (mfma_prologue) {
        if (nct == 1) hipLaunchKernelGGL(prologue_mfma_kernel<1>, dim3(B * Hkv), dim3(64), 0, st, pp);
        else if (nct == 2) hipLaunchKernelGGL(prologue_mfma_kernel<2>, dim3(B * Hkv), dim3(64), 0, st, pp);
        else hipLaunchKernelGGL(prologue_mfma_kernel<3>, dim3(B * Hkv), dim3(64), 0, st, pp);
    } else {
        hipLaunchKernelGGL(prologue_kernel, dim3(B * Hkv), dim3(256), 0, st, pp);
    }
    rc = check_hip(hipGetLastError(), "prologue kernel launch");
    if (rc != SLIMKV_OK) return rc;

    SplitParams prm{};
    prm.B = B; prm.Lq = Lq; prm.Hq = Hq;
    prm.scale_log2 = (float)(a->scale * 1.4426950408889634);
    prm.nseg = has_lat ? 2 : 1;
    if (fused) {
        prm.qrope = QRope{pp.q, pp.q_sb, pp.q_sl, pp.q_sh, pp.pos, pp.pos_sb, pp.cos, pp.sin, pp.rope_rows};
        prm.absorb = QAbsorb{pp.ut, pp.wq};
        if (pp.shift) prm.kshift = QShift{pp.up_k_bias, pp.shift, pp.scale};
    }
    // Latent rows (the bulk, pipelined) are segment 0; the short raw segment is
    // segment 1, whose workgroups split_kernel places first in the grid.
    Seg& r = prm.seg[has_lat ? 1 : 0];
    r.q = q_rot; r.q_sb = (int64_t)Lq * Hq * D; r.q_sl = (int64_t)Hq * D; r.q_sh = D;
    r.k = static_cast<const uint16_t*>(a->raw_k); r.k_sb = a->rk_sb; r.k_sn = a->rk_sn; r.k_sh = a->rk_sh;
    r.v = static_cast<const uint16_t*>(a->raw_v); r.v_sb = a->rv_sb; r.v_sn = a->rv_sn; r.v_sh = a->rv_sh;
    r.seqlens = a->raw_lengths;
    r.n = (int)a->raw_keys;
    r.hk = Hkv; r.g = g; r.wk = D; r.wv = D; r.causal = 0;
    r.tiles = p.raw.tiles; r.cols = p.raw.cols; r.splits = p.raw.splits; r.rows_per_split = p.raw.rows_per_split;
    r.part_ml = reinterpret_cast<float*>(ws + p.rml_off);
    r.part_acc = reinterpret_cast<float*>(ws + p.racc_off);
    r.wown = D;
    r.nwg = p.raw.nwg;
    if (pg && pg->raw_pages && has_lat) {
        r.k = pg->raw_pages; r.k_sb = 0; r.k_sn = pg->raw_tok_stride; r.k_sh = pg->raw_head_stride;
        r.v = pg->raw_pages + pg->raw_kind_stride; r.v_sb = 0; r.v_sn = pg->raw_tok_stride;
        r.v_sh = pg->raw_head_stride;
        r.status = pg->status;
        prm.rawp.table = pg->raw_table; prm.rawp.t_sb = pg->raw_t_sb;
        prm.rawp.blk_stride = pg->raw_blk_stride; prm.rawp.num_blocks = pg->raw_blocks;
        prm.rawp.block_shift = __builtin_ctzll((unsigned long long)pg->raw_block);
    }
    int ka = 8, kb = 0;
    if (has_lat) {
        Seg& l = prm.seg[0];
        l.q = q_lat; l.q_sb = (int64_t)Lq * Hq * p.wq; l.q_sl = (int64_t)Hq * p.wq; l.q_sh = p.wq;
        l.k = static_cast<const uint16_t*>(a->lat_k); l.k_sb = a->lk_sb; l.k_sn = a->lk_sn; l.k_sh = 0;
        l.v = static_cast<const uint16_t*>(a->lat_v); l.v_sb = a->lv_sb; l.v_sn = a->lv_sn; l.v_sh = 0;
        l.seqlens = a->lat_lengths;
        l.n = (int)a->lat_keys;
        l.hk = 1; l.g = Hq; l.wk = Rk; l.wv = Rv; l.causal = a->lat_causal ? 1 : 0;
        l.tiles = p.lat.tiles; l.cols = p.lat.cols; l.splits = p.lat.splits;
        l.rows_per_split = p.lat.rows_per_split;
        if (bd) {
            l.blk_heads = g; l.blk_k = Rk / Hkv; l.blk_v = Rv / Hkv; l.q_compact = 1;
        }
        l.part_ml = reinterpret_cast<float*>(ws + p.lml_off);
        l.part_acc = reinterpret_cast<float*>(ws + p.lacc_off);
        l.wown = bd ? Rv / Hkv : Rv;
        l.nwg = p.lat.nwg;
        if (a->lat_k2) {
            prm.two.k2 = static_cast<const uint16_t*>(a->lat_k2); prm.two.k2_sb = a->lk2_sb; prm.two.k2_sn = a->lk2_sn;
            prm.two.v2 = static_cast<const uint16_t*>(a->lat_v2); prm.two.v2_sb = a->lv2_sb; prm.two.v2_sn = a->lv2_sn;
            prm.two.n1 = (int)a->lat_split;
        }
        if (pg) {
            l.k = pg->pages + pg->sink; l.v = pg->pages + pg->sink + Rk;
            l.k_sb = l.v_sb = 0; l.k_sn = l.v_sn = Rk + Rv;
            l.table = pg->table; l.t_sb = pg->t_sb; l.page_stride = pg->page_stride; l.num_pages = pg->num_pages;
            l.slots = (int)pg->slots;
            l.slots_shift = (pg->slots & (pg->slots - 1)) == 0 ? __builtin_ctzll((unsigned long long)pg->slots) : -1;
            l.status = pg->status;
            l.compact = 1;
        }
        ka = p.lat.ks;
        kb = 8;
    }
    const bool paged = pg && has_lat;
    if (paged && ka > 8) return fail(SLIMKV_EUNSUP, "paged decode handles latent tiles up to 128 wide");
    const int grid = prm.seg[0].nwg + (has_lat ? prm.seg[1].nwg : 0);
    if (stages & SLIMKV_STAGE_ATTEND) {
        const bool seg2 = has_lat && a->lat_k2 != nullptr;
        rc = check_hip(fused ? launch_split_fused(ka, prm, grid, st, paged, seg2)
                             : launch_split_any(ka, kb, prm, grid, st, paged, seg2),
                       "split kernel launch");
        if (rc != SLIMKV_OK) return rc;
    }
    if (!(stages & SLIMKV_STAGE_COMBINE)) return SLIMKV_OK;

    CombineParams cp{};
    cp.a_ml = r.part_ml; cp.a_acc = r.part_acc; cp.a_splits = r.splits; cp.a_w = D;
    if (has_lat) {
        cp.b_ml = prm.seg[0].part_ml; cp.b_acc = prm.seg[0].part_acc;
        cp.b_splits = prm.seg[0].splits; cp.b_w = prm.seg[0].wown;
        cp.up_v = static_cast<const uint16_t*>(a->up_v); cp.up_v_ld = Rv;
        cp.up_v_bias = static_cast<const uint16_t*>(a->up_v_bias);
        cp.blockdiag = bd ? 1 : 0;
        cp.b_shift = pp.shift;
        if (prm.seg[0].compact) {
            cp.b_len = a->lat_lengths; cp.b_rps = prm.seg[0].rows_per_split; cp.b_n = prm.seg[0].n;
        }
    }
    cp.B = B; cp.Lq = Lq; cp.Hq = Hq; cp.Hkv = Hkv; cp.D = D;
    cp.out = static_cast<uint16_t*>(a->out); cp.o_sb = a->o_sb; cp.o_sl = a->o_sl; cp.o_sh = a->o_sh;
    cp.lse = a->lse;
    launch_combine(cp, B * Hq * Lq, st);
    return check_hip(hipGetLastError(), "combine kernel launch");
}

PagedRows paged_rows(const slimkv_paged_latent_decode_args* a) {
    return PagedRows{static_cast<const uint16_t*>(a->pages), a->num_pages, a->page_stride, a->table, a->t_sb,
                     a->t_cols, a->slots, a->sink_elements, a->rows_total, a->status,
                     static_cast<const uint16_t*>(a->raw_pages), a->raw_num_blocks, a->raw_block_size,
                     a->raw_block_stride, a->raw_token_stride, a->raw_kind_stride, a->raw_head_stride, a->raw_table,
                     a->raw_t_sb, a->raw_t_cols};
}

}  // namespace

extern "C" int slimkv_latent_decode(const slimkv_latent_decode_args* a, void* workspace,
                                    size_t workspace_bytes, void* stream) {
    return latent_decode_run(a, nullptr, workspace, workspace_bytes, stream);
}

extern "C" int slimkv_latent_decode_stages(const slimkv_latent_decode_args* a, int stages, void* workspace,
                                           size_t workspace_bytes, void* stream) {
    return latent_decode_run(a, nullptr, workspace, workspace_bytes, stream, stages);
}

// ---------------------------------------------------------------------------
// allocation-free latent decode: the workspace is a file-scope device array
// ---------------------------------------------------------------------------

// One copy per GPU, allocated when the library's code object is loaded on that
// GPU and held until the process ends.  In host code `scratch` names a
// host-side stand-in: its device address comes from hipGetSymbolAddress.
static __device__ __align__(256) unsigned char scratch[SLIMKV_NOALLOC_SCRATCH_BYTES];

namespace {

std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;   // device address of `scratch`, per device ordinal

// The address of the current device's `scratch`, looked up once per device
// with that device current.
int scratch_address(void** out) {
    int dev = 0;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc != SLIMKV_OK) return rc;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (rc != SLIMKV_OK) return rc;
        if (!p) return fail(SLIMKV_EHIP, "hipGetSymbolAddress(scratch) returned a null address");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return SLIMKV_OK;
}

}  // namespace

extern "C" int slimkv_latent_decode_noalloc(const slimkv_latent_decode_args* a, void* stream) {
    LatentPlan p{};
    int rc = plan_latent(a, &p);
    if (rc != SLIMKV_OK) return rc;
    if (p.total > (size_t)SLIMKV_NOALLOC_SCRATCH_BYTES)
        return fail(SLIMKV_EWORKSPACE, "slimkv_latent_decode_noalloc: this call needs " + std::to_string(p.total) +
                                           " bytes of workspace, more than the " +
                                           std::to_string((size_t)SLIMKV_NOALLOC_SCRATCH_BYTES) +
                                           "-byte device scratch; use slimkv_latent_decode with a caller workspace");
    void* ws = nullptr;
    rc = scratch_address(&ws);
    if (rc != SLIMKV_OK) return rc;
    return latent_decode_run(a, nullptr, ws, (size_t)SLIMKV_NOALLOC_SCRATCH_BYTES, stream);
}

extern "C" size_t slimkv_paged_latent_decode_workspace(const slimkv_paged_latent_decode_args* a) {
    if (!a) return 0;
    const PagedRows pg = paged_rows(a);
    LatentPlan p{};
    if (plan_latent(&a->base, &p, &pg) != SLIMKV_OK) return 0;
    return p.total;
}

extern "C" int slimkv_paged_latent_decode(const slimkv_paged_latent_decode_args* a, void* workspace,
                                          size_t workspace_bytes, void* stream) {
    if (!a) return fail(SLIMKV_EINVAL, "null arguments");
    const PagedRows pg = paged_rows(a);
    return latent_decode_run(&a->base, &pg, workspace, workspace_bytes, stream);
}

extern "C" int slimkv_paged_latent_decode_stages(const slimkv_paged_latent_decode_args* a, int stages,
                                                 void* workspace, size_t workspace_bytes, void* stream) {
    if (!a) return fail(SLIMKV_EINVAL, "null arguments");
    const PagedRows pg = paged_rows(a);
    return latent_decode_run(&a->base, &pg, workspace, workspace_bytes, stream, stages);
}

// ---------------------------------------------------------------------------
// reconstruction decode
// ---------------------------------------------------------------------------

namespace {

struct ReconPlan {
    SegPlan raw, rec;
    int v_latent, v_width;   // V stays latent (width v_width per KV head) and is lifted in the combine
    int fused, ksr, vl;      // K rebuilt per tile inside the split kernel (recon_split_kernel<ksr, vl>)
    size_t qrot_off, k_off, v_off, rml_off, racc_off, bml_off, bacc_off, total;
};

// The fused route: block-diagonal bases, per-head K rank 16, 32 or 48 and V
// rank 32 or 64, the alignment its 8- and 16-byte loads need, and prepared RoPE pairs
// when the beacon keys are rotated.
bool recon_fused_ok(const slimkv_recon_decode_args* r) {
    const slimkv_latent_decode_args* a = &r->base;
    if (a->lat_keys <= 0 || !a->block_diagonal) return false;
    const int64_t Hkv = a->kv_heads;
    if (a->rank_k % Hkv || a->rank_v % Hkv) return false;
    const int64_t rk = a->rank_k / Hkv, rv = a->rank_v / Hkv;
    if (rk % 16 || rk < 16 || rk > 48 || (rv != 32 && rv != 64) || (rk == 48 && rv == 64)) return false;
    auto al = [](const void* ptr, uintptr_t m) { return (reinterpret_cast<uintptr_t>(ptr) & (m - 1)) == 0; };
    // 16-byte latent K and U_K pieces at per-head K ranks of 32 and 48 (the
    // 32-deep rebuild MFMA), 8-byte ones at 16
    const int64_t km = rk >= 32 ? 8 : 4;
    if (!al(a->lat_k, 2 * km) || (a->lk_sb % km) || (a->lk_sn % km) || !al(a->up_k, 2 * km) || (a->rank_k % km))
        return false;
    if (a->up_k_bias && !al(a->up_k_bias, 8)) return false;
    if (!al(a->lat_v, 16) || !aligned8(a->lv_sb) || !aligned8(a->lv_sn)) return false;
    if (!al(a->up_v, 16) || !aligned8(a->rank_v)) return false;
    if (r->beacon_positions && (!r->rope_pairs || !r->rope_repeats || !al(r->rope_pairs, 16) || a->rope_rows <= 0))
        return false;
    return true;
}

// V is linear in its latent, so sum_n p_n (U_V l_n + b) = U_V (sum_n p_n l_n) + b sum_n p_n:
// the split kernel can attend over the latent rows and the combine lifts once per
// (b, head).  K cannot follow when beacon keys are rotated after the
// up-projection, so only V takes this route; it needs the latent decode's layout.
bool recon_v_latent(const slimkv_latent_decode_args* a) {
    if (a->lat_keys <= 0 || !a->lat_v) return false;
    const bool bd = a->block_diagonal != 0;
    if (bd && a->rank_v % a->kv_heads) return false;
    const int64_t w = bd ? a->rank_v / a->kv_heads : a->rank_v;
    return w > 0 && w <= a->head_dim && aligned8(w) && aligned8(a->rank_v) && aligned8(a->lv_sb) &&
           aligned8(a->lv_sn) && ptr_aligned16(a->lat_v) && ptr_aligned16(a->up_v);
}

int plan_recon(const slimkv_recon_decode_args* r, ReconPlan* p) {
    const slimkv_latent_decode_args* a = &r->base;
    if (!a->q || !a->raw_k || !a->raw_v || !a->out || !a->up_k || !a->up_v) return fail(SLIMKV_EINVAL, "null tensor pointer");
    const int64_t B = a->batch, Lq = a->queries, Hq = a->heads, Hkv = a->kv_heads, D = a->head_dim;
    if (B <= 0 || Lq <= 0 || Lq > 2 || Hq <= 0 || Hkv <= 0 || Hq % Hkv) return fail(SLIMKV_EINVAL, "invalid sizes");
    if (D != 128) return fail(SLIMKV_EUNSUP, "reconstruction decode is built for head_dim 128");
    if (a->raw_keys <= 0 || a->lat_keys < 0) return fail(SLIMKV_EINVAL, "invalid key counts");
    if (a->lat_keys > 0 && (!a->lat_k || !a->lat_v)) return fail(SLIMKV_EINVAL, "null latent pointer");
    if (r->beacon_positions && B > 1 && r->bpos_sb < a->lat_keys)
        return fail(SLIMKV_EINVAL, "beacon position rows are shorter than the beacon count");
    if (r->beacon_positions && !a->cos) return fail(SLIMKV_EINVAL, "beacon RoPE needs the tables");
    if (a->cos && (!a->sin || a->rope_rows <= 0)) return fail(SLIMKV_EINVAL, "RoPE needs sin and a table size");
    if (a->cos && !a->q_positions && (r->beacon_positions || a->rope_rows < B * Lq))
        return fail(SLIMKV_EINVAL, "beacon RoPE needs the full tables and query positions");
    const int g = (int)(Hq / Hkv);
    if (g * Lq > kMaxRows) return fail(SLIMKV_EUNSUP, "more than 16 query rows per KV head");
    const int cu = device_cu_count();
    const int nl = (int)std::max<int64_t>(a->lat_keys, 1);
    // raw rows in splits of two 16-row tiles (as the latent decode)
    const int raw_req = a->raw_splits > 0 ? a->raw_splits : (int)std::max<int64_t>(1, (a->raw_keys + 31) / 32);
    p->raw = plan_segment((int)B, (int)Hkv, (int)Lq * g, 16, (int)a->raw_keys, (int)D, (int)D, raw_req, 0);
    p->fused = recon_fused_ok(r) ? 1 : 0;
    if (p->fused) {
        p->ksr = (int)(a->rank_k / Hkv / 16);
        p->vl = (int)(a->rank_v / Hkv / 32);
        // One beacon workgroup per CU (the split count rounded down): a
        // launch whose workgroups do not spread evenly over the CUs lasts as
        // long as its most loaded CU, and two per CU measured slower than one
        // (B8 layer, 40/8 heads, 8192 beacons of rank 32: 16 splits, one a
        // CU, 34.8 us; 32 splits 40.1 us; 8, 12, 20, 24 or 48 splits 41.6-52.9
        // us).  The short raw workgroups run ahead of them.
        const int64_t groups = (int64_t)B * ((Hkv + kWaves - 1) / kWaves);
        // as for the latent decode: stay within the fast combine's split count
        const int wv = 32 * p->vl;
        const int fast_cap = std::max(1, std::min(fast_lat_splits(wv, 256), 256 - raw_req));
        int req = a->lat_splits;
        if (req <= 0) req = (int)std::max<int64_t>(1, std::min<int64_t>({(int64_t)cu / groups, fast_cap, kMaxSplits}));
        p->rec = plan_segment((int)B, (int)Hkv, (int)Lq * g, 16, nl, (int)D, wv, req, 0);
        // recon_split_kernel: a workgroup per (b, group of kWaves KV heads, split)
        p->rec.nwg = (int)(groups * p->rec.splits);
    } else {
        p->rec = plan_segment((int)B, (int)Hkv, (int)Lq * g, 16, nl, (int)D, (int)D, a->lat_splits,
                              cu * split_occupancy(8, 8));
    }
    size_t off = 0;
    p->v_latent = (p->fused || recon_v_latent(a)) ? 1 : 0;
    p->v_width = p->v_latent ? (int)(a->block_diagonal ? a->rank_v / Hkv : a->rank_v) : (int)D;
    p->qrot_off = off; off = align256(off + (size_t)B * Lq * Hq * D * 2);
    p->k_off = off; off = align256(off + (p->fused ? 0 : (size_t)B * nl * Hkv * D * 2));
    p->v_off = off; off = align256(off + (p->v_latent ? 0 : (size_t)B * nl * Hkv * D * 2));
    const size_t rr = (size_t)B * Hq * Lq * p->raw.splits;
    p->rml_off = off; off = align256(off + rr * 8);
    p->racc_off = off; off = align256(off + rr * D * 4);
    const size_t br = (size_t)B * Hq * Lq * p->rec.splits;
    p->bml_off = off; off = align256(off + br * 8);
    p->bacc_off = off; off = align256(off + br * D * 4);
    p->total = off;
    return SLIMKV_OK;
}

// Raw rows and rebuilt-per-tile beacon rows in one launch, then the combine
// with the latent V lift.  q_rot already holds the rotated queries.
int recon_fused_run(const slimkv_recon_decode_args* r, const ReconPlan& p, char* ws, uint16_t* q_rot, hipStream_t st,
                    int stages) {
    const slimkv_latent_decode_args* a = &r->base;
    const int B = (int)a->batch, Lq = (int)a->queries, Hq = (int)a->heads, Hkv = (int)a->kv_heads, D = (int)a->head_dim;
    const int g = Hq / Hkv;
    SplitParams prm{};
    prm.B = B; prm.Lq = Lq; prm.Hq = Hq;
    prm.scale_log2 = (float)(a->scale * 1.4426950408889634);
    prm.nseg = 1;
    Seg& rs = prm.seg[0];
    rs.q = q_rot; rs.q_sb = (int64_t)Lq * Hq * D; rs.q_sl = (int64_t)Hq * D; rs.q_sh = D;
    rs.k = static_cast<const uint16_t*>(a->raw_k); rs.k_sb = a->rk_sb; rs.k_sn = a->rk_sn; rs.k_sh = a->rk_sh;
    rs.v = static_cast<const uint16_t*>(a->raw_v); rs.v_sb = a->rv_sb; rs.v_sn = a->rv_sn; rs.v_sh = a->rv_sh;
    rs.seqlens = a->raw_lengths; rs.n = (int)a->raw_keys;
    rs.hk = Hkv; rs.g = g; rs.wk = D; rs.wv = D; rs.causal = 0;
    rs.tiles = p.raw.tiles; rs.cols = p.raw.cols; rs.splits = p.raw.splits; rs.rows_per_split = p.raw.rows_per_split;
    rs.part_ml = reinterpret_cast<float*>(ws + p.rml_off); rs.part_acc = reinterpret_cast<float*>(ws + p.racc_off);
    rs.wown = D; rs.nwg = p.raw.nwg;

    QRope& qr = prm.qrope;
    qr.q = static_cast<const uint16_t*>(a->q); qr.q_sb = a->q_sb; qr.q_sl = a->q_sl; qr.q_sh = a->q_sh;
    qr.pos = a->q_positions; qr.pos_sb = a->pos_sb;
    qr.cos = a->cos; qr.sin = a->sin; qr.rope_rows = a->rope_rows;

    ReconSeg bs{};
    bs.q = q_rot; bs.q_sb = rs.q_sb; bs.q_sl = rs.q_sl; bs.q_sh = rs.q_sh;
    bs.qr = qr;
    bs.lk = static_cast<const uint16_t*>(a->lat_k); bs.lk_sb = a->lk_sb; bs.lk_sn = a->lk_sn;
    bs.lv = static_cast<const uint16_t*>(a->lat_v); bs.lv_sb = a->lv_sb; bs.lv_sn = a->lv_sn;
    bs.w = static_cast<const uint16_t*>(a->up_k); bs.bias = static_cast<const uint16_t*>(a->up_k_bias);
    bs.w_ld = a->rank_k;
    if (r->beacon_positions) {
        bs.pairs = r->rope_pairs; bs.rope_rows = a->rope_rows;
        bs.pos = r->beacon_positions; bs.pos_sb = r->bpos_sb;
    }
    bs.seqlens = a->lat_lengths; bs.n = (int)a->lat_keys; bs.hk = Hkv; bs.g = g; bs.causal = a->lat_causal ? 1 : 0;
    bs.splits = p.rec.splits; bs.rows_per_split = p.rec.rows_per_split; bs.nwg = p.rec.nwg;
    bs.part_ml = reinterpret_cast<float*>(ws + p.bml_off); bs.part_acc = reinterpret_cast<float*>(ws + p.bacc_off);

    const int grid = rs.nwg + bs.nwg;
    int rc = SLIMKV_OK;
    if (stages & SLIMKV_STAGE_ATTEND) {
#define SLIMKV_LAUNCH(K, V)                                                                                       \
    if (p.ksr == K && p.vl == V) {                                                                                \
        if (bs.pairs && r->rope_fp32)                                                                              \
            hipLaunchKernelGGL((recon_split_kernel<K, V, 2>), dim3(grid), dim3(kThreads), 0, st, prm, bs);           \
        else if (bs.pairs)                                                                                        \
            hipLaunchKernelGGL((recon_split_kernel<K, V, 1>), dim3(grid), dim3(kThreads), 0, st, prm, bs);           \
        else                                                                                                      \
            hipLaunchKernelGGL((recon_split_kernel<K, V, 0>), dim3(grid), dim3(kThreads), 0, st, prm, bs);           \
    }
        SLIMKV_LAUNCH(1, 1) SLIMKV_LAUNCH(2, 1) SLIMKV_LAUNCH(3, 1) SLIMKV_LAUNCH(1, 2) SLIMKV_LAUNCH(2, 2)
#undef SLIMKV_LAUNCH
        rc = check_hip(hipGetLastError(), "reconstruction split kernel launch");
        if (rc != SLIMKV_OK) return rc;
    }
    if (!(stages & SLIMKV_STAGE_COMBINE)) return SLIMKV_OK;

    CombineParams cp{};
    cp.a_ml = rs.part_ml; cp.a_acc = rs.part_acc; cp.a_splits = rs.splits; cp.a_w = D;
    cp.b_ml = bs.part_ml; cp.b_acc = bs.part_acc; cp.b_splits = bs.splits; cp.b_w = 32 * p.vl;
    cp.up_v = static_cast<const uint16_t*>(a->up_v); cp.up_v_ld = a->rank_v;
    cp.up_v_bias = static_cast<const uint16_t*>(a->up_v_bias);
    cp.blockdiag = 1;
    cp.B = B; cp.Lq = Lq; cp.Hq = Hq; cp.Hkv = Hkv; cp.D = D;
    cp.out = static_cast<uint16_t*>(a->out); cp.o_sb = a->o_sb; cp.o_sl = a->o_sl; cp.o_sh = a->o_sh;
    cp.lse = a->lse;
    launch_combine(cp, B * Hq * Lq, st);
    return check_hip(hipGetLastError(), "combine kernel launch");
}

}  // namespace

extern "C" size_t slimkv_recon_decode_workspace(const slimkv_recon_decode_args* r) {
    ReconPlan p{};
    if (!r || plan_recon(r, &p) != SLIMKV_OK) return 0;
    return p.total;
}

namespace {

int recon_decode_run(const slimkv_recon_decode_args* r, void* workspace, size_t workspace_bytes, void* stream,
                     int stages) {
    if (!r) return fail(SLIMKV_EINVAL, "null arguments");
    int rc = check_stages(stages);
    if (rc != SLIMKV_OK) return rc;
    ReconPlan p{};
    rc = plan_recon(r, &p);
    if (rc != SLIMKV_OK) return rc;
    if (!workspace || workspace_bytes < p.total) return fail(SLIMKV_EWORKSPACE, "workspace too small");
    const slimkv_latent_decode_args* a = &r->base;
    char* ws = static_cast<char*>(workspace);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int B = (int)a->batch, Lq = (int)a->queries, Hq = (int)a->heads, Hkv = (int)a->kv_heads, D = (int)a->head_dim;
    const int g = Hq / Hkv;
    const bool has_lat = a->lat_keys > 0;
    uint16_t* q_rot = reinterpret_cast<uint16_t*>(ws + p.qrot_off);
    uint16_t* kbuf = reinterpret_cast<uint16_t*>(ws + p.k_off);
    uint16_t* vbuf = reinterpret_cast<uint16_t*>(ws + p.v_off);

    // 1. query RoPE (no absorption)
    PrologueParams pp{};
    pp.q = static_cast<const uint16_t*>(a->q); pp.q_sb = a->q_sb; pp.q_sl = a->q_sl; pp.q_sh = a->q_sh;
    pp.pos = a->q_positions; pp.pos_sb = a->pos_sb;
    pp.cos = a->cos; pp.sin = a->sin; pp.rope_rows = a->rope_rows;
    pp.q_rot = q_rot;
    pp.wq = 0;
    pp.B = B; pp.Lq = Lq; pp.Hq = Hq; pp.Hkv = Hkv; pp.D = D; pp.Rk = (int)a->rank_k; pp.parts = 1;
    pp.scale = (float)a->scale;
    // The fused reconstruction decode rotates its queries where its split
    // kernel reads them (no prologue launch; the prologue stage does nothing).
    if (p.fused) return recon_fused_run(r, p, ws, q_rot, st, stages);
    if (stages & SLIMKV_STAGE_PROLOGUE) {
        hipLaunchKernelGGL(prologue_kernel, dim3(B * Hkv), dim3(256), 0, st, pp);
        rc = check_hip(hipGetLastError(), "prologue kernel launch");
        if (rc != SLIMKV_OK) return rc;
    }

    // 2. rebuild beacon K (optionally RoPE'd) and, unless it stays latent, V: [B, Nl, Hkv, D]
    if (has_lat && (stages & SLIMKV_STAGE_ATTEND)) {
        for (int kind = 0; kind < (p.v_latent ? 1 : 2); ++kind) {
            slimkv_reconstruct_args ra{};
            ra.latent = kind ? a->lat_v : a->lat_k;
            ra.l_sb = kind ? a->lv_sb : a->lk_sb;
            ra.l_sn = kind ? a->lv_sn : a->lk_sn;
            ra.weight = kind ? a->up_v : a->up_k;
            ra.bias = kind ? a->up_v_bias : a->up_k_bias;
            ra.out = kind ? (void*)vbuf : (void*)kbuf;
            ra.o_sb = (int64_t)a->lat_keys * Hkv * D; ra.o_sn = (int64_t)Hkv * D; ra.o_sh = D;
            if (!kind && r->beacon_positions) {
                ra.cos = a->cos; ra.sin = a->sin; ra.rope_rows = a->rope_rows;
                ra.positions = r->beacon_positions; ra.pos_sb = r->bpos_sb;
            }
            ra.batch = B; ra.rows = a->lat_keys; ra.rank = kind ? a->rank_v : a->rank_k;
            ra.kv_heads = Hkv; ra.head_dim = D; ra.block_diagonal = a->block_diagonal;
            rc = reconstruct(&ra, st);
            if (rc != SLIMKV_OK) return rc;
        }
    }

    // 3. split-K attention over [rebuilt beacons ; raw rows]
    SplitParams prm{};
    prm.B = B; prm.Lq = Lq; prm.Hq = Hq;
    prm.scale_log2 = (float)(a->scale * 1.4426950408889634);
    prm.nseg = has_lat ? 2 : 1;
    Seg& rs = prm.seg[has_lat ? 1 : 0];
    rs.q = q_rot; rs.q_sb = (int64_t)Lq * Hq * D; rs.q_sl = (int64_t)Hq * D; rs.q_sh = D;
    rs.k = static_cast<const uint16_t*>(a->raw_k); rs.k_sb = a->rk_sb; rs.k_sn = a->rk_sn; rs.k_sh = a->rk_sh;
    rs.v = static_cast<const uint16_t*>(a->raw_v); rs.v_sb = a->rv_sb; rs.v_sn = a->rv_sn; rs.v_sh = a->rv_sh;
    rs.seqlens = a->raw_lengths; rs.n = (int)a->raw_keys;
    rs.hk = Hkv; rs.g = g; rs.wk = D; rs.wv = D; rs.causal = 0;
    rs.tiles = p.raw.tiles; rs.cols = p.raw.cols; rs.splits = p.raw.splits; rs.rows_per_split = p.raw.rows_per_split;
    rs.part_ml = reinterpret_cast<float*>(ws + p.rml_off); rs.part_acc = reinterpret_cast<float*>(ws + p.racc_off);
    rs.wown = D; rs.nwg = p.raw.nwg;
    if (has_lat) {
        Seg& bs = prm.seg[0];
        bs = rs;
        bs.k = kbuf; bs.k_sb = (int64_t)a->lat_keys * Hkv * D; bs.k_sn = (int64_t)Hkv * D; bs.k_sh = D;
        if (p.v_latent) {
            bs.v = static_cast<const uint16_t*>(a->lat_v); bs.v_sb = a->lv_sb; bs.v_sn = a->lv_sn;
            bs.v_sh = a->block_diagonal ? p.v_width : 0;
            bs.wv = p.v_width; bs.wown = p.v_width;
        } else {
            bs.v = vbuf; bs.v_sb = bs.k_sb; bs.v_sn = bs.k_sn; bs.v_sh = D;
        }
        bs.seqlens = a->lat_lengths; bs.n = (int)a->lat_keys; bs.causal = a->lat_causal ? 1 : 0;
        bs.tiles = p.rec.tiles; bs.cols = p.rec.cols; bs.splits = p.rec.splits; bs.rows_per_split = p.rec.rows_per_split;
        bs.part_ml = reinterpret_cast<float*>(ws + p.bml_off); bs.part_acc = reinterpret_cast<float*>(ws + p.bacc_off);
        bs.nwg = p.rec.nwg;
    }
    const int grid = prm.seg[0].nwg + (has_lat ? prm.seg[1].nwg : 0);
    if (stages & SLIMKV_STAGE_ATTEND) {
        rc = check_hip(launch_split_any(8, has_lat ? 8 : 0, prm, grid, st), "split kernel launch");
        if (rc != SLIMKV_OK) return rc;
    }
    if (!(stages & SLIMKV_STAGE_COMBINE)) return SLIMKV_OK;

    // 4. merge the two segments
    CombineParams cp{};
    cp.a_ml = rs.part_ml; cp.a_acc = rs.part_acc; cp.a_splits = rs.splits; cp.a_w = D;
    if (has_lat) {
        cp.b_ml = prm.seg[0].part_ml; cp.b_acc = prm.seg[0].part_acc; cp.b_splits = prm.seg[0].splits;
        cp.b_w = prm.seg[0].wown;
        if (p.v_latent) {
            cp.up_v = static_cast<const uint16_t*>(a->up_v); cp.up_v_ld = a->rank_v;
            cp.up_v_bias = static_cast<const uint16_t*>(a->up_v_bias);
            cp.blockdiag = a->block_diagonal ? 1 : 0;
        } else {
            cp.up_v = nullptr;
        }
    }
    cp.B = B; cp.Lq = Lq; cp.Hq = Hq; cp.Hkv = Hkv; cp.D = D;
    cp.out = static_cast<uint16_t*>(a->out); cp.o_sb = a->o_sb; cp.o_sl = a->o_sl; cp.o_sh = a->o_sh;
    cp.lse = a->lse;
    launch_combine(cp, B * Hq * Lq, st);
    return check_hip(hipGetLastError(), "combine kernel launch");
}

}  // namespace

extern "C" int slimkv_recon_decode(const slimkv_recon_decode_args* r, void* workspace, size_t workspace_bytes,
                                   void* stream) {
    return recon_decode_run(r, workspace, workspace_bytes, stream, SLIMKV_STAGE_ALL);
}

extern "C" int slimkv_recon_decode_stages(const slimkv_recon_decode_args* r, int stages, void* workspace,
                                          size_t workspace_bytes, void* stream) {
    return recon_decode_run(r, workspace, workspace_bytes, stream, stages);
}

// ---------------------------------------------------------------------------
// per-head transposed K bases for the in-kernel query absorption
// ---------------------------------------------------------------------------

namespace {

__global__ void __launch_bounds__(256)
prepare_bases_kernel(const uint16_t* up_k, int Hkv, int D, int R, uint16_t* out) {
    const int r = R / Hkv;
    const int64_t total = (int64_t)Hkv * r * D;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int d = (int)(i % D);
    const int c = (int)((i / D) % r);
    const int h = (int)(i / ((int64_t)D * r));
    out[i] = up_k[((int64_t)h * D + d) * R + (int64_t)h * r + c];
}

}  // namespace

__global__ void __launch_bounds__(256)
prepare_pairs_kernel(const float* cos, const float* sin, int64_t total, uint32_t* out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    out[i] = pack_bf16(cos[i], sin[i]);
}

extern "C" int slimkv_prepare_rope_pairs(const float* cos, const float* sin, int64_t rows, int64_t dim, uint32_t* out,
                                         void* stream) {
    if (!cos || !sin || !out) return fail(SLIMKV_EINVAL, "null pointer");
    if (rows <= 0 || dim <= 0 || rows > ((int64_t)1 << 40) / dim) return fail(SLIMKV_EINVAL, "invalid table size");
    const int64_t total = rows * dim;
    hipLaunchKernelGGL(prepare_pairs_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), cos, sin, total, out);
    return check_hip(hipGetLastError(), "pair preparation launch");
}

extern "C" int slimkv_prepare_latent_bases(const void* up_k, int64_t kv_heads, int64_t head_dim, int64_t rank,
                                           void* out, void* stream) {
    if (!up_k || !out) return fail(SLIMKV_EINVAL, "null pointer");
    if (kv_heads <= 0 || head_dim <= 0 || rank <= 0 || rank % kv_heads || kv_heads * head_dim * rank > (1LL << 31))
        return fail(SLIMKV_EINVAL, "invalid base shape");
    const int64_t total = kv_heads * (rank / kv_heads) * head_dim;
    hipLaunchKernelGGL(prepare_bases_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(up_k), (int)kv_heads,
                       (int)head_dim, (int)rank, static_cast<uint16_t*>(out));
    return check_hip(hipGetLastError(), "prepare bases launch");
}
