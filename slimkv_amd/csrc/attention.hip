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
// The combine kernel merges the split partials of both segments in fp32, lifts
// the latent accumulator through U_V once per (b, head), folds both biases and
// writes bf16 output plus the natural-log LSE.

#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
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
    int tiles, splits, rows_per_split;
    int blk_heads, blk_k, blk_v;                     // block-diagonal layout (0 = full rows)
    int q_compact;                                   // q operand holds only the own block slice
    float* part_ml;                                  // [B][Hq*Lq][splits][2]
    float* part_acc;                                 // [B][Hq*Lq][splits][wown]
    int wown;
    int nwg;
};

struct SplitParams {
    Seg seg[2];
    int nseg;
    int B, Lq, Hq;
    float scale_log2;
};

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;

template <int KS>
struct SplitLds {
    static constexpr int RS = 16 * KS + 8;                       // padded V row (bf16)
    static constexpr int vbytes = kWaves * 2 * 16 * RS * 2;      // double-buffered V tiles
    static constexpr int mbytes = kWaves * 16 * 16 * KS * 4;     // per-wave accumulators
    static constexpr int bytes = (vbytes > mbytes ? vbytes : mbytes) + kWaves * 16 * 2 * 4;
};

template <int KS>
__device__ __forceinline__ void split_segment(const Seg& sg, int w, int Lq, int Hq,
                                              float scale_log2, char* lds) {
    constexpr int VT = KS;                   // V tiles of 16 (same width budget as K)
    constexpr int RS = SplitLds<KS>::RS;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;
    const int grp = lane >> 4;

    const int s = w % sg.splits;
    int rem = w / sg.splits;
    const int t = rem % sg.tiles;
    rem /= sg.tiles;
    const int h = rem % sg.hk;
    const int b = rem / sg.hk;

    const int P = Lq * sg.g;
    const int p0 = t * 16;
    const int pl = p0 + col;
    const bool colv = pl < P;
    const int jj = colv ? pl / Lq : 0;
    const int lq = colv ? pl % Lq : 0;
    const int j = h * sg.g + jj;

    int k_off = 0, v_off = 0;
    int span_k = sg.wk, span_v = sg.wv;
    int own_k_lo = 0, own_k_w = sg.wk, own_v_lo = 0, own_v_w = sg.wv;
    if (sg.blk_heads) {
        const int pend = (P < p0 + 16 ? P : p0 + 16) - 1;
        const int first_blk = (p0 / Lq) / sg.blk_heads;
        const int last_blk = (pend / Lq) / sg.blk_heads;
        k_off = first_blk * sg.blk_k;
        v_off = first_blk * sg.blk_v;
        span_k = (last_blk - first_blk + 1) * sg.blk_k;
        span_v = (last_blk - first_blk + 1) * sg.blk_v;
        const int blk = jj / sg.blk_heads;
        own_k_lo = blk * sg.blk_k - k_off;
        own_k_w = sg.blk_k;
        own_v_lo = blk * sg.blk_v - v_off;
        own_v_w = sg.blk_v;
    }
    if (k_off + span_k > sg.wk) span_k = sg.wk - k_off;
    if (v_off + span_v > sg.wv) span_v = sg.wv - v_off;

    // Query operand (B of the score MFMA): lane group `grp` owns the contiguous
    // tile-relative k range [grp*4*KS, (grp+1)*4*KS); step s uses 4 of them.
    v4s qb[KS];
    {
        const uint16_t* qrow = sg.q + (int64_t)b * sg.q_sb + (int64_t)lq * sg.q_sl + (int64_t)j * sg.q_sh;
#pragma unroll
        for (int c = 0; c < KS / 2; ++c) {
            const int kk = grp * 4 * KS + 8 * c;
            u32x4 val = {0u, 0u, 0u, 0u};
            const bool in = colv && kk >= own_k_lo && kk + 8 <= own_k_lo + own_k_w && kk + 8 <= span_k;
            if (in) {
                const int idx = sg.q_compact ? (kk - own_k_lo) : (k_off + kk);
                val = *reinterpret_cast<const u32x4*>(qrow + idx);
            }
            qb[2 * c] = as_v4s(val.x, val.y);
            qb[2 * c + 1] = as_v4s(val.z, val.w);
        }
    }

    int Nb = sg.n;
    if (sg.seqlens) {
        const int sl = sg.seqlens[b];
        Nb = sl < 0 ? 0 : (sl < sg.n ? sl : sg.n);
    }
    const int lim = !colv ? 0 : (sg.causal ? Nb - Lq + lq + 1 : Nb);
    const int r_begin = s * sg.rows_per_split;
    const int r_end = min(r_begin + sg.rows_per_split, Nb);
    const int ntile = r_end > r_begin ? (r_end - r_begin + 15) / 16 : 0;
    const int niter = (ntile + kWaves - 1) / kWaves;
    const int vis = min(lim, r_end);

    float m = kNegInf, lsum = 0.f;
    v4f acc[VT];
#pragma unroll
    for (int i = 0; i < VT; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};

    uint16_t* vbuf = reinterpret_cast<uint16_t*>(lds) + wave * 2 * 16 * RS;
    const uint16_t* kbase = sg.k + (int64_t)b * sg.k_sb + (int64_t)h * sg.k_sh + k_off;
    const uint16_t* vbase = sg.v + (int64_t)b * sg.v_sb + (int64_t)h * sg.v_sh + v_off;
    const int vrow = lane >> 2;
    const int vpart = lane & 3;

    for (int it = 0; it < niter; ++it) {
        const int rt = it * kWaves + wave;
        const int r0 = r_begin + rt * 16;
        const bool act = rt < ntile;

        // K tile as the A operand: lane row = col, contiguous 4*KS elements.
        v4s ka[KS];
        {
            const int row = r0 + col;
            const bool rv = act && row < r_end;
            const uint16_t* src = kbase + (int64_t)row * sg.k_sn;
#pragma unroll
            for (int c = 0; c < KS / 2; ++c) {
                const int kk = grp * 4 * KS + 8 * c;
                u32x4 val = {0u, 0u, 0u, 0u};
                if (rv && kk + 8 <= span_k) val = *reinterpret_cast<const u32x4*>(src + kk);
                ka[2 * c] = as_v4s(val.x, val.y);
                ka[2 * c + 1] = as_v4s(val.z, val.w);
            }
        }
        // V tile staged in LDS: lane copies 4*VT elements of row vrow.
        {
            const int row = r0 + vrow;
            const bool rv = act && row < r_end;
            const uint16_t* src = vbase + (int64_t)row * sg.v_sn;
            uint16_t* dst = vbuf + (it & 1) * 16 * RS + vrow * RS + vpart * 4 * VT;
#pragma unroll
            for (int c = 0; c < VT / 2; ++c) {
                const int vv = vpart * 4 * VT + 8 * c;
                u32x4 val = {0u, 0u, 0u, 0u};
                if (rv && vv + 8 <= span_v) val = *reinterpret_cast<const u32x4*>(src + vv);
                *reinterpret_cast<u32x4*>(dst + 8 * c) = val;
            }
        }

        uint32_t pw0 = 0, pw1 = 0;
        if (act) {
            v4f sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) sc = mfma16(ka[ks], qb[ks], sc);
            float sv[4];
            float tmax = kNegInf;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int n = r0 + 4 * grp + i;
                const float x = n < vis ? sc[i] * scale_log2 : kNegInf;
                sv[i] = x;
                tmax = fmaxf(tmax, x);
            }
            tmax = fmaxf(tmax, shfl_xor_f(tmax, 16));
            tmax = fmaxf(tmax, shfl_xor_f(tmax, 32));
            const float mnew = fmaxf(m, tmax);
            const float mref = mnew == kNegInf ? 0.f : mnew;
            const float alpha = fast_exp2(m - mref);
            float p[4];
            float psum = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[i] = fast_exp2(sv[i] - mref);
                psum += p[i];
            }
            lsum = lsum * alpha + psum;
            m = mnew;
#pragma unroll
            for (int i = 0; i < VT; ++i) acc[i] *= alpha;
            pw0 = f32_to_bf16(p[0]) | (f32_to_bf16(p[1]) << 16);
            pw1 = f32_to_bf16(p[2]) | (f32_to_bf16(p[3]) << 16);
        }
        __syncthreads();
        if (act) {
            const v4s pb = as_v4s(pw0, pw1);
            const uint16_t* vb = vbuf + (it & 1) * 16 * RS;
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
        }
    }

    // Per-wave column sums: every lane group holds a quarter of the keys.
    lsum += shfl_xor_f(lsum, 16);
    lsum += shfl_xor_f(lsum, 32);

    // Merge the four wavefront states through LDS (reusing the V buffers).
    __syncthreads();
    float* macc = reinterpret_cast<float*>(lds);                      // [wave][col][16*VT]
    float* mml = reinterpret_cast<float*>(lds + SplitLds<KS>::bytes - kWaves * 16 * 2 * 4);
    {
        float* dst = macc + (wave * 16 + col) * 16 * VT;
#pragma unroll
        for (int u = 0; u < VT / 2; ++u) {
            // lane holds v = 32u + 8*grp + 2i + e in acc[2u+e][i]
            float o[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                o[2 * i] = acc[2 * u][i];
                o[2 * i + 1] = acc[2 * u + 1][i];
            }
            float4* d4 = reinterpret_cast<float4*>(dst + 32 * u + 8 * grp);
            d4[0] = make_float4(o[0], o[1], o[2], o[3]);
            d4[1] = make_float4(o[4], o[5], o[6], o[7]);
        }
        if (grp == 0) {
            mml[(wave * 16 + col) * 2] = m;
            mml[(wave * 16 + col) * 2 + 1] = lsum;
        }
    }
    __syncthreads();
    {
        const int c = threadIdx.x & 15;
        const int chunk = threadIdx.x >> 4;        // 16 chunks of VT values
        const int pc = p0 + c;
        if (pc < P) {
            const int cj = h * sg.g + pc / Lq;
            const int cl = pc % Lq;
            const int pr = cj * Lq + cl;
            float mw[kWaves];
            float M = kNegInf;
#pragma unroll
            for (int ww = 0; ww < kWaves; ++ww) {
                mw[ww] = mml[(ww * 16 + c) * 2];
                M = fmaxf(M, mw[ww]);
            }
            const float Mref = M == kNegInf ? 0.f : M;
            float wt[kWaves];
            float L = 0.f;
#pragma unroll
            for (int ww = 0; ww < kWaves; ++ww) {
                wt[ww] = fast_exp2(mw[ww] - Mref);
                L += mml[(ww * 16 + c) * 2 + 1] * wt[ww];
            }
            const int64_t slot = ((int64_t)b * Hq * Lq + pr) * sg.splits + s;
            if (chunk == 0) {
                sg.part_ml[slot * 2] = M;
                sg.part_ml[slot * 2 + 1] = L;
            }
            int c_own_lo = 0;
            if (sg.blk_heads) {
                const int first_blk = (p0 / Lq) / sg.blk_heads;
                c_own_lo = (pc / Lq / sg.blk_heads) * sg.blk_v - first_blk * sg.blk_v;
            }
            float* dst = sg.part_acc + slot * sg.wown;
#pragma unroll
            for (int e = 0; e < VT; ++e) {
                const int vv = chunk * VT + e;
                const int o = vv - c_own_lo;
                if (o >= 0 && o < sg.wown && vv < span_v) {
                    float sum = 0.f;
#pragma unroll
                    for (int ww = 0; ww < kWaves; ++ww)
                        sum += macc[(ww * 16 + c) * 16 * VT + vv] * wt[ww];
                    dst[o] = sum;
                }
            }
        }
    }
    (void)own_v_lo;
    (void)own_v_w;
}

template <int KA, int KB>
__global__ void __launch_bounds__(kThreads)
split_kernel(SplitParams prm) {
    constexpr int LA = SplitLds<KA>::bytes;
    constexpr int LB = KB > 0 ? SplitLds<(KB > 0 ? KB : 2)>::bytes : 0;
    __shared__ __attribute__((aligned(16))) char lds[LA > LB ? LA : LB];
    int w = blockIdx.x;
    if (w < prm.seg[0].nwg) {
        split_segment<KA>(prm.seg[0], w, prm.Lq, prm.Hq, prm.scale_log2, lds);
    } else if constexpr (KB > 0) {
        w -= prm.seg[0].nwg;
        split_segment<KB>(prm.seg[1], w, prm.Lq, prm.Hq, prm.scale_log2, lds);
    }
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
    int B, Lq, Hq, Hkv, D;                                       // D = output width
    uint16_t* out; int64_t o_sb, o_sl, o_sh;
    float* lse;                                                  // [B, Hq, Lq] or null
};

constexpr int kMaxSplits = 256;
constexpr int kMaxLatW = 1024;

__global__ void __launch_bounds__(256)
combine_kernel(CombineParams cp) {
    __shared__ float wa[kMaxSplits];
    __shared__ float wb[kMaxSplits];
    __shared__ float accb[kMaxLatW];
    __shared__ float red[4];
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

    if (threadIdx.x == 0) {
        float M = kNegInf;
        for (int s = 0; s < cp.a_splits; ++s) M = fmaxf(M, aml[2 * s]);
        for (int s = 0; s < cp.b_splits; ++s) {
            const float mb = bml[2 * s];
            if (mb != kNegInf) M = fmaxf(M, mb + shift);
        }
        const float Mref = M == kNegInf ? 0.f : M;
        float LA = 0.f, LB = 0.f;
        for (int s = 0; s < cp.a_splits; ++s) {
            const float wgt = fast_exp2(aml[2 * s] - Mref);
            wa[s] = wgt;
            LA += aml[2 * s + 1] * wgt;
        }
        for (int s = 0; s < cp.b_splits; ++s) {
            const float mb = bml[2 * s];
            const float wgt = mb == kNegInf ? 0.f : fast_exp2(mb + shift - Mref);
            wb[s] = wgt;
            LB += bml[2 * s + 1] * wgt;
        }
        red[0] = M;
        red[1] = LA;
        red[2] = LB;
    }
    __syncthreads();
    const float M = red[0], LA = red[1], LB = red[2];
    const float L = LA + LB;
    if (cp.b_splits) {
        const float* bacc = cp.b_acc + row * cp.b_splits * cp.b_w;
        for (int k = threadIdx.x; k < cp.b_w; k += blockDim.x) {
            float sum = 0.f;
            for (int s = 0; s < cp.b_splits; ++s) sum += bacc[(int64_t)s * cp.b_w + k] * wb[s];
            accb[k] = sum;
        }
        __syncthreads();
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    const float* aacc = cp.a_acc + row * cp.a_splits * cp.a_w;
    uint16_t* orow = cp.out + (int64_t)b * cp.o_sb + (int64_t)lq * cp.o_sl + (int64_t)j * cp.o_sh;
    for (int dd = threadIdx.x; dd < cp.D; dd += blockDim.x) {
        float sum = 0.f;
        for (int s = 0; s < cp.a_splits; ++s) sum += aacc[(int64_t)s * cp.a_w + dd] * wa[s];
        if (cp.b_splits) {
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
        orow[dd] = (uint16_t)f32_to_bf16(sum * inv);
    }
    if (cp.lse && threadIdx.x == 0) {
        cp.lse[((int64_t)b * cp.Hq + j) * cp.Lq + lq] = L > 0.f ? (M + __log2f(L)) * kLn2 : kNegInf;
    }
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
    int B, Lq, Hq, Hkv, D, Rk, parts;
    float scale;
};

constexpr int kMaxRows = 16;

__global__ void __launch_bounds__(256)
prologue_kernel(PrologueParams pp) {
    extern __shared__ float sh[];          // [rows][D] rotated q, then [parts][rows][wq chunk]
    const int h = blockIdx.x % pp.Hkv;
    const int b = blockIdx.x / pp.Hkv;
    const int g = pp.Hq / pp.Hkv;
    const int rows = g * pp.Lq;            // r = jj*Lq + l
    float* qs = sh;
    // RoPE (or copy) each query row of this KV head.
    for (int e = threadIdx.x; e < rows * pp.D; e += blockDim.x) {
        const int r = e / pp.D, dd = e % pp.D;
        const int jj = r / pp.Lq, l = r % pp.Lq;
        const int jh = h * g + jj;
        const uint16_t* qrow = pp.q + (int64_t)b * pp.q_sb + (int64_t)l * pp.q_sl + (int64_t)jh * pp.q_sh;
        float x = bf16_to_f32(qrow[dd]);
        if (pp.cos) {
            const int half = pp.D / 2;
            const float partner = bf16_to_f32(qrow[(dd + half) % pp.D]);
            const float rot = dd < half ? -partner : partner;
            const int64_t ps = clamp_i64(pp.pos[(int64_t)b * pp.pos_sb + l], 0, pp.rope_rows - 1);
            const float c = round_bf16(pp.cos[ps * pp.D + dd]);
            const float sn = round_bf16(pp.sin[ps * pp.D + dd]);
            x = round_bf16(round_bf16(x * c) + round_bf16(rot * sn));
        }
        qs[e] = x;
        pp.q_rot[(((int64_t)b * pp.Lq + l) * pp.Hq + jh) * pp.D + dd] = (uint16_t)f32_to_bf16(x);
    }
    __syncthreads();
    if (pp.shift && threadIdx.x < rows) {
        const int r = threadIdx.x;
        const int jj = r / pp.Lq, l = r % pp.Lq;
        float sum = 0.f;
        for (int dd = 0; dd < pp.D; ++dd)
            sum += qs[r * pp.D + dd] * bf16_to_f32(pp.up_k_bias[(int64_t)h * pp.D + dd]);
        pp.shift[(int64_t)b * pp.Hq * pp.Lq + (h * g + jj) * pp.Lq + l] = sum * pp.scale;
    }
    // Absorption: q_lat[r][k] = sum_dd qs[r][dd] * W[h*D+dd][kg].
    float* part = sh + rows * pp.D;        // [parts][rows][256]
    const int parts = pp.parts;
    const int per = pp.D / parts;
    for (int k0 = 0; k0 < pp.wq; k0 += 256 / parts) {
        const int kc = 256 / parts;
        const int tk = threadIdx.x % kc, tp = threadIdx.x / kc;
        const int k = k0 + tk;
        float accr[kMaxRows];
#pragma unroll
        for (int r = 0; r < kMaxRows; ++r) accr[r] = 0.f;
        if (k < pp.wq && tp < parts) {
            const int kg = pp.blockdiag ? h * pp.wq + k : k;
            const uint16_t* wcol = pp.up_k + ((int64_t)h * pp.D) * pp.Rk + kg;
            for (int dd = tp * per; dd < (tp + 1) * per; ++dd) {
                const float wv = bf16_to_f32(wcol[(int64_t)dd * pp.Rk]);
#pragma unroll
                for (int r = 0; r < kMaxRows; ++r)
                    if (r < rows) accr[r] += qs[r * pp.D + dd] * wv;
            }
        }
        __syncthreads();
        if (k < pp.wq && tp < parts) {
#pragma unroll
            for (int r = 0; r < kMaxRows; ++r)
                if (r < rows) part[(tp * rows + r) * kc + tk] = accr[r];
        }
        __syncthreads();
        for (int e = threadIdx.x; e < rows * kc; e += blockDim.x) {
            const int r = e / kc, kk = e % kc;
            const int kq = k0 + kk;
            if (kq >= pp.wq) continue;
            float sum = 0.f;
            for (int p = 0; p < parts; ++p) sum += part[(p * rows + r) * kc + kk];
            const int jj = r / pp.Lq, l = r % pp.Lq;
            pp.q_lat[(((int64_t)b * pp.Lq + l) * pp.Hq + h * g + jj) * pp.wq + kq] = (uint16_t)f32_to_bf16(sum);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

namespace {

thread_local std::string g_error;
thread_local hipEvent_t g_before = nullptr;
thread_local hipEvent_t g_after = nullptr;

// Launch the split kernel bracketed by the caller's profiling events, if set.
hipError_t dispatch_split(int ka, int kb, const struct SplitParams& prm, int grid, hipStream_t st);
hipError_t timed_split(int ka, int kb, const SplitParams& prm, int grid, hipStream_t st) {
    if (g_before) {
        hipError_t e = hipEventRecord(g_before, st);
        if (e != hipSuccess) return e;
    }
    hipError_t e = dispatch_split(ka, kb, prm, grid, st);
    if (e == hipSuccess && g_after) e = hipEventRecord(g_after, st);
    return e;
}

int round_even_tile(int width) {
    // MFMA k-steps of 16 needed for `width`, rounded to the instantiated set.
    const int ks = (width + 15) / 16;
    const int set[] = {4, 8, 12, 16, 24};
    for (int v : set)
        if (ks <= v) return v;
    return -1;
}

bool aligned8(int64_t x) { return (x & 7) == 0; }
bool ptr_aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct SegPlan {
    int tiles, splits, rows_per_split, nwg, wown, ks;
};

// Split the key range so the launch holds a few workgroups per CU.
SegPlan plan_segment(int B, int hk, int P, int n, int span_k, int wown, int req_splits, int target_wg) {
    SegPlan sp{};
    sp.tiles = (P + 15) / 16;
    sp.ks = round_even_tile(span_k);
    sp.wown = wown;
    const int groups = B * hk * sp.tiles;
    int splits = req_splits;
    if (splits <= 0) {
        const int max_by_rows = std::max(1, (n + 63) / 64);
        splits = std::max(1, std::min(max_by_rows, (target_wg + groups - 1) / groups));
        splits = std::min(splits, kMaxSplits);
    }
    splits = std::min(splits, kMaxSplits);
    int rps = (n + splits - 1) / splits;
    rps = std::max(64, (rps + 63) / 64 * 64);
    splits = std::max(1, (n + rps - 1) / rps);
    sp.splits = splits;
    sp.rows_per_split = rps;
    sp.nwg = groups * splits;
    return sp;
}

template <int KA, int KB>
hipError_t launch_split(const SplitParams& prm, int grid, hipStream_t st) {
    hipLaunchKernelGGL((split_kernel<KA, KB>), dim3(grid), dim3(kThreads), 0, st, prm);
    return hipGetLastError();
}

hipError_t dispatch_split(int ka, int kb, const SplitParams& prm, int grid, hipStream_t st) {
#define SLIMKV_CASE_B(A)                                            \
    switch (kb) {                                                   \
        case 0: return launch_split<A, 0>(prm, grid, st);           \
        case 4: return launch_split<A, 4>(prm, grid, st);           \
        case 8: return launch_split<A, 8>(prm, grid, st);           \
        case 12: return launch_split<A, 12>(prm, grid, st);         \
        case 16: return launch_split<A, 16>(prm, grid, st);         \
        case 24: return launch_split<A, 24>(prm, grid, st);         \
        default: return hipErrorInvalidValue;                       \
    }
    switch (ka) {
        case 4: if (kb != 0) return hipErrorInvalidValue; return launch_split<4, 0>(prm, grid, st);
        case 8: SLIMKV_CASE_B(8)
        case 12: if (kb != 0) return hipErrorInvalidValue; return launch_split<12, 0>(prm, grid, st);
        case 16: if (kb != 0) return hipErrorInvalidValue; return launch_split<16, 0>(prm, grid, st);
        case 24: if (kb != 0) return hipErrorInvalidValue; return launch_split<24, 0>(prm, grid, st);
        default: return hipErrorInvalidValue;
    }
#undef SLIMKV_CASE_B
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
    const int target = 4 * device_cu_count();
    plan->sp = plan_segment((int)B, (int)Hk, P, (int)N, span, (int)a->width_v, a->splits, target);
    if (plan->sp.ks < 0) return fail(SLIMKV_EUNSUP, "width not supported");
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

extern "C" int slimkv_abi_version(void) { return 1; }

extern "C" int slimkv_set_profile_events(void* before, void* after) {
    if ((before == nullptr) != (after == nullptr)) return fail(SLIMKV_EINVAL, "set both events or neither");
    g_before = static_cast<hipEvent_t>(before);
    g_after = static_cast<hipEvent_t>(after);
    return SLIMKV_OK;
}

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
    sg.splits = plan.sp.splits;
    sg.rows_per_split = plan.sp.rows_per_split;
    sg.part_ml = reinterpret_cast<float*>(ws + plan.ml_off);
    sg.part_acc = reinterpret_cast<float*>(ws + plan.acc_off);
    sg.wown = (int)a->width_v;
    sg.nwg = plan.sp.nwg;
    hipStream_t st = static_cast<hipStream_t>(stream);
    rc = check_hip(timed_split(plan.sp.ks, 0, prm, sg.nwg, st), "split kernel launch");
    if (rc != SLIMKV_OK) return rc;
    CombineParams cp{};
    cp.a_ml = sg.part_ml; cp.a_acc = sg.part_acc; cp.a_splits = sg.splits; cp.a_w = sg.wown;
    cp.b_splits = 0;
    cp.B = prm.B; cp.Lq = Lq; cp.Hq = Hq; cp.Hkv = Hk; cp.D = (int)a->width_v;
    cp.out = static_cast<uint16_t*>(a->out); cp.o_sb = a->o_sb; cp.o_sl = a->o_sl; cp.o_sh = a->o_sh;
    cp.lse = a->lse;
    hipLaunchKernelGGL(combine_kernel, dim3(prm.B * Hq * Lq), dim3(128), 0, st, cp);
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

int plan_latent(const slimkv_latent_decode_args* a, LatentPlan* p) {
    if (!a || !a->q || !a->raw_k || !a->raw_v || !a->out || !a->up_k || !a->up_v)
        return fail(SLIMKV_EINVAL, "null tensor pointer");
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
    if (a->lat_keys > 0 && (!a->lat_k || !a->lat_v)) return fail(SLIMKV_EINVAL, "null latent pointer");
    if (a->cos && (!a->sin || !a->q_positions || a->rope_rows <= 0))
        return fail(SLIMKV_EINVAL, "RoPE needs sin, positions and a table size");
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
    // Raw: one column tile per KV head over the full head width.
    p->raw = plan_segment((int)B, (int)Hkv, (int)Lq * g, (int)a->raw_keys, (int)D, (int)D, a->raw_splits, cu);
    if (p->raw.tiles != 1 || p->raw.ks != 8) return fail(SLIMKV_EUNSUP, "raw tile shape");
    // Latent: every query head against shared rows; block-diagonal tiles only
    // span the latent slices of their own heads.
    const int P = (int)(Lq * Hq);
    int span = (int)std::max(Rk, Rv);
    if (bd) {
        int worst = 0;
        for (int t = 0; t * 16 < P; ++t) {
            const int p0 = t * 16, pend = std::min(P, p0 + 16) - 1;
            const int blocks = (pend / (int)Lq) / g - (p0 / (int)Lq) / g + 1;
            worst = std::max(worst, blocks * std::max(rk, rv));
        }
        span = worst;
    }
    const int64_t nl = std::max<int64_t>(a->lat_keys, 1);
    p->lat = plan_segment((int)B, 1, P, (int)nl, span, rv, a->lat_splits, 4 * cu);
    if (p->lat.ks < 0) return fail(SLIMKV_EUNSUP, "latent width not supported");
    p->wq = rk;
    int parts = 1;
    while (parts < 8 && p->wq * parts * 2 <= 256) parts *= 2;
    p->parts = parts;
    const int rows = g * (int)Lq;
    p->prologue_lds = (size_t)rows * D * 4 + (size_t)parts * rows * (256 / parts) * 4;
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

extern "C" int slimkv_latent_decode(const slimkv_latent_decode_args* a, void* workspace,
                                    size_t workspace_bytes, void* stream) {
    LatentPlan p{};
    int rc = plan_latent(a, &p);
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
    hipLaunchKernelGGL(prologue_kernel, dim3(B * Hkv), dim3(256), p.prologue_lds, st, pp);
    rc = check_hip(hipGetLastError(), "prologue kernel launch");
    if (rc != SLIMKV_OK) return rc;

    SplitParams prm{};
    prm.B = B; prm.Lq = Lq; prm.Hq = Hq;
    prm.scale_log2 = (float)(a->scale * 1.4426950408889634);
    prm.nseg = has_lat ? 2 : 1;
    Seg& r = prm.seg[0];
    r.q = q_rot; r.q_sb = (int64_t)Lq * Hq * D; r.q_sl = (int64_t)Hq * D; r.q_sh = D;
    r.k = static_cast<const uint16_t*>(a->raw_k); r.k_sb = a->rk_sb; r.k_sn = a->rk_sn; r.k_sh = a->rk_sh;
    r.v = static_cast<const uint16_t*>(a->raw_v); r.v_sb = a->rv_sb; r.v_sn = a->rv_sn; r.v_sh = a->rv_sh;
    r.seqlens = a->raw_lengths;
    r.n = (int)a->raw_keys;
    r.hk = Hkv; r.g = g; r.wk = D; r.wv = D; r.causal = 0;
    r.tiles = p.raw.tiles; r.splits = p.raw.splits; r.rows_per_split = p.raw.rows_per_split;
    r.part_ml = reinterpret_cast<float*>(ws + p.rml_off);
    r.part_acc = reinterpret_cast<float*>(ws + p.racc_off);
    r.wown = D;
    r.nwg = p.raw.nwg;
    int kb = 0;
    if (has_lat) {
        Seg& l = prm.seg[1];
        l.q = q_lat; l.q_sb = (int64_t)Lq * Hq * p.wq; l.q_sl = (int64_t)Hq * p.wq; l.q_sh = p.wq;
        l.k = static_cast<const uint16_t*>(a->lat_k); l.k_sb = a->lk_sb; l.k_sn = a->lk_sn; l.k_sh = 0;
        l.v = static_cast<const uint16_t*>(a->lat_v); l.v_sb = a->lv_sb; l.v_sn = a->lv_sn; l.v_sh = 0;
        l.seqlens = a->lat_lengths;
        l.n = (int)a->lat_keys;
        l.hk = 1; l.g = Hq; l.wk = Rk; l.wv = Rv; l.causal = a->lat_causal ? 1 : 0;
        l.tiles = p.lat.tiles; l.splits = p.lat.splits; l.rows_per_split = p.lat.rows_per_split;
        if (bd) {
            l.blk_heads = g; l.blk_k = Rk / Hkv; l.blk_v = Rv / Hkv; l.q_compact = 1;
        }
        l.part_ml = reinterpret_cast<float*>(ws + p.lml_off);
        l.part_acc = reinterpret_cast<float*>(ws + p.lacc_off);
        l.wown = bd ? Rv / Hkv : Rv;
        l.nwg = p.lat.nwg;
        kb = p.lat.ks;
    }
    const int grid = r.nwg + (has_lat ? prm.seg[1].nwg : 0);
    rc = check_hip(timed_split(8, kb, prm, grid, st), "split kernel launch");
    if (rc != SLIMKV_OK) return rc;

    CombineParams cp{};
    cp.a_ml = r.part_ml; cp.a_acc = r.part_acc; cp.a_splits = r.splits; cp.a_w = D;
    if (has_lat) {
        cp.b_ml = prm.seg[1].part_ml; cp.b_acc = prm.seg[1].part_acc;
        cp.b_splits = prm.seg[1].splits; cp.b_w = prm.seg[1].wown;
        cp.up_v = static_cast<const uint16_t*>(a->up_v); cp.up_v_ld = Rv;
        cp.up_v_bias = static_cast<const uint16_t*>(a->up_v_bias);
        cp.blockdiag = bd ? 1 : 0;
        cp.b_shift = pp.shift;
    }
    cp.B = B; cp.Lq = Lq; cp.Hq = Hq; cp.Hkv = Hkv; cp.D = D;
    cp.out = static_cast<uint16_t*>(a->out); cp.o_sb = a->o_sb; cp.o_sl = a->o_sl; cp.o_sh = a->o_sh;
    cp.lse = a->lse;
    hipLaunchKernelGGL(combine_kernel, dim3(B * Hq * Lq), dim3(128), 0, st, cp);
    return check_hip(hipGetLastError(), "combine kernel launch");
}
