// Beacon reconstruction (up-projection) on MFMA, with the bias, an optional
// bf16-exact RoPE epilogue and an optional row scatter.
//
// out[b, dst(n), h, :] = rope?(bf16(latent[b, n, :] @ W[h*D:(h+1)*D, :]^T + bias))
//
// One wavefront computes a 16-row x 128-feature block of one KV head as
// C^T[o, n] = W[o, :] . latent[n, :] on v_mfma_f32_16x16x16_bf16: the A operand
// (W rows) and the B operand (latent rows) are both contiguous along the
// contraction, so neither needs a transpose, and lane (n, g) ends with features
// o = 16t + 4g + i of row n for t = 0..7 -- d and d + 64 sit in the same lane,
// so rotate-half RoPE is applied in registers before the 8-byte stores.

#include "common.hpp"

#include <algorithm>

namespace slimkv {

struct ReconParams {
    const uint16_t* latent; int64_t l_sb, l_sn;
    const uint16_t* w; const uint16_t* bias; int64_t w_ld;   // W [Hkv*D, R] row-major
    uint16_t* out; int64_t o_sb, o_sn, o_sh;
    const int64_t* dst_rows;                                  // [n] or null (identity)
    const float* cos; const float* sin; int64_t rope_rows;
    const int64_t* positions; int64_t pos_sb;                 // [B, n] or null
    int B, n, R, Hkv, blockdiag, k_lo_step;                   // k_lo_step: per-head latent slice width
};

constexpr int kReconWaves = 4;

template <int KSTEPS>
__global__ void __launch_bounds__(kReconWaves * 64)
recon_kernel(ReconParams p) {
    constexpr int D = 128;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int tiles = (p.n + 16 * kReconWaves - 1) / (16 * kReconWaves);
    const int h = blockIdx.x % p.Hkv;
    const int rt = (blockIdx.x / p.Hkv) % tiles;
    const int b = blockIdx.x / (p.Hkv * tiles);
    const int row = (rt * kReconWaves + wave) * 16 + col;
    const bool rv = row < p.n;
    const int k_lo = p.blockdiag ? h * p.k_lo_step : 0;

    const uint16_t* lrow = p.latent + (int64_t)b * p.l_sb + (int64_t)(rv ? row : 0) * p.l_sn + k_lo;
    v4f acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
        const int k = 16 * ks + 4 * grp;
        u32x2 bl = *reinterpret_cast<const u32x2*>(lrow + k);
        if (!rv) bl = u32x2{0u, 0u};
        const v4s bop = as_v4s(bl.x, bl.y);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint16_t* wr = p.w + ((int64_t)h * D + 16 * t + col) * p.w_ld + k_lo + k;
            const u32x2 al = *reinterpret_cast<const u32x2*>(wr);
            acc[t] = mfma16(as_v4s(al.x, al.y), bop, acc[t]);
        }
    }
    if (!rv) return;
    // lane holds x[d] for d = 16t + 4*grp + i
    float x[8][4];
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = 16 * t + 4 * grp + i;
            float v = acc[t][i];
            if (p.bias) v += bf16_to_f32(p.bias[(int64_t)h * D + d]);
            x[t][i] = round_bf16_hw(v);
        }
    if (p.positions) {
        const int64_t pos = clamp_i64(p.positions[(int64_t)b * p.pos_sb + row], 0, p.rope_rows - 1);
        const float* cr = p.cos + pos * D;
        const float* sr = p.sin + pos * D;
        float y[8][4];
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int d = 16 * t + 4 * grp + i;
                const float partner = t < 4 ? -x[t + 4][i] : x[t - 4][i];
                y[t][i] = round_bf16_hw(round_bf16_hw(x[t][i] * round_bf16_hw(cr[d])) + round_bf16_hw(partner * round_bf16_hw(sr[d])));
            }
#pragma unroll
        for (int t = 0; t < 8; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) x[t][i] = y[t][i];
    }
    const int64_t dst = p.dst_rows ? p.dst_rows[row] : row;
    uint16_t* orow = p.out + (int64_t)b * p.o_sb + dst * p.o_sn + (int64_t)h * p.o_sh;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        const uint32_t lo = pack_bf16(x[t][0], x[t][1]);
        const uint32_t hi = pack_bf16(x[t][2], x[t][3]);
        *reinterpret_cast<u32x2*>(orow + 16 * t + 4 * grp) = u32x2{lo, hi};
    }
}

// Streaming variant for narrow contractions (kw <= 64): the wavefront keeps its
// head's W tile (A operand, 128 x kw) in registers and walks 16-row tiles with
// the next tile's latent rows already in flight, so W is read once per
// wavefront instead of once per tile.  Same epilogue as recon_kernel.
template <int KSTEPS>
__device__ __forceinline__ void recon_stream_body(const ReconParams& p, int segs, int block) {
    constexpr int D = 128;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int col = lane & 15, grp = lane >> 4;
    const int h = block % p.Hkv;
    const int seg = (block / p.Hkv) % segs;
    const int b = block / (p.Hkv * segs);
    const int tiles = (p.n + 15) / 16;
    const int stride = segs * kReconWaves;
    const int k_lo = p.blockdiag ? h * p.k_lo_step : 0;
    u32x2 wa[8][KSTEPS];
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
            wa[t][ks] = *reinterpret_cast<const u32x2*>(p.w + ((int64_t)h * D + 16 * t + col) * p.w_ld + k_lo + 16 * ks +
                                                        4 * grp);
    float bias[8][4];
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            bias[t][i] = p.bias ? bf16_to_f32(p.bias[(int64_t)h * D + 16 * t + 4 * grp + i]) : 0.f;
    const uint16_t* lbase = p.latent + (int64_t)b * p.l_sb + k_lo + 4 * grp;
    auto load_rows = [&](u32x2 (&lr)[KSTEPS], int tile) {
        const int row = min(tile * 16 + col, p.n - 1);
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) lr[ks] = *reinterpret_cast<const u32x2*>(lbase + (int64_t)row * p.l_sn + 16 * ks);
    };
    int tile = seg * kReconWaves + wave;
    if (tile >= tiles) return;
    u32x2 cur[KSTEPS], nxt[KSTEPS];
    load_rows(cur, tile);
    for (; tile < tiles; tile += stride) {
        const bool more = tile + stride < tiles;
        load_rows(nxt, more ? tile + stride : tile);
        v4f acc[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
            const v4s bop = as_v4s(cur[ks].x, cur[ks].y);
#pragma unroll
            for (int t = 0; t < 8; ++t) acc[t] = mfma16(as_v4s(wa[t][ks].x, wa[t][ks].y), bop, acc[t]);
        }
        const int row = tile * 16 + col;
        if (row < p.n) {
            float x[8][4];
#pragma unroll
            for (int t = 0; t < 8; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) x[t][i] = round_bf16_hw(p.bias ? acc[t][i] + bias[t][i] : acc[t][i]);
            if (p.positions) {
                const int64_t pos = clamp_i64(p.positions[(int64_t)b * p.pos_sb + row], 0, p.rope_rows - 1);
                const float* cr = p.cos + pos * D;
                const float* sr = p.sin + pos * D;
                float y[8][4];
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const float4 c4 = *reinterpret_cast<const float4*>(cr + 16 * t + 4 * grp);
                    const float4 s4 = *reinterpret_cast<const float4*>(sr + 16 * t + 4 * grp);
                    const float cv[4] = {c4.x, c4.y, c4.z, c4.w}, sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float partner = t < 4 ? -x[t + 4][i] : x[t - 4][i];
                        y[t][i] = round_bf16_hw(round_bf16_hw(x[t][i] * round_bf16_hw(cv[i])) + round_bf16_hw(partner * round_bf16_hw(sv[i])));
                    }
                }
#pragma unroll
                for (int t = 0; t < 8; ++t)
#pragma unroll
                    for (int i = 0; i < 4; ++i) x[t][i] = y[t][i];
            }
            const int64_t dst = p.dst_rows ? p.dst_rows[row] : row;
            uint16_t* orow = p.out + (int64_t)b * p.o_sb + dst * p.o_sn + (int64_t)h * p.o_sh;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const uint32_t lo = pack_bf16(x[t][0], x[t][1]);
                const uint32_t hi = pack_bf16(x[t][2], x[t][3]);
                *reinterpret_cast<u32x2*>(orow + 16 * t + 4 * grp) = u32x2{lo, hi};
            }
        }
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) cur[ks] = nxt[ks];
    }
}

template <int KSTEPS>
__global__ void __launch_bounds__(kReconWaves * 64)
recon_stream_kernel(ReconParams p, int segs) {
    recon_stream_body<KSTEPS>(p, segs, blockIdx.x);
}

// Two reconstructions of the same latent width in one launch (the K and the
// V rebuild of a window's beacons): the first `blocks0` workgroups run the
// first, the rest the second -- each the single kernel's workgroup, so the
// results are the single launches' bits.
template <int KSTEPS>
__global__ void __launch_bounds__(kReconWaves * 64)
recon_stream_pair_kernel(ReconParams p0, ReconParams p1, int segs0, int segs1, int blocks0) {
    if ((int)blockIdx.x < blocks0) recon_stream_body<KSTEPS>(p0, segs0, blockIdx.x);
    else recon_stream_body<KSTEPS>(p1, segs1, blockIdx.x - blocks0);
}

namespace {
bool al4(int64_t x) { return (x & 3) == 0; }
bool pal8(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 7) == 0; }

template <int K>
hipError_t launch_recon(const ReconParams& p, int grid, hipStream_t st) {
    hipLaunchKernelGGL((recon_kernel<K>), dim3(grid), dim3(kReconWaves * 64), 0, st, p);
    return hipGetLastError();
}

template <int K>
hipError_t launch_stream(const ReconParams& p, int segs, hipStream_t st) {
    hipLaunchKernelGGL((recon_stream_kernel<K>), dim3(p.B * p.Hkv * segs), dim3(kReconWaves * 64), 0, st, p, segs);
    return hipGetLastError();
}
}  // namespace

// Checks a reconstruction and fills its kernel parameters; `segs` > 0 when it
// takes the streaming kernel (latent width kw <= 64), whose workgroup count is
// B * Hkv * segs.
int prepare_recon(const slimkv_reconstruct_args* a, ReconParams* out, int* segs, int* kw_out) {
    if (!a) return fail(SLIMKV_EINVAL, "null pointer");
    if (a->batch <= 0 || a->rows < 0 || a->rank <= 0 || a->kv_heads <= 0 || a->head_dim != 128)
        return fail(SLIMKV_EINVAL, "invalid reconstruction sizes (head_dim must be 128)");
    *segs = 0;
    *kw_out = 0;
    if (a->rows == 0) return SLIMKV_OK;               // nothing to read or write (empty tensors may be null)
    if (!a->latent || !a->weight || !a->out) return fail(SLIMKV_EINVAL, "null pointer");
    const bool bd = a->block_diagonal != 0;
    const int64_t kw = bd ? a->rank / a->kv_heads : a->rank;
    if ((bd && a->rank % a->kv_heads) || kw % 16 || kw > 512)
        return fail(SLIMKV_EUNSUP, "the contracted latent width must be a multiple of 16 up to 512");
    const int64_t strides[] = {a->l_sb, a->l_sn, a->o_sb, a->o_sn, a->o_sh, a->rank};
    for (int64_t s : strides)
        if (!al4(s)) return fail(SLIMKV_EINVAL, "strides must be multiples of 4 elements");
    if (!pal8(a->latent) || !pal8(a->weight) || !pal8(a->out)) return fail(SLIMKV_EINVAL, "tensors must be 8-byte aligned");
    if (a->positions && (!a->cos || !a->sin || a->rope_rows <= 0)) return fail(SLIMKV_EINVAL, "RoPE needs tables");
    if (a->positions && a->batch > 1 && a->pos_sb < a->rows)
        return fail(SLIMKV_EINVAL, "positions rows are shorter than the row count");
    ReconParams& p = *out;
    p = ReconParams{};
    p.latent = static_cast<const uint16_t*>(a->latent); p.l_sb = a->l_sb; p.l_sn = a->l_sn;
    p.w = static_cast<const uint16_t*>(a->weight); p.bias = static_cast<const uint16_t*>(a->bias); p.w_ld = a->rank;
    p.out = static_cast<uint16_t*>(a->out); p.o_sb = a->o_sb; p.o_sn = a->o_sn; p.o_sh = a->o_sh;
    p.dst_rows = a->dst_rows;
    p.cos = a->cos; p.sin = a->sin; p.rope_rows = a->rope_rows;
    p.positions = a->positions; p.pos_sb = a->pos_sb;
    p.B = (int)a->batch; p.n = (int)a->rows; p.R = (int)a->rank; p.Hkv = (int)a->kv_heads;
    p.blockdiag = bd ? 1 : 0; p.k_lo_step = (int)kw;
    *kw_out = (int)kw;
    const bool tables16 = !a->positions || (((reinterpret_cast<uintptr_t>(a->cos) | reinterpret_cast<uintptr_t>(a->sin)) & 15) == 0);
    if (kw <= 64 && tables16) {
        // streaming kernel: about 1024 workgroups, each wavefront at least one tile
        const int row_tiles = (p.n + 15) / 16;
        const int64_t heads = (int64_t)p.B * p.Hkv;
        const int sg = (int)std::max<int64_t>(1, std::min<int64_t>((row_tiles + kReconWaves - 1) / kReconWaves,
                                                                   (1024 + heads - 1) / heads));
        if ((int64_t)p.B * p.Hkv * sg > 0x3fffffff) return fail(SLIMKV_EINVAL, "reconstruction grid too large");
        *segs = sg;
    }
    return SLIMKV_OK;
}

int launch_prepared(const ReconParams& p, int segs, int kw, hipStream_t st) {
    hipError_t e;
    if (segs > 0) {
        switch (kw / 16) {
            case 1: e = launch_stream<1>(p, segs, st); break;
            case 2: e = launch_stream<2>(p, segs, st); break;
            case 3: e = launch_stream<3>(p, segs, st); break;
            default: e = launch_stream<4>(p, segs, st); break;
        }
        return check_hip(e, "reconstruction kernel launch");
    }
    const int tiles = (p.n + 16 * kReconWaves - 1) / (16 * kReconWaves);
    const int grid = p.B * tiles * p.Hkv;
    switch (kw / 16) {
        case 1: e = launch_recon<1>(p, grid, st); break;
        case 2: e = launch_recon<2>(p, grid, st); break;
        case 3: e = launch_recon<3>(p, grid, st); break;
        case 4: e = launch_recon<4>(p, grid, st); break;
        case 8: e = launch_recon<8>(p, grid, st); break;
        case 12: e = launch_recon<12>(p, grid, st); break;
        case 16: e = launch_recon<16>(p, grid, st); break;
        case 24: e = launch_recon<24>(p, grid, st); break;
        case 32: e = launch_recon<32>(p, grid, st); break;
        default: return fail(SLIMKV_EUNSUP, "latent width not instantiated");
    }
    return check_hip(e, "reconstruction kernel launch");
}

template <int K>
hipError_t launch_stream_pair(const ReconParams& p0, int segs0, const ReconParams& p1, int segs1, hipStream_t st) {
    const int blocks0 = p0.B * p0.Hkv * segs0;
    const int blocks1 = p1.B * p1.Hkv * segs1;
    hipLaunchKernelGGL((recon_stream_pair_kernel<K>), dim3(blocks0 + blocks1), dim3(kReconWaves * 64), 0, st, p0, p1,
                       segs0, segs1, blocks0);
    return hipGetLastError();
}

int reconstruct(const slimkv_reconstruct_args* a, hipStream_t st) {
    ReconParams p;
    int segs = 0, kw = 0;
    const int rc = prepare_recon(a, &p, &segs, &kw);
    if (rc != SLIMKV_OK || a->rows == 0) return rc;
    return launch_prepared(p, segs, kw, st);
}

int reconstruct_pair(const slimkv_reconstruct_args* a, const slimkv_reconstruct_args* b, hipStream_t st) {
    ReconParams pa, pb;
    int sa = 0, sb = 0, ka = 0, kb = 0;
    int rc = prepare_recon(a, &pa, &sa, &ka);
    if (rc != SLIMKV_OK) return rc;
    rc = prepare_recon(b, &pb, &sb, &kb);
    if (rc != SLIMKV_OK) return rc;
    if (a->rows == 0) return b->rows == 0 ? SLIMKV_OK : launch_prepared(pb, sb, kb, st);
    if (b->rows == 0) return launch_prepared(pa, sa, ka, st);
    if (sa > 0 && sb > 0 && ka == kb) {
        hipError_t e;
        switch (ka / 16) {
            case 1: e = launch_stream_pair<1>(pa, sa, pb, sb, st); break;
            case 2: e = launch_stream_pair<2>(pa, sa, pb, sb, st); break;
            case 3: e = launch_stream_pair<3>(pa, sa, pb, sb, st); break;
            default: e = launch_stream_pair<4>(pa, sa, pb, sb, st); break;
        }
        return check_hip(e, "reconstruction pair launch");
    }
    // different kernels or widths: two launches
    rc = launch_prepared(pa, sa, ka, st);
    return rc != SLIMKV_OK ? rc : launch_prepared(pb, sb, kb, st);
}

}  // namespace slimkv

extern "C" int slimkv_reconstruct(const slimkv_reconstruct_args* a, void* stream) {
    return slimkv::reconstruct(a, static_cast<hipStream_t>(stream));
}

extern "C" int slimkv_reconstruct_pair(const slimkv_reconstruct_args* a, const slimkv_reconstruct_args* b,
                                       void* stream) {
    return slimkv::reconstruct_pair(a, b, static_cast<hipStream_t>(stream));
}
