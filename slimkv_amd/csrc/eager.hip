// fp32 eager attention for every model dtype, and the two-branch LSE merge for
// every model dtype.
//
// slimkv_eager_attention follows latent_decode.eager_forward
// (slimkv/llama3/latent_decode.py:16-41): q and k of any model dtype meet in fp32
// (scores = (q . k) * scale), the bottom-right causal mask, the log-sum-exp of
// each query row, probabilities that are zero where that LSE is -inf, out =
// P . V in fp32, cast once to the input dtype.  It is the arithmetic the
// reference keeps as its fp32 baseline, so nothing here rounds P to bf16 as the
// MFMA decode kernels do.  Two launches: one workgroup per query row computes
// the row's scores into a caller workspace, its LSE, and then its
// probabilities in place; one workgroup per query row then forms the output
// row (threads over output features, coalesced V reads).
//
// slimkv_merge_typed is slimkv_merge (rope.hip) for bf16, fp16 and fp32
// branch outputs: merge_attention's arithmetic (slimkv/llama3/fa2_decode.py:
// 57-66) in fp32, rounded once to the outputs' dtype.

#include "common.hpp"

#include <algorithm>

namespace slimkv {

namespace {

constexpr int kEagerThreads = 256;

template <int DT>
struct Elem;

template <>
struct Elem<SLIMKV_DTYPE_BF16> {
    static __device__ __forceinline__ float load(const void* p, int64_t i) {
        return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    }
    static __device__ __forceinline__ void store(void* p, int64_t i, float x) {
        static_cast<uint16_t*>(p)[i] = (uint16_t)pack_bf16(x, 0.f);
    }
};

template <>
struct Elem<SLIMKV_DTYPE_F16> {
    static __device__ __forceinline__ float load(const void* p, int64_t i) {
        return (float)static_cast<const _Float16*>(p)[i];
    }
    static __device__ __forceinline__ void store(void* p, int64_t i, float x) {
        static_cast<_Float16*>(p)[i] = (_Float16)x;       // round to nearest even
    }
};

template <>
struct Elem<SLIMKV_DTYPE_F32> {
    static __device__ __forceinline__ float load(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
    static __device__ __forceinline__ void store(void* p, int64_t i, float x) { static_cast<float*>(p)[i] = x; }
};

// Maximum / sum over the workgroup (4 wavefronts), result in every thread.
__device__ __forceinline__ float block_reduce(float x, bool is_max, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float y = __shfl_xor(x, o);
        x = is_max ? fmaxf(x, y) : x + y;
    }
    const int wave = threadIdx.x >> 6;
    __syncthreads();                         // red is reused by consecutive reductions
    if ((threadIdx.x & 63) == 0) red[wave] = x;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < kEagerThreads / 64; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
    return r;
}

struct EagerRow {
    int64_t row;
    int b, h, l, kvh, visible;
};

__device__ __forceinline__ EagerRow eager_row(const slimkv_eager_attention_args& a) {
    EagerRow r;
    r.row = blockIdx.x;
    r.l = (int)(r.row % a.queries);
    r.h = (int)((r.row / a.queries) % a.heads);
    r.b = (int)(r.row / (a.queries * a.heads));
    r.kvh = r.h / (int)(a.heads / a.kv_heads);
    // key n is visible unless n > l + keys - queries (bottom-right causal)
    const int64_t vis = a.causal ? std::min<int64_t>(a.keys, (int64_t)r.l + a.keys - a.queries + 1) : a.keys;
    r.visible = (int)std::max<int64_t>(vis, 0);
    return r;
}

template <int DT>
__global__ void __launch_bounds__(kEagerThreads) eager_scores_kernel(slimkv_eager_attention_args a) {
    extern __shared__ float qs[];            // the query row in fp32, then 4 reduction slots
    float* red = qs + a.rank;
    const EagerRow r = eager_row(a);
    const int64_t qoff = (int64_t)r.b * a.q_sb + (int64_t)r.l * a.q_sl + (int64_t)r.h * a.q_sh;
    for (int e = threadIdx.x; e < a.rank; e += kEagerThreads) qs[e] = Elem<DT>::load(a.q, qoff + e);
    __syncthreads();
    float* srow = a.scores + r.row * a.keys;
    const float scale = (float)a.scale;
    const int64_t kbase = (int64_t)r.b * a.k_sb + (int64_t)r.kvh * a.k_sh;
    float mx = kNegInf;
    for (int n = threadIdx.x; n < a.keys; n += kEagerThreads) {
        float s = kNegInf;
        if (n < r.visible) {
            const int64_t ko = kbase + (int64_t)n * a.k_sn;
            float acc = 0.f;
            for (int e = 0; e < a.rank; ++e) acc = fmaf(qs[e], Elem<DT>::load(a.k, ko + e), acc);
            s = acc * scale;
        }
        srow[n] = s;
        mx = fmaxf(mx, s);
    }
    mx = block_reduce(mx, true, red);
    float sum = 0.f;
    if (mx != kNegInf)
        for (int n = threadIdx.x; n < r.visible; n += kEagerThreads) sum += expf(srow[n] - mx);
    sum = block_reduce(sum, false, red);
    const float lse = mx == kNegInf ? kNegInf : mx + logf(sum);
    // probabilities in place: exp(s - lse), zero where the row sees no key
    for (int n = threadIdx.x; n < a.keys; n += kEagerThreads)
        srow[n] = (lse == kNegInf || n >= r.visible) ? 0.f : expf(srow[n] - lse);
    if (threadIdx.x == 0) a.lse[r.row] = lse;
}

template <int DT>
__global__ void __launch_bounds__(kEagerThreads) eager_output_kernel(slimkv_eager_attention_args a) {
    const EagerRow r = eager_row(a);
    const float* prow = a.scores + r.row * a.keys;
    const int64_t vbase = (int64_t)r.b * a.v_sb + (int64_t)r.kvh * a.v_sh;
    const int64_t obase = (int64_t)r.b * a.o_sb + (int64_t)r.l * a.o_sl + (int64_t)r.h * a.o_sh;
    for (int d = threadIdx.x; d < a.rank_v; d += kEagerThreads) {
        float acc = 0.f;
        for (int n = 0; n < r.visible; ++n) acc = fmaf(prow[n], Elem<DT>::load(a.v, vbase + (int64_t)n * a.v_sn + d), acc);
        Elem<DT>::store(a.out, obase + d, acc);
    }
}

template <int DT>
__global__ void __launch_bounds__(256) merge_typed_kernel(slimkv_merge_args a) {
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t rows = a.batch * a.heads * a.length;
    if (gid >= rows * a.dim) return;
    const int64_t row = gid / a.dim;
    const int64_t d = gid % a.dim;
    const int64_t q = row % a.length;
    const int64_t hh = (row / a.length) % a.heads;
    const int64_t b = row / (a.length * a.heads);
    const float r = a.raw_lse[b * a.rl_sb + hh * a.rl_sh + q * a.rl_sl];
    const float l = a.latent_lse[b * a.ll_sb + hh * a.ll_sh + q * a.ll_sl];
    const float total = fmaxf(r, l) + log1pf(expf(-fabsf(r - l)));
    const float x = Elem<DT>::load(a.raw, b * a.r_sb + hh * a.r_sh + q * a.r_sl + d);
    const float y = Elem<DT>::load(a.latent, b * a.l_sb + hh * a.l_sh + q * a.l_sl + d);
    Elem<DT>::store(a.out, gid, expf(r - total) * x + expf(l - total) * y);
}

}  // namespace

}  // namespace slimkv

using namespace slimkv;

extern "C" int slimkv_eager_attention(const slimkv_eager_attention_args* a, void* stream) {
    if (!a || !a->q || !a->k || !a->v || !a->out || !a->lse || !a->scores) return fail(SLIMKV_EINVAL, "null pointer");
    if (a->batch <= 0 || a->queries <= 0 || a->heads <= 0 || a->kv_heads <= 0 || a->heads % a->kv_heads ||
        a->keys <= 0 || a->rank <= 0 || a->rank_v <= 0)
        return fail(SLIMKV_EINVAL, "invalid eager attention sizes or GQA head counts");
    if (a->rank > 4096 || a->keys >= ((int64_t)1 << 31) || a->batch * a->heads * a->queries >= ((int64_t)1 << 31))
        return fail(SLIMKV_EUNSUP, "eager attention supports ranks up to 4096 and 2^31 keys and query rows");
    if (a->dtype != SLIMKV_DTYPE_BF16 && a->dtype != SLIMKV_DTYPE_F16 && a->dtype != SLIMKV_DTYPE_F32)
        return fail(SLIMKV_EINVAL, "dtype must be SLIMKV_DTYPE_BF16, _F16 or _F32");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const unsigned rows = (unsigned)(a->batch * a->heads * a->queries);
    const size_t lds = (size_t)(a->rank + kEagerThreads / 64) * sizeof(float);
    switch (a->dtype) {
        case SLIMKV_DTYPE_BF16:
            hipLaunchKernelGGL(eager_scores_kernel<SLIMKV_DTYPE_BF16>, dim3(rows), dim3(kEagerThreads), lds, st, *a);
            hipLaunchKernelGGL(eager_output_kernel<SLIMKV_DTYPE_BF16>, dim3(rows), dim3(kEagerThreads), 0, st, *a);
            break;
        case SLIMKV_DTYPE_F16:
            hipLaunchKernelGGL(eager_scores_kernel<SLIMKV_DTYPE_F16>, dim3(rows), dim3(kEagerThreads), lds, st, *a);
            hipLaunchKernelGGL(eager_output_kernel<SLIMKV_DTYPE_F16>, dim3(rows), dim3(kEagerThreads), 0, st, *a);
            break;
        default:
            hipLaunchKernelGGL(eager_scores_kernel<SLIMKV_DTYPE_F32>, dim3(rows), dim3(kEagerThreads), lds, st, *a);
            hipLaunchKernelGGL(eager_output_kernel<SLIMKV_DTYPE_F32>, dim3(rows), dim3(kEagerThreads), 0, st, *a);
            break;
    }
    return check_hip(hipGetLastError(), "eager attention launch");
}

extern "C" int slimkv_merge_typed(const slimkv_merge_args* a, int dtype, void* stream) {
    if (!a || !a->raw || !a->latent || !a->raw_lse || !a->latent_lse || !a->out)
        return fail(SLIMKV_EINVAL, "null pointer");
    if (a->batch <= 0 || a->heads <= 0 || a->length <= 0 || a->dim <= 0)
        return fail(SLIMKV_EINVAL, "invalid merge sizes");
    const int64_t items = a->batch * a->heads * a->length * a->dim;
    const int64_t blocks = (items + 255) / 256;
    if (blocks >= ((int64_t)1 << 31)) return fail(SLIMKV_EINVAL, "merge too large");
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case SLIMKV_DTYPE_BF16:
            hipLaunchKernelGGL(merge_typed_kernel<SLIMKV_DTYPE_BF16>, dim3((unsigned)blocks), dim3(256), 0, st, *a);
            break;
        case SLIMKV_DTYPE_F16:
            hipLaunchKernelGGL(merge_typed_kernel<SLIMKV_DTYPE_F16>, dim3((unsigned)blocks), dim3(256), 0, st, *a);
            break;
        case SLIMKV_DTYPE_F32:
            hipLaunchKernelGGL(merge_typed_kernel<SLIMKV_DTYPE_F32>, dim3((unsigned)blocks), dim3(256), 0, st, *a);
            break;
        default:
            return fail(SLIMKV_EINVAL, "dtype must be SLIMKV_DTYPE_BF16, _F16 or _F32");
    }
    return check_hip(hipGetLastError(), "merge kernel launch");
}
