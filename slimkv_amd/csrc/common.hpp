// Shared device helpers for the gfx950 kernels: bf16 bit conversions, 16-byte
// vector types, the bf16 MFMA tile, wavefront reductions and error plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/slimkv_hip.h"

namespace slimkv {

typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kNegInf = -__builtin_inff();
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float bf16_to_f32(uint32_t bits) {
    return __uint_as_float(bits << 16);
}

// bf16(a) | bf16(b) << 16 with the gfx950 packed conversion: round to nearest
// even, as torch's float -> bfloat16 conversion, for every non-NaN input; a
// NaN keeps its payload, quieted (torch writes the canonical 0x7fc0).
typedef __bf16 bf16x2_hw __attribute__((ext_vector_type(2)));
typedef float f32x2_hw __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_hw{a, b}, bf16x2_hw));
}
// bf16(x) as a float in one packed conversion: bf16(0) lands in the low half.
__device__ __forceinline__ float round_bf16_hw(float x) { return __uint_as_float(pack_bf16(0.f, x)); }
__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Four bf16 held in two dwords, as the MFMA operand wants them.
__device__ __forceinline__ v4s as_v4s(uint32_t lo, uint32_t hi) {
    u32x2 t = {lo, hi};
    return __builtin_bit_cast(v4s, t);
}

// D = A(16x16) * B(16x16) + C, bf16 inputs, fp32 accumulate.  Lane l holds
// A[l%16][4*(l/16)+i], B[4*(l/16)+i][l%16], and D[4*(l/16)+i][l%16], i = 0..3.
__device__ __forceinline__ v4f mfma16(v4s a, v4s b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// D = A(16x32) * B(32x16) + C on the gfx950 16x16x32 bf16 MFMA.  Lane l holds
// A[l%16][8*(l/16)+j], B[8*(l/16)+j][l%16] (j = 0..7, eight bf16 in a u32x4)
// and D[4*(l/16)+i][l%16].
__device__ __forceinline__ v4f mfma32(u32x4 a, u32x4 b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) {
    return __builtin_amdgcn_exp2f(x);
}

__device__ __forceinline__ float shfl_xor_f(float v, int mask) {
    return __shfl_xor(v, mask, 64);
}

// Reductions over the four 16-lane rows of a wave (lanes l, l ^ 16, l ^ 32,
// l ^ 48) with gfx950's row swaps (v_permlane16_swap / v_permlane32_swap,
// VALU instructions: no LDS round trip).  With both operands equal a swap
// hands lane l the pair (x_l, x_l^16) (resp. x_l^32) in an order symmetric
// over the pair, so every lane of the group ends with the same value, summed
// as (x_l + x_l^16) + (x_l^32 + x_l^48) as the xor shuffles would.
__device__ __forceinline__ float rows_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float rows_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ int64_t clamp_i64(int64_t x, int64_t lo, int64_t hi) {
    return x < lo ? lo : (x > hi ? hi : x);
}

// Block-table entry -> page index with torch's indexing rules: [-n, 0) counts
// from the end of the pool; -1 marks an entry outside [-n, n) (an index error).
__device__ __forceinline__ int64_t table_page(int64_t id, int64_t n) {
    const int64_t p = id < 0 ? id + n : id;
    return (p >= 0 && p < n) ? p : -1;
}

// Index-error report: an ordinary store of the status code (any number of
// lanes may store the same value).
__device__ __forceinline__ void report_bad_page(int32_t* status) {
    if (status) *status = SLIMKV_STATUS_BAD_PAGE;
}

// Thread-local message behind slimkv_last_error().
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_hip(hipError_t err, const char* what);
int device_cu_count();
int reconstruct(const slimkv_reconstruct_args* a, hipStream_t st);

}  // namespace slimkv
