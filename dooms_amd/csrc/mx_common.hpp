// Shared device helpers of the gfx950 attention kernels: vector types, MFMA wrappers whose register layouts the kernels
// rely on, wave-level reductions, and base-2 exponentials.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mx {

typedef _Float16 half_t;
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

// D = A (16x32) * B (32x16) + C on the matrix cores (v_mfma_f32_16x16x32_f16). Register layout, for lane l of the wave:
//   a: A[l % 16][8 * (l / 16) + e], e = 0..7        b: B[8 * (l / 16) + e][l % 16]
//   c, result: C[4 * (l / 16) + v][l % 16], v = 0..3
// The position of the 8 reduction elements inside a lane's operand only has to agree between a and b.
__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// D = A (32x16) * B (16x32) + C (v_mfma_f32_32x32x16_f16). For lane l:
//   a: A[l % 32][8 * (l / 32) + e]                   b: B[8 * (l / 32) + e][l % 32]
//   c, result: C[8 * (v / 4) + 4 * (l / 32) + v % 4][l % 32], v = 0..15
__device__ __forceinline__ float16_t mfma32x32x16(half8_t a, half8_t b, float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// 2^x on the transcendental unit (v_exp_f32); 2^-inf = 0.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float log2_fast(float x) { return __builtin_amdgcn_logf(x); }

// Exchange with the lane `mask` away (xor) inside the wave, through ds_bpermute.
__device__ __forceinline__ float shfl_xor(float v, int mask) {
    const int lane = __lane_id();
    return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}

__device__ __forceinline__ half8_t as_half8(u32x4 v) { return __builtin_bit_cast(half8_t, v); }

// 16-byte global load through the vector memory path.
__device__ __forceinline__ u32x4 load16(const void * p) { return *reinterpret_cast<const u32x4 *>(p); }

// Maps a workgroup index to a work index so that each XCD (the chip has 8, and consecutive workgroups are dealt out to
// them round-robin) runs a contiguous range of the work order: neighbours in that order share keys/values in one L2.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t n) {
    constexpr uint32_t kXcd = 8;
    const uint32_t per = n / kXcd, rem = n % kXcd, x = bid % kXcd, i = bid / kXcd;
    // XCDs 0..rem-1 get per + 1 items, the others per
    return (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + i;
}

}  // namespace mx
