// Shared device helpers of the gfx950 attention kernels: vector types, MFMA wrappers whose register layouts the kernels
// rely on, wave-level reductions, and base-2 exponentials.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

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

// max / sum of v and its value in lane ^ 32 (lane ^ 16) without the LDS round trip of a bpermute: v_permlane32_swap
// (v_permlane16_swap) hands lane l the value of lane l ^ 32 (l ^ 16) in one of its two results and keeps its own in the
// other, so the max or sum of the two is the pair's in every lane (the same sum in both lanes of a pair: a + b = b + a).
// Every lane of the wave must be active.
// The max is one v_max_f32 in asm: fmaxf on the swap's results costs a canonicalizing v_max of each first (the
// compiler cannot tell that they are not signaling NaNs); scores are never NaN here.
__device__ __forceinline__ float vmax_raw(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ float xor32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return vmax_raw(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_add(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return vmax_raw(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_add(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over the 64 lanes of a wave, in every lane, without LDS: within each row of 16 lanes row_mirror (lane i with
// 15 - i), row_half_mirror (i with 7 - i inside each half) and two quad permutations (xor 2, xor 1) pair distinct lanes
// at each step, so after four DPP moves every lane holds its row's sum; then the xor-16 and xor-32 swaps. Every lane of
// the wave must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_pair_add(float v) {
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ float dpp_pair_max(float v) {
    return vmax_raw(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false)));
}
// the maximum over each row of 16 lanes, in every lane of the row (the same pairing as wave_sum)
__device__ __forceinline__ float row16_max(float v) {
    v = dpp_pair_max<0x140>(v);
    v = dpp_pair_max<0x141>(v);
    v = dpp_pair_max<0x4E>(v);
    return dpp_pair_max<0xB1>(v);
}
__device__ __forceinline__ float row16_sum(float v) {
    v = dpp_pair_add<0x140>(v);
    v = dpp_pair_add<0x141>(v);
    v = dpp_pair_add<0x4E>(v);
    return dpp_pair_add<0xB1>(v);
}
__device__ __forceinline__ float wave_sum(float v) {
    // row_mirror (0x140), row_half_mirror (0x141), quad_perm [2, 3, 0, 1] (0x4E), quad_perm [1, 0, 3, 2] (0xB1)
    return xor32_add(xor16_add(row16_sum(v)));
}

// f(std::integral_constant<int, i>) for i = B .. E - 1, each i a compile-time constant (immediate operands of inline asm)
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F && f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

__device__ __forceinline__ half8_t as_half8(u32x4 v) { return __builtin_bit_cast(half8_t, v); }

// 16-byte global load through the vector memory path.
// 16-byte load from global memory. The address space is explicit so that a pointer the compiler cannot trace back to a
// kernel argument (one pinned into registers by an asm statement) still gives a global load, not a flat one, which
// also counts against the LDS/scalar wait counter and so turns the waits for LDS into waits for memory.
__device__ __forceinline__ u32x4 load16(const void * p) { return *(const __attribute__((address_space(1))) u32x4 *)(p); }

// Maps a workgroup index to a work index so that each XCD (the chip has 8, and consecutive workgroups are dealt out to
// them round-robin) runs a contiguous range of the work order: neighbours in that order share keys/values in one L2.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t n) {
    constexpr uint32_t kXcd = 8;
    const uint32_t per = n / kXcd, rem = n % kXcd, x = bid % kXcd, i = bid / kXcd;
    // XCDs 0..rem-1 get per + 1 items, the others per
    return (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + i;
}

// ---- rotary embedding (the reference's rotate_pair / pair_index, src/backend/metal/llama_kernels.h:508-518) ----

// sin and cos of an f32 angle (|x| up to ~1e9): Cody-Waite reduction by pi/2 in double (pi/2 split in two doubles,
// fma), so the reduced |r| <= pi/4 is exact to f32, then the Taylor series of sin and cos to degree 11 / 12 in f32
// (truncation below 2e-9 there). Error a few f32 ulps of 1; no large-argument slow path, no private memory.
__device__ __forceinline__ void sincos_rope(float x, float & s_out, float & c_out) {
    constexpr double kTwoOverPi = 0.63661977236758134308, kPio2Hi = 1.5707963267948966, kPio2Lo = 6.123233995736766e-17;
    const double k = __builtin_rint((double)x * kTwoOverPi);
    const float r = (float)__builtin_fma(-k, kPio2Lo, __builtin_fma(-k, kPio2Hi, (double)x));
    const float r2 = r * r;
    float sp = -1.f / 39916800.f;
    sp = __builtin_fmaf(sp, r2, 1.f / 362880.f);
    sp = __builtin_fmaf(sp, r2, -1.f / 5040.f);
    sp = __builtin_fmaf(sp, r2, 1.f / 120.f);
    sp = __builtin_fmaf(sp, r2, -1.f / 6.f);
    const float sn = __builtin_fmaf(sp * r2, r, r);
    float cp = 1.f / 479001600.f;
    cp = __builtin_fmaf(cp, r2, -1.f / 3628800.f);
    cp = __builtin_fmaf(cp, r2, 1.f / 40320.f);
    cp = __builtin_fmaf(cp, r2, -1.f / 720.f);
    cp = __builtin_fmaf(cp, r2, 1.f / 24.f);
    cp = __builtin_fmaf(cp, r2, -0.5f);
    const float cs = __builtin_fmaf(cp, r2, 1.f);
    const int q = (int)((long long)k & 3);
    s_out = q == 0 ? sn : q == 1 ? cs : q == 2 ? -sn : -cs;
    c_out = q == 0 ? cs : q == 1 ? -sn : q == 2 ? -cs : sn;
}

// Rotates the N 8-element chunks of one head row that a lane holds, chunk c covering head dims STRIDE c + off .. + 8
// (off a multiple of 8 below STRIDE, N * STRIDE = head_dim), in f32. Pair i turns by the angle whose (cos, sin)
// cs_of(i) returns (a float2): theta = pos * base^(-2i / head_dim). mode 0: adjacent pairs (2i, 2i + 1), llama.cpp's
// "normal"; 1: split halves (i, i + head_dim / 2), "neox" (qwen2) -- the partner of chunk c is chunk c + N / 2 of the
// same lane; 2: none.
template <int N, int STRIDE, class CsOf>
__device__ __forceinline__ void rope_rotate(float (&x)[N][8], int off, int mode, CsOf cs_of) {
    auto rot = [&](float & a, float & b, int i) {
        const float2 t = cs_of(i);
        const float ra = a * t.x - b * t.y, rb = a * t.y + b * t.x;
        a = ra;
        b = rb;
    };
    if (mode == 0) {
#pragma unroll
        for (int c = 0; c < N; c++)
#pragma unroll
            for (int e = 0; e < 8; e += 2) rot(x[c][e], x[c][e + 1], (STRIDE * c + off + e) / 2);
    } else if (mode == 1) {
#pragma unroll
        for (int c = 0; c < N / 2; c++)
#pragma unroll
            for (int e = 0; e < 8; e++) rot(x[c][e], x[c + N / 2][e], STRIDE * c + off + e);
    }
}

__device__ __forceinline__ void load8f(const float * src, float (&x)[8]) {  // global memory (global loads, not flat)
    typedef const __attribute__((address_space(1))) float4_t * gp;
    const float4_t a = *(gp)(src), b = *(gp)(src + 4);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        x[e] = a[e];
        x[4 + e] = b[e];
    }
}

// bf16 <-> f32: a bf16 value is the upper half of an f32; to_bf16 rounds to nearest even, NaN stays a (quiet) NaN
__device__ __forceinline__ uint16_t to_bf16(float v) {
    const uint32_t b = __float_as_uint(v);
    return v != v ? (uint16_t)0x7FC0u : (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ void bf16x8_to_f32(u32x4 w, float (&x)[8]) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
        x[2 * e] = __uint_as_float(w[e] << 16);
        x[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
    }
}

__device__ __forceinline__ u32x4 to_half8(const float (&x)[8]) {
    half8_t h;
#pragma unroll
    for (int e = 0; e < 8; e++) h[e] = (half_t)x[e];
    return __builtin_bit_cast(u32x4, h);
}

}  // namespace mx
