// Projections over f16 weights: Y = X W^T (+ bias), optionally RMS-normalized input, accumulate, f16 output.
//
// Reference behaviour (dooms.cpp 0.6.1, src/backend/metal/llama_kernels.h):
//   * matvec1 (96-126) / matvecm (809-842), one to eight tokens: f32 input rows, y = (W . (x * gamma)) * scale + bias,
//     scale = 1 / sqrt(sum x^2 / K + eps) reduced over the row (stage_input, 62-80);
//   * matmul / matmul_big (222-255, 418-450), prompt chunks: the input tile staged as half(x * gamma * scale) with the
//     row scale from rms_scale (312-328), half x half products accumulated in f32, then + bias, or added into y.
//   * the Whisper cross-attention cache: matmul_big into an f32 scratch, then to_half (metal_whisper_decoder.mm:295-316);
//     here the GEMM rounds to half in its epilogue and writes the cache row directly.
//
// MI355X design:
//   * M <= 8 (decode): gemv_kernel, HBM-bound on the weights (2 N K bytes, each read once). One workgroup per CU
//     (1 to 8 waves, as the rows divide) stages the (normalized) input rows in LDS once; each wave owns 2 or 4 weight rows and
//     streams them in 16-byte non-temporal loads (the weights are read once per step; the cache lines are not kept:
//     q|k|v 12.9 -> 11.7 us, attn_output 10.1 -> 9.3 us, a 14336-column down projection 26.0 -> 23.2 us), 4 sweeps
//     (8 with eight input rows) of 2 or 4 loads in flight per lane. The input rows' loads go out first, in one
//     batch, then the first sweeps of weight loads, so that the staging waits only for the input; the dot products
//     stay f32 and are reduced across the wave at the end.
//   * M > 8 (prompt): stage_kernel writes each input row once as half(x * gamma * scale) into the workspace (the
//     reference stages the same values per tile); gemm_kernel, v_mfma_f32_32x32x16_f16 on 128 x 128 output tiles, K in
//     steps of 64 through LDS (double buffer, rows padded to 72 halves so that the 16-byte operand reads of 16
//     consecutive rows hit 16 distinct 4-bank groups), the step after next loading while the current step multiplies.
//     Each wave owns a 64 x 64 block (2 x 2 MFMA tiles); two workgroups per CU.
//   * Several matrices with the same input and shape (the cross cache's K and V of every layer) run in one launch.
//   * mx_linear runs these kernels only: no vendor GEMM library is loaded or linked.

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "mx_common.hpp"
#include "mx_kernels.hpp"

namespace mx {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// ---- M > 8: the input rows staged once as half, as the reference's matmul staging does per tile
// (half(x * gamma * rms_scale), llama_kernels.h:186-199, with rms_scale from llama_kernels.h:312-328): one workgroup
// per row; the GEMM then multiplies half operands only ----
template <bool NORM>
__global__ __launch_bounds__(kThreads) void stage_kernel(LinearParams p) {
    __shared__ float red[kWaves];
    const float * row = p.x + (int64_t)blockIdx.x * p.x_stride;
    const int kp = (p.K + 63) / 64 * 64;  // staged rows are zero-padded to a multiple of 64 columns
    half_t * dst = p.xh + (int64_t)blockIdx.x * kp;
    const int K4 = p.K / 4;
    constexpr int SJ = 8;  // 16-byte pieces per thread held in registers
    if (K4 <= SJ * kThreads) {
        // the row (and gamma) loaded once, all pieces in flight together; the sum of squares and the conversion then
        // work from registers
        float4_t v[SJ], g[SJ];
#pragma unroll
        for (int j = 0; j < SJ; j++) {
            const int kk = min(j * kThreads + (int)threadIdx.x, K4 - 1);
            v[j] = *reinterpret_cast<const float4_t *>(row + 4 * kk);
            if constexpr (NORM) g[j] = *reinterpret_cast<const float4_t *>(p.gamma + 4 * kk);
        }
        float s = 1.f;
        if constexpr (NORM) {
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < SJ; j++)
                if (j * kThreads + (int)threadIdx.x < K4)
                    ss += v[j][0] * v[j][0] + v[j][1] * v[j][1] + v[j][2] * v[j][2] + v[j][3] * v[j][3];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) ss += shfl_xor(ss, o);
            if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = ss;
            __syncthreads();
            float t = 0.f;
#pragma unroll
            for (int w = 0; w < kWaves; w++) t += red[w];
            s = 1.f / __builtin_sqrtf(t / (float)p.K + p.eps);
        }
#pragma unroll
        for (int j = 0; j < SJ; j++) {
            const int kk = j * kThreads + (int)threadIdx.x;
            if (kk >= K4) continue;
            half4_t h;
#pragma unroll
            for (int e = 0; e < 4; e++) h[e] = (half_t)(NORM ? v[j][e] * (g[j][e] * s) : v[j][e]);
            *reinterpret_cast<half4_t *>(dst + 4 * kk) = h;
        }
        for (int k = p.K + threadIdx.x * 8; k < kp; k += kThreads * 8) *reinterpret_cast<u32x4 *>(dst + k) = u32x4{0u, 0u, 0u, 0u};
        return;
    }
    float s = 1.f;
    if constexpr (NORM) {
        float ss = 0.f;
        for (int k = threadIdx.x * 4; k < p.K; k += kThreads * 4) {
            const float4_t v = *reinterpret_cast<const float4_t *>(row + k);
            ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += shfl_xor(ss, o);
        if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = ss;
        __syncthreads();
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) t += red[w];
        s = 1.f / __builtin_sqrtf(t / (float)p.K + p.eps);
    }
    for (int k = threadIdx.x * 8; k < p.K; k += kThreads * 8) {
        float x[8];
        load8f(row + k, x);
        if constexpr (NORM) {
            float g[8];
            load8f(p.gamma + k, g);
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] *= g[e] * s;  // x * (gamma * scale), as the reference's staging
        }
        *reinterpret_cast<u32x4 *>(dst + k) = to_half8(x);
    }
    for (int k = p.K + threadIdx.x * 8; k < kp; k += kThreads * 8) *reinterpret_cast<u32x4 *>(dst + k) = u32x4{0u, 0u, 0u, 0u};
}

// y (+)= v (+ bias) into row m, column n of output matrix mi.
template <bool OUT16>
__device__ __forceinline__ void store_y(const LinearParams & p, int mi, int m, int n, float v) {
    if (p.flags & kLinearBias) {
        const float * b = p.bias[mi];
        if (b) v += b[n];
    }
    const int64_t o = (int64_t)m * p.y_stride + n;
    if constexpr (OUT16) {
        half_t * y = static_cast<half_t *>(p.y[mi]);
        if (p.flags & kLinearAccumulate) v += (float)y[o];
        y[o] = (half_t)v;
    } else {
        float * y = static_cast<float *>(p.y[mi]);
        if (p.flags & kLinearAccumulate) v += y[o];
        y[o] = v;
    }
}

// Epilogue of the tiled GEMMs: the lane's 16 outputs of column n of an MFMA tile (rows mbase + 8 (v / 4) + v % 4),
// y (+)= acc (+ bias), the same sums as store_y. The bias and the previous outputs are all loaded before the first
// store: a store to y may alias them as far as the compiler can tell, so with loads and stores interleaved each
// element waited for one or two memory round trips in turn. Rows past M read row M - 1 (a valid address) and store
// nothing.
template <bool OUT16>
__device__ __forceinline__ void store_col16(const LinearParams & p, int mi, int n, int mbase, const float16_t & acc) {
    const float * b = (p.flags & kLinearBias) ? p.bias[mi] : nullptr;
    const float bv = b ? b[n] : 0.f;
    const bool accum = p.flags & kLinearAccumulate;
    float prev[16];
    if (accum) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int m = min(mbase + 8 * (v / 4) + v % 4, p.M - 1);
            const int64_t o = (int64_t)m * p.y_stride + n;
            if constexpr (OUT16) prev[v] = (float)static_cast<const half_t *>(p.y[mi])[o];
            else prev[v] = static_cast<const float *>(p.y[mi])[o];
        }
    }
    // every sum before the first store, so that no loaded value is used behind a store (the compiler's waits at the
    // stores' branches would otherwise drain the stores before it)
    float x[16];
#pragma unroll
    for (int v = 0; v < 16; v++) {
        x[v] = acc[v];
        if (b) x[v] += bv;
        if (accum) x[v] += prev[v];
    }
#pragma unroll
    for (int v = 0; v < 16; v++) {
        const int m = mbase + 8 * (v / 4) + v % 4;
        if (m >= p.M) continue;
        const int64_t o = (int64_t)m * p.y_stride + n;
        if constexpr (OUT16) static_cast<half_t *>(p.y[mi])[o] = (half_t)x[v];
        else static_cast<float *>(p.y[mi])[o] = x[v];
    }
}

// ---- M <= 8: f32 input rows in LDS, 2 or 4 weight rows per wave ----
constexpr int kGemvRows = 4;       // weight rows per wave (the most)
constexpr int kGemvMaxWaves = 8;   // waves per workgroup (the launch sizes workgroups so that each CU gets one)
// 64-lane sweeps of 16-byte weight loads in flight per wave: 4, and 8 with eight input rows (more arithmetic per
// weight byte; Llama-3-8B attention output at 8 rows 19.7 -> 17.2 us, while at 1, 2 and 4 rows 8 sweeps were 3-25 %
// slower than 4)
template <int MT>
constexpr int gemv_depth() { return MT == 8 ? 8 : 4; }

// STAGE: the input rows (times gamma) fit the LDS budget and are staged once; otherwise every wave reads them from
// L2 as it goes (the reference's kStageInput = false variant, metal_llama_decoder.mm:45-47).
// The wave's first gemv_depth sweeps of weight loads are issued before the input is staged, so the staging and its
// barriers overlap the first HBM round trip.
template <int MT, bool STAGE, bool OUT16, bool NORM, int RW>
__global__ __launch_bounds__(kGemvMaxWaves * kWave) void gemv_kernel(LinearParams p) {
    extern __shared__ float xs[];  // [MT][K]: x (* gamma) of each input row, when staged
    __shared__ float red[MT][kGemvMaxWaves];
    __shared__ float s_scale[MT];
    constexpr int kGemvDepth = gemv_depth<MT>();
    const int K = p.K, M = p.M;
    constexpr bool norm = NORM;  // p.flags & kLinearNorm
    const int nw = blockDim.x / kWave;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;

    // work item: (matrix, group of RW rows) per wave
    const int groups = (p.N + RW - 1) / RW;
    const int item = __builtin_amdgcn_readfirstlane(blockIdx.x * nw + wave);  // wave-uniform: scalar loads of p.w[mi]
    const bool active = item < groups * p.count;
    const int mi = active ? item / groups : 0;
    const int r0 = active ? (item % groups) * RW : 0;
    const half_t * w = p.w[mi];
    const half_t * wr[RW];
#pragma unroll
    for (int i = 0; i < RW; i++) wr[i] = w + (int64_t)min(r0 + i, p.N - 1) * K;
    const int C8 = K / 8;  // 16-byte chunks per row
    half8_t wv[kGemvDepth][RW];
    auto load_sweep = [&](int j, int c) __attribute__((always_inline)) {
        const int cc = min(c, C8 - 1);  // past the row: a valid chunk, not used
#pragma unroll
        for (int i = 0; i < RW; i++)  // non-temporal: each weight is read once per step
            wv[j][i] = as_half8(__builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4 *)(wr[i] + 8 * cc)));
    };

    // The input rows (and gamma) in batches: batch b covers the 16-byte chunks kk = (b XJ + j) blockDim + tid, j < XJ,
    // of every input row. All of a batch's loads go out before any wait (clamped, unconditional), and batch 0 goes out
    // ahead of the weight loads: loads complete in issue order, so its wait leaves the weights in flight.
    constexpr int XJ = MT >= 4 ? 1 : 4 / MT;
    const int K4 = K / 4;
    const int nxb = (STAGE || NORM) ? (K4 + XJ * (int)blockDim.x - 1) / (XJ * (int)blockDim.x) : 0;
    float4_t xv[MT][XJ], gv[XJ];
    float ss[MT];
#pragma unroll
    for (int m = 0; m < MT; m++) ss[m] = 0.f;
    auto xload = [&](int b) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < XJ; j++) {
            const int kk = min((b * XJ + j) * (int)blockDim.x + (int)threadIdx.x, K4 - 1);
            if constexpr (NORM) gv[j] = *reinterpret_cast<const float4_t *>(p.gamma + 4 * kk);
#pragma unroll
            for (int m = 0; m < MT; m++)
                xv[m][j] = *reinterpret_cast<const float4_t *>(p.x + (int64_t)min(m, M - 1) * p.x_stride + 4 * kk);
        }
    };
    // sums of squares (stage_input, llama_kernels.h:62-80) and the staged x (* gamma)
    auto xstage = [&](int b) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < XJ; j++) {
            const int kk = (b * XJ + j) * (int)blockDim.x + (int)threadIdx.x;
            if (kk >= K4) continue;
#pragma unroll
            for (int m = 0; m < MT; m++) {
                const float4_t v = xv[m][j];
                if constexpr (NORM) ss[m] += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
                if constexpr (STAGE)
                    if (m < M) *reinterpret_cast<float4_t *>(xs + m * K + 4 * kk) = NORM ? v * gv[j] : v;
            }
        }
    };
    if constexpr (STAGE || NORM) xload(0);
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order: the input first, then the weights
    // unconditional (an idle wave reads valid rows of matrix 0 and returns below): a branch here would make every
    // later wait assume that the input loads are the newest ones
#pragma unroll
    for (int j = 0; j < kGemvDepth; j++) load_sweep(j, lane + kWave * j);
    // what the epilogue adds to lane i MT + m's output (row r0 + i, input row m): the bias and the previous output,
    // loaded here behind the weights (by every lane, at clamped valid addresses) rather than after the reduction,
    // where each was one more memory round trip at the end of the kernel
    float y_prev = 0.f, y_bias = 0.f;
    {
        const int i = min(lane / MT, RW - 1), m = min(lane % MT, M - 1), n = min(r0 + i, p.N - 1);
        if (p.flags & kLinearAccumulate) {
            const int64_t o = (int64_t)m * p.y_stride + n;
            if constexpr (OUT16) y_prev = (float)static_cast<const half_t *>(p.y[mi])[o];
            else y_prev = static_cast<const float *>(p.y[mi])[o];
        }
        if (p.flags & kLinearBias) {
            const float * b = p.bias[mi];
            if (b) y_bias = b[n];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (STAGE || NORM) xstage(0);
    for (int b = 1; b < nxb; b++) {  // inputs longer than one batch (the waits of these drain the weight loads too)
        xload(b);
        xstage(b);
        // nothing in flight after the loop (else the compiler, for a register whose load may still be pending past
        // the loop, drains every weight load ahead of the sweeps, also where the loop never runs: q|k|v 11.85 ->
        // 11.11 us, Whisper attention output 3.64 -> 3.38)
        __builtin_amdgcn_s_waitcnt(0);
    }
    if (norm) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
            float t = ss[m];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) t += shfl_xor(t, o);
            if (lane == 0) red[m][wave] = t;
        }
    }
    __syncthreads();
    if (norm && threadIdx.x < MT) {
        float t = 0.f;
        for (int w2 = 0; w2 < nw; w2++) t += red[threadIdx.x][w2];
        s_scale[threadIdx.x] = 1.f / __builtin_sqrtf(t / (float)K + p.eps);
    }
    __syncthreads();
    if (!active) return;  // after the last barrier

    float acc[RW][MT];
#pragma unroll
    for (int i = 0; i < RW; i++)
#pragma unroll
        for (int m = 0; m < MT; m++) acc[i][m] = 0.f;
    auto sweep = [&](int j, int c) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < MT; m++) {
            float4_t x0, x1;
            if constexpr (STAGE) {
                x0 = *reinterpret_cast<const float4_t *>(xs + m * K + 8 * c);
                x1 = *reinterpret_cast<const float4_t *>(xs + m * K + 8 * c + 4);
            } else {
                const float * xr = p.x + (int64_t)min(m, M - 1) * p.x_stride + 8 * c;
                x0 = *reinterpret_cast<const float4_t *>(xr);
                x1 = *reinterpret_cast<const float4_t *>(xr + 4);
                if (norm) {
                    x0 = x0 * *reinterpret_cast<const float4_t *>(p.gamma + 8 * c);
                    x1 = x1 * *reinterpret_cast<const float4_t *>(p.gamma + 8 * c + 4);
                }
            }
#pragma unroll
            for (int i = 0; i < RW; i++) {
                float a = acc[i][m];
#pragma unroll
                for (int e = 0; e < 4; e++) a = __builtin_fmaf((float)wv[j][i][e], x0[e], a);
#pragma unroll
                for (int e = 0; e < 4; e++) a = __builtin_fmaf((float)wv[j][i][4 + e], x1[e], a);
                acc[i][m] = a;
            }
        }
    };
    // sweep j of pass q covers chunk 256 q + 64 j + lane; its registers are reloaded for the next pass right after use.
    // The loads are unconditional inside the loop and the last pass is peeled off (no loads), so the compiler's waits
    // track each sweep's own loads instead of draining every load at the top of a pass.
    constexpr int kPass = kWave * kGemvDepth;
    const int npass = (C8 + kPass - 1) / kPass;
    for (int q = 0; q + 1 < npass; q++) {
#pragma unroll
        for (int j = 0; j < kGemvDepth; j++) {
            const int c = q * kPass + kWave * j + lane;  // < C8: not the last pass
            sweep(j, c);
            load_sweep(j, c + kPass);
        }
    }
#pragma unroll
    for (int j = 0; j < kGemvDepth; j++) {
        const int c = (npass - 1) * kPass + kWave * j + lane;
        if (c < C8) sweep(j, c);
    }
    // reduce over the wave; lane i * MT + m stores (row r0 + i, input row m)
    float mine = 0.f;
#pragma unroll
    for (int i = 0; i < RW; i++)
#pragma unroll
        for (int m = 0; m < MT; m++) {
            const float s = wave_sum(acc[i][m]);
            if (lane == i * MT + m) mine = s;
        }
    if (lane < RW * MT) {
        const int i = lane / MT, m = lane % MT, n = r0 + i;
        if (m < M && n < p.N) {  // store_y's sums, with the bias and the previous output loaded above
            float v = norm ? mine * s_scale[m] : mine;
            if (p.flags & kLinearBias) v += y_bias;
            if (p.flags & kLinearAccumulate) v += y_prev;
            const int64_t o = (int64_t)m * p.y_stride + n;
            if constexpr (OUT16) static_cast<half_t *>(p.y[mi])[o] = (half_t)v;
            else static_cast<float *>(p.y[mi])[o] = v;
        }
    }
}

// ---- M > 8: MFMA GEMM on the staged half rows, 128 x 128 tiles, K in steps of 64 ----
constexpr int kTM = 128, kTN = 128, kTK = 64;
constexpr int kPitch = kTK + 8;  // halves per staged row: the 16-byte reads of 16 consecutive rows hit distinct banks
constexpr int kChunks = kTM * (kTK / 8) / kThreads;  // 16-byte chunks per thread per tile and step (4)

template <bool OUT16>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(LinearParams p) {
    __shared__ half_t xs[2][kTM * kPitch];
    __shared__ half_t ws[2][kTN * kPitch];
    const int n_tiles = (p.N + kTN - 1) / kTN, m_tiles = (p.M + kTM - 1) / kTM;
    // consecutive work items share a weight tile (different token tiles); contiguous ranges per XCD
    const uint32_t t = xcd_remap(blockIdx.x, (uint32_t)(p.count * n_tiles * m_tiles));
    const int mt = t % m_tiles, nt = (t / m_tiles) % n_tiles, mi = t / (m_tiles * n_tiles);
    const int m0 = mt * kTM, n0 = nt * kTN;
    const half_t * w = p.w[mi];
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int l32 = lane % 32, hi = lane / 32;

    // staging map: chunk c = threadIdx.x + 256 j is row c / 8, columns 8 (c % 8) .. + 8 of the step. The staged rows are
    // zero-padded to a multiple of 64 columns (kp); a weight column past K (K an odd multiple of 32) is read from the
    // row's last 8 columns instead, finite values that meet the zero padding
    const int kp = (p.K + kTK - 1) / kTK * kTK;
    const int kc = threadIdx.x % 8;  // the same for every j: 256 is a multiple of 8
    const half_t * a0 = p.xh + (int64_t)min(m0 + (int)threadIdx.x / 8, p.M - 1) * kp + 8 * kc;
    const half_t * b0 = w + (int64_t)min(n0 + (int)threadIdx.x / 8, p.N - 1) * p.K;
    const int64_t a_step = (int64_t)(kThreads / 8) * kp, b_step = (int64_t)(kThreads / 8) * p.K;  // 32 rows per j
    const int brow_max = p.N - 1 - n0, arow_max = p.M - 1 - m0;  // rows past N (M) repeat the last row
    // two register sets: step i's tiles travel in set i % 2, loaded two steps before they are stored into LDS
    u32x4 ar[2][kChunks], br[2][kChunks];
    auto load = [&](int step, auto S) __attribute__((always_inline)) {
        constexpr int st = decltype(S)::value;
        const int k0 = step * kTK;
        const int bcol = min(k0 + 8 * kc, p.K - 8);
#pragma unroll
        for (int j = 0; j < kChunks; j++) {
            const int64_t aoff = (int)threadIdx.x / 8 + 32 * j <= arow_max ? j * a_step : (int64_t)(arow_max - (int)threadIdx.x / 8) * kp;
            ar[st][j] = load16(a0 + aoff + k0);
            const int64_t boff = (int)threadIdx.x / 8 + 32 * j <= brow_max ? j * b_step : (int64_t)(brow_max - (int)threadIdx.x / 8) * p.K;
            br[st][j] = load16(b0 + boff + bcol);
        }
    };
    auto store = [&](int buf, auto S) __attribute__((always_inline)) {
        constexpr int st = decltype(S)::value;
#pragma unroll
        for (int j = 0; j < kChunks; j++) {
            const int c = threadIdx.x + kThreads * j, row = c / 8, kc = c % 8;
            *reinterpret_cast<u32x4 *>(&xs[buf][row * kPitch + 8 * kc]) = ar[st][j];
            *reinterpret_cast<u32x4 *>(&ws[buf][row * kPitch + 8 * kc]) = br[st][j];
        }
    };

    float16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

    const int wm = wave / 2, wn = wave % 2;  // this wave's 64 x 64 block
    const int a_base = (64 * wm + l32) * kPitch + 8 * hi;
    const int b_base = (64 * wn + l32) * kPitch + 8 * hi;
    const int nk = kp / kTK;
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    load(0, S0{});
    store(0, S0{});
    load(min(1, nk - 1), S1{});
    load(min(2, nk - 1), S0{});
    // step ib: its tiles are in LDS buffer ib % 2; step ib + 1's go from register set (ib + 1) % 2 into the other
    // buffer, and that set is refilled with step ib + 3's
    // The loads and stores are unconditional (past the last step the last step's tiles are loaded again and go into a
    // buffer nobody reads), so the loop has one path and the waits for one register set leave the other set in flight.
    auto step = [&](int ib, auto S) __attribute__((always_inline)) {
        const int buf = ib & 1;
        __syncthreads();  // step ib is in buffer buf; buffer buf ^ 1 is free
        store(buf ^ 1, S);
        load(min(ib + 3, nk - 1), S);
        const half_t * a_s = xs[buf];
        const half_t * b_s = ws[buf];
#pragma unroll
        for (int ks = 0; ks < kTK / 16; ks++) {
            half8_t a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; i++) a[i] = as_half8(*reinterpret_cast<const u32x4 *>(a_s + a_base + 32 * i * kPitch + 16 * ks));
#pragma unroll
            for (int j = 0; j < 2; j++) b[j] = as_half8(*reinterpret_cast<const u32x4 *>(b_s + b_base + 32 * j * kPitch + 16 * ks));
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) acc[i][j] = mfma32x32x16(a[i], b[j], acc[i][j]);
        }
    };
    int ib = 0;
    for (; ib + 1 < nk; ib += 2) {
        step(ib, S1{});
        step(ib + 1, S0{});
    }
    if (ib < nk) step(ib, S1{});

    // lane holds Y[m0 + 64 wm + 32 i + 8 (v / 4) + 4 hi + v % 4][n0 + 64 wn + 32 j + l32]
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = n0 + 64 * wn + 32 * j + l32;
            if (n < p.N) store_col16<OUT16>(p, mi, n, m0 + 64 * wm + 32 * i + 4 * hi, acc[i][j]);
        }
}

// ---- M > 8, large products: 256 x 256 tiles of 8 waves (each 128 x 64, 4 x 2 MFMA tiles), K in steps of 32 ----
// A 128 x 128 tile streams 64 bytes per clock and CU from L2 at the MFMA rate, the whole of an XCD's L2 bandwidth;
// 256 x 256 halves the bytes per product (and 128 x 64 per wave cuts the LDS reads per product by a quarter). The
// tiles go from HBM/L2 straight into LDS (global_load_lds_dwordx4: lane l's 16 bytes land at byte 16 l of the
// instruction's 1 KB destination), three buffers deep (the loads of step s + 2 in flight while step s multiplies), no
// registers in between. An operand tile (256 rows x 32 columns, 64 bytes per row) is 16 blocks of 16 rows, one load
// instruction each; 16-byte chunk c of row r sits at 16 (c ^ ((r % 16) / 4)) within its row's 64 bytes, so the 16-byte
// operand reads of 16 consecutive rows at one chunk land on 16 distinct 4-bank groups. 96 KB of LDS: one workgroup per
// CU, two waves per SIMD.
// BN = 128 (256 x 128 tiles, 8 waves of 64 x 64) and BN = 192 (256 x 192, 8 waves of 64 x 96) serve products whose
// 256 x 256 tiles would leave CUs idle.
constexpr int kBM = 256;
constexpr int kGemmCUs = 256;
constexpr int kBigWaves = 8, kBigThreads = kBigWaves * kWave;
// WC: columns per wave (64, or 96 for 256 x 192 tiles: 8 waves of 64 x 96). BK: columns per step, 32 (three buffers)
// or 64 (two buffers, half the barriers and load instructions per product; K a multiple of 64).
template <bool OUT16, int BN, int WC = 64, int BK = 32>
__device__ __forceinline__ void gemm_big_tile(const LinearParams & p) {
    constexpr int kBN = BN, kBK = BK;
    constexpr int kBigBufs = BK == 32 ? 3 : 2;
    constexpr int kBigLoads = kBM * kBK * 2 / 1024 / kBigWaves;  // 1 KB direct loads of A per wave and step
    constexpr int RA = kBM / 16, RBB = BN / 16;                  // 16-row blocks per chunk group of A and of B
    constexpr int WN = BN / WC, WM = kBigWaves / WN;         // waves along N and along M
    constexpr int kBigMI = kBM / WM / 32, kBigNJ = WC / 32;  // 32 x 32 MFMA tiles per wave
    constexpr int BBlocks = BN * kBK * 2 / 1024;             // 1 KB blocks of a step's B tile
    constexpr int BLoads = (BBlocks + kBigWaves - 1) / kBigWaves;  // direct loads of B per wave and step; past the
                                                                   // tile's blocks a wave reloads one it already loads
    static_assert(BLoads >= 1 && kBigMI >= 1 && WN * WM == kBigWaves, "whole loads and tiles per wave");
    __shared__ __attribute__((aligned(1024))) half_t xs[kBigBufs][kBM * kBK];
    __shared__ __attribute__((aligned(1024))) half_t ws[kBigBufs][BN * kBK];
    const int n_tiles = (p.N + kBN - 1) / kBN, m_tiles = (p.M + kBM - 1) / kBM;
    // consecutive work items share a weight tile (different token tiles); contiguous ranges per XCD
    const uint32_t t = xcd_remap(blockIdx.x, (uint32_t)(p.count * n_tiles * m_tiles));
    const int mt = t % m_tiles, nt = (t / m_tiles) % n_tiles, mi = t / (m_tiles * n_tiles);
    const int m0 = mt * kBM, n0 = nt * kBN;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x % kWave;
    const int l32 = lane % 32, hi = lane / 32;

    // Each lane's source bytes relative to the step's first column are fixed: rows past M (N) repeat the last row.
    // The staged rows are kp halves apart (K rounded up to 64, zero-padded); the weight rows K halves apart.
    const int kp = (p.K + 63) / 64 * 64;
    const char * a_base = reinterpret_cast<const char *>(p.xh + (int64_t)m0 * kp);
    const char * b_base = reinterpret_cast<const char *>(p.w[mi] + (int64_t)n0 * p.K);
    uint32_t a_off[kBigLoads], b_off[BLoads];
    const int c = (lane % 4) ^ (lane / 16);  // the chunk a lane fetches for position lane % 4 of its row's 64 bytes
    // block j of a tile: chunk group j / R (64-byte column group), rows 16 (j % R) ..
#pragma unroll
    for (int i = 0; i < kBigLoads; i++) {
        const int j = i * kBigWaves + wave;
        const int row = 16 * (j % RA) + lane / 4;  // the row this lane fills
        a_off[i] = (uint32_t)(min(m0 + row, p.M - 1) - m0) * kp * 2 + 64 * (j / RA) + 16 * c;
    }
#pragma unroll
    for (int i = 0; i < BLoads; i++) {
        const int j = i * kBigWaves + wave, jb = j < BBlocks ? j : j - kBigWaves;  // (identical bytes written twice)
        const int row = 16 * (jb % RBB) + lane / 4;
        b_off[i] = (uint32_t)(min(n0 + row, p.N - 1) - n0) * p.K * 2 + 64 * (jb / RBB) + 16 * c;
    }
    auto issue = [&](int step, int buf) __attribute__((always_inline)) {
        const int64_t k0 = (int64_t)step * kBK * 2;  // bytes
        // A and B loads interleaved
#pragma unroll
        for (int i = 0; i < kBigLoads; i++) {
            __builtin_amdgcn_global_load_lds(a_base + k0 + a_off[i],
                                             (__attribute__((address_space(3))) void *)&xs[buf][512 * (i * kBigWaves + wave)],
                                             16, 0, 0);
            if (i < BLoads) {
                const int j = i * kBigWaves + wave, jb = j < BBlocks ? j : j - kBigWaves;
                __builtin_amdgcn_global_load_lds(b_base + k0 + b_off[i],
                                                 (__attribute__((address_space(3))) void *)&ws[buf][512 * jb], 16, 0, 0);
            }
        }
    };

    float16_t acc[kBigMI][kBigNJ];
#pragma unroll
    for (int i = 0; i < kBigMI; i++)
#pragma unroll
        for (int j = 0; j < kBigNJ; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

    // this wave's block: rows (256 / WM) wm + 32 i + l32 of A, columns 64 wn + 32 j + l32 (rows of B); fragment
    // (row, chunk 2 ks + hi) at halves 512 (row / 16) + 32 (row % 16) + 8 ((2 ks + hi) ^ ((row % 16) / 4))
    const int wm = wave / WN, wn = wave % WN;
    int rd[2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) rd[ks] = 512 * (l32 / 16) + 32 * (l32 % 16) + 8 * ((2 * ks + hi) ^ ((l32 % 16) / 4));
    const int nk = p.K / kBK;
#pragma unroll
    for (int a = 0; a < kBigBufs - 1; a++)
        if (a < nk) issue(a, a);
    for (int s = 0; s < nk; s++) {
        const int buf = s % kBigBufs;
        // this wave's loads of step s are complete (those of up to kBigBufs - 2 later steps may be in flight), then
        // every wave's are; the buffer refilled below was last read in step s - 1
        if (kBigBufs > 2 && s + 1 < nk) __builtin_amdgcn_s_waitcnt(0x0F70 | (kBigLoads + BLoads));  // vmcnt(next step)
        else __builtin_amdgcn_s_waitcnt(0x0F70);                                                     // vmcnt(0)
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (s + kBigBufs - 1 < nk) issue(s + kBigBufs - 1, (s + kBigBufs - 1) % kBigBufs);
        // the operand reads as inline asm (the compiler cannot tell them from the direct loads in flight, and would
        // wait for those), all of the step's in flight, the products of each 16-column slice behind their reads
        const uint32_t xa = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) half_t *)xs[buf] + 2 * 32 * (kBM / WM) * wm;
        const uint32_t wa = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) half_t *)ws[buf] + 2 * 32 * WC * wn;
        if constexpr (BK == 64) {
            // 4 slices of 16 columns: slices s + 1's reads in flight behind slice s's products (at most 2 slices of
            // reads outstanding, within the 15 that lgkmcnt counts); the waits are ordered by sched_barrier
            constexpr int R = kBigMI + kBigNJ;  // reads per slice
            u32x4 fa[4][kBigMI], fb[4][kBigNJ];
            auto reads = [&](auto KS) __attribute__((always_inline)) {
                constexpr int ks = decltype(KS)::value;
                const uint32_t ra_ = xa + 2 * (rd[ks % 2] + 512 * RA * (ks / 2)), rb_ = wa + 2 * (rd[ks % 2] + 512 * RBB * (ks / 2));
                static_for<0, kBigMI>([&](auto I) __attribute__((always_inline)) {
                    u32x4 r;
                    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(ra_), "i"(2 * 1024 * decltype(I)::value));
                    fa[ks][decltype(I)::value] = r;
                });
                static_for<0, kBigNJ>([&](auto J) __attribute__((always_inline)) {
                    u32x4 r;
                    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(rb_), "i"(2 * 1024 * decltype(J)::value));
                    fb[ks][decltype(J)::value] = r;
                });
            };
            reads(std::integral_constant<int, 0>{});
            reads(std::integral_constant<int, 1>{});
            static_for<0, 4>([&](auto KS) __attribute__((always_inline)) {
                constexpr int ks = decltype(KS)::value;
                if constexpr (ks < 3) asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(R) : "memory");
                else asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < kBigMI; i++)
#pragma unroll
                    for (int j = 0; j < kBigNJ; j++)
                        acc[i][j] = mfma32x32x16(as_half8(fa[ks][i]), as_half8(fb[ks][j]), acc[i][j]);
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (ks + 2 < 4) reads(std::integral_constant<int, ks + 2>{});
            });
        } else {
            u32x4 fa[2][kBigMI], fb[2][kBigNJ];
            static_for<0, 2>([&](auto KS) __attribute__((always_inline)) {
                constexpr int ks = decltype(KS)::value;
                const uint32_t ra_ = xa + 2 * rd[ks], rb_ = wa + 2 * rd[ks];
                static_for<0, kBigMI>([&](auto I) __attribute__((always_inline)) {
                    constexpr int i = decltype(I)::value;
                    u32x4 r;
                    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(ra_), "i"(2 * 1024 * i));
                    fa[ks][i] = r;
                });
                static_for<0, kBigNJ>([&](auto J) __attribute__((always_inline)) {
                    constexpr int j = decltype(J)::value;
                    u32x4 r;
                    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(rb_), "i"(2 * 1024 * j));
                    fb[ks][j] = r;
                });
            });
            static_for<0, 2>([&](auto KS) __attribute__((always_inline)) {
                constexpr int ks = decltype(KS)::value;
                // slice 0 waits for its reads (slice 1's in flight), slice 1 for all: one wait per slice, tied to the
                // slice's fragments
                static_assert((kBigNJ == 2 && (kBigMI == 4 || kBigMI == 2)) || (kBigNJ == 3 && kBigMI == 2),
                              "the waits below name every fragment");
                if constexpr (kBigNJ == 3) {
                    if constexpr (ks == 0)
                        asm volatile("s_waitcnt lgkmcnt(5)" : "+v"(fa[0][0]), "+v"(fa[0][1]), "+v"(fb[0][0]), "+v"(fb[0][1]),
                                     "+v"(fb[0][2]));
                    else
                        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fa[1][0]), "+v"(fa[1][1]), "+v"(fb[1][0]), "+v"(fb[1][1]),
                                     "+v"(fb[1][2]));
                } else if constexpr (kBigMI == 4) {
                    if constexpr (ks == 0)
                        asm volatile("s_waitcnt lgkmcnt(6)" : "+v"(fa[0][0]), "+v"(fa[0][1]), "+v"(fa[0][2]), "+v"(fa[0][3]),
                                     "+v"(fb[0][0]), "+v"(fb[0][1]));
                    else
                        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fa[1][0]), "+v"(fa[1][1]), "+v"(fa[1][2]), "+v"(fa[1][3]),
                                     "+v"(fb[1][0]), "+v"(fb[1][1]));
                } else {
                    if constexpr (ks == 0)
                        asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(fa[0][0]), "+v"(fa[0][1]), "+v"(fb[0][0]), "+v"(fb[0][1]));
                    else
                        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fa[1][0]), "+v"(fa[1][1]), "+v"(fb[1][0]), "+v"(fb[1][1]));
                }
#pragma unroll
                for (int i = 0; i < kBigMI; i++)
#pragma unroll
                    for (int j = 0; j < kBigNJ; j++)
                        acc[i][j] = mfma32x32x16(as_half8(fa[ks][i]), as_half8(fb[ks][j]), acc[i][j]);
                __builtin_amdgcn_sched_barrier(0);
            });
        }
    }

    // lane holds Y[m0 + (256 / WM) wm + 32 i + 8 (v / 4) + 4 hi + v % 4][n0 + WC wn + 32 j + l32]
#pragma unroll
    for (int i = 0; i < kBigMI; i++)
#pragma unroll
        for (int j = 0; j < kBigNJ; j++) {
            const int n = n0 + WC * wn + 32 * j + l32;
            if (n < p.N) store_col16<OUT16>(p, mi, n, m0 + (kBM / WM) * wm + 32 * i + 4 * hi, acc[i][j]);
        }
}

// K in steps of 64 columns when K is a multiple of 64 (BK = 64), else 32
template <bool OUT16, int BK>
__global__ __launch_bounds__(kBigThreads, 1) void gemm_big_kernel(LinearParams p) { gemm_big_tile<OUT16, 256, 64, BK>(p); }
template <bool OUT16, int BK>
__global__ __launch_bounds__(kBigThreads, 1) void gemm_mid_kernel(LinearParams p) { gemm_big_tile<OUT16, 128, 64, BK>(p); }
template <bool OUT16, int BK>
__global__ __launch_bounds__(kBigThreads, 1) void gemm_w192_kernel(LinearParams p) { gemm_big_tile<OUT16, 192, 96, BK>(p); }

// Waves per workgroup: the (matrix, RW-row group) items spread evenly over the CUs, one workgroup per CU (the weight
// stream of each CU then ends at the same time), up to 8 waves; beyond 2048 items, several workgroups of 8 per CU.
template <int MT, int RW>
hipError_t launch_gemv_rw(const LinearParams & p, hipStream_t stream) {
    const int64_t items = (int64_t)((p.N + RW - 1) / RW) * p.count;
    const int nw = (int)std::min<int64_t>(kGemvMaxWaves, std::max<int64_t>(1, (items + 255) / 256));
    const dim3 grid((uint32_t)((items + nw - 1) / nw));
    const dim3 block((uint32_t)(nw * kWave));
    const size_t lds = (size_t)MT * p.K * sizeof(float);
    const int v = (lds <= kLinearGemvLds ? 4 : 0) | ((p.flags & kLinearOutF16) ? 2 : 0) | ((p.flags & kLinearNorm) ? 1 : 0);
    const size_t dyn = (v & 4) ? lds : 0;
    switch (v) {
        case 0: hipLaunchKernelGGL((gemv_kernel<MT, false, false, false, RW>), grid, block, dyn, stream, p); break;
        case 1: hipLaunchKernelGGL((gemv_kernel<MT, false, false, true, RW>), grid, block, dyn, stream, p); break;
        case 2: hipLaunchKernelGGL((gemv_kernel<MT, false, true, false, RW>), grid, block, dyn, stream, p); break;
        case 3: hipLaunchKernelGGL((gemv_kernel<MT, false, true, true, RW>), grid, block, dyn, stream, p); break;
        case 4: hipLaunchKernelGGL((gemv_kernel<MT, true, false, false, RW>), grid, block, dyn, stream, p); break;
        case 5: hipLaunchKernelGGL((gemv_kernel<MT, true, false, true, RW>), grid, block, dyn, stream, p); break;
        case 6: hipLaunchKernelGGL((gemv_kernel<MT, true, true, false, RW>), grid, block, dyn, stream, p); break;
        default: hipLaunchKernelGGL((gemv_kernel<MT, true, true, true, RW>), grid, block, dyn, stream, p); break;
    }
    return hipGetLastError();
}

// Rows per wave: 2 where the items still fit one workgroup per CU, i.e. twice the waves streaming the same bytes
// (A/B on one box, us per launch: Llama-3-8B attention output 8.77 -> 8.41, a 14336-column down projection
// 23.36 -> 22.69, Whisper attention output 3.73 -> 3.63, Qwen2.5-0.5B 3.33 -> 3.24, eight input rows 21.2 -> 19.7;
// unchanged at two rows and the q|k|v width, which takes 4 rows per wave to fit). Four input rows keep 4 rows per
// wave: with 2 they ran 16.5 -> 20.2 us.
template <int MT>
hipError_t launch_gemv_t(const LinearParams & p, hipStream_t stream) {
    const int64_t cap = (int64_t)256 * kGemvMaxWaves;  // one workgroup of at most 8 waves per CU
    if (MT != 4 && (int64_t)((p.N + 1) / 2) * p.count <= cap) return launch_gemv_rw<MT, 2>(p, stream);
    return launch_gemv_rw<MT, kGemvRows>(p, stream);
}

}  // namespace

hipError_t launch_stage(const LinearParams & p, hipStream_t stream) {
    if (p.flags & kLinearNorm) hipLaunchKernelGGL(stage_kernel<true>, dim3((uint32_t)p.M), dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL(stage_kernel<false>, dim3((uint32_t)p.M), dim3(kThreads), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_linear(const LinearParams & p, hipStream_t stream) {
    if (p.M <= kLinearGemvMaxRows) {
        if (p.M <= 1) return launch_gemv_t<1>(p, stream);
        if (p.M <= 2) return launch_gemv_t<2>(p, stream);
        if (p.M <= 4) return launch_gemv_t<4>(p, stream);
        return launch_gemv_t<8>(p, stream);
    }
    if (hipError_t e = launch_stage(p, stream); e != hipSuccess) return e;
    return launch_gemm(p, stream);
}

hipError_t launch_gemm(const LinearParams & p, hipStream_t stream) {
    // 256-row tiles 256, 192 or 128 columns wide (one workgroup per CU), whichever costs the fewest rounds on the CUs
    // times its width, the narrower tiles weighted for their lower efficiency (measured: the Llama-3-8B q|k|v chunk,
    // 2048 x 6144, as 256 tiles of 256 x 192 rather than 192 of 256 x 256); when even the 256 x 128 tiles leave a
    // quarter of the CUs idle, 128 x 128 tiles (three workgroups per CU)
    const int mtl = (p.M + kBM - 1) / kBM;
    const int64_t t256 = (int64_t)p.count * ((p.N + 255) / 256) * mtl, t192 = (int64_t)p.count * ((p.N + 191) / 192) * mtl,
                  t128 = (int64_t)p.count * ((p.N + 127) / 128) * mtl;
    const bool f16 = p.flags & kLinearOutF16;
    if (4 * t128 >= 3 * kGemmCUs || 4 * t256 >= 3 * kGemmCUs) {
        auto rounds = [](int64_t t) { return (double)((t + kGemmCUs - 1) / kGemmCUs); };
        const double c256 = rounds(t256) * 256 * (4 * t256 >= 3 * kGemmCUs ? 1.0 : 1.35);  // a partial round idles CUs
        const double c192 = rounds(t192) * 192 * 1.05 * (4 * t192 >= 3 * kGemmCUs ? 1.0 : 1.35);
        const double c128 = rounds(t128) * 128 * 1.15;
        const bool k64 = p.K % 64 == 0;
        const int sel = 2 * (k64 ? 1 : 0) + (f16 ? 1 : 0);
        void (*const big[4])(LinearParams) = {gemm_big_kernel<false, 32>, gemm_big_kernel<true, 32>,
                                              gemm_big_kernel<false, 64>, gemm_big_kernel<true, 64>};
        void (*const w192[4])(LinearParams) = {gemm_w192_kernel<false, 32>, gemm_w192_kernel<true, 32>,
                                               gemm_w192_kernel<false, 64>, gemm_w192_kernel<true, 64>};
        void (*const mid[4])(LinearParams) = {gemm_mid_kernel<false, 32>, gemm_mid_kernel<true, 32>,
                                              gemm_mid_kernel<false, 64>, gemm_mid_kernel<true, 64>};
        if (c256 <= c192 && c256 <= c128)
            hipLaunchKernelGGL(big[sel], dim3((uint32_t)t256), dim3(kBigThreads), 0, stream, p);
        else if (c192 <= c128)
            hipLaunchKernelGGL(w192[sel], dim3((uint32_t)t192), dim3(kBigThreads), 0, stream, p);
        else
            hipLaunchKernelGGL(mid[sel], dim3((uint32_t)t128), dim3(kBigThreads), 0, stream, p);
        return hipGetLastError();
    }
    const int tiles = p.count * ((p.N + kTN - 1) / kTN) * ((p.M + kTM - 1) / kTM);
    const dim3 grid((uint32_t)tiles);
    if (p.flags & kLinearOutF16) hipLaunchKernelGGL(gemm_kernel<true>, grid, dim3(kThreads), 0, stream, p);
    else hipLaunchKernelGGL(gemm_kernel<false>, grid, dim3(kThreads), 0, stream, p);
    return hipGetLastError();
}

}  // namespace mx
