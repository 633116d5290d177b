// Attention for head dims below 64 (powers of two 4 .. 32): the reference's per-query kernel shape, for the small test
// models of its decoder (the default tiny llama of tests/unit/test_metal_llama_decoder.cpp:56-57 has head_dim 16).
//
// Reference behaviour (dooms.cpp 0.6.1): `attention` (src/backend/metal/llama_kernels.h:552-630), which runs every head
// dim the llama decoder accepts (powers of two in [4, 256], metal_llama_decoder.mm:432-435): per (query row, head) the
// scores s_j = scale * q.k_j over the visible keys, softmax with the running maximum, out = sum_j p_j v_j / sum_j p_j,
// kv head h / (n_head / n_head_kv). Scores, softmax and accumulation are f32 here, on the f16 cache values and the query
// as given (f32 rows stay f32: these dims need no matrix cores).
//
// MI355X design: the MFMA kernels tile head_dim in 32- and 64-wide steps, so head dims below 64 run here instead. One
// workgroup of 4 waves per (sequence, query row, query head); each wave takes every fourth step of keys, and within a
// wave each key is read by HD / 4 lanes, 4 dims (8 bytes) each, so 64 / (HD / 4) keys go per step (16 at head dim 16).
// The step's scores are reduced across those lanes with xor shuffles; each key slot keeps its own running (m, l, acc),
// and the slots, then the waves (through LDS), are merged with the same log-sum-exp formula at the end. The next step's
// keys and values are loaded before the current step's arithmetic. Work is HBM/latency-bound and tiny at these dims.
#include "mx_common.hpp"
#include "mx_kernels.hpp"

namespace mx {

namespace {

constexpr int kSmallWaves = 4;

// (m, l, acc) of one partial softmax; merged with another by the log-sum-exp rule (m in base-2 units).
template <int D>
__device__ __forceinline__ void merge_into(float & m, float & l, float (&acc)[D], float m2, float l2, const float (&acc2)[D]) {
    if (!(l2 > 0.f)) return;
    if (!(l > 0.f)) {
        m = m2;
        l = l2;
#pragma unroll
        for (int d = 0; d < D; d++) acc[d] = acc2[d];
        return;
    }
    const float mn = fmaxf(m, m2), c1 = exp2_fast(m - mn), c2 = exp2_fast(m2 - mn);
    m = mn;
    l = l * c1 + l2 * c2;
#pragma unroll
    for (int d = 0; d < D; d++) acc[d] = acc[d] * c1 + acc2[d] * c2;
}

template <int HD>
__global__ __launch_bounds__(kSmallWaves * kWave) void small_attn_kernel(SmallAttnParams p) {
    constexpr int DPL = 4;           // head dims per lane
    constexpr int LPK = HD / DPL;    // lanes per key
    constexpr int KPW = kWave / LPK; // keys per wave step
    static_assert(HD % DPL == 0 && LPK <= kWave, "head dim");
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int slot = lane / LPK, part = lane % LPK, d0 = DPL * part;

    const int bl = blockIdx.y;
    const int t = blockIdx.x / p.n_head, h = blockIdx.x % p.n_head;
    const SmallSeq sq = p.seq[bl];
    const int g = h / p.group;
    const int pos = sq.p0 + t;                          // cache position of the query row
    const int nvis = p.causal ? min(pos + 1, sq.len) : sq.len;  // visible keys 0 .. nvis - 1
    const int64_t qrow = (int64_t)sq.row0 + t;

    // this lane's 4 query dims, f32 (rotated for `pos` when asked: pair partners are read from the row directly)
    float q[DPL];
    auto qval = [&](int d) -> float {
        const int64_t off = qrow * p.q_stride + (int64_t)h * HD + d;
        return p.q_f32 ? static_cast<const float *>(p.q)[off] : (float)static_cast<const half_t *>(p.q)[off];
    };
#pragma unroll
    for (int e = 0; e < DPL; e++) {
        const int d = d0 + e;
        float a = qval(d);
        if (p.rope_mode != 2) {
            // pair i = (2i, 2i + 1) adjacent or (i, i + HD / 2) neox; this element is its pair's first or second
            const bool neox = p.rope_mode == 1;
            const int i = neox ? d % (HD / 2) : d / 2;
            const bool first = neox ? d < HD / 2 : (d % 2) == 0;
            const float b = qval(neox ? (first ? d + HD / 2 : d - HD / 2) : (first ? d + 1 : d - 1));
            float sn, cs;
            sincos_rope((float)pos * p.rope_freq[i], sn, cs);
            a = first ? a * cs - b * sn : b * sn + a * cs;
        }
        q[e] = a * p.scale_log2;
    }

    const half_t * kb = sq.k + (int64_t)g * HD + d0;
    const half_t * vb = sq.v + (int64_t)g * HD + d0;
    auto ld4 = [&](const half_t * base, int j) -> u32x2 {
        return *reinterpret_cast<const u32x2 *>(base + (int64_t)j * p.kv_stride);
    };
    float m = kNegInf, l = 0.f, acc[DPL] = {};
    constexpr int kStep = KPW * kSmallWaves;  // keys per workgroup step
    int j = wave * KPW + slot;
    u32x2 kc = ld4(kb, min(j, max(nvis - 1, 0))), vc = ld4(vb, min(j, max(nvis - 1, 0)));
    for (; j - slot < nvis; j += kStep) {
        const int jn = j + kStep;
        const u32x2 kn = ld4(kb, min(jn, max(nvis - 1, 0))), vn = ld4(vb, min(jn, max(nvis - 1, 0)));
        const half4_t kh = __builtin_bit_cast(half4_t, kc), vh = __builtin_bit_cast(half4_t, vc);
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; e++) s = __builtin_fmaf(q[e], (float)kh[e], s);
#pragma unroll
        for (int mask = LPK / 2; mask >= 1; mask /= 2) s += shfl_xor(s, mask);
        if (j < nvis) {
            const float mn = fmaxf(m, s), c = exp2_fast(m - mn), pj = exp2_fast(s - mn);
            m = mn;
            l = l * c + pj;
#pragma unroll
            for (int e = 0; e < DPL; e++) acc[e] = acc[e] * c + pj * (float)vh[e];
        }
        kc = kn;
        vc = vn;
    }
    // the wave's key slots (lanes LPK apart hold the same dims), then the waves through LDS
#pragma unroll
    for (int mask = LPK; mask < kWave; mask *= 2) {
        float acc2[DPL];
#pragma unroll
        for (int e = 0; e < DPL; e++) acc2[e] = shfl_xor(acc[e], mask);
        const float m2 = shfl_xor(m, mask), l2 = shfl_xor(l, mask);
        merge_into<DPL>(m, l, acc, m2, l2, acc2);
    }
    __shared__ float s_part[kSmallWaves][HD + 2];
    if (slot == 0) {
#pragma unroll
        for (int e = 0; e < DPL; e++) s_part[wave][d0 + e] = acc[e];
        if (part == 0) {
            s_part[wave][HD] = m;
            s_part[wave][HD + 1] = l;
        }
    }
    __syncthreads();
    if (wave != 0 || slot != 0) return;
#pragma unroll
    for (int w = 1; w < kSmallWaves; w++) {
        float acc2[DPL];
#pragma unroll
        for (int e = 0; e < DPL; e++) acc2[e] = s_part[w][d0 + e];
        merge_into<DPL>(m, l, acc, s_part[w][HD], s_part[w][HD + 1], acc2);
    }
    const float inv = 1.f / l;
    const int64_t o = qrow * p.out_stride + (int64_t)h * HD + d0;
#pragma unroll
    for (int e = 0; e < DPL; e++) {
        if (p.out_f32) static_cast<float *>(p.out)[o + e] = acc[e] * inv;
        else static_cast<half_t *>(p.out)[o + e] = (half_t)(acc[e] * inv);
    }
    if (part == 0 && p.lse) p.lse[qrow * p.n_head + h] = (m + log2_fast(l)) * kLn2;
}

}  // namespace

hipError_t launch_small_attn(const SmallAttnParams & p, int head_dim, int n_seq, hipStream_t stream) {
    const dim3 grid((uint32_t)(p.n_q * p.n_head), (uint32_t)n_seq), block(kSmallWaves * kWave);
    switch (head_dim) {
        case 4: hipLaunchKernelGGL(small_attn_kernel<4>, grid, block, 0, stream, p); break;
        case 8: hipLaunchKernelGGL(small_attn_kernel<8>, grid, block, 0, stream, p); break;
        case 16: hipLaunchKernelGGL(small_attn_kernel<16>, grid, block, 0, stream, p); break;
        case 32: hipLaunchKernelGGL(small_attn_kernel<32>, grid, block, 0, stream, p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mx
