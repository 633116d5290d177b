// Prefill (prompt chunk) flash attention, causal GQA, f16 Q/K/V, f32 statistics and accumulation.
//
// Reference behaviour (dooms.cpp 0.6.1): `attention_prefill<HD>` (src/backend/metal/llama_kernels.h:632-769) as dispatched by
// MetalLlamaDecoder::Impl::attention (src/backend/metal/metal_llama_decoder.mm:284-296): query row t of a chunk of M rows
// sits at position p0 + t and sees keys 0 .. p0 + t of the cache; S = Q K^T (half operands, f32 accumulation), running max
// m and sum l with the rescale factor exp(m_old - m_new), P rounded to half, O += P V, and O / l at the end.
//
// MI355X design:
//   * One workgroup = 4 waves = 128 query rows of one query head; each wave owns 32 rows. Key/value blocks of 64 rows
//     stream through LDS (K row-major, V transposed), shared by the 4 waves; the next block is loaded from HBM/L2 into
//     registers while the current one is multiplied.
//   * Transposed scores: S^T (keys x queries) = K Q^T on v_mfma_f32_32x32x16_f16. In the MFMA result each lane holds 16
//     keys of ONE query (and the lane 32 away the other 16), so the row max and row sum need a single cross-lane step,
//     and the probabilities are already in the register layout of the B operand of O^T += V^T P^T: P never goes through
//     LDS. Q^T (the B operand of the first product) is loaded once into registers.
//   * The softmax runs in base 2 (scale * log2 e folded into one multiply), masking only in blocks that cross the
//     causal diagonal or the end of the cache; blocks past a wave's last row are skipped.
//   * Workgroups are dealt out so that the heaviest query tiles start first and the heads of one GQA group run next to
//     each other on the same XCD (shared K/V in that XCD's L2).
#include "mx_common.hpp"
#include "mx_kernels.hpp"

namespace mx {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kBK = 64;              // keys per block
constexpr int kVtPitch = kBK + 4;    // halves per row of V^T in LDS (conflict-free 8-byte reads and 2-byte writes)

template <int HD>
struct PrefillSmem {
    static constexpr int kKPitch = HD + 8;  // halves per row of K in LDS
    half_t k[kBK * kKPitch];
    half_t vt[HD * kVtPitch];
};

template <int HD>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillParams p) {
    constexpr int KS = HD / 16;          // MFMA steps along head_dim for S^T
    constexpr int DT = HD / 32;          // 32-wide output tiles along head_dim
    constexpr int C8 = HD / 8;           // 16-byte chunks per key row
    constexpr int NB = (kBK / 16) * (C8 / 4);  // (16 keys x 4 chunks) blocks per tile
    constexpr int NI = NB / kWaves;      // loads per thread per tile, for each of K and V
    constexpr int KP = PrefillSmem<HD>::kKPitch;
    __shared__ PrefillSmem<HD> sm;

    // ---- work item: heavy query tiles first, GQA groups adjacent, contiguous ranges per XCD ----
    const uint32_t n_work = (uint32_t)p.n_qtiles * p.n_head;
    const uint32_t w = xcd_remap(blockIdx.x, n_work);
    const int G = p.group;
    const int gi = w % G;
    const int kvh = (w / G) % p.n_head_kv;
    const int qt_order = w / (G * p.n_head_kv);
    const int qt = p.causal ? p.n_qtiles - 1 - qt_order : qt_order;
    const int h = kvh * G + gi;
    const int q0 = qt * kPrefillRows;

    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int l32 = lane % 32, hgrp = lane / 32;
    const int qrow = q0 + 32 * wave + l32;      // this lane's query row (chunk index)
    const int qpos = p.p0 + qrow;               // its cache position
    const int wave_last = p.p0 + q0 + 32 * wave + 31;  // the wave's last query position

    // keys this workgroup must visit
    const int last_row = min(q0 + kPrefillRows, p.n_q) - 1;
    const int kend = p.causal ? min(p.n_kv, p.p0 + last_row + 1) : p.n_kv;

    // Q^T operand: lane holds Q[qrow][16 ks + 8 hgrp .. + 8]
    half8_t qb[KS];
    {
        const half_t * qp = p.q + (int64_t)qrow * p.q_stride + (int64_t)h * HD + 8 * hgrp;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            u32x4 v = {0u, 0u, 0u, 0u};
            if (qrow < p.n_q) v = load16(qp + 16 * ks);
            qb[ks] = as_half8(v);
        }
    }

    float16_t o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int v = 0; v < 16; v++) o[dt][v] = 0.f;
    float m_run = kNegInf, l_run = 0.f;

    const half_t * kg = p.k + (int64_t)kvh * HD;
    const half_t * vg = p.v + (int64_t)kvh * HD;
    // tile-load mapping: block b = i * 4 + wave covers keys 16 (b % 4) + lane % 16 and chunks 4 (b / 4) + lane / 16
    u32x4 kreg[NI], vreg[NI];
    auto load_tile = [&](int kb) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int b = i * kWaves + wave;
            const int key = min(kb + 16 * (b % (kBK / 16)) + lane % 16, p.n_kv - 1);
            const int c8 = 4 * (b / (kBK / 16)) + lane / 16;
            const int64_t off = (int64_t)key * p.kv_stride + 8 * c8;
            kreg[i] = load16(kg + off);
            vreg[i] = load16(vg + off);
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int b = i * kWaves + wave;
            const int key = 16 * (b % (kBK / 16)) + lane % 16;
            const int c8 = 4 * (b / (kBK / 16)) + lane / 16;
            *reinterpret_cast<u32x4 *>(&sm.k[key * KP + 8 * c8]) = kreg[i];
            const half8_t vv = as_half8(vreg[i]);
#pragma unroll
            for (int e = 0; e < 8; e++) sm.vt[(8 * c8 + e) * kVtPitch + key] = vv[e];
        }
    };

    if (kend > 0) load_tile(0);
    for (int kb = 0; kb < kend; kb += kBK) {
        __syncthreads();  // the previous block's products are done with LDS
        store_tile();
        __syncthreads();
        if (kb + kBK < kend) load_tile(kb + kBK);
        if (p.causal && kb > wave_last) continue;  // every key of the block is past this wave's rows

        // S^T = K Q^T: 2 tiles of 32 keys
        float16_t sc[2];
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            float16_t acc;
#pragma unroll
            for (int v = 0; v < 16; v++) acc[v] = 0.f;
            const half_t * kr = &sm.k[(32 * mt + l32) * KP + 8 * hgrp];
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const half8_t a = as_half8(*reinterpret_cast<const u32x4 *>(kr + 16 * ks));
                acc = mfma32x32x16(a, qb[ks], acc);
            }
            sc[mt] = acc;
        }
        // scale, mask, block max
        const bool need_mask = (p.causal && kb + kBK - 1 > p.p0 + q0 + 32 * wave) || kb + kBK > p.n_kv;
        float bmax = kNegInf;
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                float x = sc[mt][v] * p.scale_log2;
                if (need_mask) {
                    const int key = kb + 32 * mt + 8 * (v / 4) + 4 * hgrp + (v % 4);
                    if (key >= p.n_kv || (p.causal && key > qpos)) x = kNegInf;
                }
                sc[mt][v] = x;
                bmax = fmaxf(bmax, x);
            }
        bmax = fmaxf(bmax, shfl_xor(bmax, 32));
        const float m_new = fmaxf(m_run, bmax);
        const bool none = m_new == kNegInf;
        const float corr = none ? 1.f : exp2_fast(m_run - m_new);
        m_run = m_new;
        float bsum = 0.f;
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const float e = none ? 0.f : exp2_fast(sc[mt][v] - m_new);
                sc[mt][v] = e;
                bsum += e;
            }
        l_run = l_run * corr + bsum;
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int v = 0; v < 16; v++) o[dt][v] *= corr;

        // O^T += V^T P^T: 4 steps of 16 keys; step u takes values 8 (u % 2) .. + 8 of score tile u / 2, which are keys
        // 16 u + 8 (e / 4) + 4 hgrp + e % 4 for e = 0..7 -- the same keys the V^T operand reads below.
#pragma unroll
        for (int u = 0; u < 4; u++) {
            half8_t pb;
#pragma unroll
            for (int e = 0; e < 8; e++) pb[e] = (half_t)sc[u / 2][8 * (u % 2) + e];
#pragma unroll
            for (int dt = 0; dt < DT; dt++) {
                const half_t * vr = &sm.vt[(32 * dt + l32) * kVtPitch + 16 * u + 4 * hgrp];
                const u32x2 lo = *reinterpret_cast<const u32x2 *>(vr);
                const u32x2 hi = *reinterpret_cast<const u32x2 *>(vr + 8);
                const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
                o[dt] = mfma32x32x16(as_half8(a), pb, o[dt]);
            }
        }
    }

    // ---- normalize and store: lane holds O[qrow][32 dt + 8 (v / 4) + 4 hgrp + v % 4] ----
    l_run += shfl_xor(l_run, 32);
    if (qrow < p.n_q) {
        const float inv = 1.f / l_run;
        half_t * op = p.out + (int64_t)qrow * p.out_stride + (int64_t)h * HD + 4 * hgrp;
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int gq = 0; gq < 4; gq++) {
                half4_t r;
#pragma unroll
                for (int e = 0; e < 4; e++) r[e] = (half_t)(o[dt][4 * gq + e] * inv);
                *reinterpret_cast<half4_t *>(op + 32 * dt + 8 * gq) = r;
            }
        if (p.lse && hgrp == 0) p.lse[(int64_t)qrow * p.n_head + h] = (m_run + log2_fast(l_run)) * kLn2;
    }
}

}  // namespace

hipError_t launch_prefill(const PrefillParams & p, int head_dim, hipStream_t stream) {
    const dim3 grid((uint32_t)p.n_qtiles * p.n_head);
    if (head_dim == 64)
        hipLaunchKernelGGL(prefill_kernel<64>, grid, dim3(kThreads), 0, stream, p);
    else
        hipLaunchKernelGGL(prefill_kernel<128>, grid, dim3(kThreads), 0, stream, p);
    return hipGetLastError();
}

}  // namespace mx
