// Decode attention over per-sequence f16 KV caches: split-KV ("flash-decoding") plus a log-sum-exp merge.
//
// Reference behaviour (dooms.cpp 0.6.1): the per-query kernel `attention` (src/backend/metal/llama_kernels.h:552-630) for
// short decodes and Whisper self-attention, `attention_split` (llama_kernels.h:856-910) for decodes of >= 512 positions
// and Whisper cross-attention, and `attention_combine` (llama_kernels.h:912-929) for the merge. The math is the same:
// scores s_j = scale * q.k_j over the visible keys, softmax with the running max, out = sum_j p_j v_j / sum_j p_j, and the
// merge out = sum_s e^{m_s - M} acc_s / sum_s e^{m_s - M} l_s over non-empty splits (l_s > 0).
//
// MI355X design (not a translation of the Metal kernels):
//   * One workgroup per (sequence, key/value head, split of the keys, tile of query rows). All query rows that read the
//     same key/value head (the G = n_head / n_head_kv heads of a GQA group, times the n_q query rows of the sequence) are
//     processed together, so each K/V byte is read from HBM once, not G times as in the reference's per-head kernels.
//   * Scores on the matrix cores: S^T (16 keys x 16 rows) = K (16 keys x head_dim) . Q^T, v_mfma_f32_16x16x32_f16. K goes
//     from HBM straight into the MFMA operand registers with 16-byte loads (4 lanes cover 64 contiguous bytes of a row).
//   * Probabilities times values on the vector ALUs: each lane owns 8 contiguous head dimensions of a value row (one
//     16-byte load) and accumulates rows x 8 f32 sums with mixed f16/f32 FMAs; the probabilities come from LDS as
//     broadcast reads. At decode's 4 FLOP per byte this keeps the ALUs well under the HBM rate.
//   * The 4 waves of a workgroup take interleaved 32-key blocks of the split and are merged through LDS, so one partial
//     (m, l, acc[head_dim]) per split and row reaches HBM; splits are then merged by a second, small kernel.
#include "mx_common.hpp"
#include "mx_kernels.hpp"

namespace mx {

namespace {

constexpr int kDecodeWaves = 4;
constexpr int kDecodeThreads = kDecodeWaves * kWave;
constexpr int kBlockKeys = 32;  // keys per wave iteration

// HD: head_dim. RT: query rows per tile (4, 8 or 16; the MFMA tile always has 16 rows, the extra ones are zero).
template <int HD, int RT>
__global__ __launch_bounds__(kDecodeThreads) void decode_split_kernel(DecodeParams p) {
    constexpr int KS = HD / 32;           // MFMA steps along head_dim
    constexpr int LPR = HD / 8;           // lanes per value row (8 halves per lane)
    constexpr int KPL = kWave / LPR;      // value rows per wave load
    constexpr int NLV = kBlockKeys / KPL; // value loads per lane per block
    constexpr int PS = RT;                // floats per key in the probability buffer

    __shared__ float s_p[kDecodeWaves][kBlockKeys * PS];
    __shared__ float s_corr[kDecodeWaves][RT];
    __shared__ float s_m[kDecodeWaves][RT], s_l[kDecodeWaves][RT];
    __shared__ float s_o[kDecodeWaves][RT * HD];

    const int s = blockIdx.x;
    int y = blockIdx.y;
    const int rt = y % p.n_rowtiles;
    y /= p.n_rowtiles;
    const int g = y % p.n_head_kv;
    const int bl = y / p.n_head_kv;
    const DecodeSeq sq = p.seq[bl];
    if (s >= sq.n_split) return;  // uniform over the workgroup, before any barrier

    const int L = sq.len;
    const int j0 = s * p.chunk;
    const int j1 = min(j0 + p.chunk, L);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int G = p.group;
    const int64_t seq_row0 = (int64_t)(p.seq0 + bl) * p.n_q;  // first query row of the sequence

    // ---- this lane's score row (lane % 16) and its query operand ----
    const int srow = lane % 16, sgrp = lane / 16;
    const int rr = rt * RT + srow;  // row index inside the (sequence, kv head) problem: rr = t * G + gi
    const bool srow_ok = srow < RT && rr < p.rows;
    const int st = rr / G, sh = g * G + rr % G;
    const int lim = p.causal ? L - p.n_q + st : L - 1;  // last visible key of the row
    half8_t qb[KS];
    {
        const half_t * qrow = p.q + (seq_row0 + st) * p.q_stride + (int64_t)sh * HD;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            u32x4 v = {0u, 0u, 0u, 0u};
            if (srow_ok) v = load16(qrow + 32 * ks + 8 * sgrp);
            qb[ks] = as_half8(v);
        }
    }

    const half_t * kbase = sq.k + (int64_t)g * HD;
    const half_t * vbase = sq.v + (int64_t)g * HD;
    const int vslot = lane / LPR, vcol = 8 * (lane % LPR);

    float m_run = kNegInf, l_run = 0.f;  // per score lane (row srow); l is this lane's partial sum
    float o[RT][8];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int e = 0; e < 8; e++) o[r][e] = 0.f;

    for (int jb = j0 + kBlockKeys * wave; jb < j1; jb += kBlockKeys * kDecodeWaves) {
        // issue every load of the block first: keys into MFMA operands, values into registers
        u32x4 kr[2][KS], vr[NLV];
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            const int key = min(jb + 16 * mt + lane % 16, L - 1);
            const half_t * kp = kbase + (int64_t)key * p.kv_stride + 8 * sgrp;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) kr[mt][ks] = load16(kp + 32 * ks);
        }
#pragma unroll
        for (int i = 0; i < NLV; i++) {
            const int key = min(jb + KPL * i + vslot, L - 1);
            vr[i] = load16(vbase + (int64_t)key * p.kv_stride + vcol);
        }
        // S^T = K Q^T, 2 tiles of 16 keys
        float sc[2][4];
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
            float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ks++) acc = mfma16x16x32(as_half8(kr[mt][ks]), qb[ks], acc);
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int key = jb + 16 * mt + 4 * sgrp + v;
                sc[mt][v] = (key < j1 && key <= lim) ? acc[v] * p.scale_log2 : kNegInf;
            }
        }
        float bmax = kNegInf;
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int v = 0; v < 4; v++) bmax = fmaxf(bmax, sc[mt][v]);
        bmax = fmaxf(bmax, shfl_xor(bmax, 16));
        bmax = fmaxf(bmax, shfl_xor(bmax, 32));
        const float m_new = fmaxf(m_run, bmax);
        const bool none = m_new == kNegInf;  // no visible key yet for this row
        const float corr = none ? 1.f : exp2_fast(m_run - m_new);
        float bsum = 0.f;
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const float pv = none ? 0.f : exp2_fast(sc[mt][v] - m_new);
                sc[mt][v] = pv;
                bsum += pv;
            }
        l_run = l_run * corr + bsum;
        m_run = m_new;
        if (srow < RT) {
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int v = 0; v < 4; v++) s_p[wave][(16 * mt + 4 * sgrp + v) * PS + srow] = sc[mt][v];
            if (sgrp == 0) s_corr[wave][srow] = corr;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // O = diag(corr) O + P V over this lane's value rows
        float cr[RT];
#pragma unroll
        for (int r = 0; r < RT; r++) cr[r] = s_corr[wave][r];
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int e = 0; e < 8; e++) o[r][e] *= cr[r];
#pragma unroll
        for (int i = 0; i < NLV; i++) {
            const half8_t vv = as_half8(vr[i]);
            const float * pk = &s_p[wave][(KPL * i + vslot) * PS];
            float pr[RT];
#pragma unroll
            for (int r = 0; r < RT; r++) pr[r] = pk[r];
#pragma unroll
            for (int r = 0; r < RT; r++)
#pragma unroll
                for (int e = 0; e < 8; e++) o[r][e] = __builtin_fmaf(pr[r], (float)vv[e], o[r][e]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // ---- wave totals: l over the 4 score-lane groups, O over the value slots ----
    l_run += shfl_xor(l_run, 16);
    l_run += shfl_xor(l_run, 32);
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float v = o[r][e];
#pragma unroll
            for (int msk = LPR; msk < kWave; msk *= 2) v += shfl_xor(v, msk);
            o[r][e] = v;
        }
    if (lane < RT) {
        s_m[wave][lane] = m_run;
        s_l[wave][lane] = l_run;
    }
    if (lane < LPR) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int e = 0; e < 8; e++) s_o[wave][r * HD + vcol + e] = o[r][e];
    }
    __syncthreads();

    // ---- merge the 4 waves; write the output (one split) or this split's partial ----
    const bool single = sq.n_split == 1;
    for (int idx = threadIdx.x; idx < RT * HD; idx += kDecodeThreads) {
        const int r = idx / HD, d = idx % HD;
        const int row = rt * RT + r;
        if (row >= p.rows) continue;
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; w++)
            if (s_l[w][r] > 0.f) M = fmaxf(M, s_m[w][r]);
        float tot = 0.f, acc = 0.f;
#pragma unroll
        for (int w = 0; w < kDecodeWaves; w++) {
            if (!(s_l[w][r] > 0.f)) continue;
            const float wt = exp2_fast(s_m[w][r] - M);
            tot += s_l[w][r] * wt;
            acc += s_o[w][r * HD + d] * wt;
        }
        const int t = row / G, h = g * G + row % G;
        if (single) {
            p.out[(seq_row0 + t) * p.out_stride + (int64_t)h * HD + d] = (half_t)(acc / tot);
            if (d == 0 && p.lse) p.lse[(seq_row0 + t) * p.n_head + h] = (M + log2_fast(tot)) * kLn2;
        } else {
            const int64_t pidx = ((((int64_t)bl * p.n_head_kv + g) * p.n_rowtiles + rt) * p.max_split + s) * RT + r;
            float * pe = p.part + pidx * (HD + 4);
            pe[d] = acc;
            if (d == 0) {
                pe[HD] = M;
                pe[HD + 1] = tot;
            }
        }
    }
}

// Merge of the split partials of one (sequence, query row, head): out = sum_s 2^{m_s - M} acc_s / sum_s 2^{m_s - M} l_s
// over the splits with l_s > 0 (the reference's attention_combine, llama_kernels.h:912-929, with base-2 statistics).
template <int HD, int RT>
__global__ __launch_bounds__(HD) void decode_merge_kernel(DecodeParams p) {
    const int bl = blockIdx.y;
    const DecodeSeq sq = p.seq[bl];
    if (sq.n_split == 1) return;  // written by the split kernel
    const int th = blockIdx.x;  // t * n_head + h
    const int t = th / p.n_head, h = th % p.n_head;
    const int G = p.group, g = h / G, row = t * G + h % G, rt = row / RT, r = row % RT;
    const int d = threadIdx.x;
    const int64_t base = (((int64_t)bl * p.n_head_kv + g) * p.n_rowtiles + rt) * p.max_split;
    float M = kNegInf;
    for (int s = 0; s < sq.n_split; s++) {
        const float * pe = p.part + ((base + s) * RT + r) * (HD + 4);
        if (pe[HD + 1] > 0.f) M = fmaxf(M, pe[HD]);
    }
    float tot = 0.f, acc = 0.f;
    for (int s = 0; s < sq.n_split; s++) {
        const float * pe = p.part + ((base + s) * RT + r) * (HD + 4);
        const float l = pe[HD + 1];
        if (!(l > 0.f)) continue;
        const float wt = exp2_fast(pe[HD] - M);
        tot += l * wt;
        acc += pe[d] * wt;
    }
    const int64_t qrow = (int64_t)(p.seq0 + bl) * p.n_q + t;
    p.out[qrow * p.out_stride + (int64_t)h * HD + d] = (half_t)(acc / tot);
    if (d == 0 && p.lse) p.lse[qrow * p.n_head + h] = (M + log2_fast(tot)) * kLn2;
}

template <int HD, int RT>
hipError_t launch_decode_t(const DecodeParams & p, int n_seq, hipStream_t stream) {
    const dim3 grid(p.max_split, n_seq * p.n_head_kv * p.n_rowtiles);
    hipLaunchKernelGGL((decode_split_kernel<HD, RT>), grid, dim3(kDecodeThreads), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.max_split == 1) return e;
    hipLaunchKernelGGL((decode_merge_kernel<HD, RT>), dim3(p.n_q * p.n_head, n_seq), dim3(HD), 0, stream, p);
    return hipGetLastError();
}

}  // namespace

int decode_rows_per_tile(int rows) { return rows <= 4 ? 4 : rows <= 8 ? 8 : 16; }

hipError_t launch_decode(const DecodeParams & p, int n_seq, int head_dim, int rt, hipStream_t stream) {
    if (head_dim == 64) {
        if (rt == 4) return launch_decode_t<64, 4>(p, n_seq, stream);
        if (rt == 8) return launch_decode_t<64, 8>(p, n_seq, stream);
        return launch_decode_t<64, 16>(p, n_seq, stream);
    }
    if (rt == 4) return launch_decode_t<128, 4>(p, n_seq, stream);
    if (rt == 8) return launch_decode_t<128, 8>(p, n_seq, stream);
    return launch_decode_t<128, 16>(p, n_seq, stream);
}

}  // namespace mx
