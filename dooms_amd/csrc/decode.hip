// Decode attention over per-sequence f16 KV caches: split-KV ("flash-decoding") with the log-sum-exp merge in the same
// kernel.
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
//   * Probabilities times values on the matrix cores too: O^T (head dims x rows) += V^T P^T. Each wave stages its 32-key
//     V block row-major in LDS and reads the V^T operand back through ds_read_b64_tr_b16 (whose 16-lane transpose
//     hands each lane 4 consecutive keys of one head dimension); P^T is the score MFMA's result layout, rounded to
//     f16, so the probabilities never leave registers and the vector ALUs only run the softmax.
//   * Each wave walks 32-key blocks of its workgroup's split with the next block's K/V already in flight (register
//     double buffer); the NW (4 or 8) waves are merged through LDS.
//   * Splits are merged inside the same launch: each workgroup publishes its partial (acc[head_dim], m, l per row) with
//     device-scope atomic stores, waits for their completion, and bumps a per-tile counter; the workgroup that brings the
//     counter to the split count merges and resets it to 0. Publishing with atomic stores (coherent at device scope by
//     construction) instead of plain stores plus a release fence avoids the fence's full L2 write-back, which on a
//     multi-XCD part serializes the workgroups; and merging in-kernel saves a second launch (~2.5 us on MI355X, more
//     than half of the ideal time of an 8192-token Llama-3-8B decode step).
#include "mx_common.hpp"
#include "mx_kernels.hpp"

// Phase trace (a separate build, libmx_attn_trace.so, compiled with MX_ATTN_TRACE): each decode workgroup stamps the
// shader's real-time clock (100 MHz) at its start, at the end of each wave's key/value walk, after the waves' merge,
// after its partial is published, after the split counter returns and (the merging workgroup) after the merge, into
// g_decode_trace[workgroup][16]; mx_attn_trace_read copies it out. The product build compiles the stamps away.
#ifdef MX_ATTN_TRACE
__device__ unsigned long long g_decode_trace[8192 * 16];
#define MX_TRACE(slot) \
    (g_decode_trace[(size_t)(blockIdx.x + blockIdx.y * gridDim.x) % 8192 * 16 + (slot)] = __builtin_amdgcn_s_memrealtime())
#define MX_TRACE_CLEAR(slot) (g_decode_trace[(size_t)(blockIdx.x + blockIdx.y * gridDim.x) % 8192 * 16 + (slot)] = 0)
#else
#define MX_TRACE(slot) ((void)0)
#define MX_TRACE_CLEAR(slot) ((void)0)
#endif

namespace mx {

namespace {

constexpr int kBlockKeys = 32;  // keys per wave iteration

typedef short short4_t __attribute__((ext_vector_type(4)));

constexpr int kMergeChunk = 16;  // splits whose partials one thread has in flight at once during the merge
constexpr int kMaxSplitsPerTile = 64;  // the host's split plan never makes more

// Relaxed device-scope atomic accesses of float pairs: coherent across the XCDs without cache maintenance.
__device__ __forceinline__ void publish2(float * p, float a, float b) {
    const uint64_t v = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
    __hip_atomic_store(reinterpret_cast<uint64_t *>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void collect2(const float * p, float & a, float & b) {
    const uint64_t v = __hip_atomic_load(reinterpret_cast<uint64_t *>(const_cast<float *>(p)), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    a = __uint_as_float((uint32_t)v);
    b = __uint_as_float((uint32_t)(v >> 32));
}

// 16-byte device-scope (sc1) buffer loads: coherent across the XCDs, a quarter of the instructions of 4-byte atomic
// loads. The resource is built from a wave-uniform base (a per-lane base would make the compiler loop over the distinct
// descriptors of the wave); lanes differ in their byte offsets.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dev_rsrc(const void * base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, 0x7fffffff, 0x00020000);
}
constexpr int kCpolSc1 = 16;  // the cache-policy bit that makes a buffer access device-scope on gfx950
__device__ __forceinline__ u32x4 load16_dev(__amdgpu_buffer_rsrc_t r, int byte_off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCpolSc1));
}
__device__ __forceinline__ void store16_dev(__amdgpu_buffer_rsrc_t r, int byte_off, float4_t v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, byte_off, 0, kCpolSc1);
}

// XCD-local publishing (the XCD-mapped grid, where every split of a tile runs on one XCD): plain stores, complete once
// they reach that XCD's L2, where the merging workgroup's device-scope loads find them (a store-load round trip on one
// XCD: 0.96 us, against 1.50 us with device-scope stores). Batch 1 at 8192 keys 11.07-11.35 -> 10.70-10.89 us per
// launch. Workgroups are dealt to the XCDs round-robin, so ids 8 apart share an XCD; the split counter checks it (below).
__device__ __forceinline__ void store16_xcd(__amdgpu_buffer_rsrc_t r, int byte_off, float4_t v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, byte_off, 0, 0);
}
__device__ __forceinline__ void publish2_xcd(float * p, float a, float b) {
    const uint64_t v = (uint64_t)__float_as_uint(a) | ((uint64_t)__float_as_uint(b) << 32);
    __hip_atomic_store(reinterpret_cast<uint64_t *>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// The XCD this wave runs on (HW_REG_XCC_ID, bits 0..3).
__device__ __forceinline__ uint32_t xcc_id() { return __builtin_amdgcn_s_getreg((3 << 11) | 20) & 7u; }
// XCD-local split counter: 64 bits, six per XCD (the host keeps the XCD-mapped grid to at most 32 splits), each split
// adding one to its XCD's field. The split that completes the count merges only if every field but its own is zero.
constexpr int kXccField = 6;

// K/V loads; NT: non-temporal (the cache lines are not kept), for launches whose keys and values stream from HBM once
template <bool NT>
__device__ __forceinline__ u32x4 load16_kv(const void * p) {
    if constexpr (NT) return __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4 *)(p));
    else return load16(p);
}

template <int HD>
struct KvBlock {
    static constexpr int KS = HD / 32;            // MFMA steps along head_dim
    static constexpr int LPR = HD / 8;            // lanes per value row (8 halves per lane)
    static constexpr int KPL = kWave / LPR;       // value rows per wave load
    static constexpr int NLV = kBlockKeys / KPL;  // value (and key) loads per lane per block
    // Keys and values are both loaded as whole row slices, LPR consecutive lanes per row: a load instruction that
    // reads 16 rows x 64 bytes (the MFMA operand layout) streams ~10 % slower, and the row slices whose address
    // bits 8..9 are 01 (two of Llama-3-8B's eight kv heads) ~17 % slower still; the keys reach the operand layout
    // through LDS.
    u32x4 k[NLV];
    u32x4 v[NLV];
};

// Two adjacent output elements: half, or f32 for the fused step (the reference's f32 attention output).
template <bool F32>
__device__ __forceinline__ void store_pair(const DecodeParams & p, int64_t off, float a, float b) {
    if constexpr (F32) {
        *reinterpret_cast<float2 *>(p.out32 + off) = make_float2(a, b);
    } else {
        p.out[off] = (half_t)a;
        p.out[off + 1] = (half_t)b;
    }
}

// The cross-split merge of a head-dim-128 tile: every (m, l) pair of the tile is loaded once (split = lane, one wave per row) and turned into per-split weights
// 2^(m - M) and the row's total by reductions inside the wave (a thread per row looping over the splits took ~0.6 us),
// while the accumulator columns come in 16-byte device-scope loads, each column's splits striped over SF threads and
// the stripes summed through LDS. Half the bytes of the per-pair merge through the merging CU, whose threads would
// each load their row's (m, l) for every split: Llama-3-8B at 8192 keys (32 splits) 13.85 -> 13.44 us per launch.
// It serves every head-dim-128 tile of more than one split, in the 4- and 8-wave kernels (Llama-3-8B batch 4 at 8192
// keys 33.6 -> 32.7 us, 1024 keys 7.07 -> 7.00 us). The head-dim-64 kernels keep the per-pair merge: there the path's
// registers cost a wave of occupancy (112 -> 136 VGPRs), +0.4 us on Qwen2.5-0.5B and the Whisper shapes; head dim 256
// has no registers to spare.
template <int HD, int RT, bool F32, int NW, size_t LDS_BYTES, int MCR>
__device__ __forceinline__ void merge_wide(const DecodeParams & p, const float * part_tile, int ns, int rt, int g, int G,
                                           int64_t seq_row0, char * lds) {
    constexpr int kThreads = NW * kWave;
    constexpr int SS = RT * (HD + 4);                       // floats between the partials of consecutive splits
    constexpr int NC = RT * HD / 4;                         // float4 columns of the tile
    constexpr int SF = kThreads >= NC ? kThreads / NC : 1;  // threads per column (stripes of the splits)
    constexpr int CPT = NC > kThreads ? NC / kThreads : 1;  // columns per thread
    // splits of each column loaded per round: MCR (the caller's choice, enough to cover the tile's splits in one
    // round where the registers allow) up to 16 / CPT. A round that covered 64 split slots for at most 32 splits
    // loaded each column of the last split up to 32 times over (clamped addresses), doubling the merging CU's bytes.
    constexpr int MC = (16 / CPT > 0 ? 16 / CPT : 1) < MCR ? (16 / CPT > 0 ? 16 / CPT : 1) : MCR;
    constexpr int NPAIR = kMaxSplitsPerTile * RT;           // weight slots: [split][row]
    constexpr int RPW = (RT + NW - 1) / NW;                 // rows per wave for the (m, l) reductions
    static_assert(kMaxSplitsPerTile <= kWave, "one lane per split");
    constexpr int kStatBytes = (NPAIR * 4 + RT * 8 + 15) / 16 * 16;
    float * s_w = reinterpret_cast<float *>(lds);               // [split][row] 2^(m - M)
    float2 * s_row = reinterpret_cast<float2 *>(s_w + NPAIR);  // [row] (M, total)
    float4_t * s_acc = reinterpret_cast<float4_t *>(lds + kStatBytes);  // [stripe - 1][column]
    static_assert(kStatBytes + (SF - 1) * NC * 16 <= (int64_t)LDS_BYTES, "merge scratch fits the V staging areas");
    const __amdgpu_buffer_rsrc_t rsrc = dev_rsrc(part_tile);
    const int stripe = SF > 1 ? (int)threadIdx.x / NC : 0;  // wave-uniform
    auto column = [&](int j) { return SF > 1 ? (int)threadIdx.x % NC : (int)threadIdx.x + j * kThreads; };
    // (m, l) of split `lane` and row `wave + NW i`, so that each row's maximum and total are reductions inside one wave
    const int wave = (int)threadIdx.x / kWave, lane = (int)threadIdx.x % kWave;
    float2 ml[RPW];
#pragma unroll
    for (int i = 0; i < RPW; i++) {
        const int r = min(wave + NW * i, RT - 1), k = min(lane, ns - 1);  // past the end: a valid pair, not used
        collect2(part_tile + k * SS + r * (HD + 4) + HD, ml[i].x, ml[i].y);
    }
    u32x4 px[CPT][MC];
    auto load_round = [&](int s0) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < CPT; j++) {
            const int col = column(j), pc = (col / (HD / 4)) * (HD + 4) + 4 * (col % (HD / 4));
#pragma unroll
            for (int e = 0; e < MC; e++) px[j][e] = load16_dev(rsrc, 4 * (pc + min(s0 + SF * e, ns - 1) * SS));
        }
    };
    load_round(stripe);
    // (the (m, l) loads went out first: the waits below leave the accumulator loads in flight)
    // each row: M = max over its splits, the splits' weights 2^(m - M) and the total, in the row's wave; an empty or
    // missing split has m = -inf (weight 0) and l = 0
#pragma unroll
    for (int i = 0; i < RPW; i++) {
        const int r = wave + NW * i;  // wave-uniform
        if (r >= RT) break;
        const bool ok = lane < ns && ml[i].y > 0.f;
        const float m = ok ? ml[i].x : kNegInf, l = ok ? ml[i].y : 0.f;
        const float M = row16_max(xor16_max(xor32_max(m)));  // in-register steps: no LDS round trips in the tail
        const float Mu = M == kNegInf ? 0.f : M;
        const float w = exp2_fast(m - Mu);
        const float tot = row16_sum(xor16_add(xor32_add(l * w)));
        if (lane < kMaxSplitsPerTile) s_w[lane * RT + r] = w;
        if (lane == 0) s_row[r] = make_float2(M, tot);
    }
    __syncthreads();
    if (threadIdx.x == 0) MX_TRACE(13);
    float4_t acc[CPT];
#pragma unroll
    for (int j = 0; j < CPT; j++) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};
    for (int s0 = stripe;;) {
#pragma unroll
        for (int j = 0; j < CPT; j++) {
            const int r = column(j) / (HD / 4);
#pragma unroll
            for (int e = 0; e < MC; e++) {
                const int k = s0 + SF * e;  // past the last split the slots' weights are 0 up to kMaxSplitsPerTile
                const float w = k < kMaxSplitsPerTile ? s_w[min(k, kMaxSplitsPerTile - 1) * RT + r] : 0.f;
                acc[j] += __builtin_bit_cast(float4_t, px[j][e]) * w;
            }
        }
        s0 += SF * MC;
        if (s0 >= ns) break;  // wave-uniform
        load_round(s0);
    }
    if (threadIdx.x == 0) MX_TRACE(15);
    if constexpr (SF > 1) {
        if (stripe > 0) s_acc[(stripe - 1) * NC + threadIdx.x % NC] = acc[0];
        __syncthreads();
        if (stripe > 0) return;
#pragma unroll
        for (int k = 1; k < SF; k++) acc[0] += s_acc[(k - 1) * NC + threadIdx.x];
    }
#pragma unroll
    for (int j = 0; j < CPT; j++) {
        const int col = column(j), r = col / (HD / 4), c = 4 * (col % (HD / 4));
        const int row = rt * RT + r;
        if (row >= p.rows) continue;
        const int t = row / G, h = g * G + row % G;
        const float2 mt = s_row[r];
        const float inv = 1.f / mt.y;
        const int64_t off = (seq_row0 + t) * p.out_stride + (int64_t)h * HD + c;
        if constexpr (F32) {
            *reinterpret_cast<float4_t *>(p.out32 + off) = acc[j] * inv;
        } else {
            typedef half_t half4_t __attribute__((ext_vector_type(4)));
            *reinterpret_cast<half4_t *>(p.out + off) =
                half4_t{(half_t)(acc[j][0] * inv), (half_t)(acc[j][1] * inv), (half_t)(acc[j][2] * inv),
                        (half_t)(acc[j][3] * inv)};
        }
        if (c == 0 && p.lse) p.lse[(seq_row0 + t) * p.n_head + h] = (mt.x + log2_fast(mt.y)) * kLn2;
    }
}

// HD: head_dim. RT: query rows per tile (4, 8 or 16; the MFMA tile always has 16 rows, the extra ones are zero).
// F32: the query rows and the output are f32, as in the reference's buffers (the query is rounded to half here).
// With p.append it is the fused decode step (one query row per sequence): q, k and v of the new token come unrotated
// from the q|k|v row; q and the new key are rotated for position kv_len - 1 and rounded to half, the new key and value
// are used from registers for that position and written into the caches by the one workgroup whose split holds it.
// NT: the keys and values are loaded non-temporally (p.kv_nt: a launch whose K/V stream from HBM once).
template <int HD, int RT, bool F32, int NW, bool NT = false>
__global__ __launch_bounds__(NW * kWave) void decode_kernel(DecodeParams p) {
    using B = KvBlock<HD>;
    constexpr int KS = B::KS, LPR = B::LPR, KPL = B::KPL, NLV = B::NLV;

    constexpr int VP = HD + 16;  // halves per row of a wave's V block in LDS (conflict-free transposing reads)
    constexpr int KPD = HD + 8;  // halves per row of its K block (16 rows' 16-byte reads at one column: distinct banks)
    static_assert(kBlockKeys * KPD <= kBlockKeys * VP, "the K block shares the V block's LDS");
    constexpr int kThreads = NW * kWave;
    static_assert(RT * HD * 4 <= kBlockKeys * VP * 2, "a wave's O rows reuse its V block's LDS");
    __shared__ half_t s_v[NW][kBlockKeys * VP];
    __shared__ float s_m[NW][RT], s_l[NW][RT];
    // after its last block each wave's V staging area holds its O rows (RT x HD f32)
    auto s_o = [&](int w) { return reinterpret_cast<float *>(s_v[w]); };
    __shared__ int s_last;
    __shared__ float2 s_cs[F32 ? HD / 2 : 1];  // fused step: (cos, sin) of each rotary pair's angle

    // Every argument the start of the kernel needs is fetched in one batch of scalar loads: pinned into registers here,
    // before the first branch. Otherwise the compiler issues each load after the branch before its first use, and the
    // kernel waits for up to four dependent round trips to the argument memory before its first K/V load. The sequence
    // is blockIdx.y, so its descriptor's address is known at once.
    const int bl = blockIdx.y;
    const half_t * seq_k = p.seq[bl].k;
    const half_t * seq_v = p.seq[bl].v;
    int32_t L = p.seq[bl].len, n_split = p.seq[bl].n_split;
    uint32_t T = p.n_rowtiles;
    int32_t max_split = p.max_split, n_head_kv = p.n_head_kv, chunk = p.chunk, G = p.group, seq0 = p.seq0, n_q = p.n_q;
    int32_t rows = p.rows, causal = p.causal, xcd_heads = p.xcd_heads;
    int64_t q_stride = p.q_stride, kv_stride = p.kv_stride;
    const half_t * qp = p.q;
    asm volatile("" : "+s"(seq_k), "+s"(seq_v), "+s"(L), "+s"(n_split), "+s"(T), "+s"(max_split), "+s"(n_head_kv),
                 "+s"(chunk), "+s"(G), "+s"(seq0), "+s"(n_q), "+s"(rows), "+s"(causal), "+s"(xcd_heads), "+s"(q_stride),
                 "+s"(kv_stride), "+s"(qp));
    // the fused step's own arguments likewise (fetched behind branches they cost dependent scalar round trips ahead
    // of the first K/V load)
    const float * qkv = p.qkv;
    int32_t n_head = p.n_head, append = p.append, rope_mode = p.rope_mode;
    if constexpr (F32) asm volatile("" : "+s"(qkv), "+s"(n_head), "+s"(append), "+s"(rope_mode));
    // fused step: this thread's rotary frequency (threads 0 .. HD / 2 - 1 use theirs) as one vector load of the
    // kernel arguments, issued before the first K/V block so that it returns ahead of it (loads return in order) and
    // is waited for with the new key and value. As uniform-index scalar loads the compiler issued them after the block
    // and waited for them behind the whole chip's burst; pinned here as scalar loads they took three dependent batches.
    float freq = 0.f;
    if constexpr (F32) freq = p.rope_freq[threadIdx.x % (HD / 2)];

    // Work item. The row tiles of one (sequence, kv head, split) read the same keys and values, so they run as
    // consecutive workgroups of one XCD (workgroups are dealt to the 8 XCDs round-robin: ids 8 apart share one), where
    // all but the first read hit that XCD's L2. With one row tile this is the identity. With xcd_heads (kv heads in
    // multiples of 8, or one short sequence with its kv heads padded to a multiple of 8) every split of kv head g runs
    // on XCD g % 8 instead (the sequence is blockIdx.y; the grid's x extent is a multiple of 8): each XCD streams whole
    // kv heads and the merging workgroup finds the partials of its head in its own XCD's L2.
    if (threadIdx.x == 0) {
        MX_TRACE(0);
        MX_TRACE_CLEAR(12);
        MX_TRACE_CLEAR(13);
        MX_TRACE_CLEAR(15);
    }
    const uint32_t id = blockIdx.x, k8 = id / 8, u = k8 / T;
    const int rt = k8 % T;
    int s, g;  // split, kv head
    if (xcd_heads) {
        s = u % max_split;
        g = (u / max_split) * 8 + id % 8;
    } else {
        const uint32_t grp = u * 8 + id % 8;  // (split, kv head) group of the sequence
        s = grp % max_split;
        g = grp / max_split;
    }
    if (g >= n_head_kv) return;  // padding of the grid to whole XCD rounds
    if (s >= n_split) return;    // uniform over the workgroup, before any barrier

    const int j0 = s * chunk;
    const int j1 = min(j0 + chunk, L);
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int64_t seq_row0 = (int64_t)(seq0 + bl) * n_q;  // first query row of the sequence

    const half_t * kbase = seq_k + (int64_t)g * HD;
    const half_t * vbase = seq_v + (int64_t)g * HD;
    const int srow = lane % 16, sgrp = lane / 16;          // score lanes: row srow, keys 4 sgrp .. + 4 of a 16-key tile
    const int vslot = lane / LPR, vcol = 8 * (lane % LPR); // value lanes: key slot, first head dim

    auto load_block = [&](int jb, B & blk) {
#pragma unroll
        for (int i = 0; i < NLV; i++) {
            const int key = min(jb + KPL * i + vslot, L - 1);
            blk.k[i] = load16_kv<NT>(kbase + (int64_t)key * kv_stride + vcol);
        }
#pragma unroll
        for (int i = 0; i < NLV; i++) {
            const int key = min(jb + KPL * i + vslot, L - 1);
            blk.v[i] = load16_kv<NT>(vbase + (int64_t)key * kv_stride + vcol);
        }
    };

    // ---- this lane's score row and its query operand ----
    const int rr = rt * RT + srow;  // row index inside the (sequence, kv head) problem: rr = t * G + gi
    const bool srow_ok = srow < RT && rr < rows;
    const int st = rr / G, sh = g * G + rr % G;
    const int lim = causal ? L - n_q + st : L - 1;  // last visible key of the row
    half8_t qb[KS];
    float xq[F32 ? KS : 1][8] = {};  // the f32 query (fused step: rotated once the first block's loads are out)
    if constexpr (F32) {
        const float * qrow = qkv + (seq_row0 + st) * q_stride + (int64_t)sh * HD;
        if (srow_ok) {
#pragma unroll
            for (int ks = 0; ks < KS; ks++) load8f(qrow + 32 * ks + 8 * sgrp, xq[ks]);
        }
    }
    // f16 query rows: loaded unconditionally behind the first block of keys and values (below); a conditional load
    // would make the compiler drain it before the block's loads
    u32x4 qv[F32 ? 1 : KS];
    const half_t * qrow = qp + (seq_row0 + (srow_ok ? st : 0)) * q_stride + (int64_t)(srow_ok ? sh : g * G) * HD;

    // fused step: the new position L - 1 lies in the block starting at jb_new, walked by one wave of the last split
    const int jb_new = (L - 1) & ~(kBlockKeys - 1);
    const bool wave_new = F32 && append && j1 == L && jb_new >= j0 && ((jb_new - j0) / kBlockKeys) % NW == wave;
    const bool k_lane_new = wave_new && srow == (L - 1) % 16;       // holds the new key in tile (L - 1) % 32 / 16
    const bool v_lane_new = wave_new && vslot == (L - 1) % KPL;     // holds the new value in load (L - 1) % 32 / KPL
    // The fused step's own loads (the new key and value) go out before the first block of keys
    // and values: a wait for them then leaves that block's loads in flight (loads complete in the order issued).
    float x[F32 ? KS : 1][8], xv[8];
    if constexpr (F32) {
        const float * row = qkv + seq_row0 * q_stride;
        if (k_lane_new) {
            const float * kr = row + (int64_t)(n_head + g) * HD + 8 * sgrp;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) load8f(kr + 32 * ks, x[ks]);
        }
        if (v_lane_new) load8f(row + (int64_t)(n_head + n_head_kv + g) * HD + vcol, xv);
    }

    // the first block of keys and values goes out right behind the query (unconditionally: keys past the split are
    // clamped to valid rows and never used, and the compiler then knows how many loads follow the ones above)
    int jb = j0 + kBlockKeys * wave;
    B cur, nxt;
    load_block(jb, cur);
    // f16 query rows: loaded by every lane (rows past the tile read the problem's first row, a valid address) behind the
    // first block and zeroed where they are first used, in the walk behind the next block's prefetch. All the waves of
    // a kv head's splits read the same query bytes; behind the keys and values that read no longer holds back their
    // stream (loads return in order): batch 16 56.8 -> 55.7 us, the short shapes within +-0.1 us.
    if constexpr (!F32) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) qv[ks] = load16(qrow + 32 * ks + 8 * sgrp);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (F32) {
        // the new key and value (and the frequency) are used only from here on, so any wait for them leaves the block's
        // loads in flight
        asm volatile("" : "+v"(freq)::"memory");
#pragma unroll
        for (int e = 0; e < 8; e++) asm volatile("" : "+v"(xv[e])::"memory");
#pragma unroll
        for (int ks = 0; ks < KS; ks++)
#pragma unroll
            for (int e = 0; e < 8; e++) asm volatile("" : "+v"(x[ks][e])::"memory");
    }

    u32x4 kn[KS], vn = {0u, 0u, 0u, 0u};
    if constexpr (F32) {  // fused step: the query and the new key rotated, the new key and value rounded to half
        if (append && rope_mode != 2) {  // the 64 (hd 128) angles of position L - 1, once per workgroup
            if (threadIdx.x < HD / 2) {
                float sn, cs;
                sincos_rope((float)(L - 1) * freq, sn, cs);
                s_cs[threadIdx.x] = make_float2(cs, sn);
            }
            __syncthreads();
        }
        if (srow_ok && append) rope_rotate<KS, 32>(xq, 8 * sgrp, rope_mode, [&](int i) { return s_cs[i]; });
#pragma unroll
        for (int ks = 0; ks < KS; ks++) qb[ks] = as_half8(to_half8(xq[ks]));
        if (k_lane_new) {
            rope_rotate<KS, 32>(x, 8 * sgrp, rope_mode, [&](int i) { return s_cs[i]; });
#pragma unroll
            for (int ks = 0; ks < KS; ks++) kn[ks] = to_half8(x[ks]);
            if (rt == 0) {
                half_t * kd = const_cast<half_t *>(kbase) + (int64_t)(L - 1) * p.kv_stride + 8 * sgrp;
#pragma unroll
                for (int ks = 0; ks < KS; ks++) *reinterpret_cast<u32x4 *>(kd + 32 * ks) = kn[ks];
            }
        }
        if (v_lane_new) {
            vn = to_half8(xv);
            if (rt == 0) *reinterpret_cast<u32x4 *>(const_cast<half_t *>(vbase) + (int64_t)(L - 1) * p.kv_stride + vcol) = vn;
        }
    }

    float m_run = kNegInf, l_run = 0.f;  // per score lane (row srow); l is this lane's partial sum
    // O^T accumulators (16 head dims x 16 rows per tile): lane holds O[row srow][16 dtile + 4 sgrp + v], v = 0..3
    float4_t o[HD / 16];
#pragma unroll
    for (int dt = 0; dt < HD / 16; dt++) o[dt] = float4_t{0.f, 0.f, 0.f, 0.f};
    // transposing read of V^T: lane a of 16-lane group g supplies V[4 g + a / 4 (+ 16)][16 dtile + 4 (a % 4)] and
    // receives V[4 g + 0..3 (+ 16)][16 dtile + a]
    half_t * vw = s_v[wave];
    const int v_rd = (4 * sgrp + (lane % 16) / 4) * VP + 4 * (lane % 4);

    bool q_pending = !F32;
    for (; jb < j1; jb += kBlockKeys * NW) {
        const int jn = jb + kBlockKeys * NW;
        if (jn < j1) load_block(jn, nxt);
        if constexpr (!F32) {
            if (q_pending) {  // the first block: the query operand, its wait leaving the next block in flight
                q_pending = false;
#pragma unroll
                for (int ks = 0; ks < KS; ks++) {
                    asm volatile("" : "+v"(qv[ks])::"memory");
                    qb[ks] = as_half8(srow_ok ? qv[ks] : u32x4{0u, 0u, 0u, 0u});
                }
            }
        }
        if constexpr (F32) {
            if (wave_new && jb == jb_new) {  // the new key and value replace what the cache held at L - 1
                const int i_new = ((L - 1) % kBlockKeys) / KPL;
                // Key slots past L - 1 were clamped to row L - 1, whose memory holds what the cache had before this
                // step (and which the row-tile-0 workgroup is overwriting). Their scores are masked, but a stale
                // Inf/NaN there would survive the p = 0 product, so their value operand is zero instead.
#pragma unroll
                for (int i = 0; i < NLV; i++) {
                    if (v_lane_new && i == i_new) cur.v[i] = vn;
                    else if (jb + KPL * i + vslot > L - 1) cur.v[i] = u32x4{0u, 0u, 0u, 0u};
                }
            }
        }
        // the wave's K block into LDS row-major, read back as the MFMA operand: lane holds K[16 mt + srow][32 ks + 8 sgrp
        // .. + 8] (the buffer is the V block's, written below once these reads are done)
#pragma unroll
        for (int i = 0; i < NLV; i++)
            *reinterpret_cast<u32x4 *>(vw + (KPL * i + vslot) * KPD + vcol) = cur.k[i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        u32x4 kr[2][KS];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
                kr[mt][ks] = *reinterpret_cast<const u32x4 *>(vw + (16 * mt + srow) * KPD + 32 * ks + 8 * sgrp);
        if constexpr (F32) {
            if (wave_new && jb == jb_new) {  // the new key replaces what the cache held at L - 1
                const int mt_new = ((L - 1) % kBlockKeys) / 16;
#pragma unroll
                for (int mt = 0; mt < 2; mt++)  // constant register indices: a runtime one would go through memory
#pragma unroll
                    for (int ks = 0; ks < KS; ks++)
                        if (k_lane_new && mt == mt_new) kr[mt][ks] = kn[ks];
            }
        }
        // S^T = K Q^T, 2 tiles of 16 keys: lane holds keys 16 mt + 4 sgrp + v of row srow
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
        bmax = xor32_max(xor16_max(bmax));
        const float m_new = fmaxf(m_run, bmax);
        const bool none = m_new == kNegInf;      // no visible key yet for this row
        const float m_use = none ? 0.f : m_new;  // then every exponent below is 2^-inf = 0
        const float corr = none ? 1.f : exp2_fast(m_run - m_new);
        half8_t pb;  // P^T operand: slot (sgrp, e) is key 16 (e / 4) + 4 sgrp + e % 4, the same keys the V^T reads fetch
        float bsum = 0.f;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float pv = exp2_fast(sc[e / 4][e % 4] - m_use);
            bsum += pv;
            pb[e] = (half_t)pv;
        }
        l_run = l_run * corr + bsum;
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < HD / 16; dt++) o[dt] *= corr;
        // the wave's V block into LDS, row-major (one 16-byte chunk per lane per load)
#pragma unroll
        for (int i = 0; i < NLV; i++)
            *reinterpret_cast<u32x4 *>(vw + (KPL * i + vslot) * VP + vcol) = cur.v[i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // O^T += V^T P^T on the matrix cores, one 16x16x32 product per 16 head dims
#pragma unroll
        for (int dt = 0; dt < HD / 16; dt++) {
            const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) short4_t *)(vw + v_rd + 16 * dt));
            const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) short4_t *)(vw + v_rd + 16 * VP + 16 * dt));
            const half8_t a = __builtin_bit_cast(half8_t, (short __attribute__((ext_vector_type(8)))){
                lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
            o[dt] = mfma16x16x32(a, pb, o[dt]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        cur = nxt;
    }

    if (lane == 0) MX_TRACE(1 + wave);
    // ---- wave totals: l over the 4 score-lane groups; O is complete per lane (the products summed every key) ----
    l_run = xor32_add(xor16_add(l_run));
    if (lane < RT) {
        s_m[wave][lane] = l_run > 0.f ? m_run : kNegInf;  // a wave with no visible key counts as -inf
        s_l[wave][lane] = l_run;
    }
    if (srow < RT) {
#pragma unroll
        for (int dt = 0; dt < HD / 16; dt++)
            *reinterpret_cast<float4_t *>(s_o(wave) + srow * HD + 16 * dt + 4 * sgrp) = o[dt];
    }
    __syncthreads();

    if (threadIdx.x == 0) MX_TRACE(9);
    // ---- merge the NW waves; write the output (one split) or publish this split's partial ----
    // Each thread owns head-dim pairs (r, 2 dp .. + 2) of the tile's RT x HD outputs.
    const bool single = n_split == 1;
    const int64_t tile = ((int64_t)bl * p.n_head_kv + g) * p.n_rowtiles + rt;  // (sequence, kv head, row tile)
    float * part_tile = p.part + tile * p.max_split * RT * (HD + 4);
    constexpr int64_t SS = (int64_t)RT * (HD + 4);  // floats between the partials of consecutive splits
    constexpr int NP = RT * HD / 2;                 // output pairs of the tile
    // Head dim 128, several splits: the partial goes out in 16-byte device-scope stores, four outputs per thread (half
    // the store instructions of the pairs below, whose completion the count then waits for; batch 1 at 8192 keys
    // 11.72 -> 11.55 us per launch).
    constexpr bool kQuadPublish = HD == 128;
    const bool local = xcd_heads;  // the XCD-mapped grid: partials published XCD-locally
    if (kQuadPublish && !single) {
        constexpr int NQ = RT * HD / 4;
        const __amdgpu_buffer_rsrc_t prs = dev_rsrc(part_tile + s * SS);
        for (int idx = threadIdx.x; idx < NQ; idx += kThreads) {
            const int r = idx / (HD / 4), d = 4 * (idx % (HD / 4));
            if (rt * RT + r >= p.rows) continue;
            float mw[NW];
#pragma unroll
            for (int w = 0; w < NW; w++) mw[w] = s_m[w][r];
            float M = kNegInf;
#pragma unroll
            for (int w = 0; w < NW; w++) M = fmaxf(M, mw[w]);
            const float Mu = M == kNegInf ? 0.f : M;
            float tot = 0.f;
            float4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int w = 0; w < NW; w++) {
                const float wt = exp2_fast(mw[w] - Mu);
                tot += s_l[w][r] * wt;
                a += *reinterpret_cast<const float4_t *>(s_o(w) + r * HD + d) * wt;
            }
            float * ml = part_tile + s * SS + (int64_t)r * (HD + 4) + HD;
            if (local) {
                store16_xcd(prs, 4 * (r * (HD + 4) + d), a);
                if (d == 0) publish2_xcd(ml, M, tot);
            } else {
                store16_dev(prs, 4 * (r * (HD + 4) + d), a);
                if (d == 0) publish2(ml, M, tot);
            }
        }
    }
    for (int idx = threadIdx.x; idx < ((kQuadPublish && !single) ? 0 : NP); idx += kThreads) {
        const int r = idx / (HD / 2), d = 2 * (idx % (HD / 2));
        const int row = rt * RT + r;
        if (row >= p.rows) continue;
        // branch-free: a wave without keys has m = -inf, weight 2^-inf = 0 and O = 0, so every read is independent
        // (a test of l > 0 per wave compiled to a chain of dependent LDS reads and branches in the launch's tail)
        float mw[NW];
#pragma unroll
        for (int w = 0; w < NW; w++) mw[w] = s_m[w][r];
        float M = kNegInf;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, mw[w]);
        const float Mu = M == kNegInf ? 0.f : M;
        float tot = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float wt = exp2_fast(mw[w] - Mu);
            tot += s_l[w][r] * wt;
            a0 += s_o(w)[r * HD + d] * wt;
            a1 += s_o(w)[r * HD + d + 1] * wt;
        }
        if (single) {
            const int t = row / G, h = g * G + row % G;
            store_pair<F32>(p, (seq_row0 + t) * p.out_stride + (int64_t)h * HD + d, a0 / tot, a1 / tot);
            if (d == 0 && p.lse) p.lse[(seq_row0 + t) * p.n_head + h] = (M + log2_fast(tot)) * kLn2;
        } else {
            float * pe = part_tile + s * SS + (int64_t)r * (HD + 4);
            if (local) {
                publish2_xcd(pe + d, a0, a1);
                if (d == 0) publish2_xcd(pe + HD, M, tot);
            } else {
                publish2(pe + d, a0, a1);
                if (d == 0) publish2(pe + HD, M, tot);
            }
        }
    }
    if (single) return;

    // Every thread waits until its partial stores are complete (performed at device scope, or in the XCD's L2 when
    // published XCD-locally), then one thread counts the split in. The merging workgroup reads the partials with
    // device-scope loads after seeing the final count.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) MX_TRACE(10);
    uint32_t * const counter = p.counters + tile * kCounterStride;
    if (threadIdx.x == 0) {
        if (local) {
            const uint32_t x = xcc_id();
            const uint64_t now = __hip_atomic_fetch_add(reinterpret_cast<uint64_t *>(counter), 1ull << (kXccField * x),
                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) +
                                 (1ull << (kXccField * x));
            uint32_t n = 0;
#pragma unroll
            for (int f = 0; f < 8; f++) n += (uint32_t)(now >> (kXccField * f)) & 63u;
            s_last = n == (uint32_t)n_split ? 1 + ((uint32_t)(now >> (kXccField * x) & 63u) != (uint32_t)n_split) : 0;
        } else {
            const uint32_t done = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = done == (uint32_t)(n_split - 1);
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) MX_TRACE(11);
    if (!s_last) return;
    __builtin_amdgcn_s_waitcnt(0);
    auto reset_counter = [&]() {
        if (threadIdx.x != 0) return;
        if (local) __hip_atomic_store(reinterpret_cast<uint64_t *>(counter), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    if (s_last == 2) {
        // Some split of the tile ran on another XCD: its partial may sit in that XCD's L2, out of reach. The dispatch
        // rule this grid relies on did not hold; the tile's outputs are NaN rather than a merge of what is visible.
        for (int idx = threadIdx.x; idx < NP; idx += kThreads) {
            const int r = idx / (HD / 2), d = 2 * (idx % (HD / 2)), row = rt * RT + r;
            if (row >= p.rows) continue;
            const int t = row / G, h = g * G + row % G;
            store_pair<F32>(p, (seq_row0 + t) * p.out_stride + (int64_t)h * HD + d, __builtin_nanf(""), __builtin_nanf(""));
            if (d == 0 && p.lse) p.lse[(seq_row0 + t) * p.n_head + h] = __builtin_nanf("");
        }
        reset_counter();
        return;
    }

    // ---- cross-split merge (attention_combine, llama_kernels.h:912-929). Each thread merges its output pairs on its
    // own: per chunk of kMergeChunk splits it issues every load first ((m, l) of its row and its pair, for all the
    // chunk's splits; the row's (m, l) loads of a wave coalesce), then folds them with a running maximum. One memory
    // round trip per chunk, no LDS, no barrier. ----
    const int ns = n_split;
    if constexpr (HD == 128) {
        if (ns > 1) {
            // the smallest round (splits per column and stripe) that covers the tile's splits
            constexpr int SFW = NW * kWave >= RT * HD / 4 ? NW * kWave / (RT * HD / 4) : 1;
            char * lds = reinterpret_cast<char *>(s_v);
            if (ns <= 2 * SFW) merge_wide<HD, RT, F32, NW, sizeof s_v, 2>(p, part_tile, ns, rt, g, G, seq_row0, lds);
            else if (ns <= 4 * SFW) merge_wide<HD, RT, F32, NW, sizeof s_v, 4>(p, part_tile, ns, rt, g, G, seq_row0, lds);
            else if (ns <= 8 * SFW) merge_wide<HD, RT, F32, NW, sizeof s_v, 8>(p, part_tile, ns, rt, g, G, seq_row0, lds);
            else merge_wide<HD, RT, F32, NW, sizeof s_v, 16>(p, part_tile, ns, rt, g, G, seq_row0, lds);
            reset_counter();
#ifdef MX_ATTN_TRACE
            __syncthreads();
            if (threadIdx.x == 0) MX_TRACE(12);
#endif
            return;
        }
    }
    constexpr int PPT = (NP + kThreads - 1) / kThreads;  // output pairs per thread
    // CH: splits whose loads are in flight at once, the smallest of 4, 6, 8, 12, 16 that holds them all (beyond 16,
    // chunks of 16); past the last split the loads repeat it and weigh 0, so every CH >= ns gives the same sums
    auto merge_pairs = [&](auto CHC) __attribute__((always_inline)) {
        constexpr int CH = decltype(CHC)::value;
#pragma unroll
        for (int j = 0; j < PPT; j++) {
            const int idx = threadIdx.x + j * kThreads;
            if (idx >= NP) break;
            const int r = idx / (HD / 2), d = 2 * (idx % (HD / 2));
            const int row = rt * RT + r;
            if (row >= p.rows) continue;
            const float * pr = part_tile + (int64_t)r * (HD + 4);
            float M = kNegInf, tot = 0.f, a0 = 0.f, a1 = 0.f;
            for (int k0 = 0; k0 < ns; k0 += CH) {
                float m[CH], l[CH], u[CH], v[CH];
#pragma unroll
                for (int e = 0; e < CH; e++) {
                    const int k = min(k0 + e, ns - 1);  // past the end: repeat the last split, weighted 0 below
                    collect2(pr + k * SS + HD, m[e], l[e]);
                    collect2(pr + k * SS + d, u[e], v[e]);
                }
                float cm = M;
#pragma unroll
                for (int e = 0; e < CH; e++)
                    if (k0 + e < ns && l[e] > 0.f) cm = fmaxf(cm, m[e]);
                const float c = cm == M ? 1.f : exp2_fast(M - cm);  // rescale of what was summed so far
                tot *= c;
                a0 *= c;
                a1 *= c;
                M = cm;
#pragma unroll
                for (int e = 0; e < CH; e++) {
                    const float w = (k0 + e < ns && l[e] > 0.f) ? exp2_fast(m[e] - M) : 0.f;
                    tot = __builtin_fmaf(l[e], w, tot);
                    a0 = __builtin_fmaf(u[e], w, a0);
                    a1 = __builtin_fmaf(v[e], w, a1);
                }
            }
            const int t = row / G, h = g * G + row % G;
            const float inv = 1.f / tot;
            store_pair<F32>(p, (seq_row0 + t) * p.out_stride + (int64_t)h * HD + d, a0 * inv, a1 * inv);
            if (d == 0 && p.lse) p.lse[(seq_row0 + t) * p.n_head + h] = (M + log2_fast(tot)) * kLn2;
        }
    };
    static_assert(kMergeChunk == 16, "the chunk sizes below");
    if (ns <= 4) merge_pairs(std::integral_constant<int, 4>{});
    else if (ns <= 6) merge_pairs(std::integral_constant<int, 6>{});
    else if (ns <= 8) merge_pairs(std::integral_constant<int, 8>{});
    else if (ns <= 12) merge_pairs(std::integral_constant<int, 12>{});
    else merge_pairs(std::integral_constant<int, 16>{});
    reset_counter();
#ifdef MX_ATTN_TRACE
    __syncthreads();
    if (threadIdx.x == 0) MX_TRACE(12);
#endif
}

template <int HD, int RT, int NW>
hipError_t launch_decode_t(const DecodeParams & p, int n_seq, hipStream_t stream) {
    // x: groups of (split, kv head), 8 per round of XCDs, each group's row tiles on one XCD; y: the sequence
    // (the XCD-mapped grid: kv head g's splits at ids = g mod 8, so the kv heads round up to a multiple of 8)
    const int64_t groups = (int64_t)p.max_split * (p.xcd_heads ? (p.n_head_kv + 7) / 8 * 8 : p.n_head_kv);
    const dim3 grid((uint32_t)(((groups + 7) / 8) * 8 * p.n_rowtiles), (uint32_t)n_seq);
    if constexpr (HD == 128 && RT == 4) {  // one query row per Llama-3-8B-shaped sequence (4 query heads per kv head)
        if (p.kv_nt) {
            if (p.f32)
                hipLaunchKernelGGL((decode_kernel<HD, RT, true, NW, true>), grid, dim3(NW * kWave), 0, stream, p);
            else
                hipLaunchKernelGGL((decode_kernel<HD, RT, false, NW, true>), grid, dim3(NW * kWave), 0, stream, p);
            return hipGetLastError();
        }
    }
    if (p.f32)
        hipLaunchKernelGGL((decode_kernel<HD, RT, true, NW>), grid, dim3(NW * kWave), 0, stream, p);
    else
        hipLaunchKernelGGL((decode_kernel<HD, RT, false, NW>), grid, dim3(NW * kWave), 0, stream, p);
    return hipGetLastError();
}

template <int HD, int NW>
hipError_t launch_decode_hd(const DecodeParams & p, int n_seq, int rt, hipStream_t stream) {
    if (rt == 4) return launch_decode_t<HD, 4, NW>(p, n_seq, stream);
    if (rt == 8) return launch_decode_t<HD, 8, NW>(p, n_seq, stream);
    return launch_decode_t<HD, 16, NW>(p, n_seq, stream);
}

// Zero fill (the split counters start at 0); a kernel rather than a memset so that a caller may capture it in a graph.
__global__ void fill_zero_kernel(uint32_t * p, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}

}  // namespace

int decode_rows_per_tile(int rows) { return rows <= 4 ? 4 : rows <= 8 ? 8 : 16; }

hipError_t launch_decode(const DecodeParams & p, int n_seq, int head_dim, int rt, int waves, hipStream_t stream) {
    // head dim 256: 4 waves only (8 would spill: the double-buffered K/V block and O take every register of a wave)
    if (head_dim == 256) return launch_decode_hd<256, 4>(p, n_seq, rt, stream);
    if (head_dim == 64)
        return waves == 8 ? launch_decode_hd<64, 8>(p, n_seq, rt, stream) : launch_decode_hd<64, 4>(p, n_seq, rt, stream);
    return waves == 8 ? launch_decode_hd<128, 8>(p, n_seq, rt, stream) : launch_decode_hd<128, 4>(p, n_seq, rt, stream);
}

hipError_t launch_fill_zero(void * p, size_t bytes, hipStream_t stream) {
    const size_t n = bytes / 4;
    if (n == 0) return hipSuccess;
    const unsigned blocks = (unsigned)((n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024);
    hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, stream, static_cast<uint32_t *>(p), n);
    return hipGetLastError();
}

}  // namespace mx

#ifdef MX_ATTN_TRACE
// Copies the trace (8192 workgroups x 16 stamps, uint64) to host memory; returns a hipError_t.
extern "C" __attribute__((visibility("default"))) int mx_attn_trace_read(void * host, size_t bytes) {
    if (bytes > sizeof g_decode_trace) bytes = sizeof g_decode_trace;
    return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_decode_trace), bytes, 0, hipMemcpyDeviceToHost);
}
#endif
