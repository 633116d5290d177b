// Prefill (prompt chunk) flash attention, causal GQA, f16 Q/K/V, f32 statistics and accumulation.
//
// Reference behaviour (dooms.cpp 0.6.1): `attention_prefill<HD>` (src/backend/metal/llama_kernels.h:632-769) as dispatched by
// MetalLlamaDecoder::Impl::attention (src/backend/metal/metal_llama_decoder.mm:284-296): query row t of a chunk of M rows
// sits at position p0 + t and sees keys 0 .. p0 + t of the cache; S = Q K^T (half operands, f32 accumulation), running max
// m and sum l with the rescale factor exp(m_old - m_new), P rounded to half, O += P V, and O / l at the end.
//
// MI355X design:
//   * One workgroup = 8 waves = 256 query rows of one query head (4 waves = 128 rows for short prompts); each wave owns
//     32 rows. When even those would leave most CUs idle, two waves share a 32-row tile and split its key blocks. The register budget is held to 256 per lane, so each SIMD interleaves two waves: one wave's softmax runs
//     on the vector ALU while the other's products run on the matrix core; all waves of a CU share each K/V tile.
//   * Key/value blocks of 64 rows pass through LDS. Every plan on f16 operands at head dims 64 and 128 loads them
//     straight into LDS (global_load_lds_dwordx4), two to four buffers deep, as 1 KB blocks of 16 rows x 64 bytes with
//     a bank swizzle chosen by which bytes each lane fetches; the IR self-attention's converted rows and head dim 256
//     double-buffer through registers: block i + 1 goes from registers into the free LDS buffer and block i + 2 is
//     loaded into registers while block i is multiplied, in row-major tiles with padded rows. Either way the K reads and the transposing V reads are free of bank conflicts
//     and address with per-lane bases plus compile-time offsets; one barrier per block.
//   * Transposed scores: S^T (keys x queries) = K Q^T on v_mfma_f32_32x32x16_f16. In the result each lane holds 16 keys
//     of ONE query (the lane 32 away the other 16), so the row max and sum need one cross-lane step, and the
//     probabilities already sit in the B-operand layout of O^T += V^T P^T: P never touches LDS. Q^T is loaded once into
//     registers. The V^T operand comes straight from the row-major V tile through ds_read_b64_tr_b16, whose 16-lane
//     transpose hands every lane four consecutive keys of one head dimension.
//   * The softmax runs in base 2: the block maximum is taken on raw scores and scale * log2 e folded into the FMA that
//     feeds v_exp_f32; masking only in blocks that cross the causal diagonal or the end of the cache; blocks past a
//     wave's last row are skipped; the output is rescaled only when the running maximum of some row moved.
//   * Workgroups are dealt out so that the heaviest query tiles start first and the heads of one GQA group run next to
//     each other on the same XCD (shared K/V in that XCD's L2).
#include "mx_common.hpp"
#include "mx_kernels.hpp"

#include <type_traits>


namespace mx {

namespace {

constexpr int kBK = 64;  // keys per block

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef half_t half2_t __attribute__((ext_vector_type(2)));
constexpr half2_t kOnes2 = {(half_t)1.f, (half_t)1.f};
// The largest per-lane sum of a block's half probabilities (32 of them) at the kept reference maximum before the
// exact update runs: below it every probability is below 2^8.
constexpr float kProbSumMax = 256.f;

// Relaxed device-scope accesses of the stream-K partials: coherent across the XCDs without cache maintenance.
__device__ __forceinline__ void put_f32(float * a, float v) {
    __hip_atomic_store(reinterpret_cast<uint32_t *>(a), __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float get_f32(const float * a) {
    return __uint_as_float(__hip_atomic_load(reinterpret_cast<uint32_t *>(const_cast<float *>(a)), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT));
}

// LDS tiles are row-major with padded rows: K rows HD + 8 halves apart (the 16-byte reads of 16 consecutive rows at one
// column land on 16 distinct 4-bank groups), V rows HD + 32 halves apart (a row step of 16 banks mod 64: the 4 rows x
// 32 bytes that each 16-lane group reads through the transposing read, for both groups of a 32-lane phase, land on 64
// distinct banks; the tile store writes 4 rows x 4 chunks per 16 lanes, also 16 distinct 4-bank groups). Every read
// address is a per-lane base plus a compile-time offset, so the loop spends no ALU on addressing.
template <int HD, int KSP, bool DL = false, int W = 8>
struct PrefillSmem {
    static constexpr int KP = HD + 8;
    static constexpr int VP = HD + 32;
    half_t k[2][KSP * kBK * KP];
    half_t v[2][KSP * kBK * VP];
};

// Direct-to-LDS tiles (DL: the 8-wave, head-dim-128 plan on f16 operands). global_load_lds_dwordx4 writes the 16 bytes
// of lane l to LDS byte 16 l of the instruction's 1 KB destination, so a tile is a grid of 1 KB blocks, each one
// instruction: block (cb, rb) = 4 cb + rb holds rows 16 rb .. + 16 x 16-byte chunks 4 cb .. + 4 (64 contiguous bytes of
// each row in memory), row r % 16 at block byte 64 (r % 16). Which chunk a lane fetches sets the bank spread:
//   K: chunk c of row r sits at 16 ((c % 4) ^ ((r % 16) / 4)) in its row's 64 bytes: the 16-byte reads of 16
//      consecutive rows at one chunk land on 16 distinct 4-bank groups, and the swizzle leaves the compile-time part of
//      a read's chunk index (its 32-byte half) additive: two per-lane bases, the rest instruction offsets;
//   V: no swizzle: each 32-lane phase of the transposing read takes 4 consecutive rows x 64 bytes, 256 contiguous bytes.
// Three buffers: the loads of step i + 2 go out while step i is multiplied, with no registers in between.
// buffers (PrefillSmem::NBUF): three (two steps ahead) for the 8-wave plan, where a fourth measured the same; in the
// 4-wave plans four at head dim 64 (their steps are short against a memory round trip) and two at head dim 128 (the
// key-split plan's 64 KB steps; the 32-row plan's two workgroups per CU)
template <int HD, int W, int KSP, int SA>
constexpr bool prefill_dl() {
    return SA == 0 && ((HD == 128 && W == 8 && KSP == 1) || (W == 4 && (HD == 64 || HD == 128)));
}

template <int HD, int KSP, int W>
struct PrefillSmem<HD, KSP, true, W> {
    // 8 waves (one workgroup per CU): 3; 4 waves: 4 at head dim 64, 2 at 128 (64 KB, two workgroups per CU)
    static constexpr int NBUF = W == 8 ? 3 : (HD == 64 ? 4 : 2);
    half_t k[NBUF][KSP * kBK * HD];
    half_t v[NBUF][KSP * kBK * HD];
};

// Work order of the prefill grid (o = 0 .. n_qtiles * n_head - 1), cut by xcd_remap into one contiguous range per XCD:
// kv head slowest, so an XCD serves the GQA group of one kv head (or of a few, with more than 8 kv heads) and streams
// only that head's keys and values through its L2. When c = 8 / n_kv XCDs share a kv head (n_kv in {1, 2, 4}), its
// query tiles are dealt to them round-robin (tile orders u, u + c, u + 2c, ... to the u-th), so each gets an equal
// share of the causal work; within a range the heaviest tiles come first and the G heads of one tile are adjacent
// (they read the same keys at the same time). The earlier order (query tile slowest, contiguous ranges) gave the
// first XCD all the heaviest tiles of a multi-round launch and every XCD every kv head's K/V: Llama-3-8B 4096-token
// prompt 250 -> 166 us, the 32k Qwen2.5-7B prompt in one call 12.7 -> 7.8 ms; a snake order that balances the tiles
// but keeps every head on every XCD measured the same as this one, so the balance is what pays.
__device__ __forceinline__ void prefill_work(uint32_t o, int nq, int G, int n_kv, int & kvh, int & gi, int & qt_order) {
    const int per_kv = nq * G;
    kvh = (int)(o / per_kv);
    const int r = (int)(o % per_kv);
    gi = r % G;
    const int qi = r / G;  // position of the query tile in its kv head's list
    const int c = (n_kv < 8 && 8 % n_kv == 0) ? 8 / n_kv : 1;
    const int base = nq / c, extra = nq % c;  // sub-lists 0 .. extra - 1 hold base + 1 tiles, the others base
    int u, i;
    if (qi < extra * (base + 1)) {
        u = qi / (base + 1);
        i = qi % (base + 1);
    } else {
        u = extra + (qi - extra * (base + 1)) / base;
        i = (qi - extra * (base + 1)) % base;
    }
    qt_order = i * c + u;
}

// POS: the scale is > 0, so the block maximum can be taken on raw scores and the scale folded into the exponent's FMA.
// W: waves per workgroup; all W waves share each K/V tile in LDS.
// KSP: waves per 32-row query tile. With KSP = 1 each wave owns 32 query rows and walks every key block; with KSP = 2
// (short prompts, where the workgroups would not fill the chip) the two waves of a row tile take alternate 64-key
// blocks of each 128-key step and merge their (m, l, O) through LDS at the end, halving the chain of dependent blocks.
// ROPE: the reference's prompt path (rope_store, then attention_prefill on f32 q rows, llama_kernels.h:520-545, 660):
// query rows are read in f32 from the q|k|v rows, rotated for their position and rounded to half; the output is f32.
// SA: the IR self-attention's own [B][N][3E] rows read in place (0: no, the f16 operands of the attention entry
// points): 1 f32, 2 bf16, 3 f16 rows with head_dim p.hdv (a multiple of 8, at most HD) and heads p.head_stride
// elements apart. Q, K and V are rounded to half as they are loaded (K and V when the tile goes into LDS, so the
// prefetch stays in flight), columns past p.hdv read as zeros, and the output is written in the rows' type.
// SK (stream-K, W = 8, KSP = 1, SA = 0 only): the tile's key blocks ib0 .. ib1 - 1 only. When that is not the whole
// tile, the partial (m, l, O) goes to this range's slot (sk_slot) of p.sk_part and the tile's counter counts it in; the
// range that completes the count merges every slot of the tile and writes the output.
struct SkSegment {
    int32_t ib0, ib1;   // key blocks of this segment
    int32_t range;      // the workgroup's range
    int64_t start;      // the tile's first unit
    int64_t tile;       // the tile's index in the launch order (its counter)
};

template <int HD, bool POS, int W, bool ROPE, int KSP, int SA, bool SK>
__device__ __forceinline__ void prefill_tile(const PrefillParams & p, PrefillSmem<HD, KSP, prefill_dl<HD, W, KSP, SA>(), W> & sm,
                                             int kvh, int gi, int qt, const SkSegment & seg) {
    constexpr bool DL = prefill_dl<HD, W, KSP, SA>();
    constexpr int DLB = DL ? PrefillSmem<HD, KSP, true, W>::NBUF : 1;  // direct-to-LDS buffers
    constexpr int RB = KSP * kBK / 16;                              // 16-row blocks per chunk group of a step's tile
    constexpr int kWaves = W, RPW = W / KSP, kPrefillRows = 32 * RPW;  // RPW: 32-row query tiles per workgroup
    static_assert(W % KSP == 0, "whole row tiles");
    static_assert(!(ROPE && SA), "the rotated prompt path reads f16 operands");
    static_assert(!SK || (W == 8 && KSP == 1 && SA == 0), "stream-K: the 8-wave plan on the attention operands");
    constexpr int ES = SA == 1 ? 4 : 2;  // bytes per element of the q, k, v rows
    constexpr int NR = SA == 1 ? 2 : 1;  // 16-byte loads per 8 elements
    constexpr int KS = HD / 16;          // MFMA steps along head_dim for S^T
    constexpr int DT = HD / 32;          // 32-wide output tiles along head_dim
    constexpr int C8 = HD / 8;           // 16-byte chunks per key row
    constexpr int KB = KSP * kBK;        // keys per step (one 64-key block per wave of a row tile)
    constexpr int NB = (KB / 16) * (C8 / 4);  // (16 keys x 4 chunks) load blocks per step
    constexpr int NI = NB / kWaves;      // loads per thread per step, for each of K and V
    static_assert(NB % kWaves == 0, "whole loads per thread");
    constexpr int KP = PrefillSmem<HD, KSP>::KP, VP = PrefillSmem<HD, KSP>::VP;  // padded row pitches (not DL)

    const int G = p.group;
    const int h = kvh * G + gi;
    const int q0 = qt * kPrefillRows;
    // problem blockIdx.y of a batch: its own query, cache, output and lse blocks
    const int64_t bq = blockIdx.y * p.q_batch, bkv = blockIdx.y * p.kv_batch, bo = blockIdx.y * p.out_batch;
    float * const lse_g = p.lse ? p.lse + blockIdx.y * p.lse_batch : nullptr;

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform, in a scalar register
    const int rt = wave % RPW, kh = wave / RPW;  // the wave's row tile and its block of each step
    const int lane = threadIdx.x % kWave;
    const int l32 = lane % 32, hgrp = lane / 32;
    const int qrow = q0 + 32 * rt + l32;        // this lane's query row (chunk index)
    const int qpos = p.p0 + qrow;               // its cache position
    const int wave_last = p.p0 + q0 + 32 * rt + 31;  // the wave's last query position

    // keys this workgroup must visit
    const int last_row = min(q0 + kPrefillRows, p.n_q) - 1;
    const int kend = p.causal ? min(p.n_kv, p.p0 + last_row + 1) : p.n_kv;
    const int nblk = (kend + KB - 1) / KB;  // steps of KB keys
    const int ib0 = SK ? seg.ib0 : 0, ib1 = SK ? seg.ib1 : nblk;  // the steps of this call
    const int nb = ib1 - ib0;

    const int64_t hstride = SA ? p.head_stride : HD;  // elements between consecutive heads of a row
    const char * kg = reinterpret_cast<const char *>(p.k) + (bkv + (int64_t)kvh * hstride) * ES;
    const char * vg = reinterpret_cast<const char *>(p.v) + (bkv + (int64_t)kvh * hstride) * ES;
    // 8 elements of column col (a multiple of 8) from byte address a, as loaded (NR 16-byte words); columns past the
    // rows' head_dim load the row's last 8 instead (a valid address; half8() then gives zeros)
    auto ld8 = [&](const char * row, int col, u32x4 (&r)[NR]) __attribute__((always_inline)) {
        const int c = SA ? min(col, p.hdv - 8) : col;
#pragma unroll
        for (int j = 0; j < NR; j++) r[j] = load16(row + (int64_t)c * ES + 16 * j);
    };
    auto half8 = [&](const u32x4 (&r)[NR], int col) __attribute__((always_inline)) -> u32x4 {
        if constexpr (SA == 0 || SA == 3) {
            if (SA == 3 && col >= p.hdv) return u32x4{0u, 0u, 0u, 0u};
            return r[0];
        } else {
            float x[8];
            if constexpr (SA == 1) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    x[e] = __uint_as_float(r[0][e]);
                    x[4 + e] = __uint_as_float(r[NR - 1][e]);
                }
            } else {
                bf16x8_to_f32(r[0], x);
            }
            if (col >= p.hdv) return u32x4{0u, 0u, 0u, 0u};
            return to_half8(x);
        }
    };
    // tile-load mapping, block b = i * W + wave of 16 rows x 4 chunks (64 contiguous bytes per row):
    //   K: row 16 (b % 4) + lane % 16, chunk 4 (b / 4) + lane / 16 (16 lanes of one LDS write phase: 16 rows, one chunk)
    //   V: row 16 (b % 4) + 4 (lane / 16) + (lane % 16) / 4, chunk 4 (b / 4) + lane % 4 (16 lanes: 4 rows x 4 chunks)
    u32x4 kreg[NI][NR], vreg[NI][NR];
    auto krow = [&](int b) { return 16 * (b % (KB / 16)) + lane % 16; };
    auto kchunk = [&](int b) { return 4 * (b / (KB / 16)) + lane / 16; };
    auto vrow = [&](int b) { return 16 * (b % (KB / 16)) + 4 * (lane / 16) + (lane % 16) / 4; };
    auto vchunk = [&](int b) { return 4 * (b / (KB / 16)) + lane % 4; };
    auto load_tile_into = [&](int kb, u32x4 (&kr)[NI][NR], u32x4 (&vr)[NI][NR]) __attribute__((always_inline)) {
        if constexpr (DL) return;
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int b = i * kWaves + wave;
            const int kkey = min(kb + krow(b), p.n_kv - 1), vkey = min(kb + vrow(b), p.n_kv - 1);
            ld8(kg + (int64_t)kkey * p.kv_stride * ES, 8 * kchunk(b), kr[i]);
            ld8(vg + (int64_t)vkey * p.kv_stride * ES, 8 * vchunk(b), vr[i]);
        }
    };
    auto load_tile = [&](int kb) __attribute__((always_inline)) { load_tile_into(kb, kreg, vreg); };
    auto store_tile = [&](int buf) {
        if constexpr (DL) return;  // the DL plan has no register staging
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int b = i * kWaves + wave;
            *reinterpret_cast<u32x4 *>(&sm.k[buf][krow(b) * KP + 8 * kchunk(b)]) = half8(kreg[i], 8 * kchunk(b));
            *reinterpret_cast<u32x4 *>(&sm.v[buf][vrow(b) * VP + 8 * vchunk(b)]) = half8(vreg[i], 8 * vchunk(b));
        }
    };

    // DL: step kb's K and V tiles straight into LDS buffer buf, instruction j = i W + wave filling block j
    // Each lane's source bytes relative to the step's first key row are fixed for the kernel: 32-bit offsets from a
    // uniform step base (the loads' scalar-base form, no per-load address arithmetic); only a step that runs past the
    // cache clamps its rows to the last one.
    uint32_t dl_ko[DL ? NI : 1], dl_vo[DL ? NI : 1];
    int dl_row[DL ? NI : 1];
    const uint32_t row_bytes = (uint32_t)p.kv_stride * 2;
    if constexpr (DL) {
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const int j = i * kWaves + wave, rb = j % RB, cb = j / RB;  // this instruction's block
            dl_row[i] = 16 * rb + lane / 4;                             // the row this lane fills
            dl_ko[i] = dl_row[i] * row_bytes + 16 * (4 * cb + ((lane % 4) ^ (lane / 16)));
            dl_vo[i] = dl_row[i] * row_bytes + 16 * (4 * cb + lane % 4);
        }
    }
    auto issue_tile = [&](int kb, int buf) __attribute__((always_inline)) {
        if constexpr (DL) {
            const char * kst = kg + (int64_t)kb * row_bytes, * vst = vg + (int64_t)kb * row_bytes;
            const bool partial = kb + KB > p.n_kv;
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const int j = i * kWaves + wave;
                uint32_t ko = dl_ko[i], vo = dl_vo[i];
                if (__builtin_expect(partial, 0)) {
                    const uint32_t back = (uint32_t)max(kb + dl_row[i] - (p.n_kv - 1), 0) * row_bytes;
                    ko -= back;
                    vo -= back;
                }
                __builtin_amdgcn_global_load_lds(kst + ko, (__attribute__((address_space(3))) void *)&sm.k[buf][512 * j],
                                                 16, 0, 0);
                __builtin_amdgcn_global_load_lds(vst + vo, (__attribute__((address_space(3))) void *)&sm.v[buf][512 * j],
                                                 16, 0, 0);
            }
        }
    };

    // Q^T operand: lane holds Q[qrow][16 ks + 8 hgrp .. + 8]
    half8_t qb[KS];
    if constexpr (ROPE) {
        // the rotary frequencies into LDS: compile-time indices make scalar loads of the kernel arguments, one LDS
        // store each (a per-lane index into the arguments would be a vector load, waited for one by one)
        __shared__ float s_freq[HD / 2];
        float fr = 0.f;
#pragma unroll
        for (int i = 0; i < HD / 2; i++)
            if (threadIdx.x == i) fr = p.rope_freq[i];
        if (threadIdx.x < HD / 2) s_freq[threadIdx.x] = fr;
        __syncthreads();
        float x[KS][8] = {};
        if (qrow < p.n_q) {
            const float * qp = p.qkv + bq + (int64_t)qrow * p.q_stride + (int64_t)h * HD + 8 * hgrp;
#pragma unroll
            for (int ks = 0; ks < KS; ks++) load8f(qp + 16 * ks, x[ks]);
            rope_rotate<KS, 16>(x, 8 * hgrp, p.rope_mode, [&](int i) {
                float sn, cs;
                sincos_rope((float)qpos * s_freq[i], sn, cs);
                return make_float2(cs, sn);
            });
        }
#pragma unroll
        for (int ks = 0; ks < KS; ks++) qb[ks] = as_half8(to_half8(x[ks]));
    }
    // f16/f32/bf16 query rows: loaded by every lane (rows past the chunk read its last row, a valid address) and turned
    // into the operand only once the first tile's loads are out, so that waiting for the query leaves them in flight
    u32x4 qr[ROPE ? 1 : KS][NR];
    auto q_operand = [&]() __attribute__((always_inline)) {
        if constexpr (!ROPE) {
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                const int col = 16 * ks + 8 * hgrp;
                const u32x4 hq = half8(qr[ks], col);
                qb[ks] = as_half8(qrow < p.n_q ? hq : u32x4{0u, 0u, 0u, 0u});
            }
        }
    };
    if constexpr (!ROPE) {
        const char * qp = reinterpret_cast<const char *>(p.q) +
                          (bq + (int64_t)min(qrow, p.n_q - 1) * p.q_stride + (int64_t)h * hstride) * ES;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) ld8(qp, 16 * ks + 8 * hgrp, qr[ks]);
    }
    if constexpr (DL) {
        // the query went out first; steps 0 and 1 follow straight into LDS (the wait for the query leaves them in flight)
        if (nb > 0) issue_tile(ib0 * KB, 0);
#pragma unroll
        for (int a = 1; a < DLB - 1; a++)
            if (nb > a) issue_tile((ib0 + a) * KB, a);
        if constexpr (!ROPE) {
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
#pragma unroll
                for (int j = 0; j < NR; j++) asm volatile("" : "+v"(qr[ks][j])::"memory");
        }
        q_operand();
    } else if (nb > 0 && W == 4) {
        // the short-prompt plans: steps 0 and 1 go out together (step 1 into registers of its own, unconditionally:
        // past the cache its rows are clamped to the last one and never used), so the prologue waits for one round
        // trip instead of two (the 8-wave plan's long chunks keep the plain order)
        u32x4 k1[NI][NR], v1[NI][NR];
        load_tile(ib0 * KB);
        __builtin_amdgcn_sched_barrier(0);
        load_tile_into((ib0 + 1) * KB, k1, v1);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (!ROPE) {  // the query is used from here on (the compiler would otherwise hoist its use above)
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
#pragma unroll
                for (int j = 0; j < NR; j++) asm volatile("" : "+v"(qr[ks][j])::"memory");
        }
        q_operand();
        store_tile(0);
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int j = 0; j < NR; j++) {
                kreg[i][j] = k1[i][j];
                vreg[i][j] = v1[i][j];
            }
    } else if (nb > 0) {
        load_tile(ib0 * KB);
        if constexpr (!ROPE) {
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
#pragma unroll
                for (int j = 0; j < NR; j++) asm volatile("" : "+v"(qr[ks][j])::"memory");
        }
        q_operand();
        store_tile(0);
        if (nb > 1) load_tile((ib0 + 1) * KB);
    } else {
        q_operand();
    }
    // Wait here for the query operand (and the prologue's loads): inside the loop the only loads in flight are then the
    // prefetch of a later block, whose registers the block's math does not read, so no wait inside the loop has to
    // drain them (a wait the compiler would otherwise place before the first product, serializing loads and math).
    if (!DL) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

    float16_t o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int v = 0; v < 16; v++) o[dt][v] = 0.f;
    float m_run = kNegInf, l_run = 0.f;  // reference maximum (base 2, scaled) and row sum of this lane's keys
    float nm_use = 0.f;                   // -m_run (0 while m_run = -inf)

    // per-lane LDS read bases (halves); everything else is a compile-time offset
    const int k_base = l32 * KP + 8 * hgrp;  // K[32 mt + l32][16 kk + 8 hgrp]
    // transposing read: lane a of 16-lane group c supplies V[4 hgrp + a / 4][16 (c % 2) + 4 (a % 4)] (+ 16 u + 8 s8 rows,
    // + 32 dt columns) and receives V[rows + 0..3][32 dt + lane % 32]
    const int v_base = (4 * hgrp + (lane % 16) / 4) * VP + 16 * ((lane / 16) % 2) + 4 * (lane % 4);
    // DL read bases (halves): K chunk 2 kk + hgrp of row l32 in block (kk / 2, l32 / 16), one base per kk % 2; V as the
    // padded read with 64-byte rows
    int dl_k[2];
#pragma unroll
    for (int b = 0; b < 2; b++) dl_k[b] = 512 * (l32 / 16) + 32 * (l32 % 16) + 8 * ((2 * b + hgrp) ^ ((l32 % 16) / 4));
    const int dl_v = (4 * hgrp + (lane % 16) / 4) * 32 + 16 * ((lane / 16) % 2) + 4 * (lane % 4);

    for (int jb = 0; jb < nb; jb++) {
        const int ib = ib0 + jb;
        const int kb = ib * KB + kh * kBK;  // this wave's block of the step
        int buf;
        if constexpr (DL) {
            buf = jb % DLB;
            // this wave's loads of step ib are complete (those of up to DLB - 2 later steps may be in flight), then
            // every wave's are: step ib is in buffer `buf`, and the buffer refilled below was last read in step ib - 1
            const int later = min(DLB - 2, nb - 1 - jb);
            static_for<0, DLB - 1>([&](auto R) __attribute__((always_inline)) {
                constexpr int r = decltype(R)::value;
                if (later == r) __builtin_amdgcn_s_waitcnt(0x0F70 | (r * 2 * NI));  // vmcnt(r steps' loads)
            });
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (jb + DLB - 1 < nb) issue_tile((ib + DLB - 1) * KB, (jb + DLB - 1) % DLB);
        } else {
            buf = jb & 1;
            __syncthreads();  // step ib is in LDS buffer `buf`; buffer buf ^ 1 is no longer read
            if (jb + 1 < nb) {
                store_tile(buf ^ 1);
                if (jb + 2 < nb) load_tile((ib + 2) * KB);
            }
        }
        if (kb >= kend || (p.causal && kb > wave_last)) continue;  // every key of the block is past this wave's rows
        const half_t * ks_ = DL ? sm.k[buf] : sm.k[buf] + kh * kBK * KP;
        const half_t * vs_ = DL ? sm.v[buf] : sm.v[buf] + kh * kBK * VP;

        // S^T = K Q^T: 2 tiles of 32 keys. The K operand of step i + 1 is read before the product of step i, so each
        // product waits only for reads issued one product earlier.
        float16_t sc[2];
        {
            constexpr int NS = 2 * KS;  // products
            // (kk, mt) order: the two key tiles' products alternate, so consecutive products are independent (cfg5 +0.8 %)
            constexpr int RA = 1;  // reads in flight ahead of the product (2 or 3 measured no faster)
            u32x4 ka[RA + 1];
            // DL: K[32 mt + l32][16 kk + 8 hgrp] in block (kk / 2, 2 mt + l32 / 16), at dl_k[kk % 2] + the block's offset
            auto kread = [&](int i) {
                return *reinterpret_cast<const u32x4 *>(ks_ + k_base + 32 * (i % 2) * KP + 16 * (i / 2));
            };
#pragma unroll
            for (int v = 0; v < 16; v++) sc[0][v] = sc[1][v] = 0.f;
            u32x4 kf[DL ? NS : 1];
            const uint32_t kb0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) half_t *)ks_;
            const uint32_t ka0 = kb0 + 2 * (dl_k[0] + 2048 * kh), ka1 = kb0 + 2 * (dl_k[1] + 2048 * kh);
            if constexpr (DL) {
                // every K fragment of the block in flight at once (inline asm, as the V reads below), each product
                // waiting for its own: LDS reads complete in order, so product i needs lgkmcnt(NS - 1 - i)
                static_assert(NS <= 16, "lgkmcnt counts at most 15 later reads");
                static_for<0, NS>([&](auto I) __attribute__((always_inline)) {
                    constexpr int i = decltype(I)::value;
                    constexpr int off = 2 * (512 * RB * (i / 4) + 1024 * (i % 2));
                    const uint32_t a = (i / 2) % 2 ? ka1 : ka0;
                    u32x4 t;
                    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(t) : "v"(a), "i"(off));
                    kf[i] = t;
                });
                static_for<0, NS>([&](auto I) __attribute__((always_inline)) {
                    constexpr int i = decltype(I)::value;
                    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(kf[i]) : "i"(NS - 1 - i));
                    sc[i % 2] = mfma32x32x16(as_half8(kf[i]), qb[i / 2], sc[i % 2]);
                    __builtin_amdgcn_sched_barrier(0);  // each product right behind its wait
                });
            } else {
#pragma unroll
                for (int i = 0; i < RA; i++) ka[i] = kread(i);
#pragma unroll
                for (int i = 0; i < NS; i++) {
                    if (i + RA < NS) ka[(i + RA) % (RA + 1)] = kread(i + RA);
                    const int mt = i % 2, kk = i / 2;
                    sc[mt] = mfma32x32x16(as_half8(ka[i % (RA + 1)]), qb[kk], sc[mt]);
                }
            }
        }
        // The mask only where a block crosses the diagonal or the end of the cache (a wave-uniform branch).
        const bool need_mask = (p.causal && kb + kBK - 1 > p.p0 + q0 + 32 * rt) || kb + kBK > p.n_kv;
        const float c = p.scale_log2;
        // DL: the first VA products' transposing V reads go out now, so that the softmax below covers their latency
        // (no other LDS access comes between them and the products' waits, which count them as before)
        constexpr int VA = 2;  // products whose V reads are in flight ahead of the one multiplied (1: -0.6 %, 3: -0.5 %)
        short4_t vr[VA + 1][2];
        const uint32_t va = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) half_t *)vs_ +
                            2 * (dl_v + 2048 * kh);
        auto vread_dl = [&](auto TC) __attribute__((always_inline)) {
            constexpr int t = decltype(TC)::value;
            constexpr int off = 2 * (512 * (RB * (t % DT) + t / DT));
            short4_t r0, r1;
            asm volatile("ds_read_b64_tr_b16 %0, %2 offset:%3\n\tds_read_b64_tr_b16 %1, %2 offset:%4"
                         : "=&v"(r0), "=&v"(r1)
                         : "v"(va), "i"(off), "i"(off + 512));
            vr[t % (VA + 1)][0] = r0;
            vr[t % (VA + 1)][1] = r1;
        };
        if constexpr (DL) static_for<0, VA>(vread_dl);
        if (need_mask) {
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int key = kb + 32 * mt + 8 * (v / 4) + 4 * hgrp + (v % 4);
                    const bool hide = key >= p.n_kv || (p.causal && key > qpos);
                    sc[mt][v] = hide ? kNegInf : (POS ? sc[mt][v] : sc[mt][v] * c);
                }
        } else if constexpr (!POS) {
#pragma unroll
            for (int mt = 0; mt < 2; mt++)
#pragma unroll
                for (int v = 0; v < 16; v++) sc[mt][v] *= c;
        }
        // Probabilities at the kept reference maximum m_run, straight to half (the P^T operand: step u takes values
        // 8 (u % 2) .. + 8 of score tile u / 2), and their per-lane sum on v_dot2_f32_f16, in two halves of 32 keys. The block's maximum is not
        // computed on this path: a sum above 2^8 (some probability above 2^8, or an overflow to inf) or a row that has
        // no reference yet sends the wave to the exact update below, which moves m_run to the running maximum, rescales
        // O and l, and recomputes the block. While the sum stays below 2^8 every probability is below 2^8, well inside
        // half; a block whose scores sit a few units (base 2) above the reference takes the exact update once, so the
        // common path is the exponentials alone (cfg5: 16 v_max3 and a cross-lane step fewer per block).
        half8_t pb[4];
        // score tiles H0 .. H1 - 1 (32 keys each): their probabilities at a valid reference, added to l. With
        // kSplitHalves the second half runs between the P V products of the first (the matrix cores busy with those
        // while the vector ALUs compute these); an exact update there rescales O with the first half's products
        // already in it, as for any earlier block.
        auto settle = [&](auto H0C, auto H1C) __attribute__((always_inline)) {
            constexpr int H0 = decltype(H0C)::value, H1 = decltype(H1C)::value;  // score tiles H0 .. H1 - 1
            float bs;
            auto probs = [&]() __attribute__((always_inline)) {
#pragma unroll
                for (int u = 2 * H0; u < 2 * H1; u++)
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        const float x = sc[u / 2][8 * (u % 2) + e];
                        pb[u][e] = (half_t)exp2_fast(POS ? __builtin_fmaf(x, c, nm_use) : x + nm_use);
                    }
                bs = 0.f;
#pragma unroll
                for (int u = 2 * H0; u < 2 * H1; u++)
#pragma unroll
                    for (int e = 0; e < 8; e += 2) bs = __builtin_amdgcn_fdot2(half2_t{pb[u][e], pb[u][e + 1]}, kOnes2, bs, false);
            };
            probs();
            if (__builtin_amdgcn_ballot_w64(bs > kProbSumMax || m_run == kNegInf)) {
                float bmax = kNegInf;
#pragma unroll
                for (int mt = H0; mt < H1; mt++)
#pragma unroll
                    for (int v = 0; v < 16; v++) bmax = fmaxf(bmax, sc[mt][v]);
                bmax = xor32_max(bmax);
                const float bm = POS ? bmax * c : bmax;
                const float m_new = fmaxf(m_run, bm);
                const float corr = m_new == kNegInf ? 1.f : exp2_fast(m_run - m_new);
                m_run = m_new;
                nm_use = m_new == kNegInf ? 0.f : -m_new;  // no visible key yet: every exponent below is 2^-inf = 0
                l_run *= corr;
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
#pragma unroll
                    for (int v = 0; v < 16; v++) o[dt][v] *= corr;
                probs();
            }
            l_run += bs;
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        // Split at head dims 64 and 256 (Qwen2.5-0.5B 4096-token prompt 352 -> 366 TFLOP/s, a head-dim-256 2048-token
        // prompt 108 -> 125); at 128 both halves come first (cfg5 1013 -> 997 split).
        constexpr bool kSplitHalves = HD != 128;
        if constexpr (kSplitHalves) settle(I0{}, I1{});
        else settle(I0{}, I2{});

        // O^T += V^T P^T: 4 steps of 16 keys; step u takes values 8 (u % 2) .. + 8 of score tile u / 2, which are keys
        // 16 u + 8 (e / 4) + 4 hgrp + e % 4 for e = 0..7; two transposing reads fetch the same keys of V. The reads of
        // product i + 1 are issued before product i.
        {
            constexpr int NP = 4 * DT;  // products: (u, dt) in order
            short4_t vt[2][2];
            auto vread = [&](int i, short4_t (&t)[2]) {
                const int u = i / DT, dt = i % DT;
#pragma unroll
                for (int s8 = 0; s8 < 2; s8++) {
                    const half_t * a = vs_ + v_base + (16 * u + 8 * s8) * VP + 32 * dt;
                    t[s8] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t *)a);
                }
            };
            auto pv = [&](int i, const short4_t (&t)[2]) __attribute__((always_inline)) {
                const short4_t lo = t[0], hi = t[1];
                const half8_t a = __builtin_bit_cast(half8_t, (short __attribute__((ext_vector_type(8)))){
                    lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
                o[i % DT] = mfma32x32x16(a, pb[i / DT], o[i % DT]);
            };
            if constexpr (DL) {
                // The transposing reads as inline asm with their own waits: the compiler cannot tell the intrinsic's
                // LDS read from the direct loads still writing another buffer, and would drain them (vmcnt(0)) before
                // the first read of every block. Rows 16 u + 8 s8 + 4 hgrp + (lane % 16) / 4 of block (dt, u).
                // (the reads of products 0 .. VA - 1 went out before the softmax)
                static_for<0, NP + VA>([&](auto I) __attribute__((always_inline)) {
                    constexpr int t = decltype(I)::value;
                    if constexpr (t >= VA && t < NP) vread_dl(I);
                    if constexpr (t >= VA) {  // product j: its two reads done, those of the later products in flight
                        constexpr int j = t - VA;
                        if constexpr (kSplitHalves && j == NP / 2) settle(I1{}, I2{});
                        constexpr int later = 2 * ((t < NP - 1 ? t : NP - 1) - j);
                        asm volatile("s_waitcnt lgkmcnt(%2)"
                                     : "+v"(vr[j % (VA + 1)][0]), "+v"(vr[j % (VA + 1)][1])
                                     : "i"(later));
                        pv(j, vr[j % (VA + 1)]);
                    }
                });
            } else {
                vread(0, vt[0]);
#pragma unroll
                for (int i = 0; i < NP / 2; i++) {
                    vread(i + 1, vt[(i + 1) & 1]);
                    pv(i, vt[i & 1]);
                }
                if constexpr (kSplitHalves) settle(I1{}, I2{});
#pragma unroll
                for (int i = NP / 2; i < NP; i++) {
                    if (i + 1 < NP) vread(i + 1, vt[(i + 1) & 1]);
                    pv(i, vt[i & 1]);
                }
            }
        }
    }

    l_run = xor32_add(l_run);
    if constexpr (KSP > 1) {
        // ---- the KSP waves of a row tile merge their (m, l, O): waves kh > 0 leave theirs in LDS (the tiles are no
        // longer read), the wave kh = 0 folds them in ----
        constexpr int XS = DT * 16 + 2;  // floats per lane
        static_assert((int64_t)RPW * (KSP - 1) * kWave * XS * 4 <= (int64_t)sizeof(sm), "merge scratch fits the tiles");
        float * xs = reinterpret_cast<float *>(&sm);
        __syncthreads();
        if (kh > 0) {
            float * d = xs + ((rt * (KSP - 1) + kh - 1) * kWave + lane) * XS;
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int v = 0; v < 16; v++) d[16 * dt + v] = o[dt][v];
            d[16 * DT] = m_run;
            d[16 * DT + 1] = l_run;
        }
        __syncthreads();
        if (kh > 0) return;
#pragma unroll
        for (int j = 0; j < KSP - 1; j++) {
            const float * d = xs + ((rt * (KSP - 1) + j) * kWave + lane) * XS;
            const float m1 = d[16 * DT], l1 = d[16 * DT + 1];
            const float mn = fmaxf(m_run, m1);
            const float w0 = m_run == kNegInf ? 0.f : exp2_fast(m_run - mn);
            const float w1 = m1 == kNegInf ? 0.f : exp2_fast(m1 - mn);
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int v = 0; v < 16; v++) o[dt][v] = o[dt][v] * w0 + d[16 * dt + v] * w1;
            l_run = l_run * w0 + l1 * w1;
            m_run = mn;
        }
    }

    if constexpr (SK) {
        if (ib0 != 0 || ib1 != nblk) {
            // ---- part of a tile: its (m, l, O) into this range's slot with device-scope stores, which are complete
            // before the tile's counter counts it in; the range that brings the count to the tile's number of ranges
            // folds every slot of the tile, in range order (its own read back too, so that the result does not depend
            // on which range finished last), and writes the output ----
            constexpr int J = HD / 2 + 2;  // floats per lane: O, m, l
            __shared__ int s_sk_last;
            const int64_t total = p.sk_total;
            const int32_t R = p.sk_ranges;
            auto lane_slot = [&](int64_t slot) {
                return p.sk_part + slot * kPrefillSlotFloats<HD> + (int64_t)wave * J * kWave + lane;
            };
            const int64_t own = sk_slot(total, R, seg.range, seg.start);
            {
                float * d = lane_slot(own);
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
#pragma unroll
                    for (int v = 0; v < 16; v++) put_f32(d + (16 * dt + v) * kWave, o[dt][v]);
                put_f32(d + (J - 2) * kWave, m_run);
                put_f32(d + (J - 1) * kWave, l_run);
            }
            const int32_t r_first = sk_range_of(total, R, seg.start), r_last = sk_range_of(total, R, seg.start + nblk - 1);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            if (threadIdx.x == 0) {
                const uint32_t done =
                    __hip_atomic_fetch_add(p.sk_counters + seg.tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_sk_last = done == (uint32_t)(r_last - r_first);
            }
            __syncthreads();
            if (!s_sk_last) return;
            __builtin_amdgcn_s_waitcnt(0);
            m_run = kNegInf;
            l_run = 0.f;
#pragma unroll
            for (int dt = 0; dt < DT; dt++)
#pragma unroll
                for (int v = 0; v < 16; v++) o[dt][v] = 0.f;
            for (int32_t r = r_first; r <= r_last; r++) {
                const float * d = lane_slot(sk_slot(total, R, r, seg.start));
                float x[DT][16];
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
#pragma unroll
                    for (int v = 0; v < 16; v++) x[dt][v] = get_f32(d + (16 * dt + v) * kWave);
                const float m1 = get_f32(d + (J - 2) * kWave), l1 = get_f32(d + (J - 1) * kWave);
                const float mn = fmaxf(m_run, m1);
                const float w0 = m_run == kNegInf ? 0.f : exp2_fast(m_run - mn);
                const float w1 = m1 == kNegInf ? 0.f : exp2_fast(m1 - mn);
#pragma unroll
                for (int dt = 0; dt < DT; dt++)
#pragma unroll
                    for (int v = 0; v < 16; v++) o[dt][v] = o[dt][v] * w0 + x[dt][v] * w1;
                l_run = l_run * w0 + l1 * w1;
                m_run = mn;
            }
            if (threadIdx.x == 0) __hip_atomic_store(p.sk_counters + seg.tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }

    // ---- normalize and store: lane holds O[qrow][32 dt + 8 (v / 4) + 4 hgrp + v % 4] ----
    if (qrow < p.n_q) {
        const float inv = 1.f / l_run;
        const int64_t off = (int64_t)qrow * p.out_stride + (int64_t)h * hstride + 4 * hgrp;
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
#pragma unroll
            for (int gq = 0; gq < 4; gq++) {
                if constexpr (SA) {
                    const int col = 32 * dt + 8 * gq + 4 * hgrp;
                    if (col >= p.hdv) continue;
                    float r[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) r[e] = o[dt][4 * gq + e] * inv;
                    if constexpr (SA == 1) {
                        *reinterpret_cast<float4_t *>(p.out32 + bo + off + 32 * dt + 8 * gq) = float4_t{r[0], r[1], r[2], r[3]};
                    } else if constexpr (SA == 2) {
                        *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(p.out) + bo + off + 32 * dt + 8 * gq) =
                            u32x2{(uint32_t)to_bf16(r[0]) | ((uint32_t)to_bf16(r[1]) << 16),
                                  (uint32_t)to_bf16(r[2]) | ((uint32_t)to_bf16(r[3]) << 16)};
                    } else {
                        *reinterpret_cast<half4_t *>(p.out + bo + off + 32 * dt + 8 * gq) =
                            half4_t{(half_t)r[0], (half_t)r[1], (half_t)r[2], (half_t)r[3]};
                    }
                } else if constexpr (ROPE) {
                    float4_t r;
#pragma unroll
                    for (int e = 0; e < 4; e++) r[e] = o[dt][4 * gq + e] * inv;
                    *reinterpret_cast<float4_t *>(p.out32 + bo + off + 32 * dt + 8 * gq) = r;
                } else {
                    half4_t r;
#pragma unroll
                    for (int e = 0; e < 4; e++) r[e] = (half_t)(o[dt][4 * gq + e] * inv);
                    *reinterpret_cast<half4_t *>(p.out + bo + off + 32 * dt + 8 * gq) = r;
                }
            }
        if (lse_g && hgrp == 0) lse_g[(int64_t)qrow * p.n_head + h] = (m_run + log2_fast(l_run)) * kLn2;
    }
}

template <int HD, bool POS, int W, bool ROPE, int KSP, int SA>
__global__ __launch_bounds__(W * kWave) __attribute__((amdgpu_waves_per_eu(KSP == 1 && HD <= 128 ? 2 : 1, KSP == 1 && HD <= 128 ? 2 : 1)))
void prefill_kernel(PrefillParams p) {
    __shared__ PrefillSmem<HD, KSP, prefill_dl<HD, W, KSP, SA>(), W> sm;
    // ---- work item: each XCD a contiguous range of a kv-head-major order, heavy query tiles first ----
    const uint32_t n_work = (uint32_t)p.n_qtiles * p.n_head;
    int kvh, gi, qt_order;
    prefill_work(xcd_remap(blockIdx.x, n_work), p.n_qtiles, p.group, p.n_head_kv, kvh, gi, qt_order);
    const int qt = p.causal ? p.n_qtiles - 1 - qt_order : qt_order;
    prefill_tile<HD, POS, W, ROPE, KSP, SA, false>(p, sm, kvh, gi, qt, SkSegment{});
}

// Stream-K: p.sk_ranges workgroups (one per CU), each over an equal range of the (tile, key block) units, so that no CU
// idles while another finishes a tile (a 2048-row chunk of 28 heads is 224 equal tiles for 256 CUs; a causal prompt's
// tiles differ in length). Workgroup b runs on XCD b % 8 (workgroups are dealt to the XCDs round-robin) and takes range
// (b % 8) R / 8 + b / 8: each XCD walks one contiguous eighth of the kv-head-major order, so its L2 streams the K/V of
// few kv heads. R is a multiple of 8 (the host's plan), so every range is dealt exactly once.
template <int HD, bool POS, bool ROPE>
__global__ __launch_bounds__(8 * kWave) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_sk_kernel(PrefillParams p) {
    __shared__ PrefillSmem<HD, 1, prefill_dl<HD, 8, 1, 0>(), 8> sm;
    const int32_t R = p.sk_ranges;
    const int32_t r = (int32_t)(blockIdx.x % 8) * (R / 8) + (int32_t)(blockIdx.x / 8);
    const int64_t total = p.sk_total, lo = sk_lo(total, R, r), hi = sk_lo(total, R, r + 1);
    int64_t per_kv = 0;
    for (int q = 0; q < p.n_qtiles; q++) per_kv += prefill_tile_blocks(q, p.n_q, p.p0, p.n_kv, p.causal);
    per_kv *= p.group;
    for (int64_t x = lo; x < hi;) {
        const SkTile t = sk_locate(x, per_kv, p.group, p.n_qtiles, p.n_q, p.p0, p.n_kv, p.causal);
        SkSegment seg;
        seg.ib0 = (int32_t)(x - t.start);
        seg.ib1 = (int32_t)(hi - t.start < t.nblk ? hi - t.start : t.nblk);
        seg.range = r;
        seg.start = t.start;
        seg.tile = ((int64_t)t.kvh * p.n_qtiles + t.qt) * p.group + t.gi;
        __syncthreads();  // the previous segment's waves are done with the LDS tiles
        prefill_tile<HD, POS, 8, ROPE, 1, 0, true>(p, sm, t.kvh, t.gi, t.qt, seg);
        x = t.start + seg.ib1;
    }
}

}  // namespace

// Waves per workgroup: 8 (256 query rows, one workgroup per CU, every K/V tile shared by all 8 waves) or 4 (128 rows,
// two workgroups per CU), whichever leaves the least work on the busiest CU: rounds of workgroups per CU times the
// rows of one, with the 8-wave tile's rows weighted 0.8 for its shared K/V tiles (measured: a 2048-row chunk of 28
// heads runs ~20 % faster as 224 workgroups of 8 waves than as 448 of 4; 96 problems of 577 rows run 1.6x faster as
// 480 workgroups of 4 waves than as 288 of 8, of which 32 would wait for a second round). n_head counts every
// (batch, head) problem of the launch.
// When even the 128-row workgroups would leave half the CUs idle and there are at least 512 keys, the plan is 64-row
// workgroups of 4 waves, two per row tile splitting the key blocks (KSP = 2): one round on the CUs, half the chain of
// dependent blocks per wave, but twice the K/V bytes through the load path per step. Measured: the Qwen2.5-0.5B
// 512-token prompt 12.0 -> 10.8 us per layer, a 16-row chunk at 30k keys (28 heads, hd 128) 629 -> 559 us; a
// 300-token Llama-3-8B prompt (5 blocks) ran 7 % slower split, hence the 512-key floor. At head dim 64 (half the
// K/V bytes per key) and with the 128-row workgroups filling at most a quarter of the CUs, the split pays from 128
// keys: Qwen2.5-0.5B prompts of 128, 256 and 384 tokens 6.06 -> 5.9, 8.2 -> 7.5 and 10.0 -> 9.3 us per layer (a
// 448-token prompt of 20 heads, 80 such workgroups, ran 9 % slower split).
// Plans: 8 = 8 waves x 32 rows, 4 = 4 waves x 32 rows, 2 = 4 waves over 2 row tiles x 2 key halves (64 rows).
constexpr int kCUs = 256;
int prefill_plan(int n_q, int n_head, int n_kv, int head_dim, int forced) {
    // head dim 256: 4 waves of 32 rows, one workgroup per CU (the K/V double buffer takes 141 KB of LDS; 8 waves or
    // the key-split plan would not fit the registers or the LDS)
    if (head_dim == 256) return 4;
    if (forced == 2 || forced == 4 || forced == 8) return forced;
    const int64_t wg8 = (int64_t)((n_q + 255) / 256) * n_head, wg4 = (int64_t)((n_q + 127) / 128) * n_head;
    if (2 * wg4 <= kCUs && n_kv >= 8 * kBK) return 2;
    if (4 * wg4 <= kCUs && head_dim <= 64 && n_kv >= 2 * kBK) return 2;
    const double cost8 = (double)((wg8 + kCUs - 1) / kCUs) * 256 * 0.8;
    const double cost4 = (double)((wg4 + kCUs - 1) / kCUs) * 128;
    return cost8 <= cost4 ? 8 : 4;
}

int prefill_rows_per_workgroup(int n_q, int n_head, int n_kv, int head_dim, int forced) {
    return 32 * prefill_plan(n_q, n_head, n_kv, head_dim, forced);
}

// ---- the IR self-attention's operand packing (row f4): one thread per 8 consecutive padded head dims ----
__global__ __launch_bounds__(256) void self_attn_pack_kernel(SelfAttnPackParams p) {
    const int H = p.heads, hd = p.hd, hdp = p.hdp, E = H * hd;
    const int64_t per_row = (int64_t)3 * H * (hdp / 8);  // 8-wide groups of q, k and v per row
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= p.rows * per_row) return;
    const int64_t row = i / per_row;
    int r = (int)(i % per_row);
    const int part = r / (H * (hdp / 8));  // 0 q, 1 k, 2 v
    r %= H * (hdp / 8);
    const int h = r / (hdp / 8), d0 = 8 * (r % (hdp / 8));
    float x[8];
    const int64_t src = row * 3 * E + (int64_t)part * E + (int64_t)h * hd + d0;
    if (hd % 8 == 0) {  // uniform: whole 8-wide groups, 16-byte (f16/bf16) or 2 x 16-byte (f32) loads, or padding
        if (d0 < hd) {
            if (p.dtype == 0) {
                load8f(static_cast<const float *>(p.qkv) + src, x);
            } else {
                const u32x4 v = load16(static_cast<const uint16_t *>(p.qkv) + src);
                const uint16_t * u = reinterpret_cast<const uint16_t *>(&v);
#pragma unroll
                for (int e = 0; e < 8; e++)
                    x[e] = p.dtype == 1 ? (float)__builtin_bit_cast(half_t, u[e]) : __uint_as_float((uint32_t)u[e] << 16);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] = 0.f;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
            x[e] = 0.f;
            if (d0 + e < hd) {
                if (p.dtype == 1) x[e] = (float)static_cast<const half_t *>(p.qkv)[src + e];
                else if (p.dtype == 2) x[e] = __uint_as_float((uint32_t)static_cast<const uint16_t *>(p.qkv)[src + e] << 16);
                else x[e] = static_cast<const float *>(p.qkv)[src + e];
            }
        }
    }
    if (part == 0) {
        float * dst = p.q + row * H * hdp + (int64_t)h * hdp + d0;
        *reinterpret_cast<float4_t *>(dst) = float4_t{x[0], x[1], x[2], x[3]};
        *reinterpret_cast<float4_t *>(dst + 4) = float4_t{x[4], x[5], x[6], x[7]};
    } else {
        *reinterpret_cast<u32x4 *>(p.kv + row * 2 * H * hdp + (int64_t)(part - 1) * H * hdp + (int64_t)h * hdp + d0) = to_half8(x);
    }
}

// one thread per 4 consecutive outputs of a head (head_dim a multiple of 4), else per output

__global__ __launch_bounds__(256) void self_attn_unpack_kernel(SelfAttnUnpackParams p) {
    const int H = p.heads, hd = p.hd, E = H * hd;
    const int V = hd % 4 == 0 ? 4 : 1;
    const int64_t i = (blockIdx.x * (int64_t)blockDim.x + threadIdx.x) * V;
    if (i >= p.rows * E) return;
    const int64_t row = i / E;
    const int c = (int)(i % E), h = c / hd, d = c % hd;
    const float * o = p.o + row * H * p.hdp + (int64_t)h * p.hdp + d;
    if (V == 4) {
        const float4_t v = *reinterpret_cast<const float4_t *>(o);
        if (p.dtype == 1) {
            *reinterpret_cast<half4_t *>(static_cast<half_t *>(p.y) + i) = half4_t{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
        } else if (p.dtype == 2) {
            const u32x2 w = {(uint32_t)to_bf16(v[0]) | ((uint32_t)to_bf16(v[1]) << 16), (uint32_t)to_bf16(v[2]) | ((uint32_t)to_bf16(v[3]) << 16)};
            *reinterpret_cast<u32x2 *>(static_cast<uint16_t *>(p.y) + i) = w;
        } else {
            *reinterpret_cast<float4_t *>(static_cast<float *>(p.y) + i) = v;
        }
        return;
    }
    const float v = o[0];
    if (p.dtype == 1) static_cast<half_t *>(p.y)[i] = (half_t)v;
    else if (p.dtype == 2) static_cast<uint16_t *>(p.y)[i] = to_bf16(v);
    else static_cast<float *>(p.y)[i] = v;
}

hipError_t launch_self_attn_pack(const SelfAttnPackParams & p, hipStream_t stream) {
    const int64_t n = p.rows * 3 * p.heads * (p.hdp / 8);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(self_attn_pack_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_self_attn_unpack(const SelfAttnUnpackParams & p, hipStream_t stream) {
    const int64_t n = p.rows * p.heads * p.hd / (p.hd % 4 == 0 ? 4 : 1);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(self_attn_unpack_kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, stream, p);
    return hipGetLastError();
}

template <int HD, bool POS, bool ROPE, int SA>
void launch_prefill_r(const PrefillParams & p, int plan, int n_batch, hipStream_t stream) {
    if constexpr (SA == 0) {
        if (p.sk_ranges > 0) {  // planned by the caller for plan 8 and one problem only
            hipLaunchKernelGGL((prefill_sk_kernel<HD, POS, ROPE>), dim3((uint32_t)p.sk_ranges), dim3(8 * kWave), 0, stream, p);
            return;
        }
    }
    const dim3 grid((uint32_t)p.n_qtiles * p.n_head, (uint32_t)n_batch);
    if (plan == 8) hipLaunchKernelGGL((prefill_kernel<HD, POS, 8, ROPE, 1, SA>), grid, dim3(8 * kWave), 0, stream, p);
    else if (plan == 4) hipLaunchKernelGGL((prefill_kernel<HD, POS, 4, ROPE, 1, SA>), grid, dim3(4 * kWave), 0, stream, p);
    else hipLaunchKernelGGL((prefill_kernel<HD, POS, 4, ROPE, 2, SA>), grid, dim3(4 * kWave), 0, stream, p);
}

template <int HD, bool POS>
void launch_prefill_t(const PrefillParams & p, int plan, int n_batch, int sa, hipStream_t stream) {
    if (sa == 1) launch_prefill_r<HD, POS, false, 1>(p, plan, n_batch, stream);
    else if (sa == 2) launch_prefill_r<HD, POS, false, 2>(p, plan, n_batch, stream);
    else if (sa == 3) launch_prefill_r<HD, POS, false, 3>(p, plan, n_batch, stream);
    else if (p.rope) launch_prefill_r<HD, POS, true, 0>(p, plan, n_batch, stream);
    else launch_prefill_r<HD, POS, false, 0>(p, plan, n_batch, stream);
}

hipError_t launch_prefill_batched(const PrefillParams & p, int head_dim, int n_batch, int sa, hipStream_t stream) {
    const bool pos = p.scale_log2 > 0.f;
    const int plan = prefill_plan(p.n_q, p.n_head * n_batch, p.n_kv, head_dim, p.plan);
    if (p.n_qtiles != (p.n_q + 32 * plan - 1) / (32 * plan)) return hipErrorInvalidValue;  // planned with other inputs
    if (head_dim == 256) {  // plan 4 only (prefill_plan), f16 or rotated f32 query rows (no self-attention variants)
        if (sa != 0 || plan != 4) return hipErrorInvalidValue;
        const dim3 grid((uint32_t)p.n_qtiles * p.n_head, (uint32_t)n_batch), block(4 * kWave);
        if (p.rope && pos) hipLaunchKernelGGL((prefill_kernel<256, true, 4, true, 1, 0>), grid, block, 0, stream, p);
        else if (p.rope) hipLaunchKernelGGL((prefill_kernel<256, false, 4, true, 1, 0>), grid, block, 0, stream, p);
        else if (pos) hipLaunchKernelGGL((prefill_kernel<256, true, 4, false, 1, 0>), grid, block, 0, stream, p);
        else hipLaunchKernelGGL((prefill_kernel<256, false, 4, false, 1, 0>), grid, block, 0, stream, p);
    } else if (head_dim == 64) {
        if (pos) launch_prefill_t<64, true>(p, plan, n_batch, sa, stream);
        else launch_prefill_t<64, false>(p, plan, n_batch, sa, stream);
    } else {
        if (pos) launch_prefill_t<128, true>(p, plan, n_batch, sa, stream);
        else launch_prefill_t<128, false>(p, plan, n_batch, sa, stream);
    }
    return hipGetLastError();
}

hipError_t launch_prefill(const PrefillParams & p, int head_dim, hipStream_t stream) {
    return launch_prefill_batched(p, head_dim, 1, 0, stream);
}

}  // namespace mx
