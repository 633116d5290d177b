// Kernel parameter blocks and launchers shared between the C ABI layer (api.hip) and the kernels. Parameters travel by
// value as kernel arguments, so a call needs no device-side metadata buffer and can be captured in a HIP graph.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace mx {

typedef _Float16 half_t;

// Sequences per decode launch: their cache pointers, lengths and split counts ride in the kernel arguments.
constexpr int kMaxHeadDim = 256;
constexpr int kMaxSeqPerLaunch = 32;
// Keys per split are a multiple of this (4 waves x 32-key blocks), and never fewer.
constexpr int kDecodeChunkQuantum = 128;
// Split counters kCounterStride uint32 (256 bytes) apart: each on a line of its own, so that the atomics of different
// tiles do not serialize on one line.
constexpr int kCounterStride = 64;

struct DecodeSeq {
    const half_t * k;
    const half_t * v;
    int32_t len;      // keys in the cache
    int32_t n_split;  // splits of `chunk` keys covering them
};

struct DecodeParams {
    const half_t * q;
    half_t * out;
    float * lse;
    float * part;  // [n_seq][n_head_kv][n_rowtiles][max_split][RT][head_dim + 4] f32: acc[head_dim], m, l, 2 spare
    uint32_t * counters;  // [n_seq][n_head_kv][n_rowtiles]: splits finished per tile; back at 0 after every call
    int64_t q_stride, kv_stride, out_stride;
    int32_t n_head, n_head_kv, group, n_q, causal;
    int32_t rows;        // n_q * group: query rows that share one key/value head
    int32_t n_rowtiles;  // ceil(rows / RT)
    int32_t chunk;       // keys per split
    int32_t max_split;   // max over the launch's sequences of n_split
    int32_t seq0;        // index of the launch's first sequence in the caller's batch (query/output rows)
    int32_t xcd_heads;   // 1: kv head g's splits run on XCD g % 8 (one sequence, n_head_kv a multiple of 8)
    int32_t kv_nt;       // 1: non-temporal K/V loads (one long sequence with xcd_heads, or at least 256 MB of K/V);
                         // honoured by the head-dim-128 kernels with 4-row tiles
    float scale_log2;    // scale * log2(e): scores are kept in base-2 units
    int32_t f32;         // 1: f32 query rows in qkv (q_stride floats apart) and f32 output in out32
    int32_t append;      // 1 (with f32): fused decode step, the rows are q|k|v of each sequence's new token
    const float * qkv;
    float * out32;
    int32_t rope_mode;   // 0 adjacent pairs, 1 split halves (neox), 2 none
    float rope_freq[kMaxHeadDim / 2];  // base^(-2i / head_dim) in f32 for rotary pair i
    DecodeSeq seq[kMaxSeqPerLaunch];
};

// The per-query kernel for head dims below 64 (small.hip): query row t of sequence s sits at cache position
// seq[s].p0 + t (its rotary angle; with causal it sees keys 0 .. p0 + t), its row index is seq[s].row0 + t.
struct SmallSeq {
    const half_t * k;
    const half_t * v;
    int32_t len;   // keys in the cache
    int32_t p0;    // position of the first query row
    int64_t row0;  // first query / output row
};
struct SmallAttnParams {
    const void * q;  // half rows, or f32 rows (q_f32)
    void * out;      // half rows, or f32 rows (out_f32)
    float * lse;
    int64_t q_stride, kv_stride, out_stride;
    int32_t n_head, n_head_kv, group, n_q, causal, q_f32, out_f32;
    int32_t rope_mode;  // 0 adjacent pairs, 1 split halves (neox), 2 none: the query rotated for its position
    float scale_log2;
    float rope_freq[kMaxHeadDim / 2];
    SmallSeq seq[kMaxSeqPerLaunch];
};

struct PrefillParams {
    const half_t * q;
    const half_t * k;
    const half_t * v;
    half_t * out;
    float * lse;
    int64_t q_stride, kv_stride, out_stride;
    int32_t n_head, n_head_kv, group, n_q, p0, n_kv, causal, n_qtiles;
    float scale_log2;
    int32_t rope;       // 1: query rows come unrotated in f32 from qkv (q_stride floats apart), rotated for position
                        // p0 + t in the kernel and rounded to half; the output is f32 (out32)
    const float * qkv;
    float * out32;
    int32_t rope_mode;  // 0 adjacent pairs, 1 split halves (neox), 2 none
    // independent problems along blockIdx.y (the IR self-attention's batch): elements between the q (or qkv), cache,
    // output and lse blocks of consecutive problems; 0 for one problem
    int64_t q_batch, kv_batch, out_batch, lse_batch;
    // the IR self-attention's rows read in place (kernel variants for f32, bf16 or f16 rows): head_dim of the rows
    // (<= the kernel's, a multiple of 8; columns past it are zeros) and the elements between consecutive heads
    int32_t hdv, head_stride;
    int32_t plan;  // workgroup plan fixed by the caller (8, 4 or 2), or 0: prefill_plan's choice
    // Stream-K launch (plan 8, one problem; sk_ranges 0 otherwise): sk_ranges workgroups each take an equal range of
    // the launch's sk_total (query tile, 64-key block) units; a tile split between ranges is merged through sk_part
    // (2 slots of kPrefillSlotFloats<HD> per range) and sk_counters (one uint32 per tile, zero between calls).
    int32_t sk_ranges;
    int64_t sk_total;
    float * sk_part;
    uint32_t * sk_counters;
    float rope_freq[kMaxHeadDim / 2];
};

// ---- Stream-K partition of an 8-wave prefill launch (host and device) ----
// Tiles are the launch's (kv head, query tile of 256 rows, head of the group) triples in that order, each with
// prefill_tile_blocks 64-key blocks; the blocks of all tiles in that order form the units 0 .. total - 1, and range r
// is the units [lo(r), lo(r + 1)).
constexpr int kPrefillSkRows = 256;  // query rows per tile (8 waves x 32)
constexpr int kPrefillSkKeys = 64;   // keys per block
// floats of one partial slot: per lane of the 8 waves its O values (head_dim / 2 of them), m and l
template <int HD>
constexpr int64_t kPrefillSlotFloats = 8 * (int64_t)(HD / 2 + 2) * 64;

__host__ __device__ inline int32_t prefill_tile_blocks(int32_t qt, int32_t n_q, int32_t p0, int32_t n_kv, int32_t causal) {
    const int32_t last_row = (qt + 1) * kPrefillSkRows < n_q ? (qt + 1) * kPrefillSkRows : n_q;  // one past the tile's last row
    const int64_t kend = causal ? ((int64_t)p0 + last_row < n_kv ? (int64_t)p0 + last_row : n_kv) : n_kv;
    return (int32_t)((kend + kPrefillSkKeys - 1) / kPrefillSkKeys);
}
__host__ __device__ inline int64_t sk_lo(int64_t total, int32_t ranges, int32_t r) { return (int64_t)r * total / ranges; }
// the range that holds unit x (ranges are never empty: total >= ranges)
__host__ __device__ inline int32_t sk_range_of(int64_t total, int32_t ranges, int64_t x) {
    const int64_t r = ((x + 1) * ranges - 1) / total;
    return (int32_t)(r < ranges - 1 ? r : ranges - 1);
}
struct SkTile {
    int32_t kvh, qt, gi, nblk;  // kv head, query tile, head within the group, blocks of the tile
    int64_t start;               // its first unit
};
// The tile that holds unit x; per_kv = group * sum over query tiles of their blocks (the units of one kv head).
__host__ __device__ inline SkTile sk_locate(int64_t x, int64_t per_kv, int32_t group, int32_t n_qtiles, int32_t n_q,
                                            int32_t p0, int32_t n_kv, int32_t causal) {
    SkTile t;
    t.kvh = (int32_t)(x / per_kv);
    const int64_t rem = x - (int64_t)t.kvh * per_kv;
    int64_t acc = 0;
    t.qt = n_qtiles - 1;
    t.nblk = prefill_tile_blocks(t.qt, n_q, p0, n_kv, causal);
    for (int32_t q = 0; q < n_qtiles; q++) {
        const int32_t nb = prefill_tile_blocks(q, n_q, p0, n_kv, causal);
        if (rem < acc + (int64_t)group * nb) {
            t.qt = q;
            t.nblk = nb;
            break;
        }
        acc += (int64_t)group * nb;
    }
    t.gi = (int32_t)((rem - acc) / t.nblk);
    t.start = (int64_t)t.kvh * per_kv + acc + (int64_t)t.gi * t.nblk;
    return t;
}
// Slot of the partial that range r holds for a tile starting at unit `start`: 2 r when it is the range's first
// segment (the tile started in an earlier range, or exactly at lo(r)), else 2 r + 1 (the range's last segment).
__host__ __device__ inline int64_t sk_slot(int64_t total, int32_t ranges, int32_t r, int64_t start) {
    return 2 * (int64_t)r + (start > sk_lo(total, ranges, r) ? 1 : 0);
}

// Packing of the IR self-attention's [B][N][3E] q|k|v rows into the attention kernel's operands when the rows cannot be
// read in place (head_dim not a multiple of 8): f32 query rows and f16 key|value rows with head_dim padded to hdp
// (zeros), and back.
struct SelfAttnPackParams {
    const void * qkv;     // [rows][3 E], of dtype (0 f32, 1 f16, 2 bf16)
    float * q;            // [rows][H hdp] f32
    half_t * kv;          // [rows][2 H hdp] f16: keys at column 0, values at column H hdp
    int64_t rows;         // B N
    int32_t heads, hd, hdp, dtype;
};
struct SelfAttnUnpackParams {
    const float * o;      // [rows][H hdp] f32
    void * y;             // [rows][E], of dtype (0 f32, 1 f16, 2 bf16)
    int64_t rows;
    int32_t heads, hd, hdp, dtype;
};

// rope_store (llama_kernels.h:520-545) for the keys and values of n_rows new tokens: key head g of row t rotated for
// position p0 + t and, like value head g, rounded to half into row p0 + t of the caches.
struct RopeStoreParams {
    const float * qkv;  // [n_rows][qkv_stride] f32: q | k | v
    half_t * k;
    half_t * v;
    float * q_out;      // [n_rows][n_head head_dim] f32: the rotated query rows, or null (not written)
    int64_t qkv_stride, kv_stride;
    int32_t n_head, n_head_kv, n_rows, p0, rope_mode;
    float rope_freq[kMaxHeadDim / 2];
};

// Projections (linear.hip): Y[i] = X W[i]^T for count matrices sharing X and the shape.
constexpr uint32_t kLinearNorm = 1, kLinearAccumulate = 2, kLinearBias = 4, kLinearOutF16 = 8;
constexpr int kLinearMaxMats = 64;
constexpr int kLinearGemvMaxRows = 8;        // M up to this runs the f32-input GEMV, above it the MFMA GEMM
constexpr size_t kLinearGemvLds = 64 * 1024;  // staged input rows up to this many bytes per workgroup

struct LinearParams {
    const float * x;
    const float * gamma;
    half_t * xh;    // [M][K] the staged input rows (M > 8): written by stage_kernel, read by the GEMM
    int64_t x_stride, y_stride;
    int32_t M, N, K, count;
    uint32_t flags;
    float eps;
    const half_t * w[kLinearMaxMats];
    void * y[kLinearMaxMats];
    const float * bias[kLinearMaxMats];
};

int decode_rows_per_tile(int rows);
hipError_t launch_decode(const DecodeParams & p, int n_seq, int head_dim, int rt, int waves, hipStream_t stream);
hipError_t launch_fill_zero(void * p, size_t bytes, hipStream_t stream);

// query rows one prefill workgroup covers (forced: a plan fixed by the caller, or 0)
int prefill_rows_per_workgroup(int n_q, int n_head, int n_kv, int head_dim, int forced);
hipError_t launch_prefill(const PrefillParams & p, int head_dim, hipStream_t stream);
hipError_t launch_linear(const LinearParams & p, hipStream_t stream);
hipError_t launch_stage(const LinearParams & p, hipStream_t stream);  // M > 8: the staged half input rows
hipError_t launch_gemm(const LinearParams & p, hipStream_t stream);   // M > 8: gemm_kernel on the staged rows
hipError_t launch_rope_store(const RopeStoreParams & p, int head_dim, hipStream_t stream);
hipError_t launch_small_attn(const SmallAttnParams & p, int head_dim, int n_seq, hipStream_t stream);
// n_batch problems of the prefill kernel along blockIdx.y, offsets from p.*_batch
hipError_t launch_prefill_batched(const PrefillParams & p, int head_dim, int n_batch, int sa, hipStream_t stream);
hipError_t launch_self_attn_pack(const SelfAttnPackParams & p, hipStream_t stream);
hipError_t launch_self_attn_unpack(const SelfAttnUnpackParams & p, hipStream_t stream);

}  // namespace mx
