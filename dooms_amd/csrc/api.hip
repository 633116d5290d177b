// C ABI of the attention hot path (include/mx_attn.h): argument checks, split planning and kernel launches.
//
// Error behaviour follows the reference's C API (include/dooms/dooms_c.h:24-36 in dooms.cpp 0.6.1): an integer code with
// dooms_code's numbering, never an abort, and a thread-local message for the last failure. Every check runs on the host
// before anything is enqueued, so a rejected call leaves the stream untouched.
#include "mx_attn.h"
#include "mx_linear.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <mutex>
#include <queue>
#include <string>

#include "mx_kernels.hpp"

namespace {

thread_local std::string g_last_error;

int32_t fail(int32_t code, const char * fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

bool aligned16(const void * p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int32_t check_tuning(const mx_attn_tuning * t) {
    if (!t) return MX_ATTN_OK;
    if (t->decode_splits < 0 || t->decode_splits > 64)
        return fail(MX_ATTN_INVALID_ARGUMENT, "tuning->decode_splits (%d) must be 0 (planned) or 1..64", t->decode_splits);
    if (t->decode_waves != 0 && t->decode_waves != 4 && t->decode_waves != 8)
        return fail(MX_ATTN_INVALID_ARGUMENT, "tuning->decode_waves (%d) must be 0 (planned), 4 or 8", t->decode_waves);
    if (t->decode_max_workgroups < 0)
        return fail(MX_ATTN_INVALID_ARGUMENT, "tuning->decode_max_workgroups (%d) must be >= 0", t->decode_max_workgroups);
    if (t->prefill_plan != 0 && t->prefill_plan != 2 && t->prefill_plan != 4 && t->prefill_plan != 8)
        return fail(MX_ATTN_INVALID_ARGUMENT, "tuning->prefill_plan (%d) must be 0 (planned), 2, 4 or 8", t->prefill_plan);
    if (t->prefill_stream < -1 || t->prefill_stream > 1)
        return fail(MX_ATTN_INVALID_ARGUMENT, "tuning->prefill_stream (%d) must be -1, 0 (planned) or 1", t->prefill_stream);
    return MX_ATTN_OK;
}

// Checks shared by prefill and decode.
int32_t check_desc(const mx_attn_desc * d) {
    if (!d) return fail(MX_ATTN_INVALID_ARGUMENT, "desc is null");
    if (d->reserved != 0) return fail(MX_ATTN_INVALID_ARGUMENT, "desc->reserved must be 0");
    if (d->n_head < 1 || d->n_head_kv < 1)
        return fail(MX_ATTN_INVALID_ARGUMENT, "n_head (%d) and n_head_kv (%d) must be >= 1", d->n_head, d->n_head_kv);
    if (d->n_head % d->n_head_kv != 0)
        return fail(MX_ATTN_INVALID_ARGUMENT, "n_head (%d) is not a multiple of n_head_kv (%d)", d->n_head, d->n_head_kv);
    if (d->head_dim < 1) return fail(MX_ATTN_INVALID_ARGUMENT, "head_dim (%d) must be >= 1", d->head_dim);
    if (d->head_dim < 4 || d->head_dim > 256 || (d->head_dim & (d->head_dim - 1)) != 0)
        return fail(MX_ATTN_UNSUPPORTED, "head_dim %d is not supported (a power of two in [4, 256])", d->head_dim);
    if (d->n_q < 0) return fail(MX_ATTN_INVALID_ARGUMENT, "n_q (%d) must be >= 0", d->n_q);
    if (d->causal != 0 && d->causal != 1) return fail(MX_ATTN_INVALID_ARGUMENT, "causal must be 0 or 1");
    if (!std::isfinite(d->scale)) return fail(MX_ATTN_INVALID_ARGUMENT, "scale is not finite");
    const int64_t qw = (int64_t)d->n_head * d->head_dim, kvw = (int64_t)d->n_head_kv * d->head_dim;
    if (d->q_stride < qw) return fail(MX_ATTN_INVALID_ARGUMENT, "q_stride (%lld) < n_head * head_dim (%lld)", (long long)d->q_stride, (long long)qw);
    if (d->out_stride < qw)
        return fail(MX_ATTN_INVALID_ARGUMENT, "out_stride (%lld) < n_head * head_dim (%lld)", (long long)d->out_stride, (long long)qw);
    if (d->kv_stride < kvw)
        return fail(MX_ATTN_INVALID_ARGUMENT, "kv_stride (%lld) < n_head_kv * head_dim (%lld)", (long long)d->kv_stride, (long long)kvw);
    const int unit = std::min(8, d->head_dim);  // 16-byte rows (8-byte ones at head dim 4)
    if (d->q_stride % unit || d->kv_stride % unit || d->out_stride % unit)
        return fail(MX_ATTN_INVALID_ARGUMENT, "strides must be multiples of %d elements", unit);
    return check_tuning(d->tuning);
}

int32_t hip_status(hipError_t e, const char * what) {
    if (e == hipSuccess) return MX_ATTN_OK;
    return fail(MX_ATTN_INTERNAL, "%s: %s", what, hipGetErrorString(e));
}

// Decode split plan. Splits are whole multiples of kDecodeChunkQuantum (128) keys, and
//   * as short as that allows with at most kMaxSplits splits per sequence: every wave of a 4-wave workgroup then
//     walks one 32-key block (more splits lengthen the in-kernel merge: 64 splits of an 8192-key Llama-3-8B row cost
//     ~5 us more than 32);
//   * then as small as possible while the launch stays within workgroup_cap() workgroups (measured on MI355X for
//     Llama-3-8B batches of 4 and 16: 1536 streams best; two workgroups per CU are resident at once, 512 in all).
// With every split counter on a line of its own (kCounterStride), splitting pays down to the shortest caches: one
// split per sequence (no merge) no longer wins anywhere measured, e.g. Qwen2.5-0.5B at 513 keys 7.0 us as one split
// of 8 waves vs 6.5 us as 5 splits of 4 waves, Whisper self-attention at 449 keys 7.1 -> 6.7 us; and 128-key splits
// beat 256-key ones at every size measured below 32 x 256 keys (Whisper cross-attention over 1500 frames: 7.8 ->
// 7.25 us, Llama-3-8B at 1024 keys 8.9 -> 8.1 us).
// The bound n_split <= ceil(len / quantum) keeps the workspace a function of the longest sequence alone.
constexpr int kMaxSplits = 32;
// One head-dim-128 sequence of at least 32k keys whose 32-split grid would leave CUs idle (fewer than 8 kv heads x row
// tiles) takes up to 64 splits: Qwen2.5-7B (4 kv heads) at 32768 keys 24.4 -> 22.3 us, at 131072 keys 72-73 -> 62 us.
// Shorter sequences keep 32 (at 8192 keys 64 splits ran 10.6 -> 12.4 us: the longer merge outweighs the stream), as do
// head dim 64 (Qwen2.5-0.5B at 32768 keys 12.2 -> 13.0) and batches (4 x 8192 keys 20.6 -> 24.9).
constexpr int kMaxSplitsFew = 64;
constexpr int64_t kMaxSplitsFewKeys = 32768;
int max_splits(const mx_attn_desc * d, int n_rowtiles, int64_t n_seq, int64_t lmax) {
    const bool few = (int64_t)d->n_head_kv * n_rowtiles * kMaxSplits < 256;
    return few && d->head_dim == 128 && n_seq == 1 && lmax >= kMaxSplitsFewKeys ? kMaxSplitsFew : kMaxSplits;
}
int workgroup_cap(const mx_attn_tuning * t) {
    return t && t->decode_max_workgroups > 0 ? t->decode_max_workgroups : 1536;
}

// Waves per workgroup: 8 when splits of at least 256 keys give each of them a 32-key block and the launch runs in one
// round on the CUs (at most 256 workgroups), each wave then walking half as many blocks (Llama-3-8B at 8192 keys, 256
// workgroups, 15.1 -> 14.4 us; Qwen2.5-7B at 32768 keys, 128 workgroups of 1024 keys, 32.2 -> 29.0 us); else 4: with
// 128-key splits the 4-wave workgroup's merge is cheaper (Whisper cross-attention 7.8 -> 7.25 us; Llama-3-8B at 1024
// keys 8.8 -> 8.1 us), and with more workgroups 8-wave ones would not all be resident at once (Llama-3-8B batch 4:
// 26.0 -> 20.6 us).
int decode_waves(const mx_attn_tuning * t, int64_t chunk, int64_t wgs) {
    if (t && t->decode_waves) return t->decode_waves;
    return chunk >= 256 && wgs <= 256 ? 8 : 4;
}

struct DecodeShape {
    int rows, rt, n_rowtiles;
};

DecodeShape decode_shape(const mx_attn_desc * d) {
    DecodeShape s;
    s.rows = d->n_q * (d->n_head / d->n_head_kv);
    s.rt = mx::decode_rows_per_tile(s.rows);
    s.n_rowtiles = (s.rows + s.rt - 1) / s.rt;
    return s;
}

// Workspace layout: kMaxTilesPerLaunch split counters (one per (sequence of a launch, kv head, row tile), each on a
// 256-byte line of its own) at a fixed place, then the partials. The counters must be zero when a call starts, and
// every call leaves the ones it used at zero; the partials are left as they are. So the counter region has the same
// place and size in every call, whatever its shape: a call of another shape on the same workspace must never write
// partials where a counter lies. Launches of more sequences than fit run one after another and reuse both.
constexpr int64_t kMaxTilesPerLaunch = 2048;
constexpr size_t kCounterRegion = (size_t)kMaxTilesPerLaunch * mx::kCounterStride * 4;  // 512 KiB

// Head dims below this run on the per-query kernel (small.hip), at and above it on the matrix-core kernels.
constexpr int kMfmaMinHeadDim = 64;

// Sequences one decode launch takes (0: a sequence alone has more tiles than a launch holds).
int64_t decode_seqs_per_launch(const mx_attn_desc * d, int64_t n_rowtiles) {
    const int64_t tiles_per_seq = (int64_t)d->n_head_kv * n_rowtiles;
    return std::min<int64_t>(mx::kMaxSeqPerLaunch, kMaxTilesPerLaunch / tiles_per_seq);
}

struct WsLayout {
    size_t counter_bytes, part_bytes;
};

WsLayout decode_ws_layout(const mx_attn_desc * d, int32_t batch, int32_t max_kv_len) {
    const DecodeShape s = decode_shape(d);
    const int64_t seqs = std::min<int64_t>(batch, std::max<int64_t>(1, decode_seqs_per_launch(d, s.n_rowtiles)));
    // the split plan never makes more than kMaxSplits splits of a sequence, nor more than one per quantum of keys
    const int64_t max_split = std::min<int64_t>(std::max(max_splits(d, s.n_rowtiles, batch, max_kv_len),
                                                         d->tuning ? d->tuning->decode_splits : 0),
                                                ((int64_t)max_kv_len + mx::kDecodeChunkQuantum - 1) / mx::kDecodeChunkQuantum);
    WsLayout w{0, 0};
    if (max_split <= 1 || d->head_dim < kMfmaMinHeadDim) return w;  // one split per sequence (or the per-query kernel)
    w.counter_bytes = kCounterRegion;
    w.part_bytes = (size_t)(seqs * d->n_head_kv * s.n_rowtiles * max_split * s.rt * (d->head_dim + 4) * (int64_t)sizeof(float));
    return w;
}

size_t decode_ws_bytes(const mx_attn_desc * d, int32_t batch, int32_t max_kv_len) {
    const WsLayout w = decode_ws_layout(d, batch, max_kv_len);
    return w.counter_bytes + w.part_bytes;
}

}  // namespace

namespace {

// The GEMM path (M > 8) stages the input rows as half, zero-padded to a multiple of 64 columns, 256-byte rounded.
size_t linear_ws_bytes(const mx_linear_desc & d) {
    if (d.M <= mx::kLinearGemvMaxRows) return 0;
    return ((size_t)d.M * (size_t)((d.K + 63) / 64 * 64) * 2 + 255) / 256 * 256;
}

// Rotary frequencies base^(-2i / head_dim) in f32 (rotate_pair, llama_kernels.h:513-518), computed once per call
// on the host with the C library's powf; 0 past head_dim / 2 or without rotation.
void fill_freq(float (&freq)[mx::kMaxHeadDim / 2], const mx_attn_rope * rope, int head_dim) {
    for (int i = 0; i < mx::kMaxHeadDim / 2; i++)
        freq[i] = (rope && rope->mode != 2 && i < head_dim / 2) ? std::pow(rope->base, -2.f * (float)i / (float)head_dim) : 0.f;
}

// rope_store of n_rows q|k|v rows (f32, q_stride floats apart) at positions p0 .. into the caches.
int32_t rope_store_rows(const mx_attn_desc & d, const mx_attn_rope * rope, const float * qkv, int32_t n_rows,
                        int32_t p0, void * k_cache, void * v_cache, float * q_out, hipStream_t st) {
    mx::RopeStoreParams r;
    r.qkv = qkv;
    r.k = static_cast<mx::half_t *>(k_cache);
    r.v = static_cast<mx::half_t *>(v_cache);
    r.qkv_stride = d.q_stride;
    r.kv_stride = d.kv_stride;
    r.n_head = d.n_head;
    r.n_head_kv = d.n_head_kv;
    r.n_rows = n_rows;
    r.p0 = p0;
    r.rope_mode = rope->mode;
    r.q_out = q_out;
    fill_freq(r.rope_freq, rope, d.head_dim);
    return hip_status(mx::launch_rope_store(r, d.head_dim, st), "rope_store launch");
}

// The per-query kernel's parameters (head dims below kMfmaMinHeadDim) without the sequences.
mx::SmallAttnParams small_params(const mx_attn_desc & d, const void * q, void * out, float * lse, bool f32,
                                 const mx_attn_rope * rope) {
    mx::SmallAttnParams sp{};
    sp.q = q;
    sp.out = out;
    sp.lse = lse;
    sp.q_stride = d.q_stride;
    sp.kv_stride = d.kv_stride;
    sp.out_stride = d.out_stride;
    sp.n_head = d.n_head;
    sp.n_head_kv = d.n_head_kv;
    sp.group = d.n_head / d.n_head_kv;
    sp.n_q = d.n_q;
    sp.causal = d.causal;
    sp.q_f32 = sp.out_f32 = f32 ? 1 : 0;
    sp.rope_mode = rope ? rope->mode : 2;
    sp.scale_log2 = d.scale * 1.4426950408889634f;
    fill_freq(sp.rope_freq, rope, d.head_dim);
    return sp;
}

// Stream-K plan of a flash prefill: ranges (0: the one-tile-per-workgroup grid) and the launch's (tile, key block) units.
struct SkPlan {
    int32_t ranges = 0;
    int64_t total = 0;
};
constexpr int32_t kSkRanges = 256;  // one range per CU
constexpr int64_t kSkMaxTiles = (int64_t)kCounterRegion / 4;
// At least this many blocks per range (below, the merge and the lost prefetch at the segment edges cost more).
constexpr int64_t kSkMinBlocksPerRange = 8;
constexpr int32_t kSkMinRanges = 192;

size_t prefill_sk_ws_bytes(int head_dim) {
    const int64_t slot = head_dim == 64 ? mx::kPrefillSlotFloats<64> : mx::kPrefillSlotFloats<128>;
    return kCounterRegion + (size_t)(2 * kSkRanges) * (size_t)slot * sizeof(float);
}

// When stream-K is planned (tuning->prefill_stream 0; 1 forces it wherever it applies, -1 never):
//   * head dim 64 only. The head-dim-128 kernel runs the chip at its power limit, so CUs the grid leaves idle let the
//     busy ones clock higher: a 2048-row chunk of 28 heads (224 tiles for 256 CUs) ran 920 TFLOP/s on the grid and 913
//     split, 224 non-causal tiles 876 against 860. At head dim 64 a 4096-token Qwen2.5-0.5B prompt (224 tiles) went
//     81.9 -> 71.0 us.
//   * fewer than 4 tiles per CU, and the grid's time at least 8 % over the split's. The grid deals its tiles heaviest
//     first and hands the next to the CU that frees first (its time is simulated so), which already balances a causal
//     prompt of many tiles: a 4096-token Llama-3-8B prompt (512 tiles) ran 167 us on the grid, 217 split.
SkPlan prefill_sk_plan(const mx_attn_desc & d, int64_t n_kv, int plan) {
    SkPlan k;
    const int forced = d.tuning ? d.tuning->prefill_stream : 0;
    if (forced < 0 || plan != 8 || (d.head_dim != 64 && d.head_dim != 128)) return k;
    if (forced == 0 && d.head_dim != 64) {
        // head dim 128: only a chunk of at most 128 tiles (half the CUs) behind a prefix at least 3x its length
        const int64_t wg8 = (int64_t)((d.n_q + mx::kPrefillSkRows - 1) / mx::kPrefillSkRows) * d.n_head;
        if (wg8 > kSkRanges / 2 || n_kv < 4 * (int64_t)d.n_q) return k;
    }
    const int32_t n_qtiles = (d.n_q + mx::kPrefillSkRows - 1) / mx::kPrefillSkRows;
    const int64_t n_tiles = (int64_t)n_qtiles * d.n_head;
    if (n_tiles > kSkMaxTiles || (forced == 0 && n_tiles >= 4 * kSkRanges)) return k;
    int64_t total = 0;
    for (int32_t qt = 0; qt < n_qtiles; qt++)
        total += (int64_t)d.n_head * mx::prefill_tile_blocks(qt, d.n_q, d.p0, (int32_t)n_kv, d.causal);
    // fewer ranges (down to kSkMinRanges) when the launch has too few blocks to give every CU kSkMinBlocksPerRange
    // (A/B on one box, us: Qwen2.5-0.5B 128 rows at 8k keys 75 -> 41, 512 rows at 4k 46.5 -> 37.8, Qwen2.5-7B 128
    // rows at 4k 61 -> 49; at ~130 ranges, chunks at 2k keys, the split was 7 % slower, hence the floor of 192)
    // (a multiple of 8: the kernel deals range (b % 8) R / 8 + b / 8 to workgroup b, one eighth per XCD)
    const int32_t R = (int32_t)(std::min<int64_t>(kSkRanges, total / kSkMinBlocksPerRange) / 8 * 8);
    if (R < kSkMinRanges) return k;
    if (forced == 0) {
        // the grid: tiles heaviest first (causal: by query tile descending), each to the CU that frees first
        std::priority_queue<int64_t, std::vector<int64_t>, std::greater<int64_t>> cu;
        for (int32_t i = 0; i < kSkRanges; i++) cu.push(0);
        int64_t grid_time = 0;
        for (int32_t i = 0; i < n_qtiles; i++) {
            const int32_t qt = d.causal ? n_qtiles - 1 - i : i;
            const int64_t nb = mx::prefill_tile_blocks(qt, d.n_q, d.p0, (int32_t)n_kv, d.causal);
            for (int32_t h = 0; h < d.n_head; h++) {
                const int64_t t = cu.top() + nb;
                cu.pop();
                cu.push(t);
                grid_time = std::max(grid_time, t);
            }
        }
        if ((double)total / R > 0.92 * (double)grid_time) return k;
    }
    k.ranges = R;
    k.total = total;
    return k;
}

// Waves per workgroup of a causal prefill at head dims 64 and 128 (prefill_plan's cost model otherwise; sk_ok: the
// workspace holds the stream-K slots). At head dim 64, measured per plan (TFLOP/s, forced plans 4 and 8,
// Qwen2.5-0.5B-shaped unless stated):
//   * a chunk behind a prefix at least as long as itself, whose 8-wave grid leaves CUs idle: the 8-wave plan split by
//     stream-K over every CU (8192 tokens in 2048-row chunks 415 -> 535, 16384 in 2048-row chunks 482 -> 657, 16 heads
//     8192 in 2048-row chunks 474 -> 576, 8192 in 1024-row chunks 363 (the key-split plan) -> 393);
//   * otherwise 4 waves (two workgroups per CU, whose barriers do not couple the waves sharing a SIMD) where the cost
//     model took 8: one-call prompts of 4096 tokens 398 -> 470 (16 heads 388 -> 526, 12 heads 372 -> 411), 8192
//     tokens 555 -> 688 (32 heads 738 -> 761), a 32-head 8192-token prompt in 2048-row chunks 682 -> 724; one case
//     measured the other way, a 32-head 4096-token prompt 716 -> 698. The key-split plan for short prompts stays.
// At head dim 128: a chunk of at most 128 8-wave tiles behind a prefix at least 3x its length takes the split 8-wave
// plan (the grid leaves over half the CUs idle, which the clock under this kernel's power draw does not repay):
// Qwen2.5-7B 16384 tokens in 1024-row chunks 777 -> 882, 8192 in 512-row chunks 481 -> 589, Llama-3-8B 16384 in
// 1024-row chunks 863 -> 958, 8192 in 256-row chunks 294 -> 439; a whole prompt whose 8-wave grid is one round takes
// 4 waves: Llama-3-8B 2048 tokens 508-539 -> 585-594, Qwen2.5-7B 2048 443-465 -> 554-559. 2048-row chunks (cfg5),
// 4096-token prompts and short prompts unchanged.
int prefill_choose_plan(const mx_attn_desc & d, int64_t n_kv, bool sk_ok) {
    const int forced = d.tuning ? d.tuning->prefill_plan : 0;
    const int plan = mx::prefill_rows_per_workgroup(d.n_q, d.n_head, (int)n_kv, d.head_dim, forced) / 32;
    // (a forced stream-K choice, tuning->prefill_stream 1 or -1, keeps the cost model's plan)
    if (forced != 0 || (d.tuning && d.tuning->prefill_stream != 0) || !d.causal) return plan;
    const int64_t wg8 = (int64_t)((d.n_q + 255) / 256) * d.n_head;
    if (d.head_dim == 64) {
        if (sk_ok && n_kv >= 2 * (int64_t)d.n_q && wg8 < kSkRanges && prefill_sk_plan(d, n_kv, 8).ranges > 0) return 8;
        return plan == 2 ? 2 : 4;
    }
    if (d.head_dim == 128) {
        if (sk_ok && prefill_sk_plan(d, n_kv, 8).ranges > 0) return 8;
        if (d.p0 == 0 && n_kv == d.n_q && plan == 8 && wg8 <= kSkRanges) return 4;
    }
    return plan;
}

int32_t prefill_impl(const mx_attn_desc * desc, const void * q, const void * k_cache, const void * v_cache, void * out,
                     float * lse, mx_attn_stream stream, const mx_attn_rope * rope, void * ws = nullptr,
                     size_t ws_bytes = 0) {
    const mx_attn_desc & d = *desc;
    if (d.p0 < 0) return fail(MX_ATTN_INVALID_ARGUMENT, "p0 (%d) must be >= 0", d.p0);
    if (d.n_kv < 0) return fail(MX_ATTN_INVALID_ARGUMENT, "n_kv (%d) must be >= 0", d.n_kv);
    if (d.n_q == 0) return MX_ATTN_OK;
    const int64_t n_kv = d.n_kv == 0 ? (int64_t)d.p0 + d.n_q : d.n_kv;
    if (n_kv > INT32_MAX) return fail(MX_ATTN_INVALID_ARGUMENT, "p0 + n_q overflows");
    if ((d.causal || rope) && n_kv < (int64_t)d.p0 + d.n_q)
        return fail(MX_ATTN_INVALID_ARGUMENT, "n_kv (%lld) must be >= p0 + n_q (%lld): the chunk's own rows are in the cache",
                    (long long)n_kv, (long long)d.p0 + d.n_q);
    if (!q || !k_cache || !v_cache || !out) return fail(MX_ATTN_INVALID_ARGUMENT, "q, k_cache, v_cache and out must not be null");
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
        return fail(MX_ATTN_INVALID_ARGUMENT, "q, k_cache, v_cache and out must be 16-byte aligned");
    if (lse && (reinterpret_cast<uintptr_t>(lse) & 3u)) return fail(MX_ATTN_INVALID_ARGUMENT, "lse must be 4-byte aligned");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (d.head_dim < kMfmaMinHeadDim) {  // the per-query kernel: the chunk's keys and values first (stream order)
        if (rope)
            if (int32_t rc = rope_store_rows(d, rope, static_cast<const float *>(q), d.n_q, d.p0, const_cast<void *>(k_cache),
                                             const_cast<void *>(v_cache), nullptr, st))
                return rc;
        mx::SmallAttnParams sp = small_params(d, q, out, lse, rope != nullptr, rope);
        sp.seq[0] = mx::SmallSeq{static_cast<const mx::half_t *>(k_cache), static_cast<const mx::half_t *>(v_cache),
                                 (int32_t)n_kv, d.p0, 0};
        return hip_status(mx::launch_small_attn(sp, d.head_dim, 1, st), "attention launch");
    }

    mx::PrefillParams p;
    p.q = static_cast<const mx::half_t *>(q);
    p.k = static_cast<const mx::half_t *>(k_cache);
    p.v = static_cast<const mx::half_t *>(v_cache);
    p.out = static_cast<mx::half_t *>(out);
    p.lse = lse;
    p.q_stride = d.q_stride;
    p.kv_stride = d.kv_stride;
    p.out_stride = d.out_stride;
    p.n_head = d.n_head;
    p.n_head_kv = d.n_head_kv;
    p.group = d.n_head / d.n_head_kv;
    p.n_q = d.n_q;
    p.p0 = d.p0;
    p.n_kv = (int32_t)n_kv;
    p.causal = d.causal;
    // stream-K when planned and the workspace holds its slots
    const bool sk_ok = ws && !(reinterpret_cast<uintptr_t>(ws) & 255u) && ws_bytes >= prefill_sk_ws_bytes(d.head_dim);
    p.plan = prefill_choose_plan(d, n_kv, sk_ok);
    const int rows = 32 * p.plan;
    p.n_qtiles = (d.n_q + rows - 1) / rows;
    p.scale_log2 = d.scale * 1.4426950408889634f;
    p.rope = rope != nullptr;
    p.qkv = static_cast<const float *>(q);
    p.out32 = static_cast<float *>(out);
    p.rope_mode = rope ? rope->mode : 2;
    p.q_batch = p.kv_batch = p.out_batch = p.lse_batch = 0;
    p.hdv = p.head_stride = d.head_dim;
    fill_freq(p.rope_freq, rope, d.head_dim);
    p.sk_ranges = 0;
    p.sk_total = 0;
    p.sk_part = nullptr;
    p.sk_counters = nullptr;
    if (sk_ok) {
        const SkPlan k = prefill_sk_plan(d, n_kv, p.plan);
        if (k.ranges > 0) {
            p.sk_ranges = k.ranges;
            p.sk_total = k.total;
            p.sk_counters = static_cast<uint32_t *>(ws);
            p.sk_part = reinterpret_cast<float *>(static_cast<char *>(ws) + kCounterRegion);
        }
    }
    if (rope)  // the chunk's keys and values go into the caches first (stream order)
        if (int32_t rc = rope_store_rows(d, rope, static_cast<const float *>(q), d.n_q, d.p0, const_cast<void *>(k_cache),
                                         const_cast<void *>(v_cache), nullptr, st))
            return rc;
    return hip_status(mx::launch_prefill(p, d.head_dim, st), "prefill launch");
}

// Checks of the rotary parameters and the q|k|v row width shared by the two fused entry points.
int32_t check_rope(const mx_attn_desc & d, const mx_attn_rope * rope) {
    if (!rope) return fail(MX_ATTN_INVALID_ARGUMENT, "rope is null");
    if (rope->mode < 0 || rope->mode > 2) return fail(MX_ATTN_INVALID_ARGUMENT, "rope->mode (%d) must be 0, 1 or 2", rope->mode);
    if (rope->mode != 2 && !(std::isfinite(rope->base) && rope->base > 0.f))
        return fail(MX_ATTN_INVALID_ARGUMENT, "rope->base must be finite and > 0");
    const int64_t row = (int64_t)(d.n_head + 2 * d.n_head_kv) * d.head_dim;
    if (d.q_stride < row)
        return fail(MX_ATTN_INVALID_ARGUMENT, "q_stride (%lld) < (n_head + 2 n_head_kv) * head_dim (%lld)", (long long)d.q_stride, (long long)row);
    return MX_ATTN_OK;
}

// The decode entry points' checks of everything but the workspace (the descriptor and batch already checked): pointers,
// alignment, every kv_len, and whether a launch holds one sequence's rows. Sets max_len, the longest kv_len.
int32_t check_decode_args(const mx_attn_desc * desc, int32_t batch, const int32_t * kv_len, const void * q,
                          const void * const * k_caches, const void * const * v_caches, const void * out,
                          const float * lse, int32_t & max_len) {
    const mx_attn_desc & d = *desc;
    if (!kv_len || !k_caches || !v_caches) return fail(MX_ATTN_INVALID_ARGUMENT, "kv_len, k_caches and v_caches must not be null");
    if (!q || !out) return fail(MX_ATTN_INVALID_ARGUMENT, "q and out must not be null");
    if (!aligned16(q) || !aligned16(out)) return fail(MX_ATTN_INVALID_ARGUMENT, "q and out must be 16-byte aligned");
    if (lse && (reinterpret_cast<uintptr_t>(lse) & 3u)) return fail(MX_ATTN_INVALID_ARGUMENT, "lse must be 4-byte aligned");
    max_len = 0;
    for (int32_t b = 0; b < batch; b++) {
        const int32_t n = kv_len[b];
        if (n < 1) return fail(MX_ATTN_INVALID_ARGUMENT, "kv_len[%d] = %d: every sequence needs at least one key", b, n);
        if (d.causal && n < d.n_q)
            return fail(MX_ATTN_INVALID_ARGUMENT, "kv_len[%d] = %d < n_q = %d: causal rows must all be in the cache", b, n, d.n_q);
        if (!k_caches[b] || !v_caches[b]) return fail(MX_ATTN_INVALID_ARGUMENT, "cache pointers of sequence %d are null", b);
        if (!aligned16(k_caches[b]) || !aligned16(v_caches[b]))
            return fail(MX_ATTN_INVALID_ARGUMENT, "cache pointers of sequence %d must be 16-byte aligned", b);
        max_len = std::max(max_len, n);
    }
    if (d.head_dim >= kMfmaMinHeadDim && decode_seqs_per_launch(desc, decode_shape(desc).n_rowtiles) < 1)
        return fail(MX_ATTN_UNSUPPORTED, "n_head * n_q (%lld query rows per sequence) is too large for one decode launch",
                    (long long)d.n_head * d.n_q);
    return MX_ATTN_OK;
}

// Shared by mx_attn_decode (half q rows and output), mx_attn_decode_f32 (f32 q rows and output) and
// mx_attn_decode_rope (f32 q|k|v rows and output, the new token's key and value appended to the caches by the kernel).
int32_t decode_impl(const mx_attn_desc * desc, int32_t batch, const int32_t * kv_len, const void * q,
                    const void * const * k_caches, const void * const * v_caches, void * out, float * lse,
                    void * workspace, size_t ws_bytes, mx_attn_stream stream, const mx_attn_rope * rope, bool f32) {
    const mx_attn_desc & d = *desc;
    int32_t max_len = 0;
    if (int32_t rc = check_decode_args(desc, batch, kv_len, q, k_caches, v_caches, out, lse, max_len)) return rc;
    const size_t need = decode_ws_bytes(desc, batch, max_len);
    if (need > 0 && !workspace) return fail(MX_ATTN_INVALID_ARGUMENT, "workspace is null but %zu bytes are needed", need);
    if (ws_bytes < need) return fail(MX_ATTN_RESOURCE_EXHAUSTED, "workspace of %zu bytes is smaller than the %zu bytes needed", ws_bytes, need);
    if (need > 0 && (reinterpret_cast<uintptr_t>(workspace) & 255u))
        return fail(MX_ATTN_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
    const WsLayout wl = decode_ws_layout(desc, batch, max_len);

    const DecodeShape s = decode_shape(desc);
    if (d.head_dim < kMfmaMinHeadDim) {  // the per-query kernel; the fused step's cache rows written first
        const hipStream_t st = static_cast<hipStream_t>(stream);
        for (int32_t b0 = 0; b0 < batch; b0 += mx::kMaxSeqPerLaunch) {
            const int n_seq = std::min<int32_t>(mx::kMaxSeqPerLaunch, batch - b0);
            mx::SmallAttnParams sp = small_params(d, q, out, lse, f32, rope);
            for (int i = 0; i < n_seq; i++) {
                const int32_t b = b0 + i, L = kv_len[b];
                if (rope)
                    if (int32_t rc = rope_store_rows(d, rope, static_cast<const float *>(q) + (int64_t)b * d.q_stride, 1,
                                                     L - 1, const_cast<void *>(k_caches[b]),
                                                     const_cast<void *>(v_caches[b]), nullptr, st))
                        return rc;
                sp.seq[i] = mx::SmallSeq{static_cast<const mx::half_t *>(k_caches[b]),
                                         static_cast<const mx::half_t *>(v_caches[b]), L, L - d.n_q, (int64_t)b * d.n_q};
            }
            if (int32_t rc = hip_status(mx::launch_small_attn(sp, d.head_dim, n_seq, st), "attention launch")) return rc;
        }
        return MX_ATTN_OK;
    }
    // one launch holds at most kMaxTilesPerLaunch (sequence, kv head, row tile) tiles (so its 1-D grid of up to 32
    // splits per tile stays far inside the grid's range)
    const int32_t seq_per_launch = (int32_t)decode_seqs_per_launch(desc, s.n_rowtiles);  // >= 1: checked above
    const hipStream_t st = static_cast<hipStream_t>(stream);
    for (int32_t b0 = 0; b0 < batch; b0 += seq_per_launch) {
        const int n_seq = std::min<int32_t>(seq_per_launch, batch - b0);
        mx::DecodeParams p;
        p.q = static_cast<const mx::half_t *>(q);
        p.out = static_cast<mx::half_t *>(out);
        p.f32 = f32 ? 1 : 0;
        p.append = rope != nullptr;
        p.qkv = static_cast<const float *>(q);
        p.out32 = static_cast<float *>(out);
        p.rope_mode = rope ? rope->mode : 2;
        fill_freq(p.rope_freq, rope, d.head_dim);
        p.lse = lse;
        p.counters = static_cast<uint32_t *>(workspace);
        p.part = reinterpret_cast<float *>(static_cast<char *>(workspace) + wl.counter_bytes);
        p.q_stride = d.q_stride;
        p.kv_stride = d.kv_stride;
        p.out_stride = d.out_stride;
        p.n_head = d.n_head;
        p.n_head_kv = d.n_head_kv;
        p.group = d.n_head / d.n_head_kv;
        p.n_q = d.n_q;
        p.causal = d.causal;
        p.rows = s.rows;
        p.n_rowtiles = s.n_rowtiles;
        p.seq0 = b0;
        // The XCD-mapped grid (kv head g's splits on XCD g mod 8, partials published into that XCD's L2) for kv heads in
        // multiples of 8, also for batches: Llama-3-8B batch 4 (ragged, 55 MB) 16.97 -> 15.7 us, batch 16 ragged 55.3
        // -> 50.4, 32 x 4096 keys 100.8 -> 97.2 (widened below for short caches)
        p.xcd_heads = d.n_head_kv % 8 == 0;
        // Non-temporal K/V loads on the XCD-mapped grid with at least 16 MB of K/V, or any grid with at least 256 MB
        // (K/V streamed from HBM once per step in a decoder): Llama-3-8B batch 1 at 8192 keys 11.93 -> 11.76 us per
        // launch, batch 16 x 8192 keys -3.5 %; on the XCD-mapped grid batch 4 (55 MB) 16.7 -> 15.7 us and batch 16
        // ragged 55.9 -> 50.4; but slower where the bench's caches stay in the Infinity Cache between replays
        // (Qwen2.5-0.5B +8 %, Whisper cross-attention +10 %), hence the 16 MB floor.
        int64_t kv_keys = 0;
        for (int i = 0; i < n_seq; i++) kv_keys += kv_len[b0 + i];
        const int64_t kv_bytes = kv_keys * d.kv_stride * 2 * 2;
        p.kv_nt = (p.xcd_heads && kv_bytes >= ((int64_t)16 << 20)) || kv_bytes >= ((int64_t)256 << 20);
        p.scale_log2 = d.scale * 1.4426950408889634f;
        // split plan (see workgroup_cap)
        const int64_t quantum = mx::kDecodeChunkQuantum;
        int64_t lmax = 0;
        for (int i = 0; i < n_seq; i++) lmax = std::max<int64_t>(lmax, kv_len[b0 + i]);
        auto round_up = [&](int64_t x) { return (x + quantum - 1) / quantum * quantum; };
        const int64_t msplit = max_splits(&d, s.n_rowtiles, n_seq, lmax);
        int64_t chunk = round_up((lmax + msplit - 1) / msplit);
        auto launch_wgs = [&](int64_t c) {
            int64_t n = 0;
            for (int i = 0; i < n_seq; i++) n += (kv_len[b0 + i] + c - 1) / c;
            return n * d.n_head_kv * s.n_rowtiles;
        };
        const int64_t cap = workgroup_cap(d.tuning);
        // A batch of at least 4 sequences of about one length (within 1.5x) and at least 4096 keys: at most 8 splits
        // per sequence. A/B on one box, us per launch (8 splits of 4 waves against the plan of up to 32): Llama-3-8B
        // 4 x 8192 keys 29.9 -> 26.4, 8 x 8192 51.9 -> 48.8, 16 x 8192 95.5 -> 90.1, 12 x 4096 42.3 -> 39.9,
        // Qwen2.5-7B 8 x 4096 22.0 -> 17.7, 4 x 8192 19.5 -> 18.8, Qwen2.5-0.5B 8 x 4096 12.1 -> 9.8. Ragged batches
        // keep the plan (Llama-3-8B 1.6k-6.8k keys x 4: 16.4 -> 19.9 at 8 splits; Qwen2.5-7B 1.3k-7.3k x 16 35 ->
        // 41.7 at 16), as do shorter caches (4 x 2048: 11.5 -> 12.6).
        int64_t lmin = lmax;
        for (int i = 0; i < n_seq; i++) lmin = std::min<int64_t>(lmin, kv_len[b0 + i]);
        const bool uniform = n_seq >= 4 && lmin >= 4096 && 2 * lmax <= 3 * lmin;
        if (uniform && !(d.tuning && d.tuning->decode_splits > 0)) chunk = std::max(chunk, round_up((lmax + 7) / 8));
        if (d.tuning && d.tuning->decode_splits > 0) {
            // the caller's split count (of the longest sequence): never more than one split per quantum of keys
            chunk = round_up((lmax + d.tuning->decode_splits - 1) / d.tuning->decode_splits);
        } else if (launch_wgs(chunk) > cap) {  // smallest chunk within the cap: bisect over multiples of the quantum
            int64_t lo = chunk / quantum, hi = round_up(lmax) / quantum;
            while (lo < hi) {
                const int64_t mid = (lo + hi) / 2;
                if (launch_wgs(mid * quantum) > cap) lo = mid + 1;
                else hi = mid;
            }
            chunk = lo * quantum;
        }
        p.chunk = (int32_t)std::min<int64_t>(chunk, INT32_MAX / 2);
        p.max_split = 1;
        for (int i = 0; i < n_seq; i++) {
            const int32_t n = kv_len[b0 + i];
            p.seq[i].k = static_cast<const mx::half_t *>(k_caches[b0 + i]);
            p.seq[i].v = static_cast<const mx::half_t *>(v_caches[b0 + i]);
            p.seq[i].len = n;
            p.seq[i].n_split = (int32_t)((n + p.chunk - 1) / p.chunk);
            p.max_split = std::max(p.max_split, p.seq[i].n_split);
        }
        for (int i = n_seq; i < mx::kMaxSeqPerLaunch; i++) p.seq[i] = mx::DecodeSeq{nullptr, nullptr, 0, 0};
        // The XCD-mapped grid (partials published into one XCD's L2) also for one short sequence whatever its kv heads:
        // a few splits over at most 4 MB of keys and values, where the merge chain outweighs the stream, which the
        // grid concentrates on min(kv heads, 8) XCDs. Qwen2.5-0.5B at 513 keys 4.99 -> 4.50 us per launch, Whisper
        // self-attention at 449 keys 5.25 -> 4.89, Qwen2.5-7B at 1024 keys 6.67 -> 6.42; 16 splits (Qwen2.5-0.5B at
        // 2048 keys, two XCDs streaming) measured 5.87 -> 6.02, Whisper cross-attention (12 splits, 7.7 MB) no gain.
        if (n_seq == 1 && p.max_split <= 8 && kv_bytes <= ((int64_t)4 << 20)) p.xcd_heads = 1;
        if (p.max_split > 32) p.xcd_heads = 0;  // the XCD-local counter counts at most 63 splits per XCD field
        const int waves = decode_waves(d.tuning, p.chunk, launch_wgs(p.chunk));
        if (int32_t rc = hip_status(mx::launch_decode(p, n_seq, d.head_dim, s.rt, waves, st), "decode launch")) return rc;
    }
    return MX_ATTN_OK;
}

// ---- prefill chunks on the split-KV decode kernel ----
// A chunk whose rows per kv head (n_q x group, the decode kernel's packed GQA rows) are at most kPrefillSplitRows runs
// on the decode kernel: its causal rows at the end of the cache are the chunk's own semantics (row t sees keys
// 0 .. p0 + t), and it spreads the keys over the CUs, which the flash kernel (one workgroup per head and query tile,
// every workgroup walking all keys) cannot. Measured (28 q / 4 kv heads, hd 128): 2 rows at 30k keys 610 -> 28 us, 16
// rows 611 -> 74 us, 128 rows 598 -> 306 us; at 256 rows and 4k keys the flash kernel wins (87 vs 113 us). Up to 512
// packed rows always, up to 1024 when the cache holds at least 64 keys per query row (Llama-3-8B, 256 rows at 30k keys:
// 607 vs 640 us, the one measured loss at that bound).
constexpr int64_t kPrefillSplitRows = 512, kPrefillSplitRowsLong = 1024, kPrefillSplitKeysPerRow = 64;
int64_t prefill_split_keys(const mx_attn_desc & d);
bool prefill_sk_room(const mx_attn_desc & d, const void * ws, size_t ws_bytes) {
    return !(reinterpret_cast<uintptr_t>(ws) & 255u) && ws_bytes >= prefill_sk_ws_bytes(d.head_dim);
}
// At head dim 128 the flash kernel split by stream-K over the CUs (planned for a chunk of few tiles behind a long
// prefix) takes the chunks of 128 rows and more, and of 64 rows over at least 16k keys, from this route (A/B on one box,
// us: Qwen2.5-7B 128 rows at 30k keys 248 -> 135-139, Llama-3-8B 128 rows at 30k 244-247 -> 133, 256 rows at 30k
// 452-465 -> 148, 128 rows at 8k 80-82 -> 56, 64 rows at 30k 134-139 -> 120-122; the route stays ahead up to 48 rows
// at every length measured, and for 64 rows over 2k-8k keys). At head dim 64 from 96 rows over at least 16k keys
// (Qwen2.5-0.5B at 30k keys: 96 rows 71 -> 66, 128 rows 86 -> 67, 144 rows 77 -> 67; 20 heads of 64, 128 rows 100 ->
// 78; below 96 rows, or over 8k keys, the route is ahead or level).
// sk_room: the workspace holds the stream-K slots (a chunk that the split flash kernel would take stays on this route
// when it does not)
bool prefill_split_route(const mx_attn_desc & d, bool sk_room) {
    if (d.n_q < 1 || d.head_dim < kMfmaMinHeadDim) return false;
    const int64_t rows = (int64_t)d.n_q * (d.n_head / d.n_head_kv);
    if (decode_seqs_per_launch(&d, decode_shape(&d).n_rowtiles) < 1) return false;
    const int64_t keys = prefill_split_keys(d);
    if (!(rows <= kPrefillSplitRows || (rows <= kPrefillSplitRowsLong && keys >= kPrefillSplitKeysPerRow * d.n_q)))
        return false;
    const bool flash = d.head_dim == 128 ? d.n_q >= 128 || (d.n_q >= 64 && keys >= 16384)
                                         : d.head_dim == 64 && d.n_q >= 96 && keys >= 16384;
    if (flash && sk_room && d.causal && d.p0 >= 0) {
        const int64_t n_kv = d.n_kv == 0 ? (int64_t)d.p0 + d.n_q : d.n_kv;
        if (n_kv <= INT32_MAX && prefill_sk_plan(d, n_kv, prefill_choose_plan(d, n_kv, true)).ranges > 0) return false;
    }
    return true;
}
// keys the decode kernel walks: a causal chunk's rows see keys up to p0 + n_q - 1 (keys past them are masked anyway)
int64_t prefill_split_keys(const mx_attn_desc & d) {
    if (d.causal) return (int64_t)d.p0 + d.n_q;
    return d.n_kv == 0 ? (int64_t)d.p0 + d.n_q : d.n_kv;
}
// workspace of the split route: the decode workspace, then (for mx_attn_prefill_rope_ws) the rotated f32 query rows
size_t prefill_split_q_offset(const mx_attn_desc & d, int32_t L) { return (decode_ws_bytes(&d, 1, L) + 255) / 256 * 256; }

// ---- IR SelfAttention (src/ir/op.h:31-32) ----

constexpr int kSelfAttnMaxHeadDim = 128;  // the IR op's heads are padded to the prefill kernel's 64 or 128

int32_t check_self_attn(const mx_self_attn_desc * d) {
    if (!d) return fail(MX_ATTN_INVALID_ARGUMENT, "desc is null");
    if (d->batch < 1 || d->batch > 65535 || d->n_tok < 0)
        return fail(MX_ATTN_INVALID_ARGUMENT, "batch (%d) must be in [1, 65535] and n_tok (%d) >= 0", d->batch, d->n_tok);
    if (d->heads < 1) return fail(MX_ATTN_INVALID_ARGUMENT, "self_attention: heads must be >= 1, got %d", d->heads);
    if (d->embed < 1 || d->embed % d->heads)
        return fail(MX_ATTN_INVALID_ARGUMENT, "self_attention: embedding %d is not divisible by %d heads", d->embed, d->heads);
    if (d->dtype < MX_ATTN_F32 || d->dtype > MX_ATTN_BF16) return fail(MX_ATTN_INVALID_ARGUMENT, "dtype %d is not f32, f16 or bf16", d->dtype);
    if (!std::isfinite(d->scale)) return fail(MX_ATTN_INVALID_ARGUMENT, "self_attention: scale must be finite");
    if (int32_t rc = check_tuning(d->tuning)) return rc;
    if (d->embed / d->heads > kSelfAttnMaxHeadDim)
        return fail(MX_ATTN_UNSUPPORTED, "head_dim %d is above %d", d->embed / d->heads, kSelfAttnMaxHeadDim);
    if ((int64_t)d->batch * d->n_tok * 3 * d->embed > ((int64_t)1 << 40)) return fail(MX_ATTN_INVALID_ARGUMENT, "qkv is too large");
    return MX_ATTN_OK;
}

// How a descriptor runs: 0 the f16 rows in place (head_dim 64 or 128); 1 the rows in place through the kernel variant
// for their type (f32, bf16, or f16 with another head_dim), when head_dim is a multiple of 8 (every 8-element chunk
// 16-byte aligned): Q, K, V rounded to half as they are loaded, zero columns up to the kernel's head_dim, the output
// in the rows' type; 2 otherwise: packed into padded f32 Q and f16 K|V in the workspace, and unpacked afterwards.
struct SelfAttnPlan {
    int mode;       // 0 in place, 1 in place with conversion, 2 packed
    int hd, hdp;    // head_dim and the kernel's head_dim
    size_t q_off, kv_off, o_off, bytes;  // workspace layout
};

SelfAttnPlan self_attn_plan(const mx_self_attn_desc & d) {
    SelfAttnPlan s{};
    s.hd = d.embed / d.heads;
    const bool native = s.hd == 64 || s.hd == 128;
    s.mode = native && d.dtype == MX_ATTN_F16 ? 0 : s.hd % 8 == 0 ? 1 : 2;
    s.hdp = s.hd <= 64 ? 64 : 128;
    const int64_t rows = (int64_t)d.batch * d.n_tok;
    auto up = [](size_t x) { return (x + 255) / 256 * 256; };
    if (s.mode == 2) {
        const size_t w = (size_t)rows * d.heads * s.hdp;
        s.q_off = 0;
        s.kv_off = up(w * 4);
        s.o_off = s.kv_off + up(w * 2 * 2);
        s.bytes = s.o_off + up(w * 4);
    }
    return s;
}

// ---- scratch of mx_attn_decode_noalloc: the decode workspace held by the library ----
// One array per GPU (each device that runs the library holds its own copy until the process ends). In host code the
// name `scratch` is a host-side stand-in, not a device address: the address of a device's copy comes from
// hipGetSymbolAddress, called once per device with that device current, and only that address is handed to kernels.
constexpr size_t kScratchBytes = (size_t)16 << 20;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;  // taken only by the first call on a device

// The current device's scratch address; on the first call on a device, its split counters are zeroed with a kernel on
// `stream` (ordered before the call's own launch; no memset, no allocation).
int32_t device_scratch(hipStream_t stream, void ** out) {
    int dev = 0;
    if (int32_t rc = hip_status(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (dev < 0 || dev >= kMaxDevices) return fail(MX_ATTN_UNSUPPORTED, "device %d: at most %d devices", dev, kMaxDevices);
    void * p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_acquire);
        if (!p) {
            void * addr = nullptr;
            if (int32_t rc = hip_status(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"))
                return rc;
            if (!addr) return fail(MX_ATTN_INTERNAL, "hipGetSymbolAddress(scratch) returned null");
            if (int32_t rc = hip_status(mx::launch_fill_zero(addr, kScratchBytes, stream), "scratch init")) return rc;
            g_scratch[dev].store(addr, std::memory_order_release);
            p = addr;
        }
    }
    *out = p;
    return MX_ATTN_OK;
}

int32_t check_linear_desc(const mx_linear_desc * desc, int32_t count) {
    if (!desc) return fail(MX_ATTN_INVALID_ARGUMENT, "desc is null");
    const mx_linear_desc & d = *desc;
    if (d.reserved != 0) return fail(MX_ATTN_INVALID_ARGUMENT, "desc->reserved must be 0");
    if (d.M < 0 || d.N < 1 || d.K < 1) return fail(MX_ATTN_INVALID_ARGUMENT, "need M >= 0, N >= 1, K >= 1 (M %d, N %d, K %d)", d.M, d.N, d.K);
    if (d.K % 32) return fail(MX_ATTN_UNSUPPORTED, "K (%d) must be a multiple of 32", d.K);
    if (d.flags & ~15u) return fail(MX_ATTN_INVALID_ARGUMENT, "unknown flags 0x%x", d.flags);
    const bool out16 = d.flags & MX_LINEAR_OUT_F16;
    if (d.x_stride < d.K || d.x_stride % 4) return fail(MX_ATTN_INVALID_ARGUMENT, "x_stride (%lld) must be >= K and a multiple of 4", (long long)d.x_stride);
    if (d.y_stride < d.N || d.y_stride % (out16 ? 8 : 4))
        return fail(MX_ATTN_INVALID_ARGUMENT, "y_stride (%lld) must be >= N and a multiple of %d", (long long)d.y_stride, out16 ? 8 : 4);
    if ((d.flags & MX_LINEAR_RMS_NORM) && !(std::isfinite(d.eps) && d.eps >= 0.f)) return fail(MX_ATTN_INVALID_ARGUMENT, "eps must be finite and >= 0");
    if (count < 1 || count > mx::kLinearMaxMats) return fail(MX_ATTN_INVALID_ARGUMENT, "count (%d) must be in [1, %d]", count, mx::kLinearMaxMats);
    return MX_ATTN_OK;
}

// Checks of an mx_linear call and its kernel parameters (for M == 0 only the descriptor is checked).
int32_t linear_params(const mx_linear_desc * desc, int32_t count, const uint16_t * const * W, const float * X,
                      void * const * Y, const float * gamma, const float * const * bias, void * workspace,
                      size_t ws_bytes, mx::LinearParams & p) {
    if (int32_t rc = check_linear_desc(desc, count)) return rc;
    const mx_linear_desc & d = *desc;
    if (d.M == 0) return MX_ATTN_OK;
    if (!W || !Y || !X) return fail(MX_ATTN_INVALID_ARGUMENT, "W, X and Y must not be null");
    if (!aligned16(X)) return fail(MX_ATTN_INVALID_ARGUMENT, "X must be 16-byte aligned");
    if ((d.flags & MX_LINEAR_RMS_NORM) && (!gamma || !aligned16(gamma))) return fail(MX_ATTN_INVALID_ARGUMENT, "gamma must be a 16-byte aligned pointer with MX_LINEAR_RMS_NORM");
    if ((d.flags & MX_LINEAR_BIAS) && !bias) return fail(MX_ATTN_INVALID_ARGUMENT, "bias is null with MX_LINEAR_BIAS");
    for (int32_t i = 0; i < count; i++) {
        if (!W[i] || !Y[i]) return fail(MX_ATTN_INVALID_ARGUMENT, "W[%d] or Y[%d] is null", i, i);
        if (!aligned16(W[i]) || !aligned16(Y[i])) return fail(MX_ATTN_INVALID_ARGUMENT, "W[%d] and Y[%d] must be 16-byte aligned", i, i);
        p.w[i] = reinterpret_cast<const mx::half_t *>(W[i]);
        p.y[i] = Y[i];
        p.bias[i] = (d.flags & MX_LINEAR_BIAS) ? bias[i] : nullptr;
    }
    const size_t need = linear_ws_bytes(d);
    if (need && (!workspace || (reinterpret_cast<uintptr_t>(workspace) & 255u)))
        return fail(MX_ATTN_INVALID_ARGUMENT, "a 256-byte aligned workspace of %zu bytes is needed", need);
    if (ws_bytes < need) return fail(MX_ATTN_RESOURCE_EXHAUSTED, "workspace of %zu bytes is smaller than the %zu bytes needed", ws_bytes, need);
    p.x = X;
    p.gamma = gamma;
    p.xh = static_cast<mx::half_t *>(workspace);
    p.x_stride = d.x_stride;
    p.y_stride = d.y_stride;
    p.M = d.M;
    p.N = d.N;
    p.K = d.K;
    p.count = count;
    p.flags = d.flags;
    p.eps = d.eps;
    return MX_ATTN_OK;
}

}  // namespace

extern "C" {

MX_ATTN_API size_t mx_self_attention_workspace_bytes(const mx_self_attn_desc * desc) {
    if (check_self_attn(desc)) return 0;
    return self_attn_plan(*desc).bytes;
}

MX_ATTN_API int32_t mx_self_attention(const mx_self_attn_desc * desc, const void * qkv, void * y, void * workspace,
                                      size_t ws_bytes, mx_attn_stream stream) {
    if (int32_t rc = check_self_attn(desc)) return rc;
    const mx_self_attn_desc & d = *desc;
    if (d.n_tok == 0) return MX_ATTN_OK;
    if (!qkv || !y) return fail(MX_ATTN_INVALID_ARGUMENT, "qkv and y must not be null");
    if (!aligned16(qkv) || !aligned16(y)) return fail(MX_ATTN_INVALID_ARGUMENT, "qkv and y must be 16-byte aligned");
    const SelfAttnPlan s = self_attn_plan(d);
    const int64_t rows = (int64_t)d.batch * d.n_tok, E = d.embed;
    const size_t esz = d.dtype == MX_ATTN_F32 ? 4 : 2;
    {  // y must not overlap qkv
        const char * a = static_cast<const char *>(qkv), * b = static_cast<const char *>(y);
        if (a < b + (size_t)rows * E * esz && b < a + (size_t)rows * 3 * E * esz)
            return fail(MX_ATTN_INVALID_ARGUMENT, "y overlaps qkv");
    }
    if (s.bytes > 0 && !workspace) return fail(MX_ATTN_INVALID_ARGUMENT, "workspace is null but %zu bytes are needed", s.bytes);
    if (ws_bytes < s.bytes) return fail(MX_ATTN_RESOURCE_EXHAUSTED, "workspace of %zu bytes is smaller than the %zu bytes needed", ws_bytes, s.bytes);
    if (s.bytes > 0 && (reinterpret_cast<uintptr_t>(workspace) & 255u)) return fail(MX_ATTN_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    char * ws = static_cast<char *>(workspace);

    mx::PrefillParams p{};
    p.n_head = p.n_head_kv = d.heads;
    p.group = 1;
    p.n_q = p.n_kv = d.n_tok;
    p.p0 = 0;
    p.causal = 0;
    p.plan = d.tuning ? d.tuning->prefill_plan : 0;
    const int rpw = mx::prefill_rows_per_workgroup(d.n_tok, d.heads * d.batch, d.n_tok, s.hdp, p.plan);
    p.n_qtiles = (d.n_tok + rpw - 1) / rpw;
    p.scale_log2 = d.scale * 1.4426950408889634f;
    p.rope_mode = 2;
    p.lse = nullptr;
    p.lse_batch = 0;
    fill_freq(p.rope_freq, nullptr, s.hdp);
    if (s.mode != 2) {  // the rows in place: q at column 0, k at E, v at 2E of each 3E row (elements of the rows' type)
        const char * x = static_cast<const char *>(qkv);
        p.q = reinterpret_cast<const mx::half_t *>(x);
        p.k = reinterpret_cast<const mx::half_t *>(x + E * esz);
        p.v = reinterpret_cast<const mx::half_t *>(x + 2 * E * esz);
        p.out = static_cast<mx::half_t *>(y);
        p.out32 = static_cast<float *>(y);
        p.q_stride = p.kv_stride = 3 * E;
        p.out_stride = E;
        p.q_batch = p.kv_batch = (int64_t)d.n_tok * 3 * E;
        p.out_batch = (int64_t)d.n_tok * E;
        p.rope = 0;
        p.hdv = s.hd;
        p.head_stride = s.hd;
        const int sa = s.mode == 0 ? 0 : d.dtype == MX_ATTN_F32 ? 1 : d.dtype == MX_ATTN_BF16 ? 2 : 3;
        return hip_status(mx::launch_prefill_batched(p, s.hdp, d.batch, sa, st), "self_attention launch");
    }
    mx::SelfAttnPackParams pk;
    pk.qkv = qkv;
    pk.q = reinterpret_cast<float *>(ws + s.q_off);
    pk.kv = reinterpret_cast<mx::half_t *>(ws + s.kv_off);
    pk.rows = rows;
    pk.heads = d.heads;
    pk.hd = s.hd;
    pk.hdp = s.hdp;
    pk.dtype = d.dtype;
    if (int32_t rc = hip_status(mx::launch_self_attn_pack(pk, st), "self_attention pack launch")) return rc;
    const int64_t W = (int64_t)d.heads * pk.hdp;  // padded row width of one third
    p.k = pk.kv;
    p.v = pk.kv + W;
    p.kv_stride = 2 * W;
    p.kv_batch = (int64_t)d.n_tok * 2 * W;
    p.rope = 1;  // f32 query rows (no rotation, rope_mode 2) and f32 output
    p.qkv = pk.q;
    p.q_stride = W;
    p.q_batch = (int64_t)d.n_tok * W;
    float * o = reinterpret_cast<float *>(ws + s.o_off);
    p.out32 = o;
    p.out_stride = W;
    p.out_batch = (int64_t)d.n_tok * W;
    if (int32_t rc = hip_status(mx::launch_prefill_batched(p, s.hdp, d.batch, 0, st), "self_attention launch")) return rc;
    mx::SelfAttnUnpackParams u;
    u.o = o;
    u.y = y;
    u.rows = rows;
    u.heads = d.heads;
    u.hd = s.hd;
    u.hdp = s.hdp;
    u.dtype = d.dtype;
    return hip_status(mx::launch_self_attn_unpack(u, st), "self_attention unpack launch");
}

MX_ATTN_API int32_t mx_attn_abi_version(void) { return MX_ATTN_ABI_VERSION; }

MX_ATTN_API const char * mx_attn_last_error(void) { return g_last_error.c_str(); }

MX_ATTN_API int32_t mx_attn_prefill(const mx_attn_desc * desc, const uint16_t * q, const uint16_t * k_cache, const uint16_t * v_cache,
                                    uint16_t * out, float * lse, mx_attn_stream stream) {
    if (int32_t rc = check_desc(desc)) return rc;
    return prefill_impl(desc, q, k_cache, v_cache, out, lse, stream, nullptr);
}

MX_ATTN_API size_t mx_attn_prefill_workspace_bytes(const mx_attn_desc * desc) {
    if (check_desc(desc)) return 0;
    if (!prefill_split_route(*desc, true)) {  // the flash kernel: the stream-K slots when that plan is taken
        const mx_attn_desc & d = *desc;
        if (d.n_q < 1 || d.head_dim < kMfmaMinHeadDim || d.p0 < 0 || d.n_kv < 0) return 0;
        const int64_t n_kv = d.n_kv == 0 ? (int64_t)d.p0 + d.n_q : d.n_kv;
        if (n_kv > INT32_MAX) return 0;
        return prefill_sk_plan(d, n_kv, prefill_choose_plan(d, n_kv, true)).ranges > 0 ? prefill_sk_ws_bytes(d.head_dim) : 0;
    }
    const int64_t L = prefill_split_keys(*desc);
    if (L < 1 || L > INT32_MAX) return 0;
    return prefill_split_q_offset(*desc, (int32_t)L) + (size_t)desc->n_q * desc->n_head * desc->head_dim * sizeof(float);
}

MX_ATTN_API int32_t mx_attn_prefill_ws(const mx_attn_desc * desc, const uint16_t * q, const uint16_t * k_cache,
                                       const uint16_t * v_cache, uint16_t * out, float * lse, void * workspace,
                                       size_t ws_bytes, mx_attn_stream stream) {
    if (int32_t rc = check_desc(desc)) return rc;
    const mx_attn_desc & d = *desc;
    if (!workspace || !prefill_split_route(d, prefill_sk_room(d, workspace, ws_bytes)))
        return prefill_impl(desc, q, k_cache, v_cache, out, lse, stream, nullptr, workspace, ws_bytes);
    if (d.p0 < 0) return fail(MX_ATTN_INVALID_ARGUMENT, "p0 (%d) must be >= 0", d.p0);
    if (d.n_kv < 0) return fail(MX_ATTN_INVALID_ARGUMENT, "n_kv (%d) must be >= 0", d.n_kv);
    if (d.n_q == 0) return MX_ATTN_OK;
    if (d.causal && d.n_kv != 0 && d.n_kv < (int64_t)d.p0 + d.n_q)
        return fail(MX_ATTN_INVALID_ARGUMENT, "n_kv (%d) must be >= p0 + n_q (%lld): the chunk's own rows are in the cache",
                    d.n_kv, (long long)d.p0 + d.n_q);
    const int64_t L = prefill_split_keys(d);
    if (L > INT32_MAX) return fail(MX_ATTN_INVALID_ARGUMENT, "p0 + n_q overflows");
    const int32_t kv_len = (int32_t)L;
    const void * kp = k_cache, * vp = v_cache;
    return decode_impl(desc, 1, &kv_len, q, &kp, &vp, out, lse, workspace, ws_bytes, stream, nullptr, false);
}

MX_ATTN_API int32_t mx_attn_prefill_rope(const mx_attn_desc * desc, const mx_attn_rope * rope, const float * qkv, uint16_t * k_cache,
                                         uint16_t * v_cache, float * out, float * lse, mx_attn_stream stream) {
    if (int32_t rc = check_desc(desc)) return rc;
    if (int32_t rc = check_rope(*desc, rope)) return rc;
    return prefill_impl(desc, qkv, k_cache, v_cache, out, lse, stream, rope);
}

MX_ATTN_API int32_t mx_attn_prefill_rope_ws(const mx_attn_desc * desc, const mx_attn_rope * rope, const float * qkv,
                                            uint16_t * k_cache, uint16_t * v_cache, float * out, float * lse,
                                            void * workspace, size_t ws_bytes, mx_attn_stream stream) {
    if (int32_t rc = check_desc(desc)) return rc;
    if (int32_t rc = check_rope(*desc, rope)) return rc;
    const mx_attn_desc & d = *desc;
    if (!workspace || !prefill_split_route(d, prefill_sk_room(d, workspace, ws_bytes)))
        return prefill_impl(desc, qkv, k_cache, v_cache, out, lse, stream, rope, workspace, ws_bytes);
    if (d.p0 < 0) return fail(MX_ATTN_INVALID_ARGUMENT, "p0 (%d) must be >= 0", d.p0);
    if (d.n_kv < 0) return fail(MX_ATTN_INVALID_ARGUMENT, "n_kv (%d) must be >= 0", d.n_kv);
    if (d.n_q == 0) return MX_ATTN_OK;
    const int64_t n_kv = d.n_kv == 0 ? (int64_t)d.p0 + d.n_q : d.n_kv;
    if (n_kv > INT32_MAX) return fail(MX_ATTN_INVALID_ARGUMENT, "p0 + n_q overflows");
    if (n_kv < (int64_t)d.p0 + d.n_q)
        return fail(MX_ATTN_INVALID_ARGUMENT, "n_kv (%lld) must be >= p0 + n_q (%lld): the chunk's own rows are in the cache",
                    (long long)n_kv, (long long)d.p0 + d.n_q);
    if (!qkv || !k_cache || !v_cache || !out) return fail(MX_ATTN_INVALID_ARGUMENT, "qkv, k_cache, v_cache and out must not be null");
    if (!aligned16(qkv) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
        return fail(MX_ATTN_INVALID_ARGUMENT, "qkv, k_cache, v_cache and out must be 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(workspace) & 255u) return fail(MX_ATTN_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
    const int32_t L = (int32_t)prefill_split_keys(d);
    const size_t q_off = prefill_split_q_offset(d, L);
    const size_t need = q_off + (size_t)d.n_q * d.n_head * d.head_dim * sizeof(float);
    if (ws_bytes < need) return fail(MX_ATTN_RESOURCE_EXHAUSTED, "workspace of %zu bytes is smaller than the %zu bytes needed", ws_bytes, need);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    // the chunk's keys and values into the caches, its query rows rotated into the workspace, then the split-KV
    // kernel on those f32 rows (rounded to half as it loads them, as the flash kernel's rotated path does)
    mx::RopeStoreParams r;
    r.qkv = qkv;
    r.k = reinterpret_cast<mx::half_t *>(k_cache);
    r.v = reinterpret_cast<mx::half_t *>(v_cache);
    r.q_out = reinterpret_cast<float *>(static_cast<char *>(workspace) + q_off);
    r.qkv_stride = d.q_stride;
    r.kv_stride = d.kv_stride;
    r.n_head = d.n_head;
    r.n_head_kv = d.n_head_kv;
    r.n_rows = d.n_q;
    r.p0 = d.p0;
    r.rope_mode = rope->mode;
    fill_freq(r.rope_freq, rope, d.head_dim);
    if (int32_t rc = hip_status(mx::launch_rope_store(r, d.head_dim, st), "rope_store launch")) return rc;
    mx_attn_desc dq = d;
    dq.q_stride = (int64_t)d.n_head * d.head_dim;
    const void * kp = k_cache, * vp = v_cache;
    return decode_impl(&dq, 1, &L, r.q_out, &kp, &vp, out, lse, workspace, q_off, stream, nullptr, true);
}

MX_ATTN_API size_t mx_attn_decode_workspace_bytes(const mx_attn_desc * desc, int32_t batch, int32_t max_kv_len) {
    if (check_desc(desc)) return 0;
    if (batch < 1 || max_kv_len < 0) {
        fail(MX_ATTN_INVALID_ARGUMENT, "batch (%d) must be >= 1 and max_kv_len (%d) >= 0", batch, max_kv_len);
        return 0;
    }
    return decode_ws_bytes(desc, batch, max_kv_len);
}

MX_ATTN_API int32_t mx_attn_decode_workspace_init(void * workspace, size_t ws_bytes, mx_attn_stream stream) {
    if (ws_bytes == 0) return MX_ATTN_OK;
    if (!workspace) return fail(MX_ATTN_INVALID_ARGUMENT, "workspace is null");
    if (reinterpret_cast<uintptr_t>(workspace) & 255u) return fail(MX_ATTN_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
    return hip_status(mx::launch_fill_zero(workspace, ws_bytes, static_cast<hipStream_t>(stream)), "workspace init");
}

MX_ATTN_API int32_t mx_attn_decode(const mx_attn_desc * desc, int32_t batch, const int32_t * kv_len, const uint16_t * q,
                                   const uint16_t * const * k_caches, const uint16_t * const * v_caches, uint16_t * out, float * lse,
                                   void * workspace, size_t ws_bytes, mx_attn_stream stream) {
    if (int32_t rc = check_desc(desc)) return rc;
    if (batch < 1) return fail(MX_ATTN_INVALID_ARGUMENT, "batch (%d) must be >= 1", batch);
    if (desc->n_q == 0) return MX_ATTN_OK;
    return decode_impl(desc, batch, kv_len, q, reinterpret_cast<const void * const *>(k_caches),
                       reinterpret_cast<const void * const *>(v_caches), out, lse, workspace, ws_bytes, stream, nullptr, false);
}

MX_ATTN_API int32_t mx_attn_decode_noalloc(const mx_attn_desc * desc, int32_t batch, const int32_t * kv_len,
                                           const uint16_t * q, const uint16_t * const * k_caches,
                                           const uint16_t * const * v_caches, uint16_t * out, float * lse,
                                           mx_attn_stream stream) {
    if (int32_t rc = check_desc(desc)) return rc;
    if (batch < 1) return fail(MX_ATTN_INVALID_ARGUMENT, "batch (%d) must be >= 1", batch);
    if (desc->n_q == 0) return MX_ATTN_OK;
    // every argument check of mx_attn_decode first, so that a call refused for its arguments enqueues nothing
    int32_t max_len = 0;
    if (int32_t rc = check_decode_args(desc, batch, kv_len, q, reinterpret_cast<const void * const *>(k_caches),
                                       reinterpret_cast<const void * const *>(v_caches), out, lse, max_len))
        return rc;
    const size_t need = decode_ws_bytes(desc, batch, max_len);
    if (need > kScratchBytes)
        return fail(MX_ATTN_RESOURCE_EXHAUSTED,
                    "this decode needs %zu bytes of scratch; the library holds %zu per GPU (mx_attn_decode takes a larger "
                    "workspace)", need, kScratchBytes);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    void * ws = nullptr;
    if (int32_t rc = device_scratch(st, &ws)) return rc;
    return decode_impl(desc, batch, kv_len, q, reinterpret_cast<const void * const *>(k_caches),
                       reinterpret_cast<const void * const *>(v_caches), out, lse, ws, kScratchBytes, stream, nullptr, false);
}

MX_ATTN_API int32_t mx_attn_decode_f32(const mx_attn_desc * desc, int32_t batch, const int32_t * kv_len, const float * q,
                                       const uint16_t * const * k_caches, const uint16_t * const * v_caches, float * out,
                                       float * lse, void * workspace, size_t ws_bytes, mx_attn_stream stream) {
    if (int32_t rc = check_desc(desc)) return rc;
    if (batch < 1) return fail(MX_ATTN_INVALID_ARGUMENT, "batch (%d) must be >= 1", batch);
    if (desc->n_q == 0) return MX_ATTN_OK;
    return decode_impl(desc, batch, kv_len, q, reinterpret_cast<const void * const *>(k_caches),
                       reinterpret_cast<const void * const *>(v_caches), out, lse, workspace, ws_bytes, stream, nullptr, true);
}

MX_ATTN_API int32_t mx_attn_decode_rope(const mx_attn_desc * desc, const mx_attn_rope * rope, int32_t batch, const int32_t * kv_len,
                                        const float * qkv, uint16_t * const * k_caches, uint16_t * const * v_caches, float * out,
                                        float * lse, void * workspace, size_t ws_bytes, mx_attn_stream stream) {
    if (int32_t rc = check_desc(desc)) return rc;
    const mx_attn_desc & d = *desc;
    if (int32_t rc = check_rope(d, rope)) return rc;
    if (batch < 1) return fail(MX_ATTN_INVALID_ARGUMENT, "batch (%d) must be >= 1", batch);
    if (d.n_q != 1) return fail(MX_ATTN_INVALID_ARGUMENT, "n_q (%d) must be 1: one new token per sequence", d.n_q);
    // the same k/v cache under two sequences would be appended twice at different positions
    for (int32_t b = 0; b < batch && k_caches && v_caches; b++)
        for (int32_t c = 0; c < b; c++)
            if (k_caches[b] == k_caches[c] || v_caches[b] == v_caches[c])
                return fail(MX_ATTN_INVALID_ARGUMENT, "sequences %d and %d share a cache: each sequence appends to its own", c, b);
    return decode_impl(desc, batch, kv_len, qkv, reinterpret_cast<const void * const *>(k_caches),
                       reinterpret_cast<const void * const *>(v_caches), out, lse, workspace, ws_bytes, stream, rope, true);
}

MX_ATTN_API size_t mx_linear_workspace_bytes(const mx_linear_desc * desc) {
    if (!desc) {
        fail(MX_ATTN_INVALID_ARGUMENT, "desc is null");
        return 0;
    }
    return linear_ws_bytes(*desc);
}

MX_ATTN_API int32_t mx_linear(const mx_linear_desc * desc, int32_t count, const uint16_t * const * W, const float * X,
                              void * const * Y, const float * gamma, const float * const * bias, void * workspace,
                              size_t ws_bytes, mx_attn_stream stream) {
    mx::LinearParams p;
    if (int32_t rc = linear_params(desc, count, W, X, Y, gamma, bias, workspace, ws_bytes, p)) return rc;
    if (desc->M == 0) return MX_ATTN_OK;
    return hip_status(mx::launch_linear(p, static_cast<hipStream_t>(stream)), "linear launch");
}

}  // extern "C"
