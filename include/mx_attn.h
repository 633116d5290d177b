/*
 * mx_attn.h — C ABI of the MI355X (gfx950) attention hot path.
 *
 * Drop-in for the attention step of dooms.cpp's fixed-model decoders. The reference encodes its attention as Metal
 * dispatches with a parameter struct and raw buffers; this header replaces them with plain C entry points that take a
 * descriptor, device pointers and a HIP stream:
 *
 *   reference (file:line, relative to the dooms.cpp 0.6.1 tree)                      replaced by
 *   -------------------------------------------------------------------------------   -----------------------------
 *   attention_prefill<64|128>  src/backend/metal/llama_kernels.h:640-769,              mx_attn_prefill
 *       dispatched by MetalLlamaDecoder::Impl::attention                               (causal GQA, chunk offset p0)
 *       src/backend/metal/metal_llama_decoder.mm:284-296
 *   attention (per-query causal)  llama_kernels.h:552-630, dispatched at               mx_attn_decode (n_q rows,
 *       metal_llama_decoder.mm:298-306 and metal_whisper_decoder.mm:167-203            causal = 1)
 *   attention_split + attention_combine  llama_kernels.h:856-929, dispatched at        mx_attn_decode (split-KV +
 *       metal_llama_decoder.mm:252-271 and metal_whisper_decoder.mm:205-225            log-sum-exp merge)
 *   partial buffer split_part  metal_llama_decoder.mm:672-677                          mx_attn_decode_workspace_bytes
 *   dooms_last_error / dooms_code  include/dooms/dooms_c.h:24-36                       mx_attn_last_error / MX_ATTN_*
 *   AttnParams / SplitParams  llama_kernels.h:496-507, 844-854                         mx_attn_desc
 *   IR SelfAttention (packed [B,N,3E], no mask)  src/ir/op.h:31-32, lowered at          mx_self_attention
 *       src/backend/ggml/ggml_backend.cpp:398-412
 *
 * What the boundary takes over from the reference and what it leaves to the caller:
 *   - Q, K, V and the output are IEEE binary16 (passed as uint16_t bit patterns, so the header needs no half type);
 *     scores, the softmax statistics and the accumulation are f32. The reference keeps q/out in f32 and rounds q to half
 *     inside the prefill kernel (llama_kernels.h:660); here the caller hands over half already.
 *   - Rotary embedding and the cache append (rope_store, llama_kernels.h:520-545) happen before the call: K/V rows for
 *     every position the call reads are already in the caches, Q is already rotated.
 *   - Caches follow the reference layout: row `pos` of a layer's cache holds n_head_kv * head_dim halves (head kvh at
 *     column kvh * head_dim), consecutive rows kv_stride elements apart (metal_llama_decoder.mm:664,
 *     llama_kernels.h:535,593). Query row r holds n_head * head_dim halves, head h at column h * head_dim; rows
 *     q_stride apart. Output rows likewise with out_stride.
 *   - Query head h reads key/value head h / (n_head / n_head_kv) (llama_kernels.h:560,656,873).
 *
 * Threading: every call is asynchronous and ordered on `stream`; nothing inside synchronizes with the host. Calls on
 * distinct streams with distinct output/workspace buffers may run concurrently. The library allocates no device memory.
 *
 * Errors: entry points return one of the MX_ATTN_* codes (numbering of dooms_code, dooms_c.h:24-33) and never abort; the
 * message of the last failure on the calling thread is returned by mx_attn_last_error().
 */
#ifndef MX_ATTN_H
#define MX_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MX_ATTN_API __attribute__((visibility("default")))
#define MX_ATTN_ABI_VERSION 3

/* Return codes: the numbering of dooms_code (include/dooms/dooms_c.h:24-33). */
#define MX_ATTN_OK 0
#define MX_ATTN_INVALID_ARGUMENT 1    /* null pointer, bad stride, n_head % n_head_kv != 0, kv_len < n_q, ... */
#define MX_ATTN_UNSUPPORTED 4         /* head_dim not a power of two in [4, 256], or a shape one launch cannot hold */
#define MX_ATTN_RESOURCE_EXHAUSTED 5  /* the workspace is smaller than mx_attn_decode_workspace_bytes asks for */
#define MX_ATTN_INTERNAL 7            /* the HIP runtime reported an error (launch failure, ...) */

/* A HIP stream (hipStream_t); NULL is the legacy default stream. */
typedef void * mx_attn_stream;

/*
 * Launch-plan choices a decoder may fix in its configuration instead of taking the library's plan: the counterpart of
 * the reference's per-decoder tuning fields WhisperDecoderConfig::cross_splits (src/backend/whisper_text_decoder.h:25)
 * and LlamaDecoderConfig::prefill_tile (src/backend/metal/metal_llama_decoder.h:37). Every field's 0 means "the
 * library's plan"; results agree within the tolerance whatever the plan (only the summation order changes). The
 * library reads no environment variable: these fields are the only way to change a plan.
 */
typedef struct mx_attn_tuning {
    int32_t decode_splits;         /* decode: splits of each sequence's keys, 1..64 (cross_splits); 0: planned */
    int32_t decode_waves;          /* decode: waves per workgroup, 4 or 8; 0: planned */
    int32_t decode_max_workgroups; /* decode: workgroup cap of one launch for the split plan, >= 1; 0: 1536 */
    int32_t prefill_plan;          /* flash prefill workgroups (prefill_tile): 8 = 8 waves x 32 query rows, 4 = 4 waves x
                                      32 rows, 2 = 4 waves over 2 row tiles splitting each tile's key blocks; 0: planned */
    int32_t prefill_stream;        /* the 8-wave plan's stream-K split over the CUs (mx_attn_prefill_ws and
                                      mx_attn_prefill_rope_ws only): 1 whenever it applies, -1 never, 0: planned */
} mx_attn_tuning;

/*
 * One attention problem: a superset of the reference's AttnParams (llama_kernels.h:496-507) without the rotary fields,
 * plus the non-causal key count of SplitParams (llama_kernels.h:844-854).
 */
typedef struct mx_attn_desc {
    int32_t n_head;      /* query heads */
    int32_t n_head_kv;   /* key/value heads; n_head % n_head_kv == 0 */
    int32_t head_dim;    /* a power of two in [4, 256] (metal_llama_decoder.mm:432-435) */
    int32_t n_q;         /* query rows (per sequence for mx_attn_decode) */
    int32_t p0;          /* mx_attn_prefill: cache position of query row 0 (the chunk offset); decode: ignored */
    int32_t n_kv;        /* mx_attn_prefill: keys in the cache (0 means p0 + n_q); decode: ignored (kv_len[]) */
    int32_t causal;      /* 1: query row t sees keys j <= p0 + t (prefill) or j <= kv_len - n_q + t (decode); 0: all */
    int32_t reserved;    /* must be 0 */
    int64_t q_stride;    /* elements between query rows   (>= n_head * head_dim) */
    int64_t kv_stride;   /* elements between cache rows   (>= n_head_kv * head_dim) */
    int64_t out_stride;  /* elements between output rows  (>= n_head * head_dim) */
    float scale;         /* score scale, normally 1 / sqrt(head_dim); 0 is valid (uniform attention) */
    const mx_attn_tuning * tuning;  /* NULL: the library's plans; else read during the call only */
} mx_attn_desc;

/* MX_ATTN_ABI_VERSION of the library. */
MX_ATTN_API int32_t mx_attn_abi_version(void);

/* Message of the last failure on this thread ("" if none). Replaces dooms_last_error (dooms_c.h:36). */
MX_ATTN_API const char * mx_attn_last_error(void);

/*
 * Prefill (prompt chunk) flash attention. Replaces attention_prefill<64|128> (llama_kernels.h:640-769) as dispatched by
 * MetalLlamaDecoder::Impl::attention(enc, cache_off, M, p0, fused_rope = false) (metal_llama_decoder.mm:284-296), and the
 * reference's chunked prompt loop against the growing cache (metal_llama_decoder.mm:703-723).
 *
 *   q       [n_q rows][q_stride]            query row t is at position p0 + t
 *   k_cache [n_kv rows][kv_stride]          keys 0 .. n_kv - 1 (for a causal chunk n_kv = p0 + n_q)
 *   v_cache [n_kv rows][kv_stride]
 *   out     [n_q rows][out_stride]          softmax(scale * q k^T + mask) v per head, rounded to half
 *   lse     [n_q rows][n_head] f32, or NULL: natural-log log-sum-exp of the scaled, masked scores of each row
 *
 * All pointers are device pointers. No workspace is needed.
 */
MX_ATTN_API int32_t mx_attn_prefill(const mx_attn_desc * desc, const uint16_t * q, const uint16_t * k_cache,
                                    const uint16_t * v_cache, uint16_t * out, float * lse, mx_attn_stream stream);

/*
 * mx_attn_prefill with a workspace: a chunk of few rows (n_q * n_head / n_head_kv <= 512, or <= 1024 with at least 64
 * keys per query row) runs on the split-KV decode kernel, which spreads a long cache over the whole chip (the flash
 * kernel has one workgroup per head and 256 query rows, each walking every key): for example 16 rows of a
 * 28 q / 4 kv-head model at 30k keys, 611 -> 74 us. Larger chunks,
 * and any call with workspace == NULL, run the flash kernel exactly as mx_attn_prefill. Same arguments, semantics and
 * results within the stated tolerance (the summation order differs). No counterpart in the reference, whose chunks
 * always take attention_prefill; the extra argument is the decode workspace:
 *
 *   workspace  device, 256-byte aligned, at least mx_attn_prefill_workspace_bytes(desc) bytes, zeroed once by
 *              mx_attn_decode_workspace_init; every call leaves its counters at zero. Calls sharing it (with each other
 *              or with mx_attn_decode) must be ordered on one stream. NULL runs the flash kernel.
 */
MX_ATTN_API int32_t mx_attn_prefill_ws(const mx_attn_desc * desc, const uint16_t * q, const uint16_t * k_cache,
                                       const uint16_t * v_cache, uint16_t * out, float * lse, void * workspace,
                                       size_t ws_bytes, mx_attn_stream stream);

/* Workspace bytes mx_attn_prefill_ws and mx_attn_prefill_rope_ws need for desc (0 when the chunk runs on the flash
 * kernel); 0 and the last error set for an invalid descriptor. */
MX_ATTN_API size_t mx_attn_prefill_workspace_bytes(const mx_attn_desc * desc);

/*
 * Decode attention over per-sequence caches: split-KV over the keys, then a log-sum-exp merge of the splits. Replaces the
 * per-query `attention` kernel (llama_kernels.h:552-630; decode dispatch metal_llama_decoder.mm:298-306, Whisper self
 * attention metal_whisper_decoder.mm:167-203) and attention_split + attention_combine (llama_kernels.h:856-929; long
 * decode metal_llama_decoder.mm:252-271, Whisper cross-attention metal_whisper_decoder.mm:205-225).
 *
 *   batch            sequences (>= 1)
 *   kv_len           HOST array [batch]: keys in sequence b's cache (>= n_q when causal, >= 1 otherwise)
 *   q                device, [batch * n_q rows][q_stride]: row b * n_q + t is query t of sequence b
 *   k_caches         HOST array [batch] of device pointers to sequence b's key cache ([kv_len[b]][kv_stride])
 *   v_caches         HOST array [batch] of device pointers to sequence b's value cache
 *                    (entries may repeat: beam search over one shared cross-attention cache)
 *   out              device, [batch * n_q rows][out_stride]
 *   lse              device, [batch * n_q rows][n_head] f32 natural-log LSE, or NULL
 *   workspace        device scratch of at least mx_attn_decode_workspace_bytes(desc, batch, max_b kv_len[b]) bytes,
 *                    256-byte aligned, zeroed once by mx_attn_decode_workspace_init before its first use: it holds
 *                    split counters that every call leaves at zero again. Calls that share a workspace must be
 *                    ordered on one stream. NULL is allowed when the size needed is 0.
 *
 * With causal = 1 query row t of sequence b attends keys 0 .. kv_len[b] - n_q + t (the decoder's prompt rows appended
 * at the end of the cache, as the reference's per-query kernel with p0 = kv_len - n_q); with causal = 0 every row
 * attends all kv_len[b] keys (cross-attention, or one decode row). desc->p0 and desc->n_kv are ignored.
 * MX_ATTN_UNSUPPORTED when one sequence has more than 2048 (kv head, 16-row tile) pairs, n_head * n_q beyond about
 * 32768 query rows (a prompt that size is a prefill).
 */
MX_ATTN_API int32_t mx_attn_decode(const mx_attn_desc * desc, int32_t batch, const int32_t * kv_len, const uint16_t * q,
                                   const uint16_t * const * k_caches, const uint16_t * const * v_caches, uint16_t * out,
                                   float * lse, void * workspace, size_t ws_bytes, mx_attn_stream stream);

/*
 * mx_attn_decode without a workspace argument: the split partials and counters live in a device array the library
 * holds, MX_ATTN_SCRATCH_BYTES on each GPU it runs on (until the process ends). No counterpart in the reference; it is
 * for callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): it calls no hipMalloc, hipFree or other allocating routine. Arguments and results as mx_attn_decode.
 *
 * Returns MX_ATTN_RESOURCE_EXHAUSTED when the shape needs more scratch than that (mx_attn_decode_workspace_bytes >
 * MX_ATTN_SCRATCH_BYTES; e.g. 32 Llama-3-8B sequences at 8192 keys need 17 MB). All calls on one GPU share its array,
 * which each call leaves ready for the next: calls that overlap on one GPU (concurrent streams) race, so order them
 * on one stream. The first call on a GPU initialises the array with a kernel on its stream; a call on another stream
 * must be ordered after that one.
 */
#define MX_ATTN_SCRATCH_BYTES ((size_t)16 << 20)
MX_ATTN_API int32_t mx_attn_decode_noalloc(const mx_attn_desc * desc, int32_t batch, const int32_t * kv_len,
                                           const uint16_t * q, const uint16_t * const * k_caches,
                                           const uint16_t * const * v_caches, uint16_t * out, float * lse,
                                           mx_attn_stream stream);

/*
 * mx_attn_decode on the reference's f32 buffers: q rows and the output are f32 (q_stride / out_stride in floats), the
 * caches f16; the query is rounded to half in the kernel. Replaces attention_split + attention_combine on the Whisper
 * decoder's f32 q / attn buffers (metal_whisper_decoder.mm:205-225, llama_kernels.h:856-929) and the per-query
 * `attention` kernel without fused_rope (llama_kernels.h:552-630). Everything else as mx_attn_decode.
 */
MX_ATTN_API int32_t mx_attn_decode_f32(const mx_attn_desc * desc, int32_t batch, const int32_t * kv_len, const float * q,
                                       const uint16_t * const * k_caches, const uint16_t * const * v_caches, float * out,
                                       float * lse, void * workspace, size_t ws_bytes, mx_attn_stream stream);

/* Rotary embedding of the fused decode step: the reference's AttnParams.neox / base (llama_kernels.h:501-506). */
typedef struct mx_attn_rope {
    int32_t mode; /* 0: adjacent pairs (2i, 2i + 1), llama.cpp's "normal" (llama); 1: split halves (i, i + head_dim / 2),
                     "neox" (qwen2); 2: none (positions come from a learned table, as in Whisper) */
    float base;   /* frequency base (rope.freq_base); pair i of position pos turns by pos * base^(-2i / head_dim) */
} mx_attn_rope;

/*
 * The fused decode step: rotary embedding of the new token's query and key, append of its key and value to the caches,
 * and decode attention, in one launch. Replaces the reference's `attention` kernel with fused_rope = 1
 * (llama_kernels.h:552-630, dispatched by MetalLlamaDecoder::Impl::attention at metal_llama_decoder.mm:298-306), and
 * rope_store + attention_split + attention_combine for long caches (llama_kernels.h:521-549, 856-929;
 * metal_llama_decoder.mm:241-271).
 *
 *   rope             rotary layout and base (mode 2: no rotation, the Whisper decoder's self-attention step)
 *   kv_len           HOST array [batch]: keys of sequence b INCLUDING the new token, which goes to position kv_len[b] - 1
 *   qkv              device, f32, [batch rows][q_stride floats]: the reference's q | k | v projection row of sequence b's
 *                    new token, unrotated: n_head query heads, then n_head_kv key heads, then n_head_kv value heads
 *   k_caches         HOST array [batch] of device pointers to distinct key caches, written at row kv_len[b] - 1 with the
 *                    rotated key rounded to half (as the reference's rope_store / fused attention store it)
 *   v_caches         the same for the values
 *   out              device, f32, [batch rows][out_stride floats] (the reference's attention output is f32)
 *   lse, workspace   as for mx_attn_decode
 *
 * desc->n_q must be 1 and desc->causal is irrelevant (one row sees every key). The query is rotated in f32 and then
 * rounded to half for the matrix cores; positions below kv_len[b] - 1 are read from the caches as they stand.
 */
MX_ATTN_API int32_t mx_attn_decode_rope(const mx_attn_desc * desc, const mx_attn_rope * rope, int32_t batch,
                                        const int32_t * kv_len, const float * qkv, uint16_t * const * k_caches,
                                        uint16_t * const * v_caches, float * out, float * lse, void * workspace,
                                        size_t ws_bytes, mx_attn_stream stream);

/*
 * The reference's prompt path on its own buffers: rope_store of the chunk's keys and values into the caches, then
 * flash attention of its query rows read from the f32 q|k|v rows (rotated and rounded to half in the kernel, as the
 * reference rounds q at llama_kernels.h:660). Replaces rope_store + attention_prefill<64|128> (llama_kernels.h:520-545,
 * 632-769) as dispatched by MetalLlamaDecoder::Impl::attention(enc, cache_off, M, p0, fused_rope = false)
 * (metal_llama_decoder.mm:276-296), and with rope->mode = 2 the Whisper prompt (metal_whisper_decoder.mm:182-203).
 *
 *   qkv     device, f32, [n_q rows][q_stride floats]: token t (position p0 + t) as q | k | v, unrotated
 *   k_cache [n_kv rows][kv_stride] f16: rows p0 .. p0 + n_q - 1 are written (rotated keys), then all rows visible to a
 *           query are read; n_kv (0: p0 + n_q) must cover the chunk
 *   v_cache the same for the values
 *   out     device, f32, [n_q rows][out_stride floats]
 *   lse     as for mx_attn_prefill
 *
 * Two launches on `stream` (the cache write, then the attention); no workspace.
 */
MX_ATTN_API int32_t mx_attn_prefill_rope(const mx_attn_desc * desc, const mx_attn_rope * rope, const float * qkv,
                                         uint16_t * k_cache, uint16_t * v_cache, float * out, float * lse,
                                         mx_attn_stream stream);

/*
 * mx_attn_prefill_rope with a workspace (sized by mx_attn_prefill_workspace_bytes, zeroed once by
 * mx_attn_decode_workspace_init; NULL runs mx_attn_prefill_rope): a chunk of few rows (n_q * n_head / n_head_kv <= 512)
 * writes its keys and values into the caches and its rotated query rows into the workspace, then attends on the
 * split-KV decode kernel, as mx_attn_prefill_ws does. No counterpart in the reference.
 */
MX_ATTN_API int32_t mx_attn_prefill_rope_ws(const mx_attn_desc * desc, const mx_attn_rope * rope, const float * qkv,
                                            uint16_t * k_cache, uint16_t * v_cache, float * out, float * lse,
                                            void * workspace, size_t ws_bytes, mx_attn_stream stream);

/*
 * Zero-fills a decode workspace on `stream` (with a kernel, not a memset, so that a caller may capture it in a HIP
 * graph). Call it once after allocating the workspace; mx_attn_decode keeps it ready for the next call. It has no
 * counterpart in the reference, whose split partials need no counters (attention_combine runs as a second dispatch,
 * llama_kernels.h:912-929); here the merge runs in the split kernel itself.
 */
MX_ATTN_API int32_t mx_attn_decode_workspace_init(void * workspace, size_t ws_bytes, mx_attn_stream stream);

/*
 * Workspace bytes mx_attn_decode needs for `batch` sequences of at most max_kv_len keys (the reference sizes its
 * split_part buffer the same way from n_ctx: metal_llama_decoder.mm:672-677). Returns 0 and sets the last error for an
 * invalid descriptor.
 */
MX_ATTN_API size_t mx_attn_decode_workspace_bytes(const mx_attn_desc * desc, int32_t batch, int32_t max_kv_len);

/* Element types of mx_self_attention's tensors: the order of the reference's DType (src/core/dtype.h:13). */
#define MX_ATTN_F32 0
#define MX_ATTN_F16 1
#define MX_ATTN_BF16 2

/*
 * The IR's SelfAttention op (src/ir/op.h:31-32, 64-71): packed q|k|v rows [batch][n_tok][3 embed] -> [batch][n_tok][embed],
 * per head softmax(scale * q k^T) v, no mask, head h the h-th run of head_dim = embed / heads values of each third.
 */
typedef struct mx_self_attn_desc {
    int32_t batch;   /* B, 1 .. 65535 */
    int32_t n_tok;   /* N >= 0 (0: nothing to do) */
    int32_t heads;   /* >= 1 (self_attention_params, src/ir/op.cpp:69-76) */
    int32_t embed;   /* E, a multiple of heads (infer_self_attention, src/ir/shape_infer.cpp:156-171); head_dim <= 128 */
    int32_t dtype;   /* MX_ATTN_F32, MX_ATTN_F16 or MX_ATTN_BF16: of qkv and of y (the op keeps the input's dtype) */
    float scale;     /* finite; multiplies q k^T before the softmax (0: uniform attention) */
    const mx_attn_tuning * tuning;  /* NULL, or prefill_plan fixes the workgroup plan (the decode fields are unused) */
} mx_self_attn_desc;

/*
 * Device workspace bytes mx_self_attention needs: 0 when head_dim is a multiple of 8 (the kernel reads the packed rows
 * in place in every dtype, rounding Q, K and V to half as it loads them, as the reference's GPU path rounds them,
 * ggml_backend.cpp:332-335); for any other head_dim the operands padded to head_dim 64 or 128. Returns 0 and sets the
 * last error for an invalid descriptor.
 */
MX_ATTN_API size_t mx_self_attention_workspace_bytes(const mx_self_attn_desc * desc);

/*
 * SelfAttention on the GPU. Replaces the reference's lowering of the op (ggml_backend.cpp:398-412: the fused
 * ggml_flash_attn_ext of lower_attention_fused, :325-340, the unfused chain of :342-356 for head dims flash attention does
 * not take, and the CPU op attention_cpu_op, :292-312). One prefill-kernel launch (non-causal, every batch element along
 * the grid) on the packed rows, plus a packing launch before and an unpacking launch after it when head_dim is not a
 * multiple of 8. Scores and accumulation are f32 over half operands (as the reference's GPU path, which rounds Q/K/V to
 * half).
 *
 *   qkv        device, [batch][n_tok][3 embed] of desc->dtype, contiguous, 16-byte aligned
 *   y          device, [batch][n_tok][embed] of desc->dtype, contiguous, 16-byte aligned, not overlapping qkv
 *   workspace  device, 256-byte aligned, at least mx_self_attention_workspace_bytes(desc) bytes (NULL when that is 0)
 */
MX_ATTN_API int32_t mx_self_attention(const mx_self_attn_desc * desc, const void * qkv, void * y, void * workspace,
                                      size_t ws_bytes, mx_attn_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* MX_ATTN_H */
