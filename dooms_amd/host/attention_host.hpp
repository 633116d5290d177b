// C++ host layer above the C ABI (include/mx_attn.h): the attention step of dooms.cpp's fixed-model decoders, with the
// reference's call shapes, so that a decoder written against the reference's interface calls this instead.
//
//   reference (dooms.cpp 0.6.1)                                               here
//   MetalLlamaDecoder::Impl::attention(enc, cache_off, M, p0, false)          LlamaAttention::attention(layer, q, out, M, p0)
//   MetalLlamaDecoder::Impl::attention(enc, cache_off, 1, p, true)            LlamaAttention::decode_step(layer, qkv, out, p)
//     (and with rope_store for a prompt chunk, f32 q|k|v rows)               LlamaAttention::prompt(layer, qkv, out, M, p0)
//     (src/backend/metal/metal_llama_decoder.mm:238-307)
//   MetalWhisperDecoder::Impl::self_attention(cache_off, p)                    WhisperAttention::self_attention(layer, q, out, p)
//   MetalWhisperDecoder::Impl::self_attention_prompt(cache_off, p0, M)         WhisperAttention::self_attention_prompt(...)
//   MetalWhisperDecoder::Impl::cross_attention(cache_off, M)                   WhisperAttention::cross_attention(layer, q, out, M)
//     (src/backend/metal/metal_whisper_decoder.mm:167-225); each also on the reference's own f32 buffers (overloads
//     taking float q|k|v rows and float output: the cache write of the step / prompt happens in the library)
//   MetalLlamaDecoder::profile_pass / MetalWhisperDecoder::profile_step      set_profile(&times) + the calls; KernelTime
//     (metal_llama_decoder.mm:789-812, metal_whisper_decoder.mm:613-626)
//   Status / Code (src/core/status.h:13-81)                                     Status / Code below (same numbering)
//
// The caches keep the reference's layout: per layer [n_ctx][n_head_kv * head_dim] f16, layer l at l * n_ctx rows
// (metal_llama_decoder.mm:657-667; the Whisper self cache [n_text_ctx][n_state] and cross cache [n_audio_ctx][n_state],
// metal_whisper_decoder.mm:460-461). The caller owns them. Rotary embedding is the caller's (the reference's
// rope_store, llama_kernels.h:520-545) for prompt chunks: q arrives rotated, and append() copies rotated keys/values
// into the cache rows; decode_step() is the reference's fused_rope decode (rotation and cache write in the kernel). Like the reference's decoders these objects are not thread-safe; all work is
// ordered on the stream given at create, and nothing synchronizes with the host except create/destroy and calls made while profiling.
//
// Header-only: include it, link libmx_attn.so and the HIP runtime.
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "mx_attn.h"

namespace dooms_amd {

enum class Code : int32_t {  // the numbering of dooms::Code / dooms_code for the codes this layer can return
    Ok = MX_ATTN_OK,
    InvalidArgument = MX_ATTN_INVALID_ARGUMENT,
    Unsupported = MX_ATTN_UNSUPPORTED,
    ResourceExhausted = MX_ATTN_RESOURCE_EXHAUSTED,
    Internal = MX_ATTN_INTERNAL,
};

struct Status {
    Code code = Code::Ok;
    std::string message;
    bool is_ok() const { return code == Code::Ok; }
    static Status from(int32_t rc) { return rc == MX_ATTN_OK ? Status{} : Status{Code(rc), mx_attn_last_error()}; }
    static Status hip(hipError_t e, const char * what) {
        return e == hipSuccess ? Status{} : Status{Code::Internal, std::string(what) + ": " + hipGetErrorString(e)};
    }
};

// Decode workspace owned by a decoder (allocated at create, as the reference allocates split_part,
// metal_llama_decoder.mm:672-677).
class Workspace {
public:
    Workspace() = default;
    Workspace(const Workspace &) = delete;
    Workspace & operator=(const Workspace &) = delete;
    ~Workspace() {
        if (ptr_) (void)hipFree(ptr_);
    }
    Status reserve(size_t bytes, hipStream_t stream) {
        if (bytes <= bytes_) return {};
        if (ptr_) (void)hipFree(ptr_);
        ptr_ = nullptr;
        bytes_ = 0;
        if (Status st = Status::hip(hipMalloc(&ptr_, bytes), "workspace allocation"); !st.is_ok()) {
            ptr_ = nullptr;
            return Status{Code::ResourceExhausted, st.message};
        }
        bytes_ = bytes;
        return Status::from(mx_attn_decode_workspace_init(ptr_, bytes_, stream));
    }
    void * data() const { return ptr_; }
    size_t size() const { return bytes_; }

private:
    void * ptr_ = nullptr;
    size_t bytes_ = 0;
};

// GPU time of one kind of call over a profiling pass (MetalLlamaDecoder::KernelTime, metal_llama_decoder.h:99).
struct KernelTime {
    std::string kind;
    int32_t dispatches = 0;
    double gpu_ms = 0.0;
};

// Per-kind timing of a decoder's calls, for profiling passes in the manner of the reference's after_dispatch
// (metal_llama_decoder.mm:118-135) and cut (metal_whisper_decoder.mm:98-103): while a vector is attached, every call
// is bracketed by two events on the decoder's stream and waited for (so it runs alone), and its time is added to its
// kind's entry. Detached (the default) it creates no events and adds no waits.
class DispatchTimer {
public:
    DispatchTimer() = default;
    DispatchTimer(const DispatchTimer &) = delete;
    DispatchTimer & operator=(const DispatchTimer &) = delete;
    ~DispatchTimer() {
        for (hipEvent_t e : ev_)
            if (e) (void)hipEventDestroy(e);
    }
    void attach(std::vector<KernelTime> * out) { out_ = out; }
    bool attached() const { return out_ != nullptr; }

    template <class F> Status run(const char * kind, hipStream_t stream, F && call) {
        if (!out_) return call();
        for (hipEvent_t & e : ev_)
            if (!e)
                if (Status st = Status::hip(hipEventCreate(&e), "profiling event"); !st.is_ok()) return st;
        if (Status st = Status::hip(hipEventRecord(ev_[0], stream), "profiling event"); !st.is_ok()) return st;
        if (Status st = call(); !st.is_ok()) return st;
        if (Status st = Status::hip(hipEventRecord(ev_[1], stream), "profiling event"); !st.is_ok()) return st;
        if (Status st = Status::hip(hipEventSynchronize(ev_[1]), "profiling wait"); !st.is_ok()) return st;
        float ms = 0.f;
        if (Status st = Status::hip(hipEventElapsedTime(&ms, ev_[0], ev_[1]), "profiling time"); !st.is_ok()) return st;
        auto it = std::find_if(out_->begin(), out_->end(), [&](const KernelTime & k) { return k.kind == kind; });
        if (it == out_->end()) out_->push_back({kind, 1, (double)ms});
        else {
            it->dispatches++;
            it->gpu_ms += ms;
        }
        return {};
    }

private:
    std::vector<KernelTime> * out_ = nullptr;
    hipEvent_t ev_[2] = {nullptr, nullptr};
};

// ---- llama / Qwen2 ----

struct LlamaAttentionConfig {  // the attention fields of LlamaDecoderConfig (metal_llama_decoder.h:20-39)
    int32_t n_layer = 0;
    int32_t n_ctx = 0;       // positions per layer cache
    int32_t n_head = 0;
    int32_t n_head_kv = 0;
    int32_t head_dim = 0;    // a power of two in [4, 256]
    float rope_base = 10000.f;  // rotary frequency base (rope.freq_base)
    bool rope_neox = false;     // rotary pairs (i, i + head_dim / 2) (qwen2) instead of (2i, 2i + 1) (llama)
    int32_t n_batch = 0;        // the largest prompt chunk prompt() is given (n_batch, metal_llama_decoder.h:33); 0: 2048
    // Launch plans fixed for measuring, as the reference's prefill_tile (metal_llama_decoder.h:35-37); all 0: the
    // library's plans. Not model metadata.
    mx_attn_tuning tuning{};
};

class LlamaAttention {
public:
    //   InvalidArgument  bad sizes or null caches     Unsupported  head_dim not a power of two in [4, 256]
    //   ResourceExhausted  workspace
    static Status create(const LlamaAttentionConfig & c, uint16_t * k_cache, uint16_t * v_cache, hipStream_t stream,
                         std::unique_ptr<LlamaAttention> & out) {
        if (c.n_layer < 1 || c.n_ctx < 1 || c.n_head < 1 || c.n_head_kv < 1 || c.head_dim < 1)
            return {Code::InvalidArgument, "n_layer, n_ctx, n_head, n_head_kv and head_dim must be >= 1"};
        if (!k_cache || !v_cache) return {Code::InvalidArgument, "caches must not be null"};
        if (c.n_head % c.n_head_kv) return {Code::InvalidArgument, "n_head must be a multiple of n_head_kv"};
        if (c.head_dim < 4 || c.head_dim > 256 || (c.head_dim & (c.head_dim - 1)) != 0)  // metal_llama_decoder.mm:432-435
            return {Code::Unsupported, "head_dim must be a power of two in [4, 256], got " + std::to_string(c.head_dim)};
        std::unique_ptr<LlamaAttention> a(new LlamaAttention(c, k_cache, v_cache, stream));
        // one workspace for the decode rows and for the prompt chunks of few rows that mx_attn_prefill_ws runs on the
        // split-KV kernel (up to 512, or with a long enough cache 1024, rows per kv head), at the full context
        mx_attn_desc d = a->desc(1, 0, 0);
        size_t bytes = mx_attn_decode_workspace_bytes(&d, 1, c.n_ctx);
        for (int32_t rows : {512, 1024}) {
            const int32_t m_split = std::min<int32_t>(c.n_ctx, std::max(1, rows / (c.n_head / c.n_head_kv)));
            mx_attn_desc dp = a->desc(m_split, 0, 0);
            dp.p0 = c.n_ctx - m_split;
            dp.causal = 1;
            bytes = std::max(bytes, mx_attn_prefill_workspace_bytes(&dp));
        }
        // and the flash kernel's stream-K slots, when its plan splits the largest chunk over the CUs (at the end of the
        // context, where its tiles are longest; a chunk that finds the workspace short of them runs unsplit)
        const int32_t n_batch = std::min<int32_t>(c.n_ctx, c.n_batch > 0 ? c.n_batch : 2048);
        mx_attn_desc db = a->desc(n_batch, 0, 0);
        db.p0 = c.n_ctx - n_batch;
        db.causal = 1;
        bytes = std::max(bytes, mx_attn_prefill_workspace_bytes(&db));
        if (Status st = a->ws_.reserve(bytes, stream); !st.is_ok()) return st;
        out = std::move(a);
        return {};
    }

    const LlamaAttentionConfig & config() const { return cfg_; }
    // Profiling (null: off): the calls made meanwhile add their GPU time under "cache k/v" (append), "attention"
    // (attention, decode_step) and "rope_store + attention" (prompt), as MetalLlamaDecoder::profile_pass reports by
    // kind (metal_llama_decoder.mm:789-812).
    void set_profile(std::vector<KernelTime> * out) { timer_.attach(out); }
    int32_t kv_width() const { return cfg_.n_head_kv * cfg_.head_dim; }
    int32_t q_width() const { return cfg_.n_head * cfg_.head_dim; }
    uint16_t * k_layer(int32_t l) const { return k_ + (size_t)l * cfg_.n_ctx * kv_width(); }
    uint16_t * v_layer(int32_t l) const { return v_ + (size_t)l * cfg_.n_ctx * kv_width(); }

    // Copies M rows of (rotated) keys and values, rows k_stride / v_stride halves apart, into layer l's cache at
    // positions p0 .. p0 + M - 1 (the cache write of rope_store).   ResourceExhausted  past n_ctx
    Status append(int32_t layer, const uint16_t * k, int64_t k_stride, const uint16_t * v, int64_t v_stride, int32_t M,
                  int32_t p0) {
        if (layer < 0 || layer >= cfg_.n_layer || M < 1 || p0 < 0 || !k || !v)
            return {Code::InvalidArgument, "append: bad layer, rows, position or pointer"};
        if ((int64_t)p0 + M > cfg_.n_ctx) return {Code::ResourceExhausted, "append: the context would overflow"};
        const size_t w = (size_t)kv_width() * 2;
        return timer_.run("cache k/v", stream_, [&]() -> Status {
            if (Status st = Status::hip(hipMemcpy2DAsync(k_layer(layer) + (size_t)p0 * kv_width(), w, k, (size_t)k_stride * 2, w,
                                                         M, hipMemcpyDeviceToDevice, stream_), "append k");
                !st.is_ok())
                return st;
            return Status::hip(hipMemcpy2DAsync(v_layer(layer) + (size_t)p0 * kv_width(), w, v, (size_t)v_stride * 2, w, M,
                                                hipMemcpyDeviceToDevice, stream_), "append v");
        });
    }

    // Attention of M query rows at positions p0 .. p0 + M - 1 of layer l over cache rows 0 .. p0 + M - 1 (already
    // appended): one decode row (M == 1) through the split-KV decode path, a prompt chunk through mx_attn_prefill_ws
    // (flash prefill, or the split-KV kernel for chunks of few rows). q rows are q_stride halves apart, out rows
    // out_stride.
    Status attention(int32_t layer, const uint16_t * q, int64_t q_stride, uint16_t * out, int64_t out_stride, int32_t M,
                     int32_t p0) {
        if (layer < 0 || layer >= cfg_.n_layer) return {Code::InvalidArgument, "layer out of range"};
        if (M < 1 || p0 < 0) return {Code::InvalidArgument, "need M >= 1 rows at a position p0 >= 0"};
        if ((int64_t)p0 + M > cfg_.n_ctx) return {Code::ResourceExhausted, "the context would overflow"};
        const uint16_t * k = k_layer(layer);
        const uint16_t * v = v_layer(layer);
        if (M == 1) {
            mx_attn_desc d = desc(1, q_stride, out_stride);
            d.causal = 0;
            const int32_t n = p0 + 1;
            return timer_.run("attention", stream_, [&] {
                return Status::from(mx_attn_decode(&d, 1, &n, q, &k, &v, out, nullptr, ws_.data(), ws_.size(), stream_));
            });
        }
        mx_attn_desc d = desc(M, q_stride, out_stride);
        d.p0 = p0;
        d.causal = 1;
        return timer_.run("attention", stream_, [&] {
            return Status::from(mx_attn_prefill_ws(&d, q, k, v, out, nullptr, ws_.data(), ws_.size(), stream_));
        });
    }

    // A prompt chunk of M tokens at positions p0 .. p0 + M - 1 on the reference's buffers (rope_store + attention with
    // fused_rope = false, metal_llama_decoder.mm:276-296): qkv holds the chunk's f32 q | k | v rows, unrotated; their
    // keys and values are rotated and written into the layer's cache, and out (f32) gets the causal attention.
    Status prompt(int32_t layer, const float * qkv, float * out, int32_t M, int32_t p0) {
        if (layer < 0 || layer >= cfg_.n_layer) return {Code::InvalidArgument, "layer out of range"};
        if (M < 1 || p0 < 0) return {Code::InvalidArgument, "need M >= 1 rows at a position p0 >= 0"};
        if ((int64_t)p0 + M > cfg_.n_ctx) return {Code::ResourceExhausted, "the context would overflow"};
        mx_attn_desc d = desc(M, q_width() + 2 * kv_width(), q_width());
        d.p0 = p0;
        d.causal = 1;
        const mx_attn_rope rope{cfg_.rope_neox ? 1 : 0, cfg_.rope_base};
        return timer_.run("rope_store + attention", stream_, [&] {
            return Status::from(mx_attn_prefill_rope_ws(&d, &rope, qkv, k_layer(layer), v_layer(layer), out, nullptr,
                                                        ws_.data(), ws_.size(), stream_));
        });
    }

    // One decode step of layer l at position p, the reference's attention(enc, cache_off, 1, p, fused_rope = true)
    // (metal_llama_decoder.mm:298-306): qkv is the new token's f32 q | k | v projection row, unrotated; q and k are
    // rotated for position p, k and v are written into the layer's cache at p, and out (f32, q_width floats) gets the
    // attention over positions 0 .. p.   ResourceExhausted  p past n_ctx
    Status decode_step(int32_t layer, const float * qkv, float * out, int32_t p) {
        if (layer < 0 || layer >= cfg_.n_layer) return {Code::InvalidArgument, "layer out of range"};
        if (p < 0) return {Code::InvalidArgument, "position must be >= 0"};
        if (p >= cfg_.n_ctx) return {Code::ResourceExhausted, "the context would overflow"};
        mx_attn_desc d = desc(1, q_width() + 2 * kv_width(), q_width());
        d.causal = 0;
        const mx_attn_rope rope{cfg_.rope_neox ? 1 : 0, cfg_.rope_base};
        const int32_t n = p + 1;
        uint16_t * k = k_layer(layer);
        uint16_t * v = v_layer(layer);
        return timer_.run("attention", stream_, [&] {
            return Status::from(mx_attn_decode_rope(&d, &rope, 1, &n, qkv, &k, &v, out, nullptr, ws_.data(), ws_.size(), stream_));
        });
    }

private:
    LlamaAttention(const LlamaAttentionConfig & c, uint16_t * k, uint16_t * v, hipStream_t s) : cfg_(c), k_(k), v_(v), stream_(s) {}
    mx_attn_desc desc(int32_t n_q, int64_t q_stride, int64_t out_stride) const {
        mx_attn_desc d{};
        d.n_head = cfg_.n_head;
        d.n_head_kv = cfg_.n_head_kv;
        d.head_dim = cfg_.head_dim;
        d.n_q = n_q;
        d.q_stride = q_stride ? q_stride : q_width();
        d.kv_stride = kv_width();
        d.out_stride = out_stride ? out_stride : q_width();
        d.scale = 1.0f / std::sqrt((float)cfg_.head_dim);
        d.tuning = &cfg_.tuning;
        return d;
    }
    LlamaAttentionConfig cfg_;
    uint16_t * k_;
    uint16_t * v_;
    hipStream_t stream_;
    Workspace ws_;
    DispatchTimer timer_;
};

// ---- Whisper (MHA: n_head_kv = n_head, head_dim = n_state / n_head) ----

struct WhisperAttentionConfig {  // the attention fields of WhisperDecoderConfig (whisper_text_decoder.h:16-30)
    int32_t n_layer = 0;
    int32_t n_state = 0;
    int32_t n_head = 0;
    int32_t n_text_ctx = 0;   // self-attention cache positions (448)
    int32_t n_audio_ctx = 0;  // cross-attention positions (1500)
    int32_t max_rows = 8;     // query rows per call: prompt rows, or beams for cross-attention
    // cross-attention: splits of the audio positions (the reference's cross_splits, whisper_text_decoder.h:25);
    // 0: the library's plan
    int32_t cross_splits = 0;
    mx_attn_tuning tuning{};  // the other plans (its decode_splits applies to self-attention); all 0: the library's
};

class WhisperAttention {
public:
    static Status create(const WhisperAttentionConfig & c, uint16_t * self_k, uint16_t * self_v, uint16_t * cross_k,
                         uint16_t * cross_v, hipStream_t stream, std::unique_ptr<WhisperAttention> & out) {
        if (c.n_layer < 1 || c.n_state < 1 || c.n_head < 1 || c.n_text_ctx < 1 || c.n_audio_ctx < 1 || c.max_rows < 1)
            return {Code::InvalidArgument, "sizes must be >= 1"};
        if (c.cross_splits < 0 || c.cross_splits > 32) return {Code::InvalidArgument, "cross_splits must be in [0, 32]"};
        if (c.n_state % c.n_head) return {Code::InvalidArgument, "n_state must be a multiple of n_head"};
        const int32_t hd = c.n_state / c.n_head;
        // the reference's Whisper decoder takes 64 or 128 (metal_whisper_decoder.mm:342-343)
        if (hd != 64 && hd != 128) return {Code::Unsupported, "head_dim " + std::to_string(hd) + " is not supported (64 or 128)"};
        if (!self_k || !self_v || !cross_k || !cross_v) return {Code::InvalidArgument, "caches must not be null"};
        std::unique_ptr<WhisperAttention> a(new WhisperAttention(c, self_k, self_v, cross_k, cross_v, stream));
        size_t ws = 0;
        for (int32_t causal = 0; causal < 2; causal++) {
            mx_attn_desc d = a->desc(c.max_rows, causal);
            const size_t self_ws = mx_attn_decode_workspace_bytes(&d, 1, c.n_text_ctx);
            const size_t cross_ws = mx_attn_decode_workspace_bytes(&d, 1, c.n_audio_ctx);
            ws = std::max(ws, std::max(self_ws, cross_ws));
        }
        if (Status st = a->ws_.reserve(ws, stream); !st.is_ok()) return st;
        out = std::move(a);
        return {};
    }

    int32_t head_dim() const { return cfg_.n_state / cfg_.n_head; }
    // Profiling (null: off): the calls made meanwhile add their GPU time under "self attention" and "cross
    // attention", the kinds MetalWhisperDecoder::profile_step reports (metal_whisper_decoder.mm:179, 218, 613-626).
    void set_profile(std::vector<KernelTime> * out) { timer_.attach(out); }
    const WhisperAttentionConfig & config() const { return cfg_; }
    uint16_t * self_k(int32_t l) const { return sk_ + (size_t)l * cfg_.n_text_ctx * cfg_.n_state; }
    uint16_t * self_v(int32_t l) const { return sv_ + (size_t)l * cfg_.n_text_ctx * cfg_.n_state; }
    uint16_t * cross_k(int32_t l) const { return ck_ + (size_t)l * cfg_.n_audio_ctx * cfg_.n_state; }
    uint16_t * cross_v(int32_t l) const { return cv_ + (size_t)l * cfg_.n_audio_ctx * cfg_.n_state; }

    // One new token at position p (its key/value already in the self cache): attends positions 0 .. p.
    Status self_attention(int32_t layer, const uint16_t * q, uint16_t * out, int32_t p) {
        if (p < 0 || p >= cfg_.n_text_ctx) return {Code::ResourceExhausted, "text position out of the context"};
        return run(layer, q, out, 1, p + 1, 0, self_k(layer), self_v(layer));
    }
    // M prompt tokens at positions p0 .. p0 + M - 1 (cached): row t attends positions 0 .. p0 + t.
    Status self_attention_prompt(int32_t layer, const uint16_t * q, uint16_t * out, int32_t p0, int32_t M) {
        if (p0 < 0 || M < 1 || (int64_t)p0 + M > cfg_.n_text_ctx) return {Code::ResourceExhausted, "prompt out of the context"};
        return run(layer, q, out, M, p0 + M, 1, self_k(layer), self_v(layer));
    }
    // M query rows (greedy 1, or one per beam) over the layer's n_audio_ctx encoder keys/values.
    Status cross_attention(int32_t layer, const uint16_t * q, uint16_t * out, int32_t M) {
        return run(layer, q, out, M, cfg_.n_audio_ctx, 0, cross_k(layer), cross_v(layer), true);
    }

    // The same three calls on the reference's f32 buffers (metal_whisper_decoder.mm:167-225): qkv rows are
    // q | k | v (3 n_state floats), unrotated (Whisper's positions are learned); the step and the prompt write their
    // keys/values into the self cache themselves; out is f32.
    Status self_attention(int32_t layer, const float * qkv, float * out, int32_t p) {
        if (layer < 0 || layer >= cfg_.n_layer) return {Code::InvalidArgument, "layer out of range"};
        if (p < 0 || p >= cfg_.n_text_ctx) return {Code::ResourceExhausted, "text position out of the context"};
        mx_attn_desc d = desc(1, 0);
        d.q_stride = 3 * cfg_.n_state;
        const mx_attn_rope none{2, 0.f};
        const int32_t n = p + 1;
        uint16_t * k = self_k(layer);
        uint16_t * v = self_v(layer);
        return timer_.run("self attention", stream_, [&] {
            return Status::from(mx_attn_decode_rope(&d, &none, 1, &n, qkv, &k, &v, out, nullptr, ws_.data(), ws_.size(), stream_));
        });
    }
    Status self_attention_prompt(int32_t layer, const float * qkv, float * out, int32_t p0, int32_t M) {
        if (layer < 0 || layer >= cfg_.n_layer) return {Code::InvalidArgument, "layer out of range"};
        if (p0 < 0 || M < 1 || (int64_t)p0 + M > cfg_.n_text_ctx) return {Code::ResourceExhausted, "prompt out of the context"};
        mx_attn_desc d = desc(M, 1);
        d.q_stride = 3 * cfg_.n_state;
        d.p0 = p0;
        const mx_attn_rope none{2, 0.f};
        return timer_.run("self attention", stream_, [&] {
            return Status::from(mx_attn_prefill_rope(&d, &none, qkv, self_k(layer), self_v(layer), out, nullptr, stream_));
        });
    }
    Status cross_attention(int32_t layer, const float * q, float * out, int32_t M) {
        if (layer < 0 || layer >= cfg_.n_layer) return {Code::InvalidArgument, "layer out of range"};
        if (M < 1 || M > cfg_.max_rows) return {Code::InvalidArgument, "rows must be in [1, max_rows]"};
        mx_attn_desc d = desc(M, 0);
        d.tuning = &cross_tuning_;
        const int32_t n = cfg_.n_audio_ctx;
        const uint16_t * k = cross_k(layer);
        const uint16_t * v = cross_v(layer);
        return timer_.run("cross attention", stream_, [&] {
            return Status::from(mx_attn_decode_f32(&d, 1, &n, q, &k, &v, out, nullptr, ws_.data(), ws_.size(), stream_));
        });
    }

private:
    WhisperAttention(const WhisperAttentionConfig & c, uint16_t * sk, uint16_t * sv, uint16_t * ck, uint16_t * cv, hipStream_t s)
        : cfg_(c), sk_(sk), sv_(sv), ck_(ck), cv_(cv), stream_(s), cross_tuning_(c.tuning) {
        cross_tuning_.decode_splits = c.cross_splits;
    }
    mx_attn_desc desc(int32_t n_q, int32_t causal) const {
        mx_attn_desc d{};
        d.n_head = cfg_.n_head;
        d.n_head_kv = cfg_.n_head;
        d.head_dim = head_dim();
        d.n_q = n_q;
        d.causal = causal;
        d.q_stride = d.kv_stride = d.out_stride = cfg_.n_state;
        d.scale = 1.0f / std::sqrt((float)head_dim());
        d.tuning = &cfg_.tuning;
        return d;
    }
    Status run(int32_t layer, const uint16_t * q, uint16_t * out, int32_t M, int32_t n_keys, int32_t causal, const uint16_t * k,
               const uint16_t * v, bool cross = false) {
        if (layer < 0 || layer >= cfg_.n_layer) return {Code::InvalidArgument, "layer out of range"};
        if (M < 1 || M > cfg_.max_rows) return {Code::InvalidArgument, "rows must be in [1, max_rows]"};
        mx_attn_desc d = desc(M, causal);
        if (cross) d.tuning = &cross_tuning_;
        return timer_.run(cross ? "cross attention" : "self attention", stream_, [&] {
            return Status::from(mx_attn_decode(&d, 1, &n_keys, q, &k, &v, out, nullptr, ws_.data(), ws_.size(), stream_));
        });
    }
    WhisperAttentionConfig cfg_;
    uint16_t * sk_;
    uint16_t * sv_;
    uint16_t * ck_;
    uint16_t * cv_;
    hipStream_t stream_;
    mx_attn_tuning cross_tuning_;
    Workspace ws_;
    DispatchTimer timer_;
};

}  // namespace dooms_amd
