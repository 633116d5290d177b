// C++ host layer above the C ABI for the two rows either side of the decoders' attention:
//
//   reference (dooms.cpp 0.6.1)                                               here
//   OpKind::SelfAttention lowered by the ggml backend                          SelfAttentionOp::create / run
//     (src/ir/op.h:31-32, 64-71; src/backend/ggml/ggml_backend.cpp:398-412;
//     self_attention_params src/ir/op.cpp:69-76)
//   the decoders' matvec / matmul dispatches around the attention             Projection::create / run
//     (src/backend/metal/metal_llama_decoder.mm:160-235, 318-352)
//   MetalWhisperDecoder::set_audio / encode_cross: every layer's cross-       WhisperCrossCache::create / set_audio
//     attention K (no bias) and V (bias) from the encoder states, rounded
//     to half into the cross caches (metal_whisper_decoder.mm:295-316, 500-520)
//
// As in the reference's Executable::run (src/backend/backend.h:50-53: no device allocation in run), the workspace is
// sized once, at create, for the largest shape the caller declares; run() with a larger shape returns
// ResourceExhausted. Not thread-safe; all work is ordered on the stream given at create.
//
// Header-only: include it, link libmx_attn.so and the HIP runtime.
#pragma once

#include <cmath>
#include <memory>
#include <string>

#include "attention_host.hpp"
#include "mx_linear.h"

namespace dooms_amd {

// Device memory owned by an op (no counters to initialize, unlike the decode workspace).
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer & operator=(const DeviceBuffer &) = delete;
    ~DeviceBuffer() {
        if (ptr_) (void)hipFree(ptr_);
    }
    Status reserve(size_t bytes) {
        if (bytes <= bytes_) return {};
        if (ptr_) (void)hipFree(ptr_);
        ptr_ = nullptr;
        bytes_ = 0;
        if (Status st = Status::hip(hipMalloc(&ptr_, bytes), "workspace allocation"); !st.is_ok()) {
            ptr_ = nullptr;
            return Status{Code::ResourceExhausted, st.message};
        }
        bytes_ = bytes;
        return {};
    }
    void * data() const { return ptr_; }
    size_t size() const { return bytes_; }

private:
    void * ptr_ = nullptr;
    size_t bytes_ = 0;
};

// The IR's SelfAttention op: packed q|k|v rows [B][N][3E] -> [B][N][E], softmax(scale q k^T) v per head, no mask.
enum class DType : int32_t { F32 = MX_ATTN_F32, F16 = MX_ATTN_F16, BF16 = MX_ATTN_BF16 };  // src/core/dtype.h:13 order

class SelfAttentionOp {
public:
    // heads >= 1 and a finite scale (self_attention_params); the workspace covers every shape up to
    // max_batch x max_tokens x embed in dtype
    static Status create(int64_t heads, float scale, int32_t max_batch, int32_t max_tokens, int32_t embed, DType dtype,
                         hipStream_t stream, std::unique_ptr<SelfAttentionOp> & out) {
        if (heads < 1) return {Code::InvalidArgument, "self_attention: heads must be >= 1, got " + std::to_string(heads)};
        if (!std::isfinite(scale)) return {Code::InvalidArgument, "self_attention: scale must be finite"};
        if (max_batch < 1 || max_tokens < 0 || embed < 1 || embed % heads)
            return {Code::InvalidArgument, "self_attention: embedding " + std::to_string(embed) + " is not divisible by " +
                                               std::to_string(heads) + " heads, or an empty batch"};
        if (embed / heads > 128) return {Code::Unsupported, "head_dim " + std::to_string(embed / heads) + " is above 128"};
        std::unique_ptr<SelfAttentionOp> op(new SelfAttentionOp((int32_t)heads, scale, dtype, stream));
        const mx_self_attn_desc d = op->desc(max_batch, max_tokens, embed);
        if (Status st = op->ws_.reserve(mx_self_attention_workspace_bytes(&d)); !st.is_ok()) return st;
        out = std::move(op);
        return {};
    }

    // qkv [batch][tokens][3 embed], y [batch][tokens][embed], device memory of the op's dtype
    Status run(const void * qkv, void * y, int32_t batch, int32_t tokens, int32_t embed) {
        const mx_self_attn_desc d = desc(batch, tokens, embed);
        return Status::from(mx_self_attention(&d, qkv, y, ws_.data(), ws_.size(), stream_));
    }

private:
    SelfAttentionOp(int32_t heads, float scale, DType dtype, hipStream_t stream)
        : heads_(heads), scale_(scale), dtype_(dtype), stream_(stream) {}
    mx_self_attn_desc desc(int32_t batch, int32_t tokens, int32_t embed) const {
        mx_self_attn_desc d{};
        d.batch = batch;
        d.n_tok = tokens;
        d.heads = heads_;
        d.embed = embed;
        d.dtype = (int32_t)dtype_;
        d.scale = scale_;
        return d;
    }
    int32_t heads_;
    float scale_;
    DType dtype_;
    hipStream_t stream_;
    DeviceBuffer ws_;
};

// One projection Y = X W^T of a decoder layer (flags MX_LINEAR_*), for up to max_rows input rows, on mx_linear's
// kernels. Nothing allocates in run().
class Projection {
public:
    static Status create(int32_t N, int32_t K, uint32_t flags, float eps, int32_t max_rows, hipStream_t stream,
                         std::unique_ptr<Projection> & out) {
        if (N < 1 || K < 1 || max_rows < 1) return {Code::InvalidArgument, "N, K and max_rows must be >= 1"};
        std::unique_ptr<Projection> p(new Projection(N, K, flags, eps, stream));
        const mx_linear_desc d = p->desc(max_rows, K, N);
        if (Status st = p->ws_.reserve(mx_linear_workspace_bytes(&d)); !st.is_ok()) return st;
        out = std::move(p);
        return {};
    }

    // X f32 [M][x_stride], Y[i] [M][y_stride] (f32, or f16 with MX_LINEAR_OUT_F16); count matrices W[i] [N][K] f16
    // sharing X; gamma f32 [K] with MX_LINEAR_RMS_NORM; bias[i] f32 [N] with MX_LINEAR_BIAS. All device memory; the
    // pointer arrays are host arrays.
    Status run(int32_t M, int32_t count, const uint16_t * const * W, const float * X, int64_t x_stride, void * const * Y,
               int64_t y_stride, const float * gamma = nullptr, const float * const * bias = nullptr) {
        mx_linear_desc d = desc(M, x_stride, y_stride);
        return Status::from(mx_linear(&d, count, W, X, Y, gamma, bias, ws_.data(), ws_.size(), stream_));
    }

private:
    Projection(int32_t N, int32_t K, uint32_t flags, float eps, hipStream_t stream)
        : N_(N), K_(K), flags_(flags), eps_(eps), stream_(stream) {}
    mx_linear_desc desc(int32_t M, int64_t x_stride, int64_t y_stride) const {
        mx_linear_desc d;
        d.M = M;
        d.N = N_;
        d.K = K_;
        d.flags = flags_;
        d.x_stride = x_stride;
        d.y_stride = y_stride;
        d.eps = eps_;
        d.reserved = 0;
        return d;
    }
    int32_t N_, K_;
    uint32_t flags_;
    float eps_;
    hipStream_t stream_;
    DeviceBuffer ws_;
};

// The Whisper decoder's cross-attention cache producer: for every layer l, K_l = X W_k[l]^T and V_l = X W_v[l]^T + b_v[l]
// over the n_audio_ctx encoder states X [n_audio_ctx][n_state] (f32), rounded to half into the caches of a
// WhisperAttention (layer l at l * n_audio_ctx rows). One mx_linear call for all 2 n_layer matrices (n_layer <= 32).
class WhisperCrossCache {
public:
    static Status create(const WhisperAttentionConfig & c, hipStream_t stream, std::unique_ptr<WhisperCrossCache> & out) {
        if (c.n_layer < 1 || 2 * c.n_layer > 64) return {Code::InvalidArgument, "n_layer must be in [1, 32]"};
        std::unique_ptr<Projection> proj;
        if (Status st = Projection::create(c.n_state, c.n_state, MX_LINEAR_OUT_F16 | MX_LINEAR_BIAS, 0.f, c.n_audio_ctx,
                                           stream, proj);
            !st.is_ok())
            return st;
        out.reset(new WhisperCrossCache(c, std::move(proj)));
        return {};
    }

    // states: device, f32 [n_audio_ctx][n_state]; w_k, w_v: host arrays [n_layer] of device f16 [n_state][n_state]
    // weights; b_v: host array [n_layer] of device f32 [n_state] biases (an entry may be null).
    Status set_audio(WhisperAttention & attn, const float * states, const uint16_t * const * w_k,
                     const uint16_t * const * w_v, const float * const * b_v) {
        const WhisperAttentionConfig & a = attn.config();
        if (a.n_layer != cfg_.n_layer || a.n_state != cfg_.n_state || a.n_audio_ctx != cfg_.n_audio_ctx)
            return {Code::InvalidArgument, "the attention's shape differs from the producer's"};
        if (!states || !w_k || !w_v) return {Code::InvalidArgument, "states and weights must not be null"};
        const uint16_t * W[64];
        void * Y[64];
        const float * B[64];
        for (int32_t l = 0; l < cfg_.n_layer; l++) {
            W[2 * l] = w_k[l];
            W[2 * l + 1] = w_v[l];
            Y[2 * l] = attn.cross_k(l);
            Y[2 * l + 1] = attn.cross_v(l);
            B[2 * l] = nullptr;  // the key projection has no bias
            B[2 * l + 1] = b_v ? b_v[l] : nullptr;
        }
        return proj_->run(cfg_.n_audio_ctx, 2 * cfg_.n_layer, W, states, cfg_.n_state, Y, cfg_.n_state, nullptr, B);
    }

private:
    WhisperCrossCache(const WhisperAttentionConfig & c, std::unique_ptr<Projection> p) : cfg_(c), proj_(std::move(p)) {}
    WhisperAttentionConfig cfg_;
    std::unique_ptr<Projection> proj_;
};

}  // namespace dooms_amd
