// C++ host layer above the C ABI for the two rows either side of the decoders' attention:
//
//   reference (dooms.cpp 0.6.1)                                               here
//   OpKind::SelfAttention lowered by the ggml backend                          SelfAttentionOp::create / run
//     (src/ir/op.h:31-32, 64-71; src/backend/ggml/ggml_backend.cpp:398-412;
//     self_attention_params src/ir/op.cpp:69-76)
//   the decoders' matvec / matmul dispatches around the attention             Projection::create / run
//     (src/backend/metal/metal_llama_decoder.mm:160-235, 318-352;
//     encode_cross, src/backend/metal/metal_whisper_decoder.mm:295-316)
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
        mx_self_attn_desc d;
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

// One projection Y = X W^T of a decoder layer (flags MX_LINEAR_*), for up to max_rows input rows.
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

}  // namespace dooms_amd
