// rope_store for a prompt chunk: the keys and values of n_rows new tokens into the f16 caches.
//
// Reference behaviour (dooms.cpp 0.6.1): rope_store (src/backend/metal/llama_kernels.h:520-545), dispatched before the
// prompt chunk's attention (metal_llama_decoder.mm:276-283, metal_whisper_decoder.mm:187-193): key head g of token t is
// rotated for position p0 + t (rotate_pair, llama_kernels.h:513-518) and stored as half at cache row p0 + t; value head
// g is stored as half. The query heads are rotated inside the prefill kernel instead (prefill.hip); only for a chunk
// that runs on the split-KV decode kernel are they rotated here too, into an f32 buffer (q_out).
//
// MI355X design: HBM-bound byte work (per row: 8 n_head_kv hd bytes read, 4 n_head_kv hd written). One workgroup per
// token row; each thread owns one rotary pair of one key head and the same two elements of the value head, so the f32
// reads and f16 writes of a wave are contiguous (adjacent pairs) or two contiguous halves (neox).
#include <algorithm>

#include "mx_common.hpp"
#include "mx_kernels.hpp"

namespace mx {

namespace {

template <int HD>
__global__ __launch_bounds__(1024) void rope_store_kernel(RopeStoreParams p) {
    const int t = blockIdx.x;
    const int pos = p.p0 + t;
    const float * row = p.qkv + (int64_t)t * p.qkv_stride;
    half_t * kd = p.k + (int64_t)pos * p.kv_stride;
    half_t * vd = p.v + (int64_t)pos * p.kv_stride;
    const int nq = p.q_out ? p.n_head * (HD / 2) : 0;  // query pairs first, when they are wanted
    for (int idx = threadIdx.x; idx < nq + p.n_head_kv * (HD / 2); idx += blockDim.x) {
        const int qi = idx < nq ? idx : idx - nq;
        const int g = qi / (HD / 2), i = qi % (HD / 2);
        const int i0 = p.rope_mode == 1 ? i : 2 * i, i1 = p.rope_mode == 1 ? i + HD / 2 : 2 * i + 1;
        if (idx < nq) {  // query head g: rotated, kept in f32
            const float * qx = row + (int64_t)g * HD;
            float a = qx[i0], b = qx[i1];
            if (p.rope_mode != 2) {
                float sn, cs;
                sincos_rope((float)pos * p.rope_freq[i], sn, cs);
                const float ra = a * cs - b * sn, rb = a * sn + b * cs;
                a = ra;
                b = rb;
            }
            float * qd = p.q_out + (int64_t)t * p.n_head * HD + (int64_t)g * HD;
            qd[i0] = a;
            qd[i1] = b;
            continue;
        }
        const float * kx = row + (int64_t)(p.n_head + g) * HD;
        const float * vx = row + (int64_t)(p.n_head + p.n_head_kv + g) * HD;
        float a = kx[i0], b = kx[i1];
        if (p.rope_mode != 2) {
            float sn, cs;
            sincos_rope((float)pos * p.rope_freq[i], sn, cs);
            const float ra = a * cs - b * sn, rb = a * sn + b * cs;
            a = ra;
            b = rb;
        }
        kd[g * HD + i0] = (half_t)a;
        kd[g * HD + i1] = (half_t)b;
        vd[g * HD + 2 * i] = (half_t)vx[2 * i];
        vd[g * HD + 2 * i + 1] = (half_t)vx[2 * i + 1];
    }
}

}  // namespace

hipError_t launch_rope_store(const RopeStoreParams & p, int head_dim, hipStream_t stream) {
    const int pairs = ((p.q_out ? p.n_head : 0) + p.n_head_kv) * head_dim / 2;
    // one pair per thread where the row has at most 1024 (each further pass of the loop is another dependent round trip)
    const int threads = std::min(1024, ((pairs + kWave - 1) / kWave) * kWave);
    const dim3 grid(p.n_rows), block(threads);
    switch (head_dim) {
        case 4: hipLaunchKernelGGL((rope_store_kernel<4>), grid, block, 0, stream, p); break;
        case 8: hipLaunchKernelGGL((rope_store_kernel<8>), grid, block, 0, stream, p); break;
        case 16: hipLaunchKernelGGL((rope_store_kernel<16>), grid, block, 0, stream, p); break;
        case 32: hipLaunchKernelGGL((rope_store_kernel<32>), grid, block, 0, stream, p); break;
        case 64: hipLaunchKernelGGL((rope_store_kernel<64>), grid, block, 0, stream, p); break;
        case 128: hipLaunchKernelGGL((rope_store_kernel<128>), grid, block, 0, stream, p); break;
        case 256: hipLaunchKernelGGL((rope_store_kernel<256>), grid, block, 0, stream, p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace mx
