// The C ABI's host-side argument handling under AddressSanitizer and UndefinedBehaviorSanitizer (host code only; no GPU
// needed): every entry point with null, misaligned, out-of-range and inconsistent arguments, which must be refused
// with the documented code before anything is enqueued, and the workspace-size functions over many shapes. Built and
// run by dooms_amd.build.build_sanitized_abi_check (tests/test_abi.py).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "mx_attn.h"
#include "mx_linear.h"

static int g_fail = 0;
#define EXPECT(c) do { if (!(c)) { std::fprintf(stderr, "FAILED %s:%d: %s (%s)\n", __FILE__, __LINE__, #c, mx_attn_last_error()); g_fail++; } } while (0)

static mx_attn_desc desc(int nh = 32, int nkv = 8, int hd = 128, int nq = 1) {
    mx_attn_desc d{};
    d.n_head = nh;
    d.n_head_kv = nkv;
    d.head_dim = hd;
    d.n_q = nq;
    d.q_stride = d.out_stride = (int64_t)nh * hd;
    d.kv_stride = (int64_t)nkv * hd;
    d.scale = 1.f / std::sqrt((float)hd);
    return d;
}

int main() {
    // fake, never dereferenced, 256-byte aligned device addresses
    uint16_t * const A = reinterpret_cast<uint16_t *>(uintptr_t(1) << 20);
    float * const F = reinterpret_cast<float *>(A);
    void * const W = A;
    const int32_t lens[3] = {100, 0, 5000};
    const uint16_t * kp[3] = {A, A, A};
    uint16_t * kpw[3] = {A, A, A};

    // descriptors
    for (int hd : {0, 2, 3, 12, 48, 80, 96, 512, -4}) {
        mx_attn_desc d = desc(32, 8, hd);
        EXPECT(mx_attn_prefill(&d, A, A, A, A, nullptr, nullptr) != MX_ATTN_OK);
        EXPECT(mx_attn_decode(&d, 1, lens, A, kp, kp, A, nullptr, W, 1 << 20, nullptr) != MX_ATTN_OK);
        EXPECT(mx_attn_decode_workspace_bytes(&d, 4, 8192) == 0);
        EXPECT(mx_attn_prefill_workspace_bytes(&d) == 0);
    }
    EXPECT(mx_attn_prefill(nullptr, A, A, A, A, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
    {
        mx_attn_desc d = desc();
        d.reserved = 7;
        EXPECT(mx_attn_prefill(&d, A, A, A, A, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        mx_attn_tuning t{};
        t.decode_splits = 99;
        d = desc();
        d.tuning = &t;
        EXPECT(mx_attn_decode(&d, 1, lens, A, kp, kp, A, nullptr, W, 1 << 20, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        d = desc(14, 3);
        EXPECT(mx_attn_prefill(&d, A, A, A, A, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        d = desc();
        d.q_stride = 4100;
        EXPECT(mx_attn_prefill(&d, A, A, A, A, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        d = desc();
        d.scale = NAN;
        EXPECT(mx_attn_prefill(&d, A, A, A, A, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
    }
    // prefill arguments
    {
        mx_attn_desc d = desc(32, 8, 128, 10);
        d.causal = 1;
        d.p0 = 5;
        d.n_kv = 12;  // a causal chunk's own rows must be in the cache
        EXPECT(mx_attn_prefill(&d, A, A, A, A, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        d.n_kv = 0;
        EXPECT(mx_attn_prefill(&d, nullptr, A, A, A, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        EXPECT(mx_attn_prefill(&d, A + 1, A, A, A, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        EXPECT(mx_attn_prefill(&d, A, A, A, A, reinterpret_cast<float *>(A + 1), nullptr) == MX_ATTN_INVALID_ARGUMENT);
        d.n_q = 0;
        EXPECT(mx_attn_prefill(&d, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr) == MX_ATTN_OK);
        mx_attn_rope bad{5, 10000.f};
        d = desc(28, 4, 128, 16);
        d.q_stride = (28 + 8) * 128;
        EXPECT(mx_attn_prefill_rope(&d, &bad, F, A, A, F, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        EXPECT(mx_attn_prefill_rope(&d, nullptr, F, A, A, F, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        d.p0 = 30000;
        const size_t n = mx_attn_prefill_workspace_bytes(&d);
        EXPECT(n > 0);
        mx_attn_rope rope{0, 500000.f};
        EXPECT(mx_attn_prefill_rope_ws(&d, &rope, F, A, A, F, nullptr, W, n - 1, nullptr) == MX_ATTN_RESOURCE_EXHAUSTED);
        EXPECT(mx_attn_prefill_ws(&d, A, A, A, A, nullptr, reinterpret_cast<char *>(W) + 16, n, nullptr) ==
               MX_ATTN_INVALID_ARGUMENT);
    }
    // decode arguments
    {
        mx_attn_desc d = desc();
        EXPECT(mx_attn_decode(&d, 0, lens, A, kp, kp, A, nullptr, W, 1 << 20, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        EXPECT(mx_attn_decode(&d, 2, lens, A, kp, kp, A, nullptr, W, 1 << 20, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        EXPECT(mx_attn_decode(&d, 1, nullptr, A, kp, kp, A, nullptr, W, 1 << 20, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        EXPECT(mx_attn_decode(&d, 1, lens + 2, A, kp, kp, A, nullptr, W, 16, nullptr) == MX_ATTN_RESOURCE_EXHAUSTED);
        EXPECT(mx_attn_decode(&d, 1, lens + 2, A, kp, kp, A, nullptr, nullptr, 1 << 30, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        const uint16_t * mis[1] = {A + 4};
        EXPECT(mx_attn_decode(&d, 1, lens, A, mis, kp, A, nullptr, W, 1 << 20, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        d.n_q = 40000;
        EXPECT(mx_attn_decode(&d, 1, lens, A, kp, kp, A, nullptr, W, 1 << 20, nullptr) == MX_ATTN_UNSUPPORTED);
        // the no-allocation entry point refuses what mx_attn_decode refuses, with the same code, before it touches the
        // device (on a host without a GPU any device call would fail with INTERNAL instead)
        EXPECT(mx_attn_decode_noalloc(&d, 1, lens, A, kp, kp, A, nullptr, nullptr) == MX_ATTN_UNSUPPORTED);
        d = desc();
        EXPECT(mx_attn_decode_noalloc(&d, 2, lens, A, kp, kp, A, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);  // kv_len 0
        EXPECT(mx_attn_decode_noalloc(&d, 1, nullptr, A, kp, kp, A, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        EXPECT(mx_attn_decode_noalloc(&d, 1, lens, nullptr, kp, kp, A, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        EXPECT(mx_attn_decode_noalloc(&d, 1, lens, A, kp, kp, nullptr, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        EXPECT(mx_attn_decode_noalloc(&d, 1, lens, A, mis, kp, A, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        EXPECT(mx_attn_decode_noalloc(&d, 1, lens, A + 4, kp, kp, A, nullptr, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        {
            // 32 sequences of 8192 keys need more scratch than the library holds: refused by size
            std::vector<int32_t> big(32, 8192);
            std::vector<const uint16_t *> bp(32, A);
            EXPECT(mx_attn_decode_workspace_bytes(&d, 32, 8192) > ((size_t)16 << 20));
            EXPECT(mx_attn_decode_noalloc(&d, 32, big.data(), A, bp.data(), bp.data(), A, nullptr, nullptr) ==
                   MX_ATTN_RESOURCE_EXHAUSTED);
        }
        mx_attn_rope rope{0, 500000.f};
        d.q_stride = (32 + 16) * 128;
        uint16_t * shared[2] = {A, A};
        const int32_t two[2] = {10, 11};
        EXPECT(mx_attn_decode_rope(&d, &rope, 2, two, F, shared, shared, F, nullptr, W, 1 << 20, nullptr) ==
               MX_ATTN_INVALID_ARGUMENT);
        d.n_q = 2;
        EXPECT(mx_attn_decode_rope(&d, &rope, 1, two, F, kpw, kpw, F, nullptr, W, 1 << 20, nullptr) ==
               MX_ATTN_INVALID_ARGUMENT);
        EXPECT(mx_attn_decode_workspace_init(reinterpret_cast<char *>(W) + 4, 256, nullptr) == MX_ATTN_INVALID_ARGUMENT);
    }
    // workspace sizes over many shapes (the arithmetic of the layout functions)
    for (int hd = 4; hd <= 256; hd *= 2)
        for (int nkv : {1, 2, 8, 20})
            for (int g : {1, 4, 7})
                for (int nq : {1, 5, 64, 300})
                    for (int L : {1, 129, 8192, 1 << 20}) {
                        mx_attn_desc d = desc(nkv * g, nkv, hd, nq);
                        const size_t a = mx_attn_decode_workspace_bytes(&d, 1, L), b = mx_attn_decode_workspace_bytes(&d, 40, L);
                        EXPECT(a <= b);
                        d.p0 = L;
                        d.causal = 1;
                        (void)mx_attn_prefill_workspace_bytes(&d);
                    }
    // self-attention and projections
    {
        mx_self_attn_desc s{};
        s.batch = 0;
        EXPECT(mx_self_attention(&s, A, A, nullptr, 0, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        s = mx_self_attn_desc{2, 10, 5, 30, MX_ATTN_F32, 0.1f, nullptr};  // head_dim 6: packed into a workspace
        EXPECT(mx_self_attention_workspace_bytes(&s) > 0);
        EXPECT(mx_self_attention(&s, A, A, nullptr, 0, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        EXPECT(mx_self_attention(&s, A, A + 8, W, 1 << 20, nullptr) == MX_ATTN_INVALID_ARGUMENT);  // y overlaps qkv
        mx_linear_desc l{100, 64, 128, 0, 128, 64, 1e-5f, 0};
        EXPECT(mx_linear_workspace_bytes(&l) == 100 * 128 * 2);
        EXPECT(mx_linear(&l, 0, nullptr, F, nullptr, nullptr, nullptr, nullptr, 0, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        const uint16_t * ws[1] = {A};
        void * ys[1] = {A};
        EXPECT(mx_linear(&l, 1, ws, F, ys, nullptr, nullptr, nullptr, 0, nullptr) == MX_ATTN_INVALID_ARGUMENT);
        l.flags = MX_LINEAR_RMS_NORM;
        EXPECT(mx_linear(&l, 1, ws, F, ys, nullptr, nullptr, W, 1 << 20, nullptr) == MX_ATTN_INVALID_ARGUMENT);
    }
    if (g_fail) {
        std::fprintf(stderr, "%d checks failed\n", g_fail);
        return 1;
    }
    std::printf("abi_checks_sanitized: ok\n");
    return 0;
}
