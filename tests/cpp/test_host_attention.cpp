// C++ host-layer test (dooms_amd/host/attention_host.hpp) in the reference's style: a dependency-free TEST/EXPECT
// harness whose exit code is the number of failed tests (tests/unit/check.h:1-71 in dooms.cpp 0.6.1), and a decoder's
// call sequence checked against an independent double-precision reference (the reference's own approach,
// tests/unit/test_metal_llama_decoder.cpp:110-192), here the CPU oracle (oracle/oracle.c).
//
// Llama: a 45-token prompt in chunks of 20 through the flash path, then decode steps one at a time
// (test_metal_llama_decoder.cpp:497-532 evaluates the same prompt in chunks of 20), two layers, GQA 4/2, head_dim 64.
// Whisper: prompt rows, single-token self-attention steps, greedy and 5-beam cross-attention over 150 encoder rows.
// Error paths: unsupported head_dim, context overflow, bad layer.
// The two rows beside the attention (ops_host.hpp): the IR SelfAttention op and a q|k|v projection.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "attention_host.hpp"
#include "ops_host.hpp"

extern "C" int oracle_attention_f64(int32_t n_head, int32_t n_head_kv, int32_t head_dim, int32_t n_q, int32_t p0, int32_t n_kv,
                                    int32_t causal, double scale, const uint16_t * q, int64_t q_stride, const uint16_t * k,
                                    const uint16_t * v, int64_t kv_stride, double * out, int64_t out_stride, double * lse);

extern "C" int oracle_linear_f64(int32_t M, int32_t N, int32_t K, uint32_t flags, int32_t half_input, float eps, const float * X,
                                 int64_t x_stride, const uint16_t * W, const float * gamma, const float * bias, double * Y);

extern "C" void oracle_rope_f32(int32_t mode, float base, int32_t head_dim, int32_t pos, const float * x, float * y, int64_t n_vec);

namespace {

int g_failed = 0, g_checks = 0;
std::vector<std::pair<const char *, std::function<void()>>> & registry() {
    static std::vector<std::pair<const char *, std::function<void()>>> r;
    return r;
}
struct Reg {
    Reg(const char * n, std::function<void()> f) { registry().emplace_back(n, std::move(f)); }
};
#define TEST(name) static void name(); static Reg reg_##name(#name, name); static void name()
#define EXPECT(cond) do { g_checks++; if (!(cond)) { g_failed++; std::fprintf(stderr, "  FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond); } } while (0)

#define HIP_OK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); std::exit(100); } } while (0)

uint16_t to_half(float f) {
    const _Float16 h = (_Float16)f;
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}
double from_half(uint16_t b) {
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return (double)(float)h;
}

// splitmix64 and Box-Muller: portable seeded normals
struct Rng {
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniform() { return ((next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
    float normal() { return (float)(std::sqrt(-2.0 * std::log(uniform())) * std::cos(6.283185307179586 * uniform())); }
};
std::vector<uint16_t> random_half(Rng & r, size_t n) {
    std::vector<uint16_t> v(n);
    for (auto & x : v) x = to_half(r.normal());
    return v;
}

struct Dev {
    uint16_t * p = nullptr;
    explicit Dev(size_t n) { HIP_OK(hipMalloc(&p, n * 2)); }
    ~Dev() { (void)hipFree(p); }
};

// |got - ref| <= 2e-3 + 1e-2 |ref| for every element
bool close(const std::vector<uint16_t> & got, const std::vector<double> & ref, const char * what) {
    double worst = 0;
    size_t bad = 0;
    for (size_t i = 0; i < ref.size(); i++) {
        const double e = std::fabs(from_half(got[i]) - ref[i]);
        worst = std::max(worst, e);
        if (!(e <= 2e-3 + 1e-2 * std::fabs(ref[i]))) bad++;
    }
    if (bad) std::fprintf(stderr, "  %s: %zu elements out of tolerance, max abs err %.3e\n", what, bad, worst);
    return bad == 0;
}

}  // namespace

// The reference's tiny llama (4 q / 2 kv heads, test_metal_llama_decoder.cpp:56-57) at its default head_dim 16 (the
// per-query kernel) and at 64 (the flash kernel, as the reference's test also runs it): a 45-token prompt in chunks of
// 20, then decode steps, two layers.
static void prompt_in_chunks_then_decode_steps(int hd);
TEST(llama_prompt_in_chunks_then_decode_steps) {
    prompt_in_chunks_then_decode_steps(16);
    prompt_in_chunks_then_decode_steps(64);
}

static void prompt_in_chunks_then_decode_steps(int hd) {
    using namespace dooms_amd;
    const int n_layer = 2, n_ctx = 96, nh = 4, nkv = 2, qw = nh * hd, kw = nkv * hd;
    Dev kc((size_t)n_layer * n_ctx * kw), vc((size_t)n_layer * n_ctx * kw);
    std::unique_ptr<LlamaAttention> attn;
    Status st = LlamaAttention::create({n_layer, n_ctx, nh, nkv, hd}, kc.p, vc.p, nullptr, attn);
    EXPECT(st.is_ok());
    if (!st.is_ok()) return;
    Rng rng{7};
    const int prompt = 45, steps = 12;
    // per layer: all rows' rotated q, k, v (host copies for the reference)
    std::vector<std::vector<uint16_t>> Q(n_layer), K(n_layer), V(n_layer);
    for (int l = 0; l < n_layer; l++) {
        Q[l] = random_half(rng, (size_t)(prompt + steps) * qw);
        K[l] = random_half(rng, (size_t)(prompt + steps) * kw);
        V[l] = random_half(rng, (size_t)(prompt + steps) * kw);
    }
    Dev dq((size_t)(prompt + steps) * qw), dk((size_t)(prompt + steps) * kw), dv((size_t)(prompt + steps) * kw),
        dout((size_t)(prompt + steps) * qw);
    auto run_rows = [&](int l, int p0, int M) -> bool {
        HIP_OK(hipMemcpy(dq.p, Q[l].data() + (size_t)p0 * qw, (size_t)M * qw * 2, hipMemcpyHostToDevice));
        HIP_OK(hipMemcpy(dk.p, K[l].data() + (size_t)p0 * kw, (size_t)M * kw * 2, hipMemcpyHostToDevice));
        HIP_OK(hipMemcpy(dv.p, V[l].data() + (size_t)p0 * kw, (size_t)M * kw * 2, hipMemcpyHostToDevice));
        Status a = attn->append(l, dk.p, kw, dv.p, kw, M, p0);
        Status b = attn->attention(l, dq.p, qw, dout.p, qw, M, p0);
        HIP_OK(hipDeviceSynchronize());
        if (!a.is_ok() || !b.is_ok()) {
            std::fprintf(stderr, "  %s %s\n", a.message.c_str(), b.message.c_str());
            return false;
        }
        std::vector<uint16_t> got((size_t)M * qw);
        HIP_OK(hipMemcpy(got.data(), dout.p, got.size() * 2, hipMemcpyDeviceToHost));
        std::vector<double> ref((size_t)M * qw);
        oracle_attention_f64(nh, nkv, hd, M, p0, p0 + M, 1, 1.0 / std::sqrt((double)hd), Q[l].data() + (size_t)p0 * qw, qw,
                             K[l].data(), V[l].data(), kw, ref.data(), qw, nullptr);
        return close(got, ref, (std::string("layer ") + std::to_string(l) + " rows at " + std::to_string(p0)).c_str());
    };
    for (int p0 = 0; p0 < prompt; p0 += 20)
        for (int l = 0; l < n_layer; l++) EXPECT(run_rows(l, p0, std::min(20, prompt - p0)));
    for (int p = prompt; p < prompt + steps; p++)
        for (int l = 0; l < n_layer; l++) EXPECT(run_rows(l, p, 1));
}

// Qwen2-style (neox rope, base 1e6) on the reference's f32 buffers: a 37-token prompt in chunks of 16 through prompt()
// (rope_store + flash attention), then fused decode steps; every output and every cache row written is checked against
// the oracle's rope and attention.
TEST(llama_f32_prompt_then_fused_decode_steps) {
    using namespace dooms_amd;
    const int n_ctx = 64, nh = 14, nkv = 2, hd = 64, qw = nh * hd, kw = nkv * hd, rw = qw + 2 * kw;
    const float base = 1e6f;
    Dev kc((size_t)n_ctx * kw), vc((size_t)n_ctx * kw);
    std::unique_ptr<LlamaAttention> attn;
    LlamaAttentionConfig cfg{1, n_ctx, nh, nkv, hd};
    cfg.rope_base = base;
    cfg.rope_neox = true;
    Status st = LlamaAttention::create(cfg, kc.p, vc.p, nullptr, attn);
    EXPECT(st.is_ok());
    if (!st.is_ok()) return;
    Rng rng{23};
    const int prompt = 37, steps = 6, chunk = 16;
    std::vector<uint16_t> K((size_t)n_ctx * kw), V((size_t)n_ctx * kw);  // host image of the cache
    float *dqkv = nullptr, *dout = nullptr;
    HIP_OK(hipMalloc(&dqkv, (size_t)chunk * rw * 4));
    HIP_OK(hipMalloc(&dout, (size_t)chunk * qw * 4));
    // runs M rows at p0 (prompt chunk, or one fused step) and checks cache rows and outputs
    auto run = [&](int p0, int M) {
        std::vector<float> rows((size_t)M * rw);
        for (auto & x : rows) x = rng.normal();
        HIP_OK(hipMemcpy(dqkv, rows.data(), rows.size() * 4, hipMemcpyHostToDevice));
        Status s = M == 1 && p0 >= prompt ? attn->decode_step(0, dqkv, dout, p0) : attn->prompt(0, dqkv, dout, M, p0);
        HIP_OK(hipDeviceSynchronize());
        EXPECT(s.is_ok());
        std::vector<uint16_t> qh((size_t)M * qw);
        int worst_k = 0;
        bool v_ok = true;
        std::vector<uint16_t> gk((size_t)M * kw), gv((size_t)M * kw);
        HIP_OK(hipMemcpy(gk.data(), kc.p + (size_t)p0 * kw, gk.size() * 2, hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(gv.data(), vc.p + (size_t)p0 * kw, gv.size() * 2, hipMemcpyDeviceToHost));
        for (int t = 0; t < M; t++) {
            const float * row = rows.data() + (size_t)t * rw;
            std::vector<float> qr(qw), kr(kw);
            oracle_rope_f32(1, base, hd, p0 + t, row, qr.data(), nh);
            oracle_rope_f32(1, base, hd, p0 + t, row + qw, kr.data(), nkv);
            for (int i = 0; i < qw; i++) qh[(size_t)t * qw + i] = to_half(qr[i]);
            for (int i = 0; i < kw; i++) {
                worst_k = std::max(worst_k, std::abs((int)(int16_t)gk[(size_t)t * kw + i] - (int)(int16_t)to_half(kr[i])));
                v_ok = v_ok && gv[(size_t)t * kw + i] == to_half(row[qw + kw + i]);
            }
        }
        EXPECT(worst_k <= 1);  // one half ulp for a sine/cosine rounding difference
        EXPECT(v_ok);
        std::memcpy(&K[(size_t)p0 * kw], gk.data(), gk.size() * 2);
        std::memcpy(&V[(size_t)p0 * kw], gv.data(), gv.size() * 2);
        std::vector<double> ref((size_t)M * qw);
        oracle_attention_f64(nh, nkv, hd, M, p0, p0 + M, 1, 1.0 / std::sqrt((double)hd), qh.data(), qw, K.data(), V.data(), kw,
                             ref.data(), qw, nullptr);
        std::vector<float> got((size_t)M * qw);
        HIP_OK(hipMemcpy(got.data(), dout, got.size() * 4, hipMemcpyDeviceToHost));
        size_t bad = 0;
        for (size_t i = 0; i < got.size(); i++)
            if (!(std::fabs(got[i] - ref[i]) <= 2e-3 + 1e-2 * std::fabs(ref[i]))) bad++;
        EXPECT(bad == 0);
    };
    for (int p0 = 0; p0 < prompt; p0 += chunk) run(p0, std::min(chunk, prompt - p0));
    for (int p = prompt; p < prompt + steps; p++) run(p, 1);
    EXPECT(attn->decode_step(0, dqkv, dout, n_ctx).code == Code::ResourceExhausted);
    EXPECT(attn->prompt(0, dqkv, dout, 2, n_ctx - 1).code == Code::ResourceExhausted);
    (void)hipFree(dqkv);
    (void)hipFree(dout);
}

// Profiling by kind (profile_pass, metal_llama_decoder.mm:789-812): every call made while a vector is attached is
// counted under its kind with a positive GPU time; detached, nothing more is recorded and results stay correct.
TEST(profile_by_kind) {
    using namespace dooms_amd;
    const int n_ctx = 256, nh = 8, nkv = 2, hd = 128, qw = nh * hd, kw = nkv * hd, rw = qw + 2 * kw;
    Dev kc((size_t)n_ctx * kw), vc((size_t)n_ctx * kw), dq((size_t)64 * qw), dout((size_t)64 * qw);
    std::unique_ptr<LlamaAttention> attn;
    EXPECT(LlamaAttention::create({1, n_ctx, nh, nkv, hd}, kc.p, vc.p, nullptr, attn).is_ok());
    if (!attn) return;
    float *dqkv = nullptr, *dof = nullptr;
    HIP_OK(hipMalloc(&dqkv, (size_t)64 * rw * 4));
    HIP_OK(hipMalloc(&dof, (size_t)64 * qw * 4));
    HIP_OK(hipMemset(dqkv, 0, (size_t)64 * rw * 4));
    HIP_OK(hipMemset(dq.p, 0, (size_t)64 * qw * 2));
    std::vector<KernelTime> times;
    attn->set_profile(&times);
    EXPECT(attn->prompt(0, dqkv, dof, 64, 0).is_ok());
    for (int p = 64; p < 67; p++) EXPECT(attn->decode_step(0, dqkv, dof, p).is_ok());
    EXPECT(attn->append(0, kc.p, kw, vc.p, kw, 4, 67).is_ok());
    EXPECT(attn->attention(0, dq.p, qw, dout.p, qw, 1, 70).is_ok());
    auto find = [&](const char * kind) -> const KernelTime * {
        for (const KernelTime & k : times)
            if (k.kind == kind) return &k;
        return nullptr;
    };
    const KernelTime * pr = find("rope_store + attention");
    const KernelTime * at = find("attention");
    const KernelTime * ca = find("cache k/v");
    EXPECT(times.size() == 3);
    EXPECT(pr && pr->dispatches == 1 && pr->gpu_ms > 0);
    EXPECT(at && at->dispatches == 4 && at->gpu_ms > 0);
    EXPECT(ca && ca->dispatches == 1 && ca->gpu_ms > 0);
    attn->set_profile(nullptr);
    EXPECT(attn->decode_step(0, dqkv, dof, 71).is_ok());
    HIP_OK(hipDeviceSynchronize());
    EXPECT(at && at->dispatches == 4);
    // Whisper: self and cross kinds
    const int ns = 256, wh = 4, n_audio = 96;
    Dev sk((size_t)32 * ns), sv((size_t)32 * ns), ck((size_t)n_audio * ns), cv((size_t)n_audio * ns);
    HIP_OK(hipMemset(ck.p, 0, (size_t)n_audio * ns * 2));
    HIP_OK(hipMemset(cv.p, 0, (size_t)n_audio * ns * 2));
    WhisperAttentionConfig wc{};
    wc.n_layer = 1;
    wc.n_state = ns;
    wc.n_head = wh;
    wc.n_text_ctx = 32;
    wc.n_audio_ctx = n_audio;
    wc.max_rows = 5;
    std::unique_ptr<WhisperAttention> w;
    EXPECT(WhisperAttention::create(wc, sk.p, sv.p, ck.p, cv.p, nullptr, w).is_ok());
    if (!w) return;
    std::vector<KernelTime> wt;
    w->set_profile(&wt);
    EXPECT(w->self_attention_prompt(0, dqkv, dof, 0, 3).is_ok());
    EXPECT(w->self_attention(0, dqkv, dof, 3).is_ok());
    EXPECT(w->cross_attention(0, dq.p, dout.p, 5).is_ok());
    EXPECT(wt.size() == 2);
    EXPECT(wt.size() == 2 && wt[0].kind == "self attention" && wt[0].dispatches == 2 && wt[0].gpu_ms > 0);
    EXPECT(wt.size() == 2 && wt[1].kind == "cross attention" && wt[1].dispatches == 1 && wt[1].gpu_ms > 0);
    (void)hipFree(dqkv);
    (void)hipFree(dof);
}

TEST(llama_errors) {
    using namespace dooms_amd;
    Dev kc(1024), vc(1024);
    std::unique_ptr<LlamaAttention> attn;
    EXPECT(LlamaAttention::create({1, 4, 4, 2, 80}, kc.p, vc.p, nullptr, attn).code == Code::Unsupported);
    EXPECT(LlamaAttention::create({1, 4, 4, 3, 64}, kc.p, vc.p, nullptr, attn).code == Code::InvalidArgument);
    EXPECT(LlamaAttention::create({1, 4, 4, 2, 64}, nullptr, vc.p, nullptr, attn).code == Code::InvalidArgument);
    EXPECT(LlamaAttention::create({1, 4, 4, 2, 64}, kc.p, vc.p, nullptr, attn).is_ok());
    if (!attn) return;
    EXPECT(attn->attention(1, kc.p, 0, vc.p, 0, 1, 0).code == Code::InvalidArgument);   // no layer 1
    EXPECT(attn->attention(0, kc.p, 0, vc.p, 0, 2, 3).code == Code::ResourceExhausted);  // positions 3, 4 of 4
    EXPECT(attn->append(0, kc.p, 128, vc.p, 128, 5, 0).code == Code::ResourceExhausted);
}

TEST(whisper_prompt_steps_and_cross_attention) {
    using namespace dooms_amd;
    const int n_state = 256, nh = 4, hd = 64, n_text = 32, n_audio = 150;
    Dev sk((size_t)n_text * n_state), sv((size_t)n_text * n_state), ck((size_t)n_audio * n_state), cv((size_t)n_audio * n_state);
    std::unique_ptr<WhisperAttention> w;
    Status st = WhisperAttention::create({1, n_state, nh, n_text, n_audio, 8}, sk.p, sv.p, ck.p, cv.p, nullptr, w);
    EXPECT(st.is_ok());
    if (!st.is_ok()) return;
    Rng rng{11};
    const std::vector<uint16_t> SK = random_half(rng, (size_t)n_text * n_state), SV = random_half(rng, (size_t)n_text * n_state);
    const std::vector<uint16_t> CK = random_half(rng, (size_t)n_audio * n_state), CV = random_half(rng, (size_t)n_audio * n_state);
    const std::vector<uint16_t> Qs = random_half(rng, (size_t)n_text * n_state);
    HIP_OK(hipMemcpy(sk.p, SK.data(), SK.size() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(sv.p, SV.data(), SV.size() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(ck.p, CK.data(), CK.size() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(cv.p, CV.data(), CV.size() * 2, hipMemcpyHostToDevice));
    Dev dq(8 * n_state), dout(8 * n_state);
    const double scale = 1.0 / 8.0;
    auto check = [&](const uint16_t * qhost, int M, const std::vector<uint16_t> & Kh, const std::vector<uint16_t> & Vh, int n_kv,
                     int p0, int causal, const char * what, const std::function<Status()> & call) {
        HIP_OK(hipMemcpy(dq.p, qhost, (size_t)M * n_state * 2, hipMemcpyHostToDevice));
        Status s = call();
        HIP_OK(hipDeviceSynchronize());
        EXPECT(s.is_ok());
        std::vector<uint16_t> got((size_t)M * n_state);
        HIP_OK(hipMemcpy(got.data(), dout.p, got.size() * 2, hipMemcpyDeviceToHost));
        std::vector<double> ref((size_t)M * n_state);
        oracle_attention_f64(nh, nh, hd, M, p0, n_kv, causal, scale, qhost, n_state, Kh.data(), Vh.data(), n_state, ref.data(),
                             n_state, nullptr);
        EXPECT(close(got, ref, what));
    };
    // prompt rows 0..4, then single steps at 5..9
    check(Qs.data(), 5, SK, SV, 5, 0, 1, "self prompt", [&] { return w->self_attention_prompt(0, dq.p, dout.p, 0, 5); });
    for (int p = 5; p < 10; p++)
        check(Qs.data() + (size_t)p * n_state, 1, SK, SV, p + 1, p, 1, "self step", [&] { return w->self_attention(0, dq.p, dout.p, p); });
    check(Qs.data(), 1, CK, CV, n_audio, 0, 0, "cross greedy", [&] { return w->cross_attention(0, dq.p, dout.p, 1); });
    check(Qs.data(), 5, CK, CV, n_audio, 0, 0, "cross beam 5", [&] { return w->cross_attention(0, dq.p, dout.p, 5); });
    EXPECT(w->self_attention(0, dq.p, dout.p, n_text).code == Code::ResourceExhausted);
    EXPECT(w->cross_attention(0, dq.p, dout.p, 9).code == Code::InvalidArgument);  // more rows than max_rows
    std::unique_ptr<WhisperAttention> w80;
    EXPECT(WhisperAttention::create({1, 320, 4, 8, 8, 1}, sk.p, sv.p, ck.p, cv.p, nullptr, w80).code == Code::Unsupported);
}

// The Whisper calls on the reference's f32 buffers: prompt rows and single steps write the self cache themselves (no
// rotation), cross-attention reads f32 query rows; f32 outputs against the oracle with the query rounded to half.
TEST(whisper_f32_buffers) {
    using namespace dooms_amd;
    const int n_state = 256, nh = 4, hd = 64, n_text = 32, n_audio = 150, rw = 3 * n_state;
    Dev sk((size_t)n_text * n_state), sv((size_t)n_text * n_state), ck((size_t)n_audio * n_state), cv((size_t)n_audio * n_state);
    std::unique_ptr<WhisperAttention> w;
    Status st = WhisperAttention::create({1, n_state, nh, n_text, n_audio, 8}, sk.p, sv.p, ck.p, cv.p, nullptr, w);
    EXPECT(st.is_ok());
    if (!st.is_ok()) return;
    Rng rng{31};
    const std::vector<uint16_t> CK = random_half(rng, (size_t)n_audio * n_state), CV = random_half(rng, (size_t)n_audio * n_state);
    HIP_OK(hipMemcpy(ck.p, CK.data(), CK.size() * 2, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(cv.p, CV.data(), CV.size() * 2, hipMemcpyHostToDevice));
    std::vector<uint16_t> SK((size_t)n_text * n_state), SV((size_t)n_text * n_state);
    float *dq = nullptr, *dout = nullptr;
    HIP_OK(hipMalloc(&dq, (size_t)8 * rw * 4));
    HIP_OK(hipMalloc(&dout, (size_t)8 * n_state * 4));
    const double scale = 1.0 / 8.0;
    auto compare = [&](const std::vector<uint16_t> & qh, int M, const std::vector<uint16_t> & Kh, const std::vector<uint16_t> & Vh,
                       int n_kv, int p0, int causal) {
        std::vector<double> ref((size_t)M * n_state);
        oracle_attention_f64(nh, nh, hd, M, p0, n_kv, causal, scale, qh.data(), n_state, Kh.data(), Vh.data(), n_state, ref.data(),
                             n_state, nullptr);
        std::vector<float> got((size_t)M * n_state);
        HIP_OK(hipMemcpy(got.data(), dout, got.size() * 4, hipMemcpyDeviceToHost));
        size_t bad = 0;
        for (size_t i = 0; i < got.size(); i++)
            if (!(std::fabs(got[i] - ref[i]) <= 2e-3 + 1e-2 * std::fabs(ref[i]))) bad++;
        return bad == 0;
    };
    // self: M rows of q | k | v at p0 (prompt when M > 1), checked after the library wrote the cache
    auto self_rows = [&](int p0, int M) {
        std::vector<float> rows((size_t)M * rw);
        for (auto & x : rows) x = rng.normal();
        HIP_OK(hipMemcpy(dq, rows.data(), rows.size() * 4, hipMemcpyHostToDevice));
        Status s = M == 1 ? w->self_attention(0, dq, dout, p0) : w->self_attention_prompt(0, dq, dout, p0, M);
        HIP_OK(hipDeviceSynchronize());
        EXPECT(s.is_ok());
        std::vector<uint16_t> qh((size_t)M * n_state);
        bool cache_ok = true;
        std::vector<uint16_t> gk((size_t)M * n_state), gv((size_t)M * n_state);
        HIP_OK(hipMemcpy(gk.data(), sk.p + (size_t)p0 * n_state, gk.size() * 2, hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(gv.data(), sv.p + (size_t)p0 * n_state, gv.size() * 2, hipMemcpyDeviceToHost));
        for (int t = 0; t < M; t++)
            for (int i = 0; i < n_state; i++) {
                const float * row = rows.data() + (size_t)t * rw;
                qh[(size_t)t * n_state + i] = to_half(row[i]);
                cache_ok = cache_ok && gk[(size_t)t * n_state + i] == to_half(row[n_state + i]) &&
                           gv[(size_t)t * n_state + i] == to_half(row[2 * n_state + i]);
                SK[(size_t)(p0 + t) * n_state + i] = to_half(row[n_state + i]);
                SV[(size_t)(p0 + t) * n_state + i] = to_half(row[2 * n_state + i]);
            }
        EXPECT(cache_ok);
        EXPECT(compare(qh, M, SK, SV, p0 + M, p0, 1));
    };
    self_rows(0, 5);
    for (int p = 5; p < 9; p++) self_rows(p, 1);
    for (int M : {1, 5}) {  // cross: greedy and 5 beams over the shared encoder cache
        std::vector<float> q((size_t)M * n_state);
        for (auto & x : q) x = rng.normal();
        HIP_OK(hipMemcpy(dq, q.data(), q.size() * 4, hipMemcpyHostToDevice));
        Status s = w->cross_attention(0, dq, dout, M);
        HIP_OK(hipDeviceSynchronize());
        EXPECT(s.is_ok());
        std::vector<uint16_t> qh(q.size());
        for (size_t i = 0; i < q.size(); i++) qh[i] = to_half(q[i]);
        EXPECT(compare(qh, M, CK, CV, n_audio, 0, 0));
    }
    EXPECT(w->self_attention(0, dq, dout, n_text).code == Code::ResourceExhausted);
    (void)hipFree(dq);
    (void)hipFree(dout);
}

// The IR SelfAttention op through SelfAttentionOp: f16 rows read in place (head_dim 64), f32 rows with padded head_dim
// 80 (the ViT-H shape's head size), batch 2; oracle_attention_f64 per batch element on the half-rounded operands.
TEST(ir_self_attention_op) {
    using namespace dooms_amd;
    struct Case { int B, N, H, D; DType dt; };
    for (const Case c : {Case{2, 37, 3, 64, DType::F16}, Case{2, 29, 2, 80, DType::F32}}) {
        const int E = c.H * c.D;
        const size_t n_in = (size_t)c.B * c.N * 3 * E, n_out = (size_t)c.B * c.N * E;
        Rng rng{(uint64_t)(900 + c.D)};
        std::vector<float> x(n_in);
        for (auto & v : x) v = (float)(2 * rng.uniform() - 1);
        std::vector<uint16_t> xh(n_in);
        for (size_t i = 0; i < n_in; i++) xh[i] = to_half(x[i]);
        const bool f32 = c.dt == DType::F32;
        void * dx = nullptr, * dy = nullptr;
        HIP_OK(hipMalloc(&dx, n_in * (f32 ? 4 : 2)));
        HIP_OK(hipMalloc(&dy, n_out * (f32 ? 4 : 2)));
        HIP_OK(hipMemcpy(dx, f32 ? (const void *)x.data() : (const void *)xh.data(), n_in * (f32 ? 4 : 2), hipMemcpyHostToDevice));
        std::unique_ptr<SelfAttentionOp> op;
        const float scale = 1.f / std::sqrt((float)c.D);
        EXPECT(SelfAttentionOp::create(c.H, scale, c.B, c.N, E, c.dt, nullptr, op).is_ok());
        EXPECT(op->run(dx, dy, c.B, c.N, E).is_ok());
        // more tokens than the op was created for: rejected before any launch (ResourceExhausted for the workspace, or
        // InvalidArgument first when the larger extents of the two adjacent buffers overlap)
        if (f32) EXPECT(!op->run(dx, dy, c.B, c.N + 1, E).is_ok());
        EXPECT(op->run(dx, dy, c.B, c.N, E).is_ok());
        HIP_OK(hipDeviceSynchronize());
        std::vector<uint16_t> got(n_out);
        if (f32) {
            std::vector<float> g(n_out);
            HIP_OK(hipMemcpy(g.data(), dy, n_out * 4, hipMemcpyDeviceToHost));
            for (size_t i = 0; i < n_out; i++) got[i] = to_half(g[i]);  // compared at the f16 tolerance
        } else {
            HIP_OK(hipMemcpy(got.data(), dy, n_out * 2, hipMemcpyDeviceToHost));
        }
        std::vector<double> ref(n_out);
        for (int b = 0; b < c.B; b++) {
            const uint16_t * base = xh.data() + (size_t)b * c.N * 3 * E;
            EXPECT(oracle_attention_f64(c.H, c.H, c.D, c.N, 0, c.N, 0, scale, base, 3 * E, base + E, base + 2 * E, 3 * E,
                                        ref.data() + (size_t)b * c.N * E, E, nullptr) == 0);
        }
        EXPECT(close(got, ref, f32 ? "self_attention f32 hd80" : "self_attention f16 hd64"));
        (void)hipFree(dx);
        (void)hipFree(dy);
    }
    std::unique_ptr<SelfAttentionOp> op;
    EXPECT(SelfAttentionOp::create(0, 1.f, 1, 4, 64, DType::F16, nullptr, op).code == Code::InvalidArgument);
    EXPECT(SelfAttentionOp::create(3, 1.f, 1, 4, 64, DType::F16, nullptr, op).code == Code::InvalidArgument);
    EXPECT(SelfAttentionOp::create(2, NAN, 1, 4, 64, DType::F16, nullptr, op).code == Code::InvalidArgument);
    EXPECT(SelfAttentionOp::create(1, 1.f, 1, 4, 192, DType::F16, nullptr, op).code == Code::Unsupported);
}

// A q|k|v projection with the RMS norm and bias through Projection: a 3-row decode step (GEMV) and a 20-row prompt
// chunk (GEMM) against oracle_linear_f64, and a chunk larger than the declared maximum.
TEST(projection_decode_and_prompt_rows) {
    using namespace dooms_amd;
    const int N = 48, K = 96, maxM = 20;
    Rng rng{77};
    std::vector<float> x((size_t)maxM * K), g(K), bias(N);
    std::vector<uint16_t> w((size_t)N * K);
    for (auto & v : x) v = 2 * rng.normal();
    for (auto & v : g) v = (float)(0.2 + 1.8 * rng.uniform());
    for (auto & v : bias) v = rng.normal();
    for (auto & v : w) v = to_half(rng.normal() / std::sqrt((float)K));
    float * dx = nullptr, * dg = nullptr, * db = nullptr, * dy = nullptr;
    uint16_t * dw = nullptr;
    HIP_OK(hipMalloc(&dx, x.size() * 4));
    HIP_OK(hipMalloc(&dg, g.size() * 4));
    HIP_OK(hipMalloc(&db, bias.size() * 4));
    HIP_OK(hipMalloc(&dy, (size_t)maxM * N * 4));
    HIP_OK(hipMalloc(&dw, w.size() * 2));
    HIP_OK(hipMemcpy(dx, x.data(), x.size() * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dg, g.data(), g.size() * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(db, bias.data(), bias.size() * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dw, w.data(), w.size() * 2, hipMemcpyHostToDevice));
    const uint32_t flags = MX_LINEAR_RMS_NORM | MX_LINEAR_BIAS;
    std::unique_ptr<Projection> proj;
    EXPECT(Projection::create(N, K, flags, 1e-5f, maxM, nullptr, proj).is_ok());
    const uint16_t * W[1] = {dw};
    void * Y[1] = {dy};
    const float * B[1] = {db};
    for (int M : {3, 9, maxM}) {
        EXPECT(proj->run(M, 1, W, dx, K, Y, N, dg, B).is_ok());
        HIP_OK(hipDeviceSynchronize());
        std::vector<float> got((size_t)M * N);
        HIP_OK(hipMemcpy(got.data(), dy, got.size() * 4, hipMemcpyDeviceToHost));
        std::vector<double> ref((size_t)M * N, 0.0);
        EXPECT(oracle_linear_f64(M, N, K, flags, M > 8, 1e-5f, x.data(), K, w.data(), g.data(), bias.data(), ref.data()) == 0);
        double worst = 0;
        for (size_t i = 0; i < ref.size(); i++) worst = std::max(worst, std::fabs(got[i] - ref[i]));
        if (!(worst <= 2e-2)) std::fprintf(stderr, "  projection M=%d: max abs err %.3e\n", M, worst);
        EXPECT(worst <= 2e-2);  // |y| ~ 2 sqrt(K) / sqrt(K): f32 accumulation of half operands stays far below this
    }
    EXPECT(proj->run(maxM + 1, 1, W, dx, K, Y, N, dg, B).code == Code::ResourceExhausted);
    (void)hipFree(dx);
    (void)hipFree(dg);
    (void)hipFree(db);
    (void)hipFree(dy);
    (void)hipFree(dw);
}

// The Whisper cross-attention cache from encoder states (set_audio / encode_cross, metal_whisper_decoder.mm:295-316,
// 500-520): two layers' K (no bias) and V (bias) through WhisperCrossCache, checked against oracle_linear_f64 (the
// half-staged form, rounded to half), then cross-attention over the produced cache against the attention oracle.
TEST(whisper_cross_cache_from_encoder_states) {
    using namespace dooms_amd;
    const int n_layer = 2, n_state = 128, nh = 2, hd = 64, n_text = 16, n_audio = 150;
    Dev sk((size_t)n_layer * n_text * n_state), sv((size_t)n_layer * n_text * n_state);
    Dev ck((size_t)n_layer * n_audio * n_state), cv((size_t)n_layer * n_audio * n_state);
    const WhisperAttentionConfig cfg{n_layer, n_state, nh, n_text, n_audio, 8};
    std::unique_ptr<WhisperAttention> w;
    std::unique_ptr<WhisperCrossCache> prod;
    EXPECT(WhisperAttention::create(cfg, sk.p, sv.p, ck.p, cv.p, nullptr, w).is_ok());
    EXPECT(WhisperCrossCache::create(cfg, nullptr, prod).is_ok());
    if (!w || !prod) return;
    Rng rng{31};
    std::vector<float> X((size_t)n_audio * n_state);
    for (auto & x : X) x = rng.normal();
    std::vector<std::vector<uint16_t>> Wk(n_layer), Wv(n_layer);
    std::vector<std::vector<float>> Bv(n_layer);
    float * dX = nullptr;
    HIP_OK(hipMalloc(&dX, X.size() * 4));
    HIP_OK(hipMemcpy(dX, X.data(), X.size() * 4, hipMemcpyHostToDevice));
    std::vector<uint16_t *> dWk(n_layer), dWv(n_layer);
    std::vector<float *> dBv(n_layer);
    for (int l = 0; l < n_layer; l++) {
        Wk[l].resize((size_t)n_state * n_state);
        Wv[l].resize((size_t)n_state * n_state);
        Bv[l].resize(n_state);
        for (auto & x : Wk[l]) x = to_half(rng.normal() / std::sqrt((float)n_state));
        for (auto & x : Wv[l]) x = to_half(rng.normal() / std::sqrt((float)n_state));
        for (auto & x : Bv[l]) x = rng.normal();
        HIP_OK(hipMalloc(&dWk[l], Wk[l].size() * 2));
        HIP_OK(hipMalloc(&dWv[l], Wv[l].size() * 2));
        HIP_OK(hipMalloc(&dBv[l], Bv[l].size() * 4));
        HIP_OK(hipMemcpy(dWk[l], Wk[l].data(), Wk[l].size() * 2, hipMemcpyHostToDevice));
        HIP_OK(hipMemcpy(dWv[l], Wv[l].data(), Wv[l].size() * 2, hipMemcpyHostToDevice));
        HIP_OK(hipMemcpy(dBv[l], Bv[l].data(), Bv[l].size() * 4, hipMemcpyHostToDevice));
    }
    EXPECT(prod->set_audio(*w, dX, dWk.data(), dWv.data(), dBv.data()).is_ok());
    HIP_OK(hipDeviceSynchronize());
    for (int l = 0; l < n_layer; l++) {
        for (int kv = 0; kv < 2; kv++) {
            std::vector<uint16_t> got((size_t)n_audio * n_state);
            HIP_OK(hipMemcpy(got.data(), kv ? w->cross_v(l) : w->cross_k(l), got.size() * 2, hipMemcpyDeviceToHost));
            std::vector<double> ref((size_t)n_audio * n_state, 0.0);
            EXPECT(oracle_linear_f64(n_audio, n_state, n_state, kv ? 4u : 0u, 1, 0.f, X.data(), n_state,
                                     kv ? Wv[l].data() : Wk[l].data(), nullptr, kv ? Bv[l].data() : nullptr, ref.data()) == 0);
            double worst = 0;
            for (size_t i = 0; i < ref.size(); i++) worst = std::max(worst, std::fabs(from_half(got[i]) - ref[i]) / (1.0 + std::fabs(ref[i])));
            if (!(worst <= 4e-3)) std::fprintf(stderr, "  cross cache layer %d %s: max scaled err %.3e\n", l, kv ? "V" : "K", worst);
            EXPECT(worst <= 4e-3);  // f32 accumulation of half operands, then one rounding to half (2^-11 relative)
        }
        // cross-attention (greedy row) over the produced cache
        std::vector<uint16_t> CK((size_t)n_audio * n_state), CV((size_t)n_audio * n_state);
        HIP_OK(hipMemcpy(CK.data(), w->cross_k(l), CK.size() * 2, hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(CV.data(), w->cross_v(l), CV.size() * 2, hipMemcpyDeviceToHost));
        const std::vector<uint16_t> q = random_half(rng, n_state);
        Dev dq(n_state), dout(n_state);
        HIP_OK(hipMemcpy(dq.p, q.data(), q.size() * 2, hipMemcpyHostToDevice));
        EXPECT(w->cross_attention(l, dq.p, dout.p, 1).is_ok());
        HIP_OK(hipDeviceSynchronize());
        std::vector<uint16_t> got(n_state);
        HIP_OK(hipMemcpy(got.data(), dout.p, got.size() * 2, hipMemcpyDeviceToHost));
        std::vector<double> ref(n_state);
        oracle_attention_f64(nh, nh, hd, 1, 0, n_audio, 0, 1.0 / 8.0, q.data(), n_state, CK.data(), CV.data(), n_state,
                             ref.data(), n_state, nullptr);
        EXPECT(close(got, ref, "cross-attention over the produced cache"));
    }
    (void)hipFree(dX);
    for (int l = 0; l < n_layer; l++) {
        (void)hipFree(dWk[l]);
        (void)hipFree(dWv[l]);
        (void)hipFree(dBv[l]);
    }
}

int main() {
    int dev_count = 0;
    if (hipGetDeviceCount(&dev_count) != hipSuccess || dev_count < 1) {
        std::fprintf(stderr, "no GPU\n");
        return 125;
    }
    for (auto & [name, fn] : registry()) {
        const int before = g_failed;
        std::fprintf(stderr, "%s\n", name);
        fn();
        std::fprintf(stderr, "  %s\n", g_failed == before ? "ok" : "FAILED");
    }
    std::fprintf(stderr, "%d checks, %d failed\n", g_checks, g_failed);
    return g_failed;
}
