// Library GEMM plans for a prompt chunk's projection (mx_linear_plan_* in include/mx_linear.h): after stage_kernel the
// product is a plain f16 x f16 -> f32 (or f16) GEMM with a bias epilogue and beta = 1 for the residual, which a plan
// runs on hipBLASLt.
//
// Everything that allocates, locks or searches happens when the plan is created: hipBLASLt itself is loaded then
// (dlopen, so that the attention library does not depend on it), and the plan's handle, matrix descriptors and the
// algorithm hipBLASLt's heuristic picks for the exact shape are made and kept. Running a plan stages the input rows and
// enqueues one hipblasLtMatmul: no allocation, no lock, no search.
//
// hipBLASLt is column-major; with row-major Y [M][y_stride] = X W^T this is Y^T (N x M, ld y_stride) = op(W) (N x K) .
// X^T (K x M): A is W read transposed (col-major K x N, ld K), B the staged rows (col-major K x M, ld kp).
#include <dlfcn.h>
#include <hipblaslt/hipblaslt.h>

#include <mutex>
#include <string>

#include "mx_kernels.hpp"

namespace mx {

namespace {

// The hipBLASLt entry points a plan uses, resolved once from the shared library.
struct BlasApi {
    decltype(&hipblasLtCreate) create;
    decltype(&hipblasLtDestroy) destroy;
    decltype(&hipblasLtMatmulDescCreate) desc_create;
    decltype(&hipblasLtMatmulDescDestroy) desc_destroy;
    decltype(&hipblasLtMatmulDescSetAttribute) desc_set;
    decltype(&hipblasLtMatrixLayoutCreate) layout_create;
    decltype(&hipblasLtMatrixLayoutDestroy) layout_destroy;
    decltype(&hipblasLtMatmulPreferenceCreate) pref_create;
    decltype(&hipblasLtMatmulPreferenceDestroy) pref_destroy;
    decltype(&hipblasLtMatmulPreferenceSetAttribute) pref_set;
    decltype(&hipblasLtMatmulAlgoGetHeuristic) heuristic;
    decltype(&hipblasLtMatmul) matmul;
};

const BlasApi * blas_api(std::string & err) {
    static std::once_flag once;
    static BlasApi api;
    static bool ok = false;
    static std::string load_err;
    std::call_once(once, [] {
        void * h = dlopen("libhipblaslt.so.1", RTLD_NOW | RTLD_LOCAL);
        if (!h) h = dlopen("libhipblaslt.so", RTLD_NOW | RTLD_LOCAL);
        if (!h) {
            const char * e = dlerror();
            load_err = std::string("cannot load hipBLASLt: ") + (e ? e : "unknown error");
            return;
        }
        bool all = true;
        auto sym = [&](auto & fn, const char * name) {
            fn = reinterpret_cast<std::remove_reference_t<decltype(fn)>>(dlsym(h, name));
            if (!fn) {
                all = false;
                load_err = std::string("hipBLASLt lacks ") + name;
            }
        };
        sym(api.create, "hipblasLtCreate");
        sym(api.destroy, "hipblasLtDestroy");
        sym(api.desc_create, "hipblasLtMatmulDescCreate");
        sym(api.desc_destroy, "hipblasLtMatmulDescDestroy");
        sym(api.desc_set, "hipblasLtMatmulDescSetAttribute");
        sym(api.layout_create, "hipblasLtMatrixLayoutCreate");
        sym(api.layout_destroy, "hipblasLtMatrixLayoutDestroy");
        sym(api.pref_create, "hipblasLtMatmulPreferenceCreate");
        sym(api.pref_destroy, "hipblasLtMatmulPreferenceDestroy");
        sym(api.pref_set, "hipblasLtMatmulPreferenceSetAttribute");
        sym(api.heuristic, "hipblasLtMatmulAlgoGetHeuristic");
        sym(api.matmul, "hipblasLtMatmul");
        ok = all;  // the library stays loaded for the process
    });
    if (!ok) err = load_err;
    return ok ? &api : nullptr;
}

}  // namespace

struct BlasPlan {
    const BlasApi * api = nullptr;
    hipblasLtHandle_t handle = nullptr;
    hipblasLtMatmulDesc_t op = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    int device = 0;
    bool bias = false;

    ~BlasPlan() {
        if (!api) return;
        if (a) api->layout_destroy(a);
        if (b) api->layout_destroy(b);
        if (c) api->layout_destroy(c);
        if (op) api->desc_destroy(op);
        if (handle) api->destroy(handle);
    }
};

BlasPlan * blas_plan_create(const LinearParams & p, int device, std::string & err) {
    const BlasApi * api = blas_api(err);
    if (!api) return nullptr;
    BlasPlan * pl = new BlasPlan;
    pl->api = api;
    pl->device = device;
    pl->bias = p.flags & kLinearBias;
    const int kp = (p.K + 63) / 64 * 64;  // staged rows, zero-padded to a multiple of 64 columns
    const hipDataType yt = (p.flags & kLinearOutF16) ? HIP_R_16F : HIP_R_32F;
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    const hipblasLtEpilogue_t ep = pl->bias ? HIPBLASLT_EPILOGUE_BIAS : HIPBLASLT_EPILOGUE_DEFAULT;
    const hipDataType bt = HIP_R_32F;
    hipblasLtMatmulPreference_t pref = nullptr;
    bool ok = api->create(&pl->handle) == HIPBLAS_STATUS_SUCCESS;
    if (!ok) pl->handle = nullptr;
    ok = ok && api->desc_create(&pl->op, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
         api->desc_set(pl->op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta) == HIPBLAS_STATUS_SUCCESS &&
         api->desc_set(pl->op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb) == HIPBLAS_STATUS_SUCCESS &&
         api->desc_set(pl->op, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof ep) == HIPBLAS_STATUS_SUCCESS &&
         api->desc_set(pl->op, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof bt) == HIPBLAS_STATUS_SUCCESS &&
         api->layout_create(&pl->a, HIP_R_16F, p.K, p.N, p.K) == HIPBLAS_STATUS_SUCCESS &&
         api->layout_create(&pl->b, HIP_R_16F, p.K, p.M, kp) == HIPBLAS_STATUS_SUCCESS &&
         api->layout_create(&pl->c, yt, p.N, p.M, p.y_stride) == HIPBLAS_STATUS_SUCCESS &&
         api->pref_create(&pref) == HIPBLAS_STATUS_SUCCESS;
    if (!ok) err = "hipBLASLt refused the plan's descriptors";
    if (ok) {
        const uint64_t ws = 0;  // no workspace: a plan needs nothing beyond mx_linear's staging buffer
        api->pref_set(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof ws);
        hipblasLtMatmulHeuristicResult_t res{};
        int n = 0;
        ok = api->heuristic(pl->handle, pl->op, pl->a, pl->b, pl->c, pl->c, pref, 1, &res, &n) == HIPBLAS_STATUS_SUCCESS &&
             n > 0 && res.state == HIPBLAS_STATUS_SUCCESS;
        if (ok) pl->algo = res.algo;
        else err = "hipBLASLt has no algorithm for this shape (mx_linear runs it)";
    }
    if (pref) api->pref_destroy(pref);
    if (!ok) {
        delete pl;
        return nullptr;
    }
    return pl;
}

void blas_plan_destroy(BlasPlan * pl) { delete pl; }

int blas_plan_device(const BlasPlan * pl) { return pl->device; }

// Stages the rows and enqueues the product. The bias pointer is an attribute of the plan's descriptor, set for each
// run: a plan runs on one thread at a time.
hipError_t blas_plan_run(BlasPlan * pl, const LinearParams & p, hipStream_t stream) {
    if (hipError_t e = launch_stage(p, stream); e != hipSuccess) return e;
    const BlasApi * api = pl->api;
    const float alpha = 1.f, beta = (p.flags & kLinearAccumulate) ? 1.f : 0.f;
    const hipblasLtEpilogue_t ep = (pl->bias && p.bias[0]) ? HIPBLASLT_EPILOGUE_BIAS : HIPBLASLT_EPILOGUE_DEFAULT;
    const void * bias = p.bias[0];
    const bool ok =
        api->desc_set(pl->op, HIPBLASLT_MATMUL_DESC_EPILOGUE, &ep, sizeof ep) == HIPBLAS_STATUS_SUCCESS &&
        api->desc_set(pl->op, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof bias) == HIPBLAS_STATUS_SUCCESS &&
        api->matmul(pl->handle, pl->op, &alpha, p.w[0], pl->a, p.xh, pl->b, &beta, p.y[0], pl->c, p.y[0], pl->c,
                    &pl->algo, nullptr, 0, stream) == HIPBLAS_STATUS_SUCCESS;
    // a refused call (an operand alignment the algorithm does not take, say) enqueues nothing: the hand-written GEMM
    // runs on the staged rows instead
    if (!ok) return launch_gemm(p, stream);
    return hipGetLastError();
}

}  // namespace mx
