// ksq_abi.hip - the C ABI of libksq.so (declared in include/ksq.h).
//
// Validation, error reporting, the per-device workspace pool and path
// selection live here; kernels live in the other .hip files.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/ksq.h"
#include "ksq_internal.h"

namespace ksq {
hipError_t launch_mmq_block_sumi(int wtype, const uint8_t* W, const uint8_t* A, int32_t* out, int M, int N,
                                 int K, hipStream_t s);
}

namespace {

thread_local int g_status = KSQ_OK;
thread_local char g_message[256] = "ok";
int g_path = 0;

int set_error(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int set_error(int status, const char* fmt, ...) {
    g_status = status;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_message, sizeof(g_message), fmt, ap);
    va_end(ap);
    return status;
}

int ok() {
    g_status = KSQ_OK;
    std::strcpy(g_message, "ok");
    return KSQ_OK;
}

int hip_error(hipError_t e, const char* where) {
    return set_error(KSQ_ERR_HIP, "%s: %s", where, hipGetErrorString(e));
}

// Per-device scratch for the Q8_1 copy of fp32 activations.
struct Pool {
    void* ptr = nullptr;
    size_t size = 0;
};
std::mutex g_pool_mu;
std::vector<Pool> g_pools;

int pool_get(size_t bytes, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_error(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_pool_mu);
    if ((int)g_pools.size() <= dev) g_pools.resize(dev + 1);
    Pool& p = g_pools[dev];
    if (p.size < bytes) {
        if (p.ptr) {
            e = hipFree(p.ptr);  // synchronises the device: no launch still reads the old buffer
            p.ptr = nullptr;
            p.size = 0;
            if (e != hipSuccess) return hip_error(e, "hipFree(workspace)");
        }
        size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
        e = hipMalloc(&p.ptr, want);
        if (e != hipSuccess) return hip_error(e, "hipMalloc(workspace)");
        p.size = want;
    }
    *out = p.ptr;
    return KSQ_OK;
}

int block_elems(int wtype) { return (wtype == KSQ_W_Q4_K || wtype == KSQ_W_Q6_K) ? 256 : 32; }

int check_common(int wtype, int atype, const void* weight, const void* activation, const void* output, int M,
                 int N, int K) {
    if (wtype < KSQ_W_Q4_0 || wtype > KSQ_W_Q6_K) return set_error(KSQ_ERR_TYPE, "unknown weight type %d", wtype);
    if (atype != KSQ_A_F32 && atype != KSQ_A_Q8_1)
        return set_error(KSQ_ERR_TYPE, "unknown activation type %d", atype);
    if (M < 0 || N < 0 || K < 0) return set_error(KSQ_ERR_SHAPE, "negative shape M=%d N=%d K=%d", M, N, K);
    const int be = block_elems(wtype);
    if (K % be != 0) return set_error(KSQ_ERR_SHAPE, "K=%d is not a multiple of %d", K, be);
    if (M == 0 || N == 0) return KSQ_OK;
    if (!output) return set_error(KSQ_ERR_NULL, "output is NULL");
    if (K == 0) return KSQ_OK;
    if (!weight || !activation) return set_error(KSQ_ERR_NULL, "weight or activation is NULL");
    const uintptr_t w = (uintptr_t)weight, a = (uintptr_t)activation, o = (uintptr_t)output;
    if (w & 1u) return set_error(KSQ_ERR_ALIGN, "weight must be 2-byte aligned");
    if ((wtype == KSQ_W_Q4_K || wtype == KSQ_W_Q6_K) && (w & 3u))
        return set_error(KSQ_ERR_ALIGN, "K-quant weight must be 4-byte aligned");
    if (atype == KSQ_A_F32 && (a & 15u)) return set_error(KSQ_ERR_ALIGN, "fp32 activation must be 16-byte aligned");
    if (atype == KSQ_A_Q8_1 && (a & 3u)) return set_error(KSQ_ERR_ALIGN, "Q8_1 activation must be 4-byte aligned");
    if (o & 3u) return set_error(KSQ_ERR_ALIGN, "output must be 4-byte aligned");
    return KSQ_OK;
}

int run_matmul(int wtype, const uint8_t* W, const uint8_t* Aq, float* C, int M, int N, int K, hipStream_t s) {
    hipError_t e;
    const bool use_mmq = (g_path != 1) && ksq::mmq_supported(wtype, M, N, K, W, Aq) && (g_path == 2 || M > 8);
    if (use_mmq)
        e = ksq::launch_mmq(wtype, W, Aq, C, M, N, K, s);
    else
        e = ksq::launch_gemv(wtype, W, Aq, C, M, N, K, s);
    if (e != hipSuccess) return hip_error(e, use_mmq ? "mmq launch" : "gemv launch");
    return KSQ_OK;
}

}  // namespace

extern "C" {

int ksq_last_error(void) { return g_status; }
const char* ksq_last_error_message(void) { return g_message; }

const char* ksq_error_string(int status) {
    switch (status) {
        case KSQ_OK: return "ok";
        case KSQ_ERR_NULL: return "null pointer";
        case KSQ_ERR_SHAPE: return "invalid shape";
        case KSQ_ERR_ALIGN: return "misaligned pointer";
        case KSQ_ERR_TYPE: return "unknown type";
        case KSQ_ERR_WORKSPACE: return "workspace too small";
        case KSQ_ERR_HIP: return "HIP runtime error";
        default: return "unknown status";
    }
}

const char* ksq_version(void) { return "ksq 0.1 gfx950"; }

void ksq_release(void) {
    std::lock_guard<std::mutex> lk(g_pool_mu);
    int cur = 0;
    (void)hipGetDevice(&cur);
    for (size_t d = 0; d < g_pools.size(); d++) {
        if (g_pools[d].ptr) {
            (void)hipSetDevice((int)d);
            (void)hipFree(g_pools[d].ptr);
        }
        g_pools[d] = Pool{};
    }
    (void)hipSetDevice(cur);
}

int ksq_set_path(int path) {
    if (path < 0 || path > 2) return set_error(KSQ_ERR_TYPE, "unknown path %d", path);
    g_path = path;
    return ok();
}

int ksq_quantize_q8_1(const float* x, uint8_t* y, int M, int K, void* stream) {
    if (M < 0 || K < 0 || K % 32) return set_error(KSQ_ERR_SHAPE, "bad shape M=%d K=%d", M, K);
    if (M == 0 || K == 0) return ok();
    if (!x || !y) return set_error(KSQ_ERR_NULL, "x or y is NULL");
    if (((uintptr_t)x & 15u) || ((uintptr_t)y & 3u))
        return set_error(KSQ_ERR_ALIGN, "x must be 16-byte and y 4-byte aligned");
    hipError_t e = ksq::launch_quantize_q8_1(x, y, M, K, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "quantize launch");
    return ok();
}

size_t ksq_gemm_workspace_size(int wtype, int atype, int M, int N, int K) {
    (void)wtype;
    (void)N;
    if (atype != KSQ_A_F32 || M <= 0 || K <= 0) return 0;
    return (size_t)M * (size_t)(K / 32) * 36u;
}

int ksq_gemm(int wtype, int atype, const void* weight, const void* activation, float* output, int M, int N,
             int K, void* workspace, size_t workspace_bytes, void* stream) {
    int st = check_common(wtype, atype, weight, activation, output, M, N, K);
    if (st != KSQ_OK) return st;
    if (M == 0 || N == 0) return ok();
    hipStream_t s = (hipStream_t)stream;
    if (K == 0) {
        hipError_t e = ksq::launch_fill_zero(output, (int64_t)M * N, s);
        return e == hipSuccess ? ok() : hip_error(e, "fill launch");
    }
    const uint8_t* Aq = (const uint8_t*)activation;
    if (atype == KSQ_A_F32) {
        const size_t need = ksq_gemm_workspace_size(wtype, atype, M, N, K);
        void* ws = workspace;
        if (ws) {
            if (workspace_bytes < need)
                return set_error(KSQ_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, need);
            if ((uintptr_t)ws & 15u) return set_error(KSQ_ERR_ALIGN, "workspace must be 16-byte aligned");
        } else {
            st = pool_get(need, &ws);
            if (st != KSQ_OK) return st;
        }
        hipError_t e = ksq::launch_quantize_q8_1((const float*)activation, (uint8_t*)ws, M, K, s);
        if (e != hipSuccess) return hip_error(e, "quantize launch");
        Aq = (const uint8_t*)ws;
    }
    st = run_matmul(wtype, (const uint8_t*)weight, Aq, output, M, N, K, s);
    return st == KSQ_OK ? ok() : st;
}

int ksq_debug_block_sumi(int wtype, const void* weight, const uint8_t* act_q8_1, int32_t* out, int M, int N,
                         int K, void* stream) {
    int st = check_common(wtype, KSQ_A_Q8_1, weight, act_q8_1, out, M, N, K);
    if (st != KSQ_OK) return st;
    if (M == 0 || N == 0 || K == 0) return ok();
    hipError_t e = ksq::launch_block_sumi(wtype, (const uint8_t*)weight, act_q8_1, out, M, N, K, (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_error(e, "block_sumi launch");
}

int ksq_debug_block_sumi_mfma(int wtype, const void* weight, const uint8_t* act_q8_1, int32_t* out, int M, int N,
                              int K, void* stream) {
    int st = check_common(wtype, KSQ_A_Q8_1, weight, act_q8_1, out, M, N, K);
    if (st != KSQ_OK) return st;
    if (M == 0 || N == 0 || K == 0) return ok();
    if (!ksq::mmq_supported(wtype, M, N, K, weight, act_q8_1))
        return set_error(KSQ_ERR_SHAPE, "MFMA path needs Q4_0/Q8_0, K %% 256 == 0 and 16-byte aligned operands");
    hipError_t e = ksq::launch_mmq_block_sumi(wtype, (const uint8_t*)weight, act_q8_1, out, M, N, K, (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_error(e, "mfma block_sumi launch");
}

#define KSQ_DROPIN(NAME, WT, AT, ACT_T)                                                              \
    void NAME(const uint8_t* weight, const ACT_T* activation, float* output, int M, int N, int K) { \
        (void)ksq_gemm(WT, AT, weight, activation, output, M, N, K, nullptr, 0, nullptr);             \
    }

KSQ_DROPIN(gemm_w4a32c8_q4_0_fp32_int8, KSQ_W_Q4_0, KSQ_A_F32, float)
KSQ_DROPIN(gemm_w8a32c8_q8_0_fp32_int8, KSQ_W_Q8_0, KSQ_A_F32, float)
KSQ_DROPIN(gemm_w4a32c8_q4_k_fp32_int8, KSQ_W_Q4_K, KSQ_A_F32, float)
KSQ_DROPIN(gemm_w6a32c8_q6_k_fp32_int8, KSQ_W_Q6_K, KSQ_A_F32, float)
KSQ_DROPIN(ksq_gemm_q4_0_q8_1, KSQ_W_Q4_0, KSQ_A_Q8_1, uint8_t)
KSQ_DROPIN(ksq_gemm_q8_0_q8_1, KSQ_W_Q8_0, KSQ_A_Q8_1, uint8_t)
KSQ_DROPIN(ksq_gemm_q4_k_q8_1, KSQ_W_Q4_K, KSQ_A_Q8_1, uint8_t)
KSQ_DROPIN(ksq_gemm_q6_k_q8_1, KSQ_W_Q6_K, KSQ_A_Q8_1, uint8_t)

}  // extern "C"
