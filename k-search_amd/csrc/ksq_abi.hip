// ksq_abi.hip - the C ABI of libksq.so (declared in include/ksq.h).
//
// Validation, error reporting, the per-device workspace pool and path
// selection live here; kernels live in the other .hip files.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
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
thread_local int g_path = 0;              // ksq_set_path: a per-thread routing override
thread_local uint32_t g_engines = 0;      // kernel families of the thread's last call

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

// Library scratch: the quantised copy of fp32 activations, split-K partial sums and the MoE
// routing tables when the caller passes no workspace.  One pool per (device, stream): calls on
// one stream run in stream order and share it; eager calls on two streams of one GPU get two
// buffers and cannot race.  A pool that must grow takes a new, larger buffer and keeps the
// outgrown one until ksq_release(): a graph captured earlier may still read and write it.
// Growing is refused while the stream captures a graph; a capturing stream whose own pool is too
// small uses the device's largest pool that is large enough (the usual warm-up-then-capture
// sequence: the call was made eagerly on another stream first), so such a graph shares that
// stream's pool and must not run concurrently with its calls.
struct Pool {
    void* ptr = nullptr;
    size_t size = 0;
    std::vector<void*> retired;
};
std::mutex g_pool_mu;
std::map<std::pair<int, uintptr_t>, Pool> g_pools;

int pool_get(size_t bytes, hipStream_t s, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_error(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_pool_mu);
    Pool& p = g_pools[{dev, (uintptr_t)s}];
    if (p.size < bytes) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (s && hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
            const Pool* big = nullptr;
            for (const auto& kv : g_pools)
                if (kv.first.first == dev && kv.second.size >= bytes && (!big || kv.second.size > big->size))
                    big = &kv.second;
            if (big) {
                *out = big->ptr;
                return KSQ_OK;
            }
            return set_error(KSQ_ERR_WORKSPACE,
                             "the workspace pool would have to grow to %zu bytes during graph capture; "
                             "pass a workspace",
                             bytes);
        }
        size_t want = 2 * p.size;
        if (want < bytes) want = bytes;
        if (want < (1u << 20)) want = 1u << 20;
        void* np = nullptr;
        e = hipMalloc(&np, want);
        if (e != hipSuccess) return hip_error(e, "hipMalloc(workspace)");
        if (p.ptr) p.retired.push_back(p.ptr);
        p.ptr = np;
        p.size = want;
    }
    *out = p.ptr;
    return KSQ_OK;
}

// ksq_gemm_noalloc's scratch: a file-scope device array (one copy per GPU, allocated with the
// code object and held until the process ends).  Host code never passes `scratch` itself to a
// kernel: that name is a host-side stand-in.  The device address of each GPU's copy comes from
// hipGetSymbolAddress, once per device, with that device current.
__device__ __attribute__((aligned(256))) uint8_t scratch[KSQ_NOALLOC_SCRATCH_BYTES];
std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;

int scratch_get(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_error(e, "hipGetDevice");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return KSQ_OK;
}

int block_elems(int wtype) { return (wtype == KSQ_W_Q4_K || wtype == KSQ_W_Q6_K) ? 256 : 32; }

bool atype_q8f(int atype) {
    return atype == KSQ_A_Q8F || atype == KSQ_A_F32_Q8F_RNE || atype == KSQ_A_F32_Q8F_LROUND;
}
bool atype_f32(int atype) {
    return atype == KSQ_A_F32 || atype == KSQ_A_F32_Q8S || atype == KSQ_A_F32_Q8F_RNE || atype == KSQ_A_F32_Q8F_LROUND;
}
// activations that arrive unquantised (fp32 or fp16) and are quantised into the workspace
bool atype_raw(int atype) { return atype_f32(atype) || atype == KSQ_A_F16; }
int atype_fmt(int atype) {
    if (atype == KSQ_A_F32_Q8S || atype == KSQ_A_Q8S) return ksq::kAQ8S;
    return atype_q8f(atype) ? ksq::kAQ8F : ksq::kAQ81;
}
// bytes of one quantised activation block
size_t atype_block_bytes(int atype) { return atype_q8f(atype) ? 40u : 36u; }

int check_common(int wtype, int atype, const void* weight, const void* activation, const void* output, int M,
                 int N, int K) {
    if (wtype < KSQ_W_Q4_0 || wtype > KSQ_W_Q5_1) return set_error(KSQ_ERR_TYPE, "unknown weight type %d", wtype);
    if (atype < KSQ_A_F32 || atype > KSQ_A_F32_Q8F_LROUND)
        return set_error(KSQ_ERR_TYPE, "unknown activation type %d", atype);
    if (atype_fmt(atype) == ksq::kAQ8S && wtype != KSQ_W_Q8_0)
        return set_error(KSQ_ERR_TYPE, "block_q8s activations pair with Q8_0 weights only (weight type %d)", wtype);
    if (atype_q8f(atype) && wtype != KSQ_W_Q4_0 && wtype != KSQ_W_Q5_0 && wtype != KSQ_W_Q8_0)
        return set_error(KSQ_ERR_TYPE, "block_q8f activations pair with Q4_0, Q5_0 and Q8_0 weights (weight type %d)",
                         wtype);
    if (M < 0 || N < 0 || K < 0) return set_error(KSQ_ERR_SHAPE, "negative shape M=%d N=%d K=%d", M, N, K);
    const int be = atype_q8f(atype) ? 256 : block_elems(wtype);
    if (K % be != 0) return set_error(KSQ_ERR_SHAPE, "K=%d is not a multiple of %d", K, be);
    if (M == 0 || N == 0) return KSQ_OK;
    if (!output) return set_error(KSQ_ERR_NULL, "output is NULL");
    if (K == 0) return KSQ_OK;
    if (!weight || !activation) return set_error(KSQ_ERR_NULL, "weight or activation is NULL");
    const uintptr_t w = (uintptr_t)weight, a = (uintptr_t)activation, o = (uintptr_t)output;
    if (w & 1u) return set_error(KSQ_ERR_ALIGN, "weight must be 2-byte aligned");
    if ((wtype == KSQ_W_Q4_K || wtype == KSQ_W_Q6_K) && (w & 3u))
        return set_error(KSQ_ERR_ALIGN, "K-quant weight must be 4-byte aligned");
    if (atype_raw(atype) && (a & 15u)) return set_error(KSQ_ERR_ALIGN, "fp32 / fp16 activation must be 16-byte aligned");
    if (!atype_raw(atype) && (a & 3u)) return set_error(KSQ_ERR_ALIGN, "quantised activation must be 4-byte aligned");
    if (atype == KSQ_A_Q8F && (a & 15u)) return set_error(KSQ_ERR_ALIGN, "block_q8f activation must be 16-byte aligned");
    if (atype_q8f(atype) && (w & 15u)) return set_error(KSQ_ERR_ALIGN, "weight must be 16-byte aligned with block_q8f");
    if (o & 3u) return set_error(KSQ_ERR_ALIGN, "output must be 4-byte aligned");
    return KSQ_OK;
}

// The MFMA GEMM above 8 rows or past the measured small-M crossovers (or when forced), the
// small-batch or v_dot4 decode kernels otherwise.
bool use_mmq(int wtype, int M, int N, int K, const void* W, bool a_aligned16) {
    if (g_path == 1 || !ksq::mmq_supported(wtype, M, N, K, W, a_aligned16)) return false;
    if (g_path == 2) return true;
    if (g_path == 3) return M > 32;
    return ksq::mmq_preferred(wtype, M, N, K);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The 4x4x4-MFMA small-batch kernel where it beats the decode kernel (path 3 forces it where it
// applies).  Checked after use_mmq.
bool use_skinny(int wtype, int afmt, int M, int N, int K, const void* W, const void* A) {
    if (!ksq::skinny_supported(wtype, afmt, M, N, K, W, A)) return false;
    return g_path == 3 || (g_path == 0 && ksq::skinny_preferred(wtype, M, N, K));
}


size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Workspace of one ksq_gemm call: [quantised activations][split-K partial sums], each part
// 256-byte aligned.  `mmq` is whether the int8 MFMA path runs (alignment permitting).
struct GemmWs {
    size_t q, p, total;
};

// Whether fp32 activations are quantised to planar block_q8_1 for the LDS-DMA GEMM (given that
// the MFMA GEMM runs).
bool use_planar(int wtype, int atype, int M, int N, int K, bool mmq) {
    return mmq && atype == KSQ_A_F32 && (K % 256) == 0 && ksq::mmq_planar_preferred(wtype, M, N, K);
}

GemmWs gemm_ws(int wtype, int atype, int M, int N, int K, bool mmq) {
    GemmWs w{};
    w.q = use_planar(wtype, atype, M, N, K, mmq)
              ? align256(ksq::planar_bytes(M, K))
              : atype_raw(atype) ? align256((size_t)M * (size_t)(K / 32) * atype_block_bytes(atype)) : 0;
    const int splits = mmq ? ksq::mmq_splits(wtype, M, N, K) : 1;
    w.p = splits > 1 ? align256((size_t)splits * (size_t)M * (size_t)N * sizeof(float)) : 0;
    w.total = w.q + w.p;
    return w;
}

int run_matmul(int wtype, int afmt, const uint8_t* W, const uint8_t* Aq, float* C, int M, int N, int K,
               float* partials, hipStream_t s) {
    hipError_t e;
    // pre-quantised block_q8f runs on the MFMA GEMM (check_common has checked its shape and
    // alignment); fp32 rows at decode sizes were taken by the fused decode kernel before
    const bool mmq = afmt == ksq::kAQ8F || use_mmq(wtype, M, N, K, W, aligned16(Aq));
    if (mmq) {
        e = ksq::launch_mmq(wtype, afmt, W, Aq, C, M, N, K, partials, s);
        if (e != hipSuccess) return hip_error(e, "mmq launch");
    } else if (use_skinny(wtype, afmt, M, N, K, W, Aq)) {
        e = ksq::launch_skinny(wtype, afmt, W, Aq, C, M, N, K, s);
        if (e != hipSuccess) return hip_error(e, "skinny launch");
    } else {
        e = ksq::launch_gemv(wtype, afmt, W, Aq, C, M, N, K, s);
        if (e != hipSuccess) return hip_error(e, "gemv launch");
    }
    return KSQ_OK;
}

}  // namespace

namespace ksq {
void note_engine(uint32_t bits) { g_engines |= bits; }
}  // namespace ksq

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
    for (auto& kv : g_pools) {
        Pool& p = kv.second;
        if (p.ptr || !p.retired.empty()) {
            (void)hipSetDevice(kv.first.first);
            if (p.ptr) (void)hipFree(p.ptr);
            for (void* r : p.retired) (void)hipFree(r);
        }
    }
    g_pools.clear();
    (void)hipSetDevice(cur);
}

uint32_t ksq_debug_last_engines(void) { return g_engines; }

int ksq_set_path(int path) {
    if (path < 0 || path > 3) return set_error(KSQ_ERR_TYPE, "unknown path %d", path);
    g_path = path;
    return ok();
}

int ksq_set_mmq_config(int config) {
    if (ksq::mmq_set_config(config) != 0) return set_error(KSQ_ERR_TYPE, "unknown MFMA tile configuration %d", config);
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

int ksq_quantize_q8_1_variant(int variant, const void* x, uint8_t* y, int M, int K, void* stream) {
    if (variant < KSQ_Q81_REF || variant > KSQ_Q81_FUSED_F16)
        return set_error(KSQ_ERR_TYPE, "unknown Q8_1 quantiser variant %d", variant);
    if (M < 0 || K < 0 || K % 32) return set_error(KSQ_ERR_SHAPE, "bad shape M=%d K=%d", M, K);
    if (M == 0 || K == 0) return ok();
    if (!x || !y) return set_error(KSQ_ERR_NULL, "x or y is NULL");
    if (((uintptr_t)x & 15u) || ((uintptr_t)y & 3u))
        return set_error(KSQ_ERR_ALIGN, "x must be 16-byte and y 4-byte aligned");
    hipError_t e = ksq::launch_quantize_variant(variant, x, y, M, K, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "quantize launch");
    return ok();
}

int ksq_quantize_weights(int wtype, int rule, const float* x, uint8_t* y, int64_t k, void* stream) {
    if (wtype != KSQ_W_Q4_0 && wtype != KSQ_W_Q8_0)
        return set_error(KSQ_ERR_TYPE, "weight quantiser for Q4_0 or Q8_0 only (wtype=%d)", wtype);
    if (rule != KSQ_WQ_DEVICE && rule != KSQ_WQ_REF) return set_error(KSQ_ERR_TYPE, "unknown weight quantiser rule %d", rule);
    if (k < 0 || k % 32) return set_error(KSQ_ERR_SHAPE, "bad element count k=%lld", (long long)k);
    if (k == 0) return ok();
    if (!x || !y) return set_error(KSQ_ERR_NULL, "x or y is NULL");
    if (((uintptr_t)x & 15u) || ((uintptr_t)y & 1u))
        return set_error(KSQ_ERR_ALIGN, "x must be 16-byte and y 2-byte aligned");
    hipError_t e = ksq::launch_quantize_weights(wtype, rule, x, y, k / 32, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "weight quantize launch");
    return ok();
}

size_t ksq_gemm_q4_0_fp16_fused_workspace_size(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    return align256(ksq_gemm_workspace_size(KSQ_W_Q4_0, KSQ_A_F16, N, M, K)) +
           align256((size_t)M * (size_t)N * sizeof(float));
}

int ksq_gemm_q4_0_fp16_fused(const uint8_t* weight, const uint16_t* fp16_activation, float* output, int M, int N,
                             int K, void* workspace, size_t workspace_bytes, void* stream) {
    // the reference's orientation: M weight rows, N activation rows, output [M][N].  Routes:
    //  * decode shapes (N <= 2): the decode kernel quantises the fp16 activations in LDS inside
    //    every workgroup and writes the [M][N] output directly (one launch, no workspace);
    //  * the int8 MFMA GEMM without split-K: quantise once into the workspace, then the GEMM
    //    writes its tile transposed, straight into [M][N];
    //  * otherwise ksq_gemm's [N][M] into the workspace, then a transpose.
    g_engines = 0;
    int st = check_common(KSQ_W_Q4_0, KSQ_A_F16, weight, fp16_activation, output, N, M, K);
    if (st != KSQ_OK) return st;
    if (M == 0 || N == 0) return ok();
    hipStream_t s = (hipStream_t)stream;
    if (K == 0) {
        hipError_t e = ksq::launch_fill_zero(output, (int64_t)M * N, s);
        return e == hipSuccess ? ok() : hip_error(e, "fill launch");
    }
    const bool mmq = use_mmq(KSQ_W_Q4_0, N, M, K, weight, true);
    if (!mmq && g_path != 3 && ksq::gemv_fused_profitable(KSQ_W_Q4_0, N, M, K, weight, true)) {
        hipError_t e = ksq::launch_gemv_fused(KSQ_W_Q4_0, ksq::kAQ81, true, weight, fp16_activation, output, N, M, K,
                                              /*ldc=*/1, /*ldr=*/N, s);
        return e == hipSuccess ? ok() : hip_error(e, "gemv launch");
    }
    const size_t need = ksq_gemm_q4_0_fp16_fused_workspace_size(M, N, K);
    void* p = workspace;
    if (p) {
        if (workspace_bytes < need) return set_error(KSQ_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, need);
        if ((uintptr_t)p & 255u) return set_error(KSQ_ERR_ALIGN, "workspace must be 256-byte aligned");
    } else {
        st = pool_get(need, s, &p);
        if (st != KSQ_OK) return st;
    }
    if (mmq && ksq::mmq_splits(KSQ_W_Q4_0, N, M, K) == 1) {
        uint8_t* aq = (uint8_t*)p;
        hipError_t e = ksq::launch_quantize_variant(KSQ_Q81_FUSED_F16, fp16_activation, aq, N, K, s);
        if (e != hipSuccess) return hip_error(e, "quantize launch");
        g_engines |= KSQ_ENG_QUANTIZE;
        e = ksq::launch_mmq(KSQ_W_Q4_0, ksq::kAQ81, weight, aq, output, N, M, K, nullptr, s, /*trans=*/true);
        return e == hipSuccess ? ok() : hip_error(e, "mmq launch");
    }
    if (N <= 8 && g_path != 2 && g_path != 3) {
        // up to 8 activation rows: quantise once, then the decode kernels write [M][N] directly.
        // Two launches; the small-batch MFMA kernel or the split MFMA GEMM would add a transpose
        // (and a reduction), measured slower at every shape tried (whole call, us: 4096 weight
        // rows, K = 4096, 8 rows 14.0 -> 11.8; 14336 x 4096, 7 rows 26.5 -> 23.6; 2048 x 4096,
        // 6 rows 12.8 -> 8.5; 4096 x 14336, 8 rows 26.1 vs 26.4 the one tie)
        uint8_t* aq = (uint8_t*)p;
        hipError_t e = ksq::launch_quantize_variant(KSQ_Q81_FUSED_F16, fp16_activation, aq, N, K, s);
        if (e != hipSuccess) return hip_error(e, "quantize launch");
        g_engines |= KSQ_ENG_QUANTIZE;
        e = ksq::launch_gemv_strided(KSQ_W_Q4_0, ksq::kAQ81, weight, aq, output, N, M, K, /*ldc=*/1, /*ldr=*/N, s);
        return e == hipSuccess ? ok() : hip_error(e, "gemv launch");
    }
    const size_t gws = align256(ksq_gemm_workspace_size(KSQ_W_Q4_0, KSQ_A_F16, N, M, K));
    float* tmp = (float*)((uint8_t*)p + gws);
    st = ksq_gemm(KSQ_W_Q4_0, KSQ_A_F16, weight, fp16_activation, tmp, N, M, K, gws ? p : nullptr, gws, stream);
    if (st != KSQ_OK) return st;
    hipError_t e = ksq::launch_transpose_f32(tmp, output, N, M, s);
    g_engines |= KSQ_ENG_TRANSPOSE;
    return e == hipSuccess ? ok() : hip_error(e, "transpose launch");
}

int ksq_quantize_q8s(const float* x, uint8_t* y, int M, int K, void* stream) {
    if (M < 0 || K < 0 || K % 32) return set_error(KSQ_ERR_SHAPE, "bad shape M=%d K=%d", M, K);
    if (M == 0 || K == 0) return ok();
    if (!x || !y) return set_error(KSQ_ERR_NULL, "x or y is NULL");
    if (((uintptr_t)x & 15u) || ((uintptr_t)y & 3u))
        return set_error(KSQ_ERR_ALIGN, "x must be 16-byte and y 4-byte aligned");
    hipError_t e = ksq::launch_quantize(ksq::kAQ8S, x, y, M, K, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "quantize launch");
    return ok();
}

size_t ksq_gemm_w16_workspace_size(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const int sp = ksq::w16_splits(M, N, K);
    return sp > 1 ? align256((size_t)sp * (size_t)M * (size_t)N * sizeof(float)) : 0;
}

int ksq_gemm_w16(int wtype, const float* A, const uint8_t* B, float* C, int M, int N, int K, void* workspace,
                 size_t workspace_bytes, void* stream) {
    g_engines = 0;
    if (wtype != KSQ_W_Q4_0 && wtype != KSQ_W_Q8_0)
        return set_error(KSQ_ERR_TYPE, "the dequantise-then-fp32 GEMM takes Q4_0 or Q8_0 weights (weight type %d)",
                         wtype);
    if (M < 0 || N < 0 || K < 0) return set_error(KSQ_ERR_SHAPE, "negative shape M=%d N=%d K=%d", M, N, K);
    if (K % 64) return set_error(KSQ_ERR_SHAPE, "K=%d is not a multiple of 64", K);
    if (M == 0 || N == 0) return ok();
    if (!C) return set_error(KSQ_ERR_NULL, "C is NULL");
    hipStream_t s = (hipStream_t)stream;
    if (K == 0) {
        hipError_t e = ksq::launch_fill_zero(C, (int64_t)M * N, s);
        return e == hipSuccess ? ok() : hip_error(e, "fill launch");
    }
    if (!A || !B) return set_error(KSQ_ERR_NULL, "A or B is NULL");
    if (((uintptr_t)A & 15u) || ((uintptr_t)B & 3u) || ((uintptr_t)C & 3u))
        return set_error(KSQ_ERR_ALIGN, "A must be 16-byte aligned, B and C 4-byte aligned");
    const size_t need = ksq_gemm_w16_workspace_size(M, N, K);
    void* ws = workspace;
    if (need) {
        if (ws) {
            if (workspace_bytes < need) return set_error(KSQ_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, need);
            if ((uintptr_t)ws & 15u) return set_error(KSQ_ERR_ALIGN, "workspace must be 16-byte aligned");
        } else {
            int st = pool_get(need, s, &ws);
            if (st != KSQ_OK) return st;
        }
    }
    hipError_t e = ksq::launch_w16(wtype, A, B, C, M, N, K, need ? (float*)ws : nullptr, s);
    return e == hipSuccess ? ok() : hip_error(e, "w16 launch");
}

int ksq_gemm_w4a16(const float* A, const uint8_t* B, float* C, int M, int N, int K, void* stream) {
    return ksq_gemm_w16(KSQ_W_Q4_0, A, B, C, M, N, K, nullptr, 0, stream);
}

int ksq_gemm_w8a16(const float* A, const uint8_t* B, float* C, int M, int N, int K, void* stream) {
    return ksq_gemm_w16(KSQ_W_Q8_0, A, B, C, M, N, K, nullptr, 0, stream);
}

int ksq_quantize_q8f(int rule, const float* x, uint8_t* y, int M, int K, void* stream) {
    if (rule != KSQ_Q8F_RNE && rule != KSQ_Q8F_LROUND)
        return set_error(KSQ_ERR_TYPE, "unknown block_q8f quantiser rule %d", rule);
    if (M < 0 || K < 0 || K % 32) return set_error(KSQ_ERR_SHAPE, "bad shape M=%d K=%d", M, K);
    if (M == 0 || K == 0) return ok();
    if (!x || !y) return set_error(KSQ_ERR_NULL, "x or y is NULL");
    if (((uintptr_t)x & 15u) || ((uintptr_t)y & 3u))
        return set_error(KSQ_ERR_ALIGN, "x must be 16-byte and y 4-byte aligned");
    hipError_t e = ksq::launch_quantize_q8f(rule, x, y, M, K, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "quantize launch");
    return ok();
}

size_t ksq_gemm_workspace_size(int wtype, int atype, int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    const bool mmq_possible = atype_q8f(atype) ||
        ((g_path != 1) && (g_path == 2 || ksq::mmq_preferred(wtype, M, N, K)) && (K % 256) == 0);
    return gemm_ws(wtype, atype, M, N, K, mmq_possible).total;
}

int ksq_gemm(int wtype, int atype, const void* weight, const void* activation, float* output, int M, int N,
             int K, void* workspace, size_t workspace_bytes, void* stream) {
    g_engines = 0;
    int st = check_common(wtype, atype, weight, activation, output, M, N, K);
    if (st != KSQ_OK) return st;
    if (M == 0 || N == 0) return ok();
    hipStream_t s = (hipStream_t)stream;
    if (K == 0) {
        hipError_t e = ksq::launch_fill_zero(output, (int64_t)M * N, s);
        return e == hipSuccess ? ok() : hip_error(e, "fill launch");
    }
    const uint8_t* Aq = (const uint8_t*)activation;
    const int afmt = atype_fmt(atype);
    // decode shapes: the activations are quantised inside every workgroup of the decode kernel
    // (fp32, or fp16 by the fused FP16 kernels' rules), no quantise launch and no workspace
    const bool xh = atype == KSQ_A_F16;
    if (((atype_f32(atype) && !atype_q8f(atype)) || xh) && ksq::gemv_fused_profitable(wtype, M, N, K, weight, xh) &&
        !use_mmq(wtype, M, N, K, weight, true) && g_path != 3) {
        hipError_t e = ksq::launch_gemv_fused(wtype, afmt, xh, (const uint8_t*)weight, activation, output, M, N, K, N,
                                              1, s);
        return e == hipSuccess ? ok() : hip_error(e, "gemv launch");
    }
    // block_q8f rules on 1-2 fp32 rows: the decode kernel quantises them in every workgroup too
    if ((atype == KSQ_A_F32_Q8F_RNE || atype == KSQ_A_F32_Q8F_LROUND) && g_path != 2 && g_path != 3 &&
        ksq::gemv_q8f_profitable(wtype, M, N, K, weight)) {
        hipError_t e = ksq::launch_gemv_q8f(atype == KSQ_A_F32_Q8F_RNE ? KSQ_Q8F_RNE : KSQ_Q8F_LROUND, wtype,
                                            (const uint8_t*)weight, (const float*)activation, output, M, N, K, s);
        return e == hipSuccess ? ok() : hip_error(e, "gemv launch");
    }
    // fp32 / fp16 activations are quantised to the start of the (16-byte aligned) workspace,
    // which is what the GEMM then reads
    const bool f32 = atype_f32(atype), f16 = atype == KSQ_A_F16;
    const bool mmq = atype_q8f(atype) || use_mmq(wtype, M, N, K, weight, f32 || f16 || aligned16(activation));
    const GemmWs L = gemm_ws(wtype, atype, M, N, K, mmq);
    uint8_t* ws = (uint8_t*)workspace;
    if (L.total) {
        if (ws) {
            if (workspace_bytes < L.total)
                return set_error(KSQ_ERR_WORKSPACE, "workspace %zu < %zu bytes", workspace_bytes, L.total);
            if ((uintptr_t)ws & 15u) return set_error(KSQ_ERR_ALIGN, "workspace must be 16-byte aligned");
        } else {
            void* p = nullptr;
            st = pool_get(L.total, s, &p);
            if (st != KSQ_OK) return st;
            ws = (uint8_t*)p;
        }
    }
    float* partials = L.p ? (float*)(ws + L.q) : nullptr;
    if (use_planar(wtype, atype, M, N, K, mmq)) {
        // the LDS-DMA GEMM's own activation layout (same blocks, split into planes)
        const ksq::PlanarQ81 P = ksq::planar_at(ws, M, K);
        hipError_t e = ksq::launch_quantize_planar((const float*)activation, P, M, K, ksq::planar_da_scale(wtype), s);
        if (e != hipSuccess) return hip_error(e, "quantize launch");
        g_engines |= KSQ_ENG_QUANTIZE;
        e = ksq::launch_mmq_planar(wtype, (const uint8_t*)weight, P, output, M, N, K, partials, s);
        if (e != hipSuccess) return hip_error(e, "mmq launch");
        return ok();
    }
    if (f32 || f16) {
        // fp16 input takes the fused FP16 kernels' quantiser (kernels/gemm/gemm_fused.cuh:76-145)
        hipError_t e;
        if (f16) e = ksq::launch_quantize_variant(KSQ_Q81_FUSED_F16, activation, ws, M, K, s);
        else if (atype_q8f(atype))
            e = ksq::launch_quantize_q8f(atype == KSQ_A_F32_Q8F_RNE ? KSQ_Q8F_RNE : KSQ_Q8F_LROUND,
                                         (const float*)activation, ws, M, K, s);
        else e = ksq::launch_quantize(afmt, (const float*)activation, ws, M, K, s);
        if (e != hipSuccess) return hip_error(e, "quantize launch");
        g_engines |= KSQ_ENG_QUANTIZE;
        Aq = ws;
    }
    st = run_matmul(wtype, afmt, (const uint8_t*)weight, Aq, output, M, N, K, partials, s);
    return st == KSQ_OK ? ok() : st;
}

int ksq_gemm_noalloc(int wtype, int atype, const void* weight, const void* activation, float* output, int M, int N,
                     int K, void* stream) {
    g_engines = 0;
    int st = check_common(wtype, atype, weight, activation, output, M, N, K);
    if (st != KSQ_OK) return st;
    if (M == 0 || N == 0) return ok();
    // the workspace ksq_gemm would ask for (an upper bound of what this call uses)
    const size_t need = ksq_gemm_workspace_size(wtype, atype, M, N, K);
    if (need > (size_t)KSQ_NOALLOC_SCRATCH_BYTES)
        return set_error(KSQ_ERR_WORKSPACE,
                         "ksq_gemm_noalloc: this call needs %zu bytes of scratch, more than the %u-byte static "
                         "scratch; use ksq_gemm with a workspace",
                         need, (unsigned)KSQ_NOALLOC_SCRATCH_BYTES);
    void* p = nullptr;
    st = scratch_get(&p);
    if (st != KSQ_OK) return st;
    // every byte of the scratch a call reads is written first by the same call (quantised
    // activations, split-K partials), so nothing needs clearing
    return ksq_gemm(wtype, atype, weight, activation, output, M, N, K, p, (size_t)KSQ_NOALLOC_SCRATCH_BYTES, stream);
}

size_t ksq_debug_planar_bytes(int M, int K) {
    if (M <= 0 || K <= 0 || K % 256) return 0;
    return ksq::planar_bytes(M, K);
}

int ksq_debug_quantize_planar(int wtype, const float* x, void* planar, int M, int K, void* stream) {
    if (wtype != KSQ_W_Q4_0 && wtype != KSQ_W_Q4_1)
        return set_error(KSQ_ERR_TYPE, "the LDS-DMA GEMM takes Q4_0 and Q4_1 weights (weight type %d)", wtype);
    if (M < 0 || K < 0 || K % 256) return set_error(KSQ_ERR_SHAPE, "bad shape M=%d K=%d (K %% 256 == 0)", M, K);
    if (M == 0 || K == 0) return ok();
    if (!x || !planar) return set_error(KSQ_ERR_NULL, "x or planar is NULL");
    if (((uintptr_t)x & 15u) || ((uintptr_t)planar & 255u))
        return set_error(KSQ_ERR_ALIGN, "x must be 16-byte and planar 256-byte aligned");
    hipError_t e = ksq::launch_quantize_planar(x, ksq::planar_at(planar, M, K), M, K, ksq::planar_da_scale(wtype),
                                               (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_error(e, "quantize launch");
}

int ksq_debug_gemm_planar(int wtype, const void* weight, const void* planar, float* output, int M, int N, int K,
                          void* stream) {
    g_engines = 0;
    if (wtype != KSQ_W_Q4_0 && wtype != KSQ_W_Q4_1)
        return set_error(KSQ_ERR_TYPE, "the LDS-DMA GEMM takes Q4_0 and Q4_1 weights (weight type %d)", wtype);
    if (M < 0 || N < 0 || K < 0 || K % 256) return set_error(KSQ_ERR_SHAPE, "bad shape M=%d N=%d K=%d", M, N, K);
    if (M == 0 || N == 0 || K == 0) return ok();
    if (!weight || !planar || !output) return set_error(KSQ_ERR_NULL, "weight, planar or output is NULL");
    if (((uintptr_t)weight & 15u) || ((uintptr_t)planar & 255u) || ((uintptr_t)output & 3u))
        return set_error(KSQ_ERR_ALIGN, "weight must be 16-byte, planar 256-byte and output 4-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    float* partials = nullptr;
    const int splits = ksq::mmq_planar_splits(wtype, M, N, K);
    if (splits > 1) {
        void* p = nullptr;
        int st = pool_get((size_t)splits * (size_t)M * (size_t)N * sizeof(float), s, &p);
        if (st != KSQ_OK) return st;
        partials = (float*)p;
    }
    // the planes are only read: the const view is the layout of planar_at
    const ksq::PlanarQ81 P = ksq::planar_at(const_cast<void*>(planar), M, K);
    hipError_t e = ksq::launch_mmq_planar(wtype, (const uint8_t*)weight, P, output, M, N, K, partials, s);
    return e == hipSuccess ? ok() : hip_error(e, "mmq launch");
}

size_t ksq_debug_stream_read_outputs(size_t bytes) { return ksq::stream_read_outputs(bytes, 32768); }

size_t ksq_debug_stream_read_wg_outputs(size_t bytes, size_t wg_bytes) {
    return (wg_bytes == 0 || wg_bytes % 4096) ? 0 : ksq::stream_read_outputs(bytes, wg_bytes);
}

int ksq_debug_stream_read_wg(const void* p, size_t bytes, size_t wg_bytes, uint32_t* out, void* stream) {
    if (wg_bytes == 0 || wg_bytes % 4096 || wg_bytes > ((size_t)1 << 30))
        return set_error(KSQ_ERR_SHAPE, "wg_bytes must be a positive multiple of 4096, at most 1 GiB");
    if (bytes == 0) return ok();
    if (!p || !out) return set_error(KSQ_ERR_NULL, "p or out is NULL");
    if (((uintptr_t)p & 15u) || (bytes & 15u) || ((uintptr_t)out & 3u))
        return set_error(KSQ_ERR_ALIGN, "p must be 16-byte aligned, bytes a multiple of 16, out 4-byte aligned");
    if (ksq::stream_read_outputs(bytes, wg_bytes) > 0x7FFFFFFFu)
        return set_error(KSQ_ERR_SHAPE, "too many workgroups for this wg_bytes");
    hipError_t e = ksq::launch_stream_read(p, bytes, wg_bytes, out, (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_error(e, "stream read launch");
}

int ksq_debug_stream_read(const void* p, size_t bytes, uint32_t* out, void* stream) {
    return ksq_debug_stream_read_wg(p, bytes, 32768, out, stream);
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
    if (!ksq::mmq_supported(wtype, M, N, K, weight, aligned16(act_q8_1)))
        return set_error(KSQ_ERR_SHAPE, "MFMA path needs K %% 256 == 0 and 16-byte aligned operands");
    hipError_t e = ksq::launch_mmq_block_sumi(wtype, (const uint8_t*)weight, act_q8_1, out, M, N, K, (hipStream_t)stream);
    return e == hipSuccess ? ok() : hip_error(e, "mfma block_sumi launch");
}

// ---- expert-grouped MoE --------------------------------------------------------
namespace {

#ifndef KSQ_MOE_SCRATCH_MIN_TOPK
#define KSQ_MOE_SCRATCH_MIN_TOPK 3
#endif
// Whether the grouped GEMM writes per-entry rows to scratch (combined afterwards in slot order)
// instead of adding into the output with atomics.
bool moe_uses_scratch(int top_k) { return top_k >= KSQ_MOE_SCRATCH_MIN_TOPK; }

struct MoeLayout {
    size_t aq, ids, wts, rows, inv, eend, ntiles, texp, trow0, scratch, total;
    int max_tiles;
};

// Rows per tile of the grouped GEMM's schedule: 128 for the LDS-DMA form, else mmq_kernel's.
static int moe_tile_rows(int wtype, int T, int N, int K, int E, int top_k) {
    (void)N;
    return ksq::mmq_moe_planar(wtype, T, E, top_k, K) ? 128 : ksq::mmq_moe_tile_rows(wtype, T, E, top_k);
}

// Planar rows of the LDS-DMA form's activations: one per entry, plus one tile's worth so that a
// tile starting at any entry reads its (d, nc) and -s rows inside the planes.
static int moe_planar_rows(int T, int top_k) { return T * top_k + 128; }

MoeLayout moe_layout(int wtype, int T, int N, int K, int E, int top_k) {
    MoeLayout L{};
    const size_t ent = (size_t)T * top_k;
    const int tile_rows = moe_tile_rows(wtype, T, N, K, E, top_k);
    L.max_tiles = (int)((ent + tile_rows - 1) / tile_rows) + E;
    size_t off = 0;
    L.aq = off;
    off = align256(off + (ksq::mmq_moe_planar(wtype, T, E, top_k, K) ? ksq::planar_bytes(moe_planar_rows(T, top_k), K)
                                                                     : (size_t)T * (K / 32) * 36));
    L.ids = off; off = align256(off + ent * 4);
    L.wts = off; off = align256(off + ent * 4);
    L.rows = off; off = align256(off + ent * 4);
    L.inv = off; off = align256(off + ent * 4);
    L.eend = off; off = align256(off + (size_t)E * 4);
    L.ntiles = off; off = align256(off + 4);
    L.texp = off; off = align256(off + (size_t)L.max_tiles * 4);
    L.trow0 = off; off = align256(off + (size_t)L.max_tiles * 4);
    L.scratch = off; off = align256(off + (moe_uses_scratch(top_k) ? ent * (size_t)N * 4 : 0));
    L.total = off;
    return L;
}

// Routing inside the grouping workgroup (one launch, 1024 threads routing T / 1024 tokens each)
// while T * E stays under this threshold; from it on routing takes its own launch over the chip
// (one thread per token) before the grouping workgroup.  Measured on MI355X, whole ksq_moe_gemm
// call at N = K = 256, top-2 (us, one launch vs two): E = 8: T = 512 22.4 vs 22.1, T = 1024
// 26.5 vs 24.5, T = 8192 98.5 vs 72.1, T = 16384 187.5 vs 130.8; E = 64: T = 512 44.4 vs 38.7,
// T = 4096 189.3 vs 92.2, T = 16384 695.2 vs 283.9.  The grouping workgroup's counting sort stays
// on one CU and is what grows with T past that.
#ifndef KSQ_MOE_ROUTE_SPLIT_TE
#define KSQ_MOE_ROUTE_SPLIT_TE 8192
#endif
static bool moe_route_in_group(int T, int E) { return (long long)T * E < (long long)KSQ_MOE_ROUTE_SPLIT_TE; }

int moe_run(int wtype, const void* weights, const float* activation, const float* logits, const int32_t* ids_in,
            const float* wts_in, float* output, int T, int N, int K, int E, int top_k, int renorm, int32_t* ids_out,
            float* wts_out, void* workspace, size_t ws_bytes, hipStream_t s) {
    g_engines = 0;
    if (wtype < KSQ_W_Q4_0 || wtype > KSQ_W_Q5_1 || wtype == KSQ_W_Q4_K || wtype == KSQ_W_Q6_K)
        return set_error(KSQ_ERR_TYPE, "MoE GEMM supports the 32-element block types (Q4_0, Q8_0, Q4_1, Q5_0, Q5_1)");
    if (T < 0 || N < 0 || K < 0 || E < 1 || E > 256 || top_k < 1 || top_k > E)
        return set_error(KSQ_ERR_SHAPE, "bad MoE shape T=%d N=%d K=%d E=%d top_k=%d", T, N, K, E, top_k);
    if (K % 256) return set_error(KSQ_ERR_SHAPE, "MoE GEMM needs K %% 256 == 0 (K=%d)", K);
    if (T == 0 || N == 0) return ok();
    if (!weights || !activation || !output || (!logits && (!ids_in || !wts_in)))
        return set_error(KSQ_ERR_NULL, "null MoE argument");
    if (((uintptr_t)weights & 15u) || ((uintptr_t)activation & 15u) || ((uintptr_t)output & 3u))
        return set_error(KSQ_ERR_ALIGN, "MoE weights/activation must be 16-byte aligned, output 4-byte");
    const MoeLayout L = moe_layout(wtype, T, N, K, E, top_k);
    const int tile_rows = moe_tile_rows(wtype, T, N, K, E, top_k);
    const bool planar = ksq::mmq_moe_planar(wtype, T, E, top_k, K);
    void* ws = workspace;
    if (ws) {
        if (ws_bytes < L.total) return set_error(KSQ_ERR_WORKSPACE, "workspace %zu < %zu bytes", ws_bytes, L.total);
        if ((uintptr_t)ws & 255u) return set_error(KSQ_ERR_ALIGN, "MoE workspace must be 256-byte aligned");
    } else {
        int st = pool_get(L.total, s, &ws);
        if (st != KSQ_OK) return st;
    }
    uint8_t* base = (uint8_t*)ws;
    uint8_t* aq = base + L.aq;
    int32_t* ids = ids_out ? ids_out : (int32_t*)(base + L.ids);
    float* wts = wts_out ? wts_out : (float*)(base + L.wts);
    // top_k <= 2 accumulates straight into the output, which the quantiser's launch zeroes
    // beside its own work when the output allows 16-byte stores; top_k > 2 writes per-entry
    // rows to scratch and combines them
    float* scratch = moe_uses_scratch(top_k) ? (float*)(base + L.scratch) : nullptr;
    const int64_t nout = (int64_t)T * N;
    const bool zero_fused = !scratch && ((uintptr_t)output & 15u) == 0 && (nout & 3) == 0;
    hipError_t e = hipSuccess;
    if (!planar) {
        // mmq_kernel's form: quantise the tokens first (rows are gathered inside the GEMM)
        e = zero_fused ? ksq::launch_quantize_q8_1_zero(activation, aq, T, K, output, nout, s)
                       : ksq::launch_quantize_q8_1(activation, aq, T, K, s);
        if (e != hipSuccess) return hip_error(e, "quantize launch");
    }
    if (!scratch && !zero_fused) {
        e = ksq::launch_fill_zero(output, nout, s);
        if (e != hipSuccess) return hip_error(e, "fill launch");
    }
    int32_t* rows = (int32_t*)(base + L.rows);
    int32_t* inv = planar ? (int32_t*)(base + L.inv) : nullptr;   // the scatter quantiser's map
    int32_t* eend = (int32_t*)(base + L.eend);
    int32_t* ntiles = (int32_t*)(base + L.ntiles);
    int32_t* texp = (int32_t*)(base + L.texp);
    int32_t* trow0 = (int32_t*)(base + L.trow0);
    // the LDS-DMA form clears the output in the routing launch when routing runs in one
    // workgroup (the rest of the chip is idle meanwhile), else in the quantiser's launch
    const bool zero_in_route = planar && zero_fused && logits && moe_route_in_group(T, E);
    if (logits && moe_route_in_group(T, E)) {
        e = ksq::launch_moe_route_group(logits, T, E, top_k, renorm, ids, wts, tile_rows, rows, inv, eend, ntiles,
                                        texp, trow0, zero_in_route ? output : nullptr, zero_in_route ? nout : 0, s);
        if (e != hipSuccess) return hip_error(e, "route launch");
        g_engines |= KSQ_ENG_MOE_ROUTE;
    } else if (logits) {
        // many tokens: one thread per token over the whole chip, then the grouping workgroup
        e = ksq::launch_moe_route(logits, T, E, top_k, renorm, ids, wts, s);
        if (e != hipSuccess) return hip_error(e, "route launch");
        e = ksq::launch_moe_group(ids, T, top_k, E, tile_rows, rows, inv, eend, ntiles, texp, trow0, s);
        if (e != hipSuccess) return hip_error(e, "group launch");
        g_engines |= KSQ_ENG_MOE_ROUTE;
    } else {
        ids = (int32_t*)ids_in;
        wts = (float*)wts_in;
        e = ksq::launch_moe_group(ids, T, top_k, E, tile_rows, rows, inv, eend, ntiles, texp, trow0, s);
        if (e != hipSuccess) return hip_error(e, "group launch");
    }
    g_engines |= KSQ_ENG_QUANTIZE | KSQ_ENG_MOE_GROUP;
    ksq::MoeTilesArgs a{ntiles, texp, trow0, eend, rows, wts, scratch, top_k};
    if (planar) {
        // the LDS-DMA form: each token quantised once into its entries' places in expert-sorted
        // order (the output zeroed in the routing launch or in this one), then 128-row tiles of each
        // expert
        const ksq::PlanarQ81 P = ksq::planar_at(aq, moe_planar_rows(T, top_k), K);
        const bool zero_here = zero_fused && !zero_in_route;
        e = ksq::launch_quantize_planar_scatter(activation, P, T, K, ksq::planar_da_scale(wtype), inv, top_k,
                                                zero_here ? output : nullptr, zero_here ? nout : 0, s);
        if (e != hipSuccess) return hip_error(e, "quantize launch");
        e = ksq::launch_mmq_planar_moe(wtype, (const uint8_t*)weights, P, output, N, K, L.max_tiles, a, s);
    } else {
        e = ksq::launch_mmq_moe(wtype, (const uint8_t*)weights, aq, output, N, K, L.max_tiles, tile_rows, a, s);
    }
    if (e != hipSuccess) return hip_error(e, "grouped gemm launch");
    if (scratch) {
        e = ksq::launch_moe_combine(scratch, ids, output, T, N, top_k, E, s);
        if (e != hipSuccess) return hip_error(e, "combine launch");
        g_engines |= KSQ_ENG_MOE_COMBINE;
    }
    return ok();
}
}  // namespace

size_t ksq_moe_workspace_size(int wtype, int T, int N, int K, int E, int top_k) {
    if (T <= 0 || N <= 0 || K <= 0 || E <= 0 || top_k <= 0) return 0;
    return moe_layout(wtype, T, N, K, E, top_k).total;
}

int ksq_moe_gemm(int wtype, const void* weights, const float* activation, const float* router_logits,
                 float* output, int T, int N, int K, int E, int top_k, int renorm, int32_t* topk_ids_out,
                 float* topk_weights_out, void* workspace, size_t workspace_bytes, void* stream) {
    if (!router_logits && T > 0 && N > 0) return set_error(KSQ_ERR_NULL, "router_logits is NULL");
    return moe_run(wtype, weights, activation, router_logits, nullptr, nullptr, output, T, N, K, E, top_k, renorm,
                   topk_ids_out, topk_weights_out, workspace, workspace_bytes, (hipStream_t)stream);
}

int ksq_moe_gemm_routed(int wtype, const void* weights, const float* activation, const int32_t* topk_ids,
                        const float* topk_weights, float* output, int T, int N, int K, int E, int top_k,
                        void* workspace, size_t workspace_bytes, void* stream) {
    return moe_run(wtype, weights, activation, nullptr, topk_ids, topk_weights, output, T, N, K, E, top_k, 0,
                   nullptr, nullptr, workspace, workspace_bytes, (hipStream_t)stream);
}

void moe_w4a32c8_q4_0_fp32_int8(const uint8_t* weight, const float* activation, const float* router_logits,
                                float* output, int T, int N, int K, int E, int top_k) {
    (void)ksq_moe_gemm(KSQ_W_Q4_0, weight, activation, router_logits, output, T, N, K, E, top_k, 0, nullptr,
                       nullptr, nullptr, 0, nullptr);
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
KSQ_DROPIN(gemm_w4a32c8_q4_1_fp32_int8, KSQ_W_Q4_1, KSQ_A_F32, float)
KSQ_DROPIN(gemm_w5a32c8_q5_0_fp32_int8, KSQ_W_Q5_0, KSQ_A_F32, float)
KSQ_DROPIN(gemm_w5a32c8_q5_1_fp32_int8, KSQ_W_Q5_1, KSQ_A_F32, float)
KSQ_DROPIN(ksq_gemm_q4_1_q8_1, KSQ_W_Q4_1, KSQ_A_Q8_1, uint8_t)
KSQ_DROPIN(ksq_gemm_q5_0_q8_1, KSQ_W_Q5_0, KSQ_A_Q8_1, uint8_t)
KSQ_DROPIN(ksq_gemm_q5_1_q8_1, KSQ_W_Q5_1, KSQ_A_Q8_1, uint8_t)
KSQ_DROPIN(gemm_w8a8c8_q8_0_q8_1, KSQ_W_Q8_0, KSQ_A_F32_Q8S, float)
KSQ_DROPIN(gemm_w4a32c8_q4_0_fp32_int8_deepseek_v2, KSQ_W_Q4_0, KSQ_A_F32_Q8F_RNE, float)

}  // extern "C"
