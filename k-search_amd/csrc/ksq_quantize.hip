// ksq_quantize.hip - fp32 activations -> block_q8_1 (or block_q8s, block_q8f) on gfx950.
//
// Same arithmetic as quantize_row_q8_1_ref (kernelevalplus-main/include/quantize.h:165-193);
// the reference's own device kernel (quantize.h:302-337) rounds half-even with
// __float2int_rn, the CPU reference rounds half away from zero with roundf, and
// this kernel follows the CPU reference bit for bit.
//
// Layout of the work: one lane per 32-float block; each wave owns 64 consecutive blocks
// (8 KiB of input) and works alone (no workgroup barrier, so the waves of a workgroup do
// not wait for each other's loads).  The wave reads its input with coalesced 16-byte
// loads into its own LDS region (33-float row pitch, so the per-lane block reads below
// are conflict free), each lane quantises its block from LDS (the sum must be the
// sequential left-to-right fp32 sum, so one lane owns a whole block), and the 36-byte
// results go back out through the same LDS region as coalesced dword stores.
#include "ksq_device.h"
#include "ksq_internal.h"

namespace ksq {

constexpr int kQWaves = 4;                       // waves per workgroup
constexpr int kQBlocksPerWG = 64 * kQWaves;
constexpr int kQPitch = 33;  // floats per staged block

// LDS written and read back by lanes of the same wave: wait for this wave's LDS
// operations, then keep the compiler from moving LDS accesses across the point.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    wave_lds_exchange();
}

// Output formats: kQF81 block_q8_1 (quantize_row_q8_1_ref), kQF8S block_q8s (the native W8A8C8
// operator's rules), both 36-byte blocks of 9 dwords; kQF8FRne / kQF8FLround block_q8f (fp32 d
// and s, 40-byte blocks of 10 dwords) by the two rules of quantize_block_q8f.
constexpr int kQF81 = 0, kQF8S = 1, kQF8FRne = 2, kQF8FLround = 3;
template <int FMT>
constexpr int out_words() { return FMT >= kQF8FRne ? 10 : 9; }

// The 64 blocks of wave w of workgroup `wg`.
template <int FMT>
__device__ __forceinline__ void quantize_wave(const float* __restrict__ x, uint8_t* __restrict__ y, int64_t nblocks,
                                              int64_t wg, float* stage_all) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    float* stage = stage_all + w * 64 * kQPitch;
    const int64_t blk0 = (wg * kQWaves + w) * 64;
    if (blk0 >= nblocks) return;
    const int nblk = (int)((nblocks - blk0) < 64 ? (nblocks - blk0) : 64);

    // 64 blocks x 8 float4 = 512 float4; lane l moves float4 l + 64*j.
    const f32x4* src = (const f32x4*)(x + blk0 * 32);
    f32x4 in[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int idx = lane + 64 * j;
        if (idx < nblk * 8) in[j] = __builtin_nontemporal_load(src + idx);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int idx = lane + 64 * j;
        if (idx < nblk * 8) {
            float* dst = stage + (idx >> 3) * kQPitch + (idx & 7) * 4;
            dst[0] = in[j].x;
            dst[1] = in[j].y;
            dst[2] = in[j].z;
            dst[3] = in[j].w;
        }
    }
    wave_lds_sync();

    constexpr int OW = out_words<FMT>();
    uint32_t q[OW];
    if (lane < nblk) {
        float v[32];
#pragma unroll
        for (int j = 0; j < 32; j++) v[j] = stage[lane * kQPitch + j];
        if constexpr (FMT == kQF8S) quantize_block_q8s(v, q);
        else if constexpr (FMT == kQF8FRne) quantize_block_q8f<kQ8FRne>(v, q);
        else if constexpr (FMT == kQF8FLround) quantize_block_q8f<kQ8FLround>(v, q);
        else quantize_block_q8_1(v, q);
    }
    wave_lds_sync();
    // 64 x OW dwords (9: odd pitch, conflict free; 10: two-way conflicts)
    uint32_t* ostage = (uint32_t*)stage;
    if (lane < nblk) {
#pragma unroll
        for (int j = 0; j < OW; j++) ostage[lane * OW + j] = q[j];
    }
    wave_lds_sync();
    uint32_t* dst = (uint32_t*)(y + blk0 * (4 * OW));
#pragma unroll
    for (int j = 0; j < OW; j++) {
        const int idx = lane + 64 * j;
        if (idx < nblk * OW) dst[idx] = ostage[idx];
    }
}

template <int FMT>
__global__ __launch_bounds__(64 * kQWaves) void quantize_q8_1_kernel(const float* __restrict__ x,
                                                                     uint8_t* __restrict__ y, int64_t nblocks) {
    __shared__ float stage_all[kQWaves * 64 * kQPitch];
    quantize_wave<FMT>(x, y, nblocks, blockIdx.x, stage_all);
}

// The quantiser's workgroups plus zero-filling ones: workgroups from qgrid on clear 32 KiB each
// of `zero` (n4 16-byte groups), so an output that is accumulated into later needs no launch
// of its own.
constexpr int kZeroBytesPerWG = 32768;

__global__ __launch_bounds__(64 * kQWaves) void quantize_zero_kernel(const float* __restrict__ x,
                                                                     uint8_t* __restrict__ y, int64_t nblocks,
                                                                     int64_t qgrid, float* __restrict__ zero,
                                                                     int64_t n4) {
    __shared__ float stage_all[kQWaves * 64 * kQPitch];
    if ((int64_t)blockIdx.x < qgrid) {
        quantize_wave<kQF81>(x, y, nblocks, blockIdx.x, stage_all);
        return;
    }
    const int64_t base = ((int64_t)blockIdx.x - qgrid) * (kZeroBytesPerWG / 16);
    f32x4* z = (f32x4*)zero;
#pragma unroll
    for (int i = 0; i < kZeroBytesPerWG / 16 / (64 * kQWaves); i++) {
        const int64_t k = base + i * (64 * kQWaves) + threadIdx.x;
        if (k < n4) z[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
}

hipError_t launch_quantize(int afmt, const float* x, uint8_t* y, int64_t rows, int K, hipStream_t s) {
    const int64_t nblocks = rows * (int64_t)(K / 32);
    if (nblocks == 0) return hipSuccess;
    const int64_t grid = (nblocks + kQBlocksPerWG - 1) / kQBlocksPerWG;
    if (afmt == kAQ8S)
        hipLaunchKernelGGL(quantize_q8_1_kernel<kQF8S>, dim3((unsigned)grid), dim3(64 * kQWaves), 0, s, x, y,
                           nblocks);
    else
        hipLaunchKernelGGL(quantize_q8_1_kernel<kQF81>, dim3((unsigned)grid), dim3(64 * kQWaves), 0, s, x, y,
                           nblocks);
    return hipGetLastError();
}

hipError_t launch_quantize_q8f(int rule, const float* x, uint8_t* y, int64_t rows, int K, hipStream_t s) {
    const int64_t nblocks = rows * (int64_t)(K / 32);
    if (nblocks == 0) return hipSuccess;
    const int64_t grid = (nblocks + kQBlocksPerWG - 1) / kQBlocksPerWG;
    if (rule == kQ8FRne)
        hipLaunchKernelGGL(quantize_q8_1_kernel<kQF8FRne>, dim3((unsigned)grid), dim3(64 * kQWaves), 0, s, x, y,
                           nblocks);
    else if (rule == kQ8FLround)
        hipLaunchKernelGGL(quantize_q8_1_kernel<kQF8FLround>, dim3((unsigned)grid), dim3(64 * kQWaves), 0, s, x, y,
                           nblocks);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_quantize_q8_1(const float* x, uint8_t* y, int64_t rows, int K, hipStream_t s) {
    return launch_quantize(kAQ81, x, y, rows, K, s);
}

hipError_t launch_quantize_q8_1_zero(const float* x, uint8_t* y, int64_t rows, int K, float* zero, int64_t nzero,
                                     hipStream_t s) {
    const int64_t nblocks = rows * (int64_t)(K / 32);
    const int64_t qgrid = (nblocks + kQBlocksPerWG - 1) / kQBlocksPerWG;
    const int64_t n4 = nzero / 4;
    const int64_t zgrid = (n4 * 16 + kZeroBytesPerWG - 1) / kZeroBytesPerWG;
    if (qgrid + zgrid == 0) return hipSuccess;
    hipLaunchKernelGGL(quantize_zero_kernel, dim3((unsigned)(qgrid + zgrid)), dim3(64 * kQWaves), 0, s, x, y, nblocks,
                       qgrid, zero, n4);
    return hipGetLastError();
}

// ---- planar block_q8_1 (the LDS-DMA GEMM's input) ---------------------------------------
// The same blocks as quantize_q8_1_kernel<kQF81> (same device quantiser, bit for bit), written
// as the planes of PlanarQ81.  A workgroup owns R rows x 4 blocks: it reads the R row
// segments of 512 bytes with coalesced 16-byte loads into LDS ([row][block] with a 33-float
// pitch, so the per-lane block reads are conflict free), and lane t quantises block t % 4 of row
// t / 4, so that the 4 lanes of a row write its 128 quant bytes, its (d, nc) pairs and its 4 sa
// halves side by side.  Rows M .. mp-1 quantise zeros: their dn and sa entries are written,
// their quants are not.
// SCATTER (the grouped MoE GEMM's input): the rows are the T tokens, read once each, and token m's
// blocks go to planar rows inv[m * top_k + s] for each of its top_k entries (inv: each (token,
// slot) entry's place in the expert-sorted order; -1 for an entry the grouping did not place), so
// that the planar rows come out in expert-sorted order without a second read of any token.  Planar
// rows that no entry maps to (the padding past the entries) are left as they are: the grouped GEMM
// reads them only for tile rows whose outputs it discards.  Workgroups from x = ceil(T / 64) on
// clear 32 KiB each of `zero` (n4 16-byte groups; chunk (x - ceil(T / 64)) * gridDim.y + y).
// R rows per workgroup (4 R threads, each loading 8 16-byte pieces): the dense form takes 16 rows
// (8 KiB per workgroup, the read curve's best shape at this size): 10.47 -> 10.00 us at config 2
// against 64 rows, three trace pairs.
template <bool SCATTER, int R = 64>
__global__ __launch_bounds__(4 * R) void quantize_planar_kernel(const float* __restrict__ x, PlanarQ81 y, int M, int K,
                                                              float da_scale, const int32_t* __restrict__ inv,
                                                              int top_k, float* __restrict__ zero, int64_t n4) {
    static_assert(!SCATTER || R == 64, "the scatter form's clearing workgroups are 256 threads");
    __shared__ float stage[R * 4 * kQPitch];
    const int t = threadIdx.x;
    if constexpr (SCATTER) {
        const int qx = (M + 63) / 64;
        if ((int)blockIdx.x >= qx) {
            const int64_t chunk = ((int64_t)blockIdx.x - qx) * gridDim.y + blockIdx.y;
            const int64_t base = chunk * (kZeroBytesPerWG / 16);
            if (base >= n4) return;
            f32x4* z = (f32x4*)zero;
#pragma unroll
            for (int i = 0; i < kZeroBytesPerWG / 16 / 256; i++) {
                const int64_t k = base + i * 256 + t;
                if (k < n4) z[k] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
            return;
        }
    }
    const int r0 = (int)blockIdx.x * R, kb0 = (int)blockIdx.y * 4;
#pragma unroll
    for (int p = 0; p < 8; p++) {
        const int idx = p * 4 * R + t, row = idx >> 5, c = idx & 31;   // c: float4 of the row segment
        f32x4 v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (r0 + row < M) v = __builtin_nontemporal_load((const f32x4*)(x + (size_t)(r0 + row) * K + kb0 * 32) + c);
        float* dst = stage + (row * 4 + (c >> 3)) * kQPitch + (c & 7) * 4;
        dst[0] = v.x;
        dst[1] = v.y;
        dst[2] = v.z;
        dst[3] = v.w;
    }
    __syncthreads();
    const int row = t >> 2, blk = t & 3, m = r0 + row, kb = kb0 + blk;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; j++) v[j] = stage[t * kQPitch + j];
    uint32_t q[9];
    quantize_block_q8_1(v, q);
    const float d = f16_to_f32(q[0] & 0xFFFFu) * da_scale;
    const uint16_t sa = (uint16_t)((q[0] >> 16) ^ 0x8000u);
    auto put = [&](int pm, bool quants) __attribute__((always_inline)) {
        if (quants) {
            u32x4* dq = (u32x4*)(y.q + (size_t)pm * K + (size_t)kb * 32);
            dq[0] = u32x4{q[1], q[2], q[3], q[4]};
            dq[1] = u32x4{q[5], q[6], q[7], q[8]};
        }
        *(f32x2*)(y.dn + 2 * ((size_t)kb * y.mp + pm)) = f32x2{d, -12582912.0f * d};
        y.sa[((size_t)(kb0 >> 2) * y.mp + pm) * 4 + blk] = sa;
    };
    if constexpr (SCATTER) {
        if (m < M)
            for (int s = 0; s < top_k; s++) {
                const int pm = inv[(size_t)m * top_k + s];
                if (pm >= 0) put(pm, true);
            }
    } else {
        put(m, m < M);
    }
}

size_t planar_bytes(int M, int K) {
    auto a256 = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t mp = (size_t)((M + 127) / 128) * 128, nb = (size_t)(K / 32);
    return a256((size_t)M * K) + a256(nb * mp * 8) + a256(nb / 4 * mp * 8);
}

PlanarQ81 planar_at(void* ws, int M, int K) {
    auto a256 = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t mp = (size_t)((M + 127) / 128) * 128, nb = (size_t)(K / 32);
    uint8_t* p = (uint8_t*)ws;
    PlanarQ81 y;
    y.q = (int8_t*)p;
    p += a256((size_t)M * K);
    y.dn = (float*)p;
    p += a256(nb * mp * 8);
    y.sa = (uint16_t*)p;
    y.mp = (int)mp;
    return y;
}

hipError_t launch_quantize_planar(const float* x, const PlanarQ81& y, int M, int K, float da_scale, hipStream_t s) {
    if (M <= 0 || K <= 0) return hipSuccess;
    if (K % 128) return hipErrorInvalidValue;
    constexpr int R = 16;
    const dim3 grid((unsigned)(y.mp / R), (unsigned)(K / 128));
    hipLaunchKernelGGL((quantize_planar_kernel<false, R>), grid, dim3(4 * R), 0, s, x, y, M, K, da_scale, nullptr, 1,
                       nullptr, (int64_t)0);
    return hipGetLastError();
}

hipError_t launch_quantize_planar_scatter(const float* x, const PlanarQ81& y, int T, int K, float da_scale,
                                          const int32_t* inv, int top_k, float* zero, int64_t nzero, hipStream_t s) {
    if (K <= 0 || K % 128) return hipErrorInvalidValue;
    if (T < 0 || top_k < 1 || y.mp < T * top_k) return hipErrorInvalidValue;
    const int64_t n4 = zero ? nzero / 4 : 0;
    const int64_t zchunks = (n4 * 16 + kZeroBytesPerWG - 1) / kZeroBytesPerWG;
    const int64_t zgrid = (zchunks + K / 128 - 1) / (K / 128);   // chunks spread over grid y too
    const int64_t qx = (T + 63) / 64;
    if (qx + zgrid == 0) return hipSuccess;
    const dim3 grid((unsigned)(qx + zgrid), (unsigned)(K / 128));
    hipLaunchKernelGGL(quantize_planar_kernel<true>, grid, dim3(256), 0, s, x, y, T, K, da_scale, inv, top_k, zero,
                       n4);
    return hipGetLastError();
}

// ---- the reference's other Q8_1 quantisers (ksq_quantize_q8_1_variant) -----------------
// One lane per 32-value block, as the reference's own device quantiser runs; block_q8_1 out.
//   1 quantize_q8_1_kernel (include/quantize.h:301-336): fmaxf/sequential-sum, id = 1/d,
//     round half to even (__float2int_rn: NaN -> 0), clamp [-128, 127]
//   2 quantize_to_q8_1 (llm_kernel_test/reference/quantize.py:165-214, NumPy): d = amax/127
//     or 1 when amax is 0, q = round_half_even(x / d) by true division, s = NumPy's pairwise
//     float32 sum (eight strided accumulators, tree-combined)
//   3 quantize_fp16_to_q8_1_smem (kernels/gemm/gemm_fused.cuh:76-145): fp16 input, max and
//     sum by the shared-memory tree (16, 8, 4, 2 apart, then 0 with 1), id = 1 / half(d),
//     q = roundf (half away from zero), saturated to int8, then clamp [-127, 127]

// (int) of an already-rounded float as the device converts it (NaN -> 0), clamped to int8.
__device__ __forceinline__ int sat_i8(float r) {
    return (r != r) ? 0 : (int)__builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);
}

template <int VAR>
__device__ __forceinline__ void quantize_block_variant(const float* v, uint32_t* out) {
#pragma clang fp contract(off)
    if constexpr (VAR == 3) {
        quantize_block_q8_1_f16tree(v, out);
        return;
    }
    float d, sum;
    if constexpr (VAR == 1) {
        float amax = 0.0f;
        sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 32; j++) {
            amax = __builtin_fmaxf(amax, __builtin_fabsf(v[j]));
            sum += v[j];
        }
        d = amax / 127.0f;
    } else {
        float amax = 0.0f;
        bool nan = false;
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const float a = __builtin_fabsf(v[j]);
            nan |= (a != a);
            amax = a > amax ? a : amax;
        }
        d = (!nan && amax > 0.0f) ? amax / 127.0f : 1.0f;
        float r[8];
#pragma unroll
        for (int j = 0; j < 8; j++) r[j] = v[j];
#pragma unroll
        for (int i = 8; i < 32; i += 8)
#pragma unroll
            for (int j = 0; j < 8; j++) r[j] += v[i + j];
        sum = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    }
    out[0] = f32_to_f16(d) | (f32_to_f16(sum) << 16);
    float id = 0.0f;
    if constexpr (VAR == 1) id = (d > 0.0f) ? 1.0f / d : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float x = v[4 * i + k];
            const int q = (VAR == 1) ? sat_i8(__builtin_rintf(x * id)) : sat_i8(__builtin_rintf(x / d));
            w |= (uint32_t)(q & 0xFF) << (8 * k);
        }
        out[1 + i] = w;
    }
}

template <int VAR>
__global__ __launch_bounds__(256) void quantize_q8_1_variant_kernel(const void* __restrict__ x, uint8_t* __restrict__ y,
                                                                    int64_t nblocks) {
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    float v[32];
    if constexpr (VAR == 3) {
        const u32x4* src = (const u32x4*)((const uint16_t*)x + b * 32);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const u32x4 w = src[i];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                v[8 * i + 2 * k] = f16_to_f32(ws[k] & 0xFFFFu);
                v[8 * i + 2 * k + 1] = f16_to_f32(ws[k] >> 16);
            }
        }
    } else {
        const f32x4* src = (const f32x4*)((const float*)x + b * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const f32x4 q = src[i];
            v[4 * i] = q.x; v[4 * i + 1] = q.y; v[4 * i + 2] = q.z; v[4 * i + 3] = q.w;
        }
    }
    uint32_t out[9];
    quantize_block_variant<VAR>(v, out);
    uint32_t* dst = (uint32_t*)(y + b * kQ81Bytes);
#pragma unroll
    for (int i = 0; i < 9; i++) dst[i] = out[i];
}

hipError_t launch_quantize_variant(int variant, const void* x, uint8_t* y, int64_t rows, int K, hipStream_t s) {
    if (variant == 0) return launch_quantize_q8_1((const float*)x, y, rows, K, s);
    const int64_t nblocks = rows * (int64_t)(K / 32);
    if (nblocks == 0) return hipSuccess;
    const dim3 grid((unsigned)((nblocks + 255) / 256)), blk(256);
    switch (variant) {
        case 1: hipLaunchKernelGGL(quantize_q8_1_variant_kernel<1>, grid, blk, 0, s, x, y, nblocks); break;
        case 2: hipLaunchKernelGGL(quantize_q8_1_variant_kernel<2>, grid, blk, 0, s, x, y, nblocks); break;
        case 3: hipLaunchKernelGGL(quantize_q8_1_variant_kernel<3>, grid, blk, 0, s, x, y, nblocks); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- device weight quantisers (fp32 -> block_q4_0 / block_q8_0), one lane per block --------
// RULE 0, the reference's device kernels quantize_q4_0_kernel / quantize_q8_0_kernel
// (include/quantize.h:221-297): amax by fmaxf, d = amax / 7 (Q4_0) or / 127 (Q8_0), stored as
// half(d); id = 1 / d (0 when d = 0); q = __float2int_rn(x * id) (half to even, NaN -> 0,
// saturating), then Q4_0 adds 8 (with 32-bit wrap, as the device's add does) and clamps to
// [0, 15], Q8_0 clamps to [-128, 127].  RULE 1, the CPU references quantize_row_q4_0_ref /
// quantize_row_q8_0_ref (include/quantize.h:34-68, 110-131): the same with (int)roundf(x * id)
// (half away from zero; a NaN or out-of-range value converts to INT32_MIN, as on x86).
// Q4_0 packs element j in the low nibble and element j + 16 in the high nibble of byte j.
__device__ __forceinline__ int32_t cvt_rn_sat(float r) {   // __float2int_rn of a rounded value
    if (r != r) return 0;
    if (r >= 2147483648.0f) return INT32_MAX;
    if (r < -2147483648.0f) return INT32_MIN;
    return (int32_t)r;
}
__device__ __forceinline__ int32_t cvt_x86(float r) {      // (int) of a rounded value on x86
    return (r >= -2147483648.0f && r < 2147483648.0f) ? (int32_t)r : INT32_MIN;
}

template <int WT, int RULE>
__global__ __launch_bounds__(256) void quantize_weights_kernel(const float* __restrict__ x, uint16_t* __restrict__ y,
                                                               int64_t nblocks) {
    static_assert(WT == kWQ40 || WT == kWQ80, "Q4_0 or Q8_0 blocks");
    const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblocks) return;
    float v[32];
    const f32x4* src = (const f32x4*)(x + b * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const f32x4 q = src[i];
        v[4 * i] = q.x; v[4 * i + 1] = q.y; v[4 * i + 2] = q.z; v[4 * i + 3] = q.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[j]));
    const float d = amax / (WT == kWQ40 ? 7.0f : 127.0f);
    const float id = (d > 0.0f) ? 1.0f / d : 0.0f;
    auto qv = [&](float f) -> int32_t {
        return RULE == 0 ? cvt_rn_sat(__builtin_rintf(f * id)) : cvt_x86(__builtin_roundf(f * id));
    };
    constexpr int NH = block_bytes(WT) / 2;   // 9 or 17 halves
    uint16_t* dst = y + b * NH;
    dst[0] = (uint16_t)f32_to_f16(d);
    if constexpr (WT == kWQ40) {
#pragma unroll
        for (int h = 0; h < 8; h++) {
            uint32_t pair = 0;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int j = 2 * h + e;
                int32_t q0 = qv(v[j]), q1 = qv(v[j + 16]);
                if (RULE == 0) {
                    q0 = (int32_t)((uint32_t)q0 + 8u);
                    q1 = (int32_t)((uint32_t)q1 + 8u);
                } else {
                    q0 = q0 == INT32_MIN ? q0 : q0 + 8;
                    q1 = q1 == INT32_MIN ? q1 : q1 + 8;
                }
                q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
                q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
                pair |= (uint32_t)((q1 << 4) | q0) << (8 * e);
            }
            dst[1 + h] = (uint16_t)pair;
        }
    } else {
#pragma unroll
        for (int h = 0; h < 16; h++) {
            uint32_t pair = 0;
#pragma unroll
            for (int e = 0; e < 2; e++) {
                int32_t q = qv(v[2 * h + e]);
                q = q < -128 ? -128 : (q > 127 ? 127 : q);
                pair |= (uint32_t)(q & 0xFF) << (8 * e);
            }
            dst[1 + h] = (uint16_t)pair;
        }
    }
}

hipError_t launch_quantize_weights(int wtype, int rule, const float* x, uint8_t* y, int64_t nblocks, hipStream_t s) {
    if (nblocks <= 0) return hipSuccess;
    const dim3 grid((unsigned)((nblocks + 255) / 256)), blk(256);
    uint16_t* out = (uint16_t*)y;
    if (wtype == kWQ40 && rule == 0)
        hipLaunchKernelGGL((quantize_weights_kernel<kWQ40, 0>), grid, blk, 0, s, x, out, nblocks);
    else if (wtype == kWQ40 && rule == 1)
        hipLaunchKernelGGL((quantize_weights_kernel<kWQ40, 1>), grid, blk, 0, s, x, out, nblocks);
    else if (wtype == kWQ80 && rule == 0)
        hipLaunchKernelGGL((quantize_weights_kernel<kWQ80, 0>), grid, blk, 0, s, x, out, nblocks);
    else if (wtype == kWQ80 && rule == 1)
        hipLaunchKernelGGL((quantize_weights_kernel<kWQ80, 1>), grid, blk, 0, s, x, out, nblocks);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// out[c][r] = in[r][c] for in [rows][cols]: 32 x 32 tiles through LDS (33-float pitch, so
// the column reads are conflict free), 256 threads = 32 columns x 8 row groups.
__global__ __launch_bounds__(256) void transpose_f32_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                            int rows, int cols) {
    __shared__ float tile[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
    for (int i = 0; i < 32; i += 8) {
        const int r = r0 + ty + i, c = c0 + tx;
        if (r < rows && c < cols) tile[ty + i][tx] = in[(size_t)r * cols + c];
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 32; i += 8) {
        const int c = c0 + ty + i, r = r0 + tx;
        if (r < rows && c < cols) out[(size_t)c * rows + r] = tile[tx][ty + i];
    }
}

hipError_t launch_transpose_f32(const float* in, float* out, int rows, int cols, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const dim3 grid((unsigned)((cols + 31) / 32), (unsigned)((rows + 31) / 32));
    hipLaunchKernelGGL(transpose_f32_kernel, grid, dim3(256), 0, s, in, out, rows, cols);
    return hipGetLastError();
}

__global__ void fill_zero_kernel(float* __restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t k = i; k < n; k += stride) p[k] = 0.0f;
}

hipError_t launch_fill_zero(float* p, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    int64_t grid = (n + 255) / 256;
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)grid), dim3(256), 0, s, p, n);
    return hipGetLastError();
}

}  // namespace ksq
