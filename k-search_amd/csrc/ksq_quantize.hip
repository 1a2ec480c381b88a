// ksq_quantize.hip - fp32 activations -> block_q8_1 (or block_q8s) on gfx950.
//
// Same arithmetic as quantize_row_q8_1_ref (kernelevalplus-main/include/quantize.h:165-193);
// the reference's own device kernel (quantize.h:302-337) rounds half-even with
// __float2int_rn, the CPU reference rounds half away from zero with roundf, and
// this kernel follows the CPU reference bit for bit.
//
// Layout of the work: one thread per 32-float block, 256 blocks (32 KiB of
// input) per workgroup.  Input is read with coalesced 16-byte loads into LDS
// (33-float row pitch, so the per-thread block reads below are conflict free),
// each thread quantises its block from LDS (the sum must be the sequential
// left-to-right fp32 sum, so one lane owns a whole block), and the 36-byte
// results go back out through LDS as coalesced dword stores.
#include "ksq_device.h"
#include "ksq_internal.h"

namespace ksq {

constexpr int kQBlocksPerWG = 256;
constexpr int kQPitch = 33;  // floats per staged block

// Q8S = false: block_q8_1 (quantize_row_q8_1_ref); true: block_q8s (the native W8A8C8
// operator's rules).  Both are 36-byte blocks of 9 dwords.
template <bool Q8S>
__global__ __launch_bounds__(256) void quantize_q8_1_kernel(const float* __restrict__ x,
                                                            uint8_t* __restrict__ y, int64_t nblocks) {
    __shared__ float stage[kQBlocksPerWG * kQPitch];
    const int t = threadIdx.x;
    const int64_t blk0 = (int64_t)blockIdx.x * kQBlocksPerWG;
    const int nblk = (int)((nblocks - blk0) < kQBlocksPerWG ? (nblocks - blk0) : kQBlocksPerWG);

    // 256 blocks x 8 float4 = 2048 float4; thread t moves float4 t + 256*j.
    const f32x4* src = (const f32x4*)(x + blk0 * 32);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int idx = t + 256 * j;
        if (idx < nblk * 8) {
            const f32x4 v = __builtin_nontemporal_load(src + idx);
            float* dst = stage + (idx >> 3) * kQPitch + (idx & 7) * 4;
            dst[0] = v.x;
            dst[1] = v.y;
            dst[2] = v.z;
            dst[3] = v.w;
        }
    }
    __syncthreads();

    uint32_t q[9];
    if (t < nblk) {
        float v[32];
#pragma unroll
        for (int j = 0; j < 32; j++) v[j] = stage[t * kQPitch + j];
        if constexpr (Q8S) quantize_block_q8s(v, q);
        else quantize_block_q8_1(v, q);
    }
    __syncthreads();
    uint32_t* ostage = (uint32_t*)stage;  // 256 x 9 dwords, odd pitch: conflict free
    if (t < nblk) {
#pragma unroll
        for (int j = 0; j < 9; j++) ostage[t * 9 + j] = q[j];
    }
    __syncthreads();
    uint32_t* dst = (uint32_t*)(y + blk0 * 36);
#pragma unroll
    for (int j = 0; j < 9; j++) {
        const int idx = t + 256 * j;
        if (idx < nblk * 9) dst[idx] = ostage[idx];
    }
}

hipError_t launch_quantize(int afmt, const float* x, uint8_t* y, int64_t rows, int K, hipStream_t s) {
    const int64_t nblocks = rows * (int64_t)(K / 32);
    if (nblocks == 0) return hipSuccess;
    const int64_t grid = (nblocks + kQBlocksPerWG - 1) / kQBlocksPerWG;
    if (afmt == kAQ8S)
        hipLaunchKernelGGL(quantize_q8_1_kernel<true>, dim3((unsigned)grid), dim3(256), 0, s, x, y, nblocks);
    else
        hipLaunchKernelGGL(quantize_q8_1_kernel<false>, dim3((unsigned)grid), dim3(256), 0, s, x, y, nblocks);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_1(const float* x, uint8_t* y, int64_t rows, int K, hipStream_t s) {
    return launch_quantize(kAQ81, x, y, rows, K, s);
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
