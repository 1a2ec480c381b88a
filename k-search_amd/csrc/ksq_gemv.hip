// ksq_gemv.hip - decode GEMV on v_dot4c_i32_i8 (the mul_mat_vec_q analogue).
//
// Reference path: the GEMV family in kernelevalplus-main/kernels/gemm/gemm_warp_optimized.cuh:108-1212
// (one warp per weight row, lanes striding K-blocks, DP4A, shuffle reduce) and the
// CPU dot vec_dot_q4_0_q8_1 / vec_dot_q8_0_q8_1 (include/gemm_reference.h:276-336).
//
// gfx950 design:
//  * A row group of L lanes (L = 16/32/64 by K) owns one weight row; each lane owns
//    "chunks" of 8 consecutive blocks.  Eight Q4_0 blocks are 144 B = 9 x 16 B and
//    eight Q8_0 blocks 272 B = 17 x 16 B, so a lane streams its chunk with 16-byte
//    global_load_dwordx4 and pulls the 18/34-byte blocks out of registers with
//    v_alignbyte_b32 (blocks are only 2-byte aligned in memory).
//  * Nibbles are unpacked in registers (q & 0x0F0F0F0F, (q >> 4) & 0x0F0F0F0F) and
//    fed to v_dot4c_i32_i8 against the Q8_1 quants; the per-block fp32 epilogue is
//    the reference formula.
//  * The weight chunk stays in registers while the lane walks the MR activation
//    rows, so weights cross HBM once per launch for M <= 8.
//  * Lane partial sums are combined with xor shuffles inside the row group.
//  * K-quant rows: one 256-element super-block per lane (Q4_K 144 B, Q6_K 210 B).
#include "ksq_device.h"
#include "ksq_internal.h"

namespace ksq {

constexpr int kWaves = 4;  // 256-thread workgroups

template <int L>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = L / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// 16-byte load from a 4-byte aligned address.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ void load_u32x4(uint32_t* dst, const uint8_t* p) {
    const u32x4_a4 v = __builtin_nontemporal_load((const u32x4_a4*)p);
    dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
}

__device__ __forceinline__ void load_u32x4_a4(uint32_t* dst, const uint8_t* p) {
    const u32x4_a4 v = *(const u32x4_a4*)p;
    dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
}

// ---------------------------------------------------------------------------
// Q4_0 / Q8_0, aligned fast path: weight base 16-byte aligned, K % 256 == 0.
// ---------------------------------------------------------------------------
template <int WT, int MR, int L>
__global__ __launch_bounds__(256) void gemv_q_chunk_kernel(const uint8_t* __restrict__ W,
                                                           const uint8_t* __restrict__ A,
                                                           float* __restrict__ C, int N, int nb,
                                                           int ldc) {
    constexpr int BB = (WT == 0) ? kQ40Bytes : kQ80Bytes;  // block bytes
    constexpr int CB = 8 * BB;                             // chunk bytes: 144 or 272
    constexpr int CW = CB / 16;                            // 16-byte loads per chunk: 9 or 17
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row = (blockIdx.x * kWaves + wave) * (64 / L) + lane / L;
    const int sub = lane % L;
    const int nchunks = nb >> 3;

    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) acc[m] = 0.0f;

    if (row < N) {
        const uint8_t* wrow = W + (size_t)row * nb * BB;
        for (int c = sub; c < nchunks; c += L) {
            uint32_t w[CW * 4];
#pragma unroll
            for (int i = 0; i < CW; i++) load_u32x4(w + 4 * i, wrow + (size_t)c * CB + 16 * i);
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const uint8_t* arow = A + ((size_t)m * nb + (size_t)c * 8) * kQ81Bytes;
                uint32_t a[72];
#pragma unroll
                for (int i = 0; i < 18; i++) load_u32x4_a4(a + 4 * i, arow + 16 * i);
                float s = 0.0f;
#pragma unroll
                for (int b = 0; b < 8; b++) {
                    if constexpr (WT == 0)
                        s += block_q4_0(w, b * BB, a + 9 * b);
                    else
                        s += block_q8_0(w, b * BB, a + 9 * b);
                }
                acc[m] += s;
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; m++) acc[m] = group_sum<L>(acc[m]);
    if (row < N && sub == 0) {
#pragma unroll
        for (int m = 0; m < MR; m++) C[(size_t)m * ldc + row] = acc[m];
    }
}

// ---------------------------------------------------------------------------
// Q4_0 / Q8_0 generic path: any 2-byte aligned weight base, K % 32 == 0.  One
// block per lane step, weight bytes gathered with 16-bit loads.
// ---------------------------------------------------------------------------
template <int WT, int MR, int L>
__global__ __launch_bounds__(256) void gemv_q_block_kernel(const uint8_t* __restrict__ W,
                                                           const uint8_t* __restrict__ A,
                                                           float* __restrict__ C, int N, int nb,
                                                           int ldc) {
    constexpr int BB = (WT == 0) ? kQ40Bytes : kQ80Bytes;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row = (blockIdx.x * kWaves + wave) * (64 / L) + lane / L;
    const int sub = lane % L;
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) acc[m] = 0.0f;
    if (row < N) {
        const uint8_t* wrow = W + (size_t)row * nb * BB;
        for (int b = sub; b < nb; b += L) {
            uint32_t w[BB / 2 + 1];
            const uint16_t* p = (const uint16_t*)(wrow + (size_t)b * BB);
#pragma unroll
            for (int i = 0; i < BB / 4; i++) w[i] = (uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 16);
            w[BB / 4] = (uint32_t)p[(BB - 2) / 2];  // last half-word (BB % 4 == 2)
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const uint32_t* ap = (const uint32_t*)(A + ((size_t)m * nb + b) * kQ81Bytes);
                uint32_t a[9];
#pragma unroll
                for (int i = 0; i < 9; i++) a[i] = ap[i];
                if constexpr (WT == 0)
                    acc[m] += block_q4_0(w, 0, a);
                else
                    acc[m] += block_q8_0(w, 0, a);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; m++) acc[m] = group_sum<L>(acc[m]);
    if (row < N && sub == 0) {
#pragma unroll
        for (int m = 0; m < MR; m++) C[(size_t)m * ldc + row] = acc[m];
    }
}

// ---------------------------------------------------------------------------
// K-quants: one 256-element super-block per lane step.
// ---------------------------------------------------------------------------

// 6-bit scale and min j of a Q4_K super-block; s0..s2 are the 12 scale bytes.
__device__ __forceinline__ void q4_K_scale_min(int j, uint32_t s0, uint32_t s1, uint32_t s2, int& sc,
                                               int& m) {
    const uint32_t q[3] = {s0, s1, s2};
    auto byte = [&](int k) -> int { return (int)((q[k >> 2] >> (8 * (k & 3))) & 0xFFu); };
    if (j < 4) {
        sc = byte(j) & 63;
        m = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 0x0F) | ((byte(j - 4) >> 6) << 4);
        m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// Q4_K super-block (registers w[0..35]) against 8 Q8_1 blocks a[0..71]
// (vec_dot_q4_K_q8_1_impl_mmq form: d * sum_j d8_j*sc_j*sumi_j - dmin * sum_j s8_j*m_j).
__device__ __forceinline__ float sb_q4_K(const uint32_t* w, const uint32_t* a) {
    float sumf_d = 0.0f, sumf_m = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int g = j >> 1;
        int sumi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t q = w[4 + 8 * g + i];
            const uint32_t v = (j & 1) ? ((q >> 4) & 0x0F0F0F0Fu) : (q & 0x0F0F0F0Fu);
            sumi = dot4((int)v, (int)a[9 * j + 1 + i], sumi);
        }
        int sc, m;
        q4_K_scale_min(j, w[1], w[2], w[3], sc, m);
        sumf_d += f16_to_f32(a[9 * j] & 0xFFFFu) * (float)(sc * sumi);
        sumf_m += f16_to_f32(a[9 * j] >> 16) * (float)m;
    }
    return f16_to_f32(w[0] & 0xFFFFu) * sumf_d - f16_to_f32(w[0] >> 16) * sumf_m;
}

// Q6_K super-block held as 53 dwords starting `sh` bytes (0 or 2) into w.
__device__ __forceinline__ float sb_q6_K(const uint32_t* w, int sh, const uint32_t* a) {
    auto W32 = [&](int off) -> uint32_t { return __builtin_amdgcn_alignbyte(w[(off >> 2) + 1], w[off >> 2], sh); };
    const uint32_t scw0 = W32(192), scw1 = W32(196), scw2 = W32(200), scw3 = W32(204);
    const uint32_t scw[4] = {scw0, scw1, scw2, scw3};
    const float d = f16_to_f32(W32(208) & 0xFFFFu);
    float sumf = 0.0f;
#pragma unroll
    for (int n = 0; n < 2; n++) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int j = 4 * n + g;
            int s0 = 0, s1 = 0, z0 = 0, z1 = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint32_t qa = W32(64 * n + 4 * i);
                const uint32_t qb = W32(64 * n + 32 + 4 * i);
                const uint32_t h = W32(128 + 32 * n + 4 * i);
                uint32_t v;
                if (g == 0) v = (qa & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
                else if (g == 1) v = (qb & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
                else if (g == 2) v = ((qa >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
                else v = ((qb >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
                const int av = (int)a[9 * j + 1 + i];
                if (i < 4) { s0 = dot4((int)v, av, s0); z0 = dot4(0x01010101, av, z0); }
                else       { s1 = dot4((int)v, av, s1); z1 = dot4(0x01010101, av, z1); }
            }
            const int is0 = s0 - 32 * z0, is1 = s1 - 32 * z1;  // quants offset by -32
            const int sc0 = (int)(int8_t)((scw[j >> 1] >> (16 * (j & 1))) & 0xFFu);
            const int sc1 = (int)(int8_t)((scw[j >> 1] >> (16 * (j & 1) + 8)) & 0xFFu);
            sumf += f16_to_f32(a[9 * j] & 0xFFFFu) * (float)(sc0 * is0 + sc1 * is1);
        }
    }
    return d * sumf;
}

template <int WT, int MR, int L>
__global__ __launch_bounds__(256) void gemv_kquant_kernel(const uint8_t* __restrict__ W,
                                                          const uint8_t* __restrict__ A,
                                                          float* __restrict__ C, int N, int nb,
                                                          int ldc) {
    constexpr int SB = (WT == 2) ? kQ4KBytes : kQ6KBytes;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row = (blockIdx.x * kWaves + wave) * (64 / L) + lane / L;
    const int sub = lane % L;
    const int nsb = nb >> 3;
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) acc[m] = 0.0f;
    if (row < N) {
        const uint8_t* wrow = W + (size_t)row * nsb * SB;
        for (int s = sub; s < nsb; s += L) {
            const size_t byte = (size_t)s * SB;
            uint32_t w[56];
            int sh = 0;
            if constexpr (WT == 2) {
#pragma unroll
                for (int i = 0; i < 9; i++) load_u32x4(w + 4 * i, wrow + byte + 16 * i);
            } else {
                // 210-byte super-blocks: start at the 4-byte boundary below and realign by sh bytes.
                const uint8_t* blk = wrow + byte;
                sh = (int)((uintptr_t)blk & 3u);
                const uint8_t* base = blk - sh;
#pragma unroll
                for (int i = 0; i < 13; i++) load_u32x4_a4(w + 4 * i, base + 16 * i);
                // the last 2 bytes past a 4-byte aligned super-block belong to the next one
                // (or lie past the buffer), so only the half-word is read then
                w[52] = sh ? *(const uint32_t*)(base + 208) : (uint32_t)*(const uint16_t*)(base + 208);
                w[53] = 0;
            }
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const uint8_t* arow = A + ((size_t)m * nb + (size_t)s * 8) * kQ81Bytes;
                uint32_t a[72];
#pragma unroll
                for (int i = 0; i < 18; i++) load_u32x4_a4(a + 4 * i, arow + 16 * i);
                if constexpr (WT == 2)
                    acc[m] += sb_q4_K(w, a);
                else
                    acc[m] += sb_q6_K(w, sh, a);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; m++) acc[m] = group_sum<L>(acc[m]);
    if (row < N && sub == 0) {
#pragma unroll
        for (int m = 0; m < MR; m++) C[(size_t)m * ldc + row] = acc[m];
    }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------

#define KSQ_GEMV_CASE(KERN, WT, MR, L)                                                            \
    hipLaunchKernelGGL((KERN<WT, MR, L>), dim3(grid), dim3(256), 0, s, W, A + (size_t)m0 * nb * 36, \
                       C + (size_t)m0 * N, N, nb, N)

template <int WT, int L>
static void gemv_launch_rows(int kind, int mr, const uint8_t* W, const uint8_t* A, float* C, int m0,
                             int N, int nb, unsigned grid, hipStream_t s) {
    // kind 0: chunked Q4_0/Q8_0, 1: per-block Q4_0/Q8_0, 2: K-quant
#define KSQ_MR_SWITCH(KERN)                                  \
    switch (mr) {                                            \
        case 1: KSQ_GEMV_CASE(KERN, WT, 1, L); break;        \
        case 2: KSQ_GEMV_CASE(KERN, WT, 2, L); break;        \
        case 3: KSQ_GEMV_CASE(KERN, WT, 3, L); break;        \
        case 4: KSQ_GEMV_CASE(KERN, WT, 4, L); break;        \
        case 5: KSQ_GEMV_CASE(KERN, WT, 5, L); break;        \
        case 6: KSQ_GEMV_CASE(KERN, WT, 6, L); break;        \
        case 7: KSQ_GEMV_CASE(KERN, WT, 7, L); break;        \
        default: KSQ_GEMV_CASE(KERN, WT, 8, L); break;       \
    }
    if constexpr (WT <= 1) {
        if (kind == 0) { KSQ_MR_SWITCH(gemv_q_chunk_kernel) }
        else { KSQ_MR_SWITCH(gemv_q_block_kernel) }
    } else {
        KSQ_MR_SWITCH(gemv_kquant_kernel)
    }
#undef KSQ_MR_SWITCH
}

template <int WT>
static void gemv_launch_L(int L, int kind, int mr, const uint8_t* W, const uint8_t* A, float* C, int m0,
                          int N, int nb, hipStream_t s) {
    const int rows_per_wg = kWaves * (64 / L);
    const unsigned grid = (unsigned)((N + rows_per_wg - 1) / rows_per_wg);
    switch (L) {
        case 8: gemv_launch_rows<WT, 8>(kind, mr, W, A, C, m0, N, nb, grid, s); break;
        case 16: gemv_launch_rows<WT, 16>(kind, mr, W, A, C, m0, N, nb, grid, s); break;
        case 32: gemv_launch_rows<WT, 32>(kind, mr, W, A, C, m0, N, nb, grid, s); break;
        default: gemv_launch_rows<WT, 64>(kind, mr, W, A, C, m0, N, nb, grid, s); break;
    }
}

// Lanes per row: enough lanes that each has ~1 work item, at least 8, at most 64.
static int pick_lanes(int items) {
    int L = 8;
    while (L < 64 && L < items) L <<= 1;
    return L;
}

hipError_t launch_gemv(int wtype, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int K,
                       hipStream_t s) {
    const int nb = K / 32;
    if (M <= 0 || N <= 0 || nb == 0) return hipSuccess;
    int kind, items;
    if (wtype <= 1) {
        const bool chunked = (K % 256 == 0) && (((uintptr_t)W & 15u) == 0) && (((uintptr_t)A & 15u) == 0);
        kind = chunked ? 0 : 1;
        items = chunked ? nb / 8 : nb;
    } else {
        kind = 2;
        items = nb / 8;
    }
    const int L = pick_lanes(items);
    for (int m0 = 0; m0 < M; m0 += 8) {
        const int mr = (M - m0) < 8 ? (M - m0) : 8;
        switch (wtype) {
            case 0: gemv_launch_L<0>(L, kind, mr, W, A, C, m0, N, nb, s); break;
            case 1: gemv_launch_L<1>(L, kind, mr, W, A, C, m0, N, nb, s); break;
            case 2: gemv_launch_L<2>(L, kind, mr, W, A, C, m0, N, nb, s); break;
            default: gemv_launch_L<3>(L, kind, mr, W, A, C, m0, N, nb, s); break;
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// ---------------------------------------------------------------------------
// Debug: per-block integer dots from the same device block-dot helpers.
// ---------------------------------------------------------------------------
__global__ void block_sumi_kernel(int wtype, const uint8_t* __restrict__ W, const uint8_t* __restrict__ A,
                                  int32_t* __restrict__ out, int M, int N, int K) {
    const int nb = K / 32;
    const int nblk = (wtype == 3) ? K / 16 : nb;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t total = (int64_t)M * N * nblk;
    if (idx >= total) return;
    const int b = (int)(idx % nblk);
    const int64_t mn = idx / nblk;
    const int n = (int)(mn % N), m = (int)(mn / N);
    int r = 0;
    if (wtype <= 1) {
        const int BB = wtype == 0 ? kQ40Bytes : kQ80Bytes;
        const uint16_t* p = (const uint16_t*)(W + ((size_t)n * nb + b) * BB);
        uint32_t w[18];
        for (int i = 0; i < BB / 4; i++) w[i] = (uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 16);
        w[BB / 4] = (uint32_t)p[(BB - 2) / 2];
        const uint32_t* ap = (const uint32_t*)(A + ((size_t)m * nb + b) * kQ81Bytes);
        uint32_t a[9];
        for (int i = 0; i < 9; i++) a[i] = ap[i];
        r = (wtype == 0) ? sumi_q4_0(w, 0, a) : sumi_q8_0(w, 0, a);
    } else if (wtype == 2) {
        const int nsb = K / 256;
        const uint32_t* wp = (const uint32_t*)(W + ((size_t)n * nsb + b / 8) * kQ4KBytes);
        const uint32_t* ap = (const uint32_t*)(A + ((size_t)m * nb + b) * kQ81Bytes);
        const int j = b % 8, g = j >> 1;
        for (int i = 0; i < 8; i++) {
            const uint32_t q = wp[4 + 8 * g + i];
            const uint32_t v = (j & 1) ? ((q >> 4) & 0x0F0F0F0Fu) : (q & 0x0F0F0F0Fu);
            r = dot4((int)v, (int)ap[1 + i], r);
        }
    } else {
        const int nsb = K / 256;
        const uint8_t* wp = W + ((size_t)n * nsb + b / 16) * kQ6KBytes;
        const int u = b % 16;                  // sub-block in the super-block
        const int j = u >> 1, nh = j >> 2, g = j & 3;
        const uint32_t* ap = (const uint32_t*)(A + ((size_t)m * nb + b / 2) * kQ81Bytes);
        for (int i = 4 * (u & 1); i < 4 * (u & 1) + 4; i++) {
            uint32_t qa = 0, qb = 0, h = 0;
            for (int t = 0; t < 4; t++) {
                qa |= (uint32_t)wp[64 * nh + 4 * i + t] << (8 * t);
                qb |= (uint32_t)wp[64 * nh + 32 + 4 * i + t] << (8 * t);
                h |= (uint32_t)wp[128 + 32 * nh + 4 * i + t] << (8 * t);
            }
            uint32_t v;
            if (g == 0) v = (qa & 0x0F0F0F0Fu) | ((h << 4) & 0x30303030u);
            else if (g == 1) v = (qb & 0x0F0F0F0Fu) | ((h << 2) & 0x30303030u);
            else if (g == 2) v = ((qa >> 4) & 0x0F0F0F0Fu) | (h & 0x30303030u);
            else v = ((qb >> 4) & 0x0F0F0F0Fu) | ((h >> 2) & 0x30303030u);
            r = dot4((int)v, (int)ap[1 + i], r);
            r -= 32 * dot4(0x01010101, (int)ap[1 + i], 0);
        }
    }
    out[idx] = r;
}

hipError_t launch_block_sumi(int wtype, const uint8_t* W, const uint8_t* A, int32_t* out, int M, int N,
                             int K, hipStream_t s) {
    const int nblk = (wtype == 3) ? K / 16 : K / 32;
    const int64_t total = (int64_t)M * N * nblk;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(block_sumi_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, wtype, W, A,
                       out, M, N, K);
    return hipGetLastError();
}

}  // namespace ksq
