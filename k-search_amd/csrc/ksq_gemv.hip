// ksq_gemv.hip - decode GEMV on v_dot4c_i32_i8 (the mul_mat_vec_q analogue).
//
// Reference path: the GEMV family in kernelevalplus-main/kernels/gemm/gemm_warp_optimized.cuh:108-1212
// (one warp per weight row, lanes striding K-blocks, DP4A, shuffle reduce) and the
// CPU dots vec_dot_q4_0_q8_1 / vec_dot_q8_0_q8_1 (include/gemm_reference.h:276-336).
//
// gfx950 design (one weight row per wave):
//  * A 256-thread workgroup owns 4 consecutive weight rows, one per wave.  Each wave
//    copies its row (a contiguous byte range) into LDS with global_load_lds_dwordx4
//    (1 KiB per wave instruction, no VGPRs), and the workgroup stages the Q8_1
//    activation rows in LDS once for all four waves.  One-shot reads of a few MB
//    are fastest as many small, fully coalesced requests spread over the whole
//    chip, which is what this layout issues.
//  * Lanes then stride over 32-element units of the row (a Q4_0/Q8_0/Q4_1/Q5_0/Q5_1
//    block, or one Q8_1-block-sized slice of a Q4_K/Q6_K super-block), pull the unit's
//    bytes out of LDS with dword reads re-aligned by v_alignbyte_b32 (blocks are
//    18/34/20/22/24/144/210 B, only 2-byte aligned), unpack nibbles (and Q5 high bits)
//    in registers and run v_dot4c_i32_i8 against the activation quants; the per-unit
//    fp32 epilogue is the reference formula.
//  * The 64 lane partials are combined with xor shuffles; lane 0 stores.
//  * Rows longer than the LDS tile are walked in K tiles.
#include "ksq_device.h"
#include "ksq_internal.h"

namespace ksq {

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// NW little-endian words starting at byte pointer p (2-byte aligned, LDS or global):
// NW+1 aligned dword reads re-aligned with v_alignbyte_b32.
template <int NW>
__device__ __forceinline__ void read_words(const uint8_t* p, uint32_t* w) {
    const int sh = (int)((uintptr_t)p & 3u);
    const uint32_t* q = (const uint32_t*)(p - sh);
    uint32_t raw[NW + 1];
#pragma unroll
    for (int i = 0; i <= NW; i++) raw[i] = q[i];
#pragma unroll
    for (int i = 0; i < NW; i++) w[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], sh);
}

__device__ __forceinline__ uint32_t read_u16(const uint8_t* p) { return *(const uint16_t*)p; }

// ---- integer parts of the unit dots (shared with the debug entry) -------------
// a[0] = Q8_1 ds word, a[1..8] = the 32 activation quants.

// Q4_0 block (gemm_reference.h:200-212): sum qa[k]*(qs[k]&15) + qa[k+16]*(qs[k]>>4)
__device__ __forceinline__ int unit_sumi_q4_0(const uint8_t* blk, const uint32_t* a) {
    uint32_t q[4];
    read_words<4>(blk + 2, q);
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        s = dot4((int)(q[i] & 0x0F0F0F0Fu), (int)a[1 + i], s);
        s = dot4((int)((q[i] >> 4) & 0x0F0F0F0Fu), (int)a[5 + i], s);
    }
    return s;
}

// Q8_0 block (gemm_reference.h:253-256)
__device__ __forceinline__ int unit_sumi_q8_0(const uint8_t* blk, const uint32_t* a) {
    uint32_t q[8];
    read_words<8>(blk + 2, q);
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) s = dot4((int)q[i], (int)a[1 + i], s);
    return s;
}

// Q4_1 block (gemm_quant_formats.cuh:126-137): the same nibble dot as Q4_0, quants at offset 4.
__device__ __forceinline__ int unit_sumi_q4_1(const uint8_t* blk, const uint32_t* a) {
    uint32_t q[4];
    read_words<4>(blk + 4, q);
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        s = dot4((int)(q[i] & 0x0F0F0F0Fu), (int)a[1 + i], s);
        s = dot4((int)((q[i] >> 4) & 0x0F0F0F0Fu), (int)a[5 + i], s);
    }
    return s;
}

// Q5_0 / Q5_1 block (gemm_quant_formats.cuh:170-200, 230-257): low 4 bits from the nibbles
// at qs_off, bit 4 of element e from bit e of the qh word at qh_off; quants 0..31.
template <int QH_OFF, int QS_OFF>
__device__ __forceinline__ int unit_sumi_q5(const uint8_t* blk, const uint32_t* a) {
    uint32_t q[4], h[1];
    read_words<4>(blk + QS_OFF, q);
    read_words<1>(blk + QH_OFF, h);
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t lo = (q[i] & 0x0F0F0F0Fu) | qh_to_bit4(h[0] >> (4 * i));
        const uint32_t hi = ((q[i] >> 4) & 0x0F0F0F0Fu) | qh_to_bit4(h[0] >> (16 + 4 * i));
        s = dot4((int)lo, (int)a[1 + i], s);
        s = dot4((int)hi, (int)a[5 + i], s);
    }
    return s;
}

// Integer block dot of any 32-element block type against the 9-dword activation block a.
template <int WT>
__device__ __forceinline__ int unit_sumi_legacy(const uint8_t* blk, const uint32_t* a) {
    if constexpr (WT == kWQ40) return unit_sumi_q4_0(blk, a);
    else if constexpr (WT == kWQ80) return unit_sumi_q8_0(blk, a);
    else if constexpr (WT == kWQ41) return unit_sumi_q4_1(blk, a);
    else if constexpr (WT == kWQ50) return unit_sumi_q5<2, 6>(blk, a);
    else return unit_sumi_q5<4, 8>(blk, a);
}

// Q4_K sub-block j (32 elements) of super-block sb: 64-element group g = j/2 holds its
// quants in qs[32g .. 32g+31], low nibbles for even j, high nibbles for odd j.
__device__ __forceinline__ int unit_sumi_q4_K(const uint8_t* sb, int j, const uint32_t* a) {
    uint32_t q[8];
    read_words<8>(sb + 16 + 32 * (j >> 1), q);
    const int sft = 4 * (j & 1);
    int s = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) s = dot4((int)((q[i] >> sft) & 0x0F0F0F0Fu), (int)a[1 + i], s);
    return s;
}

// 6-bit scale and min j of a Q4_K super-block (get_scale_min_k4); sc3 = the 12 scale bytes.
__device__ __forceinline__ void q4_K_scale_min(int j, const uint32_t* sc3, int& sc, int& m) {
    auto byte = [&](int k) -> int { return (int)((sc3[k >> 2] >> (8 * (k & 3))) & 0xFFu); };
    if (j < 4) {
        sc = byte(j) & 63;
        m = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 0x0F) | ((byte(j - 4) >> 6) << 4);
        m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// Q6_K slice j (elements 32j .. 32j+31 = sub-blocks 2j, 2j+1) of super-block sb:
// half n = j/4, quarter g = j%4; low 4 bits from ql[64n + 32*(g&1) + l] (low nibble
// for g < 2, high for g >= 2), high 2 bits from qh[32n + l] bits 2g..2g+1; the
// stored value minus 32 is the quant.  is0/is1: the two 16-element integer dots.
__device__ __forceinline__ void unit_sumi_q6_K(const uint8_t* sb, int j, const uint32_t* a, int& is0, int& is1) {
    const int n = j >> 2, g = j & 3;
    uint32_t ql[8], qh[8];
    read_words<8>(sb + 64 * n + 32 * (g & 1), ql);
    read_words<8>(sb + 128 + 32 * n, qh);
    const int lsft = (g < 2) ? 0 : 4;
    int s0 = 0, s1 = 0, z0 = 0, z1 = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t v = ((ql[i] >> lsft) & 0x0F0F0F0Fu) | (((qh[i] >> (2 * g)) << 4) & 0x30303030u);
        if (i < 4) { s0 = dot4((int)v, (int)a[1 + i], s0); z0 = dot4(0x01010101, (int)a[1 + i], z0); }
        else       { s1 = dot4((int)v, (int)a[1 + i], s1); z1 = dot4(0x01010101, (int)a[1 + i], z1); }
    }
    is0 = s0 - 32 * z0;
    is1 = s1 - 32 * z1;
}

// ---- the decode kernel -------------------------------------------------------
template <int WT>
struct Fmt {
    // bytes of one 256-element span (8 blocks or one super-block)
    static constexpr int span = (WT == kWQ4K) ? kQ4KBytes : (WT == kWQ6K) ? kQ6KBytes : 8 * block_bytes(WT);
};

constexpr int kRowsPerWG = 4;
constexpr int kTileSlack = 32;  // bytes after each staged row: head offset + read-ahead of read_words

// Copy `bytes` from global g (2-byte aligned) into LDS at dst = region + (g & 15), one wave:
// 16-bit head up to the next 16-byte boundary, LDS DMA for the body, 16-bit tail.
__device__ __forceinline__ void wave_copy_to_lds(const uint8_t* __restrict__ g, uint8_t* dst, int bytes, int lane) {
    const int head = (int)((16 - ((uintptr_t)g & 15)) & 15);
    const int h = head < bytes ? head : bytes;
    const int nvec = (bytes - h) >> 4;
    const int t0 = h + (nvec << 4);
    if (lane < (h >> 1)) ((uint16_t*)dst)[lane] = ((const uint16_t*)g)[lane];
    if (lane < ((bytes - t0) >> 1)) ((uint16_t*)(dst + t0))[lane] = ((const uint16_t*)(g + t0))[lane];
    const u32x4* src = (const u32x4*)(g + h);
    u32x4* d = (u32x4*)(dst + h);
    for (int base = 0; base < nvec; base += 64) {
        if (base + lane < nvec)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(src + base + lane),
                                             (__attribute__((address_space(3))) void*)(d + base), 16, 0, 0);
    }
}

// C[m][row] = sum over the row's units, for m < MR.  KT = blocks per K tile (multiple of 8).
// AS: the activations are block_q8s (fp32 scale, no sum) instead of block_q8_1.
template <int WT, int MR, bool ALDS, bool AS>
__global__ __launch_bounds__(256) void gemv_row_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ A,
                                                       float* __restrict__ C, int N, int nb, int KT, int ldc,
                                                       int a_vec16) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * kRowsPerWG + wave;
    constexpr bool kq = is_kquant(WT);
    const size_t RB = kq ? (size_t)(nb / 8) * Fmt<WT>::span : (size_t)nb * block_bytes(WT);  // row bytes
    const int tile_w = kq ? (KT / 8) * Fmt<WT>::span : KT * block_bytes(WT);
    const int wpitch = ((tile_w + kTileSlack + 15) & ~15);
    uint8_t* wreg = smem + wave * wpitch;
    uint8_t* areg = smem + kRowsPerWG * wpitch;  // [MR][KT] Q8_1 blocks, 36 B each

    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) acc[m] = 0.0f;

    for (int kt0 = 0; kt0 < nb; kt0 += KT) {
        const int kt = (nb - kt0) < KT ? (nb - kt0) : KT;
        const uint8_t* g = nullptr;
        uint8_t* wt = nullptr;
        if (row < N) {
            const size_t off = kq ? (size_t)(kt0 / 8) * Fmt<WT>::span : (size_t)kt0 * block_bytes(WT);
            const int bytes = kq ? (kt / 8) * Fmt<WT>::span : kt * block_bytes(WT);
            g = W + (size_t)row * RB + off;
            wt = wreg + ((uintptr_t)g & 15);
            wave_copy_to_lds(g, wt, bytes, lane);
        }
        // activations: MR rows x kt blocks, 36 B each (staged in LDS only when ALDS)
        if (!ALDS) {
        } else if (a_vec16) {
            const int nv = kt * 36 / 16;  // per activation row (kt % 4 == 0 here)
            for (int v = threadIdx.x; v < MR * nv; v += 256) {
                const int m = v / nv, j = v - m * nv;
                const u32x4 x = *(const u32x4*)(A + ((size_t)m * nb + kt0) * kQ81Bytes + 16 * j);
                *(u32x4*)(areg + (size_t)m * KT * kQ81Bytes + 16 * j) = x;
            }
        } else {
            const int nv = kt * 9;
            for (int v = threadIdx.x; v < MR * nv; v += 256) {
                const int m = v / nv, j = v - m * nv;
                ((uint32_t*)(areg + (size_t)m * KT * kQ81Bytes))[j] =
                    ((const uint32_t*)(A + ((size_t)m * nb + kt0) * kQ81Bytes))[j];
            }
        }
        wait_vmem();
        __syncthreads();

        if (row < N) {
            for (int u = lane; u < kt; u += 64) {   // unit u = 32-element slice, Q8_1 block kt0 + u
                if constexpr (!kq) {
                    const uint8_t* blk = wt + u * block_bytes(WT);
                    const float dw = f16_to_f32(read_u16(blk));
                    float mw = 0.0f;
                    if constexpr (WT == kWQ41 || WT == kWQ51) mw = f16_to_f32(read_u16(blk + 2));
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        const uint32_t* ap = ALDS ? (const uint32_t*)(areg + ((size_t)m * KT + u) * kQ81Bytes)
                                             : (const uint32_t*)(A + ((size_t)m * nb + kt0 + u) * kQ81Bytes);
                        uint32_t a[9];
#pragma unroll
                        for (int i = 0; i < 9; i++) a[i] = ap[i];
                        const float da = AS ? __builtin_bit_cast(float, a[0]) : f16_to_f32(a[0] & 0xFFFFu);
                        const int sumi = unit_sumi_legacy<WT>(blk, a);
                        // block formulas of gemm_reference.h:216 / :259 and gemm_quant_formats.cuh:148,
                        // :207, :266 (the last two without the reference's /4 on the m*s term)
                        if constexpr (WT == kWQ40) {
                            acc[m] += dw * (da * (float)sumi - 8.0f * f16_to_f32(a[0] >> 16));
                        } else if constexpr (WT == kWQ80) {
                            acc[m] += AS ? dw * da * (float)sumi : (float)sumi * da * dw;
                        } else if constexpr (WT == kWQ50) {
                            acc[m] += dw * (da * (float)sumi - 16.0f * f16_to_f32(a[0] >> 16));
                        } else {
                            acc[m] += dw * da * (float)sumi + mw * f16_to_f32(a[0] >> 16);
                        }
                    }
                } else {
                    const uint8_t* sb = wt + (u >> 3) * Fmt<WT>::span;
                    const int j = u & 7;
                    if constexpr (WT == kWQ4K) {
                        uint32_t hd[1], sc3[3];
                        read_words<1>(sb, hd);
                        read_words<3>(sb + 4, sc3);
                        int sc, mn;
                        q4_K_scale_min(j, sc3, sc, mn);
                        const float d = f16_to_f32(hd[0] & 0xFFFFu), dmin = f16_to_f32(hd[0] >> 16);
#pragma unroll
                        for (int m = 0; m < MR; m++) {
                            const uint32_t* ap = ALDS ? (const uint32_t*)(areg + ((size_t)m * KT + u) * kQ81Bytes)
                                             : (const uint32_t*)(A + ((size_t)m * nb + kt0 + u) * kQ81Bytes);
                            uint32_t a[9];
#pragma unroll
                            for (int i = 0; i < 9; i++) a[i] = ap[i];
                            const int sumi = unit_sumi_q4_K(sb, j, a);
                            acc[m] += d * (f16_to_f32(a[0] & 0xFFFFu) * (float)(sc * sumi)) -
                                      dmin * (f16_to_f32(a[0] >> 16) * (float)mn);
                        }
                    } else {
                        const uint32_t scw = read_u16(sb + 192 + 2 * j);
                        const int sc0 = (int)(int8_t)(scw & 0xFFu), sc1 = (int)(int8_t)(scw >> 8);
                        const float d = f16_to_f32(read_u16(sb + 208));
#pragma unroll
                        for (int m = 0; m < MR; m++) {
                            const uint32_t* ap = ALDS ? (const uint32_t*)(areg + ((size_t)m * KT + u) * kQ81Bytes)
                                             : (const uint32_t*)(A + ((size_t)m * nb + kt0 + u) * kQ81Bytes);
                            uint32_t a[9];
#pragma unroll
                            for (int i = 0; i < 9; i++) a[i] = ap[i];
                            int is0, is1;
                            unit_sumi_q6_K(sb, j, a, is0, is1);
                            acc[m] += d * (f16_to_f32(a[0] & 0xFFFFu) * (float)(sc0 * is0 + sc1 * is1));
                        }
                    }
                }
            }
        }
        if (kt0 + KT < nb) __syncthreads();  // the next tile overwrites LDS
    }
#pragma unroll
    for (int m = 0; m < MR; m++) acc[m] = wave_sum(acc[m]);
    if (row < N && lane == 0) {
#pragma unroll
        for (int m = 0; m < MR; m++) C[(size_t)m * ldc + row] = acc[m];
    }
}

// ---- host dispatch -------------------------------------------------------------
constexpr size_t kGemvLdsBudget = 48 * 1024;

static int span_bytes(int wtype) {
    return wtype == kWQ4K ? kQ4KBytes : wtype == kWQ6K ? kQ6KBytes : 8 * block_bytes(wtype);
}

// Activation rows are staged in LDS (once per workgroup) for M > 2; for M <= 2 each
// lane reads its Q8_1 blocks straight from L2, which measured faster at M = 1.
constexpr int kActLdsMinRows = 3;

static size_t gemv_lds_bytes(int wtype, int mr, int KT) {
    const int tile_w = (KT / 8) * span_bytes(wtype);
    const size_t wpitch = (size_t)((tile_w + kTileSlack + 15) & ~15);
    return kRowsPerWG * wpitch + (mr >= kActLdsMinRows ? (size_t)mr * KT * kQ81Bytes : 0);
}

template <int WT, int MR, bool AS>
static hipError_t row_launch(const uint8_t* W, const uint8_t* A, float* C, int N, int nb, int KT, int ldc, int av16,
                             hipStream_t s) {
    const size_t lds = gemv_lds_bytes(WT, MR, KT);
    auto k = gemv_row_kernel<WT, MR, (MR >= kActLdsMinRows), AS>;
    if (lds > 65536) (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    const unsigned grid = (unsigned)((N + kRowsPerWG - 1) / kRowsPerWG);
    hipLaunchKernelGGL(k, dim3(grid), dim3(256), lds, s, W, A, C, N, nb, KT, ldc, av16);
    return hipGetLastError();
}

template <int WT, bool AS = false>
static hipError_t row_launch_mr(int mr, const uint8_t* W, const uint8_t* A, float* C, int N, int nb, int KT, int ldc,
                                int av16, hipStream_t s) {
    switch (mr) {
        case 1: return row_launch<WT, 1, AS>(W, A, C, N, nb, KT, ldc, av16, s);
        case 2: return row_launch<WT, 2, AS>(W, A, C, N, nb, KT, ldc, av16, s);
        case 3: return row_launch<WT, 3, AS>(W, A, C, N, nb, KT, ldc, av16, s);
        case 4: return row_launch<WT, 4, AS>(W, A, C, N, nb, KT, ldc, av16, s);
        case 5: return row_launch<WT, 5, AS>(W, A, C, N, nb, KT, ldc, av16, s);
        case 6: return row_launch<WT, 6, AS>(W, A, C, N, nb, KT, ldc, av16, s);
        case 7: return row_launch<WT, 7, AS>(W, A, C, N, nb, KT, ldc, av16, s);
        default: return row_launch<WT, 8, AS>(W, A, C, N, nb, KT, ldc, av16, s);
    }
}

hipError_t launch_gemv(int wtype, int afmt, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int K,
                       hipStream_t s) {
    if (afmt == kAQ8S && wtype != kWQ80) return hipErrorNotSupported;
    const int nb = K / 32;
    if (M <= 0 || N <= 0 || nb == 0) return hipSuccess;
    for (int m0 = 0; m0 < M; m0 += 8) {
        const int mr = (M - m0) < 8 ? (M - m0) : 8;
        // K tile: the whole row if it fits the LDS budget, else the largest multiple of 64 blocks
        int KT = (nb + 7) & ~7;
        while (KT > 64 && gemv_lds_bytes(wtype, mr, KT) > kGemvLdsBudget) KT = ((KT / 2) + 63) & ~63;
        const uint8_t* Am = A + (size_t)m0 * nb * kQ81Bytes;
        const int av16 = ((((uintptr_t)Am) & 15u) == 0) && (nb % 4 == 0) && (KT % 4 == 0);
        float* Cm = C + (size_t)m0 * N;
        hipError_t e;
        switch (wtype) {
            case kWQ40: e = row_launch_mr<kWQ40>(mr, W, Am, Cm, N, nb, KT, N, av16, s); break;
            case kWQ80:
                e = (afmt == kAQ8S) ? row_launch_mr<kWQ80, true>(mr, W, Am, Cm, N, nb, KT, N, av16, s)
                                    : row_launch_mr<kWQ80>(mr, W, Am, Cm, N, nb, KT, N, av16, s);
                break;
            case kWQ4K: e = row_launch_mr<kWQ4K>(mr, W, Am, Cm, N, nb, KT, N, av16, s); break;
            case kWQ6K: e = row_launch_mr<kWQ6K>(mr, W, Am, Cm, N, nb, KT, N, av16, s); break;
            case kWQ41: e = row_launch_mr<kWQ41>(mr, W, Am, Cm, N, nb, KT, N, av16, s); break;
            case kWQ50: e = row_launch_mr<kWQ50>(mr, W, Am, Cm, N, nb, KT, N, av16, s); break;
            default: e = row_launch_mr<kWQ51>(mr, W, Am, Cm, N, nb, KT, N, av16, s); break;
        }
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
    // copy the unit's weight bytes with exact-size 16-bit loads (the unit readers may
    // read a few bytes past a block, which is fine in LDS but not at the end of W)
    const int ub = (wtype == kWQ4K) ? kQ4KBytes : (wtype == kWQ6K) ? kQ6KBytes : block_bytes(wtype);
    const uint8_t* src;
    if (!is_kquant(wtype)) src = W + ((size_t)n * nb + b) * ub;
    else src = W + ((size_t)n * (K / 256) + (wtype == kWQ6K ? b / 16 : b / 8)) * ub;
    uint32_t buf[56] = {0};
    for (int i = 0; i < ub / 2; i++) {
        const uint32_t h = ((const uint16_t*)src)[i];
        buf[i >> 1] |= h << (16 * (i & 1));
    }
    const uint8_t* blk = (const uint8_t*)buf;
    const int ab = (wtype == 3) ? b / 2 : b;
    const uint32_t* ap = (const uint32_t*)(A + ((size_t)m * nb + ab) * kQ81Bytes);
    uint32_t a[9];
    for (int i = 0; i < 9; i++) a[i] = ap[i];
    int r;
    if (wtype == kWQ40) r = unit_sumi_q4_0(blk, a);
    else if (wtype == kWQ80) r = unit_sumi_q8_0(blk, a);
    else if (wtype == kWQ41) r = unit_sumi_q4_1(blk, a);
    else if (wtype == kWQ50) r = unit_sumi_q5<2, 6>(blk, a);
    else if (wtype == kWQ51) r = unit_sumi_q5<4, 8>(blk, a);
    else if (wtype == kWQ4K) r = unit_sumi_q4_K(blk, b % 8, a);
    else {
        int is0, is1;
        unit_sumi_q6_K(blk, (b % 16) >> 1, a, is0, is1);
        r = (b & 1) ? is1 : is0;
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
