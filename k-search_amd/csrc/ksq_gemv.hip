// ksq_gemv.hip - decode GEMV on v_dot4c_i32_i8 (the mul_mat_vec_q analogue).
//
// Reference path: the GEMV family in kernelevalplus-main/kernels/gemm/gemm_warp_optimized.cuh:108-1212
// (one warp per weight row, lanes striding K-blocks, DP4A, shuffle reduce) and the
// CPU dots vec_dot_q4_0_q8_1 / vec_dot_q8_0_q8_1 (include/gemm_reference.h:276-336).
//
// gfx950 design (weight rows streamed into LDS by DMA):
//  * A 256-thread workgroup owns 4, 2 or 1 consecutive weight rows (fewer rows when N is
//    small, so the grid still covers the chip; the waves of a row then split it).  Each
//    wave copies its row or row part (a contiguous byte range) into LDS with
//    global_load_lds_dwordx4 (1 KiB per wave instruction, no VGPRs).  One-shot reads of
//    a few MB are fastest as many small, fully coalesced requests spread over the whole
//    chip, which is what this layout issues.
//  * Activations: 1-2 rows are read by each lane straight from L2; 3-8 rows are DMA'd
//    into LDS once per workgroup beside the weights; fp32 activations of 1-2 rows can be
//    quantised inside every workgroup (see kAFQ), saving the quantise launch.
//  * Lanes then stride over 32-element units of the row (a Q4_0/Q8_0/Q4_1/Q5_0/Q5_1
//    block, or one Q8_1-block-sized slice of a Q4_K/Q6_K super-block), pull the unit's
//    bytes out of LDS with dword reads re-aligned by v_alignbyte_b32 (blocks are
//    18/34/20/22/24/144/210 B, only 2-byte aligned), unpack nibbles (and Q5 high bits)
//    in registers and run v_dot4c_i32_i8 against the activation quants; the per-unit
//    fp32 epilogue is the reference formula.
//  * The 64 lane partials are combined with xor shuffles; lane 0 stores.
//  * Rows longer than the LDS tile are walked in K tiles.
//  * 1-2 quantised activation rows (Q6_K: 1) take the register-direct kernels instead: lanes
//    load 4-byte-aligned block pairs (K-quants: unit pairs) straight into VGPRs, no LDS round
//    trip; fp32 rows of 32-element block types are quantised per workgroup beside them.
#include "ksq_device.h"
#include "ksq_internal.h"

namespace ksq {

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

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

// Activation staging modes of the decode kernel.
//   kAL2   each lane reads its activation blocks from global memory (L2) after the weight wait
//          (1 or 2 activation rows short of kGemvDmaMinBlocks1/2 blocks: no barrier)
//   kADMA  the activation rows of the K tile are copied into LDS by DMA, issued together with
//          the weight DMA, so one wait covers both (3 or more rows, or long rows; read once
//          per workgroup)
//   kAFQ   the activations arrive as fp32 and every workgroup quantises the K tile's blocks
//          itself into LDS while its weight DMA is in flight (the same device quantiser as
//          ksq_quantize.hip, so the blocks are bit-identical); no separate quantise launch
//   kAFQH  the same from fp16 activations, by the fused FP16 kernels' quantiser
//          (kernels/gemm/gemm_fused.cuh:76-145; their kernel :158-310 quantises its activation
//          columns into shared memory the same way)
constexpr int kAL2 = 0, kADMA = 1, kAFQ = 2, kAFQH = 3;
__host__ __device__ constexpr bool is_fq(int amode) { return amode == kAFQ || amode == kAFQH; }
constexpr int kMaxL2Rows = 2, kMaxFusedRows = 2;
// With 1-2 activation rows kAL2 reads each row once per wave, i.e. 4x the activation bytes of
// kADMA, as many bytes again as the weights for M = 1.  Shorter rows are latency-bound and kAL2
// (no workgroup barrier) wins; on the longest rows the L2 traffic dominates and kADMA wins
// (measured on MI355X, us, weights streamed from HBM): M = 1 from 576 blocks (Q4_1 N = 3584,
// K = 18944: 13.1 vs 15.7; Q8_0 N = 7168, K = 18432: 29.6 vs 36.4; but Q4_0 N = 4096,
// K = 14336: 12.2 vs 10.7 the other way), M = 2 from 256 blocks (Q4_0 N = 4096, K = 14336: 11.6
// vs 13.8).
constexpr int kGemvDmaMinBlocks1 = 576, kGemvDmaMinBlocks2 = 256;

// Part `part` of `nparts` of a copy of `bytes` from g into LDS at dst (dst = g mod 16): the
// parts split at 16-byte boundaries of g, so each is a valid wave_copy_to_lds.
__device__ __forceinline__ void wave_copy_part(const uint8_t* g, uint8_t* dst, int bytes, int part, int nparts,
                                               int lane) {
    if (nparts == 1) {
        wave_copy_to_lds(g, dst, bytes, lane);
        return;
    }
    const int sh = (int)((uintptr_t)g & 15);
    auto cut = [&](int k) -> int {   // offset of the k-th split point, 16-byte aligned in g
        if (k <= 0) return 0;
        if (k >= nparts) return bytes;
        const int c = ((sh + (int)(((int64_t)bytes * k) / nparts) + 15) & ~15) - sh;
        return c < 0 ? 0 : (c > bytes ? bytes : c);
    };
    const int b0 = cut(part), b1 = cut(part + 1);
    if (b1 > b0) wave_copy_to_lds(g + b0, dst + b0, b1 - b0, lane);
}

// C[m][row] = sum over the row's units, for m < MR.  KT = blocks per K tile (multiple of 8).
// RPW weight rows per workgroup: with 1 or 2 the 4 / RPW waves of a row split its units
// (and its weight copy) and add their partial sums through LDS at the end; with 8 every
// wave owns 2 rows, so each activation block it reads serves both.
// AS: the activations are block_q8s (fp32 scale, no sum) instead of block_q8_1.
// Ain: block_q8_1 / block_q8s bytes [MR][nb] (kAL2, kADMA), fp32 [MR][32 nb] (kAFQ) or fp16
// [MR][32 nb] (kAFQH).  Output C[m * ldc + row * ldr].
template <int WT, int MR, int AMODE, bool AS, int RPW>
__global__ __launch_bounds__(256) void gemv_row_kernel(const uint8_t* __restrict__ W, const void* __restrict__ Ain,
                                                       float* __restrict__ C, int N, int nb, int KT, int ldc, int ldr) {
    static_assert(RPW == 1 || RPW == 2 || RPW == 4 || RPW == 8, "1, 2, 4 or 8 rows per workgroup");
    constexpr int WPR = RPW >= 4 ? 1 : 4 / RPW;  // waves per row
    constexpr int VR = RPW >= 4 ? RPW / 4 : 1;   // rows per wave
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ float red[4][MR];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rloc = wave / WPR, part = wave % WPR;
    const int row0 = blockIdx.x * RPW + rloc * VR;   // this wave's rows: row0 .. row0 + VR - 1
    constexpr bool kq = is_kquant(WT);
    const uint8_t* A = (const uint8_t*)Ain;
    const size_t RB = kq ? (size_t)(nb / 8) * Fmt<WT>::span : (size_t)nb * block_bytes(WT);  // row bytes
    const int tile_w = kq ? (KT / 8) * Fmt<WT>::span : KT * block_bytes(WT);
    const int wpitch = ((tile_w + kTileSlack + 15) & ~15);
    const int apitch = ((KT * kQ81Bytes + 16 + 15) & ~15);
    uint8_t* wreg = smem + rloc * VR * wpitch;
    uint8_t* areg = smem + RPW * wpitch;  // [MR][apitch]: the K tile's activation blocks, 36 B each

    float acc[VR][MR];
#pragma unroll
    for (int v = 0; v < VR; v++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[v][m] = 0.0f;

    for (int kt0 = 0; kt0 < nb; kt0 += KT) {
        const int kt = (nb - kt0) < KT ? (nb - kt0) : KT;
        uint8_t* wt[VR];
#pragma unroll
        for (int v = 0; v < VR; v++) {
            wt[v] = nullptr;
            if (row0 + v < N) {
                const size_t off = kq ? (size_t)(kt0 / 8) * Fmt<WT>::span : (size_t)kt0 * block_bytes(WT);
                const int bytes = kq ? (kt / 8) * Fmt<WT>::span : kt * block_bytes(WT);
                const uint8_t* g = W + (size_t)(row0 + v) * RB + off;
                wt[v] = wreg + v * wpitch + ((uintptr_t)g & 15);
                wave_copy_part(g, wt[v], bytes, part, WPR, lane);
            }
        }
        // per activation row, the byte offset of its first staged block inside its LDS region
        int ashift[MR];
#pragma unroll
        for (int m = 0; m < MR; m++) ashift[m] = 0;
        if constexpr (AMODE == kADMA) {
            // activation row m is copied by wave m % 4
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const uint8_t* g = A + ((size_t)m * nb + kt0) * kQ81Bytes;
                ashift[m] = (int)((uintptr_t)g & 15);
                if ((m & 3) == wave) wave_copy_to_lds(g, areg + m * apitch + ashift[m], kt * kQ81Bytes, lane);
            }
        } else if constexpr (is_fq(AMODE)) {
            const int K = nb * 32;
            for (int v = threadIdx.x; v < MR * kt; v += 256) {
                const int m = v / kt, u = v - m * kt;
                float x[32];
                load_x32<AMODE == kAFQH>(Ain, (size_t)m * K + (size_t)(kt0 + u) * 32, x);
                uint32_t blk[9];
                if constexpr (AS) quantize_block_q8s(x, blk);
                else if constexpr (AMODE == kAFQH) quantize_block_q8_1_f16tree(x, blk);
                else quantize_block_q8_1(x, blk);
                uint32_t* dst = (uint32_t*)(areg + m * apitch + u * kQ81Bytes);
#pragma unroll
                for (int i = 0; i < 9; i++) dst[i] = blk[i];
            }
        }
        const int ustep = 64 * WPR, u0 = part * 64 + lane;
        auto load_act = [&](int u, uint32_t (&av)[MR][9]) {
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const uint32_t* ap = (AMODE == kAL2) ? (const uint32_t*)(A + ((size_t)m * nb + kt0 + u) * kQ81Bytes)
                                                     : (const uint32_t*)(areg + m * apitch + ashift[m] + u * kQ81Bytes);
#pragma unroll
                for (int i = 0; i < 9; i++) av[m][i] = ap[i];
            }
        };
        // LDS written by other waves (shared activations, or a row split over waves) needs the
        // workgroup barrier; a wave that reads only the row it copied itself just waits for its
        // own loads
        constexpr bool shared_lds = (AMODE != kAL2) || (WPR > 1);
        wait_vmem();
        if constexpr (shared_lds) __syncthreads();

        // one unit u (activation block kt0 + u) of weight row row0 + v for all MR activation rows
        auto unit = [&](int v, int u, const uint32_t (&av)[MR][9]) {
            if constexpr (!kq) {
                const uint8_t* blk = wt[v] + u * block_bytes(WT);
                const float dw = f16_to_f32(read_u16(blk));
                float mw = 0.0f;
                if constexpr (WT == kWQ41 || WT == kWQ51) mw = f16_to_f32(read_u16(blk + 2));
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    const uint32_t* a = av[m];
                    const float da = AS ? __builtin_bit_cast(float, a[0]) : f16_to_f32(a[0] & 0xFFFFu);
                    const int sumi = unit_sumi_legacy<WT>(blk, a);
                    // block formulas of gemm_reference.h:216 / :259 and gemm_quant_formats.cuh:148,
                    // :207, :266 (the last two without the reference's /4 on the m*s term)
                    if constexpr (WT == kWQ40) {
                        acc[v][m] += dw * (da * (float)sumi - 8.0f * f16_to_f32(a[0] >> 16));
                    } else if constexpr (WT == kWQ80) {
                        acc[v][m] += AS ? dw * da * (float)sumi : (float)sumi * da * dw;
                    } else if constexpr (WT == kWQ50) {
                        acc[v][m] += dw * (da * (float)sumi - 16.0f * f16_to_f32(a[0] >> 16));
                    } else {
                        acc[v][m] += dw * da * (float)sumi + mw * f16_to_f32(a[0] >> 16);
                    }
                }
            } else {
                const uint8_t* sb = wt[v] + (u >> 3) * Fmt<WT>::span;
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
                        const uint32_t* a = av[m];
                        const int sumi = unit_sumi_q4_K(sb, j, a);
                        acc[v][m] += d * (f16_to_f32(a[0] & 0xFFFFu) * (float)(sc * sumi)) -
                                  dmin * (f16_to_f32(a[0] >> 16) * (float)mn);
                    }
                } else {
                    const uint32_t scw = read_u16(sb + 192 + 2 * j);
                    const int sc0 = (int)(int8_t)(scw & 0xFFu), sc1 = (int)(int8_t)(scw >> 8);
                    const float d = f16_to_f32(read_u16(sb + 208));
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        const uint32_t* a = av[m];
                        int is0, is1;
                        unit_sumi_q6_K(sb, j, a, is0, is1);
                        acc[v][m] += d * (f16_to_f32(a[0] & 0xFFFFu) * (float)(sc0 * is0 + sc1 * is1));
                    }
                }
            }
        };

        if (row0 < N) {
            for (int u = u0; u < kt; u += ustep) {
                uint32_t av[MR][9];
                load_act(u, av);
#pragma unroll
                for (int v = 0; v < VR; v++)
                    if (row0 + v < N) unit(v, u, av);
            }
        }
        if (shared_lds && kt0 + KT < nb) __syncthreads();  // the next tile overwrites LDS
    }
#pragma unroll
    for (int v = 0; v < VR; v++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[v][m] = wave_sum(acc[v][m]);
    if constexpr (WPR > 1) {
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MR; m++) red[wave][m] = acc[0][m];
        }
        __syncthreads();
        if (part == 0) {
#pragma unroll
            for (int m = 0; m < MR; m++)
                for (int p = 1; p < WPR; p++) acc[0][m] += red[wave + p][m];
        }
    }
    if (part == 0 && lane == 0) {
#pragma unroll
        for (int v = 0; v < VR; v++)
            if (row0 + v < N) {
#pragma unroll
                for (int m = 0; m < MR; m++) C[(size_t)m * ldc + (size_t)(row0 + v) * ldr] = acc[v][m];
            }
    }
}

// ---- the register-direct decode kernel ------------------------------------------
// For 32-element block types with 1-2 activation rows read from L2 (kAL2), every lane owns
// pairs of adjacent blocks: a pair is 36/40/44/48/68 bytes, 4-byte aligned whenever the row
// start is (even block count, 4-byte aligned W), so the lane pulls it with dwordx4 loads
// straight into VGPRs: no LDS round trip, no barrier, no wait for other lanes.  Measured on
// MI355X against gemv_row_kernel (weights streamed from HBM, us): Q4_0 M = 1 N = K = 4096
// 4.78 -> 4.14, N = 14336 K = 4096 11.2 -> 8.7, N = 512 K = 7168 3.11 -> 2.57; Q8_0
// N = K = 4096 6.1 -> 5.4; Q5_1 N = 4096 K = 14336 14.3 -> 11.0; Q4_K N = 14336 K = 4096
// 11.9 -> 8.8; Q6_K 15.8 -> 13.8.  Issuing two pairs' loads ahead was mixed (-5% to +3%);
// long rows that stage activations by DMA keep gemv_row_kernel.

// NW dwords from p (4-byte aligned) by 16-, 8- and 4-byte loads.
template <int NW>
__device__ __forceinline__ void load_dwords(const uint32_t* __restrict__ p, uint32_t* w) {
#pragma unroll
    for (int i = 0; i + 4 <= NW; i += 4) {
        const u32x4a4 v = *(const u32x4a4*)(p + i);
        w[i] = v.x; w[i + 1] = v.y; w[i + 2] = v.z; w[i + 3] = v.w;
    }
    constexpr int r0 = NW & ~3;
    if constexpr (NW - r0 >= 2) {
        const u32x2a4 v = *(const u32x2a4*)(p + r0);
        w[r0] = v.x; w[r0 + 1] = v.y;
    }
    if constexpr ((NW - r0) & 1) w[NW - 1] = p[NW - 1];
}

// Little-endian word i / 16-bit field of the byte string at compile-time offset OFF of raw.
template <int OFF>
__device__ __forceinline__ uint32_t word_at(const uint32_t* raw, int i) {
    constexpr int q = OFF / 4, r = OFF % 4;
    if constexpr (r == 0) return raw[q + i];
    else return __builtin_amdgcn_alignbyte(raw[q + i + 1], raw[q + i], r);
}
template <int OFF>
__device__ __forceinline__ uint32_t half_at(const uint32_t* raw) {
    return (raw[OFF / 4] >> (8 * (OFF % 4))) & 0xFFFFu;
}

// The block at byte OFF of raw dotted with activation block a[9]: the same integer dots and
// fp32 block formulas as unit_sumi_legacy and gemv_row_kernel's epilogue.
template <int WT, bool AS, int OFF>
__device__ __forceinline__ float reg_block_dot(const uint32_t* raw, const uint32_t* a) {
    int s = 0;
    if constexpr (WT == kWQ40 || WT == kWQ41) {
        constexpr int QO = OFF + (WT == kWQ40 ? 2 : 4);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = word_at<QO>(raw, i);
            s = dot4((int)(q & 0x0F0F0F0Fu), (int)a[1 + i], s);
            s = dot4((int)((q >> 4) & 0x0F0F0F0Fu), (int)a[5 + i], s);
        }
    } else if constexpr (WT == kWQ80) {
#pragma unroll
        for (int i = 0; i < 8; i++) s = dot4((int)word_at<OFF + 2>(raw, i), (int)a[1 + i], s);
    } else {
        constexpr int QH = OFF + (WT == kWQ50 ? 2 : 4), QS = OFF + (WT == kWQ50 ? 6 : 8);
        const uint32_t h = word_at<QH>(raw, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = word_at<QS>(raw, i);
            s = dot4((int)((q & 0x0F0F0F0Fu) | qh_to_bit4(h >> (4 * i))), (int)a[1 + i], s);
            s = dot4((int)(((q >> 4) & 0x0F0F0F0Fu) | qh_to_bit4(h >> (16 + 4 * i))), (int)a[5 + i], s);
        }
    }
    const float dw = f16_to_f32(half_at<OFF>(raw));
    const float da = AS ? __builtin_bit_cast(float, a[0]) : f16_to_f32(a[0] & 0xFFFFu);
    if constexpr (WT == kWQ40) return dw * (da * (float)s - 8.0f * f16_to_f32(a[0] >> 16));
    else if constexpr (WT == kWQ80) return AS ? dw * da * (float)s : (float)s * da * dw;
    else if constexpr (WT == kWQ50) return dw * (da * (float)s - 16.0f * f16_to_f32(a[0] >> 16));
    else return dw * da * (float)s + f16_to_f32(half_at<OFF + 2>(raw)) * f16_to_f32(a[0] >> 16);
}

// The block at byte OFF of raw dotted with a block_q8f activation block a[10] (fp32 d, fp32 s, 32
// quants): the integer dot, then the deepseek_v2 operator's block term d_w * (d_a * sumi - c * s_a)
// (c = 8 for Q4_0, 16 for Q5_0; none for Q8_0), as ksq_ref_gemm_q8f states it.
template <int WT, int OFF>
__device__ __forceinline__ float reg_block_dot_q8f(const uint32_t* raw, const uint32_t* a) {
    static_assert(WT == kWQ40 || WT == kWQ50 || WT == kWQ80, "block_q8f pairs with Q4_0, Q5_0 and Q8_0");
    int s = 0;
    if constexpr (WT == kWQ40) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = word_at<OFF + 2>(raw, i);
            s = dot4((int)(q & 0x0F0F0F0Fu), (int)a[2 + i], s);
            s = dot4((int)((q >> 4) & 0x0F0F0F0Fu), (int)a[6 + i], s);
        }
    } else if constexpr (WT == kWQ80) {
#pragma unroll
        for (int i = 0; i < 8; i++) s = dot4((int)word_at<OFF + 2>(raw, i), (int)a[2 + i], s);
    } else {
        const uint32_t h = word_at<OFF + 2>(raw, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q = word_at<OFF + 6>(raw, i);
            s = dot4((int)((q & 0x0F0F0F0Fu) | qh_to_bit4(h >> (4 * i))), (int)a[2 + i], s);
            s = dot4((int)(((q >> 4) & 0x0F0F0F0Fu) | qh_to_bit4(h >> (16 + 4 * i))), (int)a[6 + i], s);
        }
    }
    const float dw = f16_to_f32(half_at<OFF>(raw));
    const float da = __builtin_bit_cast(float, a[0]), sa = __builtin_bit_cast(float, a[1]);
    if constexpr (WT == kWQ40) return dw * (da * (float)s - 8.0f * sa);
    else if constexpr (WT == kWQ50) return dw * (da * (float)s - 16.0f * sa);
    else return dw * (da * (float)s);
}

// C[m][row] for m < MR (1 or 2); RPW rows per 256-thread workgroup: 8 = two rows per wave (each
// activation pair a lane loads serves both), 4 = one, 2 or 1 = 4 / RPW waves per row (their
// partial sums meet in LDS).  A: block_q8_1 (or block_q8s when AS) [MR][nb], nb even.
template <int WT, int MR, bool AS, int RPW>
__global__ __launch_bounds__(256) void gemv_direct_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ A,
                                                          float* __restrict__ C, int N, int nb, int ldc) {
    static_assert(!is_kquant(WT) && (MR == 1 || MR == 2), "32-element block types, 1-2 activation rows");
    constexpr int WPR = RPW >= 4 ? 1 : 4 / RPW;  // waves per row
    constexpr int VR = RPW >= 4 ? RPW / 4 : 1;   // rows per wave
    constexpr int BB = block_bytes(WT), PW = BB / 2;  // dwords per block pair
    __shared__ float red[4][MR];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int part = wave % WPR;
    const int row0 = blockIdx.x * RPW + (wave / WPR) * VR;
    float acc[VR][MR];
#pragma unroll
    for (int v = 0; v < VR; v++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[v][m] = 0.0f;
    if (row0 < N) {
        const int np = nb >> 1;
        for (int p = part * 64 + lane; p < np; p += 64 * WPR) {
            uint32_t w[VR][PW], a[MR][18];
#pragma unroll
            for (int v = 0; v < VR; v++)
                if (row0 + v < N) load_dwords<PW>((const uint32_t*)(W + (size_t)(row0 + v) * nb * BB) + (size_t)p * PW, w[v]);
#pragma unroll
            for (int m = 0; m < MR; m++)
                load_dwords<18>((const uint32_t*)(A + ((size_t)m * nb + 2 * p) * kQ81Bytes), a[m]);
#pragma unroll
            for (int v = 0; v < VR; v++)
                if (row0 + v < N) {
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        acc[v][m] += reg_block_dot<WT, AS, 0>(w[v], a[m]);
                        acc[v][m] += reg_block_dot<WT, AS, BB>(w[v], a[m] + 9);
                    }
                }
        }
    }
#pragma unroll
    for (int v = 0; v < VR; v++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[v][m] = wave_sum(acc[v][m]);
    if constexpr (WPR > 1) {
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MR; m++) red[wave][m] = acc[0][m];
        }
        __syncthreads();
        if (part == 0) {
#pragma unroll
            for (int m = 0; m < MR; m++)
                for (int q = 1; q < WPR; q++) acc[0][m] += red[wave + q][m];
        }
    }
    if (part == 0 && lane == 0) {
#pragma unroll
        for (int v = 0; v < VR; v++)
            if (row0 + v < N) {
#pragma unroll
                for (int m = 0; m < MR; m++) C[(size_t)m * ldc + row0 + v] = acc[v][m];
            }
    }
}

// 3-8 activation rows (quantised input, 32-element block types): the same register-direct
// weight loads, with the K tile's activation rows staged in LDS once per workgroup by LDS DMA
// while the first weight pair of every lane is in flight.  A lane reads each activation pair once and
// applies it to its VR weight rows.
// LDS bytes per staged activation row of ktp block pairs: 72 B a pair, plus the DMA's
// alignment shift and read-ahead slack
__host__ __device__ constexpr int direct_mr_apitch(int ktp) { return (ktp * 72 + 16 + 15) & ~15; }

// Weight words of block pair p of a row for the 3-8-row kernel: the pair's bytes for 32-element
// types; for Q4_K the 16-byte head of super-block p / 4 and the 32 quant bytes of its unit pair
// p % 4 (units 2(p % 4), +1: the low / high nibbles), whose activation blocks are again pair p.
template <int WT>
struct MrW { static constexpr int NW = (WT == kWQ4K) ? 12 : block_bytes(WT) / 2; };

template <int WT>
__device__ __forceinline__ void mr_load_w(const uint8_t* __restrict__ W, int row, int nb, int p, uint32_t* w) {
    if constexpr (WT == kWQ4K) {
        const uint8_t* sb = W + ((size_t)row * (nb / 8) + (size_t)(p >> 2)) * kQ4KBytes;
        load_dwords<4>((const uint32_t*)sb, w);
        load_dwords<8>((const uint32_t*)(sb + 16 + 32 * (p & 3)), w + 4);
    } else {
        constexpr int BB = block_bytes(WT), PW = BB / 2;
        load_dwords<PW>((const uint32_t*)(W + (size_t)row * nb * BB) + (size_t)p * PW, w);
    }
}

// Per-pair weight context decoded once for all activation rows (Q4_K: d, dmin and the two
// units' 6-bit scales and mins; nothing for the 32-element types).
template <int WT>
struct MrCtx {
    float d = 0.0f, dmin = 0.0f;
    int sc0 = 0, mn0 = 0, sc1 = 0, mn1 = 0;
    __device__ __forceinline__ void prep(const uint32_t* w, int p) {
        if constexpr (WT == kWQ4K) {
            const int sub = p & 3;
            q4_K_scale_min(2 * sub, w + 1, sc0, mn0);
            q4_K_scale_min(2 * sub + 1, w + 1, sc1, mn1);
            d = f16_to_f32(w[0] & 0xFFFFu);
            dmin = f16_to_f32(w[0] >> 16);
        }
    }
};

// acc += the pair's two unit dots against activation blocks a[0..8], a[9..17]
template <int WT, bool AS>
__device__ __forceinline__ void mr_pair_acc(float& acc, const MrCtx<WT>& c, const uint32_t* w, const uint32_t* a) {
    if constexpr (WT == kWQ4K) {
        int s0 = 0, s1 = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            s0 = dot4((int)(w[4 + i] & 0x0F0F0F0Fu), (int)a[1 + i], s0);
            s1 = dot4((int)((w[4 + i] >> 4) & 0x0F0F0F0Fu), (int)a[10 + i], s1);
        }
        acc += c.d * (f16_to_f32(a[0] & 0xFFFFu) * (float)(c.sc0 * s0)) - c.dmin * (f16_to_f32(a[0] >> 16) * (float)c.mn0);
        acc += c.d * (f16_to_f32(a[9] & 0xFFFFu) * (float)(c.sc1 * s1)) - c.dmin * (f16_to_f32(a[9] >> 16) * (float)c.mn1);
    } else {
        acc += reg_block_dot<WT, AS, 0>(w, a);
        acc += reg_block_dot<WT, AS, block_bytes(WT)>(w, a + 9);
    }
}

// FQ: the activations arrive as fp32 [MR][32 nb] and the workgroup quantises the (single) K
// tile into the same LDS layout instead (the device quantiser, bit-identical blocks); with XH they
// arrive as fp16 and are quantised by the fused FP16 kernels' rules (kernels/gemm/gemm_fused.cuh:
// 76-145, quantize_block_q8_1_f16tree).  Output element (m, row) at C[m * ldc + row * ldr].
template <int WT, int MR, bool AS, int RPW, bool FQ, bool XH = false>
__global__ __launch_bounds__(256) void gemv_direct_mr_kernel(const uint8_t* __restrict__ W, const void* __restrict__ Ain,
                                                             float* __restrict__ C, int N, int nb, int ktp, int ldc,
                                                             int ldr) {
    static_assert((!is_kquant(WT) || WT == kWQ4K) && MR >= 1 && MR <= 8 && !(FQ && is_kquant(WT)),
                  "32-element block types or Q4_K, 1-8 activation rows");
    static_assert(!XH || (FQ && !AS), "fp16 rows are quantised to block_q8_1 inside the workgroup");
    constexpr int WPR = RPW >= 4 ? 1 : 4 / RPW;  // waves per row
    constexpr int VR = RPW >= 4 ? RPW / 4 : 1;   // rows per wave
    constexpr int PW = MrW<WT>::NW;
    extern __shared__ __attribute__((aligned(16))) uint32_t sact[];   // [MR][apitch bytes]
    const int apitch = direct_mr_apitch(ktp);
    __shared__ float red[4][MR];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int part = wave % WPR;
    const int row0 = blockIdx.x * RPW + (wave / WPR) * VR;
    const int np = nb >> 1;
    float acc[VR][MR];
#pragma unroll
    for (int v = 0; v < VR; v++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[v][m] = 0.0f;
    for (int t0 = 0; t0 < np; t0 += ktp) {
        const int tp = (np - t0) < ktp ? (np - t0) : ktp;
        int p = t0 + part * 64 + lane;
        // FQ: this thread's first activation block is loaded before the weight pairs, so its
        // quantisation runs while the weight loads are in flight (loads complete in issue order)
        float x0[FQ ? 32 : 1];
        if constexpr (FQ) {
            const int e = (int)threadIdx.x;
            if (e < MR * 2 * tp) {
                const int m = e / (2 * tp), u = e - m * 2 * tp;
                load_x32<XH>(Ain, (size_t)m * nb * 32 + (size_t)(2 * t0 + u) * 32, x0);
            }
        }
        // unconditional loads (row and pair clamped in range), so that the fused quantisation
        // below waits only for its own activation loads (see gemv_direct_fq_kernel)
        uint32_t w[VR][PW];
#pragma unroll
        for (int v = 0; v < VR; v++) mr_load_w<WT>(W, min(row0 + v, N - 1), nb, min(p, t0 + tp - 1), w[v]);
        // stage the tile: row m's tp pairs (tp * 72 contiguous bytes from pair t0) are copied by
        // wave m % 4 with LDS DMA; its first byte lands at ashift[m] (the source's offset mod 16)
        int ashift[MR];
        if constexpr (FQ) {
            const int K = nb * 32;
            for (int e = threadIdx.x; e < MR * 2 * tp; e += 256) {
                const int m = e / (2 * tp), u = e - m * 2 * tp;   // block u of row m's tile
                float x[32];
                if (e == (int)threadIdx.x) {
#pragma unroll
                    for (int i = 0; i < 32; i++) x[i] = x0[i];
                } else {
                    load_x32<XH>(Ain, (size_t)m * K + (size_t)(2 * t0 + u) * 32, x);
                }
                uint32_t blk[9];
                if constexpr (AS) quantize_block_q8s(x, blk);
                else if constexpr (XH) quantize_block_q8_1_f16tree(x, blk);
                else quantize_block_q8_1(x, blk);
                uint32_t* dst = (uint32_t*)((uint8_t*)sact + (size_t)m * apitch + (size_t)u * kQ81Bytes);
#pragma unroll
                for (int i = 0; i < 9; i++) dst[i] = blk[i];
            }
#pragma unroll
            for (int m = 0; m < MR; m++) ashift[m] = 0;
        } else {
            const uint8_t* A = (const uint8_t*)Ain;
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const uint8_t* g = A + ((size_t)m * nb + 2 * (size_t)t0) * kQ81Bytes;
                ashift[m] = (int)((uintptr_t)g & 15);
                if ((m & 3) == wave) wave_copy_to_lds(g, (uint8_t*)sact + (size_t)m * apitch + ashift[m], tp * 72, lane);
            }
            wait_vmem();
        }
        __syncthreads();
        if (row0 < N) {
            for (bool first = true; p < t0 + tp; p += 64 * WPR, first = false) {
                if (!first) {
#pragma unroll
                    for (int v = 0; v < VR; v++)
                        if (row0 + v < N) mr_load_w<WT>(W, row0 + v, nb, p, w[v]);
                }
                MrCtx<WT> ctx[VR];
#pragma unroll
                for (int v = 0; v < VR; v++) ctx[v].prep(w[v], p);
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    const uint32_t* src = (const uint32_t*)((const uint8_t*)sact + (size_t)m * apitch + ashift[m] +
                                                            (size_t)(p - t0) * 72);
                    uint32_t a[18];
#pragma unroll
                    for (int i = 0; i < 18; i++) a[i] = src[i];
#pragma unroll
                    for (int v = 0; v < VR; v++)
                        if (row0 + v < N) mr_pair_acc<WT, AS>(acc[v][m], ctx[v], w[v], a);
                }
            }
        }
        if (t0 + ktp < np) __syncthreads();   // the next tile overwrites the LDS
    }
#pragma unroll
    for (int v = 0; v < VR; v++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[v][m] = wave_sum(acc[v][m]);
    if constexpr (WPR > 1) {
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MR; m++) red[wave][m] = acc[0][m];
        }
        __syncthreads();
        if (part == 0) {
#pragma unroll
            for (int m = 0; m < MR; m++)
                for (int q = 1; q < WPR; q++) acc[0][m] += red[wave + q][m];
        }
    }
    if (part == 0 && lane == 0) {
#pragma unroll
        for (int v = 0; v < VR; v++)
            if (row0 + v < N) {
#pragma unroll
                for (int m = 0; m < MR; m++) C[(size_t)m * ldc + (size_t)(row0 + v) * ldr] = acc[v][m];
            }
    }
}

// K-quant form: a lane task is a pair of 32-element units that share their quant bytes.
//   Q4_K (144-byte super-blocks, 16-byte aligned in rows of K/256 of them): units 2g, 2g+1
//        = the low / high nibbles of qs[32g .. 32g+31]; the lane loads the 16-byte head
//        (d, dmin, 12 scale bytes) and those 32 quant bytes.
//   Q6_K (210-byte super-blocks, 2-byte aligned): units j, j+2 (j = 4n + h, h < 2) = the low /
//        high nibbles of ql[64n + 32h ..] with bits 2g.. of qh[32n ..]; the lane loads both
//        32-byte spans, the 16 scale bytes and d, re-aligning odd super-blocks with alignbyte.
// Integer dots and fp32 unit formulas are those of gemv_row_kernel.
// A span of NW little-endian words at p (2-byte aligned), loaded as NW + 1 aligned dwords and
// re-aligned later (raw_span / realign), so that all loads of a lane task issue before the first
// v_alignbyte waits on one (left to itself the scheduler starts on the first spans and issues
// the rest one memory latency later).
//   fwd:  from p rounded down to 4 bytes; the caller guarantees 4 readable bytes after the span.
//   back: from 4 (p 4-byte aligned) or 2 bytes before p, ending at p + 4 NW - 1 or p + 4 NW + 1;
//         the caller guarantees 4 readable bytes before p and, for p = 2 mod 4, 2 after the span.
template <int NW, bool BACK>
__device__ __forceinline__ void raw_span(const uint8_t* __restrict__ p, uint32_t* raw) {
    const int sh = (int)((uintptr_t)p & 3u);
    load_dwords<NW + 1>((const uint32_t*)(BACK ? p - 4 + sh : p - sh), raw);
}
template <int NW, bool BACK>
__device__ __forceinline__ void realign(const uint8_t* p, const uint32_t* raw, uint32_t* w) {
    const int sh = (int)((uintptr_t)p & 3u);
#pragma unroll
    for (int i = 0; i < NW; i++)
        w[i] = BACK ? (sh ? __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], 2) : raw[i + 1])
                    : __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], sh);
}

template <int WT, int MR, int RPW>
__global__ __launch_bounds__(256) void gemv_direct_kq_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ A,
                                                             float* __restrict__ C, int N, int nb, int ldc) {
    static_assert(is_kquant(WT) && (MR == 1 || MR == 2), "K-quant types, 1-2 activation rows");
    constexpr int WPR = 4 / RPW;
    constexpr int SB = Fmt<WT>::span;
    __shared__ float red[4][MR];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int part = wave % WPR;
    const int row = blockIdx.x * RPW + wave / WPR;
    float acc[MR];
#pragma unroll
    for (int m = 0; m < MR; m++) acc[m] = 0.0f;
    if (row < N) {
        const uint8_t* wrow = W + (size_t)row * (nb / 8) * SB;
        const int ntask = (nb / 8) * 4;
        for (int t = part * 64 + lane; t < ntask; t += 64 * WPR) {
            const int sbi = t >> 2, sub = t & 3;
            const uint8_t* sb = wrow + (size_t)sbi * SB;
            if constexpr (WT == kWQ4K) {
                uint32_t hd[4], q[8], a[MR][18];
                load_dwords<4>((const uint32_t*)sb, hd);
                load_dwords<8>((const uint32_t*)(sb + 16 + 32 * sub), q);
#pragma unroll
                for (int m = 0; m < MR; m++)
                    load_dwords<18>((const uint32_t*)(A + ((size_t)m * nb + 8 * sbi + 2 * sub) * kQ81Bytes), a[m]);
                int sc0, mn0, sc1, mn1;
                q4_K_scale_min(2 * sub, hd + 1, sc0, mn0);
                q4_K_scale_min(2 * sub + 1, hd + 1, sc1, mn1);
                const float d = f16_to_f32(hd[0] & 0xFFFFu), dmin = f16_to_f32(hd[0] >> 16);
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    int s0 = 0, s1 = 0;
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        s0 = dot4((int)(q[i] & 0x0F0F0F0Fu), (int)a[m][1 + i], s0);
                        s1 = dot4((int)((q[i] >> 4) & 0x0F0F0F0Fu), (int)a[m][10 + i], s1);
                    }
                    acc[m] += d * (f16_to_f32(a[m][0] & 0xFFFFu) * (float)(sc0 * s0)) -
                              dmin * (f16_to_f32(a[m][0] >> 16) * (float)mn0);
                    acc[m] += d * (f16_to_f32(a[m][9] & 0xFFFFu) * (float)(sc1 * s1)) -
                              dmin * (f16_to_f32(a[m][9] >> 16) * (float)mn1);
                }
            } else {
                const int n = sub >> 1, h = sub & 1;
                const int j0 = 4 * n + h, j1 = j0 + 2;
                const uint8_t* pl = sb + 64 * n + 32 * h;  // ql span, ends <= byte 127 (+4 read) of 210
                const uint8_t* ph = sb + 128 + 32 * n;     // qh span, ends <= byte 191 (+4 read)
                const uint8_t* ps = sb + 192;              // scales: reads 188 or 190 .. 207 or 209
                uint32_t rl[9], rh[9], rs[5], a[MR][2][9];
                raw_span<8, false>(pl, rl);
                raw_span<8, false>(ph, rh);
                raw_span<4, true>(ps, rs);
                const uint32_t dbits = read_u16(sb + 208);
#pragma unroll
                for (int m = 0; m < MR; m++) {
                    load_dwords<9>((const uint32_t*)(A + ((size_t)m * nb + 8 * sbi + j0) * kQ81Bytes), a[m][0]);
                    load_dwords<9>((const uint32_t*)(A + ((size_t)m * nb + 8 * sbi + j1) * kQ81Bytes), a[m][1]);
                }
                __builtin_amdgcn_sched_barrier(0);
                uint32_t ql[8], qh[8], sc[4];
                realign<8, false>(pl, rl, ql);
                realign<8, false>(ph, rh, qh);
                realign<4, true>(ps, rs, sc);
                const float d = f16_to_f32(dbits);
                // scales 2j, 2j + 1 of unit j = 4n + h (+ 2): bytes 8n + 2h (+ 4) of the 16, i.e.
                // the low or high half of word 2n (2n + 1); no register array indexed at run time
                const uint32_t sw0 = n ? sc[2] : sc[0], sw1 = n ? sc[3] : sc[1];
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const int g = 2 * e + h;
                    const int lsft = e ? 4 : 0;
                    const uint32_t sw = (e ? sw1 : sw0) >> (16 * h);
                    const int c0 = (int)(int8_t)(sw & 0xFFu), c1 = (int)(int8_t)((sw >> 8) & 0xFFu);
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        const uint32_t* av = a[m][e];
                        int s0 = 0, s1 = 0, z0 = 0, z1 = 0;
#pragma unroll
                        for (int i = 0; i < 8; i++) {
                            const uint32_t v = ((ql[i] >> lsft) & 0x0F0F0F0Fu) | (((qh[i] >> (2 * g)) << 4) & 0x30303030u);
                            if (i < 4) { s0 = dot4((int)v, (int)av[1 + i], s0); z0 = dot4(0x01010101, (int)av[1 + i], z0); }
                            else       { s1 = dot4((int)v, (int)av[1 + i], s1); z1 = dot4(0x01010101, (int)av[1 + i], z1); }
                        }
                        const int is0 = s0 - 32 * z0, is1 = s1 - 32 * z1;
                        acc[m] += d * (f16_to_f32(av[0] & 0xFFFFu) * (float)(c0 * is0 + c1 * is1));
                    }
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; m++) acc[m] = wave_sum(acc[m]);
    if constexpr (WPR > 1) {
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MR; m++) red[wave][m] = acc[m];
        }
        __syncthreads();
        if (part == 0) {
#pragma unroll
            for (int m = 0; m < MR; m++)
                for (int q = 1; q < WPR; q++) acc[m] += red[wave + q][m];
        }
    }
    if (part == 0 && lane == 0 && row < N) {
#pragma unroll
        for (int m = 0; m < MR; m++) C[(size_t)m * ldc + row] = acc[m];
    }
}

// The same with fp32 activations quantised inside every workgroup (the kAFQ idea): each lane
// first issues the loads of its first weight pair, the workgroup then quantises the MR
// activation rows into LDS (hiding the weight latency), and after one barrier the lanes walk
// their pairs with the activation blocks read from LDS.  RPW 8: two rows per wave, halving
// the quantisation each row costs.  XH: X holds fp16 activations, quantised by the fused FP16
// kernels' rules.  QF 1 / 2: the rows are quantised to block_q8f by the deepseek_v2 (RNE) /
// lm_head (LROUND) rule instead.  Output C[m * ldc + row * ldr].
template <int WT, int MR, bool AS, int RPW, bool XH, int QF = 0>
__global__ __launch_bounds__(256) void gemv_direct_fq_kernel(const uint8_t* __restrict__ W, const void* __restrict__ X,
                                                             float* __restrict__ C, int N, int nb, int ldc, int ldr) {
    static_assert(!is_kquant(WT) && (MR == 1 || MR == 2), "32-element block types, 1-2 activation rows");
    static_assert(!QF || (!AS && !XH && (WT == kWQ40 || WT == kWQ50 || WT == kWQ80)),
                  "block_q8f: fp32 rows against Q4_0, Q5_0 or Q8_0 weights");
    constexpr int QW = QF ? 10 : 9, QB = 4 * QW;   // words / bytes per staged activation block
    constexpr int WPR = RPW >= 4 ? 1 : 4 / RPW;  // waves per row
    constexpr int VR = RPW >= 4 ? RPW / 4 : 1;   // rows per wave
    constexpr int BB = block_bytes(WT), PW = BB / 2;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];  // [MR][nb] activation blocks
    __shared__ float red[4][MR];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int part = wave % WPR;
    const int row0 = blockIdx.x * RPW + (wave / WPR) * VR;
    const int np = nb >> 1;
    int p = part * 64 + lane;
    const int K = nb * 32;
    // this thread's first activation block is loaded before the weight pairs: global loads
    // complete in issue order, so its quantisation waits only for it and runs while the weight
    // loads are in flight (loaded after them, the quantisation would wait for the weights too)
    // fp32 or fp16 -> block_q8_1 (or block_q8f): each block is quantised by a lane pair (16
    // elements a lane), which spreads the quantisation over all four waves (config 0, fp32 entry:
    // 5.40 -> 4.57 us); block_q8s quantises a block per lane
    constexpr bool PAIR = !AS;
    const int nq = PAIR ? 2 * MR * nb : MR * nb;   // half blocks or blocks to quantise
    float x0[PAIR ? 16 : 32];
    const bool has0 = (int)threadIdx.x < nq;
    if (has0) {
        if constexpr (PAIR) {
            const int u = (int)threadIdx.x >> 1, m = u / nb, ub = u - m * nb;
            load_x16<XH>(X, (size_t)m * K + (size_t)ub * 32 + 16 * (threadIdx.x & 1), x0);
        } else {
            const int m = (int)threadIdx.x / nb, u = (int)threadIdx.x - m * nb;
            load_x32<XH>(X, (size_t)m * K + (size_t)u * 32, x0);
        }
    }
    // unconditional loads (row and pair clamped in range; lanes past them discard the data): with a
    // conditional load the compiler must assume none is pending on the other path and would wait
    // for every load, weights included, before the quantisation
    uint32_t w[VR][PW];
#pragma unroll
    for (int v = 0; v < VR; v++)
        load_dwords<PW>((const uint32_t*)(W + (size_t)min(row0 + v, N - 1) * nb * BB) + (size_t)min(p, np - 1) * PW,
                        w[v]);
    for (int t = threadIdx.x; t < nq; t += 256) {
        if constexpr (PAIR) {
            // half block t & 1 of block u (the partner lane t ^ 1 holds the other half)
            const int u = t >> 1, m = u / nb, ub = u - m * nb;
            float x[16];
            if (t == (int)threadIdx.x) {
#pragma unroll
                for (int i = 0; i < 16; i++) x[i] = x0[i];
            } else {
                load_x16<XH>(X, (size_t)m * K + (size_t)ub * 32 + 16 * (t & 1), x);
            }
            uint32_t* dst = (uint32_t*)(smem + (size_t)u * QB);
            if constexpr (QF) quantize_block_q8f_pair<QF - 1>(x, t & 1, dst);
            else if constexpr (XH) quantize_block_q8_1_f16tree_pair(x, t & 1, dst);
            else quantize_block_q8_1_pair(x, t & 1, dst);
        } else {
            const int m = t / nb, u = t - m * nb;
            float x[32];
            if (t == (int)threadIdx.x) {
#pragma unroll
                for (int i = 0; i < 32; i++) x[i] = x0[i];
            } else {
                load_x32<XH>(X, (size_t)m * K + (size_t)u * 32, x);
            }
            uint32_t blk[9];
            if constexpr (AS) quantize_block_q8s(x, blk);
            else if constexpr (XH) quantize_block_q8_1_f16tree(x, blk);
            else quantize_block_q8_1(x, blk);
            uint32_t* dst = (uint32_t*)(smem + (size_t)t * kQ81Bytes);
#pragma unroll
            for (int i = 0; i < 9; i++) dst[i] = blk[i];
        }
    }
    __syncthreads();
    float acc[VR][MR];
#pragma unroll
    for (int v = 0; v < VR; v++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[v][m] = 0.0f;
    if (row0 < N) {
        for (bool first = true; p < np; p += 64 * WPR, first = false) {
            if (!first) {
#pragma unroll
                for (int v = 0; v < VR; v++)
                    if (row0 + v < N)
                        load_dwords<PW>((const uint32_t*)(W + (size_t)(row0 + v) * nb * BB) + (size_t)p * PW, w[v]);
            }
            uint32_t a[MR][2 * QW];
#pragma unroll
            for (int m = 0; m < MR; m++)
                load_dwords<2 * QW>((const uint32_t*)(smem + ((size_t)m * nb + 2 * p) * QB), a[m]);
#pragma unroll
            for (int v = 0; v < VR; v++)
                if (row0 + v < N) {
#pragma unroll
                    for (int m = 0; m < MR; m++) {
                        if constexpr (QF) {
                            acc[v][m] += reg_block_dot_q8f<WT, 0>(w[v], a[m]);
                            acc[v][m] += reg_block_dot_q8f<WT, BB>(w[v], a[m] + QW);
                        } else {
                            acc[v][m] += reg_block_dot<WT, AS, 0>(w[v], a[m]);
                            acc[v][m] += reg_block_dot<WT, AS, BB>(w[v], a[m] + 9);
                        }
                    }
                }
        }
    }
#pragma unroll
    for (int v = 0; v < VR; v++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[v][m] = wave_sum(acc[v][m]);
    if constexpr (WPR > 1) {
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MR; m++) red[wave][m] = acc[0][m];
        }
        __syncthreads();
        if (part == 0) {
#pragma unroll
            for (int m = 0; m < MR; m++)
                for (int q = 1; q < WPR; q++) acc[0][m] += red[wave + q][m];
        }
    }
    if (part == 0 && lane == 0) {
#pragma unroll
        for (int v = 0; v < VR; v++)
            if (row0 + v < N) {
#pragma unroll
                for (int m = 0; m < MR; m++) C[(size_t)m * ldc + (size_t)(row0 + v) * ldr] = acc[v][m];
            }
    }
}

// ---- host dispatch -------------------------------------------------------------
constexpr size_t kGemvLdsBudget = 48 * 1024;

static int span_bytes(int wtype) {
    return wtype == kWQ4K ? kQ4KBytes : wtype == kWQ6K ? kQ6KBytes : 8 * block_bytes(wtype);
}

static size_t gemv_lds_bytes(int wtype, int mr, int KT, int amode, int rpw) {
    const int tile_w = (KT / 8) * span_bytes(wtype);
    const size_t wpitch = (size_t)((tile_w + kTileSlack + 15) & ~15);
    const size_t apitch = (size_t)((KT * kQ81Bytes + 16 + 15) & ~15);
    return rpw * wpitch + (amode == kAL2 ? 0 : (size_t)mr * apitch);
}

// Rows per workgroup: 4 while that still gives at least kGemvMinWGs workgroups, else 2 or 1
// (the waves of a row then split its K range), so small-N matrices still cover the chip.
#ifndef KSQ_GEMV_MIN_WGS
#define KSQ_GEMV_MIN_WGS 256
#endif
constexpr int kGemvMinWGs = KSQ_GEMV_MIN_WGS;

// Staging modes (bit AMODE) that use 8 rows per workgroup (2 rows per wave) when N allows.
// Only the fused mode does: it halves the quantisation every workgroup repeats.  For the DMA
// mode the halved activation traffic did not pay for the halved grid (measured over the 87
// definitions: neutral at N = 4096, 8-24% slower at N >= 9728 with 8 activation rows).
#ifndef KSQ_GEMV_RPW8_MODES
#define KSQ_GEMV_RPW8_MODES 0xC
#endif

static int pick_rpw(int N, int amode) {
    if (((KSQ_GEMV_RPW8_MODES >> amode) & 1) && (N + 7) / 8 >= kGemvMinWGs) return 8;
    if ((N + 3) / 4 >= kGemvMinWGs) return 4;
    if ((N + 1) / 2 >= kGemvMinWGs) return 2;
    return 1;
}

template <int WT, int MR, int AMODE, bool AS, int RPW>
static hipError_t row_launch(const uint8_t* W, const void* A, float* C, int N, int nb, int KT, int ldc, int ldr,
                             hipStream_t s) {
    if constexpr ((AMODE == kAL2 && MR > kMaxL2Rows) || (is_fq(AMODE) && MR > kMaxFusedRows) ||
                  (AMODE == kAFQH && AS)) {
        return hipErrorNotSupported;  // combinations the dispatcher never asks for are not compiled
    } else {
        const size_t lds = gemv_lds_bytes(WT, MR, KT, AMODE, RPW);
        auto k = gemv_row_kernel<WT, MR, AMODE, AS, RPW>;
        if (lds > 65536)
            (void)hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        const unsigned grid = (unsigned)((N + RPW - 1) / RPW);
        hipLaunchKernelGGL(k, dim3(grid), dim3(256), lds, s, W, A, C, N, nb, KT, ldc, ldr);
        return hipGetLastError();
    }
}

template <int WT, int MR, int AMODE, bool AS>
static hipError_t row_launch_rpw(int rpw, const uint8_t* W, const void* A, float* C, int N, int nb, int KT, int ldc,
                                 int ldr, hipStream_t s) {
    switch (rpw) {
        case 8:
            if constexpr ((KSQ_GEMV_RPW8_MODES >> AMODE) & 1) return row_launch<WT, MR, AMODE, AS, 8>(W, A, C, N, nb, KT, ldc, ldr, s);
            else return hipErrorNotSupported;
        case 4: return row_launch<WT, MR, AMODE, AS, 4>(W, A, C, N, nb, KT, ldc, ldr, s);
        case 2: return row_launch<WT, MR, AMODE, AS, 2>(W, A, C, N, nb, KT, ldc, ldr, s);
        default: return row_launch<WT, MR, AMODE, AS, 1>(W, A, C, N, nb, KT, ldc, ldr, s);
    }
}

template <int WT, int AMODE, bool AS>
static hipError_t row_launch_mr(int mr, int rpw, const uint8_t* W, const void* A, float* C, int N, int nb, int KT,
                                int ldc, int ldr, hipStream_t s) {
    switch (mr) {
        case 1: return row_launch_rpw<WT, 1, AMODE, AS>(rpw, W, A, C, N, nb, KT, ldc, ldr, s);
        case 2: return row_launch_rpw<WT, 2, AMODE, AS>(rpw, W, A, C, N, nb, KT, ldc, ldr, s);
        case 3: return row_launch_rpw<WT, 3, AMODE, AS>(rpw, W, A, C, N, nb, KT, ldc, ldr, s);
        case 4: return row_launch_rpw<WT, 4, AMODE, AS>(rpw, W, A, C, N, nb, KT, ldc, ldr, s);
        case 5: return row_launch_rpw<WT, 5, AMODE, AS>(rpw, W, A, C, N, nb, KT, ldc, ldr, s);
        case 6: return row_launch_rpw<WT, 6, AMODE, AS>(rpw, W, A, C, N, nb, KT, ldc, ldr, s);
        case 7: return row_launch_rpw<WT, 7, AMODE, AS>(rpw, W, A, C, N, nb, KT, ldc, ldr, s);
        default: return row_launch_rpw<WT, 8, AMODE, AS>(rpw, W, A, C, N, nb, KT, ldc, ldr, s);
    }
}

// Two rows per wave once that still leaves 1024 workgroups, or 256 on rows of 384+ blocks
// (measured, us: Q4_0 M = 1 N = 14336 K = 4096 8.7 -> 8.0, N = 4096 K = 14336 10.0 -> 8.3;
// fewer workgroups lost: Q4_0 N = K = 2560 2.91 -> 3.16, Q5_0 N = K = 4096 4.41 -> 4.69).
static int direct_rpw(int rpw, int N, int nb) {
    const int wgs8 = (N + 7) / 8;
    return (rpw == 4 && (wgs8 >= 1024 || (nb >= 384 && wgs8 >= kGemvMinWGs))) ? 8 : rpw;
}

template <int WT, bool AS, int MR>
static hipError_t direct_launch_rpw(int rpw, const uint8_t* W, const uint8_t* A, float* C, int N, int nb, int ldc,
                                    hipStream_t s) {
    const dim3 blk(256);
    switch (direct_rpw(rpw, N, nb)) {
        case 8: hipLaunchKernelGGL((gemv_direct_kernel<WT, MR, AS, 8>), dim3((N + 7) / 8), blk, 0, s, W, A, C, N, nb, ldc); break;
        case 4: hipLaunchKernelGGL((gemv_direct_kernel<WT, MR, AS, 4>), dim3((N + 3) / 4), blk, 0, s, W, A, C, N, nb, ldc); break;
        case 2: hipLaunchKernelGGL((gemv_direct_kernel<WT, MR, AS, 2>), dim3((N + 1) / 2), blk, 0, s, W, A, C, N, nb, ldc); break;
        default: hipLaunchKernelGGL((gemv_direct_kernel<WT, MR, AS, 1>), dim3(N), blk, 0, s, W, A, C, N, nb, ldc); break;
    }
    return hipGetLastError();
}

template <int WT, bool AS, int MR, bool XH>
static hipError_t direct_fq_launch_rpw(int rpw, const uint8_t* W, const void* X, float* C, int N, int nb, int ldc,
                                       int ldr, hipStream_t s) {
    const dim3 blk(256);
    const size_t lds = (size_t)MR * nb * kQ81Bytes;
    switch (rpw) {
        case 8: hipLaunchKernelGGL((gemv_direct_fq_kernel<WT, MR, AS, 8, XH>), dim3((N + 7) / 8), blk, lds, s, W, X, C, N, nb, ldc, ldr); break;
        case 4: hipLaunchKernelGGL((gemv_direct_fq_kernel<WT, MR, AS, 4, XH>), dim3((N + 3) / 4), blk, lds, s, W, X, C, N, nb, ldc, ldr); break;
        case 2: hipLaunchKernelGGL((gemv_direct_fq_kernel<WT, MR, AS, 2, XH>), dim3((N + 1) / 2), blk, lds, s, W, X, C, N, nb, ldc, ldr); break;
        default: hipLaunchKernelGGL((gemv_direct_fq_kernel<WT, MR, AS, 1, XH>), dim3(N), blk, lds, s, W, X, C, N, nb, ldc, ldr); break;
    }
    return hipGetLastError();
}

// QUANT: pre-quantised activations (gemv_direct_kernel), else fp32 or, with xh, fp16
// (gemv_direct_fq_kernel).
template <int WT, bool AS>
static hipError_t direct_launch(bool quant, bool xh, int mr, int rpw, const uint8_t* W, const void* A, float* C, int N,
                                int nb, int ldc, int ldr, hipStream_t s) {
    if (!quant) {
        if constexpr (AS) {
            if (xh) return hipErrorNotSupported;
            return mr == 1 ? direct_fq_launch_rpw<WT, AS, 1, false>(rpw, W, A, C, N, nb, ldc, ldr, s)
                           : direct_fq_launch_rpw<WT, AS, 2, false>(rpw, W, A, C, N, nb, ldc, ldr, s);
        } else {
            if (xh)
                return mr == 1 ? direct_fq_launch_rpw<WT, AS, 1, true>(rpw, W, A, C, N, nb, ldc, ldr, s)
                               : direct_fq_launch_rpw<WT, AS, 2, true>(rpw, W, A, C, N, nb, ldc, ldr, s);
            return mr == 1 ? direct_fq_launch_rpw<WT, AS, 1, false>(rpw, W, A, C, N, nb, ldc, ldr, s)
                           : direct_fq_launch_rpw<WT, AS, 2, false>(rpw, W, A, C, N, nb, ldc, ldr, s);
        }
    }
    return mr == 1 ? direct_launch_rpw<WT, AS, 1>(rpw, W, (const uint8_t*)A, C, N, nb, ldc, s)
                   : direct_launch_rpw<WT, AS, 2>(rpw, W, (const uint8_t*)A, C, N, nb, ldc, s);
}

// Pairs per K tile of gemv_direct_mr_kernel: the whole row while MR rows of it fit the LDS
// budget, else the largest multiple of 64 pairs that does.
static int direct_mr_ktp(int mr, int nb) {
    const int np = nb >> 1;
    if ((size_t)mr * direct_mr_apitch(np) <= kGemvLdsBudget) return np;
    int ktp = 64;
    while ((size_t)mr * direct_mr_apitch(ktp + 64) <= kGemvLdsBudget) ktp += 64;
    return ktp;
}

template <int WT, bool AS, int MR, bool FQ, bool XH = false>
static hipError_t direct_mr_launch_rpw(int rpw, const uint8_t* W, const void* A, float* C, int N, int nb, int ldc,
                                       int ldr, hipStream_t s) {
    const int ktp = direct_mr_ktp(MR, nb);
    if (FQ && ktp != (nb >> 1)) return hipErrorNotSupported;   // fused quantisation: one K tile
    const size_t lds = (size_t)MR * direct_mr_apitch(ktp);
    const dim3 blk(256);
    // two rows per wave on long rows for up to 5 activation rows (past that the doubled
    // accumulators cost occupancy): Q4_0 N = 4096, K = 14336, M = 3 14.8 -> 11.7 us, M = 8
    // 24.4 -> 28.2 the other way
    if (rpw == 4 && MR <= 5 && nb >= 384 && (N + 7) / 8 >= kGemvMinWGs) rpw = 8;
    switch (rpw) {
        case 8:
            if constexpr (MR <= 5)
                hipLaunchKernelGGL((gemv_direct_mr_kernel<WT, MR, AS, 8, FQ, XH>), dim3((N + 7) / 8), blk, lds, s, W, A, C, N, nb, ktp, ldc, ldr);
            break;
        case 4: hipLaunchKernelGGL((gemv_direct_mr_kernel<WT, MR, AS, 4, FQ, XH>), dim3((N + 3) / 4), blk, lds, s, W, A, C, N, nb, ktp, ldc, ldr); break;
        case 2: hipLaunchKernelGGL((gemv_direct_mr_kernel<WT, MR, AS, 2, FQ, XH>), dim3((N + 1) / 2), blk, lds, s, W, A, C, N, nb, ktp, ldc, ldr); break;
        default: hipLaunchKernelGGL((gemv_direct_mr_kernel<WT, MR, AS, 1, FQ, XH>), dim3(N), blk, lds, s, W, A, C, N, nb, ktp, ldc, ldr); break;
    }
    return hipGetLastError();
}

template <int WT, bool AS>
static hipError_t direct_mr_launch(bool quant, bool xh, int mr, int rpw, const uint8_t* W, const void* A, float* C,
                                   int N, int nb, int ldc, int ldr, hipStream_t s) {
#define KSQ_MR_CASE(MRV)                                                                                          \
    if constexpr (is_kquant(WT)) return quant ? direct_mr_launch_rpw<WT, AS, MRV, false>(rpw, W, A, C, N, nb, ldc, ldr, s) \
                                              : hipErrorNotSupported;                                             \
    else if constexpr (AS) return quant ? direct_mr_launch_rpw<WT, AS, MRV, false>(rpw, W, A, C, N, nb, ldc, ldr, s)    \
                                        : xh ? hipErrorNotSupported                                               \
                                             : direct_mr_launch_rpw<WT, AS, MRV, true>(rpw, W, A, C, N, nb, ldc, ldr, s); \
    else return quant ? direct_mr_launch_rpw<WT, AS, MRV, false>(rpw, W, A, C, N, nb, ldc, ldr, s)                     \
                : xh  ? direct_mr_launch_rpw<WT, AS, MRV, true, true>(rpw, W, A, C, N, nb, ldc, ldr, s)               \
                      : direct_mr_launch_rpw<WT, AS, MRV, true>(rpw, W, A, C, N, nb, ldc, ldr, s);
    switch (mr) {
        case 3: KSQ_MR_CASE(3)
        case 4: KSQ_MR_CASE(4)
        case 5: KSQ_MR_CASE(5)
        case 6: KSQ_MR_CASE(6)
        case 7: KSQ_MR_CASE(7)
        default: KSQ_MR_CASE(8)
    }
#undef KSQ_MR_CASE
}

// The register-direct kernels take 1-2 activation rows (quantised ones read from L2, or fp32
// ones quantised per workgroup) for 32-element block types when every block pair is 4-byte
// aligned; the fp32 form also needs the quantised rows to fit the LDS budget.
// Build-time switches (-DKSQ_GEMV_DIRECT_FQ=0 etc.) that route the register-direct cases back to
// gemv_row_kernel, for A/B measurement; both sides compute the same block formulas.
#ifndef KSQ_GEMV_DIRECT_FQ
#define KSQ_GEMV_DIRECT_FQ 1
#endif
#ifndef KSQ_GEMV_DIRECT_KQ
#define KSQ_GEMV_DIRECT_KQ 1
#endif
#ifndef KSQ_GEMV_DIRECT_MR
#define KSQ_GEMV_DIRECT_MR 1
#endif
// 3-8 rows: the register-direct form measured 9% faster over 108 decode shapes (M = 3..8, Q4_0 /
// Q8_0 / Q4_1), but for grids of 256-511 four-row workgroups (N = 1536, K = 5120: 5.6 vs 5.1 us
// at M = 4), where gemv_row_kernel stays.
static bool direct_eligible(int wtype, int amode, int mr, int nb, int N, int rpw, const void* W, const void* A) {
    // Q4_K included: measured 5-33% faster over 36 shapes at M = 3..8 (N = 3584, K = 18944, M = 4:
    // 25.9 -> 17.3 us), once the scale decode is done once per pair rather than per activation row
    if (amode == kADMA && mr >= 3)
        return KSQ_GEMV_DIRECT_MR && (!is_kquant(wtype) || (KSQ_GEMV_DIRECT_KQ && wtype == kWQ4K && (nb & 7) == 0)) &&
               (nb & 1) == 0 && ((uintptr_t)W & 3) == 0 && ((uintptr_t)A & 3) == 0 && direct_mr_ktp(mr, nb) > 0 &&
               !(rpw == 4 && (N + 3) / 4 < 512);
    if (is_fq(amode) && mr >= 3)   // gemv_fused_profitable admitted it: one K tile, no grid exclusion
        return !is_kquant(wtype) && (nb & 1) == 0 && ((uintptr_t)W & 3) == 0 && direct_mr_ktp(mr, nb) == (nb >> 1);
    // Q6_K with 2 activation rows measured level with gemv_row_kernel (N = 14336, K = 4096: 17.3
    // vs 17.0 us), 1 row 13-18% faster; Q4_K 10-20% faster with 1 or 2
    if (is_kquant(wtype))
        return KSQ_GEMV_DIRECT_KQ && amode == kAL2 && mr <= (wtype == kWQ4K ? 2 : 1) && (nb & 7) == 0 &&
               ((uintptr_t)A & 3) == 0 && ((uintptr_t)W & (wtype == kWQ4K ? 3 : 1)) == 0;
    if (mr > 2 || (nb & 1) || ((uintptr_t)W & 3) || ((uintptr_t)A & 3)) return false;
    if (is_fq(amode)) return KSQ_GEMV_DIRECT_FQ && (size_t)mr * nb * kQ81Bytes <= kGemvLdsBudget;
    return amode == kAL2;
}

static hipError_t direct_dispatch(int wtype, int afmt, bool quant, bool xh, int mr, int rpw, const uint8_t* W,
                                  const void* A, float* C, int N, int nb, int ldc, int ldr, hipStream_t s) {
    if (mr >= 3 && wtype == kWQ4K) return direct_mr_launch<kWQ4K, false>(quant, false, mr, rpw, W, A, C, N, nb, N, 1, s);
    if (wtype == kWQ4K || wtype == kWQ6K) {
        const uint8_t* Aq = (const uint8_t*)A;
        const dim3 blk(256);
#define KSQ_KQ_LAUNCH(WT)                                                                                          \
    if (mr == 1) {                                                                                                 \
        if (rpw == 4) hipLaunchKernelGGL((gemv_direct_kq_kernel<WT, 1, 4>), dim3((N + 3) / 4), blk, 0, s, W, Aq, C, N, nb, N); \
        else if (rpw == 2) hipLaunchKernelGGL((gemv_direct_kq_kernel<WT, 1, 2>), dim3((N + 1) / 2), blk, 0, s, W, Aq, C, N, nb, N); \
        else hipLaunchKernelGGL((gemv_direct_kq_kernel<WT, 1, 1>), dim3(N), blk, 0, s, W, Aq, C, N, nb, N);          \
    } else {                                                                                                       \
        if (rpw == 4) hipLaunchKernelGGL((gemv_direct_kq_kernel<WT, 2, 4>), dim3((N + 3) / 4), blk, 0, s, W, Aq, C, N, nb, N); \
        else if (rpw == 2) hipLaunchKernelGGL((gemv_direct_kq_kernel<WT, 2, 2>), dim3((N + 1) / 2), blk, 0, s, W, Aq, C, N, nb, N); \
        else hipLaunchKernelGGL((gemv_direct_kq_kernel<WT, 2, 1>), dim3(N), blk, 0, s, W, Aq, C, N, nb, N);          \
    }
        if (wtype == kWQ4K) { KSQ_KQ_LAUNCH(kWQ4K) } else { KSQ_KQ_LAUNCH(kWQ6K) }
#undef KSQ_KQ_LAUNCH
        return hipGetLastError();
    }
    if (mr >= 3) {
        switch (wtype) {
            case kWQ40: return direct_mr_launch<kWQ40, false>(quant, xh, mr, rpw, W, A, C, N, nb, ldc, ldr, s);
            case kWQ80:
                return afmt == kAQ8S ? direct_mr_launch<kWQ80, true>(quant, xh, mr, rpw, W, A, C, N, nb, ldc, ldr, s)
                                     : direct_mr_launch<kWQ80, false>(quant, xh, mr, rpw, W, A, C, N, nb, ldc, ldr, s);
            case kWQ41: return direct_mr_launch<kWQ41, false>(quant, xh, mr, rpw, W, A, C, N, nb, ldc, ldr, s);
            case kWQ50: return direct_mr_launch<kWQ50, false>(quant, xh, mr, rpw, W, A, C, N, nb, ldc, ldr, s);
            default: return direct_mr_launch<kWQ51, false>(quant, xh, mr, rpw, W, A, C, N, nb, ldc, ldr, s);
        }
    }
    switch (wtype) {
        case kWQ40: return direct_launch<kWQ40, false>(quant, xh, mr, rpw, W, A, C, N, nb, ldc, ldr, s);
        case kWQ80:
            return afmt == kAQ8S ? direct_launch<kWQ80, true>(quant, xh, mr, rpw, W, A, C, N, nb, ldc, ldr, s)
                                 : direct_launch<kWQ80, false>(quant, xh, mr, rpw, W, A, C, N, nb, ldc, ldr, s);
        case kWQ41: return direct_launch<kWQ41, false>(quant, xh, mr, rpw, W, A, C, N, nb, ldc, ldr, s);
        case kWQ50: return direct_launch<kWQ50, false>(quant, xh, mr, rpw, W, A, C, N, nb, ldc, ldr, s);
        default: return direct_launch<kWQ51, false>(quant, xh, mr, rpw, W, A, C, N, nb, ldc, ldr, s);
    }
}

// QUANT: the activations are already quantised (kAL2 / kADMA by row count and length), else fp32 (kAFQ).
template <int AMODE>
static hipError_t gemv_dispatch_mode(int wtype, int afmt, int mr, const uint8_t* W, const void* Am, float* Cm,
                                     int N, int nb, int KT, int rpw, int ldc, int ldr,
                                     hipStream_t s) {
    switch (wtype) {
        case kWQ40: return row_launch_mr<kWQ40, AMODE, false>(mr, rpw, W, Am, Cm, N, nb, KT, ldc, ldr, s);
        case kWQ80:
            return (afmt == kAQ8S) ? row_launch_mr<kWQ80, AMODE, true>(mr, rpw, W, Am, Cm, N, nb, KT, ldc, ldr, s)
                                   : row_launch_mr<kWQ80, AMODE, false>(mr, rpw, W, Am, Cm, N, nb, KT, ldc, ldr, s);
        case kWQ4K: return row_launch_mr<kWQ4K, AMODE, false>(mr, rpw, W, Am, Cm, N, nb, KT, ldc, ldr, s);
        case kWQ6K: return row_launch_mr<kWQ6K, AMODE, false>(mr, rpw, W, Am, Cm, N, nb, KT, ldc, ldr, s);
        case kWQ41: return row_launch_mr<kWQ41, AMODE, false>(mr, rpw, W, Am, Cm, N, nb, KT, ldc, ldr, s);
        case kWQ50: return row_launch_mr<kWQ50, AMODE, false>(mr, rpw, W, Am, Cm, N, nb, KT, ldc, ldr, s);
        default: return row_launch_mr<kWQ51, AMODE, false>(mr, rpw, W, Am, Cm, N, nb, KT, ldc, ldr, s);
    }
}

// QUANT: pre-quantised activations; else fp32 (or fp16 with xh) quantised in every workgroup.
// Output element (m, n) at C[m * ldc + n * ldr].
template <bool QUANT>
static hipError_t gemv_dispatch(int wtype, int afmt, bool xh, const uint8_t* W, const void* A, float* C, int M, int N,
                                int K, int ldc, int ldr, hipStream_t s) {
    if (afmt == kAQ8S && (wtype != kWQ80 || xh)) return hipErrorNotSupported;
    const int nb = K / 32;
    if (M <= 0 || N <= 0 || nb == 0) return hipSuccess;
    const int chunk = (QUANT || M > kMaxFusedRows) ? 8 : kMaxFusedRows;
    for (int m0 = 0; m0 < M; m0 += chunk) {
        const int mr = (M - m0) < chunk ? (M - m0) : chunk;
        const int dma_min = mr == 1 ? kGemvDmaMinBlocks1 : kGemvDmaMinBlocks2;
        const int AMODE = !QUANT ? (xh ? kAFQH : kAFQ) : (mr <= kMaxL2Rows && nb < dma_min ? kAL2 : kADMA);
        // K tile: the whole row if it fits the LDS budget, else the largest multiple of 64 blocks
        const int rpw = pick_rpw(N, (is_fq(AMODE) && mr > kMaxFusedRows) ? kADMA : AMODE);
        int KT = (nb + 7) & ~7;
        while (KT > 64 && gemv_lds_bytes(wtype, mr, KT, AMODE, rpw) > kGemvLdsBudget) KT = ((KT / 2) + 63) & ~63;
        const void* Am = QUANT ? (const void*)((const uint8_t*)A + (size_t)m0 * nb * kQ81Bytes)
                       : xh    ? (const void*)((const uint16_t*)A + (size_t)m0 * K)
                               : (const void*)((const float*)A + (size_t)m0 * K);
        float* Cm = C + (size_t)m0 * ldc;
        hipError_t e;
        if (direct_eligible(wtype, AMODE, mr, nb, N, rpw, W, Am)) {
            note_engine(is_kquant(wtype) && mr <= 2 ? KSQ_ENG_GEMV_KQ
                        : mr >= 3 ? (QUANT ? KSQ_ENG_GEMV_MR : KSQ_ENG_GEMV_MR_FQ)
                                  : (QUANT ? KSQ_ENG_GEMV_DIRECT : KSQ_ENG_GEMV_DIRECT_FQ));
            // the K-quant multi-row form writes a row-major output only
            if (mr >= 3 && QUANT && wtype == kWQ4K && (ldc != N || ldr != 1)) return hipErrorNotSupported;
            e = direct_dispatch(wtype, afmt, QUANT, xh, mr, rpw, W, Am, Cm, N, nb, ldc, ldr, s);
        } else {
            note_engine(is_fq(AMODE) ? KSQ_ENG_GEMV_ROW_FQ : KSQ_ENG_GEMV_ROW);
            if (AMODE == kAL2) e = gemv_dispatch_mode<kAL2>(wtype, afmt, mr, W, Am, Cm, N, nb, KT, rpw, ldc, ldr, s);
            else if (AMODE == kADMA) e = gemv_dispatch_mode<kADMA>(wtype, afmt, mr, W, Am, Cm, N, nb, KT, rpw, ldc, ldr, s);
            else if (AMODE == kAFQH) e = gemv_dispatch_mode<kAFQH>(wtype, afmt, mr, W, Am, Cm, N, nb, KT, rpw, ldc, ldr, s);
            else e = gemv_dispatch_mode<kAFQ>(wtype, afmt, mr, W, Am, Cm, N, nb, KT, rpw, ldc, ldr, s);
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_gemv(int wtype, int afmt, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int K,
                       hipStream_t s) {
    return gemv_dispatch<true>(wtype, afmt, false, W, A, C, M, N, K, N, 1, s);
}

hipError_t launch_gemv_strided(int wtype, int afmt, const uint8_t* W, const uint8_t* A, float* C, int M, int N,
                               int K, int ldc, int ldr, hipStream_t s) {
    return gemv_dispatch<true>(wtype, afmt, false, W, A, C, M, N, K, ldc, ldr, s);
}

// The in-workgroup quantisation is repeated by every workgroup; it beats the separate quantise
// launch while that repeated work stays small (measured crossover: between 4.0e5 and 4.6e5
// block quantisations, e.g. N = K = 7168 fused is faster, N = 14336, K = 4096 is not).
#ifndef KSQ_GEMV_FUSED_MAX_WORK
#define KSQ_GEMV_FUSED_MAX_WORK 420000ll
#endif
#ifndef KSQ_GEMV_FUSED_MR_MAX_WORK
#define KSQ_GEMV_FUSED_MR_MAX_WORK 200000ll
#endif

bool gemv_fused_profitable(int wtype, int M, int N, int K, const void* W, bool xh) {
    if (M < 1 || M > 8) return false;
#ifndef KSQ_GEMV_FUSED_MR
#define KSQ_GEMV_FUSED_MR 1
#endif
    if (M > kMaxFusedRows) {
        if (!KSQ_GEMV_FUSED_MR) return false;
        // 3-8 rows: gemv_direct_mr_kernel quantising its single K tile, where the quantised path
        // would take the decode kernel too (not the small-batch kernel), while the repeated work
        // stays under 2e5 block quantisations (measured: Q4_0 N = 512, K = 7168, M = 3 7.0 -> 6.4
        // us at 1.7e5; N = K = 4096, M = 3 9.3 -> 10.3 the other way at 3.9e5)
        const int nb = K / 32;
        if (is_kquant(wtype) || (nb & 1) || ((uintptr_t)W & 3) || direct_mr_ktp(M, nb) != (nb >> 1)) return false;
        if (skinny_preferred(wtype, M, N, K)) return false;
        int rpw = pick_rpw(N, kADMA);
        if (rpw == 4 && M <= 5 && nb >= 384 && (N + 7) / 8 >= kGemvMinWGs) rpw = 8;
        const long long wgs = (N + rpw - 1) / rpw;
        return (long long)M * wgs * nb <= KSQ_GEMV_FUSED_MR_MAX_WORK;
    }
    const int rpw = pick_rpw(N, kAFQ);
    const int nb = K / 32, KT = (nb + 7) & ~7;
    // one K tile only: with several, each tile's quantisation would wait for the previous tile
    // (the register-direct form stages only the activation rows, for 4-byte aligned weights)
    const bool direct = !is_kquant(wtype) && (nb & 1) == 0 && (size_t)M * nb * kQ81Bytes <= kGemvLdsBudget;
    if (!direct && gemv_lds_bytes(wtype, M, KT, kAFQ, rpw) > kGemvLdsBudget) return false;
    const long long wgs = (N + rpw - 1) / rpw;
    return (long long)M * wgs * nb <= KSQ_GEMV_FUSED_MAX_WORK;
}

hipError_t launch_gemv_f32(int wtype, int afmt, const uint8_t* W, const float* X, float* C, int M, int N, int K,
                           hipStream_t s) {
    return gemv_dispatch<false>(wtype, afmt, false, W, X, C, M, N, K, N, 1, s);
}

hipError_t launch_gemv_fused(int wtype, int afmt, bool xh, const uint8_t* W, const void* X, float* C, int M, int N,
                             int K, int ldc, int ldr, hipStream_t s) {
    return gemv_dispatch<false>(wtype, afmt, xh, W, X, C, M, N, K, ldc, ldr, s);
}

// ---- block_q8f decode (the deepseek_v2 / lm_head operators at 1-2 activation rows) ----------
template <int WT, int MR, int QF>
static hipError_t q8f_launch_rpw(int rpw, const uint8_t* W, const float* X, float* C, int N, int nb, hipStream_t s) {
    const dim3 blk(256);
    const size_t lds = (size_t)MR * nb * 40;
    switch (rpw) {
        case 8: hipLaunchKernelGGL((gemv_direct_fq_kernel<WT, MR, false, 8, false, QF>), dim3((N + 7) / 8), blk, lds, s, W, X, C, N, nb, N, 1); break;
        case 4: hipLaunchKernelGGL((gemv_direct_fq_kernel<WT, MR, false, 4, false, QF>), dim3((N + 3) / 4), blk, lds, s, W, X, C, N, nb, N, 1); break;
        case 2: hipLaunchKernelGGL((gemv_direct_fq_kernel<WT, MR, false, 2, false, QF>), dim3((N + 1) / 2), blk, lds, s, W, X, C, N, nb, N, 1); break;
        default: hipLaunchKernelGGL((gemv_direct_fq_kernel<WT, MR, false, 1, false, QF>), dim3(N), blk, lds, s, W, X, C, N, nb, N, 1); break;
    }
    return hipGetLastError();
}

template <int WT, int QF>
static hipError_t q8f_launch(int M, int rpw, const uint8_t* W, const float* X, float* C, int N, int nb, hipStream_t s) {
    return M == 1 ? q8f_launch_rpw<WT, 1, QF>(rpw, W, X, C, N, nb, s) : q8f_launch_rpw<WT, 2, QF>(rpw, W, X, C, N, nb, s);
}

// The fused decode kernel applies: 1-2 rows of a Q4_0 / Q5_0 / Q8_0 matrix with an even block
// count, dword-aligned weights, the rows' block_q8f blocks within the LDS budget, and the work
// the workgroups repeat (every one quantises the rows) under the fused kernels' limit.  The MFMA
// GEMM with split-K took 2.4x as long at M = 1 (N = K = 5120: 17.2 us; the block_q8_1 fused path
// 7.0 us on the same box).
bool gemv_q8f_profitable(int wtype, int M, int N, int K, const void* W) {
    if (M < 1 || M > 2 || !(wtype == kWQ40 || wtype == kWQ50 || wtype == kWQ80)) return false;
    const int nb = K / 32;
    if ((nb & 1) || ((uintptr_t)W & 3) || (size_t)M * nb * 40 > kGemvLdsBudget) return false;
    const int rpw = pick_rpw(N, kAFQ);
    return (long long)M * ((N + rpw - 1) / rpw) * nb <= KSQ_GEMV_FUSED_MAX_WORK;
}

hipError_t launch_gemv_q8f(int rule, int wtype, const uint8_t* W, const float* X, float* C, int M, int N, int K,
                           hipStream_t s) {
    if (!gemv_q8f_profitable(wtype, M, N, K, W) || (rule != kQ8FRne && rule != kQ8FLround)) return hipErrorNotSupported;
    const int nb = K / 32, rpw = pick_rpw(N, kAFQ);
    note_engine(KSQ_ENG_GEMV_DIRECT_FQ);
    switch (wtype) {
        case kWQ40: return rule == kQ8FRne ? q8f_launch<kWQ40, 1>(M, rpw, W, X, C, N, nb, s)
                                           : q8f_launch<kWQ40, 2>(M, rpw, W, X, C, N, nb, s);
        case kWQ50: return rule == kQ8FRne ? q8f_launch<kWQ50, 1>(M, rpw, W, X, C, N, nb, s)
                                           : q8f_launch<kWQ50, 2>(M, rpw, W, X, C, N, nb, s);
        default: return rule == kQ8FRne ? q8f_launch<kWQ80, 1>(M, rpw, W, X, C, N, nb, s)
                                        : q8f_launch<kWQ80, 2>(M, rpw, W, X, C, N, nb, s);
    }
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

// Calibration: a plain streaming read of `bytes` (16-byte aligned, a multiple of 16) with the
// decode kernels' load width.  Workgroup g reads the per16 16-byte words from g * per16 (per16 a
// multiple of 256) in rounds of 8 loads per thread, XOR-folding what it read into one word of
// out (so the loads cannot be elided).
constexpr int kReadBytesPerWG = 32768;

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ p, int64_t n16, int64_t per16,
                                                          uint32_t* __restrict__ out) {
    const int64_t beg = (int64_t)blockIdx.x * per16;
    const int64_t end = beg + per16 < n16 ? beg + per16 : n16;
    uint32_t x = 0;
    for (int64_t k0 = beg; k0 < end; k0 += 8 * 256) {
        u32x4 v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int64_t k = k0 + i * 256 + threadIdx.x;
            v[i] = k < end ? p[k] : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < 8; i++) x ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
    for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
    __shared__ uint32_t red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

size_t stream_read_outputs(size_t bytes, size_t wg_bytes) { return (bytes + wg_bytes - 1) / wg_bytes; }

hipError_t launch_stream_read(const void* p, size_t bytes, size_t wg_bytes, uint32_t* out, hipStream_t s) {
    const int64_t n16 = (int64_t)(bytes / 16);
    const size_t grid = stream_read_outputs(bytes, wg_bytes);
    if (grid == 0) return hipSuccess;
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)grid), dim3(256), 0, s, (const u32x4*)p, n16,
                       (int64_t)(wg_bytes / 16), out);
    return hipGetLastError();
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
