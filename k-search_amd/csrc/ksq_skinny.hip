// ksq_skinny.hip - small-batch GEMM: up to 8 activation rows on the 4x4x4 int8 MFMA, 9-32 rows on the
// 16x16x32 int8 MFMA (skinny16_kernel, below).
//
// Reference path: the decode GEMVs of kernelevalplus-main/kernels/gemm/gemm_warp_optimized.cuh:108-1212
// run with batch > 1 (one warp per weight row, DP4A per activation row) and the block formulas of
// include/gemm_reference.h:200-259 and include/gemm_quant_formats.cuh:126-266.
//
// gfx950 design:
//  * v_mfma_i32_4x4x4_16b_i8 computes 16 independent 4 x 4 x 4 int8 products.  Lane
//    l = 16 g + 4 kb + q: product (g, kb) is weight rows 4g .. 4g+3 x activation rows q of block
//    kb of the current K step; the lane supplies weight row 4g + q and activation row q of that
//    block.  Eight instructions (k = 0..31) leave the reference's integer block dot sumi of
//    4 weight rows x 4 activation rows in every lane's four result registers, for 16 rows x
//    4 blocks per wave and step; activation rows 4..7 take a second set of eight.  The
//    activation fragment is used by all 16 rows, so the integer work per (row, block, column)
//    is 1/16 of an MFMA issue slot instead of the 8 v_dot4 of the decode kernel.
//  * A workgroup owns 16 weight rows and its waves split the K steps (4 blocks each).  Lanes
//    load their weight block and activation block straight from global memory into registers
//    kSkPD steps ahead of the MFMAs (the 16 rows x 4 blocks of one step are 16 contiguous runs
//    of 4 blocks), so each wave keeps several KB in flight with no LDS staging and no barrier
//    in the K loop.  The loads are bounds-checked buffer loads: blocks past K and activation
//    rows past M read zeros without branches.
//  * Per-block epilogue as the MFMA GEMM: the MFMA accumulates onto the bit pattern of
//    12582912.0f, X = fma(f, d_a, -12582912 d_a) = d_a * sumi with one rounding; the four weight
//    rows' scales come from the lanes of the quad by DPP broadcast.
//  * The 4 blocks of a step are summed over lanes by DPP row rotation once at the end, the
//    waves' K ranges through LDS.
#include "ksq_device.h"
#include "ksq_internal.h"

namespace ksq {

namespace {

constexpr uint32_t kSkMagic = 0x4B400000u;  // 12582912.0f
constexpr float kSkMagicF = 12582912.0f;
constexpr int kSkRows = 16;                 // weight rows per workgroup
constexpr int kSkPD2 = 4;                   // K steps in flight per wave (up to 8 rows)

// Per-lane weight registers of one block: the WD dwords from the 4-byte aligned address at or
// below the block start (Q4_0 18 B, Q8_0 34 B and Q5_0 22 B blocks are only 2-byte aligned; the
// window covers the block wherever it starts).  NP payload dwords follow the fp16 scale(s).
template <int WT>
struct SkFmt {
    static constexpr bool al4 = (WT == kWQ41 || WT == kWQ51);
    static constexpr int BB = block_bytes(WT);
    static constexpr int WD = (BB + (al4 ? 3 : 5)) / 4;
    static constexpr int NP = (WT == kWQ80) ? 8 : (WT == kWQ50 || WT == kWQ51) ? 5 : 4;  // payload dwords
};

constexpr uint32_t kOOB = 0x80000000u;  // buffer offset past every buffer this kernel reads: loads give 0

// ND consecutive dwords at byte offset off of the buffer (dword aligned), as 16-byte loads
// plus one 4-, 8- or 12-byte load.
template <int ND>
__device__ __forceinline__ void buf_load(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t* out) {
#pragma unroll
    for (int i = 0; i + 4 <= ND; i += 4) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 4 * i, 0, 0);
        out[i] = v.x; out[i + 1] = v.y; out[i + 2] = v.z; out[i + 3] = v.w;
    }
    constexpr int R = ND & 3, B = ND - R;
    if constexpr (R == 1) {
        out[B] = __builtin_amdgcn_raw_buffer_load_b32(r, off + 4 * B, 0, 0);
    } else if constexpr (R == 2) {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off + 4 * B, 0, 0);
        out[B] = v.x; out[B + 1] = v.y;
    } else if constexpr (R == 3) {
        typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
        const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(r, off + 4 * B, 0, 0);
        out[B] = v.x; out[B + 1] = v.y; out[B + 2] = v.z;
    }
}

// One weight block from its load window (F::WD dwords from the 4-byte aligned address at or below
// the block start, sh = the block start's byte offset in the first dword): the fp16 scale (and
// min), and the 32 quants as int8 in 8 dwords (elements 4j .. 4j+3 in a8[j]; the nibble types'
// 0..15 / 0..31 codes, whose offsets the block formula carries).
template <int WT>
__device__ __forceinline__ void sk_unpack(const uint32_t* w, int sh, uint32_t (&a8)[8], float& dw, float& mw) {
    using F = SkFmt<WT>;
    uint32_t pay[F::NP];
    mw = 0.0f;
    if constexpr (F::al4) {
        dw = f16_to_f32(w[0] & 0xFFFFu);
        mw = f16_to_f32(w[0] >> 16);
#pragma unroll
        for (int i = 0; i < F::NP; i++) pay[i] = w[1 + i];
    } else {
        // d at byte sh of the window, the payload from byte sh + 2 (2 or 4)
        dw = f16_to_f32((w[0] >> (8 * sh)) & 0xFFFFu);
#pragma unroll
        for (int i = 0; i < F::NP; i++) pay[i] = sh ? w[i + 1] : __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
    }
    if constexpr (WT == kWQ80) {
#pragma unroll
        for (int j = 0; j < 8; j++) a8[j] = pay[j];
    } else if constexpr (WT == kWQ40 || WT == kWQ41) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            a8[j] = pay[j] & 0x0F0F0F0Fu;
            a8[4 + j] = (pay[j] >> 4) & 0x0F0F0F0Fu;
        }
    } else {
        const uint32_t h = pay[0];  // qh: bit e = bit 4 of element e
#pragma unroll
        for (int j = 0; j < 4; j++) {
            a8[j] = (pay[1 + j] & 0x0F0F0F0Fu) | qh_to_bit4(h >> (4 * j));
            a8[4 + j] = ((pay[1 + j] >> 4) & 0x0F0F0F0Fu) | qh_to_bit4(h >> (16 + 4 * j));
        }
    }
}

__device__ __forceinline__ float dpp_quad_bcast(float v, int r) {
    const int x = __builtin_bit_cast(int, v);
    int y;
    switch (r) {
        case 0: y = __builtin_amdgcn_mov_dpp(x, 0x00, 0xF, 0xF, false); break;
        case 1: y = __builtin_amdgcn_mov_dpp(x, 0x55, 0xF, 0xF, false); break;
        case 2: y = __builtin_amdgcn_mov_dpp(x, 0xAA, 0xF, 0xF, false); break;
        default: y = __builtin_amdgcn_mov_dpp(x, 0xFF, 0xF, 0xF, false); break;
    }
    return __builtin_bit_cast(float, y);
}

__device__ __forceinline__ float dpp_row_ror(float v, int n) {
    const int x = __builtin_bit_cast(int, v);
    const int y = (n == 4) ? __builtin_amdgcn_mov_dpp(x, 0x124, 0xF, 0xF, false)
                           : __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false);
    return __builtin_bit_cast(float, y);
}

// C[m][n] = sum over blocks of the reference block formula, m < M <= 4*MP, for the 16 rows
// n0 .. n0+15 of this workgroup.  NWV waves split the K steps.  AS: block_q8s activations
// (Q8_0 weights only).  wbytes / abytes: readable bytes of W and A (W's rounded up to a dword:
// the last dword of the weights is read whole).  Loads are buffer loads: a block past K or an
// activation row past M reads at an offset beyond the buffer and gets zeros.
// AL (K % 128 == 0, A 16-byte aligned): a step's activation blocks (4 MP rows x 4 blocks, 36 MP
// 16-byte pieces) are loaded once per wave, one piece per lane, and exchanged through the wave's
// LDS region, instead of every lane loading its 9 dwords (each block then came through 4 lanes:
// removing the activation traffic altogether took Q8_0 N = K = 4096, M = 8 from 9.8 to 7.0 us).
template <int WT, int MP, bool AS, int NWV, bool AL = false>
__global__ __launch_bounds__(64 * NWV) void skinny_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ A,
                                                          float* __restrict__ C, int M, int N, int nb, int ldc,
                                                          uint32_t wbytes, uint32_t abytes) {
    using F = SkFmt<WT>;
    constexpr int BB = F::BB;
    constexpr int AP = 36 * MP;                  // activation pieces of 16 bytes per step (AL)
    constexpr int APL = (AP + 63) / 64;          // pieces per lane
    __shared__ float red[NWV][kSkRows][4 * MP];
    __shared__ __attribute__((aligned(16))) uint32_t sact[AL ? NWV : 1][AL ? 4 * AP : 4];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, kb = (lane >> 2) & 3, q = lane & 3;
    const int n0 = blockIdx.x * kSkRows;
    const int wrow = min(n0 + 4 * g + q, N - 1);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, (int)wbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, (int)abytes, 0x00020000);
    // this lane's block starts at row offset + (4 s + kb) * BB; its offset mod 4 is the same at
    // every step, since a step advances 4 blocks
    const uint32_t wrow_off = (uint32_t)wrow * (uint32_t)nb * (uint32_t)BB + (uint32_t)kb * BB;
    const int sh = (int)(((uintptr_t)W + wrow_off) & 3u);   // block start within its dword (0 or 2)
    uint32_t aoff0[MP];
#pragma unroll
    for (int pp = 0; pp < MP; pp++) {
        const int m = q + 4 * pp;
        aoff0[pp] = m < M ? ((uint32_t)m * (uint32_t)nb + (uint32_t)kb) * (uint32_t)kQ81Bytes : kOOB;
    }
    // AL: piece p = lane + 64 i of a step is bytes 16 (p % 9) .. of activation row p / 9's 4 blocks
    uint32_t poff0[APL];
#pragma unroll
    for (int i = 0; i < APL; i++) {
        const int p = lane + 64 * i, row = p / 9;
        poff0[i] = (p < AP && row < M) ? (uint32_t)row * (uint32_t)nb * (uint32_t)kQ81Bytes + 16u * (uint32_t)(p % 9)
                                       : kOOB;
    }

    const int S = (nb + 3) >> 2;
    const int s_lo = (int)((long long)S * wave / NWV), s_hi = (int)((long long)S * (wave + 1) / NWV);

    i32x4 bias;
#pragma unroll
    for (int r = 0; r < 4; r++) bias[r] = (int)kSkMagic;
    float acc[MP][4];
#pragma unroll
    for (int p = 0; p < MP; p++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[p][r] = 0.0f;

    struct Step {
        uint32_t w[F::WD];
        uint32_t a[AL ? 1 : MP][9];
        u32x4 ap[AL ? APL : 1];
    };
    auto load = [&](int s, Step& st) {
        const bool bok = 4 * s + kb < nb;
        const uint32_t woff = bok ? wrow_off + (uint32_t)(4 * s) * BB - (uint32_t)sh : kOOB;
        buf_load<F::WD>(rw, woff, st.w);
        if constexpr (AL) {
#pragma unroll
            for (int i = 0; i < APL; i++)
                st.ap[i] = __builtin_amdgcn_raw_buffer_load_b128(
                    ra, poff0[i] == kOOB ? kOOB : poff0[i] + (uint32_t)(4 * s) * kQ81Bytes, 0, 0);
        } else {
#pragma unroll
            for (int pp = 0; pp < MP; pp++) {
                const uint32_t aoff = bok ? aoff0[pp] + (uint32_t)(4 * s) * kQ81Bytes : kOOB;
                buf_load<9>(ra, aoff, st.a[pp]);
            }
        }
    };
    uint32_t* sap = &sact[AL ? wave : 0][0];

    auto compute = [&](const Step& st) {
        // AL: the wave's step pieces into its LDS region, then every lane's activation blocks
        if constexpr (AL) {
            wave_lds_exchange();   // the previous step's reads come first
#pragma unroll
            for (int i = 0; i < APL; i++)
                if (lane + 64 * i < AP) *(u32x4*)&sap[4 * (lane + 64 * i)] = st.ap[i];
            wave_lds_exchange();   // every lane reads pieces other lanes wrote (per pass, below)
        }
        // weight scale(s) and the 8 A-operand dwords (elements 4j .. 4j+3)
        float dw, mw;
        uint32_t a8[8];
        sk_unpack<WT>(st.w, sh, a8, dw, mw);
        float dwr[4], mwr[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
            dwr[r] = dpp_quad_bcast(dw, r);
            if constexpr (WT == kWQ41 || WT == kWQ51) mwr[r] = dpp_quad_bcast(mw, r);
        }
#pragma unroll
        for (int pp = 0; pp < MP; pp++) {
            if (pp * 4 >= M) break;  // uniform: no activation rows in this pass
            i32x4 d = bias;
            uint32_t al[9];
            if constexpr (AL) {
#pragma unroll
                for (int i = 0; i < 9; i++) al[i] = sap[(q + 4 * pp) * 36 + kb * 9 + i];
            }
            const uint32_t* av = AL ? al : st.a[AL ? 0 : pp];
#pragma unroll
            for (int j = 0; j < 8; j++)
                d = __builtin_amdgcn_mfma_i32_4x4x4i8((int)a8[j], (int)av[1 + j], d, 0, 0, 0);
            const uint32_t ds = av[0];
            // block_q8s: fp32 scale with its two lowest mantissa bits cleared so that
            // 12582912 * d_a stays exact (relative change < 2^-21)
            const float da = AS ? __builtin_bit_cast(float, ds & ~3u) : f16_to_f32(ds & 0xFFFFu);
            const float sa = AS ? 0.0f : f16_to_f32(ds >> 16);
            const float nc = -kSkMagicF * da;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int e = d[r];
                const float X = fmaf(__builtin_bit_cast(float, e), da, nc);  // d_a * sumi
                if constexpr (WT == kWQ40) acc[pp][r] = fmaf(dwr[r], fmaf(-8.0f, sa, X), acc[pp][r]);
                else if constexpr (WT == kWQ50) acc[pp][r] = fmaf(dwr[r], fmaf(-16.0f, sa, X), acc[pp][r]);
                else if constexpr (WT == kWQ80) acc[pp][r] = fmaf(dwr[r], X, acc[pp][r]);
                else acc[pp][r] = fmaf(mwr[r], sa, fmaf(dwr[r], X, acc[pp][r]));
            }
        }
    };

    // PD steps in flight (wave-uniform branches only)
    constexpr int kSkPD = MP <= 2 ? kSkPD2 : 2;
    Step buf[kSkPD];
#pragma unroll
    for (int d = 0; d < kSkPD; d++)
        if (s_lo + d < s_hi) load(s_lo + d, buf[d]);
    for (int s0 = s_lo; s0 < s_hi; s0 += kSkPD) {
#pragma unroll
        for (int d = 0; d < kSkPD; d++) {
            if (s0 + d < s_hi) {
                compute(buf[d]);
                if (s0 + d + kSkPD < s_hi) load(s0 + d + kSkPD, buf[d]);
            }
        }
    }

    // sum the 4 blocks of a step (lanes kb = 0..3 of a 16-lane row), then the waves
#pragma unroll
    for (int pp = 0; pp < MP; pp++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float v = acc[pp][r];
            v += dpp_row_ror(v, 4);
            v += dpp_row_ror(v, 8);
            acc[pp][r] = v;
        }
    if (kb == 0) {
#pragma unroll
        for (int pp = 0; pp < MP; pp++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[wave][4 * g + r][q + 4 * pp] = acc[pp][r];
    }
    __syncthreads();
    const int t = threadIdx.x;
    if (t < kSkRows * 4 * MP) {
        const int row = t % kSkRows, m = t / kSkRows;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NWV; w++) v += red[w][row][m];
        if (m < M && n0 + row < N) C[(size_t)m * ldc + n0 + row] = v;
    }
}

// 9-32 activation rows on the 16x16x32 int8 MFMA (one issue per block, weight rows x 16
// activation rows, in place of 4 activation rows per 4x4x4 pass).  Lane l = 16 c + r loads block
// c of the step for weight row r (the skinny_kernel's loads: 16 contiguous 4-block runs per
// instruction), and the MFMA wants lane l to hold dwords 2c, 2c+1 of one block for every
// 16-lane row c: the 4 x 4 lane-row x dword-pair transpose is two swap stages, v_permlane32_swap
// (the off-diagonal 2 x 2 blocks of lane rows 0-1 / 2-3) and v_permlane16_swap (inside each),
// 8 swaps per lane and step.  The activation pieces are shared through the wave's LDS region as
// in skinny_kernel; the MFMA's B operand (activation row r of the half, dwords 2c, 2c+1) and the
// result rows (weight rows 4c .. 4c+3 x activation row r) read their scales from there and from
// the wave's weight-scale slots.  MH halves of 16 activation rows.  Requires K % 128 == 0 and a
// 16-byte aligned A (the shared pieces); every other rule is skinny_kernel's.
// WST (16-byte aligned W): the step's 16 weight-row runs are loaded as 16-byte aligned chunks
// (one coalesced segment per row, ~2.5x fewer cache lines touched per load instruction than the
// per-lane block windows) into the wave's LDS region, and each lane reads its block window from
// there; the loads, not the MFMA or LDS work, bound this kernel (per-wave timestamps: each K
// step ~1.2-1.4 us, ~4x its compute).
template <int WT, bool AS, int MH, int NWV, bool WST = false>
__global__ __launch_bounds__(64 * NWV) void skinny16_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ A,
                                                            float* __restrict__ C, int M, int N, int nb, int ldc,
                                                            uint32_t wbytes, uint32_t abytes) {
    using F = SkFmt<WT>;
    constexpr int BB = F::BB;
    constexpr int AR = 16 * MH;                  // activation rows of the step pieces
    constexpr int AP = 9 * AR;                   // 16-byte pieces per step (4 blocks of 36 bytes a row)
    constexpr int APL = (AP + 63) / 64;
    constexpr bool MIN = (WT == kWQ41 || WT == kWQ51);
    constexpr int RED = NWV * kSkRows * AR;      // floats of the cross-wave sum
    __shared__ __attribute__((aligned(16))) uint32_t sact[NWV * 4 * AP > RED ? NWV * 4 * AP : RED];
    __shared__ __attribute__((aligned(16))) float swd[NWV][MIN ? 2 : 1][4][kSkRows];
    // WST: the step's weight rows as 16-byte aligned chunks (RUN bytes of a row at any even offset)
    // rows RS dwords apart: 4 WCH + 4 puts the 16 rows' window reads 2 to a bank instead of 4
    // (Q8_0 M = 32: 10.66 -> 10.45 us, M = 16 8.1 -> 7.8)
    constexpr int RUN = 4 * BB, WCH = (RUN + 14 + 15) / 16, WQ = kSkRows * WCH, WQL = (WQ + 63) / 64;
    constexpr int RS = 4 * WCH + 4;
    __shared__ __attribute__((aligned(16))) uint32_t swc[WST ? NWV : 1][WST ? kSkRows * RS : 4];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane >> 4, r = lane & 15;
    const int n0 = blockIdx.x * kSkRows;
    const int wrow = min(n0 + r, N - 1);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, (int)wbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, (int)abytes, 0x00020000);
    const uint32_t wrow_off = (uint32_t)wrow * (uint32_t)nb * (uint32_t)BB + (uint32_t)c * BB;
    const int sh = (int)(((uintptr_t)W + wrow_off) & 3u);
    // WST: this lane's row start, and the chunk (row q / WCH, byte 16 (q % WCH) of the row's run)
    // each of its loads brings in, q = lane + 64 i (-1: no chunk)
    const uint32_t rs_own = (uint32_t)wrow * (uint32_t)nb * (uint32_t)BB;
    uint32_t wrs[WST ? WQL : 1];
    int wch[WST ? WQL : 1];
    if constexpr (WST) {
#pragma unroll
        for (int i = 0; i < WQL; i++) {
            const int q = lane + 64 * i, row = q / WCH;
            wrs[i] = (uint32_t)min(n0 + min(row, kSkRows - 1), N - 1) * (uint32_t)nb * (uint32_t)BB;
            wch[i] = q < WQ ? 16 * (q % WCH) : -1;
        }
    }
    uint32_t poff0[APL];
#pragma unroll
    for (int i = 0; i < APL; i++) {
        const int p = lane + 64 * i, row = p / 9;
        poff0[i] = (p < AP && row < M) ? (uint32_t)row * (uint32_t)nb * (uint32_t)kQ81Bytes + 16u * (uint32_t)(p % 9)
                                       : kOOB;
    }
    const int S = nb >> 2;
    const int s_lo = (int)((long long)S * wave / NWV), s_hi = (int)((long long)S * (wave + 1) / NWV);

    i32x4 bias;
#pragma unroll
    for (int q = 0; q < 4; q++) bias[q] = (int)kSkMagic;
    float acc[MH][4];
#pragma unroll
    for (int h = 0; h < MH; h++)
#pragma unroll
        for (int q = 0; q < 4; q++) acc[h][q] = 0.0f;

    struct Step {
        uint32_t w[WST ? 1 : F::WD];
        u32x4 wc[WST ? WQL : 1];
        u32x4 ap[APL];
    };
    auto load = [&](int s, Step& st) {
        if constexpr (WST) {
#pragma unroll
            for (int i = 0; i < WQL; i++)
                st.wc[i] = __builtin_amdgcn_raw_buffer_load_b128(
                    rw, wch[i] >= 0 ? ((wrs[i] + (uint32_t)(RUN * s)) & ~15u) + (uint32_t)wch[i] : kOOB, 0, 0);
        } else {
            const bool bok = 4 * s + c < nb;
            buf_load<F::WD>(rw, bok ? wrow_off + (uint32_t)(4 * s) * BB - (uint32_t)sh : kOOB, st.w);
        }
#pragma unroll
        for (int i = 0; i < APL; i++)
            st.ap[i] = __builtin_amdgcn_raw_buffer_load_b128(
                ra, poff0[i] == kOOB ? kOOB : poff0[i] + (uint32_t)(4 * s) * kQ81Bytes, 0, 0);
    };
    uint32_t* sap = &sact[wave * 4 * AP];

    auto compute = [&](const Step& st, int s) {
        float dw, mw;
        uint32_t a8[8];
        wave_lds_exchange();   // the previous step's reads come first
        if constexpr (WST) {
#pragma unroll
            for (int i = 0; i < WQL; i++)
                if (wch[i] >= 0) {
                    const int q = lane + 64 * i;
                    *(u32x4*)&swc[wave][(q / WCH) * RS + 4 * (q % WCH)] = st.wc[i];
                }
            wave_lds_exchange();
            const uint32_t o = ((rs_own + (uint32_t)(RUN * s)) & 15u) + (uint32_t)(BB * c);
            const uint32_t* wp = &swc[wave][r * RS + (o >> 2)];
            uint32_t wv[F::WD];
#pragma unroll
            for (int i = 0; i < F::WD; i++) wv[i] = wp[i];
            sk_unpack<WT>(wv, (int)(o & 3u), a8, dw, mw);
        } else {
            sk_unpack<WT>(st.w, sh, a8, dw, mw);
        }
#pragma unroll
        for (int i = 0; i < APL; i++)
            if (lane + 64 * i < AP) *(u32x4*)&sap[4 * (lane + 64 * i)] = st.ap[i];
        swd[wave][0][c][r] = dw;
        if constexpr (MIN) swd[wave][1][c][r] = mw;
        wave_lds_exchange();
        // x[j] = dwords 2j, 2j+1 of this lane's block (lane row c = block c): after the transpose
        // x[k] of lane row c holds dwords 2c, 2c+1 of block k (for this lane's weight row)
        uint32_t x[4][2];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            x[j][0] = a8[2 * j];
            x[j][1] = a8[2 * j + 1];
        }
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const auto v = __builtin_amdgcn_permlane32_swap(x[j][e], x[j + 2][e], false, false);
                x[j][e] = v[0];
                x[j + 2][e] = v[1];
            }
#pragma unroll
        for (int j = 0; j < 4; j += 2)
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const auto v = __builtin_amdgcn_permlane16_swap(x[j][e], x[j + 1][e], false, false);
                x[j][e] = v[0];
                x[j + 1][e] = v[1];
            }
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const long wa = (long)(((uint64_t)x[k][1] << 32) | x[k][0]);
            const f32x4 dwr = *(const f32x4*)&swd[wave][0][k][4 * c];
            f32x4 mwr;
            if constexpr (MIN) mwr = *(const f32x4*)&swd[wave][1][k][4 * c];
#pragma unroll
            for (int h = 0; h < MH; h++) {
                const uint32_t* ab = &sap[(16 * h + r) * 36 + 9 * k];
                const long bv = (long)(((uint64_t)ab[2 + 2 * c] << 32) | ab[1 + 2 * c]);
                const i32x4 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(wa, bv, bias, 0, 0, 0);
                const uint32_t ds = ab[0];
                const float da = AS ? __builtin_bit_cast(float, ds & ~3u) : f16_to_f32(ds & 0xFFFFu);
                const float sa = AS ? 0.0f : f16_to_f32(ds >> 16);
                const float nc = -kSkMagicF * da;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int e = d[q];
                    const float X = fmaf(__builtin_bit_cast(float, e), da, nc);  // d_a * sumi
                    if constexpr (WT == kWQ40) acc[h][q] = fmaf(dwr[q], fmaf(-8.0f, sa, X), acc[h][q]);
                    else if constexpr (WT == kWQ50) acc[h][q] = fmaf(dwr[q], fmaf(-16.0f, sa, X), acc[h][q]);
                    else if constexpr (WT == kWQ80) acc[h][q] = fmaf(dwr[q], X, acc[h][q]);
                    else acc[h][q] = fmaf(mwr[q], sa, fmaf(dwr[q], X, acc[h][q]));
                }
            }
        }
    };

    // one step in flight per wave: a second (loaded under the current step's MFMAs) needs ~30 more
    // VGPRs per lane, and at 8 waves the kernel was 2-15% slower with it (Q8_0 N = K = 4096, M = 32:
    // 11.6 vs 11.3 us; Q4_0 M = 24: 8.9 vs 7.2)
    constexpr int PD = 1;
    Step buf[PD];
#pragma unroll
    for (int d = 0; d < PD; d++)
        if (s_lo + d < s_hi) load(s_lo + d, buf[d]);
    for (int s0 = s_lo; s0 < s_hi; s0 += PD) {
#pragma unroll
        for (int d = 0; d < PD; d++) {
            if (s0 + d < s_hi) {
                compute(buf[d], s0 + d);
                if (s0 + d + PD < s_hi) load(s0 + d + PD, buf[d]);
            }
        }
    }

    // result lane (c, r): weight rows 4c .. 4c+3, activation row 16h + r; the waves' K ranges
    // summed through LDS (the activation regions, free after the K loop)
    __syncthreads();
    float* red = (float*)sact;
#pragma unroll
    for (int h = 0; h < MH; h++)
#pragma unroll
        for (int q = 0; q < 4; q++) red[(wave * kSkRows + 4 * c + q) * AR + 16 * h + r] = acc[h][q];
    __syncthreads();
    for (int t = threadIdx.x; t < kSkRows * AR; t += 64 * NWV) {
        const int row = t % kSkRows, m = t / kSkRows;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NWV; w++) v += red[(w * kSkRows + row) * AR + m];
        if (m < M && n0 + row < N) C[(size_t)m * ldc + n0 + row] = v;
    }
}

template <int WT, int MP, bool AS>
hipError_t skinny_launch_nwv(int nwv, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int nb,
                             hipStream_t s) {
    const uint32_t wbytes = (uint32_t)(((uint64_t)N * nb * block_bytes(WT) + 3) & ~(uint64_t)3);
    const uint32_t abytes = (uint32_t)((uint64_t)M * nb * kQ81Bytes);
    const dim3 grid((unsigned)((N + kSkRows - 1) / kSkRows));
    // the shared activation pieces: whole 4-block steps, 16-byte aligned rows
    const bool al = (nb % 4) == 0 && ((uintptr_t)A & 15u) == 0;
    static_assert(MP <= 2, "9-32 rows take skinny16_kernel");
    // 16 waves leave 128 VGPRs per lane: enough for one activation pass, or two with the shared
    // pieces (the 5-8-row launch rule asks for 16 only then)
    if (nwv == 16 && al)
        hipLaunchKernelGGL((skinny_kernel<WT, MP, AS, 16, true>), grid, dim3(1024), 0, s, W, A, C, M, N, nb, N, wbytes,
                           abytes);
    else if (MP == 1 && nwv == 16)
        hipLaunchKernelGGL((skinny_kernel<WT, 1, AS, 16>), grid, dim3(1024), 0, s, W, A, C, M, N, nb, N, wbytes, abytes);
    else if (nwv >= 8 && al)
        hipLaunchKernelGGL((skinny_kernel<WT, MP, AS, 8, true>), grid, dim3(512), 0, s, W, A, C, M, N, nb, N, wbytes, abytes);
    else if (nwv >= 8)
        hipLaunchKernelGGL((skinny_kernel<WT, MP, AS, 8>), grid, dim3(512), 0, s, W, A, C, M, N, nb, N, wbytes, abytes);
    else if (al)
        hipLaunchKernelGGL((skinny_kernel<WT, MP, AS, 4, true>), grid, dim3(256), 0, s, W, A, C, M, N, nb, N, wbytes, abytes);
    else
        hipLaunchKernelGGL((skinny_kernel<WT, MP, AS, 4>), grid, dim3(256), 0, s, W, A, C, M, N, nb, N, wbytes, abytes);
    return hipGetLastError();
}

// 8 waves per workgroup (4 when the K steps are too few): 16 measured 2-25% slower at 9-32 rows
// (Q8_0 N = K = 4096, M = 16: 8.8 vs 8.6 us; N = 14336, K = 4096, M = 32: 42.4 vs 34.4), as did
// 4 on N <= 4096 (M = 32: 12.0 vs 11.3)
template <int WT, bool AS, int MH>
hipError_t skinny16_launch(int nwv, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int nb,
                           hipStream_t s) {
    const uint32_t wbytes = (uint32_t)(((uint64_t)N * nb * block_bytes(WT) + 3) & ~(uint64_t)3);
    const uint32_t abytes = (uint32_t)((uint64_t)M * nb * kQ81Bytes);
    const dim3 grid((unsigned)((N + kSkRows - 1) / kSkRows));
    if constexpr (WT == kWQ80) {
        // Q8_0: the weights staged as aligned row chunks (us, N = K = 4096, M = 32: 11.35 -> 10.74;
        // M = 16 8.61 -> 8.19; N = 14336, K = 4096, M = 16 26.0 -> 23.6).  The shorter blocks of the
        // other types lose with it at N = 4096 (Q4_0 M = 32 7.87 -> 8.36).
        if (nwv >= 8 && ((uintptr_t)W & 15u) == 0) {
            hipLaunchKernelGGL((skinny16_kernel<WT, AS, MH, 8, true>), grid, dim3(512), 0, s, W, A, C, M, N, nb, N, wbytes,
                               abytes);
            return hipGetLastError();
        }
    }
    if (nwv >= 8)
        hipLaunchKernelGGL((skinny16_kernel<WT, AS, MH, 8>), grid, dim3(512), 0, s, W, A, C, M, N, nb, N, wbytes, abytes);
    else
        hipLaunchKernelGGL((skinny16_kernel<WT, AS, MH, 4>), grid, dim3(256), 0, s, W, A, C, M, N, nb, N, wbytes, abytes);
    return hipGetLastError();
}

template <int WT, bool AS>
hipError_t skinny_launch_mp(int nwv, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int nb,
                            hipStream_t s) {
    if (M <= 4) return skinny_launch_nwv<WT, 1, AS>(nwv, W, A, C, M, N, nb, s);
    if (M <= 8) return skinny_launch_nwv<WT, 2, AS>(nwv, W, A, C, M, N, nb, s);
    // 9-32 rows: the 16x16x32 MFMA form (skinny_supported has required the shared pieces)
    if (M <= 16) return skinny16_launch<WT, AS, 1>(nwv, W, A, C, M, N, nb, s);
    return skinny16_launch<WT, AS, 2>(nwv, W, A, C, M, N, nb, s);
}

}  // namespace

bool skinny_supported(int wtype, int afmt, int M, int N, int K, const void* W, const void* A) {
    const bool type_ok = wtype == kWQ40 || wtype == kWQ80 || wtype == kWQ41 || wtype == kWQ50 || wtype == kWQ51;
    if (!type_ok || !(afmt == kAQ81 || (afmt == kAQ8S && wtype == kWQ80)) || M < 1 || M > 32 || N < 1 || K < 32 ||
        (K % 32) != 0 || (((uintptr_t)W | (uintptr_t)A) & 3u) != 0)
        return false;
    // 9-32 rows only with the shared activation pieces (whole 4-block steps, 16-byte aligned)
    if (M > 8 && ((K % 128) != 0 || ((uintptr_t)A & 15u) != 0)) return false;
    // buffer offsets are 32-bit and kOOB (2^31) must lie past both buffers
    const uint64_t wbytes = (uint64_t)N * (K / 32) * block_bytes(wtype) + 4, abytes = (uint64_t)M * (K / 32) * kQ81Bytes;
    return wbytes < (1ull << 31) && abytes < (1ull << 31);
}

// Measured on MI355X against the decode kernel over the quant_gemm definition shapes (block_q8_1
// activations, M = 1 .. 8, us): with ~16 waves per CU the small-batch kernel wins from M = 2 on
// rows of up to 4096 elements once N >= 2048 gives enough 16-row workgroups (Q4_0 N = 9728,
// K = 2560: 7.4 vs 9.2 at M = 3, 7.6 vs 10.9 at M = 4; N = 7168, K = 512: 2.8 vs 5.9 at M = 3),
// on rows up to 8192 elements only for N >= 7168 (Q4_0 N = 12288, K = 5120: 15.2 vs 17.3 at
// M = 4; N = 5120, K = 5120: 11.0 vs 9.6 the other way), at M = 1 only on very short rows
// (N = 7168, K = 512: 2.7 vs 3.7); below N = 2048 (N = 512, K = 7168: 5.8 vs 3.4 at M = 2) and on
// long rows (N = 5120, K = 12288: 19.8 vs 11.1 at M = 2) the decode kernel wins.  At M = 2 the
// register-direct decode kernel wins everywhere but on very short rows (N = 7168, K = 512: 2.7
// vs 4.8) and for Q8_0 on 3584..8192-square shapes (N = K = 7168: 16.6 vs 18.0); elsewhere it is
// 5-32% faster (Q4_0 N = 14336, K = 4096: 9.8 vs 13.0; N = K = 4096: 4.8 vs 5.2).
bool skinny_preferred(int wtype, int M, int N, int K) {
    if (M == 1) return K <= 1024 && N >= 4096;
    if (M == 2)
        return (K <= 1024 && N >= 4096) ||
               (wtype == kWQ80 && N >= 3584 && N <= 8192 && K >= 3584 && K <= 8192);
    // 3-8 rows, fitted on the definition shapes x M = 3, 4, 5, 6, 8 (430 cases, fp32 entry, whole
    // call, this kernel with its activation pieces shared through LDS against the decode kernels
    // and the MFMA GEMM): the automatic route lands 0.2% above the per-case best (geometric
    // mean), no case more than 6.1% above it.  Examples (us, decode vs this kernel): Q8_0 N = K =
    // 4096, M = 8 15.2 vs 13.4; Q4_0 N = 2560, K = 9728, M = 5 15.4 vs 13.5; the other way
    // N = 512, K = 7168, M = 8 the decode kernel wins by 10-18% and N = 5120, K = 12288, M = 6 by
    // 2-29%.
    const bool nib = (wtype == kWQ40 || wtype == kWQ41);
    if (M > 8) {
        // 9-32 rows on the 16x16x32-MFMA form (Q8_1 input, graph replays, us, against the split
        // MFMA GEMM): 9-16 rows but on large square-ish matrices (N = K = 4096, M = 16: Q8_0 8.6
        // vs 9.3 (the 4x4x4 passes took 9.3), Q4_0 5.9 vs 7.6, Q5_0 6.7 vs 15.6, Q5_1 6.8 vs 15.5;
        // N = 14336, K = 4096: Q8_0 26.1 vs 27.4, Q4_0 15.9 vs 17.5; the other way N = K = 7168:
        // Q8_0 25.2 vs 25.0, Q4_0 17.0 vs 16.7), 17-32 rows up to 4096 x 4096 (M = 32: Q8_0 11.3
        // vs 13.4-16.0, Q4_0 7.9 vs 9.9 (4x4x4 passes 11.4), Q5_0 9.7 vs 16.3; M = 24: Q8_0 10.3
        // vs 12.7-14.5; larger matrices go to the MFMA GEMM: N = 14336, K = 4096, M = 32: Q8_0
        // 34.4 vs 30.6, Q4_0 23.2 vs 21.3; N = K = 7168: 28.9 vs 26.7, 19.9 vs 18.4)
        if (!(nib || wtype == kWQ80 || wtype == kWQ50 || wtype == kWQ51)) return false;  // K-quants
        if (M <= 16) return !(N >= 7168 && K >= 7168);
        return (long long)N * K <= 16777216ll;
    }
    if (M == 3) return N >= 2048 && (K <= 1536 || (nib && N >= 100000 && K <= 2560));
    if (M == 4) {
        if (N < 2048) return false;
        if (K <= 3584) return true;
        if (K <= 4096) return N < 100000;
        if (K <= 7168) return (N >= 7168 && N < 14336) || N >= 100000;
        return N <= 4096;
    }
    if (N < 1536) return false;
    if (K <= 3584) return true;
    if (K <= 8192) {
        if (M <= 6 && N < 4096 && K > 4096) return false;
        if (M == 5 && K > 4096 && (N < 7168 || (N >= 14336 && N < 100000 && K >= 7168))) return false;
        return true;
    }
    return N <= 4096 || (M >= 6 && N >= 7168);
}

hipError_t launch_skinny(int wtype, int afmt, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int K,
                         hipStream_t s) {
    if (!skinny_supported(wtype, afmt, M, N, K, W, A)) return hipErrorNotSupported;
    const int nb = K / 32;
    // waves per workgroup: enough workgroups x waves to put ~16 waves on every CU for M <= 4
    // (~4 for 5-8 rows, whose waves hold twice the accumulators), but at least two K steps
    // (4 blocks each) per wave.  Measured (us, M = 2 / 4): Q4_0 N = 4096, K = 14336 20.2 / 20.9
    // with ~4 waves per CU, 13.4 / 15.8 with ~16; at M = 8 ~16 waves per CU lose (Q4_0
    // N = 14336, K = 4096: 29.3 vs 24.4).  With the shared activation pieces (K % 128 == 0,
    // 16-byte aligned activations) 5-8 rows fit 16 waves too and take the M <= 4 rule (kernel
    // alone, us, 8 waves -> this rule: Q8_0 N = K = 4096, M = 8 8.19 -> 7.68; Q4_0 N = 14336,
    // K = 4096, M = 8 17.19 -> 14.79; Q8_0 N = 4096, K = 14336, M = 8 21.18 vs 21.35 level).
    const bool al = (nb % 4) == 0 && ((uintptr_t)A & 15u) == 0;
    const int wgs = (N + kSkRows - 1) / kSkRows;
    const int steps = (nb + 3) / 4;
    const int max_nwv = (M <= 4 || al) ? 16 : 8;
    const long long wave_target = (M <= 4 || al) ? 4096 : 1024;
    int nwv = 4;
    while (nwv < max_nwv && (long long)wgs * nwv < wave_target && steps >= 2 * nwv) nwv *= 2;
    // 5-8 rows on a grid of at most one workgroup per CU: 8 waves (whole call, us: Q8_0 N = K =
    // 4096, M = 8 14.3 -> 13.6, M = 6 13.8 -> 12.7; Q4_0 M = 8 13.1 -> 12.4); with 448 workgroups
    // 4 stay better (Q8_0 N = K = 7168, M = 8: 27.2 vs 29.6)
    if (M > 4 && wgs <= 256 && nwv < 8 && steps >= 16) nwv = 8;
    // 9-32 rows: at most 8 (skinny16_launch)
    if (M > 8) nwv = min(nwv, 8);
    note_engine(KSQ_ENG_SKINNY);
    switch (wtype) {
        case kWQ40: return skinny_launch_mp<kWQ40, false>(nwv, W, A, C, M, N, nb, s);
        case kWQ80:
            return afmt == kAQ8S ? skinny_launch_mp<kWQ80, true>(nwv, W, A, C, M, N, nb, s)
                                 : skinny_launch_mp<kWQ80, false>(nwv, W, A, C, M, N, nb, s);
        case kWQ41: return skinny_launch_mp<kWQ41, false>(nwv, W, A, C, M, N, nb, s);
        case kWQ50: return skinny_launch_mp<kWQ50, false>(nwv, W, A, C, M, N, nb, s);
        default: return skinny_launch_mp<kWQ51, false>(nwv, W, A, C, M, N, nb, s);
    }
}

}  // namespace ksq
