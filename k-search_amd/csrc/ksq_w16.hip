// ksq_w16.hip - the dequantise-then-fp32 GEMM (W4A16 / W8A16: fp32 activations, Q4_0 / Q8_0
// weights, no activation quantisation) on the gfx950 bf16 MFMA.
//
// Reference path: gemm_w4a16_naive / gemm_w4a16_tiled / gemm_w8a16_naive
// (include/gemm_cuda_naive.cuh:66-150, launchers :267-283; include/gemm_cuda_tiled.cuh:108-190,
// launcher :284-291), CPU references gemm_w4a16_reference / gemm_w8a16_reference
// (include/gemm_reference.h:73-147) and the harness oracle reference_q4_0_fp32_gemm
// (llm_kernel_test/reference/gemm_ref.py:51-97): C[m][n] = sum_k A[m][k] * d_w * q_w[n][k] in
// fp32, with q_w = q - 8 for Q4_0 and the signed quant for Q8_0.
//
// gfx950 design:
//  * Exact products on the bf16 MFMA.  Each fp32 activation is split into three bf16 terms
//    a = hi + mid + lo (hi = bf16(a), mid = bf16(a - hi), lo = bf16(a - hi - mid)): both
//    differences are exact in fp32 and the three terms carry all 24 significant bits (finite
//    |a| below the largest bf16).  The weight quants (q - 8 for Q4_0, q for Q8_0) are integers
//    of at most 8 bits, exact in bf16.  So every product of v_mfma_f32_32x32x16_bf16 is exact
//    and only the fp32 sums round, as in the reference's fp32 loop (in another order).  The
//    terms go in smallest first: lo, mid, hi.
//  * The K loop steps over two 32-element blocks.  Per block, six MFMAs (two 16-element halves
//    x three terms) give the block's partial sum P = sum_k a_k q_k for a 32 x 32 patch, then
//    acc = fma(d_w, P, acc): one VALU op per output and block (the reference multiplies d_w into
//    every weight element instead; the same value up to rounding).
//  * Staging: the activation tile is converted to the three bf16 planes and the weight quants
//    to bf16 once per workgroup and K step, into LDS (row pitch 144 bytes: the 16-byte fragment
//    reads of 16 consecutive rows hit distinct banks).  The next step's global loads are issued
//    into registers before the current step's MFMAs.
//  * Tiles: 128 x 128 (four waves of 64 x 64) for M > 32; 32 x 128 (four waves side by side)
//    for M <= 32.  Grids below 256 workgroups are split along K; the partial sums are added in
//    split order by the int8 GEMM's split-K reduction (deterministic).
//  * Rows / columns past M or N load a clamped in-range row and are not stored.
#include "ksq_device.h"
#include "ksq_internal.h"

namespace ksq {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int BM_, int BN_, int TM_, int TN_>
struct W16Tile {
    static constexpr int BM = BM_, BN = BN_, TM = TM_, TN = TN_;
    static constexpr int WN = BN / (32 * TN);   // waves along N
    static constexpr int WM = BM / (32 * TM);   // waves along M
    static_assert(WN * WM == 4, "four waves per workgroup");
    static_assert(BN == 128, "the weight staging maps 128 rows x 2 blocks onto 256 threads");
    static_assert(BM % 16 == 0 && BM * 16 % 256 == 0, "the activation staging maps 16 float4 per row");
};
using W16Big = W16Tile<128, 128, 2, 2>;
using W16Skinny = W16Tile<32, 128, 1, 1>;

constexpr int kW16Pitch = 72;         // bf16 per staged row: 64 values of the step + 8 padding

typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two fp32 values as a bf16 pair (round to nearest even), lo in the low half: one packed
// conversion (v_cvt_pk_bf16_f32) instead of two single ones and the shift and or that merge them.
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{lo, hi}, bf16x2));
}
__device__ __forceinline__ float bf16_low_f32(uint32_t p) { return __builtin_bit_cast(float, p << 16); }
__device__ __forceinline__ float bf16_high_f32(uint32_t p) { return __builtin_bit_cast(float, p & 0xFFFF0000u); }

// 32 weight quants of one block as bf16 into dst (32 values), the block's scale into *d.  v: the
// dwords holding the block, which starts at byte O of v.
template <int WT, int O>
__device__ __forceinline__ void w16_stage_block(const uint32_t* v, uint16_t* dst, float* d) {
    *d = f16_to_f32(half_at(v, O));
    if constexpr (WT == kWQ40) {
        // element e < 16: low nibble of qs[e]; e >= 16: high nibble of qs[e - 16]; value q - 8
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t w = word_at(v, O + 2 + 4 * i);
            float lo[4], hi[4];
#pragma unroll
            for (int b = 0; b < 4; b++) {
                lo[b] = (float)((w >> (8 * b)) & 0x0Fu) - 8.0f;
                hi[b] = (float)((w >> (8 * b + 4)) & 0x0Fu) - 8.0f;
            }
            *(u32x2*)(dst + 4 * i) = u32x2{bf16_pair(lo[0], lo[1]), bf16_pair(lo[2], lo[3])};
            *(u32x2*)(dst + 16 + 4 * i) = u32x2{bf16_pair(hi[0], hi[1]), bf16_pair(hi[2], hi[3])};
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t w = word_at(v, O + 2 + 4 * i);
            float q[4];
#pragma unroll
            for (int b = 0; b < 4; b++) q[b] = (float)(int8_t)((w >> (8 * b)) & 0xFFu);
            *(u32x2*)(dst + 4 * i) = u32x2{bf16_pair(q[0], q[1]), bf16_pair(q[2], q[3])};
        }
    }
}

// WT: kWQ40 or kWQ80.  W: [N][K/32] blocks (4-byte aligned); A: fp32 [M][K] (16-byte aligned);
// C: fp32 [M][N], or split z's partial [M][N] at C + z*M*N.  nb = K/32, even.
// XG: workgroup x is a linear tile index whose tiles each XCD takes as one contiguous run in
// row-major tile order (xcd_tile): whole rows of tiles per XCD, so each XCD's L2 fetches its
// activation rows once (the plain grid spreads each 128-row tile's column tiles over all 8 XCDs).
template <class T, int WT, bool XG = false>
__global__ __launch_bounds__(256, 2) void w16_kernel(const uint8_t* __restrict__ W, const float* __restrict__ A,
                                                     float* __restrict__ C, int M, int N, int nb) {
    constexpr int BM = T::BM, BN = T::BN, TM = T::TM, TN = T::TN, P = kW16Pitch;
    constexpr int BB = block_bytes(WT);                    // 18 or 34
    constexpr int AC = BM * 16 / 256;                      // activation float4 chunks per thread
    constexpr int WW = (WT == kWQ40) ? 5 : 9;              // weight dwords a thread loads per step
    __shared__ __attribute__((aligned(16))) uint16_t sA[3][BM][P];     // lo, mid, hi planes
    __shared__ __attribute__((aligned(16))) uint16_t sW[BN][P];
    __shared__ __attribute__((aligned(16))) float sD[2][BN];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / T::WN, wn = wave % T::WN;
    const int l32 = lane & 31, hi = lane >> 5;
    int tm = (int)blockIdx.y, tn = (int)blockIdx.x;
    if constexpr (XG) {
        const int gn = (N + BN - 1) / BN, tiles = gn * ((M + BM - 1) / BM);
        const int L = xcd_tile((int)blockIdx.x, (int)gridDim.x);
        if (L >= tiles) return;   // padding of the grid to a multiple of 8 (whole workgroup)
        tm = L / gn;
        tn = L % gn;
    }
    const int m0 = tm * BM, n0 = tn * BN;

    // split z covers K steps [s_lo, s_hi) of two blocks each
    const int nsteps = nb / 2, Z = (int)gridDim.z, z = (int)blockIdx.z;
    const int s_lo = (int)((long long)nsteps * z / Z), s_hi = (int)((long long)nsteps * (z + 1) / Z);
    C += (size_t)z * (size_t)M * (size_t)N;
    const size_t K = (size_t)nb * 32;

    // staging assignment: activation chunk c = t + 256 i is row c / 16, float4 c % 16 of the
    // step's 64 floats (16 lanes read 256 contiguous bytes of a row); weight row t % 128,
    // block t / 128 of the step (wave-uniform)
    const int wr = t % BN, wb = t / BN;
    const uint8_t* wrow = W + (size_t)min(n0 + wr, N - 1) * nb * BB;
    f32x4 pa[AC];
    uint32_t pw[WW];
    auto load = [&](int s) {
#pragma unroll
        for (int i = 0; i < AC; i++) {
            const int c = t + 256 * i, r = c >> 4, q = c & 15;
            pa[i] = *(const f32x4*)(A + (size_t)min(m0 + r, M - 1) * K + (size_t)s * 64 + 4 * q);
        }
        // Q4_0: the step's 36 bytes are dwords 0..8 and block wb starts at byte 18 wb, so dwords
        // 4 wb .. 4 wb + 4 hold it from byte 2 wb on; Q8_0: 68 bytes, block wb at byte 34 wb,
        // dwords 8 wb .. 8 wb + 8, from byte 2 wb on
        const uint32_t* src = (const uint32_t*)(wrow + (size_t)s * 2 * BB) + (WT == kWQ40 ? 4 : 8) * wb;
#pragma unroll
        for (int i = 0; i < WW; i++) pw[i] = src[i];
    };
    auto store = [&]() {
#pragma unroll
        for (int i = 0; i < AC; i++) {
            const int c = t + 256 * i, r = c >> 4, q = c & 15;
            const float a[4] = {pa[i].x, pa[i].y, pa[i].z, pa[i].w};
            uint32_t ph[2], pm[2], pl[2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                ph[j] = bf16_pair(a[2 * j], a[2 * j + 1]);
                const float r0 = a[2 * j] - bf16_low_f32(ph[j]), r1 = a[2 * j + 1] - bf16_high_f32(ph[j]);
                pm[j] = bf16_pair(r0, r1);
                pl[j] = bf16_pair(r0 - bf16_low_f32(pm[j]), r1 - bf16_high_f32(pm[j]));
            }
            *(u32x2*)&sA[0][r][4 * q] = u32x2{pl[0], pl[1]};
            *(u32x2*)&sA[1][r][4 * q] = u32x2{pm[0], pm[1]};
            *(u32x2*)&sA[2][r][4 * q] = u32x2{ph[0], ph[1]};
        }
        if (wb == 0) w16_stage_block<WT, 0>(pw, &sW[wr][0], &sD[0][wr]);
        else w16_stage_block<WT, 2>(pw, &sW[wr][32], &sD[1][wr]);
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    f32x16 zero;
#pragma unroll
    for (int r = 0; r < 16; r++) zero[r] = 0.0f;
    const bool wave_has_rows = M - m0 - wm * 32 * TM > 0;   // wave-uniform

    if (s_lo < s_hi) load(s_lo);
    for (int s = s_lo; s < s_hi; s++) {
        store();
        __syncthreads();
        if (s + 1 < s_hi) load(s + 1);
        if (wave_has_rows) {
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
                bf16x8 wf[TN][2], af[3][TM][2];
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int ko = 32 * kb + 16 * h + 8 * hi;
#pragma unroll
                    for (int j = 0; j < TN; j++) wf[j][h] = *(const bf16x8*)&sW[wn * 32 * TN + 32 * j + l32][ko];
#pragma unroll
                    for (int e = 0; e < 3; e++)
#pragma unroll
                        for (int i = 0; i < TM; i++) af[e][i][h] = *(const bf16x8*)&sA[e][wm * 32 * TM + 32 * i + l32][ko];
                }
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int nbase = wn * 32 * TN + 32 * j + 4 * hi;
                    f32x4 dw[4];
#pragma unroll
                    for (int q = 0; q < 4; q++) dw[q] = *(const f32x4*)&sD[kb][nbase + 8 * q];
#pragma unroll
                    for (int i = 0; i < TM; i++) {
                        // the MFMA computes D[n][m]: A operand = weight fragment, B = activations
                        f32x16 p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j][0], af[0][i][0], zero, 0, 0, 0);
                        p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j][1], af[0][i][1], p, 0, 0, 0);
                        p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j][0], af[1][i][0], p, 0, 0, 0);
                        p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j][1], af[1][i][1], p, 0, 0, 0);
                        p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j][0], af[2][i][0], p, 0, 0, 0);
                        p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j][1], af[2][i][1], p, 0, 0, 0);
#pragma unroll
                        for (int q = 0; q < 4; q++)
#pragma unroll
                            for (int r = 0; r < 4; r++)
                                acc[i][j][4 * q + r] = fmaf(dw[q][r], p[4 * q + r], acc[i][j][4 * q + r]);
                    }
                }
            }
        }
        __syncthreads();
    }

    // lane l holds activation row m = l % 32 and weight rows n = 8 (r / 4) + 4 (l / 32) + r % 4
    const bool vec_ok = (N % 4) == 0 && (((uintptr_t)C & 15u) == 0);
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const int gm = m0 + wm * 32 * TM + 32 * i + l32;
        if (gm >= M) continue;
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int nbase = n0 + wn * 32 * TN + 32 * j + 4 * hi;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int gn = nbase + 8 * q;
                if (vec_ok && gn + 3 < N) {
                    *(f32x4*)(C + (size_t)gm * N + gn) =
                        f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                } else {
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        if (gn + r < N) C[(size_t)gm * N + gn + r] = acc[i][j][4 * q + r];
                }
            }
        }
    }
}

// ---- decode form (1-4 activation rows) ------------------------------------------------------
// A GEMV on the VALU: the bf16-MFMA tile wastes 31 of its 32 rows at M = 1 and splits K to fill
// the chip (13 us at N = K = 4096); here every lane owns pairs of adjacent weight blocks (36 or 68
// bytes, loaded straight into VGPRs), the workgroup stages the activation rows of a K tile in LDS
// with each block's fp32 sum, and a lane's block contributes
//     d_w * (sum_k a_k q_k - 8 * sum_k a_k)      (Q4_0; Q8_0: d_w * sum_k a_k q_k)
// with q_k converted once per element (v_cvt_f32_ubyte) and one fma per element and activation
// row: the reference's sum of a_k * (q_k - 8) * d_w regrouped (fp32 rounding differs).  RPW
// weight rows per 256-thread workgroup, RPW / 4 per wave, every activation value read from LDS
// serving all of them.
constexpr int kW16KTile = 4096;   // activation elements per row and K tile
// LDS layout of a staged activation row: pair p of the tile (64 floats) at p * 68 floats, so the
// 16-byte reads of 16 lanes (consecutive pairs, 272 bytes apart) hit distinct bank groups
constexpr int kW16PairPitch = 68;

// NW dwords from p (4-byte aligned) by 16-, 8- and 4-byte loads.
template <int NW>
__device__ __forceinline__ void load_dwords_a4(const uint32_t* __restrict__ p, uint32_t* w) {
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

template <int WT, int MR, int RPW>
__global__ __launch_bounds__(256) void w16_gemv_kernel(const uint8_t* __restrict__ W, const float* __restrict__ A,
                                                       float* __restrict__ C, int N, int nb) {
    constexpr int VR = RPW / 4;                                  // weight rows per wave
    constexpr int BB = block_bytes(WT), PW = BB / 2;             // pair: 36 / 68 bytes = 9 / 17 dwords
    __shared__ __attribute__((aligned(16))) float sx[MR][kW16KTile / 64 * kW16PairPitch];
    __shared__ float ssum[MR][kW16KTile / 32];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (int)blockIdx.x * RPW + wave * VR;
    const size_t K = (size_t)nb * 32;
    float acc[VR][MR];
#pragma unroll
    for (int v = 0; v < VR; v++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[v][m] = 0.0f;

    for (int kb0 = 0; kb0 < nb; kb0 += kW16KTile / 32) {
        const int kbn = min(kW16KTile / 32, nb - kb0);          // blocks in this K tile (even)
        const int np = kbn / 2;
        // this lane's first pair of weight blocks for its rows, issued before the staging loads
        int p = lane;
        uint32_t w[VR][PW];
#pragma unroll
        for (int v = 0; v < VR; v++)
            if (p < np && row0 + v < N)
                load_dwords_a4<PW>((const uint32_t*)(W + ((size_t)(row0 + v) * nb + kb0 + 2 * p) * BB), w[v]);
        // stage the K tile's activations, 8 floats per thread and step, and the block sums
        for (int e = threadIdx.x; e < MR * kbn * 4; e += 256) {
            const int m = e / (kbn * 4), c = e - m * kbn * 4;        // c: 8-float chunk of row m
            const f32x4* src = (const f32x4*)(A + (size_t)m * K + (size_t)kb0 * 32 + 8 * c);
            const f32x4 x0 = src[0], x1 = src[1];
            // chunk c = elements 8c .. 8c + 7 of the tile: pair c / 8, offset 8 (c % 8) in it
            float* dst = &sx[m][(c >> 3) * kW16PairPitch + 8 * (c & 7)];
            *(f32x4*)dst = x0;
            *(f32x4*)(dst + 4) = x1;
            // the 4 chunks of a block sit in 4 consecutive lanes: their partial sums meet by DPP
            float part = ((x0.x + x0.y) + (x0.z + x0.w)) + ((x1.x + x1.y) + (x1.z + x1.w));
            part += dpp_mov<0xB1>(part);   // quad_perm [1,0,3,2]
            part += dpp_mov<0x4E>(part);   // quad_perm [2,3,0,1]
            if ((c & 3) == 0) ssum[m][c >> 2] = part;
        }
        __syncthreads();
        if (row0 < N) {
            for (bool first = true; p < np; p += 64, first = false) {
                if (!first) {
#pragma unroll
                    for (int v = 0; v < VR; v++)
                        if (row0 + v < N)
                            load_dwords_a4<PW>((const uint32_t*)(W + ((size_t)(row0 + v) * nb + kb0 + 2 * p) * BB), w[v]);
                }
#pragma unroll
                for (int h = 0; h < 2; h++) {       // block 2p + h of the tile
                    const int b = 2 * p + h;
                    float part[VR][MR];
#pragma unroll
                    for (int v = 0; v < VR; v++)
#pragma unroll
                        for (int m = 0; m < MR; m++) part[v][m] = 0.0f;
#pragma unroll
                    for (int i = 0; i < (WT == kWQ40 ? 4 : 8); i++) {
                        // 4 quants of each row: Q4_0 elements 4i..4i+3 (low nibbles) and
                        // 16+4i..16+4i+3 (high nibbles); Q8_0 elements 4i..4i+3
                        float q[VR][WT == kWQ40 ? 8 : 4];
#pragma unroll
                        for (int v = 0; v < VR; v++) {
                            const uint32_t wd = word_at(w[v], h * BB + 2 + 4 * i);
                            if constexpr (WT == kWQ40) {
                                const uint32_t lo = wd & 0x0F0F0F0Fu, hi = (wd >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                                for (int j = 0; j < 4; j++) {
                                    q[v][j] = (float)((lo >> (8 * j)) & 0xFFu);
                                    q[v][4 + j] = (float)((hi >> (8 * j)) & 0xFFu);
                                }
                            } else {
#pragma unroll
                                for (int j = 0; j < 4; j++) q[v][j] = (float)(int8_t)((wd >> (8 * j)) & 0xFFu);
                            }
                        }
#pragma unroll
                        for (int m = 0; m < MR; m++) {
                            const float* xp = &sx[m][p * kW16PairPitch + 32 * h];
                            const f32x4 xl = *(const f32x4*)(xp + 4 * i);
#pragma unroll
                            for (int v = 0; v < VR; v++) {
                                part[v][m] = fmaf(xl.x, q[v][0], part[v][m]);
                                part[v][m] = fmaf(xl.y, q[v][1], part[v][m]);
                                part[v][m] = fmaf(xl.z, q[v][2], part[v][m]);
                                part[v][m] = fmaf(xl.w, q[v][3], part[v][m]);
                            }
                            if constexpr (WT == kWQ40) {
                                const f32x4 xh = *(const f32x4*)(xp + 16 + 4 * i);
#pragma unroll
                                for (int v = 0; v < VR; v++) {
                                    part[v][m] = fmaf(xh.x, q[v][4], part[v][m]);
                                    part[v][m] = fmaf(xh.y, q[v][5], part[v][m]);
                                    part[v][m] = fmaf(xh.z, q[v][6], part[v][m]);
                                    part[v][m] = fmaf(xh.w, q[v][7], part[v][m]);
                                }
                            }
                        }
                    }
#pragma unroll
                    for (int v = 0; v < VR; v++) {
                        const float d = f16_to_f32(half_at(w[v], h * BB));
#pragma unroll
                        for (int m = 0; m < MR; m++) {
                            const float t = (WT == kWQ40) ? fmaf(-8.0f, ssum[m][b], part[v][m]) : part[v][m];
                            acc[v][m] = fmaf(d, t, acc[v][m]);
                        }
                    }
                }
            }
        }
        if (kb0 + kW16KTile / 32 < nb) __syncthreads();   // the next tile overwrites the LDS
    }
#pragma unroll
    for (int v = 0; v < VR; v++)
#pragma unroll
        for (int m = 0; m < MR; m++) acc[v][m] = wave_sum(acc[v][m]);
    if (lane == 0) {
#pragma unroll
        for (int v = 0; v < VR; v++)
            if (row0 + v < N) {
#pragma unroll
                for (int m = 0; m < MR; m++) C[(size_t)m * N + row0 + v] = acc[v][m];
            }
    }
}

namespace {
constexpr int kW16MinWGs = 256, kW16TargetWGs = 512, kW16MaxSplits = 16;
constexpr int kW16GemvMaxRows = 4;
bool w16_uses_gemv(int M) { return M >= 1 && M <= kW16GemvMaxRows; }

bool w16_skinny(int M) { return M <= 32; }

int w16_grid_wgs(int M, int N) {
    const int bm = w16_skinny(M) ? W16Skinny::BM : W16Big::BM;
    return ((N + 127) / 128) * ((M + bm - 1) / bm);
}
}  // namespace

int w16_splits(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || w16_uses_gemv(M)) return 1;
    const int wgs = w16_grid_wgs(M, N), steps = K / 64;
    if (wgs >= kW16MinWGs) return 1;
    int sp = (kW16TargetWGs + wgs - 1) / wgs;
    sp = sp < steps / 4 ? sp : steps / 4;            // at least 4 K steps per split
    sp = sp < kW16MaxSplits ? sp : kW16MaxSplits;
    return sp < 1 ? 1 : sp;
}

template <int WT>
static hipError_t w16_launch(const float* A, const uint8_t* W, float* C, int M, int N, int K, int splits,
                             hipStream_t s) {
    const int nb = K / 32;
    if (w16_skinny(M)) {
        const dim3 grid((unsigned)((N + 127) / 128), (unsigned)((M + 31) / 32), (unsigned)splits);
        hipLaunchKernelGGL((w16_kernel<W16Skinny, WT>), grid, dim3(256), 0, s, W, A, C, M, N, nb);
    } else {
        const int tiles = ((N + 127) / 128) * ((M + 127) / 128);
        const dim3 grid((unsigned)((tiles + 7) / 8 * 8), 1u, (unsigned)splits);
        hipLaunchKernelGGL((w16_kernel<W16Big, WT, true>), grid, dim3(256), 0, s, W, A, C, M, N, nb);
    }
    return hipGetLastError();
}

template <int WT, int MR>
static hipError_t w16_gemv_launch(const float* A, const uint8_t* W, float* C, int N, int K, hipStream_t s) {
    const int nb = K / 32;
    // 4 weight rows per wave while that keeps 512 workgroups, else 2 or 1 (whole call, us, with 256
    // in place of 512: N = K = 4096 M = 1 6.84 -> 5.6, M = 2 8.66 -> 6.56; N = 4096, K = 14336,
    // M = 4 33.4 -> 26.3; N = 14336 level; 1024 loses at M = 4: 35.6)
    constexpr int kGemvMinWGs = 512;
    if ((N + 15) / 16 >= kGemvMinWGs)
        hipLaunchKernelGGL((w16_gemv_kernel<WT, MR, 16>), dim3((N + 15) / 16), dim3(256), 0, s, W, A, C, N, nb);
    else if ((N + 7) / 8 >= kGemvMinWGs)
        hipLaunchKernelGGL((w16_gemv_kernel<WT, MR, 8>), dim3((N + 7) / 8), dim3(256), 0, s, W, A, C, N, nb);
    else
        hipLaunchKernelGGL((w16_gemv_kernel<WT, MR, 4>), dim3((N + 3) / 4), dim3(256), 0, s, W, A, C, N, nb);
    return hipGetLastError();
}

template <int WT>
static hipError_t w16_gemv_dispatch(const float* A, const uint8_t* W, float* C, int M, int N, int K, hipStream_t s) {
    switch (M) {
        case 1: return w16_gemv_launch<WT, 1>(A, W, C, N, K, s);
        case 2: return w16_gemv_launch<WT, 2>(A, W, C, N, K, s);
        case 3: return w16_gemv_launch<WT, 3>(A, W, C, N, K, s);
        default: return w16_gemv_launch<WT, 4>(A, W, C, N, K, s);
    }
}

hipError_t launch_w16(int wtype, const float* A, const uint8_t* W, float* C, int M, int N, int K, float* partials,
                      hipStream_t s) {
    if (wtype != kWQ40 && wtype != kWQ80) return hipErrorNotSupported;
    if (w16_uses_gemv(M)) {
        note_engine(KSQ_ENG_W16);
        return wtype == kWQ40 ? w16_gemv_dispatch<kWQ40>(A, W, C, M, N, K, s)
                              : w16_gemv_dispatch<kWQ80>(A, W, C, M, N, K, s);
    }
    const int splits = w16_splits(M, N, K);
    note_engine(KSQ_ENG_W16 | (splits > 1 ? KSQ_ENG_SPLITK : 0u));
    float* out = C;
    if (splits > 1) {
        if (!partials) return hipErrorInvalidValue;
        out = partials;
    }
    hipError_t e = wtype == kWQ40 ? w16_launch<kWQ40>(A, W, out, M, N, K, splits, s)
                                  : w16_launch<kWQ80>(A, W, out, M, N, K, splits, s);
    if (e != hipSuccess || splits == 1) return e;
    return launch_splitk_reduce(partials, C, (int64_t)M * N, splits, s);
}

}  // namespace ksq
