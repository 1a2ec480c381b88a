// ksq_mmq.hip - prefill GEMM on the gfx950 int8 MFMA (the mul_mat_q analogue).
//
// Reference path: the tiled GEMMs of kernelevalplus-main/include/gemm_cuda_tiled.cuh:191-262 and
// gemm_cuda_dp4a.cuh:275-351 (32x32 shared-memory tiles, DP4A on CUDA cores) with the
// block formula of gemm_w4a8_reference / gemm_w8a8_reference (include/gemm_reference.h:175-267).
//
// gfx950 design:
//  * Workgroup tile 128 activation rows x 128 weight rows, 4 waves each owning a
//    64 x 64 quadrant = 2 x 2 tiles of v_mfma_i32_32x32x32_i8.  One MFMA contracts
//    exactly one 32-element Q block, so its i32 result IS the reference's integer
//    block dot sumi for a 32 x 32 patch of outputs.
//  * Per K step 8 blocks (256 K) are staged in LDS: Q8_1 quants as int8 rows, Q4_0
//    weights as packed nibbles (the MFMA lane that holds k = 0..15 takes the low
//    nibbles, the lane that holds k = 16..31 the high ones, which is exactly the
//    Q4_0 element order), Q8_0 weights as int8 rows, plus the per-block scales.
//  * Epilogue without an int->float conversion: the MFMA accumulates onto the bit
//    pattern of 12582912.0f (0x4B400000), so the result read as a float is exactly
//    12582912 + sumi (|sumi| < 2^22).  Then
//        X   = fma(f, d_a', -12582912 * d_a')    = sumi * d_a'   (one rounding; the
//              product 12582912 * d_a' is exact because d_a' has 11 significant bits)
//        acc = fma(d_w, X, acc)
//    two VALU ops per output per block.  For Q4_0 the -8 * d_w * s_a term of the
//    reference formula is a rank-(K/32) product of fp16 fields, so it runs on the
//    f16 MFMA (exact products) straight into the same accumulators; to fold its
//    factor 8 exactly the main term uses d_a' = d_a / 8 and the result is scaled
//    by 8 at the end (powers of two: exact).  Q8_0 uses d_a' = d_a and no side term.
//  * The MFMA for the next tile is issued before the epilogue of the current one,
//    so matrix and vector pipes overlap within a wave.
//  * Row / column tiles past M or N load a clamped in-range row and are not stored.
#include "ksq_device.h"
#include "ksq_internal.h"

namespace ksq {

constexpr int kBM = 128, kBN = 128, kKB = 8;
constexpr int kAPitch = kKB * 32 + 16;  // bytes per staged activation row (conflict-free b128 reads)
constexpr uint32_t kMagic = 0x4B400000u;  // 12582912.0f
constexpr float kMagicF = 12582912.0f;

typedef uint32_t u32x2_a8 __attribute__((ext_vector_type(2), aligned(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

template <int WT>
struct MmqShape {
    static constexpr int WQ = (WT == 0) ? 16 : 32;     // staged weight bytes per block
    static constexpr int WPitch = kKB * WQ + 16;       // bytes per staged weight row
    static constexpr int BB = (WT == 0) ? kQ40Bytes : kQ80Bytes;
    static constexpr int HalfBytes = 4 * BB;           // 72 or 136: half a row's K step
};

// Expert-grouped mode (MoE): workgroup tile y is entry blockIdx.x of a tile schedule;
// its activation rows are gathered through a sorted (token, slot) list and its output is
// added, weighted by the routing probability, into C[token][n].
struct MoeTiles {
    const int32_t* num_tiles;   // [1]
    const int32_t* tile_expert; // [max_tiles]
    const int32_t* tile_row0;   // [max_tiles] first entry in `rows` of this tile
    const int32_t* expert_end;  // [E] one past the expert's last entry in `rows`
    const int32_t* rows;        // [T*top_k] entry j = token*top_k + slot, grouped by expert
    const float* weights;       // [T*top_k] routing weight of entry j
    float* scratch;             // [T*top_k][N] per-entry outputs when top_k > 2, else null
    int top_k;
    size_t expert_stride;       // weight bytes per expert
};

template <int WT, bool DUMP, bool MOE = false>
__global__ __launch_bounds__(256, 2) void mmq_kernel(const uint8_t* __restrict__ W, const uint8_t* __restrict__ A,
                                                     float* __restrict__ C, int32_t* __restrict__ dump, int M,
                                                     int N, int nb, MoeTiles moe = MoeTiles{}) {
    using S = MmqShape<WT>;
    __shared__ __attribute__((aligned(16))) uint8_t sA[kBM * kAPitch];
    __shared__ __attribute__((aligned(16))) uint8_t sW[kBN * S::WPitch];
    __shared__ __attribute__((aligned(16))) float sDa[kKB][kBM];     // d_a' (d_a/8 for Q4_0)
    __shared__ __attribute__((aligned(16))) float sNc[kKB][kBM];     // -12582912 * d_a'
    __shared__ __attribute__((aligned(16))) float sDw[kKB][kBN];     // d_w
    __shared__ __attribute__((aligned(16))) uint16_t sSaH[kBM][kKB]; // -s_a, fp16 bits (Q4_0 side term)
    __shared__ __attribute__((aligned(16))) uint16_t sDwH[kBN][kKB]; //  d_w, fp16 bits

    __shared__ int32_t sRows[kBM];  // MoE: entry index of each tile row
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int m0 = blockIdx.y * kBM;
    const int n0 = (MOE ? blockIdx.y : blockIdx.x) * kBN;
    if constexpr (MOE) {
        const int tile = blockIdx.x;
        if (tile >= moe.num_tiles[0]) return;           // surplus workgroups of the worst-case grid
        const int e = moe.tile_expert[tile];
        const int r0 = moe.tile_row0[tile];
        const int rend = moe.expert_end[e];
        M = min(kBM, rend - r0);                         // valid rows of this tile
        m0 = 0;
        W += (size_t)e * moe.expert_stride;
        if (t < kBM) sRows[t] = moe.rows[r0 + min(t, M - 1)];
        __syncthreads();
    }
    const int l32 = lane & 31, hi = lane >> 5;
    const float da_scale = (WT == 0) ? 0.125f : 1.0f;

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    i32x16 bias;
#pragma unroll
    for (int r = 0; r < 16; r++) bias[r] = DUMP ? 0 : (int)kMagic;

    // staging assignment: thread t owns row t/2, blocks 4*(t&1) .. 4*(t&1)+3 of the K step
    const int sr = t >> 1, sh = t & 1;
    const int am = MOE ? (sRows[sr] / moe.top_k) : min(m0 + sr, M - 1);
    const int wn_row = min(n0 + sr, N - 1);
    const uint8_t* a_src = A + (size_t)am * nb * kQ81Bytes + (size_t)sh * 4 * kQ81Bytes;
    const uint8_t* w_src = W + (size_t)wn_row * nb * S::BB + (size_t)sh * S::HalfBytes;

    for (int kb0 = 0; kb0 < nb; kb0 += kKB) {
        // ---- stage activations: 4 Q8_1 blocks = 144 B = 9 x 16 B
        {
            uint32_t v[36];
            const uint8_t* p = a_src + (size_t)kb0 * kQ81Bytes;
#pragma unroll
            for (int i = 0; i < 9; i++) {
                const u32x4 x = *(const u32x4*)(p + 16 * i);
                v[4 * i] = x.x; v[4 * i + 1] = x.y; v[4 * i + 2] = x.z; v[4 * i + 3] = x.w;
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int kb = 4 * sh + j;
                u32x4* dst = (u32x4*)(sA + sr * kAPitch + kb * 32);
                dst[0] = u32x4{v[9 * j + 1], v[9 * j + 2], v[9 * j + 3], v[9 * j + 4]};
                dst[1] = u32x4{v[9 * j + 5], v[9 * j + 6], v[9 * j + 7], v[9 * j + 8]};
                const float da = f16_to_f32(v[9 * j] & 0xFFFFu) * da_scale;
                sDa[kb][sr] = da;
                sNc[kb][sr] = -kMagicF * da;
                sSaH[sr][kb] = (uint16_t)((v[9 * j] >> 16) ^ 0x8000u);
            }
        }
        // ---- stage weights: 4 blocks = 72 B (Q4_0) / 136 B (Q8_0), 8-byte aligned
        {
            constexpr int NW = S::HalfBytes / 4;
            uint32_t v[NW + 2];
            const uint8_t* p = w_src + (size_t)kb0 * S::BB;
#pragma unroll
            for (int i = 0; i < NW / 2; i++) {
                const u32x2_a8 x = *(const u32x2_a8*)(p + 8 * i);
                v[2 * i] = x.x; v[2 * i + 1] = x.y;
            }
            v[NW] = 0; v[NW + 1] = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int kb = 4 * sh + j, off = j * S::BB;
                const uint32_t dwb = half_at(v, off);
                sDw[kb][sr] = f16_to_f32(dwb);
                sDwH[sr][kb] = (uint16_t)dwb;
                if constexpr (WT == 0) {
                    *(u32x4*)(sW + sr * S::WPitch + kb * 16) =
                        u32x4{word_at(v, off + 2), word_at(v, off + 6), word_at(v, off + 10), word_at(v, off + 14)};
                } else {
                    u32x4* dst = (u32x4*)(sW + sr * S::WPitch + kb * 32);
                    dst[0] = u32x4{word_at(v, off + 2), word_at(v, off + 6), word_at(v, off + 10), word_at(v, off + 14)};
                    dst[1] = u32x4{word_at(v, off + 18), word_at(v, off + 22), word_at(v, off + 26), word_at(v, off + 30)};
                }
            }
        }
        __syncthreads();

        // 32 (block, tile) MFMAs per K step; tile index q = 4*b + 2*i + j.  The MFMA of
        // step q+1 is issued before the epilogue of step q.
        auto frag_a = [&](int b, int i) -> i32x4 {
            return *(const i32x4*)(sA + (wm * 64 + i * 32 + l32) * kAPitch + b * 32 + 16 * hi);
        };
        auto frag_b = [&](int b, int j) -> i32x4 {
            if constexpr (WT == 0) {
                const u32x4 x = *(const u32x4*)(sW + (wn * 64 + j * 32 + l32) * S::WPitch + b * 16);
                const int s4 = 4 * hi;
                return i32x4{(int)((x.x >> s4) & 0x0F0F0F0Fu), (int)((x.y >> s4) & 0x0F0F0F0Fu),
                             (int)((x.z >> s4) & 0x0F0F0F0Fu), (int)((x.w >> s4) & 0x0F0F0F0Fu)};
            } else {
                return *(const i32x4*)(sW + (wn * 64 + j * 32 + l32) * S::WPitch + b * 32 + 16 * hi);
            }
        };
        auto epilogue = [&](int b, int i, int j, const i32x16& res) {
            // 32x32 accumulator layout: column = lane % 32, row = 8*(r/4) + 4*(lane/32) + r%4
            const int col = wn * 64 + j * 32 + l32;
            const int rowb = wm * 64 + i * 32 + 4 * hi;
            if constexpr (DUMP) {
                const int gn = n0 + col;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int gm = m0 + rowb + 8 * (r >> 2) + (r & 3);
                    if (gm < M && gn < N) dump[((size_t)gm * N + gn) * nb + kb0 + b] = res[r];
                }
            } else {
                const float dw = sDw[b][col];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const f32x4 da = *(const f32x4*)&sDa[b][rowb + 8 * q];
                    const f32x4 nc = *(const f32x4*)&sNc[b][rowb + 8 * q];
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        // copy the element out first: bit_cast of an ext-vector element lvalue
                        // reads element 0 with this compiler
                        const int e = res[4 * q + p];
                        const float f = __builtin_bit_cast(float, e);
                        acc[i][j][4 * q + p] = fmaf(dw, fmaf(f, da[p], nc[p]), acc[i][j][4 * q + p]);
                    }
                }
            }
        };

        i32x4 af[2], bf[2];
        af[0] = frag_a(0, 0); af[1] = frag_a(0, 1);
        bf[0] = frag_b(0, 0); bf[1] = frag_b(0, 1);
        i32x16 cur = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[0], bf[0], bias, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4 * kKB; q++) {
            const int b = q >> 2, i = (q >> 1) & 1, j = q & 1;
            i32x16 nxt = bias;
            if (q + 1 < 4 * kKB) {
                const int b1 = (q + 1) >> 2, i1 = ((q + 1) >> 1) & 1, j1 = (q + 1) & 1;
                if (((q + 1) & 3) == 0) {
                    af[0] = frag_a(b1, 0); af[1] = frag_a(b1, 1);
                    bf[0] = frag_b(b1, 0); bf[1] = frag_b(b1, 1);
                }
                nxt = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i1], bf[j1], bias, 0, 0, 0);
            }
            epilogue(b, i, j, cur);
            cur = nxt;
        }

        if constexpr (WT == 0 && !DUMP) {
            // side term: acc += sum_k (-s_a[m][k]) * d_w[n][k] over the 8 blocks (f16 MFMA, exact products)
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const f16x4 sa4 = *(const f16x4*)&sSaH[wm * 64 + i * 32 + l32][4 * hi];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const f16x4 dw4 = *(const f16x4*)&sDwH[wn * 64 + j * 32 + l32][4 * hi];
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x8f16(sa4, dw4, acc[i][j], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }

    if constexpr (!DUMP) {
        const float out_scale = (WT == 0) ? 8.0f : 1.0f;
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int gn = n0 + wn * 64 + j * 32 + l32;
                const int rowb = m0 + wm * 64 + i * 32 + 4 * hi;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int gm = rowb + 8 * (r >> 2) + (r & 3);
                    if (gm < M && gn < N) {
                        if constexpr (MOE) {
                            const int ent = sRows[gm];
                            const float v = out_scale * acc[i][j][r] * moe.weights[ent];
                            if (moe.scratch) moe.scratch[(size_t)ent * N + gn] = v;
                            else unsafeAtomicAdd(C + (size_t)(ent / moe.top_k) * N + gn, v);
                        } else {
                            C[(size_t)gm * N + gn] = out_scale * acc[i][j][r];
                        }
                    }
                }
            }
    }
}

bool mmq_supported(int wtype, int M, int N, int K, const void* W, const void* A) {
    return (wtype == 0 || wtype == 1) && M > 0 && N > 0 && K > 0 && (K % 256) == 0 &&
           (((uintptr_t)W & 15u) == 0) && (((uintptr_t)A & 15u) == 0);
}

hipError_t launch_mmq(int wtype, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int K, hipStream_t s) {
    const dim3 grid((unsigned)((N + kBN - 1) / kBN), (unsigned)((M + kBM - 1) / kBM));
    const int nb = K / 32;
    if (wtype == 0)
        hipLaunchKernelGGL((mmq_kernel<0, false>), grid, dim3(256), 0, s, W, A, C, nullptr, M, N, nb);
    else
        hipLaunchKernelGGL((mmq_kernel<1, false>), grid, dim3(256), 0, s, W, A, C, nullptr, M, N, nb);
    return hipGetLastError();
}

hipError_t launch_mmq_moe(int wtype, const uint8_t* W, const uint8_t* Aq, float* C, int N, int K, int max_tiles,
                          const MoeTilesArgs& a, hipStream_t s) {
    MoeTiles mt;
    mt.num_tiles = a.num_tiles;
    mt.tile_expert = a.tile_expert;
    mt.tile_row0 = a.tile_row0;
    mt.expert_end = a.expert_end;
    mt.rows = a.rows;
    mt.weights = a.weights;
    mt.scratch = a.scratch;
    mt.top_k = a.top_k;
    const int nb = K / 32;
    mt.expert_stride = (size_t)N * nb * (wtype == 0 ? kQ40Bytes : kQ80Bytes);
    const dim3 grid((unsigned)max_tiles, (unsigned)((N + kBN - 1) / kBN));
    if (wtype == 0)
        hipLaunchKernelGGL((mmq_kernel<0, false, true>), grid, dim3(256), 0, s, W, Aq, C, nullptr, 0, N, nb, mt);
    else
        hipLaunchKernelGGL((mmq_kernel<1, false, true>), grid, dim3(256), 0, s, W, Aq, C, nullptr, 0, N, nb, mt);
    return hipGetLastError();
}

hipError_t launch_mmq_block_sumi(int wtype, const uint8_t* W, const uint8_t* A, int32_t* out, int M, int N, int K,
                                 hipStream_t s) {
    if (!mmq_supported(wtype, M, N, K, W, A)) return hipErrorNotSupported;
    const dim3 grid((unsigned)((N + kBN - 1) / kBN), (unsigned)((M + kBM - 1) / kBM));
    const int nb = K / 32;
    if (wtype == 0)
        hipLaunchKernelGGL((mmq_kernel<0, true>), grid, dim3(256), 0, s, W, A, nullptr, out, M, N, nb);
    else
        hipLaunchKernelGGL((mmq_kernel<1, true>), grid, dim3(256), 0, s, W, A, nullptr, out, M, N, nb);
    return hipGetLastError();
}

}  // namespace ksq
