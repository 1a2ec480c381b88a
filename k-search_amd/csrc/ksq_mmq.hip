// ksq_mmq.hip - prefill GEMM on the gfx950 int8 MFMA (the mul_mat_q analogue).
//
// Reference path: the tiled GEMMs of kernelevalplus-main/include/gemm_cuda_tiled.cuh:191-262 and
// gemm_cuda_dp4a.cuh:275-351 (32x32 shared-memory tiles, DP4A on CUDA cores) with the
// block formula of gemm_w4a8_reference / gemm_w8a8_reference (include/gemm_reference.h:175-267).
//
// gfx950 design:
//  * A BM x BN workgroup tile, four waves each owning TM x TN tiles of 32 x 32 computed
//    with v_mfma_i32_32x32x32_i8.  One MFMA contracts exactly one 32-element Q block,
//    so its i32 result IS the reference's integer block dot sumi for a 32 x 32 patch.
//  * Per K step KB blocks are staged in LDS: Q8_1 quants as int8 rows, Q4_0 / Q4_1
//    weights as packed nibbles (the MFMA lane that holds k = 0..15 takes the low nibbles,
//    the lane that holds k = 16..31 the high ones, which is exactly the element order),
//    Q8_0 weights as int8 rows, Q5_0 / Q5_1 widened to one byte per 5-bit quant, plus the
//    per-block scales widened once to fp32.
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
//    by 8 at the end (powers of two: exact).  Q5_0 does the same with 16; Q4_1 and
//    Q5_1 add m * s_a the same way with factor 1.  Q8_0 uses d_a' = d_a and no side term.
//  * The MFMA for the next tile is issued before the epilogue of the current one,
//    so matrix and vector pipes overlap within a wave.
//  * Row / column tiles past M or N load a clamped in-range row and are not stored.
//  * Tile shapes are template parameters; the host picks one by (M, N) so that small-M
//    problems still put a workgroup on every CU.
#include "ksq_device.h"
#include "ksq_internal.h"

namespace ksq {

#ifndef KSQ_KQ_PIPE
#define KSQ_KQ_PIPE 1   // K-quant staging loads of the next K step prefetched into registers
#endif

constexpr uint32_t kMagic = 0x4B400000u;  // 12582912.0f
constexpr float kMagicF = 12582912.0f;

typedef uint32_t u32x2_a8 __attribute__((ext_vector_type(2), aligned(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

template <int V>
struct IntC {
    static constexpr int value = V;
};

// f(IntC<0>{}), ..., f(IntC<N - 1>{}) with compile-time indices
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(IntC<I>{});
        static_for<N, I + 1>(f);
    }
}

template <int BM_, int BN_, int KB_, int TM_, int TN_, int OCC_, bool PIPE_ = false>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, KB = KB_, TM = TM_, TN = TN_, OCC = OCC_;
    static constexpr bool PIPE = PIPE_;   // staging loads of the next K step prefetched into registers
    static constexpr int WN = BN / (32 * TN);          // waves along N
    static constexpr int WM = BM / (32 * TM);          // waves along M
    static constexpr int NT = 64 * WN * WM;            // threads per workgroup
    static_assert(WN * WM == 4 || WN * WM == 8, "four or eight waves per workgroup");
    static_assert(KB == 4 || KB == 8, "K step of 4 or 8 blocks");
    static constexpr int APitch = KB * 32 + 16;        // bytes per staged activation row
};

// Staged weight format per type: Q4_0 / Q4_1 / Q4_K keep packed nibbles (16 B per
// 32-element block); Q8_0 / Q6_K / Q5_0 / Q5_1 int8 values (32 B per block; the 5-bit
// quants are widened while staging).  SUB = scale groups per 32-element block (2 for
// Q6_K's 16-element sub-blocks).
template <int WT, int KB>
struct WShape {
    static constexpr bool nib = (WT == kWQ40 || WT == kWQ41 || WT == kWQ4K);
    static constexpr int WQ = nib ? 16 : 32;                    // staged weight bytes per block
    static constexpr int WPitch = KB * WQ + 16;                 // bytes per staged weight row
    static constexpr int BB = is_kquant(WT) ? 0 : block_bytes(WT);
    static constexpr int Chunk = 4 * BB;                        // 4 blocks: 72 / 136 / 80 / 88 / 96 bytes
    static constexpr int SUB = (WT == kWQ6K) ? 2 : 1;
    // the s_a side term: -8 d_w s_a (Q4_0), -dmin m s_a (Q4_K), -16 d_w s_a (Q5_0), +m s_a (Q4_1, Q5_1)
    static constexpr bool side = !(WT == kWQ80 || WT == kWQ6K);
    // the main term runs on d_a / out_scale so that the side factor is an fp16 field as stored
    static constexpr float out_scale = (WT == kWQ40 || WT == kWQ4K) ? 8.0f : (WT == kWQ50) ? 16.0f : 1.0f;
    static constexpr int SB = (WT == kWQ4K) ? kQ4KBytes : kQ6KBytes;  // K-quant super-block bytes
};

// Expert-grouped mode (MoE): workgroup x is entry blockIdx.x of a tile schedule; its
// activation rows are gathered through a sorted (token, slot) list and its output is
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

// 6-bit scale and min j of a Q4_K super-block (get_scale_min_k4); s3 = the 12 scale bytes.
__device__ __forceinline__ void q4_K_scale_min_regs(int j, const uint32_t* s3, int& sc, int& m) {
    auto byte = [&](int k) -> int { return (int)((s3[k >> 2] >> (8 * (k & 3))) & 0xFFu); };
    if (j < 4) {
        sc = byte(j) & 63;
        m = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 0x0F) | ((byte(j - 4) >> 6) << 4);
        m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// NW words starting at the 2-byte aligned global byte pointer p: aligned dword reads
// re-aligned with v_alignbyte_b32.  The extra dword is read only when p is not 4-byte
// aligned, so no byte past p + 4*NW is touched.
template <int NW>
__device__ __forceinline__ void read_words_g(const uint8_t* p, uint32_t* w) {
    const int sh = (int)((uintptr_t)p & 3u);
    const uint32_t* q = (const uint32_t*)(p - sh);
    uint32_t raw[NW + 1];
#pragma unroll
    for (int i = 0; i < NW; i++) raw[i] = q[i];
    raw[NW] = sh ? q[NW] : 0u;
#pragma unroll
    for (int i = 0; i < NW; i++) w[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], sh);
}

// AF: activation block format: kAQ81 block_q8_1 (fp16 d, s), kAQ8S block_q8s (fp32 d, no sum;
// Q8_0 weights only), kAQ8F block_q8f (fp32 d and s, 40 bytes; Q4_0, Q5_0, Q8_0 weights), whose
// s_a term is subtracted in the epilogue instead of running on the f16 MFMA.
// T::PIPE (tiles of 128 x 128 with K steps of 4 blocks; 32-element block types, no MoE): the
// global loads of K step k+1 are issued into registers before step k computes (threads 0..127
// hold an activation chunk, 128..255 a weight chunk), so their latency hides behind the MFMAs.
// Slot of 32-byte block kb (0..7) in a staged row: the second chunk's blocks 4..7 swapped in
// pairs (4 <-> 6, 5 <-> 7), so that the lane pair staging a row's two chunks writes blocks j and
// 4 + j 64 bytes apart mod 128, i.e. 16 banks apart, instead of 128 bytes apart on the same banks.
__device__ __forceinline__ constexpr int kslot(int kb) { return kb ^ ((kb >> 1) & 2); }
// Half (4 block slots, 8 bytes) h of row r of the side-term planes (16-byte rows): the halves of
// rows 8..15 of every 16 swapped, so that the side-term MFMA's 8-byte reads (lane: row l % 32,
// half l / 32) of rows r and r + 8 fall 8 bytes apart instead of on the same banks.
__device__ __forceinline__ constexpr int shalf(int r, int h) { return h ^ ((r >> 3) & 1); }

template <class T, int WT, bool DUMP, bool MOE, int AF>
__global__ __launch_bounds__(T::NT, T::OCC) void mmq_kernel(const uint8_t* __restrict__ W,
                                                          const uint8_t* __restrict__ A, float* __restrict__ C,
                                                          int32_t* __restrict__ dump, int M, int N, int nb,
                                                          MoeTiles moe, int trans) {
    using S = WShape<WT, T::KB>;
    constexpr int BM = T::BM, BN = T::BN, KB = T::KB, TM = T::TM, TN = T::TN;
    constexpr bool AS = AF == kAQ8S, AFS = AF == kAQ8F;
    constexpr int ABW = AFS ? 10 : 9;                  // dwords per activation block
    constexpr int AQ = AFS ? 2 : 1;                    // dword offset of the quants in a block
    // the s_a term: f16 MFMA for block_q8_1, an epilogue subtraction for block_q8f
    constexpr bool SIDE_MFMA = S::side && AF == kAQ81, SIDE_BF = S::side && AFS;
    __shared__ __attribute__((aligned(16))) uint8_t sA[BM * T::APitch];
    // Q6_K: one more row, all zeros, that the lanes outside a sub-block read
    __shared__ __attribute__((aligned(16))) uint8_t sW[(BN + (S::SUB == 2 ? 1 : 0)) * S::WPitch];
    // The lane pair staging a row's two chunks of 4 blocks writes blocks j and 4 + j at once.
    // Unpadded, the scale planes put those 4 rows of BM (BN) floats apart, a multiple of the
    // 32 banks that serve one write; 4 floats of padding per row put them 16 banks apart.  (The
    // 32-byte blocks of a staged row are placed by kslot for the same reason.)
    constexpr int SP = 4;
    __shared__ __attribute__((aligned(16))) float sDa[KB][BM + SP];     // d_a' (d_a/8 for Q4_0)
    __shared__ __attribute__((aligned(16))) float sNc[KB][BM + SP];     // -12582912 * d_a'
    __shared__ __attribute__((aligned(16))) float sDw[KB * S::SUB][BN + SP]; // weight scale per (sub-)block
    __shared__ __attribute__((aligned(16))) uint16_t sSaH[BM][8];  // -s_a, fp16 bits (side term)
    // block_q8f: -s_a as three bf16 parts (hi + mid + lo, exact), d_w as two (hi + lo, exact)
    __shared__ __attribute__((aligned(16))) uint16_t sSaB[SIDE_BF ? 3 : 1][SIDE_BF ? BM : 1][8];
    __shared__ __attribute__((aligned(16))) uint16_t sDwB[SIDE_BF ? 2 : 1][SIDE_BF ? BN : 1][8];
    __shared__ __attribute__((aligned(16))) uint16_t sDwH[BN][8];  // side-term weight factor, fp16 bits
    __shared__ __attribute__((aligned(16))) uint16_t sDwL[WT == kWQ4K ? BN : 1][8];  // Q4_K: its low part
    __shared__ int32_t sRows[MOE ? BM : 1];                        // MoE: entry index of each tile row
    __shared__ int32_t sTok[MOE ? BM : 1];                         // MoE: its token (activation row)
    __shared__ float sWt[MOE ? BM : 1];                            // MoE: its routing weight * out_scale

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave / T::WN, wn = wave % T::WN;
    // MoE grid: x = column tile, y = entry of the tile schedule, so the row tiles that share a
    // column of an expert's weights are dispatched N / BN workgroups apart, i.e. to the same XCD
    // (and its L2) when N / BN is a multiple of 8
    const int m0 = (MOE ? 0 : (int)blockIdx.y) * BM;
    const int n0 = (int)blockIdx.x * BN;
    const int l32 = lane & 31, hi = lane >> 5;
    constexpr float da_scale = 1.0f / S::out_scale;
    static_assert(!is_kquant(WT) || KB == 8, "K-quants stage one 256-element super-block per K step");
    static_assert(!AS || WT == kWQ80, "block_q8s activations pair with Q8_0 weights only");
    static_assert(!AFS || WT == kWQ40 || WT == kWQ50 || WT == kWQ80,
                  "block_q8f activations pair with Q4_0, Q5_0 and Q8_0 weights");
    static_assert(!(AFS && MOE), "the grouped GEMM reads block_q8_1 activations");

    if constexpr (S::SUB == 2) {
        for (int i = t; i < S::WPitch / 16; i += T::NT) *(u32x4*)(sW + BN * S::WPitch + 16 * i) = u32x4{0, 0, 0, 0};
    }
    if constexpr (KB == 4) {
        // the f16 side-term MFMA contracts 8 block slots; slots 4..7 stay zero
        if (t < BM) *(uint4*)&sSaH[t][0] = uint4{0, 0, 0, 0};
        if (t < BN) *(uint4*)&sDwH[t][0] = uint4{0, 0, 0, 0};
        if constexpr (SIDE_BF) {
            if (t < BM)
                for (int e = 0; e < 3; e++) *(uint4*)&sSaB[e][t][0] = uint4{0, 0, 0, 0};
            if (t < BN)
                for (int e = 0; e < 2; e++) *(uint4*)&sDwB[e][t][0] = uint4{0, 0, 0, 0};
        }
    }
    if constexpr (MOE) {
        const int tile = blockIdx.y;
        if (tile >= moe.num_tiles[0]) return;           // surplus workgroups of the worst-case grid
        const int e = moe.tile_expert[tile];
        const int r0 = moe.tile_row0[tile];
        M = min(BM, moe.expert_end[e] - r0);             // valid rows of this tile
        W += (size_t)e * moe.expert_stride;
        if (t < BM) {
            // per-row routing data read once here, so neither the staging nor the epilogue waits
            // on a global load or divides per element
            const int ent = moe.rows[r0 + min(t, M - 1)];
            sRows[t] = ent;
            sTok[t] = ent / moe.top_k;
            sWt[t] = moe.weights[ent] * S::out_scale;
        }
    }
    __syncthreads();

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;
    i32x16 bias;
#pragma unroll
    for (int r = 0; r < 16; r++) bias[r] = DUMP ? 0 : (int)kMagic;

    const int wave_rows = M - m0 - wm * 32 * TM;            // rows of this wave's tiles (wave-uniform)
    const bool wave_has_rows = wave_rows > 0;

    // split-K: workgroup z of gridDim.z covers K steps [z*steps/Z, (z+1)*steps/Z) and writes its
    // partial sums to C + z*M*N (the caller adds the partials)
    const int nsteps = nb / KB, Z = (int)gridDim.z, z = (int)blockIdx.z;
    const int kb_lo = (int)((long long)nsteps * z / Z) * KB, kb_hi = (int)((long long)nsteps * (z + 1) / Z) * KB;
    if constexpr (!MOE) C += (size_t)z * (size_t)M * (size_t)N;
    // ---- staging of 32-element blocks, split into the global loads and the LDS writes
    // activation chunk g (4 blocks = 144 B = 9 x 16 B, or 160 B = 10 x 16 B for block_q8f) of
    // staged row sr
    auto load_act = [&](int sr, int g, int kb0, uint32_t* v) {
        const int am = MOE ? sTok[sr] : min(m0 + sr, M - 1);
        const uint8_t* p = A + ((size_t)am * nb + kb0 + 4 * g) * (4 * ABW);
#pragma unroll
        for (int i = 0; i < ABW; i++) {
            const u32x4 x = *(const u32x4*)(p + 16 * i);
            v[4 * i] = x.x; v[4 * i + 1] = x.y; v[4 * i + 2] = x.z; v[4 * i + 3] = x.w;
        }
    };
    // (each row's four 2-byte side values of a chunk leave as one 8-byte write: 2-byte writes 16
    // bytes apart were LDS bank conflicts)
    auto store_act = [&](int sr, int g, const uint32_t* v) {
        uint32_t sah[2] = {0u, 0u}, sab[3][2] = {{0u, 0u}, {0u, 0u}, {0u, 0u}};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int kb = 4 * g + j;
            const uint32_t* bv = v + ABW * j;
            u32x4* dst = (u32x4*)(sA + sr * T::APitch + kslot(kb) * 32);
            dst[0] = u32x4{bv[AQ], bv[AQ + 1], bv[AQ + 2], bv[AQ + 3]};
            dst[1] = u32x4{bv[AQ + 4], bv[AQ + 5], bv[AQ + 6], bv[AQ + 7]};
            // fp32 scales (block_q8s, block_q8f) with their two lowest mantissa bits cleared (22
            // significant bits), so that 12582912 * d_a' stays exact (relative change < 2^-21);
            // da_scale is a power of two
            const float da = (AS || AFS) ? __builtin_bit_cast(float, bv[0] & ~3u) * da_scale
                                         : f16_to_f32(bv[0] & 0xFFFFu) * da_scale;
            sDa[kb][sr] = da;
            sNc[kb][sr] = -kMagicF * da;
            // block_q8f: the term -c*s_a in the main term's units (c = out_scale: 8 for Q4_0,
            // 16 for Q5_0), i.e. -s_a
            if constexpr (SIDE_BF) {
                // -s_a in the main term's units (the factor c cancels against d_a / c), split into
                // bf16 parts whose sum is exact: hi = bf16(x), mid = bf16(x - hi), lo = the rest
                const float x = -__builtin_bit_cast(float, bv[1]);
                const __bf16 h = (__bf16)x;
                const float r = x - (float)h;
                const __bf16 m = (__bf16)r;
                const uint32_t sh = 16 * (j & 1);
                sab[0][j >> 1] |= (uint32_t)__builtin_bit_cast(uint16_t, h) << sh;
                sab[1][j >> 1] |= (uint32_t)__builtin_bit_cast(uint16_t, m) << sh;
                sab[2][j >> 1] |= (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(r - (float)m)) << sh;
            }
            if constexpr (SIDE_MFMA) sah[j >> 1] |= ((bv[0] >> 16) ^ 0x8000u) << (16 * (j & 1));
        }
        if constexpr (SIDE_BF) {
#pragma unroll
            for (int e = 0; e < 3; e++) *(u32x2*)&sSaB[e][sr][4 * g] = u32x2{sab[e][0], sab[e][1]};
        }
        if constexpr (SIDE_MFMA) *(u32x2*)&sSaH[sr][4 * shalf(sr, g)] = u32x2{sah[0], sah[1]};
    };
    // weight chunk g (4 blocks: 72 / 136 / 80 / 88 / 96 B, 8-byte aligned) of staged row sr
    constexpr int WNW = is_kquant(WT) ? 2 : S::Chunk / 4;
    auto load_w = [&](int sr, int g, int kb0, uint32_t* v) {
        if constexpr (!is_kquant(WT)) {
            const int wr = min(n0 + sr, N - 1);
            const uint8_t* p = W + (size_t)wr * nb * S::BB + (size_t)(kb0 + 4 * g) * S::BB;
#pragma unroll
            for (int i = 0; i < WNW / 2; i++) {
                const u32x2_a8 x = *(const u32x2_a8*)(p + 8 * i);
                v[2 * i] = x.x; v[2 * i + 1] = x.y;
            }
            v[WNW] = 0; v[WNW + 1] = 0;
        }
    };
    auto store_w = [&](int sr, int g, const uint32_t* v) {
        if constexpr (!is_kquant(WT)) {
            uint32_t dwh[2] = {0u, 0u}, dwbf[2][2] = {{0u, 0u}, {0u, 0u}};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int kb = 4 * g + j, off = j * S::BB;
                const uint32_t dwb = half_at(v, off);
                sDw[kb][sr] = f16_to_f32(dwb);
                // side factor against -s_a: d_w (Q4_0, Q5_0) or -m (Q4_1, Q5_1)
                const uint32_t sh = 16 * (j & 1);
                if constexpr (WT == kWQ41 || WT == kWQ51) dwh[j >> 1] |= ((half_at(v, off + 2) ^ 0x8000u) & 0xFFFFu) << sh;
                else dwh[j >> 1] |= (dwb & 0xFFFFu) << sh;
                if constexpr (SIDE_BF) {
                    // d_w (11 significant bits) as bf16 hi + lo, exact
                    const float dwf = f16_to_f32(dwb);
                    const __bf16 h = (__bf16)dwf;
                    dwbf[0][j >> 1] |= (uint32_t)__builtin_bit_cast(uint16_t, h) << sh;
                    dwbf[1][j >> 1] |= (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(dwf - (float)h)) << sh;
                }
                if constexpr (WT == kWQ40 || WT == kWQ41) {
                    constexpr int q = (WT == kWQ40) ? 2 : 4;  // offset of qs
                    *(u32x4*)(sW + sr * S::WPitch + kb * 16) =
                        u32x4{word_at(v, off + q), word_at(v, off + q + 4), word_at(v, off + q + 8),
                              word_at(v, off + q + 12)};
                } else if constexpr (WT == kWQ80) {
                    u32x4* dst = (u32x4*)(sW + sr * S::WPitch + kslot(kb) * 32);
                    dst[0] = u32x4{word_at(v, off + 2), word_at(v, off + 6), word_at(v, off + 10), word_at(v, off + 14)};
                    dst[1] = u32x4{word_at(v, off + 18), word_at(v, off + 22), word_at(v, off + 26), word_at(v, off + 30)};
                } else {
                    // Q5_0 / Q5_1: widen to one byte per quant (0..31); element 4i+t takes nibble
                    // t of word i and qh bit 4i+t, element 16+4i+t the high nibble and bit 16+4i+t
                    constexpr int qh = (WT == kWQ50) ? 2 : 4, q = qh + 4;
                    const uint32_t h = word_at(v, off + qh);
                    uint32_t o[8];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const uint32_t w4 = word_at(v, off + q + 4 * i);
                        o[i] = (w4 & 0x0F0F0F0Fu) | qh_to_bit4(h >> (4 * i));
                        o[4 + i] = ((w4 >> 4) & 0x0F0F0F0Fu) | qh_to_bit4(h >> (16 + 4 * i));
                    }
                    u32x4* dst = (u32x4*)(sW + sr * S::WPitch + kslot(kb) * 32);
                    dst[0] = u32x4{o[0], o[1], o[2], o[3]};
                    dst[1] = u32x4{o[4], o[5], o[6], o[7]};
                }
            }
            *(u32x2*)&sDwH[sr][4 * shalf(sr, g)] = u32x2{dwh[0], dwh[1]};
            if constexpr (SIDE_BF) {
#pragma unroll
                for (int e = 0; e < 2; e++) *(u32x2*)&sDwB[e][sr][4 * g] = u32x2{dwbf[e][0], dwbf[e][1]};
            }
        }
    };
    // ---- K-quant super-blocks, split into the global loads and the LDS writes.  Work item c is
    // weight row c (Q4_K: 144 bytes, 16-byte aligned) or, for Q6_K (210 bytes, 2-byte aligned),
    // half h = c / BN of row c % BN: items c < BN take the first halves (consecutive lanes write
    // consecutive rows; lane pairs sharing a row were 2-way LDS bank conflicts on every scale
    // write).  The loads keep raw words: Q6_K's are re-aligned with v_alignbyte_b32 when stored.
    constexpr int KQW = (WT == kWQ6K) ? 2 * BN : BN;     // weight work items per K step
    auto load_kq = [&](int c, int kb0, uint32_t* v) {
        const int nsb = nb / 8, s0 = kb0 / 8;
        if constexpr (WT == kWQ4K) {
            const int wr = min(n0 + c, N - 1);
            const uint8_t* p = W + ((size_t)wr * nsb + s0) * kQ4KBytes;
#pragma unroll
            for (int i = 0; i < 9; i++) {
                const u32x4 x = *(const u32x4*)(p + 16 * i);
                v[4 * i] = x.x; v[4 * i + 1] = x.y; v[4 * i + 2] = x.z; v[4 * i + 3] = x.w;
            }
        } else if constexpr (WT == kWQ6K) {
            // v[0..16] the ql half (64 B at 64h), v[17..25] the qh half (32 B at 128 + 32h),
            // v[26..28] the 8 scales (at 192 + 8h), v[29] d, v[30] the byte shift; the last raw
            // word of each field is read only when the super-block is not 4-byte aligned, so no
            // byte past the field is touched
            const int sr = c % BN, h = c / BN;
            const int wr = min(n0 + sr, N - 1);
            const uint8_t* sb = W + ((size_t)wr * nsb + s0) * kQ6KBytes;
            const int sh = (int)((uintptr_t)sb & 3u);
            const uint32_t* q = (const uint32_t*)(sb - sh);
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = q[16 * h + i];
            v[16] = sh ? q[16 * h + 16] : 0u;
#pragma unroll
            for (int i = 0; i < 8; i++) v[17 + i] = q[32 + 8 * h + i];
            v[25] = sh ? q[40 + 8 * h] : 0u;
            v[26] = q[48 + 2 * h];
            v[27] = q[49 + 2 * h];
            v[28] = sh ? q[50 + 2 * h] : 0u;
            v[29] = *(const uint16_t*)(sb + 208);
            v[30] = (uint32_t)sh;
        }
    };
    auto store_kq = [&](int c, const uint32_t* v) {
        if constexpr (WT == kWQ4K) {
            const int sr = c;
            const float d = f16_to_f32(v[0] & 0xFFFFu), dmin = f16_to_f32(v[0] >> 16);
            // the row's 8 side factors leave as one 16-byte write per plane (8 two-byte
            // writes per row 16 bytes apart were 4-way LDS bank conflicts)
            uint32_t hh[4], ll[4];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                int sc, mn;
                q4_K_scale_min_regs(j, v + 1, sc, mn);
                sDw[j][sr] = d * (float)sc;                     // exact: 11 x 6 bits
                // side factor dmin*m/8 (17 significant bits) as an fp16 hi + lo pair
                const float f = dmin * (float)mn * 0.125f;
                const _Float16 h = (_Float16)f;
                const _Float16 l = (_Float16)(f - (float)h);
                const uint32_t hb = __builtin_bit_cast(uint16_t, h), lb = __builtin_bit_cast(uint16_t, l);
                if (j & 1) {
                    hh[j >> 1] |= hb << 16;
                    ll[j >> 1] |= lb << 16;
                } else {
                    hh[j >> 1] = hb;
                    ll[j >> 1] = lb;
                }
            }
            if (shalf(sr, 0)) {
                *(u32x4*)&sDwH[sr][0] = u32x4{hh[2], hh[3], hh[0], hh[1]};
                *(u32x4*)&sDwL[sr][0] = u32x4{ll[2], ll[3], ll[0], ll[1]};
            } else {
                *(u32x4*)&sDwH[sr][0] = u32x4{hh[0], hh[1], hh[2], hh[3]};
                *(u32x4*)&sDwL[sr][0] = u32x4{ll[0], ll[1], ll[2], ll[3]};
            }
#pragma unroll
            for (int i = 0; i < 8; i++)
                *(u32x4*)(sW + sr * S::WPitch + 16 * i) =
                    u32x4{v[4 + 4 * i], v[5 + 4 * i], v[6 + 4 * i], v[7 + 4 * i]};
        } else if constexpr (WT == kWQ6K) {
            // unpack one 128-element half to int8 (q - 32)
            const int sr = c % BN, h = c / BN;
            const int sh = (int)v[30];
            uint32_t ql[16], qh[8], scw[2];
#pragma unroll
            for (int i = 0; i < 16; i++) ql[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], sh);
#pragma unroll
            for (int i = 0; i < 8; i++) qh[i] = __builtin_amdgcn_alignbyte(v[18 + i], v[17 + i], sh);
#pragma unroll
            for (int i = 0; i < 2; i++) scw[i] = __builtin_amdgcn_alignbyte(v[27 + i], v[26 + i], sh);
            const float d = f16_to_f32(v[29]);
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int sc = (int)(int8_t)((scw[u >> 2] >> (8 * (u & 3))) & 0xFFu);
                sDw[8 * h + u][sr] = d * (float)sc;              // exact: 11 x 8 bits
            }
#pragma unroll
            for (int g = 0; g < 4; g++) {
                uint32_t o[8];
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const uint32_t lo = (ql[8 * (g & 1) + i] >> (4 * (g >> 1))) & 0x0F0F0F0Fu;
                    const uint32_t hb = ((qh[i] >> (2 * g)) << 4) & 0x30303030u;
                    // 6-bit values b, one per byte; (b + 96) ^ 128 = b - 32 as int8, and b + 96
                    // <= 159 carries into no neighbouring byte
                    o[i] = ((lo | hb) + 0x60606060u) ^ 0x80808080u;
                }
                // elements 128h + 32g .. +31 = block 4h + g of this K step
                u32x4* dst = (u32x4*)(sW + sr * S::WPitch + (4 * h + g) * 32);
                dst[0] = u32x4{o[0], o[1], o[2], o[3]};
                dst[1] = u32x4{o[4], o[5], o[6], o[7]};
            }
        }
    };
    constexpr bool PIPE = T::PIPE && !MOE && !is_kquant(WT);
    static_assert(!PIPE || (KB == 4 && BM == 128 && BN == 128 && T::NT == 256),
                  "the pipelined staging covers 128 x 128 tiles with 4-block K steps");
    // KPIPE (Q6_K, no MoE, tiles whose K step is at most 128 weight items and 128 activation
    // chunks): threads 0..127 hold weight item t, 128..255 activation chunk t - 128 of the next K
    // step, the same way (Q6_K M = 128, N = 14336, K = 4096 on 64 x 64: 70.9 -> 62.5 us with the
    // quantiser).  Q4_K's prefetched form spills at three workgroups per CU (64 x 128: 42.9 ->
    // 50.9 us) and stays unprefetched.
    constexpr int ACH = BM * (KB / 4);                   // activation chunks per K step
    constexpr bool KPIPE = KSQ_KQ_PIPE && WT == kWQ6K && !MOE && T::NT == 256 && KQW <= 128 && ACH <= 128;
    // PIPE: one chunk per thread and K step; threads 0..127 activation row t, 128..255 weight row t-128
    uint32_t pre[(PIPE || KPIPE) ? 4 * ABW : 1];
    static_assert(!KPIPE || 4 * ABW >= 36, "a prefetched super-block fits the chunk registers");
    const bool pre_act = t < 128;
    auto pre_load = [&](int kb0) {
        if constexpr (PIPE) {
            if (pre_act) load_act(t, 0, kb0, pre);
            else load_w(t - 128, 0, kb0, pre);
        } else if constexpr (KPIPE) {
            if (t < KQW) load_kq(t, kb0, pre);
            else if (t >= 128 && t - 128 < ACH) load_act((t - 128) / (KB / 4), (t - 128) % (KB / 4), kb0, pre);
        }
    };
    if constexpr (PIPE || KPIPE) {
        if (kb_lo < kb_hi) pre_load(kb_lo);
    }

    for (int kb0 = kb_lo; kb0 < kb_hi; kb0 += KB) {
        if constexpr (PIPE) {
            if (pre_act) store_act(t, 0, pre);
            else store_w(t - 128, 0, pre);
            __syncthreads();
            if (kb0 + KB < kb_hi) pre_load(kb0 + KB);
        } else if constexpr (KPIPE) {
            if (t < KQW) store_kq(t, pre);
            else if (t >= 128 && t - 128 < ACH) store_act((t - 128) / (KB / 4), (t - 128) % (KB / 4), pre);
            __syncthreads();
            if (kb0 + KB < kb_hi) pre_load(kb0 + KB);
        } else {
        // ---- stage activations
        for (int c = t; c < BM * (KB / 4); c += T::NT) {
            const int sr = c / (KB / 4), g = c % (KB / 4);
            uint32_t v[4 * ABW];
            load_act(sr, g, kb0, v);
            store_act(sr, g, v);
        }
        if constexpr (!is_kquant(WT)) {
            // ---- stage weights
            for (int c = t; c < BN * (KB / 4); c += T::NT) {
                const int sr = c / (KB / 4), g = c % (KB / 4);
                uint32_t v[WNW + 2];
                load_w(sr, g, kb0, v);
                store_w(sr, g, v);
            }
        } else {
            // ---- K-quants: one super-block per weight row (Q4_K) or half-row (Q6_K) and K step
            for (int c = t; c < KQW; c += T::NT) {
                uint32_t v[36];
                load_kq(c, kb0, v);
                store_kq(c, v);
            }
        }
        __syncthreads();
        }  // staging without prefetch

        auto frag_a = [&](int b, int i) -> i32x4 {
            return *(const i32x4*)(sA + (wm * 32 * TM + i * 32 + l32) * T::APitch + kslot(b) * 32 + 16 * hi);
        };
        auto frag_b = [&](int b, int j) -> i32x4 {
            if constexpr (WT == kWQ4K) {
                // sub-block b: bytes 32*(b/2) + 16*hi .. +15 of the staged qs, low nibbles for
                // even b, high nibbles for odd b
                const u32x4 x =
                    *(const u32x4*)(sW + (wn * 32 * TN + j * 32 + l32) * S::WPitch + 32 * (b >> 1) + 16 * hi);
                const int s4 = 4 * (b & 1);
                return i32x4{(int)((x.x >> s4) & 0x0F0F0F0Fu), (int)((x.y >> s4) & 0x0F0F0F0Fu),
                             (int)((x.z >> s4) & 0x0F0F0F0Fu), (int)((x.w >> s4) & 0x0F0F0F0Fu)};
            } else if constexpr (S::nib) {
                const u32x4 x = *(const u32x4*)(sW + (wn * 32 * TN + j * 32 + l32) * S::WPitch + b * 16);
                const int s4 = 4 * hi;
                return i32x4{(int)((x.x >> s4) & 0x0F0F0F0Fu), (int)((x.y >> s4) & 0x0F0F0F0Fu),
                             (int)((x.z >> s4) & 0x0F0F0F0Fu), (int)((x.w >> s4) & 0x0F0F0F0Fu)};
            } else {
                return *(const i32x4*)(sW + (wn * 32 * TN + j * 32 + l32) * S::WPitch + kslot(b) * 32 + 16 * hi);
            }
        };
        // Q6_K sub-block h of block b: the lanes holding the other half (hi != h) read the zero
        // row, so the MFMA sums only this sub-block's 16 products
        auto frag_b_sub = [&](int b, int j, int h) -> i32x4 {
            const int row = (hi == h) ? wn * 32 * TN + j * 32 + l32 : BN;
            return *(const i32x4*)(sW + row * S::WPitch + b * 32 + 16 * hi);
        };
        // The MFMA computes the transposed tile D[n][m] (A operand = weight fragment, B operand =
        // activation fragment): lane l holds activation row m = l % 32 and the 16 weight rows
        // n = 8*(r/4) + 4*(l/32) + r%4, so its activation scales are two scalars and its weight
        // scales 16 floats that stay in registers across the TM row tiles of a block.
        f32x4 edw[4];
        auto epilogue = [&](int b, int u, int i, int j, const i32x16& res) {
            const int lm = wm * 32 * TM + i * 32 + l32;          // local activation row
            if constexpr (DUMP) {
                const int nbase = wn * 32 * TN + j * 32 + 4 * hi;    // local weight row of r = 0
                const int gm = m0 + lm;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int gn = n0 + nbase + 8 * (r >> 2) + (r & 3);
                    if (gm < M && gn < N)
                        dump[((size_t)gm * N + gn) * nb * S::SUB + (kb0 + b) * S::SUB + (u - b * S::SUB)] = res[r];
                }
            } else {
                const int nbase = wn * 32 * TN + j * 32 + 4 * hi;    // local weight row of r = 0
                if (i == 0) {
#pragma unroll
                    for (int q = 0; q < 4; q++) edw[q] = *(const f32x4*)&sDw[u][nbase + 8 * q];
                }
                const float da = sDa[b][lm], nc = sNc[b][lm];
#pragma unroll
                for (int q = 0; q < 4; q++) {
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        // copy the element out first: bit_cast of an ext-vector element lvalue
                        // reads element 0 with this compiler
                        const int e = res[4 * q + p];
                        const float f = __builtin_bit_cast(float, e);
                        const float x = fmaf(f, da, nc);        // sumi * d_a'
                        acc[i][j][4 * q + p] = fmaf(edw[q][p], x, acc[i][j][4 * q + p]);
                    }
                }
            }
        };

        // KB*SUB*TN*TA MFMAs per K step, over the wave's first TA of its TM row tiles; step
        // q = ((b*SUB + h)*TN + j)*TA + i.  For Q6_K the two 16-element sub-blocks of a block are
        // separate MFMAs whose weight fragment keeps only the lanes holding that half
        // (k = 16*hi ..; the others read the zero row); one K = 16 MFMA per sub-block instead measured slower (M = 128,
        // N = 14336, K = 4096: 65.6 vs 63.0 us, its fragments cost registers the 64 x 64 tile
        // then spills).  The MFMA of step q+1 is issued before the epilogue of step q.
        constexpr int SUBN = S::SUB;
        auto compute = [&](auto ta) __attribute__((always_inline)) {
            constexpr int TA = decltype(ta)::value;
            constexpr int NQ = KB * SUBN * TA * TN;
            i32x4 af[TA], bf[TN];
            auto mfma_step = [&](int q) -> i32x16 {
                const int b = q / (SUBN * TA * TN), h = (q / (TA * TN)) % SUBN;
                const int j = (q / TA) % TN, i = q % TA;
                if (q % (SUBN * TA * TN) == 0) {
#pragma unroll
                    for (int ii = 0; ii < TA; ii++) af[ii] = frag_a(b, ii);
                    if constexpr (SUBN == 1) {
#pragma unroll
                        for (int jj = 0; jj < TN; jj++) bf[jj] = frag_b(b, jj);
                    }
                }
                if constexpr (SUBN == 2) {
                    if (q % (TA * TN) == 0) {
#pragma unroll
                        for (int jj = 0; jj < TN; jj++) bf[jj] = frag_b_sub(b, jj, h);
                    }
                }
                return __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j], af[i], bias, 0, 0, 0);
            };
            // the compute phase of this wave goes first at instruction issue: with two workgroups
            // per CU the other one is usually staging (Q4_K M = 128: 50.0 -> 45.8 us, Q8_0
            // M = 2048 -2%, the rest level)
            __builtin_amdgcn_s_setprio(2);
            i32x16 cur = mfma_step(0);
#pragma unroll
            for (int q = 0; q < NQ; q++) {
                const int b = q / (SUBN * TA * TN), h = (q / (TA * TN)) % SUBN;
                const int j = (q / TA) % TN, i = q % TA;
                i32x16 nxt = bias;
                if (q + 1 < NQ) nxt = mfma_step(q + 1);
                epilogue(b, b * SUBN + h, i, j, cur);
                cur = nxt;
            }
            __builtin_amdgcn_s_setprio(0);
        };
        // A wave whose rows all lie past the tile's last row (ragged MoE tiles, the last row
        // tile of a ragged M) skips its MFMAs and epilogues; staging and barriers stay shared.
        // In a ragged MoE tile a wave also skips those of its row tiles that hold no row.
        if (wave_has_rows) {
            if constexpr (MOE && TM > 1) {
                // explicit cases (a recursive dispatch was not inlined: the accumulators then
                // went to scratch memory, 15x slower)
                static_assert(TM <= 4, "row tiles per wave");
                const int nta = min(TM, (wave_rows + 31) / 32);   // row tiles with rows, >= 1
                if (nta >= TM) {
                    compute(IntC<TM>{});
                } else if (nta == 1) {
                    compute(IntC<1>{});
                } else if constexpr (TM >= 3) {
                    if (nta == 2) compute(IntC<2>{});
                    else if constexpr (TM >= 4) compute(IntC<3>{});
                }
            } else {
                compute(IntC<TM>{});
            }
        }

        if constexpr (SIDE_MFMA && !DUMP) {
            // side term: acc[n][m] += sum_k f[n][k] * (-s_a[m][k]) over the staged blocks, f = d_w
            // (Q4_0, Q5_0), -m (Q4_1, Q5_1) or dmin*m/8 as an fp16 hi + lo pair (Q4_K); f16 MFMA
            // over 8 block slots, exact products
#pragma unroll
            for (int i = 0; i < TM; i++) {
                if (MOE && wave_rows <= 32 * i) continue;   // a row tile without rows (wave-uniform)
                const int arow = wm * 32 * TM + i * 32 + l32;
                const f16x4 sa4 = *(const f16x4*)&sSaH[arow][4 * shalf(arow, hi)];
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int wrow = wn * 32 * TN + j * 32 + l32;
                    const f16x4 dw4 = *(const f16x4*)&sDwH[wrow][4 * shalf(wrow, hi)];
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x8f16(dw4, sa4, acc[i][j], 0, 0, 0);
                    if constexpr (WT == kWQ4K) {
                        const f16x4 dl4 = *(const f16x4*)&sDwL[wrow][4 * shalf(wrow, hi)];
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x8f16(dl4, sa4, acc[i][j], 0, 0, 0);
                    }
                }
            }
        }
        if constexpr (SIDE_BF && !DUMP) {
            // block_q8f side term: acc[n][m] += sum over the staged blocks of d_w * (-s_a), as the six
            // exact products of the bf16 parts (d_w hi, lo) x (-s_a hi, mid, lo) on the bf16 MFMA:
            // MFMA e covers part pairs 2e (k = 0..7, the lanes with hi = 0) and 2e + 1 (k = 8..15)
            // over the 8 block slots, pair p = (d_w part p / 3, s_a part p % 3)
            typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const int arow = wm * 32 * TM + i * 32 + l32;
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int wrow = wn * 32 * TN + j * 32 + l32;
#pragma unroll
                    for (int e = 0; e < 3; e++) {
                        const int pr = 2 * e + hi;
                        const bf16x8 wv = *(const bf16x8*)&sDwB[pr / 3][wrow][0];
                        const bf16x8 av = *(const bf16x8*)&sSaB[pr % 3][arow][0];
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wv, av, acc[i][j], 0, 0, 0);
                    }
                }
            }
        }
        __syncthreads();
    }

    if constexpr (MOE) {
        // Gathered rows scatter-add into out[token][n]: route each wave's tile through LDS (the
        // staging buffer is free after the last K step's barrier) so that the atomics of one
        // instruction cover 32 consecutive columns of one token instead of 32 tokens.
        constexpr int kTP = 33;   // padded row pitch (floats) of the [32 m][32 n] transpose
        static_assert(T::NT / 64 * 32 * kTP * 4 <= BM * T::APitch, "transpose scratch fits the activation tile");
        float* tp = (float*)sA + wave * 32 * kTP;
#pragma unroll
        for (int i = 0; i < TM; i++) {
            if (wave_rows <= 32 * i) break;   // no rows in this or a later row tile (wave-uniform)
#pragma unroll
            for (int j = 0; j < TN; j++) {
#pragma unroll
                for (int r = 0; r < 16; r++) tp[l32 * kTP + 8 * (r >> 2) + 4 * hi + (r & 3)] = acc[i][j][r];
                __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes done
                wave_lds_exchange();
                const int gn = n0 + wn * 32 * TN + j * 32 + l32;
#pragma unroll
                for (int p = 0; p < 16; p++) {
                    const int lm = wm * 32 * TM + i * 32 + 2 * p + hi;   // local activation row
                    if (lm < M && gn < N) {
                        const float v = tp[(2 * p + hi) * kTP + l32] * sWt[lm];
                        if (moe.scratch) moe.scratch[(size_t)sRows[lm] * N + gn] = v;
                        else unsafeAtomicAdd(C + (size_t)sTok[lm] * N + gn, v);
                    }
                }
                wave_lds_exchange();
            }
        }
    } else if constexpr (!DUMP) {
        constexpr float out_scale = S::out_scale;
        const bool vec_ok = (N % 4) == 0 && (((uintptr_t)C & 15u) == 0);
        if (trans) {
            // transposed output [N][M]: for each of its 16 weight rows the 32 lanes of a half-wave
            // write 32 consecutive activation rows
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int gm = m0 + wm * 32 * TM + i * 32 + l32;
                    if (gm >= M) continue;
                    const int nbase = n0 + wn * 32 * TN + j * 32 + 4 * hi;
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int gn = nbase + 8 * (r >> 2) + (r & 3);
                        if (gn < N) C[(size_t)gn * M + gm] = out_scale * acc[i][j][r];
                    }
                }
            return;
        }
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int lm = wm * 32 * TM + i * 32 + l32;
                const int gm = m0 + lm;
                if (gm >= M) continue;
                const int nbase = n0 + wn * 32 * TN + j * 32 + 4 * hi;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int gn = nbase + 8 * q;   // this lane's 4 consecutive outputs gn .. gn + 3
                    if (vec_ok && gn + 3 < N) {
                        *(f32x4*)(C + (size_t)gm * N + gn) =
                            f32x4{out_scale * acc[i][j][4 * q], out_scale * acc[i][j][4 * q + 1],
                                  out_scale * acc[i][j][4 * q + 2], out_scale * acc[i][j][4 * q + 3]};
                    } else {
#pragma unroll
                        for (int p = 0; p < 4; p++)
                            if (gn + p < N) C[(size_t)gm * N + gn + p] = out_scale * acc[i][j][4 * q + p];
                    }
                }
            }
    }
}

// ---- the LDS-DMA GEMM: planar block_q8_1 activations, nibble weights --------------------------
// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane (no VGPRs); the
// caller waits with s_waitcnt vmcnt before the data is read.
__device__ __forceinline__ void dma16(const void* src, void* lds) {
    __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                     (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
__device__ __forceinline__ void wait_vmem_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// 128 x 128 tiles of Q4_0 / Q4_1 weights against planar block_q8_1 activations, the same
// arithmetic as mmq_kernel (magic-bias epilogue, f16-MFMA side term) in K steps of 4 blocks
// with every LDS array double-buffered, so the loads of step k+1 run under the MFMAs of step k:
//  * every wave copies its share of step k+1's activation planes into the other buffer by DMA
//    (21 wave instructions per step: 16 KiB of quants, 4 KiB of (d, nc) pairs, 1 KiB of sa)
//    and loads half a weight row of step k+1 per thread (2 blocks) into VGPRs;
//  * all four waves compute step k (each 128 rows x 32 columns, as the 128 x 128 tile of
//    mmq_kernel); then the weight halves are unpacked into the other buffer, the DMA is waited
//    for, and one barrier ends the step.
// (Every wave does the same work: splitting the roles between waves left a register copy of
// the weight words at the branches' join that made every wave wait for its loads before
// computing.)
// The quants are stored without padding, with the 16-byte pieces of a row XOR-swizzled (piece p
// of row r at slot p ^ ((r / 2) % 8)): a 128-byte row spans half of the 64 banks, so rows of
// one parity share a bank half, and the swizzle spreads the 8 rows of each parity among a
// fragment read's 16 consecutive rows over the 8 slots; the 16 lanes served together then hit
// 16 different bank groups (the plain p ^ (r % 8) left 2-way conflicts: 5.5e6 conflict cycles
// per launch).  The slots of one DMA instruction are 8 consecutive rows, so lane l of
// instruction i sources piece (l % 8) ^ ((4 i + l / 16) % 8).
// MOE (the expert-grouped GEMM): workgroup y is entry y of the tile schedule (128-row tiles of one
// expert; surplus workgroups of the worst-case grid return at once).  Its planar rows are the
// tile's rows of the expert-sorted entries (the gathered planar quantiser wrote them), the weights
// are its expert's, a tile of at most 32 or 64 rows runs a K loop over that many rows (the others
// stage no activation quants), and the output is added, weighted by the routing probability, into
// C[token][n] through an LDS transpose (coalesced atomics; per-entry rows into moe.scratch when
// top_k > 2).
template <int WT, bool MOE = false>
__global__ __launch_bounds__(256, 2) void mmq_planar_kernel(const uint8_t* __restrict__ W, PlanarQ81 A,
                                                           float* __restrict__ C, int M, int N, int nb, MoeTiles moe) {
    static_assert(WT == kWQ40 || WT == kWQ41, "nibble-staged weights");
    constexpr int KB = 4, BM = 128, BN = 128, TM = 4;
    using S = WShape<WT, KB>;
    constexpr int WNW = S::Chunk / 4;   // weight words per row and step
    __shared__ __attribute__((aligned(16))) uint8_t sA0[BM * 128], sA1[BM * 128];
    __shared__ __attribute__((aligned(16))) uint8_t sW0[BN * S::WPitch], sW1[BN * S::WPitch];
    __shared__ __attribute__((aligned(16))) float sDn0[KB * BM * 2], sDn1[KB * BM * 2];   // (d, nc) pairs
    __shared__ __attribute__((aligned(16))) float sDw0[KB * BN], sDw1[KB * BN];
    __shared__ __attribute__((aligned(16))) uint16_t sSa0[BM * 4], sSa1[BM * 4];
    // side-term weight factor per row and block; row BN stays zero (read by the lanes holding
    // the f16 MFMA's k = 4..7, for which a step has no blocks)
    __shared__ __attribute__((aligned(16))) uint16_t sDh0[(BN + 1) * 4], sDh1[(BN + 1) * 4];

    __shared__ int32_t sRows[MOE ? BM : 1];   // MoE: entry index of each tile row
    __shared__ int32_t sTok[MOE ? BM : 1];    // MoE: its token (output row)
    __shared__ float sWt[MOE ? BM : 1];       // MoE: its routing weight * out_scale

    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int l32 = lane & 31, hi = lane >> 5;
    int m0 = (int)blockIdx.y * BM;
    int n0 = (int)blockIdx.x * BN;
    if constexpr (!MOE) {
        // workgroup x is a linear tile index, each XCD (x % 8) taking a contiguous run of row-major
        // tiles: whole rows of tiles per XCD, so each XCD's L2 fetches its activation rows once
        const int gn = (N + BN - 1) / BN, tiles = gn * ((M + BM - 1) / BM);
        const int L = xcd_tile((int)blockIdx.x, (int)gridDim.x);
        if (L >= tiles) return;   // padding of the grid to a multiple of 8 (whole workgroup)
        m0 = (L / gn) * BM;
        n0 = (L % gn) * BN;
    }
    int rows_here = BM;   // MoE: rows of this tile
    if constexpr (MOE) {
        // schedule values are wave-uniform (read once, broadcast), so the row-count dispatch below
        // is a scalar branch
        const int tile = blockIdx.y;
        if (tile >= __builtin_amdgcn_readfirstlane(moe.num_tiles[0])) return;   // surplus workgroups
        const int e = __builtin_amdgcn_readfirstlane(moe.tile_expert[tile]);
        m0 = __builtin_amdgcn_readfirstlane(moe.tile_row0[tile]);
        rows_here = min(BM, __builtin_amdgcn_readfirstlane(moe.expert_end[e]) - m0);
        M = m0 + rows_here;                              // DMA sources past the tile's rows read its last row
        W += (size_t)e * moe.expert_stride;
        if (t < BM) {
            const int ent = moe.rows[m0 + min(t, rows_here - 1)];
            sRows[t] = ent;
            sTok[t] = ent / moe.top_k;
            sWt[t] = moe.weights[ent] * S::out_scale;
        }
    }
    const int K = nb * 32;
    const int nsteps = nb / KB, Z = (int)gridDim.z, z = (int)blockIdx.z;
    const int kb_lo = (int)((long long)nsteps * z / Z) * KB, kb_hi = (int)((long long)nsteps * (z + 1) / Z) * KB;
    C += (size_t)z * (size_t)M * (size_t)N;

    // ---- per-lane DMA source offsets ----
    // quants: wave w fills slots 256 w .. 256 w + 255 (rows 32 w .. 32 w + 31; rows past M read
    // row M-1); (d, nc): wave w copies block w of the step, lane -> rows 2 lane, 2 lane + 1; sa:
    // one instruction of wave 3, lane -> rows 2 lane, 2 lane + 1
    const int8_t* qtile = A.q + (size_t)m0 * K;
    uint32_t qoff[4];
    {
#pragma unroll
        for (int ii = 0; ii < 4; ii++) {
            const int p = (lane & 7) ^ ((4 * ii + (lane >> 4)) & 7);
            const int r = min(m0 + 32 * wave + 8 * ii + (lane >> 3), M - 1) - m0;
            qoff[ii] = (uint32_t)r * (uint32_t)K + 16u * p;
        }
    }
    auto dma_act = [&](auto par, int kb0, bool qa) __attribute__((always_inline)) {
        constexpr int P = decltype(par)::value;
        uint8_t* dA = P ? sA1 : sA0;
        const int8_t* qs = qtile + (size_t)kb0 * 32;
        if (qa) {
#pragma unroll
            for (int ii = 0; ii < 4; ii++) dma16(qs + qoff[ii], dA + (4 * wave + ii) * 1024);
        }
        dma16(A.dn + 2 * ((size_t)(kb0 + wave) * A.mp + m0 + 2 * lane), (P ? sDn1 : sDn0) + 256 * wave);
        if (wave == 3) dma16(A.sa + ((size_t)(kb0 >> 2) * A.mp + m0 + 2 * lane) * 4, P ? sSa1 : sSa0);
    };

    // ---- weights: thread t stages blocks 2h, 2h + 1 (h = t / 128) of row t % 128 ----
    // (consecutive lanes write consecutive rows' scales and quants, free of LDS bank conflicts;
    // lane pairs sharing a row left 2-way conflicts on every scale write: 1.3e6 conflict cycles
    // per launch.  4-byte loads of the 36- / 40-byte half chunk: 8-byte loads from the 8-byte
    // boundary below, with Q4_0's second half re-aligned by a word, measured 1% slower.)
    constexpr int HW = WNW / 2;   // words per half chunk
    const int wsr = t & 127, wh = t >> 7;
    uint32_t pre[HW + 1];
    auto load_w = [&](int kb0) __attribute__((always_inline)) {
        const int wr = min(n0 + wsr, N - 1);
        const uint32_t* p = (const uint32_t*)(W + (size_t)wr * nb * S::BB + (size_t)(kb0 + 2 * wh) * S::BB);
#pragma unroll
        for (int i = 0; i < HW; i++) pre[i] = p[i];
        pre[HW] = 0;
    };
    auto store_w = [&](auto par) __attribute__((always_inline)) {
        constexpr int P = decltype(par)::value;
        uint8_t* dW = P ? sW1 : sW0;
        float* dDw = P ? sDw1 : sDw0;
        uint16_t* dDh = P ? sDh1 : sDh0;
        uint32_t dh[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int kb = 2 * wh + j, off = j * S::BB;
            const uint32_t dwb = half_at(pre, off);
            dDw[kb * BN + wsr] = f16_to_f32(dwb);
            // side factor against -s_a: d_w (Q4_0) or -m (Q4_1)
            dh[j] = (WT == kWQ41) ? (half_at(pre, off + 2) ^ 0x8000u) : dwb;
            constexpr int q = (WT == kWQ40) ? 2 : 4;   // offset of qs
            *(u32x4*)(dW + wsr * S::WPitch + kb * 16) =
                u32x4{word_at(pre, off + q), word_at(pre, off + q + 4), word_at(pre, off + q + 8),
                      word_at(pre, off + q + 12)};
        }
        *(uint32_t*)(dDh + 4 * wsr + 2 * wh) = dh[0] | (dh[1] << 16);
    };

    // ---- compute ----
    f32x16 acc[TM];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][r] = 0.0f;
    i32x16 bias;
#pragma unroll
    for (int r = 0; r < 16; r++) bias[r] = (int)kMagic;
    const int wn = wave;   // four waves side by side along N, each over all 128 rows
    int aoff[KB];          // swizzled byte offset of piece 2b + hi of row l32
#pragma unroll
    for (int b = 0; b < KB; b++) aoff[b] = l32 * 128 + (((2 * b + hi) ^ ((l32 >> 1) & 7)) << 4);
    const int woff = (wn * 32 + l32) * S::WPitch;
    const int dh_idx = hi ? BN * 4 : (wn * 32 + l32) * 4;
    const int nbase = wn * 32 + 4 * hi;   // local weight row of r = 0

    // TA: the row sub-tiles a K loop computes (TM, or fewer for a ragged MoE tile; each value
    // is a K loop of its own, free of per-sub-tile branches: a wave-uniform branch around each
    // sub-tile's epilogue inside the loop cost 10% on full tiles)
    auto compute = [&](auto par, auto tav) __attribute__((always_inline)) {
        constexpr int P = decltype(par)::value;
        constexpr int TA = decltype(tav)::value;
        const uint8_t* cA = P ? sA1 : sA0;
        const uint8_t* cW = P ? sW1 : sW0;
        const float* cDn = P ? sDn1 : sDn0;
        const float* cDw = P ? sDw1 : sDw0;
        const uint16_t* cSa = P ? sSa1 : sSa0;
        const uint16_t* cDh = P ? sDh1 : sDh0;
        constexpr int NQ = KB * TA;
        i32x4 af[TA], afn[TA], bf;
        u32x4 bxn;
        f32x4 edw[4];
        auto unpack = [&](const u32x4& x) -> i32x4 {
            const int s4 = 4 * hi;
            return i32x4{(int)((x.x >> s4) & 0x0F0F0F0Fu), (int)((x.y >> s4) & 0x0F0F0F0Fu),
                         (int)((x.z >> s4) & 0x0F0F0F0Fu), (int)((x.w >> s4) & 0x0F0F0F0Fu)};
        };
        if constexpr (TA >= 2) {
            // software pipeline, one region per MFMA q: issue the MFMA of q + 1, run the first
            // quarter of q's epilogue (its LDS operands were read during region q - 1), read the
            // operands of q + 1 (its (d, nc) pair; at a block's first sub-tile the next block's
            // fragments; a sub-tile before its last one the next block's weight scales), then the
            // rest of q's epilogue.  The scheduling barriers hold that order: left to itself the
            // compiler sank each MFMA to its first use and waited on the LDS reads it had just
            // issued (config 2, GEMM alone: 93.4 -> 91.5 us, MoE config 4: 264 -> 257, same bits).
            auto quarter = [&](const i32x16& c, auto iv, int qq, const f32x2& dn) __attribute__((always_inline)) {
                constexpr int i = decltype(iv)::value;
                float x[4];
#pragma unroll
                for (int p = 0; p < 4; p++) {
                    // through an int: hipcc's __builtin_bit_cast of the vector element itself
                    // read element 0 for every p
                    const int e = c[4 * qq + p];
                    x[p] = fmaf(__builtin_bit_cast(float, e), dn.x, dn.y);   // sumi * d_a'
                }
#pragma unroll
                for (int p = 0; p < 4; p++) acc[i][4 * qq + p] = fmaf(edw[qq][p], x[p], acc[i][4 * qq + p]);
            };
            f32x4 edwn[4];
            f32x2 dnc = *(const f32x2*)&cDn[2 * l32];
#pragma unroll
            for (int qq = 0; qq < 4; qq++) edw[qq] = *(const f32x4*)&cDw[nbase + 8 * qq];
#pragma unroll
            for (int ii = 0; ii < TA; ii++) af[ii] = *(const i32x4*)(cA + ii * 32 * 128 + aoff[0]);
            bf = unpack(*(const u32x4*)(cW + woff));
            __builtin_amdgcn_s_setprio(2);
            i32x16 cur = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf, af[0], bias, 0, 0, 0);
            static_for<NQ>([&](auto qv) __attribute__((always_inline)) {
                constexpr int q = decltype(qv)::value;
                constexpr int b = q / TA, i = q % TA;
                i32x16 nxt = bias;
                if constexpr (q + 1 < NQ) {
                    if constexpr (i + 1 < TA) {
                        nxt = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf, af[i + 1], bias, 0, 0, 0);
                    } else {
                        bf = unpack(bxn);
#pragma unroll
                        for (int ii = 0; ii < TA; ii++) af[ii] = afn[ii];
                        nxt = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf, af[0], bias, 0, 0, 0);
                    }
                    asm volatile("" : "+v"(nxt));   // pins the issue here, ahead of q's epilogue
                }
                __builtin_amdgcn_sched_barrier(0);
                quarter(cur, IntC<i>{}, 0, dnc);
                __builtin_amdgcn_sched_barrier(0);
                f32x2 dnn = dnc;
                if constexpr (q + 1 < NQ) {
                    constexpr int bn = (q + 1) / TA, in = (q + 1) % TA;
                    dnn = *(const f32x2*)&cDn[2 * (bn * BM + in * 32 + l32)];
                }
                if constexpr (i == 0 && b + 1 < KB) {
#pragma unroll
                    for (int ii = 0; ii < TA; ii++) afn[ii] = *(const i32x4*)(cA + ii * 32 * 128 + aoff[b + 1]);
                    bxn = *(const u32x4*)(cW + woff + (b + 1) * 16);
                }
                if constexpr (i == TA - 2 && b + 1 < KB) {
#pragma unroll
                    for (int qq = 0; qq < 4; qq++) edwn[qq] = *(const f32x4*)&cDw[(b + 1) * BN + nbase + 8 * qq];
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int qq = 1; qq < 4; qq++) quarter(cur, IntC<i>{}, qq, dnc);
                if constexpr (i == TA - 1 && b + 1 < KB) {
#pragma unroll
                    for (int qq = 0; qq < 4; qq++) edw[qq] = edwn[qq];
                }
                dnc = dnn;
                cur = nxt;
            });
        } else {
    #pragma unroll
            for (int ii = 0; ii < TA; ii++) af[ii] = *(const i32x4*)(cA + ii * 32 * 128 + aoff[0]);
            bf = unpack(*(const u32x4*)(cW + woff));
            __builtin_amdgcn_s_setprio(2);
            i32x16 cur = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf, af[0], bias, 0, 0, 0);
    #pragma unroll
            for (int q = 0; q < NQ; q++) {
                const int b = q / TA, i = q % TA;
                if (i == 0 && b + 1 < KB) {
                    // the next block's fragments, a block ahead of their MFMAs
    #pragma unroll
                    for (int ii = 0; ii < TA; ii++) afn[ii] = *(const i32x4*)(cA + ii * 32 * 128 + aoff[b + 1]);
                    bxn = *(const u32x4*)(cW + woff + (b + 1) * 16);
                    __builtin_amdgcn_sched_barrier(0);
                }
                i32x16 nxt = bias;
                if (q + 1 < NQ) {
                    if (i + 1 < TA) {
                        nxt = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf, af[i + 1], bias, 0, 0, 0);
                    } else {
                        bf = unpack(bxn);
    #pragma unroll
                        for (int ii = 0; ii < TA; ii++) af[ii] = afn[ii];
                        nxt = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf, af[0], bias, 0, 0, 0);
                    }
                }
                if (i == 0) {
    #pragma unroll
                    for (int qq = 0; qq < 4; qq++) edw[qq] = *(const f32x4*)&cDw[b * BN + nbase + 8 * qq];
                }
                {
                    const int lm = i * 32 + l32;
                    const f32x2 dn = *(const f32x2*)&cDn[2 * (b * BM + lm)];
                    const float da = dn.x, nc = dn.y;
    #pragma unroll
                    for (int qq = 0; qq < 4; qq++) {
    #pragma unroll
                        for (int p = 0; p < 4; p++) {
                            const int e = cur[4 * qq + p];
                            const float f = __builtin_bit_cast(float, e);
                            const float x = fmaf(f, da, nc);   // sumi * d_a'
                            acc[i][4 * qq + p] = fmaf(edw[qq][p], x, acc[i][4 * qq + p]);
                        }
                    }
                }
                cur = nxt;
            }
        }
        __builtin_amdgcn_s_setprio(0);
        // side term over the step's 4 blocks (f16 MFMA, exact products; k = 4..7 read zeros)
        const f16x4 dw4 = *(const f16x4*)&cDh[dh_idx];
#pragma unroll
        for (int i = 0; i < TA; i++) {
            const f16x4 sa4 = *(const f16x4*)&cSa[(i * 32 + l32) * 4];
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x8f16(dw4, sa4, acc[i], 0, 0, 0);
        }
    };

    // ---- pipeline ----
    if (t < 4) {
        sDh0[BN * 4 + t] = 0;
        sDh1[BN * 4 + t] = 0;
    }
    auto run = [&](auto tav) __attribute__((always_inline)) {
        constexpr int TA = decltype(tav)::value;
        // waves past the computed sub-tiles stage no activation quants (no wave reads them)
        const bool qa = wave < TA;
        if (kb_lo < kb_hi) {
            dma_act(IntC<0>{}, kb_lo, qa);
            load_w(kb_lo);
            store_w(IntC<0>{});
            wait_vmem_all();
        }
        __syncthreads();
        auto step = [&](auto par, int kb0) __attribute__((always_inline)) {
            constexpr int P = decltype(par)::value;
            const bool more = kb0 + KB < kb_hi;
            if (more) {
                dma_act(IntC<1 - P>{}, kb0 + KB, qa);
                load_w(kb0 + KB);
            }
            compute(par, tav);
            if (more) {
                store_w(IntC<1 - P>{});
                wait_vmem_all();
            }
            __syncthreads();
        };
        for (int kb0 = kb_lo; kb0 < kb_hi; kb0 += 2 * KB) {
            step(IntC<0>{}, kb0);
            if (kb0 + KB < kb_hi) step(IntC<1>{}, kb0 + KB);
        }
    };
    if constexpr (MOE) {
        // wave-uniform: the tile's row count comes from the broadcast schedule
        const int ta = (rows_here + 31) >> 5;
        if (ta >= 3) run(IntC<TM>{});
        else if (ta == 2) run(IntC<2>{});
        else run(IntC<1>{});
    } else {
        run(IntC<TM>{});
    }

    // ---- output ----
    if constexpr (MOE) {
        // the staging buffers are free after the last K step's barrier: each wave transposes its
        // [32 rows][32 columns] sub-tiles through a 33-float-pitch scratch, so that one atomic
        // instruction covers 32 consecutive columns of one token
        constexpr int kTP = 33;
        static_assert(2 * 32 * kTP * 4 <= BM * 128, "two waves' transpose scratch fits one activation buffer");
        float* tp = (float*)(wave < 2 ? sA0 : sA1) + (wave & 1) * 32 * kTP;
        const int gn = n0 + nbase - 4 * hi + l32;   // this lane's column after the transpose
#pragma unroll
        for (int i = 0; i < TM; i++) {
            if (32 * i >= rows_here) break;   // no rows in this or a later sub-tile (wave-uniform)
#pragma unroll
            for (int r = 0; r < 16; r++) tp[l32 * kTP + 8 * (r >> 2) + 4 * hi + (r & 3)] = acc[i][r];
            __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS writes done
            wave_lds_exchange();
#pragma unroll
            for (int p = 0; p < 16; p++) {
                const int lm = i * 32 + 2 * p + hi;   // tile row
                if (lm < rows_here && gn < N) {
                    const float v = tp[(2 * p + hi) * kTP + l32] * sWt[lm];
                    if (moe.scratch) moe.scratch[(size_t)sRows[lm] * N + gn] = v;
                    else unsafeAtomicAdd(C + (size_t)sTok[lm] * N + gn, v);
                }
            }
            wave_lds_exchange();
        }
        return;
    }
    constexpr float out_scale = S::out_scale;
    const bool vec_ok = (N % 4) == 0 && (((uintptr_t)C & 15u) == 0);
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const int gm = m0 + i * 32 + l32;
        if (gm >= M) continue;
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            const int gn = n0 + nbase + 8 * qq;   // this lane's 4 consecutive outputs gn .. gn + 3
            if (vec_ok && gn + 3 < N) {
                *(f32x4*)(C + (size_t)gm * N + gn) =
                    f32x4{out_scale * acc[i][4 * qq], out_scale * acc[i][4 * qq + 1], out_scale * acc[i][4 * qq + 2],
                          out_scale * acc[i][4 * qq + 3]};
            } else {
#pragma unroll
                for (int p = 0; p < 4; p++)
                    if (gn + p < N) C[(size_t)gm * N + gn + p] = out_scale * acc[i][4 * qq + p];
            }
        }
    }
}

// ---- tile configurations ----------------------------------------------------------
// 128 rows x 32 columns per wave: one weight fragment (the one that needs its nibbles unpacked)
// per four MFMAs (Q4_0 M = 2048, N = K = 4096: 99 vs 101 us for 64 x 64 per wave)
using TileL = Tile<128, 128, 8, 4, 1, 2>;   // large M
using TileN = Tile<128, 64, 8, 2, 1, 2>;    // half the columns per workgroup: twice the workgroups
using TileS = Tile<64, 64, 8, 1, 1, 3>;     // 32 x 32 per wave, 4x the workgroups of TileL
// half the K step without prefetch (selected only explicitly: its exposed load latency makes it
// the slowest 128 x 128 form, Q4_0 M = 2048, N = K = 4096: 192 us); two workgroups per CU, as
// three would need more registers than a wave then has
using TileK4 = Tile<128, 128, 4, 2, 2, 2>;
using TileT = Tile<32, 128, 8, 1, 1, 3>;    // skinny: M <= 32, the four waves side by side along N
using TileP = Tile<128, 128, 4, 2, 2, 2, true>;  // 128 x 128, K step 4, next step's loads prefetched
// 64 x 128, 64 x 32 per wave, 64-row granularity (MoE config 4: 294 vs 310 us for 32 x 64 per
// wave; Q4_K M = 128, N = 14336: 42.8 vs 45.5)
using TileW = Tile<64, 128, 8, 2, 1, 3>;

static thread_local int g_mmq_config = 0;  // 0 = automatic; set per host thread

int mmq_set_config(int c) {
    if (c < 0 || c > 8) return -1;
    g_mmq_config = c;
    return 0;
}

template <class T>
static int grid_wgs(int M, int N) {
    return ((N + T::BN - 1) / T::BN) * ((M + T::BM - 1) / T::BM);
}

// Measured on MI355X (M = 3 .. 2048, N = 512 .. 18944, K = 2560 .. 18944, block_q8_1 input, us):
//  * nibble-staged Q4_0 / Q4_1: the 128 x 128 tile from M = 256 on while it covers the CUs
//    (Q4_0 M = 2048, N = K = 4096: 103 vs 113 prefetched K-step-4), or with long rows (K >= 9728)
//    when the 64 x 64 grid has 512 workgroups or more (M = 512, N = 4096, K = 14336: 103 vs
//    117; M = 1024, N = 3584, K = 18944: 243 vs 273), else 64 x 64 (M = 512, N = K = 4096: 42.5
//    vs 46.5); 32 x 128 at M <= 32 (N = 14336, K = 4096: 21.1 vs 25.2 at M = 8) and for larger
//    grids below M = 256 (M = 64, N = 18944, K = 3584: 37.2 vs 53.7 for 128 x 64);
//  * byte-staged Q8_0 / Q5_0 / Q5_1 need 86 KB of LDS for the 128 x 128 K-step-8 tile (one
//    workgroup per CU); its K-step-4 form with prefetched loads wins on large grids (Q8_0
//    M = 2048, N = K = 4096: 113 vs 128 for 128 x 64 and 187 for K-step 8), 128 x 64 when its
//    grid of 416 .. 512 workgroups fills the CUs in one round (Q8_0 M = 512, N = K = 7168:
//    104 vs 131; M = 1024, N = K = 4096: 71 vs 84), else 64 x 64 (M = 512, N = K = 4096: 41.6
//    vs 46.2 and 46.6);
//  * Q4_K / Q6_K stage one super-block per K step: 128 x 64 while that grid covers the CUs or
//    for long rows below M = 256 (Q6_K M = 128, N = 4096, K = 14336: 58.8 vs 70.0 for 64 x 64),
//    else 64 x 64; Q4_K (nibble-staged) like Q4_0 takes 32 x 128 at M <= 32 (N = 14336,
//    K = 4096, M = 16: 20.5 vs 26.7) up to M = 96, 64 x 128 from there to M = 255, 128 x 128
//    from M = 256 while it covers the CUs (M = 2048, N = K = 4096: 114.5 vs 131.9).
static int pick_config(int wtype, int M, int N, int K) {
    // configuration 8 (the LDS-DMA GEMM, mmq_planar_preferred) is the 128 x 128 tile elsewhere
    if (g_mmq_config == 8) return 1;
    if (g_mmq_config && !(is_kquant(wtype) && (g_mmq_config == 4 || g_mmq_config == 6))) return g_mmq_config;
    constexpr int kCUs = 256;
    const bool nib = (wtype == kWQ40 || wtype == kWQ41), kq = is_kquant(wtype);
    if (nib && M <= 32) return 5;
    if (nib && M >= 256) {
        if (grid_wgs<TileL>(M, N) >= kCUs) return 1;
        if (K >= 9728 && grid_wgs<TileS>(M, N) >= 2 * kCUs) return 1;
        return 3;
    }
    if (nib) return grid_wgs<TileN>(M, N) >= kCUs ? 5 : 3;
    if (!kq) {
        if (grid_wgs<TileP>(M, N) >= 384) return 6;
        const int gn = grid_wgs<TileN>(M, N);
        return (gn >= 416 && gn <= 2 * kCUs) ? 2 : 3;
    }
    if (wtype == kWQ4K) {
        // 33..96 rows: 32 x 128 (N = 14336, K = 4096, M = 96: 36.2 vs 44.8 us for 64 x 64);
        // 97..255 rows: 64 x 128, split along K while its grid is small (M = 128: 40.8 vs 45.4 for
        // 32 x 128; M = 192: 53.3 vs 55.0)
        if (M <= 96) return 5;
        if (M >= 256 && grid_wgs<TileL>(M, N) >= kCUs) return 1;
        if (M < 256) return 7;
    }
    if (M < 256 && K >= 9728) return 2;
    if (grid_wgs<TileN>(M, N) >= kCUs) return 2;
    return 3;
}

// Below M = 9 the decode and small-batch kernels usually win; their time grows with M * N * K
// while the MFMA kernel's stays near its ~10 us floor, so for large matrices the MFMA kernel
// takes over.  Fitted to measurements over the quant_gemm definition shapes (M = 5 .. 8,
// block_q8_1 activations, us): the nibble types from M = 7 once N * K >= 2e7 (Q4_0 N = K = 5120,
// M = 8: 12.7 vs 17.9 decode, 15.5 small-batch) and at M = 5, 6 from N * K >= 6e7 (N = 3584,
// K = 18944: 21.6 vs 27.4 decode); Q8_0 from M = 7 once N * K >= 2e7 (N = K = 7168, M = 8: 26.1
// vs 30.7 decode), never at M = 5, 6 (N = 18944, K = 3584: 36.7 vs 27.1 decode).  Where the small-batch
// kernel also applies it keeps rows of up to 3584 elements (Q8_0 N = 18944, K = 3584, M = 8:
// 26.4 vs 36.5).
// K-quants (decode kernel vs MFMA GEMM only): Q4_K from M = 7 once N * K >= 1.2e7 (N = K = 4096,
// M = 8: 1.08x), at M = 5, 6 as below; Q6_K from M = 7 on
// rows of up to 7168 elements once N * K >= 1.5e7 (N = 12288, K = 5120, M = 8: 1.30x; with
// K = 14336 the decode kernel stays 1.15x faster).
bool mmq_preferred(int wtype, int M, int N, int K) {
    // 9-32 rows: the small-batch kernel where it applies (shared activation pieces: K % 128 == 0)
    // and measured faster
    if (M > 8) return !(M <= 32 && (K % 128) == 0 && skinny_preferred(wtype, M, N, K));
    const bool nib = (wtype == kWQ40 || wtype == kWQ41);
    const double nk = (double)N * (double)K;
    // Q4_K at M = 5, 6 against the register-direct decode kernel: the MFMA GEMM on rows of up to
    // 5120 elements once N * K >= 2e7 (N = 12288, K = 5120: 20.9 vs 23.4 us) and on very short
    // rows (N = 7168, K = 512: 6.6 vs 8.2); longer rows stay on the decode kernel (N = 4096,
    // K = 14336: 16.6 vs 19.6)
    if (wtype == kWQ4K)
        return (M >= 7 && nk >= 1.2e7) || (M >= 5 && M <= 6 && ((nk >= 2.0e7 && K <= 5120) || K <= 1024));
    if (wtype == kWQ6K) return M >= 7 && K <= 7168 && nk >= 1.5e7;
    // 3-8 rows of the 32-element types, fitted on the definition shapes (430 cases, fp32 entry;
    // the small-batch kernel with shared activation pieces and the decode kernels are the
    // alternatives): Q8_0 never (the MFMA GEMM was 5-120% slower on every such case), the nibble
    // types on rows of at least 4096 elements once the grid is wide (N >= 18432 from 6 rows on,
    // N >= 100000 from 4) or the matrix large from 7 rows on (N = 128256, K = 4096, Q4_1, M = 8:
    // 0.81x the better alternative; N = 7168, K = 18432, M = 8: 0.94-1.01x; N = 14336, K = 4096,
    // M = 8: 1.20-1.31x, so not there)
    if (!nib) return false;
    return K >= 4096 && ((M >= 6 && N >= 18432) || (M >= 4 && N >= 100000) || (M >= 7 && nk >= 1.3e8));
}

bool mmq_supported(int wtype, int M, int N, int K, const void* W, bool a_aligned16) {
    const uintptr_t wal = (wtype == kWQ6K) ? 3u : 15u;  // Q6_K rows are read per dword
    return (wtype >= kWQ40 && wtype <= kWQ51) && M > 0 && N > 0 && K > 0 && (K % 256) == 0 &&
           (((uintptr_t)W & wal) == 0) && a_aligned16;
}

// Split-K factor for a (tile, M, N, K): grids of fewer than kSplitMinWGs workgroups are split
// along K (at least kSplitMinSteps K steps per split) so that small-M problems still occupy
// the chip; the partial sums go to a workspace and splitk_reduce_kernel adds them in order.
// Larger grids that still leave most CUs below the tile's residency (at most 2/3 of
// 256 x OCC workgroups for the nibble types, 1/2 for the others) are split too when K >= 4096,
// up to that residency with at least 8 K steps per split.  Measured on MI355X against the
// unsplit grid (us, Q4_0 / Q8_0): M = 256, N = 4096, K = 14336 on 64 x 64 tiles 129 -> 77 /
// 130 -> 85; M = 512, N = 2048, K = 7168 64 -> 44 / 59 -> 44; M = 1024, N = 4096, K = 14336 on
// 128 x 128 tiles 254 -> 194.  Past those fractions the reduction costs more than the fuller
// chip gains (Q8_0 M = 512, N = 4096, K = 14336 with 512 of 768: 145 -> 162).
constexpr int kSplitMinWGs = 256, kSplitTargetWGs = 512, kSplitMinSteps = 2, kSplitMax = 16;
constexpr int kCUCount = 256;

template <class T>
static int split_for(int wtype, int M, int N, int K) {
    const int wgs = ((N + T::BN - 1) / T::BN) * ((M + T::BM - 1) / T::BM);
    const int steps = (K / 32) / T::KB;
    if (wgs >= kSplitMinWGs) {
        const int target = kCUCount * T::OCC;
        const bool nib = (wtype == kWQ40 || wtype == kWQ41);
        const int limit = nib ? (2 * target) / 3 : target / 2;
        if (wgs > limit || K < 4096) return 1;
        int sp = (target + wgs - 1) / wgs;
        sp = sp < steps / 8 ? sp : steps / 8;
        return sp < 1 ? 1 : sp;
    }
    int sp = (kSplitTargetWGs + wgs - 1) / wgs;
    sp = sp < steps / kSplitMinSteps ? sp : steps / kSplitMinSteps;
    sp = sp < kSplitMax ? sp : kSplitMax;
    return sp < 1 ? 1 : sp;
}

// C[i] = P[0][i] + P[1][i] + ... in split order (deterministic).  All the splits' loads are
// issued before the first add (the split count is at most kSplitMax), so the kernel costs one
// memory latency instead of one per split.  VEC: 4 consecutive elements per thread as 16-byte
// accesses (mn % 4 == 0 and C 16-byte aligned).
template <bool VEC>
__global__ void splitk_reduce_kernel(const float* __restrict__ P, float* __restrict__ C, int64_t mn, int splits) {
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * (VEC ? 4 : 1);
    if (i >= mn) return;
    if constexpr (VEC) {
        f32x4 v[kSplitMax];
#pragma unroll
        for (int z = 0; z < kSplitMax; z++)
            if (z < splits) v[z] = *(const f32x4*)(P + (size_t)z * (size_t)mn + (size_t)i);
        f32x4 acc = v[0];
#pragma unroll
        for (int z = 1; z < kSplitMax; z++)
            if (z < splits) acc = f32x4{acc.x + v[z].x, acc.y + v[z].y, acc.z + v[z].z, acc.w + v[z].w};
        *(f32x4*)(C + i) = acc;
    } else {
        float v[kSplitMax];
#pragma unroll
        for (int z = 0; z < kSplitMax; z++)
            if (z < splits) v[z] = P[(size_t)z * (size_t)mn + (size_t)i];
        float acc = v[0];
#pragma unroll
        for (int z = 1; z < kSplitMax; z++)
            if (z < splits) acc += v[z];
        C[i] = acc;
    }
}

template <class T, int WT, bool DUMP, bool MOE, int AF = kAQ81>
static hipError_t launch_k(dim3 grid, const uint8_t* W, const uint8_t* A, float* C, int32_t* dump, int M, int N,
                           int nb, const MoeTiles& mt, hipStream_t s, int trans = 0) {
    if constexpr (is_kquant(WT) && (T::KB != 8 || MOE)) {
        return hipErrorNotSupported;
    } else {
        hipLaunchKernelGGL((mmq_kernel<T, WT, DUMP, MOE, AF>), grid, dim3(T::NT), 0, s, W, A, C, dump, M, N, nb, mt, trans);
        return hipGetLastError();
    }
}

template <class T, bool DUMP, bool MOE>
static hipError_t launch_t(int wtype, int afmt, dim3 grid, const uint8_t* W, const uint8_t* A, float* C,
                           int32_t* dump, int M, int N, int nb, const MoeTiles& mt, hipStream_t s, int trans = 0) {
    if (afmt != kAQ81) {
        // the fp32-scale activation blocks: plain GEMM only (no block-dot dump, no MoE)
        if constexpr (DUMP || MOE) {
            return hipErrorNotSupported;
        } else {
            if (afmt == kAQ8S) {
                if (wtype != kWQ80) return hipErrorNotSupported;
                return launch_k<T, kWQ80, false, false, kAQ8S>(grid, W, A, C, dump, M, N, nb, mt, s, trans);
            }
            if (afmt != kAQ8F) return hipErrorNotSupported;
            switch (wtype) {
                case kWQ40: return launch_k<T, kWQ40, false, false, kAQ8F>(grid, W, A, C, dump, M, N, nb, mt, s, trans);
                case kWQ50: return launch_k<T, kWQ50, false, false, kAQ8F>(grid, W, A, C, dump, M, N, nb, mt, s, trans);
                case kWQ80: return launch_k<T, kWQ80, false, false, kAQ8F>(grid, W, A, C, dump, M, N, nb, mt, s, trans);
                default: return hipErrorNotSupported;
            }
        }
    }
    switch (wtype) {
        case kWQ40: return launch_k<T, kWQ40, DUMP, MOE>(grid, W, A, C, dump, M, N, nb, mt, s, trans);
        case kWQ80: return launch_k<T, kWQ80, DUMP, MOE>(grid, W, A, C, dump, M, N, nb, mt, s, trans);
        case kWQ4K: return launch_k<T, kWQ4K, DUMP, MOE>(grid, W, A, C, dump, M, N, nb, mt, s, trans);
        case kWQ6K: return launch_k<T, kWQ6K, DUMP, MOE>(grid, W, A, C, dump, M, N, nb, mt, s, trans);
        case kWQ41: return launch_k<T, kWQ41, DUMP, MOE>(grid, W, A, C, dump, M, N, nb, mt, s, trans);
        case kWQ50: return launch_k<T, kWQ50, DUMP, MOE>(grid, W, A, C, dump, M, N, nb, mt, s, trans);
        case kWQ51: return launch_k<T, kWQ51, DUMP, MOE>(grid, W, A, C, dump, M, N, nb, mt, s, trans);
        default: return hipErrorNotSupported;
    }
}

static int split_cfg(int cfg, int wtype, int M, int N, int K) {
    switch (cfg) {
        case 1: return split_for<TileL>(wtype, M, N, K);
        case 2: return split_for<TileN>(wtype, M, N, K);
        case 3: return split_for<TileS>(wtype, M, N, K);
        case 5: return split_for<TileT>(wtype, M, N, K);
        case 6: return split_for<TileP>(wtype, M, N, K);
        case 7: return split_for<TileW>(wtype, M, N, K);
        default: return split_for<TileK4>(wtype, M, N, K);
    }
}

// splits > 1: C receives splits partial [M][N] results back to back.
template <bool DUMP>
static hipError_t launch_cfg(int cfg, int wtype, int afmt, const uint8_t* W, const uint8_t* A, float* C,
                             int32_t* dump, int M, int N, int K, int splits, hipStream_t s, int trans = 0) {
    const int nb = K / 32;
    const MoeTiles mt{};
    auto grid = [&](int BM, int BN) {
        return dim3((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM), (unsigned)splits);
    };
    switch (cfg) {
        case 1: return launch_t<TileL, DUMP, false>(wtype, afmt, grid(128, 128), W, A, C, dump, M, N, nb, mt, s, trans);
        case 2: return launch_t<TileN, DUMP, false>(wtype, afmt, grid(128, 64), W, A, C, dump, M, N, nb, mt, s, trans);
        case 3: return launch_t<TileS, DUMP, false>(wtype, afmt, grid(64, 64), W, A, C, dump, M, N, nb, mt, s, trans);
        case 5: return launch_t<TileT, DUMP, false>(wtype, afmt, grid(32, 128), W, A, C, dump, M, N, nb, mt, s, trans);
        case 6: return launch_t<TileP, DUMP, false>(wtype, afmt, grid(128, 128), W, A, C, dump, M, N, nb, mt, s, trans);
        case 7: return launch_t<TileW, DUMP, false>(wtype, afmt, grid(64, 128), W, A, C, dump, M, N, nb, mt, s, trans);
        default: return launch_t<TileK4, DUMP, false>(wtype, afmt, grid(128, 128), W, A, C, dump, M, N, nb, mt, s, trans);
    }
}

hipError_t launch_splitk_reduce(const float* P, float* C, int64_t mn, int splits, hipStream_t s) {
    if (splits < 1 || splits > kSplitMax) return hipErrorInvalidValue;
    if ((mn % 4) == 0 && ((uintptr_t)C & 15u) == 0 && ((uintptr_t)P & 15u) == 0) {
        const int64_t n4 = mn / 4;
        hipLaunchKernelGGL(splitk_reduce_kernel<true>, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, P, C, mn,
                           splits);
    } else {
        hipLaunchKernelGGL(splitk_reduce_kernel<false>, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, s, P, C, mn,
                           splits);
    }
    return hipGetLastError();
}

int mmq_splits(int wtype, int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0) return 1;
    return split_cfg(pick_config(wtype, M, N, K), wtype, M, N, K);
}

hipError_t launch_mmq(int wtype, int afmt, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int K,
                      float* partials, hipStream_t s, bool trans) {
    const int cfg = pick_config(wtype, M, N, K);
    const int splits = split_cfg(cfg, wtype, M, N, K);
    if (trans && splits > 1) return hipErrorNotSupported;
    note_engine(KSQ_ENG_MMQ_CFG(cfg) | (splits > 1 ? KSQ_ENG_SPLITK : 0u));
    if (splits == 1) return launch_cfg<false>(cfg, wtype, afmt, W, A, C, nullptr, M, N, K, 1, s, trans ? 1 : 0);
    if (!partials) return hipErrorInvalidValue;
    hipError_t e = launch_cfg<false>(cfg, wtype, afmt, W, A, partials, nullptr, M, N, K, splits, s);
    if (e != hipSuccess) return e;
    return launch_splitk_reduce(partials, C, (int64_t)M * N, splits, s);
}

// The LDS-DMA GEMM takes fp32 activations against Q4_0 / Q4_1 wherever the 128 x 128 tile is
// the automatic pick (or configuration 8 forces it).
#ifndef KSQ_MMQ_PLANAR
#define KSQ_MMQ_PLANAR 1
#endif
bool mmq_planar_preferred(int wtype, int M, int N, int K) {
    if (wtype != kWQ40 && wtype != kWQ41) return false;
    if (g_mmq_config == 8) return true;
    return KSQ_MMQ_PLANAR && g_mmq_config == 0 && pick_config(wtype, M, N, K) == 1;
}

int mmq_planar_splits(int wtype, int M, int N, int K) { return split_for<TileL>(wtype, M, N, K); }

float planar_da_scale(int wtype) { return wtype == kWQ40 ? 1.0f / WShape<kWQ40, 4>::out_scale : 1.0f; }

hipError_t launch_mmq_planar(int wtype, const uint8_t* W, const PlanarQ81& A, float* C, int M, int N, int K,
                             float* partials, hipStream_t s) {
    if (K % 256) return hipErrorInvalidValue;
    const int splits = split_for<TileL>(wtype, M, N, K);
    if (splits > 1 && !partials) return hipErrorInvalidValue;
    note_engine(KSQ_ENG_MMQ_PLANAR | (splits > 1 ? KSQ_ENG_SPLITK : 0u));
    const int tiles = ((N + 127) / 128) * ((M + 127) / 128);
    const dim3 grid((unsigned)((tiles + 7) / 8 * 8), 1u, (unsigned)splits);   // tile order: xcd_tile
    float* out = splits > 1 ? partials : C;
    if (wtype == kWQ40)
        hipLaunchKernelGGL((mmq_planar_kernel<kWQ40, false>), grid, dim3(256), 0, s, W, A, out, M, N, K / 32, MoeTiles{});
    else if (wtype == kWQ41)
        hipLaunchKernelGGL((mmq_planar_kernel<kWQ41, false>), grid, dim3(256), 0, s, W, A, out, M, N, K / 32, MoeTiles{});
    else
        return hipErrorNotSupported;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    return launch_splitk_reduce(partials, C, (int64_t)M * N, splits, s);
}

// 64-row tiles (64 x 128, little padding per expert).  The 128 x 128 form (empty 32-row tiles of a
// ragged tile skipped) measured slower at every routed size but one on MI355X (Q4_0, top-2 of 8
// experts, us, 64- vs 128-row tiles): 512 tokens N = 14336, K = 4096: 257 vs 301; 1024 tokens:
// 450 vs 470; 2048 tokens N = 4096, K = 14336: 808 vs 885; 4096 tokens N = K = 4096: 487 vs 514;
// 2048 tokens N = 14336, K = 4096: 842 vs 830.  It stays selectable through this build-time
// threshold (rows per expert).
#ifndef KSQ_MOE_TILE128_MIN_ROWS
#define KSQ_MOE_TILE128_MIN_ROWS 100000
#endif
int mmq_moe_tile_rows(int wtype, int T, int E, int top_k) {
    const bool nib = (wtype == kWQ40 || wtype == kWQ41);
    return (nib && (long long)T * top_k >= (long long)KSQ_MOE_TILE128_MIN_ROWS * E) ? 128 : 64;
}

hipError_t launch_mmq_moe(int wtype, const uint8_t* W, const uint8_t* Aq, float* C, int N, int K, int max_tiles,
                          int tile_rows, const MoeTilesArgs& a, hipStream_t s) {
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
    if (is_kquant(wtype)) return hipErrorNotSupported;
    mt.expert_stride = (size_t)N * nb * block_bytes(wtype);
    note_engine(tile_rows == TileL::BM ? KSQ_ENG_MOE_TILE128 : KSQ_ENG_MOE_TILE64);
    if (tile_rows == TileL::BM) {
        const dim3 grid((unsigned)((N + TileL::BN - 1) / TileL::BN), (unsigned)max_tiles);
        return launch_t<TileL, false, true>(wtype, kAQ81, grid, W, Aq, C, nullptr, 0, N, nb, mt, s);
    }
    if (tile_rows != 64) return hipErrorInvalidValue;
#ifndef KSQ_MOE_TILEW
#define KSQ_MOE_TILEW 1
#endif
    if (KSQ_MOE_TILEW) {
        const dim3 grid((unsigned)((N + TileW::BN - 1) / TileW::BN), (unsigned)max_tiles);
        return launch_t<TileW, false, true>(wtype, kAQ81, grid, W, Aq, C, nullptr, 0, N, nb, mt, s);
    }
    const dim3 grid((unsigned)((N + TileS::BN - 1) / TileS::BN), (unsigned)max_tiles);
    return launch_t<TileS, false, true>(wtype, kAQ81, grid, W, Aq, C, nullptr, 0, N, nb, mt, s);
}

// The grouped GEMM on the LDS-DMA kernel (Q4_0 / Q4_1, fp32 activations quantised to planar
// rows in expert-sorted order): from an average of KSQ_MOE_PLANAR_MIN_ROWS entries per expert on.
#ifndef KSQ_MOE_PLANAR_MIN_ROWS
#define KSQ_MOE_PLANAR_MIN_ROWS 96
#endif
bool mmq_moe_planar(int wtype, int T, int E, int top_k, int K) {
    return (wtype == kWQ40 || wtype == kWQ41) && K % 256 == 0 &&
           (long long)T * top_k >= (long long)KSQ_MOE_PLANAR_MIN_ROWS * E;
}

hipError_t launch_mmq_planar_moe(int wtype, const uint8_t* W, const PlanarQ81& A, float* C, int N, int K,
                                 int max_tiles, const MoeTilesArgs& a, hipStream_t s) {
    if (K % 256) return hipErrorInvalidValue;
    MoeTiles mt;
    mt.num_tiles = a.num_tiles;
    mt.tile_expert = a.tile_expert;
    mt.tile_row0 = a.tile_row0;
    mt.expert_end = a.expert_end;
    mt.rows = a.rows;
    mt.weights = a.weights;
    mt.scratch = a.scratch;
    mt.top_k = a.top_k;
    mt.expert_stride = (size_t)N * (K / 32) * block_bytes(wtype);
    note_engine(KSQ_ENG_MOE_PLANAR);
    const dim3 grid((unsigned)((N + 127) / 128), (unsigned)max_tiles);
    if (wtype == kWQ40)
        hipLaunchKernelGGL((mmq_planar_kernel<kWQ40, true>), grid, dim3(256), 0, s, W, A, C, 0, N, K / 32, mt);
    else if (wtype == kWQ41)
        hipLaunchKernelGGL((mmq_planar_kernel<kWQ41, true>), grid, dim3(256), 0, s, W, A, C, 0, N, K / 32, mt);
    else
        return hipErrorNotSupported;
    return hipGetLastError();
}

hipError_t launch_mmq_block_sumi(int wtype, const uint8_t* W, const uint8_t* A, int32_t* out, int M, int N, int K,
                                 hipStream_t s) {
    if (!mmq_supported(wtype, M, N, K, W, ((uintptr_t)A & 15u) == 0)) return hipErrorNotSupported;
    return launch_cfg<true>(pick_config(wtype, M, N, K), wtype, kAQ81, W, A, nullptr, out, M, N, K, 1, s);
}

}  // namespace ksq
