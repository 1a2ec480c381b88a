// ksq_mmqh.hip - prefill GEMM for Q4_0 weights on the gfx950 f16 MFMA with exact integer dots.
//
// Reference path: the tiled GEMMs of kernelevalplus-main/include/gemm_cuda_tiled.cuh:191-262 and
// gemm_cuda_dp4a.cuh:275-351 with the block formula of gemm_w4a8_reference
// (include/gemm_reference.h:200-216): per 32-element block, d_w * (d_a * sumi - 8 * s_a).
//
// Why f16: on the int8 MFMA the block dot arrives as an int32 that must be converted and then
// scaled by d_w * d_a, two VALU ops per output per block, which bounds that kernel by the vector
// ALU (the matrix unit idles ~85% of the time).  Here both operands are exact small integers
// in f16 (Q4_0 nibbles 0..15; Q8_1 quants as q/8, 7 significant bits), every product is exact
// and every partial sum is a multiple of 1/8 below 2^16, so v_mfma_f32_32x32x16_f16 returns the
// reference's sumi / 8 exactly, already as a float.  A second f16 MFMA with one live k slot
// forms the outer product E = d_w x d_a of the block (products of two fp16 values are exact in
// fp32), and the epilogue is a single FMA per output and block: acc += E * S.  The -8 d_w s_a
// term is a rank-(K/32) product of fp16 fields (d_w, -s_a) on the same f16 MFMA, accumulated
// into acc at 1/8 scale like the main term; the result is scaled by 8 at the end.
//
// Activations arrive in the "q8h" layout written by the quantiser (or converted from block_q8_1):
// QH [M][K] fp16 holding q/8 and DS [M][K/32] the block_q8_1 ds word (fp16 d, fp16 s).
//
// Tiling: 128 x 128 workgroup tile, 4 waves of 64 x 64 (16 x 16 MFMA sub-tiles, the weight rows
// as the A operand), K steps of 2 blocks with double-buffered LDS: the activation tile of the
// next step is copied by LDS DMA (global_load_lds, 16 B per lane, into an XOR-swizzled layout so
// that the fragment reads are conflict free) and the next weight blocks are loaded into
// registers while the current step computes; the nibbles are widened to fp16 once per workgroup
// when they are written to LDS.  One barrier per step.
//
// Status: exact (bit-identical block dots) but measured slower on MI355X than the int8 kernel
// (M = 2048, N = K = 4096: 138 vs 113 us; MFMA 35 % and VALU 46 % busy, little overlap between
// the two; without any per-step copies it still takes 101 us), so it is an opt-in engine
// (ksq_set_path(4)) and the automatic path keeps the int8 MFMA GEMM.
#include "ksq_device.h"
#include "ksq_internal.h"

namespace ksq {

namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

constexpr int kHBM = 128, kHBN = 128;  // workgroup tile
constexpr int kHKB = 2;                // blocks per K step
constexpr int kHKH = kHKB * 32;        // fp16 values per staged row and step (128 B = 8 chunks of 16 B)

// 16-byte chunk c of staged row r lives at chunk c ^ (r & 7): the 32 rows of a fragment read
// hit 8 different chunk positions, i.e. all banks.
__device__ __forceinline__ int hswz(int r, int c) { return c ^ (r & 7); }

// Four nibbles (low nibbles of bytes o, o+1 of x for o = 0 or 2) -> two fp16 values.
// v_perm_b32 puts bytes o, o+1 of x under 0x64 high bytes: fp16 1024 + byte; the mask keeps
// the low nibble, and the packed subtract of 1024 leaves the nibble value exactly.
__device__ __forceinline__ uint32_t nib2h(uint32_t x, int o) {
    const uint32_t sel = o ? 0x04030402u : 0x04010400u;  // result bytes: x[o], 0x64, x[o+1], 0x64
    const uint32_t p = __builtin_amdgcn_perm(0x64646464u, x, sel) & 0xFF0FFF0Fu;
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 v = __builtin_bit_cast(h2, p) - h2{(_Float16)1024.0f, (_Float16)1024.0f};
    return __builtin_bit_cast(uint32_t, v);
}

// LDS of one pipeline stage (one K step of kHKB blocks).
struct HStage {
    _Float16 a[kHBM * kHKH];          // activations q/8, rows of 8 swizzled 16-byte chunks
    _Float16 w[kHBN * kHKH];          // weights widened to fp16, same layout
    uint16_t da[kHKB][kHBM];          // [block][row]: d_a
    uint16_t dw[kHKB][kHBN];          // d_w
    uint16_t sa[kHBM][kHKB];          // [row][block]: -s_a (the side term's k slots)
    uint16_t ds[kHBN][kHKB];          // d_w, same shape
};

template <bool DUMP>
__global__ __launch_bounds__(256, 2) void mmqh_q4_0_kernel(const uint8_t* __restrict__ W, const _Float16* __restrict__ QH,
                                                           const uint32_t* __restrict__ DS, float* __restrict__ C,
                                                           int32_t* __restrict__ dump, int M, int N, int nb) {
    // two stages as separate objects: the LDS DMA into one provably does not alias the reads of
    // the other, so the compiler does not make the compute of a step wait for the next step's copy
    __shared__ __attribute__((aligned(16))) HStage st0;
    __shared__ __attribute__((aligned(16))) HStage st1;

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * kHBM, n0 = blockIdx.x * kHBN;
    const int K = nb * 32;

    // split-K: workgroup z covers steps [z*S/Z, (z+1)*S/Z) and writes its partial sums to C + z*M*N
    const int S = nb / kHKB, Z = (int)gridDim.z, z = (int)blockIdx.z;
    const int s_lo = (int)((long long)S * z / Z), s_hi = (int)((long long)S * (z + 1) / Z);
    C += (size_t)z * (size_t)M * (size_t)N;

    // ---- staging roles: thread t -> row t/2, block t%2 of the step (weights and activation scales)
    const int sr = t >> 1, sj = t & 1;
    const int wr = min(n0 + sr, N - 1), ar = min(m0 + sr, M - 1);
    // this thread's weight block of step s starts at wblk0 + 36 s; its offset mod 4 is fixed
    const uint8_t* wblk0 = W + (size_t)wr * nb * kQ40Bytes + (size_t)sj * kQ40Bytes;
    const int wsh = (int)((uintptr_t)wblk0 & 3u);           // d at byte wsh (0 or 2) of its dword
    const int wpsh = (wsh + 2) & 3;                         // the 16 quant bytes start at byte wpsh
    const uint32_t* wd0 = (const uint32_t*)(wblk0 - wsh);   // dword holding d
    const uint32_t* wq0 = (const uint32_t*)(wblk0 + 2 - wpsh);  // first dword of the quants
    const uint32_t* ds0 = DS + (size_t)ar * nb + sj;
    // activation DMA: lane i of instruction q moves physical chunk i % 8 of row 32 w + 8 q + i / 8
    // (element offsets into QH; M * K < 2^31)
    int asrc[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int pr = 32 * wave + 8 * q + (lane >> 3), c = (lane & 7) ^ (pr & 7);
        asrc[q] = min(m0 + pr, M - 1) * K + 8 * c;
    }

    struct WReg {
        uint32_t d, q[5], ds;
    };
    auto load_stage = [&](int s, WReg& r) {
        const int o = (kHKB * kQ40Bytes / 4) * s;   // 9 dwords per step
        r.d = wd0[o];
#pragma unroll
        for (int i = 0; i < 4; i++) r.q[i] = wq0[o + i];
        r.q[4] = wpsh ? wq0[o + 4] : 0u;   // only when re-aligning (stays inside the block)
        r.ds = ds0[kHKB * s];
    };
    auto dma_a = [&](int s, HStage& st) {
#pragma unroll
        for (int q = 0; q < 4; q++)
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(QH + (asrc[q] + kHKH * s)),
                                             (__attribute__((address_space(3))) void*)(st.a + (32 * wave + 8 * q) * kHKH),
                                             16, 0, 0);
    };
    auto store_stage = [&](HStage& st, const WReg& r) {
        const uint32_t d = (r.d >> (8 * wsh)) & 0xFFFFu;
        uint32_t qs[4];
#pragma unroll
        for (int i = 0; i < 4; i++) qs[i] = __builtin_amdgcn_alignbyte(r.q[i + 1], r.q[i], wpsh);
        // element e: low nibble of byte e (e < 16), high nibble of byte e - 16 (e >= 16)
        uint32_t o[16];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            o[j] = nib2h(qs[j >> 1], 2 * (j & 1));
            o[8 + j] = nib2h(qs[j >> 1] >> 4, 2 * (j & 1));
        }
        _Float16* row = st.w + sr * kHKH;
#pragma unroll
        for (int c = 0; c < 4; c++)
            *(u32x4*)(row + 8 * hswz(sr, 4 * sj + c)) = u32x4{o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]};
        st.dw[sj][sr] = (uint16_t)d;
        st.ds[sr][sj] = (uint16_t)d;
        st.da[sj][sr] = (uint16_t)(r.ds & 0xFFFFu);
        st.sa[sr][sj] = (uint16_t)((r.ds >> 16) ^ 0x8000u);
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // The wave's 64 x 64 outputs are 2 x 2 regions of 32 x 32, each 2 x 2 sub-tiles of 16 x 16
    // computed by v_mfma_f32_16x16x32_f16 (one instruction per block: K = 32, no dependent pair).
    // Sub-tile blk = 2 rj + ci of region (I, J) holds weight rows 32 J + 16 rj + 4 (l/16) + i and
    // activation row 32 I + 16 ci + l % 16 in registers 4 blk + i of acc[I][J] - the layout of the
    // 4-block v_mfma_f32_16x16x4_4b_f16 that forms E = d_w x d_a for all four sub-tiles at once.
    const int l16 = lane & 15, g4 = lane >> 4;
    // per-lane LDS element offsets of the 16-row fragment groups (row 16 q + l16, k = 8 g4 .. +7)
    int wfo[kHKB][4], afo[kHKB][4];
#pragma unroll
    for (int b = 0; b < kHKB; b++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int n = 64 * wn + 16 * q + l16, m = 64 * wm + 16 * q + l16;
            wfo[b][q] = n * kHKH + 8 * hswz(n, 4 * b + g4);
            afo[b][q] = m * kHKH + 8 * hswz(m, 4 * b + g4);
        }
    // the E operands: lane l supplies the scale of sub-tile g4's row / column l16
    const int erow = 64 * wn + 16 * (g4 >> 1) + l16;   // + 32 J: weight row of the sub-tile
    const int ecol = 64 * wm + 16 * (g4 & 1) + l16;    // + 32 I: activation row

    auto compute = [&](const HStage& st, int s) {
#pragma unroll
        for (int b = 0; b < kHKB; b++) {
            h8 wf[4], af[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                wf[q] = *(const h8*)(st.w + wfo[b][q]);
                af[q] = *(const h8*)(st.a + afo[b][q]);
            }
            h4 ew[2], ea[2];
#pragma unroll
            for (int x = 0; x < 2; x++) {
                ew[x] = __builtin_bit_cast(h4, u16x4{st.dw[b][erow + 32 * x], 0, 0, 0});
                ea[x] = __builtin_bit_cast(h4, u16x4{st.da[b][ecol + 32 * x], 0, 0, 0});
            }
            // region r = (I, J) = (r / 2, r % 2); its MFMAs are issued before the FMAs of region r-1
            auto region_s = [&](int r, f32x16& Sv) {
                const int I = r >> 1, J = r & 1;
#pragma unroll
                for (int blk = 0; blk < 4; blk++) {
                    const f32x4 v = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[2 * J + (blk >> 1)], af[2 * I + (blk & 1)],
                                                                          f32x4{}, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) Sv[4 * blk + i] = v[i];
                }
            };
            auto region_e = [&](int r) -> f32x16 {
                return __builtin_amdgcn_mfma_f32_16x16x4f16(ew[r & 1], ea[r >> 1], f32x16{}, 0, 0, 0);
            };
            auto finish = [&](int r, const f32x16& Sv, const f32x16& Ev) {
                const int I = r >> 1, J = r & 1;
                if constexpr (DUMP) {
#pragma unroll
                    for (int blk = 0; blk < 4; blk++) {
                        const int gm = m0 + 64 * wm + 32 * I + 16 * (blk & 1) + l16;
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int gn = n0 + 64 * wn + 32 * J + 16 * (blk >> 1) + 4 * g4 + i;
                            if (gm < M && gn < N)
                                dump[((size_t)gm * N + gn) * nb + kHKB * s + b] = (int32_t)(Sv[4 * blk + i] * 8.0f);
                        }
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 16; e++) acc[I][J][e] = fmaf(Ev[e], Sv[e], acc[I][J][e]);
                }
            };
            if constexpr (DUMP) {
                f32x16 Sv;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    region_s(r, Sv);
                    finish(r, Sv, f32x16{});
                }
            } else {
                // Software pipeline over the 4 regions: the 5 MFMAs of region r+1 are interleaved one
                // by one with the 16 FMAs of region r (sched_group_barrier pins the order: the
                // scheduler would otherwise issue the MFMAs back to back, and an in-order wave cannot
                // issue its FMAs while it waits for the matrix pipe to accept the next MFMA).
                f32x16 Sc, Ec = region_e(0);
                region_s(0, Sc);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int I = r >> 1, J = r & 1;
                    f32x16 Sn = Sc, En = Ec;
                    if (r + 1 < 4) {
                        const int In = (r + 1) >> 1, Jn = (r + 1) & 1;
#pragma unroll
                        for (int blk = 0; blk < 4; blk++) {
                            const f32x4 v = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[2 * Jn + (blk >> 1)],
                                                                                  af[2 * In + (blk & 1)], f32x4{}, 0, 0, 0);
#pragma unroll
                            for (int i = 0; i < 4; i++) Sn[4 * blk + i] = v[i];
#pragma unroll
                            for (int e = 4 * blk; e < 4 * blk + 4; e++) acc[I][J][e] = fmaf(Ec[e], Sc[e], acc[I][J][e]);
                            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
                        }
                        En = region_e(r + 1);
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    } else {
#pragma unroll
                        for (int e = 0; e < 16; e++) acc[I][J][e] = fmaf(Ec[e], Sc[e], acc[I][J][e]);
                    }
                    Sc = Sn;
                    Ec = En;
                }
            }
        }
        if constexpr (!DUMP) {
            // side term: acc += sum over the step's blocks of d_w[n] * (-s_a[m]) (2 of 4 k slots)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int I = r >> 1, J = r & 1;
                const u32x2 dwp{*(const uint32_t*)&st.ds[erow + 32 * J][0], 0u};
                const u32x2 sap{*(const uint32_t*)&st.sa[ecol + 32 * I][0], 0u};
                acc[I][J] = __builtin_amdgcn_mfma_f32_16x16x4f16(__builtin_bit_cast(h4, dwp), __builtin_bit_cast(h4, sap),
                                                                 acc[I][J], 0, 0, 0);
            }
        }
    };

    // one step: copy step s+1 into `nx` (DMA + weight registers) while step s computes from `cu`
    auto step = [&](int s, const HStage& cu, HStage& nx) {
        const bool more = s + 1 < s_hi;
        WReg r{};
        if (more) {
            dma_a(s + 1, nx);
            load_stage(s + 1, r);
        }
        compute(cu, s);
        if (more) store_stage(nx, r);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    };

    if (s_lo < s_hi) {
        WReg r{};
        dma_a(s_lo, st0);
        load_stage(s_lo, r);
        store_stage(st0, r);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }
    for (int s = s_lo; s < s_hi; s += 2) {
        step(s, st0, st1);
        if (s + 1 < s_hi) step(s + 1, st1, st0);
    }

    if constexpr (!DUMP) {
        const bool vec_ok = (N % 4) == 0 && (((uintptr_t)C & 15u) == 0);
#pragma unroll
        for (int I = 0; I < 2; I++)
#pragma unroll
            for (int J = 0; J < 2; J++)
#pragma unroll
                for (int blk = 0; blk < 4; blk++) {
                    const int gm = m0 + 64 * wm + 32 * I + 16 * (blk & 1) + l16;
                    const int gn = n0 + 64 * wn + 32 * J + 16 * (blk >> 1) + 4 * g4;
                    if (gm >= M) continue;
                    float a[4];
#pragma unroll
                    for (int p = 0; p < 4; p++) a[p] = acc[I][J][4 * blk + p];
                    if (vec_ok && gn + 3 < N) {
                        *(f32x4*)(C + (size_t)gm * N + gn) = f32x4{8.0f * a[0], 8.0f * a[1], 8.0f * a[2], 8.0f * a[3]};
                    } else {
#pragma unroll
                        for (int p = 0; p < 4; p++)
                            if (gn + p < N) C[(size_t)gm * N + gn + p] = 8.0f * a[p];
                    }
                }
    }
}

// Split-K factor: grids below 256 workgroups split along K (>= 4 steps per split, <= 16 splits).
int mmqh_split(int M, int N, int K) {
    const int wgs = ((N + kHBN - 1) / kHBN) * ((M + kHBM - 1) / kHBM);
    const int steps = (K / 32) / kHKB;
    if (wgs >= 256) return 1;
    int sp = (512 + wgs - 1) / wgs;
    sp = sp < steps / 4 ? sp : steps / 4;
    sp = sp < 16 ? sp : 16;
    return sp < 1 ? 1 : sp;
}

}  // namespace

bool mmqh_supported(int wtype, int M, int N, int K, const void* W) {
    return wtype == kWQ40 && M >= 1 && N >= 1 && K >= 64 && (K % 64) == 0 && (((uintptr_t)W) & 1u) == 0 &&
           (long long)M * K < (1ll << 31);
}

int mmqh_splits(int M, int N, int K) { return mmqh_split(M, N, K); }

hipError_t launch_mmqh(const uint8_t* W, const _Float16* QH, const uint32_t* DS, float* C, int M, int N, int K,
                       float* partials, hipStream_t s) {
    const int nb = K / 32;
    const int splits = mmqh_split(M, N, K);
    const dim3 grid((unsigned)((N + kHBN - 1) / kHBN), (unsigned)((M + kHBM - 1) / kHBM), (unsigned)splits);
    if (splits == 1) {
        hipLaunchKernelGGL(mmqh_q4_0_kernel<false>, grid, dim3(256), 0, s, W, QH, DS, C, nullptr, M, N, nb);
        return hipGetLastError();
    }
    if (!partials) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mmqh_q4_0_kernel<false>, grid, dim3(256), 0, s, W, QH, DS, partials, nullptr, M, N, nb);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_splitk_reduce(partials, C, (int64_t)M * N, splits, s);
}

hipError_t launch_mmqh_block_sumi(const uint8_t* W, const _Float16* QH, const uint32_t* DS, int32_t* out, int M,
                                  int N, int K, hipStream_t s) {
    const int nb = K / 32;
    const dim3 grid((unsigned)((N + kHBN - 1) / kHBN), (unsigned)((M + kHBM - 1) / kHBM), 1u);
    hipLaunchKernelGGL(mmqh_q4_0_kernel<true>, grid, dim3(256), 0, s, W, QH, DS, nullptr, out, M, N, nb);
    return hipGetLastError();
}

}  // namespace ksq
