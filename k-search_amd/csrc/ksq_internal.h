// ksq_internal.h - host-side launchers shared between the kernel files and
// the C ABI layer (ksq_abi.hip).  Launchers assume their arguments were
// validated by the ABI layer (shapes, alignment, non-null pointers) and
// return the hipError_t of the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/ksq.h"

namespace ksq {

// Kernel families a call launched, recorded per host thread (ksq_debug_last_engines; the bit
// values are the KSQ_ENG_* constants of include/ksq.h).  The launchers add their bit; the ABI
// layer clears the record when a call starts.
void note_engine(uint32_t bits);

// Quantised-activation formats: block_q8_1 (fp16 d and s), block_q8s (fp32 d, the native
// W8A8C8 operator's block; used with Q8_0 weights only) or block_q8f (fp32 d and s, 40 bytes;
// int8 MFMA GEMM only, with Q4_0, Q5_0 and Q8_0 weights).
constexpr int kAQ81 = 0, kAQ8S = 1, kAQ8F = 2;

// fp32 [rows][K] -> [rows][K/32] 36-byte blocks of format afmt; x 16-byte aligned, y 4-byte aligned.
hipError_t launch_quantize(int afmt, const float* x, uint8_t* y, int64_t rows, int K, hipStream_t s);
hipError_t launch_quantize_q8_1(const float* x, uint8_t* y, int64_t rows, int K, hipStream_t s);
// fp32 [rows][K] -> block_q8f [rows][K/32] by rule KSQ_Q8F_RNE / KSQ_Q8F_LROUND (0 / 1).
hipError_t launch_quantize_q8f(int rule, const float* x, uint8_t* y, int64_t rows, int K, hipStream_t s);
// The same quantisation plus zeroing nzero floats at `zero` (16-byte aligned, nzero % 4 == 0) in
// the same launch.
hipError_t launch_quantize_q8_1_zero(const float* x, uint8_t* y, int64_t rows, int K, float* zero, int64_t nzero,
                                     hipStream_t s);
// Planar block_q8_1: the blocks of quantize_row_q8_1 split into planes, so that every piece
// the LDS-DMA GEMM stages is a 16-byte-aligned run it copies into LDS without VGPRs.
//   q  [M][K]          int8 quants (block kb of row m at q + m*K + 32*kb)
//   dn [K/32][mp][2]   fp32 pairs (d, nc): d = d_a * da_scale (d_a the block's fp16 scale,
//                      da_scale a power of two), nc = -12582912 * d
//   sa [K/128][mp][4]  fp16 bits of -s_a
// mp = M rounded up to a multiple of 128; rows M .. mp-1 of dn and sa hold zeros.
struct PlanarQ81 {
    int8_t* q;
    float* dn;
    uint16_t* sa;
    int mp;
};
// Workspace bytes of the planes (each 256-byte aligned) and their addresses in a workspace.
size_t planar_bytes(int M, int K);
PlanarQ81 planar_at(void* ws, int M, int K);
// fp32 [M][K] (16-byte aligned, K % 128 == 0) -> planar block_q8_1.
hipError_t launch_quantize_planar(const float* x, const PlanarQ81& y, int M, int K, float da_scale, hipStream_t s);
// The same for the grouped MoE GEMM: x row m (m < T) goes to planar rows inv[m * top_k + s] (s <
// top_k; -1: none); planar rows no entry maps to are not written.  With zero non-null the same
// launch also clears nzero floats there (16-byte aligned, nzero % 4 == 0).
hipError_t launch_quantize_planar_scatter(const float* x, const PlanarQ81& y, int T, int K, float da_scale,
                                          const int32_t* inv, int top_k, float* zero, int64_t nzero, hipStream_t s);
// The LDS-DMA GEMM (Q4_0 / Q4_1 weights, K % 256 == 0, W 16-byte aligned) on planar
// activations quantised with da_scale = planar_da_scale(wtype); whether it is the pick for this
// shape (fp32 activations); partials as launch_mmq (mmq_splits(...) > 1).
bool mmq_planar_preferred(int wtype, int M, int N, int K);
int mmq_planar_splits(int wtype, int M, int N, int K);
float planar_da_scale(int wtype);
hipError_t launch_mmq_planar(int wtype, const uint8_t* W, const PlanarQ81& A, float* C, int M, int N, int K,
                             float* partials, hipStream_t s);
// variant 0-3 of ksq_quantize_q8_1_variant (x fp32, or fp16 bits for variant 3)
hipError_t launch_quantize_variant(int variant, const void* x, uint8_t* y, int64_t rows, int K, hipStream_t s);
// fp32 weights -> nblocks block_q4_0 (wtype kWQ40) or block_q8_0 (kWQ80) by the reference's device
// rule (rule 0) or CPU-reference rule (rule 1); x 16-byte aligned, y 2-byte aligned.
hipError_t launch_quantize_weights(int wtype, int rule, const float* x, uint8_t* y, int64_t nblocks, hipStream_t s);
// out [cols][rows] = in [rows][cols], fp32
hipError_t launch_transpose_f32(const float* in, float* out, int rows, int cols, hipStream_t s);
// Decode GEMV/GEMM on v_dot4 (mul_mat_vec_q family), any M.
// wtype: 0 Q4_0, 1 Q8_0, 2 Q4_K, 3 Q6_K, 4 Q4_1, 5 Q5_0, 6 Q5_1.
hipError_t launch_gemv(int wtype, int afmt, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int K,
                       hipStream_t s);
// The same with output element (m, n) at C[m * ldc + n * ldr] (not for Q4_K at 3-8 rows).
hipError_t launch_gemv_strided(int wtype, int afmt, const uint8_t* W, const uint8_t* A, float* C, int M, int N,
                               int K, int ldc, int ldr, hipStream_t s);

// The same decode kernels on fp32 activations [M][K] (16-byte aligned): every workgroup
// quantises the activation blocks it needs (block_q8_1, or block_q8s for afmt kAQ8S) into
// LDS while its weight loads are in flight, so no quantise launch or workspace is needed.
hipError_t launch_gemv_f32(int wtype, int afmt, const uint8_t* W, const float* X, float* C, int M, int N, int K,
                           hipStream_t s);
// The same from fp32 (xh false) or fp16 (xh true, quantised by the fused FP16 kernels' rules,
// M <= 2) activations, with output element (m, n) at C[m * ldc + n * ldr] (ldr > 1 only for
// M <= 2): ldc = 1, ldr = M writes the transposed [N][M] output.
hipError_t launch_gemv_fused(int wtype, int afmt, bool xh, const uint8_t* W, const void* X, float* C, int M, int N,
                             int K, int ldc, int ldr, hipStream_t s);
// Whether the in-workgroup quantisation beats quantise + launch_gemv for this shape (M <= 2, or
// M <= 8 for fp32, and a bounded amount of repeated quantisation).
bool gemv_fused_profitable(int wtype, int M, int N, int K, const void* W, bool xh = false);
// fp32 [M][K] activations (M = 1, 2) quantised to block_q8f by `rule` (kQ8FRne / kQ8FLround)
// inside every workgroup of the decode kernel, against Q4_0 / Q5_0 / Q8_0 weights; C [M][N].
bool gemv_q8f_profitable(int wtype, int M, int N, int K, const void* W);
hipError_t launch_gemv_q8f(int rule, int wtype, const uint8_t* W, const float* X, float* C, int M, int N, int K,
                           hipStream_t s);

// Small-batch GEMM (1 <= M <= 8) on the 4x4x4 int8 MFMA for the 32-element block types
// (Q4_0, Q8_0, Q4_1, Q5_0, Q5_1; block_q8s activations with Q8_0).  W and A 4-byte aligned.
bool skinny_supported(int wtype, int afmt, int M, int N, int K, const void* W, const void* A);
// Whether it is expected to beat the decode kernel (measured crossovers by type, M and N).
bool skinny_preferred(int wtype, int M, int N, int K);
hipError_t launch_skinny(int wtype, int afmt, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int K,
                         hipStream_t s);

// Prefill GEMM on int8 MFMA (mul_mat_q family); returns hipErrorNotSupported
// for shapes it does not tile.
// a_aligned16: the quantised activations the GEMM will read are 16-byte aligned.
bool mmq_supported(int wtype, int M, int N, int K, const void* W, bool a_aligned16);
// Whether the MFMA kernel is expected to beat the decode kernel for this shape (M > 8, or
// a large matrix with M >= 5 .. 7 by the measured crossovers).
bool mmq_preferred(int wtype, int M, int N, int K);
// Number of K splits launch_mmq uses for this shape (1: none).  With splits > 1 it needs
// `partials`, splits * M * N floats of device scratch.
int mmq_splits(int wtype, int M, int N, int K);
// trans: write the output transposed, [N][M] (only without split-K: mmq_splits(...) == 1).
hipError_t launch_mmq(int wtype, int afmt, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int K,
                      float* partials, hipStream_t s, bool trans = false);
// In-order sum of `splits` partial [M][N] results (P) into C.
hipError_t launch_splitk_reduce(const float* P, float* C, int64_t mn, int splits, hipStream_t s);

// Force one of the MFMA tile configurations (1..7; 8: the LDS-DMA GEMM where it applies, the
// 128 x 128 tile elsewhere) or automatic choice (0) for the calling host thread; -1 if out of
// range.
int mmq_set_config(int c);

// Expert-grouped prefill GEMM (MoE).  Arrays are device arrays produced by launch_moe_route /
// launch_moe_group; C must be zeroed first when scratch is null (top_k <= 2).
struct MoeTilesArgs {
    const int32_t* num_tiles;
    const int32_t* tile_expert;
    const int32_t* tile_row0;
    const int32_t* expert_end;
    const int32_t* rows;
    const float* weights;
    float* scratch;
    int top_k;
};
// Rows per grouped-GEMM tile (the MoE tile schedule's granularity) for a routing shape.
int mmq_moe_tile_rows(int wtype, int T, int E, int top_k);
// Whether the grouped GEMM runs on the LDS-DMA kernel (128-row tiles over planar activations in
// expert-sorted order, launch_quantize_planar_scatter), and that launch.
bool mmq_moe_planar(int wtype, int T, int E, int top_k, int K);
hipError_t launch_mmq_planar_moe(int wtype, const uint8_t* W, const PlanarQ81& A, float* C, int N, int K,
                                 int max_tiles, const MoeTilesArgs& a, hipStream_t s);
hipError_t launch_mmq_moe(int wtype, const uint8_t* W, const uint8_t* Aq, float* C, int N, int K, int max_tiles,
                          int tile_rows, const MoeTilesArgs& a, hipStream_t s);

// MoE routing: softmax over E logits per token, top_k by logit (ties -> lower expert).
hipError_t launch_moe_route(const float* logits, int T, int E, int top_k, int renorm, int32_t* ids, float* w,
                            hipStream_t s);
// Routing and grouping in one launch (one workgroup): launch_moe_route then launch_moe_group.
// With zero != nullptr, more workgroups of the same launch clear zero[0, nzero) (nzero % 4 == 0,
// zero 16-byte aligned) meanwhile.
hipError_t launch_moe_route_group(const float* logits, int T, int E, int top_k, int renorm, int32_t* ids, float* w,
                                  int tile_rows, int32_t* rows, int32_t* inv, int32_t* expert_end, int32_t* num_tiles,
                                  int32_t* tile_expert, int32_t* tile_row0, float* zero, int64_t nzero,
                                  hipStream_t s);
// Stable grouping of the T*top_k (token, slot) entries by expert, plus the tile schedule
// for tiles of `tile_rows` rows.  max_tiles = T*top_k/tile_rows + E bounds num_tiles.
// rows[p] = the entry at place p; inv (if non-null) the inverse: inv[entry] = its place, -1 for an
// entry with an expert id outside [0, E).
hipError_t launch_moe_group(const int32_t* ids, int T, int top_k, int E, int tile_rows, int32_t* rows, int32_t* inv,
                            int32_t* expert_end, int32_t* num_tiles, int32_t* tile_expert, int32_t* tile_row0,
                            hipStream_t s);
// out[t][n] = sum_s scratch[t*top_k + s][n] in slot order over the slots whose id is in [0, E)
// (top_k > 2 combine).
hipError_t launch_moe_combine(const float* scratch, const int32_t* ids, float* out, int T, int N, int top_k, int E,
                              hipStream_t s);

// Per-block integer dots [M][N][nblk] from the same device block-dot code the
// decode kernels use (debug entry for the bit-exact check).
hipError_t launch_block_sumi(int wtype, const uint8_t* W, const uint8_t* A, int32_t* out, int M, int N,
                             int K, hipStream_t s);

// Calibration read of `bytes` bytes at p (16-byte aligned, bytes % 16 == 0), wg_bytes (a multiple
// of 4096) per workgroup; writes stream_read_outputs(bytes, wg_bytes) words to out.
size_t stream_read_outputs(size_t bytes, size_t wg_bytes);
hipError_t launch_stream_read(const void* p, size_t bytes, size_t wg_bytes, uint32_t* out, hipStream_t s);

// Dequantise-then-fp32 GEMM (W4A16 / W8A16) on the bf16 MFMA: C[M][N] = A . dequant(W)^T,
// wtype kWQ40 or kWQ80, K % 64 == 0.  With w16_splits(M, N, K) > 1 it needs `partials`, that
// many M x N float planes of device scratch.
int w16_splits(int M, int N, int K);
hipError_t launch_w16(int wtype, const float* A, const uint8_t* W, float* C, int M, int N, int K, float* partials,
                      hipStream_t s);

// Fill `n` floats with zero (a kernel, so it can be captured in a graph).
hipError_t launch_fill_zero(float* p, int64_t n, hipStream_t s);

}  // namespace ksq
