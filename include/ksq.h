/*
 * ksq.h - C ABI of the MI355X (gfx950) quantized GGML matmul library (libksq.so).
 *
 * Convention (the reference's quant_gemm operator boundary):
 *     output[M][N] = activation[M][K] . weight[N][K]^T
 *   weight      device bytes, [N][K/32] GGML blocks (or [N][K/256] K-quant super-blocks)
 *   activation  device fp32 [M][K] (the "a32" definitions) or block_q8_1 [M][K/32]
 *   output      device fp32 [M][N], every element written
 * All pointers are device pointers owned by the caller.  Shapes are ints as in the
 * reference signature.  M == 0 or N == 0 is an empty call; K == 0 writes zeros.
 *
 * Reference interface each entry replaces:
 *   extern "C" void <entry_point>(const uint8_t* weight, const <act_t>* activation,
 *                                 float* output, int M, int N, int K);
 *   (k_search/tasks/kernelevalplus_prompts.py:38-48; wrapper generated at
 *    kernelevalplus-main/llm_kernel_test/op_test_handler.py:298-349; a concrete
 *    instance is kernelevalplus-main/core/operators/quant_gemm/variants/deepseek_v3/
 *    w8a8c8_q8_0_q8_1/kernel.cu:119-130.)
 * As in the reference, the void entries launch on the default (null) stream and
 * return before the work finishes; unlike the reference they validate their
 * arguments and record failures for ksq_last_error() instead of launching.
 */
#ifndef KSQ_H
#define KSQ_H

#include <stddef.h>
#include <stdint.h>

#include "ksq_blocks.h"

#if defined(__GNUC__) || defined(__clang__)
#define KSQ_API __attribute__((visibility("default")))
#else
#define KSQ_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------- */
enum ksq_status {
    KSQ_OK = 0,
    KSQ_ERR_NULL = 1,        /* a required pointer is NULL */
    KSQ_ERR_SHAPE = 2,       /* negative size, K not a multiple of the block size, ... */
    KSQ_ERR_ALIGN = 3,       /* pointer alignment the kernels cannot honour */
    KSQ_ERR_TYPE = 4,        /* unknown weight / activation type code */
    KSQ_ERR_WORKSPACE = 5,   /* caller workspace smaller than ksq_gemm_workspace_size() */
    KSQ_ERR_HIP = 6,         /* HIP runtime error (launch, allocation, device) */
};

/* Status of the last ksq call on this host thread, and a message for it. */
KSQ_API int ksq_last_error(void);
KSQ_API const char* ksq_last_error_message(void);
KSQ_API const char* ksq_error_string(int status);

/* Library version string. */
KSQ_API const char* ksq_version(void);

/* Free the workspace pools (one per device and stream) the void entries allocate on demand. */
KSQ_API void ksq_release(void);

/* ---- drop-in entries: the reference's quant_gemm signature --------------- */

/* W4A32C8: Q4_0 weights, fp32 activations quantised to Q8_1 inside the call
 * (quantize_row_q8_1_ref arithmetic), int8 compute.  Replaces the entry of the
 * w4a32c8_q4_0_fp32_int8_* definitions (e.g. kernelevalplus-main/definitions/
 * quant_gemm/llama3_8b/w4a32c8_q4_0_fp32_int8_llama3_8b_att_out_n4096_k4096.json)
 * and KernelEvalPlus' gemm_w4a8_reference (include/gemm_reference.h:175-222). */
KSQ_API void gemm_w4a32c8_q4_0_fp32_int8(const uint8_t* weight, const float* activation, float* output,
                                 int M, int N, int K);

/* W8A32C8: Q8_0 weights, fp32 activations -> Q8_1, int8 compute (the
 * w8a32c8_q8_0_fp32_int8_* definitions; gemm_w8a8_reference, gemm_reference.h:233-267). */
KSQ_API void gemm_w8a32c8_q8_0_fp32_int8(const uint8_t* weight, const float* activation, float* output,
                                 int M, int N, int K);

/* K-quant weights (no reference counterpart; named by the reference's naming
 * scheme, kernelevalplus-main/definitions/NAMING_CONVENTION.md:21-33).  K % 256 == 0. */
KSQ_API void gemm_w4a32c8_q4_k_fp32_int8(const uint8_t* weight, const float* activation, float* output,
                                 int M, int N, int K);
KSQ_API void gemm_w6a32c8_q6_k_fp32_int8(const uint8_t* weight, const float* activation, float* output,
                                 int M, int N, int K);

/* W4A32C8 / W5A32C8 with the other legacy GGML blocks of the reference
 * (kernels/gemm/gemm_quant_formats.cuh:119-267, core/operators/common/types.py:94-140):
 * Q4_1 replaces the entry of the w4a32c8_q4_1_fp32_int8_* definitions (e.g.
 * kernelevalplus-main/definitions/quant_gemm/qwen3_4b/
 * w4a32c8_q4_1_fp32_int8_qwen3_4b_att_out_n2560_k2560.json).  Block contributions:
 *   Q4_1, Q5_1  d_w*d_a*sumi + m_w*s_a   (the harness oracle gemm_ref.py:274-330; the
 *               reference's device dot divides the m*s term by 4, gemm_quant_formats.cuh:148,
 *               :266, which disagrees with that oracle and with the dequantised values)
 *   Q5_0        d_w*(d_a*sumi - 16*s_a)  (gemm_quant_formats.cuh:207)
 * No definitions exist for Q5_0 / Q5_1; their names follow NAMING_CONVENTION.md:21-33. */
KSQ_API void gemm_w4a32c8_q4_1_fp32_int8(const uint8_t* weight, const float* activation, float* output,
                                 int M, int N, int K);
KSQ_API void gemm_w5a32c8_q5_0_fp32_int8(const uint8_t* weight, const float* activation, float* output,
                                 int M, int N, int K);
KSQ_API void gemm_w5a32c8_q5_1_fp32_int8(const uint8_t* weight, const float* activation, float* output,
                                 int M, int N, int K);

/* The native W8A8C8 operator (kernelevalplus-main/core/operators/quant_gemm/variants/
 * deepseek_v3/w8a8c8_q8_0_q8_1/kernel.cu:119-130, same symbol and signature): Q8_0 weights,
 * fp32 activations re-quantised per 32-element block with an fp32 scale (d = amax/127, 1 when
 * below 1e-6; q = roundf(x / d) by true division, kernel.cu:66-93), contribution
 * d_w*d_a*sumi.  Quantised once per activation row here (block_q8s), not once per output. */
KSQ_API void gemm_w8a8c8_q8_0_q8_1(const uint8_t* weight, const float* activation, float* output,
                                   int M, int N, int K);

/* Pre-quantised activations (the harness' uint8_t activation form,
 * op_test_handler.py:319-323): activation is block_q8_1 [M][K/32]. */
KSQ_API void ksq_gemm_q4_0_q8_1(const uint8_t* weight, const uint8_t* activation, float* output, int M, int N, int K);
KSQ_API void ksq_gemm_q8_0_q8_1(const uint8_t* weight, const uint8_t* activation, float* output, int M, int N, int K);
KSQ_API void ksq_gemm_q4_k_q8_1(const uint8_t* weight, const uint8_t* activation, float* output, int M, int N, int K);
KSQ_API void ksq_gemm_q6_k_q8_1(const uint8_t* weight, const uint8_t* activation, float* output, int M, int N, int K);
KSQ_API void ksq_gemm_q4_1_q8_1(const uint8_t* weight, const uint8_t* activation, float* output, int M, int N, int K);
KSQ_API void ksq_gemm_q5_0_q8_1(const uint8_t* weight, const uint8_t* activation, float* output, int M, int N, int K);
KSQ_API void ksq_gemm_q5_1_q8_1(const uint8_t* weight, const uint8_t* activation, float* output, int M, int N, int K);

/* ---- checked, stream-taking entries -------------------------------------- */

/* fp32 [M][K] -> block_q8_1 [M][K/32] (quantize_row_q8_1_ref,
 * kernelevalplus-main/include/quantize.h:165-193, bit for bit; replaces the launcher
 * quantize_q8_1_cuda, quantize.h:361-368, whose kernel rounds half-even instead).
 * x 16-byte aligned, y 4-byte aligned.  stream: hipStream_t or NULL. */
KSQ_API int ksq_quantize_q8_1(const float* x, uint8_t* y, int M, int K, void* stream);

/* The reference's other Q8_1 quantisers, [M][K] -> block_q8_1 [M][K/32], each bit for bit
 * (x 16-byte and y 4-byte aligned; KSQ_ERR_TYPE for an unknown variant):
 *   KSQ_Q81_REF        quantize_row_q8_1_ref, the same as ksq_quantize_q8_1
 *   KSQ_Q81_CUDA       the reference's device kernel quantize_q8_1_kernel
 *                      (include/quantize.h:301-336): half-to-even rounding
 *   KSQ_Q81_NUMPY      the test harness' quantize_to_q8_1
 *                      (llm_kernel_test/reference/quantize.py:165-214): true division,
 *                      d = 1 for an all-zero block, NumPy's pairwise float32 sum; finite x
 *   KSQ_Q81_FUSED_F16  the fused FP16-activation kernels' quantize_fp16_to_q8_1_smem
 *                      (kernels/gemm/gemm_fused.cuh:76-145): x is fp16 (uint16 bits), tree
 *                      max/sum, q from 1/half(d), clamp [-127, 127]
 * x is fp32 for the first three. */
#define KSQ_Q81_REF 0
#define KSQ_Q81_CUDA 1
#define KSQ_Q81_NUMPY 2
#define KSQ_Q81_FUSED_F16 3
KSQ_API int ksq_quantize_q8_1_variant(int variant, const void* x, uint8_t* y, int M, int K, void* stream);

/* Weight quantisers: fp32 x [k] (k % 32 == 0, 16-byte aligned) -> k/32 blocks of block_q4_0
 * (wtype KSQ_W_Q4_0, 18 bytes) or block_q8_0 (KSQ_W_Q8_0, 34 bytes) at y (2-byte aligned):
 *   KSQ_WQ_DEVICE  the reference's device kernels quantize_q4_0_kernel / quantize_q8_0_kernel
 *                  and their launchers quantize_q4_0_cuda / quantize_q8_0_cuda
 *                  (include/quantize.h:221-297, 343-359): round half to even, NaN -> 0
 *   KSQ_WQ_REF     quantize_row_q4_0_ref / quantize_row_q8_0_ref (include/quantize.h:34-68,
 *                  110-131): roundf, a NaN or out-of-range product converts to INT32_MIN
 * KSQ_ERR_TYPE for another weight type or rule. */
#define KSQ_WQ_DEVICE 0
#define KSQ_WQ_REF 1
KSQ_API int ksq_quantize_weights(int wtype, int rule, const float* x, uint8_t* y, int64_t k, void* stream);

/* The reference's fused FP16-activation GEMM gemm_q4_0_fp16_fused (kernels/gemm/gemm_fused.cuh:
 * 311-338) in its orientation: Q4_0 weight [M][K/32] (M weight rows), fp16 activations [N][K]
 * (uint16 bits, 16-byte aligned), output fp32 [M][N] (weight-row major).  Activations are
 * quantised by its quantize_fp16_to_q8_1_smem rules (KSQ_Q81_FUSED_F16, bit-exact), block
 * dots bit-exact.  For decode shapes (N <= 2 activation rows) the quantisation runs inside the
 * decode kernel's workgroups, into LDS, as the reference's fused kernel does (one launch, no
 * workspace used); with the int8 MFMA GEMM the activations are quantised once and the GEMM
 * writes the [M][N] output directly.  workspace: ksq_gemm_q4_0_fp16_fused_workspace_size(M, N,
 * K) bytes of device memory (an upper bound), 256-byte aligned, or NULL for the library's
 * per-device pool (which may allocate). */
KSQ_API size_t ksq_gemm_q4_0_fp16_fused_workspace_size(int M, int N, int K);
KSQ_API int ksq_gemm_q4_0_fp16_fused(const uint8_t* weight, const uint16_t* fp16_activation, float* output,
                                     int M, int N, int K, void* workspace, size_t workspace_bytes,
                                     void* stream);

/* fp32 [M][K] -> block_q8s [M][K/32] by the native W8A8C8 operator's per-block rules
 * (variants/deepseek_v3/w8a8c8_q8_0_q8_1/kernel.cu:66-93, bit for bit).  Same alignment
 * rules as ksq_quantize_q8_1. */
KSQ_API int ksq_quantize_q8s(const float* x, uint8_t* y, int M, int K, void* stream);

/* fp32 [M][K] -> block_q8f [M][K/32] (fp32 d and s), bit for bit with one of two reference
 * quantisers (same alignment rules as ksq_quantize_q8_1; KSQ_ERR_TYPE for an unknown rule):
 *   KSQ_Q8F_RNE     the deepseek_v2 W4A32C8 operator (core/operators/quant_gemm/variants/
 *                   deepseek_v2/w4a32c8_q4_0_fp32_int8/reference.py:50-73, float32 scalar
 *                   arithmetic as NumPy >= 2 evaluates it): d = amax / 127 (1 for an
 *                   all-zero block), q = round-half-even(x / d) by true division, clamped to
 *                   [-128, 127], s = sequential fp32 sum
 *   KSQ_Q8F_LROUND  the generated lm_head kernel (best_kernels_GLM-5/quant_gemm/
 *                   w4a32c8_q4_0_fp32_int8_llama3_8b_lm_head_n128256_k4096/kernel.cu:85-107):
 *                   d = amax / 127 when amax > 1e-10 (else 1), q = lroundf(x * (127 /
 *                   max(amax, 1e-10))) (half away from zero), s = sequential fp32 sum */
#define KSQ_Q8F_RNE 0
#define KSQ_Q8F_LROUND 1
KSQ_API int ksq_quantize_q8f(int rule, const float* x, uint8_t* y, int M, int K, void* stream);

/* The deepseek_v2 W4A32C8 operator (core/operators/quant_gemm/variants/deepseek_v2/
 * w4a32c8_q4_0_fp32_int8: spec.json entry "forward", reference.py:5-94): Q4_0 weights, fp32
 * activations quantised per block by its rules (KSQ_Q8F_RNE: fp32 d_a and s_a), contribution
 * d_w*(d_a*sumi - 8*s_a) in fp32 (reference.py:86).  K % 256 == 0. */
KSQ_API void gemm_w4a32c8_q4_0_fp32_int8_deepseek_v2(const uint8_t* weight, const float* activation, float* output,
                                                     int M, int N, int K);

/* ---- dequantise-then-fp32 GEMM (W4A16 / W8A16) ---------------------------- */

/* C[M][N] = A[M][K] . dequant(B)[N][K]^T with fp32 activations A and Q4_0 (wtype KSQ_W_Q4_0)
 * or Q8_0 (KSQ_W_Q8_0) weights B [N][K/32], no activation quantisation: the reference's W4A16 /
 * W8A16 path (gemm_w4a16_naive / gemm_w4a16_tiled / gemm_w8a16_naive, include/gemm_cuda_naive.cuh:
 * 267-283 and include/gemm_cuda_tiled.cuh:284-291 over the kernels :66-150 and :108-190; CPU
 * references gemm_w4a16_reference / gemm_w8a16_reference, include/gemm_reference.h:73-147) and
 * the harness oracle of the fp32-activation definitions (llm_kernel_test/reference/gemm_ref.py:
 * 51-97).  Every product a * q is exact (bf16 MFMA on a three-term split of each activation);
 * the fp32 sums round in another order than the reference's loop (agreement within fp32
 * accumulation error).  Argument order of the reference launchers: A, B, C.  A 16-byte
 * aligned, finite, |a| < 3.38e38; B and C 4-byte aligned; K % 64 == 0.  workspace: the split-K
 * partial sums, ksq_gemm_w16_workspace_size(M, N, K) bytes (0 when the grid needs no split), or
 * NULL for the library's per-device pool.  Returns a ksq_status. */
KSQ_API size_t ksq_gemm_w16_workspace_size(int M, int N, int K);
KSQ_API int ksq_gemm_w16(int wtype, const float* A, const uint8_t* B, float* C, int M, int N, int K,
                         void* workspace, size_t workspace_bytes, void* stream);
/* The reference launchers' form (stream, pool workspace): gemm_w4a16_naive / gemm_w4a16_tiled
 * (Q4_0) and gemm_w8a16_naive (Q8_0). */
KSQ_API int ksq_gemm_w4a16(const float* A, const uint8_t* B, float* C, int M, int N, int K, void* stream);
KSQ_API int ksq_gemm_w8a16(const float* A, const uint8_t* B, float* C, int M, int N, int K, void* stream);

/* Workspace bytes ksq_gemm needs for (wtype, atype, M, N, K): the quantised copy of fp32 or
 * fp16 activations (block_q8_1 rows, or the LDS-DMA GEMM's planar form for fp32 x Q4_0 / Q4_1
 * at large M, 42 bytes per block), plus the split-K partial sums of small MFMA grids (so it can
 * be non-zero for pre-quantised activations too).  The workspace must be 16-byte aligned. */
KSQ_API size_t ksq_gemm_workspace_size(int wtype, int atype, int M, int N, int K);

/* General entry: wtype = enum ksq_wtype, atype = enum ksq_atype (the block_q8s forms pair
 * with Q8_0 weights only, KSQ_ERR_TYPE otherwise; KSQ_A_F16 takes fp16 activations, 16-byte
 * aligned, quantised by the fused FP16 kernels' rules as KSQ_Q81_FUSED_F16; the block_q8f forms
 * pair with Q4_0, Q5_0 and Q8_0 weights and need K % 256 == 0; fp32 rows take the decode kernel
 * (quantising in every workgroup) at M <= 2 where it applies, else the int8 MFMA GEMM, block
 * contribution d_w*(d_a*sumi - c*s_a) with c = 8 / 16 / 0 in fp32).  workspace may be
 * NULL (then a per-device pool owned by the library is used, which makes the call
 * allocate on first use and when sizes grow).  Returns a ksq_status. */
KSQ_API int ksq_gemm(int wtype, int atype, const void* weight, const void* activation, float* output,
             int M, int N, int K, void* workspace, size_t workspace_bytes, void* stream);

/* No counterpart in the reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): ksq_gemm whose scratch
 * (the quantised copy of fp32 / fp16 activations, split-K partial sums) is a static device array
 * of KSQ_NOALLOC_SCRATCH_BYTES on each GPU, held until the process ends.  Makes no hipMalloc /
 * hipFree.  A call whose ksq_gemm_workspace_size() exceeds KSQ_NOALLOC_SCRATCH_BYTES returns
 * KSQ_ERR_WORKSPACE without launching.  All calls on one GPU share that GPU's array: calls that
 * overlap on one GPU (concurrent streams) race; calls in one stream are ordered. */
#define KSQ_NOALLOC_SCRATCH_BYTES (32u << 20)
KSQ_API int ksq_gemm_noalloc(int wtype, int atype, const void* weight, const void* activation, float* output,
                             int M, int N, int K, void* stream);

/* Debug / calibration: a plain streaming read of `bytes` device bytes at p (16-byte aligned,
 * bytes % 16 == 0) with the decode kernels' 16-byte loads, 32 KiB per workgroup; writes one XOR
 * word per workgroup to out (ksq_debug_stream_read_outputs(bytes) words).  The read-only speed of
 * a given byte count, the ceiling a bandwidth-bound kernel of that size is measured against. */
KSQ_API size_t ksq_debug_stream_read_outputs(size_t bytes);
KSQ_API int ksq_debug_stream_read(const void* p, size_t bytes, uint32_t* out, void* stream);
/* The same read with wg_bytes (a positive multiple of 4096, at most 1 GiB) per workgroup instead
 * of 32 KiB, so a read-size curve can pick the launch shape that covers the CUs evenly; writes
 * ksq_debug_stream_read_wg_outputs(bytes, wg_bytes) XOR words (0 for an invalid wg_bytes). */
KSQ_API size_t ksq_debug_stream_read_wg_outputs(size_t bytes, size_t wg_bytes);
KSQ_API int ksq_debug_stream_read_wg(const void* p, size_t bytes, size_t wg_bytes, uint32_t* out, void* stream);

/* Debug / measurement: the two launches of an fp32 ksq_gemm call that takes the LDS-DMA GEMM
 * (Q4_0 / Q4_1 weights, K % 256 == 0, the 128 x 128-tile shapes), run separately so that the
 * GEMM kernel can be timed alone.  ksq_debug_quantize_planar writes the planar block_q8_1
 * activations of x [M][K] (fp32, 16-byte aligned) for weight type wtype into `planar`
 * (ksq_debug_planar_bytes(M, K) bytes, 256-byte aligned): the same blocks as
 * ksq_quantize_q8_1, split into an int8 quant plane [M][K], (d, -12582912 d) fp32 pairs
 * [K/32][Mp] (d = the fp16 scale, divided by 8 for Q4_0) and -s fp16 bits [K/128][Mp][4]
 * (Mp = M rounded up to 128).  ksq_debug_gemm_planar runs the GEMM on them; it splits along K
 * where ksq_gemm would, with its partial sums in the library's workspace pool.  The two in a
 * row write what ksq_gemm writes for the same fp32 input. */
KSQ_API size_t ksq_debug_planar_bytes(int M, int K);
KSQ_API int ksq_debug_quantize_planar(int wtype, const float* x, void* planar, int M, int K, void* stream);
KSQ_API int ksq_debug_gemm_planar(int wtype, const void* weight, const void* planar, float* output, int M, int N,
                                  int K, void* stream);

/* Debug: per-block integer dot products out[M][N][nblk] (nblk = K/32, or K/16 for
 * Q6_K) computed by the device block-dot code of the decode kernels. */
KSQ_API int ksq_debug_block_sumi(int wtype, const void* weight, const uint8_t* act_q8_1, int32_t* out,
                         int M, int N, int K, void* stream);

/* Debug: the same per-block integer dots taken from the int8 MFMA tiles of the
 * prefill GEMM (all weight types).  K % 256 == 0, act_q8_1 16-byte aligned, weight
 * 16-byte aligned (4-byte for Q6_K). */
KSQ_API int ksq_debug_block_sumi_mfma(int wtype, const void* weight, const uint8_t* act_q8_1, int32_t* out,
                              int M, int N, int K, void* stream);

/* ---- expert-grouped MoE (no reference counterpart for GGML types) ----------
 * output[t][n] = sum over the top_k experts e chosen for token t of
 *                w[t][e] * (Q8_1(activation[t]) . weight[e][n]),
 * weight = E experts, each [N][K/32] blocks (Q4_0, Q8_0, Q4_1, Q5_0 or Q5_1), back to back.
 * Routing: softmax over router_logits[t][0..E-1] (fp32), the top_k experts by logit
 * (ties -> lower index); w = the softmax probabilities of the chosen experts, or those
 * divided by their sum when renorm != 0.  K % 256 == 0, E <= 256, top_k <= E.
 * For top_k <= 2 every output element receives exactly top_k fp32 additions onto
 * zero, so the result does not depend on their order.
 * Structure after the reference's FP8 MoE kernel (results/moe/moe_fp8_block_scale_ds_
 * routing_topk8_ng8_kg4_e32_h7168_i2048/ksearch_best_moe.cu:44,193-236,525-582). */
KSQ_API size_t ksq_moe_workspace_size(int wtype, int T, int N, int K, int E, int top_k);
/* topk_ids_out [T][top_k] / topk_weights_out [T][top_k]: optional device outputs of the routing. */
KSQ_API int ksq_moe_gemm(int wtype, const void* weights, const float* activation, const float* router_logits,
                         float* output, int T, int N, int K, int E, int top_k, int renorm,
                         int32_t* topk_ids_out, float* topk_weights_out,
                         void* workspace, size_t workspace_bytes, void* stream);
/* The same with caller-supplied routing (ids in [0, E); other ids contribute nothing). */
KSQ_API int ksq_moe_gemm_routed(int wtype, const void* weights, const float* activation,
                                const int32_t* topk_ids, const float* topk_weights, float* output,
                                int T, int N, int K, int E, int top_k,
                                void* workspace, size_t workspace_bytes, void* stream);
/* Drop-in style void entry for the Q4_0 up-projection (default stream, internal workspace). */
KSQ_API void moe_w4a32c8_q4_0_fp32_int8(const uint8_t* weight, const float* activation,
                                        const float* router_logits, float* output,
                                        int T, int N, int K, int E, int top_k);

/* Path selection for testing and benchmarking, for calls made from the calling host thread
 * (other threads keep their own setting): 0 = automatic (default), 1 = always the v_dot4 decode
 * kernels, 2 = always the int8 MFMA GEMM where it applies, 3 = the 4x4x4-MFMA small-batch
 * kernel where it applies (M <= 8; M <= 32 with K % 128 == 0 and 16-byte aligned activations). */
KSQ_API int ksq_set_path(int path);

/* MFMA tile configuration for tuning, for calls made from the calling host thread: 0 = chosen
 * from (M, N) (default); 1 = 128x128 tile, K step 8; 2 = 128x64; 3 = 64x64; 4 = 128x128 with
 * K step 4; 5 = 32x128; 6 = 128x128 with K step 4 and the next step's loads prefetched into
 * registers; 7 = 64x128. */
KSQ_API int ksq_set_mmq_config(int config);

/* Debug: the kernel families the last ksq_gemm / drop-in / MoE / fused-FP16 call made on the
 * calling host thread launched, as a bit set of: */
#define KSQ_ENG_QUANTIZE (1u << 0)        /* separate activation quantise launch */
#define KSQ_ENG_GEMV_ROW (1u << 1)        /* gemv_row_kernel (LDS-staged v_dot4 decode) */
#define KSQ_ENG_GEMV_ROW_FQ (1u << 2)     /* gemv_row_kernel quantising fp32 rows per workgroup */
#define KSQ_ENG_GEMV_DIRECT (1u << 3)     /* gemv_direct_kernel (1-2 rows, register-direct) */
#define KSQ_ENG_GEMV_DIRECT_FQ (1u << 4)  /* gemv_direct_fq_kernel (fp32 rows quantised per workgroup) */
#define KSQ_ENG_GEMV_MR (1u << 5)         /* gemv_direct_mr_kernel (3-8 rows) */
#define KSQ_ENG_GEMV_MR_FQ (1u << 6)      /* gemv_direct_mr_kernel quantising fp32 rows */
#define KSQ_ENG_GEMV_KQ (1u << 7)         /* gemv_direct_kq_kernel (Q4_K / Q6_K, 1-2 rows) */
#define KSQ_ENG_SKINNY (1u << 8)          /* skinny_kernel (4x4x4 int8 MFMA, M <= 8) */
#define KSQ_ENG_MMQ_CFG(c) (1u << (8 + (c))) /* mmq_kernel with tile configuration c = 1..7 */
#define KSQ_ENG_SPLITK (1u << 16)         /* the MFMA GEMM split along K, plus its reduction */
#define KSQ_ENG_MOE_ROUTE (1u << 17)      /* MoE routing */
#define KSQ_ENG_MOE_GROUP (1u << 18)      /* MoE grouping / tile schedule */
#define KSQ_ENG_MOE_TILE64 (1u << 19)     /* grouped mmq_kernel, 64-row tiles */
#define KSQ_ENG_MOE_TILE128 (1u << 20)    /* grouped mmq_kernel, 128-row tiles */
#define KSQ_ENG_MOE_COMBINE (1u << 21)    /* slot-ordered combine of per-entry rows */
#define KSQ_ENG_TRANSPOSE (1u << 22)      /* output transpose (fused FP16 orientation) */
#define KSQ_ENG_W16 (1u << 23)            /* w16_kernel (dequantise-then-fp32 GEMM on the bf16 MFMA) */
#define KSQ_ENG_MMQ_PLANAR (1u << 24)     /* mmq_planar_kernel (planar block_q8_1 staged by LDS DMA) */
#define KSQ_ENG_MOE_PLANAR (1u << 25)     /* grouped mmq_planar_kernel (128-row tiles, expert-sorted planar rows) */
KSQ_API uint32_t ksq_debug_last_engines(void);

#ifdef __cplusplus
}
#endif

#endif /* KSQ_H */
