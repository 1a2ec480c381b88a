/*
 * ksq_blocks.h - byte layouts of the GGML quantisation blocks used by the
 * quantized-matmul path.  Plain C11, no GPU or fp16 types: every half-precision
 * field is carried as its raw IEEE binary16 bit pattern (uint16_t).
 *
 * Reference layouts (kept byte-identical, so buffers produced for the
 * reference can be handed over unchanged):
 *   block_q4_0  kernelevalplus-main/include/quant_types.h:59-64
 *               offsets kernelevalplus-main/core/operators/common/types.py:80-91
 *   block_q8_0  quant_types.h:116-121, types.py:142-153
 *   block_q8_1  quant_types.h:147-152, types.py:156-169
 *               (ds = half2: d in the low half, s = sum of the source floats
 *                in the high half)
 *   block_q4_1  quant_types.h:88-95, types.py:94-108
 *   block_q5_0  types.py:110-123 (used by kernels/gemm/gemm_quant_formats.cuh:162-208)
 *   block_q5_1  types.py:125-140 (gemm_quant_formats.cuh:222-267)
 * block_q8s is the activation block of the native W8A8C8 operator
 * (core/operators/quant_gemm/variants/deepseek_v3/w8a8c8_q8_0_q8_1/kernel.cu:66-93):
 * that kernel keeps the per-block scale in fp32 and never stores a sum, so its
 * quantised activations are {float d; int8 qs[32]}, 36 B with qs at the same
 * offset as block_q8_1.
 * block_q8f is the activation block of the generated kernels that keep the Q8_1 scale and sum
 * in fp32: the deepseek_v2 W4A32C8 operator's reference
 * (core/operators/quant_gemm/variants/deepseek_v2/w4a32c8_q4_0_fp32_int8/reference.py:50-73)
 * and the lm_head kernel's quantiser (best_kernels_GLM-5/quant_gemm/
 * w4a32c8_q4_0_fp32_int8_llama3_8b_lm_head_n128256_k4096/kernel.cu:85-107) compute d_a and
 * s_a as fp32 and never round them to fp16; {float d; float s; int8 qs[32]}, 40 B.
 * The K-quant super-blocks are absent from the reference; they follow the
 * public GGML layout (ggml-common.h, QK_K = 256):
 *   block_q4_K  {half d; half dmin; u8 scales[12]; u8 qs[128]}      144 B
 *   block_q6_K  {u8 ql[128]; u8 qh[64]; i8 scales[16]; half d}      210 B
 *
 * Blocks are only 2-byte aligned inside a row (18- and 34-byte blocks), so
 * device code never dereferences these structs directly; they document the
 * layout and pin it with static assertions.
 */
#ifndef KSQ_BLOCKS_H
#define KSQ_BLOCKS_H

#include <stddef.h>
#include <stdint.h>

#define KSQ_QK4_0 32
#define KSQ_QK8_0 32
#define KSQ_QK8_1 32
#define KSQ_QK4_1 32
#define KSQ_QK5_0 32
#define KSQ_QK5_1 32
#define KSQ_QK_K 256
#define KSQ_K_SCALE_SIZE 12

typedef struct {
    uint16_t d;                 /* fp16 scale */
    uint8_t qs[KSQ_QK4_0 / 2];  /* element j<16 in the low nibble of qs[j], j>=16 in the high nibble of qs[j-16] */
} ksq_block_q4_0;

typedef struct {
    uint16_t d;                 /* fp16 scale */
    int8_t qs[KSQ_QK8_0];
} ksq_block_q8_0;

typedef struct {
    uint16_t d;                 /* fp16 scale (low half of the reference's half2 ds) */
    uint16_t s;                 /* fp16 sum of the 32 source floats (high half) */
    int8_t qs[KSQ_QK8_1];
} ksq_block_q8_1;

typedef struct {
    uint16_t d;                 /* fp16 scale */
    uint16_t m;                 /* fp16 offset: value = q * d + m, q in 0..15 */
    uint8_t qs[KSQ_QK4_1 / 2];  /* nibble order as block_q4_0 */
} ksq_block_q4_1;

typedef struct {
    uint16_t d;                 /* fp16 scale: value = (q - 16) * d, q in 0..31 */
    uint8_t qh[4];              /* bit j of the little-endian word = bit 4 of element j */
    uint8_t qs[KSQ_QK5_0 / 2];  /* low 4 bits, nibble order as block_q4_0 */
} ksq_block_q5_0;

typedef struct {
    uint16_t d;                 /* fp16 scale */
    uint16_t m;                 /* fp16 offset: value = q * d + m, q in 0..31 */
    uint8_t qh[4];
    uint8_t qs[KSQ_QK5_1 / 2];
} ksq_block_q5_1;

typedef struct {
    float d;                    /* fp32 scale (amax / 127, or 1 when that is below 1e-6) */
    int8_t qs[KSQ_QK8_1];
} ksq_block_q8s;

typedef struct {
    float d;                    /* fp32 scale */
    float s;                    /* fp32 sequential sum of the 32 source floats */
    int8_t qs[KSQ_QK8_1];
} ksq_block_q8f;

typedef struct {
    uint16_t d;                          /* super-block scale for the 6-bit sub-block scales */
    uint16_t dmin;                       /* super-block scale for the 6-bit sub-block mins */
    uint8_t scales[KSQ_K_SCALE_SIZE];    /* 8 scales + 8 mins, 6 bits each */
    uint8_t qs[KSQ_QK_K / 2];            /* 4-bit quants, 64-element groups: low nibbles then high nibbles */
} ksq_block_q4_K;

typedef struct {
    uint8_t ql[KSQ_QK_K / 2];            /* low 4 bits of the 6-bit quants */
    uint8_t qh[KSQ_QK_K / 4];            /* high 2 bits */
    int8_t scales[KSQ_QK_K / 16];        /* 16 signed 8-bit sub-block scales */
    uint16_t d;                          /* fp16 super-block scale */
} ksq_block_q6_K;

#if defined(__cplusplus)
#define KSQ_STATIC_ASSERT static_assert
#else
#define KSQ_STATIC_ASSERT _Static_assert
#endif

KSQ_STATIC_ASSERT(sizeof(ksq_block_q4_0) == 18, "block_q4_0 must be 18 bytes");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q4_0, qs) == 2, "block_q4_0.qs at offset 2");
KSQ_STATIC_ASSERT(sizeof(ksq_block_q8_0) == 34, "block_q8_0 must be 34 bytes");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q8_0, qs) == 2, "block_q8_0.qs at offset 2");
KSQ_STATIC_ASSERT(sizeof(ksq_block_q8_1) == 36, "block_q8_1 must be 36 bytes");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q8_1, s) == 2, "block_q8_1.s (high half of ds) at offset 2");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q8_1, qs) == 4, "block_q8_1.qs at offset 4");
KSQ_STATIC_ASSERT(sizeof(ksq_block_q4_1) == 20, "block_q4_1 must be 20 bytes");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q4_1, m) == 2, "block_q4_1.m at offset 2");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q4_1, qs) == 4, "block_q4_1.qs at offset 4");
KSQ_STATIC_ASSERT(sizeof(ksq_block_q5_0) == 22, "block_q5_0 must be 22 bytes");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q5_0, qh) == 2, "block_q5_0.qh at offset 2");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q5_0, qs) == 6, "block_q5_0.qs at offset 6");
KSQ_STATIC_ASSERT(sizeof(ksq_block_q5_1) == 24, "block_q5_1 must be 24 bytes");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q5_1, qh) == 4, "block_q5_1.qh at offset 4");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q5_1, qs) == 8, "block_q5_1.qs at offset 8");
KSQ_STATIC_ASSERT(sizeof(ksq_block_q8s) == 36, "block_q8s must be 36 bytes");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q8s, qs) == 4, "block_q8s.qs at offset 4, as in block_q8_1");
KSQ_STATIC_ASSERT(sizeof(ksq_block_q8f) == 40, "block_q8f must be 40 bytes");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q8f, s) == 4, "block_q8f.s at offset 4");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q8f, qs) == 8, "block_q8f.qs at offset 8");
KSQ_STATIC_ASSERT(sizeof(ksq_block_q4_K) == 144, "block_q4_K must be 144 bytes");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q4_K, scales) == 4, "block_q4_K.scales at offset 4");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q4_K, qs) == 16, "block_q4_K.qs at offset 16");
KSQ_STATIC_ASSERT(sizeof(ksq_block_q6_K) == 210, "block_q6_K must be 210 bytes");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q6_K, qh) == 128, "block_q6_K.qh at offset 128");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q6_K, scales) == 192, "block_q6_K.scales at offset 192");
KSQ_STATIC_ASSERT(offsetof(ksq_block_q6_K, d) == 208, "block_q6_K.d at offset 208");

/* Weight-type codes shared by the C ABI and the Python host layer. */
enum ksq_wtype {
    KSQ_W_Q4_0 = 0,
    KSQ_W_Q8_0 = 1,
    KSQ_W_Q4_K = 2,
    KSQ_W_Q6_K = 3,
    KSQ_W_Q4_1 = 4,
    KSQ_W_Q5_0 = 5,
    KSQ_W_Q5_1 = 6,
};

/* Activation-type codes. */
enum ksq_atype {
    KSQ_A_F32 = 0,   /* fp32 [M][K], quantised to Q8_1 inside the call */
    KSQ_A_Q8_1 = 1,  /* pre-quantised block_q8_1 [M][K/32] */
    KSQ_A_F32_Q8S = 2, /* fp32 [M][K], quantised to block_q8s inside the call (native W8A8C8 rules) */
    KSQ_A_Q8S = 3,   /* pre-quantised block_q8s [M][K/32] */
    KSQ_A_F16 = 4,   /* fp16 [M][K], quantised to Q8_1 inside the call by the fused FP16 kernels' rules */
    KSQ_A_Q8F = 5,   /* pre-quantised block_q8f [M][K/32] (Q4_0, Q5_0, Q8_0 weights; K % 256 == 0) */
    KSQ_A_F32_Q8F_RNE = 6,    /* fp32 [M][K] -> block_q8f inside the call, rule KSQ_Q8F_RNE */
    KSQ_A_F32_Q8F_LROUND = 7, /* fp32 [M][K] -> block_q8f inside the call, rule KSQ_Q8F_LROUND */
};

#endif /* KSQ_BLOCKS_H */
