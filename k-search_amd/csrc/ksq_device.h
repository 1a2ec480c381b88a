// ksq_device.h - device helpers shared by the gfx950 kernels.
//
// Blocks inside a weight row are only 2-byte aligned (18- and 34-byte
// blocks), so kernels load whole 16-byte chunks of a row into registers and
// pull fields out at compile-time byte offsets with v_alignbyte_b32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ksq {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kQ40Bytes = 18;
constexpr int kQ80Bytes = 34;
constexpr int kQ81Bytes = 36;
constexpr int kQ4KBytes = 144;
constexpr int kQ6KBytes = 210;

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ uint32_t f32_to_f16(float f) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32, round to nearest even
}

// 32-bit little-endian word at byte offset `off` of a register array; `off`
// must fold to a constant after unrolling.
__device__ __forceinline__ uint32_t word_at(const uint32_t* w, int off) {
    const int i = off >> 2, s = off & 3;
    return s == 0 ? w[i] : __builtin_amdgcn_alignbyte(w[i + 1], w[i], s);
}

// 16-bit field at an even byte offset of a register array.
__device__ __forceinline__ uint32_t half_at(const uint32_t* w, int off) {
    return (off & 2) ? (w[off >> 2] >> 16) : (w[off >> 2] & 0xFFFFu);
}

// v_dot4c_i32_i8: c + sum of four signed byte products.
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// Round half away from zero, then convert; out-of-range and NaN give INT32_MIN,
// the value (int)roundf(v) produces on the x86-64 host of the reference CPU path.
__device__ __forceinline__ int32_t round_to_i32(float v) {
    const float r = roundf(v);
    return (r >= -2147483648.0f && r < 2147483648.0f) ? (int32_t)r : INT32_MIN;
}

__device__ __forceinline__ uint32_t clamp_i8(int32_t q) {
    q = q < -128 ? -128 : (q > 127 ? 127 : q);
    return (uint32_t)q & 0xFFu;
}

// Quantise 32 floats to one block_q8_1, bit-exact with quantize_row_q8_1_ref
// (kernelevalplus-main/include/quantize.h:165-193): sequential fp32 sum,
// IEEE d = amax/127, id = 1/d (fp32 d), q = clamp(roundf(x*id)), ds = half2(d, sum).
// out[0] = ds word, out[1..8] = the 32 quants.
__device__ __forceinline__ void quantize_block_q8_1(const float* v, uint32_t* out) {
#pragma clang fp contract(off)
    float amax = 0.0f, sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const float a = fabsf(v[j]);
        amax = (amax < a) ? a : amax;
        sum += v[j];
    }
    const float d = amax / 127.0f;
    const float id = (d > 0.0f) ? 1.0f / d : 0.0f;
    out[0] = f32_to_f16(d) | (f32_to_f16(sum) << 16);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint32_t packed = 0;
#pragma unroll
        for (int t = 0; t < 4; t++) packed |= clamp_i8(round_to_i32(v[4 * j + t] * id)) << (8 * t);
        out[1 + j] = packed;
    }
}

// ---------------------------------------------------------------------------
// Block dot products on register-resident blocks.  `w` holds weight bytes,
// `a` points at the 9 dwords of one block_q8_1 (ds, then 8 quant words).
// ---------------------------------------------------------------------------

// Integer part of vec_dot_q4_0_q8_1 (kernelevalplus-main/include/gemm_reference.h:200-212):
// sumi = sum_k qa[k]*(qs[k]&15) + qa[k+16]*(qs[k]>>4).
__device__ __forceinline__ int sumi_q4_0(const uint32_t* w, int off, const uint32_t* a) {
    int sumi = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t q = word_at(w, off + 2 + 4 * i);
        sumi = dot4((int)(q & 0x0F0F0F0Fu), (int)a[1 + i], sumi);
        sumi = dot4((int)((q >> 4) & 0x0F0F0F0Fu), (int)a[5 + i], sumi);
    }
    return sumi;
}

// Integer part of vec_dot_q8_0_q8_1 (gemm_reference.h:253-256).
__device__ __forceinline__ int sumi_q8_0(const uint32_t* w, int off, const uint32_t* a) {
    int sumi = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) sumi = dot4((int)word_at(w, off + 2 + 4 * i), (int)a[1 + i], sumi);
    return sumi;
}

// Block contribution d_w * (d_a * sumi - 8 * s_a) (gemm_reference.h:216).
__device__ __forceinline__ float block_q4_0(const uint32_t* w, int off, const uint32_t* a) {
    const int sumi = sumi_q4_0(w, off, a);
    const float dw = f16_to_f32(half_at(w, off));
    const float da = f16_to_f32(a[0] & 0xFFFFu), sa = f16_to_f32(a[0] >> 16);
    return dw * (da * (float)sumi - 8.0f * sa);
}

// Block contribution sumi * d_a * d_w (gemm_reference.h:259).
__device__ __forceinline__ float block_q8_0(const uint32_t* w, int off, const uint32_t* a) {
    const int sumi = sumi_q8_0(w, off, a);
    const float dw = f16_to_f32(half_at(w, off));
    const float da = f16_to_f32(a[0] & 0xFFFFu);
    return (float)sumi * da * dw;
}

template <typename T>
__device__ __forceinline__ T ldg_nt(const T* p) {
    return __builtin_nontemporal_load(p);
}

}  // namespace ksq
