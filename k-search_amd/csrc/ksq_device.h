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
typedef float f32x2 __attribute__((ext_vector_type(2)));
// the same vectors at 4-byte alignment: global loads of 16 / 8 bytes from dword-aligned addresses
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2a4 __attribute__((ext_vector_type(2), aligned(4)));

// Linear tile of workgroup x in a 1-D grid of gx (a multiple of 8) workgroups: workgroups go to
// the 8 XCDs round robin (XCD = x % 8), so XCD j takes tiles j * gx / 8 .. (j + 1) * gx / 8 - 1,
// a contiguous run of the row-major tile order (whole rows of tiles for grids of 8 rows or more).
__device__ __forceinline__ int xcd_tile(int x, int gx) { return (x % 8) * (gx / 8) + x / 8; }

// LDS written by some lanes of a wave and read by other lanes of the same wave.  The
// wavefront-scope release / acquire pair keeps the compiler from moving LDS accesses across
// the point or reusing a value read before it (a lane that wrote nothing may otherwise keep its
// earlier read of the same address); LDS operations of one wave complete in order, so no
// wait instruction is needed for the hardware.
__device__ __forceinline__ void wave_lds_exchange() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int kQ40Bytes = 18;
constexpr int kQ80Bytes = 34;
constexpr int kQ81Bytes = 36;
constexpr int kQ4KBytes = 144;
constexpr int kQ6KBytes = 210;
constexpr int kQ41Bytes = 20;
constexpr int kQ50Bytes = 22;
constexpr int kQ51Bytes = 24;

// Weight-type codes (enum ksq_wtype of include/ksq_blocks.h).
constexpr int kWQ40 = 0, kWQ80 = 1, kWQ4K = 2, kWQ6K = 3, kWQ41 = 4, kWQ50 = 5, kWQ51 = 6;

// The K-quant super-block types (256 elements) versus the 32-element block types.
__host__ __device__ constexpr bool is_kquant(int wt) { return wt == kWQ4K || wt == kWQ6K; }

// Bytes of one 32-element block of a non-K-quant type.
__host__ __device__ constexpr int block_bytes(int wt) {
    return wt == kWQ40 ? kQ40Bytes : wt == kWQ80 ? kQ80Bytes : wt == kWQ41 ? kQ41Bytes
         : wt == kWQ50 ? kQ50Bytes : kQ51Bytes;
}

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
//
// Two paths with identical results.  When the sum is finite every input is finite, so
// max|x| is a plain v_max3 reduction; when 1/d is finite as well, |x * id| <= 127 * (1 + 2^-22),
// and roundf(y) = trunc(y + copysign(0.49999997f, y)) there (0.49999997f = the float below
// 0.5: the sum is exact or rounds away from the next integer, checked exhaustively on the
// CPU over every float in [0.25, 128]), so each quant is mul, bfi, add, cvt with no clamp
// (|q| <= 127).  Blocks holding inf / NaN, or so small that 1/d overflows, take the general
// path: the reference's comparison-based max and roundf with out-of-range -> INT32_MIN.
__device__ __forceinline__ void quantize_block_q8_1(const float* v, uint32_t* out) {
#pragma clang fp contract(off)
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) sum += v[j];
    const bool finite = __builtin_isfinite(sum);
    float amax = 0.0f;
    if (finite) {
#pragma unroll
        for (int j = 0; j < 32; j++) amax = __builtin_fmaxf(amax, fabsf(v[j]));
    } else {
#pragma unroll
        for (int j = 0; j < 32; j++) {
            const float a = fabsf(v[j]);
            amax = (amax < a) ? a : amax;
        }
    }
    const float d = amax / 127.0f;
    const float id = (d > 0.0f) ? 1.0f / d : 0.0f;
    out[0] = f32_to_f16(d) | (f32_to_f16(sum) << 16);
    if (finite && __builtin_isfinite(id)) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            int q[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const float y = v[4 * j + t] * id;
                q[t] = (int)(y + __builtin_copysignf(0.49999997f, y));
            }
            const uint32_t lo = (uint32_t)__builtin_bit_cast(int, __builtin_amdgcn_cvt_pk_i16(q[0], q[1]));
            const uint32_t hi = (uint32_t)__builtin_bit_cast(int, __builtin_amdgcn_cvt_pk_i16(q[2], q[3]));
            out[1 + j] = __builtin_amdgcn_perm(hi, lo, 0x06040200u);  // bytes 0, 2 of lo, then of hi
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t packed = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) packed |= clamp_i8(round_to_i32(v[4 * j + t] * id)) << (8 * t);
            out[1 + j] = packed;
        }
    }
}

// Quantise 32 floats to one block_q8s, the activation block of the native W8A8C8 operator
// (kernelevalplus-main/core/operators/quant_gemm/variants/deepseek_v3/w8a8c8_q8_0_q8_1/
// kernel.cu:66-93): amax = fmaxf over |x| from 0, d = amax / 127 in fp32 (1 when below 1e-6,
// kept in fp32), q = clamp((int)roundf(x / d), -128, 127) with a true division.  That
// operator's float -> int conversion is the device one (NaN -> 0, saturation); clamping the
// rounded value before converting gives the same bytes.  out[0] = d bits, out[1..8] = quants.
__device__ __forceinline__ void quantize_block_q8s(const float* v, uint32_t* out) {
#pragma clang fp contract(off)
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(v[j]));
    float d = amax / 127.0f;
    if (d < 1e-6f) d = 1.0f;
    out[0] = __builtin_bit_cast(uint32_t, d);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint32_t packed = 0;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float r = roundf(v[4 * j + t] / d);
            const int q = (r != r) ? 0 : (r >= 127.0f ? 127 : (r <= -128.0f ? -128 : (int)r));
            packed |= ((uint32_t)q & 0xFFu) << (8 * t);
        }
        out[1 + j] = packed;
    }
}

// Quantise 32 values (fp16 inputs widened to fp32) to one block_q8_1 by the fused FP16 kernels'
// rules (quantize_fp16_to_q8_1_smem, kernels/gemm/gemm_fused.cuh:76-145): max |x| and the sum
// by the shared-memory tree (pairs 16, 8, 4, 2 apart, then element 0 with element 1),
// d = max / 127, ds = (half(d), half(sum)), id = 1 / half(d) (0 when half(d) is 0),
// q = roundf(x * id) saturated to int8, then clamped to [-127, 127].
__device__ __forceinline__ void quantize_block_q8_1_f16tree(const float* v, uint32_t* out) {
#pragma clang fp contract(off)
    float m[32], t[32];
#pragma unroll
    for (int j = 0; j < 32; j++) {
        m[j] = __builtin_fabsf(v[j]);
        t[j] = v[j];
    }
#pragma unroll
    for (int w = 16; w >= 2; w >>= 1)
#pragma unroll
        for (int j = 0; j < w; j++) {
            m[j] = __builtin_fmaxf(m[j], m[j + w]);
            t[j] += t[j + w];
        }
    const float d = __builtin_fmaxf(m[0], m[1]) / 127.0f;
    const float sum = t[0] + t[1];
    const uint32_t dh = f32_to_f16(d);
    out[0] = dh | (f32_to_f16(sum) << 16);
    const float dr = f16_to_f32(dh);
    const float id = (dr != 0.0f) ? 1.0f / dr : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float r = roundf(v[4 * i + k] * id);
            int q = (r != r) ? 0 : (int)__builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);
            q = q < -127 ? -127 : q;
            w |= (uint32_t)(q & 0xFF) << (8 * k);
        }
        out[1 + i] = w;
    }
}

// 32 consecutive activations starting at element `off` of X, as fp32: X holds fp32 values, or
// fp16 bit patterns when XH (16-byte aligned either way).
template <bool XH>
__device__ __forceinline__ void load_x32(const void* X, size_t off, float* x) {
    if constexpr (XH) {
        const u32x4* src = (const u32x4*)((const uint16_t*)X + off);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const u32x4 w = src[i];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                x[8 * i + 2 * k] = f16_to_f32(ws[k] & 0xFFFFu);
                x[8 * i + 2 * k + 1] = f16_to_f32(ws[k] >> 16);
            }
        }
    } else {
        const f32x4* src = (const f32x4*)((const float*)X + off);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const f32x4 q = src[i];
            x[4 * i] = q.x; x[4 * i + 1] = q.y; x[4 * i + 2] = q.z; x[4 * i + 3] = q.w;
        }
    }
}

// Quantise 32 floats to one block_q8f (fp32 d and s).  out[0] = d bits, out[1] = s bits,
// out[2..9] = quants.  s is the sequential fp32 sum in both rules.
//   RNE (deepseek_v2/w4a32c8_q4_0_fp32_int8/reference.py:50-73, float32 scalar arithmetic
//       as NumPy >= 2 evaluates it): d = amax / 127, 1 when amax is 0; q = round-half-even of
//       the fp32 quotient x / d, clamped to [-128, 127]
//   LROUND (best_kernels_GLM-5/.../lm_head_n128256_k4096/kernel.cu:85-107): d = amax / 127
//       when amax > 1e-10, else 1; q = lroundf(x * (127 / fmaxf(amax, 1e-10))), half away from
//       zero; |x * scale| <= 127 * (1 + 2^-23) for finite x, so q fits int8 without a clamp
constexpr int kQ8FRne = 0, kQ8FLround = 1;
template <int RULE>
__device__ __forceinline__ void quantize_block_q8f(const float* v, uint32_t* out) {
#pragma clang fp contract(off)
    float amax = 0.0f, sum = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) {
        amax = __builtin_fmaxf(amax, __builtin_fabsf(v[j]));
        sum += v[j];
    }
    float d, scale = 0.0f;
    if constexpr (RULE == kQ8FRne) {
        d = amax > 0.0f ? amax / 127.0f : 1.0f;
    } else {
        d = amax > 1e-10f ? amax / 127.0f : 1.0f;
        scale = 127.0f / __builtin_fmaxf(amax, 1e-10f);
    }
    out[0] = __builtin_bit_cast(uint32_t, d);
    out[1] = __builtin_bit_cast(uint32_t, sum);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint32_t packed = 0;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float x = v[4 * j + t];
            const float r = (RULE == kQ8FRne) ? __builtin_rintf(x / d) : roundf(x * scale);
            const int q = (r != r) ? 0 : (int)__builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);
            packed |= ((uint32_t)q & 0xFFu) << (8 * t);
        }
        out[2 + j] = packed;
    }
}

// Sum over the 64 lanes, returned in every lane.  Rows of 16 lanes reduce through DPP (quad_perm
// swaps of 1 and 2 lanes, then rotations by 4 and 8 within the row), and the 4 row sums are read
// out with v_readlane: register-only steps instead of 6 dependent ds_bpermute round trips
// through the LDS unit at the tail of every decode wave.
#ifndef KSQ_WAVE_SUM_DPP
#define KSQ_WAVE_SUM_DPP 1
#endif
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float v) {
#if KSQ_WAVE_SUM_DPP
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x124>(v);  // row_ror:4
    v += dpp_mov<0x128>(v);  // row_ror:8
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (r0 + r1) + (r2 + r3);
#else
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
#endif
}

// 16 consecutive activations starting at element `off` of X, as fp32: X holds fp32 values, or
// fp16 bit patterns when XH (16-byte aligned either way).
template <bool XH>
__device__ __forceinline__ void load_x16(const void* X, size_t off, float* x) {
    if constexpr (XH) {
        const u32x4* src = (const u32x4*)((const uint16_t*)X + off);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const u32x4 w = src[i];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                x[8 * i + 2 * k] = f16_to_f32(ws[k] & 0xFFFFu);
                x[8 * i + 2 * k + 1] = f16_to_f32(ws[k] >> 16);
            }
        }
    } else {
        const f32x4* src = (const f32x4*)((const float*)X + off);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const f32x4 q = src[i];
            x[4 * i] = q.x; x[4 * i + 1] = q.y; x[4 * i + 2] = q.z; x[4 * i + 3] = q.w;
        }
    }
}

// One block_q8_1 quantised by a lane pair: lanes 2i and 2i+1 of a wave hold elements 0..15 and
// 16..31 (h = lane & 1) of the same block in v[0..15].  The bytes are those of
// quantize_block_q8_1:
//  * amax is the larger of the two halves' maxima (a max that skips NaN, as both forms there do);
//  * both lanes compute d = amax / 127 and 1/d;
//  * the sum stays the left-to-right fp32 sum: the odd lane continues from the even lane's
//    partial sum of elements 0..15, and hands the total back;
//  * each lane quantises its own 16 values.
// The even lane writes words 1..4 of the block at dst, the odd lane words 0 (d, s) and 5..8.
// Both lanes of every pair must be active.
__device__ __forceinline__ void quantize_block_q8_1_pair(const float* v, int h, uint32_t* dst) {
#pragma clang fp contract(off)
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; j++) part += v[j];
    float sum = dpp_mov<0xB1>(part);                 // quad_perm [1,0,3,2]: the partner's value
#pragma unroll
    for (int j = 0; j < 16; j++) sum += v[j];       // the total on the odd lane
    const float sum_odd = dpp_mov<0xB1>(sum);
    const float s = h ? sum : sum_odd;
    const bool finite = __builtin_isfinite(s);
    float am = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const float a = fabsf(v[j]);
        am = (am < a) ? a : am;
    }
    const float am_other = dpp_mov<0xB1>(am);
    const float amax = (am < am_other) ? am_other : am;
    const float d = amax / 127.0f;
    const float id = (d > 0.0f) ? 1.0f / d : 0.0f;
    uint32_t q4[4];
    if (finite && __builtin_isfinite(id)) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int q[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const float y = v[4 * j + t] * id;
                q[t] = (int)(y + __builtin_copysignf(0.49999997f, y));
            }
            const uint32_t lo = (uint32_t)__builtin_bit_cast(int, __builtin_amdgcn_cvt_pk_i16(q[0], q[1]));
            const uint32_t hi = (uint32_t)__builtin_bit_cast(int, __builtin_amdgcn_cvt_pk_i16(q[2], q[3]));
            q4[j] = __builtin_amdgcn_perm(hi, lo, 0x06040200u);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t packed = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) packed |= clamp_i8(round_to_i32(v[4 * j + t] * id)) << (8 * t);
            q4[j] = packed;
        }
    }
    if (h) {
        dst[0] = f32_to_f16(d) | (f32_to_f16(s) << 16);
#pragma unroll
        for (int j = 0; j < 4; j++) dst[5 + j] = q4[j];
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++) dst[1 + j] = q4[j];
    }
}

// block_q8f (quantize_block_q8f, either rule) on a lane pair laid out as for
// quantize_block_q8_1_pair: the larger of the halves' fmaxf maxima, the left-to-right sum
// continued by the odd lane, d and the scale on both lanes, 16 quants a lane.  The even lane
// writes words 2..5 of the 10-word block at dst, the odd lane words 0 (d), 1 (s) and 6..9.
template <int RULE>
__device__ __forceinline__ void quantize_block_q8f_pair(const float* v, int h, uint32_t* dst) {
#pragma clang fp contract(off)
    float part = 0.0f, am = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        am = __builtin_fmaxf(am, __builtin_fabsf(v[j]));
        part += v[j];
    }
    float sum = dpp_mov<0xB1>(part);                 // quad_perm [1,0,3,2]: the partner's value
#pragma unroll
    for (int j = 0; j < 16; j++) sum += v[j];       // the total on the odd lane
    const float amax = __builtin_fmaxf(am, dpp_mov<0xB1>(am));
    float d, scale = 0.0f;
    if constexpr (RULE == kQ8FRne) {
        d = amax > 0.0f ? amax / 127.0f : 1.0f;
    } else {
        d = amax > 1e-10f ? amax / 127.0f : 1.0f;
        scale = 127.0f / __builtin_fmaxf(amax, 1e-10f);
    }
    uint32_t q4[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t packed = 0;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const float x = v[4 * j + t];
            const float r = (RULE == kQ8FRne) ? __builtin_rintf(x / d) : roundf(x * scale);
            const int q = (r != r) ? 0 : (int)__builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);
            packed |= ((uint32_t)q & 0xFFu) << (8 * t);
        }
        q4[j] = packed;
    }
    if (h) {
        dst[0] = __builtin_bit_cast(uint32_t, d);
        dst[1] = __builtin_bit_cast(uint32_t, sum);
#pragma unroll
        for (int j = 0; j < 4; j++) dst[6 + j] = q4[j];
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++) dst[2 + j] = q4[j];
    }
}

// The fused FP16 kernels' quantiser (quantize_block_q8_1_f16tree) on a lane pair laid out as for
// quantize_block_q8_1_pair.  Its reduction tree first combines elements j and j + 16, which sit
// in the two lanes of the pair: each lane takes its partner's 16 values, and both lanes run the
// same tree, so both hold d and the sum; each lane then quantises its own 16 values.  Same words
// to dst as quantize_block_q8_1_pair.
__device__ __forceinline__ void quantize_block_q8_1_f16tree_pair(const float* v, int h, uint32_t* dst) {
#pragma clang fp contract(off)
    float m[16], t[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const float o = dpp_mov<0xB1>(v[j]);        // the partner's element: j + 16 or j
        const float lo = h ? o : v[j], hi = h ? v[j] : o;
        m[j] = __builtin_fmaxf(__builtin_fabsf(lo), __builtin_fabsf(hi));
        t[j] = lo + hi;
    }
#pragma unroll
    for (int w = 8; w >= 2; w >>= 1)
#pragma unroll
        for (int j = 0; j < w; j++) {
            m[j] = __builtin_fmaxf(m[j], m[j + w]);
            t[j] += t[j + w];
        }
    const float d = __builtin_fmaxf(m[0], m[1]) / 127.0f;
    const float sum = t[0] + t[1];
    const uint32_t dh = f32_to_f16(d);
    const float dr = f16_to_f32(dh);
    const float id = (dr != 0.0f) ? 1.0f / dr : 0.0f;
    uint32_t q4[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float r = roundf(v[4 * i + k] * id);
            int q = (r != r) ? 0 : (int)__builtin_fminf(__builtin_fmaxf(r, -128.0f), 127.0f);
            q = q < -127 ? -127 : q;
            w |= (uint32_t)(q & 0xFF) << (8 * k);
        }
        q4[i] = w;
    }
    if (h) {
        dst[0] = dh | (f32_to_f16(sum) << 16);
#pragma unroll
        for (int j = 0; j < 4; j++) dst[5 + j] = q4[j];
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++) dst[1 + j] = q4[j];
    }
}

// Bits 0..3 of x moved to bit 4 of the four bytes of a word: the fifth bit of four
// consecutive Q5_0 / Q5_1 quants.  The product places bit k of x at bit 8k (its shifted
// copies x, x<<7, x<<14, x<<21 do not overlap, so nothing carries).
__device__ __forceinline__ uint32_t qh_to_bit4(uint32_t x) { return (((x & 0xFu) * 0x00204081u) & 0x01010101u) << 4; }

}  // namespace ksq
