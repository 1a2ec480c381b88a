// ksq_internal.h - host-side launchers shared between the kernel files and
// the C ABI layer (ksq_abi.hip).  Launchers assume their arguments were
// validated by the ABI layer (shapes, alignment, non-null pointers) and
// return the hipError_t of the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ksq {

// fp32 [rows][K] -> block_q8_1 [rows][K/32]; x 16-byte aligned, y 4-byte aligned.
hipError_t launch_quantize_q8_1(const float* x, uint8_t* y, int64_t rows, int K, hipStream_t s);

// Decode GEMV/GEMM on v_dot4 (mul_mat_vec_q family), any M; activations are Q8_1.
// wtype: 0 Q4_0, 1 Q8_0, 2 Q4_K, 3 Q6_K.
hipError_t launch_gemv(int wtype, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int K,
                       hipStream_t s);

// Prefill GEMM on int8 MFMA (mul_mat_q family); returns hipErrorNotSupported
// for shapes it does not tile.
bool mmq_supported(int wtype, int M, int N, int K, const void* W, const void* A);
hipError_t launch_mmq(int wtype, const uint8_t* W, const uint8_t* A, float* C, int M, int N, int K,
                      hipStream_t s);

// Per-block integer dots [M][N][nblk] from the same device block-dot code the
// decode kernels use (debug entry for the bit-exact check).
hipError_t launch_block_sumi(int wtype, const uint8_t* W, const uint8_t* A, int32_t* out, int M, int N,
                             int K, hipStream_t s);

// Fill `n` floats with zero (a kernel, so it can be captured in a graph).
hipError_t launch_fill_zero(float* p, int64_t n, hipStream_t s);

}  // namespace ksq
