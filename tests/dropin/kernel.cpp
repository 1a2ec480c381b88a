// kernel.cpp - the forwarding file a KernelEvalPlus maintainer compiles in place of a quant_gemm
// definition's kernel.cu to run it on libksq: each entry point forwards to the libksq symbol of
// the same name.
//
// The reference harness generates a pybind wrapper around the definition's entry point
// (kernelevalplus-main/llm_kernel_test/op_test_handler.py:298-349) which declares
//     extern "C" void <entry>(const uint8_t* weight, const <act_t>* activation, float* output,
//                             int M, int N, int K);
// and calls it with device pointers on the default stream.  libksq.so exports those entry names
// itself (include/ksq.h), so this file only includes the header and forwards; linking -lksq
// resolves them.  dropin_forward() is the C-callable stand-in for that generated wrapper: it
// looks the definition's entry point up by name and calls it exactly as the wrapper would.
#include <cstdint>
#include <cstring>

#include "ksq.h"

namespace {
using EntryF32 = void (*)(const uint8_t*, const float*, float*, int, int, int);
using EntryU8 = void (*)(const uint8_t*, const uint8_t*, float*, int, int, int);

struct Entry {
    const char* name;
    EntryF32 f32;
    EntryU8 u8;
};

const Entry kEntries[] = {
    {"gemm_w4a32c8_q4_0_fp32_int8", gemm_w4a32c8_q4_0_fp32_int8, nullptr},
    {"gemm_w8a32c8_q8_0_fp32_int8", gemm_w8a32c8_q8_0_fp32_int8, nullptr},
    {"gemm_w4a32c8_q4_1_fp32_int8", gemm_w4a32c8_q4_1_fp32_int8, nullptr},
    {"gemm_w8a8c8_q8_0_q8_1", gemm_w8a8c8_q8_0_q8_1, nullptr},
    {"gemm_w4a32c8_q4_k_fp32_int8", gemm_w4a32c8_q4_k_fp32_int8, nullptr},
    {"gemm_w6a32c8_q6_k_fp32_int8", gemm_w6a32c8_q6_k_fp32_int8, nullptr},
    {"ksq_gemm_q4_0_q8_1", nullptr, ksq_gemm_q4_0_q8_1},
    {"ksq_gemm_q8_0_q8_1", nullptr, ksq_gemm_q8_0_q8_1},
};
}  // namespace

// Returns ksq_last_error() after the call, or -1 for an entry name libksq does not export.
extern "C" int dropin_forward(const char* entry, const uint8_t* weight, const void* activation, float* output, int M,
                              int N, int K) {
    for (const Entry& e : kEntries) {
        if (std::strcmp(e.name, entry) != 0) continue;
        if (e.f32) e.f32(weight, static_cast<const float*>(activation), output, M, N, K);
        else e.u8(weight, static_cast<const uint8_t*>(activation), output, M, N, K);
        return ksq_last_error();
    }
    return -1;
}
