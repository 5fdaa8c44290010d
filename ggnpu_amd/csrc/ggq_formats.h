// ggq_formats.h -- GGUF block geometry shared by host and device code.
//
// Block sizes and byte sizes follow the GGUF type table
// (ggnpu src/gguf/tensor.cpp:18-38, ids include/ggnpu/tensor.h:11-42).
// A "group" is the run of values sharing one scale: the granularity of the
// int32 block dot products the prefill GEMM accumulates before scaling.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define GGQ_HD __host__ __device__ __forceinline__
#else
#define GGQ_HD inline
#endif

namespace ggq {

enum Type : uint32_t {
    T_F32 = 0,
    T_Q8_0 = 8,
    T_Q4_K = 12,
    T_Q5_K = 13,
    T_Q6_K = 14,
    T_IQ4_NL = 20,
    T_IQ4_XS = 23,
};

GGQ_HD int block_elems(uint32_t t) {
    return (t == T_Q8_0 || t == T_IQ4_NL) ? 32
         : (t == T_Q4_K || t == T_Q5_K || t == T_Q6_K || t == T_IQ4_XS) ? 256 : 0;
}

GGQ_HD int block_bytes(uint32_t t) {
    switch (t) {
    case T_Q8_0: return 34;
    case T_IQ4_NL: return 18;
    case T_Q4_K: return 144;
    case T_Q5_K: return 176;
    case T_Q6_K: return 210;
    case T_IQ4_XS: return 136;
    default: return 0;
    }
}

// Values per scale group (Q6_K has one int8 scale per 16 values).
GGQ_HD int group_elems(uint32_t t) { return t == T_Q6_K ? 16 : (block_elems(t) ? 32 : 0); }

GGQ_HD bool supported(uint32_t t) { return block_elems(t) != 0; }

GGQ_HD int64_t row_bytes(uint32_t t, int64_t K) { return (K / block_elems(t)) * block_bytes(t); }

// Device copies of weights are padded by this many bytes so that the
// realigning loads (which may touch up to 4 bytes past a block) stay inside
// the allocation.
constexpr int kWeightPad = 256;

}  // namespace ggq
