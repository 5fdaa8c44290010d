// ggq_kernels.hip -- CDNA4 (gfx950) kernels of the quantized-matmul backend.
//
// Raw GGUF weight blocks are read straight from HBM (no re-quantization);
// block decode is fused into every kernel through ggq_device.h.
//
//   dequant_kernel     bit-exact fp32 dequant (parity probe for the decoders)
//   block_dot_kernel   int32 per-group dot products of codes x int8 activations
//   quant_act_*        per-row / per-32-block int8 activation quantization
//   gemv_kernel        decode GEMV (batch 1..8, also expert-grouped for MoE)
//   gemm_i8_kernel     prefill GEMM on int8 MFMA (v_mfma_i32_32x32x32_i8)
//   moe_*              top-k routing, expert grouping, SwiGLU, weighted combine
//
// The reference path these replace: CpuRefBackend::mul_mat_q
// (src/backends/cpu_ref/cpu_ref.cpp:25-137) and the XDNA int8 tile loop
// (src/backends/amd_xdna/amd_xdna.cpp:491-952).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <mutex>
#include <set>
#include <vector>

#include "ggq_device.h"
#include "ggq_launch.h"

namespace ggq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

#define GGQ_DISPATCH_TYPE(t, F)                 \
    switch (t) {                                \
    case T_Q4_K: F(T_Q4_K); break;              \
    case T_Q5_K: F(T_Q5_K); break;              \
    case T_Q6_K: F(T_Q6_K); break;              \
    case T_Q8_0: F(T_Q8_0); break;              \
    case T_IQ4_NL: F(T_IQ4_NL); break;          \
    case T_IQ4_XS: F(T_IQ4_XS); break;          \
    default: return hipErrorInvalidValue;       \
    }

// =================================================================== dequant
// One thread per 16 values: codes16 + group_scale, then the reference's
// rounding order (dequant_value).
template <int T>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ raw, int64_t n16,
                                                      float* __restrict__ out) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n16) return;
    constexpr int be = T == T_Q8_0 || T == T_IQ4_NL ? 32 : 256;
    constexpr int bb = T == T_Q8_0 ? 34 : T == T_IQ4_NL ? 18 : T == T_Q4_K ? 144
                     : T == T_Q5_K ? 176 : T == T_Q6_K ? 210 : 136;
    const int64_t b = g / (be / 16);
    const int k = (int)(g % (be / 16)) * 16;
    const uint8_t* blk = raw + b * bb;
    const uint4 c = codes16<T>(blk, k);
    const GroupScale gs = group_scale<T>(blk, k);
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
    float4* o = (float4*)(out + b * be + k);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float4 v;
        v.x = dequant_value(gs, (int)(int8_t)(w[i] & 0xFFu));
        v.y = dequant_value(gs, (int)(int8_t)((w[i] >> 8) & 0xFFu));
        v.z = dequant_value(gs, (int)(int8_t)((w[i] >> 16) & 0xFFu));
        v.w = dequant_value(gs, (int)(int8_t)(w[i] >> 24));
        o[i] = v;
    }
}

hipError_t launch_dequant(uint32_t type, const void* raw, int64_t n_blocks, float* out, hipStream_t s) {
    const int64_t n16 = n_blocks * (block_elems(type) / 16);
    if (n16 == 0) return hipSuccess;
    const dim3 grid((unsigned)((n16 + 255) / 256));
#define L(TT) dequant_kernel<TT><<<grid, 256, 0, s>>>((const uint8_t*)raw, n16, out)
    GGQ_DISPATCH_TYPE(type, L)
#undef L
    return hipGetLastError();
}

// ================================================================= block dot
template <int T>
__global__ __launch_bounds__(256) void block_dot_kernel(const uint8_t* __restrict__ W, int N, int K,
                                                        const int8_t* __restrict__ qa, int M,
                                                        int32_t* __restrict__ out) {
    constexpr int ge = T == T_Q6_K ? 16 : 32;
    const int G = K / ge;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)M * N * G) return;
    const int g = (int)(idx % G);
    const int n = (int)((idx / G) % N);
    const int m = (int)(idx / ((int64_t)G * N));
    const uint8_t* row = W + (int64_t)n * row_bytes(T, K);
    int acc = 0;
#pragma unroll
    for (int h = 0; h < ge / 16; h++) {
        const int k = g * ge + 16 * h;
        const uint4 c = codes16<T>(row, k);
        const uint4 a = *(const uint4*)(qa + (int64_t)m * K + k);
        acc = __builtin_amdgcn_sdot4((int)c.x, (int)a.x, acc, false);
        acc = __builtin_amdgcn_sdot4((int)c.y, (int)a.y, acc, false);
        acc = __builtin_amdgcn_sdot4((int)c.z, (int)a.z, acc, false);
        acc = __builtin_amdgcn_sdot4((int)c.w, (int)a.w, acc, false);
    }
    out[idx] = acc;
}

hipError_t launch_block_dot(uint32_t type, const void* W, int N, int K, const int8_t* qa, int M,
                            int32_t* out, hipStream_t s) {
    const int64_t total = (int64_t)M * N * (K / group_elems(type));
    if (total == 0) return hipSuccess;
    const dim3 grid((unsigned)((total + 255) / 256));
#define L(TT) block_dot_kernel<TT><<<grid, 256, 0, s>>>((const uint8_t*)W, N, K, qa, M, out)
    GGQ_DISPATCH_TYPE(type, L)
#undef L
    return hipGetLastError();
}

// ========================================================= activation quant
// Reference: amd_xdna.cpp:633-639 (scale = amax/127, or 1 for a zero row) and
// :598-603, :757-771 (q = clamp(nearbyint(a * (1/scale)), -128, 127)).
// Division and rint are IEEE (correctly rounded / half-to-even).
__device__ __forceinline__ int8_t to_i8(float v) {
    float r = __builtin_rintf(v);
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    return (int8_t)(int)r;
}

// Sum over the 256 threads of a workgroup (four wavefronts), in a fixed
// order; every thread gets the total.
__device__ __forceinline__ float wg_sum256(float v, float* red4) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red4[0] + red4[1]) + (red4[2] + red4[3]);
}

// Producers that may run ahead of the quantization, in the same launch:
// PROD_RMS is CpuRefBackend::rms_norm (cpu_ref.cpp:139-156), x * (1 /
// sqrt(sum(x^2) / K + eps)) * w[k] (w null = 1), the sum of squares taken
// over the workgroup in a fixed order; PROD_SWIGLU is silu(g) * u with
// silu(g) = g / (1 + exp(-g)) (main.cpp:3164-3165, 3474-3477).
enum { PROD_NONE = 0, PROD_RMS = 1, PROD_SWIGLU = 2 };

// The row of up to 16384 values (K a multiple of 4, 16-byte aligned) held
// in registers, 16 float4 per thread: all loads issued before the first is
// used and each value read once; produced, then quantized as below.
template <int P>
__device__ __forceinline__ void quant_row_regs(const float* a, const float* aux, float eps, int m, int K,
                                               int8_t* __restrict__ q, float* __restrict__ scales,
                                               float* __restrict__ x_eff, float* __restrict__ prod_out = nullptr,
                                               float* __restrict__ gsum = nullptr) {
    __shared__ float wmax[4];
    constexpr int R = 16;
    float4 v[R];
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int k = 4 * threadIdx.x + 1024 * i;
        v[i] = k < K ? *(const float4*)(a + k) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    if constexpr (P == PROD_SWIGLU) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int k = 4 * threadIdx.x + 1024 * i;
            if (k >= K) break;
            const float4 u = *(const float4*)(aux + k);
            v[i].x = (v[i].x / (1.0f + expf(-v[i].x))) * u.x;
            v[i].y = (v[i].y / (1.0f + expf(-v[i].y))) * u.y;
            v[i].z = (v[i].z / (1.0f + expf(-v[i].z))) * u.z;
            v[i].w = (v[i].w / (1.0f + expf(-v[i].w))) * u.w;
        }
    }
    if constexpr (P == PROD_RMS) {
        __shared__ float wss[4];
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < R; i++)
            ss = fmaf(v[i].w, v[i].w, fmaf(v[i].z, v[i].z, fmaf(v[i].y, v[i].y, fmaf(v[i].x, v[i].x, ss))));
        ss = wg_sum256(ss, wss);
        // 1 / sqrt(v) with each step correctly rounded, as the reference's
        // fp32 code computes it: the fp64 square root rounded once to fp32
        // is the correctly rounded fp32 square root (53 >= 2 * 24 + 2 bits).
        const float var = __fadd_rn(__fdiv_rn(ss, (float)K), eps);
        const float is = __fdiv_rn(1.0f, (float)__dsqrt_rn((double)var));
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int k = 4 * threadIdx.x + 1024 * i;
            if (k >= K) break;
            const float4 w = aux ? *(const float4*)(aux + k) : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            v[i].x = __fmul_rn(__fmul_rn(v[i].x, is), w.x);
            v[i].y = __fmul_rn(__fmul_rn(v[i].y, is), w.y);
            v[i].z = __fmul_rn(__fmul_rn(v[i].z, is), w.z);
            v[i].w = __fmul_rn(__fmul_rn(v[i].w, is), w.w);
        }
    }
    // The produced row itself, when asked for (stage-by-stage checks of the
    // layers that quantize a produced row).
    if (prod_out) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int k = 4 * threadIdx.x + 1024 * i;
            if (k >= K) break;
            *(float4*)(prod_out + (int64_t)m * K + k) = v[i];
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < R; i++)
        amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v[i].x), fabsf(v[i].y))), fmaxf(fabsf(v[i].z), fabsf(v[i].w)));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float sc = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 1.0f;
    const float inv = __fdiv_rn(1.0f, sc);
    if (threadIdx.x == 0 && scales) scales[m] = sc;
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int k = 4 * threadIdx.x + 1024 * i;
        if (k >= K) break;
        const int8_t c0 = to_i8(__fmul_rn(v[i].x, inv)), c1 = to_i8(__fmul_rn(v[i].y, inv));
        const int8_t c2 = to_i8(__fmul_rn(v[i].z, inv)), c3 = to_i8(__fmul_rn(v[i].w, inv));
        if (q)
            *(uint32_t*)(q + (int64_t)m * K + k) = (uint32_t)(uint8_t)c0 | (uint32_t)(uint8_t)c1 << 8 |
                                                   (uint32_t)(uint8_t)c2 << 16 | (uint32_t)(uint8_t)c3 << 24;
        if (x_eff)
            *(float4*)(x_eff + (int64_t)m * K + k) =
                make_float4(__fmul_rn((float)c0, sc), __fmul_rn((float)c1, sc), __fmul_rn((float)c2, sc),
                            __fmul_rn((float)c3, sc));
        if (gsum) {  // code sums per 32 values (eight consecutive threads), exact in fp32
            int cs = (int)c0 + (int)c1 + (int)c2 + (int)c3;
            cs += __shfl_xor(cs, 1, 64);
            cs += __shfl_xor(cs, 2, 64);
            cs += __shfl_xor(cs, 4, 64);
            if ((threadIdx.x & 7) == 0) gsum[(int64_t)m * (K / 32) + k / 32] = (float)cs;
        }
    }
}

// Producer + row quantization, one workgroup per row (register path only).
template <int P>
__global__ __launch_bounds__(256) void produce_quant_row_kernel(const float* __restrict__ A,
                                                                const float* __restrict__ aux, int lda, int K,
                                                                float eps, int8_t* __restrict__ q,
                                                                float* __restrict__ scales,
                                                                float* __restrict__ prod_out,
                                                                float* __restrict__ gsum) {
    const int m = blockIdx.x;
    const float* au = P == PROD_SWIGLU ? aux + (int64_t)m * lda : aux;
    quant_row_regs<P>(A + (int64_t)m * lda, au, eps, m, K, q, scales, nullptr, prod_out, gsum);
}

// One workgroup per row: absolute maximum, then codes.  With 16-byte
// aligned rows (lda, K multiples of 4) each thread moves float4 / 4 codes
// at a time; the arithmetic per element is the same either way.
__global__ __launch_bounds__(256) void quant_act_row_kernel(const float* __restrict__ A, int lda, int K,
                                                            int8_t* __restrict__ q, float* __restrict__ scales,
                                                            float* __restrict__ x_eff, int vec4) {
    __shared__ float wmax[4];
    const int m = blockIdx.x;
    const float* a = A + (int64_t)m * lda;
    float amax = 0.0f;
    if (vec4 && K <= 1024 * 16) {
        quant_row_regs<PROD_NONE>(a, nullptr, 0.0f, m, K, q, scales, x_eff);
        return;
    }
    if (vec4) {
        for (int k = 4 * threadIdx.x; k < K; k += 1024) {
            const float4 v = *(const float4*)(a + k);
            amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
        }
    } else {
        for (int k = threadIdx.x; k < K; k += 256) amax = fmaxf(amax, fabsf(a[k]));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float sc = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 1.0f;
    const float inv = __fdiv_rn(1.0f, sc);
    if (threadIdx.x == 0 && scales) scales[m] = sc;
    if (vec4) {
        for (int k = 4 * threadIdx.x; k < K; k += 1024) {
            const float4 v = *(const float4*)(a + k);
            const int8_t c0 = to_i8(__fmul_rn(v.x, inv)), c1 = to_i8(__fmul_rn(v.y, inv));
            const int8_t c2 = to_i8(__fmul_rn(v.z, inv)), c3 = to_i8(__fmul_rn(v.w, inv));
            if (q)
                *(uint32_t*)(q + (int64_t)m * K + k) = (uint32_t)(uint8_t)c0 | (uint32_t)(uint8_t)c1 << 8 |
                                                       (uint32_t)(uint8_t)c2 << 16 | (uint32_t)(uint8_t)c3 << 24;
            if (x_eff)
                *(float4*)(x_eff + (int64_t)m * K + k) =
                    make_float4(__fmul_rn((float)c0, sc), __fmul_rn((float)c1, sc), __fmul_rn((float)c2, sc),
                                __fmul_rn((float)c3, sc));
        }
        return;
    }
    for (int k = threadIdx.x; k < K; k += 256) {
        const int8_t v = to_i8(__fmul_rn(a[k], inv));
        if (q) q[(int64_t)m * K + k] = v;
        if (x_eff) x_eff[(int64_t)m * K + k] = __fmul_rn((float)v, sc);
    }
}

__global__ __launch_bounds__(256) void quant_act_b32_kernel(const float* __restrict__ A, int lda, int M, int K,
                                                            int8_t* __restrict__ q, float* __restrict__ scales,
                                                            float* __restrict__ x_eff) {
    const int nb = K / 32;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)M * nb) return;
    const int m = (int)(idx / nb), b = (int)(idx % nb);
    const float* a = A + (int64_t)m * lda + 32 * b;
    float amax = 0.0f;
    for (int k = 0; k < 32; k++) amax = fmaxf(amax, fabsf(a[k]));
    const float sc = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 1.0f;
    const float inv = __fdiv_rn(1.0f, sc);
    if (scales) scales[idx] = sc;
    for (int k = 0; k < 32; k++) {
        const int8_t v = to_i8(__fmul_rn(a[k], inv));
        if (q) q[(int64_t)m * K + 32 * b + k] = v;
        if (x_eff) x_eff[(int64_t)m * K + 32 * b + k] = __fmul_rn((float)v, sc);
    }
}

template <int P>
__global__ void produce_quant_wave_kernel(const float* __restrict__ A, const float* __restrict__ aux, int lda, int M,
                                          int K, int8_t* __restrict__ q, float* __restrict__ scales,
                                          float* __restrict__ prod_out, float* __restrict__ gsum);

hipError_t launch_quant_act(const float* A, int lda, int M, int K, int mode, int8_t* q,
                            float* scales, float* x_eff, hipStream_t s) {
    if (M == 0 || K == 0) return hipSuccess;
    if (mode == 1 && !x_eff && K <= 2048 && K % 8 == 0 && (uintptr_t)A % 16 == 0 && lda % 4 == 0 &&
        (uintptr_t)q % 8 == 0) {
        // rows of up to 2048 values: a wavefront per row (the same codes)
        produce_quant_wave_kernel<PROD_NONE><<<(M + 3) / 4, 256, 0, s>>>(A, nullptr, lda, M, K, q, scales, nullptr,
                                                                         nullptr);
    } else if (mode == 1) {
        const int vec4 = ((uintptr_t)A % 16 == 0) && lda % 4 == 0 && K % 4 == 0 && ((uintptr_t)q % 4 == 0) &&
                         ((uintptr_t)x_eff % 16 == 0);
        quant_act_row_kernel<<<M, 256, 0, s>>>(A, lda, K, q, scales, x_eff, vec4);
    } else {
        const int64_t n = (int64_t)M * (K / 32);
        quant_act_b32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(A, lda, M, K, q, scales, x_eff);
    }
    return hipGetLastError();
}

// Producer (none or SwiGLU) + row quantization for rows of up to 2048
// values: one wavefront per row, four rows per workgroup, lane l holding the
// 8-value chunks l, l + 64, ...; the row maximum by a wavefront reduction
// (no barrier).  Same arithmetic per value as quant_row_regs, so the codes
// and scales are identical; code sums per 32 values from 4 lanes.
template <int P>
__device__ __forceinline__ void quant_row_wave(const float* __restrict__ A, const float* __restrict__ aux,
                                               int lda, int m, int K, int8_t* __restrict__ q,
                                               float* __restrict__ scales, float* __restrict__ prod_out,
                                               float* __restrict__ gsum, int lane);
template <int P>
__global__ __launch_bounds__(256) void produce_quant_wave_kernel(const float* __restrict__ A,
                                                                 const float* __restrict__ aux, int lda, int M,
                                                                 int K, int8_t* __restrict__ q,
                                                                 float* __restrict__ scales,
                                                                 float* __restrict__ prod_out,
                                                                 float* __restrict__ gsum) {
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;
    quant_row_wave<P>(A, aux, lda, m, K, q, scales, prod_out, gsum, lane);
}

// Row m by one wavefront (lane = its lane), K <= 2048.
template <int P>
__device__ __forceinline__ void quant_row_wave(const float* __restrict__ A, const float* __restrict__ aux,
                                               int lda, int m, int K, int8_t* __restrict__ q,
                                               float* __restrict__ scales, float* __restrict__ prod_out,
                                               float* __restrict__ gsum, int lane) {
    constexpr int R = 4;  // chunks per lane (K <= 2048)
    const float* a = A + (int64_t)m * lda;
    const float* u = P == PROD_SWIGLU ? aux + (int64_t)m * lda : nullptr;
    float4 v[R][2];
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int k = 8 * (lane + 64 * i);
        if (k < K) {
            v[i][0] = *(const float4*)(a + k);
            v[i][1] = *(const float4*)(a + k + 4);
        } else {
            v[i][0] = v[i][1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    if constexpr (P == PROD_SWIGLU) {
        auto sw = [](float g, float uu) { return (g / (1.0f + expf(-g))) * uu; };
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int k = 8 * (lane + 64 * i);
            if (k >= K) continue;
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const float4 uv = *(const float4*)(u + k + 4 * hh);
                float4& x = v[i][hh];
                x = make_float4(sw(x.x, uv.x), sw(x.y, uv.y), sw(x.z, uv.z), sw(x.w, uv.w));
            }
        }
    }
    if (prod_out) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int k = 8 * (lane + 64 * i);
            if (k >= K) continue;
            *(float4*)(prod_out + (int64_t)m * K + k) = v[i][0];
            *(float4*)(prod_out + (int64_t)m * K + k + 4) = v[i][1];
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
            amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v[i][hh].x), fabsf(v[i][hh].y))), fmaxf(fabsf(v[i][hh].z), fabsf(v[i][hh].w)));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    const float sc = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 1.0f;
    const float inv = __fdiv_rn(1.0f, sc);
    if (lane == 0 && scales) scales[m] = sc;
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int k = 8 * (lane + 64 * i);
        int cs = 0;
        uint32_t w[2];
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const float4 x = v[i][hh];
            const int8_t c0 = to_i8(__fmul_rn(x.x, inv)), c1 = to_i8(__fmul_rn(x.y, inv));
            const int8_t c2 = to_i8(__fmul_rn(x.z, inv)), c3 = to_i8(__fmul_rn(x.w, inv));
            cs += (int)c0 + (int)c1 + (int)c2 + (int)c3;
            w[hh] = (uint32_t)(uint8_t)c0 | (uint32_t)(uint8_t)c1 << 8 | (uint32_t)(uint8_t)c2 << 16 |
                    (uint32_t)(uint8_t)c3 << 24;
        }
        if (k < K && q) *(uint2*)(q + (int64_t)m * K + k) = make_uint2(w[0], w[1]);
        if (gsum) {  // 32 values = 4 consecutive lanes (exact in fp32)
            cs += __shfl_xor(cs, 1, 64);
            cs += __shfl_xor(cs, 2, 64);
            if (k < K && (lane & 3) == 0) gsum[(int64_t)m * (K / 32) + k / 32] = (float)cs;
        }
    }
}

hipError_t launch_produce_quant(int producer, const float* A, const float* aux, int lda, int M, int K, float eps,
                                int8_t* q, float* scales, hipStream_t s, float* prod_out, float* gsum) {
    if (M == 0) return hipSuccess;
    if (K <= 0 || K > 1024 * 16 || K % 4 || lda % 4 || (uintptr_t)A % 16 || (uintptr_t)aux % 16 ||
        (uintptr_t)q % 4 || (uintptr_t)prod_out % 16 || (gsum && K % 32))
        return hipErrorInvalidValue;
    // rows of up to 2048 values: a wavefront per row
    const bool wave = K <= 2048 && K % 8 == 0 && (uintptr_t)q % 8 == 0;
    if (wave && producer == PROD_SWIGLU && aux)
        produce_quant_wave_kernel<PROD_SWIGLU><<<(M + 3) / 4, 256, 0, s>>>(A, aux, lda, M, K, q, scales, prod_out, gsum);
    else if (wave && producer == PROD_NONE)
        produce_quant_wave_kernel<PROD_NONE><<<(M + 3) / 4, 256, 0, s>>>(A, aux, lda, M, K, q, scales, prod_out, gsum);
    else if (producer == PROD_RMS)
        produce_quant_row_kernel<PROD_RMS><<<M, 256, 0, s>>>(A, aux, lda, K, eps, q, scales, prod_out, gsum);
    else if (producer == PROD_SWIGLU && aux)
        produce_quant_row_kernel<PROD_SWIGLU><<<M, 256, 0, s>>>(A, aux, lda, K, eps, q, scales, prod_out, gsum);
    else if (producer == PROD_NONE)
        produce_quant_row_kernel<PROD_NONE><<<M, 256, 0, s>>>(A, aux, lda, K, eps, q, scales, prod_out, gsum);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// ===================================================================== GEMV
// Work layout (256 threads, 4 wavefronts):
//   * a row of K values is P = K/32 pieces; LPR = 2^lpr_log2 threads share a
//     row (LPR = min(256, pow2ceil(P))), so one row-iteration covers 256/LPR
//     rows; thread t owns pieces lp, lp+LPR, ... (PPT of them) of row t/LPR.
//   * the thread's activations for its pieces (32 fp32 per piece and batch
//     row) stay in VGPRs for the whole row loop, so HBM carries only weight
//     blocks; activations are read once per wavefront and M-chunk.
//   * weight dwords are fetched one row-iteration ahead (register double
//     buffer) when `prefetch` is set; the first fetch is issued before the
//     activations are read.
//   * the grid is sized to the resident capacity (occupancy x CUs) and each
//     workgroup loops over its rows, so no launch runs a partial second
//     round of workgroups.
//   * partial sums are reduced with DPP / swizzle steps inside a wavefront
//     and through LDS when a row spans several wavefronts (LPR >= 128).
struct GemvArgs {
    const uint8_t* W;
    int64_t w_group_stride;
    int64_t row_bytes;
    int N, K;
    const float* X;
    int ldx;
    float* Y;
    int ldy;
    int M;
    const int* grp_off;
    const int* x_idx;
    int lpr_log2;
    int x_vec4;    // X rows are 16-byte aligned (float4 loads)
    uint32_t p_div; // ceil(2^32 / P), P = K / 32: s / P == umulhi(s, p_div) for s < 8 P
    int prefetch;  // fetch the next row-iteration while computing the current one
    // Fused neighbours of the matmul (all off when zero / null):
    const float* X2;       // elementwise product input: the activation is X * X2 (X2 like X)
    int silu;              // epilogue: Y = silu(result), silu(v) = v / (1 + exp(-v))
    int rms;               // RMSNorm each activation row first: x * (1/sqrt(mean(x^2) + eps)) * norm_w
    float eps;
    const float* norm_w;   // [K] or null (weight 1)
    const float* R;        // residual: Y = R + result, R [M][ldr] (may alias Y)
    int ldr;
    // Paired matrices (n1 > 0): rows [0, n1) come from W / go to Y, rows
    // [n1, N) are rows 0.. of W2 / Y2 (same type, K, group stride and ldy):
    // e.g. an expert's gate and up in one launch, one activation load each.
    const uint8_t* W2;
    float* Y2;
    int n1;
    // Per-row int8 activations (GGQ_ACT_Q8_ROW, LDS-staged single-row
    // launches): the staging replaces the row by its codes q = clamp(rint(x /
    // s)), s = max|x| / 127, and the outputs are scaled by s.
    int q8row;
};

// Weight row `row` of a (group's) matrix, or of the paired one.  With no
// paired matrix (n1 == 0 known at the call) the base is the uniform W.
__device__ __forceinline__ RowRef weight_row(const uint8_t* W, const uint8_t* W2, int n1, int64_t row_bytes, int row) {
    const bool second = n1 > 0 && row >= n1;
    return make_row(second ? W2 : W, (uint32_t)(second ? row - n1 : row) * (uint32_t)row_bytes);
}

// Sum over aligned groups of 2^lg lanes (lg = 0..6): afterwards every lane of
// a group of <= 32 lanes holds the group sum; for lg = 6 lane 0 holds the
// wavefront sum.
template <int CTRL> __device__ __forceinline__ float dpp_addc(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float group_sum(float v, int lg) {
    if (lg >= 1) v = dpp_addc<0xB1>(v);   // quad_perm [1,0,3,2]: xor 1
    if (lg >= 2) v = dpp_addc<0x4E>(v);   // quad_perm [2,3,0,1]: xor 2
    if (lg >= 3) v = dpp_addc<0x141>(v);  // row_half_mirror: the other quad of 8
    if (lg >= 4) v = dpp_addc<0x140>(v);  // row_mirror: the other half of 16
    if (lg >= 5) v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));  // xor 16
    if (lg >= 6) v += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    return v;
}

// Largest value over the wavefront (lane 0 holds it), the steps of
// group_sum with max.
template <int CTRL> __device__ __forceinline__ float dpp_maxc(float v) {
    return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false)));
}
__device__ __forceinline__ float wave_max_lane0(float v) {
    v = dpp_maxc<0xB1>(v);
    v = dpp_maxc<0x4E>(v);
    v = dpp_maxc<0x141>(v);
    v = dpp_maxc<0x140>(v);
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F)));
    return fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32)));
}

// Fetches are unconditional: out-of-range rows / pieces read row 0 / piece 0
// (always valid memory) and their contribution is discarded later.  Keeping
// the loads unpredicated avoids per-lane branches and register copies.
template <int T, int PPT, int U>
__device__ __forceinline__ void gemv_fetch(typename Piece<T>::Raw (&raw)[U][PPT], const uint8_t* W, int64_t row_bytes,
                                           int it, int stride, int n_iters, int rpi, int rsub, int N, int lp, int lpr,
                                           int P, const uint8_t* W2 = nullptr, int n1 = 0) {
    // Two copies of the loop: without a paired matrix the row base is the
    // uniform W (scalar-base loads).
    if (n1 > 0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int iu = it + u * stride, row = iu * rpi + rsub;
            const bool rvalid = iu < n_iters && row < N;
            const RowRef wrow = weight_row(W, W2, n1, row_bytes, rvalid ? row : 0);
#pragma unroll
            for (int i = 0; i < PPT; i++) {
                const int p = lp + i * lpr;
                raw[u][i] = Piece<T>::fetch(wrow, p < P ? p : 0);
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int iu = it + u * stride, row = iu * rpi + rsub;
            const bool rvalid = iu < n_iters && row < N;
            const RowRef wrow = weight_row(W, nullptr, 0, row_bytes, rvalid ? row : 0);
#pragma unroll
            for (int i = 0; i < PPT; i++) {
                const int p = lp + i * lpr;
                raw[u][i] = Piece<T>::fetch(wrow, p < P ? p : 0);
            }
        }
    }
}

template <int T, int MB, int PPT, int U, bool F, bool Q8 = false>
__device__ __forceinline__ void gemv_rows(const typename Piece<T>::Raw (&raw)[U][PPT], const GemvArgs& a,
                                          const uint8_t* W, const uint8_t* W2, int it, int stride, int n_iters, int rpi, int lp, int lpr,
                                          int P, int wave, int lane, int rsub, int m0, int mc, int mcount,
                                          const float (&xr)[PPT][MB][32], const float (&xs)[PPT][MB][2],
                                          float (&red)[2][4][U * MB], int& parity, float q8s) {
    float acc[U][MB];
    // The writer lane reads its residual values first, so their latency
    // overlaps the row's decode and reduction.
    float res[U][MB];
    if (F && a.R && lp == 0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int iu = it + u * stride, row = iu * rpi + rsub;
            const int rr = iu < n_iters && row < a.N ? row : 0;
#pragma unroll
            for (int m = 0; m < MB; m++) res[u][m] = a.R[(int64_t)(m0 + mc + (mc + m < mcount ? m : 0)) * a.ldr + rr];
        }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
#pragma unroll
        for (int m = 0; m < MB; m++) acc[u][m] = 0.0f;
        const int iu = it + u * stride, row = iu * rpi + rsub;
        const bool rvalid = iu < n_iters && row < a.N;
        const RowRef wrow = weight_row(W, W2, a.n1, a.row_bytes, rvalid ? row : 0);
#pragma unroll
        for (int i = 0; i < PPT; i++) {
            const int p = lp + i * lpr;
            const bool ok = p < P;
            const PieceCodes pc = Piece<T>::decode(raw[u][i], wrow, ok ? p : 0);
            float tp[MB];
#pragma unroll
            for (int r = 0; r < 2; r++) {
                float f[16];
                ubytes_to_f32(pc.u[r], f);
#pragma unroll
                for (int m = 0; m < MB; m++) {
                    float s0 = 0.0f, s1 = 0.0f;  // two chains for ILP
#pragma unroll
                    for (int j = 0; j < 16; j += 2) {
                        s0 = fmaf(xr[i][m][16 * r + j], f[j], s0);
                        s1 = fmaf(xr[i][m][16 * r + j + 1], f[j + 1], s1);
                    }
                    if (r == 0) {
                        tp[m] = fmaf(pc.a[0], s0 + s1, pc.b[0] * xs[i][m][0]);
                    } else {
                        tp[m] = fmaf(pc.a[1], s0 + s1, tp[m]);
                        tp[m] = fmaf(pc.b[1], xs[i][m][1], tp[m]);
                    }
                }
            }
#pragma unroll
            // Pieces past the row end (p >= P) decode piece 0 again but meet
            // activations zeroed when they were loaded: tp is exactly 0.
            for (int m = 0; m < MB; m++) acc[u][m] += tp[m];
        }
    }
    // A row spans at least a wavefront in the common case (K >= 2048): the
    // fixed-count reduction has no per-step branches.
    if (a.lpr_log2 >= 6) {
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int m = 0; m < MB; m++) acc[u][m] = group_sum(acc[u][m], 6);
    } else {
        const int lg = a.lpr_log2;
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int m = 0; m < MB; m++) acc[u][m] = group_sum(acc[u][m], lg);
    }
    if (a.lpr_log2 > 6) {
        if (lane == 0) {
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int m = 0; m < MB; m++) red[parity][wave][u * MB + m] = acc[u][m];
        }
        __syncthreads();
        if (lp == 0) {
            const int wpr = lpr >> 6, w0 = rsub * wpr;
#pragma unroll
            for (int u = 0; u < U; u++)
#pragma unroll
                for (int m = 0; m < MB; m++) {
                    float sum = 0.0f;
                    for (int w = 0; w < wpr; w++) sum += red[parity][w0 + w][u * MB + m];
                    acc[u][m] = sum;
                }
        }
        parity ^= 1;
    }
    if (lp == 0) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int iu = it + u * stride, row = iu * rpi + rsub;
            if (iu < n_iters && row < a.N) {
#pragma unroll
                for (int m = 0; m < MB; m++)
                    if (mc + m < mcount) {
                        float v = acc[u][m];
                        if constexpr (Q8) v = v * q8s;  // the row's int8 scale
                        if (F && a.silu) v = v / (1.0f + expf(-v));  // cpu_ref.cpp:200-209
                        const int64_t mrow = m0 + mc + m;
                        if (F && a.R) v = res[u][m] + v;
                        if (a.n1 > 0 && row >= a.n1) a.Y2[mrow * a.ldy + (row - a.n1)] = v;
                        else a.Y[mrow * a.ldy + row] = v;
                    }
            }
        }
    }
}

// RMSNorm of the activation rows held in registers (cpu_ref.cpp:139-156):
// x * (1 / sqrt(sum(x^2) / K + eps)) * w, in that order.  The sum of squares
// of a row is spread over the LPR threads that hold its pieces: DPP inside a
// wavefront, LDS across the wavefronts of a row when LPR > 64.  (The
// reference adds the squares sequentially; the order differs, the rounding
// of the sum by a few ulps.)
template <int T, int MB, int PPT>
__device__ __forceinline__ void gemv_rms_norm(const GemvArgs& a, float (&xr)[PPT][MB][32], int lp, int lpr, int P,
                                              int wave, int lane, int rsub, int mc, int mcount) {
    __shared__ float nrm[4][MB];
    float tot[MB];
#pragma unroll
    for (int m = 0; m < MB; m++) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < PPT; i++)
#pragma unroll
            for (int j = 0; j < 32; j++) ss = fmaf(xr[i][m][j], xr[i][m][j], ss);
        const int lg = a.lpr_log2 < 6 ? a.lpr_log2 : 6;
        ss = group_sum(ss, lg);
        if (lg == 6) ss = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, ss)));
        tot[m] = ss;
    }
    if (a.lpr_log2 > 6) {
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MB; m++) nrm[wave][m] = tot[m];
        }
        __syncthreads();
        const int wpr = lpr >> 6, w0 = rsub * wpr;
#pragma unroll
        for (int m = 0; m < MB; m++) {
            float t = 0.0f;
            for (int w = 0; w < wpr; w++) t += nrm[w0 + w][m];
            tot[m] = t;
        }
        __syncthreads();
    }
#pragma unroll
    for (int m = 0; m < MB; m++) {
        if (mc + m >= mcount) continue;
        const float is = 1.0f / sqrtf(tot[m] / (float)a.K + a.eps);
#pragma unroll
        for (int i = 0; i < PPT; i++) {
            const int p = lp + i * lpr;
            const int pc = p < P ? p : 0;
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const int k0 = Piece<T>::run_k(pc, r);  // a multiple of 16: float4-aligned in norm_w
                float w[16];
                if (a.norm_w) {
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float4 v = *(const float4*)(a.norm_w + k0 + 4 * j);
                        w[4 * j] = v.x; w[4 * j + 1] = v.y; w[4 * j + 2] = v.z; w[4 * j + 3] = v.w;
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 16; j++) w[j] = 1.0f;
                }
#pragma unroll
                for (int j = 0; j < 16; j++) xr[i][m][16 * r + j] = __fmul_rn(__fmul_rn(xr[i][m][16 * r + j], is), w[j]);
            }
        }
    }
}

// One workgroup's share of a GEMV problem: workgroup bx of gx working on
// group `by` (the expert in grouped mode) and on the MB-row chunks
// bz, bz + gz, ... of its activation rows.
// F: compiled with the fused options (RMSNorm, product input, silu,
// residual); the plain instantiations carry none of their code.
template <int T, int MB, int PPT, int U, bool F, bool XL = false, bool Q8 = false>
__device__ __forceinline__ void gemv_body(const GemvArgs& a, int bx, int gx, int by, int bz, int gz,
                                          float (&red)[2][4][U * MB]) {
    static_assert(!XL || MB == 1, "LDS-staged activations: one activation row per pass");
    static_assert(!Q8 || (!F && MB == 1), "per-row int8 codes: plain single-row kernels");
    if constexpr (XL) {
        // Every kernel argument the launch reads, in one round of scalar
        // loads: left to itself the compiler loads them next to their first
        // use, three dependent rounds before the first weight fetch.
        asm volatile("" ::"s"(a.W), "s"(a.w_group_stride), "s"(a.row_bytes), "s"(a.N), "s"(a.K), "s"(a.X),
                     "s"(a.ldx), "s"(a.Y), "s"(a.ldy), "s"(a.M), "s"(a.lpr_log2), "s"(a.p_div), "s"(a.prefetch),
                     "s"(a.W2), "s"(a.n1));
    }
    typedef typename Piece<T>::Raw Raw;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lpr_log2 = a.lpr_log2;
    const int lpr = 1 << lpr_log2, lp = tid & (lpr - 1), rsub = tid >> lpr_log2;
    const int rpi = 256 >> lpr_log2;
    const int P = a.K >> 5;
    const uint8_t* W = a.W + (int64_t)by * a.w_group_stride;
    const uint8_t* W2 = a.n1 > 0 ? a.W2 + (int64_t)by * a.w_group_stride : nullptr;
    int m0 = 0, mcount = a.M;
    // (The LDS-staged launches are never grouped: no dependent read of the
    // group offsets before the first weight fetch.)
    if (!XL && a.grp_off) {
        m0 = a.grp_off[by];
        mcount = a.grp_off[by + 1] - m0;
    }
    const int n_iters = (a.N + rpi - 1) / rpi;
    const int stride = gx;
    const int step = U * stride;
    int parity = 0;
    float q8s = 1.0f;  // per-row int8 activations: the row's scale

    for (int mc = bz * MB; mc < mcount; mc += gz * MB) {
        Raw ra[U][PPT], rb[U][PPT];
        int it = bx;
        // Without staging the first weight fetch is issued before the
        // activations are read.
        if constexpr (!XL) gemv_fetch<T, PPT, U>(ra, W, a.row_bytes, it, stride, n_iters, rpi, rsub, a.N, lp, lpr, P, W2, a.n1);
        float xr[PPT][MB][32];
        float xs[PPT][MB][2];
        if constexpr (XL) {
            // The activation row is read from memory once per workgroup and
            // staged in LDS as float4 slots s = 8 p' + ... transposed to
            // s = j P + p (j = 4 r + quad of run r of piece p): the stores
            // and each lane's reads of its pieces are consecutive 16-byte
            // words across lanes (no bank conflicts).  Its loads (8 P <= 1024
            // slots, at most 4 per thread) are all issued before the weight
            // fetch: loads complete in issue order, so the LDS stores wait
            // only for the (cache-resident) activations, not for the weights.
            extern __shared__ float4 xl[];
            if (mc != bz * MB) __syncthreads();  // the previous chunk's row is read by every wavefront
            const float* xp = a.X + (int64_t)(m0 + mc) * a.ldx;
            // (Unconditional loads, slots past the row reading slot 0: a
            // branch around a load makes the compiler wait for every load
            // in flight.)
            float4 xv[4], uv[F ? 4 : 1];
            const int nq = (8 * P + 255) >> 8;  // (uniform)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                if (q == 0 || q < nq) {
                    const int sl = tid + 256 * q < 8 * P ? tid + 256 * q : 0;
                    const int j = (int)__umulhi((uint32_t)sl, a.p_div);
                    const int p = sl - j * P;
                    const int k = Piece<T>::run_k(p, j >> 2) + 4 * (j & 3);
                    xv[q] = *(const float4*)(xp + k);
                    if (F && a.X2) uv[F ? q : 0] = *(const float4*)(a.X2 + (int64_t)(m0 + mc) * a.ldx + k);
                }
            }
            gemv_fetch<T, PPT, U>(ra, W, a.row_bytes, it, stride, n_iters, rpi, rsub, a.N, lp, lpr, P, W2, a.n1);
            float q8inv = 0.0f;
            if constexpr (Q8) {
                // The row's largest magnitude over the workgroup, then the
                // reference's per-row scale and codes (amd_xdna.cpp:598-603,
                // 633-639): s = max / 127, q = clamp(rint(x * (1 / s))).
                __shared__ float q8max[4];
                float mx = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if ((q == 0 || q < nq) && tid + 256 * q < 8 * P)
                        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(xv[q].x), fabsf(xv[q].y)), fmaxf(fabsf(xv[q].z), fabsf(xv[q].w))));
                mx = wave_max_lane0(mx);
                if (lane == 0) q8max[wave] = mx;
                __syncthreads();
                const float amax = fmaxf(fmaxf(q8max[0], q8max[1]), fmaxf(q8max[2], q8max[3]));
                q8s = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 1.0f;
                q8inv = __fdiv_rn(1.0f, q8s);
            }
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int sl = tid + 256 * q;
                if (sl < 8 * P) {
                    float4 v = xv[q];
                    if constexpr (Q8) {
                        auto code = [&](float x) { return fminf(fmaxf(__builtin_rintf(__fmul_rn(x, q8inv)), -128.0f), 127.0f); };
                        v = make_float4(code(v.x), code(v.y), code(v.z), code(v.w));
                    }
                    if (F && a.X2) {  // SwiGLU's product: silu(gate) (already applied) * up, main.cpp:3474-3477
                        const float4 u = uv[F ? q : 0];
                        v = make_float4(__fmul_rn(v.x, u.x), __fmul_rn(v.y, u.y), __fmul_rn(v.z, u.z), __fmul_rn(v.w, u.w));
                    }
                    xl[sl] = v;
                }
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < PPT; i++) {
                const int p = lp + i * lpr;
                const int pc = p < P ? p : 0;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float4 v = xl[j * P + pc];
                    const bool ok = p < P;
                    xr[i][0][4 * j + 0] = ok ? v.x : 0.0f; xr[i][0][4 * j + 1] = ok ? v.y : 0.0f;
                    xr[i][0][4 * j + 2] = ok ? v.z : 0.0f; xr[i][0][4 * j + 3] = ok ? v.w : 0.0f;
                }
            }
        } else
#pragma unroll
        for (int i = 0; i < PPT; i++) {
            const int p = lp + i * lpr;
            const int pc = p < P ? p : 0;
#pragma unroll
            for (int m = 0; m < MB; m++) {
                const bool ok = p < P && mc + m < mcount;
                if (mc + m >= mcount) {  // uniform over the workgroup: no load for absent rows
#pragma unroll
                    for (int j = 0; j < 32; j++) xr[i][m][j] = 0.0f;
                    xs[i][m][0] = xs[i][m][1] = 0.0f;
                    continue;
                }
                int xrow = m0 + mc + m;
                if (a.x_idx) xrow = a.x_idx[xrow];
                const float* xp = a.X + (int64_t)xrow * a.ldx;
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const int k0 = Piece<T>::run_k(pc, r);
                    if (a.x_vec4) {
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const float4 v = *(const float4*)(xp + k0 + 4 * j);
                            xr[i][m][16 * r + 4 * j + 0] = v.x; xr[i][m][16 * r + 4 * j + 1] = v.y;
                            xr[i][m][16 * r + 4 * j + 2] = v.z; xr[i][m][16 * r + 4 * j + 3] = v.w;
                        }
                    } else {
#pragma unroll
                        for (int j = 0; j < 16; j++) xr[i][m][16 * r + j] = xp[k0 + j];
                    }
                    if (F && a.X2) {  // SwiGLU's product: silu(gate) (already applied) * up, main.cpp:3474-3477
                        const float* up = a.X2 + (int64_t)xrow * a.ldx + k0;
                        float uv[16];
                        if (a.x_vec4) {
#pragma unroll
                            for (int j = 0; j < 4; j++) {
                                const float4 v = *(const float4*)(up + 4 * j);
                                uv[4 * j] = v.x; uv[4 * j + 1] = v.y; uv[4 * j + 2] = v.z; uv[4 * j + 3] = v.w;
                            }
                        } else {
#pragma unroll
                            for (int j = 0; j < 16; j++) uv[j] = up[j];
                        }
#pragma unroll
                        for (int j = 0; j < 16; j++) xr[i][m][16 * r + j] = __fmul_rn(xr[i][m][16 * r + j], uv[j]);
                    }
#pragma unroll
                    for (int j = 0; j < 16; j++) xr[i][m][16 * r + j] = ok ? xr[i][m][16 * r + j] : 0.0f;
                }
            }
        }
        if (F && a.rms) gemv_rms_norm<T, MB, PPT>(a, xr, lp, lpr, P, wave, lane, rsub, mc, mcount);
        if constexpr (Q8 && !XL) {
            // Per-row int8 codes of the row held in registers: every row
            // group of the workgroup holds all of the row's pieces, so the
            // workgroup's largest magnitude is the row's (amd_xdna.cpp:598-603,
            // 633-639: s = max / 127, q = clamp(rint(x * (1 / s)))).
            __shared__ float q8max[4];
            float mx = 0.0f;
#pragma unroll
            for (int i = 0; i < PPT; i++)
#pragma unroll
                for (int j = 0; j < 32; j++) mx = fmaxf(mx, fabsf(xr[i][0][j]));
            mx = wave_max_lane0(mx);
            if (mc != bz * MB) __syncthreads();  // the previous row's maxima are read
            if (lane == 0) q8max[wave] = mx;
            __syncthreads();
            const float amax = fmaxf(fmaxf(q8max[0], q8max[1]), fmaxf(q8max[2], q8max[3]));
            q8s = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 1.0f;
            const float inv = __fdiv_rn(1.0f, q8s);
#pragma unroll
            for (int i = 0; i < PPT; i++)
#pragma unroll
                for (int j = 0; j < 32; j++) xr[i][0][j] = fminf(fmaxf(__builtin_rintf(__fmul_rn(xr[i][0][j], inv)), -128.0f), 127.0f);
        }
#pragma unroll
        for (int i = 0; i < PPT; i++)
#pragma unroll
            for (int m = 0; m < MB; m++)
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    float sum = 0.0f;
#pragma unroll
                    for (int j = 0; j < 16; j++) sum += xr[i][m][16 * r + j];
                    xs[i][m][r] = sum;
                }

        if (!a.prefetch) {
            // Fetch, then decode/multiply/reduce; latency is hidden by the
            // other resident wavefronts.
            while (true) {
                gemv_rows<T, MB, PPT, U, F, Q8>(ra, a, W, W2, it, stride, n_iters, rpi, lp, lpr, P, wave, lane, rsub, m0, mc,
                                         mcount, xr, xs, red, parity, q8s);
                it += step;
                if (it >= n_iters) break;
                gemv_fetch<T, PPT, U>(ra, W, a.row_bytes, it, stride, n_iters, rpi, rsub, a.N, lp, lpr, P, W2, a.n1);
            }
            continue;
        }
        // Ping-pong between ra and rb: fetch the next U row-iterations, then
        // decode/multiply/reduce the current ones.
        while (it < n_iters) {
            gemv_fetch<T, PPT, U>(rb, W, a.row_bytes, it + step, stride, n_iters, rpi, rsub, a.N, lp, lpr, P, W2, a.n1);
            gemv_rows<T, MB, PPT, U, F, Q8>(ra, a, W, W2, it, stride, n_iters, rpi, lp, lpr, P, wave, lane, rsub, m0, mc, mcount,
                                     xr, xs, red, parity, q8s);
            it += step;
            if (it >= n_iters) break;
            gemv_fetch<T, PPT, U>(ra, W, a.row_bytes, it + step, stride, n_iters, rpi, rsub, a.N, lp, lpr, P, W2, a.n1);
            gemv_rows<T, MB, PPT, U, F, Q8>(rb, a, W, W2, it, stride, n_iters, rpi, lp, lpr, P, wave, lane, rsub, m0, mc, mcount,
                                     xr, xs, red, parity, q8s);
            it += step;
        }
    }
}

template <int T, int MB, int PPT, int U, bool F = false, bool XL = false, bool Q8 = false>
// Two rows per pass: held to 3 wavefronts per SIMD (168 VGPRs; Q4_K spills
// a few registers), where the natural allocation gave 2.  That variant is
// the MoE default (each expert sees ~2 tokens: the decoded codes are shared).
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MB == 2 ? 3 : 1))) void gemv_kernel(GemvArgs a) {
    __shared__ float red[2][4][U * MB];
    if constexpr (MB > 1) {
        if (a.grp_off) {
            // Grouped launch: each group (expert) has its own row count, so
            // the rows per pass follow it instead of the launch maximum.
            const int cnt = a.grp_off[blockIdx.y + 1] - a.grp_off[blockIdx.y];
            if (cnt <= 0) return;
            if (cnt == 1) {
                gemv_body<T, 1, PPT, U, F>(a, blockIdx.x, gridDim.x, blockIdx.y, 0, 1,
                                        *reinterpret_cast<float(*)[2][4][U]>(&red));
                return;
            }
            if (MB > 2 && cnt == 2) {
                gemv_body<T, 2, PPT, U, F>(a, blockIdx.x, gridDim.x, blockIdx.y, 0, 1,
                                        *reinterpret_cast<float(*)[2][4][U * 2]>(&red));
                return;
            }
        }
    }
    gemv_body<T, MB, PPT, U, F, XL, Q8>(a, blockIdx.x, gridDim.x, blockIdx.y, blockIdx.z, gridDim.z, red);
}

// Several independent GEMV problems (any mix of formats, same pieces-per-
// thread) in one launch: workgroups [begin[q], begin[q+1]) serve problem q.
// Used where matmuls share a dependency level, e.g. the q/k/v projections
// (one input) or gate/up of a decode step.
constexpr int kMaxMulti = 8;
struct MultiArgs {
    GemvArgs p[kMaxMulti];
    uint32_t type[kMaxMulti];
    int begin[kMaxMulti + 1];
    int n;
};

// KQ: compiled for Q4_K and Q6_K only (the Q4_K_M decode levels), so the
// register budget is not set by the other formats' decoders (Q5_K's needs
// one more wavefront's worth of VGPRs than Q4_K's).
template <int MB, int PPT, int U, bool F = false, bool KQ = false, bool XL = false, bool Q8 = false>
__global__ __launch_bounds__(256) void gemv_multi_kernel(MultiArgs ma) {
    __shared__ float red[2][4][U * MB];
    int q = 0;
    while (q + 1 < ma.n && (int)blockIdx.x >= ma.begin[q + 1]) q++;
    const int bx = blockIdx.x - ma.begin[q], gx = ma.begin[q + 1] - ma.begin[q];
    const int bz = blockIdx.z, gz = gridDim.z;
    if constexpr (KQ) {
        if (ma.type[q] == T_Q4_K) gemv_body<T_Q4_K, MB, PPT, U, F, XL, Q8>(ma.p[q], bx, gx, 0, bz, gz, red);
        else gemv_body<T_Q6_K, MB, PPT, U, F, XL, Q8>(ma.p[q], bx, gx, 0, bz, gz, red);
        return;
    }
    switch (ma.type[q]) {
    case T_Q4_K: gemv_body<T_Q4_K, MB, PPT, U, F, XL, Q8>(ma.p[q], bx, gx, 0, bz, gz, red); break;
    case T_Q5_K: gemv_body<T_Q5_K, MB, PPT, U, F, XL, Q8>(ma.p[q], bx, gx, 0, bz, gz, red); break;
    case T_Q6_K: gemv_body<T_Q6_K, MB, PPT, U, F, XL, Q8>(ma.p[q], bx, gx, 0, bz, gz, red); break;
    case T_Q8_0: gemv_body<T_Q8_0, MB, PPT, U, F, XL, Q8>(ma.p[q], bx, gx, 0, bz, gz, red); break;
    case T_IQ4_NL: gemv_body<T_IQ4_NL, MB, PPT, U, F, XL, Q8>(ma.p[q], bx, gx, 0, bz, gz, red); break;
    case T_IQ4_XS: gemv_body<T_IQ4_XS, MB, PPT, U, F, XL, Q8>(ma.p[q], bx, gx, 0, bz, gz, red); break;
    default: break;
    }
}

// ============================================ GEMV on the matrix cores
// Several activation rows (M >= 2, fp32 activations): the weight codes of a
// piece are decoded once and multiplied against up to 4*MS activation rows
// with v_mfma_f32_4x4x4_16b_f16 instead of one fp32 FMA chain per row.
//
// Layout: lane = 4*blk + j (blk 0..15 per wavefront).  The 64 blocks of the
// workgroup are piece slots; S = 2^lpr_log2 (16, 32 or 64) slots serve one
// group of 4 weight rows, so a row-iteration covers 4*(64/S) rows.  Lane j
// of a block owns weight row 4*group + j and activation row j (+4t) at the
// block's pieces sg, sg+S, ... (PPT of them).  One MFMA multiplies the 4x4
// activation slice A[m][k] (lane j supplies row m = j) by the 4x4 code slice
// B[k][n] (lane j supplies its own row's codes); D[m][n] lands in lane j,
// register m.  A run's 16 codes are 4 such slices of one lane, so the run's
// scale a[r] and bias b[r] (per weight row) apply to D as in the fp32 path:
//   sum_k x_k w_k = sum_r a[r] * D_r + b[r] * sum(x_run_r).
// Codes are small unsigned integers (<= 255), exact in fp16.  Activations
// are scaled per row by a power of two that puts the row's largest
// magnitude (over the workgroup's slots) in [2^14, 2^15) and split as
// hi + lo (both fp16, hi rounded toward zero, lo = x - hi rounded toward
// zero): |x - hi - lo| <= 2^-20 |x| for values above 2^-18 of the row
// maximum, 2^-40 of the maximum below that; the power of two is undone
// exactly at the store.  The MFMA accumulates in fp32; hi and lo go into
// one accumulator per run.
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));

// Two codes (bytes 0,1 or 2,3 of w, by selector) as an fp16 pair: the byte
// becomes the low mantissa byte of 1024.0 (0x64 high byte), then 1024 is
// subtracted (exact).
__device__ __forceinline__ uint32_t codes_f16x2(uint32_t w, uint32_t sel) {
    const h2v v = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, w, sel));
    const h2v off = {(_Float16)1024.0f, (_Float16)1024.0f};
    return __builtin_bit_cast(uint32_t, v - off);
}
__device__ __forceinline__ h4v codes_slice(uint32_t w) {
    return __builtin_bit_cast(h4v, make_uint2(codes_f16x2(w, 0x04010400u), codes_f16x2(w, 0x04030402u)));
}
__device__ __forceinline__ uint32_t u4_at(const uint4& u, int i) { return i == 0 ? u.x : i == 1 ? u.y : i == 2 ? u.z : u.w; }

// Broadcast of lane m (0..3) of each 4-lane block.
template <int M> __device__ __forceinline__ float quad_bcast(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), M * 0x55, 0xF, 0xF, false));
}
__device__ __forceinline__ void quad_bcast4(float v, float (&o)[4]) {
    o[0] = quad_bcast<0>(v); o[1] = quad_bcast<1>(v); o[2] = quad_bcast<2>(v); o[3] = quad_bcast<3>(v);
}

// ONE: a single activation row (M == 1): only row 0 of each MFMA result is
// scaled, reduced and stored.
// Grouped mode (grp_off set): workgroup row `by` serves group (expert) by,
// whose weights start at by * w_group_stride and whose activation rows are
// grp_off[by] .. grp_off[by+1]-1 (through x_idx when set); paired matrices
// (n1 > 0) as in gemv_body.
template <int T, int PPT, int MS, bool ONE = false, bool X32 = false, bool XL = false>
__device__ __forceinline__ void gemv_mfma_body(const GemvArgs& a, int bx, int gx, int by, int bz, int gz,
                                               float (&red)[2][4][2][4][4 * MS]) {
    constexpr int NM = ONE ? 1 : 4;  // result rows per row set that are used
    typedef typename Piece<T>::Raw Raw;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 3, blk = lane >> 2;
    const int slot = (wave << 4) | blk;
    const int sl2 = a.lpr_log2, S = 1 << sl2;
    const int grp = slot >> sl2, sg = slot & (S - 1);
    const int G = 64 >> sl2;               // row groups per iteration
    const int wpg = S >> 4;                // wavefronts per row group
    const int P = a.K >> 5;
    const int n_iters = (a.N + 4 * G - 1) / (4 * G);
    const uint8_t* const W = a.W + (int64_t)by * a.w_group_stride;
    const uint8_t* const W2 = a.n1 > 0 ? a.W2 + (int64_t)by * a.w_group_stride : nullptr;
    int m0 = 0, mcount = a.M;
    if (a.grp_off) {
        m0 = a.grp_off[by];
        mcount = a.grp_off[by + 1] - m0;
    }
    int parity = 0;

    for (int mc = bz * 4 * MS; mc < mcount; mc += gz * 4 * MS) {
        Raw ra[PPT], rb[PPT];
        auto fetch = [&](Raw (&r)[PPT], int it) {
            const int row = (it * G + grp) * 4 + j;
            const bool rv = it < n_iters && row < a.N;
            if (a.n1 > 0) {
                const RowRef wrow = weight_row(W, W2, a.n1, a.row_bytes, rv ? row : 0);
#pragma unroll
                for (int i = 0; i < PPT; i++) {
                    const int p = sg + i * S;
                    r[i] = Piece<T>::fetch(wrow, p < P ? p : 0);
                }
            } else {
                const RowRef wrow = weight_row(W, nullptr, 0, a.row_bytes, rv ? row : 0);
#pragma unroll
                for (int i = 0; i < PPT; i++) {
                    const int p = sg + i * S;
                    r[i] = Piece<T>::fetch(wrow, p < P ? p : 0);
                }
            }
        };
        int it = bx;
        if constexpr (!XL) fetch(ra, it);

        // Activations of this lane's row (j + 4t) at its pieces.
        float x[PPT][MS][32];
        float amax[MS];
#pragma unroll
        for (int t = 0; t < MS; t++) amax[t] = 0.0f;
        if constexpr (XL) {
            // The workgroup's 4 MS activation rows are read from memory once
            // (16-byte words, consecutive k across lanes) and staged in LDS
            // as float4 slot (j8, p, m) at j8 (4 MS P + 1) + 4 MS p + m, with
            // j8 = 4 r + quad of run r of piece p: each lane's reads of its
            // (piece, row) are consecutive slots across the wavefront.
            // P <= 32: at most 4 MS slots per thread, all loaded (rows past
            // the batch and slots past the rows reading row 0 / slot 0,
            // without a branch) before the weight fetch, so that the LDS
            // stores wait only for them (loads complete in issue order).
            extern __shared__ float4 xls[];
            constexpr int R4 = 4 * MS;
            const int pstride = R4 * P + 1;
            if (mc != bz * 4 * MS) __syncthreads();  // every wavefront has read the previous rows
            float4 xv[R4];
#pragma unroll
            for (int q = 0; q < R4; q++) {
                const int sl = tid + 256 * q < 8 * R4 * P ? tid + 256 * q : 0, rest = sl >> 3;
                const int mrow = (int)__umulhi((uint32_t)rest, a.p_div);
                const int p = rest - mrow * P;
                const int k = Piece<T>::run_k(p, (sl & 7) >> 2) + 4 * (sl & 3);
                xv[q] = *(const float4*)(a.X + (int64_t)(mc + mrow < mcount ? mc + mrow : 0) * a.ldx + k);
            }
            fetch(ra, it);
#pragma unroll
            for (int q = 0; q < R4; q++) {
                const int sl = tid + 256 * q, rest = sl >> 3;
                const int mrow = (int)__umulhi((uint32_t)rest, a.p_div);
                const int p = rest - mrow * P;
                if (sl < 8 * R4 * P)
                    xls[(sl & 7) * pstride + p * R4 + mrow] = mc + mrow < mcount ? xv[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
            __syncthreads();
#pragma unroll
            for (int i = 0; i < PPT; i++) {
                const int p = sg + i * S;
                const bool ok = p < P;
                const int pc = ok ? p : 0;
#pragma unroll
                for (int t = 0; t < MS; t++)
#pragma unroll
                    for (int j8 = 0; j8 < 8; j8++) {
                        const float4 v = xls[j8 * pstride + pc * R4 + 4 * t + j];
                        x[i][t][4 * j8] = ok ? v.x : 0.0f; x[i][t][4 * j8 + 1] = ok ? v.y : 0.0f;
                        x[i][t][4 * j8 + 2] = ok ? v.z : 0.0f; x[i][t][4 * j8 + 3] = ok ? v.w : 0.0f;
                    }
#pragma unroll
                for (int t = 0; t < MS; t++)
#pragma unroll
                    for (int q = 0; q < 32; q++) amax[t] = fmaxf(amax[t], fabsf(x[i][t][q]));
            }
        } else
#pragma unroll
        for (int i = 0; i < PPT; i++) {
            const int p = sg + i * S;
            const int pc = p < P ? p : 0;
#pragma unroll
            for (int t = 0; t < MS; t++) {
                const int m = mc + 4 * t + j;
                const bool ok = p < P && m < mcount;
                int xrow = m0 + (m < mcount ? m : 0);
                if (a.x_idx) xrow = a.x_idx[xrow];
                const float* xp = a.X + (int64_t)xrow * a.ldx;
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    const int k0 = Piece<T>::run_k(pc, r);
                    if (a.x_vec4) {
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const float4 v = *(const float4*)(xp + k0 + 4 * q);
                            x[i][t][16 * r + 4 * q] = v.x; x[i][t][16 * r + 4 * q + 1] = v.y;
                            x[i][t][16 * r + 4 * q + 2] = v.z; x[i][t][16 * r + 4 * q + 3] = v.w;
                        }
                    } else {
#pragma unroll
                        for (int q = 0; q < 16; q++) x[i][t][16 * r + q] = xp[k0 + q];
                    }
                }
#pragma unroll
                for (int q = 0; q < 32; q++) {
                    x[i][t][q] = ok ? x[i][t][q] : 0.0f;
                    amax[t] = fmaxf(amax[t], fabsf(x[i][t][q]));
                }
            }
        }
        // X32: the fp32 activations go into the fp32 matrix-core product as
        // they are (4x4x1 steps, one value of k per step); only the run sums
        // of the bias term are formed here.
        float xs[PPT][MS][2][4];
        h4v xh[PPT][MS][X32 ? 1 : 8], xl[PPT][MS][X32 ? 1 : 8];
        float out_inv = 1.0f;
        const int out_t = (lane >> 4) & (MS - 1), out_m = (lane >> 2) & 3;
        if constexpr (X32) {
#pragma unroll
            for (int i = 0; i < PPT; i++)
#pragma unroll
                for (int t = 0; t < MS; t++) {
                    float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                    for (int q = 0; q < 16; q++) {
                        s0 += x[i][t][q];
                        s1 += x[i][t][16 + q];
                    }
                    quad_bcast4(s0, xs[i][t][0]);
                    quad_bcast4(s1, xs[i][t][1]);
                }
        } else {
        // Largest magnitude of each activation row over the workgroup's
        // slots (all groups of a workgroup read the same rows): lanes of
        // equal j inside the wavefront, then its two halves and the
        // wavefronts through LDS.  Row m then gets the power of two
        // 2^sh[m] that puts that maximum in [2^14, 2^15).
#pragma unroll
        for (int t = 0; t < MS; t++) {
            float v = amax[t];
            v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xF, 0xF, false)));
            v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false)));
            v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F)));
            if ((lane & 31) < 4) red[parity][wave][lane >> 5][j][4 * t] = v;
        }
        __syncthreads();
        int sh[MS];
        float scl[MS];
#pragma unroll
        for (int t = 0; t < MS; t++) {
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; w++) v = fmaxf(v, fmaxf(red[parity][w][0][j][4 * t], red[parity][w][1][j][4 * t]));
            int e = 15 - __builtin_amdgcn_frexp_expf(v);
            e = v > 0.0f ? (e < 126 ? e : 126) : 0;
            sh[t] = e;
            scl[t] = __builtin_amdgcn_ldexpf(1.0f, e);
        }
        // The output lane of (j, m, t) = (L & 3, (L >> 2) & 3, L >> 4) needs
        // the scale of row 4t + m: lane 4m + j' of any block holds it for
        // j' = m.
#pragma unroll
        for (int t = 0; t < MS; t++) {
            const int e = __builtin_amdgcn_ds_bpermute(4 * ((lane & ~3) | out_m), sh[t]);
            if (t == out_t) out_inv = __builtin_amdgcn_ldexpf(1.0f, -e);
        }
        parity ^= 1;
        // Split into fp16 hi + lo after the row's scale; run sums of the
        // scaled values for the bias term, gathered for all four rows.
#pragma unroll
        for (int i = 0; i < PPT; i++)
#pragma unroll
            for (int t = 0; t < MS; t++) {
                float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                for (int q = 0; q < 16; q++) {
                    s0 += x[i][t][q] * scl[t];
                    s1 += x[i][t][16 + q] * scl[t];
                }
                quad_bcast4(s0, xs[i][t][0]);
                quad_bcast4(s1, xs[i][t][1]);
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    float v[4], l[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = x[i][t][4 * q + e] * scl[t];
                    const auto h01 = __builtin_amdgcn_cvt_pkrtz(v[0], v[1]), h23 = __builtin_amdgcn_cvt_pkrtz(v[2], v[3]);
                    l[0] = v[0] - (float)h01[0]; l[1] = v[1] - (float)h01[1];
                    l[2] = v[2] - (float)h23[0]; l[3] = v[3] - (float)h23[1];
                    const auto l01 = __builtin_amdgcn_cvt_pkrtz(l[0], l[1]), l23 = __builtin_amdgcn_cvt_pkrtz(l[2], l[3]);
                    xh[i][t][q] = __builtin_bit_cast(h4v, make_uint2(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23)));
                    xl[i][t][q] = __builtin_bit_cast(h4v, make_uint2(__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23)));
                }
            }
        }

        while (it < n_iters) {
            if (it + gx < n_iters) fetch(rb, it + gx);
            const int row = (it * G + grp) * 4 + j;
            const RowRef wrow = weight_row(W, W2, a.n1, a.row_bytes, row < a.N ? row : 0);
            float acc[MS][4];
#pragma unroll
            for (int t = 0; t < MS; t++)
#pragma unroll
                for (int m = 0; m < 4; m++) acc[t][m] = 0.0f;
#pragma unroll
            for (int i = 0; i < PPT; i++) {
                const int p = sg + i * S;
                const PieceCodes pc = Piece<T>::decode(ra[i], wrow, p < P ? p : 0);
#pragma unroll
                for (int r = 0; r < 2; r++) {
                    h4v B[4];
                    float Bf[16];
                    if constexpr (X32) {
#pragma unroll
                        for (int q = 0; q < 16; q++) Bf[q] = (float)((u4_at(pc.u[r], q >> 2) >> (8 * (q & 3))) & 0xFFu);
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; q++) B[q] = codes_slice(u4_at(pc.u[r], q));
                    }
#pragma unroll
                    for (int t = 0; t < MS; t++) {
                        f4v D = {0.0f, 0.0f, 0.0f, 0.0f};
                        if constexpr (X32) {
#pragma unroll
                            for (int q = 0; q < 16; q++) D = __builtin_amdgcn_mfma_f32_4x4x1f32(x[i][t][16 * r + q], Bf[q], D, 0, 0, 0);
                        } else {
#pragma unroll
                            for (int q = 0; q < 4; q++) {
                                D = __builtin_amdgcn_mfma_f32_4x4x4f16(xh[i][t][4 * r + q], B[q], D, 0, 0, 0);
                                D = __builtin_amdgcn_mfma_f32_4x4x4f16(xl[i][t][4 * r + q], B[q], D, 0, 0, 0);
                            }
                        }
#pragma unroll
                        for (int m = 0; m < NM; m++) {
                            acc[t][m] = fmaf(pc.a[r], D[m], acc[t][m]);
                            acc[t][m] = fmaf(pc.b[r], xs[i][t][r][m], acc[t][m]);
                        }
                    }
                }
            }
            // Sum over the wavefront's 16 blocks (lanes of equal j): rotate
            // by 4 and 8 inside each row of 16, then xor 16; lanes 0-3 and
            // 32-35 hold the two halves.
#pragma unroll
            for (int t = 0; t < MS; t++)
#pragma unroll
                for (int m = 0; m < NM; m++) {
                    float v = dpp_addc<0x124>(acc[t][m]);
                    v = dpp_addc<0x128>(v);
                    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
                    acc[t][m] = v;
                }
            if ((lane & 31) < 4) {
#pragma unroll
                for (int t = 0; t < MS; t++)
#pragma unroll
                    for (int m = 0; m < NM; m++) red[parity][wave][lane >> 5][j][4 * t + m] = acc[t][m];
            }
            __syncthreads();
            // Lane L of the group's first wavefront finishes output (row j =
            // L & 3, activation row 4t + m with m = (L >> 2) & 3, t = L >> 4).
            if ((wave & (wpg - 1)) == 0 && lane < 16 * MS && (!ONE || lane < 4)) {
                const int orow = (it * G + grp) * 4 + (lane & 3);
                const int mr = mc + 4 * out_t + out_m;
                if (orow < a.N && mr < mcount) {
                    float v = 0.0f;
                    for (int w = 0; w < wpg; w++)
                        v += red[parity][wave + w][0][lane & 3][4 * out_t + out_m] + red[parity][wave + w][1][lane & 3][4 * out_t + out_m];
                    v *= out_inv;
                    const int64_t o = (int64_t)(m0 + mr) * a.ldy;
                    if (a.n1 > 0 && orow >= a.n1) a.Y2[o + (orow - a.n1)] = v;
                    else a.Y[o + orow] = v;
                }
            }
            parity ^= 1;
            it += gx;
#pragma unroll
            for (int i = 0; i < PPT; i++) ra[i] = rb[i];
        }
    }
}

template <int T, int PPT, int MS, bool ONE = false, bool X32 = false, bool XL = false>
__global__ __launch_bounds__(256) void gemv_mfma_kernel(GemvArgs a) {
    __shared__ float red[2][4][2][4][4 * MS];
    gemv_mfma_body<T, PPT, MS, ONE, X32, XL>(a, blockIdx.x, gridDim.x, blockIdx.y, blockIdx.z, gridDim.z, red);
}

template <int PPT, int MS, bool X32 = false, bool XL = false>
__global__ __launch_bounds__(256) void gemv_mfma_multi_kernel(MultiArgs ma) {
    __shared__ float red[2][4][2][4][4 * MS];
    int q = 0;
    while (q + 1 < ma.n && (int)blockIdx.x >= ma.begin[q + 1]) q++;
    const int bx = blockIdx.x - ma.begin[q], gx = ma.begin[q + 1] - ma.begin[q];
    switch (ma.type[q]) {
#define C(TT) case TT: gemv_mfma_body<TT, PPT, MS, false, X32, XL>(ma.p[q], bx, gx, 0, blockIdx.z, gridDim.z, red); break;
    C(T_Q4_K) C(T_Q5_K) C(T_Q6_K) C(T_Q8_0) C(T_IQ4_NL) C(T_IQ4_XS)
#undef C
    default: break;
    }
}

// Straightforward GEMV for shapes the piece kernel does not take (K not a
// multiple of 64, i.e. an odd number of 32-value blocks): one thread per
// (row, batch row), codes16 + group scales.
template <int T>
__global__ __launch_bounds__(256) void gemv_simple_kernel(GemvArgs a) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    const int g = blockIdx.y;
    if (n >= a.N) return;
    int m0 = 0, mcount = a.M;
    if (a.grp_off) {
        m0 = a.grp_off[g];
        mcount = a.grp_off[g + 1] - m0;
    }
    const uint8_t* row = a.W + (int64_t)g * a.w_group_stride + (int64_t)n * a.row_bytes;
    for (int mi = 0; mi < mcount; mi++) {
        int xrow = m0 + mi;
        if (a.x_idx) xrow = a.x_idx[xrow];
        const float* x = a.X + (int64_t)xrow * a.ldx;
        float acc = 0.0f;
        for (int k = 0; k < a.K; k += 16) {
            const uint4 c = codes16<T>(row, k);
            const GroupScale gs = group_scale<T>(row, k);
            const uint32_t w[4] = {c.x, c.y, c.z, c.w};
            float s = 0.0f, sx = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; j++) {
                s = fmaf(x[k + j], (float)(int8_t)(w[j >> 2] >> (8 * (j & 3))), s);
                sx += x[k + j];
            }
            acc += gs.dl * s - gs.ml * sx;
        }
        a.Y[(int64_t)(m0 + mi) * a.ldy + n] = acc;
    }
}

static int ilog2_ceil(int v) {
    int l = 0;
    while ((1 << l) < v) l++;
    return l;
}

static int device_cus() {
    static int v = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    return v;
}

// Resident 256-thread workgroups per CU of a kernel at an LDS size, asked
// of the runtime once per (kernel, LDS size) and thread: the occupancy query
// costs about as much host time as a launch.
static int occupancy_per_cu(const void* kernel, size_t lds) {
    struct Entry { const void* k; size_t lds; int v; };
    thread_local std::vector<Entry> cache;
    for (const Entry& e : cache)
        if (e.k == kernel && e.lds == lds) return e.v;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, lds) != hipSuccess || per_cu <= 0) per_cu = 1;
    cache.push_back({kernel, lds, per_cu});
    return per_cu;
}

// Workgroups of a non-grouped launch: exactly as many as can be resident at
// once (occupancy x CUs), each looping over its share of rows, so no launch
// runs a partial second round.
template <typename K>
static int resident_blocks(K kernel, size_t lds) {
    return occupancy_per_cu((const void*)kernel, lds) * device_cus();
}

static bool fused(const GemvProblem& p) { return p.rms || p.X2 || p.R || p.silu; }

// Single-row launches stage the activation row in LDS once per workgroup
// (K <= 4096, at most 4 slots per thread; 16-byte aligned rows) instead of
// every wavefront reading it from memory.
static bool gemv_xlds(const GemvProblem& p, const GemvArgs& a) {
    return p.M <= 1 && !p.grp_off && !p.x_idx && a.x_vec4 && a.lpr_log2 < 8 && p.K >= 64 && p.K <= 4096 && p.K % 32 == 0;
}

static int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    return e && *e ? atoi(e) : dflt;
}
// Grouped (MoE) launches on the FMA kernels take two token rows per pass
// and size their grid to four resident rounds shared among the groups.
// Plain multi-row launches on the FMA kernels take one row per pass (two or
// four rows per pass hold 2x / 4x the activations in VGPRs and measured
// slower: the extra weight passes of one row per pass are served from
// cache).
constexpr int kMoeRowsPerPass = 2;
constexpr int kMoeRounds = 4;


// Matrix-core GEMV (gemv_mfma_kernel) for M >= 2 plain fp32-activation
// problems: S = 2^sl2 piece slots per group of 4 rows (16, 32 or 64), PPT
// pieces per lane (at most 2: the split activations take 32 VGPRs per piece
// and row set), MS row sets of 4 per pass (2 when PPT is 1 and M > 4).
// GGQ_GEMV_MFMA=0 selects the fp32 FMA kernels instead (read at every
// multi-row launch).
struct MfmaPlan {
    int sl2, ppt, ms, n_iters;
    bool x32, xl;
};
// LDS bytes of the staged activation rows (8 float4 slots per piece and row,
// one pad slot per run quad).
static size_t mfma_xl_bytes(int K, int ms) { return (size_t)8 * (4 * ms * (K / 32) + 1) * 16; }
static bool mfma_plan(const GemvProblem& p, int M, MfmaPlan& m) {
    if (env_int("GGQ_GEMV_MFMA", 1) == 0 || p.q8row) return false;
    if (M < 2 || fused(p) || (p.K % 32) != 0 || p.K <= 0) return false;
    const int P = p.K / 32;
    m.sl2 = P <= 16 ? 4 : (P <= 32 ? 5 : 6);
    const int S = 1 << m.sl2;
    m.ppt = (P + S - 1) / S;
    if (m.ppt > 2) return false;
    // 8 rows per pass (MS 2) halves the passes over each weight row but
    // holds twice the activations: it pays off for expert groups averaging
    // 8 rows or more (prefill-sized MoE batches), not for plain batches.
    const bool eight = p.grp_off && p.groups > 1 && (int64_t)p.M >= 8LL * p.groups;
    m.ms = (M > 4 && m.ppt == 1 && eight) ? 2 : 1;
    // Plain batches of up to 8 rows: fp32 activations straight into 4x4x1
    // fp32 products.  Grouped (expert) launches and larger batches: the fp16
    // hi + lo split into 4x4x4 fp16 products (half the MFMA issues per row
    // set), faster there.
    m.x32 = !p.grp_off && M <= 8;
    // Rows staged in LDS once per workgroup when two or more row groups of
    // the workgroup would read the same activations (K <= 1024).
    m.xl = P >= 2 && P <= 32 && !p.grp_off && !p.x_idx && (uintptr_t)p.X % 16 == 0 && p.ldx % 4 == 0;
    const int rows_per_iter = 4 * (64 / S);
    m.n_iters = (p.N + rows_per_iter - 1) / rows_per_iter;
    return true;
}

struct GemvPlan {
    GemvArgs a;
    int ppt, n_iters, mrows;
    bool simple;
};

// Rows are addressed as a matrix base plus a 32-bit byte offset: each
// matrix (each group's matrix; each of a pair) must stay below 4 GiB.
static bool offsets_fit(const GemvProblem& p) {
    const int64_t rows = p.n1 > 0 ? (p.n1 > p.N - p.n1 ? p.n1 : p.N - p.n1) : p.N;
    return rows * row_bytes(p.type, p.K) <= (int64_t)0xFFFFFFFF;
}

static GemvPlan plan_gemv(const GemvProblem& p) {
    GemvPlan g;
    GemvArgs& a = g.a;
    g.simple = (p.K % 32) != 0;
    const int P = p.K / 32 > 0 ? p.K / 32 : 1;
    const int lpr_log2 = ilog2_ceil(P < 256 ? P : 256);
    const int lpr = 1 << lpr_log2;
    const int rpi = 256 / lpr;
    a.W = (const uint8_t*)p.W;
    a.w_group_stride = p.w_group_stride;
    a.row_bytes = row_bytes(p.type, p.K);
    a.N = p.N; a.K = p.K;
    a.X = p.X; a.ldx = p.ldx;
    a.Y = p.Y; a.ldy = p.ldy;
    a.M = p.M;
    a.grp_off = p.grp_off;
    a.x_idx = p.x_idx;
    a.lpr_log2 = lpr_log2;
    a.x_vec4 = ((uintptr_t)p.X % 16 == 0) && (p.ldx % 4 == 0) && ((uintptr_t)p.X2 % 16 == 0);
    a.p_div = (uint32_t)((0x100000000ull + P - 1) / P);
    a.prefetch = 1;
    a.X2 = p.X2;
    a.silu = p.silu;
    a.rms = p.rms;
    a.eps = p.eps;
    a.norm_w = p.norm_w;
    a.R = p.R;
    a.ldr = p.ldr;
    a.W2 = (const uint8_t*)p.W2;
    a.Y2 = p.Y2;
    a.n1 = p.n1;
    a.q8row = p.q8row;
    g.ppt = (P + lpr - 1) / lpr;
    g.n_iters = (p.N + rpi - 1) / rpi;
    g.mrows = p.grp_off ? p.max_group_rows : p.M;
    return g;
}

template <int T, int PPT, int MS, bool ONE>
static void launch_mfma_one(const GemvArgs& a, const MfmaPlan& mp, int K, int groups, int gz, hipStream_t s) {
    void (*k)(GemvArgs) = mp.x32 ? (mp.xl ? gemv_mfma_kernel<T, PPT, MS, ONE, true, true> : gemv_mfma_kernel<T, PPT, MS, ONE, true, false>)
                                 : (mp.xl ? gemv_mfma_kernel<T, PPT, MS, ONE, false, true> : gemv_mfma_kernel<T, PPT, MS, ONE, false, false>);
    const size_t lds = mp.xl ? mfma_xl_bytes(K, MS) : 0;
    int gx = resident_blocks(k, lds) * (groups > 1 ? kMoeRounds : 1) / (gz * groups);
    gx = gx < 1 ? 1 : (gx > mp.n_iters ? mp.n_iters : gx);
    hipLaunchKernelGGL(k, dim3(gx, groups, gz), dim3(256), lds, s, a);
}

template <int PPT, int MS>
static void launch_mfma_multi(const MultiArgs& mm, const MfmaPlan* mp, int n, int kmax, int gz, hipStream_t s) {
    void (*k)(MultiArgs) = mp[0].x32 ? (mp[0].xl ? gemv_mfma_multi_kernel<PPT, MS, true, true> : gemv_mfma_multi_kernel<PPT, MS, true, false>)
                                     : (mp[0].xl ? gemv_mfma_multi_kernel<PPT, MS, false, true> : gemv_mfma_multi_kernel<PPT, MS, false, false>);
    const size_t lds = mp[0].xl ? mfma_xl_bytes(kmax, MS) : 0;
    hipLaunchKernelGGL(k, dim3(mm.begin[n], 1, gz), dim3(256), lds, s, mm);
}

template <int T>
static hipError_t launch_gemv_t(const GemvProblem& p, hipStream_t s) {
    const GemvPlan g = plan_gemv(p);
    GemvArgs a = g.a;
    const int groups = p.groups > 0 ? p.groups : 1;
    if (p.n1 > 0 && (g.simple || fused(p) || !p.W2 || !p.Y2 || p.n1 >= p.N)) return hipErrorInvalidValue;
    if (!offsets_fit(p)) return hipErrorInvalidValue;
    if (g.simple) {
        if (p.X2 || p.rms || p.R || p.silu) return hipErrorInvalidValue;  // fused options need K % 32 == 0
        gemv_simple_kernel<T><<<dim3((p.N + 255) / 256, groups), 256, 0, s>>>(a);
        return hipGetLastError();
    }
    const int ppt = g.ppt, mrows = g.mrows;
    {
        MfmaPlan mp;
        if ((groups == 1 || p.grp_off) && mfma_plan(p, mrows, mp)) {
            a.lpr_log2 = mp.sl2;
            // Grouped: one workgroup row per group, each looping over its
            // own row sets (as the FMA kernels' grouped launches).
            const int gz = groups > 1 ? 1 : (mrows + 4 * mp.ms - 1) / (4 * mp.ms);
            if (mrows == 1) {
                if (mp.ppt == 2) launch_mfma_one<T, 2, 1, true>(a, mp, p.K, groups, gz, s);
                else launch_mfma_one<T, 1, 1, true>(a, mp, p.K, groups, gz, s);
            } else if (mp.ppt == 2) launch_mfma_one<T, 2, 1, false>(a, mp, p.K, groups, gz, s);
            else if (mp.ms == 2) launch_mfma_one<T, 1, 2, false>(a, mp, p.K, groups, gz, s);
            else launch_mfma_one<T, 1, 1, false>(a, mp, p.K, groups, gz, s);
            return hipGetLastError();
        }
    }
    // Batch rows per pass (MB) and pieces per thread (PPT) keep the
    // activation registers at 32*MB*PPT <= 128 floats.  Plain launches with
    // more rows than MB run their MB-row chunks in parallel (grid z) and
    // share the resident capacity among them; grouped (MoE) launches share
    // it among the groups (experts), each looping over its own chunks, so
    // each wavefront covers many weight rows per activation load.
#define GO(MB_, PPT_, U_)                                                                        \
    do {                                                                                         \
        const int gz = groups > 1 ? 1 : (mrows + MB_ - 1) / MB_;                                 \
        int gx = resident_blocks(gemv_kernel<T, MB_, PPT_, U_>, 0) * (groups > 1 ? kMoeRounds : 1) / (gz * groups); \
        gx = gx < 1 ? 1 : (gx > g.n_iters ? g.n_iters : gx);                                     \
        gemv_kernel<T, MB_, PPT_, U_><<<dim3(gx, groups, gz), 256, 0, s>>>(a);                   \
    } while (0)
    // (Fused launches reading a product input per wavefront read twice the
    // activation bytes per workgroup: half the resident grid, two row
    // iterations each, halves those reads; 11.2 -> 9.7 us on the K = 8192
    // down projection.)
#define GO_F(PPT_)                                                                               \
    do {                                                                                         \
        const int gz = mrows;                                                                    \
        int gx = resident_blocks(gemv_kernel<T, 1, PPT_, 1, true>, 0) / (gz * (p.X2 ? 2 : 1));   \
        gx = gx < 1 ? 1 : (gx > g.n_iters ? g.n_iters : gx);                                     \
        gemv_kernel<T, 1, PPT_, 1, true><<<dim3(gx, 1, gz), 256, 0, s>>>(a);                     \
    } while (0)
#define GO_X(PPT_)                                                                               \
    do {                                                                                         \
        const size_t lds = (size_t)p.K * sizeof(float);                                          \
        void (*k_)(GemvArgs) = p.q8row ? gemv_kernel<T, 1, PPT_, 1, false, true, true> : gemv_kernel<T, 1, PPT_, 1, false, true>; \
        int gx = resident_blocks(k_, lds);                                                       \
        gx = gx < 1 ? 1 : (gx > g.n_iters ? g.n_iters : gx);                                     \
        hipLaunchKernelGGL(k_, dim3(gx, 1, 1), dim3(256), lds, s, a);                            \
    } while (0)
#define GO_FX(PPT_)                                                                              \
    do {                                                                                         \
        const size_t lds = (size_t)p.K * sizeof(float);                                          \
        int gx = resident_blocks(gemv_kernel<T, 1, PPT_, 1, true, true>, lds);                   \
        gx = gx < 1 ? 1 : (gx > g.n_iters ? g.n_iters : gx);                                     \
        gemv_kernel<T, 1, PPT_, 1, true, true><<<dim3(gx, 1, 1), 256, lds, s>>>(a);              \
    } while (0)
    if (p.q8row && !(groups == 1 && !fused(p) && mrows == 1 && ppt <= 4)) return hipErrorInvalidValue;
    if (p.q8row && !gemv_xlds(p, a)) {  // the row quantized in registers (non-staged kernels)
#define GQ(PPT_)                                                                                 \
    do {                                                                                         \
        int gx = resident_blocks(gemv_kernel<T, 1, PPT_, 1, false, false, true>, 0);             \
        gx = gx < 1 ? 1 : (gx > g.n_iters ? g.n_iters : gx);                                     \
        gemv_kernel<T, 1, PPT_, 1, false, false, true><<<dim3(gx, 1, 1), 256, 0, s>>>(a);        \
    } while (0)
        if (ppt == 1) GQ(1);
        else if (ppt == 2) GQ(2);
        else GQ(4);
#undef GQ
        return hipGetLastError();
    }
    if (groups == 1 && fused(p) && gemv_xlds(p, a)) {
        if (ppt == 1) GO_FX(1);
        else if (ppt == 2) GO_FX(2);
        else if (ppt <= 4) GO_FX(4);
        else return hipErrorInvalidValue;
#undef GO_FX
        return hipGetLastError();
    }
    if (groups == 1 && !fused(p) && gemv_xlds(p, a)) {
        if (ppt == 1) GO_X(1);
        else if (ppt == 2) GO_X(2);
        else if (ppt <= 4) GO_X(4);
        else return hipErrorInvalidValue;
#undef GO_X
        return hipGetLastError();
    }
    if (fused(p)) {  // one activation row per pass, the fused options compiled in
        if (groups > 1) return hipErrorInvalidValue;
        if (ppt == 1) GO_F(1);
        else if (ppt == 2) GO_F(2);
        else if (ppt <= 4) GO_F(4);
        else return hipErrorInvalidValue;
    } else if (groups > 1 && ppt == 1 && mrows > 1) {
        GO(kMoeRowsPerPass, 1, 1);
    } else if (ppt == 1) {
        GO(1, 1, 1);
    } else if (ppt == 2) {
        GO(1, 2, 1);
    } else if (ppt <= 4) {
        GO(1, 4, 1);
    } else {
        return hipErrorInvalidValue;
    }
#undef GO
#undef GO_F
    return hipGetLastError();
}

template <int MB, int PPT, int U, bool F = false, bool KQ = false>
static int multi_resident() {
    return resident_blocks(gemv_multi_kernel<MB, PPT, U, F, KQ>, 0);
}

// Independent problems with the same number of activation rows M in one
// launch when they share the pieces-per-thread count; otherwise one launch
// per problem.
hipError_t launch_gemv_multi(const GemvProblem* ps, int n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (n == 1) return launch_gemv(ps[0], s);  // the single-problem kernel sizes its grid for one problem
    for (int i = 0; i < n; i++)
        if (!offsets_fit(ps[i])) return hipErrorInvalidValue;
    {
        if (i8_gemv_eligible(ps, n, 0)) return launch_i8_gemv(ps, n, 0, nullptr, nullptr, s);
    }
    MultiArgs ma;
    int ppt = -1, total_iters = 0;
    const int M = ps[0].M;
    bool fuse = n <= kMaxMulti;
    GemvPlan plans[kMaxMulti];
    for (int i = 0; fuse && i < n; i++) {
        if (ps[i].M != M || ps[i].grp_off || !supported(ps[i].type)) {
            fuse = false;
        } else {
            plans[i] = plan_gemv(ps[i]);
            if (ppt < 0) ppt = plans[i].ppt;
            if (plans[i].simple || plans[i].ppt != ppt || ppt > 2) fuse = false;
            total_iters += plans[i].n_iters;
        }
    }
    if (!fuse || M == 0) {
        for (int i = 0; i < n; i++) {
            const hipError_t e = launch_gemv(ps[i], s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    {
        MfmaPlan mp[kMaxMulti];
        bool all = M >= 2;
        for (int i = 0; all && i < n; i++) all = mfma_plan(ps[i], M, mp[i]) && mp[i].ppt == mp[0].ppt && mp[i].ms == mp[0].ms;
        int kmax = 0;
        for (int i = 0; all && i < n; i++) {
            mp[0].xl = mp[0].xl && mp[i].xl;
            kmax = ps[i].K > kmax ? ps[i].K : kmax;
        }
        if (all) {
            MultiArgs mm;
            const int ms = mp[0].ms, pp = mp[0].ppt;
            const int gz = (M + 4 * ms - 1) / (4 * ms);
            const size_t lds = mp[0].xl ? mfma_xl_bytes(kmax, ms) : 0;
            int tgt = pp == 2 ? resident_blocks(gemv_mfma_multi_kernel<2, 1>, lds)
                              : (ms == 2 ? resident_blocks(gemv_mfma_multi_kernel<1, 2>, lds) : resident_blocks(gemv_mfma_multi_kernel<1, 1>, lds));
            tgt = tgt / gz > 0 ? tgt / gz : 1;
            int tot = 0;
            for (int i = 0; i < n; i++) tot += mp[i].n_iters;
            int b = 0;
            for (int i = 0; i < n; i++) {
                mm.p[i] = plans[i].a;
                mm.p[i].lpr_log2 = mp[i].sl2;
                mm.type[i] = ps[i].type;
                mm.begin[i] = b;
                int nb = (int)((int64_t)tgt * mp[i].n_iters / (tot > 0 ? tot : 1));
                nb = nb < 1 ? 1 : (nb > mp[i].n_iters ? mp[i].n_iters : nb);
                b += nb;
            }
            mm.begin[n] = b;
            mm.n = n;
            if (pp == 2) launch_mfma_multi<2, 1>(mm, mp, n, kmax, gz, s);
            else if (ms == 2) launch_mfma_multi<1, 2>(mm, mp, n, kmax, gz, s);
            else launch_mfma_multi<1, 1>(mm, mp, n, kmax, gz, s);
            return hipGetLastError();
        }
    }
    bool any_fused = false, kq = true, xl = true;
    int kmax = 0;
    for (int i = 0; i < n; i++) {
        any_fused = any_fused || fused(ps[i]);
        kq = kq && (ps[i].type == T_Q4_K || ps[i].type == T_Q6_K);
        xl = xl && gemv_xlds(ps[i], plans[i].a);
        kmax = ps[i].K > kmax ? ps[i].K : kmax;
    }
    const int gz = M;  // one activation row per pass
    kq = kq && ppt == 1;  // the variants compiled with KQ
    xl = xl && M == 1;
    const bool q8 = ps[0].q8row != 0;
    for (int i = 0; i < n; i++)
        if ((ps[i].q8row != 0) != q8 || (q8 && any_fused)) return hipErrorInvalidValue;
    if (q8 && !xl) {  // the non-staged kernels quantize the row per launch
        for (int i = 0; i < n; i++) {
            const hipError_t e = launch_gemv(ps[i], s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const size_t lds = xl ? (size_t)kmax * sizeof(float) : 0;
    int target;
    if (xl && any_fused) {
        target = ppt == 1 ? (kq ? resident_blocks(gemv_multi_kernel<1, 1, 1, true, true, true>, lds)
                                : resident_blocks(gemv_multi_kernel<1, 1, 1, true, false, true>, lds))
                          : resident_blocks(gemv_multi_kernel<1, 2, 1, true, false, true>, lds);
    } else if (xl) {
        target = kq ? resident_blocks(gemv_multi_kernel<1, 1, 1, false, true, true>, lds)
                    : ppt == 1 ? resident_blocks(gemv_multi_kernel<1, 1, 1, false, false, true>, lds)
                               : resident_blocks(gemv_multi_kernel<1, 2, 1, false, false, true>, lds);
    } else if (any_fused) {
        target = ppt == 1 ? (kq ? multi_resident<1, 1, 1, true, true>() : multi_resident<1, 1, 1, true>())
                          : multi_resident<1, 2, 1, true>();
    } else if (kq) {
        target = multi_resident<1, 1, 1, false, true>();
    } else if (ppt == 1) {
        target = multi_resident<1, 1, 1>();
    } else {
        target = multi_resident<1, 2, 1>();
    }
    target = target / gz > 0 ? target / gz : 1;
    int b = 0;
    for (int i = 0; i < n; i++) {
        ma.p[i] = plans[i].a;
        ma.type[i] = ps[i].type;
        ma.begin[i] = b;
        int nb = (int)((int64_t)target * plans[i].n_iters / (total_iters > 0 ? total_iters : 1));
        if (nb < 1) nb = 1;
        if (nb > plans[i].n_iters) nb = plans[i].n_iters;
        b += nb;
    }
    ma.begin[n] = b;
    ma.n = n;
    const dim3 grid(b, 1, gz);
    if (xl && any_fused) {
        if (kq) gemv_multi_kernel<1, 1, 1, true, true, true><<<grid, 256, lds, s>>>(ma);
        else if (ppt == 1) gemv_multi_kernel<1, 1, 1, true, false, true><<<grid, 256, lds, s>>>(ma);
        else gemv_multi_kernel<1, 2, 1, true, false, true><<<grid, 256, lds, s>>>(ma);
    } else if (xl && q8) {
        if (kq) gemv_multi_kernel<1, 1, 1, false, true, true, true><<<grid, 256, lds, s>>>(ma);
        else if (ppt == 1) gemv_multi_kernel<1, 1, 1, false, false, true, true><<<grid, 256, lds, s>>>(ma);
        else gemv_multi_kernel<1, 2, 1, false, false, true, true><<<grid, 256, lds, s>>>(ma);
    } else if (xl) {
        if (kq) gemv_multi_kernel<1, 1, 1, false, true, true><<<grid, 256, lds, s>>>(ma);
        else if (ppt == 1) gemv_multi_kernel<1, 1, 1, false, false, true><<<grid, 256, lds, s>>>(ma);
        else gemv_multi_kernel<1, 2, 1, false, false, true><<<grid, 256, lds, s>>>(ma);
    } else if (any_fused) {
        if (kq) gemv_multi_kernel<1, 1, 1, true, true><<<grid, 256, 0, s>>>(ma);
        else if (ppt == 1) gemv_multi_kernel<1, 1, 1, true><<<grid, 256, 0, s>>>(ma);
        else gemv_multi_kernel<1, 2, 1, true><<<grid, 256, 0, s>>>(ma);
    } else if (kq) {
        gemv_multi_kernel<1, 1, 1, false, true><<<grid, 256, 0, s>>>(ma);
    } else if (ppt == 1) {
        gemv_multi_kernel<1, 1, 1><<<grid, 256, 0, s>>>(ma);
    } else {
        gemv_multi_kernel<1, 2, 1><<<grid, 256, 0, s>>>(ma);
    }
    return hipGetLastError();
}

// Single-row GGQ_ACT_Q8_ROW problems that the fp32 kernels take with the row
// quantized in their LDS staging or, for rows they do not stage (K > 4096,
// unaligned rows), in registers (GemvArgs::q8row): K a multiple of 32, no
// fused options or grouping, and together fewer weight bytes than the int8
// matrix-core GEMV's threshold (its fixed set-up only pays off above it).
bool gemv_q8row_eligible(const GemvProblem* ps, int n) {
    if (n < 1 || n > kMaxMulti) return false;
    int64_t bytes = 0;
    for (int i = 0; i < n; i++) {
        const GemvProblem& p = ps[i];
        if (p.M != 1 || !supported(p.type) || fused(p) || p.grp_off || p.x_idx || p.groups > 1 || p.n1 > 0 || p.W2)
            return false;
        GemvProblem q = p;
        q.q8row = 1;
        const GemvPlan g = plan_gemv(q);
        if (g.simple || g.ppt > 4 || !offsets_fit(p)) return false;
        bytes += (int64_t)p.N * row_bytes(p.type, p.K);
    }
    return bytes < (int64_t)env_int("GGQ_I8_MIN_BYTES", 16 << 20);
}

hipError_t launch_gemv(const GemvProblem& p, hipStream_t s) {
    if (p.N == 0 || p.M == 0) return hipSuccess;
    if (offsets_fit(p) && i8_gemv_eligible(&p, 1, 0)) return launch_i8_gemv(&p, 1, 0, nullptr, nullptr, s);
#define L(TT) return launch_gemv_t<TT>(p, s)
    GGQ_DISPATCH_TYPE(p.type, L)
#undef L
    return hipSuccess;
}

// ================================================================ GEMM (i8)
// 128x128 output tile per 256-thread workgroup; each wavefront owns a 64x64
// quadrant as 2x2 blocks of v_mfma_i32_32x32x32_i8 (A = activation rows,
// B = weight rows, so every lane's output column n is fixed and the
// per-group weight scale is one scalar per lane).  Each MFMA covers one
// 32-value scale group: the int32 result is converted and scaled into fp32
// accumulators; the Q4_K/Q5_K min term uses the activation group sums from
// a second MFMA against a ones operand.  Q6_K (16-value groups) uses
// v_mfma_i32_32x32x16_i8.
//
// MFMA operand layout: lane l supplies row/column (l % 32) and the K-slice
// 16*(l/32) .. +16; output element r of lane l is row 8*(r/4) + 4*(l/32) +
// r%4, column l%32.
struct GemmArgs {
    const uint8_t* W;
    int64_t row_bytes;
    int N, K;
    const int8_t* QA;
    const float* sa;
    float* C;
    int ldc;
    int M;
    int steps_per_split;  // K-steps per blockIdx.z slice (split-K)
    float* Cpart;         // [splits][M][N] partial sums when split, else null
};

constexpr int kGemmMaxProb = 4;
struct GemmProb {
    const uint8_t* W;
    float* C;
    int N;
    int ldc;
    int tile_begin;  // first blockIdx.x of this weight
};
struct GemmMultiArgs {
    GemmProb p[kGemmMaxProb];
    int np;
    int64_t row_bytes;
    int K, M;
    const int8_t* QA;
    const float* sa;
    int splits, steps_per_split;
    float* part;  // [tiles][splits][BM*BN] partial sums when splits > 1
};

template <int T>
__global__ __launch_bounds__(256) void gemm_i8_kernel(GemmArgs a) {
    constexpr bool kMin = T == T_Q4_K || T == T_Q5_K;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, lk = lane >> 5;
    const int m_base = blockIdx.y * 128 + (wave >> 1) * 64;
    const int n_base = blockIdx.x * 128 + (wave & 1) * 64;

    const int8_t* arow[2];
    bool aval[2];
    const uint8_t* brow[2];
    bool bval[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int m = m_base + 32 * i + li;
        aval[i] = m < a.M;
        arow[i] = a.QA + (int64_t)(aval[i] ? m : 0) * a.K;
        const int n = n_base + 32 * i + li;
        bval[i] = n < a.N;
        brow[i] = a.W + (int64_t)(bval[i] ? n : 0) * a.row_bytes;
    }

    float acc[2][2][16];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const v16i zero = {};
    for (int k0 = 0; k0 < a.K; k0 += 32) {
        if constexpr (T != T_Q6_K) {
            v4i A[2], B[2];
            GroupScale gs[2];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const uint4 av = aval[i] ? *(const uint4*)(arow[i] + k0 + 16 * lk) : make_uint4(0, 0, 0, 0);
                A[i] = v4i{(int)av.x, (int)av.y, (int)av.z, (int)av.w};
                const uint4 bv = bval[i] ? codes16<T>(brow[i], k0 + 16 * lk) : make_uint4(0, 0, 0, 0);
                B[i] = v4i{(int)bv.x, (int)bv.y, (int)bv.z, (int)bv.w};
                gs[i] = bval[i] ? group_scale<T>(brow[i], k0) : GroupScale{0.0f, 0.0f};
            }
            v16i S[2];
            if constexpr (kMin) {
                const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
#pragma unroll
                for (int i = 0; i < 2; i++) S[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[i], ones, zero, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const v16i Pm = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[i], B[j], zero, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        acc[i][j][r] = fmaf(gs[j].dl, (float)Pm[r], acc[i][j][r]);
                        if constexpr (kMin) acc[i][j][r] = fmaf(-gs[j].ml, (float)S[i][r], acc[i][j][r]);
                    }
                }
        } else {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int kk = k0 + 16 * h;
                long A[2], B[2];
                GroupScale gs[2];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    A[i] = aval[i] ? *(const long*)(arow[i] + kk + 8 * lk) : 0;
                    const uint4 c = bval[i] ? codes16<T>(brow[i], kk) : make_uint4(0, 0, 0, 0);
                    const uint32_t lo = lk ? c.z : c.x, hi = lk ? c.w : c.y;
                    B[i] = (long)(((uint64_t)hi << 32) | lo);
                    gs[i] = bval[i] ? group_scale<T>(brow[i], kk) : GroupScale{0.0f, 0.0f};
                }
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++) {
                        const v16i Pm = __builtin_amdgcn_mfma_i32_32x32x16_i8(A[i], B[j], zero, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[i][j][r] = fmaf(gs[j].dl, (float)Pm[r], acc[i][j][r]);
                    }
            }
        }
    }

#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = m_base + 32 * i + 8 * (r >> 2) + 4 * lk + (r & 3);
            if (m >= a.M) continue;
            const float s = a.sa[m];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int n = n_base + 32 * j + li;
                if (n < a.N) a.C[(int64_t)m * a.ldc + n] = acc[i][j][r] * s;
            }
        }
}

// ------------------------------------------------------ LDS-tiled GEMM (i8)
// Workgroup tile BM x BN x BK(=128, four 32-value scale groups), 4
// wavefronts in a 2x2 layout, each computing (BM/2) x (BN/2) with
// v_mfma_i32_32x32x32_i8.  Per K-step the workgroup stages
//   As[m][k]   int8 activations (16-byte rows padded by 16 B: conflict-free)
//   Bs[n][k]   int8 weight codes decoded once from the raw blocks
//   Bd[n][g]   fp32 group scales dl (and Bm[n][g] mins ml for Q4_K/Q5_K)
// in LDS, double-buffered: the global loads of step k+1 are issued before
// the MFMAs of step k and written to the other buffer after them.  Each
// MFMA covers one scale group; its int32 result is converted and scaled
// into fp32 accumulators (acc += dl * P, and -= ml * S with S the
// activation group sums from an MFMA against a ones operand).
constexpr int kGemmBK = 128;
constexpr int kGemmPad = 16;
constexpr int kGemmLd = kGemmBK + kGemmPad;

// Weight staging: fetch() issues the global loads of one (row, 32-group)
// slot, store() decodes it into LDS codes + scales.  The generic version
// loads at store time through codes16 / group_scale; Q8_0 prefetches the
// raw block window.
template <int T> struct BStage {
    const uint8_t* row;
    int k;
    bool ok;
    __device__ __forceinline__ void fetch(const uint8_t* r, int kk, bool v) { row = r; k = kk; ok = v; }
    __device__ __forceinline__ void store(int8_t* codes, float* dl, float* ml) const {
        uint4 c0 = make_uint4(0, 0, 0, 0), c1 = c0;
        GroupScale gs{0.0f, 0.0f};
        if (ok) {
            c0 = codes16<T>(row, k);
            c1 = codes16<T>(row, k + 16);
            gs = group_scale<T>(row, k);
        }
        *(uint4*)codes = c0;
        *(uint4*)(codes + 16) = c1;
        *dl = gs.dl;
        *ml = gs.ml;
    }
};

template <> struct BStage<T_Q8_0> {
    uint32_t w[9];
    const uint8_t* b;
    bool ok;
    __device__ __forceinline__ void fetch(const uint8_t* r, int kk, bool v) {
        b = r + (kk >> 5) * 34;
        ok = v;
        ld_dw<9>(align_down4(b), w);
    }
    // A slot outside the matrix (row >= N, or k >= K) reads block 0 of a
    // valid row; its scale is stored as 0 and its codes are left as read:
    // they only meet zero activation codes (k >= K) or feed output columns
    // that are never written (row >= N).
    __device__ __forceinline__ void store(int8_t* codes, float* dl, float* ml) const {
        const uint32_t sel = half_sel(b);
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = half_pick(w[i + 1], w[i], sel);
        *(uint4*)codes = make_uint4(q[0], q[1], q[2], q[3]);
        *(uint4*)(codes + 16) = make_uint4(q[4], q[5], q[6], q[7]);
        *dl = ok ? half_d(w[0], b) : 0.0f;
        *ml = 0.0f;
    }
};

// One launch serves up to kGemmMaxProb weights of one type that share the
// activation rows (q/k/v, or gate/up): blockIdx.x runs over the N-tiles of
// all of them, blockIdx.y over M-tiles, blockIdx.z over K-slices.
//
// With split-K every slice writes its partial tile to workspace in
// accumulator register order (element e of thread t at e*256 + t, so writes
// and reads are coalesced) and gemm_reduce_kernel adds the slices in slice
// order, which keeps results independent of scheduling.  (A last-arriving-
// workgroup reduction inside this kernel needs an agent-scope release fence
// per workgroup, which writes back the XCD's L2 and measured several times
// slower than the extra launch.)
template <int T, int BM, int BN, int PF>
__global__ __launch_bounds__(256) void gemm_i8_lds_kernel(GemmMultiArgs a) {
    constexpr bool kMin = T == T_Q4_K || T == T_Q5_K;
    constexpr int WM = BM / 2, WN = BN / 2;       // wavefront tile
    constexpr int TM = WM / 32, TN = WN / 32;     // MFMA tiles per wavefront
    constexpr int G = kGemmBK / 32;               // scale groups per K-step
    constexpr int A_CHUNKS = BM * kGemmBK / 16;   // 16-byte chunks of the A tile
    constexpr int A_PER_T = A_CHUNKS / 256;
    constexpr int B_SLOTS = BN * G;               // (row, group) slots of the B tile
    constexpr int B_PER_T = (B_SLOTS + 255) / 256;
    static_assert(A_CHUNKS % 256 == 0, "A tile must split evenly");

    __shared__ __attribute__((aligned(16))) int8_t As[2][BM][kGemmLd];
    __shared__ __attribute__((aligned(16))) int8_t Bs[2][BN][kGemmLd];
    __shared__ __attribute__((aligned(16))) float Bd[2][BN][G];
    __shared__ __attribute__((aligned(16))) float Bm[2][BN][G];
    static_assert(G % 4 == 0, "group scales are read four at a time");

    int q = 0;
    while (q + 1 < a.np && (int)blockIdx.x >= a.p[q + 1].tile_begin) q++;
    const uint8_t* const W = a.p[q].W;
    const int N = a.p[q].N;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, lk = lane >> 5;
    const int m_tile = blockIdx.y * BM, n_tile = ((int)blockIdx.x - a.p[q].tile_begin) * BN;
    const int wm = (wave >> 1) * WM, wn = (wave & 1) * WN;
    const int nsteps = (a.K + kGemmBK - 1) / kGemmBK;

    // PF register stages: the global loads of K-step st+PF are in flight
    // while step st computes.
    uint4 areg[PF][A_PER_T];
    BStage<T> breg[PF][B_PER_T];
    // Per-thread source rows, computed once; each K-step advances k.
    const int8_t* aptr[A_PER_T];
    bool arow_ok[A_PER_T];
    int akc[A_PER_T];
#pragma unroll
    for (int i = 0; i < A_PER_T; i++) {
        const int c = tid + 256 * i, r = c / (kGemmBK / 16);
        akc[i] = (c % (kGemmBK / 16)) * 16;
        const int m = m_tile + r;
        arow_ok[i] = m < a.M;
        aptr[i] = a.QA + (int64_t)(arow_ok[i] ? m : 0) * a.K + akc[i];
    }
    const uint8_t* bptr[B_PER_T];
    bool brow_ok[B_PER_T];
    int bkg[B_PER_T];
#pragma unroll
    for (int i = 0; i < B_PER_T; i++) {
        const int sl = tid + 256 * i;
        const int r = sl / G, n = n_tile + r;
        bkg[i] = 32 * (sl % G);
        brow_ok[i] = sl < B_SLOTS && n < N;
        bptr[i] = W + (int64_t)(brow_ok[i] ? n : 0) * a.row_bytes;
    }

    auto fetch = [&](int step, uint4 (&ar)[A_PER_T], BStage<T> (&br)[B_PER_T]) {
        const int k0 = step * kGemmBK;
#pragma unroll
        for (int i = 0; i < A_PER_T; i++) {
            const bool ok = arow_ok[i] && k0 + akc[i] < a.K;
            ar[i] = ok ? *(const uint4*)(aptr[i] + k0) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < B_PER_T; i++) {
            const int k = k0 + bkg[i];
            const bool ok = brow_ok[i] && k < a.K;
            br[i].fetch(bptr[i], ok ? k : 0, ok);
        }
    };
    auto store = [&](int buf, const uint4 (&ar)[A_PER_T], const BStage<T> (&br)[B_PER_T]) {
#pragma unroll
        for (int i = 0; i < A_PER_T; i++) {
            const int c = tid + 256 * i, r = c / (kGemmBK / 16), kc = (c % (kGemmBK / 16)) * 16;
            *(uint4*)&As[buf][r][kc] = ar[i];
        }
#pragma unroll
        for (int i = 0; i < B_PER_T; i++) {
            const int sl = tid + 256 * i;
            if (sl < B_SLOTS) {
                const int r = sl / G, g = sl % G;
                br[i].store(&Bs[buf][r][32 * g], &Bd[buf][r][g], &Bm[buf][r][g]);
            }
        }
    };

    float acc[TM][TN][16];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const v16i zero = {};
    // Split-K: slice z covers K-steps [st0, st1).
    const int st0 = blockIdx.z * a.steps_per_split;
    const int st1 = st0 + a.steps_per_split < nsteps ? st0 + a.steps_per_split : nsteps;
    // Step st lives in register stage (st - st0) % PF until it is stored to
    // LDS buffer (st - st0) & 1 at the end of step st - 1.
    fetch(st0, areg[0], breg[0]);
    store(0, areg[0], breg[0]);
#pragma unroll
    for (int j = 1; j <= PF; j++)
        if (st0 + j < st1) fetch(st0 + j, areg[j % PF], breg[j % PF]);
    __syncthreads();
    for (int sb = st0; sb < st1; sb += PF) {
#pragma unroll
        for (int d = 0; d < PF; d++) {
            const int st = sb + d;
            if (st >= st1) break;
            const int buf = (st - st0) & 1;
            // Formats without a min term: the epilogue of group g-1 follows
            // the MFMA of group g, pinned by scheduling barriers, so it
            // overlaps that MFMA and stays ahead of the stage stores and the
            // barrier (left to itself the scheduler issues all four MFMAs
            // and sinks every epilogue below the barrier, where the
            // workgroup's wavefronts run them together while the MFMA pipe
            // idles).  Two products are live at a time.
            constexpr bool kGLag = !kMin && TM * TN == 1;
            v16i Pq[2];
            float dq[2];
            // The group-lag path reads its row's G scales up front, 16 bytes
            // at a time: one per-group 4-byte read at a 16-byte lane stride
            // costs an extra LDS instruction and bank conflicts per group.
            float dg[G];
            if constexpr (kGLag) {
#pragma unroll
                for (int g4 = 0; g4 < G; g4 += 4) {
                    const float4 v = *(const float4*)&Bd[buf][wn + li][g4];
                    dg[g4] = v.x, dg[g4 + 1] = v.y, dg[g4 + 2] = v.z, dg[g4 + 3] = v.w;
                }
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                v4i A[TM], B[TN];
                float dl[TN], ml[TN];
#pragma unroll
                for (int i = 0; i < TM; i++) {
                    const uint4 v = *(const uint4*)&As[buf][wm + 32 * i + li][32 * g + 16 * lk];
                    A[i] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
                }
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const uint4 v = *(const uint4*)&Bs[buf][wn + 32 * j + li][32 * g + 16 * lk];
                    B[j] = v4i{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
                    if constexpr (!kGLag) {
                        dl[j] = Bd[buf][wn + 32 * j + li][g];
                        ml[j] = Bm[buf][wn + 32 * j + li][g];
                    }
                }
                if constexpr (kGLag) {
                    Pq[g & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[0], B[0], zero, 0, 0, 0);
                    dq[g & 1] = dg[g];
                    if (g > 0) {
#pragma unroll
                        for (int r = 0; r < 16; r++)
                            acc[0][0][r] = fmaf(dq[(g - 1) & 1], (float)Pq[(g - 1) & 1][r], acc[0][0][r]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    if (g == G - 1) {
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[0][0][r] = fmaf(dq[g & 1], (float)Pq[g & 1][r], acc[0][0][r]);
                        // An opaque use of the accumulators: IR-level sinking
                        // cannot move the epilogue below this point.
#pragma unroll
                        for (int r = 0; r < 16; r++) asm volatile("" : "+v"(acc[0][0][r]));
                    }
                    continue;
                }
                v16i S[TM];
                if constexpr (kMin) {
                    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
#pragma unroll
                    for (int i = 0; i < TM; i++) S[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[i], ones, zero, 0, 0, 0);
                }
#pragma unroll
                for (int i = 0; i < TM; i++)
#pragma unroll
                    for (int j = 0; j < TN; j++) {
                        const v16i Pm = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[i], B[j], zero, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            acc[i][j][r] = fmaf(dl[j], (float)Pm[r], acc[i][j][r]);
                            if constexpr (kMin) acc[i][j][r] = fmaf(-ml[j], (float)S[i][r], acc[i][j][r]);
                        }
                    }
            }
            if (st + 1 < st1) {
                const int nx = (d + 1) % PF;  // a constant once the d loop is unrolled
                store(buf ^ 1, areg[nx], breg[nx]);
                if (st + 1 + PF < st1) fetch(st + 1 + PF, areg[nx], breg[nx]);
                __syncthreads();
            }
        }
    }

    if (a.splits > 1) {
        // Partial tile in accumulator register order; gemm_reduce_kernel
        // adds the slices in slice order.
        const int tile = blockIdx.y * gridDim.x + blockIdx.x;
        float* mine = a.part + ((int64_t)tile * a.splits + blockIdx.z) * (BM * BN);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) mine[((i * TN + j) * 16 + r) * 256 + tid] = acc[i][j][r];
        return;
    }
    float* const C = a.p[q].C;
    const int ldc = a.p[q].ldc;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = m_tile + wm + 32 * i + 8 * (r >> 2) + 4 * lk + (r & 3);
            if (m >= a.M) continue;
            const float s = a.sa[m];
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int n = n_tile + wn + 32 * j + li;
                if (n < N) C[(int64_t)m * ldc + n] = acc[i][j][r] * s;
            }
        }
}

// ------------------------------------- activation-panel GEMM (prefill, i8)
// One 768-thread workgroup per (64-row activation panel, N-range): the
// panel's int8 rows for the whole K stay in LDS (64 x (K + 16) bytes, K <=
// 2048), quantized per row inside the kernel from the fp32 rows
// (amd_xdna.cpp:598-603, 633-639: scale = amax / 127, q = rint(a * (1 /
// scale)) -- the quantizer of quant_row_regs, bit for bit) or copied from
// given codes.  Each wavefront then takes (32 weight rows x 32 activation
// rows) items of its N-range and runs the whole K for one: the weight
// codes go from memory straight into the B operand of
// v_mfma_i32_32x32x32_i8 (a lane's 16 codes and its group scale, fetched
// kPanelPD groups ahead), the activation codes come from the panel, and the
// exact per-group epilogue acc += dl * P (- ml * S) runs in registers.  No
// LDS staging of the weights, no barrier after the panel is loaded, no
// split of K and hence no reduction launch, and no separate quantization
// launch.  Workgroup id = panel * ranges + range with ranges a multiple of
// 8, so the panels sharing an N-range run on one XCD (its L2 serves the
// weights to all of them).
constexpr int kPanelRows = 64;
constexpr int kPanelMaxK = 2048;
constexpr int kPanelThreads = 768;   // 12 wavefronts: 3 per SIMD, up to 168 VGPRs
constexpr int kPanelWaves = kPanelThreads / 64;
constexpr int kPanelPD = 4;        // weight groups in flight per lane
constexpr int kPanelRegK = 1536;   // rows up to this K are quantized from registers

struct PanelArgs {
    GemmProb p[kGemmMaxProb];  // tile_begin: first 32-row N-block of each weight
    int np;
    int64_t row_bytes;
    int K, M;
    const float* A;   // fp32 rows [M][lda] (quantized in the kernel), or null
    int lda;
    const int8_t* QA; // given codes [M][K] and scales sa when A is null
    const float* sa;
    int nblocks;      // 32-row N-blocks over all weights
    int ranges;       // N-ranges per panel
};

// Weight operand of one lane for one 32-value group: the 16 codes of half
// lk of the group of row `row` and the group's scales.  Generic formats
// load at decode time; Q8_0 fetches its dword window early.
template <int T> struct PStage {
    const uint8_t* row;
    int k;
    __device__ __forceinline__ void fetch(const uint8_t* r, int g, int h) { row = r; k = 32 * g + 16 * h; }
    __device__ __forceinline__ uint4 codes(GroupScale& gs) const {
        gs = group_scale<T>(row, k & ~31);
        return codes16<T>(row, k);
    }
};
template <> struct PStage<T_Q8_0> {
    uint4 c;
    uint32_t d;
    // the 16 codes of half h start 2 + 16 h bytes into the 34-byte block:
    // one 16-byte load at a 2-byte-aligned address (exact on gfx950) and
    // the fp16 scale
    __device__ __forceinline__ void fetch(const uint8_t* r, int g, int h) {
        const uint8_t* b = r + 34 * g;
        c = *(const uint4*)(b + 2 + 16 * h);
        d = ld_u16(b);
    }
    __device__ __forceinline__ uint4 codes(GroupScale& gs) const {
        gs = {h2f(d), 0.0f};
        return c;
    }
};

template <int T>
__global__ __launch_bounds__(kPanelThreads) void gemm_panel_kernel(PanelArgs a) {
    constexpr bool kMin = T == T_Q4_K || T == T_Q5_K;
    extern __shared__ __attribute__((aligned(16))) int8_t panel[];
    __shared__ float sa_s[kPanelRows];
    const int K = a.K, ld = K + 16;
    // the wavefront index as a scalar: items, and the weight each item reads
    // (a kernel-argument array indexed per item), stay uniform
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 31, lk = lane >> 5;
    const int mp = (int)blockIdx.x / a.ranges, rg = (int)blockIdx.x % a.ranges;
    const int m0 = mp * kPanelRows;

    // ---- the panel: 32 threads per row, rows tid / 32 + 24 j
    constexpr int RPP = kPanelThreads / 32;                 // rows per pass
    constexpr int NP = (kPanelRows + RPP - 1) / RPP;        // passes
    const int c = tid & 31;
    if (a.A && K <= kPanelRegK) {
        // every load of the thread's rows issued before the first is used,
        // unconditional (positions past K and rows past M read valid
        // memory and are zeroed after): a branch around a load makes the
        // compiler wait for the loads in flight
        constexpr int NV = kPanelRegK / 128;
        float4 v[NP][NV];
#pragma unroll
        for (int j = 0; j < NP; j++) {
            const int r = tid / 32 + RPP * j, m = m0 + (r < kPanelRows ? r : 0);
            const float* arow = a.A + (int64_t)(m < a.M ? m : 0) * a.lda;
#pragma unroll
            for (int i = 0; i < NV; i++) {
                const int k = 4 * c + 128 * i;
                v[j][i] = *(const float4*)(arow + (k < K ? k : 0));
            }
        }
#pragma unroll
        for (int j = 0; j < NP; j++) {
            const int r = tid / 32 + RPP * j;
            if (r >= kPanelRows) break;
            const bool ok = m0 + r < a.M;
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < NV; i++) {
                if (!ok || 4 * c + 128 * i >= K) v[j][i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v[j][i].x), fabsf(v[j][i].y))),
                             fmaxf(fabsf(v[j][i].z), fabsf(v[j][i].w)));
            }
#pragma unroll
            for (int off = 1; off < 32; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
            const float sc = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 1.0f;
            const float inv = __fdiv_rn(1.0f, sc);
            if (c == 0) sa_s[r] = sc;
            int8_t* prow = panel + r * ld;
#pragma unroll
            for (int i = 0; i < NV; i++) {
                const int k = 4 * c + 128 * i;
                if (k < K)
                    *(uint32_t*)(prow + k) = (uint32_t)(uint8_t)to_i8(__fmul_rn(v[j][i].x, inv)) |
                                             (uint32_t)(uint8_t)to_i8(__fmul_rn(v[j][i].y, inv)) << 8 |
                                             (uint32_t)(uint8_t)to_i8(__fmul_rn(v[j][i].z, inv)) << 16 |
                                             (uint32_t)(uint8_t)to_i8(__fmul_rn(v[j][i].w, inv)) << 24;
            }
        }
    }
    for (int r = tid >> 5; r < kPanelRows && !(a.A && K <= kPanelRegK); r += RPP) {
        const int m = m0 + r;
        const bool ok = m < a.M;
        int8_t* prow = panel + r * ld;
        if (a.A) {  // longer rows: the maximum, then the codes, both streamed
            const float* arow = a.A + (int64_t)(ok ? m : 0) * a.lda;
            float amax = 0.0f;
            for (int k = 4 * c; k < K; k += 128) {
                const float4 v = ok ? *(const float4*)(arow + k) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v.x), fabsf(v.y))), fmaxf(fabsf(v.z), fabsf(v.w)));
            }
#pragma unroll
            for (int off = 1; off < 32; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
            const float sc = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 1.0f;
            const float inv = __fdiv_rn(1.0f, sc);
            if (c == 0) sa_s[r] = sc;
            for (int k = 4 * c; k < K; k += 128) {
                const float4 v = ok ? *(const float4*)(arow + k) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                *(uint32_t*)(prow + k) = (uint32_t)(uint8_t)to_i8(__fmul_rn(v.x, inv)) |
                                         (uint32_t)(uint8_t)to_i8(__fmul_rn(v.y, inv)) << 8 |
                                         (uint32_t)(uint8_t)to_i8(__fmul_rn(v.z, inv)) << 16 |
                                         (uint32_t)(uint8_t)to_i8(__fmul_rn(v.w, inv)) << 24;
            }
        } else {
            const int8_t* qrow = a.QA + (int64_t)(ok ? m : 0) * K;
            constexpr int NQ = kPanelMaxK / 512;
            uint4 v[NQ];
#pragma unroll
            for (int i = 0; i < NQ; i++) {
                const int k = 16 * c + 512 * i;
                v[i] = *(const uint4*)(qrow + (k < K ? k : 0));
            }
#pragma unroll
            for (int i = 0; i < NQ; i++) {
                const int k = 16 * c + 512 * i;
                if (k < K) *(uint4*)(prow + k) = ok ? v[i] : make_uint4(0, 0, 0, 0);
            }
            if (c == 0) sa_s[r] = ok ? a.sa[m] : 1.0f;
        }
    }
    __syncthreads();

    // ---- items: 32-row N-blocks, strided over the waves; each item covers
    // the panel's 64 rows (two MFMAs per group share the weight operand)
    const int nb_here = a.nblocks > rg ? (a.nblocks - rg + a.ranges - 1) / a.ranges : 0;
    const bool two = a.M - m0 > 32;  // uniform: the panel's second half holds rows
    const int G = K / 32;
    const v16i zero = {};
    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
    // Fewer items than wavefronts (the small levels): each item's K is split
    // over ks wavefronts in whole 4-group chunks, and the slices' sums are
    // added in slice order through LDS (the panel's space, once every
    // wavefront is done with it) by the slice-0 wavefront.
    const int nch_all = (G + 3) / 4;
    int ks = nb_here > 0 ? kPanelWaves / nb_here : 1;
    if (ks > nch_all) ks = nch_all;
    if (ks < 1) ks = 1;
    const int n_work = nb_here * ks;
    float acc0[16], acc1[16];
    int n = 0, N = 0, q = 0;
    for (int w = wave; w < n_work; w += kPanelWaves) {
        const int it = w / ks, sl = w % ks;
        const int c_lo = nch_all * sl / ks, c_hi = nch_all * (sl + 1) / ks;
        const int nbk = rg + a.ranges * it;
        q = 0;
        while (q + 1 < a.np && nbk >= a.p[q + 1].tile_begin) q++;
        N = a.p[q].N;
        n = (nbk - a.p[q].tile_begin) * 32 + li;
        const uint8_t* wrow = a.p[q].W + (int64_t)(n < N ? n : 0) * a.row_bytes;
        const int8_t* arow0 = panel + li * ld + 16 * lk;
        const int8_t* arow1 = arow0 + 32 * ld;

#pragma unroll
        for (int r = 0; r < 16; r++) acc0[r] = acc1[r] = 0.0f;
        // one group's MFMAs (both panel halves) and exact epilogue
        auto group = [&](int g, const uint4& bv, const GroupScale& gs) {
            const v4i Bv = v4i{(int)bv.x, (int)bv.y, (int)bv.z, (int)bv.w};
#pragma unroll
            for (int h = 0; h < 2; h++) {
                if (h == 1 && !two) break;
                const uint4 av = *(const uint4*)((h ? arow1 : arow0) + 32 * g);
                const v4i Av = v4i{(int)av.x, (int)av.y, (int)av.z, (int)av.w};
                float* acc = h ? acc1 : acc0;
                const v16i P = __builtin_amdgcn_mfma_i32_32x32x32_i8(Av, Bv, zero, 0, 0, 0);
                if constexpr (kMin) {
                    const v16i S = __builtin_amdgcn_mfma_i32_32x32x32_i8(Av, ones, zero, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        acc[r] = fmaf(gs.dl, (float)P[r], acc[r]);
                        acc[r] = fmaf(-gs.ml, (float)S[r], acc[r]);
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[r] = fmaf(gs.dl, (float)P[r], acc[r]);
                }
            }
        };
        if constexpr (T == T_Q8_0) {
            // Chunks of four blocks (136 bytes of the row): lane (li, lk)
            // loads bytes 68 lk .. 68 lk + 67 of row li's chunk (blocks 2 lk
            // and 2 lk + 1, whole), so each cache line of the row is read
            // once; one v_permlane32_swap per dword then gives every lane
            // half lk of all four blocks (the lower lanes' half-0 codes and
            // the upper lanes' half-1 codes of the same blocks trade places).
            constexpr int CH = 2;  // chunks in flight
            const uint8_t* seg = wrow + 68 * lk;
            uint32_t R[CH][17];
            auto load = [&](int ch, uint32_t (&wv)[17]) {
                const uint32_t* p = (const uint32_t*)(seg + 136 * ch);
#pragma unroll
                for (int i = 0; i < 4; i++) *(uint4*)&wv[4 * i] = *(const uint4*)(p + 4 * i);
                wv[16] = p[16];
            };
#pragma unroll
            for (int j = 0; j < CH; j++) load(c_lo + j < c_hi ? c_lo + j : c_lo, R[j]);
            for (int c0 = c_lo; c0 < c_hi; c0 += CH) {
#pragma unroll
                for (int j = 0; j < CH; j++) {
                    const int ch = c0 + j;
                    if (ch >= c_hi) break;
                    uint32_t a0[4], a1[4], b0[4], b1[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        // block A (bytes 0..33, codes from byte 2), block B (34..67, codes from 36)
                        const auto sa = __builtin_amdgcn_permlane32_swap(__builtin_amdgcn_alignbyte(R[j][i + 1], R[j][i], 2),
                                                                         __builtin_amdgcn_alignbyte(R[j][i + 5], R[j][i + 4], 2),
                                                                         false, false);
                        const auto sb = __builtin_amdgcn_permlane32_swap(R[j][9 + i], R[j][13 + i], false, false);
                        a0[i] = sa[0], a1[i] = sa[1], b0[i] = sb[0], b1[i] = sb[1];
                    }
                    // the two fp16 scales of the lane's blocks in one dword
                    const uint32_t sc = (R[j][0] & 0xFFFFu) | (R[j][8] & 0xFFFF0000u);
                    const auto ss = __builtin_amdgcn_permlane32_swap(sc, sc, false, false);
                    if (ch + CH < c_hi) load(ch + CH, R[j]);
                    const int g = 4 * ch;
                    group(g, make_uint4(a0[0], a0[1], a0[2], a0[3]), GroupScale{h2f(ss[0] & 0xFFFFu), 0.0f});
                    if (g + 1 < G) group(g + 1, make_uint4(b0[0], b0[1], b0[2], b0[3]), GroupScale{h2f(ss[0] >> 16), 0.0f});
                    if (g + 2 < G) group(g + 2, make_uint4(a1[0], a1[1], a1[2], a1[3]), GroupScale{h2f(ss[1] & 0xFFFFu), 0.0f});
                    if (g + 3 < G) group(g + 3, make_uint4(b1[0], b1[1], b1[2], b1[3]), GroupScale{h2f(ss[1] >> 16), 0.0f});
                }
            }
        } else {
            const int g_lo = 4 * c_lo, g_hi = 4 * c_hi < G ? 4 * c_hi : G;
            PStage<T> st[kPanelPD];
#pragma unroll
            for (int j = 0; j < kPanelPD; j++) st[j].fetch(wrow, g_lo + j < g_hi ? g_lo + j : g_lo, lk);
            for (int g0 = g_lo; g0 < g_hi; g0 += kPanelPD) {
#pragma unroll
                for (int j = 0; j < kPanelPD; j++) {
                    const int g = g0 + j;
                    if (g >= g_hi) break;
                    GroupScale gs;
                    const uint4 bv = st[j].codes(gs);
                    if (g + kPanelPD < g_hi) st[j].fetch(wrow, g + kPanelPD, lk);
                    group(g, bv, gs);
                }
            }
        }
        if (ks == 1 && n < N) {
            float* const C = a.p[q].C;
            const int ldc = a.p[q].ldc;
#pragma unroll
            for (int h = 0; h < 2; h++) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int mr = 32 * h + 8 * (r >> 2) + 4 * lk + (r & 3);
                    const int m = m0 + mr;
                    if (m < a.M) C[(int64_t)m * ldc + n] = (h ? acc1[r] : acc0[r]) * sa_s[mr];
                }
            }
        }
    }
    if (ks > 1) {  // uniform over the workgroup (n_work <= kPanelWaves)
        float* red = (float*)panel;  // [wave][32 values][64 lanes]
        __syncthreads();
        if (wave < n_work) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                red[(wave * 32 + r) * 64 + lane] = acc0[r];
                red[(wave * 32 + 16 + r) * 64 + lane] = acc1[r];
            }
        }
        __syncthreads();
        if (wave < n_work && wave % ks == 0) {
            for (int sl = 1; sl < ks; sl++) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    acc0[r] += red[((wave + sl) * 32 + r) * 64 + lane];
                    acc1[r] += red[((wave + sl) * 32 + 16 + r) * 64 + lane];
                }
            }
            if (n < N) {
                float* const C = a.p[q].C;
                const int ldc = a.p[q].ldc;
#pragma unroll
                for (int h = 0; h < 2; h++) {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int mr = 32 * h + 8 * (r >> 2) + 4 * lk + (r & 3);
                        const int m = m0 + mr;
                        if (m < a.M) C[(int64_t)m * ldc + n] = (h ? acc1[r] : acc0[r]) * sa_s[mr];
                    }
                }
            }
        }
    }
}

bool gemm_panel_eligible(uint32_t type, int K, int M, const float* A, int lda) {
    if (type == T_Q6_K || K <= 0 || K > kPanelMaxK || K % 32 || M <= 0) return false;
    if (A && (((uintptr_t)A & 15u) || lda % 4)) return false;
    return true;
}

hipError_t launch_gemm_panel(uint32_t type, const GemmDesc* d, int n, int K, const float* A, int lda,
                             const int8_t* qa, const float* sa, int M, hipStream_t s) {
    if (M == 0 || n == 0) return hipSuccess;
    if (n > kGemmMaxProb || !gemm_panel_eligible(type, K, M, A, lda) || (!A && (!qa || !sa)))
        return hipErrorInvalidValue;
    PanelArgs a;
    int nb = 0;
    for (int i = 0; i < n; i++) {
        a.p[i].W = (const uint8_t*)d[i].W;
        a.p[i].C = d[i].C;
        a.p[i].N = d[i].N;
        a.p[i].ldc = d[i].ldc;
        a.p[i].tile_begin = nb;
        nb += (d[i].N + 31) / 32;
    }
    a.np = n;
    a.row_bytes = row_bytes(type, K);
    a.K = K;
    a.M = M;
    a.A = A;
    a.lda = lda;
    a.QA = qa;
    a.sa = sa;
    a.nblocks = nb;
    const int panels = (M + kPanelRows - 1) / kPanelRows;
    // ranges: a multiple of 8, at most one per N-block (rounded up), and
    // panels x ranges about one workgroup per CU
    int ranges = (device_cus() / panels) & ~7;
    if (ranges < 8) ranges = 8;
    const int nb8 = (nb + 7) & ~7;
    if (ranges > nb8) ranges = nb8;
    a.ranges = ranges;
    // the panel, and room for the K-split partial sums (8 KB per wavefront)
    const size_t lds = std::max((size_t)kPanelRows * (K + 16), (size_t)kPanelWaves * 8192);
    const void* k = nullptr;
    switch (type) {
    case T_Q8_0: k = (const void*)gemm_panel_kernel<T_Q8_0>; break;
    case T_Q4_K: k = (const void*)gemm_panel_kernel<T_Q4_K>; break;
    case T_Q5_K: k = (const void*)gemm_panel_kernel<T_Q5_K>; break;
    case T_IQ4_NL: k = (const void*)gemm_panel_kernel<T_IQ4_NL>; break;
    case T_IQ4_XS: k = (const void*)gemm_panel_kernel<T_IQ4_XS>; break;
    default: return hipErrorInvalidValue;
    }
    static std::mutex mu;
    static std::set<const void*> attr_done;
    {
        std::lock_guard<std::mutex> lock(mu);
        if (!attr_done.count(k)) {
            const hipError_t e =
                hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kPanelRows * (kPanelMaxK + 16));
            if (e != hipSuccess) return e;
            attr_done.insert(k);
        }
    }
    void* args[] = {&a};
    return hipLaunchKernel(k, dim3(panels * ranges), dim3(kPanelThreads), args, lds, s);
}

// ------------------------------------------ expert-grouped int8 GEMM (MoE)
// Prefill-sized MoE batches (tens of tokens per expert) with per-row int8
// activations: one launch multiplies every expert's weight matrix by the
// token rows routed to it.  A tile is (expert e, 32 consecutive pair rows
// of e's group, 128 weight rows); the tile list over all experts (and the
// shared expert as group E) is built on the device (moe_tiles_kernel) from
// the group offsets, so the grid is sized by an upper bound and the
// workgroups past the list end exit.  Per K-step (128 values) the
// workgroup gathers its 32 activation rows (token rows through x_idx) and
// decodes 128 weight rows' codes into LDS once; four wavefronts each take
// 32 weight rows with v_mfma_i32_32x32x32_i8 per 32-value scale group
// (Q6_K's 16-value groups: two MFMAs, each with the other half of the lane
// groups' activation codes zeroed), and the exact per-group epilogue
// acc += dl * P (- ml * S for the K-quant mins, S from an MFMA against
// ones).  Weight rows [0, n1) come from W and go to C, rows [n1, N) from W2
// to C2 (an expert's gate and up in one pass); the shared expert's
// matrices replace W / W2 for group E.
struct MoeGemmArgs {
    const uint8_t* W;
    const uint8_t* W2;
    const uint8_t* Wsh;
    const uint8_t* W2sh;
    int64_t w_stride;  // bytes per expert matrix
    int64_t row_bytes;
    int N, K, n1, E;
    const int8_t* QA;        // activation codes, rows of K
    const float* sa;         // activation row scales
    const int32_t* x_idx;    // pair row -> activation row (null: the pair row itself)
    const int32_t* grp;      // [E + 2] first pair row of each group (E: shared expert)
    const int2* tiles;       // (group, first pair row)
    const int32_t* n_tiles;  // tile count
    float* C;
    float* C2;
    int ldc;
    const float* QS;  // int8 mode, K-quant mins: code sums per 32 values [rows][K/32]
    // fp32-row mode (moe_gemm_f16_kernel): hi / lo planes [rows][K], group
    // sums [rows][K/32] and row scales 2^-e [rows] of the activation rows
    const _Float16* XH;
    const _Float16* XL;
    const float* XS;
    const float* xs;
};
constexpr int kMoeBM = kMoeTileRows, kMoeBN = 128;

// Weight staging of the grouped GEMM: fetch() issues plain loads of one
// (row, 32-value group) slot's raw bytes into registers, store() decodes
// them into LDS codes and scales one K-step later, so the loads of step
// k+1 are in flight during step k.  Q4_K: the block header and the 32 qs
// bytes holding the group's nibbles (16-byte aligned loads).  Q6_K
// (2-byte-aligned 210-byte blocks): aligned dword windows over the group's
// ql and qh bytes, realigned when stored, plus its two 16-value scales and
// d.  Other formats stage through BStage.
template <int T> struct MStage : BStage<T> {
    __device__ __forceinline__ void store2(int8_t* codes, float* dl, float* ml) const { this->store(codes, dl, ml); }
};
template <> struct MStage<T_Q4_K> {
    uint4 hd, q0, q1;
    int j;
    bool ok;
    __device__ __forceinline__ void fetch(const uint8_t* row, int k, bool v) {
        const uint8_t* b = row + (k >> 8) * 144;
        j = (k & 255) >> 5;
        ok = v;
        hd = ld16_a(b);
        q0 = ld16_a(b + 16 + 32 * (j >> 1));
        q1 = ld16_a(b + 32 + 32 * (j >> 1));
    }
    __device__ __forceinline__ void store2(int8_t* codes, float* dl, float* ml) const {
        const uint32_t sh = 4 * (j & 1);
        *(uint4*)codes = and4(shr4(q0, sh), 0x0F0F0F0Fu);
        *(uint4*)(codes + 16) = and4(shr4(q1, sh), 0x0F0F0F0Fu);
        uint32_t sc, m;
        kq_scale_min(hd.y, hd.z, hd.w, j, sc, m);
        *dl = ok ? __fmul_rn(h2f(hd.x & 0xFFFFu), (float)sc) : 0.0f;
        *ml = ok ? __fmul_rn(h2f(hd.x >> 16), (float)m) : 0.0f;
    }
};
template <> struct MStage<T_Q6_K> {
    uint32_t ql[9], qh[9], sc, d;
    uint32_t sel;
    int qd;
    bool ok;
    __device__ __forceinline__ void fetch(const uint8_t* row, int k, bool v) {
        const uint8_t* b = row + (k >> 8) * 210;
        const int kk = k & 255, h = kk >> 7;
        qd = (kk & 127) >> 5;
        ok = v;
        // the ql and qh runs start at b + (multiple of 4): dword i of a run
        // is w[i] (b 4-aligned) or bytes 2..5 of (w[i], w[i+1])
        sel = ((uint32_t)(uintptr_t)b & 2u) ? 0x05040302u : 0x03020100u;
        ld_dw<9>(align_down4(b + 64 * h + 32 * (qd & 1)), ql);
        ld_dw<9>(align_down4(b + 128 + 32 * h), qh);
        sc = ld_u16(b + 192 + (kk >> 4));
        d = ld_u16(b + 208);
    }
    // writes the scales of both 16-value groups: dl[0], dl[1]
    __device__ __forceinline__ void store2(int8_t* codes, float* dl, float*) const {
        uint32_t c[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t l = half_pick(ql[i + 1], ql[i], sel), hh = half_pick(qh[i + 1], qh[i], sel);
            c[i] = six_to_s8(((l >> (4 * (qd >> 1))) & 0x0F0F0F0Fu) | (((hh >> (2 * qd)) & 0x03030303u) << 4));
        }
        *(uint4*)codes = make_uint4(c[0], c[1], c[2], c[3]);
        *(uint4*)(codes + 16) = make_uint4(c[4], c[5], c[6], c[7]);
        const float df = h2f(d);
        dl[0] = ok ? __fmul_rn(df, (float)(int8_t)(sc & 0xFFu)) : 0.0f;
        dl[1] = ok ? __fmul_rn(df, (float)(int8_t)(sc >> 8)) : 0.0f;
    }
};

template <int T>
__global__ __launch_bounds__(256) void moe_gemm_kernel(MoeGemmArgs a) {
    constexpr bool kMin = T == T_Q4_K || T == T_Q5_K;
    constexpr bool kQ6 = T == T_Q6_K;
    constexpr int G = kGemmBK / 32;                // 32-value groups per K-step
    constexpr int GS = kQ6 ? 2 * G : G;            // scales per row and step
    __shared__ __attribute__((aligned(16))) int8_t As[2][kMoeBM][kGemmLd];
    __shared__ __attribute__((aligned(16))) int8_t Bs[2][kMoeBN][kGemmLd];
    __shared__ __attribute__((aligned(16))) float Bd[2][kMoeBN][GS];
    __shared__ __attribute__((aligned(16))) float Bm[2][kMoeBN][G];
    __shared__ __attribute__((aligned(16))) float Ss[2][G][kMoeBM];  // activation code sums (K-quant mins)

    const int tile = blockIdx.y;
    if (tile >= *a.n_tiles) return;
    const int2 te = a.tiles[tile];
    const int e = te.x, p0 = te.y, p_end = a.grp[e + 1];
    const uint8_t* const W1 = e == a.E ? a.Wsh : a.W + (int64_t)e * a.w_stride;
    const uint8_t* const W2 = e == a.E ? a.W2sh : (a.W2 ? a.W2 + (int64_t)e * a.w_stride : nullptr);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, lk = lane >> 5;
    const int n_tile = blockIdx.x * kMoeBN;
    const int nsteps = (a.K + kGemmBK - 1) / kGemmBK;
    const int KG = a.K / 32;
    // Group sums: threads 0..127 stage (group, row) entries, 4 groups x 32 rows.
    const int sr = tid & 31, sg = (tid >> 5) & 3;
    const int ps = p0 + sr;
    const int srow = a.x_idx ? a.x_idx[ps < p_end ? ps : p0] : (ps < p_end ? ps : p0);
    const float* const qsp = kMin ? a.QS + (int64_t)srow * KG + sg : nullptr;

    // Activations: 32 rows x 128 bytes per step, one 16-byte chunk per thread.
    const int ar = tid >> 3, akc = (tid & 7) * 16;
    const int pa = p0 + ar;
    const bool arow_ok = pa < p_end;
    const int arow = a.x_idx ? a.x_idx[arow_ok ? pa : p0] : (arow_ok ? pa : p0);
    const int8_t* const aptr = a.QA + (int64_t)arow * a.K + akc;
    // Weights: 128 rows x 4 groups per step, two (row, group) slots per thread.
    const uint8_t* bptr[2];
    bool brow_ok[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int sl = tid + 256 * i, n = n_tile + sl / G;
        brow_ok[i] = n < a.N;
        const int nn = brow_ok[i] ? n : 0;
        bptr[i] = nn < a.n1 ? W1 + (int64_t)nn * a.row_bytes : W2 + (int64_t)(nn - a.n1) * a.row_bytes;
    }

    uint4 areg;
    float sreg = 0.0f;
    MStage<T> breg[2];
    auto fetch = [&](int st) {
        const int k0 = st * kGemmBK;
        areg = arow_ok && k0 + akc < a.K ? *(const uint4*)(aptr + k0) : make_uint4(0, 0, 0, 0);
        if constexpr (kMin) sreg = tid < 128 && ps < p_end && k0 / 32 + sg < KG ? qsp[k0 / 32] : 0.0f;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int k = k0 + 32 * ((tid + 256 * i) % G);
            const bool ok = brow_ok[i] && k < a.K;
            breg[i].fetch(bptr[i], ok ? k : 0, ok);
        }
    };
    auto store = [&](int buf) {
        *(uint4*)&As[buf][ar][akc] = areg;
        if constexpr (kMin)
            if (tid < 128) Ss[buf][sg][sr] = sreg;
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int sl = tid + 256 * i, r = sl / G, g = sl % G;
            if constexpr (kQ6) breg[i].store2(&Bs[buf][r][32 * g], &Bd[buf][r][2 * g], nullptr);
            else breg[i].store2(&Bs[buf][r][32 * g], &Bd[buf][r][g], &Bm[buf][r][g]);
        }
    };

    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    const v16i zero = {};
    const int wn = 32 * wave;

    fetch(0);
    store(0);
    if (nsteps > 1) fetch(1);
    __syncthreads();
    for (int st = 0; st < nsteps; st++) {
        const int buf = st & 1;
#pragma unroll
        for (int g = 0; g < G; g++) {
            const uint4 av = *(const uint4*)&As[buf][li][32 * g + 16 * lk];
            const uint4 bv = *(const uint4*)&Bs[buf][wn + li][32 * g + 16 * lk];
            const v4i A = v4i{(int)av.x, (int)av.y, (int)av.z, (int)av.w};
            const v4i B = v4i{(int)bv.x, (int)bv.y, (int)bv.z, (int)bv.w};
            if constexpr (kQ6) {
                // lane group lk holds values 16 lk.. of the 32: group 2g + lk
                const v4i A0 = lk == 0 ? A : v4i{0, 0, 0, 0};
                const v4i A1 = lk == 1 ? A : v4i{0, 0, 0, 0};
                const v16i P0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A0, B, zero, 0, 0, 0);
                const v16i P1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A1, B, zero, 0, 0, 0);
                const float d0 = Bd[buf][wn + li][2 * g], d1 = Bd[buf][wn + li][2 * g + 1];
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    acc[r] = fmaf(d0, (float)P0[r], acc[r]);
                    acc[r] = fmaf(d1, (float)P1[r], acc[r]);
                }
            } else {
                const v16i P = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, zero, 0, 0, 0);
                const float dl = Bd[buf][wn + li][g];
                if constexpr (kMin) {
                    // the activation rows' code sums of this group, staged
                    // from the quantizer's output (no MFMA against ones)
                    const float ml = Bm[buf][wn + li][g];
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float4 sv = *(const float4*)&Ss[buf][g][8 * j + 4 * lk];
                        const float sj[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int r = 4 * j + i;
                            acc[r] = fmaf(dl, (float)P[r], acc[r]);
                            acc[r] = fmaf(-ml, sj[i], acc[r]);
                        }
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 16; r++) acc[r] = fmaf(dl, (float)P[r], acc[r]);
                }
            }
        }
        if (st + 1 < nsteps) {
            store(buf ^ 1);
            if (st + 2 < nsteps) fetch(st + 2);
            __syncthreads();
        }
    }

    // Lane (li, lk) holds weight row n = n_tile + wn + li and pair rows
    // p0 + 8 (r >> 2) + 4 lk + (r & 3).
    const int n = n_tile + wn + li;
    if (n >= a.N) return;
    float* const Cb = n < a.n1 ? a.C + n : a.C2 + (n - a.n1);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int p = p0 + 8 * (r >> 2) + 4 * lk + (r & 3);
        if (p < p_end) Cb[(int64_t)p * a.ldc] = acc[r] * a.sa[a.x_idx ? a.x_idx[p] : p];
    }
}

// ------------------------------- expert-grouped fp16 GEMM (MoE, fp32 rows)
// The prefill-sized MoE layer with fp32 activations.  Each activation row
// is written once (split_rows_kernel) as two fp16 planes under a power of
// two per row, x * 2^e = hi + lo with the row's largest magnitude in
// [2^14, 2^15): |x 2^e - hi - lo| <= 2^-8, i.e. 2^-23 of the row maximum.
// The weights' integer codes are exact in fp16 (|code| <= 128), so each
// product code * (hi + lo) is exact in the fp32 accumulator of
// v_mfma_f32_32x32x16_f16; per 32-value scale group four MFMAs (hi and lo
// of the two 16-value halves) chain into one fp32 sum P, and the epilogue
// is the exact-code one of the int8 GEMM: acc += dl * P (- ml * S, S the
// group sum of hi + lo from the split).  Q6_K's 16-value groups take one
// hi / lo pair each.  The result is scaled by 2^-e of its row at the
// store.  Tiles, staging of the weights and the gate / up pairing are those
// of moe_gemm_kernel; K-steps of 64 values keep the LDS at 45 KB.
constexpr int kF16BK = 64;                 // values per K-step
constexpr int kF16ALd = kF16BK + 8;        // fp16 per A row in LDS (144 B: conflict-free)
constexpr int kF16BLd = kF16BK + 16;       // code bytes per B row in LDS (80 B)

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Eight int8 codes (two dwords) as eight fp16 values: biased to unsigned,
// placed as the low mantissa byte of 1024.0, then 1024 + 128 subtracted.
__device__ __forceinline__ uint32_t s8x2_f16(uint32_t w, uint32_t sel) {
    const h2v v = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, w, sel));
    const h2v off = {(_Float16)1152.0f, (_Float16)1152.0f};
    return __builtin_bit_cast(uint32_t, v - off);
}
__device__ __forceinline__ v8h s8x8_f16(uint2 c) {
    const uint32_t a = c.x ^ 0x80808080u, b = c.y ^ 0x80808080u;
    return __builtin_bit_cast(v8h, make_uint4(s8x2_f16(a, 0x04010400u), s8x2_f16(a, 0x04030402u),
                                              s8x2_f16(b, 0x04010400u), s8x2_f16(b, 0x04030402u)));
}

template <int T, int PF>
__global__ __launch_bounds__(256) void moe_gemm_f16_kernel(MoeGemmArgs a) {
    constexpr bool kMin = T == T_Q4_K || T == T_Q5_K;
    constexpr bool kQ6 = T == T_Q6_K;
    constexpr int G = kF16BK / 32;       // 32-value groups per K-step
    constexpr int GS = kQ6 ? 2 * G : G;  // scales per row and step
    __shared__ __attribute__((aligned(16))) _Float16 Ah[2][kMoeBM][kF16ALd];
    __shared__ __attribute__((aligned(16))) _Float16 Al[2][kMoeBM][kF16ALd];
    __shared__ __attribute__((aligned(16))) int8_t Bs[2][kMoeBN][kF16BLd];
    __shared__ __attribute__((aligned(16))) float Bd[2][kMoeBN][GS];
    __shared__ __attribute__((aligned(16))) float Bm[2][kMoeBN][G];
    __shared__ __attribute__((aligned(16))) float As[2][G][kMoeBM];

    const int tile = blockIdx.y;
    if (tile >= *a.n_tiles) return;
    const int2 te = a.tiles[tile];
    const int e = te.x, p0 = te.y, p_end = a.grp[e + 1];
    const uint8_t* const W1 = e == a.E ? a.Wsh : a.W + (int64_t)e * a.w_stride;
    const uint8_t* const W2 = e == a.E ? a.W2sh : (a.W2 ? a.W2 + (int64_t)e * a.w_stride : nullptr);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, lk = lane >> 5;
    const int n_tile = blockIdx.x * kMoeBN;
    const int nsteps = a.K / kF16BK;  // K is a multiple of 256 or of 64 (checked by the caller)
    const int KG = a.K / 32;

    // Activations: thread t stages 8 values of row t / 8 from both planes.
    const int ar = tid >> 3, akc = (tid & 7) * 8;
    const int pa = p0 + ar;
    const bool arow_ok = pa < p_end;
    const int arow = a.x_idx ? a.x_idx[arow_ok ? pa : p0] : (arow_ok ? pa : p0);
    const _Float16* const hptr = a.XH + (int64_t)arow * a.K + akc;
    const _Float16* const lptr = a.XL + (int64_t)arow * a.K + akc;
    // Group sums (K-quant mins): threads 0..63 stage (group, row) entries.
    const int sr = tid & 31, sg = (tid >> 5) & 1;
    const int ps = p0 + sr;
    const int srow = a.x_idx ? a.x_idx[ps < p_end ? ps : p0] : (ps < p_end ? ps : p0);
    const float* const sptr = a.XS + (int64_t)srow * KG + sg;
    // Weights: 128 rows x 2 groups per step, one (row, group) slot per thread.
    const int br = tid / G, bg = tid % G;
    const int bn = n_tile + br;
    const bool brow_ok = bn < a.N;
    const int bnn = brow_ok ? bn : 0;
    const uint8_t* const bptr = bnn < a.n1 ? W1 + (int64_t)bnn * a.row_bytes : W2 + (int64_t)(bnn - a.n1) * a.row_bytes;

    // PF register stages: the global loads of K-step st + PF are in flight
    // while step st computes.
    uint4 ahr[PF], alr[PF];
    float asr[PF];
    MStage<T> breg[PF];
    auto fetch = [&](int st, int j) {
        const int k0 = st * kF16BK;
        ahr[j] = arow_ok ? *(const uint4*)(hptr + k0) : make_uint4(0, 0, 0, 0);
        alr[j] = arow_ok ? *(const uint4*)(lptr + k0) : make_uint4(0, 0, 0, 0);
        if constexpr (kMin) asr[j] = tid < 64 && ps < p_end ? sptr[k0 / 32] : 0.0f;
        breg[j].fetch(bptr, brow_ok ? k0 + 32 * bg : 0, brow_ok);
    };
    auto store = [&](int buf, int j) {
        *(uint4*)&Ah[buf][ar][akc] = ahr[j];
        *(uint4*)&Al[buf][ar][akc] = alr[j];
        if constexpr (kMin)
            if (tid < 64) As[buf][sg][sr] = asr[j];
        if constexpr (kQ6) breg[j].store2(&Bs[buf][br][32 * bg], &Bd[buf][br][2 * bg], nullptr);
        else breg[j].store2(&Bs[buf][br][32 * bg], &Bd[buf][br][bg], &Bm[buf][br][bg]);
    };

    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    const v16f zero = {};
    const int wn = 32 * wave;

    // Step st lives in register stage st % PF until it is stored to LDS
    // buffer st & 1 at the end of step st - 1.
    fetch(0, 0);
    store(0, 0);
#pragma unroll
    for (int j = 1; j <= PF; j++)
        if (j < nsteps) fetch(j, j % PF);
    __syncthreads();
    for (int sb = 0; sb < nsteps; sb += PF) {
#pragma unroll
        for (int d = 0; d < PF; d++) {
            const int st = sb + d;
            if (st >= nsteps) break;
            const int buf = st & 1;
#pragma unroll
            for (int g = 0; g < G; g++) {
                v8h H[2], L[2], B[2];
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    const int k = 32 * g + 16 * hh + 8 * lk;
                    H[hh] = *(const v8h*)&Ah[buf][li][k];
                    L[hh] = *(const v8h*)&Al[buf][li][k];
                    B[hh] = s8x8_f16(*(const uint2*)&Bs[buf][wn + li][k]);
                }
                if constexpr (kQ6) {
                    v16f P0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(H[0], B[0], zero, 0, 0, 0);
                    P0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(L[0], B[0], P0, 0, 0, 0);
                    v16f P1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(H[1], B[1], zero, 0, 0, 0);
                    P1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(L[1], B[1], P1, 0, 0, 0);
                    const float d0 = Bd[buf][wn + li][2 * g], d1 = Bd[buf][wn + li][2 * g + 1];
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        acc[r] = fmaf(d0, P0[r], acc[r]);
                        acc[r] = fmaf(d1, P1[r], acc[r]);
                    }
                } else {
                    v16f P = __builtin_amdgcn_mfma_f32_32x32x16_f16(H[0], B[0], zero, 0, 0, 0);
                    P = __builtin_amdgcn_mfma_f32_32x32x16_f16(L[0], B[0], P, 0, 0, 0);
                    P = __builtin_amdgcn_mfma_f32_32x32x16_f16(H[1], B[1], P, 0, 0, 0);
                    P = __builtin_amdgcn_mfma_f32_32x32x16_f16(L[1], B[1], P, 0, 0, 0);
                    const float dl = Bd[buf][wn + li][g];
                    if constexpr (kMin) {
                        const float ml = Bm[buf][wn + li][g];
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const float4 sv = *(const float4*)&As[buf][g][8 * j + 4 * lk];
                            const float sj[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
                            for (int i = 0; i < 4; i++) {
                                const int r = 4 * j + i;
                                acc[r] = fmaf(dl, P[r], acc[r]);
                                acc[r] = fmaf(-ml, sj[i], acc[r]);
                            }
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 16; r++) acc[r] = fmaf(dl, P[r], acc[r]);
                    }
                }
            }
            if (st + 1 < nsteps) {
                const int nx = (d + 1) % PF;  // a constant once the d loop is unrolled
                store(buf ^ 1, nx);
                if (st + 1 + PF < nsteps) fetch(st + 1 + PF, nx);
                __syncthreads();
            }
        }
    }

    // Lane (li, lk) holds weight row n = n_tile + wn + li and pair rows
    // p0 + 8 (r >> 2) + 4 lk + (r & 3).
    const int n = n_tile + wn + li;
    if (n >= a.N) return;
    float* const Cb = n < a.n1 ? a.C + n : a.C2 + (n - a.n1);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        const int p = p0 + 8 * (r >> 2) + 4 * lk + (r & 3);
        if (p < p_end) Cb[(int64_t)p * a.ldc] = acc[r] * a.xs[a.x_idx ? a.x_idx[p] : p];
    }
}

// Rows of fp32 activations as the fp16 hi + lo planes of the grouped fp16
// GEMM: per row the power of two 2^e that puts its largest magnitude in
// [2^14, 2^15) (e clamped to 126: all-subnormal rows keep fewer bits), hi =
// fp16(x 2^e), lo = fp16(x 2^e - hi), the group sums of hi + lo per 32
// values, and 2^-e.  P = PROD_SWIGLU forms each row as silu(g) * u first
// (the SwiGLU of quant_row_regs, same expression); prod_out receives the
// produced rows when set.  One workgroup per row, K <= 16384, K a multiple
// of 32, rows 16-byte aligned.
template <int P>
__global__ __launch_bounds__(256) void split_rows_kernel(const float* __restrict__ A, const float* __restrict__ aux,
                                                         int lda, int K, _Float16* __restrict__ XH,
                                                         _Float16* __restrict__ XL, float* __restrict__ XS,
                                                         float* __restrict__ xs, float* __restrict__ prod_out) {
    __shared__ float wmax[4];
    constexpr int R = 16;
    const int m = blockIdx.x;
    const float* a = A + (int64_t)m * lda;
    float4 v[R];
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int k = 4 * threadIdx.x + 1024 * i;
        v[i] = k < K ? *(const float4*)(a + k) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    if constexpr (P == PROD_SWIGLU) {
        const float* u = aux + (int64_t)m * lda;
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int k = 4 * threadIdx.x + 1024 * i;
            if (k >= K) break;
            const float4 w = *(const float4*)(u + k);
            v[i].x = (v[i].x / (1.0f + expf(-v[i].x))) * w.x;
            v[i].y = (v[i].y / (1.0f + expf(-v[i].y))) * w.y;
            v[i].z = (v[i].z / (1.0f + expf(-v[i].z))) * w.z;
            v[i].w = (v[i].w / (1.0f + expf(-v[i].w))) * w.w;
        }
    }
    if (prod_out) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int k = 4 * threadIdx.x + 1024 * i;
            if (k >= K) break;
            *(float4*)(prod_out + (int64_t)m * K + k) = v[i];
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < R; i++)
        amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v[i].x), fabsf(v[i].y))), fmaxf(fabsf(v[i].z), fabsf(v[i].w)));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int ex = 0;
    if (amax > 0.0f) {
        int x2;
        (void)frexpf(amax, &x2);  // amax in [2^(x2-1), 2^x2)
        ex = 15 - x2;
        if (ex > 126) ex = 126;
    }
    if (threadIdx.x == 0) xs[m] = ldexpf(1.0f, -ex);
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int k = 4 * threadIdx.x + 1024 * i;
        if (k >= K) break;
        const float y[4] = {ldexpf(v[i].x, ex), ldexpf(v[i].y, ex), ldexpf(v[i].z, ex), ldexpf(v[i].w, ex)};
        _Float16 h[4], l[4];
        float gs = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            h[j] = (_Float16)y[j];
            l[j] = (_Float16)(y[j] - (float)h[j]);
            gs += (float)h[j] + (float)l[j];
        }
        *(uint2*)(XH + (int64_t)m * K + k) = __builtin_bit_cast(uint2, h4v{h[0], h[1], h[2], h[3]});
        *(uint2*)(XL + (int64_t)m * K + k) = __builtin_bit_cast(uint2, h4v{l[0], l[1], l[2], l[3]});
        // eight consecutive threads hold one 32-value group
        gs += __shfl_xor(gs, 1, 64);
        gs += __shfl_xor(gs, 2, 64);
        gs += __shfl_xor(gs, 4, 64);
        if ((threadIdx.x & 7) == 0) XS[(int64_t)m * (K / 32) + k / 32] = gs;
    }
}

// The same for rows of up to 2048 values: one wavefront per row, four rows
// per workgroup, lane l holding the 8-value chunks l, l + 64, ...; the
// per-value arithmetic and the order of the group sums are those of
// split_rows_kernel (each 4-value sum, then pairs of them, then across 4
// lanes), so the planes and sums are identical.
template <int P>
__global__ __launch_bounds__(256) void split_rows_wave_kernel(const float* __restrict__ A,
                                                              const float* __restrict__ aux, int lda, int M, int K,
                                                              _Float16* __restrict__ XH, _Float16* __restrict__ XL,
                                                              float* __restrict__ XS, float* __restrict__ xs,
                                                              float* __restrict__ prod_out) {
    const int lane = threadIdx.x & 63;
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= M) return;
    constexpr int R = 4;
    const float* a = A + (int64_t)m * lda;
    float4 v[R][2];
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int k = 8 * (lane + 64 * i);
        if (k < K) {
            v[i][0] = *(const float4*)(a + k);
            v[i][1] = *(const float4*)(a + k + 4);
        } else {
            v[i][0] = v[i][1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    if constexpr (P == PROD_SWIGLU) {
        const float* u = aux + (int64_t)m * lda;
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int k = 8 * (lane + 64 * i);
            if (k >= K) continue;
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const float4 w = *(const float4*)(u + k + 4 * hh);
                float4& x = v[i][hh];
                x.x = (x.x / (1.0f + expf(-x.x))) * w.x;
                x.y = (x.y / (1.0f + expf(-x.y))) * w.y;
                x.z = (x.z / (1.0f + expf(-x.z))) * w.z;
                x.w = (x.w / (1.0f + expf(-x.w))) * w.w;
            }
        }
    }
    if (prod_out) {
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int k = 8 * (lane + 64 * i);
            if (k >= K) continue;
            *(float4*)(prod_out + (int64_t)m * K + k) = v[i][0];
            *(float4*)(prod_out + (int64_t)m * K + k + 4) = v[i][1];
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++)
            amax = fmaxf(fmaxf(amax, fmaxf(fabsf(v[i][hh].x), fabsf(v[i][hh].y))), fmaxf(fabsf(v[i][hh].z), fabsf(v[i][hh].w)));
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
    int ex = 0;
    if (amax > 0.0f) {
        int x2;
        (void)frexpf(amax, &x2);  // amax in [2^(x2-1), 2^x2)
        ex = 15 - x2;
        if (ex > 126) ex = 126;
    }
    if (lane == 0) xs[m] = ldexpf(1.0f, -ex);
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int k = 8 * (lane + 64 * i);
        float gq[2];
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const float4 x = v[i][hh];
            const float y[4] = {ldexpf(x.x, ex), ldexpf(x.y, ex), ldexpf(x.z, ex), ldexpf(x.w, ex)};
            _Float16 hv[4], lv[4];
            float gs = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                hv[j] = (_Float16)y[j];
                lv[j] = (_Float16)(y[j] - (float)hv[j]);
                gs += (float)hv[j] + (float)lv[j];
            }
            gq[hh] = gs;
            if (k < K) {
                *(uint2*)(XH + (int64_t)m * K + k + 4 * hh) = __builtin_bit_cast(uint2, h4v{hv[0], hv[1], hv[2], hv[3]});
                *(uint2*)(XL + (int64_t)m * K + k + 4 * hh) = __builtin_bit_cast(uint2, h4v{lv[0], lv[1], lv[2], lv[3]});
            }
        }
        float gs = gq[0] + gq[1];
        gs += __shfl_xor(gs, 1, 64);
        gs += __shfl_xor(gs, 2, 64);
        if (k < K && (lane & 3) == 0) XS[(int64_t)m * (K / 32) + k / 32] = gs;
    }
}

hipError_t launch_split_rows(int producer, const float* A, const float* aux, int lda, int M, int K, void* XH,
                             void* XL, float* XS, float* xs, float* prod_out, hipStream_t s) {
    if (M == 0) return hipSuccess;
    if (K <= 0 || K > 1024 * 16 || K % 32 || lda % 4 || (uintptr_t)A % 16 || (uintptr_t)aux % 16 ||
        (uintptr_t)XH % 8 || (uintptr_t)XL % 8 || (uintptr_t)prod_out % 16)
        return hipErrorInvalidValue;
    if (K <= 2048) {  // a wavefront per row
        if (producer == PROD_SWIGLU)
            split_rows_wave_kernel<PROD_SWIGLU><<<(M + 3) / 4, 256, 0, s>>>(A, aux, lda, M, K, (_Float16*)XH,
                                                                          (_Float16*)XL, XS, xs, prod_out);
        else
            split_rows_wave_kernel<PROD_NONE><<<(M + 3) / 4, 256, 0, s>>>(A, aux, lda, M, K, (_Float16*)XH,
                                                                        (_Float16*)XL, XS, xs, prod_out);
    } else if (producer == PROD_SWIGLU)
        split_rows_kernel<PROD_SWIGLU><<<M, 256, 0, s>>>(A, aux, lda, K, (_Float16*)XH, (_Float16*)XL, XS, xs,
                                                          prod_out);
    else
        split_rows_kernel<PROD_NONE><<<M, 256, 0, s>>>(A, aux, lda, K, (_Float16*)XH, (_Float16*)XL, XS, xs,
                                                        prod_out);
    return hipGetLastError();
}

// The tile list of the grouped GEMM: group e (experts 0..E-1, then the
// shared expert as group E with T_sh rows after the routed ones) covers
// ceil(rows / 32) tiles.  One workgroup: a prefix sum over the groups.
// Also completes the shared group's entries: grp[E + 1] and the token of
// each shared row (x_idx[grp[E] + t] = t).
__global__ __launch_bounds__(1024) void moe_tiles_kernel(int32_t* __restrict__ grp, int32_t* __restrict__ x_idx,
                                                         int E, int T_sh, int2* __restrict__ tiles,
                                                         int32_t* __restrict__ n_tiles) {
    __shared__ int cnt[1024 + 1];
    const int tid = threadIdx.x;
    const int base = grp[E];  // routed rows end (all pair rows are sorted by expert)
    if (tid == 0) grp[E + 1] = base + T_sh;
    for (int t = tid; t < T_sh; t += 1024) x_idx[base + t] = t;
    const int G = E + 1;
    int mine = 0;
    if (tid < G) {
        const int rows = tid < E ? grp[tid + 1] - grp[tid] : T_sh;
        mine = (rows + kMoeBM - 1) / kMoeBM;
    }
    cnt[tid] = mine;
    __syncthreads();
    // inclusive scan (Hillis-Steele over 1024 entries)
    for (int off = 1; off < 1024; off <<= 1) {
        const int v = tid >= off ? cnt[tid - off] : 0;
        __syncthreads();
        cnt[tid] += v;
        __syncthreads();
    }
    if (tid < G) {
        const int first = cnt[tid] - mine;
        const int p0 = tid < E ? grp[tid] : base;
        for (int i = 0; i < mine; i++) tiles[first + i] = make_int2(tid, p0 + kMoeBM * i);
    }
    if (tid == 1023) *n_tiles = cnt[1023];
}

hipError_t launch_moe_tiles(int32_t* grp, int32_t* x_idx, int E, int T_sh, int2* tiles, int32_t* n_tiles, hipStream_t s) {
    if (E + 1 > 1024) return hipErrorInvalidValue;
    moe_tiles_kernel<<<1, 1024, 0, s>>>(grp, x_idx, E, T_sh, tiles, n_tiles);
    return hipGetLastError();
}

hipError_t launch_moe_gemm(uint32_t type, const MoeGemm& g, hipStream_t s) {
    MoeGemmArgs a;
    a.W = (const uint8_t*)g.W; a.W2 = (const uint8_t*)g.W2;
    a.Wsh = (const uint8_t*)g.Wsh; a.W2sh = (const uint8_t*)g.W2sh;
    a.w_stride = g.w_stride;
    a.row_bytes = row_bytes(type, g.K);
    a.N = g.N; a.K = g.K; a.n1 = g.n1 > 0 ? g.n1 : g.N; a.E = g.E;
    a.QA = g.QA; a.sa = g.sa; a.x_idx = g.x_idx; a.grp = g.grp;
    a.tiles = (const int2*)g.tiles; a.n_tiles = g.n_tiles;
    a.C = g.C; a.C2 = g.C2; a.ldc = g.ldc;
    a.XH = (const _Float16*)g.XH; a.XL = (const _Float16*)g.XL; a.XS = g.XS; a.xs = g.xs;
    a.QS = g.QS;
    if (!g.XH && (type == T_Q4_K || type == T_Q5_K) && !g.QS) return hipErrorInvalidValue;
    const dim3 grid((g.N + kMoeBN - 1) / kMoeBN, g.max_tiles);
    if (g.max_tiles <= 0) return hipSuccess;
    if (g.XH) {  // fp32 rows as fp16 hi + lo
        if (g.K % kF16BK || !g.XL || !g.XS || !g.xs) return hipErrorInvalidValue;
        switch (type) {
        case T_Q4_K: moe_gemm_f16_kernel<T_Q4_K, 1><<<grid, 256, 0, s>>>(a); break;
        case T_Q5_K: moe_gemm_f16_kernel<T_Q5_K, 1><<<grid, 256, 0, s>>>(a); break;
        case T_Q6_K: moe_gemm_f16_kernel<T_Q6_K, 1><<<grid, 256, 0, s>>>(a); break;
        case T_Q8_0: moe_gemm_f16_kernel<T_Q8_0, 1><<<grid, 256, 0, s>>>(a); break;
        case T_IQ4_NL: moe_gemm_f16_kernel<T_IQ4_NL, 1><<<grid, 256, 0, s>>>(a); break;
        case T_IQ4_XS: moe_gemm_f16_kernel<T_IQ4_XS, 1><<<grid, 256, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    switch (type) {
    case T_Q4_K: moe_gemm_kernel<T_Q4_K><<<grid, 256, 0, s>>>(a); break;
    case T_Q5_K: moe_gemm_kernel<T_Q5_K><<<grid, 256, 0, s>>>(a); break;
    case T_Q6_K: moe_gemm_kernel<T_Q6_K><<<grid, 256, 0, s>>>(a); break;
    case T_Q8_0: moe_gemm_kernel<T_Q8_0><<<grid, 256, 0, s>>>(a); break;
    case T_IQ4_NL: moe_gemm_kernel<T_IQ4_NL><<<grid, 256, 0, s>>>(a); break;
    case T_IQ4_XS: moe_gemm_kernel<T_IQ4_XS><<<grid, 256, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// C = sa * (slice 0 + slice 1 + ...) for each output tile, with the (m, n)
// of each register element as in gemm_i8_lds_kernel.  Workgroup (x, y, z)
// covers tile (x, y) and register elements [4z, 4z + 4) of every thread, so
// each thread has four independent load streams.
template <int BM, int BN>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmMultiArgs a) {
    constexpr int WM = BM / 2, WN = BN / 2, TN = WN / 32;
    int q = 0;
    while (q + 1 < a.np && (int)blockIdx.x >= a.p[q + 1].tile_begin) q++;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, lk = lane >> 5;
    const int m_tile = blockIdx.y * BM, n_tile = ((int)blockIdx.x - a.p[q].tile_begin) * BN;
    const int wm = (wave >> 1) * WM, wn = (wave & 1) * WN;
    const int N = a.p[q].N, ldc = a.p[q].ldc;
    float* const C = a.p[q].C;
    const float* part = a.part + (int64_t)(blockIdx.y * gridDim.x + blockIdx.x) * a.splits * (BM * BN);
    const int e0 = 4 * blockIdx.z;
    float sum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int z = 0; z < a.splits; z++)
#pragma unroll
        for (int u = 0; u < 4; u++) sum[u] += part[(int64_t)z * (BM * BN) + (e0 + u) * 256 + tid];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int e = e0 + u, r = e & 15, ij = e >> 4, i = ij / TN, j = ij % TN;
        const int m = m_tile + wm + 32 * i + 8 * (r >> 2) + 4 * lk + (r & 3);
        const int n = n_tile + wn + 32 * j + li;
        if (m < a.M && n < N) C[(int64_t)m * ldc + n] = sum[u] * a.sa[m];
    }
}

// Workgroup tile 64x64 (32x32 per wavefront), register prefetch two
// K-steps ahead (128x64 tiles and depths 1, 3, 4 measured slower).
static const void* gemm_kernel_for(uint32_t type) {
    switch (type) {
    case T_Q4_K: return (const void*)gemm_i8_lds_kernel<T_Q4_K, 64, 64, 2>;
    case T_Q5_K: return (const void*)gemm_i8_lds_kernel<T_Q5_K, 64, 64, 2>;
    case T_Q8_0: return (const void*)gemm_i8_lds_kernel<T_Q8_0, 64, 64, 2>;
    case T_IQ4_NL: return (const void*)gemm_i8_lds_kernel<T_IQ4_NL, 64, 64, 2>;
    case T_IQ4_XS: return (const void*)gemm_i8_lds_kernel<T_IQ4_XS, 64, 64, 2>;
    default: return nullptr;
    }
}

// Split count for T tiles of S K-steps on R resident workgroups: split K
// only to fill the chip (T * splits <= R) and keep at least two K-steps per
// slice.  Once the tiles alone fill a round, the reduction's extra traffic
// (splits x the output in fp32, written and read back) costs more than the
// rounds it would even out.
static int choose_splits(int64_t tiles, int nsteps, int resident) {
    int s = 1;
    while (s < 8 && tiles * (s * 2) <= resident && nsteps / (s * 2) >= 2) s *= 2;
    return s;
}

GemmPlan plan_gemm_i8(uint32_t type, const int* Ns, int n, int K, int M) {
    GemmPlan pl{};
    pl.bm = 64;
    pl.bn = 64;
    pl.n_tiles = 0;
    for (int i = 0; i < n; i++) pl.n_tiles += (Ns[i] + pl.bn - 1) / pl.bn;
    pl.m_tiles = (M + pl.bm - 1) / pl.bm;
    const int nsteps = (K + kGemmBK - 1) / kGemmBK;
    pl.splits = 1;
    if (type != T_Q6_K) {
        const void* k = gemm_kernel_for(type);
        int per_cu = 0;
        per_cu = k ? occupancy_per_cu(k, 0) : 1;
        pl.splits = choose_splits((int64_t)pl.n_tiles * pl.m_tiles, nsteps, per_cu * device_cus());
    }
    pl.steps_per_split = (nsteps + pl.splits - 1) / pl.splits;
    pl.splits = (nsteps + pl.steps_per_split - 1) / pl.steps_per_split;
    pl.part_floats = pl.splits > 1 ? (size_t)pl.n_tiles * pl.m_tiles * pl.splits * pl.bm * pl.bn : 0;
    return pl;
}

hipError_t launch_gemm_i8_multi(uint32_t type, const GemmDesc* d, int n, int K, const int8_t* qa, const float* sa,
                                int M, float* part, hipStream_t s) {
    if (M == 0 || n == 0) return hipSuccess;
    if (n > kGemmMaxProb) return hipErrorInvalidValue;
    if (type == T_Q6_K) {  // 16-value groups: direct-load kernel with 32x32x16 MFMAs
        for (int i = 0; i < n; i++) {
            GemmArgs a;
            a.W = (const uint8_t*)d[i].W;
            a.row_bytes = row_bytes(type, K);
            a.N = d[i].N; a.K = K;
            a.QA = qa; a.sa = sa;
            a.C = d[i].C; a.ldc = d[i].ldc; a.M = M;
            a.Cpart = nullptr;
            a.steps_per_split = 0;
            const dim3 grid((d[i].N + 127) / 128, (M + 127) / 128);
            gemm_i8_kernel<T_Q6_K><<<grid, 256, 0, s>>>(a);
        }
        return hipGetLastError();
    }
    int Ns[kGemmMaxProb];
    for (int i = 0; i < n; i++) Ns[i] = d[i].N;
    const GemmPlan pl = plan_gemm_i8(type, Ns, n, K, M);
    GemmMultiArgs a;
    int tb = 0;
    for (int i = 0; i < n; i++) {
        a.p[i].W = (const uint8_t*)d[i].W;
        a.p[i].C = d[i].C;
        a.p[i].N = d[i].N;
        a.p[i].ldc = d[i].ldc;
        a.p[i].tile_begin = tb;
        tb += (d[i].N + pl.bn - 1) / pl.bn;
    }
    a.np = n;
    a.row_bytes = row_bytes(type, K);
    a.K = K;
    a.M = M;
    a.QA = qa;
    a.sa = sa;
    a.splits = pl.splits;
    a.steps_per_split = pl.steps_per_split;
    a.part = part;
    if (pl.splits > 1 && !part) return hipErrorInvalidValue;
    const dim3 grid(pl.n_tiles, pl.m_tiles, pl.splits);
    const void* k = gemm_kernel_for(type);
    if (!k) return hipErrorInvalidValue;
    void* args[] = {&a};
    hipError_t e = hipLaunchKernel(k, grid, dim3(256), args, 0, s);
    if (e != hipSuccess || pl.splits == 1) return e;
    // (BM*BN/256) register elements per thread, four per workgroup.
    gemm_reduce_kernel<64, 64><<<dim3(pl.n_tiles, pl.m_tiles, 64 * 64 / 1024), 256, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_gemm_i8(uint32_t type, const void* W, int N, int K, const int8_t* qa, const float* sa, int M,
                          float* C, int ldc, float* part, hipStream_t s) {
    const GemmDesc d{W, C, N, ldc};
    return launch_gemm_i8_multi(type, &d, 1, K, qa, sa, M, part, s);
}

// Byte copy by the shader cores, used between pinned host memory and HBM
// for the small per-call vectors of the synchronous entry points (a copy
// kernel's launch costs less than a DMA-engine transfer at these sizes).
// 16-byte chunks when both ends are 16-byte aligned, then the tail.
__global__ __launch_bounds__(256) void copy_bytes_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                         size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t n16 = n / 16;
    if (i < n16) {
        ((uint4*)dst)[i] = ((const uint4*)src)[i];
    } else if (i < n16 + (n & 15)) {
        const size_t b = n16 * 16 + (i - n16);
        dst[b] = src[b];
    }
}

hipError_t launch_copy_bytes(void* dst, const void* src, size_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (((uintptr_t)dst | (uintptr_t)src) & 15u) return hipMemcpyAsync(dst, src, n, hipMemcpyDefault, s);
    const size_t items = n / 16 + (n & 15);
    copy_bytes_kernel<<<(unsigned)((items + 255) / 256), 256, 0, s>>>((const uint8_t*)src, (uint8_t*)dst, n);
    return hipGetLastError();
}

// Completion word for a host that waits by polling pinned memory instead of
// a stream synchronization: one lane stores v with a system-scope release
// after everything queued before it on the stream has finished.
__global__ __launch_bounds__(64) void host_flag_kernel(uint32_t* flag, uint32_t v) {
    if (threadIdx.x == 0) __hip_atomic_store(flag, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

hipError_t launch_host_flag(uint32_t* flag, uint32_t v, hipStream_t s) {
    host_flag_kernel<<<1, 64, 0, s>>>(flag, v);
    return hipGetLastError();
}

// x_eff[m][k] = q[m][k] * scale[m] (fp32) from pre-quantized activations.
__global__ __launch_bounds__(256) void dequant_act_kernel(const int8_t* __restrict__ q, const float* __restrict__ sa,
                                                          int M, int K, float* __restrict__ x) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)M * K) return;
    x[i] = __fmul_rn((float)q[i], sa[i / K]);
}

hipError_t launch_dequant_act(const int8_t* q, const float* sa, int M, int K, float* x, hipStream_t s) {
    const int64_t n = (int64_t)M * K;
    if (n == 0) return hipSuccess;
    dequant_act_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(q, sa, M, K, x);
    return hipGetLastError();
}

// ================================================================== argmax
// Greedy token choice of sample_token (main.cpp:827-838): the first index
// with the strictly largest value; NaN never wins, and a row with nothing
// above -inf gives index 0.  (value, index) pairs merge with ties going to
// the lower index, so the result does not depend on how the row is split.
__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

// Stage 1: workgroup (p, m) reduces chunk p of row m (chunks of `chunk`
// values, a multiple of 4; float4 loads when rows are 16-byte aligned) to
// one (value, index) pair.  Each thread walks its elements in increasing
// index order, so a strict > keeps the first of equal values.
constexpr int kArgmaxParts = 64;
__global__ __launch_bounds__(256) void argmax_part_kernel(const float* __restrict__ L, int N, int ld, int chunk,
                                                          int vec4, float* __restrict__ pv, int* __restrict__ pi) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int m = blockIdx.y, p = blockIdx.x;
    const float* row = L + (int64_t)m * ld;
    const int n0 = p * chunk, n1 = n0 + chunk < N ? n0 + chunk : N;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    if (vec4) {
        for (int n = n0 + 4 * threadIdx.x; n < n1; n += 1024) {
            const float4 v = *(const float4*)(row + n);  // n1 - n >= 4: N and chunk are multiples of 4
            if (v.x > bv) { bv = v.x; bi = n; }
            if (v.y > bv) { bv = v.y; bi = n + 1; }
            if (v.z > bv) { bv = v.z; bi = n + 2; }
            if (v.w > bv) { bv = v.w; bi = n + 3; }
        }
    } else {
        for (int n = n0 + threadIdx.x; n < n1; n += 256) {
            const float v = row[n];
            if (v > bv) { bv = v; bi = n; }
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) argmax_merge(bv, bi, __shfl_xor(bv, off, 64), __shfl_xor(bi, off, 64));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; w++) argmax_merge(bv, bi, sv[w], si[w]);
        pv[m * kArgmaxParts + p] = bv;
        pi[m * kArgmaxParts + p] = bi;
    }
}

// Stage 2: one wavefront per row merges the chunk results.
__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ L, int ld, int parts,
                                                          const float* __restrict__ pv, const int* __restrict__ pi,
                                                          int32_t* __restrict__ idx, float* __restrict__ val) {
    const int m = blockIdx.x, lane = threadIdx.x;
    float bv = lane < parts ? pv[m * kArgmaxParts + lane] : -INFINITY;
    int bi = lane < parts ? pi[m * kArgmaxParts + lane] : 0x7FFFFFFF;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) argmax_merge(bv, bi, __shfl_xor(bv, off, 64), __shfl_xor(bi, off, 64));
    if (lane == 0) {
        const int i = bi == 0x7FFFFFFF ? 0 : bi;
        idx[m] = i;
        if (val) val[m] = L[(int64_t)m * ld + i];  // the chosen token's logit (NaN / -inf when nothing won)
    }
}

size_t argmax_workspace_bytes(int M) { return (size_t)M * kArgmaxParts * (sizeof(float) + sizeof(int)); }

hipError_t launch_argmax_rows(const float* L, int M, int N, int ld, int32_t* idx, float* val, void* ws,
                              hipStream_t s) {
    if (M == 0) return hipSuccess;
    int parts = (N + 2047) / 2048;
    parts = parts < 1 ? 1 : (parts > kArgmaxParts ? kArgmaxParts : parts);
    int chunk = (N + parts - 1) / parts;
    chunk = (chunk + 3) & ~3;
    parts = (N + chunk - 1) / chunk;
    const int vec4 = ((uintptr_t)L % 16 == 0) && ld % 4 == 0 && N % 4 == 0;
    float* pv = (float*)ws;
    int* pi = (int*)((char*)ws + (size_t)M * kArgmaxParts * sizeof(float));
    argmax_part_kernel<<<dim3(parts, M), 256, 0, s>>>(L, N, ld, chunk, vec4, pv, pi);
    argmax_final_kernel<<<M, 64, 0, s>>>(L, ld, parts, pv, pi, idx, val);
    return hipGetLastError();
}

// =============================================================== attention
// Decode attention over one layer's KV cache in its native layout
// [position][kv head][head_dim] (kv_cache.cpp:38-48), for query rows at
// positions pos0, pos0+1, ... (causal: row t sees positions <= pos0 + t).
// Same result as CpuRefBackend::flash_attn (cpu_ref.cpp:223-280) over the GQA-
// expanded K/V (main.cpp:3358-3379), without materialising the expansion:
// workgroup (span c, kv head h, row t) reads the positions of span c of kv
// head h once for all G = n_head / n_kv query heads that share it.
//
// A span is a whole number of 64-position steps; the span count is chosen so
// the grid fills the chip.  Per step (4 wavefronts, 16 positions each):
//   phase 1: score[g][j] = (q_g . k_j) * scale, 16 lanes per position
//            (head_dim/16 values each, DPP sum), 4 positions per wave step;
//   phase 2: online softmax, one wavefront per query head: m' = max(m, s),
//            p = exp(s - m'), alpha = exp(m - m'), l = l * alpha + sum p;
//   phase 3: o_g = o_g * alpha_g + sum_j p_gj v_j (lane layout of phase 1).
// K of the next step is fetched during phases 2-3 and V of a step during
// phases 1-2.  Scores and alphas are double-buffered in LDS, so a step needs
// two barriers.  With one span the kernel writes o / l directly; otherwise it
// writes (m, l, o) and attn_combine_kernel merges the spans:
// m = max m_c, out = sum_c e^(m_c-m) o_c / sum_c e^(m_c-m) l_c.  The
// reference does one softmax over the whole row; the results differ by fp32
// rounding.
constexpr int kAttnStep = 64;

struct AttnArgs {
    const float* Q;   // [n_tok][n_head][HD]
    const float* K;   // [ctx][n_kv][HD]
    const float* V;
    float* part_o;    // [n_tok][n_head][n_spans][HD]
    float* part_ml;   // [n_tok][n_head][n_spans][2]
    float* out;       // [n_tok][n_head][HD]
    int n_head, n_kv, n_spans, span_steps;
    int64_t ctx_len, pos0;
    float scale;
};

template <int N> __device__ __forceinline__ void ld_floats(const float* p, float (&v)[N]) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
        const float4 f = *(const float4*)(p + i);
        v[i] = f.x; v[i + 1] = f.y; v[i + 2] = f.z; v[i + 3] = f.w;
    }
}

template <int HD, int G>
__global__ __launch_bounds__(256) void attn_span_kernel(AttnArgs a) {
    constexpr int DPL = HD / 16;
    constexpr int IT = kAttnStep / 16;  // wave steps of 4 positions
    __shared__ float sc[2][G][kAttnStep];
    __shared__ float al[2][G];
    __shared__ float ml[G][2];
    __shared__ float ored[4][G][HD];
    const int span = blockIdx.x, kvh = blockIdx.y, t = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, pg = lane >> 4;
    const int64_t qpos = a.pos0 + t;
    const int64_t last = qpos < a.ctx_len - 1 ? qpos : a.ctx_len - 1;
    const int64_t s0 = (int64_t)span * a.span_steps * kAttnStep;
    int64_t s1 = s0 + (int64_t)a.span_steps * kAttnStep;
    if (s1 > last + 1) s1 = last + 1;
    const int steps = s1 > s0 ? (int)((s1 - s0 + kAttnStep - 1) / kAttnStep) : 0;
    const int64_t kstride = (int64_t)a.n_kv * HD;
    const float* Kb = a.K + (int64_t)kvh * HD + l16 * DPL;
    const float* Vb = a.V + (int64_t)kvh * HD + l16 * DPL;
    const int jbase = wave * (kAttnStep / 4) + pg;  // + it * 4

    float q[G][DPL], o[G][DPL];
#pragma unroll
    for (int g = 0; g < G; g++) {
        ld_floats<DPL>(a.Q + ((int64_t)t * a.n_head + kvh * G + g) * HD + l16 * DPL, q[g]);
#pragma unroll
        for (int i = 0; i < DPL; i++) o[g][i] = 0.0f;
    }
    float m_run = -INFINITY, l_run = 0.0f;  // for heads g == wave (+4): per wave, G <= 8
    float m_run2 = -INFINITY, l_run2 = 0.0f;

    float kk[IT][DPL], vv[IT][DPL];
    auto fetch = [&](float (&r)[IT][DPL], const float* base, int step) {
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int64_t j = s0 + (int64_t)step * kAttnStep + jbase + it * 4;
            ld_floats<DPL>(base + (j < s1 ? j : s0) * kstride, r[it]);
        }
    };
    if (steps > 0) fetch(kk, Kb, 0);
    for (int st = 0; st < steps; st++) {
        const int b = st & 1;
        const int64_t jb = s0 + (int64_t)st * kAttnStep;
        fetch(vv, Vb, st);
        // phase 1
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int jl = jbase + it * 4;
            const bool vis = jb + jl < s1;
#pragma unroll
            for (int g = 0; g < G; g++) {
                float sv = 0.0f;
#pragma unroll
                for (int i = 0; i < DPL; i++) sv = fmaf(q[g][i], kk[it][i], sv);
                sv = group_sum(sv, 4);
                if (l16 == 0) sc[b][g][jl] = vis ? sv * a.scale : -INFINITY;
            }
        }
        if (st + 1 < steps) fetch(kk, Kb, st + 1);
        __syncthreads();
        // phase 2: wavefront w owns heads w and w + 4
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int g = wave + 4 * r;
            if (g < G) {
                float& mr = r ? m_run2 : m_run;
                float& lr = r ? l_run2 : l_run;
                const float v = sc[b][g][lane];
                float mx = v;
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
                const float mn = fmaxf(mr, mx);
                const float pv = mn == -INFINITY ? 0.0f : expf(v - mn);
                const float alpha = mr == -INFINITY ? 0.0f : expf(mr - mn);
                sc[b][g][lane] = pv;
                float ls = pv;
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) ls += __shfl_xor(ls, off, 64);
                lr = lr * alpha + ls;
                mr = mn;
                if (lane == 0) al[b][g] = alpha;
            }
        }
        __syncthreads();
        // phase 3
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float alpha = al[b][g];
#pragma unroll
            for (int i = 0; i < DPL; i++) o[g][i] *= alpha;
        }
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int jl = jbase + it * 4;
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float pv = sc[b][g][jl];  // 0 where not visible
#pragma unroll
                for (int i = 0; i < DPL; i++) o[g][i] = fmaf(pv, vv[it][i], o[g][i]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const int g = wave + 4 * r;
        if (g < G && lane == 0) { ml[g][0] = r ? m_run2 : m_run; ml[g][1] = r ? l_run2 : l_run; }
    }
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int i = 0; i < DPL; i++) {
            float v = o[g][i];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            if (pg == 0) ored[wave][g][l16 * DPL + i] = v;
        }
    __syncthreads();
    const int64_t hb = (int64_t)t * a.n_head + kvh * G;
    if (a.n_spans == 1) {
        for (int e = tid; e < G * HD; e += 256) {
            const int g = e / HD, d = e % HD;
            a.out[(hb + g) * HD + d] = (ored[0][g][d] + ored[1][g][d] + ored[2][g][d] + ored[3][g][d]) / ml[g][1];
        }
        return;
    }
    for (int e = tid; e < G * HD; e += 256) {
        const int g = e / HD, d = e % HD;
        a.part_o[((hb + g) * a.n_spans + span) * HD + d] = ored[0][g][d] + ored[1][g][d] + ored[2][g][d] + ored[3][g][d];
    }
    if (tid < G) {
        a.part_ml[((hb + tid) * a.n_spans + span) * 2 + 0] = ml[tid][0];
        a.part_ml[((hb + tid) * a.n_spans + span) * 2 + 1] = ml[tid][1];
    }
}

// One workgroup of 512 threads per (head, row): merge the span partials in
// one pass.  Thread (grp, d), d = tid % HD, folds spans grp, grp + 512/HD, ...
// into a running (m, l, o) (rescaling when the maximum grows); the groups
// are then merged in a fixed order, so results are deterministic.
template <int HD>
__global__ __launch_bounds__(512) void attn_combine_kernel(AttnArgs a) {
    constexpr int NG = 512 / HD;
    __shared__ float gm[NG], gl[NG], go[NG][HD];
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int64_t hb = (int64_t)t * a.n_head + h;
    const int ns = a.n_spans;
    const float* pml = a.part_ml + hb * ns * 2;
    const int d = tid % HD, grp = tid / HD;
    const float* po = a.part_o + hb * ns * HD + d;
    // batches of 16 spans: all loads first, then one rescale per batch
    constexpr int B = 16;
    float m = -INFINITY, L = 0.0f, o = 0.0f;
    for (int c0 = grp; c0 < ns; c0 += NG * B) {
        float mc[B], lc[B], oc[B];
#pragma unroll
        for (int u = 0; u < B; u++) {
            const int c = c0 + u * NG;
            const bool ok = c < ns;
            const float2 v = *(const float2*)(pml + 2 * (ok ? c : 0));
            const float ov = po[(int64_t)(ok ? c : 0) * HD];
            mc[u] = ok ? v.x : -INFINITY;  // -inf also marks a span past this row's position
            lc[u] = v.y;
            oc[u] = ov;
        }
        float mb = m;
#pragma unroll
        for (int u = 0; u < B; u++) mb = fmaxf(mb, mc[u]);
        if (mb == -INFINITY) continue;
        const float r = m == -INFINITY ? 0.0f : expf(m - mb);
        L *= r;
        o *= r;
#pragma unroll
        for (int u = 0; u < B; u++) {
            const float e = mc[u] == -INFINITY ? 0.0f : expf(mc[u] - mb);
            L = fmaf(lc[u], e, L);
            o = fmaf(oc[u], e, o);
        }
        m = mb;
    }
    go[grp][d] = o;
    if (d == 0) { gm[grp] = m; gl[grp] = L; }
    __syncthreads();
    if (grp == 0) {
        float mx = gm[0];
#pragma unroll
        for (int k = 1; k < NG; k++) mx = fmaxf(mx, gm[k]);
        float os = 0.0f, ls = 0.0f;
#pragma unroll
        for (int k = 0; k < NG; k++) {
            const float e = gm[k] == -INFINITY ? 0.0f : expf(gm[k] - mx);
            os = fmaf(go[k][d], e, os);
            ls = fmaf(gl[k], e, ls);
        }
        a.out[hb * HD + d] = os / ls;
    }
}

static int attn_span_wgs() {
    static int v = -1;
    if (v < 0) {
        const int r = resident_blocks(attn_span_kernel<64, 4>, 0);
        v = r > 0 ? r : 1024;
    }
    return v;
}

static void attn_plan(int n_tok, int n_kv, int64_t ctx_len, int64_t pos0, int* n_spans, int* span_steps) {
    const int64_t last = pos0 + n_tok - 1 < ctx_len - 1 ? pos0 + n_tok - 1 : ctx_len - 1;
    const int64_t steps = (last + kAttnStep) / kAttnStep;
    int64_t want = env_int("GGQ_ATTN_SPANS", 0);
    if (want <= 0) want = (attn_span_wgs() + (int64_t)n_kv * n_tok - 1) / ((int64_t)n_kv * n_tok);
    if (want > steps) want = steps;
    if (want < 1) want = 1;
    const int64_t per = (steps + want - 1) / want;
    *span_steps = (int)per;
    *n_spans = (int)((steps + per - 1) / per);
}

size_t attn_workspace_floats(int n_tok, int n_head, int head_dim, int64_t ctx_len, int64_t pos0, int n_kv) {
    int ns, ss;
    attn_plan(n_tok, n_kv, ctx_len, pos0, &ns, &ss);
    return ns > 1 ? (size_t)n_tok * n_head * ns * (head_dim + 2) : 0;
}

hipError_t launch_attn_decode(const float* Q, const float* K, const float* V, int n_tok, int n_head, int n_kv,
                              int head_dim, int64_t ctx_len, int64_t pos0, float* out, float* ws, hipStream_t s) {
    if (n_tok == 0) return hipSuccess;
    const int G = n_head / n_kv;
    AttnArgs a;
    a.Q = Q; a.K = K; a.V = V; a.out = out;
    a.n_head = n_head; a.n_kv = n_kv;
    attn_plan(n_tok, n_kv, ctx_len, pos0, &a.n_spans, &a.span_steps);
    a.ctx_len = ctx_len; a.pos0 = pos0;
    a.scale = 1.0f / sqrtf((float)head_dim);  // cpu_ref.cpp:237
    a.part_o = ws;
    a.part_ml = ws ? ws + (size_t)n_tok * n_head * a.n_spans * head_dim : nullptr;
    if (a.n_spans > 1 && !ws) return hipErrorInvalidValue;
    const dim3 grid(a.n_spans, n_kv, n_tok);
#define L(HD_, G_) attn_span_kernel<HD_, G_><<<grid, 256, 0, s>>>(a)
#define BY_G(HD_)                                 \
    switch (G) {                                  \
    case 1: L(HD_, 1); break;                     \
    case 2: L(HD_, 2); break;                     \
    case 4: L(HD_, 4); break;                     \
    case 8: L(HD_, 8); break;                     \
    default: return hipErrorInvalidValue;         \
    }
    if (head_dim == 64) { BY_G(64) }
    else if (head_dim == 128) { BY_G(128) }
    else return hipErrorInvalidValue;
#undef BY_G
#undef L
    if (a.n_spans > 1) {
        if (head_dim == 64) attn_combine_kernel<64><<<dim3(n_head, n_tok), 512, 0, s>>>(a);
        else attn_combine_kernel<128><<<dim3(n_head, n_tok), 512, 0, s>>>(a);
    }
    return hipGetLastError();
}

// ====================================================================== MoE
// Routing (main.cpp:3126-3135): top-k experts by descending logit, then a
// softmax over the selected logits only: w_j = exp(l_j - l_0) / sum.
// One wavefront per token; lane i holds the logits of experts i, i+64, ...
// in registers (E <= 1024) with a bitmask of the ones already taken; ties
// break toward the lower expert id.  Selection j ends in lane j.
constexpr int kRouteMaxPerLane = 16;
// One argmax step against the lane selected by DPP control CTRL: the larger
// value wins, ties go to the lower expert index (as the reference's scan in
// index order).  -inf values with index 0x7FFFFFFF never win a tie; a free
// expert always exists (topk <= E), so the final index is below E.
template <int CTRL> __device__ __forceinline__ void route_step(float& best, int& bi) {
    const float ov = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, best), CTRL, 0xF, 0xF, false));
    const int oi = __builtin_amdgcn_mov_dpp(bi, CTRL, 0xF, 0xF, false);
    if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
}

// PL: logits per lane (E <= 64 * PL), so the per-step scan covers only the
// experts that exist.
// One wavefront routes token t (lane = its lane): selections and weights of
// the token to sel / wsel (and, when sel_l is given, the selections to
// sel_l too).
template <int PL>
__device__ __forceinline__ void route_token(const float* __restrict__ logits, int E, int topk, int t, int lane,
                                            int32_t* __restrict__ sel, float* __restrict__ wsel,
                                            int32_t* sel_l) {
    const float* l = logits + (int64_t)t * E;
    float v[PL];
    uint32_t taken = 0;
#pragma unroll
    for (int i = 0; i < PL; i++) {
        const int e = lane + 64 * i;
        // A NaN logit ranks with -inf (ties to the lower id), so every
        // selection is an expert below E whatever the logits hold.
        const float x = e < E ? l[e] : -INFINITY;
        v[i] = x != x ? -INFINITY : x;
        if (e >= E) taken |= 1u << i;
    }
    int my_sel = 0;
    float my_l = 0.0f;
    for (int j = 0; j < topk; j++) {
        float best = -INFINITY;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int i = 0; i < PL; i++) {
            const int e = lane + 64 * i;
            const bool free = !((taken >> i) & 1u);
            if (free && (v[i] > best || (v[i] == best && e < bi))) {
                best = v[i];
                bi = e;
            }
        }
        // Inside each row of 16 lanes by DPP (xor 1, xor 2, the other quad
        // of 8, the other half of 16), then across the four rows.
        route_step<0xB1>(best, bi);
        route_step<0x4E>(best, bi);
        route_step<0x141>(best, bi);
        route_step<0x140>(best, bi);
        {
            float rb = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, best), 0));
            int ri = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
            for (int r = 1; r < 4; r++) {
                const float ov = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, best), 16 * r));
                const int oi = __builtin_amdgcn_readlane(bi, 16 * r);
                if (ov > rb || (ov == rb && oi < ri)) { rb = ov; ri = oi; }
            }
            best = rb;
            bi = ri;
        }
        if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
        if (lane == j) my_sel = bi;
    }
    // The softmax takes the selected logits as given (NaN included).
    if (lane < topk) my_l = l[my_sel];
    const float l0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_l), 0));
    const float ex = lane < topk ? expf(my_l - l0) : 0.0f;
    float sum = 0.0f;  // in selection order, as the reference adds them
    for (int j = 0; j < topk; j++) sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), j));
    if (lane < topk) {
        sel[t * topk + lane] = my_sel;
        wsel[t * topk + lane] = ex / sum;
        if (sel_l) sel_l[t * topk + lane] = my_sel;
    }
}

template <int PL>
__global__ __launch_bounds__(64) void moe_route_kernel(const float* __restrict__ logits, int E, int topk,
                                                       int32_t* __restrict__ sel, float* __restrict__ wsel) {
    route_token<PL>(logits, E, topk, blockIdx.x, threadIdx.x, sel, wsel, nullptr);
}

hipError_t launch_moe_route(const float* logits, int T, int E, int topk, int32_t* sel, float* wsel,
                            hipStream_t s) {
    if (T == 0) return hipSuccess;
    if (E > 64 * kRouteMaxPerLane || topk > 64) return hipErrorInvalidValue;
    if (E <= 64) moe_route_kernel<1><<<T, 64, 0, s>>>(logits, E, topk, sel, wsel);
    else if (E <= 128) moe_route_kernel<2><<<T, 64, 0, s>>>(logits, E, topk, sel, wsel);
    else if (E <= 256) moe_route_kernel<4><<<T, 64, 0, s>>>(logits, E, topk, sel, wsel);
    else if (E <= 512) moe_route_kernel<8><<<T, 64, 0, s>>>(logits, E, topk, sel, wsel);
    else moe_route_kernel<kRouteMaxPerLane><<<T, 64, 0, s>>>(logits, E, topk, sel, wsel);
    return hipGetLastError();
}

// Scratch region of ggq_mul_mat_noalloc_dev (see kScratchBytes).  In host
// code `scratch` names a host-side stand-in, not device memory: kernels and
// copies get the address from scratch_device_ptr.
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

hipError_t scratch_device_ptr(int device, void** out) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* ptrs[kMaxDevices] = {};
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!ptrs[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        ptrs[device] = p;
    }
    *out = ptrs[device];
    return hipSuccess;
}

// Expert grouping: stable counting sort of the T*topk (token, slot) pairs by
// expert id.  grp_off[E+1] are the group boundaries, tok_idx[pos] the token of
// each sorted pair and pos_of[t*topk+j] its position.  One workgroup of 1024
// threads, E <= 1024: counts with LDS atomics, an exclusive scan over experts
// (wavefront scans + a scan of the 16 wavefront totals), then every pair's
// rank among earlier pairs of its expert, counted over an LDS copy of `sel`
// (chunks of kGroupChunk pairs; `base` carries the counts of earlier chunks).
constexpr int kGroupChunk = 8192;
// Selections come from moe_route_kernel and are below E; the clamp keeps the
// LDS histograms and the output positions in range regardless.
__device__ __forceinline__ int expert_id(int e, int E) { return e < 0 ? 0 : e >= E ? E - 1 : e; }
__global__ __launch_bounds__(1024) void moe_group_kernel(const int32_t* __restrict__ sel, int n, int E,
                                                         int topk, int32_t* __restrict__ grp_off,
                                                         int32_t* __restrict__ tok_idx,
                                                         int32_t* __restrict__ pos_of) {
    __shared__ __attribute__((aligned(16))) int32_t chunk[kGroupChunk];
    __shared__ int32_t base[1024];
    __shared__ int32_t wsum[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    base[tid] = 0;
    __syncthreads();
    for (int f = tid; f < n; f += 1024) atomicAdd(&base[expert_id(sel[f], E)], 1);
    __syncthreads();
    // Exclusive scan of the counts: base[e] = first position of expert e.
    const int c = base[tid];
    int incl = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(incl, off, 64);
        if (lane >= off) incl += o;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; w++) before += wsum[w];
    const int start = before + incl - c;
    __syncthreads();
    base[tid] = start;
    if (tid < E) grp_off[tid] = start;
    if (tid == 0) grp_off[E] = n;
    __syncthreads();
    for (int c0 = 0; c0 < n; c0 += kGroupChunk) {
        const int len = n - c0 < kGroupChunk ? n - c0 : kGroupChunk;
        for (int f = tid; f < len; f += 1024) chunk[f] = expert_id(sel[c0 + f], E);
        __syncthreads();
        for (int f = tid; f < len; f += 1024) {
            const int e = chunk[f];
            int rank = 0, g = 0;
            for (; g + 4 <= f; g += 4) {
                const int4 v = *(const int4*)&chunk[g];
                rank += (v.x == e) + (v.y == e) + (v.z == e) + (v.w == e);
            }
            for (; g < f; g++) rank += chunk[g] == e;
            const int pos = base[e] + rank;
            tok_idx[pos] = (c0 + f) / topk;
            pos_of[c0 + f] = pos;
        }
        __syncthreads();
        for (int f = tid; f < len; f += 1024) atomicAdd(&base[chunk[f]], 1);
        __syncthreads();
    }
}

// The same stable counting sort for E <= 256 experts and any number of
// pairs, in rounds of 1024 (one pair per thread): a histogram of all pairs
// gives each expert's start; within a round a pair's position is start[e]
// + (pairs of e in earlier rounds) + (pairs of e in earlier wavefronts of
// the round, from per-wavefront histograms) + (pairs of e in earlier lanes
// of its wavefront).
constexpr int kGroupFastE = 256;
// With logits given (moe_group_routes: up to 16 tokens), the launch first
// routes the tokens itself, a wavefront per token (route_token: the same selections
// and weights as moe_route_kernel), keeping the selections in LDS.
constexpr int kGroupRouteMax = 1024;
__global__ __launch_bounds__(1024) void moe_group_small_kernel(const int32_t* __restrict__ sel_in, int n, int E,
                                                               int topk, int32_t* __restrict__ grp_off,
                                                               int32_t* __restrict__ tok_idx,
                                                               int32_t* __restrict__ pos_of, int t_sh,
                                                               ChunkList l0, ChunkList l1, int n_lists,
                                                               const float* __restrict__ logits,
                                                               int32_t* __restrict__ sel_out,
                                                               float* __restrict__ wsel_out, RowQuant rq) {
    __shared__ int32_t hist[16][kGroupFastE];  // per wavefront: pairs of each expert in its slice
    __shared__ int32_t start[kGroupFastE];     // first position of each expert (then its end)
    __shared__ int32_t wsum[4];
    __shared__ int32_t sel_l[kGroupRouteMax];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int i = tid; i < 16 * kGroupFastE; i += 1024) (&hist[0][0])[i] = 0;
    if (logits)
        for (int t = wave; t < n / topk; t += 16)
            route_token<kGroupFastE / 64>(logits, E, topk, t, lane, sel_out, wsel_out, sel_l);
    if (rq.A)  // row m on wavefront (m + 8) % 16, beside the routing of token m on wavefront m
        for (int m = (wave + 8) & 15; m < rq.M; m += 16)
            quant_row_wave<PROD_NONE>(rq.A, nullptr, rq.lda, m, rq.K, rq.q, rq.scales, nullptr, rq.gsum, lane);
    const int32_t* sel = logits ? sel_l : sel_in;
    __syncthreads();
    // Wavefront w ranks the pairs of its slice [w * S, (w + 1) * S), 64 at
    // a time: lanes holding the same expert are found with one ballot per
    // bit of the expert id; a pair's rank is its count of such lanes below
    // it plus the slice's earlier pairs of that expert.  The rank goes to
    // pos_of (read back by the same lane below).
    const int S = ((n + 16 * 64 - 1) / (16 * 64)) * 64;
    const uint64_t below = (1ull << lane) - 1ull;
    for (int f0 = wave * S; f0 < (wave + 1) * S && f0 < n; f0 += 64) {
        const int f = f0 + lane;
        const bool ok = f < n;
        const int e = ok ? expert_id(sel[f], E) : 0;
        uint64_t same = __ballot(ok);
#pragma unroll
        for (int bit = 0; bit < 8; bit++) {
            const uint64_t b1 = __ballot((e >> bit) & 1);
            same &= ((e >> bit) & 1) ? b1 : ~b1;
        }
        const int before = hist[wave][e];
        if (ok && (same & below) == 0) hist[wave][e] = before + __popcll(same);  // the first such lane
        if (ok) pos_of[f] = before + __popcll(same & below);
    }
    __syncthreads();
    // Expert totals, their exclusive scan (four wavefronts cover 256
    // experts), then each wavefront's base per expert.
    if (tid < kGroupFastE) {
        int c = 0;
#pragma unroll
        for (int w = 0; w < 16; w++) c += hist[w][tid];
        int incl = c;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int o = __shfl_up(incl, off, 64);
            if (lane >= off) incl += o;
        }
        if (lane == 63) wsum[wave] = incl;
        start[tid] = incl - c;  // within its wavefront of experts, for now
    }
    __syncthreads();
    if (tid < kGroupFastE) {
        int before = 0;
        for (int w = 0; w < wave; w++) before += wsum[w];
        int b0 = start[tid] + before;
        if (tid < E) grp_off[tid] = b0;
        if (tid == 0) grp_off[E] = n;
#pragma unroll
        for (int w = 0; w < 16; w++) {
            const int c = hist[w][tid];
            hist[w][tid] = b0;
            b0 += c;
        }
        start[tid] = b0;  // the end of expert tid's rows
    }
    __syncthreads();
    for (int f0 = wave * S; f0 < (wave + 1) * S && f0 < n; f0 += 64) {
        const int f = f0 + lane;
        if (f < n) {
            const int e = expert_id(sel[f], E);
            const int pos = hist[wave][e] + pos_of[f];
            tok_idx[pos] = f / topk;
            pos_of[f] = pos;
        }
    }
    // The shared expert's group end and token rows, and the grouped int8
    // launches' chunk lists from the offsets just written, saving their own
    // launches.
    if (tid == 0) grp_off[E + 1] = n + t_sh;
    for (int t = tid; t < t_sh; t += 1024) tok_idx[n + t] = t;
    if (n_lists > 0) {
        __shared__ ChunkList lists[2];
        if (tid == 0) { lists[0] = l0; lists[1] = l1; }
        // start[e] has advanced to the end of expert e's rows
        int r0 = 0, rows = 0;
        if (tid < E) {
            r0 = tid > 0 ? start[tid - 1] : 0;
            rows = start[tid] - r0;
        } else if (tid == E && t_sh > 0) {  // the shared expert: every token after the routed rows
            r0 = n;
            rows = t_sh;
        }
        __syncthreads();
        chunk_lists_from_rows(r0, rows, lists, n_lists, &hist[0][0]);
    }
}

// (one token per wavefront: more tokens per wavefront run their routing
// serially, slower than the separate launch: 64 tokens 165 -> 191 us)
bool moe_group_routes(int T, int topk, int E) {
    return E <= kGroupFastE && topk <= 64 && T <= 16 && (int64_t)T * topk <= kGroupRouteMax;
}

hipError_t launch_moe_group(const int32_t* sel, int T, int topk, int E, int32_t* grp_off,
                            int32_t* tok_idx, int32_t* pos_of, hipStream_t s, int t_sh, const ChunkList* lists,
                            int n_lists, bool* lists_built, bool* shared_built, const float* logits,
                            int32_t* sel_out, float* wsel_out, const RowQuant* rq) {
    if (lists_built) *lists_built = false;
    if (shared_built) *shared_built = false;
    if (E > 1024 || n_lists < 0 || n_lists > 2) return hipErrorInvalidValue;
    if (logits && (!moe_group_routes(T, topk, E) || !sel_out || !wsel_out)) return hipErrorInvalidValue;
    const RowQuant rq0{};
    if (rq && rq->A &&
        (!logits || rq->M > 16 || rq->K <= 0 || rq->K > 2048 || rq->K % 8 || (uintptr_t)rq->A % 16 || rq->lda % 4 ||
         (uintptr_t)rq->q % 8 || (rq->gsum && rq->K % 32)))
        return hipErrorInvalidValue;
    if (E <= kGroupFastE) {
        const ChunkList none{0, nullptr, nullptr};
        moe_group_small_kernel<<<1, 1024, 0, s>>>(sel, T * topk, E, topk, grp_off, tok_idx, pos_of, t_sh,
                                                  n_lists > 0 ? lists[0] : none, n_lists > 1 ? lists[1] : none,
                                                  n_lists, logits, sel_out, wsel_out, rq ? *rq : rq0);
        if (lists_built) *lists_built = n_lists > 0;
        if (shared_built) *shared_built = true;
        return hipGetLastError();
    }
    moe_group_kernel<<<1, 1024, 0, s>>>(sel, T * topk, E, topk, grp_off, tok_idx, pos_of);
    return hipGetLastError();
}

// SwiGLU as main.cpp:3164-3165: h = (g / (1 + exp(-g))) * u.
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                     float* __restrict__ h, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float gv = g[i];
        h[i] = (gv / (1.0f + expf(-gv))) * u[i];
    }
}

hipError_t launch_swiglu(const float* g, const float* u, float* h, int64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    swiglu_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(g, u, h, n);
    return hipGetLastError();
}

// Weighted combine in the reference's order (main.cpp:3166-3193): routed
// experts j = 0..topk-1 by descending logit, then the shared expert.
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ D, const int32_t* __restrict__ pos_of,
                                                          const float* __restrict__ wsel, int topk, int H,
                                                          const float* __restrict__ Dsh,
                                                          const float* __restrict__ shared_w,
                                                          float* __restrict__ out) {
    const int t = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= H) return;
    float acc = 0.0f;
    for (int j = 0; j < topk; j++)
        acc += wsel[t * topk + j] * D[(int64_t)pos_of[t * topk + j] * H + i];
    if (Dsh) acc += (shared_w ? shared_w[t] : 1.0f) * Dsh[(int64_t)t * H + i];
    out[(int64_t)t * H + i] = acc;
}

// The same with 4 values a thread (16-byte loads and stores; H % 4 == 0,
// 16-byte aligned rows).
__global__ __launch_bounds__(256) void moe_combine4_kernel(const float* __restrict__ D, const int32_t* __restrict__ pos_of,
                                                           const float* __restrict__ wsel, int topk, int H,
                                                           const float* __restrict__ Dsh,
                                                           const float* __restrict__ shared_w,
                                                           float* __restrict__ out) {
    const int t = blockIdx.y;
    const int i = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= H) return;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int j = 0; j < topk; j++) {
        const float w = wsel[t * topk + j];
        const float4 v = *(const float4*)(D + (int64_t)pos_of[t * topk + j] * H + i);
        acc.x += w * v.x; acc.y += w * v.y; acc.z += w * v.z; acc.w += w * v.w;
    }
    if (Dsh) {
        const float w = shared_w ? shared_w[t] : 1.0f;
        const float4 v = *(const float4*)(Dsh + (int64_t)t * H + i);
        acc.x += w * v.x; acc.y += w * v.y; acc.z += w * v.z; acc.w += w * v.w;
    }
    *(float4*)(out + (int64_t)t * H + i) = acc;
}

hipError_t launch_moe_combine(const float* D, const int32_t* pos_of, const float* wsel, int T,
                              int topk, int H, const float* Dsh, const float* shared_w, float* out,
                              hipStream_t s) {
    if (T == 0) return hipSuccess;
    const bool v4 = H % 4 == 0 && ((uintptr_t)D & 15u) == 0 && ((uintptr_t)out & 15u) == 0 &&
                    (!Dsh || ((uintptr_t)Dsh & 15u) == 0);
    if (v4) {
        moe_combine4_kernel<<<dim3((H / 4 + 255) / 256, T), 256, 0, s>>>(D, pos_of, wsel, topk, H, Dsh, shared_w, out);
        return hipGetLastError();
    }
    moe_combine_kernel<<<dim3((H + 255) / 256, T), 256, 0, s>>>(D, pos_of, wsel, topk, H, Dsh, shared_w, out);
    return hipGetLastError();
}

}  // namespace ggq
