// ref_shim.cpp -- extern "C" entry points over the ggnpu reference sources,
// compiled (by oracle/Makefile) straight from /root/reference into
// oracle/_ref/libggnpu_ref.so.  TEST INFRASTRUCTURE ONLY: used by
// tests/golden/make_golden.py and the CPU tests in this container to check the
// oracle restatement against the reference's own code.  No reference source is
// copied; this file only calls the reference's public functions.
#include <cstdint>
#include <cstring>
#include <vector>
#include "backend.h"
#include "tensor.h"
#include "quant/kquant.h"
#include "quant/q8_0.h"
#include "quant/iq4_nl.h"
#include "quant/iq4_xs.h"
#include "quant/quant.h"

using namespace ggnpu;

extern "C" {

float ref_fp16_to_f32(uint16_t h) { return fp16_to_f32(h); }

void ref_q4k_scale_min(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    q4k_get_scale_min(j, q, sc, m);
}

// Dequantize n consecutive blocks of the given ggml type id.
int ref_dequant_blocks(uint32_t type, const uint8_t* raw, int64_t n, float* out) {
    const size_t bs = ggml_type_size(static_cast<GgmlType>(type));
    const size_t be = ggml_blck_size(static_cast<GgmlType>(type));
    for (int64_t i = 0; i < n; i++) {
        const uint8_t* b = raw + i * bs;
        float* o = out + i * be;
        switch (static_cast<GgmlType>(type)) {
        case GgmlType::Q4_K: dequant_q4_k_block(b, o); break;
        case GgmlType::Q5_K: dequant_q5_k_block(b, o); break;
        case GgmlType::Q6_K: dequant_q6_k_block(b, o); break;
        case GgmlType::Q8_0: dequant_q8_0_block(b, o); break;
        case GgmlType::IQ4_NL: dequant_iq4_nl_block(b, o); break;
        case GgmlType::IQ4_XS: dequant_iq4_xs_block(b, o); break;
        default: return 3;
        }
    }
    return 0;
}

uint64_t ref_type_size(uint32_t type) { return ggml_type_size(static_cast<GgmlType>(type)); }
uint64_t ref_blck_size(uint32_t type) { return ggml_blck_size(static_cast<GgmlType>(type)); }

// Per-row int8 weight requant (decode_*_for_npu): outputs [N][K] int8 + [N] scales.
int ref_decode_for_npu(uint32_t type, const uint8_t* raw, uint64_t size, int64_t N, int64_t K,
                       int8_t* q, float* scales) {
    std::vector<int8_t> qo;
    std::vector<float> so;
    decode_for_npu(static_cast<GgmlType>(type), raw, size, N, K, qo, so);
    if (qo.size() != static_cast<size_t>(N * K) || so.size() != static_cast<size_t>(N)) return 1;
    std::memcpy(q, qo.data(), qo.size());
    std::memcpy(scales, so.data(), so.size() * sizeof(float));
    return 0;
}

// CpuRefBackend::mul_mat_q on raw blocks (valid for Q4_K / Q6_K).
int ref_cpuref_mul_mat(uint32_t type, const void* W, int N, int K, const float* A, int M, float* C) {
    auto be = create_cpu_ref_backend();
    MulMatParams p;
    p.A = A; p.B = W; p.C = C; p.M = M; p.N = N; p.K = K;
    p.lda = K; p.ldb = K; p.ldc = N; p.n_batches = 1;
    p.B_type = static_cast<GgmlType>(type);
    return static_cast<int>(be->mul_mat_q(p));
}

// The dequantize-row + fp32 dot loop the CLI runs where no backend takes the
// weight type (main.cpp:317-326, :1380-1386): whole row through the
// reference's block decoders, then one running fp32 sum over k per row of A.
int ref_rowdot_mul_mat(uint32_t type, const uint8_t* W, int N, int K, const float* A, int M, float* C) {
    const size_t be = ggml_blck_size(static_cast<GgmlType>(type));
    const size_t bs = ggml_type_size(static_cast<GgmlType>(type));
    if (be == 0 || K % be) return 3;
    const size_t nb = K / be;
    std::vector<float> row(static_cast<size_t>(K));
    for (int n = 0; n < N; n++) {
        int st = ref_dequant_blocks(type, W + static_cast<size_t>(n) * nb * bs, static_cast<int64_t>(nb), row.data());
        if (st) return st;
        for (int m = 0; m < M; m++) {
            const float* a = A + static_cast<size_t>(m) * K;
            float acc = 0.0f;
            for (int k = 0; k < K; k++) acc += a[k] * row[k];
            C[static_cast<size_t>(m) * N + n] = acc;
        }
    }
    return 0;
}

// CpuRefBackend::rms_norm (cpu_ref.cpp:139-156) and silu (:200-209).
int ref_rms_norm(const float* x, int n, const float* w, float eps, float* out) {
    auto be = create_cpu_ref_backend();
    RmsNormParams p;
    p.input = x; p.output = out; p.size = n; p.eps = eps; p.weight = w;
    return static_cast<int>(be->rms_norm(p));
}

int ref_silu(const float* x, int n, float* out) {
    auto be = create_cpu_ref_backend();
    SiluParams p;
    p.input = x; p.output = out; p.size = n;
    return static_cast<int>(be->silu(p));
}

// CpuRefBackend::flash_attn (cpu_ref.cpp:223-280) for one query row.
int ref_flash_attn(const float* Q, const float* K, const float* V, int n_head, int hd, int64_t ctx_len,
                   int64_t query_pos, float* out) {
    auto be = create_cpu_ref_backend();
    AttnParams p;
    p.Q = Q; p.K = K; p.V = V; p.output = out;
    p.batch_size = 1; p.n_head = n_head; p.head_dim = hd; p.ctx_len = ctx_len;
    p.query_pos = query_pos; p.freq_factors = nullptr;
    return static_cast<int>(be->flash_attn(p));
}

}  // extern "C"
