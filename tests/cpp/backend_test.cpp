// Drives ggq_backend::HipBackend the way ggnpu's mul_mat_weight drives a
// Backend (src/cli/main.cpp:1408-1433): raw GGUF bytes in B, fp32 A/C,
// synchronous mul_mat_q, then sync().  Checked against the CPU oracle.
//   backend_test cpu   error paths without a device
//   backend_test gpu   parity on cuda:0 for Q4_K / Q6_K / Q8_0 / IQ4_XS
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "ggq_backend.h"
#include "ggq_oracle.h"

using namespace ggq_backend;

static int fails = 0;
#define CHECK(c, msg)                                              \
    do {                                                           \
        if (!(c)) {                                                \
            std::printf("FAIL %s (%s:%d)\n", msg, __FILE__, __LINE__); \
            fails++;                                               \
        }                                                          \
    } while (0)

static double rel_l2(const std::vector<float>& got, const std::vector<double>& ref) {
    double num = 0, den = 0;
    for (size_t i = 0; i < got.size(); i++) {
        num += (got[i] - ref[i]) * (got[i] - ref[i]);
        den += ref[i] * ref[i];
    }
    return std::sqrt(num / (den > 0 ? den : 1));
}

static int run_cpu() {
    HipBackend be(9999);
    CHECK(!be.is_available(), "no device 9999");
    MulMatParams p{};
    float a = 0, c = 0;
    unsigned char b[144] = {};
    p.A = &a; p.B = b; p.C = &c; p.M = 1; p.N = 1; p.K = 256; p.lda = 256; p.ldb = 256; p.ldc = 1;
    p.n_batches = 1; p.B_type = GgmlType::Q4_K;
    CHECK(be.mul_mat_q(p) == Status::DEVICE_UNAVAILABLE, "mul_mat_q without device");
    CHECK(be.last_error() == Status::DEVICE_UNAVAILABLE, "last_error");
    CHECK(be.name() == "hip_gfx950", "name");
    return fails;
}

static int run_gpu() {
    auto be = create_hip_backend(0);
    CHECK(be->is_available(), "device 0");
    std::mt19937 rng(7);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    const GgmlType types[] = {GgmlType::Q4_K, GgmlType::Q6_K, GgmlType::Q8_0, GgmlType::IQ4_XS};
    const int M = 2, N = 96, K = 1024;
    for (GgmlType t : types) {
        std::vector<float> w((size_t)N * K), A((size_t)M * K), C((size_t)M * N, NAN);
        for (auto& v : w) v = 0.02f * nd(rng);
        for (auto& v : A) v = nd(rng);
        std::vector<unsigned char> raw((size_t)ggq_row_bytes((uint32_t)t, K) * N);
        CHECK(ggq_encode((uint32_t)t, w.data(), N, K, raw.data()) == GGQ_OK, "encode");
        MulMatParams p{};
        p.A = A.data(); p.B = raw.data(); p.C = C.data();
        p.M = M; p.N = N; p.K = K; p.lda = K; p.ldb = K; p.ldc = N; p.n_batches = 1; p.B_type = t;
        CHECK(be->mul_mat_q(p) == Status::OK, "mul_mat_q");
        be->sync();
        CHECK(be->last_error() == Status::OK, "sync");
        std::vector<double> ref((size_t)M * N);
        orc_mul_mat_f64((uint32_t)t, raw.data(), N, K, A.data(), K, M, ORC_ACT_F32, ref.data(), N);
        const double err = rel_l2(C, ref);
        std::printf("type %u rel_l2 %.3e\n", (unsigned)t, err);
        CHECK(err < 1e-4, "parity");
        // reference error contract: null pointers -> INVALID_PARAM
        MulMatParams bad = p;
        bad.C = nullptr;
        CHECK(be->mul_mat_q(bad) == Status::INVALID_PARAM, "null C");
    }
    return fails;
}

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::strcmp(argv[1], "gpu") == 0;
    const int f = gpu ? run_gpu() : run_cpu();
    std::printf(f ? "FAILED %d\n" : "OK\n", f);
    return f ? 1 : 0;
}
