// ggq_backend.h -- C++ adapter with the shape of ggnpu's Backend interface
// (include/ggnpu/backend.h:113-160 in the ggnpu tree) over the C ABI in
// ggq.h.  Header-only; link libggq_hip.so.
//
// The types below restate the hot-path slice of ggnpu's interface with the
// same names, field order and status values, so ggnpu's caller code
// (mul_mat_weight, src/cli/main.cpp:1367-1434) reads the same against it:
//   Status        backend.h:12-19
//   GgmlType      tensor.h:11-42 (the ids this backend accepts)
//   MulMatParams  backend.h:21-35
//   Backend       backend.h:113-160 (mul_mat_q, sync, is_available, name,
//                 last_error; the non-matmul operators are not part of this
//                 backend and report DEVICE_UNAVAILABLE, i.e. the reference's
//                 Status::NPU_UNAVAILABLE value)
// Inside ggnpu itself the adapter is a ggnpu::Backend subclass that forwards
// mul_mat_q to the same C calls and reports NPU_UNAVAILABLE for the other
// operators.
#pragma once

#include <cstdint>
#include <memory>
#include <string>

#include "ggq.h"

namespace ggq_backend {

enum class Status {
    OK = GGQ_OK,
    ERROR = GGQ_ERROR,
    NOT_FOUND = GGQ_NOT_FOUND,
    INVALID_PARAM = GGQ_INVALID_PARAM,
    DEVICE_UNAVAILABLE = GGQ_DEVICE_UNAVAILABLE,
    OUT_OF_MEMORY = GGQ_OUT_OF_MEMORY,
};

enum class GgmlType : uint32_t {
    F32 = 0,
    Q8_0 = GGQ_TYPE_Q8_0,
    Q4_K = GGQ_TYPE_Q4_K,
    Q5_K = GGQ_TYPE_Q5_K,
    Q6_K = GGQ_TYPE_Q6_K,
    IQ4_NL = GGQ_TYPE_IQ4_NL,
    IQ4_XS = GGQ_TYPE_IQ4_XS,
};

struct MulMatParams {
    const void* A;
    const void* B;
    void* C;
    int M;
    int N;
    int K;
    int lda;
    int ldb;
    int ldc;
    int32_t n_batches;
    const void* scales = nullptr;
    int n_weight_scales = 0;
    GgmlType B_type = GgmlType::F32;
};

class Backend {
public:
    virtual ~Backend() = default;
    virtual Status mul_mat_q(const MulMatParams& params) = 0;
    virtual void sync() = 0;
    virtual bool is_available() const = 0;
    virtual std::string name() const = 0;
    virtual Status last_error() const = 0;
};

// mul_mat_q on raw GGUF blocks with HBM-resident weights.  `act_mode`
// selects the activation treatment for every call: GGQ_ACT_F32 (CpuRef
// semantics, the default) or GGQ_ACT_Q8_ROW (the XDNA backend's per-row int8
// activations).
class HipBackend final : public Backend {
public:
    explicit HipBackend(int device = 0, int act_mode = GGQ_ACT_F32) : act_mode_(act_mode) {
        const int st = ggq_create(device, &ctx_);
        if (st != GGQ_OK) {
            ctx_ = nullptr;
            last_ = static_cast<Status>(st);
        }
    }
    ~HipBackend() override {
        if (ctx_) ggq_destroy(ctx_);
    }
    HipBackend(const HipBackend&) = delete;
    HipBackend& operator=(const HipBackend&) = delete;

    Status mul_mat_q(const MulMatParams& p) override {
        if (!ctx_) return last_ = Status::DEVICE_UNAVAILABLE;
        ggq_mul_mat_params c;
        c.A = p.A;
        c.B = p.B;
        c.C = p.C;
        c.M = p.M;
        c.N = p.N;
        c.K = p.K;
        c.lda = p.lda;
        c.ldb = p.ldb;
        c.ldc = p.ldc;
        c.n_batches = p.n_batches;
        c.scales = p.scales;
        c.n_weight_scales = p.n_weight_scales;
        c.B_type = static_cast<uint32_t>(p.B_type);
        return last_ = static_cast<Status>(ggq_mul_mat_q(ctx_, &c, act_mode_));
    }
    void sync() override {
        if (ctx_) last_ = static_cast<Status>(ggq_sync(ctx_));
    }
    bool is_available() const override { return ctx_ != nullptr; }
    std::string name() const override { return "hip_gfx950"; }
    Status last_error() const override { return last_; }
    // Detail of the last failure reported by the library.
    std::string last_error_message() const { return ctx_ ? ggq_last_error_message(ctx_) : "no device"; }
    ggq_ctx* handle() const { return ctx_; }

private:
    ggq_ctx* ctx_ = nullptr;
    int act_mode_;
    Status last_ = Status::OK;
};

// Factory in the style of create_cpu_ref_backend() (backend.h:162-165).
inline std::shared_ptr<Backend> create_hip_backend(int device = 0, int act_mode = GGQ_ACT_F32) {
    return std::make_shared<HipBackend>(device, act_mode);
}

}  // namespace ggq_backend
