// ggq_api.cpp -- implementation of the C ABI in include/ggq.h.
//
// Control plane of the backend: validates shapes, owns HBM-resident raw
// weights and a growable workspace, and queues the kernels of
// ggq_kernels.hip on a HIP stream.  Replaces the host tile loop of the XDNA
// backend (src/backends/amd_xdna/amd_xdna.cpp:491-952): there is no host
// re-quantization, no tiling on the host and no per-tile readback; one
// launch covers a whole matmul.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <set>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/ggq.h"
#include "ggq_formats.h"
#include "ggq_launch.h"

static_assert(ggq::kScratchBytes == GGQ_NOALLOC_SCRATCH_BYTES, "scratch size of the header and the library differ");

struct ggq_weight {
    void* dev = nullptr;
    uint32_t type = 0;
    int64_t N = 0, K = 0;
    size_t bytes = 0;
};

namespace {

struct Buffer {
    void* ptr = nullptr;
    size_t size = 0;
};

// Device memory a matmul may use beyond its inputs and outputs.
struct Work {
    Buffer ws;    // activation quantization, MoE intermediates
    Buffer part;  // GEMM split-K partial tiles
};

}  // namespace

struct ggq_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::recursive_mutex mu;
    int last = GGQ_OK;
    std::string msg;
    std::map<std::tuple<const void*, uint32_t, int64_t, int64_t>, ggq_weight*> cache;
    std::set<ggq_weight*> weights;
    Work dev;   // workspace of the *_dev entry points
    Work host;  // workspace of the synchronous host-pointer entry points (never
                // shared with device calls that may still run on other streams)
    Buffer io;  // staging of host A / C for the synchronous entry points
    Buffer logits;  // vocab projection output when the caller does not keep it
    Buffer attn;  // attention chunk partials
    Buffer pin;   // pinned host staging of A and C for the synchronous host-pointer entry points
    uint32_t* done = nullptr;  // pinned completion word of the synchronous entry points
    uint32_t done_seq = 0;
    std::vector<void*> retired;  // outgrown device buffers, freed by ggq_destroy
    ggq_moe_trace trace{};       // intermediates of the last MoE call
    bool trace_rows = false;     // MoE calls keep their fp32 SwiGLU rows
};

namespace {

using ggq::block_bytes;
using ggq::block_elems;

int set_status(ggq_ctx* c, int st, const char* fmt = nullptr, ...) {
    c->last = st;
    c->msg.clear();
    if (fmt) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        c->msg = buf;
    }
    return st;
}

int hip_status(ggq_ctx* c, hipError_t e, const char* what) {
    if (e == hipSuccess) return set_status(c, GGQ_OK);
    const int st = e == hipErrorOutOfMemory ? GGQ_OUT_OF_MEMORY : GGQ_ERROR;
    return set_status(c, st, "%s: %s", what, hipGetErrorString(e));
}

// Grows `b` to at least `need` bytes for work queued on `s`.  An outgrown
// allocation is not freed before ggq_destroy: work queued earlier and HIP
// graphs captured earlier keep using its address.  Growing while `s` is being
// captured is refused (the allocation would not be part of the graph's
// ordering); one call outside the capture, or ggq_reserve, sizes it first.
int grow(ggq_ctx* c, Buffer& b, size_t need, hipStream_t s, const char* what) {
    if (b.size >= need) return GGQ_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
        return set_status(c, GGQ_ERROR,
                          "%s: %zu bytes of workspace needed while the stream is being captured (%zu reserved); "
                          "call ggq_reserve or run the call once before the capture",
                          what, need, b.size);
    const size_t sz = std::max(need + 4096, 2 * b.size);
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, sz);
    if (e != hipSuccess) return hip_status(c, e, what);
    if (b.ptr) c->retired.push_back(b.ptr);
    b.ptr = p;
    b.size = sz;
    return GGQ_OK;
}

inline size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// Where a call's scratch memory comes from: the growable buffers of a Work,
// or one fixed region (activation workspace first, split-K partials after).
struct Arena {
    ggq_ctx* c;
    Work* w;
    char* fixed;
    size_t cap;
    hipStream_t s;
    int get(size_t ws_bytes, size_t part_bytes, void** ws, float** part, const char* what) {
        *ws = nullptr;
        *part = nullptr;
        if (w) {
            int st;
            if (ws_bytes && (st = grow(c, w->ws, ws_bytes, s, what)) != GGQ_OK) return st;
            if (part_bytes && (st = grow(c, w->part, part_bytes, s, what)) != GGQ_OK) return st;
            *ws = w->ws.ptr;
            *part = part_bytes ? (float*)w->part.ptr : nullptr;
            return GGQ_OK;
        }
        const size_t off = align256(ws_bytes);
        if (off + part_bytes > cap)
            return set_status(c, GGQ_INVALID_PARAM,
                              "%s: the call needs %zu bytes of scratch; the allocation-free entry point has %zu",
                              what, off + part_bytes, cap);
        *ws = fixed;
        *part = part_bytes ? (float*)(fixed + off) : nullptr;
        return GGQ_OK;
    }
};

Arena dev_arena(ggq_ctx* c, hipStream_t s) { return Arena{c, &c->dev, nullptr, 0, s}; }

// Split-K partial bytes of a GEMM plan (0 when the plan does not split).
size_t gemm_part_bytes(const ggq::GemmPlan& pl) { return pl.splits <= 1 ? 0 : sizeof(float) * pl.part_floats; }

// Stream of a device-pointer call: the caller's, or the HIP default (null)
// stream for NULL, as HIP APIs treat a null stream argument.  (The context's
// own stream is non-blocking and is used only inside the synchronous
// entry points, which wait for it before returning.)
hipStream_t pick_stream(ggq_ctx*, void* s) { return (hipStream_t)s; }

int check_matmul_shape(ggq_ctx* c, uint32_t type, int64_t N, int64_t K, int M, int lda, int ldc,
                       int act_mode) {
    if (!ggq::supported(type)) return set_status(c, GGQ_INVALID_PARAM, "unsupported weight type %u", type);
    if (N <= 0 || K <= 0 || M < 0) return set_status(c, GGQ_INVALID_PARAM, "bad shape N=%lld K=%lld M=%d", (long long)N, (long long)K, M);
    if (K % block_elems(type)) return set_status(c, GGQ_INVALID_PARAM, "K=%lld not a multiple of the block size %d", (long long)K, block_elems(type));
    if (N > INT32_MAX || K > ggq::kGemvMaxK) return set_status(c, GGQ_INVALID_PARAM, "K=%lld exceeds the supported maximum %d", (long long)K, ggq::kGemvMaxK);
    if (lda < K || ldc < N) return set_status(c, GGQ_INVALID_PARAM, "lda/ldc smaller than K/N");
    if (N * ggq::row_bytes(type, K) > (int64_t)0xFFFFFFFF)
        return set_status(c, GGQ_INVALID_PARAM, "weight matrix of %lld bytes: at most 4 GiB per matrix",
                          (long long)(N * ggq::row_bytes(type, K)));
    if (act_mode < GGQ_ACT_F32 || act_mode > GGQ_ACT_Q8_BLOCK32) return set_status(c, GGQ_INVALID_PARAM, "bad act_mode %d", act_mode);
    return GGQ_OK;
}

// Queues C = A . W^T with the requested activation treatment.
int mul_mat_queue(ggq_ctx* c, Arena& ar, const void* W, uint32_t type, int64_t N, int64_t K, const float* A,
                  int lda, float* C, int ldc, int M, int act_mode, hipStream_t s) {
    if (M == 0) return set_status(c, GGQ_OK);
    hipError_t e;
    int st;
    ggq::GemvProblem g{};
    g.type = type;
    g.W = W;
    g.N = (int)N;
    g.K = (int)K;
    g.Y = C;
    g.ldy = ldc;
    g.M = M;
    g.groups = 1;
    if (act_mode == GGQ_ACT_F32) {
        g.X = A;
        g.ldx = lda;
        return hip_status(c, ggq::launch_gemv(g, s), "gemv");
    }
    if (act_mode == GGQ_ACT_Q8_ROW && M <= 8) {
        // Decode-sized: one row below 16 MB of weights on the LDS-staged fp32
        // kernel with the row quantized in its staging; otherwise the int8
        // matrix-core GEMV quantizes the rows itself.
        g.X = A;
        g.ldx = lda;
        if (ggq::gemv_q8row_eligible(&g, 1)) {
            g.q8row = 1;
            return hip_status(c, ggq::launch_gemv(g, s), "gemv_q8row");
        }
        if (ggq::i8_gemv_eligible(&g, 1, 1))
            return hip_status(c, ggq::launch_i8_gemv(&g, 1, 1, nullptr, nullptr, s), "gemv_i8");
    }
    if (act_mode == GGQ_ACT_Q8_ROW && M > 8 && ggq::gemm_panel_eligible(type, (int)K, M, A, lda)) {
        // quantized per row inside the GEMM (no workspace)
        const ggq::GemmDesc gd{W, C, (int)N, ldc};
        return hip_status(c, ggq::launch_gemm_panel(type, &gd, 1, (int)K, A, lda, nullptr, nullptr, M, s), "gemm_panel");
    }
    const size_t q_off = 0;
    const size_t s_off = align256(q_off + (size_t)M * K);
    const size_t x_off = align256(s_off + sizeof(float) * (size_t)M * (K / 32));
    const bool use_gemm = act_mode == GGQ_ACT_Q8_ROW && M > 8;
    const size_t need = use_gemm ? x_off : align256(x_off + sizeof(float) * (size_t)M * K);
    const int n32 = (int)N;
    const size_t part_bytes = use_gemm ? gemm_part_bytes(ggq::plan_gemm_i8(type, &n32, 1, (int)K, M)) : 0;
    void* ws;
    float* part;
    if ((st = ar.get(need, part_bytes, &ws, &part, "workspace")) != GGQ_OK) return st;
    int8_t* q = (int8_t*)ws + q_off;
    float* sc = (float*)((char*)ws + s_off);
    float* xe = (float*)((char*)ws + x_off);
    if (use_gemm) {
        if ((e = ggq::launch_quant_act(A, lda, M, (int)K, act_mode, q, sc, nullptr, s)) != hipSuccess)
            return hip_status(c, e, "quant_act");
        return hip_status(c, ggq::launch_gemm_i8(type, W, (int)N, (int)K, q, sc, M, C, ldc, part, s), "gemm_i8");
    }
    if ((e = ggq::launch_quant_act(A, lda, M, (int)K, act_mode, nullptr, nullptr, xe, s)) != hipSuccess)
        return hip_status(c, e, "quant_act");
    g.X = xe;
    g.ldx = (int)K;
    return hip_status(c, ggq::launch_gemv(g, s), "gemv");
}

// C = sa * (qa . W^T) from activations already quantized per row.
int mul_mat_q8_queue(ggq_ctx* c, Arena& ar, const void* W, uint32_t type, int64_t N, int64_t K, const int8_t* qa,
                     const float* sa, int M, float* C, int ldc, hipStream_t s) {
    if (M == 0) return set_status(c, GGQ_OK);
    hipError_t e;
    int st;
    void* ws;
    float* part;
    if (M > 8 && ggq::gemm_panel_eligible(type, (int)K, M, nullptr, 0)) {
        const ggq::GemmDesc gd{W, C, (int)N, ldc};
        return hip_status(c, ggq::launch_gemm_panel(type, &gd, 1, (int)K, nullptr, 0, qa, sa, M, s), "gemm_panel");
    }
    if (M > 8) {
        const int n32 = (int)N;
        const size_t part_bytes = gemm_part_bytes(ggq::plan_gemm_i8(type, &n32, 1, (int)K, M));
        if ((st = ar.get(0, part_bytes, &ws, &part, "workspace")) != GGQ_OK) return st;
        return hip_status(c, ggq::launch_gemm_i8(type, W, (int)N, (int)K, qa, sa, M, C, ldc, part, s), "gemm_i8");
    }
    ggq::GemvProblem g{};
    g.type = type;
    g.W = W;
    g.N = (int)N;
    g.K = (int)K;
    g.Y = C;
    g.ldy = ldc;
    g.M = M;
    g.groups = 1;
    if (ggq::i8_gemv_eligible(&g, 1, 2))
        return hip_status(c, ggq::launch_i8_gemv(&g, 1, 2, qa, sa, s), "gemv_i8");
    if ((st = ar.get(sizeof(float) * (size_t)M * K, 0, &ws, &part, "workspace")) != GGQ_OK) return st;
    float* xe = (float*)ws;
    if ((e = ggq::launch_dequant_act(qa, sa, M, (int)K, xe, s)) != hipSuccess) return hip_status(c, e, "dequant_act");
    g.X = xe;
    g.ldx = (int)K;
    return hip_status(c, ggq::launch_gemv(g, s), "gemv");
}

ggq_weight* upload(ggq_ctx* c, const void* raw, uint32_t type, int64_t N, int64_t K, int* st) {
    const size_t bytes = (size_t)N * (size_t)ggq::row_bytes(type, K);
    ggq_weight* w = new (std::nothrow) ggq_weight;
    if (!w) { *st = set_status(c, GGQ_OUT_OF_MEMORY, "host allocation"); return nullptr; }
    hipError_t e = hipMalloc(&w->dev, bytes + ggq::kWeightPad);
    if (e == hipSuccess) e = hipMemsetAsync((char*)w->dev + bytes, 0, ggq::kWeightPad, c->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(w->dev, raw, bytes, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        if (w->dev) hipFree(w->dev);
        delete w;
        *st = hip_status(c, e, "weight upload");
        return nullptr;
    }
    w->type = type;
    w->N = N;
    w->K = K;
    w->bytes = bytes;
    c->weights.insert(w);
    *st = set_status(c, GGQ_OK);
    return w;
}

// Synchronous host-pointer matmul against a resident weight.
// Pinned host buffer of at least `need` bytes (grown by reallocation;
// hipHostFree waits for the device).
hipError_t ensure_pinned(Buffer& b, size_t need) {
    if (b.size >= need) return hipSuccess;
    if (b.ptr) hipHostFree(b.ptr);
    b.ptr = nullptr;
    b.size = 0;
    const size_t sz = need + need / 4 + 4096;
    // coherent: the device's stores of C reach host memory without being
    // held in its caches
    hipError_t e = hipHostMalloc(&b.ptr, sz, hipHostMallocCoherent);
    if (e != hipSuccess) return e;
    b.size = sz;
    return hipSuccess;
}

// Waits for everything queued on the context's stream.  A one-lane kernel
// queued last stores a sequence number into pinned memory, which the host
// polls: at decode sizes a stream synchronization costs ~3 us more per
// call (its wake-up).  After 200 us of polling the wait falls back to the
// stream synchronization, which also reports a failed launch or fault.
hipError_t wait_stream(ggq_ctx* c) {
    hipError_t e;
    if (!c->done) {
        if ((e = hipHostMalloc((void**)&c->done, 256, hipHostMallocCoherent)) != hipSuccess) {
            c->done = nullptr;
            return e;
        }
        __atomic_store_n(c->done, 0u, __ATOMIC_RELAXED);
    }
    const uint32_t v = ++c->done_seq;
    if ((e = ggq::launch_host_flag(c->done, v, c->stream)) != hipSuccess) return e;
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0;; i++) {
        if (__atomic_load_n(c->done, __ATOMIC_ACQUIRE) == v) return hipSuccess;
        if ((i & 255) == 255 && std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(200)) break;
    }
    return hipStreamSynchronize(c->stream);
}

// Synchronous matmul with host A and C: the caller's rows are packed into a
// pinned staging buffer that a copy kernel reads (and the result is written
// back the same way).  Copies from pageable memory go through the runtime's
// own staging and DMA-engine copies have a fixed latency; both measured
// slower than a copy kernel for the small vectors of a decode step.
int mul_mat_host(ggq_ctx* c, const ggq_weight* w, const float* A, int lda, float* C, int ldc, int M,
                 int act_mode) {
    int st = check_matmul_shape(c, w->type, w->N, w->K, M, lda, ldc, act_mode);
    if (st != GGQ_OK) return st;
    if (M == 0) return set_status(c, GGQ_OK);
    const size_t a_bytes = sizeof(float) * (size_t)M * w->K;
    const size_t c_bytes = sizeof(float) * (size_t)M * w->N;
    if ((st = grow(c, c->io, a_bytes, c->stream, "io buffer")) != GGQ_OK) return st;
    hipError_t e;
    if ((e = ensure_pinned(c->pin, align256(a_bytes) + c_bytes)) != hipSuccess) return hip_status(c, e, "pinned buffer");
    float* dA = (float*)c->io.ptr;
    float* hA = (float*)c->pin.ptr;
    float* hC = (float*)((char*)c->pin.ptr + align256(a_bytes));
    for (int m = 0; m < M; m++) memcpy(hA + (size_t)m * w->K, A + (size_t)m * lda, sizeof(float) * w->K);
    // A is read by every workgroup, so it is copied to HBM first; C is
    // written once per element, straight into the pinned buffer.
    e = ggq::launch_copy_bytes(dA, hA, a_bytes, c->stream);
    if (e != hipSuccess) return hip_status(c, e, "copy A");
    Arena ar{c, &c->host, nullptr, 0, c->stream};
    st = mul_mat_queue(c, ar, w->dev, w->type, w->N, w->K, dA, (int)w->K, hC, (int)w->N, M, act_mode, c->stream);
    if (st != GGQ_OK) return st;
    if ((e = wait_stream(c)) != hipSuccess) return hip_status(c, e, "sync");
    for (int m = 0; m < M; m++) memcpy(C + (size_t)m * ldc, hC + (size_t)m * w->N, sizeof(float) * w->N);
    return set_status(c, GGQ_OK);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Last use of a device's fixed scratch region by ggq_mul_mat_noalloc_dev
// (eager calls; work queued under graph capture is not tracked): the stream
// it was queued on and an event recorded after it.  Process-wide, like the
// region itself.
struct ScratchGate {
    std::mutex mu;
    hipStream_t stream = nullptr;
    hipEvent_t ev = nullptr;
};
ScratchGate& scratch_gate(int device) {
    static ScratchGate gates[64];
    return gates[device & 63];
}

}  // namespace

#define GGQ_GUARD(ctx)                                   \
    if (!(ctx)) return GGQ_INVALID_PARAM;                \
    std::lock_guard<std::recursive_mutex> lock_((ctx)->mu); \
    hipSetDevice((ctx)->device);                         \
    try {
#define GGQ_END(ctx)                                                             \
    }                                                                           \
    catch (const std::bad_alloc&) {                                             \
        return set_status(ctx, GGQ_OUT_OF_MEMORY, "host allocation failed");   \
    }                                                                           \
    catch (...) {                                                               \
        return set_status(ctx, GGQ_ERROR, "internal error");                   \
    }                                                                           \
    return set_status(ctx, GGQ_ERROR, "unreachable");

extern "C" {

int ggq_create(int device, ggq_ctx** out) {
    if (!out) return GGQ_INVALID_PARAM;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return GGQ_DEVICE_UNAVAILABLE;
    ggq_ctx* c = new (std::nothrow) ggq_ctx;
    if (!c) return GGQ_OUT_OF_MEMORY;
    c->device = device;
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return GGQ_DEVICE_UNAVAILABLE;
    }
    *out = c;
    return GGQ_OK;
}

void ggq_destroy(ggq_ctx* c) {
    if (!c) return;
    hipSetDevice(c->device);
    hipDeviceSynchronize();
    for (ggq_weight* w : c->weights) {
        hipFree(w->dev);
        delete w;
    }
    for (Buffer* b : {&c->dev.ws, &c->dev.part, &c->host.ws, &c->host.part})
        if (b->ptr) hipFree(b->ptr);
    for (void* p : c->retired) hipFree(p);
    if (c->io.ptr) hipFree(c->io.ptr);
    if (c->logits.ptr) hipFree(c->logits.ptr);
    if (c->attn.ptr) hipFree(c->attn.ptr);
    if (c->pin.ptr) hipHostFree(c->pin.ptr);
    if (c->done) hipHostFree(c->done);
    hipStreamDestroy(c->stream);
    delete c;
}

int ggq_last_error(const ggq_ctx* c) { return c ? c->last : GGQ_INVALID_PARAM; }
const char* ggq_last_error_message(const ggq_ctx* c) { return c ? c->msg.c_str() : "null context"; }
const char* ggq_name(const ggq_ctx*) { return "hip_gfx950"; }
int ggq_is_available(const ggq_ctx* c) { return c != nullptr; }

int ggq_sync(ggq_ctx* c) {
    GGQ_GUARD(c)
    return hip_status(c, hipDeviceSynchronize(), "sync");  // every stream the calls used
    GGQ_END(c)
}

int64_t ggq_row_bytes(uint32_t type, int64_t K) {
    if (!ggq::supported(type) || K <= 0 || K % block_elems(type)) return 0;
    return ggq::row_bytes(type, K);
}

int ggq_weight_upload(ggq_ctx* c, const void* raw, uint32_t type, int64_t N, int64_t K, ggq_weight** out) {
    GGQ_GUARD(c)
    if (!raw || !out) return set_status(c, GGQ_INVALID_PARAM, "null pointer");
    *out = nullptr;
    int st = check_matmul_shape(c, type, N, K, 0, (int)K, (int)N, GGQ_ACT_F32);
    if (st != GGQ_OK) return st;
    *out = upload(c, raw, type, N, K, &st);
    return st;
    GGQ_END(c)
}

int ggq_weight_free(ggq_ctx* c, ggq_weight* w) {
    GGQ_GUARD(c)
    if (!w || !c->weights.count(w)) return set_status(c, GGQ_INVALID_PARAM, "unknown weight");
    hipError_t e = hipStreamSynchronize(c->stream);
    for (auto it = c->cache.begin(); it != c->cache.end();)
        it = it->second == w ? c->cache.erase(it) : std::next(it);
    c->weights.erase(w);
    hipFree(w->dev);
    delete w;
    return hip_status(c, e, "weight free");
    GGQ_END(c)
}

const void* ggq_weight_device_ptr(const ggq_weight* w) { return w ? w->dev : nullptr; }

int ggq_mul_mat(ggq_ctx* c, const ggq_weight* w, const float* A, int lda, float* C, int ldc, int M,
                int act_mode) {
    GGQ_GUARD(c)
    if (!w || !c->weights.count(const_cast<ggq_weight*>(w))) return set_status(c, GGQ_INVALID_PARAM, "unknown weight");
    if (!A || !C) return set_status(c, GGQ_INVALID_PARAM, "null A/C");
    return mul_mat_host(c, w, A, lda ? lda : (int)w->K, C, ldc ? ldc : (int)w->N, M, act_mode);
    GGQ_END(c)
}

int ggq_mul_mat_q(ggq_ctx* c, const ggq_mul_mat_params* p, int act_mode) {
    GGQ_GUARD(c)
    // Null A/B/C -> INVALID_PARAM, as cpu_ref.cpp:26 and amd_xdna.cpp:492-495.
    if (!p || !p->A || !p->B || !p->C) return set_status(c, GGQ_INVALID_PARAM, "null A/B/C");
    if (p->scales || p->n_weight_scales)
        return set_status(c, GGQ_INVALID_PARAM, "re-quantized weight scales are not used by this backend");
    const int lda = p->lda ? p->lda : p->K, ldc = p->ldc ? p->ldc : p->N;
    int st = check_matmul_shape(c, p->B_type, p->N, p->K, p->M, lda, ldc, act_mode);
    if (st != GGQ_OK) return st;
    const auto key = std::make_tuple(p->B, p->B_type, (int64_t)p->N, (int64_t)p->K);
    auto it = c->cache.find(key);
    ggq_weight* w;
    if (it != c->cache.end()) {
        w = it->second;
    } else {
        w = upload(c, p->B, p->B_type, p->N, p->K, &st);
        if (!w) return st;
        c->cache[key] = w;
    }
    return mul_mat_host(c, w, (const float*)p->A, lda, (float*)p->C, ldc, p->M, act_mode);
    GGQ_END(c)
}

int ggq_mul_mat_dev(ggq_ctx* c, const void* W, uint32_t type, int64_t N, int64_t K, const float* A, int lda,
                    float* C, int ldc, int M, int act_mode, void* stream) {
    GGQ_GUARD(c)
    if (!W || !A || !C) return set_status(c, GGQ_INVALID_PARAM, "null W/A/C");
    if (!aligned16(W)) return set_status(c, GGQ_INVALID_PARAM, "W must be 16-byte aligned");
    int st = check_matmul_shape(c, type, N, K, M, lda, ldc, act_mode);
    if (st != GGQ_OK) return st;
    const hipStream_t s = pick_stream(c, stream);
    Arena ar = dev_arena(c, s);
    return mul_mat_queue(c, ar, W, type, N, K, A, lda, C, ldc, M, act_mode, s);
    GGQ_END(c)
}

int ggq_mul_mat_noalloc_dev(ggq_ctx* c, const void* W, uint32_t type, int64_t N, int64_t K, const float* A, int lda,
                            float* C, int ldc, int M, int act_mode, void* stream) {
    GGQ_GUARD(c)
    if (!W || !A || !C) return set_status(c, GGQ_INVALID_PARAM, "null W/A/C");
    if (!aligned16(W)) return set_status(c, GGQ_INVALID_PARAM, "W must be 16-byte aligned");
    int st = check_matmul_shape(c, type, N, K, M, lda, ldc, act_mode);
    if (st != GGQ_OK) return st;
    // This device's copy of the fixed region, looked up on the first call
    // made on the device (with it current); a failed lookup fails this
    // entry point only.
    void* scratch = nullptr;
    hipError_t e = ggq::scratch_device_ptr(c->device, &scratch);
    if (e != hipSuccess) return hip_status(c, e, "scratch region lookup");
    const hipStream_t s = pick_stream(c, stream);
    // One region per GPU: refuse a call that would overlap unfinished work
    // queued by an earlier call on another stream (any context or thread).
    ScratchGate& gate = scratch_gate(c->device);
    std::lock_guard<std::mutex> lock(gate.mu);
    if (gate.ev && gate.stream != s && hipEventQuery(gate.ev) == hipErrorNotReady)
        return set_status(c, GGQ_ERROR,
                          "the scratch region of device %d is still in use by a call queued on another stream; "
                          "order the calls (same stream, or wait for the earlier one)",
                          c->device);
    Arena ar{c, nullptr, (char*)scratch, ggq::kScratchBytes, s};
    st = mul_mat_queue(c, ar, W, type, N, K, A, lda, C, ldc, M, act_mode, s);
    if (st != GGQ_OK) return st;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone) {
        if (!gate.ev && (e = hipEventCreateWithFlags(&gate.ev, hipEventDisableTiming)) != hipSuccess)
            return hip_status(c, e, "scratch event");
        if ((e = hipEventRecord(gate.ev, s)) != hipSuccess) return hip_status(c, e, "scratch event");
        gate.stream = s;
    }
    return st;
    GGQ_END(c)
}

int ggq_reserve(ggq_ctx* c, int64_t bytes) {
    GGQ_GUARD(c)
    if (bytes < 0) return set_status(c, GGQ_INVALID_PARAM, "negative size");
    const size_t b = (size_t)bytes;
    int st;
    for (Buffer* buf : {&c->dev.ws, &c->dev.part, &c->logits, &c->attn})
        if ((st = grow(c, *buf, b, c->stream, "reserve")) != GGQ_OK) return st;
    return set_status(c, GGQ_OK);
    GGQ_END(c)
}

int ggq_logits_argmax_dev(ggq_ctx* c, const void* W, uint32_t type, int64_t N, int64_t K, const float* A, int M,
                          int act_mode, float* logits, int32_t* token, float* value, void* stream) {
    GGQ_GUARD(c)
    if (!W || !A || !token) return set_status(c, GGQ_INVALID_PARAM, "null W/A/token");
    if (!aligned16(W)) return set_status(c, GGQ_INVALID_PARAM, "W must be 16-byte aligned");
    int st = check_matmul_shape(c, type, N, K, M, (int)K, (int)N, act_mode);
    if (st != GGQ_OK) return st;
    if (M == 0) return set_status(c, GGQ_OK);
    // c->logits holds the argmax partials, then the logits if the caller
    // does not keep them.
    const size_t part_bytes = align256(ggq::argmax_workspace_bytes(M));
    const size_t need = part_bytes + (logits ? 0 : sizeof(float) * (size_t)M * (size_t)N);
    const hipStream_t s = pick_stream(c, stream);
    if ((st = grow(c, c->logits, need, s, "logits workspace")) != GGQ_OK) return st;
    float* L = logits ? logits : (float*)((char*)c->logits.ptr + part_bytes);
    Arena ar = dev_arena(c, s);
    st = mul_mat_queue(c, ar, W, type, N, K, A, (int)K, L, (int)N, M, act_mode, s);
    if (st != GGQ_OK) return st;
    return hip_status(c, ggq::launch_argmax_rows(L, M, (int)N, (int)N, token, value, c->logits.ptr, s), "argmax");
    GGQ_END(c)
}

int ggq_attention_decode_dev(ggq_ctx* c, const float* Q, const float* K, const float* V, int n_tok, int n_head,
                             int n_kv_head, int head_dim, int64_t ctx_len, int64_t pos0, float* out, void* stream) {
    GGQ_GUARD(c)
    if (n_tok < 0 || n_head < 1 || n_kv_head < 1 || n_head % n_kv_head)
        return set_status(c, GGQ_INVALID_PARAM, "need n_tok >= 0 and n_head a multiple of n_kv_head");
    const int g = n_head / n_kv_head;
    if (g != 1 && g != 2 && g != 4 && g != 8)
        return set_status(c, GGQ_INVALID_PARAM, "n_head / n_kv_head must be 1, 2, 4 or 8 (got %d)", g);
    if (head_dim != 64 && head_dim != 128)
        return set_status(c, GGQ_INVALID_PARAM, "head_dim must be 64 or 128 (got %d)", head_dim);
    if (ctx_len < 1 || pos0 < 0) return set_status(c, GGQ_INVALID_PARAM, "need ctx_len >= 1 and pos0 >= 0");
    if (n_tok == 0) return set_status(c, GGQ_OK);
    if (!Q || !K || !V || !out) return set_status(c, GGQ_INVALID_PARAM, "null Q/K/V/out");
    if (!aligned16(Q) || !aligned16(K) || !aligned16(V))
        return set_status(c, GGQ_INVALID_PARAM, "Q, K and V must be 16-byte aligned");
    const size_t need = sizeof(float) * ggq::attn_workspace_floats(n_tok, n_head, head_dim, ctx_len, pos0, n_kv_head);
    const hipStream_t s = pick_stream(c, stream);
    const int st = grow(c, c->attn, need, s, "attention workspace");
    if (st != GGQ_OK) return st;
    return hip_status(c, ggq::launch_attn_decode(Q, K, V, n_tok, n_head, n_kv_head, head_dim, ctx_len, pos0, out,
                                                 (float*)c->attn.ptr, s),
                      "attention");
    GGQ_END(c)
}

int ggq_mul_mat_q8_dev(ggq_ctx* c, const void* W, uint32_t type, int64_t N, int64_t K, const int8_t* qa,
                       const float* sa, int M, float* C, int ldc, void* stream) {
    GGQ_GUARD(c)
    if (!W || !qa || !sa || !C) return set_status(c, GGQ_INVALID_PARAM, "null W/qa/sa/C");
    if (!aligned16(W) || ((uintptr_t)qa & 15u)) return set_status(c, GGQ_INVALID_PARAM, "W and qa must be 16-byte aligned");
    int st = check_matmul_shape(c, type, N, K, M, (int)K, ldc, GGQ_ACT_Q8_ROW);
    if (st != GGQ_OK) return st;
    const hipStream_t s = pick_stream(c, stream);
    Arena ar = dev_arena(c, s);
    return mul_mat_q8_queue(c, ar, W, type, N, K, qa, sa, M, C, ldc, s);
    GGQ_END(c)
}

int ggq_mul_mat_q8_batch_dev(ggq_ctx* c, const ggq_gemm_desc* d, int n, uint32_t type, int64_t K, const int8_t* qa,
                             const float* sa, int M, void* stream) {
    GGQ_GUARD(c)
    if (!d || n < 1 || n > GGQ_MAX_GEMM_BATCH) return set_status(c, GGQ_INVALID_PARAM, "need 1..%d descriptors", GGQ_MAX_GEMM_BATCH);
    if (M < 0 || (M > 0 && (!qa || !sa))) return set_status(c, GGQ_INVALID_PARAM, "bad activations");
    if (!aligned16(qa) || K % 16) return set_status(c, GGQ_INVALID_PARAM, "qa must be 16-byte aligned with K %% 16 == 0");
    for (int i = 0; i < n; i++) {
        if (!d[i].W || !d[i].C) return set_status(c, GGQ_INVALID_PARAM, "null pointer in entry %d", i);
        if (!aligned16(d[i].W)) return set_status(c, GGQ_INVALID_PARAM, "W must be 16-byte aligned");
        const int st = check_matmul_shape(c, type, d[i].N, K, M, (int)K, d[i].ldc, GGQ_ACT_Q8_ROW);
        if (st != GGQ_OK) return st;
    }
    if (M == 0) return set_status(c, GGQ_OK);
    const hipStream_t s = pick_stream(c, stream);
    Arena ar = dev_arena(c, s);
    if (M <= 8 || type == GGQ_TYPE_Q6_K) {
        for (int i = 0; i < n; i++) {
            const int st = mul_mat_q8_queue(c, ar, d[i].W, type, d[i].N, K, qa, sa, M, d[i].C, d[i].ldc, s);
            if (st != GGQ_OK) return st;
        }
        return set_status(c, GGQ_OK);
    }
    ggq::GemmDesc gd[GGQ_MAX_GEMM_BATCH];
    int Ns[GGQ_MAX_GEMM_BATCH];
    for (int i = 0; i < n; i++) {
        gd[i] = ggq::GemmDesc{d[i].W, d[i].C, (int)d[i].N, d[i].ldc};
        Ns[i] = (int)d[i].N;
    }
    if (ggq::gemm_panel_eligible(type, (int)K, M, nullptr, 0))
        return hip_status(c, ggq::launch_gemm_panel(type, gd, n, (int)K, nullptr, 0, qa, sa, M, s), "gemm_panel batch");
    void* ws;
    float* part;
    const int st = ar.get(0, gemm_part_bytes(ggq::plan_gemm_i8(type, Ns, n, (int)K, M)), &ws, &part, "workspace");
    if (st != GGQ_OK) return st;
    return hip_status(c, ggq::launch_gemm_i8_multi(type, gd, n, (int)K, qa, sa, M, part, s), "gemm_i8 batch");
    GGQ_END(c)
}

int ggq_mul_mat_batch_rows_dev(ggq_ctx* c, const ggq_gemv_desc* d, int n, int M, void* stream) {
    GGQ_GUARD(c)
    if (!d || n < 1 || n > GGQ_MAX_BATCH) return set_status(c, GGQ_INVALID_PARAM, "need 1..%d descriptors", GGQ_MAX_BATCH);
    if (M < 0 || M > GGQ_MAX_BATCH_ROWS) return set_status(c, GGQ_INVALID_PARAM, "M=%d outside 0..%d", M, GGQ_MAX_BATCH_ROWS);
    ggq::GemvProblem ps[GGQ_MAX_BATCH];
    for (int i = 0; i < n; i++) {
        if (!d[i].W || !d[i].A || !d[i].C) return set_status(c, GGQ_INVALID_PARAM, "null pointer in entry %d", i);
        if (!aligned16(d[i].W)) return set_status(c, GGQ_INVALID_PARAM, "W must be 16-byte aligned");
        int st = check_matmul_shape(c, d[i].type, d[i].N, d[i].K, M, (int)d[i].K, (int)d[i].N, GGQ_ACT_F32);
        if (st != GGQ_OK) return st;
        ps[i] = ggq::GemvProblem{};
        ps[i].type = d[i].type;
        ps[i].W = d[i].W;
        ps[i].N = (int)d[i].N;
        ps[i].K = (int)d[i].K;
        ps[i].X = d[i].A;
        ps[i].ldx = (int)d[i].K;
        ps[i].Y = d[i].C;
        ps[i].ldy = (int)d[i].N;
        ps[i].M = M;
        ps[i].groups = 1;
    }
    if (M == 0) return set_status(c, GGQ_OK);
    return hip_status(c, ggq::launch_gemv_multi(ps, n, pick_stream(c, stream)), "gemv batch");
    GGQ_END(c)
}

int ggq_mul_mat_fused_dev(ggq_ctx* c, const ggq_gemv_fused_desc* d, int n, int M, void* stream) {
    GGQ_GUARD(c)
    if (!d || n < 1 || n > GGQ_MAX_BATCH) return set_status(c, GGQ_INVALID_PARAM, "need 1..%d descriptors", GGQ_MAX_BATCH);
    if (M < 0 || M > GGQ_MAX_BATCH_ROWS) return set_status(c, GGQ_INVALID_PARAM, "M=%d outside 0..%d", M, GGQ_MAX_BATCH_ROWS);
    ggq::GemvProblem ps[GGQ_MAX_BATCH];
    for (int i = 0; i < n; i++) {
        const ggq_gemv_fused_desc& e = d[i];
        if (!e.W || !e.A || !e.C) return set_status(c, GGQ_INVALID_PARAM, "null pointer in entry %d", i);
        if (!aligned16(e.W)) return set_status(c, GGQ_INVALID_PARAM, "W must be 16-byte aligned");
        int st = check_matmul_shape(c, e.type, e.N, e.K, M, (int)e.K, (int)e.N, GGQ_ACT_F32);
        if (st != GGQ_OK) return st;
        if ((e.A_up || e.rms_norm || e.residual || e.silu) && e.K % 32)
            return set_status(c, GGQ_INVALID_PARAM, "fused options need K %% 32 == 0 (entry %d)", i);
        if (e.A_up && e.rms_norm) return set_status(c, GGQ_INVALID_PARAM, "A_up and rms_norm exclude each other");
        if (e.rms_norm && !(e.rms_eps >= 0.0f)) return set_status(c, GGQ_INVALID_PARAM, "rms_eps must be >= 0");
        if (e.rms_norm && !aligned16(e.rms_w)) return set_status(c, GGQ_INVALID_PARAM, "rms_w must be 16-byte aligned");
        ggq::GemvProblem& g = ps[i];
        g = ggq::GemvProblem{};
        g.type = e.type;
        g.W = e.W;
        g.N = (int)e.N;
        g.K = (int)e.K;
        g.X = e.A;
        g.X2 = e.A_up;
        g.ldx = (int)e.K;
        g.Y = e.C;
        g.ldy = (int)e.N;
        g.M = M;
        g.groups = 1;
        g.rms = e.rms_norm != 0;
        g.eps = e.rms_eps;
        g.norm_w = e.rms_w;
        g.R = e.residual;
        g.ldr = (int)e.N;
        g.silu = e.silu != 0;
    }
    if (M == 0) return set_status(c, GGQ_OK);
    return hip_status(c, ggq::launch_gemv_multi(ps, n, pick_stream(c, stream)), "fused gemv");
    GGQ_END(c)
}

int ggq_mul_mat_batch_dev(ggq_ctx* c, const ggq_gemv_desc* d, int n, void* stream) {
    return ggq_mul_mat_batch_rows_dev(c, d, n, 1, stream);
}

int ggq_mul_mat_batch_act_dev(ggq_ctx* c, const ggq_gemv_desc* d, int n, int M, int act_mode, void* stream) {
    if (act_mode == GGQ_ACT_F32) return ggq_mul_mat_batch_rows_dev(c, d, n, M, stream);
    GGQ_GUARD(c)
    if (!d || n < 1 || n > GGQ_MAX_BATCH) return set_status(c, GGQ_INVALID_PARAM, "need 1..%d descriptors", GGQ_MAX_BATCH);
    if (M < 0 || (M > GGQ_MAX_BATCH_ROWS && act_mode != GGQ_ACT_Q8_ROW))
        return set_status(c, GGQ_INVALID_PARAM, "M=%d outside 0..%d", M, GGQ_MAX_BATCH_ROWS);
    ggq::GemvProblem ps[GGQ_MAX_BATCH];
    for (int i = 0; i < n; i++) {
        if (!d[i].W || !d[i].A || !d[i].C) return set_status(c, GGQ_INVALID_PARAM, "null pointer in entry %d", i);
        if (!aligned16(d[i].W)) return set_status(c, GGQ_INVALID_PARAM, "W must be 16-byte aligned");
        int st = check_matmul_shape(c, d[i].type, d[i].N, d[i].K, M, (int)d[i].K, (int)d[i].N, act_mode);
        if (st != GGQ_OK) return st;
        ps[i] = ggq::GemvProblem{};
        ps[i].type = d[i].type;
        ps[i].W = d[i].W;
        ps[i].N = (int)d[i].N;
        ps[i].K = (int)d[i].K;
        ps[i].X = d[i].A;
        ps[i].ldx = (int)d[i].K;
        ps[i].Y = d[i].C;
        ps[i].ldy = (int)d[i].N;
        ps[i].M = M;
        ps[i].groups = 1;
    }
    if (M == 0) return set_status(c, GGQ_OK);
    hipStream_t s = pick_stream(c, stream);
    // Per-row int8 decode rows: one matrix-core launch quantizes and
    // multiplies every entry; otherwise one queued matmul per entry.
    if (act_mode == GGQ_ACT_Q8_ROW && M == 1 && ggq::gemv_q8row_eligible(ps, n)) {
        for (int i = 0; i < n; i++) ps[i].q8row = 1;
        return hip_status(c, ggq::launch_gemv_multi(ps, n, s), "gemv_q8row batch");
    }
    if (act_mode == GGQ_ACT_Q8_ROW && M <= 8 && ggq::i8_gemv_eligible(ps, n, 1))
        return hip_status(c, ggq::launch_i8_gemv(ps, n, 1, nullptr, nullptr, s), "gemv_i8 batch");
    bool done[GGQ_MAX_BATCH] = {};
    if (act_mode == GGQ_ACT_Q8_ROW && M > 8) {
        // Prefill-sized: entries that share the activations, type and K (q/k/v,
        // gate/up) as one activation-panel GEMM that quantizes the rows itself.
        for (int i = 0; i < n; i++) {
            if (done[i] || !ggq::gemm_panel_eligible(d[i].type, (int)d[i].K, M, d[i].A, (int)d[i].K)) continue;
            ggq::GemmDesc gd[GGQ_MAX_GEMM_BATCH];
            int ng = 0;
            for (int j = i; j < n && ng < GGQ_MAX_GEMM_BATCH; j++)
                if (!done[j] && d[j].A == d[i].A && d[j].type == d[i].type && d[j].K == d[i].K) {
                    gd[ng++] = ggq::GemmDesc{d[j].W, d[j].C, (int)d[j].N, (int)d[j].N};
                    done[j] = true;
                }
            const hipError_t e =
                ggq::launch_gemm_panel(d[i].type, gd, ng, (int)d[i].K, d[i].A, (int)d[i].K, nullptr, nullptr, M, s);
            if (e != hipSuccess) return hip_status(c, e, "gemm_panel batch");
        }
    }
    Arena ar = dev_arena(c, s);
    for (int i = 0; i < n; i++) {
        if (done[i]) continue;
        int st = mul_mat_queue(c, ar, d[i].W, d[i].type, d[i].N, d[i].K, d[i].A, (int)d[i].K, d[i].C, (int)d[i].N, M,
                               act_mode, s);
        if (st != GGQ_OK) return st;
    }
    return set_status(c, GGQ_OK);
    GGQ_END(c)
}

int ggq_dequant_dev(ggq_ctx* c, const void* raw, uint32_t type, int64_t n_blocks, float* out, void* stream) {
    GGQ_GUARD(c)
    if (!raw || !out || n_blocks < 0) return set_status(c, GGQ_INVALID_PARAM, "bad arguments");
    if (!ggq::supported(type)) return set_status(c, GGQ_INVALID_PARAM, "unsupported weight type %u", type);
    if (!aligned16(raw) || !aligned16(out)) return set_status(c, GGQ_INVALID_PARAM, "raw/out must be 16-byte aligned");
    return hip_status(c, ggq::launch_dequant(type, raw, n_blocks, out, pick_stream(c, stream)), "dequant");
    GGQ_END(c)
}

int ggq_quantize_act_dev(ggq_ctx* c, const float* A, int lda, int M, int K, int act_mode, int8_t* q,
                         float* scales, void* stream) {
    GGQ_GUARD(c)
    if (!A || !q || !scales || M < 0 || K <= 0 || lda < K) return set_status(c, GGQ_INVALID_PARAM, "bad arguments");
    if (act_mode != GGQ_ACT_Q8_ROW && act_mode != GGQ_ACT_Q8_BLOCK32)
        return set_status(c, GGQ_INVALID_PARAM, "act_mode must be Q8_ROW or Q8_BLOCK32");
    if (act_mode == GGQ_ACT_Q8_BLOCK32 && K % 32) return set_status(c, GGQ_INVALID_PARAM, "K must be a multiple of 32");
    return hip_status(c, ggq::launch_quant_act(A, lda, M, K, act_mode, q, scales, nullptr, pick_stream(c, stream)),
                      "quant_act");
    GGQ_END(c)
}

int ggq_produce_quantize_act_dev(ggq_ctx* c, int producer, const float* A, const float* aux, int lda, int M, int K,
                                 float eps, int8_t* q, float* scales, void* stream) {
    GGQ_GUARD(c)
    if (!A || !q || !scales || M < 0 || K <= 0 || lda < K) return set_status(c, GGQ_INVALID_PARAM, "bad arguments");
    if (producer != GGQ_PRODUCE_RMS_NORM && producer != GGQ_PRODUCE_SWIGLU)
        return set_status(c, GGQ_INVALID_PARAM, "producer must be GGQ_PRODUCE_RMS_NORM or GGQ_PRODUCE_SWIGLU");
    if (producer == GGQ_PRODUCE_SWIGLU && !aux) return set_status(c, GGQ_INVALID_PARAM, "SwiGLU needs the up rows");
    if (K > 16384 || K % 4 || lda % 4 || ((uintptr_t)A & 15u) || ((uintptr_t)aux & 15u) || ((uintptr_t)q & 3u))
        return set_status(c, GGQ_INVALID_PARAM, "K <= 16384, K and lda multiples of 4, A and aux 16-byte aligned");
    return hip_status(c, ggq::launch_produce_quant(producer, A, aux, lda, M, K, eps, q, scales, pick_stream(c, stream)),
                      "produce_quant");
    GGQ_END(c)
}

int ggq_block_dot_dev(ggq_ctx* c, const void* W, uint32_t type, int64_t N, int64_t K, const int8_t* qa, int M,
                      int32_t* out, void* stream) {
    GGQ_GUARD(c)
    if (!W || !qa || !out) return set_status(c, GGQ_INVALID_PARAM, "null pointer");
    if (!aligned16(W) || ((uintptr_t)qa & 15u) || (K % 16)) return set_status(c, GGQ_INVALID_PARAM, "alignment");
    int st = check_matmul_shape(c, type, N, K, M, (int)K, (int)N, GGQ_ACT_F32);
    if (st != GGQ_OK) return st;
    return hip_status(c, ggq::launch_block_dot(type, W, (int)N, (int)K, qa, M, out, pick_stream(c, stream)), "block_dot");
    GGQ_END(c)
}

// A routed (grouped) expert launch of the fp32 MoE path: on the int8
// matrix cores when the grouped form takes it (the expert's weights are
// decoded to int8 codes, about a third of the VALU work per weight of the
// fp16 matrix-core GEMV), else on the matrix-core / FMA GEMV.  The down
// projection's groups would run in passes of 1-2 rows there, each
// re-reading the expert's weights (measured slower): down takes the
// expert-grouped row tiles (Q6_K) or the GEMV.
static hipError_t moe_grouped_gemv(const ggq::GemvProblem& g, void* items, size_t items_bytes, hipStream_t s,
                                   bool down = false, const ggq::I8Shared* sh = nullptr, bool* took_shared = nullptr,
                                   bool list_ready = false) {
    if (took_shared) *took_shared = false;
    if (!down && ggq::i8_gemv_grouped_eligible(g)) {
        if (sh && ggq::i8_gemv_grouped_ws_bytes(g, sh->T) <= items_bytes) {
            if (took_shared) *took_shared = true;
            return ggq::launch_i8_gemv_grouped(g, items, s, sh, list_ready);
        }
        if (ggq::i8_gemv_grouped_ws_bytes(g) <= items_bytes) return ggq::launch_i8_gemv_grouped(g, items, s, nullptr, list_ready);
    }
    return ggq::launch_gemv(g, s);
}

// Largest average of pair rows per group (experts, plus the shared expert)
// that the grouped GEMVs take; above it the expert-grouped GEMMs / row
// tiles run.  GGQ_MOE_GEMV_MAX_AVG overrides the default: 5 for fp32
// activations (their 32-row fp16 GEMM tiles would be mostly empty below),
// 3 for per-row int8 (qwen35moe, GEMV vs the int8 row tiles: 64 tokens,
// 2.2 rows per group, 175 vs 205 us; 128 tokens, 4.5 rows, 264 vs 222 us).
static bool moe_small_groups(size_t rows, int groups, int dflt = 5) {
    const char* v = getenv("GGQ_MOE_GEMV_MAX_AVG");  // read per call: a process can switch it
    const size_t max_avg = v && *v ? (size_t)atoi(v) : (size_t)dflt;
    return rows <= max_avg * (size_t)groups;
}

// MoE layer with fp32 activations at prefill-sized batches: route, group
// (tile list over the experts and the shared expert as group E), the token
// rows split once into fp16 hi + lo planes, one expert-grouped fp16 GEMM
// for every expert's gate and up (paired when their types match), SwiGLU
// fused into the split of the pair rows, one grouped launch for down (the
// row tiles on the fp16 planes for Q6_K, else the GEMM), combine.  Requires
// H and F multiples of 64 (at most 16384), E <= 1023, x 16-byte aligned
// (checked by the caller).
static int moe_ffn_f16(ggq_ctx* c, const ggq_moe_params* p, hipStream_t s) {
    const int T = p->T, H = p->H, F = p->F, E = p->E, k = p->top_k;
    const bool shared = p->gate_shexp != nullptr;
    const size_t nk = (size_t)T * k, ts = shared ? (size_t)T : 0, rows = nk + ts;
    const int max_tiles = (int)((rows + ggq::kMoeTileRows - 1) / ggq::kMoeTileRows) + E + 1;
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off = align256(off + bytes); return o; };
    const size_t o_sel = take(4 * nk), o_w = take(4 * nk), o_go = take(4 * (size_t)(E + 2)),
                 o_tok = take(4 * rows), o_pos = take(4 * nk), o_xh = take(2 * (size_t)T * H),
                 o_xl = take(2 * (size_t)T * H), o_xs = take(4 * (size_t)T * (H / 32)), o_xe = take(4 * (size_t)T),
                 o_g = take(4 * rows * F), o_u = take(4 * rows * F), o_hh = take(2 * rows * F),
                 o_hl = take(2 * rows * F), o_hs = take(4 * rows * (F / 32)), o_he = take(4 * rows),
                 o_d = take(4 * rows * H), o_tl = take(8 * (size_t)max_tiles), o_nt = take(4);
    const size_t o_hf = c->trace_rows ? take(4 * rows * F) : 0;
    int st;
    if ((st = grow(c, c->dev.ws, off, s, "workspace")) != GGQ_OK) return st;
    hipError_t e;
    char* base = (char*)c->dev.ws.ptr;
    int32_t* sel = (int32_t*)(base + o_sel);
    float* wsel = (float*)(base + o_w);
    int32_t* grp = (int32_t*)(base + o_go);
    int32_t* tok = (int32_t*)(base + o_tok);
    int32_t* pos = (int32_t*)(base + o_pos);
    float *G = (float*)(base + o_g), *U = (float*)(base + o_u), *D = (float*)(base + o_d);
    float* hf = c->trace_rows ? (float*)(base + o_hf) : nullptr;
    void* tiles = base + o_tl;
    int32_t* ntiles = (int32_t*)(base + o_nt);

    // (decode-sized batches: the grouping launch routes the tokens itself)
    const bool route_in_group = ggq::moe_group_routes(T, k, E);
    const float* const rlog = route_in_group ? p->router_logits : nullptr;
    if (!route_in_group && (e = ggq::launch_moe_route(p->router_logits, T, E, k, sel, wsel, s)) != hipSuccess)
        return hip_status(c, e, "moe_route");
    if ((e = ggq::launch_moe_group(sel, T, k, E, grp, tok, pos, s, 0, nullptr, 0, nullptr, nullptr, rlog, sel, wsel)) !=
        hipSuccess)
        return hip_status(c, e, "moe_group");
    if ((e = ggq::launch_moe_tiles(grp, tok, E, (int)ts, (int2*)tiles, ntiles, s)) != hipSuccess)
        return hip_status(c, e, "moe_tiles");
    if ((e = ggq::launch_split_rows(0, p->x, nullptr, H, T, H, base + o_xh, base + o_xl, (float*)(base + o_xs),
                                    (float*)(base + o_xe), nullptr, s)) != hipSuccess)
        return hip_status(c, e, "split x");
    ggq::MoeGemm g{};
    g.E = E; g.grp = grp; g.tiles = tiles; g.n_tiles = ntiles; g.max_tiles = max_tiles;
    ggq::MoeGemm gu = g, gd = g;
    gu.K = H; gu.x_idx = tok; gu.ldc = F;
    gu.XH = base + o_xh; gu.XL = base + o_xl; gu.XS = (const float*)(base + o_xs); gu.xs = (const float*)(base + o_xe);
    gu.w_stride = (int64_t)F * ggq::row_bytes(p->gate_type, H);
    if (p->up_type == p->gate_type) {
        gu.W = p->gate_exps; gu.W2 = p->up_exps; gu.Wsh = p->gate_shexp; gu.W2sh = p->up_shexp;
        gu.N = 2 * F; gu.n1 = F; gu.C = G; gu.C2 = U;
        if ((e = ggq::launch_moe_gemm(p->gate_type, gu, s)) != hipSuccess) return hip_status(c, e, "moe gate+up");
    } else {
        gu.W = p->gate_exps; gu.Wsh = p->gate_shexp; gu.N = F; gu.n1 = F; gu.C = G;
        if ((e = ggq::launch_moe_gemm(p->gate_type, gu, s)) != hipSuccess) return hip_status(c, e, "moe gate");
        gu.W = p->up_exps; gu.Wsh = p->up_shexp; gu.C = U;
        gu.w_stride = (int64_t)F * ggq::row_bytes(p->up_type, H);
        if ((e = ggq::launch_moe_gemm(p->up_type, gu, s)) != hipSuccess) return hip_status(c, e, "moe up");
    }
    // SwiGLU of every pair row (routed and shared), split for down.
    if ((e = ggq::launch_split_rows(2, G, U, F, (int)rows, F, base + o_hh, base + o_hl, (float*)(base + o_hs),
                                    (float*)(base + o_he), hf, s)) != hipSuccess)
        return hip_status(c, e, "swiglu split");
    gd.K = F; gd.x_idx = nullptr; gd.ldc = H;
    gd.XH = base + o_hh; gd.XL = base + o_hl; gd.XS = (const float*)(base + o_hs); gd.xs = (const float*)(base + o_he);
    gd.W = p->down_exps; gd.Wsh = p->down_shexp;
    gd.w_stride = (int64_t)H * ggq::row_bytes(p->down_type, F);
    gd.N = H; gd.n1 = H; gd.C = D;
    // A Q6_K down projection (K <= 1024) on the row tiles with fp16 rows
    // (each expert's weights read once per 16 to 32 of its rows).
    if (ggq::i8_tile_codes_eligible(p->down_type, gd))
        e = ggq::launch_i8_tile_codes(p->down_type, gd, (int)(rows / (size_t)(E + (shared ? 1 : 0))), s);
    else
        e = ggq::launch_moe_gemm(p->down_type, gd, s);
    if (e != hipSuccess) return hip_status(c, e, "moe down");
    if ((e = ggq::launch_moe_combine(D, pos, wsel, T, k, H, shared ? D + nk * H : nullptr, p->shared_w, p->out, s)) !=
        hipSuccess)
        return hip_status(c, e, "moe combine");
    c->trace = ggq_moe_trace{GGQ_ACT_F32, T, H, F, E, k, (int)rows, shared ? 1 : 0, grp, tok, pos, G, U, hf, nullptr,
                             nullptr, D, shared ? D + nk * H : nullptr};
    if (p->sel_experts && (e = hipMemcpyAsync(p->sel_experts, sel, 4 * nk, hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return hip_status(c, e, "copy selection");
    if (p->sel_weights && (e = hipMemcpyAsync(p->sel_weights, wsel, 4 * nk, hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return hip_status(c, e, "copy weights");
    return set_status(c, GGQ_OK);
}

// MoE layer with per-row int8 activations (GGQ_ACT_Q8_ROW): route, group,
// quantize the token rows once (up to 16 tokens the grouping launch routes
// and quantizes too), one grouped int8 launch for every expert's gate and
// up (and the shared expert's, as group E: the int8 row tiles for Q4_K /
// Q6_K, else the expert-grouped GEMM, or the grouped int8 GEMV when the
// groups are small), SwiGLU fused into the row quantization of the pair
// rows, one grouped launch for down, combine.
static int moe_ffn_q8(ggq_ctx* c, const ggq_moe_params* p, hipStream_t s) {
    const int T = p->T, H = p->H, F = p->F, E = p->E, k = p->top_k;
    const bool shared = p->gate_shexp != nullptr;
    const size_t nk = (size_t)T * k, ts = shared ? (size_t)T : 0, rows = nk + ts;
    const int max_tiles = (int)((rows + ggq::kMoeTileRows - 1) / ggq::kMoeTileRows) + E + 1;
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off = align256(off + bytes); return o; };
    const size_t o_sel = take(4 * nk), o_w = take(4 * nk), o_go = take(4 * (size_t)(E + 2)),
                 o_tok = take(4 * rows), o_pos = take(4 * nk), o_qx = take((size_t)T * H), o_sx = take(4 * (size_t)T),
                 o_g = take(4 * rows * F), o_u = take(4 * rows * F), o_qh = take(rows * F), o_sh = take(4 * rows),
                 o_d = take(4 * rows * H), o_tl = take(8 * (size_t)max_tiles), o_nt = take(4),
                 o_qsx = take(4 * (size_t)T * (H / 32)), o_qsh = take(4 * rows * (F / 32));
    const size_t o_hf = c->trace_rows ? take(4 * rows * F) : 0;
    // chunk list of the grouped int8 GEMV (chunks of 4 or more rows)
    const size_t it_bytes = 8 * ((rows + 3) / 4 + std::min<size_t>((size_t)E + 1, rows)) + 16;
    const size_t o_it = take(it_bytes), o_it2 = take(it_bytes);  // gate / up, down
    int st;
    if ((st = grow(c, c->dev.ws, off, s, "workspace")) != GGQ_OK) return st;
    hipError_t e;
    char* base = (char*)c->dev.ws.ptr;
    int32_t* sel = (int32_t*)(base + o_sel);
    float* wsel = (float*)(base + o_w);
    int32_t* grp = (int32_t*)(base + o_go);
    int32_t* tok = (int32_t*)(base + o_tok);
    int32_t* pos = (int32_t*)(base + o_pos);
    int8_t* qx = (int8_t*)(base + o_qx);
    float* sx = (float*)(base + o_sx);
    float *G = (float*)(base + o_g), *U = (float*)(base + o_u), *D = (float*)(base + o_d);
    int8_t* qh = (int8_t*)(base + o_qh);
    float* sh = (float*)(base + o_sh);
    void* tiles = base + o_tl;
    int32_t* ntiles = (int32_t*)(base + o_nt);

    // (decode-sized batches: the grouping launch routes the tokens itself)
    const bool route_in_group = ggq::moe_group_routes(T, k, E);
    const float* const rlog = route_in_group ? p->router_logits : nullptr;
    if (!route_in_group && (e = ggq::launch_moe_route(p->router_logits, T, E, k, sel, wsel, s)) != hipSuccess)
        return hip_status(c, e, "moe_route");
    ggq::MoeGemm g{};
    g.E = E; g.grp = grp; g.tiles = tiles; g.n_tiles = ntiles; g.max_tiles = max_tiles;
    // Few rows per expert (decode-sized batches: up to 3 rows per group on
    // average, up to 1 for Q4_K / Q6_K): the grouped int8 GEMV in its
    // given-codes mode (chunks of 8 rows, 4 for Q6_K / IQ4), whose lanes
    // carry the rows; more rows per expert: the int8 row tiles or the
    // expert-grouped GEMM's 32-row tiles.
    const bool small = moe_small_groups(rows, E + (shared ? 1 : 0), 3);
    // Q4_K / Q6_K launches leave the grouped GEMV for the int8 row tiles
    // from 1 row per group on average (qwen35moe 32 / 64 / 128 tokens 142 ->
    // 117, 164 -> 157, 189 -> 179 us; at 16 tokens the two tie, at 4 the
    // GEMV is 5 us faster).
    const bool tiny = moe_small_groups(rows, E + (shared ? 1 : 0), 1);
    auto i8_ok = [&](uint32_t type, const ggq::MoeGemm& d) {
        return small && ggq::i8_moe_q8_eligible(type, d, (int)rows) &&
               ggq::i8_moe_q8_ws_bytes(type, d, (int)rows) <= it_bytes;
    };
    // gate and up: K = H, token rows gathered through tok; paired when the
    // types match, else two launches.  down: K = F, the pair rows themselves.
    ggq::MoeGemm gu = g, gd = g;
    gu.K = H; gu.QA = qx; gu.sa = sx; gu.x_idx = tok; gu.ldc = F;
    gu.w_stride = (int64_t)F * ggq::row_bytes(p->gate_type, H);
    gd.K = F; gd.QA = qh; gd.sa = sh; gd.x_idx = nullptr; gd.ldc = H;
    gd.W = p->down_exps; gd.W2 = nullptr; gd.Wsh = p->down_shexp; gd.W2sh = nullptr;
    gd.w_stride = (int64_t)H * ggq::row_bytes(p->down_type, F);
    gd.N = H; gd.n1 = H; gd.C = D; gd.C2 = nullptr;
    // the token rows' and pair rows' code sums per 32 values (the K-quant min term)
    float* qsx = (float*)(base + o_qsx);
    float* qsh = (float*)(base + o_qsh);
    gu.QS = qsx;
    gd.QS = qsh;
    const bool paired = p->up_type == p->gate_type;
    if (paired) {
        gu.W = p->gate_exps; gu.W2 = p->up_exps; gu.Wsh = p->gate_shexp; gu.W2sh = p->up_shexp;
        gu.N = 2 * F; gu.n1 = F; gu.C = G; gu.C2 = U;
    }
    // Above 3 rows per group on average, Q4_K / Q6_K launches (K <= 2048)
    // run on the int8 row tiles (8 to 32 rows of a group per pass, several
    // passes for larger groups), other formats on the 32-row GEMM tiles
    // (qwen35moe, tiles vs GEMM: 768 / 1024 / 2048 / 4096 / 6144 tokens
    // 303 vs 315, 374 vs 392, 593 vs 636, 1036 vs 1108, 1478 vs 1576 us).
    const int rpg = (int)(rows / (size_t)(E + (shared ? 1 : 0)));
    // A Q6_K down projection takes the row tiles from 32 routed pair rows
    // (64 tokens: 68 -> 61 us against the grouped GEMV's 4-row chunks; with
    // fewer, the few groups leave most of the tiles' resident grid idle: one
    // token of qwen35moe 41.1 vs 51.6 us on the GEMV, four 58.5 vs 54.7).
    auto tc_ok = [&](uint32_t type, const ggq::MoeGemm& d, bool down) {
        return (!tiny || (down && type == ggq::T_Q6_K && nk >= 32)) && ggq::i8_tile_codes_eligible(type, d);
    };
    const bool gu_tc = paired && tc_ok(p->gate_type, gu, false), dn_tc = tc_ok(p->down_type, gd, true);
    const bool gu_i8 = paired && !gu_tc && i8_ok(p->gate_type, gu), dn_i8 = !dn_tc && i8_ok(p->down_type, gd);
    // The grouping launch builds the chunk lists of the grouped int8
    // launches (and the shared expert's group end and token rows); the tile
    // list is built only when a launch takes the expert-grouped GEMM.
    ggq::ChunkList lists[2];
    int nl = 0;
    if (gu_i8) lists[nl++] = ggq::i8_moe_q8_list(p->gate_type, gu, (int)rows, base + o_it);
    if (dn_i8) lists[nl++] = ggq::i8_moe_q8_list(p->down_type, gd, (int)rows, base + o_it2);
    bool built = false, sh_built = false;
    // (up to 16 tokens the grouping launch also quantizes the token rows)
    ggq::RowQuant rq;
    const bool quant_in_group = route_in_group && H <= 2048 && H % 8 == 0;
    if (quant_in_group) {
        rq.A = p->x; rq.lda = H; rq.M = T; rq.K = H; rq.q = qx; rq.scales = sx; rq.gsum = qsx;
    }
    if ((e = ggq::launch_moe_group(sel, T, k, E, grp, tok, pos, s, (int)ts, lists, nl, &built, &sh_built, rlog, sel,
                                   wsel, quant_in_group ? &rq : nullptr)) !=
        hipSuccess)
        return hip_status(c, e, "moe_group");
    // The GEMM's tile list (and the shared expert's group end and token rows
    // when the grouping launch did not write them).
    const bool any_gemm = (paired ? !gu_i8 && !gu_tc : true) || (!dn_i8 && !dn_tc);
    if ((any_gemm || !sh_built) &&
        (e = ggq::launch_moe_tiles(grp, tok, E, (int)ts, (int2*)tiles, ntiles, s)) != hipSuccess)
        return hip_status(c, e, "moe_tiles");
    // the token rows' codes, and their sums per 32 values for the K-quant
    // min term of the grouped GEMM
    if (!quant_in_group &&
        (e = ggq::launch_produce_quant(0, p->x, nullptr, H, T, H, 0.0f, qx, sx, s, nullptr, qsx)) != hipSuccess)
        return hip_status(c, e, "quant x");
    auto grouped = [&](uint32_t type, const ggq::MoeGemm& d) -> hipError_t {
        if (i8_ok(type, d)) return ggq::launch_i8_moe_q8(type, d, (int)rows, base + o_it, s);
        return ggq::launch_moe_gemm(type, d, s);
    };
    if (paired) {
        if (gu_tc) e = ggq::launch_i8_tile_codes(p->gate_type, gu, rpg, s);
        else if (gu_i8) e = ggq::launch_i8_moe_q8(p->gate_type, gu, (int)rows, base + o_it, s, built);
        else e = ggq::launch_moe_gemm(p->gate_type, gu, s);
        if (e != hipSuccess) return hip_status(c, e, "moe gate+up");
    } else {
        gu.W = p->gate_exps; gu.W2 = nullptr; gu.Wsh = p->gate_shexp; gu.W2sh = nullptr;
        gu.N = F; gu.n1 = F; gu.C = G; gu.C2 = nullptr;
        if ((e = grouped(p->gate_type, gu)) != hipSuccess) return hip_status(c, e, "moe gate");
        gu.W = p->up_exps; gu.Wsh = p->up_shexp; gu.C = U;
        gu.w_stride = (int64_t)F * ggq::row_bytes(p->up_type, H);
        if ((e = grouped(p->up_type, gu)) != hipSuccess) return hip_status(c, e, "moe up");
    }
    // SwiGLU of every pair row (routed and shared) and its int8 row codes.
    float* hf = c->trace_rows ? (float*)(base + o_hf) : nullptr;
    if ((e = ggq::launch_produce_quant(GGQ_PRODUCE_SWIGLU, G, U, F, (int)rows, F, 0.0f, qh, sh, s, hf, qsh)) !=
        hipSuccess)
        return hip_status(c, e, "swiglu quant");
    if (dn_tc) e = ggq::launch_i8_tile_codes(p->down_type, gd, rpg, s);
    else if (dn_i8) e = ggq::launch_i8_moe_q8(p->down_type, gd, (int)rows, base + o_it2, s, built);
    else e = ggq::launch_moe_gemm(p->down_type, gd, s);
    if (e != hipSuccess) return hip_status(c, e, "moe down");
    if ((e = ggq::launch_moe_combine(D, pos, wsel, T, k, H, shared ? D + nk * H : nullptr, p->shared_w, p->out, s)) !=
        hipSuccess)
        return hip_status(c, e, "moe combine");
    c->trace = ggq_moe_trace{GGQ_ACT_Q8_ROW, T, H, F, E, k, (int)rows, shared ? 1 : 0, grp, tok, pos, G, U, hf, qh,
                             sh, D, shared ? D + nk * H : nullptr};
    if (p->sel_experts && (e = hipMemcpyAsync(p->sel_experts, sel, 4 * nk, hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return hip_status(c, e, "copy selection");
    if (p->sel_weights && (e = hipMemcpyAsync(p->sel_weights, wsel, 4 * nk, hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return hip_status(c, e, "copy weights");
    return set_status(c, GGQ_OK);
}

int ggq_moe_ffn_act_dev(ggq_ctx* c, const ggq_moe_params* p, int act_mode, void* stream) {
    if (act_mode == GGQ_ACT_F32) return ggq_moe_ffn_dev(c, p, stream);
    GGQ_GUARD(c)
    if (act_mode != GGQ_ACT_Q8_ROW) return set_status(c, GGQ_INVALID_PARAM, "act_mode must be F32 or Q8_ROW");
    if (!p || !p->x || !p->router_logits || !p->gate_exps || !p->up_exps || !p->down_exps || !p->out)
        return set_status(c, GGQ_INVALID_PARAM, "null pointer");
    const int T = p->T, H = p->H, F = p->F, E = p->E, k = p->top_k;
    if (T < 0 || H <= 0 || F <= 0 || E <= 0 || E > 1023 || k <= 0 || k > 64 || k > E || (int64_t)T * k > 65536)
        return set_status(c, GGQ_INVALID_PARAM, "bad MoE shape");
    int st;
    if ((st = check_matmul_shape(c, p->gate_type, F, H, T, H, F, 0)) != GGQ_OK) return st;
    if ((st = check_matmul_shape(c, p->up_type, F, H, T, H, F, 0)) != GGQ_OK) return st;
    if ((st = check_matmul_shape(c, p->down_type, H, F, T, F, H, 0)) != GGQ_OK) return st;
    if (H % 32 || F % 32 || H > 16384 || F > 16384 || H % 4 || F % 4)
        return set_status(c, GGQ_INVALID_PARAM, "Q8_ROW MoE needs H and F multiples of 32, at most 16384");
    const bool shared = p->gate_shexp != nullptr;
    if (shared && (!p->up_shexp || !p->down_shexp)) return set_status(c, GGQ_INVALID_PARAM, "partial shared expert");
    for (const void* w : {p->gate_exps, p->up_exps, p->down_exps, p->gate_shexp, p->up_shexp, p->down_shexp})
        if (w && !aligned16(w)) return set_status(c, GGQ_INVALID_PARAM, "weights must be 16-byte aligned");
    if (((uintptr_t)p->x & 15u)) return set_status(c, GGQ_INVALID_PARAM, "x must be 16-byte aligned");
    if (T == 0) return set_status(c, GGQ_OK);
    return moe_ffn_q8(c, p, pick_stream(c, stream));
    GGQ_END(c)
}

int ggq_moe_ffn_dev(ggq_ctx* c, const ggq_moe_params* p, void* stream) {
    GGQ_GUARD(c)
    if (!p || !p->x || !p->router_logits || !p->gate_exps || !p->up_exps || !p->down_exps || !p->out)
        return set_status(c, GGQ_INVALID_PARAM, "null pointer");
    const int T = p->T, H = p->H, F = p->F, E = p->E, k = p->top_k;
    if (T < 0 || H <= 0 || F <= 0 || E <= 0 || E > 1024 || k <= 0 || k > 64 || k > E || (int64_t)T * k > 65536)
        return set_status(c, GGQ_INVALID_PARAM, "bad MoE shape");
    int st;
    if ((st = check_matmul_shape(c, p->gate_type, F, H, T, H, F, 0)) != GGQ_OK) return st;
    if ((st = check_matmul_shape(c, p->up_type, F, H, T, H, F, 0)) != GGQ_OK) return st;
    if ((st = check_matmul_shape(c, p->down_type, H, F, T, F, H, 0)) != GGQ_OK) return st;
    const bool shared = p->gate_shexp != nullptr;
    if (shared && (!p->up_shexp || !p->down_shexp)) return set_status(c, GGQ_INVALID_PARAM, "partial shared expert");
    for (const void* w : {p->gate_exps, p->up_exps, p->down_exps, p->gate_shexp, p->up_shexp, p->down_shexp})
        if (w && !aligned16(w)) return set_status(c, GGQ_INVALID_PARAM, "weights must be 16-byte aligned");
    if (T == 0) return set_status(c, GGQ_OK);
    hipStream_t s = pick_stream(c, stream);
    // Prefill-sized batches: the expert-grouped fp16 GEMM, where its shape
    // limits allow.
    if (!moe_small_groups((size_t)T * k + (shared ? T : 0), E + (shared ? 1 : 0)) && E <= 1023 && H % 64 == 0 &&
        F % 64 == 0 && H <= 16384 && F <= 16384 && ((uintptr_t)p->x & 15u) == 0)
        return moe_ffn_f16(c, p, s);

    const size_t nk = (size_t)T * k;
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off = align256(off + bytes); return o; };
    // The shared expert's gate / up / SwiGLU rows follow the routed ones in
    // the same buffers (one SwiGLU launch covers both).
    const size_t ts = shared ? (size_t)T : 0;
    const size_t o_sel = take(4 * nk), o_w = take(4 * nk), o_go = take(4 * (size_t)(E + 2)),
                 o_tok = take(4 * (nk + ts)), o_pos = take(4 * nk), o_g = take(4 * (nk + ts) * F),
                 o_u = take(4 * (nk + ts) * F), o_h = take(4 * (nk + ts) * F), o_d = take(4 * nk * H);
    const size_t o_sd = shared ? take(4 * (size_t)T * H) : 0;
    // chunk list of the grouped int8 launches (chunks of 2 or more rows)
    const size_t it_bytes = 8 * ((nk + ts + 1) / 2 + std::min<size_t>((size_t)E + 1, nk + ts)) + 16;
    const size_t o_it = take(it_bytes);
    if ((st = grow(c, c->dev.ws, off, s, "workspace")) != GGQ_OK) return st;
    hipError_t e;
    char* base = (char*)c->dev.ws.ptr;
    int32_t* sel = (int32_t*)(base + o_sel);
    float* wsel = (float*)(base + o_w);
    int32_t* grp = (int32_t*)(base + o_go);
    int32_t* tok = (int32_t*)(base + o_tok);
    int32_t* pos = (int32_t*)(base + o_pos);
    float *G = (float*)(base + o_g), *U = (float*)(base + o_u), *Hh = (float*)(base + o_h), *D = (float*)(base + o_d);

    // (decode-sized batches: the grouping launch routes the tokens itself)
    const bool route_in_group = ggq::moe_group_routes(T, k, E);
    const float* const rlog = route_in_group ? p->router_logits : nullptr;
    if (!route_in_group && (e = ggq::launch_moe_route(p->router_logits, T, E, k, sel, wsel, s)) != hipSuccess)
        return hip_status(c, e, "moe_route");

    bool shared_done = false;  // the shared expert's gate / up ran in the routed launch
    ggq::GemvProblem g{};
    g.groups = E;
    g.grp_off = grp;
    g.M = (int)nk;
    g.max_group_rows = T;
    // gate / up: rows F, K = H, activations gathered by token.
    g.N = F; g.K = H; g.X = p->x; g.ldx = H; g.x_idx = tok; g.ldy = F;
    g.type = p->gate_type; g.W = p->gate_exps; g.w_group_stride = (int64_t)F * ggq::row_bytes(p->gate_type, H); g.Y = G;
    const bool paired = p->up_type == p->gate_type && H % 32 == 0;
    // The paired gate / up launch's chunk list (with the shared expert as one
    // more group) is built by the grouping launch itself when the grouped
    // int8 GEMV takes that launch (the same conditions as moe_grouped_gemv).
    ggq::GemvProblem gp = g;
    gp.W2 = p->up_exps; gp.Y2 = U; gp.n1 = F; gp.N = 2 * F;
    const int t_list = shared ? T : 0;
    const bool pre = paired && ggq::i8_gemv_grouped_eligible(gp) &&
                     ggq::i8_gemv_grouped_ws_bytes(gp, t_list) <= it_bytes;
    const ggq::ChunkList cl = pre ? ggq::i8_gemv_grouped_list(gp, base + o_it, t_list) : ggq::ChunkList{0, nullptr, nullptr};
    bool built = false;
    if ((e = ggq::launch_moe_group(sel, T, k, E, grp, tok, pos, s, pre ? t_list : 0, pre ? &cl : nullptr, pre ? 1 : 0,
                                   &built, nullptr, rlog, sel, wsel)) != hipSuccess)
        return hip_status(c, e, "moe_group");
    if (paired) {
        // gate and up of each expert in one launch: each workgroup loads a
        // token's activations once for both.
        g.W2 = p->up_exps; g.Y2 = U; g.n1 = F; g.N = 2 * F;
        // the shared expert joins the grouped int8 launch as one more group
        // (its rows nk .. nk + T - 1 of G / U), when that launch takes it
        const ggq::I8Shared shx{p->gate_shexp, p->up_shexp, T};
        if ((e = moe_grouped_gemv(g, base + o_it, it_bytes, s, false, shared ? &shx : nullptr, &shared_done, built)) !=
            hipSuccess)
            return hip_status(c, e, "moe gate+up");
        g.W2 = nullptr; g.Y2 = nullptr; g.n1 = 0;
    } else {
        if ((e = moe_grouped_gemv(g, base + o_it, it_bytes, s)) != hipSuccess) return hip_status(c, e, "moe gate");
        g.type = p->up_type; g.W = p->up_exps; g.w_group_stride = (int64_t)F * ggq::row_bytes(p->up_type, H); g.Y = U;
        if ((e = moe_grouped_gemv(g, base + o_it, it_bytes, s)) != hipSuccess) return hip_status(c, e, "moe up");
    }
    float* Dsh = nullptr;
    ggq::GemvProblem q{};
    q.groups = 1;
    q.M = T;
    if (shared) Dsh = (float*)(base + o_sd);
    if (shared && !shared_done) {
        float *SG = G + nk * F, *SU = U + nk * F;
        q.N = F; q.K = H; q.X = p->x; q.ldx = H; q.ldy = F;
        q.type = p->gate_type; q.W = p->gate_shexp; q.Y = SG;
        if (p->up_type == p->gate_type && H % 32 == 0) {
            q.W2 = p->up_shexp; q.Y2 = SU; q.n1 = F; q.N = 2 * F;
            if ((e = ggq::launch_gemv(q, s)) != hipSuccess) return hip_status(c, e, "shared gate+up");
            q.W2 = nullptr; q.Y2 = nullptr; q.n1 = 0;
        } else {
            if ((e = ggq::launch_gemv(q, s)) != hipSuccess) return hip_status(c, e, "shared gate");
            q.type = p->up_type; q.W = p->up_shexp; q.Y = SU;
            if ((e = ggq::launch_gemv(q, s)) != hipSuccess) return hip_status(c, e, "shared up");
        }
    }
    // SwiGLU of the routed pair rows and the shared expert's rows together.
    if ((e = ggq::launch_swiglu(G, U, Hh, (int64_t)(nk + ts) * F, s)) != hipSuccess) return hip_status(c, e, "swiglu");
    // down: rows H, K = F, activations are the sorted pair rows themselves.
    g.N = H; g.K = F; g.X = Hh; g.ldx = F; g.x_idx = nullptr; g.ldy = H; g.Y = D;
    g.type = p->down_type; g.W = p->down_exps; g.w_group_stride = (int64_t)H * ggq::row_bytes(p->down_type, F);
    // Q6_K down: expert-grouped row tiles on the int8 matrix cores (each
    // expert's weights decoded once per 4 of its rows), the shared expert as
    // one more group of the same launch.
    // (from 16 routed pair rows: below, the few groups leave most of the
    // tiles' resident grid idle and the grouped GEMV is faster, one token of
    // qwen35moe 43.4 vs 50.0 us; two tokens 55.4 vs 51.1 us)
    const bool tiles =
        ggq::i8_tile_grouped_eligible(p->down_type, H, F, E, g.w_group_stride, shared) && F % 4 == 0 && nk >= 16;
    if (tiles) {
        if ((e = ggq::launch_i8_tile_grouped(p->down_type, p->down_exps, g.w_group_stride, shared ? p->down_shexp : nullptr,
                                             Hh, F, grp, E, shared ? T : 0, D, Dsh, H, H, F, s)) != hipSuccess)
            return hip_status(c, e, "moe down");
    } else if ((e = moe_grouped_gemv(g, base + o_it, it_bytes, s, true)) != hipSuccess) {
        return hip_status(c, e, "moe down");
    }
    if (shared && !tiles) {
        q.N = H; q.K = F; q.X = Hh + nk * F; q.ldx = F; q.ldy = H; q.type = p->down_type; q.W = p->down_shexp; q.Y = Dsh;
        if ((e = ggq::launch_gemv(q, s)) != hipSuccess) return hip_status(c, e, "shared down");
    }
    if ((e = ggq::launch_moe_combine(D, pos, wsel, T, k, H, Dsh, p->shared_w, p->out, s)) != hipSuccess)
        return hip_status(c, e, "moe combine");
    c->trace = ggq_moe_trace{GGQ_ACT_F32, T, H, F, E, k, (int)(nk + ts), shared ? 1 : 0, grp, tok, pos, G, U, Hh,
                             nullptr, nullptr, D, Dsh};
    if (p->sel_experts && (e = hipMemcpyAsync(p->sel_experts, sel, 4 * nk, hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return hip_status(c, e, "copy selection");
    if (p->sel_weights && (e = hipMemcpyAsync(p->sel_weights, wsel, 4 * nk, hipMemcpyDeviceToDevice, s)) != hipSuccess)
        return hip_status(c, e, "copy weights");
    return set_status(c, GGQ_OK);
    GGQ_END(c)
}

int ggq_moe_trace_get(const ggq_ctx* c, ggq_moe_trace* out) {
    if (!c || !out) return GGQ_INVALID_PARAM;
    *out = c->trace;
    return c->trace.grp ? GGQ_OK : GGQ_NOT_FOUND;
}

int ggq_moe_trace_rows(ggq_ctx* c, int on) {
    if (!c) return GGQ_INVALID_PARAM;
    std::lock_guard<std::recursive_mutex> lk(c->mu);
    c->trace_rows = on != 0;
    return GGQ_OK;
}

}  // extern "C"
