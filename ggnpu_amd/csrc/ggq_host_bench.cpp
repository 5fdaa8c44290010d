// Benchmark driver for the synchronous host-pointer entry point: replays a
// sequence of ggq_mul_mat_q calls from a C++ loop, as the reference's CLI
// issues them (src/cli/main.cpp:1405-1434, one call per matmul), so that no
// interpreter runs between the calls.  The entry point is passed in as a
// function pointer (the caller's already-loaded libggq_hip.so); this library
// links nothing of its own.
#include <chrono>

#include "ggq.h"

typedef int (*ggq_mul_mat_q_fn)(ggq_ctx*, const ggq_mul_mat_params*, int);

extern "C" int ggq_host_bench_run(ggq_mul_mat_q_fn mul_mat_q, ggq_ctx* ctx, const ggq_mul_mat_params* params, int n,
                                  int act_mode, int warmup, int steps, double* sec_per_step) {
    if (!mul_mat_q || !ctx || !params || n <= 0 || warmup < 0 || steps <= 0 || !sec_per_step) return GGQ_INVALID_PARAM;
    for (int s = 0; s < warmup; s++)
        for (int i = 0; i < n; i++) {
            const int st = mul_mat_q(ctx, params + i, act_mode);
            if (st != GGQ_OK) return st;
        }
    const auto t0 = std::chrono::steady_clock::now();
    for (int s = 0; s < steps; s++)
        for (int i = 0; i < n; i++) {
            const int st = mul_mat_q(ctx, params + i, act_mode);
            if (st != GGQ_OK) return st;
        }
    const std::chrono::duration<double> dt = std::chrono::steady_clock::now() - t0;
    *sec_per_step = dt.count() / steps;
    return GGQ_OK;
}
