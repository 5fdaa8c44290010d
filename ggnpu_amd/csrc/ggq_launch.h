// ggq_launch.h -- host-side launchers of the HIP kernels (ggq_kernels.hip).
// All launchers are asynchronous on `stream` and return hipError_t from the
// launch; shape validation is done by the caller (ggq_api.cpp).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ggq {

// Standalone bit-exact dequant of n_blocks consecutive blocks.
hipError_t launch_dequant(uint32_t type, const void* raw, int64_t n_blocks, float* out, hipStream_t s);

// int32 dot products per scale group: out[(m*N+n)*G + g], G = K/group_elems.
hipError_t launch_block_dot(uint32_t type, const void* W, int N, int K, const int8_t* qa, int M,
                            int32_t* out, hipStream_t s);

// Activation quantization (mode 1 = per row, 2 = per 32-block).  Any of q,
// scales, x_eff may be null.  x_eff[m][k] = q*scale as fp32 (dense, ld = K).
hipError_t launch_quant_act(const float* A, int lda, int M, int K, int mode, int8_t* q,
                            float* scales, float* x_eff, hipStream_t s);

// RMSNorm (producer 1; aux = norm weight [K] or null) or SwiGLU (producer
// 2; A = gate rows, aux = up rows, both with row stride lda) of each row,
// then the per-row quantization of launch_quant_act mode 1.  K <= 16384,
// K and lda multiples of 4, A and aux 16-byte aligned, q dense [M][K].
// prod_out (optional, dense [M][K], 16-byte aligned) receives the produced
// fp32 rows that were quantized.
// gsum (optional, [M][K/32], K a multiple of 32) receives the sums of each
// row's codes per 32 values (the K-quant min term of the grouped GEMM);
// producer 0 quantizes the rows as they are.
hipError_t launch_produce_quant(int producer, const float* A, const float* aux, int lda, int M, int K, float eps,
                                int8_t* q, float* scales, hipStream_t s, float* prod_out = nullptr,
                                float* gsum = nullptr);

// Decode GEMV with fp32 activations: Y[y_row][n] = sum_k X[x_row][k] W[n][k].
// Plain mode: grp_off == null, rows 0..M-1.  Grouped mode (MoE): group g uses
// weights W + g*w_group_stride and output rows grp_off[g]..grp_off[g+1]-1,
// whose activation rows are x_idx[row] (or the row itself when x_idx is null).
struct GemvProblem {
    uint32_t type;
    const void* W;
    int64_t w_group_stride;
    int N, K;
    const float* X;
    int ldx;
    float* Y;
    int ldy;
    int M;
    int groups;
    const int* grp_off;
    const int* x_idx;
    int max_group_rows;  // upper bound of rows per group (grouped mode)
    // Fused neighbours (zero / null = off; plain mode only):
    const float* X2;       // the activation is X * X2 elementwise (X2 [M][ldx])
    int silu;              // Y = silu(result) (before the residual add)
    int rms;               // RMSNorm the activation rows first (norm_w may be null)
    float eps;
    const float* norm_w;
    const float* R;        // Y = R + result, R [M][ldr]
    int ldr;
    // Paired matrices (n1 > 0, N = n1 + rows of W2): rows [0, n1) from W into
    // Y, the rest from W2 (same type, K, group stride) into Y2 (same ldy).
    // Not with the fused options; K a multiple of 32.
    const void* W2;
    float* Y2;
    int n1;
    // Single-row GGQ_ACT_Q8_ROW on the LDS-staged fp32 kernels: the row is
    // replaced by its per-row int8 codes in the staging and the outputs are
    // scaled back (gemv_q8row_eligible problems only).
    int q8row;
};
hipError_t launch_gemv(const GemvProblem& p, hipStream_t s);
// Several independent M = 1 problems in as few launches as possible.
hipError_t launch_gemv_multi(const GemvProblem* ps, int n, hipStream_t s);
// Decode-sized matmuls (1..8 activation rows, K a multiple of 256, the
// fused options in modes 0 and 1, no grouping, no pairs) on the int8
// matrix cores (ggq_gemv_i8.hip).
// mode 0: fp32 activations X (exact fixed-point digits); mode 1: X
// quantized per row to int8 in the kernel (GGQ_ACT_Q8_ROW semantics);
// mode 2: given int8 codes qa [M][K] with row scales sa.  Several problems
// (same M) run as one launch.
bool i8_gemv_eligible(const GemvProblem* ps, int n, int mode);
bool gemv_q8row_eligible(const GemvProblem* ps, int n);
hipError_t launch_i8_gemv(const GemvProblem* ps, int n, int mode, const int8_t* qa, const float* sa, hipStream_t s);
// A list of (group, first row) chunks of at most mt rows over groups whose
// rows are grp_off[g] .. grp_off[g+1]-1, for grouped launches that give a
// grid row to each chunk (n_items: its length).
struct ChunkList {
    int mt;
    int2* items;
    int32_t* n_items;
};
// Grouped (MoE) fp32-activation problems on the same kernel (groups <= 1024,
// g.M = total rows): a group's rows run in chunks of up to 4 (2 for Q6_K /
// IQ4) rows, one grid row per chunk from a chunk list built on the device;
// paired gate / up halves are two problems.  `ws`: device workspace of
// i8_gemv_grouped_ws_bytes(g) bytes.
// With `sh`, the shared expert (weights sh->W / sh->W2, every one of its
// sh->T tokens) joins the launch as group g.groups: its rows follow the
// routed ones (grp_off needs g.groups + 2 entries and x_idx g.M + T).
struct I8Shared { const void* W; const void* W2; int T; };
bool i8_gemv_grouped_eligible(const GemvProblem& g);
size_t i8_gemv_grouped_ws_bytes(const GemvProblem& g, int t_sh = 0);
hipError_t launch_i8_gemv_grouped(const GemvProblem& g, void* ws, hipStream_t s, const I8Shared* sh = nullptr,
                                  bool list_ready = false);
// The chunk list that launch would use in `ws` (mt 0 when the plan fails), for
// launch_moe_group to build ahead of it (then list_ready = true).
ChunkList i8_gemv_grouped_list(const GemvProblem& g, void* ws, int t_sh);
// Expert-grouped row tiles on the int8 matrix cores (fp32 activation rows,
// 4 per pass; Q6_K, K <= 2048): Y rows grp_off[g] .. grp_off[g+1]-1 = X rows
// times group g's matrix (W + g * w_stride); with Wsh, group E is the shared
// expert (X rows grp_off[E] .. + t_sh, outputs Ysh from row 0).
bool i8_tile_grouped_eligible(uint32_t type, int N, int K, int E, int64_t w_stride, bool shared);
hipError_t launch_i8_tile_grouped(uint32_t type, const void* W, int64_t w_stride, const void* Wsh, const float* X,
                                  int ldx, const int32_t* grp_off, int E, int t_sh, float* Y, float* Ysh, int ldy,
                                  int N, int K, hipStream_t s);
// Largest K the register-resident GEMV supports.
constexpr int kGemvMaxK = 32768;

// int8-MFMA GEMM on per-row int8 activations:
//   C[m][n] = sa[m] * sum_groups dl[n,g]*P[m,n,g] - ml[n,g]*S[m,g]
// One launch covers up to 4 weights of one type sharing the activations.
struct GemmDesc {
    const void* W;
    float* C;
    int N;
    int ldc;
};
struct GemmPlan {
    int bm, bn, n_tiles, m_tiles, splits, steps_per_split;
    size_t part_floats;  // split-K workspace (floats), 0 when not split
};
GemmPlan plan_gemm_i8(uint32_t type, const int* Ns, int n, int K, int M);
// `part` sized by plan_gemm_i8 (may be null when it plans no split).
hipError_t launch_gemm_i8_multi(uint32_t type, const GemmDesc* d, int n, int K, const int8_t* qa, const float* sa,
                                int M, float* part, hipStream_t s);
hipError_t launch_gemm_i8(uint32_t type, const void* W, int N, int K, const int8_t* qa, const float* sa, int M,
                          float* C, int ldc, float* part, hipStream_t s);
// Activation-panel GEMM (gemm_panel_kernel): the per-row int8 activations of
// a 64-row panel resident in LDS for the whole K, quantized in the kernel
// from fp32 rows A [M][lda] (GGQ_ACT_Q8_ROW, bit-exact with
// launch_quant_act) or taken from given codes qa / sa when A is null.  Up to
// 4 weights of one type sharing the activations; no workspace.  Types other
// than Q6_K, K a multiple of 32 and at most 2048, A 16-byte aligned with lda
// a multiple of 4.
bool gemm_panel_eligible(uint32_t type, int K, int M, const float* A, int lda);
hipError_t launch_gemm_panel(uint32_t type, const GemmDesc* d, int n, int K, const float* A, int lda,
                             const int8_t* qa, const float* sa, int M, hipStream_t s);
// idx[m] = first index of the largest value of row m of L ([M][ld], N
// values); val[m] = that value (val may be null).  `ws`: device workspace
// of argmax_workspace_bytes(M) bytes.
size_t argmax_workspace_bytes(int M);
hipError_t launch_argmax_rows(const float* L, int M, int N, int ld, int32_t* idx, float* val, void* ws,
                              hipStream_t s);
// Decode attention over one layer's KV cache [ctx][n_kv][head_dim] for n_tok
// query rows at positions pos0.. (head_dim 64 or 128, n_head / n_kv in
// {1, 2, 4, 8}); ws holds attn_workspace_floats(...) floats.
size_t attn_workspace_floats(int n_tok, int n_head, int head_dim, int64_t ctx_len, int64_t pos0, int n_kv);
hipError_t launch_attn_decode(const float* Q, const float* K, const float* V, int n_tok, int n_head, int n_kv,
                              int head_dim, int64_t ctx_len, int64_t pos0, float* out, float* ws, hipStream_t s);
// n-byte copy by a kernel (either end may be pinned host memory).
hipError_t launch_copy_bytes(void* dst, const void* src, size_t n, hipStream_t s);
hipError_t launch_host_flag(uint32_t* flag, uint32_t v, hipStream_t s);
// x[m][k] = q[m][k] * sa[m] (dense fp32 [M][K]).
hipError_t launch_dequant_act(const int8_t* q, const float* sa, int M, int K, float* x, hipStream_t s);

// Fixed per-device scratch region of the allocation-free entry point
// (ggq_mul_mat_noalloc_dev): kScratchBytes of device memory that every GPU the
// library runs on holds until the process ends.  scratch_device_ptr returns
// the current device's address of it (looked up once per device; the caller
// makes `device` current first).
constexpr size_t kScratchBytes = size_t(32) << 20;
hipError_t scratch_device_ptr(int device, void** out);

// MoE helpers.
hipError_t launch_moe_route(const float* logits, int T, int E, int topk, int32_t* sel,
                            float* wsel, hipStream_t s);
// Pairs grouped by expert (grp_off, tok_idx, pos_of).  On the small-E path
// the same launch also writes the chunk lists asked for (*lists_built) and
// the shared expert's group end grp_off[E + 1] and token rows, t_sh of them
// (*shared_built).  With logits given (moe_group_routes(T, topk, E) must
// hold) it first routes the tokens itself, writing sel_out / wsel_out as
// launch_moe_route does, and sel is not read.
bool moe_group_routes(int T, int topk, int E);
// Rows the grouping launch also quantizes per row when it routes (M <= 16,
// K <= 2048 and a multiple of 8, A 16-byte aligned with lda % 4 == 0, q
// 8-byte aligned): the codes, scales and code sums per 32 values of
// launch_produce_quant(PROD_NONE), bit for bit.
struct RowQuant {
    const float* A = nullptr;
    int lda = 0, M = 0, K = 0;
    int8_t* q = nullptr;
    float* scales = nullptr;
    float* gsum = nullptr;
};
hipError_t launch_moe_group(const int32_t* sel, int T, int topk, int E, int32_t* grp_off,
                            int32_t* tok_idx, int32_t* pos_of, hipStream_t s, int t_sh = 0,
                            const ChunkList* lists = nullptr, int n_lists = 0, bool* lists_built = nullptr,
                            bool* shared_built = nullptr, const float* logits = nullptr, int32_t* sel_out = nullptr,
                            float* wsel_out = nullptr, const RowQuant* rq = nullptr);
// Expert-grouped int8 GEMM over a device-built tile list (see
// moe_gemm_kernel): C[p] = sa[row(p)] * codes(p) . W_e^T for every pair row
// p of group e; rows [n1, N) of the output come from W2 into C2.
struct MoeGemm {
    const void* W;
    const void* W2;   // paired matrix (rows [n1, N)) or null
    const void* Wsh;  // shared expert (group E) matrices
    const void* W2sh;
    int64_t w_stride;
    int N, K, n1, E;
    const int8_t* QA;
    const float* sa;
    const int32_t* x_idx;
    const int32_t* grp;
    const void* tiles;
    const int32_t* n_tiles;
    int max_tiles;
    float* C;
    float* C2;
    int ldc;
    // int8 codes: their sums per 32 values [rows][K/32] (needed for Q4_K /
    // Q5_K, whose min term they feed)
    const float* QS = nullptr;
    // fp32 activation rows (the fp16 hi + lo kernel) when XH is set: planes
    // from launch_split_rows (K a multiple of 64); QA / sa unused then.
    const void* XH = nullptr;
    const void* XL = nullptr;
    const float* XS = nullptr;
    const float* xs = nullptr;
};
constexpr int kMoeTileRows = 32;  // pair rows per grouped-GEMM tile
hipError_t launch_moe_tiles(int32_t* grp, int32_t* x_idx, int E, int T_sh, int2* tiles, int32_t* n_tiles, hipStream_t s);
hipError_t launch_moe_gemm(uint32_t type, const MoeGemm& g, hipStream_t s);
// The same grouped launch (int8 codes QA / sa, groups from grp with the
// shared expert as group E when Wsh is set, grp[E + 1] written) on int8 row
// tiles: Q4_K / Q6_K, K <= 2048, 16 to 32 rows of a group per pass (by
// the average rows per group).  With XH set (fp32 rows as fp16 hi / lo
// planes, XL, xs): Q6_K, K <= 1024, unpaired.
bool i8_tile_codes_eligible(uint32_t type, const MoeGemm& g);
hipError_t launch_i8_tile_codes(uint32_t type, const MoeGemm& g, int rows_per_group, hipStream_t s);
// The same layer's grouped launches on the int8 GEMV in its given-codes
// mode (per-row int8 codes g.QA / g.sa): a group's rows in chunks of up to 8
// (4 for Q6_K / IQ4) from a chunk list built on the device over the E groups
// and the shared expert (group E, when g.Wsh is set); rows = total pair rows
// (grp[E + 1]).  `ws`: i8_moe_q8_ws_bytes(...) bytes.
bool i8_moe_q8_eligible(uint32_t type, const MoeGemm& g, int rows);
size_t i8_moe_q8_ws_bytes(uint32_t type, const MoeGemm& g, int rows);
hipError_t launch_i8_moe_q8(uint32_t type, const MoeGemm& g, int rows, void* ws, hipStream_t s, bool list_ready = false);
ChunkList i8_moe_q8_list(uint32_t type, const MoeGemm& g, int rows, void* ws);
// fp32 rows (producer 0) or their SwiGLU silu(A) * aux (producer 2, both
// with row stride lda) as the fp16 hi + lo planes XH / XL [M][K] (fp16),
// group sums XS [M][K/32] and row scales xs [M] of the grouped fp16 GEMM;
// prod_out (optional, [M][K]) receives the produced rows.  K <= 16384, a
// multiple of 32; A, aux 16-byte aligned.
hipError_t launch_split_rows(int producer, const float* A, const float* aux, int lda, int M, int K, void* XH,
                             void* XL, float* XS, float* xs, float* prod_out, hipStream_t s);
hipError_t launch_swiglu(const float* g, const float* u, float* h, int64_t n, hipStream_t s);
hipError_t launch_moe_combine(const float* D, const int32_t* pos_of, const float* wsel, int T,
                              int topk, int H, const float* Dsh, const float* shared_w, float* out,
                              hipStream_t s);

}  // namespace ggq
