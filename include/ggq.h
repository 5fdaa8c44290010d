/*
 * ggq.h -- C ABI of the MI355X (gfx950) quantized-matmul backend for ggnpu.
 *
 * This is the drop-in boundary for ggnpu's `Backend::mul_mat_q` hot path
 * (include/ggnpu/backend.h:117 in the ggnpu tree) when B holds raw GGUF
 * blocks (the non-NPU branch of the caller, src/cli/main.cpp:1430-1432).
 * Plain C types only: pointers, sizes, integer status codes.  No C++ or torch
 * types cross this boundary and no exception escapes it.
 *
 * Status codes are ggnpu's `Status` values (include/ggnpu/backend.h:12-19).
 * Weight type ids are GGML ids (include/ggnpu/tensor.h:11-42); supported:
 * Q8_0 (8), Q4_K (12), Q5_K (13), Q6_K (14), IQ4_NL (20), IQ4_XS (23).
 *
 * Layouts (as in the reference, src/backends/cpu_ref/cpu_ref.cpp:87-117):
 *   W  raw GGUF bytes, N rows of K values, row n at n * (K/blck) * type_size
 *   A  fp32 activations [M][lda], C fp32 output [M][ldc] (fully overwritten)
 *
 * Activation treatments (act_mode):
 *   GGQ_ACT_F32         fp32 activations, as CpuRefBackend::mul_mat_q
 *                       (cpu_ref.cpp:87-117)
 *   GGQ_ACT_Q8_ROW      per-row int8 activations, as the XDNA backend
 *                       (amd_xdna.cpp:598-603, 633-639, 757-771): scale =
 *                       amax/127, q = clamp(rint(a*(1/scale)))
 *   GGQ_ACT_Q8_BLOCK32  per-32-value int8 activations (extension; no
 *                       reference counterpart)
 */
#ifndef GGQ_H
#define GGQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status, include/ggnpu/backend.h:12-19. */
#define GGQ_OK 0
#define GGQ_ERROR 1
#define GGQ_NOT_FOUND 2
#define GGQ_INVALID_PARAM 3
#define GGQ_DEVICE_UNAVAILABLE 4 /* Status::NPU_UNAVAILABLE */
#define GGQ_OUT_OF_MEMORY 5

/* GGML type ids, include/ggnpu/tensor.h:11-42. */
#define GGQ_TYPE_Q8_0 8
#define GGQ_TYPE_Q4_K 12
#define GGQ_TYPE_Q5_K 13
#define GGQ_TYPE_Q6_K 14
#define GGQ_TYPE_IQ4_NL 20
#define GGQ_TYPE_IQ4_XS 23

#define GGQ_ACT_F32 0
#define GGQ_ACT_Q8_ROW 1
#define GGQ_ACT_Q8_BLOCK32 2

typedef struct ggq_ctx ggq_ctx;
typedef struct ggq_weight ggq_weight;

/* ---------------------------------------------------------------- context */

/* Replaces create_amd_xdna_backend(int device_id) (backend.h:162-165).
 * Returns GGQ_DEVICE_UNAVAILABLE when no HIP device with that id exists. */
int ggq_create(int device, ggq_ctx** out);
/* Frees every device allocation the context owns (uploaded weights,
 * workspace) and its stream. */
void ggq_destroy(ggq_ctx* ctx);
/* Backend::last_error (backend.h:159): status of the most recent call. */
int ggq_last_error(const ggq_ctx* ctx);
/* Human-readable detail of the most recent error ("" when none). */
const char* ggq_last_error_message(const ggq_ctx* ctx);
/* Backend::name (backend.h:158). */
const char* ggq_name(const ggq_ctx* ctx);
/* Backend::is_available (backend.h:157). */
int ggq_is_available(const ggq_ctx* ctx);
/* Backend::sync (backend.h:155): waits for all work queued on the context's
 * device (the context stream and the streams passed to the *_dev calls). */
int ggq_sync(ggq_ctx* ctx);

/* Workspace contract.  The *_dev calls take their scratch memory (quantized
 * activations, split-K partial tiles, MoE intermediates, logits and
 * attention partials) from buffers the context grows on demand.  An outgrown
 * buffer is kept until ggq_destroy, never freed earlier, so work queued
 * before the growth and HIP graphs captured before it stay valid.  A call
 * made while its stream is being captured never allocates: if its workspace
 * is too small it fails with GGQ_ERROR and says so in
 * ggq_last_error_message.  Size the workspace before a capture by running
 * the captured calls once outside it, or with ggq_reserve.  The synchronous
 * host-pointer calls use their own buffers.  No reference counterpart (the
 * reference has no device workspace). */
/* Grows each of the context's device workspaces to at least `bytes`. */
int ggq_reserve(ggq_ctx* ctx, int64_t bytes);

/* ------------------------------------------------ host-pointer, synchronous */

/* MulMatParams (backend.h:21-35) with B = raw GGUF bytes; field order and
 * meaning as in the reference.  `scales`/`n_weight_scales` must be 0 (they
 * carry the XDNA path's re-quantized row scales, which this backend never
 * uses).  lda/ldc of 0 mean K/N. */
typedef struct {
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
    const void* scales;
    int n_weight_scales;
    uint32_t B_type;
} ggq_mul_mat_params;

/* Replaces Backend::mul_mat_q (backend.h:117) for raw-block weights.  B is
 * uploaded to HBM unchanged on first use and kept resident, keyed by
 * (B pointer, type, N, K) like the XDNA backend's resident weight BOs
 * (amd_xdna.cpp:279-310, 726-748); the caller keeps B alive and unchanged
 * while the context lives (it is an mmap'd GGUF tensor in the reference).
 * Synchronous: C is complete on return (as cpu_ref.cpp and amd_xdna.cpp). */
int ggq_mul_mat_q(ggq_ctx* ctx, const ggq_mul_mat_params* params, int act_mode);

/* Explicit upload of raw blocks (copied unchanged; host bytes stay owned by
 * the caller).  No reference counterpart: the reference re-reads mmap'd
 * bytes per call; this is the HBM-resident form of the same tensor. */
int ggq_weight_upload(ggq_ctx* ctx, const void* raw, uint32_t type, int64_t N, int64_t K,
                      ggq_weight** out);
int ggq_weight_free(ggq_ctx* ctx, ggq_weight* w);
/* Device address of an uploaded weight (for the *_dev entry points). */
const void* ggq_weight_device_ptr(const ggq_weight* w);
/* Synchronous matmul against an uploaded weight with host A and C. */
int ggq_mul_mat(ggq_ctx* ctx, const ggq_weight* w, const float* A, int lda, float* C, int ldc,
                int M, int act_mode);

/* --------------------------------------- device-pointer, asynchronous */
/* All pointers below are device pointers; work is queued on `stream`
 * (a hipStream_t; NULL = the HIP default stream, so the work is ordered
 * with the caller's default-stream work) and the call returns without
 * waiting.  W must be 16-byte aligned and readable for 256 bytes past its
 * last block (allocations made by ggq_weight_upload are). */

/* Same semantics as ggq_mul_mat_q. */
int ggq_mul_mat_dev(ggq_ctx* ctx, const void* W, uint32_t type, int64_t N, int64_t K,
                    const float* A, int lda, float* C, int ldc, int M, int act_mode, void* stream);

/* ggq_mul_mat_dev without any allocation, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  Its
 * scratch memory (quantized activations, split-K partial tiles) is one fixed
 * region of GGQ_NOALLOC_SCRATCH_BYTES per GPU, held from library load until
 * the process ends and shared by every context on that GPU; a call that
 * would need more fails with GGQ_INVALID_PARAM before queuing anything.
 * Calls that overlap on one GPU (several streams, threads or contexts) would
 * race on that region: order them.  An eager call is refused with GGQ_ERROR,
 * before queuing anything, while work an earlier eager call queued on
 * another stream is unfinished (calls queued under graph capture are not
 * tracked).  The region's address is looked up on the first call on a
 * device; if that fails only this entry point fails.  Results equal
 * ggq_mul_mat_dev's. */
#define GGQ_NOALLOC_SCRATCH_BYTES (32u << 20)
int ggq_mul_mat_noalloc_dev(ggq_ctx* ctx, const void* W, uint32_t type, int64_t N, int64_t K,
                            const float* A, int lda, float* C, int ldc, int M, int act_mode, void* stream);

/* Decode GEMVs (fp32 activations, GGQ_ACT_F32 semantics) with their
 * neighbours in the same launch, for the parts of a transformer layer that
 * surround the matmuls (no reference counterpart as a fused call; each
 * option restates a reference step):
 *   rms_norm  RMSNorm of each A row before the matmul, as
 *             CpuRefBackend::rms_norm (cpu_ref.cpp:139-156):
 *             a * (1/sqrt(sum(a^2)/K + eps)) * rms_w[k] (rms_w null = 1,
 *             else 16-byte aligned);
 *   silu      C = silu(result), silu(x) = x / (1 + exp(-x))
 *             (CpuRefBackend::silu, cpu_ref.cpp:200-209) -- the gate
 *             projection of SwiGLU;
 *   A_up      the activation is A * A_up elementwise (main.cpp:3474-3477:
 *             silu(gate) *= up) -- the down projection reading the gate
 *             (silu applied) and up outputs; A_up dense [M][K] with A's
 *             alignment; not with rms_norm;
 *   residual  C = residual + result (after silu), the residual adds of
 *             main.cpp:3424-3431 and 3491-3498 (residual may be C itself).
 * A dense [M][K], C and residual dense [M][N]; all entries share M
 * (<= GGQ_MAX_BATCH_ROWS); entries that share the pieces-per-thread count
 * run as one launch.  K must be a multiple of 32 when any option is set.
 * Results match the unfused sequence within fp32 rounding (the norm's sum
 * of squares is added in a different order). */
typedef struct {
    const void* W;
    uint32_t type;
    int64_t N;
    int64_t K;
    const float* A;
    const float* A_up;
    float* C;
    const float* residual;
    const float* rms_w;
    int rms_norm;
    float rms_eps;
    int silu;
} ggq_gemv_fused_desc;
int ggq_mul_mat_fused_dev(ggq_ctx* ctx, const ggq_gemv_fused_desc* descs, int n, int M, void* stream);

/* Vocab projection with the greedy token choice on the device: logits =
 * A . W^T as ggq_mul_mat_dev (A dense [M][K], act_mode as there), then
 * token[m] = the first index of the largest logit of row m and value[m]
 * that logit, as sample_token with temperature 0 (src/cli/main.cpp:827-838:
 * strict >, so ties go to the lower index and NaN never wins; a row with
 * nothing above -inf gives 0).  Replaces compute_logits + sample_token
 * (main.cpp:270-327, 827-838) without reading the logits back.  `logits`
 * ([M][N]) and `value` ([M]) may be null; token ([M] int32) may not. */
int ggq_logits_argmax_dev(ggq_ctx* ctx, const void* W, uint32_t type, int64_t N, int64_t K, const float* A,
                          int M, int act_mode, float* logits, int32_t* token, float* value, void* stream);

/* Decode attention of n_tok query rows over one layer's KV cache, on the
 * device.  Q is [n_tok][n_head][head_dim]; K and V are the layer's cache
 * slabs [ctx_len][n_kv_head][head_dim] (the layout of kv_cache.cpp:38-48,
 * row p = position p); out is [n_tok][n_head][head_dim]; all fp32, Q/K/V
 * 16-byte aligned.  Query row t sits at position pos0 + t and attends to
 * positions 0 .. min(pos0 + t, ctx_len - 1); query head h reads kv head
 * h / (n_head / n_kv_head).  Result: softmax(q.k / sqrt(head_dim)) . V as
 * CpuRefBackend::flash_attn (src/backends/cpu_ref.cpp:223-280) computes it
 * over the GQA-expanded K/V that src/cli/main.cpp:3358-3379 builds with
 * query_pos = pos + bt; no expanded copy is made here.  head_dim 64 or 128,
 * n_head / n_kv_head in {1, 2, 4, 8}.  Matches the reference within fp32
 * rounding (the softmax sum is taken per 64-position chunk, then merged). */
int ggq_attention_decode_dev(ggq_ctx* ctx, const float* Q, const float* K, const float* V, int n_tok, int n_head,
                             int n_kv_head, int head_dim, int64_t ctx_len, int64_t pos0, float* out, void* stream);

/* C = sa[m] * sum_k qa[m][k] * w[n][k]: the GGQ_ACT_Q8_ROW matmul on
 * activations already quantized by ggq_quantize_act_dev (row mode; qa dense
 * [M][K], 16-byte aligned, sa [M]).  Lets callers quantize an input once
 * when several weights consume it (q/k/v, gate/up).  The reference
 * quantizes inside every mul_mat_q call (amd_xdna.cpp:633-639, 757-771);
 * results are identical to ggq_mul_mat_dev with GGQ_ACT_Q8_ROW. */
int ggq_mul_mat_q8_dev(ggq_ctx* ctx, const void* W, uint32_t type, int64_t N, int64_t K, const int8_t* qa,
                       const float* sa, int M, float* C, int ldc, void* stream);

/* Several weights of one type and one K that consume the same activations
 * quantized by ggq_quantize_act_dev (the q/k/v or the gate/up projections
 * of a prefill batch), as one int8-MFMA launch.  Each entry gets what
 * ggq_mul_mat_q8_dev gives for it, up to fp32 summation order (the split of
 * K over workgroups depends on the launch's total size).  No reference
 * counterpart: the reference issues one mul_mat_q per weight
 * (src/cli/main.cpp:3256-3267).  At most GGQ_MAX_GEMM_BATCH entries. */
#define GGQ_MAX_GEMM_BATCH 4
typedef struct {
    const void* W; /* raw blocks, device memory, 16-byte aligned */
    int64_t N;     /* weight rows */
    float* C;      /* [M][ldc] device output */
    int ldc;
} ggq_gemm_desc;
int ggq_mul_mat_q8_batch_dev(ggq_ctx* ctx, const ggq_gemm_desc* descs, int n, uint32_t type, int64_t K,
                             const int8_t* qa, const float* sa, int M, void* stream);

/* Several independent single-row (decode) matmuls with fp32 activations,
 * queued as one launch where their shapes allow (a mix of weight types is
 * fine), e.g. the q/k/v projections of one token, which share an input.  No
 * reference counterpart: the reference issues one mul_mat_q per weight
 * (src/cli/main.cpp:3256-3267).  Same result as one ggq_mul_mat_dev call per
 * entry with M = 1 and GGQ_ACT_F32.  At most GGQ_MAX_BATCH entries. */
#define GGQ_MAX_BATCH 8
typedef struct {
    const void* W;
    uint32_t type;
    int64_t N, K;
    const float* A; /* [K] */
    float* C;       /* [N] */
} ggq_gemv_desc;
int ggq_mul_mat_batch_dev(ggq_ctx* ctx, const ggq_gemv_desc* descs, int n, void* stream);

/* ggq_mul_mat_batch_dev for M activation rows per entry (A dense [M][K], C
 * dense [M][N]; every entry has the same M, 0 <= M <= GGQ_MAX_BATCH_ROWS),
 * e.g. the projections of a few decode sequences batched together.  Same
 * result as one ggq_mul_mat_dev call per entry with GGQ_ACT_F32.  No
 * reference counterpart (see ggq_mul_mat_batch_dev). */
#define GGQ_MAX_BATCH_ROWS 64
int ggq_mul_mat_batch_rows_dev(ggq_ctx* ctx, const ggq_gemv_desc* descs, int n, int M, void* stream);

/* ggq_mul_mat_batch_rows_dev with an activation treatment (act_mode as for
 * ggq_mul_mat_dev): same result as one ggq_mul_mat_dev call per entry with
 * that act_mode.  GGQ_ACT_Q8_ROW with M <= 8 quantizes each entry's rows as
 * amd_xdna.cpp:598-603 and runs all entries in one int8 launch where the
 * shapes allow; with M > 8 (any M: the GGQ_MAX_BATCH_ROWS limit applies to
 * the other modes) entries that share A, type and K run as one int8 GEMM
 * launch that quantizes the rows itself, the prefill form of the
 * reference's quantize-inside-mul_mat_q (amd_xdna.cpp:633-639).  No reference counterpart as a batched call (the reference
 * issues one mul_mat_q per weight, main.cpp:3256-3267). */
int ggq_mul_mat_batch_act_dev(ggq_ctx* ctx, const ggq_gemv_desc* descs, int n, int M, int act_mode, void* stream);

/* Bit-exact fp32 dequant of n_blocks consecutive blocks, equal to the
 * reference's dequant_*_block functions (kquant.h:133-202, q8_0.cpp:19-25,
 * iq4_nl.cpp:24-31, iq4_xs.cpp:21-38). */
int ggq_dequant_dev(ggq_ctx* ctx, const void* raw, uint32_t type, int64_t n_blocks, float* out,
                    void* stream);

/* Activation quantization (act_mode GGQ_ACT_Q8_ROW or GGQ_ACT_Q8_BLOCK32).
 * q: [M][K] int8; scales: [M] (row) or [M][K/32] (block32).  Bit-exact with
 * amd_xdna.cpp:598-603, 633-639, 757-771 for the row mode. */
int ggq_quantize_act_dev(ggq_ctx* ctx, const float* A, int lda, int M, int K, int act_mode,
                         int8_t* q, float* scales, void* stream);

/* The producer of a prefill input and its per-row int8 quantization in one
 * launch (no reference counterpart as a fused call), so that a caller
 * feeding ggq_mul_mat_q8_dev / ggq_mul_mat_q8_batch_dev does not write the
 * fp32 rows out and read them back:
 *   GGQ_PRODUCE_RMS_NORM  x = CpuRefBackend::rms_norm of the row
 *                         (cpu_ref.cpp:139-156): a * (1/sqrt(sum(a^2)/K +
 *                         eps)) * aux[k]; aux = norm weight [K] or NULL (= 1);
 *   GGQ_PRODUCE_SWIGLU    x = silu(a) * aux[m][k], silu(v) = v / (1 +
 *                         exp(-v)) (main.cpp:3164-3165, 3474-3477); A holds
 *                         the gate rows, aux the up rows, both with stride lda.
 * then q[m][k], scales[m] from x as ggq_quantize_act_dev in GGQ_ACT_Q8_ROW
 * mode (amd_xdna.cpp:598-603, 633-639, 757-771).  K <= 16384, K and lda
 * multiples of 4, A and aux 16-byte aligned; q dense [M][K].  The result
 * equals the unfused sequence up to the order in which the norm's sum of
 * squares is added (and the device expf), i.e. a code may differ by one
 * where x / scale lies within fp32 rounding of a half-integer. */
#define GGQ_PRODUCE_RMS_NORM 1
#define GGQ_PRODUCE_SWIGLU 2
int ggq_produce_quantize_act_dev(ggq_ctx* ctx, int producer, const float* A, const float* aux, int lda, int M,
                                 int K, float eps, int8_t* q, float* scales, void* stream);

/* int32 dot products of the raw weight codes with int8 activations, per
 * scale group (32 values; 16 for Q6_K): out[(m*N + n)*G + g], G = K/group.
 * Codes: Q4_K nibble, Q5_K 5-bit value, Q6_K 6-bit - 32, Q8_0 int8, IQ4
 * codebook value.  These are the products the int8 tile kernel forms
 * (kernels/triton/compile_kernels.py:558-574 tl.dot int8 -> int32), here on
 * raw codes instead of re-quantized rows. */
int ggq_block_dot_dev(ggq_ctx* ctx, const void* W, uint32_t type, int64_t N, int64_t K,
                      const int8_t* qa, int M, int32_t* out, void* stream);

/* Expert-grouped MoE FFN for a batch of T tokens, replacing the per-token
 * expert loop of src/cli/main.cpp:3110-3193: top-k routing on the given
 * router logits, softmax over the selected, SwiGLU experts
 * down(silu(gate x) * up x), weighted combine, plus an optional shared
 * expert weighted by shared_w[t] (1 when NULL).  Expert tensors hold E
 * consecutive matrices (expert e at e * rows * row_bytes, main.cpp:3140-3150):
 * gate/up [F][H], down [H][F].  Device pointers; asynchronous. */
typedef struct {
    int T, H, F, E, top_k;
    const float* x;             /* [T][H] */
    const float* router_logits; /* [T][E] */
    uint32_t gate_type, up_type, down_type;
    const void* gate_exps;
    const void* up_exps;
    const void* down_exps;
    const void* gate_shexp; /* NULL: no shared expert */
    const void* up_shexp;
    const void* down_shexp;
    const float* shared_w; /* [T] or NULL */
    float* out;            /* [T][H] */
    int32_t* sel_experts;  /* optional [T][top_k] */
    float* sel_weights;    /* optional [T][top_k] */
} ggq_moe_params;
int ggq_moe_ffn_dev(ggq_ctx* ctx, const ggq_moe_params* p, void* stream);

/* ggq_moe_ffn_dev with the activation treatment of the expert matmuls:
 * GGQ_ACT_F32 is ggq_moe_ffn_dev; GGQ_ACT_Q8_ROW quantizes each expert
 * matmul's input per row as the XDNA backend does for every mul_mat_q call
 * of the per-token loop (amd_xdna.cpp:598-603): the token row for gate and
 * up, the SwiGLU row (fp32) for down.  That mode runs each expert's matmuls
 * for all its tokens as one grouped int8 GEMM (weights decoded once per 32
 * token rows) -- the prefill-sized path.  Extra requirements in that mode:
 * H and F multiples of 32 and at most 16384, E <= 1023, x 16-byte aligned. */
int ggq_moe_ffn_act_dev(ggq_ctx* ctx, const ggq_moe_params* p, int act_mode, void* stream);

/* Intermediates of the most recent MoE call on the context
 * (ggq_moe_ffn_dev or ggq_moe_ffn_act_dev), for checking the layer stage by
 * stage against the per-token loop of src/cli/main.cpp:3110-3193.  Device
 * pointers into the context's workspace, valid until the next call that uses
 * the workspace.  No reference counterpart (the reference keeps no
 * intermediates).  "Pair rows" are the (token, expert) rows sorted by expert:
 * routed rows grp[e] .. grp[e+1]-1 belong to expert e (grp[E] = T*top_k);
 * with a shared expert, rows T*top_k + t (t < T) are token t's shared-expert
 * rows. */
typedef struct {
    int act_mode;           /* GGQ_ACT_F32 or GGQ_ACT_Q8_ROW */
    int T, H, F, E, top_k;
    int rows;               /* T*top_k, plus T with a shared expert */
    int shared;
    const int32_t* grp;     /* [E + 1] */
    const int32_t* tok;     /* [T*top_k] token of each routed pair row */
    const int32_t* pos;     /* [T][top_k] pair row of each (token, slot) */
    const float* gate;      /* [rows][F] gate projection outputs */
    const float* up;        /* [rows][F] up projection outputs */
    const float* h;         /* [rows][F] SwiGLU rows silu(gate) * up: with
                               GGQ_ACT_F32 at decode-sized batches always, else
                               only after ggq_moe_trace_rows(ctx, 1) (else NULL) */
    const int8_t* h_codes;  /* [rows][F] GGQ_ACT_Q8_ROW: int8 codes of h */
    const float* h_scales;  /* [rows] their row scales */
    const float* down;      /* [T*top_k][H] down projection of each routed pair row */
    const float* down_shared; /* [T][H] the shared expert's, or NULL */
} ggq_moe_trace;
int ggq_moe_trace_get(const ggq_ctx* ctx, ggq_moe_trace* out);
/* on != 0: later MoE calls also write the fp32 SwiGLU rows (trace.h) that
 * they quantize or split into fp16 planes, from the same registers the
 * codes / planes come from. */
int ggq_moe_trace_rows(ggq_ctx* ctx, int on);

/* ------------------------------------------------------- synthetic data */

/* Host-side encoder float -> GGUF blocks for seeded synthetic weights (the
 * reference ships no quantizer).  x is [n_rows][K] fp32; out receives
 * n_rows * (K/blck) * type_size bytes.  Multi-threaded. */
int ggq_encode(uint32_t type, const float* x, int64_t n_rows, int64_t K, void* out);

/* Bytes of one row of K values of `type` (0 if unsupported or K not a
 * multiple of the block size). */
int64_t ggq_row_bytes(uint32_t type, int64_t K);

#ifdef __cplusplus
}
#endif
#endif /* GGQ_H */
