/*
 * ggq_oracle.h -- CPU restatement of ggnpu's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker (or as the timed CPU
 * baseline), never as the thing measured on the GPU.
 *
 * Every function cites the reference file:line (relative to the ggnpu tree)
 * whose behaviour it restates.  Parity of each function is pinned in tests/
 * against (1) the reference's own unit-test goldens, (2) vectors produced by
 * the reference sources compiled into oracle/_ref, and (3) closed forms /
 * brute force; see the table at the top of ggq_oracle.c.
 */
#ifndef GGQ_ORACLE_H
#define GGQ_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (include/ggnpu/tensor.h:11-42). */
enum {
    ORC_F32 = 0, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14,
    ORC_IQ4_NL = 20, ORC_IQ4_XS = 23
};

/* Activation treatments. */
enum { ORC_ACT_F32 = 0, ORC_ACT_Q8_ROW = 1, ORC_ACT_Q8_BLOCK32 = 2 };

/* Block geometry (src/gguf/tensor.cpp:18-38). Returns 0 for unsupported. */
int    orc_block_elems(uint32_t type);
int    orc_block_bytes(uint32_t type);
/* Number of scale groups per block and elements per group (the granularity
 * of the int32 "block dot" products).  Q6_K: 16 groups of 16. */
int    orc_groups_per_block(uint32_t type);

float  orc_fp16_to_f32(uint16_t h);                                   /* kquant.h:30-53 */
void   orc_q4k_scale_min(int j, const uint8_t* q, uint8_t* sc, uint8_t* m); /* kquant.h:56-64 */

void   orc_dequant_q4_k(const uint8_t* blk, float* out);   /* kquant.h:133-151 */
void   orc_dequant_q5_k(const uint8_t* blk, float* out);   /* kquant.h:157-179 */
void   orc_dequant_q6_k(const uint8_t* blk, float* out);   /* kquant.h:182-202 */
void   orc_dequant_q8_0(const uint8_t* blk, float* out);   /* q8_0.cpp:19-25 */
void   orc_dequant_iq4_nl(const uint8_t* blk, float* out); /* iq4_nl.cpp:24-31 */
void   orc_dequant_iq4_xs(const uint8_t* blk, float* out); /* iq4_xs.cpp:21-38 */

/* Dequantize n_blocks consecutive blocks. Returns 0 on success. */
int    orc_dequant_blocks(uint32_t type, const uint8_t* raw, int64_t n_blocks, float* out);

/* Raw integer codes of one block (the values the int32 block dot multiplies):
 * Q4_K nibble, Q5_K 5-bit value, Q6_K (6-bit - 32), Q8_0 int8, IQ4 kvalue. */
int    orc_block_codes(uint32_t type, const uint8_t* blk, int8_t* codes);

/* Per-row int8 activation quantization (amd_xdna.cpp:598-603, 633-639,
 * 757-771): scale = amax>0 ? amax/127 : 1; q = clamp(nearbyint(a*(1/scale))). */
void   orc_quant_act_row(const float* A, int lda, int M, int K, int8_t* q, float* scale);
/* Per-32-block variant (extension; no reference counterpart).
 * scale[m*(K/32)+b] = amax_b>0 ? amax_b/127 : 1; same rounding as above. */
void   orc_quant_act_block32(const float* A, int lda, int M, int K, int8_t* q, float* scale);

/* int32 products per scale group: out[(m*N + n)*G + g] with G = K/group. */
int    orc_block_dot(uint32_t type, const uint8_t* W, int64_t N, int64_t K,
                     const int8_t* qa, int M, int32_t* out);

/* fp64 oracle of C = A . W^T with the given activation treatment, using the
 * exactly dequantized fp32 weights. C is [M][ldc] (double). */
int    orc_mul_mat_f64(uint32_t type, const uint8_t* W, int64_t N, int64_t K,
                       const float* A, int lda, int M, int act_mode,
                       double* C, int ldc);

/* fp32, single-threaded restatement of CpuRefBackend::mul_mat_q
 * (cpu_ref.cpp:87-117) generalised to all six types through the
 * main.cpp:36-261 dequant dispatch: per-block fp32 partial sum added to C. */
int    orc_mul_mat_cpuref_f32(uint32_t type, const uint8_t* W, int64_t N, int64_t K,
                              const float* A, int lda, int M, float* C, int ldc);

/* RMSNorm, restating CpuRefBackend::rms_norm (cpu_ref.cpp:139-156) in its
 * fp32 order: sum of squares in index order, / n, + eps, 1/sqrt, then
 * out[i] = x[i] * inv * w[i] (w NULL = 1). */
/* main.cpp:317-326 dequant-row + fp32 dot (weights no backend takes) */
int    orc_mul_mat_rowdot_f32(uint32_t type, const uint8_t* W, int64_t N, int64_t K,
                              const float* A, int lda, int M, float* C, int ldc);
void   orc_rms_norm(const float* x, int n, const float* w, float eps, float* out);
/* silu, restating CpuRefBackend::silu (cpu_ref.cpp:200-209):
 * out[i] = x[i] / (1 + expf(-x[i])) in fp32. */
void   orc_silu(const float* x, int n, float* out);

/* Decode attention, restating CpuRefBackend::flash_attn (cpu_ref.cpp:223-280)
 * in its fp32 order for one query row: Q [n_head][hd]; K, V head-major
 * [n_head][ctx_len][hd] (the GQA expansion of main.cpp:3358-3379); scores for
 * positions <= query_pos (< 0: ctx_len - 1), softmax with the max
 * subtracted, out [n_head][hd] = sum_j w_j V_j. */
void   orc_flash_attn(const float* Q, const float* K, const float* V, int n_head, int hd, int64_t ctx_len,
                      int64_t query_pos, float* out);
/* The same in fp64 (the parity target). */
void   orc_flash_attn_f64(const float* Q, const float* K, const float* V, int n_head, int hd, int64_t ctx_len,
                          int64_t query_pos, double* out);

/* MoE FFN oracle (main.cpp:3110-3193) in fp64 over dequantized weights.
 *   x [T][H] fp32, logits [T][E] fp32 router logits
 *   gate/up expert tensor: E consecutive [F][H] matrices (type tg, tu)
 *   down expert tensor:    E consecutive [H][F] matrices (type td)
 *   optional shared expert (sg/su/sd, may be NULL) weighted by shared_w[t]
 *   out [T][H] double.  Top-k by descending logit; softmax over the selected. */
int    orc_moe_ffn_f64(const float* x, const float* logits, int T, int H, int F, int E, int topk,
                       uint32_t tg, const uint8_t* Wg, uint32_t tu, const uint8_t* Wu,
                       uint32_t td, const uint8_t* Wd,
                       const uint8_t* Sg, const uint8_t* Su, const uint8_t* Sd,
                       const float* shared_w, double* out,
                       int32_t* sel_experts, float* sel_weights);
/* orc_moe_ffn_f64 with each expert matmul under act_mode (ORC_ACT_F32 or
 * ORC_ACT_Q8_ROW; the SwiGLU row is rounded to fp32 before it is quantized). */
int    orc_moe_ffn_act_f64(const float* x, const float* logits, int T, int H, int F, int E, int topk,
                           uint32_t tg, const uint8_t* Wg, uint32_t tu, const uint8_t* Wu,
                           uint32_t td, const uint8_t* Wd,
                           const uint8_t* Sg, const uint8_t* Su, const uint8_t* Sd,
                           const float* shared_w, int act_mode, double* out,
                           int32_t* sel_experts, float* sel_weights);

#ifdef __cplusplus
}
#endif
#endif
