/*
 * ggq_oracle.c -- CPU restatement of ggnpu's quantized-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see ggq_oracle.h).  Compiled with
 * -O2 -ffp-contract=off and no -march, like the reference's -O3 build without
 * -march (CMakeLists.txt:19-20), so that every float expression rounds in the
 * same order as the reference's scalar code (no fused multiply-add).
 *
 * How each function is pinned (tests/test_oracle.py):
 *   orc_fp16_to_f32       all 65536 inputs vs the compiled reference and vs
 *                         numpy's float16 (closed form)
 *   orc_q4k_scale_min     brute force over random 12-byte inputs vs oracle/_ref
 *   orc_dequant_*         reference unit-test goldens (test_quant.cpp:209-288)
 *                         + committed vectors from oracle/_ref (bit-exact)
 *                         + closed forms (IQ4_NL = d*LUT, Q8_0 = d*q)
 *   orc_quant_act_row     closed form (numpy restatement with IEEE division and
 *                         round-half-even) + edge cases (zero row, clamp)
 *   orc_quant_act_block32 closed form only (no reference counterpart)
 *   orc_block_dot         brute force: integer sums recomputed in numpy from
 *                         the codes; codes pinned by codes*scale == dequant
 *   orc_mul_mat_f64       vs the compiled CpuRefBackend::mul_mat_q (Q4_K, Q6_K)
 *                         and vs numpy float64 matmul of the dequantized rows
 *   orc_moe_ffn_f64       vs a per-token numpy loop over orc_mul_mat_f64 rows
 *   orc_mul_mat_rowdot_f32  bit-identical to the reference decoders + the same
 *                         loop (oracle/_ref ref_rowdot_mul_mat) and to a numpy
 *                         float32 sequential cumsum over the dequantized row
 *                         (a per-block partial sum would differ in the bits)
 */
#include "ggq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- block geometry: src/gguf/tensor.cpp:18-38 ------------------------- */
int orc_block_elems(uint32_t t) {
    switch (t) {
    case ORC_Q8_0: case ORC_IQ4_NL: return 32;
    case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: case ORC_IQ4_XS: return 256;
    case ORC_F32: return 1;
    default: return 0;
    }
}

int orc_block_bytes(uint32_t t) {
    switch (t) {
    case ORC_Q8_0: return 34;
    case ORC_IQ4_NL: return 18;
    case ORC_Q4_K: return 144;
    case ORC_Q5_K: return 176;
    case ORC_Q6_K: return 210;
    case ORC_IQ4_XS: return 136;
    case ORC_F32: return 4;
    default: return 0;
    }
}

int orc_groups_per_block(uint32_t t) {
    switch (t) {
    case ORC_Q8_0: case ORC_IQ4_NL: return 1;
    case ORC_Q4_K: case ORC_Q5_K: case ORC_IQ4_XS: return 8;
    case ORC_Q6_K: return 16;
    default: return 0;
    }
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---- fp16 -> fp32: kquant.h:30-53 (== src/utils/bf16.cpp:22-46) --------
 * Normal numbers re-bias the exponent; subnormals are exact as
 * mantissa * 2^-24 (representable in fp32); exp==31 keeps the payload. */
float orc_fp16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31u, f = h & 1023u, bits;
    float r;
    if (e == 0) {
        r = (float)f * 0x1p-24f;            /* exact: f < 2^10 */
        memcpy(&bits, &r, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (f << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (f << 13);
    }
    memcpy(&r, &bits, 4);
    return r;
}

/* ---- 6-bit scale/min unpack: kquant.h:56-64 ---------------------------- */
void orc_q4k_scale_min(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m  = q[j + 4] & 63;
    } else {
        /* low 4 bits from the nibbles of q[8..11], top 2 bits from the
         * high bits of q[0..3] (scales) / q[4..7] (mins) */
        *sc = (uint8_t)((q[j + 4] & 15) | ((q[j - 4] >> 6) << 4));
        *m  = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ---- Q4_K: kquant.h:133-151 ---------------------------------------------
 * 4 chunks of 64 values; chunk c uses qs[32c..32c+31]: low nibbles are
 * values 64c+l (sub-block 2c), high nibbles 64c+32+l (sub-block 2c+1).
 * value = (d*sc)*q - (dmin*m), each product rounded separately. */
void orc_dequant_q4_k(const uint8_t* b, float* out) {
    const float d = orc_fp16_to_f32(rd16(b)), dmin = orc_fp16_to_f32(rd16(b + 2));
    const uint8_t* s = b + 4;
    const uint8_t* qs = b + 16;
    for (int c = 0; c < 4; c++) {
        uint8_t sc0, m0, sc1, m1;
        orc_q4k_scale_min(2 * c, s, &sc0, &m0);
        orc_q4k_scale_min(2 * c + 1, s, &sc1, &m1);
        const float dl0 = d * (float)sc0, ml0 = dmin * (float)m0;
        const float dl1 = d * (float)sc1, ml1 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            const uint8_t v = qs[32 * c + l];
            out[64 * c + l]      = dl0 * (float)(v & 15) - ml0;
            out[64 * c + 32 + l] = dl1 * (float)(v >> 4) - ml1;
        }
    }
}

/* ---- Q5_K: kquant.h:157-179 ---------------------------------------------
 * As Q4_K plus a fifth bit: chunk c takes bit 2c (low nibbles) and bit
 * 2c+1 (high nibbles) of qh[l]; a set bit adds 16 before scaling. */
void orc_dequant_q5_k(const uint8_t* b, float* out) {
    const float d = orc_fp16_to_f32(rd16(b)), dmin = orc_fp16_to_f32(rd16(b + 2));
    const uint8_t* s = b + 4;
    const uint8_t* qh = b + 16;
    const uint8_t* qs = b + 48;
    for (int c = 0; c < 4; c++) {
        uint8_t sc0, m0, sc1, m1;
        orc_q4k_scale_min(2 * c, s, &sc0, &m0);
        orc_q4k_scale_min(2 * c + 1, s, &sc1, &m1);
        const float dl0 = d * (float)sc0, ml0 = dmin * (float)m0;
        const float dl1 = d * (float)sc1, ml1 = dmin * (float)m1;
        for (int l = 0; l < 32; l++) {
            const uint8_t v = qs[32 * c + l];
            const int lo = (v & 15) + (((qh[l] >> (2 * c)) & 1) ? 16 : 0);
            const int hi = (v >> 4) + (((qh[l] >> (2 * c + 1)) & 1) ? 16 : 0);
            out[64 * c + l]      = dl0 * (float)lo - ml0;
            out[64 * c + 32 + l] = dl1 * (float)hi - ml1;
        }
    }
}

/* ---- Q6_K: kquant.h:182-202 ---------------------------------------------
 * Two halves of 128 values.  In half h, for l<32: ql[64h+l] low nibble and
 * qh[32h+l] bits 0-1 -> value 128h+l (scale sc[8h+l/16]); ql[64h+32+l] low
 * and qh bits 2-3 -> 128h+32+l (sc +2); ql[64h+l] high and bits 4-5 ->
 * 128h+64+l (sc +4); ql[64h+32+l] high and bits 6-7 -> 128h+96+l (sc +6).
 * value = (d*sc)*(q6-32). */
void orc_dequant_q6_k(const uint8_t* b, float* out) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    const float d = orc_fp16_to_f32(rd16(b + 208));
    for (int h = 0; h < 2; h++) {
        for (int l = 0; l < 32; l++) {
            const int g = 8 * h + l / 16;
            const uint8_t a = ql[64 * h + l], c = ql[64 * h + 32 + l], e = qh[32 * h + l];
            const int q0 = (int)((a & 15) | ((e & 3) << 4)) - 32;
            const int q1 = (int)((c & 15) | (((e >> 2) & 3) << 4)) - 32;
            const int q2 = (int)((a >> 4) | (((e >> 4) & 3) << 4)) - 32;
            const int q3 = (int)((c >> 4) | (((e >> 6) & 3) << 4)) - 32;
            out[128 * h + l]      = (d * (float)sc[g])     * (float)q0;
            out[128 * h + 32 + l] = (d * (float)sc[g + 2]) * (float)q1;
            out[128 * h + 64 + l] = (d * (float)sc[g + 4]) * (float)q2;
            out[128 * h + 96 + l] = (d * (float)sc[g + 6]) * (float)q3;
        }
    }
}

/* ---- Q8_0: src/quant/q8_0.cpp:19-25 ------------------------------------ */
void orc_dequant_q8_0(const uint8_t* b, float* out) {
    const float d = orc_fp16_to_f32(rd16(b));
    for (int j = 0; j < 32; j++) out[j] = (float)(int8_t)b[2 + j] * d;
}

/* Non-linear 4-bit codebook, src/quant/iq4_nl.cpp:16-18 (a fixed data table
 * of the GGUF format, shared with IQ4_XS, src/quant/iq4_xs.cpp:14-16). */
static const int8_t kIq4Values[16] = {
    -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113,
};

/* ---- IQ4_NL: src/quant/iq4_nl.cpp:24-31 --------------------------------
 * low nibble of qs[j] -> value j, high nibble -> value j+16; d*kv. */
void orc_dequant_iq4_nl(const uint8_t* b, float* out) {
    const float d = orc_fp16_to_f32(rd16(b));
    for (int j = 0; j < 16; j++) {
        out[j]      = d * (float)kIq4Values[b[2 + j] & 15];
        out[j + 16] = d * (float)kIq4Values[b[2 + j] >> 4];
    }
}

/* ---- IQ4_XS: src/quant/iq4_xs.cpp:21-38 --------------------------------
 * 8 sub-blocks of 32; 6-bit scale ls = nibble ib of scales_l | 2 bits ib of
 * scales_h << 4; dl = d*(ls-32); out = dl*kv. */
void orc_dequant_iq4_xs(const uint8_t* b, float* out) {
    const float d = orc_fp16_to_f32(rd16(b));
    const uint16_t sh = rd16(b + 2);
    for (int ib = 0; ib < 8; ib++) {
        const int ls = ((b[4 + ib / 2] >> (4 * (ib & 1))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
        const float dl = d * (float)(ls - 32);
        const uint8_t* qs = b + 8 + 16 * ib;
        for (int j = 0; j < 16; j++) {
            out[32 * ib + j]      = dl * (float)kIq4Values[qs[j] & 15];
            out[32 * ib + 16 + j] = dl * (float)kIq4Values[qs[j] >> 4];
        }
    }
}

int orc_dequant_blocks(uint32_t t, const uint8_t* raw, int64_t nb, float* out) {
    const int be = orc_block_elems(t), bb = orc_block_bytes(t);
    if (!be || t == ORC_F32) return 3;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t* b = raw + i * bb;
        float* o = out + i * be;
        switch (t) {
        case ORC_Q4_K: orc_dequant_q4_k(b, o); break;
        case ORC_Q5_K: orc_dequant_q5_k(b, o); break;
        case ORC_Q6_K: orc_dequant_q6_k(b, o); break;
        case ORC_Q8_0: orc_dequant_q8_0(b, o); break;
        case ORC_IQ4_NL: orc_dequant_iq4_nl(b, o); break;
        case ORC_IQ4_XS: orc_dequant_iq4_xs(b, o); break;
        default: return 3;
        }
    }
    return 0;
}

/* Integer codes in value order, derived from the same layouts as above. */
int orc_block_codes(uint32_t t, const uint8_t* b, int8_t* q) {
    switch (t) {
    case ORC_Q4_K:
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) {
                q[64 * c + l] = (int8_t)(b[16 + 32 * c + l] & 15);
                q[64 * c + 32 + l] = (int8_t)(b[16 + 32 * c + l] >> 4);
            }
        return 0;
    case ORC_Q5_K:
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) {
                const uint8_t v = b[48 + 32 * c + l], h = b[16 + l];
                q[64 * c + l] = (int8_t)((v & 15) + (((h >> (2 * c)) & 1) << 4));
                q[64 * c + 32 + l] = (int8_t)((v >> 4) + (((h >> (2 * c + 1)) & 1) << 4));
            }
        return 0;
    case ORC_Q6_K:
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l++) {
                const uint8_t a = b[64 * h + l], c = b[64 * h + 32 + l], e = b[128 + 32 * h + l];
                q[128 * h + l]      = (int8_t)(((a & 15) | ((e & 3) << 4)) - 32);
                q[128 * h + 32 + l] = (int8_t)(((c & 15) | (((e >> 2) & 3) << 4)) - 32);
                q[128 * h + 64 + l] = (int8_t)(((a >> 4) | (((e >> 4) & 3) << 4)) - 32);
                q[128 * h + 96 + l] = (int8_t)(((c >> 4) | (((e >> 6) & 3) << 4)) - 32);
            }
        return 0;
    case ORC_Q8_0:
        for (int j = 0; j < 32; j++) q[j] = (int8_t)b[2 + j];
        return 0;
    case ORC_IQ4_NL:
        for (int j = 0; j < 16; j++) {
            q[j] = kIq4Values[b[2 + j] & 15];
            q[j + 16] = kIq4Values[b[2 + j] >> 4];
        }
        return 0;
    case ORC_IQ4_XS:
        for (int ib = 0; ib < 8; ib++)
            for (int j = 0; j < 16; j++) {
                q[32 * ib + j] = kIq4Values[b[8 + 16 * ib + j] & 15];
                q[32 * ib + 16 + j] = kIq4Values[b[8 + 16 * ib + j] >> 4];
            }
        return 0;
    default:
        return 3;
    }
}

/* ---- activation quantization: amd_xdna.cpp:598-603, 633-639, 757-771 ---
 * The reference computes scale = amax/127 (or 1 for an all-zero row), then
 * inv = 1.0f/scale, then nearbyint(a*inv) clamped to [-128,127]. */
static inline int8_t orc_to_i8(float v) {
    float r = nearbyintf(v);          /* default rounding: half to even */
    if (r > 127.0f) r = 127.0f;
    if (r < -128.0f) r = -128.0f;
    return (int8_t)r;
}

void orc_quant_act_row(const float* A, int lda, int M, int K, int8_t* q, float* scale) {
    for (int m = 0; m < M; m++) {
        const float* a = A + (size_t)m * lda;
        float amax = 0.0f;
        for (int k = 0; k < K; k++) {
            const float v = fabsf(a[k]);
            if (v > amax) amax = v;
        }
        const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
        const float inv = 1.0f / s;
        scale[m] = s;
        for (int k = 0; k < K; k++) q[(size_t)m * K + k] = orc_to_i8(a[k] * inv);
    }
}

void orc_quant_act_block32(const float* A, int lda, int M, int K, int8_t* q, float* scale) {
    const int nb = K / 32;
    for (int m = 0; m < M; m++)
        for (int b = 0; b < nb; b++) {
            const float* a = A + (size_t)m * lda + 32 * b;
            float amax = 0.0f;
            for (int k = 0; k < 32; k++) {
                const float v = fabsf(a[k]);
                if (v > amax) amax = v;
            }
            const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
            const float inv = 1.0f / s;
            scale[(size_t)m * nb + b] = s;
            for (int k = 0; k < 32; k++) q[(size_t)m * K + 32 * b + k] = orc_to_i8(a[k] * inv);
        }
}

/* ---- int32 per-group dot products of raw codes with int8 activations --- */
int orc_block_dot(uint32_t t, const uint8_t* W, int64_t N, int64_t K,
                  const int8_t* qa, int M, int32_t* out) {
    const int be = orc_block_elems(t), bb = orc_block_bytes(t), gpb = orc_groups_per_block(t);
    if (!gpb || K % be) return 3;
    const int ge = be / gpb;
    const int64_t nb = K / be, G = K / ge;
    int8_t codes[256];
    for (int64_t n = 0; n < N; n++)
        for (int64_t b = 0; b < nb; b++) {
            orc_block_codes(t, W + (n * nb + b) * bb, codes);
            for (int m = 0; m < M; m++)
                for (int g = 0; g < gpb; g++) {
                    int32_t s = 0;
                    for (int j = 0; j < ge; j++)
                        s += (int32_t)codes[g * ge + j] * (int32_t)qa[(size_t)m * K + b * be + g * ge + j];
                    out[((size_t)m * N + n) * G + b * gpb + g] = s;
                }
        }
    return 0;
}

/* ---- fp64 matmul oracle -------------------------------------------------- */
int orc_mul_mat_f64(uint32_t t, const uint8_t* W, int64_t N, int64_t K,
                    const float* A, int lda, int M, int act_mode, double* C, int ldc) {
    const int be = orc_block_elems(t), bb = orc_block_bytes(t);
    if (!be || t == ORC_F32 || K % be) return 3;
    const int64_t nb = K / be;
    double* a = (double*)malloc(sizeof(double) * (size_t)M * K);
    float* w = (float*)malloc(sizeof(float) * (size_t)K);
    int8_t* q = NULL;
    float* s = NULL;
    if (!a || !w) { free(a); free(w); return 5; }
    if (act_mode == ORC_ACT_F32) {
        for (int m = 0; m < M; m++)
            for (int64_t k = 0; k < K; k++) a[(size_t)m * K + k] = A[(size_t)m * lda + k];
    } else {
        q = (int8_t*)malloc((size_t)M * K);
        s = (float*)malloc(sizeof(float) * (size_t)M * (K / 32));
        if (act_mode == ORC_ACT_Q8_ROW) {
            orc_quant_act_row(A, lda, M, (int)K, q, s);
            for (int m = 0; m < M; m++)
                for (int64_t k = 0; k < K; k++) a[(size_t)m * K + k] = (double)q[(size_t)m * K + k] * (double)s[m];
        } else {
            orc_quant_act_block32(A, lda, M, (int)K, q, s);
            for (int m = 0; m < M; m++)
                for (int64_t k = 0; k < K; k++)
                    a[(size_t)m * K + k] = (double)q[(size_t)m * K + k] * (double)s[(size_t)m * (K / 32) + k / 32];
        }
    }
    for (int64_t n = 0; n < N; n++) {
        orc_dequant_blocks(t, W + n * nb * bb, nb, w);
        for (int m = 0; m < M; m++) {
            double acc = 0.0;
            const double* am = a + (size_t)m * K;
            for (int64_t k = 0; k < K; k++) acc += am[k] * (double)w[k];
            C[(size_t)m * ldc + n] = acc;
        }
    }
    free(a); free(w); free(q); free(s);
    return 0;
}

/* ---- CpuRefBackend::mul_mat_q fp32 path (cpu_ref.cpp:87-117) ------------
 * For each row n and block b: dequantize, then for each m an fp32 partial
 * sum over the block, added into C[m][n] (C zeroed first, cpu_ref.cpp:33). */
int orc_mul_mat_cpuref_f32(uint32_t t, const uint8_t* W, int64_t N, int64_t K,
                           const float* A, int lda, int M, float* C, int ldc) {
    const int be = orc_block_elems(t), bb = orc_block_bytes(t);
    if (!be || t == ORC_F32 || K % be) return 3;
    const int64_t nb = K / be;
    float w[256];
    for (int m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) C[(size_t)m * ldc + n] = 0.0f;
    for (int64_t n = 0; n < N; n++)
        for (int64_t b = 0; b < nb; b++) {
            orc_dequant_blocks(t, W + (n * nb + b) * bb, 1, w);
            for (int m = 0; m < M; m++) {
                const float* am = A + (size_t)m * lda + b * be;
                float sum = 0.0f;
                for (int j = 0; j < be; j++) sum += am[j] * w[j];
                C[(size_t)m * ldc + n] += sum;
            }
        }
    return 0;
}

/* ---- dequantize-row + fp32 dot: main.cpp:317-326 and :1380-1386 -----------
 * The CLI's loop for weights no backend takes: the whole row is decoded
 * (dequant_tensor_row, main.cpp:36-...), then one running fp32 sum over k. */
int orc_mul_mat_rowdot_f32(uint32_t t, const uint8_t* W, int64_t N, int64_t K,
                           const float* A, int lda, int M, float* C, int ldc) {
    const int be = orc_block_elems(t), bb = orc_block_bytes(t);
    if (!be || t == ORC_F32 || K % be) return 3;
    const int64_t nb = K / be;
    float* row = (float*)malloc((size_t)K * sizeof(float));
    if (!row) return 2;
    for (int64_t n = 0; n < N; n++) {
        orc_dequant_blocks(t, W + n * nb * bb, nb, row);
        for (int m = 0; m < M; m++) {
            const float* am = A + (size_t)m * lda;
            float acc = 0.0f;
            for (int64_t k = 0; k < K; k++) acc += am[k] * row[k];
            C[(size_t)m * ldc + n] = acc;
        }
    }
    free(row);
    return 0;
}

/* ---- MoE FFN: main.cpp:3110-3193 ------------------------------------------
 * Per token: top-k experts by descending router logit (partial_sort, :3128);
 * weights = softmax over the selected logits (:3132-3135); for each selected
 * expert down(silu(gate x) * up x) accumulated with its weight (:3156-3169);
 * shared expert added with its gate weight (:3177-3191). Expert e of a 3-D
 * tensor starts at e * rows * row_bytes (:3140-3150). */
static double orc_silu_f64(double v) { return v / (1.0 + exp(-v)); }

int orc_moe_ffn_f64(const float* x, const float* logits, int T, int H, int F, int E, int topk,
                    uint32_t tg, const uint8_t* Wg, uint32_t tu, const uint8_t* Wu,
                    uint32_t td, const uint8_t* Wd,
                    const uint8_t* Sg, const uint8_t* Su, const uint8_t* Sd,
                    const float* shared_w, double* out,
                    int32_t* sel_experts, float* sel_weights) {
    return orc_moe_ffn_act_f64(x, logits, T, H, F, E, topk, tg, Wg, tu, Wu, td, Wd, Sg, Su, Sd, shared_w,
                               ORC_ACT_F32, out, sel_experts, sel_weights);
}

/* The same with each expert matmul under an activation treatment
 * (act_mode as orc_mul_mat_f64): with ORC_ACT_Q8_ROW the token row is
 * quantized per row for gate / up and the SwiGLU row, rounded to fp32 as
 * the reference holds it (main.cpp:3164-3165), is quantized per row for
 * down -- each mul_mat_weight call of the per-token loop quantizing its own
 * input (amd_xdna.cpp:598-603). */
int orc_moe_ffn_act_f64(const float* x, const float* logits, int T, int H, int F, int E, int topk,
                        uint32_t tg, const uint8_t* Wg, uint32_t tu, const uint8_t* Wu,
                        uint32_t td, const uint8_t* Wd,
                        const uint8_t* Sg, const uint8_t* Su, const uint8_t* Sd,
                        const float* shared_w, int act_mode, double* out,
                        int32_t* sel_experts, float* sel_weights) {
    const size_t gbytes = (size_t)F * (H / orc_block_elems(tg)) * orc_block_bytes(tg);
    const size_t ubytes = (size_t)F * (H / orc_block_elems(tu)) * orc_block_bytes(tu);
    const size_t dbytes = (size_t)H * (F / orc_block_elems(td)) * orc_block_bytes(td);
    double* g = (double*)malloc(sizeof(double) * F);
    double* u = (double*)malloc(sizeof(double) * F);
    double* d = (double*)malloc(sizeof(double) * H);
    float* act = (float*)malloc(sizeof(float) * F);
    int* idx = (int*)malloc(sizeof(int) * E);
    int sel_idx[64];
    if (topk > 64) { free(g); free(u); free(d); free(act); free(idx); return 3; }
    if (!g || !u || !d || !act || !idx) { free(g); free(u); free(d); free(act); free(idx); return 5; }
    for (int t = 0; t < T; t++) {
        const float* xt = x + (size_t)t * H;
        const float* lt = logits + (size_t)t * E;
        double* ot = out + (size_t)t * H;
        for (int i = 0; i < H; i++) ot[i] = 0.0;
        /* top-k by descending logit, ties to the lower expert id; a NaN
         * logit ranks with -inf (the reference's partial_sort has no order
         * for NaN; this rule keeps every selection a valid expert id) */
        for (int e = 0; e < E; e++) idx[e] = 0; /* taken flags */
        for (int j = 0; j < topk; j++) {
            int best = -1;
            float bv = -INFINITY;
            for (int e = 0; e < E; e++) {
                if (idx[e]) continue;
                const float v = isnan(lt[e]) ? -INFINITY : lt[e];
                if (best < 0 || v > bv) { best = e; bv = v; }
            }
            idx[best] = 1;
            sel_idx[j] = best;
        }
        double wsum = 0.0, wv[64];
        for (int j = 0; j < topk; j++) { wv[j] = exp((double)lt[sel_idx[j]] - (double)lt[sel_idx[0]]); wsum += wv[j]; }
        for (int j = 0; j < topk + 1; j++) {
            const uint8_t *pg, *pu, *pd;
            double wj;
            if (j < topk) {
                const int e = sel_idx[j];
                wj = wv[j] / wsum;
                if (sel_experts) sel_experts[t * topk + j] = e;
                if (sel_weights) sel_weights[t * topk + j] = (float)wj;
                pg = Wg + e * gbytes; pu = Wu + e * ubytes; pd = Wd + e * dbytes;
            } else {
                if (!Sg) break;
                wj = shared_w ? (double)shared_w[t] : 1.0;
                pg = Sg; pu = Su; pd = Sd;
            }
            orc_mul_mat_f64(tg, pg, F, H, xt, H, 1, act_mode, g, F);
            orc_mul_mat_f64(tu, pu, F, H, xt, H, 1, act_mode, u, F);
            for (int i = 0; i < F; i++) act[i] = (float)(orc_silu_f64(g[i]) * u[i]);
            orc_mul_mat_f64(td, pd, H, F, act, F, 1, act_mode, d, H);
            for (int i = 0; i < H; i++) ot[i] += wj * d[i];
        }
    }
    free(g); free(u); free(d); free(act); free(idx);
    return 0;
}

/* cpu_ref.cpp:139-156: variance accumulated in fp32 in index order. */
void orc_rms_norm(const float* x, int n, const float* w, float eps, float* out) {
    float variance = 0.0f;
    for (int i = 0; i < n; i++) variance += x[i] * x[i];
    variance /= (float)n;
    variance += eps;
    const float inv_std = 1.0f / sqrtf(variance);
    for (int i = 0; i < n; i++) out[i] = x[i] * inv_std * (w ? w[i] : 1.0f);
}

/* cpu_ref.cpp:200-209. */
void orc_silu(const float* x, int n, float* out) {
    for (int i = 0; i < n; i++) out[i] = x[i] / (1.0f + expf(-x[i]));
}

/* cpu_ref.cpp:223-280, fp32, one query row. */
void orc_flash_attn(const float* Q, const float* K, const float* V, int n_head, int hd, int64_t cl,
                    int64_t query_pos, float* out) {
    const int64_t qpos = query_pos >= 0 ? query_pos : cl - 1;
    const float scale = 1.0f / sqrtf((float)hd);
    float* scores = (float*)malloc(sizeof(float) * (size_t)(cl > 0 ? cl : 1));
    float* weights = (float*)malloc(sizeof(float) * (size_t)(cl > 0 ? cl : 1));
    for (int h = 0; h < n_head; h++) {
        const float* Qh = Q + (int64_t)h * hd;
        const float* Kh = K + (int64_t)h * cl * hd;
        const float* Vh = V + (int64_t)h * cl * hd;
        float* outh = out + (int64_t)h * hd;
        for (int64_t j = 0; j < cl; j++) scores[j] = -INFINITY;
        for (int64_t j = 0; j <= qpos && j < cl; j++) {
            float sum = 0.0f;
            for (int d = 0; d < hd; d++) sum += Qh[d] * Kh[j * hd + d];
            scores[j] = sum * scale;
        }
        float max_val = -INFINITY;
        for (int64_t j = 0; j < cl; j++)
            if (scores[j] > max_val) max_val = scores[j];
        float sum = 0.0f;
        for (int64_t j = 0; j < cl; j++) {
            weights[j] = expf(scores[j] - max_val);
            sum += weights[j];
        }
        for (int64_t j = 0; j < cl; j++) weights[j] /= sum;
        for (int d = 0; d < hd; d++) outh[d] = 0.0f;
        for (int64_t j = 0; j < cl; j++)
            for (int d = 0; d < hd; d++) outh[d] += weights[j] * Vh[j * hd + d];
    }
    free(scores);
    free(weights);
}

void orc_flash_attn_f64(const float* Q, const float* K, const float* V, int n_head, int hd, int64_t cl,
                        int64_t query_pos, double* out) {
    const int64_t qpos = query_pos >= 0 ? query_pos : cl - 1;
    const double scale = 1.0 / sqrt((double)hd);
    const int64_t n = qpos + 1 < cl ? qpos + 1 : cl;
    double* w = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
    for (int h = 0; h < n_head; h++) {
        const float* Qh = Q + (int64_t)h * hd;
        const float* Kh = K + (int64_t)h * cl * hd;
        const float* Vh = V + (int64_t)h * cl * hd;
        double m = -INFINITY;
        for (int64_t j = 0; j < n; j++) {
            double s = 0.0;
            for (int d = 0; d < hd; d++) s += (double)Qh[d] * (double)Kh[j * hd + d];
            w[j] = s * scale;
            if (w[j] > m) m = w[j];
        }
        double tot = 0.0;
        for (int64_t j = 0; j < n; j++) {
            w[j] = exp(w[j] - m);
            tot += w[j];
        }
        for (int d = 0; d < hd; d++) {
            double acc = 0.0;
            for (int64_t j = 0; j < n; j++) acc += w[j] * (double)Vh[j * hd + d];
            out[(int64_t)h * hd + d] = acc / tot;
        }
    }
    free(w);
}
