// ggq_device.h -- device-side decoding of raw GGUF blocks for CDNA4 (gfx950).
//
// Three views of the same block formats live here:
//   * codes16<T>(row, k): 16 signed int8 "codes" for values k..k+15 of a row,
//     packed 4 per dword in natural k order.  Codes are the integers the
//     format scales: Q4_K nibble, Q5_K 5-bit value, Q6_K (6-bit - 32), Q8_0
//     int8, IQ4_NL/IQ4_XS codebook entry.  Used by the bit-exact dequant
//     kernel, the int32 block-dot kernel and the int8-MFMA GEMM.
//   * group scales (dl, ml) per scale group, computed exactly as the
//     reference does (fp16 -> fp32, then one rounded fp32 multiply).
//   * Piece<T>: the decode-GEMV view.  A piece is 32 values of one row laid
//     out as two runs of 16 consecutive k; it is decoded to unsigned byte codes
//     u plus four coefficients so that
//        sum_k x_k w_k = a0*sum(x_run0*u0) + b0*sum(x_run0)
//                      + a1*sum(x_run1*u1) + b1*sum(x_run1).
//     Signed codes are biased to unsigned bytes (v_cvt_f32_ubyteN converts
//     them in one instruction) and the bias is removed through b*sum(x).
//
// Format references (ggnpu): include/ggnpu/quant/kquant.h:9-20 (K-quant
// layouts), :56-64 (6-bit scale/min packing), :133-202 (dequant order),
// src/quant/q8_0.cpp:19-25, src/quant/iq4_nl.cpp:16-31,
// src/quant/iq4_xs.cpp:21-38.
#pragma once
#include "ggq_launch.h"
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "ggq_formats.h"

namespace ggq {

// ---------------------------------------------------------------- loads --

// Unaligned 16-byte load: reads the dword-aligned window that covers
// [p, p+16) (5 dwords, at most 4 bytes past p+16) and realigns it with
// v_alignbyte.  Pointer arithmetic (not integer casts) keeps the global
// address space, so these are global_load_dword* instructions.
__device__ __forceinline__ uint4 ld16_u(const uint8_t* p) {
    const uint32_t s = (uint32_t)(uintptr_t)p & 3u;
    const uint32_t* q = (const uint32_t*)(p - s);
    const uint32_t d0 = q[0], d1 = q[1], d2 = q[2], d3 = q[3], d4 = q[4];
    uint4 r;
    r.x = __builtin_amdgcn_alignbyte(d1, d0, s);
    r.y = __builtin_amdgcn_alignbyte(d2, d1, s);
    r.z = __builtin_amdgcn_alignbyte(d3, d2, s);
    r.w = __builtin_amdgcn_alignbyte(d4, d3, s);
    return r;
}

// Unaligned 8-byte load (3 dwords window).
__device__ __forceinline__ uint2 ld8_u(const uint8_t* p) {
    const uint32_t s = (uint32_t)(uintptr_t)p & 3u;
    const uint32_t* q = (const uint32_t*)(p - s);
    const uint32_t d0 = q[0], d1 = q[1], d2 = q[2];
    return make_uint2(__builtin_amdgcn_alignbyte(d1, d0, s), __builtin_amdgcn_alignbyte(d2, d1, s));
}

// 16-bit little-endian load from an even address.
__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return *(const uint16_t*)p; }

__device__ __forceinline__ uint4 ld16_a(const uint8_t* p) { return *(const uint4*)p; }

// Exact IEEE half -> float (v_cvt_f32_f16; fp16 subnormals are preserved).
__device__ __forceinline__ float h2f(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

__device__ __forceinline__ uint32_t byte_at(uint32_t w0, uint32_t w1, uint32_t w2, int i) {
    const uint32_t w = i < 4 ? w0 : (i < 8 ? w1 : w2);
    return (w >> (8 * (i & 3))) & 0xFFu;
}

// 6-bit scale and min of sub-block j (0..7) from the 12 packed bytes held in
// w0..w2 (Q4_K/Q5_K header bytes 4..15).  j<4: low 6 bits of bytes j and
// j+4.  j>=4: low nibble / high nibble of byte j+4, plus the top two bits of
// bytes j-4 (scale) and j (min).
__device__ __forceinline__ void kq_scale_min(uint32_t w0, uint32_t w1, uint32_t w2, int j,
                                             uint32_t& sc, uint32_t& m) {
    if (j < 4) {
        sc = byte_at(w0, w1, w2, j) & 63u;
        m = byte_at(w0, w1, w2, j + 4) & 63u;
    } else {
        const uint32_t c = byte_at(w0, w1, w2, j + 4);
        sc = (c & 15u) | ((byte_at(w0, w1, w2, j - 4) >> 6) << 4);
        m = (c >> 4) | ((byte_at(w0, w1, w2, j) >> 6) << 4);
    }
}

// Scales and mins of the sub-block pair 2c, 2c+1 of a K-quant block as four
// bytes [sc(2c), sc(2c+1), m(2c), m(2c+1)]: the same values as kq_scale_min,
// gathered with v_perm (the byte pattern depends only on c, which is fixed
// per lane in the decode GEMV) and without branches.  With b = 2*(c&1),
// A = scale bytes b, b+1, b+4, b+5 and B = bytes b, b+1, b, b+1 of w2:
// c < 2 keeps the low 6 bits of A; c >= 2 takes the low / high nibbles of B
// for sc / m and bits 6-7 of A as bits 4-5.
__device__ __forceinline__ uint32_t kq_pair(uint32_t w0, uint32_t w1, uint32_t w2, int c) {
    const uint32_t b = 2u * (uint32_t)(c & 1);
    const uint32_t a = __builtin_amdgcn_perm(w1, w0, b | (b + 1) << 8 | (b + 4) << 16 | (b + 5) << 24);
    const uint32_t q = __builtin_amdgcn_perm(w2, w2, b | (b + 1) << 8 | b << 16 | (b + 1) << 24);
    const uint32_t hi = ((a >> 2) & 0x30303030u) | (q & 0x00000F0Fu) | ((q >> 4) & 0x0F0F0000u);
    return c >= 2 ? hi : a & 0x3F3F3F3Fu;
}

// ---------------------------------------------------- IQ4 codebook lookup --
// Codebook of IQ4_NL/IQ4_XS (src/quant/iq4_nl.cpp:16-18), packed 4 per dword
// little-endian.  kIq4S: signed entries.  kIq4U: entries + 128 (unsigned).
#define GGQ_IQ4S0 0xBFAD9881u  // -127 -104 -83 -65
#define GGQ_IQ4S1 0xF6EADDCFu  //  -49  -35 -22 -10
#define GGQ_IQ4S2 0x26190D01u  //    1   13  25  38
#define GGQ_IQ4S3 0x71594535u  //   53   69  89 113
#define GGQ_IQ4U0 0x3F2D1801u
#define GGQ_IQ4U1 0x766A5D4Fu
#define GGQ_IQ4U2 0xA6998D81u
#define GGQ_IQ4U3 0xF1D9C5B5u

// Per-byte table lookup of 4 nibbles (one per byte, values 0..15): v_perm
// picks from the 8-byte half tables, v_bfi merges on bit 3.
__device__ __forceinline__ uint32_t lut16(uint32_t nib, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
    const uint32_t sel = nib & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
    const uint32_t msk = ((nib >> 3) & 0x01010101u) * 0xFFu;
    return (hi & msk) | (lo & ~msk);
}

__device__ __forceinline__ uint4 lut16x4(uint4 n, bool biased) {
    uint4 r;
    if (biased) {
        r.x = lut16(n.x, GGQ_IQ4U0, GGQ_IQ4U1, GGQ_IQ4U2, GGQ_IQ4U3);
        r.y = lut16(n.y, GGQ_IQ4U0, GGQ_IQ4U1, GGQ_IQ4U2, GGQ_IQ4U3);
        r.z = lut16(n.z, GGQ_IQ4U0, GGQ_IQ4U1, GGQ_IQ4U2, GGQ_IQ4U3);
        r.w = lut16(n.w, GGQ_IQ4U0, GGQ_IQ4U1, GGQ_IQ4U2, GGQ_IQ4U3);
    } else {
        r.x = lut16(n.x, GGQ_IQ4S0, GGQ_IQ4S1, GGQ_IQ4S2, GGQ_IQ4S3);
        r.y = lut16(n.y, GGQ_IQ4S0, GGQ_IQ4S1, GGQ_IQ4S2, GGQ_IQ4S3);
        r.z = lut16(n.z, GGQ_IQ4S0, GGQ_IQ4S1, GGQ_IQ4S2, GGQ_IQ4S3);
        r.w = lut16(n.w, GGQ_IQ4S0, GGQ_IQ4S1, GGQ_IQ4S2, GGQ_IQ4S3);
    }
    return r;
}

__device__ __forceinline__ uint4 and4(uint4 v, uint32_t m) { return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m); }
__device__ __forceinline__ uint4 shr4(uint4 v, uint32_t s) { return make_uint4(v.x >> s, v.y >> s, v.z >> s, v.w >> s); }
__device__ __forceinline__ uint4 or4(uint4 a, uint4 b) { return make_uint4(a.x | b.x, a.y | b.y, a.z | b.z, a.w | b.w); }
__device__ __forceinline__ uint4 xor4(uint4 v, uint32_t m) { return make_uint4(v.x ^ m, v.y ^ m, v.z ^ m, v.w ^ m); }
__device__ __forceinline__ uint4 shl4(uint4 v, uint32_t s) { return make_uint4(v.x << s, v.y << s, v.z << s, v.w << s); }

// 6-bit offset-binary bytes (0..63) -> signed bytes (u - 32): flip bit 5,
// then copy bit 5 into bits 6-7 (0x20*6 = 0xC0, no carry between bytes).
__device__ __forceinline__ uint32_t six_to_s8(uint32_t u) {
    const uint32_t t = u ^ 0x20202020u;
    return t | ((t & 0x20202020u) * 6u);
}

// ------------------------------------------------------- codes16<T> ------
// 16 signed codes for values k..k+15 of the row starting at `row`
// (k a multiple of 16).
template <int T> __device__ __forceinline__ uint4 codes16(const uint8_t* row, int k);

template <> __device__ __forceinline__ uint4 codes16<T_Q4_K>(const uint8_t* row, int k) {
    const uint8_t* b = row + (k >> 8) * 144;
    const int kk = k & 255, c = kk >> 6, hi = (kk >> 5) & 1, off = kk & 16;
    const uint4 q = ld16_a(b + 16 + 32 * c + off);
    return and4(shr4(q, 4 * hi), 0x0F0F0F0Fu);
}

template <> __device__ __forceinline__ uint4 codes16<T_Q5_K>(const uint8_t* row, int k) {
    const uint8_t* b = row + (k >> 8) * 176;
    const int kk = k & 255, c = kk >> 6, hi = (kk >> 5) & 1, off = kk & 16;
    const uint4 q = ld16_a(b + 48 + 32 * c + off);
    const uint4 h = ld16_a(b + 16 + off);
    return or4(and4(shr4(q, 4 * hi), 0x0F0F0F0Fu), shl4(and4(shr4(h, 2 * c + hi), 0x01010101u), 4));
}

template <> __device__ __forceinline__ uint4 codes16<T_Q6_K>(const uint8_t* row, int k) {
    const uint8_t* b = row + (k >> 8) * 210;
    const int kk = k & 255, h = kk >> 7, r = kk & 127, qd = r >> 5, l0 = r & 16;
    const uint4 ql = ld16_u(b + 64 * h + 32 * (qd & 1) + l0);
    const uint4 qh = ld16_u(b + 128 + 32 * h + l0);
    const uint4 u = or4(and4(shr4(ql, 4 * (qd >> 1)), 0x0F0F0F0Fu), shl4(and4(shr4(qh, 2 * qd), 0x03030303u), 4));
    return make_uint4(six_to_s8(u.x), six_to_s8(u.y), six_to_s8(u.z), six_to_s8(u.w));
}

template <> __device__ __forceinline__ uint4 codes16<T_Q8_0>(const uint8_t* row, int k) {
    return ld16_u(row + (k >> 5) * 34 + 2 + (k & 16));
}

template <> __device__ __forceinline__ uint4 codes16<T_IQ4_NL>(const uint8_t* row, int k) {
    const uint4 q = ld16_u(row + (k >> 5) * 18 + 2);
    return lut16x4(and4(shr4(q, (k & 16) >> 2), 0x0F0F0F0Fu), false);
}

template <> __device__ __forceinline__ uint4 codes16<T_IQ4_XS>(const uint8_t* row, int k) {
    const uint8_t* b = row + (k >> 8) * 136;
    const int ib = (k & 255) >> 5;
    const uint2 lo = *(const uint2*)(b + 8 + 16 * ib);
    const uint2 hi = *(const uint2*)(b + 16 + 16 * ib);
    const uint4 q = make_uint4(lo.x, lo.y, hi.x, hi.y);
    return lut16x4(and4(shr4(q, (k & 16) >> 2), 0x0F0F0F0Fu), false);
}

// ------------------------------------------------------ group scales -----
// Scale (dl) and offset (ml) of the group containing value k, computed with
// the reference's rounding: dl = d*sc, ml = dmin*m (one fp32 multiply each).
// Value = dl*code - ml (ml = 0 for formats without a min).
struct GroupScale { float dl, ml; };

template <int T> __device__ __forceinline__ GroupScale group_scale(const uint8_t* row, int k);

template <> __device__ __forceinline__ GroupScale group_scale<T_Q4_K>(const uint8_t* row, int k) {
    const uint4 hd = ld16_a(row + (k >> 8) * 144);
    uint32_t sc, m;
    kq_scale_min(hd.y, hd.z, hd.w, (k & 255) >> 5, sc, m);
    return {__fmul_rn(h2f(hd.x & 0xFFFFu), (float)sc), __fmul_rn(h2f(hd.x >> 16), (float)m)};
}

template <> __device__ __forceinline__ GroupScale group_scale<T_Q5_K>(const uint8_t* row, int k) {
    const uint4 hd = ld16_a(row + (k >> 8) * 176);
    uint32_t sc, m;
    kq_scale_min(hd.y, hd.z, hd.w, (k & 255) >> 5, sc, m);
    return {__fmul_rn(h2f(hd.x & 0xFFFFu), (float)sc), __fmul_rn(h2f(hd.x >> 16), (float)m)};
}

template <> __device__ __forceinline__ GroupScale group_scale<T_Q6_K>(const uint8_t* row, int k) {
    const uint8_t* b = row + (k >> 8) * 210;
    const int sc = (int)(int8_t)b[192 + ((k & 255) >> 4)];
    return {__fmul_rn(h2f(ld_u16(b + 208)), (float)sc), 0.0f};
}

template <> __device__ __forceinline__ GroupScale group_scale<T_Q8_0>(const uint8_t* row, int k) {
    return {h2f(ld_u16(row + (k >> 5) * 34)), 0.0f};
}

template <> __device__ __forceinline__ GroupScale group_scale<T_IQ4_NL>(const uint8_t* row, int k) {
    return {h2f(ld_u16(row + (k >> 5) * 18)), 0.0f};
}

template <> __device__ __forceinline__ GroupScale group_scale<T_IQ4_XS>(const uint8_t* row, int k) {
    const uint8_t* b = row + (k >> 8) * 136;
    const uint2 hd = *(const uint2*)b;
    const int ib = (k & 255) >> 5;
    const int ls = (int)(((hd.y >> (8 * (ib >> 1) + 4 * (ib & 1))) & 15u) | (((hd.x >> (16 + 2 * ib)) & 3u) << 4));
    return {__fmul_rn(h2f(hd.x & 0xFFFFu), (float)(ls - 32)), 0.0f};
}

// Dequantized value with the reference's operation order (no contraction):
//   Q4_K/Q5_K: (d*sc)*q - (dmin*m); Q6_K, IQ4_XS: (d*sc)*q;
//   Q8_0: q*d; IQ4_NL: d*kv.
__device__ __forceinline__ float dequant_value(GroupScale g, int code) {
    return __fsub_rn(__fmul_rn(g.dl, (float)code), g.ml);
}

// ------------------------------------------------------------ pieces -----
// Decode-GEMV piece: 32 values of one row, as two runs of 16 consecutive k.
// Pieces of a row are numbered p = 0..K/32-1; run r of piece p starts at
// k = run_k(p, r).  Each format provides
//   fetch(row, p)       -> Raw: the dwords covering the piece, loaded with
//                          plain dword-aligned loads and not yet inspected, so
//                          a caller can keep loads of later rows in flight;
//   decode(raw, row, p) -> PieceCodes: unsigned byte codes u[r] and
//                          coefficients such that
//     sum_k x_k w_k = sum_r a[r] * sum(x_run_r * u[r]) + b[r] * sum(x_run_r).
// Signed codes are biased to unsigned bytes (converted by v_cvt_f32_ubyteN in
// one instruction); b[r] removes the bias (and carries the K-quant mins).
struct PieceCodes {
    uint4 u[2];
    float a[2], b[2];
};

template <int NW> struct RawW { uint32_t w[NW]; };

__device__ __forceinline__ const uint32_t* align_down4(const uint8_t* p) {
    return (const uint32_t*)(p - ((uint32_t)(uintptr_t)p & 3u));
}

template <int N> __device__ __forceinline__ void ld_dw(const uint32_t* q, uint32_t* w) {
#pragma unroll
    for (int i = 0; i < N; i++) w[i] = q[i];
}

__device__ __forceinline__ uint32_t align2(uint32_t hi, uint32_t lo, uint32_t s) {
    return __builtin_amdgcn_alignbyte(hi, lo, s);
}

// Blocks of 2-byte-aligned formats (Q8_0: 34 bytes, IQ4_NL: 18) are read as
// a dword window from the aligned-down base b4.  Dword i of the stream that
// starts 2 bytes after the block base is bytes 2..5 of (w[i], w[i+1]) when
// the base is 4-aligned and w[i+1] when it is not: one v_perm_b32 with a
// per-block selector instead of a shift and a select per dword.
__device__ __forceinline__ uint32_t half_sel(const uint8_t* base) {
    return ((uint32_t)(uintptr_t)base & 2u) ? 0x07060504u : 0x05040302u;
}
__device__ __forceinline__ uint32_t half_pick(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}
// The fp16 at the block base: the high half of w[0] when the base is not
// 4-aligned, the low half when it is.
__device__ __forceinline__ float half_d(uint32_t w0, const uint8_t* base) {
    return h2f(w0 >> (((uint32_t)(uintptr_t)base & 2u) << 3));
}
// The same two from the low address bits of the block base.
__device__ __forceinline__ uint32_t half_sel_lo(uint32_t lo) { return (lo & 2u) ? 0x07060504u : 0x05040302u; }
__device__ __forceinline__ float half_d_lo(uint32_t w0, uint32_t lo) { return h2f(w0 >> ((lo & 2u) << 3)); }

// A weight row as a 4-aligned base and a 32-bit byte offset.  Loads at
// base + (off + o) take the scalar-base form (64-bit SGPR base + 32-bit VGPR
// offset) when the base is uniform over the wavefront, which saves the
// 64-bit address arithmetic per load; one matrix (one group's matrix) must
// stay below 4 GiB.  Alignment bits come from the offset alone.
struct RowRef {
    const uint8_t* base;
    uint32_t off;
    __device__ __forceinline__ const uint8_t* at(uint32_t o) const { return base + (uint32_t)(off + o); }
    // The dword-aligned address at or below base + off + o.
    __device__ __forceinline__ const uint32_t* at_al4(uint32_t o) const {
        return (const uint32_t*)(base + ((off + o) & ~3u));
    }
    __device__ __forceinline__ uint32_t lo(uint32_t o) const { return off + o; }
};
// Row at byte offset `off` of a matrix starting at m (any alignment): the
// misalignment of m moves into the offset.
__device__ __forceinline__ RowRef make_row(const uint8_t* m, uint32_t off) {
    const uint32_t mis = (uint32_t)(uintptr_t)m & 3u;
    return RowRef{m - mis, off + mis};
}

__device__ __forceinline__ uint4 uint4_at(const uint32_t* w) { return make_uint4(w[0], w[1], w[2], w[3]); }

// Dwords i..i+3 of a byte stream held as a window shifted by `s` bytes.
__device__ __forceinline__ uint4 realign4(const uint32_t* w, uint32_t s) {
    return make_uint4(align2(w[1], w[0], s), align2(w[2], w[1], s), align2(w[3], w[2], s), align2(w[4], w[3], s));
}

template <int T> struct Piece;

// Q4_K: piece j = p%8 of block b covers qs bytes [32c+16h, +16) (c = j/2,
// h = j%2): low nibbles are values 64c+16h+i (sub-block 2c), high nibbles
// values 64c+32+16h+i (sub-block 2c+1).
template <> struct Piece<T_Q4_K> {
    typedef RawW<8> Raw;
    static __device__ __forceinline__ int run_k(int p, int r) {
        return (p >> 3) * 256 + ((p >> 1) & 3) * 64 + (p & 1) * 16 + 32 * r;
    }
    static __device__ __forceinline__ Raw fetch(RowRef row, int p) {
        const uint32_t b = (p >> 3) * 144;
        const int c = (p >> 1) & 3, h = p & 1;
        Raw r;
        const uint4 hd = ld16_a(row.at(b)), q = ld16_a(row.at(b + 16 + 32 * c + 16 * h));
        r.w[0] = hd.x; r.w[1] = hd.y; r.w[2] = hd.z; r.w[3] = hd.w;
        r.w[4] = q.x; r.w[5] = q.y; r.w[6] = q.z; r.w[7] = q.w;
        return r;
    }
    static __device__ __forceinline__ PieceCodes decode(const Raw& r, RowRef, int p) {
        const int c = (p >> 1) & 3;
        const uint32_t sm = kq_pair(r.w[1], r.w[2], r.w[3], c);
        const uint32_t sc0 = sm & 0xFFu, sc1 = (sm >> 8) & 0xFFu, m0 = (sm >> 16) & 0xFFu, m1 = sm >> 24;
        const float d = h2f(r.w[0] & 0xFFFFu), dm = h2f(r.w[0] >> 16);
        const uint4 q = uint4_at(r.w + 4);
        PieceCodes o;
        o.u[0] = and4(q, 0x0F0F0F0Fu);
        // Run 1 keeps the high nibbles in place (byte = 16 * code, no shift)
        // and takes the 1/16 in its scale; both factors are exact.
        o.u[1] = and4(q, 0xF0F0F0F0u);
        o.a[0] = d * (float)sc0; o.b[0] = -(dm * (float)m0);
        o.a[1] = (d * (float)sc1) * 0.0625f; o.b[1] = -(dm * (float)m1);
        return o;
    }
};

// Q5_K: as Q4_K, plus bits 2c (run 0) and 2c+1 (run 1) of qh[16h+i].
template <> struct Piece<T_Q5_K> {
    typedef RawW<12> Raw;
    static __device__ __forceinline__ int run_k(int p, int r) { return Piece<T_Q4_K>::run_k(p, r); }
    static __device__ __forceinline__ Raw fetch(RowRef row, int p) {
        const uint32_t b = (p >> 3) * 176;
        const int c = (p >> 1) & 3, h = p & 1;
        Raw r;
        const uint4 hd = ld16_a(row.at(b)), qh = ld16_a(row.at(b + 16 + 16 * h)), q = ld16_a(row.at(b + 48 + 32 * c + 16 * h));
        r.w[0] = hd.x; r.w[1] = hd.y; r.w[2] = hd.z; r.w[3] = hd.w;
        r.w[4] = qh.x; r.w[5] = qh.y; r.w[6] = qh.z; r.w[7] = qh.w;
        r.w[8] = q.x; r.w[9] = q.y; r.w[10] = q.z; r.w[11] = q.w;
        return r;
    }
    static __device__ __forceinline__ PieceCodes decode(const Raw& r, RowRef, int p) {
        const int c = (p >> 1) & 3;
        const uint32_t sm = kq_pair(r.w[1], r.w[2], r.w[3], c);
        const uint32_t sc0 = sm & 0xFFu, sc1 = (sm >> 8) & 0xFFu, m0 = (sm >> 16) & 0xFFu, m1 = sm >> 24;
        const float d = h2f(r.w[0] & 0xFFFFu), dm = h2f(r.w[0] >> 16);
        const uint4 qh = uint4_at(r.w + 4), q = uint4_at(r.w + 8);
        PieceCodes o;
        o.u[0] = or4(and4(q, 0x0F0F0F0Fu), shl4(and4(shr4(qh, 2 * c), 0x01010101u), 4));
        o.u[1] = or4(and4(shr4(q, 4), 0x0F0F0F0Fu), shl4(and4(shr4(qh, 2 * c + 1), 0x01010101u), 4));
        o.a[0] = d * (float)sc0; o.b[0] = -(dm * (float)m0);
        o.a[1] = d * (float)sc1; o.b[1] = -(dm * (float)m1);
        return o;
    }
};

// Q6_K: piece j = p%8 of block b: half n = j/4, l0 = 16*((j/2)%2), s = j%2.
// ql bytes [64n+32s+l0, +16) low nibbles + qh[32n+l0+i] bits 2s..2s+1 ->
// values 128n+32s+l0+i (scale sc[8n+l0/16+2s]); the high nibbles + qh bits
// 4+2s.. -> values 128n+64+32s+l0+i (scale index +4).  Codes are 6-bit,
// offset 32.  Blocks are 210 bytes, so the fields are only 2-byte aligned:
// each is fetched as the dword window covering it and realigned in decode.
template <> struct Piece<T_Q6_K> {
    typedef RawW<14> Raw;
    static __device__ __forceinline__ int run_k(int p, int r) {
        return (p >> 3) * 256 + ((p >> 2) & 1) * 128 + (p & 1) * 32 + ((p >> 1) & 1) * 16 + 64 * r;
    }
    static __device__ __forceinline__ int sc_index(int p) { return 8 * ((p >> 2) & 1) + ((p >> 1) & 1) + 2 * (p & 1); }
    static __device__ __forceinline__ Raw fetch(RowRef row, int p) {
        const uint32_t b = (p >> 3) * 210;
        const int n = (p >> 2) & 1, l0 = ((p >> 1) & 1) * 16, s = p & 1;
        Raw r;
        ld_dw<5>(row.at_al4(b + 64 * n + 32 * s + l0), r.w);
        ld_dw<5>(row.at_al4(b + 128 + 32 * n + l0), r.w + 5);
        ld_dw<3>(row.at_al4(b + 192 + sc_index(p)), r.w + 10);
        r.w[13] = ld_u16(row.at(b + 208));
        return r;
    }
    static __device__ __forceinline__ PieceCodes decode(const Raw& r, RowRef row, int p) {
        const uint32_t b = (p >> 3) * 210;
        const uint32_t sh = row.lo(b) & 3u;  // ql / qh windows (offsets are multiples of 16)
        const uint32_t ss = row.lo(b + 192 + sc_index(p)) & 3u;
        const int s = p & 1;
        const uint4 ql = realign4(r.w, sh), qh = realign4(r.w + 5, sh);
        const uint32_t sc0 = align2(r.w[11], r.w[10], ss), sc1 = align2(r.w[12], r.w[11], ss);
        const float d = h2f(r.w[13]);
        PieceCodes o;
        o.u[0] = or4(and4(ql, 0x0F0F0F0Fu), shl4(and4(shr4(qh, 2 * s), 0x03030303u), 4));
        o.u[1] = or4(and4(shr4(ql, 4), 0x0F0F0F0Fu), shl4(and4(shr4(qh, 4 + 2 * s), 0x03030303u), 4));
        o.a[0] = d * (float)(int8_t)(sc0 & 0xFFu);
        o.a[1] = d * (float)(int8_t)(sc1 & 0xFFu);
        o.b[0] = -32.0f * o.a[0];
        o.b[1] = -32.0f * o.a[1];
        return o;
    }
};

// Q8_0: one piece per 34-byte block; run 0 = qs[0..15], run 1 = qs[16..31].
// Signed bytes are biased by 128 (xor 0x80).  Block bases are even, so the
// 9-dword window from the aligned-down base covers d and qs.
template <> struct Piece<T_Q8_0> {
    typedef RawW<9> Raw;
    static __device__ __forceinline__ int run_k(int p, int r) { return p * 32 + 16 * r; }
    static __device__ __forceinline__ Raw fetch(RowRef row, int p) {
        Raw r;
        ld_dw<9>(row.at_al4(p * 34), r.w);
        return r;
    }
    static __device__ __forceinline__ PieceCodes decode(const Raw& r, RowRef row, int p) {
        const uint32_t b = row.lo(p * 34);
        const uint32_t sel = half_sel_lo(b);
        const float d = half_d_lo(r.w[0], b);
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = half_pick(r.w[i + 1], r.w[i], sel) ^ 0x80808080u;
        PieceCodes o;
        o.u[0] = make_uint4(q[0], q[1], q[2], q[3]);
        o.u[1] = make_uint4(q[4], q[5], q[6], q[7]);
        o.a[0] = o.a[1] = d;
        o.b[0] = o.b[1] = -128.0f * d;
        return o;
    }
};

// IQ4_NL: one piece per 18-byte block; low nibbles -> values 0..15, high ->
// 16..31.  5-dword window from the aligned-down (even) base.
template <> struct Piece<T_IQ4_NL> {
    typedef RawW<5> Raw;
    static __device__ __forceinline__ int run_k(int p, int r) { return p * 32 + 16 * r; }
    static __device__ __forceinline__ Raw fetch(RowRef row, int p) {
        Raw r;
        ld_dw<5>(row.at_al4(p * 18), r.w);
        return r;
    }
    static __device__ __forceinline__ PieceCodes decode(const Raw& r, RowRef row, int p) {
        const uint32_t b = row.lo(p * 18);
        const uint32_t sel = half_sel_lo(b);
        const float d = half_d_lo(r.w[0], b);
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = half_pick(r.w[i + 1], r.w[i], sel);
        const uint4 qq = make_uint4(q[0], q[1], q[2], q[3]);
        PieceCodes o;
        o.u[0] = lut16x4(and4(qq, 0x0F0F0F0Fu), true);
        o.u[1] = lut16x4(and4(shr4(qq, 4), 0x0F0F0F0Fu), true);
        o.a[0] = o.a[1] = d;
        o.b[0] = o.b[1] = -128.0f * d;
        return o;
    }
};

// IQ4_XS: piece = sub-block ib = p%8 of block b (32 values, scale d*(ls-32)).
template <> struct Piece<T_IQ4_XS> {
    typedef RawW<6> Raw;
    static __device__ __forceinline__ int run_k(int p, int r) { return p * 32 + 16 * r; }
    static __device__ __forceinline__ Raw fetch(RowRef row, int p) {
        const uint32_t b = (p >> 3) * 136;
        const int ib = p & 7;
        Raw r;
        const uint2 hd = *(const uint2*)row.at(b);
        const uint2 lo = *(const uint2*)row.at(b + 8 + 16 * ib);
        const uint2 hi = *(const uint2*)row.at(b + 16 + 16 * ib);
        r.w[0] = hd.x; r.w[1] = hd.y; r.w[2] = lo.x; r.w[3] = lo.y; r.w[4] = hi.x; r.w[5] = hi.y;
        return r;
    }
    static __device__ __forceinline__ PieceCodes decode(const Raw& r, RowRef, int p) {
        const int ib = p & 7;
        const int ls = (int)(((r.w[1] >> (8 * (ib >> 1) + 4 * (ib & 1))) & 15u) | (((r.w[0] >> (16 + 2 * ib)) & 3u) << 4));
        const float dl = h2f(r.w[0] & 0xFFFFu) * (float)(ls - 32);
        const uint4 q = uint4_at(r.w + 2);
        PieceCodes o;
        o.u[0] = lut16x4(and4(q, 0x0F0F0F0Fu), true);
        o.u[1] = lut16x4(and4(shr4(q, 4), 0x0F0F0F0Fu), true);
        o.a[0] = o.a[1] = dl;
        o.b[0] = o.b[1] = -128.0f * dl;
        return o;
    }
};

// Hides the known-zero bits of a masked word from the optimizer, so byte
// extraction stays v_cvt_f32_ubyteN (one instruction) instead of being
// narrowed to v_bfe_u32 + v_cvt_f32_ubyte0.  Emits no instruction.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// Unsigned byte codes -> floats (v_cvt_f32_ubyte0..3).
__device__ __forceinline__ void ubytes_to_f32(uint4 u, float* f) {
    const uint32_t w[4] = {opaque(u.x), opaque(u.y), opaque(u.z), opaque(u.w)};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[4 * i + 0] = (float)(w[i] & 0xFFu);
        f[4 * i + 1] = (float)((w[i] >> 8) & 0xFFu);
        f[4 * i + 2] = (float)((w[i] >> 16) & 0xFFu);
        f[4 * i + 3] = (float)(w[i] >> 24);
    }
}

// ------------------------------------------------- MoE chunk lists -----
// (group, first row) chunk lists for grouped launches (struct ChunkList,
// ggq_launch.h).

// Built by one workgroup of 1024 threads (groups <= 1024); cnt: 16 ints of
// LDS (build_chunk_lists reads the offsets from global memory;
// chunk_lists_from_rows takes each group's rows from its thread).  With t_sh > 0 the last group is the shared expert, t_sh rows (every
// token) after the others: its end grp_off[groups] = grp_off[groups - 1] +
// t_sh and the x_idx of its rows (the token itself) are written first.
// grp_off is read from global memory, so a caller that has just written it
// from the same workgroup synchronizes first.
// Thread tid < groups passes its group's first row r0 and row count; the
// other threads pass 0 rows.
__device__ inline void chunk_lists_from_rows(int r0, int rows, const ChunkList* lists, int n_lists, int* cnt) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int li = 0; li < n_lists; li++) {
        const int mt = lists[li].mt;
        const int mine = rows > 0 ? (rows + mt - 1) / mt : 0;
        // chunks of the groups before this one: a scan within the
        // wavefront, then the totals of the earlier wavefronts
        int incl = mine;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const int o = __shfl_up(incl, off, 64);
            if (lane >= off) incl += o;
        }
        if (lane == 63) cnt[wave] = incl;
        __syncthreads();
        int before = 0;
        for (int w = 0; w < wave; w++) before += cnt[w];
        const int first = before + incl - mine;
        for (int i = 0; i < mine; i++) lists[li].items[first + i] = make_int2(tid, r0 + mt * i);
        if (tid == 1023) *lists[li].n_items = before + incl;  // the last lane of the last wavefront: the total
        __syncthreads();  // cnt is reused by the next list
    }
}

__device__ inline void build_chunk_lists(int32_t* grp_off, int groups, int t_sh, int32_t* x_idx,
                                         const ChunkList* lists, int n_lists, int* cnt) {
    const int tid = threadIdx.x;
    if (t_sh > 0) {
        const int base = grp_off[groups - 1];
        for (int t = tid; t < t_sh; t += 1024) x_idx[base + t] = t;
        __syncthreads();  // every thread has read grp_off[groups - 1]
        if (tid == 0) grp_off[groups] = base + t_sh;
        __syncthreads();
    }
    int rows = 0, r0 = 0;
    if (tid < groups) {
        r0 = grp_off[tid];
        rows = grp_off[tid + 1] - r0;
    }
    chunk_lists_from_rows(r0, rows, lists, n_lists, cnt);
}

}  // namespace ggq
