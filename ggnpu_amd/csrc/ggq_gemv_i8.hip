// ggq_gemv_i8.hip -- decode-sized matmuls (1..8 activation rows) on the int8
// matrix cores of gfx950 (v_mfma_i32_16x16x64_i8), straight from raw GGUF
// blocks.
//
// One MFMA multiplies a 16 x 64 activation operand A by a 64 x 16 weight
// operand B.  B's 16 columns are 16 weight rows (a "tile").  Lane l of a
// wavefront supplies 16 bytes of B for column l%16 and of A for row l%16,
// both for the 16 K-slots of its lane group g = l/16; the result C[i][j] =
// sum over g and byte b of A(lane 16g+i)[b] * B(lane 16g+j)[b] lands in lane
// 16*(i/4)+j, register i%4.  Each lane group's 16 B-bytes are the integer
// codes (Q4_K nibble, Q5_K 5-bit value, Q6_K 6-bit value, Q8_0 int8, IQ4
// codebook entry) of 16 consecutive values of K of one scale group, taken
// from one 16-byte load per lane (two MFMAs per load for the nibble formats:
// low nibbles, then high nibbles).  A lane group therefore carries one scale
// group ("slot" s = g/2 for the 32-value groups of Q4_K, Q5_K and Q8_0, s = g
// for Q6_K's 16-value groups and for IQ4, whose 32-value blocks span two
// MFMAs), and each row of A is restricted to one slot by zeros in the other
// lane groups: output lane group q holds per-group dot products and applies
// that group's scale.  Block headers (scales, mins) are loaded by one lane
// group and broadcast, so the loads stay at 16 bytes per lane access.
//
// Activations:
//  * fp32 (CpuRefBackend::mul_mat_q semantics, cpu_ref.cpp:87-117): each row
//    is written as fixed point X = rint(x * 2^e) with the row's largest
//    magnitude scaled into [2^21, 2^22), i.e. |x - 2^-e X| <= 2^-22 of the
//    row maximum, and X as three signed int8 digits, X = 65536 d0 + 256 d1 +
//    d2.  Rows 4q, 4q+1, 4q+2 of A carry the three digits, so one MFMA gives
//    the three digit dot products of a group in registers 0..2 of one lane;
//    the lane forms P = 65536 C0 + 256 C1 + C2 in fp32 (relative rounding
//    2^-24) and accumulates a*P + b*S, where a and b are the group's scale
//    and offset (K-quant min, Q6_K's -32 code bias) and S = sum of X over the
//    group.  Two activation rows per MFMA (one for Q6_K), more in passes.
//  * int8 (the XDNA backend's per-row semantics, amd_xdna.cpp:598-603,
//    633-639, 757-771): the digit is the reference's code q = clamp(rint(a *
//    (1/scale))), computed here bit for bit, or taken as given; C is then
//    exactly the int32 block dot product of the raw codes with q, and each
//    lane register carries another activation row.
//
// Work layout: a workgroup of 16 wavefronts builds the A operand of all its
// activation rows in LDS once (8-byte digit planes per MFMA, lane group and
// half, plus a zero plane that inactive slots point at), then its
// wavefronts stream weight tiles: KW wavefronts share a tile and split its K
// into 256-value chunks (one K-quant block, or eight 32-value blocks), the
// other wavefronts take other tiles.  Each chunk's raw bytes are fetched one
// chunk ahead.  Partial sums of a tile are combined across lane groups by
// swizzles and across the KW wavefronts through LDS, in a fixed order.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ggq_device.h"
#include "ggq_launch.h"

namespace ggq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v8u __attribute__((ext_vector_type(8)));

constexpr int kWaves = 16;
constexpr int kThreads = 64 * kWaves;


__device__ __forceinline__ v4i pack_b(uint2 lo, uint2 hi) {
    v4i b;
    b.x = (int)lo.x; b.y = (int)lo.y; b.z = (int)hi.x; b.w = (int)hi.y;
    return b;
}
__device__ __forceinline__ uint2 and2(uint2 v, uint32_t m) { return make_uint2(v.x & m, v.y & m); }
__device__ __forceinline__ uint2 shr2(uint2 v, int s) { return make_uint2(v.x >> s, v.y >> s); }
__device__ __forceinline__ uint2 or2(uint2 a, uint2 b) { return make_uint2(a.x | b.x, a.y | b.y); }
__device__ __forceinline__ uint2 shl2(uint2 v, int s) { return make_uint2(v.x << s, v.y << s); }

// Byte i of w as a float (v_cvt_f32_ubyteN).
template <int I> __device__ __forceinline__ float ubyte_f(uint32_t w) {
    return (float)((opaque(w) >> (8 * I)) & 0xFFu);
}

// ------------------------------------------------------------ formats ----
// IF<T>: the int8-MFMA view of a format.  A chunk is 256 values of a row
// (4 MFMAs t = 0..3).  fetch() issues the chunk's loads for lane group g (the
// header loads only in lane group 0), bcast() copies header words to the
// other lane groups once the loads have landed, codes(t) gives the B operand
// of MFMA t, coef() each MFMA's scale a[t] and offset b[t] for output slot s
// (value = a * code + b).  kpos maps (MFMA t, lane group g) to the first of
// its 16 consecutive values within the chunk; slot(g) is its scale group.
template <int T> struct IF;

// Weight loads go through a buffer resource over the matrix: offsets are
// 32-bit, and a lane whose offset is out of range (kOOB and above) reads
// zeros without a memory access, so lanes that do not own a load and
// fetches past the last chunk cost no memory traffic and need no branch
// (branches around loads make the compiler wait for every load in flight).
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr uint32_t kOOB = 0xC0000000u;
__device__ __forceinline__ Rsrc make_rsrc(const uint8_t* W, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ v4u bl16(Rsrc rs, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, 0); }
__device__ __forceinline__ uint32_t bl4(Rsrc rs, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(rs, (int)off, 0, 0); }
__device__ __forceinline__ uint32_t bl2(Rsrc rs, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b16(rs, (int)off, 0, 0); }
__device__ __forceinline__ uint32_t own(bool mine, uint32_t off) { return mine ? off : kOOB; }

__device__ __forceinline__ uint32_t lane_bcast(uint32_t v, int src) { return (uint32_t)__shfl((int)v, src, 64); }
__device__ __forceinline__ v4i nib_lo(v4u w) {
    v4i r; r.x = (int)(w.x & 0x0F0F0F0Fu); r.y = (int)(w.y & 0x0F0F0F0Fu); r.z = (int)(w.z & 0x0F0F0F0Fu); r.w = (int)(w.w & 0x0F0F0F0Fu);
    return r;
}
__device__ __forceinline__ v4i nib_hi(v4u w) {
    v4i r; r.x = (int)((w.x >> 4) & 0x0F0F0F0Fu); r.y = (int)((w.y >> 4) & 0x0F0F0F0Fu);
    r.z = (int)((w.z >> 4) & 0x0F0F0F0Fu); r.w = (int)((w.w >> 4) & 0x0F0F0F0Fu);
    return r;
}

// Q4_K (kquant.h:9-13, 133-151): qs[128] at 16; 32-byte run c holds
// sub-block 2c (low nibbles) and 2c+1 (high nibbles).  Lane group g loads
// qs[16g, +16) and qs[64+16g, +16): runs 2u + (g>>1), values 16(g&1).. of
// them.  MFMA t = 2u + h takes the low (h = 0) or high (h = 1) nibbles, so
// slot s = g>>1 is sub-block 4u + 2s + h.
template <> struct IF<T_Q4_K> {
    static constexpr int G = 2, CHUNK = 144;
    static constexpr bool BIAS = true;
    struct Raw { v4u q0, q1, hd; };
    static __device__ __forceinline__ Raw fetch(Rsrc rs, uint32_t off, int g, int) {
        Raw r;
        r.q0 = bl16(rs, off + 16 + 16 * g);
        r.q1 = bl16(rs, off + 80 + 16 * g);
        r.hd = bl16(rs, own(g == 0, off));
        return r;
    }
    static __device__ __forceinline__ void bcast(Raw& r, int col) {
        r.hd.x = lane_bcast(r.hd.x, col); r.hd.y = lane_bcast(r.hd.y, col);
        r.hd.z = lane_bcast(r.hd.z, col); r.hd.w = lane_bcast(r.hd.w, col);
    }
    static __device__ __forceinline__ v4i codes(const Raw& r, int t, int) {
        const v4u w = (t >> 1) ? r.q1 : r.q0;
        return (t & 1) ? nib_hi(w) : nib_lo(w);
    }
    // scale / min of sub-blocks 2s, 2s+1 (t = 0, 1) and 4+2s, 5+2s (t = 2,
    // 3), kquant.h:56-64, as the pairs s and 2+s of kq_pair.
    static __device__ __forceinline__ void coef(const Raw& r, int s, float (&a)[4], float (&b)[4]) {
        const float d = h2f(r.hd.x & 0xFFFFu), dm = h2f(r.hd.x >> 16);
        const uint32_t b2 = 2u * (uint32_t)s;
        const uint32_t A = __builtin_amdgcn_perm(r.hd.z, r.hd.y, b2 | (b2 + 1) << 8 | (b2 + 4) << 16 | (b2 + 5) << 24);
        const uint32_t Q = __builtin_amdgcn_perm(r.hd.w, r.hd.w, b2 | (b2 + 1) << 8 | b2 << 16 | (b2 + 1) << 24);
        const uint32_t lo = A & 0x3F3F3F3Fu;  // sc(2s), sc(2s+1), m(2s), m(2s+1)
        const uint32_t hi = ((A >> 2) & 0x30303030u) | (Q & 0x00000F0Fu) | ((Q >> 4) & 0x0F0F0000u);
        a[0] = d * ubyte_f<0>(lo); a[1] = d * ubyte_f<1>(lo);
        b[0] = -(dm * ubyte_f<2>(lo)); b[1] = -(dm * ubyte_f<3>(lo));
        a[2] = d * ubyte_f<0>(hi); a[3] = d * ubyte_f<1>(hi);
        b[2] = -(dm * ubyte_f<2>(hi)); b[3] = -(dm * ubyte_f<3>(hi));
    }
    static __device__ __forceinline__ int slot(int g) { return g >> 1; }
    static __device__ __forceinline__ int kpos(int t, int g) { return 128 * (t >> 1) + 64 * (g >> 1) + 32 * (t & 1) + 16 * (g & 1); }
    static __device__ __forceinline__ void inv(int x, int& t, int& g) { t = 2 * (x >> 3) + ((x >> 1) & 1); g = 2 * ((x >> 2) & 1) + (x & 1); }
};

// Q5_K (kquant.h:157-179): as Q4_K with qs at 48 and the fifth bits in
// qh[32] at 16: bit 2c of qh[p] for sub-block 2c, bit 2c+1 for 2c+1.  Lane
// groups 0 and 1 load qh[16(g&1), +16) for 2 and 3 as well.
template <> struct IF<T_Q5_K> {
    static constexpr int G = 2, CHUNK = 176;
    static constexpr bool BIAS = true;
    struct Raw { v4u q0, q1, qh, hd; };
    static __device__ __forceinline__ Raw fetch(Rsrc rs, uint32_t off, int g, int) {
        Raw r;
        r.q0 = bl16(rs, off + 48 + 16 * g);
        r.q1 = bl16(rs, off + 112 + 16 * g);
        r.qh = bl16(rs, own(g < 2, off + 16 + 16 * g));
        r.hd = bl16(rs, own(g == 0, off));
        return r;
    }
    static __device__ __forceinline__ void bcast(Raw& r, int col) {
        IF<T_Q4_K>::Raw h{r.q0, r.q1, r.hd};
        IF<T_Q4_K>::bcast(h, col);
        r.hd = h.hd;
        const int src = (int)(threadIdx.x & 31);
        r.qh.x = lane_bcast(r.qh.x, src); r.qh.y = lane_bcast(r.qh.y, src);
        r.qh.z = lane_bcast(r.qh.z, src); r.qh.w = lane_bcast(r.qh.w, src);
    }
    static __device__ __forceinline__ v4i codes(const Raw& r, int t, int g) {
        const v4u w = (t >> 1) ? r.q1 : r.q0;
        v4i c = (t & 1) ? nib_hi(w) : nib_lo(w);
        // bit 2c + h of qh, c = 2u + (g>>1): moved to bit 4 of each byte
        const int sh = 4 * (t >> 1) + 2 * (g >> 1) + (t & 1);
        c.x |= (int)(((r.qh.x >> sh) & 0x01010101u) << 4); c.y |= (int)(((r.qh.y >> sh) & 0x01010101u) << 4);
        c.z |= (int)(((r.qh.z >> sh) & 0x01010101u) << 4); c.w |= (int)(((r.qh.w >> sh) & 0x01010101u) << 4);
        return c;
    }
    static __device__ __forceinline__ void coef(const Raw& r, int s, float (&a)[4], float (&b)[4]) {
        IF<T_Q4_K>::coef(IF<T_Q4_K>::Raw{r.q0, r.q1, r.hd}, s, a, b);
    }
    static __device__ __forceinline__ int slot(int g) { return g >> 1; }
    static __device__ __forceinline__ int kpos(int t, int g) { return IF<T_Q4_K>::kpos(t, g); }
    static __device__ __forceinline__ void inv(int x, int& t, int& g) { IF<T_Q4_K>::inv(x, t, g); }
};

// Q6_K (kquant.h:182-202): half n of the block: ql[64n + 16g, +16) for lane
// group g; low nibbles (MFMA t = 2n) are values 128n + 16g.., high nibbles
// (t = 2n+1) values 128n + 64 + 16g..; the top two bits come from qh[32n +
// 16(g&1) + b], bits 2(g>>1) (+4 for the high nibbles).  Codes stay unsigned
// (0..63) and the -32 goes into b.  Slot s = g: scale sc[4t + s].  Lane
// groups 0 and 1 load qh for 2 and 3; lane group 0 loads sc and d.
template <> struct IF<T_Q6_K> {
    static constexpr int G = 4, CHUNK = 210;
    static constexpr bool BIAS = true;
    struct Raw { v4u ql0, ql1, qh0, qh1, sc; uint32_t d; };
    static __device__ __forceinline__ Raw fetch(Rsrc rs, uint32_t off, int g, int) {
        Raw r;
        r.ql0 = bl16(rs, off + 16 * g);
        r.ql1 = bl16(rs, off + 64 + 16 * g);
        r.qh0 = bl16(rs, own(g < 2, off + 128 + 16 * g));
        r.qh1 = bl16(rs, own(g < 2, off + 160 + 16 * g));
        r.sc = bl16(rs, own(g == 0, off + 192));
        r.d = bl2(rs, own(g == 0, off + 208));
        return r;
    }
    static __device__ __forceinline__ void bcast(Raw& r, int col) {
        const int src = (int)(threadIdx.x & 31);
        r.qh0.x = lane_bcast(r.qh0.x, src); r.qh0.y = lane_bcast(r.qh0.y, src);
        r.qh0.z = lane_bcast(r.qh0.z, src); r.qh0.w = lane_bcast(r.qh0.w, src);
        r.qh1.x = lane_bcast(r.qh1.x, src); r.qh1.y = lane_bcast(r.qh1.y, src);
        r.qh1.z = lane_bcast(r.qh1.z, src); r.qh1.w = lane_bcast(r.qh1.w, src);
        r.sc.x = lane_bcast(r.sc.x, col); r.sc.y = lane_bcast(r.sc.y, col);
        r.sc.z = lane_bcast(r.sc.z, col); r.sc.w = lane_bcast(r.sc.w, col);
        r.d = lane_bcast(r.d, col);
    }
    static __device__ __forceinline__ v4i codes(const Raw& r, int t, int g) {
        const v4u w = (t >> 1) ? r.ql1 : r.ql0;
        const v4u qh = (t >> 1) ? r.qh1 : r.qh0;
        v4i c = (t & 1) ? nib_hi(w) : nib_lo(w);
        const int sh = 4 * (t & 1) + 2 * (g >> 1);
        c.x |= (int)(((qh.x >> sh) & 0x03030303u) << 4); c.y |= (int)(((qh.y >> sh) & 0x03030303u) << 4);
        c.z |= (int)(((qh.z >> sh) & 0x03030303u) << 4); c.w |= (int)(((qh.w >> sh) & 0x03030303u) << 4);
        return c;
    }
    static __device__ __forceinline__ void coef(const Raw& r, int s, float (&a)[4], float (&b)[4]) {
        const float d = h2f(r.d);
        const uint32_t w[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
#pragma unroll
        for (int t = 0; t < 4; t++) {
            a[t] = d * (float)(int)(int8_t)((w[t] >> (8 * s)) & 0xFFu);
            b[t] = -32.0f * a[t];
        }
    }
    static __device__ __forceinline__ int slot(int g) { return g; }
    static __device__ __forceinline__ int kpos(int t, int g) { return 128 * (t >> 1) + 64 * (t & 1) + 16 * g; }
    static __device__ __forceinline__ void inv(int x, int& t, int& g) { t = 2 * (x >> 3) + ((x >> 2) & 1); g = x & 3; }
};

// Q8_0 (q8_0.cpp:19-25): a chunk is 8 blocks of 34 bytes; MFMA t takes
// blocks 2t + (g>>1), codes 16(g&1)..+15 (signed, as they are); slot
// s = g>>1.  Each output lane loads the d of its own slot's blocks.
template <> struct IF<T_Q8_0> {
    static constexpr int G = 2, CHUNK = 272;
    static constexpr bool BIAS = false;
    struct Raw { v4u q0, q1, q2, q3; uint32_t d01, d23; };
    static __device__ __forceinline__ Raw fetch(Rsrc rs, uint32_t off, int g, int s) {
        Raw r;
        const uint32_t o = off + 34 * (g >> 1) + 2 + 16 * (g & 1);
        r.q0 = bl16(rs, o); r.q1 = bl16(rs, o + 68); r.q2 = bl16(rs, o + 136); r.q3 = bl16(rs, o + 204);
        const uint32_t od = off + 34 * s;
        r.d01 = bl2(rs, od) | bl2(rs, od + 68) << 16;
        r.d23 = bl2(rs, od + 136) | bl2(rs, od + 204) << 16;
        return r;
    }
    static __device__ __forceinline__ void bcast(Raw&, int) {}
    static __device__ __forceinline__ v4i codes(const Raw& r, int t, int) {
        const v4u w = t == 0 ? r.q0 : t == 1 ? r.q1 : t == 2 ? r.q2 : r.q3;
        v4i c; c.x = (int)w.x; c.y = (int)w.y; c.z = (int)w.z; c.w = (int)w.w;
        return c;
    }
    static __device__ __forceinline__ void coef(const Raw& r, int, float (&a)[4], float (&b)[4]) {
        a[0] = h2f(r.d01 & 0xFFFFu); a[1] = h2f(r.d01 >> 16); a[2] = h2f(r.d23 & 0xFFFFu); a[3] = h2f(r.d23 >> 16);
        b[0] = b[1] = b[2] = b[3] = 0.0f;
    }
    static __device__ __forceinline__ int slot(int g) { return g >> 1; }
    static __device__ __forceinline__ int kpos(int t, int g) { return 64 * t + 16 * g; }
    static __device__ __forceinline__ void inv(int x, int& t, int& g) { t = x >> 2; g = x & 3; }
};

// Codebook entries of four nibbles (one per byte), signed: v_perm picks from
// the two 8-entry halves of the table, and bit 3 of each nibble (moved to
// the byte's sign bit and replicated by v_perm's sign selectors) chooses.
__device__ __forceinline__ uint32_t iq4_lut(uint32_t nib) {
    const uint32_t sel = nib & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(GGQ_IQ4S1, GGQ_IQ4S0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(GGQ_IQ4S3, GGQ_IQ4S2, sel);
    const uint32_t x = nib << 4;
    const uint32_t msk = __builtin_amdgcn_perm(x << 8, x, 0x090B080Au);
    return (hi & msk) | (lo & ~msk);
}
__device__ __forceinline__ v4i iq4_codes(v4u w, int hi) {
    const v4i n = hi ? nib_hi(w) : nib_lo(w);
    v4i c;
    c.x = (int)iq4_lut((uint32_t)n.x); c.y = (int)iq4_lut((uint32_t)n.y);
    c.z = (int)iq4_lut((uint32_t)n.z); c.w = (int)iq4_lut((uint32_t)n.w);
    return c;
}

// IQ4_NL (iq4_nl.cpp:16-31): 8 blocks of 18 bytes per chunk; value j < 16 is
// the low nibble of qs[j], value j+16 the high nibble.  Lane group g loads
// the 16 qs bytes of blocks g and 4+g; MFMA t = 2w + h takes nibbles h of
// blocks 4w + g: slot s = g (block 4w + s).
template <> struct IF<T_IQ4_NL> {
    static constexpr int G = 4, CHUNK = 144;
    static constexpr bool BIAS = false;
    struct Raw { v4u q0, q1; uint32_t d0, d1; };
    static __device__ __forceinline__ Raw fetch(Rsrc rs, uint32_t off, int g, int s) {
        Raw r;
        r.q0 = bl16(rs, off + 18 * g + 2);
        r.q1 = bl16(rs, off + 18 * (4 + g) + 2);
        r.d0 = bl2(rs, off + 18 * s);
        r.d1 = bl2(rs, off + 18 * (4 + s));
        return r;
    }
    static __device__ __forceinline__ void bcast(Raw&, int) {}
    static __device__ __forceinline__ v4i codes(const Raw& r, int t, int) { return iq4_codes((t >> 1) ? r.q1 : r.q0, t & 1); }
    static __device__ __forceinline__ void coef(const Raw& r, int, float (&a)[4], float (&b)[4]) {
        a[0] = a[1] = h2f(r.d0); a[2] = a[3] = h2f(r.d1);
        b[0] = b[1] = b[2] = b[3] = 0.0f;
    }
    static __device__ __forceinline__ int slot(int g) { return g; }
    static __device__ __forceinline__ int kpos(int t, int g) { return 128 * (t >> 1) + 32 * g + 16 * (t & 1); }
    static __device__ __forceinline__ void inv(int x, int& t, int& g) { t = 2 * (x >> 3) + (x & 1); g = (x >> 1) & 3; }
};

// IQ4_XS (iq4_xs.cpp:21-38): sub-block j of the block: qs[16j, +16), low
// nibbles values 32j.., high 32j+16..; scale d * (ls - 32) with the 6-bit ls
// from scales_l / scales_h.  Lane group g loads sub-blocks g and 4+g; lane
// group 0 the 8-byte header.
template <> struct IF<T_IQ4_XS> {
    static constexpr int G = 4, CHUNK = 136;
    static constexpr bool BIAS = false;
    struct Raw { v4u q0, q1; uint32_t h0, h1; };
    static __device__ __forceinline__ Raw fetch(Rsrc rs, uint32_t off, int g, int) {
        Raw r;
        r.q0 = bl16(rs, off + 8 + 16 * g);
        r.q1 = bl16(rs, off + 72 + 16 * g);
        r.h0 = bl4(rs, own(g == 0, off));
        r.h1 = bl4(rs, own(g == 0, off + 4));
        return r;
    }
    static __device__ __forceinline__ void bcast(Raw& r, int col) {
        r.h0 = lane_bcast(r.h0, col);
        r.h1 = lane_bcast(r.h1, col);
    }
    static __device__ __forceinline__ v4i codes(const Raw& r, int t, int) { return iq4_codes((t >> 1) ? r.q1 : r.q0, t & 1); }
    static __device__ __forceinline__ void coef(const Raw& r, int s, float (&a)[4], float (&b)[4]) {
        const float d = h2f(r.h0 & 0xFFFFu);
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const int ib = 4 * w + s;
            const int ls = (int)(((r.h1 >> (4 * ib)) & 15u) | (((r.h0 >> (16 + 2 * ib)) & 3u) << 4));
            a[2 * w] = a[2 * w + 1] = __fmul_rn(d, (float)(ls - 32));
        }
        b[0] = b[1] = b[2] = b[3] = 0.0f;
    }
    static __device__ __forceinline__ int slot(int g) { return g; }
    static __device__ __forceinline__ int kpos(int t, int g) { return IF<T_IQ4_NL>::kpos(t, g); }
    static __device__ __forceinline__ void inv(int x, int& t, int& g) { IF<T_IQ4_NL>::inv(x, t, g); }
};

// ------------------------------------------------------------- launch ----
struct I8Prob {
    const uint8_t* W;
    uint32_t row_bytes;
    uint32_t type;
    int N, K;
    const float* X;     // fp32 activations [M][ldx] (modes 0, 1)
    int ldx;
    const int8_t* QA;   // given int8 activations [M][K] and row scales (mode 2)
    const float* SA;
    float* Y;
    int ldy;
    int kw_log2;        // wavefronts per tile
    int x_vec4;         // X (and X2) rows 16-byte aligned
    // Fused neighbours (modes 0 and 1; zero / null = off), as the fp32
    // kernels apply them: the activation is X * X2, then RMSNorm'd
    // (x * (1 / sqrt(sum(x^2) / K + eps)) * norm_w); the output is
    // silu(result), then R + result.
    const float* X2;
    const float* norm_w;
    const float* R;
    int ldr;
    int rms, silu;
    float eps;
    int nw_vec4;        // norm_w 16-byte aligned
};

constexpr int kMaxProbs = 8;
struct I8Args {
    I8Prob p[kMaxProbs];
    int begin[kMaxProbs + 1];
    int n;
    int M;
    int mode;  // 0: fp32 -> 3 digits; 1: fp32 -> per-row int8 codes; 2: given int8 codes
};

// Geometry of one launch instantiation.
template <int T, int D, int NE, int NP> struct Geo {
    static constexpr int G = IF<T>::G;
    static constexpr int RG = 4 / G;                     // activation row groups per pass (lane groups)
    static constexpr int RP = RG * (D == 1 ? NE : 1);    // activation rows per pass
    static constexpr int MT = RP * NP;                   // most rows of a launch
};

// LDS carve (bytes) for K values and M activation rows:
//  * A entries, 16 bytes each, per (MFMA t, lane group g): entry d*M + m =
//    digit plane d of row m at that lane group's 16 values, and a zero entry
//    last: E = D*M + 1 per (t, g);
//  * group sums S[chunk][slot s][row m][mfma t] (floats);
//  * per-row scale and exponent; the reduction buffer (two tiles' worth, by
//    parity); the per-wavefront row maxima and sums of squares; the per-row
//    RMSNorm factor.
__host__ __device__ inline int i8_entries(int D, int M) { return D * M + 1; }
__host__ __device__ inline int i8_lds_a(int K, int D, int M) { return (K / 64) * 4 * i8_entries(D, M) * 16; }
__host__ __device__ inline int i8_lds_s(int K, int G, int M) { return (K / 256) * G * M * 4 * 4; }
__host__ __device__ inline int i8_lds_red(int MT) { return 2 * kWaves * MT * 16 * 4; }
__host__ __device__ inline int i8_lds_total(int K, int G, int D, int M, int MT) {
    return i8_lds_a(K, D, M) + (D == 3 ? 2 : 1) * i8_lds_s(K, G, M) + M * 8 + i8_lds_red(MT) + 2 * kWaves * M * 4 + M * 4;
}

// Fixed-point digits of one value: X = rint(x 2^e) + 0x808080 as bytes
// (offset binary); the digits are those bytes xor 0x80.
__device__ __forceinline__ uint32_t fixed_u(float x, int e) {
    const float f = __fadd_rn(ldexpf(x, e), 12582912.0f);  // 1.5 * 2^23: rounds to an integer (ties to even)
    return __builtin_bit_cast(uint32_t, f) - 0x4B400000u + 0x808080u;
}

// Four values' digit bytes: byte k of plane dword = digit of value k.
// Plane 0 is the most significant digit (byte 2 of u), plane 2 the least.
__device__ __forceinline__ void digit_planes4(const uint32_t* v, uint32_t& p0, uint32_t& p1, uint32_t& p2) {
    const uint32_t a01 = __builtin_amdgcn_perm(v[1], v[0], 0x05010400u);  // v0.b0 v1.b0 v0.b1 v1.b1
    const uint32_t a23 = __builtin_amdgcn_perm(v[3], v[2], 0x05010400u);
    const uint32_t c01 = __builtin_amdgcn_perm(v[1], v[0], 0x0c0c0602u);  // v0.b2 v1.b2
    const uint32_t c23 = __builtin_amdgcn_perm(v[3], v[2], 0x0c0c0602u);
    p2 = __builtin_amdgcn_perm(a23, a01, 0x05040100u) ^ 0x80808080u;  // byte 0 of each
    p1 = __builtin_amdgcn_perm(a23, a01, 0x07060302u) ^ 0x80808080u;  // byte 1
    p0 = __builtin_amdgcn_perm(c23, c01, 0x05040100u) ^ 0x80808080u;  // byte 2
}

__device__ __forceinline__ int8_t code_i8(float v) {
    float r = __builtin_rintf(v);
    r = fminf(fmaxf(r, -128.0f), 127.0f);
    return (int8_t)(int)r;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// M_ activation rows; row m of the activations is row xrow[m] of X (the
// row itself when xrow is null) and its outputs go to row yrow0 + m of Y.
template <int T, int D, int NE, int NP, bool FU>
__device__ void i8_gemv_body(const I8Args& args, const I8Prob& a, int bx, int gx, uint8_t* lds, int M_,
                             const int32_t* xrow, int yrow0) {
    typedef Geo<T, D, NE, NP> GEO;
    constexpr int G = GEO::G, RG = GEO::RG, RP = GEO::RP, MT = GEO::MT;
    typedef typename IF<T>::Raw Raw;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = lane >> 4, col = lane & 15;
    const int M = M_, K = a.K, N = a.N;
    const int NC = K >> 8;
    const int KW = 1 << a.kw_log2, TPI = kWaves >> a.kw_log2;
    const int kp = w & (KW - 1), slot_t = w >> a.kw_log2;
    const int tiles = (N + 15) >> 4;
    const int n_it = (tiles + TPI - 1) / TPI;
    const int nmy = (NC - kp + KW - 1) >> a.kw_log2;
    // scale-group slot and row group of this lane's outputs
    const int s_out = g % G, rg_out = g / G;
    const int E = i8_entries(D, M);
    const uint32_t TS = 64u * (uint32_t)E;  // A bytes per MFMA

    uint8_t* lds_a = lds;
    float* lds_s = (float*)(lds + i8_lds_a(K, D, M));
    float* lds_sc = (float*)((uint8_t*)lds_s + i8_lds_s(K, G, M));  // fp32 mode: group scales
    float* row_rs = (float*)((uint8_t*)lds_s + (D == 3 ? 2 : 1) * i8_lds_s(K, G, M));
    int* row_re = (int*)(row_rs + M);
    float* red = (float*)(row_re + M);
    float* wmax = red + i8_lds_red(MT) / 4;
    // outputs of this workgroup's tiles, stored to Y after the main loop
    // (stores inside it would make the compiler wait for the weight loads
    // in flight): [row m][local output row]
    const int iters_wg = (n_it - bx + gx - 1) / gx;
    const int ROWS = iters_wg * TPI * 16;
    float* wss = wmax + kWaves * M;      // per-wavefront sums of squares (RMSNorm)
    float* row_is = wss + kWaves * M;    // per-row RMSNorm factor
    float* outl = row_is + M;

    const Rsrc rs = make_rsrc(a.W, (uint32_t)N * a.row_bytes);
    // Chunk offset of a (tile iteration, chunk) position: rows past N read
    // row N-1 (their results are dropped), positions past the last
    // iteration read nothing (out-of-range offset).
    auto chunk_off = [&](int it, int i) __attribute__((always_inline)) {
        int n = (it * TPI + slot_t) * 16 + col;
        n = n < N ? n : N - 1;
        const uint32_t o = (uint32_t)n * a.row_bytes + (uint32_t)(kp + KW * i) * IF<T>::CHUNK;
        return it < n_it ? o : kOOB;
    };
    // (tile iteration, chunk) positions: compute position and the position
    // of the next fetch, two chunks ahead.
    int it = bx, i = 0;
    int itf = bx, jf = 0;
    auto adv = [&](int& pit, int& pi) __attribute__((always_inline)) {
        if (++pi >= nmy) { pi = 0; pit += gx; }
    };
    // The first chunk's loads go out before the activation set-up, the
    // second's right after it.
    // ---- activation set-up, per hexad (16 consecutive values of K).  The
    // thread's first hexad of row 0 is loaded before anything else
    // (its latency then overlaps the first weight fetch); others are read
    // when needed.
    const int n_hex = K >> 4;
    const int mode = args.mode;
    constexpr int KR = 1;
    float xk[KR][16];
    auto load_hex = [&](int m, int x, float (&v)[16]) __attribute__((always_inline)) {
        const float* xr = a.X + (int64_t)(xrow ? xrow[m] : m) * a.ldx + 16 * x;
        if (a.x_vec4) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 f = *(const float4*)(xr + 4 * q);
                v[4 * q] = f.x; v[4 * q + 1] = f.y; v[4 * q + 2] = f.z; v[4 * q + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = xr[k];
        }
    };
    if (mode != 2 && tid < n_hex) {
#pragma unroll
        for (int m = 0; m < KR; m++)
            if (m < M) load_hex(m, tid, xk[m]);
    }
    auto get_hex = [&](int m, int x, float (&v)[16]) __attribute__((always_inline)) {
        if (x == tid && m < KR) {
#pragma unroll
            for (int r = 0; r < KR; r++)
                if (r == m) {
#pragma unroll
                    for (int k = 0; k < 16; k++) v[k] = xk[r][k];
                }
        } else {
            load_hex(m, x, v);
        }
    };
    // Fused inputs: the product with X2, then (norm = true) the RMSNorm
    // factor and weights, rounded as the fp32 kernels round them.
    auto load16 = [&](const float* p, bool vec, float (&u)[16]) __attribute__((always_inline)) {
        if (vec) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 f = *(const float4*)(p + 4 * q);
                u[4 * q] = f.x; u[4 * q + 1] = f.y; u[4 * q + 2] = f.z; u[4 * q + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < 16; k++) u[k] = p[k];
        }
    };
    auto fuse_in = [&](int m, int x, float (&v)[16], bool norm) __attribute__((always_inline)) {
        if (a.X2) {
            float u[16];
            load16(a.X2 + (int64_t)m * a.ldx + 16 * x, a.x_vec4, u);
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = __fmul_rn(v[k], u[k]);
        }
        if (norm && a.rms) {
            const float is = row_is[m];
            float u[16];
            if (a.norm_w) {
                load16(a.norm_w + 16 * x, a.nw_vec4, u);
            } else {
#pragma unroll
                for (int k = 0; k < 16; k++) u[k] = 1.0f;
            }
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = __fmul_rn(__fmul_rn(v[k], is), u[k]);
        }
    };
    Raw r0, r1, r2;
    r0 = IF<T>::fetch(rs, chunk_off(itf, jf), g, s_out);
    adv(itf, jf);

    // phase 0 (RMSNorm): each row's sum of squares over the workgroup, then
    // its factor 1 / sqrt(sum / K + eps) (cpu_ref.cpp:139-156)
    if (FU && a.rms) {
        for (int m = 0; m < M; m++) {
            float ss = 0.0f;
            for (int x = tid; x < n_hex; x += kThreads) {
                float v[16];
                get_hex(m, x, v);
                if constexpr (FU) fuse_in(m, x, v, false);
#pragma unroll
                for (int k = 0; k < 16; k++) ss = fmaf(v[k], v[k], ss);
            }
            ss = wave_sum(ss);
            if (lane == 0) wss[w * M + m] = ss;
        }
        __syncthreads();
        if (tid < M) {
            float t = 0.0f;
#pragma unroll
            for (int k = 0; k < kWaves; k++) t += wss[k * M + tid];
            row_is[tid] = 1.0f / sqrtf(t / (float)K + a.eps);
        }
        __syncthreads();
    }

    // phase 1 (int8 codes only): row maxima, the reference's per-row scale
    if (mode == 1) {
        for (int m = 0; m < M; m++) {
            float mx = 0.0f;
            for (int x = tid; x < n_hex; x += kThreads) {
                float v[16];
                get_hex(m, x, v);
                if constexpr (FU) fuse_in(m, x, v, true);
#pragma unroll
                for (int k = 0; k < 16; k++) mx = fmaxf(mx, fabsf(v[k]));
            }
            mx = wave_max(mx);
            if (lane == 0) wmax[w * M + m] = mx;
        }
        __syncthreads();
    }
    // phase 2: A entries and group sums (fp32 mode: each scale group gets its
    // own power of two, from its largest magnitude; int8 modes: per-row
    // scale and codes)
    for (int m = 0; m < M; m++) {
        float rs_m = 1.0f, inv = 0.0f;
        if (mode == 2) {
            rs_m = a.SA[xrow ? xrow[m] : m];
        } else if (mode == 1) {
            float amax = 0.0f;
#pragma unroll
            for (int k = 0; k < kWaves; k++) amax = fmaxf(amax, wmax[k * M + m]);
            rs_m = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 1.0f;
            inv = __fdiv_rn(1.0f, rs_m);
        }
        if (tid == 0) { row_rs[m] = rs_m; row_re[m] = 0; }
        for (int x = tid; x < n_hex; x += kThreads) {
            int tl, hg;
            IF<T>::inv(x & 15, tl, hg);
            const int t = 4 * (x >> 4) + tl;
            uint4 pl[3];
            float gsum = 0.0f, gscale = 1.0f;
            if (mode == 2) {
                const uint4 q = *(const uint4*)(a.QA + (int64_t)(xrow ? xrow[m] : m) * K + 16 * x);
                pl[0] = q;
                const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
                int sum = 0;
#pragma unroll
                for (int k = 0; k < 16; k++) sum += (int)(int8_t)(qq[k >> 2] >> (8 * (k & 3)));
                if (G == 2) sum += __shfl_xor(sum, 1, 64);
                gsum = (float)sum;
            } else {
                float v[16];
                get_hex(m, x, v);
                if constexpr (FU) fuse_in(m, x, v, true);
                if (mode == 0) {
                    // the group's power of two: its largest magnitude in [2^21, 2^22)
                    float mx = 0.0f;
#pragma unroll
                    for (int k = 0; k < 16; k++) mx = fmaxf(mx, fabsf(v[k]));
                    if (G == 2) mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
                    int Ex = 0;
                    frexpf(mx, &Ex);
                    const int e = mx > 0.0f ? 22 - Ex : 0;
                    gscale = ldexpf(1.0f, -e);
                    int sum = 0;
                    uint32_t p0[4], p1[4], p2[4];
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        uint32_t u[4];
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            u[k] = fixed_u(v[4 * q + k], e);
                            sum += (int)(u[k] - 0x808080u);
                        }
                        digit_planes4(u, p0[q], p1[q], p2[q]);
                    }
                    if (G == 2) sum += __shfl_xor(sum, 1, 64);
                    gsum = ldexpf((float)sum, -e);  // the group sum of the fixed-point values
                    pl[0] = make_uint4(p0[0], p0[1], p0[2], p0[3]);
                    pl[1] = make_uint4(p1[0], p1[1], p1[2], p1[3]);
                    pl[2] = make_uint4(p2[0], p2[1], p2[2], p2[3]);
                } else {
                    uint32_t c[4] = {0u, 0u, 0u, 0u};
                    int sum = 0;
#pragma unroll
                    for (int k = 0; k < 16; k++) {
                        const int8_t cq = code_i8(__fmul_rn(v[k], inv));
                        sum += cq;
                        c[k >> 2] |= (uint32_t)(uint8_t)cq << (8 * (k & 3));
                    }
                    if (G == 2) sum += __shfl_xor(sum, 1, 64);
                    gsum = (float)sum;
                    pl[0] = make_uint4(c[0], c[1], c[2], c[3]);
                }
            }
            uint4* ent = (uint4*)(lds_a + (size_t)t * TS) + hg * E;
#pragma unroll
            for (int d = 0; d < D; d++) ent[d * M + m] = pl[d];
            if (m == 0) ent[E - 1] = make_uint4(0u, 0u, 0u, 0u);  // the zero entry
            // a 32-value group is two consecutive hexads: the first writes
            if (G == 4 || (x & 1) == 0) {
                const int sl = IF<T>::slot(hg);
                const int si = (((x >> 4) * G + sl) * M + m) * 4 + tl;
                lds_s[si] = gsum;
                if (D == 3) lds_sc[si] = gscale;
            }
        }
    }
    __syncthreads();
    r1 = IF<T>::fetch(rs, chunk_off(itf, jf), g, s_out);
    adv(itf, jf);

    // ---- per-lane A entry offsets (bytes within one MFMA's entries)
    const int ai = lane & 15, ae = ai & 3, aq = ai >> 2;
    const int as = aq % G, arg = aq / G;
    uint32_t aoff[NP];
#pragma unroll
    for (int p = 0; p < NP; p++) {
        int entry = E - 1;  // zero
        if (IF<T>::slot(g) == as) {
            if (D == 3) {
                const int m = p * RP + arg;
                if (ae < 3 && m < M) entry = ae * M + m;
            } else {
                const int m = p * RP + arg * NE + ae;
                if (ae < NE && m < M) entry = m;
            }
        }
        aoff[p] = 16u * (uint32_t)(g * E + entry);
    }
    constexpr int NS = D == 3 ? 1 : NE;  // rows per lane register set
    int srow[NP][NS];
#pragma unroll
    for (int p = 0; p < NP; p++)
#pragma unroll
        for (int e2 = 0; e2 < NS; e2++) {
            const int m = p * RP + (D == 3 ? rg_out : rg_out * NE + e2);
            srow[p][e2] = m < M ? m : M - 1;
        }

    constexpr int NACC = NP * NS;
    float acc[NACC];
#pragma unroll
    for (int k = 0; k < NACC; k++) acc[k] = 0.0f;

    auto compute = [&](const Raw& r_in, int c) __attribute__((always_inline)) {
        Raw r = r_in;
        IF<T>::bcast(r, col);
        float ca[4], cb[4];
        IF<T>::coef(r, s_out, ca, cb);
        const uint8_t* abase = lds_a + (size_t)c * 4 * TS;
        float sv[NP][NS][4], sc[NP][4];
        if (IF<T>::BIAS) {
#pragma unroll
            for (int p = 0; p < NP; p++)
#pragma unroll
                for (int e2 = 0; e2 < NS; e2++) {
                    const float4 v = *(const float4*)(lds_s + ((c * G + s_out) * M + srow[p][e2]) * 4);
                    sv[p][e2][0] = v.x; sv[p][e2][1] = v.y; sv[p][e2][2] = v.z; sv[p][e2][3] = v.w;
                }
        }
        if (D == 3) {
#pragma unroll
            for (int p = 0; p < NP; p++) {
                const float4 v = *(const float4*)(lds_sc + ((c * G + s_out) * M + srow[p][0]) * 4);
                sc[p][0] = v.x; sc[p][1] = v.y; sc[p][2] = v.z; sc[p][3] = v.w;
            }
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const v4i B = IF<T>::codes(r, t, g);
#pragma unroll
            for (int p = 0; p < NP; p++) {
                const v4i A = *(const v4i*)(abase + t * TS + aoff[p]);
                const v4i Z = {0, 0, 0, 0};
                const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, Z, 0, 0, 0);
                if constexpr (D == 3) {
                    const int hi2 = (int)(((uint32_t)C.x << 8) + (uint32_t)C.y);
                    const float P = fmaf((float)hi2, 256.0f, (float)C.z);
                    acc[p] = fmaf(ca[t] * sc[p][t], P, acc[p]);
                    if (IF<T>::BIAS) acc[p] = fmaf(cb[t], sv[p][0][t], acc[p]);
                } else {
                    const int cc[4] = {C.x, C.y, C.z, C.w};
#pragma unroll
                    for (int e2 = 0; e2 < NE; e2++) {
                        acc[p * NE + e2] = fmaf(ca[t], (float)cc[e2], acc[p * NE + e2]);
                        if (IF<T>::BIAS) acc[p * NE + e2] = fmaf(cb[t], sv[p][e2][t], acc[p * NE + e2]);
                    }
                }
            }
        }
    };

    // Tile end: lane groups of one output row are added (they differ in the
    // scale-group slot), then the KW wavefronts of the tile through LDS in
    // wavefront order; the first of them stores.
    int parity = 0;
    auto finish = [&](int fit) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < NACC; k++) {
            float v = acc[k];
            v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));  // lane ^ 16
            if (G == 4) v += __shfl_xor(v, 32, 64);
            acc[k] = v;
        }
        const int rl = ((fit - bx) / gx * TPI + slot_t) * 16 + col;  // local output row
        const bool holder = G == 2 ? ((g & 1) == 0) : (g == 0);
        auto store = [&](int k, float v) __attribute__((always_inline)) {
            const int p = k / NS, e2 = k % NS;
            const int m = p * RP + (D == 3 ? rg_out : rg_out * NE + e2);
            if (m < M) outl[m * ROWS + rl] = ldexpf(v * row_rs[m], row_re[m]);
        };
        if (KW == 1) {
            if (holder) {
#pragma unroll
                for (int k = 0; k < NACC; k++) store(k, acc[k]);
            }
        } else {
            float* rb_ = red + parity * (kWaves * MT * 16);
            if (holder) {
#pragma unroll
                for (int k = 0; k < NACC; k++) rb_[(w * NACC + k) * (RG * 16) + rg_out * 16 + col] = acc[k];
            }
            __syncthreads();
            if (kp == 0 && holder) {
#pragma unroll
                for (int k = 0; k < NACC; k++) {
                    float v = 0.0f;
                    for (int q = 0; q < KW; q++) v += rb_[((w + q) * NACC + k) * (RG * 16) + rg_out * 16 + col];
                    store(k, v);
                }
            }
            parity ^= 1;
        }
#pragma unroll
        for (int k = 0; k < NACC; k++) acc[k] = 0.0f;
    };

    // ---- main loop: three register sets in rotation; each step issues the
    // fetch two chunks ahead before computing the current one.
#define GGQ_I8_STEP(CUR, NXT)                                                   \
    {                                                                           \
        NXT = IF<T>::fetch(rs, chunk_off(itf, jf), g, s_out);                 \
        adv(itf, jf);                                                           \
        __builtin_amdgcn_sched_barrier(0);                                      \
        compute(CUR, kp + KW * i);                                              \
        if (i == nmy - 1) finish(it);                                           \
        adv(it, i);                                                             \
        if (it >= n_it) break;                                                  \
    }
    if (it < n_it) {
        while (true) {
            GGQ_I8_STEP(r0, r2)
            GGQ_I8_STEP(r1, r0)
            GGQ_I8_STEP(r2, r1)
        }
    }
#undef GGQ_I8_STEP
    __syncthreads();
    // this workgroup's outputs: tile iterations bx, bx + gx, ... of TPI tiles
    for (int idx = tid; idx < M * ROWS; idx += kThreads) {
        const int m = idx / ROWS, rl = idx % ROWS;
        const int j = rl / (TPI * 16), tr = rl % (TPI * 16);
        const int n = (bx + j * gx) * TPI * 16 + tr;
        if (n < N) {
            float v = outl[idx];
            if (FU && a.silu) v = v / (1.0f + expf(-v));  // cpu_ref.cpp:200-209
            if (FU && a.R) v = a.R[(int64_t)m * a.ldr + n] + v;
            a.Y[(int64_t)(yrow0 + m) * a.ldy + n] = v;
        }
    }
}

// Format sets a kernel is compiled for (the register allocation is the
// largest over its formats).
enum : int {
    FS_Q4K = 1 << 0, FS_Q5K = 1 << 1, FS_Q6K = 1 << 2, FS_Q80 = 1 << 3, FS_IQ4NL = 1 << 4, FS_IQ4XS = 1 << 5,
    FS_ALL = 63,
    FS_FUSED = 64,  // compiled with the fused options (fp32 mode)
};
__host__ __device__ constexpr int fs_bit(uint32_t t) {
    return t == T_Q4_K ? FS_Q4K : t == T_Q5_K ? FS_Q5K : t == T_Q6_K ? FS_Q6K : t == T_Q8_0 ? FS_Q80
         : t == T_IQ4_NL ? FS_IQ4NL : t == T_IQ4_XS ? FS_IQ4XS : 0;
}

template <int D, int NE, int NP, int FS>
__device__ __forceinline__ void i8_dispatch(const I8Args& args, const I8Prob& a, int bx, int gx, uint8_t* lds, int M,
                                            const int32_t* xrow, int yrow0) {
    switch (a.type) {
    case T_Q4_K: if constexpr ((FS & FS_Q4K) != 0) i8_gemv_body<T_Q4_K, D, NE, NP, (FS & FS_FUSED) != 0>(args, a, bx, gx, lds, M, xrow, yrow0); break;
    case T_Q5_K: if constexpr ((FS & FS_Q5K) != 0) i8_gemv_body<T_Q5_K, D, NE, NP, (FS & FS_FUSED) != 0>(args, a, bx, gx, lds, M, xrow, yrow0); break;
    case T_Q6_K: if constexpr ((FS & FS_Q6K) != 0) i8_gemv_body<T_Q6_K, D, NE, NP, (FS & FS_FUSED) != 0>(args, a, bx, gx, lds, M, xrow, yrow0); break;
    case T_Q8_0: if constexpr ((FS & FS_Q80) != 0) i8_gemv_body<T_Q8_0, D, NE, NP, (FS & FS_FUSED) != 0>(args, a, bx, gx, lds, M, xrow, yrow0); break;
    case T_IQ4_NL: if constexpr ((FS & FS_IQ4NL) != 0) i8_gemv_body<T_IQ4_NL, D, NE, NP, (FS & FS_FUSED) != 0>(args, a, bx, gx, lds, M, xrow, yrow0); break;
    case T_IQ4_XS: if constexpr ((FS & FS_IQ4XS) != 0) i8_gemv_body<T_IQ4_XS, D, NE, NP, (FS & FS_FUSED) != 0>(args, a, bx, gx, lds, M, xrow, yrow0); break;
    default: break;
    }
}

template <int D, int NE, int NP, int FS>
__global__ __launch_bounds__(kThreads) void i8_gemv_kernel(I8Args args) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    int q = 0;
    while (q + 1 < args.n && (int)blockIdx.x >= args.begin[q + 1]) q++;
    const int bx = blockIdx.x - args.begin[q], gx = args.begin[q + 1] - args.begin[q];
    i8_dispatch<D, NE, NP, FS>(args, args.p[q], bx, gx, lds, args.M, nullptr, 0);
}

// Grouped launches (MoE experts; fp32 rows, mode 0, or given int8 codes and
// row scales, mode 2): the rows of group e (pair rows grp_off[e] ..
// grp_off[e+1]-1) are cut into chunks of at most args.M rows; item i = (e,
// first row) of the device-built chunk list is grid row blockIdx.y.  Its
// weights are the problem's matrix advanced by e * w_stride bytes (group
// shared_group: the shared expert's matrix wsh[problem]), its activation
// rows rows x_idx[row] of X (or of QA / SA) (the row itself when x_idx is
// null), its outputs Y rows row ..  Grid rows past the list end exit.  Each
// chunk is a full pass over its group's weights.
struct I8Group {
    const int32_t* grp_off;
    const int32_t* x_idx;
    int64_t w_stride;
    const int2* items;
    const int32_t* n_items;
    int shared_group;  // -1: none
    const uint8_t* wsh[2];
};

template <int D, int NE, int NP, int FS>
__global__ __launch_bounds__(kThreads) void i8_gemv_grouped_kernel(I8Args args, I8Group gp) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    if ((int)blockIdx.y >= *gp.n_items) return;
    const int2 it = gp.items[blockIdx.y];
    const int e = it.x, r = it.y;
    const int end = gp.grp_off[e + 1];
    const int mc = end - r < args.M ? end - r : args.M;
    int q = 0;
    while (q + 1 < args.n && (int)blockIdx.x >= args.begin[q + 1]) q++;
    const int bx = blockIdx.x - args.begin[q], gx = args.begin[q + 1] - args.begin[q];
    I8Prob a = args.p[q];
    if (e == gp.shared_group) a.W = gp.wsh[q];
    else a.W += (int64_t)e * gp.w_stride;
    if (!gp.x_idx) {  // the chunk's own rows
        if (a.X) a.X += (int64_t)r * a.ldx;
        if (a.QA) {
            a.QA += (int64_t)r * a.K;
            a.SA += r;
        }
    }
    i8_dispatch<D, NE, NP, FS>(args, a, bx, gx, lds, mc, gp.x_idx ? gp.x_idx + r : nullptr, r);
}

// The chunk list: one thread per group counts its chunks, a scan over the
// workgroup places them (groups <= 1024).  t_sh > 0 appends a last group of
// t_sh rows (the shared expert: every token) first: grp_off[groups] =
// grp_off[groups - 1] + t_sh and x_idx of its rows = the token itself.
__global__ __launch_bounds__(1024) void i8_chunks_kernel(int32_t* __restrict__ grp_off, int groups, int mt,
                                                         int t_sh, int32_t* __restrict__ x_idx,
                                                         int2* __restrict__ items, int32_t* __restrict__ n_items) {
    __shared__ int cnt[1024];
    const ChunkList l{mt, items, n_items};
    build_chunk_lists(grp_off, groups, t_sh, x_idx, &l, 1, cnt);
}

int env_i8(const char* name, int dflt) {
    const char* e = getenv(name);
    return e && *e ? atoi(e) : dflt;
}

int cu_count() {
    static int v = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        return n;
    }();
    return v;
}

// Formats with four scale slots per MFMA (one row per pass in fp32 mode).
bool g4_format(uint32_t t) { return t == T_Q6_K || t == T_IQ4_NL || t == T_IQ4_XS; }

// Instantiation choice for M rows: (D, NE, NP) and the rows per pass.
struct I8Shape { int D, NE, NP; };
bool i8_shape(int M, int mode, bool has_q6, I8Shape& sh) {  // has_q6: a format with four slots per MFMA
    if (M < 1 || M > 8) return false;
    if (mode == 0) {
        // two rows per pass (one for Q6_K)
        const int rp = has_q6 ? 1 : 2;
        const int np = (M + rp - 1) / rp;
        if (np > 2) return false;  // more passes hold more accumulators than fit without spills
        sh = {3, 1, np};
        return true;
    }
    // int8 codes: rows in registers; NE rows per lane group
    const int rg = has_q6 ? 1 : 2;
    int ne = (M + rg - 1) / rg;
    if (ne <= 1) ne = 1;
    else if (ne <= 2) ne = 2;
    else ne = 4;
    const int np = (M + rg * ne - 1) / (rg * ne);
    if (np > 1) return false;
    sh = {1, ne, np};
    return true;
}

int i8_lds_bytes(int K, int M, bool q6, const I8Shape& sh) {
    const int G = q6 ? 4 : 2;
    const int mt = (4 / G) * (sh.D == 1 ? sh.NE : 1) * sh.NP;
    return i8_lds_total(K, G, sh.D, M, mt);
}

constexpr int kMaxLds = 150 * 1024;

// Wavefronts per tile and workgroups per problem of a launch (one
// 1024-thread workgroup per CU), and the LDS it needs: lds_need (set-up and
// reduction) plus each workgroup's output rows.
struct I8Grid { int kw_log2[kMaxProbs], gx[kMaxProbs]; int lds; };
I8Grid i8_grid(const GemvProblem* ps, int n, const int* lds_need, int M) {
    I8Grid gr{};
    const int resident = cu_count();
    const int resident_waves = resident * kWaves;
    // wavefronts per tile: split K so the launch fills the resident waves
    int tiles_total = 0;
    for (int i = 0; i < n; i++) tiles_total += (ps[i].N + 15) / 16;
    const int kw_env = env_i8("GGQ_I8_KW", 0);
    int want[kMaxProbs];
    int want_total = 0;
    for (int i = 0; i < n; i++) {
        const GemvProblem& p = ps[i];
        const int nc = p.K / 256, tiles = (p.N + 15) / 16;
        int kw = 1;
        while (kw < 16 && 2 * kw <= nc && tiles_total * 2 * kw <= resident_waves) kw *= 2;
        if (kw_env > 0) {
            kw = 1;
            while (2 * kw <= kw_env && 2 * kw <= nc && kw < 16) kw *= 2;
        }
        gr.kw_log2[i] = __builtin_ctz(kw);
        const int tpi = kWaves / kw;
        want[i] = (tiles + tpi - 1) / tpi;
        want_total += want[i];
    }
    // workgroups per problem: all it can use when the launch fits the
    // resident capacity, else in proportion
    gr.lds = 0;
    for (int i = 0; i < n; i++) {
        int gxi = want[i];
        if (want_total > resident) {
            gxi = (int)((int64_t)want[i] * resident / want_total);
            gxi = gxi < 1 ? 1 : gxi;
        }
        gr.gx[i] = gxi;
        const int tpi = kWaves >> gr.kw_log2[i];
        const int rows = (want[i] + gxi - 1) / gxi * tpi * 16;
        const int need = lds_need[i] + rows * M * 4;
        gr.lds = need > gr.lds ? need : gr.lds;
    }
    return gr;
}

template <int D, int NE, int NP, int FS>
hipError_t i8_run(I8Args& args, const I8Grid& gr, int n, hipStream_t s) {
    auto kern = i8_gemv_kernel<D, NE, NP, FS>;
    // set once per process (thread-safe static initialisation); a failure
    // is reported by every launch that needs the attribute
    static const hipError_t attr =
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    if (attr != hipSuccess) return attr;
    const int lds = gr.lds;
    args.begin[0] = 0;
    for (int i = 0; i < n; i++) {
        args.p[i].kw_log2 = gr.kw_log2[i];
        args.begin[i + 1] = args.begin[i] + gr.gx[i];
    }
    args.n = n;
    kern<<<args.begin[n], kThreads, lds, s>>>(args);
    return hipGetLastError();
}

}  // namespace

bool i8_gemv_eligible(const GemvProblem* ps, int n, int mode) {
    // GGQ_GEMV_MFMA=0 keeps every GEMV on the fp32 FMA kernels
    if (env_i8("GGQ_GEMV_MFMA", 1) == 0 || n < 1 || n > kMaxProbs) return false;
    bool q6 = false;
    for (int i = 0; i < n; i++) q6 = q6 || g4_format(ps[i].type);
    I8Shape sh;
    if (!i8_shape(ps[0].M, mode, q6, sh)) return false;
    for (int i = 0; i < n; i++) {
        const GemvProblem& p = ps[i];
        if (p.M != ps[0].M || !supported(p.type)) return false;
        if (p.grp_off || p.W2 || p.n1 > 0 || p.q8row) return false;
        if (mode != 0 && (p.X2 || p.rms || p.R || p.silu)) return false;  // fused options: fp32 mode only
        if (p.K % 256 != 0 || p.K <= 0 || p.N <= 0 || p.groups > 1) return false;
        if (p.N * row_bytes(p.type, p.K) >= (int64_t)kOOB) return false;  // buffer offsets below kOOB
    }
    if (mode == 0) {
        // fp32 activations: the matrix-core kernel pays a fixed set-up (the
        // activation digits in LDS, 1024-thread workgroups, one per tile
        // group) that only launches moving enough weight bytes amortize;
        // smaller ones stay on the fp32 kernels (GGQ_I8_MIN_BYTES, bytes).
        int64_t bytes = 0;
        for (int i = 0; i < n; i++) bytes += (int64_t)ps[i].N * row_bytes(ps[i].type, ps[i].K);
        if (bytes < (int64_t)env_i8("GGQ_I8_MIN_BYTES", 16 << 20)) return false;
    }
    int lds_need[kMaxProbs];
    for (int i = 0; i < n; i++) lds_need[i] = i8_lds_bytes(ps[i].K, ps[i].M, g4_format(ps[i].type), sh);
    return i8_grid(ps, n, lds_need, ps[0].M).lds <= kMaxLds;
}

hipError_t launch_i8_gemv(const GemvProblem* ps, int n, int mode, const int8_t* qa, const float* sa, hipStream_t s) {
    if (n < 1 || n > kMaxProbs) return hipErrorInvalidValue;
    const int M = ps[0].M;
    bool q6 = false;
    for (int i = 0; i < n; i++) {
        if (ps[i].M != M) return hipErrorInvalidValue;
        q6 = q6 || g4_format(ps[i].type);
    }
    I8Shape sh;
    if (!i8_shape(M, mode, q6, sh)) return hipErrorInvalidValue;
    I8Args args{};
    args.M = M;
    args.mode = mode;
    int lds_need[kMaxProbs];
    for (int i = 0; i < n; i++) {
        const GemvProblem& g = ps[i];
        I8Prob& p = args.p[i];
        p.W = (const uint8_t*)g.W;
        p.row_bytes = (uint32_t)row_bytes(g.type, g.K);
        p.type = g.type;
        p.N = g.N;
        p.K = g.K;
        p.X = g.X;
        p.ldx = g.ldx;
        p.QA = qa;
        p.SA = sa;
        p.Y = g.Y;
        p.ldy = g.ldy;
        p.x_vec4 = g.X && ((uintptr_t)g.X % 16 == 0) && (g.ldx % 4 == 0) && ((uintptr_t)g.X2 % 16 == 0);
        p.X2 = g.X2;
        p.norm_w = g.norm_w;
        p.nw_vec4 = (uintptr_t)g.norm_w % 16 == 0;
        p.R = g.R;
        p.ldr = g.ldr;
        p.rms = g.rms;
        p.silu = g.silu;
        p.eps = g.eps;
        lds_need[i] = i8_lds_bytes(g.K, M, g4_format(g.type), sh);  // each format's own geometry
        if (lds_need[i] > kMaxLds) return hipErrorInvalidValue;
    }
    int fs = 0;
    for (int i = 0; i < n; i++) fs |= fs_bit(ps[i].type);
    // one format, or the Q4_K_M pair (Q4_K and Q6_K), each get their own
    // kernel; other mixes the kernel compiled for all formats
    const I8Grid gr = i8_grid(ps, n, lds_need, M);
    if (gr.lds > kMaxLds) return hipErrorInvalidValue;
#define R(D_, NE_, NP_)                                                                          \
    switch (fs) {                                                                                \
    case FS_Q4K: return i8_run<D_, NE_, NP_, FS_Q4K>(args, gr, n, s);                      \
    case FS_Q6K: return i8_run<D_, NE_, NP_, FS_Q6K>(args, gr, n, s);                      \
    case FS_Q4K | FS_Q6K: return i8_run<D_, NE_, NP_, FS_Q4K | FS_Q6K>(args, gr, n, s);    \
    case FS_Q80: return i8_run<D_, NE_, NP_, FS_Q80>(args, gr, n, s);                      \
    default: return i8_run<D_, NE_, NP_, FS_ALL>(args, gr, n, s);                          \
    }
    bool fused = false;
    for (int i = 0; i < n; i++) fused = fused || ps[i].X2 || ps[i].rms || ps[i].R || ps[i].silu;
    if (fused) {
        if (sh.D != 3) return hipErrorInvalidValue;
#define RF(NP_)                                                                                    \
    switch (fs) {                                                                                  \
    case FS_Q4K: return i8_run<3, 1, NP_, FS_Q4K | FS_FUSED>(args, gr, n, s);                    \
    case FS_Q6K: return i8_run<3, 1, NP_, FS_Q6K | FS_FUSED>(args, gr, n, s);                    \
    case FS_Q4K | FS_Q6K: return i8_run<3, 1, NP_, FS_Q4K | FS_Q6K | FS_FUSED>(args, gr, n, s);  \
    default: return i8_run<3, 1, NP_, FS_ALL | FS_FUSED>(args, gr, n, s);                        \
    }
        if (sh.NP == 1) RF(1);
        RF(2);
#undef RF
    }
    if (sh.D == 3) {
        if (sh.NP == 1) R(3, 1, 1);
        R(3, 1, 2);
    }
    switch (sh.NE) {
    case 1: R(1, 1, 1);
    case 2: R(1, 2, 1);
    default: R(1, 4, 1);
    }
#undef R
}

}  // namespace ggq

namespace ggq {
namespace {

template <int D, int NE, int NP, int FS>
hipError_t i8_run_grouped(I8Args& args, const I8Group& gp, int groups, int lds, hipStream_t s) {
    auto kern = i8_gemv_grouped_kernel<D, NE, NP, FS>;
    // set once per process (thread-safe static initialisation); a failure
    // is reported by every launch that needs the attribute
    static const hipError_t attr =
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    if (attr != hipSuccess) return attr;
    kern<<<dim3(args.begin[args.n], groups), kThreads, lds, s>>>(args, gp);  // groups: chunk-list bound
    return hipGetLastError();
}

// Shape of a grouped launch: rows per pass, wavefronts per tile and
// workgroups per problem and group, and the LDS it needs.
struct I8GroupedPlan { I8Shape sh; int mt, kw_log2, gx, lds; };

// Workgroups per (problem, chunk): GGQ_MOE_I8_GX when set, else enough to
// fill one 1024-thread workgroup per CU over the chunk-list bound (one per
// chunk once the chunks alone fill the chip: 64 qwen35moe tokens), at most
// one per tile iteration.
int i8_grouped_gx(int rows, int groups, int mt, int np, int n_it) {
    int gx = env_i8("GGQ_MOE_I8_GX", 0);
    if (gx <= 0) {
        const int items = (rows + mt - 1) / mt + (groups < rows ? groups : rows);
        const int per = np * (items > 0 ? items : 1);
        gx = (cu_count() + per - 1) / per;
    }
    if (gx < 1) gx = 1;
    return gx > n_it ? n_it : gx;
}

bool i8_grouped_plan(const GemvProblem& g, I8GroupedPlan& pl) {
    const bool q6 = g4_format(g.type);
    // fp32 mode: two rows per pass (one for four-slot formats), two passes
    if (!i8_shape(q6 ? 2 : 4, 0, q6, pl.sh)) return false;
    pl.mt = (q6 ? 1 : 2) * pl.sh.NP;
    const int nc = g.K / 256;
    // one workgroup per (problem, chunk), four wavefronts per tile: measured
    // best at the qwen35moe shape (GGQ_MOE_I8_GX 1 / 2 / 4 / 8: 209 / 223 /
    // 240 / 250 us per layer; the wavefront count per tile within noise)
    int kw = env_i8("GGQ_MOE_I8_KW", 4);
    int k2 = 1;
    while (2 * k2 <= kw && 2 * k2 <= nc && k2 < kWaves) k2 *= 2;
    pl.kw_log2 = __builtin_ctz(k2);
    const int n1 = g.n1 > 0 ? g.n1 : g.N;
    const int tiles = (n1 + 15) / 16, tpi = kWaves / k2;
    const int n_it = (tiles + tpi - 1) / tpi;
    pl.gx = i8_grouped_gx(g.M, g.groups, pl.mt, g.n1 > 0 ? 2 : 1, n_it);
    const int iters_wg = (n_it + pl.gx - 1) / pl.gx;
    pl.lds = i8_lds_bytes(g.K, pl.mt, q6, pl.sh) + iters_wg * tpi * 16 * pl.mt * 4;
    return pl.lds <= kMaxLds;
}

}  // namespace

// Upper bound of the chunk list: every chunk but the last of a group holds
// mt rows, and at most min(groups, rows) groups are non-empty.
static int i8_max_items(const GemvProblem& g, int mt, int t_sh = 0) {
    const int rows = g.M + t_sh, groups = g.groups + (t_sh > 0 ? 1 : 0);
    return (rows + mt - 1) / mt + (groups < rows ? groups : rows);
}

size_t i8_gemv_grouped_ws_bytes(const GemvProblem& g, int t_sh) {
    I8GroupedPlan pl;
    if (!i8_grouped_plan(g, pl)) return 0;
    return 8 * (size_t)i8_max_items(g, pl.mt, t_sh) + 16;
}

bool i8_gemv_grouped_eligible(const GemvProblem& g) {
    if (env_i8("GGQ_MOE_I8", 1) == 0 || env_i8("GGQ_GEMV_MFMA", 1) == 0) return false;
    if (!g.grp_off || g.groups < 1 || g.groups > 1023 || g.M < 1 || !supported(g.type) || g.K % 256 != 0 || g.K <= 0 || g.N <= 0) return false;
    if (g.X2 || g.rms || g.R || g.silu || g.q8row) return false;
    const int n1 = g.n1 > 0 ? g.n1 : g.N;
    if (g.n1 > 0 && (!g.W2 || !g.Y2 || g.N - g.n1 != g.n1)) return false;  // paired halves of equal size
    if ((int64_t)n1 * row_bytes(g.type, g.K) >= (int64_t)kOOB) return false;
    I8GroupedPlan pl;
    return i8_grouped_plan(g, pl) && i8_max_items(g, pl.mt) <= 65535;
}

ChunkList i8_gemv_grouped_list(const GemvProblem& g, void* ws, int t_sh) {
    I8GroupedPlan pl;
    if (!i8_grouped_plan(g, pl)) return ChunkList{0, nullptr, nullptr};
    const int max_items = i8_max_items(g, pl.mt, t_sh);
    return ChunkList{pl.mt, (int2*)ws, (int32_t*)((char*)ws + 8 * (size_t)max_items)};
}

hipError_t launch_i8_gemv_grouped(const GemvProblem& g, void* ws, hipStream_t s, const I8Shared* sh, bool list_ready) {
    I8GroupedPlan pl;
    if (!i8_grouped_plan(g, pl) || !ws || g.groups + (sh ? 1 : 0) > 1024) return hipErrorInvalidValue;
    if (sh && (!g.x_idx || sh->T < 1 || (g.n1 > 0 && !sh->W2))) return hipErrorInvalidValue;
    const int max_items = i8_max_items(g, pl.mt, sh ? sh->T : 0);
    const ChunkList cl = i8_gemv_grouped_list(g, ws, sh ? sh->T : 0);
    int2* items = cl.items;
    int32_t* n_items = cl.n_items;
    const int groups = g.groups + (sh ? 1 : 0);
    if (!list_ready)
        i8_chunks_kernel<<<1, 1024, 0, s>>>((int32_t*)g.grp_off, groups, pl.mt, sh ? sh->T : 0, (int32_t*)g.x_idx,
                                            items, n_items);
    const int n1 = g.n1 > 0 ? g.n1 : g.N;
    I8Args args{};
    args.M = pl.mt;
    args.mode = 0;
    const int np = g.n1 > 0 ? 2 : 1;
    for (int i = 0; i < np; i++) {
        I8Prob& p = args.p[i];
        p.W = (const uint8_t*)(i == 0 ? g.W : g.W2);
        p.row_bytes = (uint32_t)row_bytes(g.type, g.K);
        p.type = g.type;
        p.N = n1;
        p.K = g.K;
        p.X = g.X;
        p.ldx = g.ldx;
        p.Y = i == 0 ? g.Y : g.Y2;
        p.ldy = g.ldy;
        p.kw_log2 = pl.kw_log2;
        p.x_vec4 = ((uintptr_t)g.X % 16 == 0) && (g.ldx % 4 == 0);
        args.begin[i + 1] = args.begin[i] + pl.gx;
    }
    args.n = np;
    I8Group gp{g.grp_off, g.x_idx, g.w_group_stride, items, n_items, sh ? g.groups : -1,
               {sh ? (const uint8_t*)sh->W : nullptr, sh ? (const uint8_t*)sh->W2 : nullptr}};
    const int fs = fs_bit(g.type);
#define RG(NP_)                                                                                  \
    switch (fs) {                                                                                \
    case FS_Q4K: return i8_run_grouped<3, 1, NP_, FS_Q4K>(args, gp, max_items, pl.lds, s);      \
    case FS_Q6K: return i8_run_grouped<3, 1, NP_, FS_Q6K>(args, gp, max_items, pl.lds, s);      \
    case FS_Q80: return i8_run_grouped<3, 1, NP_, FS_Q80>(args, gp, max_items, pl.lds, s);      \
    default: return i8_run_grouped<3, 1, NP_, FS_ALL>(args, gp, max_items, pl.lds, s);          \
    }
    if (pl.sh.D != 3) return hipErrorInvalidValue;
    if (pl.sh.NP == 1) RG(1);
    RG(2);
#undef RG
}

}  // namespace ggq

namespace ggq {

// Per-row int8 MoE (mode 2: the codes and row scales are given): chunks of
// up to 8 rows (4 for the four-slot formats), the shared expert as group E.
static bool i8_moe_q8_plan(uint32_t type, const MoeGemm& g, int rows, I8GroupedPlan& pl) {
    const bool q6 = g4_format(type);
    if (!i8_shape(q6 ? 4 : 8, 2, q6, pl.sh) || pl.sh.NP != 1 || pl.sh.NE != 4) return false;
    pl.mt = (q6 ? 1 : 2) * 4;
    const int nc = g.K / 256;
    int kw = env_i8("GGQ_MOE_I8_KW", 4), k2 = 1;
    while (2 * k2 <= kw && 2 * k2 <= nc && k2 < kWaves) k2 *= 2;
    pl.kw_log2 = __builtin_ctz(k2);
    const int n1 = g.n1 > 0 ? g.n1 : g.N;
    const int tiles = (n1 + 15) / 16, tpi = kWaves / k2;
    const int n_it = (tiles + tpi - 1) / tpi;
    pl.gx = i8_grouped_gx(rows, g.E + (g.Wsh ? 1 : 0), pl.mt, g.W2 ? 2 : 1, n_it);
    const int iters_wg = (n_it + pl.gx - 1) / pl.gx;
    pl.lds = i8_lds_bytes(g.K, pl.mt, q6, pl.sh) + iters_wg * tpi * 16 * pl.mt * 4;
    return pl.lds <= kMaxLds;
}

static int i8_moe_groups(const MoeGemm& g) { return g.E + (g.Wsh ? 1 : 0); }

size_t i8_moe_q8_ws_bytes(uint32_t type, const MoeGemm& g, int rows) {
    I8GroupedPlan pl;
    if (!i8_moe_q8_plan(type, g, rows, pl)) return 0;
    const int groups = i8_moe_groups(g);
    return 8 * (size_t)((rows + pl.mt - 1) / pl.mt + (groups < rows ? groups : rows)) + 16;
}

bool i8_moe_q8_eligible(uint32_t type, const MoeGemm& g, int rows) {
    if (env_i8("GGQ_MOE_I8", 1) == 0 || env_i8("GGQ_GEMV_MFMA", 1) == 0) return false;
    if (!supported(type) || g.K % 256 != 0 || g.K <= 0 || g.N <= 0 || rows < 1) return false;
    const int groups = i8_moe_groups(g);
    if (groups > 1024) return false;
    const int n1 = g.n1 > 0 ? g.n1 : g.N;
    if (g.W2 && g.N - n1 != n1) return false;  // paired halves of equal size
    if (g.Wsh && g.W2 && !g.W2sh) return false;
    if ((int64_t)n1 * row_bytes(type, g.K) >= (int64_t)kOOB) return false;
    I8GroupedPlan pl;
    if (!i8_moe_q8_plan(type, g, rows, pl)) return false;
    return (rows + pl.mt - 1) / pl.mt + (groups < rows ? groups : rows) <= 65535;
}

ChunkList i8_moe_q8_list(uint32_t type, const MoeGemm& g, int rows, void* ws) {
    I8GroupedPlan pl;
    if (!i8_moe_q8_plan(type, g, rows, pl)) return ChunkList{0, nullptr, nullptr};
    const int groups = i8_moe_groups(g);
    const int max_items = (rows + pl.mt - 1) / pl.mt + (groups < rows ? groups : rows);
    return ChunkList{pl.mt, (int2*)ws, (int32_t*)((char*)ws + 8 * (size_t)max_items)};
}

hipError_t launch_i8_moe_q8(uint32_t type, const MoeGemm& g, int rows, void* ws, hipStream_t s, bool list_ready) {
    I8GroupedPlan pl;
    if (!i8_moe_q8_plan(type, g, rows, pl) || !ws) return hipErrorInvalidValue;
    const int groups = i8_moe_groups(g);
    if (groups > 1024) return hipErrorInvalidValue;
    const int max_items = (rows + pl.mt - 1) / pl.mt + (groups < rows ? groups : rows);
    const ChunkList cl = i8_moe_q8_list(type, g, rows, ws);
    int2* items = cl.items;
    int32_t* n_items = cl.n_items;
    if (!list_ready) i8_chunks_kernel<<<1, 1024, 0, s>>>((int32_t*)g.grp, groups, pl.mt, 0, nullptr, items, n_items);
    const int n1 = g.n1 > 0 ? g.n1 : g.N;
    I8Args args{};
    args.M = pl.mt;
    args.mode = 2;
    const int np = g.W2 ? 2 : 1;
    for (int i = 0; i < np; i++) {
        I8Prob& p = args.p[i];
        p.W = (const uint8_t*)(i == 0 ? g.W : g.W2);
        p.row_bytes = (uint32_t)row_bytes(type, g.K);
        p.type = type;
        p.N = n1;
        p.K = g.K;
        p.QA = g.QA;
        p.SA = g.sa;
        p.Y = i == 0 ? g.C : g.C2;
        p.ldy = g.ldc;
        p.kw_log2 = pl.kw_log2;
        args.begin[i + 1] = args.begin[i] + pl.gx;
    }
    args.n = np;
    I8Group gp{g.grp, g.x_idx, g.w_stride, items, n_items, g.Wsh ? g.E : -1,
               {(const uint8_t*)g.Wsh, (const uint8_t*)g.W2sh}};
    switch (fs_bit(type)) {
    case FS_Q4K: return i8_run_grouped<1, 4, 1, FS_Q4K>(args, gp, max_items, pl.lds, s);
    case FS_Q6K: return i8_run_grouped<1, 4, 1, FS_Q6K>(args, gp, max_items, pl.lds, s);
    case FS_Q80: return i8_run_grouped<1, 4, 1, FS_Q80>(args, gp, max_items, pl.lds, s);
    default: return i8_run_grouped<1, 4, 1, FS_ALL>(args, gp, max_items, pl.lds, s);
    }
}

namespace {

// ============================================ expert-grouped row tiles
// The down projection of a MoE layer at decode-sized batches (a few pair
// rows per expert), fp32 activations: a unit of work is 128 weight rows
// (a row tile) of one group (expert, or the shared expert) times up to 4 of
// the group's activation rows (a pass) on v_mfma_i32_32x32x32_i8, so the
// weight codes are decoded once per 4 rows.  The units are spread evenly
// over a grid of resident workgroups.
//
// MFMA layout (32 x 32 x 32, int8): lane l supplies row / column l % 32 of
// A / B for K-slice 16 (l / 32) .. + 16, and holds output rows 8 (r / 4) +
// 4 (l / 32) + r % 4 (register r) of column l % 32.  B column c is weight
// row n0 + c; K-step j covers values 32 j .. 32 j + 31, lane half h values
// 32 j + 16 h + [0, 16): one Q6_K 16-value scale group.  Activation rows
// are fixed point X = rint(x 2^e) with the row's largest magnitude in
// [2^29, 2^30), written as four signed int8 digits (X = sum_d digit_d
// 256^d), so |x - 2^-e X| <= 2^-30 of the row maximum.  A row 8 m + 4 s + d
// holds digit d of activation row m in lane half s and zeros in the other
// half; so output lane (c, h) finds in registers 4 m + d the digit-d dot
// products of row m with its own 16 codes (scale group sc[.., h]), and
// accumulates sc * C in int32 per Q6_K block (exact: |C| <= 2^16,
// |sc * C| <= 2^23, 8 K-steps), then d_block * sum_d I_d 256^d in fp32.
// Codes are taken signed (q - 32), so no offset term remains.  The two lane
// halves' sums are added at the end and scaled by 2^-e.
constexpr int kTileRows = 128;   // weight rows per workgroup (4 wavefronts x 32)
constexpr int kTileMR = 4;       // activation rows per pass
constexpr int kTileMaxK = 1024;  // K limit: a pass's digit planes take 16 K bytes of LDS (two buffers)
constexpr int kTilePre = 4160;   // LDS bytes of the unit prefix (up to 1024 groups + 1)

struct I8TileArgs {
    const uint8_t* W;  // group g's matrix at W + g * w_stride
    int64_t w_stride;
    const uint8_t* Wsh;  // group E (optional): the shared expert
    const float* X;      // activation rows, grouped: group g's rows grp_off[g] .. grp_off[g+1]-1
    int ldx;
    const int32_t* grp_off;
    int E, t_sh;  // routed groups; rows of the shared group (grp_off[E] ..)
    float* Y;     // output rows, as X's
    float* Ysh;   // the shared group's output rows (from 0)
    int ldy;
    int N, K;
    uint32_t row_bytes;
    int groups;  // E, plus the shared group
};

// Q6_K block (kquant.h:182-202) of one lane: for half nh, ql[64 nh + 16 h]
// (values 128 nh + 16 h + i, low nibbles; + 64, high nibbles), ql[64 nh +
// 32 + 16 h] (+ 32 / + 96) and qh[32 nh + 16 h] (2-bit fields 0, 2, 4, 6 for
// + 0, + 32, + 64, + 96); scales sc[8 nh + 2 t + h] for K-step t of the
// half; d at 208.
struct TileQ6 {
    v4u ql0[2], ql1[2], qh[2], sc;
    uint32_t d;
};
// (d and the scales are loaded first: loads complete in issue order, so
// waiting for the first codes covers them)
__device__ __forceinline__ TileQ6 tile_q6_fetch(Rsrc rs, uint32_t off, int h) {
    TileQ6 r;
    r.d = bl2(rs, off + 208);
    r.sc = bl16(rs, off + 192);
#pragma unroll
    for (int nh = 0; nh < 2; nh++) {
        r.ql0[nh] = bl16(rs, off + 64 * nh + 16 * h);
        r.ql1[nh] = bl16(rs, off + 64 * nh + 32 + 16 * h);
        r.qh[nh] = bl16(rs, off + 128 + 32 * nh + 16 * h);
    }
    return r;
}
// Signed codes q - 32 of K-step t of half nh: low 4 bits from ql, the top
// two (hh) as the 4-bit two's complement of hh - 2 in bits 4..7.
__device__ __forceinline__ uint32_t q6_signed(uint32_t ql, uint32_t qh, int t) {
    const uint32_t lo = (t >> 1) ? (ql >> 4) & 0x0F0F0F0Fu : ql & 0x0F0F0F0Fu;
    const uint32_t hh = (qh >> (2 * t)) & 0x03030303u;
    return lo | (((hh + 0x0E0E0E0Eu) & 0x0F0F0F0Fu) << 4);
}
__device__ __forceinline__ v4i tile_q6_codes(const TileQ6& r, int nh, int t) {
    const v4u ql = (t & 1) ? r.ql1[nh] : r.ql0[nh];
    const v4u qh = r.qh[nh];
    v4i c;
    c.x = (int)q6_signed(ql.x, qh.x, t); c.y = (int)q6_signed(ql.y, qh.y, t);
    c.z = (int)q6_signed(ql.z, qh.z, t); c.w = (int)q6_signed(ql.w, qh.w, t);
    return c;
}
__device__ __forceinline__ int tile_q6_scale(const TileQ6& r, int nh, int t, int h) {
    const int i = 2 * nh + (t >> 1);
    const uint32_t w = i == 0 ? r.sc.x : i == 1 ? r.sc.y : i == 2 ? r.sc.z : r.sc.w;
    return __builtin_amdgcn_sbfe((int)w, 16 * (t & 1) + 8 * h, 8);
}

// A wavefront's 32 rows of one Q6_K block, loaded coalesced: bytes 0..207
// of each row as 13 16-byte pieces, chunk c = lane + 64 i (c < 416) being
// piece c % 13 of row c / 13, staged in LDS at 240 bytes a row (stride 60
// dwords: the 16-byte reads of 8 consecutive lanes fall in distinct banks)
// and read back per lane; d (bytes 208..209) is loaded by each lane for its
// own row (a 16-byte piece there would reach past the end of the matrix).
constexpr int kTileStageRow = 240;
constexpr int kTileStage = 32 * kTileStageRow;  // LDS bytes per wavefront
struct TileRaw {
    v4u c[7];
    uint32_t d;
};
__device__ __forceinline__ TileRaw tile_raw_fetch(Rsrc rs, const uint32_t (&off)[7], uint32_t doff) {
    TileRaw r;
    r.d = bl2(rs, doff);
#pragma unroll
    for (int i = 0; i < 7; i++) r.c[i] = bl16(rs, off[i]);
    return r;
}
__device__ __forceinline__ TileQ6 tile_q6_stage(const TileRaw& r, uint8_t* st, const uint32_t (&soff)[7], int col, int h) {
#pragma unroll
    for (int i = 0; i < 7; i++)
        if (i < 6 || soff[i] != ~0u) *(v4u*)(st + soff[i]) = r.c[i];
    const uint8_t* row = st + col * kTileStageRow;
    TileQ6 q;
#pragma unroll
    for (int nh = 0; nh < 2; nh++) {
        q.ql0[nh] = *(const v4u*)(row + 64 * nh + 16 * h);
        q.ql1[nh] = *(const v4u*)(row + 64 * nh + 32 + 16 * h);
        q.qh[nh] = *(const v4u*)(row + 128 + 32 * nh + 16 * h);
    }
    q.sc = *(const v4u*)(row + 192);
    q.d = r.d;
    return q;
}

// Work units (group g, pass of up to 4 of its rows, row tile), ordered
// group-major, are split evenly over a resident grid; each workgroup
// streams its units' weight blocks with loads two blocks ahead across unit
// boundaries, and rebuilds the activation planes (double-buffered, one
// barrier) when the unit's (group, pass) changes.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void i8_tile_grouped_kernel(I8TileArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, h = lane >> 5;
    const int NB = a.K >> 8, NJ = a.K >> 5, G = a.groups;
    const int ntiles = (a.N + kTileRows - 1) / kTileRows;
    // LDS: unit prefix [G + 1], two plane buffers [m][d][j][half] (16 B
    // entries), a zero plane [j][half], the rows' exponents [2][4], the
    // scan's wavefront totals
    int* pre = (int*)lds;
    const int PB = kTileMR * 4 * NJ * 32;
    uint8_t* planes = lds + kTilePre;
    uint8_t* zero = planes + 2 * PB;
    int* lexp = (int*)(zero + NJ * 32);
    int* wsum = lexp + 2 * kTileMR;
    uint8_t* stage = lds + kTilePre + 2 * PB + NJ * 32 + 64 + w * kTileStage;
    for (int i = tid; i < NJ * 2; i += 256) ((uint4*)zero)[i] = make_uint4(0u, 0u, 0u, 0u);
    auto group_rows = [&](int g, int& r0) __attribute__((always_inline)) {
        if (g == a.E) {
            r0 = a.grp_off[a.E];
            return a.t_sh;
        }
        r0 = a.grp_off[g];
        return a.grp_off[g + 1] - r0;
    };
    // units per group, exclusive prefix over the workgroup (4 groups per
    // thread, G <= 1024)
    {
        int cnt[4], tsum = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int g = 4 * tid + i;
            int r0 = 0;
            const int rows = g < G ? group_rows(g, r0) : 0;
            cnt[i] = (rows + kTileMR - 1) / kTileMR * ntiles;
            tsum += cnt[i];
        }
        int x = tsum;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        if (lane == 63) wsum[w] = x;
        __syncthreads();
        int ex = x - tsum;
        for (int k = 0; k < w; k++) ex += wsum[k];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int g = 4 * tid + i;
            if (g <= G) pre[g] = ex;
            ex += cnt[i];
        }
        __syncthreads();
    }
    // (values read from LDS are uniform: kept in scalar registers, so the
    // buffer resource chosen from them needs no per-lane loop)
    auto upre = [&](int g) __attribute__((always_inline)) { return __builtin_amdgcn_readfirstlane(pre[g]); };
    const int U = upre(G);
    const int u0 = (int)((int64_t)U * blockIdx.x / gridDim.x), u1 = (int)((int64_t)U * (blockIdx.x + 1) / gridDim.x);
    if (u0 >= u1) return;
    // the group of unit u: the last g with pre[g] <= u (groups without units
    // have pre[g] == pre[g + 1])
    auto group_of = [&](int u) __attribute__((always_inline)) {
        int lo = 0, hi = G - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (upre(mid) <= u) lo = mid;
            else hi = mid - 1;
        }
        return lo;
    };
    const Rsrc rs_r = make_rsrc(a.W, (uint32_t)(a.E >= 0 ? a.E : G) * (uint32_t)a.w_stride);
    const Rsrc rs_s = make_rsrc(a.Wsh ? a.Wsh : a.W, (uint32_t)a.N * a.row_bytes);
    // Unit cursors (group, unit index within it, the group's unit count),
    // advanced one unit at a time: the fetch cursor runs one unit ahead of
    // the compute cursor.
    struct UCur { int g, local, end; };
    auto ucur_next = [&](UCur& c) __attribute__((always_inline)) {
        if (++c.local >= c.end) {
            do {
                ++c.g;
            } while (c.g < G && upre(c.g + 1) == upre(c.g));
            c.local = 0;
            c.end = c.g < G ? upre(c.g + 1) - upre(c.g) : 0;
        }
    };
    UCur fc;
    fc.g = group_of(u0);
    fc.local = u0 - upre(fc.g);
    fc.end = upre(fc.g + 1) - upre(fc.g);
    UCur cc = fc;
    const int n_pos = (u1 - u0) * NB;
    int fq = 0, fb = 0;
    // this lane's pieces: chunk c = lane + 64 i is piece c % 14 of row c / 14
    // of the wavefront's 32; its LDS staging offset
    uint32_t soff[7], poff[7];
    int prow[7];
#pragma unroll
    for (int i = 0; i < 7; i++) {
        const int c = lane + 64 * i;
        prow[i] = c < 416 ? c / 13 : 0;
        poff[i] = 16u * (uint32_t)(c % 13);
        soff[i] = c < 416 ? (uint32_t)(prow[i] * kTileStageRow) + poff[i] : ~0u;
    }
    // the next position's block (the wavefront's rows of the unit's tile,
    // block fb); out of range past the last position
    auto fetch = [&]() __attribute__((always_inline)) {
        uint32_t roff[7], doff = kOOB;
        bool sh = false;
        if (fq < n_pos) {
            const int n0 = (fc.local % ntiles) * kTileRows + w * 32;
            sh = fc.g == a.E;
            const uint32_t base = (sh ? 0u : (uint32_t)fc.g * (uint32_t)a.w_stride) + (uint32_t)fb * 210u;
#pragma unroll
            for (int i = 0; i < 7; i++) {
                const int n = n0 + prow[i];
                roff[i] = i == 6 && soff[i] == ~0u ? kOOB : base + (uint32_t)(n < a.N ? n : a.N - 1) * a.row_bytes + poff[i];
            }
            const int nd = n0 + col;
            doff = base + (uint32_t)(nd < a.N ? nd : a.N - 1) * a.row_bytes + 208u;
            if (++fb == NB) {
                fb = 0;
                ucur_next(fc);
            }
            fq++;
        } else {
#pragma unroll
            for (int i = 0; i < 7; i++) roff[i] = kOOB;
        }
        // (the matrix choice is uniform: one resource, no per-lane loop)
        return tile_raw_fetch(__builtin_amdgcn_readfirstlane((int)sh) ? rs_s : rs_r, roff, doff);
    };
    const int rho = lane & 31, m_l = rho >> 3, s_l = (rho >> 2) & 1, d_l = rho & 3;

    TileRaw ra = fetch();
    TileRaw rb = fetch();
    int buf = 1, mc = 0, r0 = 0, gr0 = 0;
    uint32_t abase = 0;
    int es[kTileMR];
    float acc[kTileMR];
    int tile = 0;
    bool shg = false;
    // unit start: its group, pass and tile; new planes when (group, pass)
    // changes
    // a segment: the units of one (group, pass) in this workgroup's range;
    // its activation planes are built once (set-up loads drain the load
    // queue, so they stay out of the streaming loop)
    auto start_segment = [&]() __attribute__((always_inline)) {
        const int g = __builtin_amdgcn_readfirstlane(cc.g), local = __builtin_amdgcn_readfirstlane(cc.local);
        const int pass = local / ntiles;
        tile = local % ntiles;
        shg = g == a.E;
        const int rows = group_rows(g, gr0);
        r0 = gr0 + kTileMR * pass;
        mc = rows - kTileMR * pass < kTileMR ? rows - kTileMR * pass : kTileMR;
        buf ^= 1;
        uint8_t* pl = planes + buf * PB;
        // wavefront w writes activation row r0 + w
        constexpr int KV = kTileMaxK / 512;
        float4 v[KV][2];
        const float* xr = a.X + (int64_t)(r0 + (w < mc ? w : 0)) * a.ldx;
#pragma unroll
        for (int i = 0; i < KV; i++) {
            const int k0 = 8 * lane + 512 * i;
            const int kc = k0 < a.K ? k0 : 0;
            v[i][0] = *(const float4*)(xr + kc);
            v[i][1] = *(const float4*)(xr + kc + 4);
        }
        if (w < mc) {
            float mx = 0.0f;
#pragma unroll
            for (int i = 0; i < KV; i++) {
                if (8 * lane + 512 * i >= a.K) v[i][0] = v[i][1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i][0].x), fabsf(v[i][0].y)), fmaxf(fabsf(v[i][0].z), fabsf(v[i][0].w))));
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i][1].x), fabsf(v[i][1].y)), fmaxf(fabsf(v[i][1].z), fabsf(v[i][1].w))));
            }
            mx = wave_max(mx);
            int Ex = 0;
            frexpf(mx, &Ex);
            const int e = mx > 0.0f ? 30 - Ex : 0;
            auto fx = [&](float x) __attribute__((always_inline)) {
                return (uint32_t)(int)__builtin_rintf(ldexpf(x, e)) + 0x80808080u;
            };
#pragma unroll
            for (int i = 0; i < KV; i++) {
                const int k0 = 8 * lane + 512 * i;
                if (k0 >= a.K) continue;
                uint32_t p[2][4];
#pragma unroll
                for (int qq = 0; qq < 2; qq++) {
                    const uint32_t x0 = fx(v[i][qq].x), x1 = fx(v[i][qq].y), x2 = fx(v[i][qq].z), x3 = fx(v[i][qq].w);
                    const uint32_t lo01 = __builtin_amdgcn_perm(x1, x0, 0x05010400u), hi01 = __builtin_amdgcn_perm(x1, x0, 0x07030602u);
                    const uint32_t lo23 = __builtin_amdgcn_perm(x3, x2, 0x05010400u), hi23 = __builtin_amdgcn_perm(x3, x2, 0x07030602u);
                    p[qq][0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u) ^ 0x80808080u;
                    p[qq][1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u) ^ 0x80808080u;
                    p[qq][2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u) ^ 0x80808080u;
                    p[qq][3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u) ^ 0x80808080u;
                }
                const int j = k0 >> 5, hh = (k0 >> 4) & 1;
#pragma unroll
                for (int d = 0; d < 4; d++)
                    *(uint2*)(pl + (((w * 4 + d) * NJ + j) * 2 + hh) * 16 + (k0 & 8)) = make_uint2(p[0][d], p[1][d]);
            }
            if (lane == 0) lexp[buf * kTileMR + w] = e;
        }
        // (the other buffer was last read before the previous set-up's
        // barrier: one barrier per set-up)
        __syncthreads();
        const bool act = s_l == h && m_l < mc;
        abase = act ? (uint32_t)(buf * PB + (((m_l * 4 + d_l) * NJ) * 2 + h) * 16)
                    : (uint32_t)(2 * PB + h * 16);
#pragma unroll
        for (int m = 0; m < kTileMR; m++) es[m] = lexp[buf * kTileMR + m];
    };
    auto block = [&](const TileQ6& r, int b) __attribute__((always_inline)) {
        const float dd = h2f(r.d & 0xFFFFu);
        int I[kTileMR][4];
#pragma unroll
        for (int m = 0; m < kTileMR; m++)
#pragma unroll
            for (int d = 0; d < 4; d++) I[m][d] = 0;
#pragma unroll
        for (int nh = 0; nh < 2; nh++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int j = 8 * b + 4 * nh + t;
                const v4i A = *(const v4i*)(planes + abase + (uint32_t)j * 32u);
                const v4i B = tile_q6_codes(r, nh, t);
                typedef int v16i __attribute__((ext_vector_type(16)));
                const v16i Z = {};
                const v16i C = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, Z, 0, 0, 0);
                const int sc = tile_q6_scale(r, nh, t, h);
#pragma unroll
                for (int m = 0; m < kTileMR; m++)
                    if (m < mc) {  // (uniform)
#pragma unroll
                        for (int d = 0; d < 4; d++) I[m][d] += __mul24(sc, C[4 * m + d]);
                    }
                // one K-step's results live at a time (other wavefronts
                // cover the MFMA latency): the sums are formed here
#pragma unroll
                for (int m = 0; m < kTileMR; m++)
                    asm volatile("" : "+v"(I[m][0]), "+v"(I[m][1]), "+v"(I[m][2]), "+v"(I[m][3]));
            }
#pragma unroll
        for (int m = 0; m < kTileMR; m++) {
            const float P = fmaf(fmaf(fmaf((float)I[m][3], 256.0f, (float)I[m][2]), 256.0f, (float)I[m][1]), 256.0f,
                                 (float)I[m][0]);
            acc[m] = fmaf(dd, P, acc[m]);
        }
    };
    auto finish = [&]() __attribute__((always_inline)) {
        // the two halves' scale groups, then the row's 2^-e
        const int n = tile * kTileRows + w * 32 + col;
#pragma unroll
        for (int m = 0; m < kTileMR; m++) {
            const float v = acc[m] + __shfl_xor(acc[m], 32, 64);
            if (m < mc && h == 0 && n < a.N) {
                const int r = r0 + m;
                float* y = shg ? a.Ysh + (int64_t)(r - gr0) * a.ldy : a.Y + (int64_t)r * a.ldy;
                y[n] = ldexpf(v, -es[m]);
            }
        }
    };
    int q = 0;
#define GGQ_TILE_STEP(R)                                                           \
    {                                                                              \
        const int b = q % NB;                                                      \
        if (b == 0) {                                                              \
            _Pragma("unroll") for (int m = 0; m < kTileMR; m++) acc[m] = 0.0f;     \
        }                                                                          \
        block(tile_q6_stage(R, stage, soff, col, h), b);                           \
        R = fetch();                                                               \
        if (b == NB - 1) {                                                         \
            finish();                                                              \
            tile++;                                                                \
            ucur_next(cc);                                                         \
        }                                                                          \
        if (++q >= seg_end) break;                                                 \
    }
    while (q < n_pos) {
        start_segment();
        // units left in this pass of the group, within the range
        const int seg_units = min(ntiles - tile, u1 - u0 - q / NB);
        const int seg_end = q + seg_units * NB;
        // position q is in ra when q is even, in rb when odd
        if (q & 1) {
            do GGQ_TILE_STEP(rb) while (false);
            if (q >= seg_end) continue;
        }
        while (true) {
            GGQ_TILE_STEP(ra)
            GGQ_TILE_STEP(rb)
        }
    }
#undef GGQ_TILE_STEP
}

// ------------------------------------------- row tiles, given int8 codes
// The same units (group, pass, 128-row tile) for per-row int8 activation
// codes (the XDNA semantics: codes and a scale per row, as the quantizer
// wrote them): one digit per row, A row m holding the codes of row m of the
// pass (MR of 8, 16, 24 or 32 rows), so that a K-step is one scale group for
// both lane halves and output register i of lane (c, h) is the complete
// dot product of row 8 (i / 4) + 4 h + i % 4 with weight row c (MR of 8:
// registers 0..3).  Q6_K:
// signed codes (q - 32), K-steps of 16 (v_mfma_i32_32x32x16_i8: a scale
// group), I += sc * C, acc += d * I per block.  Q4_K: unsigned nibbles,
// K-steps of 32 (v_mfma_i32_32x32x32_i8: a sub-block); the min term takes
// I += sc * C per K-step (exact integer I: |C| <= 32 * 128 * 15, sc <= 63,
// 8 K-steps), acc += d * I per block, less the min term: for more than 16
// rows a pass a product over sub-blocks on v_mfma_f32_32x32x2_f32 (A: the
// row's code sums per sub-block, from the quantizer, staged in LDS; B:
// dmin * m of the weight row; accumulated over the unit); for 16 rows
// (whose LDS must leave room for 3 workgroups per CU) the code sums from a
// second MFMA against ones, Mn += m * S, acc -= dmin * Mn per block.  Paired matrices (gate / up):
// rows [0, n1) of a group from W, [n1, N) from W2.
// F16 (Q6_K only): fp32 rows as fp16 hi + lo planes with a power-of-two row
// scale (the fp16 GEMM's split), the codes q - 32 exact in fp16, one
// v_mfma_f32_32x32x16_f16 per plane and 16-value group (products summed in
// fp32 by the matrix core), acc += d * sc * C.
constexpr int kCodeMaxK = 2048;
constexpr int kCodeF16MaxK = 1024;
// LDS bytes of one workgroup: unit prefix, code planes (rows padded by 16
// bytes, so that the rows of a K-step fall in distinct banks), row scales,
// scan totals, staging
// (fp16 rows: hi and lo planes of 2 bytes a value)
__host__ __device__ constexpr int code_lds_bytes(int G, int MR, int K, int stage_row, bool sums, bool f16 = false) {
    return (((G + 1) * 4 + 15) & ~15) + (f16 ? 2 * MR * (2 * K + 16) : MR * (K + 16)) +
           (sums ? MR * (K / 32) * 4 : 0) + 4 * MR + 16 + 4 * 32 * stage_row;
}
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
// Four 6-bit Q6_K values u (bytes of w, 0..63) as the fp16 codes u - 32,
// exactly: the half 0x6400 | u is 1024 + u.
__device__ __forceinline__ uint2 q6u_f16x4(uint32_t w) {
    const h2v off = {(_Float16)1056.0f, (_Float16)1056.0f};
    const h2v a = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u)) - off;
    const h2v b = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u)) - off;
    return make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
}

template <int T> struct CodeFmt;
template <> struct CodeFmt<T_Q6_K> {
    static constexpr int BB = 210, PIECES = 13, LOADS = 7, STAGE_ROW = 240;
};
template <> struct CodeFmt<T_Q4_K> {
    static constexpr int BB = 144, PIECES = 9, LOADS = 5, STAGE_ROW = 144;
};

// (3 wavefronts per SIMD for 16 rows a pass, 2 above: the accumulators)
template <int T, int MR, bool F16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MR > 16 ? 2 : 3))) void i8_tile_codes_kernel(
    MoeGemm a) {
    typedef CodeFmt<T> CF;
    static_assert(!F16 || T == T_Q6_K, "fp16 rows: Q6_K");
    static_assert(MR % 8 == 0 && MR <= 32, "rows per pass");
    constexpr int NA = MR / 2;  // output registers per lane
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 31, h = lane >> 5;
    const int NB = a.K >> 8, NJ = a.K >> 5;
    const int G = a.E + (a.Wsh ? 1 : 0);
    const int ntiles = (a.N + kTileRows - 1) / kTileRows;
    const uint32_t row_bytes = (uint32_t)(NB * CF::BB);
    // LDS: unit prefix [G + 1] (16-byte padded), code planes [m][j][half]
    // (16 B entries), row scales [16], wavefront totals of the scan,
    // staging (32 rows of one block per wavefront)
    const int pre_bytes = ((G + 1) * 4 + 15) & ~15;
    const int PS = F16 ? 2 * a.K + 16 : a.K + 16;  // plane row stride (bytes)
    int* pre = (int*)lds;
    uint8_t* planes = lds + pre_bytes;
    // Q4_K: code sums [m][block][h][s] of sub-block 2 s + h (one 16-byte read
    // per lane and block)
    float* sums = (float*)(planes + (F16 ? 2 : 1) * MR * PS);
    constexpr bool kSumsLds = T == T_Q4_K && MR > 16;
    float* lsc = sums + (kSumsLds ? MR * NJ : 0);
    int* wsum = (int*)(lsc + MR);
    uint8_t* stage = (uint8_t*)(wsum + 4) + w * 32 * CF::STAGE_ROW;
    // units per group, exclusive prefix over the workgroup (4 groups per
    // thread, G <= 1023)
    {
        int cnt[4], tsum = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int g = 4 * tid + i;
            const int rows = g < G ? a.grp[g + 1] - a.grp[g] : 0;
            cnt[i] = (rows + MR - 1) / MR * ntiles;
            tsum += cnt[i];
        }
        int x = tsum;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y = __shfl_up(x, o, 64);
            if (lane >= o) x += y;
        }
        if (lane == 63) wsum[w] = x;
        __syncthreads();
        int ex = x - tsum;
        for (int k = 0; k < w; k++) ex += wsum[k];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int g = 4 * tid + i;
            if (g <= G) pre[g] = ex;
            ex += cnt[i];
        }
        __syncthreads();
    }
    auto upre = [&](int g) __attribute__((always_inline)) { return __builtin_amdgcn_readfirstlane(pre[g]); };
    const int U = upre(G);
    const int u0 = (int)((int64_t)U * blockIdx.x / gridDim.x), u1 = (int)((int64_t)U * (blockIdx.x + 1) / gridDim.x);
    if (u0 >= u1) return;
    int glo = 0, ghi = G - 1;
    while (glo < ghi) {
        const int mid = (glo + ghi + 1) >> 1;
        if (upre(mid) <= u0) glo = mid;
        else ghi = mid - 1;
    }
    struct UCur { int g, local, end; };
    auto ucur_next = [&](UCur& c) __attribute__((always_inline)) {
        if (++c.local >= c.end) {
            do {
                ++c.g;
            } while (c.g < G && upre(c.g + 1) == upre(c.g));
            c.local = 0;
            c.end = c.g < G ? upre(c.g + 1) - upre(c.g) : 0;
        }
    };
    UCur fc{glo, u0 - upre(glo), upre(glo + 1) - upre(glo)};
    UCur cc = fc;
    const int n_pos = (u1 - u0) * NB;
    int fq = 0, fb = 0;
    // the four matrices (routed / shared x first / second of the pair)
    const int Er = a.E;
    const Rsrc rs0 = make_rsrc((const uint8_t*)a.W, (uint32_t)Er * (uint32_t)a.w_stride);
    const Rsrc rs1 = make_rsrc((const uint8_t*)(a.W2 ? a.W2 : a.W), (uint32_t)Er * (uint32_t)a.w_stride);
    const Rsrc rs2 = make_rsrc((const uint8_t*)(a.Wsh ? a.Wsh : a.W), (uint32_t)a.n1 * row_bytes);
    const Rsrc rs3 = make_rsrc((const uint8_t*)(a.W2sh ? a.W2sh : a.W), (uint32_t)(a.N - a.n1) * row_bytes);
    // this lane's pieces of a block: chunk c = lane + 64 i is piece c % P of
    // row c / P of the wavefront's 32
    uint32_t soff[CF::LOADS], poff[CF::LOADS];
    int prow[CF::LOADS];
#pragma unroll
    for (int i = 0; i < CF::LOADS; i++) {
        const int c = lane + 64 * i;
        const bool ok = c < 32 * CF::PIECES;
        prow[i] = ok ? c / CF::PIECES : 0;
        poff[i] = 16u * (uint32_t)(c % CF::PIECES);
        soff[i] = ok ? (uint32_t)(prow[i] * CF::STAGE_ROW) + poff[i] : ~0u;
    }
    struct Raw { v4u c[CF::LOADS]; uint32_t d; };
    auto fetch = [&]() __attribute__((always_inline)) {
        uint32_t roff[CF::LOADS], doff = kOOB;
        int which = 0;
        if (fq < n_pos) {
            const int n0 = (fc.local % ntiles) * kTileRows + w * 32;
            const bool second = n0 >= a.n1;
            which = (fc.g == Er ? 2 : 0) + (second ? 1 : 0);
            const int nr = second ? n0 - a.n1 : n0;
            const int nmax = (second ? a.N - a.n1 : a.n1) - 1;
            const uint32_t base = (fc.g == Er ? 0u : (uint32_t)fc.g * (uint32_t)a.w_stride) + (uint32_t)fb * CF::BB;
#pragma unroll
            for (int i = 0; i < CF::LOADS; i++) {
                const int n = nr + prow[i];
                roff[i] = soff[i] == ~0u ? kOOB : base + (uint32_t)(n < nmax ? n : nmax) * row_bytes + poff[i];
            }
            if (T == T_Q6_K) {
                const int n = nr + col;
                doff = base + (uint32_t)(n < nmax ? n : nmax) * row_bytes + 208u;
            }
            if (++fb == NB) {
                fb = 0;
                ucur_next(fc);
            }
            fq++;
        } else {
#pragma unroll
            for (int i = 0; i < CF::LOADS; i++) roff[i] = kOOB;
        }
        which = __builtin_amdgcn_readfirstlane(which);
        const Rsrc rs = which == 0 ? rs0 : which == 1 ? rs1 : which == 2 ? rs2 : rs3;
        Raw r;
        r.d = T == T_Q6_K ? bl2(rs, doff) : 0u;
#pragma unroll
        for (int i = 0; i < CF::LOADS; i++) r.c[i] = bl16(rs, roff[i]);
        return r;
    };
    const int m_l = lane & 31;  // activation row of this lane's A entries
    auto arow = [&](int i) __attribute__((always_inline)) { return 8 * (i >> 2) + 4 * h + (i & 3); };
    // blocks in flight: 2, or (2 wavefronts per SIMD leave the registers)
    // 3 / 4 for more than 16 rows a pass
    constexpr int NR = MR > 16 ? (T == T_Q4_K ? 4 : 3) : 2;
    Raw ra = fetch();
    Raw rb = fetch();
    Raw rc, rd;
    if constexpr (NR > 2) rc = fetch();
    if constexpr (NR > 3) rd = fetch();
    int mc = 0, r0 = 0, tile = 0;
    bool act = false;
    uint32_t abase = 0;
    float acc[NA];
    typedef float v4f __attribute__((ext_vector_type(4)));
    typedef float v16f __attribute__((ext_vector_type(16)));
    v16f Mf = {};  // Q4_K min term for more than 16 rows a pass
    uint32_t abase_s = 0;
    auto start_segment = [&]() __attribute__((always_inline)) {
        const int g = __builtin_amdgcn_readfirstlane(cc.g), local = __builtin_amdgcn_readfirstlane(cc.local);
        const int pass = local / ntiles;
        tile = local % ntiles;
        const int gr0 = a.grp[g];
        const int rows = a.grp[g + 1] - gr0;
        r0 = gr0 + MR * pass;
        mc = rows - MR * pass < MR ? rows - MR * pass : MR;
        __syncthreads();  // the previous segment's planes are read
        // codes of the pass's rows: 16-byte chunks, entry (m, j, half)
        if constexpr (F16) {
            // hi and lo planes: 8 values a 16-byte chunk
            const int per_row = a.K >> 3;
            for (int i = tid; i < mc * per_row; i += 256) {
                const int m = i / per_row, k0 = 8 * (i - m * per_row);
                const int r = r0 + m;
                const int64_t src = (int64_t)(a.x_idx ? a.x_idx[r] : r) * a.K + k0;
                *(uint4*)(planes + m * PS + 2 * k0) = *(const uint4*)((const _Float16*)a.XH + src);
                *(uint4*)(planes + (MR + m) * PS + 2 * k0) = *(const uint4*)((const _Float16*)a.XL + src);
            }
            if (tid < MR) {
                const int r = r0 + (tid < mc ? tid : 0);
                lsc[tid] = a.xs[a.x_idx ? a.x_idx[r] : r];
            }
        } else {
            const int per_row = a.K >> 4;
            for (int i = tid; i < mc * per_row; i += 256) {
                const int m = i / per_row, k0 = 16 * (i - m * per_row);
                const int r = r0 + m;
                const int ar = a.x_idx ? a.x_idx[r] : r;
                const uint4 v = *(const uint4*)(a.QA + (int64_t)ar * a.K + k0);
                *(uint4*)(planes + m * PS + k0) = v;
            }
            if (tid < MR) {
                const int r = r0 + (tid < mc ? tid : 0);
                lsc[tid] = a.sa[a.x_idx ? a.x_idx[r] : r];
            }
        }
        if constexpr (kSumsLds) {
            for (int i = tid; i < mc * NJ; i += 256) {
                const int m = i / NJ, j = i - m * NJ, t = j & 7;
                const int r = r0 + m;
                const int ar = a.x_idx ? a.x_idx[r] : r;
                sums[m * NJ + (j & ~7) + 4 * (t & 1) + (t >> 1)] = a.QS[(int64_t)ar * NJ + j];
            }
        }
        __syncthreads();
        act = m_l < mc;
        // lane half h: bytes 8 h.. of a 16-value K-step (Q6_K), 16 h.. of a 32-value one (Q4_K)
        abase = (uint32_t)(m_l * PS + (T == T_Q6_K && !F16 ? 8 : 16) * h);
        abase_s = (uint32_t)(m_l * NJ + 4 * h);
    };
    // One block: K-steps on the staged rows.
    auto block = [&](const Raw& raw, int b) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < CF::LOADS; i++)
            if (i < CF::LOADS - 1 || soff[i] != ~0u) *(v4u*)(stage + soff[i]) = raw.c[i];
        const uint8_t* row = stage + col * CF::STAGE_ROW;
        typedef int v16i __attribute__((ext_vector_type(16)));
        const v16i Z = {};
        int I[NA];
#pragma unroll
        for (int m = 0; m < NA; m++) I[m] = 0;
        if constexpr (F16) {
            // lane half h: values 8 h .. 8 h + 7 of each 16-value group (u in
            // 0..63: low 4 bits from ql, the top two from qh)
            TileQ6 q;
            auto ld2 = [&](const uint8_t* p) __attribute__((always_inline)) {
                const uint2 u0 = *(const uint2*)p, u1 = *(const uint2*)(p + 16);
                return v4u{u0.x, u0.y, u1.x, u1.y};
            };
#pragma unroll
            for (int nh = 0; nh < 2; nh++) {
                q.ql0[nh] = ld2(row + 64 * nh + 8 * h);
                q.ql1[nh] = ld2(row + 64 * nh + 32 + 8 * h);
                q.qh[nh] = ld2(row + 128 + 32 * nh + 8 * h);
            }
            q.sc = *(const v4u*)(row + 192);
            const float dd = h2f(raw.d & 0xFFFFu);
            typedef float v16f_ __attribute__((ext_vector_type(16)));
            const v16f_ Zf = {};
            const v8h Z8 = {};
#pragma unroll
            for (int nh = 0; nh < 2; nh++)
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int g = 0; g < 2; g++) {
                        const int j = 8 * b + 4 * nh + t;
                        const uint32_t ko = (uint32_t)(2 * (32 * j + 16 * g));
                        v8h Ah = *(const v8h*)(planes + abase + ko);
                        v8h Al = *(const v8h*)(planes + MR * PS + abase + ko);
                        if (!act) { Ah = Z8; Al = Z8; }
                        const v4u ql = (t & 1) ? q.ql1[nh] : q.ql0[nh];
                        const v4u qh = q.qh[nh];
                        auto u6 = [&](uint32_t l, uint32_t hb) __attribute__((always_inline)) {
                            const uint32_t lo = (t >> 1) ? (l >> 4) & 0x0F0F0F0Fu : l & 0x0F0F0F0Fu;
                            return lo | (((hb >> (2 * t)) & 0x03030303u) << 4);
                        };
                        const uint2 b0 = q6u_f16x4(u6(g ? ql.z : ql.x, g ? qh.z : qh.x));
                        const uint2 b1 = q6u_f16x4(u6(g ? ql.w : ql.y, g ? qh.w : qh.y));
                        const v8h B = __builtin_bit_cast(v8h, make_uint4(b0.x, b0.y, b1.x, b1.y));
                        v16f_ C = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ah, B, Zf, 0, 0, 0);
                        C = __builtin_amdgcn_mfma_f32_32x32x16_f16(Al, B, C, 0, 0, 0);
                        const float ds = dd * (float)tile_q6_scale(q, nh, t, g);
#pragma unroll
                        for (int m = 0; m < NA; m++) acc[m] = fmaf(ds, C[m], acc[m]);
#pragma unroll
                        for (int m = 0; m < NA; m += 4)
                            asm volatile("" : "+v"(acc[m]), "+v"(acc[m + 1]), "+v"(acc[m + 2]), "+v"(acc[m + 3]));
                    }
        } else if constexpr (T == T_Q6_K) {
            // lane half h: codes 8 h .. 8 h + 7 of each 16-value group, the
            // two groups of a 32-value step in (x, y) and (z, w)
            TileQ6 q;
            auto ld2 = [&](const uint8_t* p) __attribute__((always_inline)) {
                const uint2 u0 = *(const uint2*)p, u1 = *(const uint2*)(p + 16);
                return v4u{u0.x, u0.y, u1.x, u1.y};
            };
#pragma unroll
            for (int nh = 0; nh < 2; nh++) {
                q.ql0[nh] = ld2(row + 64 * nh + 8 * h);
                q.ql1[nh] = ld2(row + 64 * nh + 32 + 8 * h);
                q.qh[nh] = ld2(row + 128 + 32 * nh + 8 * h);
            }
            q.sc = *(const v4u*)(row + 192);
            const float dd = h2f(raw.d & 0xFFFFu);
#pragma unroll
            for (int nh = 0; nh < 2; nh++)
#pragma unroll
                for (int t = 0; t < 4; t++)
#pragma unroll
                    for (int g = 0; g < 2; g++) {
                        const int j = 8 * b + 4 * nh + t;
                        long A = *(const long*)(planes + abase + (uint32_t)(32 * j + 16 * g));
                        if (!act) A = 0;
                        const v4u ql = (t & 1) ? q.ql1[nh] : q.ql0[nh];
                        const v4u qh = q.qh[nh];
                        const uint32_t c0 = q6_signed(g ? ql.z : ql.x, g ? qh.z : qh.x, t);
                        const uint32_t c1 = q6_signed(g ? ql.w : ql.y, g ? qh.w : qh.y, t);
                        const long B = (long)(((uint64_t)c1 << 32) | c0);
                        const v16i C = __builtin_amdgcn_mfma_i32_32x32x16_i8(A, B, Z, 0, 0, 0);
                        const int sc = tile_q6_scale(q, nh, t, g);
                        // (rows past mc meet zero A entries: no branches)
#pragma unroll
                        for (int m = 0; m < NA; m++) I[m] += __mul24(sc, C[m]);
#pragma unroll
                        for (int m = 0; m < NA; m += 4)
                            asm volatile("" : "+v"(I[m]), "+v"(I[m + 1]), "+v"(I[m + 2]), "+v"(I[m + 3]));
                    }
#pragma unroll
            for (int m = 0; m < NA; m++) acc[m] = fmaf(dd, (float)I[m], acc[m]);
        } else {
            const v4u hd = *(const v4u*)row;
            v4u qs[4];
#pragma unroll
            for (int c = 0; c < 4; c++) qs[c] = *(const v4u*)(row + 16 + 32 * c + 16 * h);
            const float d = h2f(hd.x & 0xFFFFu), dmin = h2f(hd.x >> 16);
            int Mn[NA];
#pragma unroll
            for (int m = 0; m < NA; m++) Mn[m] = 0;
            // min term: sub-blocks 2 s + h of this lane half
            if constexpr (kSumsLds) {
                v4f Sa = *(const v4f*)(sums + abase_s + 8 * b);
                if (!act) Sa = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int s4 = 0; s4 < 4; s4++) {
                    const uint32_t sm = kq_pair(hd.y, hd.z, hd.w, s4);
                    const float bm = dmin * (float)((sm >> (16 + 8 * h)) & 0xFFu);
                    Mf = __builtin_amdgcn_mfma_f32_32x32x2f32(Sa[s4], bm, Mf, 0, 0, 0);
                }
            }
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const int j = 8 * b + t;
                v4i A = *(const v4i*)(planes + abase + (uint32_t)j * 32u);
                if (!act) A = v4i{0, 0, 0, 0};
                const v4u w4 = qs[t >> 1];
                v4i B;
                if (t & 1) {
                    B.x = (int)((w4.x >> 4) & 0x0F0F0F0Fu); B.y = (int)((w4.y >> 4) & 0x0F0F0F0Fu);
                    B.z = (int)((w4.z >> 4) & 0x0F0F0F0Fu); B.w = (int)((w4.w >> 4) & 0x0F0F0F0Fu);
                } else {
                    B.x = (int)(w4.x & 0x0F0F0F0Fu); B.y = (int)(w4.y & 0x0F0F0F0Fu);
                    B.z = (int)(w4.z & 0x0F0F0F0Fu); B.w = (int)(w4.w & 0x0F0F0F0Fu);
                }
                const v16i C = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, Z, 0, 0, 0);
                // scale / min of sub-block t (kquant.h:56-64): bytes t % 2 of pair t / 2
                const uint32_t sm = kq_pair(hd.y, hd.z, hd.w, t >> 1);
                const int sc = (int)((sm >> (8 * (t & 1))) & 0xFFu);
#pragma unroll
                for (int m = 0; m < NA; m++) I[m] += __mul24(sc, C[m]);
                if constexpr (!kSumsLds) {
                    const v4i ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
                    const v16i S = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, ones, Z, 0, 0, 0);
                    const int mn = (int)((sm >> (16 + 8 * (t & 1))) & 0xFFu);
#pragma unroll
                    for (int m = 0; m < NA; m++) Mn[m] += __mul24(mn, S[m]);
#pragma unroll
                    for (int m = 0; m < NA; m += 4)
                        asm volatile("" : "+v"(Mn[m]), "+v"(Mn[m + 1]), "+v"(Mn[m + 2]), "+v"(Mn[m + 3]));
                }
#pragma unroll
                for (int m = 0; m < NA; m += 4)
                    asm volatile("" : "+v"(I[m]), "+v"(I[m + 1]), "+v"(I[m + 2]), "+v"(I[m + 3]));
            }
#pragma unroll
            for (int m = 0; m < NA; m++) acc[m] = fmaf(d, (float)I[m], kSumsLds ? acc[m] : fmaf(-dmin, (float)Mn[m], acc[m]));
        }
    };
    auto finish = [&]() __attribute__((always_inline)) {
        // the row's scale
        const int n = tile * kTileRows + w * 32 + col;
        const bool second = n - col >= a.n1;  // (uniform: the wavefront's rows are in one matrix)
        float* Y = second ? a.C2 : a.C;
        const int nn = second ? n - a.n1 : n;
#pragma unroll
        for (int i = 0; i < NA; i++) {
            const int m = arow(i);
            const float v = kSumsLds ? acc[i] - Mf[i] : acc[i];
            if (m < mc && n < a.N) Y[(int64_t)(r0 + m) * a.ldc + nn] = v * lsc[m];
        }
    };
    int q = 0;
#define GGQ_CODE_STEP(R)                                                           \
    {                                                                              \
        const int b = q % NB;                                                      \
        if (b == 0) {                                                              \
            _Pragma("unroll") for (int m = 0; m < NA; m++) acc[m] = 0.0f;     \
            if (kSumsLds) Mf = v16f{};                                             \
        }                                                                          \
        block(R, b);                                                               \
        R = fetch();                                                               \
        if (b == NB - 1) {                                                         \
            finish();                                                              \
            tile++;                                                                \
            ucur_next(cc);                                                         \
        }                                                                          \
        if (++q >= seg_end) break;                                                 \
    }
    while (q < n_pos) {
        start_segment();
        const int seg_units = min(ntiles - tile, u1 - u0 - q / NB);
        const int seg_end = q + seg_units * NB;
        // position q is in register set q % NR
        const int ph = q % NR;
        if (ph != 0) {
            do {
                if (ph <= 1) GGQ_CODE_STEP(rb)
                if (NR > 2 && ph <= 2) GGQ_CODE_STEP(rc)
                if (NR > 3) GGQ_CODE_STEP(rd)
            } while (false);
            if (q >= seg_end) continue;
        }
        while (true) {
            GGQ_CODE_STEP(ra)
            GGQ_CODE_STEP(rb)
            if constexpr (NR > 2) GGQ_CODE_STEP(rc)
            if constexpr (NR > 3) GGQ_CODE_STEP(rd)
        }
    }
#undef GGQ_CODE_STEP
}

}  // namespace

bool i8_tile_grouped_eligible(uint32_t type, int N, int K, int E, int64_t w_stride, bool shared) {
    if (type != T_Q6_K || K % 256 != 0 || K <= 0 || K > kTileMaxK || N <= 0 || E < 1 || E + (shared ? 1 : 0) > 1023)
        return false;
    // one buffer resource over the routed matrices: offsets below kOOB
    return w_stride >= (int64_t)N * row_bytes(type, K) && (int64_t)E * w_stride < (int64_t)kOOB;
}

hipError_t launch_i8_tile_grouped(uint32_t type, const void* W, int64_t w_stride, const void* Wsh, const float* X,
                                  int ldx, const int32_t* grp_off, int E, int t_sh, float* Y, float* Ysh, int ldy,
                                  int N, int K, hipStream_t s) {
    const int groups = E + (Wsh && t_sh > 0 ? 1 : 0);
    if (!i8_tile_grouped_eligible(type, N, K, E, w_stride, Wsh && t_sh > 0) || ldx % 4 != 0 || ((uintptr_t)X & 15u) != 0)
        return hipErrorInvalidValue;
    I8TileArgs a{(const uint8_t*)W, w_stride, (const uint8_t*)Wsh, X, ldx, grp_off, Wsh && t_sh > 0 ? E : -1, t_sh,
                 Y, Ysh, ldy, N, K, (uint32_t)row_bytes(type, K), groups};
    const int lds = kTilePre + 2 * kTileMR * 4 * K + K + 64 + 4 * kTileStage;
    // resident grid: 3 workgroups per CU (the kernel's register budget),
    // fewer when their LDS does not fit (160 KB per CU)
    int per_cu = (160 * 1024) / lds;
    per_cu = per_cu > 3 ? 3 : per_cu < 1 ? 1 : per_cu;
    const dim3 grid((unsigned)(per_cu * cu_count()));
    static const hipError_t attr = hipFuncSetAttribute((const void*)i8_tile_grouped_kernel,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024);
    if (attr != hipSuccess) return attr;
    i8_tile_grouped_kernel<<<grid, 256, lds, s>>>(a);
    return hipGetLastError();
}

bool i8_tile_codes_eligible(uint32_t type, const MoeGemm& g) {
    if (type != T_Q6_K && type != T_Q4_K) return false;
    if (g.XH) {  // fp16 rows: Q6_K, hi / lo planes and row scales
        if (type != T_Q6_K || !g.XL || !g.xs || g.K > kCodeF16MaxK || g.W2) return false;
    } else if (!g.QA || !g.sa || (type == T_Q4_K && !g.QS)) {  // (the min term's code sums)
        return false;
    }
    const int G = g.E + (g.Wsh ? 1 : 0);
    if (g.K % 256 != 0 || g.K <= 0 || g.K > kCodeMaxK || g.N <= 0 || g.E < 1 || G > 1023) return false;
    if (g.W2 ? (g.n1 % 32 != 0 || g.n1 <= 0 || g.n1 >= g.N || !g.C2) : g.n1 != g.N) return false;
    if (g.Wsh && g.W2 && !g.W2sh) return false;
    const int64_t rb = row_bytes(type, g.K);
    return g.w_stride >= (int64_t)g.n1 * rb && (int64_t)g.E * g.w_stride < (int64_t)kOOB;
}

namespace {
template <int T, int MR, bool F16> hipError_t launch_codes_mr(const MoeGemm& g, int G, hipStream_t s) {
    const int lds = code_lds_bytes(G, MR, g.K, CodeFmt<T>::STAGE_ROW, T == T_Q4_K && MR > 16, F16);
    // resident grid: up to 3 workgroups per CU for 16 rows a pass, 2 above
    // (the kernel's register budget), as many as fit in its 160 KB of LDS
    const int max_cu = MR > 16 ? 2 : 3;
    int per_cu = (160 * 1024) / lds;
    per_cu = per_cu > max_cu ? max_cu : per_cu < 1 ? 1 : per_cu;
    static const hipError_t attr = hipFuncSetAttribute((const void*)i8_tile_codes_kernel<T, MR, F16>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (attr != hipSuccess) return attr;
    i8_tile_codes_kernel<T, MR, F16><<<dim3((unsigned)(per_cu * cu_count())), 256, lds, s>>>(g);
    return hipGetLastError();
}
template <int T, bool F16> hipError_t launch_codes(const MoeGemm& g, int G, int rows_per_group, hipStream_t s) {
    // 8 rows per pass for up to 4 rows a group on average (half the
    // products of 16-row passes), 16 up to 12; otherwise the most rows that
    // leave two workgroups per CU
    const bool sums = T == T_Q4_K;
    if (rows_per_group <= 4) return launch_codes_mr<T, 8, F16>(g, G, s);
    if (rows_per_group <= 12) return launch_codes_mr<T, 16, F16>(g, G, s);
    if (2 * code_lds_bytes(G, 32, g.K, CodeFmt<T>::STAGE_ROW, sums, F16) <= 160 * 1024)
        return launch_codes_mr<T, 32, F16>(g, G, s);
    if (2 * code_lds_bytes(G, 24, g.K, CodeFmt<T>::STAGE_ROW, sums, F16) <= 160 * 1024)
        return launch_codes_mr<T, 24, F16>(g, G, s);
    return launch_codes_mr<T, 16, F16>(g, G, s);
}
}  // namespace

hipError_t launch_i8_tile_codes(uint32_t type, const MoeGemm& g, int rows_per_group, hipStream_t s) {
    if (!i8_tile_codes_eligible(type, g)) return hipErrorInvalidValue;
    const int G = g.E + (g.Wsh ? 1 : 0);
    if (g.XH) return launch_codes<T_Q6_K, true>(g, G, rows_per_group, s);
    return type == T_Q6_K ? launch_codes<T_Q6_K, false>(g, G, rows_per_group, s)
                          : launch_codes<T_Q4_K, false>(g, G, rows_per_group, s);
}

}  // namespace ggq
