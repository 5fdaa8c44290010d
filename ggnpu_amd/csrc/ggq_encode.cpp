// ggq_encode.cpp -- float -> GGUF block encoders for seeded synthetic weights.
//
// ggnpu ships decoders only (include/ggnpu/quant/kquant.h, src/quant/*.cpp)
// and no quantizer, so the synthetic tensors of the benchmark configurations
// are produced here.  The encoders are simple round-to-nearest schemes (not
// llama.cpp's search-based ones); what matters for parity is only that the
// bytes are valid blocks: every decoder downstream (GPU kernels and oracle)
// consumes the same bytes.  The encoded layouts are the inverse of the
// reference decoders:
//   Q4_K/Q5_K  kquant.h:9-13, 56-64, 133-179   Q6_K  kquant.h:15-20, 182-202
//   Q8_0       q8_0.cpp:19-25                   IQ4_NL iq4_nl.cpp:16-31
//   IQ4_XS     iq4_xs.cpp:21-38
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/ggq.h"
#include "ggq_formats.h"

namespace {

// float -> IEEE half, round to nearest even (finite inputs of fp16 range).
uint16_t f2h(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const float a = std::fabs(f);
    if (!(a < 65520.0f)) return (uint16_t)(sign | 0x7C00u);
    if (a < 0x1p-14f) {  // subnormal half: multiple of 2^-24, rint is half-even
        return (uint16_t)(sign | (uint32_t)std::nearbyint(a * 0x1p24f));
    }
    uint32_t ax;
    std::memcpy(&ax, &a, 4);
    uint32_t e = (ax >> 23) - 112;                 // half exponent
    uint32_t m = ax & 0x7FFFFFu;
    uint32_t hm = m >> 13, rem = m & 0x1FFFu;
    uint32_t h = (e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1))) h++;  // carries into exponent correctly
    return (uint16_t)(sign | h);
}

float h2f(uint16_t h) {
    const uint32_t e = (h >> 10) & 31u, f = h & 1023u;
    float v = e == 0 ? (float)f * 0x1p-24f : std::ldexp((float)(f | 1024u), (int)e - 25);
    return (h & 0x8000u) ? -v : v;
}

void put16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xFF);
    p[1] = (uint8_t)(v >> 8);
}

int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

const int8_t kIq4[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

int nearest_iq4(float v) {
    int best = 0;
    float bd = std::fabs(v - kIq4[0]);
    for (int i = 1; i < 16; i++) {
        const float d = std::fabs(v - kIq4[i]);
        if (d < bd) { bd = d; best = i; }
    }
    return best;
}

void enc_q8_0(const float* x, uint8_t* b) {
    float amax = 0;
    for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(x[i]));
    const uint16_t dh = f2h(amax / 127.0f);
    const float d = h2f(dh);
    put16(b, dh);
    for (int i = 0; i < 32; i++) b[2 + i] = (uint8_t)(int8_t)(d > 0 ? clampi((int)std::nearbyint(x[i] / d), -127, 127) : 0);
}

void enc_iq4_nl(const float* x, uint8_t* b) {
    float amax = 0;
    for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(x[i]));
    const uint16_t dh = f2h(amax / 127.0f);
    const float d = h2f(dh);
    put16(b, dh);
    for (int j = 0; j < 16; j++) {
        const int lo = d > 0 ? nearest_iq4(x[j] / d) : 8, hi = d > 0 ? nearest_iq4(x[j + 16] / d) : 8;
        b[2 + j] = (uint8_t)(lo | (hi << 4));
    }
}

void enc_iq4_xs(const float* x, uint8_t* b) {
    float sub[8], dmax = 0;
    for (int ib = 0; ib < 8; ib++) {
        float amax = 0;
        for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(x[32 * ib + i]));
        sub[ib] = amax / 127.0f;
        dmax = std::max(dmax, sub[ib]);
    }
    const uint16_t dh = f2h(dmax / 31.0f);
    const float d = h2f(dh);
    put16(b, dh);
    uint16_t sh = 0;
    std::memset(b + 4, 0, 4);
    for (int ib = 0; ib < 8; ib++) {
        const int ls = d > 0 ? clampi((int)std::nearbyint(sub[ib] / d) + 32, 0, 63) : 32;
        b[4 + ib / 2] |= (uint8_t)((ls & 15) << (4 * (ib & 1)));
        sh |= (uint16_t)((ls >> 4) << (2 * ib));
        const float dl = d * (float)(ls - 32);
        for (int j = 0; j < 16; j++) {
            const int lo = dl != 0 ? nearest_iq4(x[32 * ib + j] / dl) : 8;
            const int hi = dl != 0 ? nearest_iq4(x[32 * ib + 16 + j] / dl) : 8;
            b[8 + 16 * ib + j] = (uint8_t)(lo | (hi << 4));
        }
    }
    put16(b + 2, sh);
}

// Packs 8 (scale, min) 6-bit pairs the way kquant.h:56-64 unpacks them.
void pack_scale_min(const int* sc, const int* mn, uint8_t* s) {
    std::memset(s, 0, 12);
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            s[j] |= (uint8_t)(sc[j] & 63);
            s[j + 4] |= (uint8_t)(mn[j] & 63);
        } else {
            s[j + 4] = (uint8_t)((sc[j] & 15) | ((mn[j] & 15) << 4));
            s[j - 4] |= (uint8_t)((sc[j] >> 4) << 6);
            s[j] |= (uint8_t)((mn[j] >> 4) << 6);
        }
    }
}

// Q4_K (levels = 15) and Q5_K (levels = 31): per 32-value sub-block an
// affine map x ~ (d*sc)*q - (dmin*m) with q in [0, levels].
void enc_kq(const float* x, uint8_t* b, int levels) {
    float scl[8], mns[8], smax = 0, mmax = 0;
    for (int j = 0; j < 8; j++) {
        float lo = 0, hi = 0;  // include 0 so that the min is >= 0
        for (int i = 0; i < 32; i++) { lo = std::min(lo, x[32 * j + i]); hi = std::max(hi, x[32 * j + i]); }
        scl[j] = (hi - lo) / levels;
        mns[j] = -lo;
        smax = std::max(smax, scl[j]);
        mmax = std::max(mmax, mns[j]);
    }
    const uint16_t dh = f2h(smax / 63.0f), mh = f2h(mmax / 63.0f);
    const float d = h2f(dh), dm = h2f(mh);
    put16(b, dh);
    put16(b + 2, mh);
    int sc[8], mn[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = d > 0 ? clampi((int)std::nearbyint(scl[j] / d), 0, 63) : 0;
        mn[j] = dm > 0 ? clampi((int)std::nearbyint(mns[j] / dm), 0, 63) : 0;
    }
    pack_scale_min(sc, mn, b + 4);
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
        const float dl = d * (float)sc[j], ml = dm * (float)mn[j];
        for (int i = 0; i < 32; i++)
            q[32 * j + i] = (uint8_t)(dl > 0 ? clampi((int)std::nearbyint((x[32 * j + i] + ml) / dl), 0, levels) : 0);
    }
    if (levels == 15) {
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) b[16 + 32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
    } else {
        std::memset(b + 16, 0, 32);
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) {
                const int lo = q[64 * c + l], hi = q[64 * c + 32 + l];
                b[48 + 32 * c + l] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
                b[16 + l] |= (uint8_t)(((lo >> 4) << (2 * c)) | ((hi >> 4) << (2 * c + 1)));
            }
    }
}

// Q6_K: per 16-value group an int8 scale, value = (d*sc)*(q-32).
void enc_q6_k(const float* x, uint8_t* b) {
    float gs[16], gmax = 0;
    for (int g = 0; g < 16; g++) {
        float amax = 0;
        for (int i = 0; i < 16; i++) amax = std::max(amax, std::fabs(x[16 * g + i]));
        gs[g] = amax / 31.0f;
        gmax = std::max(gmax, gs[g]);
    }
    const uint16_t dh = f2h(gmax / 127.0f);
    const float d = h2f(dh);
    int sc[16];
    for (int g = 0; g < 16; g++) sc[g] = d > 0 ? clampi((int)std::nearbyint(gs[g] / d), -128, 127) : 0;
    int q[256];
    for (int v = 0; v < 256; v++) {
        const float dl = d * (float)sc[v / 16];
        q[v] = dl != 0 ? clampi((int)std::nearbyint(x[v] / dl), -32, 31) + 32 : 32;
    }
    for (int h = 0; h < 2; h++)
        for (int l = 0; l < 32; l++) {
            const int q0 = q[128 * h + l], q1 = q[128 * h + 32 + l], q2 = q[128 * h + 64 + l], q3 = q[128 * h + 96 + l];
            b[64 * h + l] = (uint8_t)((q0 & 15) | ((q2 & 15) << 4));
            b[64 * h + 32 + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
            b[128 + 32 * h + l] = (uint8_t)((q0 >> 4) | ((q1 >> 4) << 2) | ((q2 >> 4) << 4) | ((q3 >> 4) << 6));
        }
    for (int g = 0; g < 16; g++) b[192 + g] = (uint8_t)(int8_t)sc[g];
    put16(b + 208, dh);
}

void encode_block(uint32_t t, const float* x, uint8_t* b) {
    switch (t) {
    case ggq::T_Q8_0: enc_q8_0(x, b); break;
    case ggq::T_IQ4_NL: enc_iq4_nl(x, b); break;
    case ggq::T_IQ4_XS: enc_iq4_xs(x, b); break;
    case ggq::T_Q4_K: enc_kq(x, b, 15); break;
    case ggq::T_Q5_K: enc_kq(x, b, 31); break;
    case ggq::T_Q6_K: enc_q6_k(x, b); break;
    default: break;
    }
}

}  // namespace

extern "C" int ggq_encode(uint32_t type, const float* x, int64_t n_rows, int64_t K, void* out) {
    if (!ggq::supported(type) || !x || !out || n_rows < 0 || K <= 0 || K % ggq::block_elems(type))
        return GGQ_INVALID_PARAM;
    const int be = ggq::block_elems(type), bb = ggq::block_bytes(type);
    const int64_t nblk = n_rows * (K / be);
    uint8_t* o = (uint8_t*)out;
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (nt > 16) nt = 16;
    if (nblk < 4096) nt = 1;
    auto work = [&](int64_t b0, int64_t b1) {
        for (int64_t i = b0; i < b1; i++) encode_block(type, x + i * be, o + i * bb);
    };
    std::vector<std::thread> th;
    const int64_t chunk = (nblk + nt - 1) / nt;
    for (unsigned t = 1; t < nt; t++) {
        const int64_t b0 = t * chunk, b1 = std::min(nblk, b0 + chunk);
        if (b0 < b1) th.emplace_back(work, b0, b1);
    }
    work(0, std::min(nblk, chunk));
    for (auto& t : th) t.join();
    return GGQ_OK;
}
