// Host-side synthetic weight quantizer and Kindi repack (include/kq_host.h).
// Built with g++ -O3 -fopenmp -ffp-contract=off: every float step below is one IEEE operation.
#include "kq_host.h"

#include <cmath>
#include <cstring>

namespace {

constexpr int QK = 256;

// fp32 -> fp16 bits, round to nearest even, with subnormals, overflow to inf and NaN.
uint16_t f2h(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          // >= 65520 rounds to inf
    if (ax < 0x38800000u) {                                            // below 2^-14: subnormal
        float a;
        std::memcpy(&a, &ax, 4);
        const uint32_t m = (uint32_t)std::nearbyint(a * 16777216.0f);  // a * 2^24 is exact
        return (uint16_t)(sign | m);
    }
    const uint32_t e = (ax >> 23) - 112;                                // rebias 127 -> 15
    uint32_t h = (e << 10) | ((ax >> 13) & 0x3ffu);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t u;
    if (e == 0) {
        if (m == 0) u = s;
        else {
            int sh = 0;
            uint32_t mm = m;
            while (!(mm & 1024u)) { mm <<= 1; sh++; }
            u = s | ((uint32_t)(113 - sh) << 23) | ((mm & 1023u) << 13);
        }
    } else if (e == 31) u = s | 0x7f800000u | (m << 13);
    else u = s | ((e + 112) << 23) | (m << 13);
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

inline int rint_clamp(float v, int lo, int hi) {
    const float r = std::nearbyint(v);
    if (!(r >= (float)lo)) return lo;   // also maps NaN to lo
    if (r > (float)hi) return hi;
    return (int)r;
}

void quant_q4k_block(const float* x, uint8_t* b) {
    float scale[8], mn[8];
    float max_scale = 0.0f, max_mn = 0.0f;
    for (int s = 0; s < 8; s++) {
        float lo = x[32 * s], hi = x[32 * s];
        for (int j = 1; j < 32; j++) {
            const float v = x[32 * s + j];
            if (v < lo) lo = v;
            if (v > hi) hi = v;
        }
        if (lo > 0.0f) lo = 0.0f;
        scale[s] = (hi - lo) / 15.0f;
        mn[s] = -lo;
        if (scale[s] > max_scale) max_scale = scale[s];
        if (mn[s] > max_mn) max_mn = mn[s];
    }
    const uint16_t d16 = f2h(max_scale / 63.0f), dm16 = f2h(max_mn / 63.0f);
    const float d = h2f(d16), dm = h2f(dm16);
    int sc[8], m[8];
    for (int s = 0; s < 8; s++) {
        sc[s] = d > 0.0f ? rint_clamp(scale[s] / d, 0, 63) : 0;
        m[s] = dm > 0.0f ? rint_clamp(mn[s] / dm, 0, 63) : 0;
    }
    std::memset(b, 0, 144);
    std::memcpy(b, &d16, 2);
    std::memcpy(b + 2, &dm16, 2);
    uint8_t* sb = b + 4;
    for (int j = 0; j < 4; j++) {    // inverse of the 6-bit unpack in q4kernels.h:17-18
        sb[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        sb[j + 4] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
        sb[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
    for (int s = 0; s < 8; s++) {
        const float ds = d * (float)sc[s], ms = dm * (float)m[s];
        for (int j = 0; j < 32; j++) {
            const int q = ds > 0.0f ? rint_clamp((x[32 * s + j] + ms) / ds, 0, 15) : 0;
            b[16 + (s / 2) * 32 + j] |= (uint8_t)(q << ((s % 2) * 4));
        }
    }
}

void quant_q6k_block(const float* x, uint8_t* b) {
    float s16[16], max_s = 0.0f;
    for (int t = 0; t < 16; t++) {
        float amax = 0.0f;
        for (int j = 0; j < 16; j++) {
            const float a = std::fabs(x[16 * t + j]);
            if (a > amax) amax = a;
        }
        s16[t] = amax / 31.0f;
        if (s16[t] > max_s) max_s = s16[t];
    }
    const uint16_t d16 = f2h(max_s / 127.0f);
    const float d = h2f(d16);
    std::memset(b, 0, 210);
    int8_t* scb = reinterpret_cast<int8_t*>(b + 192);
    for (int t = 0; t < 16; t++) scb[t] = (int8_t)(d > 0.0f ? rint_clamp(s16[t] / d, -128, 127) : 0);
    std::memcpy(b + 208, &d16, 2);
    for (int e = 0; e < QK; e++) {
        const float ds = d * (float)scb[e / 16];
        const int q = ds > 0.0f ? rint_clamp(x[e] / ds, -32, 31) : 0;
        const int u = q + 32;                       // 0..63; layout of q4kernels.h:26-28
        const int h = e / 128, k = (e % 128) / 32, j = e % 32;
        b[h * 64 + (k % 2) * 32 + j] |= (uint8_t)((u & 15) << ((k / 2) * 4));
        b[128 + h * 32 + j] |= (uint8_t)((u >> 4) << (2 * k));
    }
}

int block_bytes(int type) { return type == 12 ? 144 : type == 14 ? 210 : 0; }

}  // namespace

extern "C" {

int kq_host_quantize_q4k(const float* w, int64_t R, int C, uint8_t* out) {
    if (!w || !out || R <= 0 || C <= 0 || C % QK) return -1;
    const int64_t nb = R * (C / QK);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < nb; i++) quant_q4k_block(w + i * QK, out + i * 144);
    return 0;
}

int kq_host_quantize_q6k(const float* w, int64_t R, int C, uint8_t* out) {
    if (!w || !out || R <= 0 || C <= 0 || C % QK) return -1;
    const int64_t nb = R * (C / QK);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < nb; i++) quant_q6k_block(w + i * QK, out + i * 210);
    return 0;
}

int kq_host_tile(const uint8_t* in, int64_t R, int C, int type, uint8_t* out) {
    const int bs = block_bytes(type);
    if (!in || !out || !bs || R <= 0 || R % 8 || C <= 0 || C % QK) return -1;
    const int64_t G = C / QK;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < R; r++)
        for (int64_t g = 0; g < G; g++)
            std::memcpy(out + (((r / 8) * G + g) * 8 + r % 8) * bs, in + (r * G + g) * bs, bs);
    return 0;
}

int kq_host_untile(const uint8_t* in, int64_t R, int C, int type, uint8_t* out) {
    const int bs = block_bytes(type);
    if (!in || !out || !bs || R <= 0 || R % 8 || C <= 0 || C % QK) return -1;
    const int64_t G = C / QK;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < R; r++)
        for (int64_t g = 0; g < G; g++)
            std::memcpy(out + (r * G + g) * bs, in + (((r / 8) * G + g) * 8 + r % 8) * bs, bs);
    return 0;
}

}  // extern "C"
