// Per-lane integer kernels of the Q8_K-activation products.
//
// Lane mapping shared by every GEMV kernel: a wave covers 16 super-block columns per pass
// (slot = lane >> 2, g = slot + 16*i) and four lanes share one super-block (part = lane & 3).
//   Q4_K part p : sub-blocks 2p (low nibbles) and 2p+1 (high nibbles) = qs bytes [32p, 32p+32)
//   Q6_K part p : h = p>>1, jj = p&1 -> elements h*128 + k*32 + 16*jj + j (k<4, j<16), i.e. the
//                 four 16-element sub-blocks t = 8h + 2k + jj
// All sums here are exact int32 (|sum| < 2^31 for any byte content).
#pragma once
#include "kq_device.h"

namespace kq {

// Q4_K: quants qa (qs bytes 32p..32p+15) and qb (32p+16..32p+31); activations xl (8 dwords of
// sub-block 2p) and xh (8 dwords of sub-block 2p+1).  Returns the two 32-element dot sums.
__device__ __forceinline__ void q4k_lane_dots(const u32x4& qa, const u32x4& qb, const uint32_t* xl,
                                              const uint32_t* xh, int& plo, int& phi) {
    const uint32_t m = 0x0f0f0f0fu;
    int a = 0, b = 0;
    a = dot4(qa.x & m, xl[0], a); b = dot4((qa.x >> 4) & m, xh[0], b);
    a = dot4(qa.y & m, xl[1], a); b = dot4((qa.y >> 4) & m, xh[1], b);
    a = dot4(qa.z & m, xl[2], a); b = dot4((qa.z >> 4) & m, xh[2], b);
    a = dot4(qa.w & m, xl[3], a); b = dot4((qa.w >> 4) & m, xh[3], b);
    a = dot4(qb.x & m, xl[4], a); b = dot4((qb.x >> 4) & m, xh[4], b);
    a = dot4(qb.y & m, xl[5], a); b = dot4((qb.y >> 4) & m, xh[5], b);
    a = dot4(qb.z & m, xl[6], a); b = dot4((qb.z >> 4) & m, xh[6], b);
    a = dot4(qb.w & m, xl[7], a); b = dot4((qb.w >> 4) & m, xh[7], b);
    plo = a; phi = b;
}

// Q6_K: l0 = ql[h*64 + 16jj ..+16], l1 = ql[h*64 + 32 + 16jj ..+16], hb = qh[h*32 + 16jj ..+16];
// x[k*4 + w] = activation dword w of element group k.  P[k] = sum over the 16 elements of
// sub-block 8h+2k+jj of q6u * q8, with q6u = q6 + 32 in 0..63 (unsigned 6-bit code).
__device__ __forceinline__ void q6k_lane_dots(const u32x4& l0, const u32x4& l1, const u32x4& hb,
                                              const uint32_t* x, int* P) {
    const uint32_t m4 = 0x0f0f0f0fu, m2 = 0x30303030u;
    int p0 = 0, p1 = 0, p2 = 0, p3 = 0;
#define KQ_Q6_STEP(L0, L1, H, w)                                              \
    {                                                                         \
        const uint32_t q0 = ((L0) & m4) | (((H) << 4) & m2);                  \
        const uint32_t q1 = ((L1) & m4) | (((H) << 2) & m2);                  \
        const uint32_t q2 = (((L0) >> 4) & m4) | ((H) & m2);                  \
        const uint32_t q3 = (((L1) >> 4) & m4) | (((H) >> 2) & m2);           \
        p0 = dot4(q0, x[0 * 4 + (w)], p0);                                    \
        p1 = dot4(q1, x[1 * 4 + (w)], p1);                                    \
        p2 = dot4(q2, x[2 * 4 + (w)], p2);                                    \
        p3 = dot4(q3, x[3 * 4 + (w)], p3);                                    \
    }
    KQ_Q6_STEP(l0.x, l1.x, hb.x, 0)
    KQ_Q6_STEP(l0.y, l1.y, hb.y, 1)
    KQ_Q6_STEP(l0.z, l1.z, hb.z, 2)
    KQ_Q6_STEP(l0.w, l1.w, hb.w, 3)
#undef KQ_Q6_STEP
    P[0] = p0; P[1] = p1; P[2] = p2; P[3] = p3;
}

// Sign-extended int8 byte b of w.
__device__ __forceinline__ int sbyte(uint32_t w, int b) { return (int)(int8_t)(uint8_t)(w >> (8 * b)); }
// Sign-extended int16 half of w.
__device__ __forceinline__ int shalf(uint32_t w, int hi) { return (int)(int16_t)(uint16_t)(hi ? (w >> 16) : w); }

// ---- Per-(row, super-block) fp32 value: the numerical contract of every Q8_K product.
//   Q4_K: v = fma(d*dx, float(I1), -((dmin*dx) * float(I2)))
//   Q6_K: v = (d*dx) * float(I)
// with I1 = sum_s sc_s*S_s, I2 = sum_s m_s*(b_2s + b_2s+1), I = sum_t sc_t*S_t exact int32.
__device__ __forceinline__ float q4k_value(uint32_t dd_bits, float dx, int I1, int I2) {
    const float dd = __fmul_rn(f16_lo(dd_bits), dx);
    const float dm = __fmul_rn(f16_hi(dd_bits), dx);
    return __builtin_fmaf(dd, (float)I1, -__fmul_rn(dm, (float)I2));
}
__device__ __forceinline__ float q6k_value(float d, float dx, int I) {
    return __fmul_rn(__fmul_rn(d, dx), (float)I);
}

// Pairwise tree over super-block columns, padded with zeros to a power of two.  Per pass i the
// wave's 16 slots are reduced by slot_tree_f32 (levels 1-4 of the tree); pass results are merged
// here as a binary counter so that passes (2m, 2m+1) pair first, then (4m..4m+3), and so on.
constexpr int TREE_LEVELS = 4;   // up to 15 passes of 16 columns: C <= 61440
struct PassTree {
    float s[TREE_LEVELS];   // s[l] holds a completed subtree of 2^l passes, valid when bit l of n is set
    int n;
};
__device__ __forceinline__ void tree_init(PassTree& t) { t.n = 0; }
__device__ __forceinline__ void tree_push(PassTree& t, float v) {
    bool carry = true;   // v still has to be placed
#pragma unroll
    for (int l = 0; l < TREE_LEVELS; l++) {
        const bool bit = (t.n >> l) & 1;
        const float merged = __fadd_rn(t.s[l], v);
        if (carry && !bit) t.s[l] = v;
        if (carry && bit) v = merged;
        carry = carry && bit;
    }
    t.n += 1;
}
// Final value: merge pending subtrees from the smallest up, each padded with a zero subtree of
// its own size (x + 0 = x), i.e. partial = s[l] + partial for every set bit l in increasing l.
// The trailing +0.0f maps -0 to +0 so the sign of an exactly-zero result never depends on the
// path taken.
__device__ __forceinline__ float tree_final(const PassTree& t) {
    float r = 0.0f;
    bool have = false;
#pragma unroll
    for (int l = 0; l < TREE_LEVELS; l++) {
        if ((t.n >> l) & 1) {
            r = have ? __fadd_rn(t.s[l], r) : t.s[l];
            have = true;
        }
    }
    return __fadd_rn(r, 0.0f);
}

}  // namespace kq
