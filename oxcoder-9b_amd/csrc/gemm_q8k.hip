// Prefill GEMM for gfx950: Y[m][n] = sum_k x_q8[m][k] * W[n][k], Q4_K / Q6_K weights in the Kindi
// layout, Q8_K activations, int8 MFMA with int32 accumulation and an fp32 epilogue per super-block.
//
// Scale folding.  The 6-bit (Q4_K) or int8 (Q6_K) sub-block scale changes every 32 / 16 columns,
// faster than an MFMA K step can absorb.  It is folded into the weight: w' = sc*q is 10 bits
// (Q4_K, 0..945) or 14 bits signed (Q6_K, sc*(q+32) in [-8064, 8001]); written as w' = 128*h + l
// with l in 0..127 and h small, both are int8, so one super-block (K = 256) is two int8 MFMA
// sweeps accumulating I1 = sum_k w'*q8 exactly.  The remaining per-sub-block term (Q4_K min:
// I2 = sum_s m_s*B_s; Q6_K offset: I2 = sum_t sc_t*B_t with B from the Q8_K bsums) is one more
// small MFMA pair on B split as 64*Bh + Bl.  Per super-block the fp32 epilogue adds
//   Q4_K: dx * (d * I1 - dmin * I2)        Q6_K: dx * d * (I1 - 32 * I2)
// (the same per-super-block quantity as the GEMV; the I2 part is added first, then the I1 part,
// and the fp32 sums run along K in natural order).
//
// Work split.  A workgroup (4 waves) owns a 128 (tokens) x 128 (weight rows) output tile; each
// wave a 64 x 64 quarter = 2 x 2 MFMA 32x32 tiles.  Per super-block every thread unpacks half a
// weight row into the two int8 planes in LDS (row stride 272 B, 16-B aligned, staggered banks),
// while each lane reads its MFMA A operand (16 contiguous activation bytes) straight from the
// Q8_K block.  The next super-block's weight bytes and activation fragments are loaded into
// registers while the current one runs.  Rows past M or R are clamped for loading and not stored.
#include "kq_device.h"
#include "kq_internal.h"
#include "q4_lanes.h"

namespace kq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

constexpr int GM_BM = 128, GM_BN = 128, GM_WS = 272;   // tile rows, tile cols, LDS row stride

// ------------------------------------------------------------------ weight unpack helpers
// 4 unsigned nibbles (bytes of x, 0..15) times scale s (0..63): w' = s*q split into
// h = w' >> 7 (0..7) and l = w' & 127, returned as 4 bytes each.  Products are formed two at a
// time in 16-bit halves (each < 1024, so no carry crosses a half).
__device__ __forceinline__ void split_q4(uint32_t x, uint32_t s, uint32_t& hb, uint32_t& lb) {
    const uint32_t e = x & 0x00ff00ffu, o = (x >> 8) & 0x00ff00ffu;
    const uint32_t pe = __umul24(e, s), po = __umul24(o, s);
    lb = (pe & 0x007f007fu) | ((po & 0x007f007fu) << 8);
    hb = ((pe >> 7) & 0x00070007u) | (((po >> 7) & 0x00070007u) << 8);
}
// 4 unsigned 6-bit codes (bytes of q) times signed scale sc: w' = sc*q in [-8064, 8001] split into
// h = w' >> 7 (arithmetic, -63..62) and l = w' & 127.  16-bit lanes hold the exact signed product.
__device__ __forceinline__ void split_q6(uint32_t q, s16x2 s2, uint32_t& hb, uint32_t& lb) {
    const uint32_t e = q & 0x00ff00ffu, o = (q >> 8) & 0x00ff00ffu;
    const s16x2 pe = __builtin_bit_cast(s16x2, e) * s2, po = __builtin_bit_cast(s16x2, o) * s2;
    const uint32_t ue = __builtin_bit_cast(uint32_t, pe), uo = __builtin_bit_cast(uint32_t, po);
    lb = (ue & 0x007f007fu) | ((uo & 0x007f007fu) << 8);
    const uint32_t he = __builtin_bit_cast(uint32_t, (s16x2)(pe >> (short)7));
    const uint32_t ho = __builtin_bit_cast(uint32_t, (s16x2)(po >> (short)7));
    hb = (he & 0x00ff00ffu) | ((ho & 0x00ff00ffu) << 8);
}

__device__ __forceinline__ void st16(int8_t* p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    *reinterpret_cast<u32x4*>(p) = u32x4{a, b, c, d};
}

// Raw bytes of one half weight row (the thread's share of a super-block).
template <int TYPE> struct RawW;
template <> struct RawW<TYPE_Q4_K> { u32x4 hdr, q[4]; };
template <> struct RawW<TYPE_Q6_K> { u32x4 ql[4], qh[2]; uint32_t qle, qhe, sce, dw, sh; u32x2 sc; };

// bk: this row's block; ph: which half of the super-block (columns 128*ph .. 128*ph+127).
__device__ __forceinline__ void load_raw(RawW<TYPE_Q4_K>& r, const uint8_t* bk, int ph) {
    r.hdr = ld16(bk);
#pragma unroll
    for (int i = 0; i < 4; i++) r.q[i] = ld16(bk + 16 + 64 * ph + 16 * i);   // qs bytes 64ph .. 64ph+63
}
// Q6_K: the block starts at 0 or 2 (mod 4); words are read from the dword at or below each field
// (all fields share the shift).  The last word read ends at most 2 bytes past the block, inside
// the next row's block of the same tile column (only for blocks starting at 0 mod 4, which are
// never the last row of a tile).
__device__ __forceinline__ void load_raw(RawW<TYPE_Q6_K>& r, const uint8_t* bk, int ph) {
    r.sh = uint32_t(reinterpret_cast<uintptr_t>(bk) & 3);
    const uint8_t* b4 = bk - r.sh;
#pragma unroll
    for (int i = 0; i < 4; i++) r.ql[i] = ld16_a4(b4 + 64 * ph + 16 * i);     // ql bytes 64h .. 64h+63
    r.qle = ld4(b4 + 64 * ph + 64);
    r.qh[0] = ld16_a4(b4 + 128 + 32 * ph);                                    // qh bytes 32h .. 32h+31
    r.qh[1] = ld16_a4(b4 + 144 + 32 * ph);
    r.qhe = ld4(b4 + 160 + 32 * ph);
    r.sc = *reinterpret_cast<const u32x2_a4*>(b4 + 192 + 8 * ph);            // scales 8h .. 8h+7
    r.sce = ld4(b4 + 200 + 8 * ph);
    r.dw = ld4(b4 + 208);
}

// Unpack into the LDS planes: row pointers wh/wl (K index 0..255), aux row (16 bytes), d/dmin.
__device__ __forceinline__ void unpack(const RawW<TYPE_Q4_K>& r, int ph, int8_t* wh, int8_t* wl, uint8_t* aux,
                                       float* d, float* dm) {
#pragma unroll
    for (int pp = 0; pp < 2; pp++) {
        const int p = 2 * ph + pp;                                  // qs bytes 32p..32p+31: sub-blocks 2p, 2p+1
        const ScMin sm = q4k_scmin_pair(r.hdr.y, r.hdr.z, r.hdr.w, p);
#pragma unroll
        for (int c = 0; c < 2; c++) {                               // 16-byte chunk c: elements j = 16c .. 16c+15
            const u32x4 v = r.q[2 * pp + c];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            uint32_t lh[4], ll[4], hh[4], hl[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                split_q4(w[i] & 0x0f0f0f0fu, sm.sc_lo, lh[i], ll[i]);         // sub-block 2p
                split_q4((w[i] >> 4) & 0x0f0f0f0fu, sm.sc_hi, hh[i], hl[i]);  // sub-block 2p+1
            }
            const int k_lo = 64 * p + 16 * c, k_hi = 64 * p + 32 + 16 * c;
            st16(wh + k_lo, lh[0], lh[1], lh[2], lh[3]);
            st16(wl + k_lo, ll[0], ll[1], ll[2], ll[3]);
            st16(wh + k_hi, hh[0], hh[1], hh[2], hh[3]);
            st16(wl + k_hi, hl[0], hl[1], hl[2], hl[3]);
        }
        aux[2 * p] = (uint8_t)sm.m_lo;
        aux[2 * p + 1] = (uint8_t)sm.m_hi;
    }
    if (ph == 0) {
        *d = f16_lo(r.hdr.x);
        *dm = f16_hi(r.hdr.x);
    }
}

__device__ __forceinline__ void unpack(const RawW<TYPE_Q6_K>& r, int ph, int8_t* wh, int8_t* wl, uint8_t* aux,
                                       float* d, float* dm) {
    (void)dm;
    uint32_t ql[16], qh[8];
    {
        const uint32_t a[17] = {r.ql[0].x, r.ql[0].y, r.ql[0].z, r.ql[0].w, r.ql[1].x, r.ql[1].y, r.ql[1].z,
                                r.ql[1].w, r.ql[2].x, r.ql[2].y, r.ql[2].z, r.ql[2].w, r.ql[3].x, r.ql[3].y,
                                r.ql[3].z, r.ql[3].w, r.qle};
#pragma unroll
        for (int i = 0; i < 16; i++) ql[i] = __builtin_amdgcn_alignbyte(a[i + 1], a[i], r.sh);
        const uint32_t b[9] = {r.qh[0].x, r.qh[0].y, r.qh[0].z, r.qh[0].w, r.qh[1].x, r.qh[1].y, r.qh[1].z,
                               r.qh[1].w, r.qhe};
#pragma unroll
        for (int i = 0; i < 8; i++) qh[i] = __builtin_amdgcn_alignbyte(b[i + 1], b[i], r.sh);
    }
    const uint32_t sc0 = __builtin_amdgcn_alignbyte(r.sc.y, r.sc.x, r.sh);   // scales 8h .. 8h+3
    const uint32_t sc1 = __builtin_amdgcn_alignbyte(r.sce, r.sc.y, r.sh);    // scales 8h+4 .. 8h+7
#pragma unroll
    for (int k = 0; k < 4; k++) {                     // element e = 128h + 32k + j
#pragma unroll
        for (int c = 0; c < 2; c++) {                 // j = 16c .. 16c+15: sub-block 8h + 2k + c
            const uint32_t scw = k < 2 ? sc0 : sc1;
            const int scv = (int)(int8_t)(uint8_t)(scw >> (8 * ((2 * k + c) & 3)));
            const s16x2 s2 = {(short)scv, (short)scv};
            uint32_t hb[4], lb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t L = ql[8 * (k & 1) + 4 * c + i], H = qh[4 * c + i];
                const uint32_t q = ((L >> (4 * (k >> 1))) & 0x0f0f0f0fu) | (((H >> (2 * k)) & 0x03030303u) << 4);
                split_q6(q, s2, hb[i], lb[i]);
            }
            const int kk = 128 * ph + 32 * k + 16 * c;
            st16(wh + kk, hb[0], hb[1], hb[2], hb[3]);
            st16(wl + kk, lb[0], lb[1], lb[2], lb[3]);
        }
    }
    *reinterpret_cast<uint32_t*>(aux + 8 * ph) = sc0;
    *reinterpret_cast<uint32_t*>(aux + 8 * ph + 4) = sc1;
    if (ph == 0) *d = f16_lo(r.dw >> (8 * r.sh));
}

// ------------------------------------------------------------------ activation-side operands
// bsums of one Q8_K block (16 int16 in 8 dwords) -> the min-term A operand for this lane's half:
// Q4_K: B_s = b_2s + b_2s+1 (s < 8), half 0 gets B_s & 63, half 1 gets B_s >> 6, 8 bytes (K = 16).
// Q6_K: B_t = b_t (t < 16), same split, 16 bytes (K = 32).
__device__ __forceinline__ uint32_t pack_split(int B0, int B1, int B2, int B3, int half) {
    const int v0 = half ? (B0 >> 6) : (B0 & 63), v1 = half ? (B1 >> 6) : (B1 & 63);
    const int v2 = half ? (B2 >> 6) : (B2 & 63), v3 = half ? (B3 >> 6) : (B3 & 63);
    return (uint32_t)(v0 & 255) | ((uint32_t)(v1 & 255) << 8) | ((uint32_t)(v2 & 255) << 16) | ((uint32_t)v3 << 24);
}

// ------------------------------------------------------------------ the kernel
template <int TYPE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_gemm_q8k(const uint8_t* __restrict__ W, int R, int G, const uint8_t* __restrict__ XQ, int M,
           float* __restrict__ Y, int64_t ldy) {
    constexpr int BS = TYPE == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    __shared__ __attribute__((aligned(16))) int8_t sWh[GM_BN * GM_WS];
    __shared__ __attribute__((aligned(16))) int8_t sWl[GM_BN * GM_WS];
    __shared__ __attribute__((aligned(16))) uint8_t sAux[GM_BN * 16];
    __shared__ float sD[GM_BN], sDm[GM_BN], sDx[GM_BM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, l32 = lane & 31;
    const int n0 = blockIdx.x * GM_BN, m0 = blockIdx.y * GM_BM;
    const int64_t xrow = (int64_t)G * Q8K_BYTES;

    // activation rows this lane feeds (clamped), and the dx row this thread stages
    const uint8_t* arow[2];
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
        int m = m0 + 64 * wm + 32 * mt + l32;
        m = m < M ? m : M - 1;
        arow[mt] = XQ + m * xrow;
    }
    const uint8_t* dxrow = XQ + (int64_t)(m0 + (tid & 127) < M ? m0 + (tid & 127) : M - 1) * xrow;

    // weight half-row this thread unpacks
    const int pn = tid >> 1, ph = tid & 1;
    const int pr = n0 + pn < R ? n0 + pn : R - 1;
    const uint8_t* prow = W + ((int64_t)(pr >> 3) * G * 8 + (pr & 7)) * BS;   // block (pr, g) = prow + g*8*BS

    float yacc[2][2][16];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int a = 0; a < 16; a++) yacc[mt][nt][a] = 0.0f;

    RawW<TYPE> raw;
    u32x4 afr[2][8], bsr[2][2];
    float dxv = 0.0f;
    load_raw(raw, prow, ph);
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
#pragma unroll
        for (int ks = 0; ks < 8; ks++) afr[mt][ks] = ld16_a4(arow[mt] + 4 + 32 * ks + 16 * half);
        bsr[mt][0] = ld16_a4(arow[mt] + 260);
        bsr[mt][1] = ld16_a4(arow[mt] + 276);
    }
    dxv = __builtin_bit_cast(float, ld4(dxrow));

    for (int g = 0; g < G; g++) {
        // ---- unpack this super-block's weights into LDS
        unpack(raw, ph, sWh + pn * GM_WS, sWl + pn * GM_WS, sAux + pn * 16, sD + pn, sDm + pn);
        if (tid < GM_BM) sDx[tid] = dxv;
        __syncthreads();

        // ---- operands of this super-block, then prefetch the next one's
        u32x4 acur[2][8], bcur[2][2];
#pragma unroll
        for (int mt = 0; mt < 2; mt++) {
#pragma unroll
            for (int ks = 0; ks < 8; ks++) acur[mt][ks] = afr[mt][ks];
            bcur[mt][0] = bsr[mt][0];
            bcur[mt][1] = bsr[mt][1];
        }
        if (g + 1 < G) {
            load_raw(raw, prow + (int64_t)(g + 1) * 8 * BS, ph);
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                const uint8_t* xb = arow[mt] + (int64_t)(g + 1) * Q8K_BYTES;
#pragma unroll
                for (int ks = 0; ks < 8; ks++) afr[mt][ks] = ld16_a4(xb + 4 + 32 * ks + 16 * half);
                bsr[mt][0] = ld16_a4(xb + 260);
                bsr[mt][1] = ld16_a4(xb + 276);
            }
            dxv = __builtin_bit_cast(float, ld4(dxrow + (int64_t)(g + 1) * Q8K_BYTES));
        }

        // ---- min / offset term: I2 = 64 * (A_h . B) + A_l . B, applied to the fp32 sums at once
        //      Q4_K: y -= dx * dmin * I2          Q6_K: y -= dx * d * 32 * I2
        {
            const int ncol[2] = {64 * wn + l32, 64 * wn + 32 + l32};
            if (TYPE == TYPE_Q4_K) {
                long am[2];
#pragma unroll
                for (int mt = 0; mt < 2; mt++) {
                    const uint32_t w[8] = {bcur[mt][0].x, bcur[mt][0].y, bcur[mt][0].z, bcur[mt][0].w,
                                           bcur[mt][1].x, bcur[mt][1].y, bcur[mt][1].z, bcur[mt][1].w};
                    int B[8];
#pragma unroll
                    for (int s = 0; s < 8; s++) B[s] = shalf(w[s], 0) + shalf(w[s], 1);
                    const uint32_t lo = pack_split(B[0], B[1], B[2], B[3], half);
                    const uint32_t hi = pack_split(B[4], B[5], B[6], B[7], half);
                    am[mt] = (long)(((uint64_t)hi << 32) | lo);
                }
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    const long mn = *reinterpret_cast<const long*>(sAux + ncol[nt] * 16);
                    const long b_lo = half ? 0L : mn, b_hi = half ? mn : 0L;
                    const float dm = sDm[ncol[nt]];
#pragma unroll
                    for (int mt = 0; mt < 2; mt++) {
                        v16i c = {};
                        c = __builtin_amdgcn_mfma_i32_32x32x16_i8(am[mt], b_hi, c, 0, 0, 0);
#pragma unroll
                        for (int a = 0; a < 16; a++) c[a] <<= 6;
                        c = __builtin_amdgcn_mfma_i32_32x32x16_i8(am[mt], b_lo, c, 0, 0, 0);
#pragma unroll
                        for (int a = 0; a < 16; a++) {
                            const float dx = sDx[64 * wm + 32 * mt + (a >> 2) * 8 + half * 4 + (a & 3)];
                            yacc[mt][nt][a] = __builtin_fmaf(dx, -__fmul_rn(dm, (float)c[a]), yacc[mt][nt][a]);
                        }
                    }
                }
            } else {
                v4i am[2];
#pragma unroll
                for (int mt = 0; mt < 2; mt++) {
                    const uint32_t w[8] = {bcur[mt][0].x, bcur[mt][0].y, bcur[mt][0].z, bcur[mt][0].w,
                                           bcur[mt][1].x, bcur[mt][1].y, bcur[mt][1].z, bcur[mt][1].w};
                    uint32_t pk[4];
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        pk[i] = pack_split(shalf(w[2 * i], 0), shalf(w[2 * i], 1), shalf(w[2 * i + 1], 0),
                                           shalf(w[2 * i + 1], 1), half);
                    am[mt] = v4i{(int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3]};
                }
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    const u32x4 scv = *reinterpret_cast<const u32x4*>(sAux + ncol[nt] * 16);
                    const v4i sc = __builtin_bit_cast(v4i, scv), zero = {0, 0, 0, 0};
                    const v4i b_lo = half ? zero : sc, b_hi = half ? sc : zero;
                    const float d = sD[ncol[nt]];
#pragma unroll
                    for (int mt = 0; mt < 2; mt++) {
                        v16i c = {};
                        c = __builtin_amdgcn_mfma_i32_32x32x32_i8(am[mt], b_hi, c, 0, 0, 0);
#pragma unroll
                        for (int a = 0; a < 16; a++) c[a] <<= 6;
                        c = __builtin_amdgcn_mfma_i32_32x32x32_i8(am[mt], b_lo, c, 0, 0, 0);
#pragma unroll
                        for (int a = 0; a < 16; a++) {
                            const float dx = sDx[64 * wm + 32 * mt + (a >> 2) * 8 + half * 4 + (a & 3)];
                            yacc[mt][nt][a] = __builtin_fmaf(dx, -__fmul_rn(d, (float)(32 * c[a])), yacc[mt][nt][a]);
                        }
                    }
                }
            }
        }

        // ---- main sweeps: I1 = 128 * (A . Wh) + A . Wl over K = 256
        v16i acch[2][2], accl[2][2];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++) {
                acch[mt][nt] = v16i{};
                accl[mt][nt] = v16i{};
            }
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            v4i bh[2], bl[2];
#pragma unroll
            for (int nt = 0; nt < 2; nt++) {
                const int off = (64 * wn + 32 * nt + l32) * GM_WS + 32 * ks + 16 * half;
                bh[nt] = *reinterpret_cast<const v4i*>(sWh + off);
                bl[nt] = *reinterpret_cast<const v4i*>(sWl + off);
            }
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
                const v4i a = __builtin_bit_cast(v4i, acur[mt][ks]);
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    acch[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bh[nt], acch[mt][nt], 0, 0, 0);
                    accl[mt][nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bl[nt], accl[mt][nt], 0, 0, 0);
                }
            }
        }

        // ---- epilogue of this super-block
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const int nl = 64 * wn + 32 * nt + l32;
            const float d = sD[nl];
#pragma unroll
            for (int mt = 0; mt < 2; mt++) {
#pragma unroll
                for (int a = 0; a < 16; a++) {
                    const int ml = 64 * wm + 32 * mt + (a >> 2) * 8 + half * 4 + (a & 3);
                    const float dx = sDx[ml];
                    const int i1 = (acch[mt][nt][a] << 7) + accl[mt][nt][a];
                    yacc[mt][nt][a] = __builtin_fmaf(dx, __fmul_rn(d, (float)i1), yacc[mt][nt][a]);
                }
            }
        }
        __syncthreads();
    }

    // ---- store
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const int n = n0 + 64 * wn + 32 * nt + l32;
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int a = 0; a < 16; a++) {
                const int m = m0 + 64 * wm + 32 * mt + (a >> 2) * 8 + half * 4 + (a & 3);
                if (m < M && n < R) Y[(int64_t)m * ldy + n] = yacc[mt][nt][a];
            }
    }
}

void launch_gemm_q8k(const uint8_t* w, int R, int C, int type, const uint8_t* xq, int M, float* y, int64_t ldy,
                     hipStream_t s) {
    const int G = C / QK;
    dim3 grid((R + GM_BN - 1) / GM_BN, (M + GM_BM - 1) / GM_BM), block(256);
    if (type == TYPE_Q4_K)
        hipLaunchKernelGGL(k_gemm_q8k<TYPE_Q4_K>, grid, block, 0, s, w, R, G, xq, M, y, ldy);
    else
        hipLaunchKernelGGL(k_gemm_q8k<TYPE_Q6_K>, grid, block, 0, s, w, R, G, xq, M, y, ldy);
}

}  // namespace kq
