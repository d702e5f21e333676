// Small-batch GEMV (speculative verify, 2..16 tokens; one token for some shapes) on int8 MFMA for gfx950.
//
// A wave owns 16 weight rows x 4 consecutive super-blocks (a "chunk") for all tokens: per
// super-block it forms the exact integers of the GEMV (Q4_K: I1 = sum sc_s*S_s and
// I2 = sum m_s*B_s; Q6_K: I = sum sc_t*(S_t - 32*b_t)) with v_mfma_i32_16x16x64_i8 (tokens x rows,
// K = 64 per step), turns them into the per-super-block fp32 value with the GEMV's own formula
// (q4k_value / q6k_value) and adds the chunk's four values as ((v0+v1)+(v2+v3)).  A workgroup
// holds every chunk of its 16 rows; after one barrier the chunk sums of each 16-column pass are
// merged as ((c0+c1)+(c2+c3)) and the passes with the pass tree, which is exactly the column tree
// of the GEMV (zero-padded columns included).  Every output is therefore bit-identical to the
// GEMV of that token alone.
//
// Operands.  The scale is folded into the weights as in the prefill GEMM, split into two int8
// planes: Q4_K sc = 8a + b, planes a*q and b*q (I1 = 8*(x.H) + (x.L)); Q6_K w = sc*(q - 32),
// v = w + 128, planes high byte of v and low byte of v ^ 0x80 (I = 256*(x.H) + (x.L)).  The Q4_K
// min term is one v_mfma_f32_16x16x16_f16 with exact small-integer operands [B_s >> 6, B_s & 63]
// and [-64 m_s, -m_s], which returns -I2 exactly.  Up to 4 (Q4_K) or 8 (Q6_K) tokens a second form
// is used (k_gemv_mfma_ph, below): raw codes against sub-block-phased activations, no planes.
//
// MFMA lanes (the plane form): lane l serves token (A operand) and weight row (B operand) l & 15 and K slots
// 16q .. 16q+15 of each step, q = l >> 4.  Outputs: lane l holds tokens 4q + j (j = 0..3) of
// row l & 15.  Which super-block elements a K slot carries is free (the products are exact integer
// sums), so each type uses the assignment that loads its bytes best:
//   Q4_K: lane q reads qs bytes 32q .. 32q+31 (sub-blocks 2q and 2q+1, the GEMV's lane layout),
//         each quant byte once per row; step p takes bytes 32q + 8p .. +7, low nibbles (elements
//         64q + 8p + i) in slots 0..7 and high nibbles (64q + 32 + 8p + i) in slots 8..15, and
//         the activation bytes of those elements come from the lane's 64 contiguous ones.
//   Q6_K: step p covers elements 64p + 16q + i (h = p >> 1 selects the 128-element half).
#include "kq_device.h"
#include "kq_internal.h"
#include "q4_lanes.h"

namespace kq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short s16x2 __attribute__((ext_vector_type(2)));

#ifndef KQ_GEMV_MFMA_Q6_PLANES
#define KQ_GEMV_MFMA_Q6_PLANES 0   // 1: Q6_K through the two-plane form instead of sub-block phases
#endif
#ifndef KQ_GEMV_MFMA_RG
#define KQ_GEMV_MFMA_RG 1          // plane form with at most 32 super-blocks: two row groups per wave
#endif
#ifndef KQ_GEMV_MFMA_Q4_PH_MAX
#define KQ_GEMV_MFMA_Q4_PH_MAX 4   // Q4_K through the phase form up to this many tokens (at most 8)
#endif
#ifndef KQ_Q4P_FP1
#define KQ_Q4P_FP1 4   // super-blocks in flight per wave, Q4_K phase form, 1-4 tokens
#endif
#ifndef KQ_Q4P_FP2
#define KQ_Q4P_FP2 2   // the same, 5-8 tokens
#endif
#ifndef KQ_Q6P_FP1
#define KQ_Q6P_FP1 4   // super-blocks in flight per wave, Q6_K phase form, 1-4 tokens
#endif
#ifndef KQ_Q6P_FP2
#define KQ_Q6P_FP2 2   // the same, 5-8 tokens
#endif

constexpr int MV_ROWS = 16;     // weight rows per workgroup
constexpr int MV_CHUNK = 4;     // super-blocks per wave

struct MvGroup {
    const uint8_t* w[3];
    float* y[3];
    int64_t ldy[3];
    int R[3];
    int first[4];   // workgroups of matrix m are [first[m], first[m+1])
};
// Kernel arguments: first, as plain scalars, what the prologue needs (the three matrices' weights, the
// activations, the row counts, the first workgroups of matrices 1 and 2 packed as f1 | f2 << 16, and
// NxG = N | G << 8), 13 dwords that the dispatch preloads into scalar registers
// (-amdgpu-kernarg-preload-count), so a wave's first loads wait for no argument fetch; the matrix table
// follows for the outputs.  Matrix m's fields are picked by selects, not by an indexed load that would
// wait for m.
#define KQ_MV_HEAD                                                                                    \
    const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1, const uint8_t* __restrict__ w2,   \
        const uint8_t* __restrict__ XQ, int R0, int R1, int R2, int F12, int NxG
#define KQ_MV_PICK(wg, rows)                                                                          \
    const int N = NxG & 0xff, G = NxG >> 8;                                                           \
    const int m = (wg) >= (F12 & 0xffff) ? ((wg) >= (F12 >> 16) ? 2 : 1) : 0;                         \
    const int R = mv_pick(m, R0, R1, R2);                                                             \
    const int row0 = ((wg) - mv_pick(m, 0, F12 & 0xffff, F12 >> 16)) * (rows);                        \
    const uint8_t* const wm = mv_pick(m, w0, w1, w2)
template <class T> __device__ __forceinline__ T mv_pick(int m, T a, T b, T c) { return m == 0 ? a : m == 1 ? b : c; }

__device__ __forceinline__ uint32_t mv_mul_u8x4(uint32_t q, uint32_t s2) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, q) * __builtin_bit_cast(u16x2, s2));
}
__device__ __forceinline__ uint32_t mv_pk_f16(float a, float b) {   // exact small integers only
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}

// ------------------------------------------------------------------ per-super-block operands
template <int TYPE> struct MvW;
// Q4_K: header and the lane's 32 qs bytes 32q .. 32q+31.
template <> struct MvW<TYPE_Q4_K> { u32x4 hdr, qa, qb; };
// Q6_K: dword-aligned raw words: ql bytes 64h + 16q (h = 0, 1), qh bytes 32h + 16(q & 1), the 16
// scales and d, each 16-byte field with the dword after it; sh = block start & 3.
template <> struct MvW<TYPE_Q6_K> { u32x4 ql[2], qh[2], sc; uint32_t qle[2], qhe[2], sce, sh; };

struct MvX {
    u32x4 a[4];     // activation bytes of token l & 15: Q4_K 64q + 16k .. +15, Q6_K 64k + 16q .. +15
    u32x4 bs;       // bsums 8(q & 1) .. 8(q & 1) + 7 of token l & 15 (Q4_K min term; not loaded for Q6_K)
    float dx[4];    // d of tokens 4q + j
};

__device__ __forceinline__ void mv_load(MvW<TYPE_Q4_K>& w, const uint8_t* bk, int q) {
    w.hdr = ld16(bk);
    w.qa = ld16(bk + 16 + 32 * q);
    w.qb = ld16(bk + 32 + 32 * q);
}
// The last word read (bytes 208..211 from the aligned base) passes the block end by 2 bytes only
// for blocks starting at 0 (mod 4), which are never row 7 of a tile column.
__device__ __forceinline__ void mv_load(MvW<TYPE_Q6_K>& w, const uint8_t* bk, int q) {
    w.sh = uint32_t(reinterpret_cast<uintptr_t>(bk) & 3);
    const uint8_t* b4 = bk - w.sh;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        w.ql[h] = ld16_a4(b4 + 64 * h + 16 * q);
        w.qle[h] = ld4(b4 + 64 * h + 16 * q + 16);
        w.qh[h] = ld16_a4(b4 + 128 + 32 * h + 16 * (q & 1));
        w.qhe[h] = ld4(b4 + 144 + 32 * h + 16 * (q & 1));
    }
    w.sc = ld16_a4(b4 + 192);
    w.sce = ld4(b4 + 208);
}
// xa: Q8_K block of token l & 15; xd[j]: Q8_K block of token 4q + j (tokens clamped by the caller).
template <int TYPE>
__device__ __forceinline__ void mv_load_x(MvX& x, const uint8_t* xa, const uint8_t* const* xd, int q) {
#pragma unroll
    for (int k = 0; k < 4; k++) x.a[k] = ld16_a4(xa + 4 + (TYPE == TYPE_Q4_K ? 64 * q + 16 * k : 64 * k + 16 * q));
    if constexpr (TYPE == TYPE_Q4_K) x.bs = ld16_a4(xa + 260 + 16 * (q & 1));   // the min term's bsums
#pragma unroll
    for (int j = 0; j < 4; j++) x.dx[j] = __builtin_bit_cast(float, ld4(xd[j]));
}

__device__ __forceinline__ u32x4 mv_funnel(const u32x4& v, uint32_t e, uint32_t sh) {
    return u32x4{__builtin_amdgcn_alignbyte(v.y, v.x, sh), __builtin_amdgcn_alignbyte(v.z, v.y, sh),
                 __builtin_amdgcn_alignbyte(v.w, v.z, sh), __builtin_amdgcn_alignbyte(e, v.w, sh)};
}

// The four per-super-block values (tokens 4q + j of row l & 15).
__device__ __forceinline__ void mv_values(const MvW<TYPE_Q4_K>& w, const MvX& x, int q, float v[4]) {
    // planes of the lane's two sub-blocks 2q (low nibbles) and 2q + 1 (high nibbles)
    const ScMin sm = q4k_scmin_pair(w.hdr.y, w.hdr.z, w.hdr.w, q);
    const uint32_t al = (sm.sc_lo >> 3) * 0x10001u, bl = (sm.sc_lo & 7u) * 0x10001u;
    const uint32_t ah = (sm.sc_hi >> 3) * 0x10001u, bh = (sm.sc_hi & 7u) * 0x10001u;
    const uint32_t ws[8] = {w.qa.x, w.qa.y, w.qa.z, w.qa.w, w.qb.x, w.qb.y, w.qb.z, w.qb.w};
    const uint32_t xw[16] = {x.a[0].x, x.a[0].y, x.a[0].z, x.a[0].w, x.a[1].x, x.a[1].y, x.a[1].z, x.a[1].w,
                             x.a[2].x, x.a[2].y, x.a[2].z, x.a[2].w, x.a[3].x, x.a[3].y, x.a[3].z, x.a[3].w};
    v4i hp[4], lp[4], xa[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const uint32_t l0 = ws[2 * p] & 0x0f0f0f0fu, l1 = ws[2 * p + 1] & 0x0f0f0f0fu;
        const uint32_t h0 = (ws[2 * p] >> 4) & 0x0f0f0f0fu, h1 = (ws[2 * p + 1] >> 4) & 0x0f0f0f0fu;
        hp[p] = v4i{(int)mv_mul_u8x4(l0, al), (int)mv_mul_u8x4(l1, al), (int)mv_mul_u8x4(h0, ah), (int)mv_mul_u8x4(h1, ah)};
        lp[p] = v4i{(int)mv_mul_u8x4(l0, bl), (int)mv_mul_u8x4(l1, bl), (int)mv_mul_u8x4(h0, bh), (int)mv_mul_u8x4(h1, bh)};
        xa[p] = v4i{(int)xw[2 * p], (int)xw[2 * p + 1], (int)xw[8 + 2 * p], (int)xw[9 + 2 * p]};
    }
    v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[0], hp[0], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
    for (int p = 1; p < 4; p++) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[p], hp[p], acc, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] <<= 3;
#pragma unroll
    for (int p = 0; p < 4; p++) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[p], lp[p], acc, 0, 0, 0);

    // min term: K 4q..4q+3 = sub-blocks 4(q & 1) .. +3, the high (q < 2) or low part of B
    const ScMin m0 = q4k_scmin_pair(w.hdr.y, w.hdr.z, w.hdr.w, 2 * (q & 1));
    const ScMin m1 = q4k_scmin_pair(w.hdr.y, w.hdr.z, w.hdr.w, 2 * (q & 1) + 1);
    const float f = (q >> 1) ? -1.0f : -64.0f;
    const v4h bm = __builtin_bit_cast(v4h, u32x2{mv_pk_f16(f * (float)m0.m_lo, f * (float)m0.m_hi),
                                                 mv_pk_f16(f * (float)m1.m_lo, f * (float)m1.m_hi)});
    const uint32_t bw[4] = {x.bs.x, x.bs.y, x.bs.z, x.bs.w};
    float B[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int s = shalf(bw[k], 0) + shalf(bw[k], 1);
        B[k] = (float)((q >> 1) ? (s & 63) : (s >> 6));
    }
    const v4h am = __builtin_bit_cast(v4h, u32x2{mv_pk_f16(B[0], B[1]), mv_pk_f16(B[2], B[3])});
    const v4f cm = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);   // -I2
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = q4k_value(w.hdr.x, x.dx[j], acc[j], (int)(-cm[j]));
}

__device__ __forceinline__ void mv_values(const MvW<TYPE_Q6_K>& w, const MvX& x, int q, float v[4]) {
    const uint32_t sh = w.sh;
    u32x4 QL[2], QH[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        QL[h] = mv_funnel(w.ql[h], w.qle[h], sh);
        QH[h] = mv_funnel(w.qh[h], w.qhe[h], sh);
    }
    const u32x4 SC = mv_funnel(w.sc, w.sce, sh);          // the 16 int8 scales
    const float d = f16_lo(w.sce >> (8 * sh));             // bytes 208, 209 of the block
    const uint32_t scw[4] = {SC.x, SC.y, SC.z, SC.w};
    v4i hp[4], lp[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const int h = p >> 1, k = 2 * (p & 1) + (q >> 1);
        const int t = 8 * h + 2 * k + (q & 1);            // scale of elements 64p + 16q + i
        const int sc = sbyte(scw[t >> 2], t & 3);
        const s16x2 s2 = __builtin_bit_cast(s16x2, (uint32_t)(sc & 0xffff) * 0x10001u);
        const s16x2 c2 = __builtin_bit_cast(s16x2, (uint32_t)((128 - 32 * sc) & 0xffff) * 0x10001u);
        const uint32_t lw[4] = {QL[h].x, QL[h].y, QL[h].z, QL[h].w};
        const uint32_t hw[4] = {QH[h].x, QH[h].y, QH[h].z, QH[h].w};
        uint32_t hh[4], ll[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lq = (lw[i] >> (4 * (p & 1))) & 0x0f0f0f0fu;
            const uint32_t hq = ((hw[i] >> (2 * k)) & 0x03030303u) << 4;
            const uint32_t q6 = lq | hq;
            const uint32_t e = __builtin_amdgcn_perm(0u, q6, 0x0c020c00u);   // bytes 0, 2 -> 16-bit lanes
            const uint32_t o = __builtin_amdgcn_perm(0u, q6, 0x0c030c01u);   // bytes 1, 3
            const uint32_t ve = __builtin_bit_cast(uint32_t, (s16x2)(__builtin_bit_cast(s16x2, e) * s2 + c2));
            const uint32_t vo = __builtin_bit_cast(uint32_t, (s16x2)(__builtin_bit_cast(s16x2, o) * s2 + c2));
            hh[i] = __builtin_amdgcn_perm(vo, ve, 0x07030501u);
            ll[i] = __builtin_amdgcn_perm(vo, ve, 0x06020400u) ^ 0x80808080u;
        }
        hp[p] = v4i{(int)hh[0], (int)hh[1], (int)hh[2], (int)hh[3]};
        lp[p] = v4i{(int)ll[0], (int)ll[1], (int)ll[2], (int)ll[3]};
    }
    v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, x.a[0]), hp[0], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
    for (int p = 1; p < 4; p++) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, x.a[p]), hp[p], acc, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] <<= 8;
#pragma unroll
    for (int p = 0; p < 4; p++) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, x.a[p]), lp[p], acc, 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = q6k_value(d, x.dx[j], acc[j]);
}

// After the barrier: thread (token n, row r) merges the chunk sums of each 16-column pass as
// ((c0+c1)+(c2+c3)) (missing chunks +0) and the passes with the pass tree, and stores y.
__device__ __forceinline__ void mv_merge(const float (*part)[16][MV_ROWS], int nchunks, int G, int N, int R, int row0,
                                         float* y, int64_t ldy) {
    const int passes = (G + 15) / 16;
    for (int idx = threadIdx.x; idx < N * MV_ROWS; idx += blockDim.x) {
        const int n = idx / MV_ROWS, r = idx - n * MV_ROWS;
        if (row0 + r >= R) continue;
        PassTree tr;
        tree_init(tr);
        for (int ps = 0; ps < passes; ps++) {
            float c[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int cc = 4 * ps + k;
                c[k] = cc < nchunks ? part[cc][n][r] : 0.0f;
            }
            tree_push(tr, __fadd_rn(__fadd_rn(c[0], c[1]), __fadd_rn(c[2], c[3])));
        }
        y[(int64_t)n * ldy + row0 + r] = tree_final(tr);
    }
}

// ------------------------------------------------------------------ the kernel
// Workgroup: 16 rows of one matrix, one wave per chunk of 4 super-blocks (ceil(G/4) <= 16 waves).
// Load schedule of a wave's chunk: with PRE_ALL every super-block's loads are issued before the
// first is used (four buffers); otherwise two buffers, the next-but-one super-block loaded after
// each one is used.  SB puts a scheduling barrier behind the initial loads, so that the compiler
// cannot move the second super-block's loads behind the first one's arithmetic.  LB is the
// launch bound, which sets the register budget the compiler works to.
template <int TYPE, int LB, bool PRE_ALL, bool SB>
__global__ void __launch_bounds__(LB)
k_gemv_mfma(KQ_MV_HEAD, MvGroup mg) {
    constexpr int BS = TYPE == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    __shared__ float part[16][16][MV_ROWS];            // [chunk][token][row] chunk sums
    const int lane = threadIdx.x & 63;
    const int chunk = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, l16 = lane & 15;

    const int wg = blockIdx.x;
    KQ_MV_PICK(wg, MV_ROWS);
    const int nthr = 64 * ((G + MV_CHUNK - 1) / MV_CHUNK);   // the block: one wave per chunk
    const int nchunks = nthr >> 6;
    int row = row0 + l16;
    row = row < R ? row : R - 1;                       // rows past R are loaded clamped, not stored
    const int64_t col_bytes = 8 * BS;
    const uint8_t* wrow = wm + ((int64_t)(row >> 3) * G * 8 + (row & 7)) * BS;   // + g * col_bytes
    const int64_t xrow = (int64_t)G * Q8K_BYTES;
    const uint8_t* xa = XQ + (int64_t)(l16 < N ? l16 : N - 1) * xrow;
    const uint8_t* xd[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int n = 4 * q + j;
        xd[j] = XQ + (int64_t)(n < N ? n : N - 1) * xrow;
    }

    // the chunk's four super-blocks; columns past G are loaded clamped and contribute +0
    const int g0 = MV_CHUNK * chunk;
    auto wload = [&](int s, MvW<TYPE>& ww) {
        const int g = g0 + s < G ? g0 + s : G - 1;
        mv_load(ww, wrow + (int64_t)g * col_bytes, q);
    };
    auto xload = [&](int s, MvX& xx) {
        const int g = g0 + s < G ? g0 + s : G - 1;
        const uint8_t* xdg[4] = {xd[0] + g * Q8K_BYTES, xd[1] + g * Q8K_BYTES, xd[2] + g * Q8K_BYTES,
                                 xd[3] + g * Q8K_BYTES};
        mv_load_x<TYPE>(xx, xa + (int64_t)g * Q8K_BYTES, xdg, q);
    };
    float v[MV_CHUNK][4];
    auto keep = [&](int s, const float (&vv)[4]) {
        const bool valid = g0 + s < G;
#pragma unroll
        for (int j = 0; j < 4; j++) v[s][j] = valid ? vv[j] : 0.0f;
    };
    if constexpr (PRE_ALL) {
        MvW<TYPE> w[MV_CHUNK];
        MvX x[MV_CHUNK];
#pragma unroll
        for (int s = 0; s < MV_CHUNK; s++) { wload(s, w[s]); xload(s, x[s]); }
        if constexpr (SB) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < MV_CHUNK; s++) {
            float vv[4];
            mv_values(w[s], x[s], q, vv);
            keep(s, vv);
        }
    } else {
        MvW<TYPE> w[2];
        MvX x[2];
        wload(0, w[0]); xload(0, x[0]);
        wload(1, w[1]); xload(1, x[1]);
        if constexpr (SB) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < MV_CHUNK; s++) {
            float vv[4];
            mv_values(w[s & 1], x[s & 1], q, vv);
            keep(s, vv);
            if (s + 2 < MV_CHUNK) { wload(s + 2, w[s & 1]); xload(s + 2, x[s & 1]); }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
        part[chunk][4 * q + j][l16] = __fadd_rn(__fadd_rn(v[0][j], v[1][j]), __fadd_rn(v[2][j], v[3][j]));
    __syncthreads();

    // merge: thread (token n, row r); passes of 4 chunks, missing chunks are +0
    mv_merge(part, nchunks, G, N, R, row0, mv_pick(m, mg.y[0], mg.y[1], mg.y[2]), mv_pick(m, mg.ldy[0], mg.ldy[1], mg.ldy[2]));
}

// ------------------------------------------------------------------ the phase form (no planes)
// Instead of folding the sub-block scales into two weight planes, this form keeps the raw codes
// (Q4_K 0..15, Q6_K 0..63) as the MFMA's B operand and separates 16-element sub-block pieces on the
// A side.  A row a = 4t + p (token t of a group of four, phase p) holds token t's activations in
// K group (p + s) & 3 of step s only and zeros in the other three, so output row 4t + p of a
// K = 64 step is the sum over one 16-element piece alone, and every A lane carries data in exactly
// one step (its 16 bytes are loaded once and selected per step).  Lane l (q = l >> 4) then holds,
// for weight row l & 15 and token 4 gi + q, the four piece sums of each step and applies the
// scales with 24-bit multiply-adds (|piece sum| <= 16 * 128 * 63 < 2^23):
//   Q4_K  K group q of step s = elements 64q + 16s .. +15 (nibble s >> 1 of qs bytes
//         32q + 16(s & 1) + i: the lane's 32 qs bytes, as in the plane form), sub-block 2q + (s >> 1);
//         I1 = sum sc_j * S_j, and I2 from the same exact fp16 MFMA as the plane form.
//   Q6_K  K group q of step s = sub-block j(s, q) = 8(q >> 1) + (q & 1) + 2s: lane q reads ql bytes
//         64h + 16b and 64h + 32 + 16b, qh bytes 32h + 16b and the scales (h = q >> 1, b = q & 1),
//         52 bytes, step s taking nibble s >> 1 of ql word s & 1 and bit pair s of qh;
//         I = sum_j sc_j * S_j - 32 * sum_j sc_j * b_j, the second sum one v_mfma_f32_16x16x16_f16
//         over the Q8_K bsums b_j and the scales (exact small integers: |b_j| <= 2032,
//         |sc_j| <= 128, every partial sum < 2^23).
// The integers are the GEMV's, so the per-super-block values and every row are bit-identical to
// the one-token GEMV.  The unpack is 1.5 (Q4_K) / ~3.3 (Q6_K) VALU per 4 codes instead of ~3.5 /
// ~13 for the planes, and the operands are small enough for all four super-blocks of a wave to be
// in flight at once.  Zero A lanes and the b / B operands of lanes that carry none come from buffer
// loads past the end of the activation buffer, which return zeros.
constexpr int MV_OOB = 0x40000000;   // buffer offset beyond any activation buffer: the load returns 0

__device__ __forceinline__ constexpr int q6p_sub(int s, int q) { return 8 * (q >> 1) + (q & 1) + 2 * s; }

// Raw Q6_K words of one super-block for lane q: ql bytes 64h + 16b and 64h + 32 + 16b, qh bytes
// 128 + 32h + 16b, scales, each 16-byte field with the dword after it (funnel-shifted by sh).
struct MvW6 { u32x4 ql[2], qh, sc; uint32_t qle[2], qhe, sce, sh; };

// The last word read (bytes 208..211 from the aligned base) passes the block end by 2 bytes only
// for blocks starting at 0 (mod 4), which are never row 7 of a tile column.
__device__ __forceinline__ void mv6_load(MvW6& w, const uint8_t* bk, int q) {
    w.sh = uint32_t(reinterpret_cast<uintptr_t>(bk) & 3);
    const uint8_t* b4 = bk - w.sh;
    const int h = q >> 1, b = q & 1;
#pragma unroll
    for (int c = 0; c < 2; c++) {
        w.ql[c] = ld16_a4(b4 + 64 * h + 32 * c + 16 * b);
        w.qle[c] = ld4(b4 + 64 * h + 32 * c + 16 * b + 16);
    }
    w.qh = ld16_a4(b4 + 128 + 32 * h + 16 * b);
    w.qhe = ld4(b4 + 144 + 32 * h + 16 * b);
    w.sc = ld16_a4(b4 + 192);
    w.sce = ld4(b4 + 208);
}

template <int TYPE> struct MvPh;
template <> struct MvPh<TYPE_Q4_K> {
    typedef MvW<TYPE_Q4_K> W;
    typedef u32x4 B;   // bsums 8(q & 1) .. +7 (the min term's sub-blocks 4(q & 1) .. +3)
    static __device__ __forceinline__ int a_off(int q, int p) { return 4 + 64 * q + 16 * ((q - p) & 3); }
    static __device__ __forceinline__ int b_off(int q) { return 260 + 16 * (q & 1); }
    static __device__ __forceinline__ void load(W& w, const uint8_t* bk, int q) { mv_load(w, bk, q); }
};
template <> struct MvPh<TYPE_Q6_K> {
    typedef MvW6 W;
    typedef u32x2 B;   // bsums 4q .. 4q+3
    static __device__ __forceinline__ int a_off(int q, int p) { return 4 + 16 * q6p_sub((q - p) & 3, q); }
    static __device__ __forceinline__ int b_off(int q) { return 260 + 8 * q; }
    static __device__ __forceinline__ void load(W& w, const uint8_t* bk, int q) { mv6_load(w, bk, q); }
};

template <int TYPE, int NG> struct MvXp {
    u32x4 a[NG];                      // token 4 gi + (l & 15) / 4, the piece of its active step
    typename MvPh<TYPE>::B bs[NG];    // bsums of token 4 gi + (l & 15) / 4 where l & 3 == 0; else 0
    float dx[NG];                     // d of token 4 gi + q
};

__device__ __forceinline__ v4i byte_pieces(const u32x4& v, int shift) {
    return v4i{(int)((v.x >> shift) & 0x0f0f0f0fu), (int)((v.y >> shift) & 0x0f0f0f0fu),
               (int)((v.z >> shift) & 0x0f0f0f0fu), (int)((v.w >> shift) & 0x0f0f0f0fu)};
}

template <int NG>
__device__ __forceinline__ void mvp_values(const MvW<TYPE_Q4_K>& w, const MvXp<TYPE_Q4_K, NG>& x, int q, int p,
                                           float (&v)[NG]) {
    const uint32_t s0 = w.hdr.y, s1 = w.hdr.z, s2 = w.hdr.w;
    // the eight 6-bit scales (bytes of sca: sub-blocks 0..3, of scb: 4..7) and mins (q4kernels.h:17-18)
    const uint32_t sca = s0 & 0x3f3f3f3fu, scb = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
    const uint32_t ma = s1 & 0x3f3f3f3fu, mb = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
    const v4i bq[4] = {byte_pieces(w.qa, 0), byte_pieces(w.qb, 0), byte_pieces(w.qa, 4), byte_pieces(w.qb, 4)};
    // min term, as the plane form: K slots 4q .. 4q+3 = sub-blocks 4(q & 1) .. +3, the high (q < 2) or
    // low part of B against -64 m or -m
    const uint32_t mw = (q & 1) ? mb : ma;
    const float f = (q >> 1) ? -1.0f : -64.0f;
    const v4h bm = __builtin_bit_cast(v4h, u32x2{mv_pk_f16(f * (float)byte_of(mw, 0), f * (float)byte_of(mw, 1)),
                                                 mv_pk_f16(f * (float)byte_of(mw, 2), f * (float)byte_of(mw, 3))});
    const v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (int gi = 0; gi < NG; gi++) {
        const v4i xa = __builtin_bit_cast(v4i, x.a[gi]);
        int I1 = 0;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const v4i a = ((p + s) & 3) == q ? xa : zero;
            const v4i S = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bq[s], zero, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++) {          // output row 4q + r: K group (r + s) & 3, sub-block 2k + (s >> 1)
                const int j = 2 * ((r + s) & 3) + (s >> 1);
                I1 += (int)byte_of(j < 4 ? sca : scb, j & 3) * ((S[r] << 8) >> 8);   // 24-bit operands
            }
        }
        const uint32_t bw[4] = {x.bs[gi].x, x.bs[gi].y, x.bs[gi].z, x.bs[gi].w};
        float B[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int sb = shalf(bw[k], 0) + shalf(bw[k], 1);
            B[k] = (float)((q >> 1) ? (sb & 63) : (sb >> 6));
        }
        const v4h am = __builtin_bit_cast(v4h, u32x2{mv_pk_f16(B[0], B[1]), mv_pk_f16(B[2], B[3])});
        const v4f cm = __builtin_amdgcn_mfma_f32_16x16x16f16(am, bm, v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);   // -I2
        v[gi] = q4k_value(w.hdr.x, x.dx[gi], I1, (int)(-cm[0]));
    }
}

template <int NG>
__device__ __forceinline__ void mvp_values(const MvW6& w, const MvXp<TYPE_Q6_K, NG>& x, int q, int p, float (&v)[NG]) {
    const uint32_t sh = w.sh;
    const u32x4 QL[2] = {mv_funnel(w.ql[0], w.qle[0], sh), mv_funnel(w.ql[1], w.qle[1], sh)};
    const u32x4 QH = mv_funnel(w.qh, w.qhe, sh);
    const u32x4 SC = mv_funnel(w.sc, w.sce, sh);   // scale of sub-block j = byte j & 3 of dword j >> 2
    const float d = f16_lo(w.sce >> (8 * sh));
    const uint32_t hw[4] = {QH.x, QH.y, QH.z, QH.w};
    v4i bq[4];   // B of step s: codes of sub-block j(s, q), 6-bit, as bytes
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const u32x4 L = QL[s & 1];
        const uint32_t lw[4] = {L.x, L.y, L.z, L.w};
        uint32_t c[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t lq = (lw[i] >> (4 * (s >> 1))) & 0x0f0f0f0fu;
            const uint32_t hq = s < 2 ? hw[i] << (4 - 2 * s) : hw[i] >> (2 * s - 4);   // bit pair s to bits 4..5
            c[i] = (hq & 0x30303030u) | lq;
        }
        bq[s] = v4i{(int)c[0], (int)c[1], (int)c[2], (int)c[3]};
    }
    // B of the b term: scales of sub-blocks 4q .. 4q+3 as fp16
    const uint32_t scq = q == 0 ? SC.x : q == 1 ? SC.y : q == 2 ? SC.z : SC.w;
    const v4h bsc = __builtin_bit_cast(v4h, u32x2{mv_pk_f16((float)sbyte(scq, 0), (float)sbyte(scq, 1)),
                                                  mv_pk_f16((float)sbyte(scq, 2), (float)sbyte(scq, 3))});
    const uint32_t scw[4] = {SC.x, SC.y, SC.z, SC.w};
    const v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (int gi = 0; gi < NG; gi++) {
        const v4i xa = __builtin_bit_cast(v4i, x.a[gi]);
        int I = 0;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const v4i a = ((p + s) & 3) == q ? xa : zero;    // this lane's phase owns K group q at step s
            const v4i S = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bq[s], zero, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++) {          // output row 4q + r: phase r, sub-block j(s, (r + s) & 3)
                const int j = q6p_sub(s, (r + s) & 3);
                I += sbyte(scw[j >> 2], j & 3) * ((S[r] << 8) >> 8);   // 24-bit operands
            }
        }
        const uint32_t b0 = x.bs[gi].x, b1 = x.bs[gi].y;
        const v4h bb = __builtin_bit_cast(v4h, u32x2{mv_pk_f16((float)shalf(b0, 0), (float)shalf(b0, 1)),
                                                     mv_pk_f16((float)shalf(b1, 0), (float)shalf(b1, 1))});
        const v4f cb = __builtin_amdgcn_mfma_f32_16x16x16f16(bb, bsc, v4f{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        v[gi] = q6k_value(d, x.dx[gi], I - 32 * (int)cb[0]);
    }
}

__device__ __forceinline__ u32x4 buf_ld16(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ void buf_ld(u32x4& v, __amdgpu_buffer_rsrc_t r, int off) { v = buf_ld16(r, off); }
__device__ __forceinline__ void buf_ld(u32x2& v, __amdgpu_buffer_rsrc_t r, int off) {
    v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}

// Workgroup and merge as k_gemv_mfma; NG groups of four tokens (N <= 4 NG) share each unpack; FP of
// the wave's four super-blocks are in flight before the first is used.
template <int TYPE, int NG, int LB, int FP>
__global__ void __launch_bounds__(LB)
k_gemv_mfma_ph(KQ_MV_HEAD, MvGroup mg) {
    typedef MvPh<TYPE> Ph;
    constexpr int BS = TYPE == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    __shared__ float part[16][16][MV_ROWS];            // [chunk][token][row] chunk sums
    const int lane = threadIdx.x & 63;
    const int chunk = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, l16 = lane & 15;

    const int wg = blockIdx.x;
    KQ_MV_PICK(wg, MV_ROWS);
    const int nthr = 64 * ((G + MV_CHUNK - 1) / MV_CHUNK);   // the block: one wave per chunk
    const int nchunks = nthr >> 6;
    int row = row0 + l16;
    row = row < R ? row : R - 1;                       // rows past R are loaded clamped, not stored
    const int64_t col_bytes = 8 * BS;
    const uint8_t* wrow = wm + ((int64_t)(row >> 3) * G * 8 + (row & 7)) * BS;   // + g * col_bytes
    const int xrow = G * Q8K_BYTES;
    // raw buffer over the N activation rows: stride 0, N * xrow bytes (loads past them return 0), and
    // the gfx9 descriptor word 3 (32-bit data format)
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(XQ), 0, N * xrow, 0x00020000);
    const int t = l16 >> 2, p = lane & 3;
    int aoff[NG], boff[NG];
    const uint8_t* xd[NG];
#pragma unroll
    for (int gi = 0; gi < NG; gi++) {
        const int tok = 4 * gi + t;
        aoff[gi] = tok < N ? tok * xrow + Ph::a_off(q, p) : MV_OOB;
        boff[gi] = p == 0 && tok < N ? tok * xrow + Ph::b_off(q) : MV_OOB;
        const int n = 4 * gi + q;
        xd[gi] = XQ + (int64_t)(n < N ? n : N - 1) * xrow;
    }

    const int g0 = MV_CHUNK * chunk;
    auto load = [&](int s, typename Ph::W& ww, MvXp<TYPE, NG>& xx) {
        const int g = g0 + s < G ? g0 + s : G - 1;
        Ph::load(ww, wrow + (int64_t)g * col_bytes, q);
        const int go = g * Q8K_BYTES;
#pragma unroll
        for (int gi = 0; gi < NG; gi++) {
            xx.a[gi] = buf_ld16(xr, aoff[gi] + go);
            buf_ld(xx.bs[gi], xr, boff[gi] + go);
            xx.dx[gi] = __builtin_bit_cast(float, ld4(xd[gi] + go));
        }
    };
    float v[MV_CHUNK][NG];
    typename Ph::W w[FP];
    MvXp<TYPE, NG> x[FP];
#pragma unroll
    for (int s = 0; s < FP; s++) load(s, w[s], x[s]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < MV_CHUNK; s++) {
        float vv[NG];
        mvp_values<NG>(w[s % FP], x[s % FP], q, p, vv);
        const bool valid = g0 + s < G;          // columns past G contribute +0
#pragma unroll
        for (int gi = 0; gi < NG; gi++) v[s][gi] = valid ? vv[gi] : 0.0f;
        if (s + FP < MV_CHUNK) load(s + FP, w[s % FP], x[s % FP]);
    }
#pragma unroll
    for (int gi = 0; gi < NG; gi++)
        part[chunk][4 * gi + q][l16] = __fadd_rn(__fadd_rn(v[0][gi], v[1][gi]), __fadd_rn(v[2][gi], v[3][gi]));
    __syncthreads();

    mv_merge(part, nchunks, G, N, R, row0, mv_pick(m, mg.y[0], mg.y[1], mg.y[2]), mv_pick(m, mg.ldy[0], mg.ldy[1], mg.ldy[2]));
}

// ------------------------------------------------------------------ two row groups per wave
// The plane form with each wave on two 16-row groups x two super-blocks (a "piece": half a chunk)
// instead of one group x four: the same waves and MFMAs, but each activation operand (16 tokens x 256
// bytes per super-block, more than the weights it meets from 5 tokens on) is loaded once for 32 rows,
// so a launch loads half the activation bytes.  A workgroup holds 32 rows and every piece of them
// (ceil(G/2) <= 16 waves, so G <= 32); each wave adds its two super-block values (v0 + v1) or (v2 + v3)
// and the merge forms each chunk as (v0 + v1) + (v2 + v3) before the pass tree, so every output is the
// one k_gemv_mfma (and the one-token GEMV) gives.
constexpr int MV_ROWS2 = 32;    // weight rows per workgroup of the two-group form

template <int TYPE, int LB>
__global__ void __launch_bounds__(LB)
k_gemv_mfma_rg(KQ_MV_HEAD, MvGroup mg) {
    constexpr int BS = TYPE == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    __shared__ float part[16][16][MV_ROWS2];           // [piece][token][row] piece sums
    const int lane = threadIdx.x & 63;
    const int piece = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, l16 = lane & 15;

    const int wg = blockIdx.x;
    KQ_MV_PICK(wg, MV_ROWS2);
    const int nthr = 64 * ((G + 1) / 2);                     // the block: one wave per piece
    const int npieces = nthr >> 6;
    const int64_t col_bytes = 8 * BS;
    const uint8_t* wrow[2];
#pragma unroll
    for (int rg = 0; rg < 2; rg++) {
        int row = row0 + 16 * rg + l16;
        row = row < R ? row : R - 1;                   // rows past R are loaded clamped, not stored
        wrow[rg] = wm + ((int64_t)(row >> 3) * G * 8 + (row & 7)) * BS;   // + g * col_bytes
    }
    const int64_t xrow = (int64_t)G * Q8K_BYTES;
    const uint8_t* xa = XQ + (int64_t)(l16 < N ? l16 : N - 1) * xrow;
    const uint8_t* xd[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int n = 4 * q + j;
        xd[j] = XQ + (int64_t)(n < N ? n : N - 1) * xrow;
    }

    // the piece's two super-blocks, every load issued before the first is used; columns past G are
    // loaded clamped and contribute +0
    const int g0 = 2 * piece;
    MvW<TYPE> w[2][2];
    MvX x[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const int g = g0 + s < G ? g0 + s : G - 1;
#pragma unroll
        for (int rg = 0; rg < 2; rg++) mv_load(w[s][rg], wrow[rg] + (int64_t)g * col_bytes, q);
        const uint8_t* xdg[4] = {xd[0] + g * Q8K_BYTES, xd[1] + g * Q8K_BYTES, xd[2] + g * Q8K_BYTES,
                                 xd[3] + g * Q8K_BYTES};
        mv_load_x<TYPE>(x[s], xa + (int64_t)g * Q8K_BYTES, xdg, q);
    }
    __builtin_amdgcn_sched_barrier(0);
    float v[2][2][4];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const bool valid = g0 + s < G;
#pragma unroll
        for (int rg = 0; rg < 2; rg++) {
            float vv[4];
            mv_values(w[s][rg], x[s], q, vv);
#pragma unroll
            for (int j = 0; j < 4; j++) v[rg][s][j] = valid ? vv[j] : 0.0f;
        }
    }
#pragma unroll
    for (int rg = 0; rg < 2; rg++)
#pragma unroll
        for (int j = 0; j < 4; j++) part[piece][4 * q + j][16 * rg + l16] = __fadd_rn(v[rg][0][j], v[rg][1][j]);
    __syncthreads();

    // merge: thread (token n, row r); chunk c = pieces 2c, 2c + 1, passes of 4 chunks, missing ones +0
    const int passes = (G + 15) / 16;
    float* const y = mv_pick(m, mg.y[0], mg.y[1], mg.y[2]);
    const int64_t ldy = mv_pick(m, mg.ldy[0], mg.ldy[1], mg.ldy[2]);
    for (int idx = threadIdx.x; idx < N * MV_ROWS2; idx += nthr) {
        const int n = idx / MV_ROWS2, r = idx - n * MV_ROWS2;
        if (row0 + r >= R) continue;
        PassTree tr;
        tree_init(tr);
        for (int ps = 0; ps < passes; ps++) {
            float c[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int p0 = 2 * (4 * ps + k);
                const float a = p0 < npieces ? part[p0][n][r] : 0.0f;
                const float b = p0 + 1 < npieces ? part[p0 + 1][n][r] : 0.0f;
                c[k] = __fadd_rn(a, b);
            }
            tree_push(tr, __fadd_rn(__fadd_rn(c[0], c[1]), __fadd_rn(c[2], c[3])));
        }
        y[(int64_t)n * ldy + row0 + r] = tree_final(tr);
    }
}

// The leading arguments of the MFMA kernels (KQ_MV_HEAD) from a group; the workgroup counts fit 16
// bits (the dispatcher sends at most 65535 row groups to these forms).
#define MV_HEAD_ARGS(g) (g).w[0], (g).w[1], (g).w[2], xq, (g).R[0], (g).R[1], (g).R[2], (g).first[1] | (g).first[2] << 16, N | G << 8

template <int TYPE, int LB, bool PRE_ALL, bool SB>
static void launch_mv(const MvGroup& mg, int wgs, const uint8_t* xq, int N, int G, hipStream_t s) {
    const int nchunks = (G + MV_CHUNK - 1) / MV_CHUNK;
    hipLaunchKernelGGL((k_gemv_mfma<TYPE, LB, PRE_ALL, SB>), dim3(wgs), dim3(64 * nchunks), 0, s, MV_HEAD_ARGS(mg),
                       mg);
}

// n (1..3) matrices of one type, N = 1..16 tokens, C <= 16384 (at most 16 chunks of 4 columns).
// Schedules by shape, each the fastest measured for its case (12288x4096 and 4096x12288 Q4_K,
// 4096x12288 and 1024x4096 Q6_K; N = 3..16):
//   Q4_K up to 4 tokens and 48 super-blocks: the phase form, all four super-blocks in flight
//   (12288x4096 at N = 2 / 4: plane form 10.2 / 10.0 -> 8.0 / 8.2 us; at 5..8 tokens the plane form
//   stays faster, 9.9 / 10.6 against 10.3 / 10.8 us);
//   Q6_K up to 8 tokens and 48 super-blocks: the phase form, all four super-blocks in flight for
//   up to 4 tokens, two for 5..8 (4096x12288 at N = 3 / 4 / 5 / 8: 15.3 / 15.3 / 15.3 / 16.1 ->
//   12.7 / 12.8 / 14.0 / 14.4 us; 4096x4096 at N = 4: 7.0 -> 5.9 us);
//   otherwise the plane form: with G <= 32 (Q4_K) or G <= 16 (Q6_K) two row groups per wave
//   (k_gemv_mfma_rg: 12288x4096 Q4_K at N = 16 13.9-14.1 -> 12.8 us, N = 8 unchanged); beyond, Q4_K
//   with G <= 16 all four super-blocks in flight (3 waves per SIMD), else two in flight, behind the
//   barrier.
void launch_gemv_mfma_group(int n, const uint8_t* const* w, const int* R, int C, int type, const uint8_t* xq,
                            int N, float* const* y, const int64_t* ldy, hipStream_t s) {
    const int G = C / QK;
    MvGroup mg{};
    int wgs = 0;
    for (int i = 0; i < n; i++) {
        mg.w[i] = w[i];
        mg.y[i] = y[i];
        mg.ldy[i] = ldy[i];
        mg.R[i] = R[i];
        mg.first[i] = wgs;
        wgs += (R[i] + MV_ROWS - 1) / MV_ROWS;
    }
    for (int i = n; i < 4; i++) mg.first[i] = wgs;
    const int nchunks = (G + MV_CHUNK - 1) / MV_CHUNK;
    const dim3 grid(wgs), block(64 * nchunks);
    // the phase form up to 8 tokens and 48 super-blocks: beyond 8 tokens (three or four token groups)
    // it needs more registers than 3 waves per SIMD leave and spills, beyond 48 super-blocks a
    // workgroup has 16 waves, 4 per SIMD (128 registers: spills too)
    const bool ph = G <= 48 && N <= 8 && (type == TYPE_Q4_K ? N <= KQ_GEMV_MFMA_Q4_PH_MAX : !KQ_GEMV_MFMA_Q6_PLANES);
    if (ph && type == TYPE_Q4_K) {
        if (N <= 4) hipLaunchKernelGGL((k_gemv_mfma_ph<TYPE_Q4_K, 1, 768, KQ_Q4P_FP1>), grid, block, 0, s, MV_HEAD_ARGS(mg), mg);
        else hipLaunchKernelGGL((k_gemv_mfma_ph<TYPE_Q4_K, 2, 768, KQ_Q4P_FP2>), grid, block, 0, s, MV_HEAD_ARGS(mg), mg);
    } else if (ph) {
        if (N <= 4) hipLaunchKernelGGL((k_gemv_mfma_ph<TYPE_Q6_K, 1, 768, KQ_Q6P_FP1>), grid, block, 0, s, MV_HEAD_ARGS(mg), mg);
        else hipLaunchKernelGGL((k_gemv_mfma_ph<TYPE_Q6_K, 2, 768, KQ_Q6P_FP2>), grid, block, 0, s, MV_HEAD_ARGS(mg), mg);
    } else if (KQ_GEMV_MFMA_RG && G <= (type == TYPE_Q4_K ? 32 : 16)) {
        // two row groups per wave: workgroups of 32 rows (Q6_K beyond 16 super-blocks, 4 waves per SIMD,
        // would spill)
        MvGroup mg2 = mg;
        int wgs2 = 0;
        for (int i = 0; i < n; i++) {
            mg2.first[i] = wgs2;
            wgs2 += (R[i] + MV_ROWS2 - 1) / MV_ROWS2;
        }
        for (int i = n; i < 4; i++) mg2.first[i] = wgs2;
        const dim3 block2(64 * ((G + 1) / 2));
        if (type == TYPE_Q4_K) {
            if (G <= 16) hipLaunchKernelGGL((k_gemv_mfma_rg<TYPE_Q4_K, 512>), dim3(wgs2), block2, 0, s, MV_HEAD_ARGS(mg2), mg2);
            else hipLaunchKernelGGL((k_gemv_mfma_rg<TYPE_Q4_K, 1024>), dim3(wgs2), block2, 0, s, MV_HEAD_ARGS(mg2), mg2);
        } else {
            hipLaunchKernelGGL((k_gemv_mfma_rg<TYPE_Q6_K, 512>), dim3(wgs2), block2, 0, s, MV_HEAD_ARGS(mg2), mg2);
        }
    } else if (type == TYPE_Q4_K) {
        if (G <= 16) launch_mv<TYPE_Q4_K, 256, true, true>(mg, wgs, xq, N, G, s);
        else if (G <= 48) launch_mv<TYPE_Q4_K, 768, false, true>(mg, wgs, xq, N, G, s);
        else launch_mv<TYPE_Q4_K, 1024, false, true>(mg, wgs, xq, N, G, s);
    } else {
        launch_mv<TYPE_Q6_K, 1024, false, true>(mg, wgs, xq, N, G, s);
    }
}

}  // namespace kq
