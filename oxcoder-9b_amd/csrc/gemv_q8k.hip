// Q4_K / Q6_K x Q8_K GEMV for gfx950 (batch-1 decode and small-batch speculative verify).
//
// Work unit: RPW consecutive rows of one 8-row tile of one matrix.  Up to three matrices that
// share the activation (q/k/v, gate/up) are one launch: their units are numbered back to back.
// The grid is sized to the chip (KQ_GEMV_WAVES_PER_CU waves per CU, fewer if there are fewer
// units) and each wave walks its units in increasing order, the waves of one workgroup sharing
// whole 8-row tiles (TileWalk); while it computes one
// (unit, column pass) it already has the loads of the next one in flight, so weight streaming
// and the dot/reduce work of a wave overlap instead of alternating.
//
// Lanes: slot = lane >> 2 walks super-block columns g = slot + 16*pass, part = lane & 3 owns a
// quarter of the super-block (q4_lanes.h).  Per row a Q4_K lane reads the 16-B block header and
// 32 quant bytes (a tile column is 9 cache lines, each read once); a Q6_K lane reads 48 quant
// bytes plus scales and d with dword-aligned funnel-shifted loads.  Per (row, super-block) the
// four lanes' int32 partials are summed exactly, turned into one fp32 value and reduced by the
// column tree of q4_lanes.h, so the result does not depend on NT, RPW or grid shape.
#include <type_traits>

#include "kq_device.h"
#include "kq_internal.h"
#include "q4_lanes.h"
#include "argmax_block.h"
#include "q8k_block.h"

#ifndef KQ_GEMV_WAVES_PER_CU
#define KQ_GEMV_WAVES_PER_CU 8
#endif
#ifndef KQ_GEMV_WAVES_PER_CU_Q6
#define KQ_GEMV_WAVES_PER_CU_Q6 KQ_GEMV_WAVES_PER_CU
#endif
#ifndef KQ_GEMV_WAVES_PER_CU_NT2
#define KQ_GEMV_WAVES_PER_CU_NT2 KQ_GEMV_WAVES_PER_CU   // Q4_K, two tokens per launch
#endif
#ifndef KQ_GEMV_WAVES_PER_CU_F32
#define KQ_GEMV_WAVES_PER_CU_F32 KQ_GEMV_WAVES_PER_CU   // fp32 activations
#endif
#ifndef KQ_GEMV_WAVES_PER_CU_F32_Q6
#define KQ_GEMV_WAVES_PER_CU_F32_Q6 KQ_GEMV_WAVES_PER_CU_Q6
#endif
// Q6_K on the sequential kernel: one workgroup of 4 waves per CU, one wave per SIMD, each wave
// walking more units (4096x12288 at one token: 4 units per wave, 10.9 us against 11.6 us at 8
// waves per CU; two tokens 12.8 against 13.9 us; 2, 3, 5 or 6 waves per CU and workgroups of 1
// or 2 waves were slower).
#ifndef KQ_GEMV_WAVES_PER_CU_SEQ_Q6
#define KQ_GEMV_WAVES_PER_CU_SEQ_Q6 4
#endif
#ifndef KQ_GEMV_SEQ_DEPTH
#define KQ_GEMV_SEQ_DEPTH 2      // (unit, pass) steps in flight per wave, three-pass kernel, one token
#endif
#ifndef KQ_GEMV_SEQ_WPB
#define KQ_GEMV_SEQ_WPB 4        // waves per workgroup of the sequential kernel
#endif
#ifndef KQ_GEMV_SPLIT_WFIRST
#define KQ_GEMV_SPLIT_WFIRST 1   // pass-split kernel: the first unit's weights issued before the activations
#endif
#ifndef KQ_GEMV_SPLIT_MAX
#define KQ_GEMV_SPLIT_MAX 4      // most column passes handled by the pass-split kernel (Q4_K)
#endif
#ifndef KQ_XF_XFIRST
#define KQ_XF_XFIRST 1           // in-launch quantization: x's loads before the first unit's weights
#endif
#ifndef KQ_GEMV_SPLIT_MAX_Q6
#define KQ_GEMV_SPLIT_MAX_Q6 2   // Q6_K, 1-2 tokens: 3-4 passes run faster as sequential passes (measured)
#endif
#ifndef KQ_GEMV_WG_WAVES
#define KQ_GEMV_WG_WAVES 4
#endif
#ifndef KQ_GEMV_P3
#define KQ_GEMV_P3 1       // three-pass matrices (C = 8448..12288) keep every pass's activations in registers
#endif
#ifndef KQ_XCDS
#define KQ_XCDS 8          // accelerator complex dies per MI355X; workgroups alternate between them
#endif
#ifndef KQ_GEMV_TILE_WG
#define KQ_GEMV_TILE_WG 1  // every 8-row tile is walked by the waves of one workgroup (see TileWalk)
#endif

namespace kq {

struct MatGroup {
    const uint8_t* w[3];
    float* y[3];
    int64_t ldy[3];
    int first_unit[4];   // units of matrix m are [first_unit[m], first_unit[m+1])
    int n;
};

// Kernel arguments.  The GEMV kernels take first, as plain scalars, what their prologue needs: the
// three matrices' weights, the activations, G, the unit count, the first units of matrices 1 and 2,
// the grid size and one more count, 14 dwords that the dispatch preloads into scalar registers
// (-amdgpu-kernarg-preload-count; on firmware that does not preload, the code object's compatibility
// prologue loads them in one batch).  The matrix table follows for the loop's later units and the
// outputs.  The prologue picks the first unit's matrix by selects, not by an indexed load that would
// wait for m.  (Left to the compiler with the table first, the prologue made three or four dependent
// round trips of ~0.3 us to the kernel arguments before its first weight load: a per-wave timeline of
// the 4096x12288 Q6_K GEMV read its arguments 0.9 us after the wave's first instruction.)
#define KQ_GEMV_HEAD                                                                                  \
    const uint8_t* __restrict__ w0, const uint8_t* __restrict__ w1, const uint8_t* __restrict__ w2,   \
        const uint8_t* __restrict__ XQ, int G, int total_units, int f1, int f2, int ngrid
#define KQ_GEMV_PICK                                                                                  \
    auto mat_of = [&](int u) { return u >= f1 ? (u >= f2 ? 2 : 1) : 0; };                             \
    auto first_of = [&](int m) { return m == 0 ? 0 : m == 1 ? f1 : f2; };                             \
    auto w_of = [&](int m) { return m == 0 ? w0 : m == 1 ? w1 : w2; }

// Unit order of a wave (stream s of S streams in workgroup b of nwg; units of one 8-row tile:
// WPT).  With S >= WPT the streams of a workgroup hold whole tiles when numbered consecutively:
// unit = b*S + s + k*nwg*S.  With S < WPT (one-row Q6_K units over 4 streams, or several column
// passes per stream) the workgroup takes tiles b, b + nwg, ... and stream s walks units s, s + S,
// ... of each, so a tile's rows, whose 144- or 210-byte blocks share 128-byte lines with their
// neighbours', are read through the L2 of one XCD instead of two (the 4096x12288 Q6_K down and the
// 151936x4096 Q6_K head fetched 12 % more than their bytes from HBM with the tiles split).  TM =
// false keeps the consecutive numbering: the sequential kernel's Q6_K down projection measured
// 11.7 us with it and 12.2 us tile-major; the pass-split kernel gained from it (Q4_K two tokens
// 12288x4096 10.0 -> 9.5 us, the fused 248320x4096 head 113 -> 105 us; the Q6_K head unchanged).
template <int WPT, bool TM = true> struct TileWalk {
    int b, nwg, s, S;
    __device__ __forceinline__ bool tile_major() const { return TM && KQ_GEMV_TILE_WG && S < WPT; }
    __device__ __forceinline__ int first() const { return tile_major() ? b * WPT + s : b * S + s; }
    __device__ __forceinline__ int next(int u) const {
        if (!tile_major()) return u + nwg * S;
        return (u % WPT) + S < WPT ? u + S : u + nwg * WPT + S - WPT;
    }
    // the k-th unit of the stream, and how many units it walks in all
    __device__ __forceinline__ int unit(int k) const {
        if (!tile_major()) return b * S + s + k * nwg * S;
        const int per = WPT / S;
        return (b + (k / per) * nwg) * WPT + s + (k % per) * S;
    }
    __device__ __forceinline__ int count(int total_units) const {
        if (!tile_major()) {
            const int u0 = b * S + s;
            return u0 < total_units ? (total_units - u0 + nwg * S - 1) / (nwg * S) : 0;
        }
        const int tiles = total_units / WPT;
        return b < tiles ? ((tiles - b - 1) / nwg + 1) * (WPT / S) : 0;
    }
};

// ------------------------------------------------------------------ per-type fragments
template <int TYPE> struct Frag;
template <> struct Frag<TYPE_Q4_K> { u32x4 hdr, qa, qb; };
// Q6_K fields sit at block offset + (block start & 3): a lane multiplies its dword-aligned words
// (each 16-B field + the following dword), the scales and d, funnel-shifted by the byte shift in
// block_value.  A lane loads its three 16-B quant fields and the quad's common 16-B scale field
// and d dword (5 loads); the dword after each quant field is the first dword of a field another
// lane of the quad holds, and comes from it by a quad permutation (prepare).
struct Q6Fields { u32x4 l0, l1, hb; uint32_t l0e, l1e, hbe; u32x2 sc; uint32_t sce, dw, sh; };
template <> struct Frag<TYPE_Q6_K> { u32x4 l0, l1, hb, sc4; uint32_t dw, sh; };

template <int TYPE> struct Act;
template <> struct Act<TYPE_Q4_K> { uint32_t xl[8], xh[8]; int blo, bhi; float dx; };
template <> struct Act<TYPE_Q6_K> { uint32_t xa[16]; int corr[4]; float dx; };

// bk = first byte of this row's block; p = part.
__device__ __forceinline__ void load_frag(Frag<TYPE_Q4_K>& f, const uint8_t* bk, int p) {
    f.hdr = ld16(bk);
    f.qa = ld16(bk + 16 + 32 * p);
    f.qb = ld16(bk + 32 + 32 * p);
}
// Q6_K reads stay inside the row's 8-row tile column: quant fields end at byte 192 of the block,
// the scale window [192 + 8h, 200 + 8h) and d [208, 210) are read from the dword-aligned address
// at or below them; for even rows (block start = 0 mod 4) the last word read reaches 2 bytes
// into the next row's block, which exists because row 7 of a tile is odd.
__device__ __forceinline__ void load_frag(Frag<TYPE_Q6_K>& f, const uint8_t* bk, int p) {
    const int h = p >> 1, jj = p & 1;
    // pointer arithmetic (not an integer round trip) keeps the global address space
    f.sh = uint32_t(reinterpret_cast<uintptr_t>(bk) & 3);   // the same shift for every field
    const uint8_t* b4 = bk - f.sh;
    f.l0 = ld16_a4(b4 + h * 64 + 16 * jj);          // ql bytes 64h + 16jj ..
    f.l1 = ld16_a4(b4 + h * 64 + 32 + 16 * jj);     // ql bytes 64h + 32 + 16jj ..
    f.hb = ld16_a4(b4 + 128 + h * 32 + 16 * jj);    // qh bytes 32h + 16jj ..
    f.sc4 = ld16_a4(b4 + 192);                      // the 16 scales
    f.dw = ld4(b4 + 208);                           // d
}
// The fields a lane multiplies.  Quad lane p = 2h + jj holds the 16-B chunks at block offsets
// (relative to the dword-aligned start) l0: 64h + 16jj, l1: 64h + 32 + 16jj, hb: 128 + 32h + 16jj,
// so the dword following
//   l0 of p = 0, 1, 2, 3 (offsets 16, 32, 80, 96) is l0.x of lane 1, l1.x of lane 0, l0.x of lane 3, l1.x of lane 2;
//   l1 (offsets 48, 64, 112, 128) is l1.x of lane 1, l0.x of lane 2, l1.x of lane 3, hb.x of lane 0;
//   hb (offsets 144, 160, 176, 192) is hb.x of lanes 1, 2, 3 and, for p = 3, the first scale dword.
// Lane-dependent choice between two words as a bit select.
__device__ __forceinline__ uint32_t pick(bool c, uint32_t a, uint32_t b) {
    const uint32_t m = 0u - (uint32_t)c;
    return (a & m) | (b & ~m);
}
// SEL: the lane-dependent choices as bit selects.  Written as conditional expressions the compiler
// turns them into divergent branches with exec-mask bookkeeping; the bit selects measured faster
// in the pass-split kernel (1024x4096 Q6_K 4.03 -> 3.77 us) and for two tokens (4096x12288 Q6_K
// 12.6 -> 11.8 us), slower in the one-token three-pass kernel (10.6 -> 11.2 us, with earlier waits
// on the weight loads in flight), which keeps the branches.  The fields are the same either way.
template <bool SEL = true>
__device__ __forceinline__ Q6Fields prepare(const Frag<TYPE_Q6_K>& f, int p) {
    constexpr int QUAD_ROT1 = 0x39;   // quad_perm [1,2,3,0]: lane i <- lane (i + 1) & 3
    const int h = p >> 1, jj = p & 1;
    Q6Fields q;
    q.l0 = f.l0; q.l1 = f.l1; q.hb = f.hb; q.dw = f.dw; q.sh = f.sh;
    if constexpr (SEL) {
        q.l0e = (uint32_t)dpp<DPP_QUAD_XOR1>((int)pick(jj, f.l0.x, f.l1.x));
        q.l1e = (uint32_t)dpp<QUAD_ROT1>((int)pick(p == 0, f.hb.x, pick(p == 2, f.l0.x, f.l1.x)));
        const uint32_t hn = (uint32_t)dpp<QUAD_ROT1>((int)f.hb.x);
        q.hbe = pick(p == 3, f.sc4.x, hn);
        q.sc = u32x2{pick(h, f.sc4.z, f.sc4.x), pick(h, f.sc4.w, f.sc4.y)};   // scales 8h .. 8h+7
        q.sce = pick(h, f.dw, f.sc4.z);                                       // the dword after them
    } else {
        q.l0e = (uint32_t)dpp<DPP_QUAD_XOR1>((int)(jj ? f.l0.x : f.l1.x));
        q.l1e = (uint32_t)dpp<QUAD_ROT1>((int)(p == 0 ? f.hb.x : (p == 2 ? f.l0.x : f.l1.x)));
        const uint32_t hn = (uint32_t)dpp<QUAD_ROT1>((int)f.hb.x);
        q.hbe = p == 3 ? f.sc4.x : hn;
        q.sc = h ? u32x2{f.sc4.z, f.sc4.w} : u32x2{f.sc4.x, f.sc4.y};
        q.sce = h ? f.dw : f.sc4.z;
    }
    return q;
}
template <bool SEL = true>
__device__ __forceinline__ const Frag<TYPE_Q4_K>& prepare(const Frag<TYPE_Q4_K>& f, int) { return f; }
__device__ __forceinline__ u32x4 funnel(const u32x4& v, uint32_t e, uint32_t sh) {
    u32x4 r;
    r.x = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
    r.y = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
    r.z = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
    r.w = __builtin_amdgcn_alignbyte(e, v.w, sh);
    return r;
}

// xb = first byte of the Q8_K block of column g for one token.
__device__ __forceinline__ void load_act(Act<TYPE_Q4_K>& a, const uint8_t* xb, int p) {
    a.dx = __builtin_bit_cast(float, ld4(xb));
    const u32x4 a0 = ld16_a4(xb + 4 + 64 * p), a1 = ld16_a4(xb + 20 + 64 * p);
    const u32x4 a2 = ld16_a4(xb + 36 + 64 * p), a3 = ld16_a4(xb + 52 + 64 * p);
    a.xl[0] = a0.x; a.xl[1] = a0.y; a.xl[2] = a0.z; a.xl[3] = a0.w;
    a.xl[4] = a1.x; a.xl[5] = a1.y; a.xl[6] = a1.z; a.xl[7] = a1.w;
    a.xh[0] = a2.x; a.xh[1] = a2.y; a.xh[2] = a2.z; a.xh[3] = a2.w;
    a.xh[4] = a3.x; a.xh[5] = a3.y; a.xh[6] = a3.z; a.xh[7] = a3.w;
    const uint32_t b01 = ld4(xb + 260 + 8 * p), b23 = ld4(xb + 264 + 8 * p);
    a.blo = shalf(b01, 0) + shalf(b01, 1);
    a.bhi = shalf(b23, 0) + shalf(b23, 1);
}
__device__ __forceinline__ void load_act(Act<TYPE_Q6_K>& a, const uint8_t* xb, int p) {
    const int h = p >> 1, jj = p & 1;
    a.dx = __builtin_bit_cast(float, ld4(xb));
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const u32x4 v = ld16_a4(xb + 4 + h * 128 + k * 32 + 16 * jj);
        a.xa[4 * k + 0] = v.x; a.xa[4 * k + 1] = v.y; a.xa[4 * k + 2] = v.z; a.xa[4 * k + 3] = v.w;
    }
    const u32x4 bs = ld16_a4(xb + 260 + 16 * h);   // bsums 8h..8h+7; sub-block 8h+2k+jj = dword k, half jj
    a.corr[0] = 32 * shalf(bs.x, jj);
    a.corr[1] = 32 * shalf(bs.y, jj);
    a.corr[2] = 32 * shalf(bs.z, jj);
    a.corr[3] = 32 * shalf(bs.w, jj);
}
// Super-block value of one row for one token (same in all four lanes of the quad).
__device__ __forceinline__ float block_value(const Frag<TYPE_Q4_K>& f, const Act<TYPE_Q4_K>& a, int p) {
    const ScMin sm = q4k_scmin_pair(f.hdr.y, f.hdr.z, f.hdr.w, p);
    int plo, phi;
    q4k_lane_dots(f.qa, f.qb, a.xl, a.xh, plo, phi);
    // 24-bit multiplies (v_mul_i32_i24 / v_mad_i32_i24, full rate; the 32-bit v_mul_lo_u32 is quarter
    // rate): scales and mins < 64, |plo|, |phi| <= 32*15*128, |blo|, |bhi| <= 32*127, products exact
    const int i1 = quad_sum_i32(__mul24((int)sm.sc_lo, plo) + __mul24((int)sm.sc_hi, phi));
    const int i2 = quad_sum_i32(__mul24((int)sm.m_lo, a.blo) + __mul24((int)sm.m_hi, a.bhi));
    return q4k_value(f.hdr.x, a.dx, i1, i2);
}
__device__ __forceinline__ float block_value(const Q6Fields& f, const Act<TYPE_Q6_K>& a, int p) {
    const int jj = p & 1;
    const uint32_t w0 = __builtin_amdgcn_alignbyte(f.sc.y, f.sc.x, f.sh);   // scales 8h .. 8h+3
    const uint32_t w1 = __builtin_amdgcn_alignbyte(f.sce, f.sc.y, f.sh);    // scales 8h+4 .. 8h+7
    int P[4];
    q6k_lane_dots(funnel(f.l0, f.l0e, f.sh), funnel(f.l1, f.l1e, f.sh), funnel(f.hb, f.hbe, f.sh), a.xa, P);
    // 24-bit multiplies: |scale| <= 128, |P - corr| <= 16*63*127 + 32*16*127, products exact
    int I = __mul24(sbyte(w0, jj), P[0] - a.corr[0]);
    I += __mul24(sbyte(w0, jj + 2), P[1] - a.corr[1]);
    I += __mul24(sbyte(w1, jj), P[2] - a.corr[2]);
    I += __mul24(sbyte(w1, jj + 2), P[3] - a.corr[3]);
    I = quad_sum_i32(I);
    return q6k_value(f16_lo(f.dw >> (8 * f.sh)), a.dx, I);
}

// ------------------------------------------------------------------ fp32 activations
// The same lanes and weight fragments with fp32 activations (Kindi's q4_gemv numerics,
// q4.cu:18-27): a lane keeps its 64 activations of the column and their sums, and per weight
// accumulates code * x with one fp32 multiply-add; per sub-block the decoded scale is applied to
// the sum, w = (d*sc)*q - dmin*m, as
//   sum_j w_j x_j = (d*sc_lo) * sum_j q_j x_j - (dmin*m_lo) * sum_j x_j   (Q4_K, likewise hi)
//                 = (d*sc_k) * (sum_j q6u_j x_j - 32 * sum_j x_j)           (Q6_K, q6u = q + 32).
// The quad's four partial values are added in fp32 (lanes p^1, then p^2: the same bits in the four
// lanes) and go through the slot and pass trees like the Q8_K values.
template <int TYPE> struct ActF;
template <> struct ActF<TYPE_Q4_K> { float xl[32], xh[32], sxl, sxh; };   // elements 64p + 0..31, 64p + 32..63
template <> struct ActF<TYPE_Q6_K> { float xa[64], sx[4]; };             // xa[16k + j]: element 128h + 32k + 16jj + j

// Codes as f16 operands.  A 16-bit half whose value v < 1024 sits in the ten mantissa bits (exponent
// field zero) is the f16 subnormal v * 2^-24, exactly, and v_fma_mix_f32 takes such a half as one
// factor of an fp32 multiply-add (f16 subnormals are kept: denormal mode 3).  So a code masked into
// a half in place, at bit 0 (value c * 2^-24) or bit 4 (c * 2^-20), needs no convert instruction, and
// an accumulator of c * 2^-s * x terms is the fp32 accumulator of c * x scaled by 2^-s, rounding
// step for step the same (a power-of-two scale commutes with rounding while the partial sums stay
// at or above 2^-126 * 2^-s in magnitude; only partial sums below that, from activations near the
// fp32 subnormal range, round differently).
__device__ __forceinline__ float half_lo(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)v); }
__device__ __forceinline__ float half_hi(uint32_t v) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16)); }
// acc + c0 x[0] + c1 x[1] + c2 x[2] + c3 x[3], in that order, for codes c0 = a.lo, c1 = b.lo, c2 = a.hi,
// c3 = b.hi (each the scaled value above)
__device__ __forceinline__ float dot_halves_f32(uint32_t a, uint32_t b, const float* x, float acc) {
    acc = __builtin_fmaf(half_lo(a), x[0], acc);
    acc = __builtin_fmaf(half_lo(b), x[1], acc);
    acc = __builtin_fmaf(half_hi(a), x[2], acc);
    return __builtin_fmaf(half_hi(b), x[3], acc);
}
// Bytes 0 and 2 / 1 and 3 of w in the low bytes of the two halves: [0, w.b2, 0, w.b0] / [0, w.b3, 0, w.b1].
__device__ __forceinline__ uint32_t even_bytes(uint32_t w) { return __builtin_amdgcn_perm(w, w, 0x0c020c00u); }
__device__ __forceinline__ uint32_t odd_bytes(uint32_t w) { return __builtin_amdgcn_perm(w, w, 0x0c030c01u); }

// xg = the 256 activations of column g.
__device__ __forceinline__ void load_act(ActF<TYPE_Q4_K>& a, const float* xg, int p) {
    const float* x = xg + 64 * p;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const f32x4 lo = *reinterpret_cast<const f32x4_a4*>(x + 4 * k);
        const f32x4 hi = *reinterpret_cast<const f32x4_a4*>(x + 32 + 4 * k);
        a.xl[4 * k] = lo.x; a.xl[4 * k + 1] = lo.y; a.xl[4 * k + 2] = lo.z; a.xl[4 * k + 3] = lo.w;
        a.xh[4 * k] = hi.x; a.xh[4 * k + 1] = hi.y; a.xh[4 * k + 2] = hi.z; a.xh[4 * k + 3] = hi.w;
    }
    a.sxl = 0.0f;
    a.sxh = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) { a.sxl = __fadd_rn(a.sxl, a.xl[j]); a.sxh = __fadd_rn(a.sxh, a.xh[j]); }
}
__device__ __forceinline__ void load_act(ActF<TYPE_Q6_K>& a, const float* xg, int p) {
    const int h = p >> 1, jj = p & 1;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float* x = xg + h * 128 + k * 32 + 16 * jj;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const f32x4 v = *reinterpret_cast<const f32x4_a4*>(x + 4 * w);
            a.xa[16 * k + 4 * w] = v.x; a.xa[16 * k + 4 * w + 1] = v.y;
            a.xa[16 * k + 4 * w + 2] = v.z; a.xa[16 * k + 4 * w + 3] = v.w;
        }
        float sx = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; j++) sx = __fadd_rn(sx, a.xa[16 * k + j]);
        a.sx[k] = sx;
    }
}
__device__ __forceinline__ float quad_sum_f32(float v) {
    v = __fadd_rn(v, dppf<DPP_QUAD_XOR1>(v));
    return __fadd_rn(v, dppf<DPP_QUAD_XOR2>(v));
}
__device__ __forceinline__ float block_value(const Frag<TYPE_Q4_K>& f, const ActF<TYPE_Q4_K>& a, int p) {
    const ScMin sm = q4k_scmin_pair(f.hdr.y, f.hdr.z, f.hdr.w, p);
    const uint32_t q[8] = {f.qa.x, f.qa.y, f.qa.z, f.qa.w, f.qb.x, f.qb.y, f.qb.z, f.qb.w};
    // byte b of q[k] holds element 4k + b of the low half (low nibble) and of the high half (high
    // nibble): low nibbles in place are codes * 2^-24, high nibbles in place codes * 2^-20
    float plo = 0.0f, phi = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t odd = odd_bytes(q[k]);
        plo = dot_halves_f32(q[k] & 0x000f000fu, odd & 0x000f000fu, a.xl + 4 * k, plo);
        phi = dot_halves_f32(q[k] & 0x00f000f0u, odd & 0x00f000f0u, a.xh + 4 * k, phi);
    }
    plo = __fmul_rn(plo, 0x1p24f);
    phi = __fmul_rn(phi, 0x1p20f);
    const float d = f16_lo(f.hdr.x), dm = f16_hi(f.hdr.x);
    const float dsl = __fmul_rn(d, (float)sm.sc_lo), dsh = __fmul_rn(d, (float)sm.sc_hi);
    const float msl = __fmul_rn(dm, (float)sm.m_lo), msh = __fmul_rn(dm, (float)sm.m_hi);
    const float lo = __fsub_rn(__fmul_rn(dsl, plo), __fmul_rn(msl, a.sxl));
    const float hi = __fsub_rn(__fmul_rn(dsh, phi), __fmul_rn(msh, a.sxh));
    return quad_sum_f32(__fadd_rn(lo, hi));
}
__device__ __forceinline__ float block_value(const Q6Fields& f, const ActF<TYPE_Q6_K>& a, int p) {
    const int jj = p & 1;
    const uint32_t w0 = __builtin_amdgcn_alignbyte(f.sc.y, f.sc.x, f.sh);   // scales 8h .. 8h+3
    const uint32_t w1 = __builtin_amdgcn_alignbyte(f.sce, f.sc.y, f.sh);    // scales 8h+4 .. 8h+7
    const u32x4 l0 = funnel(f.l0, f.l0e, f.sh), l1 = funnel(f.l1, f.l1e, f.sh), hb = funnel(f.hb, f.hbe, f.sh);
    const uint32_t L0[4] = {l0.x, l0.y, l0.z, l0.w}, L1[4] = {l1.x, l1.y, l1.z, l1.w};
    const uint32_t H[4] = {hb.x, hb.y, hb.z, hb.w};
    float P[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t m4 = 0x0f0f0f0fu, m2 = 0x30303030u;
        // four 6-bit codes per word, one per byte (elements 4w .. 4w+3 of group k), codes * 2^-24
        const uint32_t c[4] = {(L0[w] & m4) | ((H[w] << 4) & m2), (L1[w] & m4) | ((H[w] << 2) & m2),
                               ((L0[w] >> 4) & m4) | (H[w] & m2), ((L1[w] >> 4) & m4) | ((H[w] >> 2) & m2)};
#pragma unroll
        for (int k = 0; k < 4; k++)
            P[k] = dot_halves_f32(even_bytes(c[k]), odd_bytes(c[k]), a.xa + k * 16 + 4 * w, P[k]);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) P[k] = __fmul_rn(P[k], 0x1p24f);
    const float d = f16_lo(f.dw >> (8 * f.sh));
    const int sc[4] = {sbyte(w0, jj), sbyte(w0, jj + 2), sbyte(w1, jj), sbyte(w1, jj + 2)};
    float v = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++)
        v = __fadd_rn(v, __fmul_rn(__fmul_rn(d, (float)sc[k]), __fsub_rn(P[k], __fmul_rn(32.0f, a.sx[k]))));
    return quad_sum_f32(v);
}

// Activation formats of the kernels below: where column g of token t starts, and its register type.
struct ActQ8K {
    template <int T> using A = Act<T>;
    static constexpr bool F32 = false;
    static __device__ __forceinline__ const uint8_t* col(const uint8_t* X, int64_t t, int G, int g) {
        return X + (t * G + g) * Q8K_BYTES;
    }
};
struct ActF32 {
    template <int T> using A = ActF<T>;
    static constexpr bool F32 = true;
    static __device__ __forceinline__ const float* col(const uint8_t* X, int64_t t, int G, int g) {
        return reinterpret_cast<const float*>(X) + (t * G + g) * QK;
    }
};

// ------------------------------------------------------------------ the kernel
// FP = 3: exactly three column passes (C = 8448 .. 12288, the FFN down projection), with the
// activations of all three held in registers instead of reloaded at every (unit, pass) step;
// the step loop is unrolled over the passes so each step's pass is a compile-time index.
template <int TYPE, int NT, int RPW, bool ONEPASS, int FP = 0, class AP = ActQ8K>
__global__ void __launch_bounds__(256)
k_gemv_q8k(KQ_GEMV_HEAD, int nwaves, MatGroup mg) {
    using ActT = typename AP::template A<TYPE>;
    constexpr int WPT = 8 / RPW;
    constexpr int BS = TYPE == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    const int lane = threadIdx.x & 63;
    // Unit bookkeeping is wave-uniform: readfirstlane keeps it in scalar registers.
    // Logical workgroup index grouped by die: workgroups are dealt to the XCDs in turn, so the
    // consecutive logical indices b, b + 1, whose streams share an 8-row tile (and the 128-byte lines
    // its rows' blocks straddle), run behind one L2 (4096x12288 Q6_K: 10.6 -> 10.4 us).
    // nwaves: waves per workgroup
    KQ_GEMV_PICK;
    int lwg = blockIdx.x;
    if (ngrid % KQ_XCDS == 0) lwg = (lwg % KQ_XCDS) * (ngrid / KQ_XCDS) + lwg / KQ_XCDS;
    const TileWalk<WPT, false> walk{lwg, ngrid, __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nwaves};
    int u = walk.first();
    if (u >= total_units) return;
    const int p = lane & 3, slot = lane >> 2;
    const int passes = ONEPASS ? 1 : FP ? FP : (G + 15) >> 4;
    const int64_t col_bytes = 8 * BS;                  // one tile column
    const int64_t tile_bytes = (int64_t)G * col_bytes;

    // Unit -> (matrix, first row) and the row-block address.  The unit index is wave-uniform,
    // so the argument-struct reads below are scalar loads and never wait on the weight stream.
    // (the first unit's from the registers of the prologue's batch; later units' from the argument
    // table, whose scalar loads the streaming loop hides: selects there made the loop's control flow
    // branchier and its wait for the current unit a wait for every load, 89 -> 96 us on a 510 MB head)
    auto unit_base0 = [&](int uu, int& m, int64_t& row0) -> const uint8_t* {
        m = mat_of(uu);
        const int v = uu - first_of(m);
        const int64_t tile = v / WPT;
        const int r0 = (v - (int)tile * WPT) * RPW;
        row0 = tile * 8 + r0;
        return w_of(m) + tile * tile_bytes + r0 * BS;
    };
    auto unit_base = [&](int uu, int& m, int64_t& row0) -> const uint8_t* {
        m = uu >= mg.first_unit[1] ? (uu >= mg.first_unit[2] ? 2 : 1) : 0;
        const int v = uu - mg.first_unit[m];
        const int64_t tile = v / WPT;
        const int r0 = (v - (int)tile * WPT) * RPW;
        row0 = tile * 8 + r0;
        return mg.w[m] + tile * tile_bytes + r0 * BS;
    };

    // Every load below is unconditional (lanes past the last column read column G-1 and their
    // values are masked to zero), so the number of loads in flight is static and the compiler
    // can wait for the current step's data without draining the next step's prefetch.
    const int slot_c = slot < G ? slot : G - 1;
    ActT act[NT];
    if (ONEPASS) {
#pragma unroll
        for (int t = 0; t < NT; t++) load_act(act[t], AP::col(XQ, t, G, slot_c), p);
    }
    // (the activations before the first weights: weights first measured slower here, 4096x12288 Q6_K
    // 10.2 -> 10.6 us, unlike the pass-split kernel)
    ActT actp[FP ? FP : 1][NT];                        // FP: every pass's activations
    if (FP) {
#pragma unroll
        for (int q = 0; q < (FP ? FP : 1); q++) {
            const int gq = slot + 16 * q < G ? slot + 16 * q : G - 1;
#pragma unroll
            for (int t = 0; t < NT; t++) load_act(actp[q][t], AP::col(XQ, t, G, gq), p);
        }
    }

    Frag<TYPE> bufA[RPW], bufB[RPW];
    int m;
    int64_t row0;
    const uint8_t* base = unit_base0(u, m, row0);
#pragma unroll
    for (int r = 0; r < RPW; r++) load_frag(bufA[r], base + (int64_t)slot_c * col_bytes + r * BS, p);
    PassTree tree[NT][RPW];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int r = 0; r < RPW; r++) tree_init(tree[t][r]);

    int pass = 0;
    // One (unit, pass) step: issue the next step's loads into `nxt`, then compute from `cur`.
    // The loop body runs two steps with the buffers swapped, so no register copy (which would
    // have to wait for the prefetch) is needed.  The last step re-reads its own unit so the
    // number of loads in flight stays fixed.
    auto step = [&](Frag<TYPE>* cur, Frag<TYPE>* nxt) -> bool {
        int un = u, pn = pass + 1;
        if (pn == passes) { pn = 0; un = walk.next(u); }
        const bool has_next = un < total_units;
        int mn = m;
        int64_t row0n = row0;
        const uint8_t* basen = base;
        if (has_next && un != u) basen = unit_base(un, mn, row0n);
        {
            int gn = slot + 16 * (has_next ? pn : pass);
            gn = gn < G ? gn : G - 1;
#pragma unroll
            for (int r = 0; r < RPW; r++) load_frag(nxt[r], basen + (int64_t)gn * col_bytes + r * BS, p);
        }
        __builtin_amdgcn_sched_barrier(0);

        const int g = slot + 16 * pass;
        const bool valid = g < G;
        if (!ONEPASS) {
            const int gc = valid ? g : G - 1;
#pragma unroll
            for (int t = 0; t < NT; t++) load_act(act[t], AP::col(XQ, t, G, gc), p);
        }
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const auto fr = prepare(cur[r], p);
#pragma unroll
            for (int t = 0; t < NT; t++) {
                const float v = block_value(fr, act[t], p);
                tree_push(tree[t][r], slot_tree_f32(valid ? v : 0.0f));
            }
        }

        if (pass == passes - 1) {
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int r = 0; r < RPW; r++) {
                    const float y = tree_final(tree[t][r]);
                    if (lane == 0) mg.y[m][t * mg.ldy[m] + row0 + r] = y;
                    tree_init(tree[t][r]);
                }
        }
        if (!has_next) return false;
        u = un; pass = pn; m = mn; row0 = row0n; base = basen;
        return true;
    };
    if constexpr (FP == 3) {
        // step with a compile-time pass PS: the same work as `step`, activations from registers
        auto stepf = [&](auto pass_c, Frag<TYPE>* cur, Frag<TYPE>* nxt) -> bool {
            constexpr int PS = decltype(pass_c)::value;
            constexpr int PN = PS + 1 == FP ? 0 : PS + 1;
            const int un = PN == 0 ? walk.next(u) : u;
            const bool has_next = un < total_units;
            int mn = m;
            int64_t row0n = row0;
            const uint8_t* basen = base;
            if (has_next && PN == 0) basen = unit_base(un, mn, row0n);
            {
                int gn = slot + 16 * (has_next ? PN : PS);
                gn = gn < G ? gn : G - 1;
#pragma unroll
                for (int r = 0; r < RPW; r++) load_frag(nxt[r], basen + (int64_t)gn * col_bytes + r * BS, p);
            }
            __builtin_amdgcn_sched_barrier(0);
            const bool valid = slot + 16 * PS < G;
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                const auto fr = prepare(cur[r], p);
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const float v = block_value(fr, actp[PS][t], p);
                    tree_push(tree[t][r], slot_tree_f32(valid ? v : 0.0f));
                }
            }
            if (PS == FP - 1) {
#pragma unroll
                for (int t = 0; t < NT; t++)
#pragma unroll
                    for (int r = 0; r < RPW; r++) {
                        const float y = tree_final(tree[t][r]);
                        if (lane == 0) mg.y[m][t * mg.ldy[m] + row0 + r] = y;
                        tree_init(tree[t][r]);
                    }
            }
            if (!has_next) return false;
            u = un; m = mn; row0 = row0n; base = basen;
            return true;
        };
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        if constexpr (NT == 1 && KQ_GEMV_SEQ_DEPTH == 2) {
            // two steps in flight: step i issues the loads of step i + 2 into the buffer step i - 1 used
            // (one token: 4096x12288 Q6_K 11.6 -> 11.1 us; two tokens were slower with it, and three
            // steps in flight slower again: 10.6 -> 11.5 us)
            Frag<TYPE> bufC[RPW];
#pragma unroll
            for (int r = 0; r < RPW; r++) load_frag(bufB[r], base + (int64_t)(slot + 16 < G ? slot + 16 : G - 1) * col_bytes + r * BS, p);
            auto step2 = [&](auto pass_c, Frag<TYPE>* cur, Frag<TYPE>* nxt2) -> bool {
                constexpr int PS = decltype(pass_c)::value;
                const int un = walk.next(u);
                const bool has_un = un < total_units;
                int mn = m;
                int64_t row0n = row0;
                const uint8_t* basen = base;
                if (has_un) basen = unit_base(un, mn, row0n);
                {
                    // step i + 2: (u, 2) when PS == 0, else (un, PS - 1); past the end this step again
                    const uint8_t* bt = PS == 0 || !has_un ? base : basen;
                    const int pt = PS == 0 ? 2 : (has_un ? PS - 1 : PS);
                    int gn = slot + 16 * pt;
                    gn = gn < G ? gn : G - 1;
#pragma unroll
                    for (int r = 0; r < RPW; r++) load_frag(nxt2[r], bt + (int64_t)gn * col_bytes + r * BS, p);
                }
                __builtin_amdgcn_sched_barrier(0);
                const bool valid = slot + 16 * PS < G;
#pragma unroll
                for (int r = 0; r < RPW; r++) {
                    const auto fr = prepare<false>(cur[r], p);
#pragma unroll
                    for (int t = 0; t < NT; t++) {
                        const float v = block_value(fr, actp[PS][t], p);
                        tree_push(tree[t][r], slot_tree_f32(valid ? v : 0.0f));
                    }
                }
                if (PS == FP - 1) {
#pragma unroll
                    for (int t = 0; t < NT; t++)
#pragma unroll
                        for (int r = 0; r < RPW; r++) {
                            const float y = tree_final(tree[t][r]);
                            if (lane == 0) mg.y[m][t * mg.ldy[m] + row0 + r] = y;
                            tree_init(tree[t][r]);
                        }
                    if (!has_un) return false;
                    u = un; m = mn; row0 = row0n; base = basen;
                }
                return true;
            };
            while (step2(I0{}, bufA, bufC) && step2(I1{}, bufB, bufA) && step2(I2{}, bufC, bufB)) {
            }
        } else {
        while (stepf(I0{}, bufA, bufB) && stepf(I1{}, bufB, bufA) && stepf(I2{}, bufA, bufB) &&
               stepf(I0{}, bufB, bufA) && stepf(I1{}, bufA, bufB) && stepf(I2{}, bufB, bufA)) {
        }
        }
    } else {
        while (step(bufA, bufB) && step(bufB, bufA)) {
        }
    }
}

// ------------------------------------------------------------------ pass-split kernel
// For C <= 16384 (at most 4 column passes).  A workgroup holds K unit streams of P waves each
// (P = passes): wave (stream, pass) keeps the activations of its pass in registers and streams
// that pass's tile columns for every unit of its stream (TileWalk order),
// prefetching the next unit.  Each (unit, token, row) pass value goes to LDS; after one barrier
// the workgroup merges them with the same pass tree as the sequential kernel and stores y.  With
// one pass the value is stored directly.
// AMAX (one matrix, one token, one pass): the argmax of the outputs as well, into *aout
// (argmax_block.h; aws is its workspace).  The body takes the workgroup's index among the
// launch's workgroups of this part (bid; the grid's own index for k_gemv_q8k_split) and the
// pass partials' LDS (part: [stream][k][t][r][pass]).
// XF (one token, one column pass): the activations arrive as fp32 (X) and every workgroup quantizes
// them to Q8_K into LDS (xs) itself, with the stand-alone quantizer's block code, while its first
// weight loads are in flight; workgroup 0 also writes the bytes to XQO when that is not null.
template <int TYPE, int NT, int RPW, bool AMAX, class AP, bool XF = false>
__device__ __forceinline__ void gemv_split_body(KQ_GEMV_HEAD, int PK, const MatGroup& mg, int kmax, uint8_t* aws,
                                                int* aout, int bid, float* part, const float* X = nullptr,
                                                uint8_t* xs = nullptr, uint8_t* XQO = nullptr) {
    using ActT = typename AP::template A<TYPE>;
    constexpr int WPT = 8 / RPW;
    constexpr int BS = TYPE == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    // PK = P | K << 8: P column passes, K unit streams per workgroup (the block holds K * P waves)
    const int P = PK & 0xff, K = PK >> 8;
    KQ_GEMV_PICK;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int pass = wave % P, stream = wave / P;
    // The WPT units of an 8-row tile fall to the streams of one workgroup (TileWalk), so the rows
    // that share cache lines (144- and 210-byte blocks do not align to 128-byte lines) are read by
    // one CU through one L2.  (Contiguous unit ranges per stream, with the streams of each XCD
    // grouped, were slower: gate+up 12.2 -> 13.1 us, the output head 95 -> 108 us.)
    const int nwg = ngrid;
    const int lwg = bid;
    const TileWalk<WPT> walk{lwg, nwg, stream, K};
    const int u_begin = walk.first(), u_end = total_units;
    const int p = lane & 3, slot = lane >> 2;
    const int64_t col_bytes = 8 * BS;
    const int64_t tile_bytes = (int64_t)G * col_bytes;
    const int g = slot + 16 * pass;
    const bool valid = g < G;
    const int gc = valid ? g : G - 1;                  // lanes past the last column read column G-1, masked

    // (the first unit's from the prologue's registers, later units' from the argument table: see
    // k_gemv_q8k)
    auto unit_base0 = [&](int uu, int& m, int64_t& row0) -> const uint8_t* {
        m = mat_of(uu);
        const int v = uu - first_of(m);
        const int64_t tile = v / WPT;
        const int r0 = (v - (int)tile * WPT) * RPW;
        row0 = tile * 8 + r0;
        return w_of(m) + tile * tile_bytes + r0 * BS + gc * col_bytes;
    };
    auto unit_base = [&](int uu, int& m, int64_t& row0) -> const uint8_t* {
        m = uu >= mg.first_unit[1] ? (uu >= mg.first_unit[2] ? 2 : 1) : 0;
        const int v = uu - mg.first_unit[m];
        const int64_t tile = v / WPT;
        const int r0 = (v - (int)tile * WPT) * RPW;
        row0 = tile * 8 + r0;
        return mg.w[m] + tile * tile_bytes + r0 * BS + gc * col_bytes;
    };

    ArgBest best = arg_init();                         // AMAX: the wave's best output so far (every lane)
    static_assert(!XF || (NT == 1 && !AMAX && !AP::F32), "XF: one token of Q8_K activations, no argmax");
    if (u_begin < u_end || XF) {
        const bool active = u_begin < u_end;           // wave-uniform
        ActT act[NT];
        Frag<TYPE> bufA[RPW], bufB[RPW];
        int u = u_begin, k = 0, m = 0;
        int64_t row0 = 0;
        const uint8_t* base = active ? unit_base0(u, m, row0) : w0;
        // the first unit's weights before the activations: the weights come from HBM, the activations
        // (written by the launch before) from the last-level cache (decode layer 37.87 -> 37.67 us)
        if constexpr (XF) {
            // blocks wave, wave + nw, ... of x, loaded first (the quantization waits for them, the
            // first unit's weights come later from HBM anyway), then the first unit's weights
            constexpr int XB = 4;                      // G <= 16 blocks over the workgroup's 4 waves
            const int nw = P * K;
            f32x4 xv[XB];
            if constexpr (!KQ_XF_XFIRST) {
                if (active) {
#pragma unroll
                    for (int r = 0; r < RPW; r++) load_frag(bufA[r], base + r * BS, p);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int i = 0; i < XB; i++) {
                const int b = wave + nw * i < G ? wave + nw * i : G - 1;
                xv[i] = *reinterpret_cast<const f32x4_a4*>(X + b * QK + 4 * lane);
            }
            if constexpr (KQ_XF_XFIRST) {
                __builtin_amdgcn_sched_barrier(0);
                if (active) {
#pragma unroll
                    for (int r = 0; r < RPW; r++) load_frag(bufA[r], base + r * BS, p);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            // the wave's blocks side by side (blocks past G go to the spare slot xs[G])
            float e[XB][4];
            uint8_t* ob[XB];
#pragma unroll
            for (int i = 0; i < XB; i++) {
                const int b = wave + nw * i;
                e[i][0] = xv[i].x; e[i][1] = xv[i].y; e[i][2] = xv[i].z; e[i][3] = xv[i].w;
                ob[i] = xs + (b < G ? b : G) * Q8K_BYTES;
            }
            q8k_blocks_store<XB>(e, lane, ob);
            // LDS-only barrier: the weight loads issued above stay in flight
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
            if (XQO != nullptr && bid == 0) {          // the bytes out of this workgroup's LDS
                const uint32_t* src = reinterpret_cast<const uint32_t*>(xs);
                uint32_t* dst = reinterpret_cast<uint32_t*>(XQO);
                for (int i = threadIdx.x; i < G * (Q8K_BYTES / 4); i += 64 * nw) dst[i] = src[i];
            }
            if (!active) return;
            load_act(act[0], xs + gc * Q8K_BYTES, p);
        } else if constexpr (KQ_GEMV_SPLIT_WFIRST) {
#pragma unroll
            for (int r = 0; r < RPW; r++) load_frag(bufA[r], base + r * BS, p);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < NT; t++) load_act(act[t], AP::col(XQ, t, G, gc), p);
        } else {
#pragma unroll
            for (int t = 0; t < NT; t++) load_act(act[t], AP::col(XQ, t, G, gc), p);
#pragma unroll
            for (int r = 0; r < RPW; r++) load_frag(bufA[r], base + r * BS, p);
        }
        float* mypart = part + (int64_t)stream * kmax * NT * RPW * P;

        auto step = [&](Frag<TYPE>* cur, Frag<TYPE>* nxt) -> bool {
            const int un = walk.next(u);
            const bool has_next = un < u_end;
            int mn = m;
            int64_t row0n = row0;
            const uint8_t* basen = has_next ? unit_base(un, mn, row0n) : base;
#pragma unroll
            for (int r = 0; r < RPW; r++) load_frag(nxt[r], basen + r * BS, p);
            // keep every prefetch load ahead of this step's compute (and its waits)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < RPW; r++) {
                const auto fr = prepare(cur[r], p);
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    const float v = block_value(fr, act[t], p);
                    const float pv = slot_tree_f32(valid ? v : 0.0f);
                    if (P == 1) {
                        // every lane holds the same pv (the slot tree is symmetric); the units of a
                        // stream come in increasing row order, so the pick runs unmasked
                        const float yv = __fadd_rn(pv, 0.0f);
                        if (lane == 0) mg.y[m][t * mg.ldy[m] + row0 + r] = yv;
                        if (AMAX) arg_take_ascending(best, yv, (int)(row0 + r));
                    } else if (lane == 0) {
                        mypart[((k * NT + t) * RPW + r) * P + pass] = pv;
                    }
                }
            }
            if (!has_next) return false;
            u = un; k++; m = mn; row0 = row0n; base = basen;
            return true;
        };
        while (step(bufA, bufB) && step(bufB, bufA)) {
        }
    }
    if (P == 1) {
        if (AMAX) arg_grid_finish(arg_wave_reduce(best), aws, aout);
        return;
    }

    __syncthreads();
    for (int st = 0; st < K; st++) {
        const TileWalk<WPT> ws{lwg, nwg, st, K};
        const int nk = ws.count(total_units);
        const float* sp = part + (int64_t)st * kmax * NT * RPW * P;
        for (int idx = threadIdx.x; idx < nk * NT * RPW; idx += 64 * K * P) {
            const int kk = idx / (NT * RPW), t = (idx / RPW) % NT, r = idx % RPW;
            const int uu = ws.unit(kk);
            const int mm = uu >= mg.first_unit[1] ? (uu >= mg.first_unit[2] ? 2 : 1) : 0;
            const int v = uu - mg.first_unit[mm];
            const int64_t rowr = (int64_t)(v / WPT) * 8 + (v % WPT) * RPW + r;
            PassTree tr;
            tree_init(tr);
            for (int q = 0; q < P; q++) tree_push(tr, sp[idx * P + q]);
            mg.y[mm][t * mg.ldy[mm] + rowr] = tree_final(tr);
        }
    }
}

template <int TYPE, int NT, int RPW, bool AMAX, class AP = ActQ8K>
__global__ void __launch_bounds__(64 * KQ_GEMV_WG_WAVES)
k_gemv_q8k_split(KQ_GEMV_HEAD, int PK, MatGroup mg, int kmax, uint8_t* aws, int* aout) {
    extern __shared__ float part[];
    gemv_split_body<TYPE, NT, RPW, AMAX, AP>(w0, w1, w2, XQ, G, total_units, f1, f2, ngrid, PK, mg, kmax, aws, aout,
                                             blockIdx.x, part);
}

// One token from fp32 activations (C <= 4096: one column pass): x quantized to Q8_K inside the
// launch (each workgroup into its LDS, bit for bit the stand-alone quantizer's bytes), so the
// quantizer's own launch is saved.  XQ (KQ_GEMV_HEAD's slot) carries x; xqo, when not null,
// receives the Q8_K bytes (from workgroup 0).
template <int TYPE, int RPW>
__global__ void __launch_bounds__(64 * KQ_GEMV_WG_WAVES)
k_gemv_q8k_x(KQ_GEMV_HEAD, MatGroup mg, uint8_t* xqo) {
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
    constexpr int PK = 1 | KQ_GEMV_WG_WAVES << 8;
    gemv_split_body<TYPE, 1, RPW, false, ActQ8K, true>(w0, w1, w2, XQ, G, total_units, f1, f2, ngrid, PK, mg, 1,
                                                       nullptr, nullptr, blockIdx.x, nullptr,
                                                       reinterpret_cast<const float*>(XQ), xs, xqo);
}

// Two weight types sharing one input, one token and one column pass, in one launch: workgroups
// [0, nwgA) run the pass-split GEMV over w0 and w1 (type TA; w1 = w0 and f1 = nA when there is
// one), the others over w2 (type TB), each part in the unit order of its own launch, so every
// output has the bits of the one-type launch.  The scalars keep KQ_GEMV_HEAD's slots (all
// preloaded): total_units = nB (units of w2), f1 = first unit of w1, f2 = nA (units of type TA),
// ngrid = both parts' workgroups; mgA / mgB hold the parts' outputs (and units for later steps).
// XF: XQ carries fp32 x, quantized in every workgroup as in k_gemv_q8k_x (xqo: the bytes, or null).
template <int TA, int RA, int TB, int RB, class AP = ActQ8K, bool XF = false>
__global__ void __launch_bounds__(64 * KQ_GEMV_WG_WAVES)
k_gemv_q8k_split2(KQ_GEMV_HEAD, int nwgA, MatGroup mgA, MatGroup mgB, uint8_t* xqo) {
    extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
    constexpr int PK = 1 | KQ_GEMV_WG_WAVES << 8;
    const float* X = XF ? reinterpret_cast<const float*>(XQ) : nullptr;
    if ((int)blockIdx.x < nwgA)
        gemv_split_body<TA, 1, RA, false, AP, XF>(w0, w1, w1, XQ, G, f2, f1, f2, nwgA, PK, mgA, 1, nullptr, nullptr,
                                                  blockIdx.x, nullptr, X, xs, xqo);
    else
        gemv_split_body<TB, 1, RB, false, AP, XF>(w2, w2, w2, XQ, G, total_units, total_units, total_units,
                                                  ngrid - nwgA, PK, mgB, 1, nullptr, nullptr, blockIdx.x - nwgA,
                                                  nullptr, X, xs, nullptr);
}

// ------------------------------------------------------------------ launch
// Rows per wave: Q4_K 2 keeps per-wave register use moderate and gives many units to balance;
// with several tokens per launch the register budget is NT*RPW <= 8 outputs per lane.  Q6_K
// takes one row per wave: twice the units, so each wave walks more (unit, pass) steps and its
// prefetch covers more of the stream (the one-pass output head 151936x4096: 96 us against 102 us
// at 2), except two tokens on the sequential kernel (3 or more passes), where 2 rows per wave
// share each pass's activations (4096x12288: 12.9 -> 12.3 us; one token: no difference).
static int pick_rpw(int nt, int type, int G) {
#ifdef KQ_GEMV_RPW
#if KQ_GEMV_RPW != 1 && KQ_GEMV_RPW != 2
#error "KQ_GEMV_RPW must be 1 or 2 (the launcher instantiates only these)"
#endif
    (void)nt; (void)type; (void)G;
    return KQ_GEMV_RPW;
#else
    if (type == TYPE_Q6_K) return nt == 2 && (G + 15) / 16 > KQ_GEMV_SPLIT_MAX_Q6 ? 2 : 1;
    return nt >= 3 ? 1 : 2;
#endif
}

template <int TYPE, int NT, int RPW, bool AMAX = false, class AP = ActQ8K>
static void launch3(const MatGroup& mg0, const uint8_t* xq, int G, hipStream_t s, uint8_t* aws = nullptr,
                    int* aout = nullptr) {
    MatGroup mg = mg0;
    int total = 0;
    for (int i = 0; i < 3; i++) {
        mg.first_unit[i] = total;
        if (i < mg.n) total += (int)((mg0.first_unit[i + 1] - mg0.first_unit[i]) * (8 / RPW));
    }
    mg.first_unit[3] = total;
    const int passes = (G + 15) / 16;
    const int wpc = AP::F32 ? (TYPE == TYPE_Q6_K ? KQ_GEMV_WAVES_PER_CU_F32_Q6 : KQ_GEMV_WAVES_PER_CU_F32)
                    : TYPE == TYPE_Q6_K ? KQ_GEMV_WAVES_PER_CU_Q6 : NT == 2 ? KQ_GEMV_WAVES_PER_CU_NT2 : KQ_GEMV_WAVES_PER_CU;
    // Q6_K with one or two tokens: sequential passes (the activations are reloaded per pass,
    // which only pays off while they are few)
    // (fp32 activations keep 64 floats per lane and pass: every pass a wave of its own)
    if (passes <= (TYPE == TYPE_Q6_K && NT <= 2 && !AP::F32 ? KQ_GEMV_SPLIT_MAX_Q6 : KQ_GEMV_SPLIT_MAX)) {
        // K unit streams of `passes` waves per workgroup (about KQ_GEMV_WG_WAVES waves per
        // workgroup); about KQ_GEMV_WAVES_PER_CU waves per CU in total
        const int K = passes >= KQ_GEMV_WG_WAVES ? 1 : KQ_GEMV_WG_WAVES / passes;
        int streams = device_cus() * wpc / passes;
        if (streams > total) streams = total;
        auto round_xcd = [](int n) { return (n + KQ_XCDS - 1) / KQ_XCDS * KQ_XCDS; };
        int nwg = round_xcd((streams + K - 1) / K);
        size_t lds = 0;
        int kmax = 1;
        if (passes > 1) {
            constexpr int WPT = 8 / RPW;
            for (;;) {
                // most units a stream walks (TileWalk::count)
                kmax = KQ_GEMV_TILE_WG && K < WPT ? (total / WPT + nwg - 1) / nwg * (WPT / K)
                                                  : (total + nwg * K - 1) / (nwg * K);
                lds = (size_t)K * kmax * NT * RPW * passes * sizeof(float);
                if (lds <= 32768 || nwg * K >= total) break;
                nwg = round_xcd(nwg * 2);
            }
        }
        hipLaunchKernelGGL((k_gemv_q8k_split<TYPE, NT, RPW, AMAX, AP>), dim3(nwg), dim3(64 * passes * K), lds, s,
                           mg.w[0], mg.w[1], mg.w[2], xq, G, total, mg.first_unit[1], mg.first_unit[2], nwg,
                           passes | K << 8, mg, kmax, aws, aout);
        return;
    }
    const int wpb = KQ_GEMV_SEQ_WPB;
    int waves = device_cus() * (TYPE == TYPE_Q6_K ? KQ_GEMV_WAVES_PER_CU_SEQ_Q6 : wpc);
    if (waves > total) waves = total;
    dim3 grid((waves + wpb - 1) / wpb), block(64 * wpb);
    if constexpr (KQ_GEMV_P3 && NT <= 2 && RPW <= 2 && !AP::F32) {
        if (passes == 3) {
            hipLaunchKernelGGL((k_gemv_q8k<TYPE, NT, RPW, false, 3>), grid, block, 0, s, mg.w[0], mg.w[1], mg.w[2], xq,
                               G, total, mg.first_unit[1], mg.first_unit[2], (int)grid.x, wpb, mg);
            return;
        }
    }
    if (G <= 16)
        hipLaunchKernelGGL((k_gemv_q8k<TYPE, NT, RPW, true, 0, AP>), grid, block, 0, s, mg.w[0], mg.w[1], mg.w[2], xq,
                           G, total, mg.first_unit[1], mg.first_unit[2], (int)grid.x, wpb, mg);
    else
        hipLaunchKernelGGL((k_gemv_q8k<TYPE, NT, RPW, false, 0, AP>), grid, block, 0, s, mg.w[0], mg.w[1], mg.w[2], xq,
                           G, total, mg.first_unit[1], mg.first_unit[2], (int)grid.x, wpb, mg);
}

template <int TYPE, int NT>
static void launch2(const MatGroup& mg, const uint8_t* xq, int G, int rpw, hipStream_t s) {
    if (rpw == 1) launch3<TYPE, NT, 1>(mg, xq, G, s);
    else launch3<TYPE, NT, 2>(mg, xq, G, s);
}

template <int TYPE>
static void launch1(const MatGroup& mg, const uint8_t* xq, int G, int nt, int rpw, hipStream_t s) {
    switch (nt) {
        case 1: launch2<TYPE, 1>(mg, xq, G, rpw, s); break;
        case 2: launch2<TYPE, 2>(mg, xq, G, rpw, s); break;
        case 3: launch2<TYPE, 3>(mg, xq, G, rpw, s); break;
        default: launch2<TYPE, 4>(mg, xq, G, rpw, s); break;
    }
}

// Whether a call goes to the MFMA forms (gemv_mfma.hip, at most 64 super-blocks per row) rather than
// the v_dot4 kernels here; every choice is the faster one measured (us, v_dot4 -> MFMA form):
//   Q4_K  one token with 17..48 super-blocks per row and at least 4096 rows (the phase form against the
//         pass-split kernel): 4096x12288 9.2 -> 8.6; below 4096 rows the v_dot4 kernel stays (2048x12288
//         6.2 against ~6.7), and so does every one-token call with at most 16 (6144 / 4096 / 12288 /
//         24576 x 4096: 5.2 / 4.5 / 8.3 / 12.7 against 5.7 / 4.7 / 8.4 / 12.7).  2..4 tokens: the phase
//         form, 12288x4096 at N = 2 9.4 -> 8.0, 4096x12288 10.4 -> 8.4, 2048x12288 at N = 2 / 3 / 4
//         7.8 / 9.0 / 11.0 -> 6.7 / 6.7 / 6.7; except below
//         4096 rows with at most 16 super-blocks and at most 3 tokens (1024x4096 at N = 2 3.8 against
//         4.4, N = 3 4.3 against 4.4), and below 4096 rows with more than 48 (not measured with the
//         phase form, which stops at 48).  5..16 tokens: the plane form.
//   Q6_K  from 3 tokens (2 tokens: 12.1 against 13.7); below 4096 rows from 5 tokens (N = 3 / 4: 1024x4096
//         4.7 / 5.5 against 5.7 / 5.7, 2048x12288 10.8 / 12.6 against 11.4 / 11.6).
static bool use_mfma_form(int type, int N, int G, int rows) {
    // (the MFMA kernels take the first workgroups of matrices 1 and 2 in 16 bits each: 16-row groups)
    if (G > 64 || rows >= 16 * 65535) return false;
    const bool few_rows = rows < 4096;
    if (type == TYPE_Q4_K) {
        if (N == 1) return G > 16 && G <= 48 && !few_rows;
        if (few_rows && N <= 4 && (G > 48 || (G <= 16 && N <= 3))) return false;
        return true;
    }
    return N >= 3 && !(few_rows && N <= 4);
}

// n matrices of one type sharing xq (N tokens); tokens go in groups of up to 4 per launch, each
// group an independent launch over the same weights.  first_unit[] is filled with row-tile
// prefix counts here and scaled to units per RPW in launch3.
void launch_gemv_q8k_group(int n, const uint8_t* const* w, const int* R, int C, int type,
                           const uint8_t* xq, int N, float* const* y, const int64_t* ldy, hipStream_t s) {
    const int G = C / QK;
    int rows = 0;
    for (int i = 0; i < n; i++) rows += R[i];
    if (use_mfma_form(type, N, G, rows)) {   // same bits

        launch_gemv_mfma_group(n, w, R, C, type, xq, N, y, ldy, s);
        return;
    }
    for (int n0 = 0; n0 < N; n0 += 4) {
        const int nt = N - n0 < 4 ? N - n0 : 4;
        MatGroup mg{};
        mg.n = n;
        int tiles = 0;
        for (int i = 0; i < n; i++) {
            mg.w[i] = w[i];
            mg.y[i] = y[i] + (int64_t)n0 * ldy[i];
            mg.ldy[i] = ldy[i];
            mg.first_unit[i] = tiles;
            tiles += R[i] / 8;
        }
        for (int i = n; i < 4; i++) mg.first_unit[i] = tiles;
        const uint8_t* xg = xq + (int64_t)n0 * G * Q8K_BYTES;
        if (type == TYPE_Q4_K) launch1<TYPE_Q4_K>(mg, xg, G, nt, pick_rpw(nt, TYPE_Q4_K, G), s);
        else launch1<TYPE_Q6_K>(mg, xg, G, nt, pick_rpw(nt, TYPE_Q6_K, G), s);
    }
}

// Both weight types sharing one input (a Q4_K_M layer's q, k and a Q6_K v): the two launches the
// type groups would make become one (k_gemv_q8k_split2), its workgroups split between the types
// in proportion to their weight bytes, each part's waves walking their units as the one-type
// launch does (a 1024x4096 Q6_K matrix alone costs a launch of ~3.7 us).
template <int TA, int RA, int TB, int RB, class AP, bool XF = false>
static void launch_mixed(const uint8_t* const* wa, const int* ra, float* const* ya, int na, const uint8_t* wb,
                         int rb, float* yb, const uint8_t* xq, int G, hipStream_t s, uint8_t* xqo = nullptr) {
    constexpr int BSA = TA == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES, BSB = TB == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    constexpr int K = KQ_GEMV_WG_WAVES;                // one column pass: K unit streams of one wave
    MatGroup mga{}, mgb{};
    mga.n = na;
    int unitsA = 0;
    int64_t rowsA = 0;
    for (int i = 0; i < na; i++) {
        mga.w[i] = wa[i];
        mga.y[i] = ya[i];
        mga.ldy[i] = ra[i];
        mga.first_unit[i] = unitsA;
        unitsA += ra[i] / RA;
        rowsA += ra[i];
    }
    for (int i = na; i < 4; i++) mga.first_unit[i] = unitsA;
    const int unitsB = rb / RB;
    mgb.n = 1;
    mgb.w[0] = wb;
    mgb.y[0] = yb;
    mgb.ldy[0] = rb;
    mgb.first_unit[0] = 0;
    for (int i = 1; i < 4; i++) mgb.first_unit[i] = unitsB;
    const double bytesA = (double)rowsA * BSA, bytesB = (double)rb * BSB;
    const int streams = device_cus() * (AP::F32 ? KQ_GEMV_WAVES_PER_CU_F32 : KQ_GEMV_WAVES_PER_CU);
    int sa = (int)(streams * bytesA / (bytesA + bytesB) + 0.5);
    sa = sa < K ? K : sa > unitsA ? unitsA : sa;
    int sb = streams - sa;
    sb = sb < K ? K : sb > unitsB ? unitsB : sb;
    auto round_xcd = [](int n) { return (n + KQ_XCDS - 1) / KQ_XCDS * KQ_XCDS; };
    const int nwga = round_xcd((sa + K - 1) / K), nwgb = round_xcd((sb + K - 1) / K);
    const size_t lds = XF ? (size_t)(G + 1) * Q8K_BYTES : 0;   // XF: the Q8_K blocks + a spare slot
    hipLaunchKernelGGL((k_gemv_q8k_split2<TA, RA, TB, RB, AP, XF>), dim3(nwga + nwgb), dim3(64 * K), lds, s, wa[0],
                       wa[na > 1 ? 1 : 0], wb, xq, G, unitsB, mga.first_unit[1], unitsA, nwga + nwgb, nwga, mga, mgb,
                       xqo);
}

template <class AP, bool XF = false>
static bool launch_mixed_group(int n, const uint8_t* const* w, const int* R, const int* type, int C, const uint8_t* xq,
                               float* const* y, hipStream_t s, uint8_t* xqo = nullptr) {
    const int G = C / QK;
    if (G > 16 || n < 2 || n > 3) return false;
    int n4 = 0;
    for (int i = 0; i < n; i++) n4 += type[i] == TYPE_Q4_K;
    if (n4 == 0 || n4 == n) return false;
    // part B: the type with one matrix (Q6_K when there is one of each)
    const int tb = n - n4 == 1 ? TYPE_Q6_K : TYPE_Q4_K;
    const uint8_t* wa[2];
    int ra[2], na = 0, ib = 0;
    float* ya[2];
    for (int i = 0; i < n; i++) {
        if (type[i] == tb) { ib = i; continue; }
        wa[na] = w[i]; ra[na] = R[i]; ya[na] = y[i]; na++;
    }
    if (tb == TYPE_Q6_K)
        launch_mixed<TYPE_Q4_K, 2, TYPE_Q6_K, 1, AP, XF>(wa, ra, ya, na, w[ib], R[ib], y[ib], xq, G, s, xqo);
    else
        launch_mixed<TYPE_Q6_K, 1, TYPE_Q4_K, 2, AP, XF>(wa, ra, ya, na, w[ib], R[ib], y[ib], xq, G, s, xqo);
    return true;
}

bool launch_gemv_q8k_x_mixed(int n, const uint8_t* const* w, const int* R, const int* type, int C, const float* x,
                             float* const* y, uint8_t* xqo, hipStream_t s) {
    return launch_mixed_group<ActQ8K, true>(n, w, R, type, C, reinterpret_cast<const uint8_t*>(x), y, s, xqo);
}

bool launch_gemv_q8k_mixed(int n, const uint8_t* const* w, const int* R, const int* type, int C, const uint8_t* xq,
                           float* const* y, hipStream_t s) {
    return launch_mixed_group<ActQ8K>(n, w, R, type, C, xq, y, s);
}

bool launch_gemv_f32_mixed(int n, const uint8_t* const* w, const int* R, const int* type, int C, const float* x,
                           float* const* y, hipStream_t s) {
    return launch_mixed_group<ActF32>(n, w, R, type, C, reinterpret_cast<const uint8_t*>(x), y, s);
}

// One token of fp32 activations, n (1..3) matrices of one type, C <= 4096: x quantized inside the GEMV
// launch (k_gemv_q8k_x); xqo (nullable) receives the Q8_K bytes.  The grid is launch3's for one pass.
void launch_gemv_q8k_x_group(int n, const uint8_t* const* w, const int* R, int C, int type, const float* x,
                             float* const* y, uint8_t* xqo, hipStream_t s) {
    const int G = C / QK;
    const int rpw = type == TYPE_Q4_K ? 2 : 1;
    MatGroup mg{};
    mg.n = n;
    int total = 0;
    for (int i = 0; i < n; i++) {
        mg.w[i] = w[i];
        mg.y[i] = y[i];
        mg.ldy[i] = R[i];
        mg.first_unit[i] = total;
        total += R[i] / rpw;
    }
    for (int i = n; i < 4; i++) mg.first_unit[i] = total;
    constexpr int K = KQ_GEMV_WG_WAVES;
    int streams = device_cus() * (type == TYPE_Q6_K ? KQ_GEMV_WAVES_PER_CU_Q6 : KQ_GEMV_WAVES_PER_CU);
    if (streams > total) streams = total;
    const int nwg = (((streams + K - 1) / K) + KQ_XCDS - 1) / KQ_XCDS * KQ_XCDS;
    const size_t lds = (size_t)(G + 1) * Q8K_BYTES;   // + a spare slot for the waves' blocks past G
    const uint8_t* xb = reinterpret_cast<const uint8_t*>(x);
    if (type == TYPE_Q4_K)
        hipLaunchKernelGGL((k_gemv_q8k_x<TYPE_Q4_K, 2>), dim3(nwg), dim3(64 * K), lds, s, mg.w[0], mg.w[1], mg.w[2], xb,
                           G, total, mg.first_unit[1], mg.first_unit[2], nwg, mg, xqo);
    else
        hipLaunchKernelGGL((k_gemv_q8k_x<TYPE_Q6_K, 1>), dim3(nwg), dim3(64 * K), lds, s, mg.w[0], mg.w[1], mg.w[2], xb,
                           G, total, mg.first_unit[1], mg.first_unit[2], nwg, mg, xqo);
}

// One token, one matrix, and the argmax of y (output head + greedy pick).  With one column pass
// (C <= 4096) the GEMV itself finds it; otherwise a separate argmax launch follows.
void launch_gemv_q8k_argmax(const uint8_t* w, int R, int C, int type, const uint8_t* xq, float* y, uint8_t* aws,
                            int* aout, hipStream_t s) {
    const int G = C / QK;
    if (G > 16) {
        int64_t ldy = R;
        launch_gemv_q8k_group(1, &w, &R, C, type, xq, 1, &y, &ldy, s);
        launch_argmax(y, R, aws, aout, s);
        return;
    }
    MatGroup mg{};
    mg.n = 1;
    mg.w[0] = w;
    mg.y[0] = y;
    mg.ldy[0] = R;
    mg.first_unit[0] = 0;
    for (int i = 1; i < 4; i++) mg.first_unit[i] = R / 8;
    if (type == TYPE_Q4_K) launch3<TYPE_Q4_K, 1, 2, true>(mg, xq, G, s, aws, aout);
    else launch3<TYPE_Q6_K, 1, 1, true>(mg, xq, G, s, aws, aout);
}

void launch_gemv_q8k(const uint8_t* w, int R, int C, int type, const uint8_t* xq, int N, float* y,
                     int64_t ldy, hipStream_t s) {
    launch_gemv_q8k_group(1, &w, &R, C, type, xq, N, &y, &ldy, s);
}

// fp32 activations: n (1..3) matrices of one type sharing x, one launch.  Two rows per unit for
// Q4_K, one for Q6_K, as the Q8_K GEMV takes them.
void launch_gemv_f32_group(int n, const uint8_t* const* w, const int* R, int C, int type, const float* x,
                           float* const* y, hipStream_t s) {
    const int G = C / QK;
    MatGroup mg{};
    mg.n = n;
    int tiles = 0;
    for (int i = 0; i < n; i++) {
        mg.w[i] = w[i];
        mg.y[i] = y[i];
        mg.ldy[i] = R[i];
        mg.first_unit[i] = tiles;
        tiles += R[i] / 8;
    }
    for (int i = n; i < 4; i++) mg.first_unit[i] = tiles;
    const uint8_t* xb = reinterpret_cast<const uint8_t*>(x);
    if (type == TYPE_Q4_K) launch3<TYPE_Q4_K, 1, 2, false, ActF32>(mg, xb, G, s);
    else launch3<TYPE_Q6_K, 1, 1, false, ActF32>(mg, xb, G, s);
}

}  // namespace kq
