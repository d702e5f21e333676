// Prefill GEMM for gfx950: Y[m][n] = sum_k x_q8[m][k] * W[n][k], Q4_K / Q6_K weights in the Kindi
// layout, Q8_K activations, int8 MFMA with int32 accumulation and an fp32 epilogue per super-block.
//
// Weight planes.  The sub-block scale changes every 32 (Q4_K) or 16 (Q6_K) columns, faster than
// an MFMA K step can absorb, so it is folded into the weights, and the folded weight is split
// into two int8 planes; one super-block (K = 256) is two int8 MFMA sweeps that accumulate exact
// integers:
//   Q4_K  sc (6 bit) = 8a + b with a, b in 0..7; plane H = a*q, plane L = b*q (both <= 105);
//         I1 = 8 * (x . H) + (x . L) = sum sc*q*x.  Each plane is one packed 16-bit multiply of
//         four nibbles by a (no carry crosses a byte since a*q < 256).
//   Q6_K  w = sc*(q-32) in [-4096, 4064] (the -32 offset is folded in as well); v = w + 128 as
//         int16: plane H = high byte of v (-16..16), plane L = low byte of v ^ 0x80 = low byte of
//         w as int8; I = 256 * (x . H) + (x . L) = sum w*x.
// The Q4_K min term I2 = sum_s m_s * B_s (B_s = sum of the activation quants of sub-block s, from
// the Q8_K bsums) is one fp16 MFMA with K = 16: activation side [B_s >> 6, B_s & 63], weight
// side [-64 m_s, -m_s]; every operand and product is an exact fp16 / fp32 integer, so the MFMA
// returns -I2 exactly.  Per super-block the fp32 epilogue adds
//   Q4_K: dx * (d * I1 - dmin * I2)          Q6_K: dx * (d * I)
// (the per-super-block quantity of the CPU reference, with fp32 sums along K).
//
// Work split.  A workgroup (4 waves) owns 128 tokens x 64 weight rows; each wave 32 tokens x 64
// rows (two 32x32 MFMA tiles sharing the A operand).  Each thread unpacks 64 of the 256 weights of
// one weight row into the two LDS planes (rows of 256 B, 16-B chunks XOR-swizzled by row so that
// 16 consecutive rows hit distinct banks); the planes are double-buffered, so the next super-block is unpacked while
// the MFMAs of the current one run, with one barrier per super-block.  A workgroup takes 80 KB of
// LDS and its waves at most 256 VGPRs, so two workgroups share a CU: each SIMD runs two waves and
// one wave's VALU work (unpack, epilogue) issues while the other's MFMAs run.
//
// Activation fragments.  An MFMA A operand holds 16 bytes of each of 32 token rows, so reading
// it straight from Q8_K rows touches 32-64 cache lines per load instruction, for every weight
// tile.  A first pass (k_q8k_frag) rewrites the quants once into fragment order,
//   frag[m/32][g][ks 0..7][lane 0..63][16 B] = qs bytes 32ks + 16(lane/32) .. +15 of row 32(m/32) + lane%32,
// so each A load is one contiguous 1 KB; rows are padded to a multiple of 256 with zeros.  This
// needs a caller workspace (kq_gemm_q8k_ws); without one (kq_gemm_q8k, which allocates nothing)
// the fragments are read from the Q8_K rows directly.  The next super-block's raw weight bytes
// and activation fragments are loaded one step ahead.  Rows past M or R are clamped for loading
// and not stored.
//
// K split.  When the output tiles are too few to fill the GPU (small M, or few weight rows), each
// tile is computed by S workgroups, each over a contiguous range of super-blocks, into S partial
// planes of the workspace; k_gemm_reduce then adds the planes in order s = 0, 1, ...  The split
// depends only on (R, C, M), so results are deterministic; it needs the workspace, so kq_gemm_q8k
// (no workspace) never splits.
//
// Matrices sharing the activations (q/k/v, gate/up) can go in one call: one fragment copy, and one
// GEMM launch per weight type whose grid holds every matrix's tiles (and splits), so that small
// matrices fill the GPU together; each matrix keeps its own split, so its results do not change.
#include <atomic>
#include <mutex>
#include <type_traits>

#include "kq_device.h"
#include "kq_internal.h"

namespace kq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));
typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int GM_BMAX = 256;  // largest token tile: the fragment workspace is padded to it


// Byte offset of 16-byte chunk `c` (0..15) of LDS plane row `r`: rows are 256 B, the chunk index
// is XORed with the row's low 4 bits.
__device__ __forceinline__ int swz(int r, int c) { return r * 256 + ((c ^ (r & 15)) << 4); }

// Four bytes q (each < 16) times s in 0..7, per byte: two 16-bit lanes multiplied at once.
__device__ __forceinline__ uint32_t mul_u8x4(uint32_t q, uint32_t s2) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, q) * __builtin_bit_cast(u16x2, s2));
}
__device__ __forceinline__ uint32_t pk_f16(float a, float b) {   // exact small integers only
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}
__device__ __forceinline__ void st16(int8_t* p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    *reinterpret_cast<u32x4*>(p) = u32x4{a, b, c, d};
}

// One LDS buffer (the kernel double-buffers with two of them: distinct objects, so the compiler
// knows the next super-block's stores never alias the current one's loads).
template <int BN, int BM> struct GemmBuf {
    int8_t wh[BN * 256];
    int8_t wl[BN * 256];
    uint32_t wmin[BN * 8];      // Q4_K: row n = 16 f16 [-64 m_0..7, -m_0..7]
    uint32_t xmin[BM * 8];      // Q4_K: row m = 16 f16 [B_0..7 >> 6, B_0..7 & 63]
    float d[BN], dm[BN], dx[BM];
};

// ------------------------------------------------------------------ weight parts
// Each thread owns one part of one weight row per super-block: part pi of PPR (2 or 4) parts.
//   Q4_K: NPP = 4/PPR consecutive 64-element chunks p (qs bytes 32p..32p+31: sub-blocks 2p, 2p+1).
//   Q6_K: half h of the super-block and NJ = 4/PPR of its two 16-column slices jj (elements
//         128h + 32k + 16jj + 0..15 for k = 0..3: ql bytes 64h + 32(k&1) + 16jj, qh bytes
//         32h + 16jj, scale 8h + 2k + jj).
template <int TYPE, int PPR> struct RawW;
template <int PPR> struct RawW<TYPE_Q4_K, PPR> {
    static constexpr int NPP = 4 / PPR;
    u32x4 hdr, q[2 * NPP];
};
struct Chunk20 { u32x4 v; uint32_t e; };   // 20 bytes from a dword-aligned address
template <int PPR> struct RawW<TYPE_Q6_K, PPR> {
    static constexpr int NJ = 4 / PPR;
    Chunk20 ql[NJ][2], qh[NJ];
    u32x2 sc;
    uint32_t sce, dw, sh;
};

template <int PPR>
__device__ __forceinline__ void load_raw(RawW<TYPE_Q4_K, PPR>& r, const uint8_t* bk, int pi) {
    constexpr int NPP = RawW<TYPE_Q4_K, PPR>::NPP;
    r.hdr = ld16(bk);
#pragma unroll
    for (int pp = 0; pp < NPP; pp++)
#pragma unroll
        for (int c = 0; c < 2; c++) r.q[2 * pp + c] = ld16(bk + 16 + 32 * (pi * NPP + pp) + 16 * c);
}

__device__ __forceinline__ Chunk20 ld20(const uint8_t* p) { return Chunk20{ld16_a4(p), ld4(p + 16)}; }

// Q6_K blocks start at 0 or 2 (mod 4); every field is read from the dword at or below it and
// funnel-shifted by the block's shift.  The last dword read (bytes 208..211 from the aligned
// base) passes the block end by 2 bytes only for blocks starting at 0 (mod 4), which are never
// row 7 of a tile column, so the bytes belong to the next block of the same buffer.
template <int PPR>
__device__ __forceinline__ void load_raw(RawW<TYPE_Q6_K, PPR>& r, const uint8_t* bk, int pi) {
    constexpr int NJ = RawW<TYPE_Q6_K, PPR>::NJ;
    const int h = NJ == 2 ? pi : pi >> 1, jj0 = NJ == 2 ? 0 : pi & 1;
    r.sh = uint32_t(reinterpret_cast<uintptr_t>(bk) & 3);
    const uint8_t* b4 = bk - r.sh;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int jj = jj0 + j;
        r.ql[j][0] = ld20(b4 + 64 * h + 16 * jj);
        r.ql[j][1] = ld20(b4 + 64 * h + 32 + 16 * jj);
        r.qh[j] = ld20(b4 + 128 + 32 * h + 16 * jj);
    }
    r.sc = *reinterpret_cast<const u32x2_a4*>(b4 + 192 + 8 * h);
    r.sce = ld4(b4 + 200 + 8 * h);
    r.dw = ld4(b4 + 208);
}

// Unpack into LDS buffer Lb, weight row `row` (0..BN-1).
template <int PPR, int BN, int BM>
__device__ __forceinline__ void unpack(const RawW<TYPE_Q4_K, PPR>& r, int pi, int row, GemmBuf<BN, BM>& Lb) {
    constexpr int NPP = RawW<TYPE_Q4_K, PPR>::NPP;
    int8_t* wh = Lb.wh;
    int8_t* wl = Lb.wl;
#pragma unroll
    for (int pp = 0; pp < NPP; pp++) {
        const int p = pi * NPP + pp;
        const ScMin sm = q4k_scmin_pair(r.hdr.y, r.hdr.z, r.hdr.w, p);
        const uint32_t alo = (sm.sc_lo >> 3) * 0x10001u, blo = (sm.sc_lo & 7u) * 0x10001u;
        const uint32_t ahi = (sm.sc_hi >> 3) * 0x10001u, bhi = (sm.sc_hi & 7u) * 0x10001u;
#pragma unroll
        for (int c = 0; c < 2; c++) {          // elements 64p + 16c + 0..15 (lo), 64p + 32 + 16c (hi)
            const u32x4 v = r.q[2 * pp + c];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            uint32_t h0[4], l0[4], h1[4], l1[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t lo = w[i] & 0x0f0f0f0fu, hi = (w[i] >> 4) & 0x0f0f0f0fu;
                h0[i] = mul_u8x4(lo, alo);
                l0[i] = mul_u8x4(lo, blo);
                h1[i] = mul_u8x4(hi, ahi);
                l1[i] = mul_u8x4(hi, bhi);
            }
            const int c0 = 4 * p + c, c1 = 4 * p + 2 + c;   // 16-byte chunk indices
            st16(wh + swz(row, c0), h0[0], h0[1], h0[2], h0[3]);
            st16(wl + swz(row, c0), l0[0], l0[1], l0[2], l0[3]);
            st16(wh + swz(row, c1), h1[0], h1[1], h1[2], h1[3]);
            st16(wl + swz(row, c1), l1[0], l1[1], l1[2], l1[3]);
        }
        const float mlo = (float)sm.m_lo, mhi = (float)sm.m_hi;
        Lb.wmin[row * 8 + p] = pk_f16(-64.0f * mlo, -64.0f * mhi);
        Lb.wmin[row * 8 + 4 + p] = pk_f16(-mlo, -mhi);
    }
    // every part of the row stores the same d / dmin: no branch in the main loop
    Lb.d[row] = f16_lo(r.hdr.x);
    Lb.dm[row] = f16_hi(r.hdr.x);
}

template <int PPR, int BN, int BM>
__device__ __forceinline__ void unpack(const RawW<TYPE_Q6_K, PPR>& r, int pi, int row, GemmBuf<BN, BM>& Lb) {
    constexpr int NJ = RawW<TYPE_Q6_K, PPR>::NJ;
    const int h = NJ == 2 ? pi : pi >> 1, jj0 = NJ == 2 ? 0 : pi & 1;
    int8_t* wh = Lb.wh;
    int8_t* wl = Lb.wl;
    const uint32_t sh = r.sh;
    const uint32_t s0 = __builtin_amdgcn_alignbyte(r.sc.y, r.sc.x, sh);   // scales 8h .. 8h+3
    const uint32_t s1 = __builtin_amdgcn_alignbyte(r.sce, r.sc.y, sh);    // scales 8h+4 .. 8h+7
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int jj = jj0 + j;
        uint32_t Lw[2][4], Hw[4];
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const Chunk20 c = r.ql[j][t];
            Lw[t][0] = __builtin_amdgcn_alignbyte(c.v.y, c.v.x, sh);
            Lw[t][1] = __builtin_amdgcn_alignbyte(c.v.z, c.v.y, sh);
            Lw[t][2] = __builtin_amdgcn_alignbyte(c.v.w, c.v.z, sh);
            Lw[t][3] = __builtin_amdgcn_alignbyte(c.e, c.v.w, sh);
        }
        {
            const Chunk20 c = r.qh[j];
            Hw[0] = __builtin_amdgcn_alignbyte(c.v.y, c.v.x, sh);
            Hw[1] = __builtin_amdgcn_alignbyte(c.v.z, c.v.y, sh);
            Hw[2] = __builtin_amdgcn_alignbyte(c.v.w, c.v.z, sh);
            Hw[3] = __builtin_amdgcn_alignbyte(c.e, c.v.w, sh);
        }
#pragma unroll
        for (int k = 0; k < 4; k++) {              // elements 128h + 32k + 16jj + 0..15
            const uint32_t scw = k < 2 ? s0 : s1;
            const int sc = (int)(int8_t)(uint8_t)(scw >> (8 * ((2 * k + jj) & 3)));
            const uint32_t s2 = (uint32_t)(sc & 0xffff) * 0x10001u;
            const uint32_t c2 = (uint32_t)((128 - 32 * sc) & 0xffff) * 0x10001u;
            uint32_t hb[4], lb[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t lq = (Lw[k & 1][i] >> (4 * (k >> 1))) & 0x0f0f0f0fu;
                const uint32_t hq = ((Hw[i] >> (2 * k)) & 0x03030303u) << 4;
                const uint32_t q = lq | hq;                                  // 6-bit codes, 4 bytes
                const uint32_t e = __builtin_amdgcn_perm(0u, q, 0x0c020c00u);    // bytes 0, 2 -> 16-bit lanes
                const uint32_t o = __builtin_amdgcn_perm(0u, q, 0x0c030c01u);    // bytes 1, 3
                const s16x2 sv = __builtin_bit_cast(s16x2, s2), cv = __builtin_bit_cast(s16x2, c2);
                const uint32_t ve = __builtin_bit_cast(uint32_t, (s16x2)(__builtin_bit_cast(s16x2, e) * sv + cv));
                const uint32_t vo = __builtin_bit_cast(uint32_t, (s16x2)(__builtin_bit_cast(s16x2, o) * sv + cv));
                hb[i] = __builtin_amdgcn_perm(vo, ve, 0x07030501u);              // high bytes, element order
                lb[i] = __builtin_amdgcn_perm(vo, ve, 0x06020400u) ^ 0x80808080u;
            }
            const int ch = 8 * h + 2 * k + jj;
            st16(wh + swz(row, ch), hb[0], hb[1], hb[2], hb[3]);
            st16(wl + swz(row, ch), lb[0], lb[1], lb[2], lb[3]);
        }
    }
    Lb.d[row] = f16_lo(r.dw >> (8 * sh));   // same value from every part of the row
}

// ------------------------------------------------------------------ activation side
// XP (2 or 4) threads share an activation row: thread part xp holds bsums (16/XP) xp .. +16/XP-1,
// i.e. NB = 8/XP of the Q4_K sub-block sums, and the row's d.
template <int XP> struct RawX {
    static constexpr int NB = 8 / XP;
    uint32_t bs[NB], d;
};

template <int XP>
__device__ __forceinline__ void load_x(RawX<XP>& r, const uint8_t* xb, int xp) {
    const uint8_t* p = xb + 260 + 4 * RawX<XP>::NB * xp;
    if constexpr (RawX<XP>::NB == 4) {
        const u32x4 v = ld16_a4(p);
        r.bs[0] = v.x; r.bs[1] = v.y; r.bs[2] = v.z; r.bs[3] = v.w;
    } else {
        const u32x2 v = *reinterpret_cast<const u32x2_a4*>(p);
        r.bs[0] = v.x; r.bs[1] = v.y;
    }
    r.d = ld4(xb);
}

template <int TYPE, int XP, int BN, int BM>
__device__ __forceinline__ void stage_x(const RawX<XP>& r, int mr, int xp, GemmBuf<BN, BM>& Lb) {
    constexpr int NB = RawX<XP>::NB;
    if (TYPE == TYPE_Q4_K) {
        // B_s = bsum[2s] + bsum[2s+1] for s = NB*xp .. NB*xp+NB-1, split as 64 * (B >> 6) + (B & 63)
        int B[NB];
#pragma unroll
        for (int i = 0; i < NB; i++) B[i] = (int)(int16_t)(r.bs[i] & 0xffffu) + (int)(int16_t)(r.bs[i] >> 16);
#pragma unroll
        for (int i = 0; i < NB; i += 2) {
            const int dw = mr * 8 + (NB * xp + i) / 2;
            Lb.xmin[dw] = pk_f16((float)(B[i] >> 6), (float)(B[i + 1] >> 6));
            Lb.xmin[dw + 4] = pk_f16((float)(B[i] & 63), (float)(B[i + 1] & 63));
        }
    }
    Lb.dx[mr] = __builtin_bit_cast(float, r.d);   // same value from every part of the row
}

// ------------------------------------------------------------------ the kernel
// One launch covers up to three matrices of one type that share the activations (q/k/v, gate/up):
// workgroup x = wg0 of its matrix + split * ntile + weight tile (weight tile fastest), y = token
// tile.  Each matrix keeps the K split a call of its own would take, so its results are those of
// that call bit for bit.
struct GemmMat {
    const uint8_t* w;
    float* y;
    float* part;      // partial planes of the K split (S of M x R floats), or null
    int64_t ldy;
    int R, ntile, gps, wg0;
};
struct GemmGroup {
    GemmMat m[3];
    int n;
};

// WN waves along n times WM along m; each wave owns MT token tiles x NT = 2/MT weight-row tiles of
// 32x32 (two MFMA tiles), the workgroup BM = 32*MT*WM tokens x BN = 32*NT*WN rows.  With MT = 1 a wave
// holds one token tile's A operands (32 VGPRs for a super-block) and uses each for both row tiles,
// reading twice the B operands from LDS instead.  FRAG: A operands from the fragment-order copy XF,
// else straight from the Q8_K rows XQ.
template <int TYPE, int BN, int WN, int WM, bool FRAG, int MT>
__global__ void __launch_bounds__(64 * WN * WM)
k_gemm_q8k(GemmGroup gg, int G, const uint8_t* __restrict__ XQ, const uint8_t* __restrict__ XF, int M) {
    constexpr int BS = TYPE == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    constexpr int BM = 32 * MT * WM;
    constexpr int NTHR = 64 * WN * WM;
    constexpr int NE = BN / WN;                   // weight rows per wave
    constexpr int NT = NE / 32;                   // 32-column MFMA tiles per wave
    constexpr int PPR = NTHR / BN;                // unpack parts per weight row
    constexpr int XP = NTHR / BM;                 // staging parts per activation row
    constexpr int SHIFT = TYPE == TYPE_Q4_K ? 3 : 8;
    static_assert(PPR == 2 || PPR == 4, "a weight row is split in 2 or 4 parts");
    static_assert(NT * MT == 2, "two 32x32 tiles per wave");
    __shared__ __attribute__((aligned(16))) GemmBuf<BN, BM> LB0;
    __shared__ __attribute__((aligned(16))) GemmBuf<BN, BM> LB1;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WM, wn = wave / WM;
    const int half = lane >> 5, l32 = lane & 31;
    // this workgroup's matrix (the argument fields picked by selects on the wave-uniform index)
    const int bx = blockIdx.x;
    const int mi = gg.n > 1 && bx >= gg.m[1].wg0 ? (gg.n > 2 && bx >= gg.m[2].wg0 ? 2 : 1) : 0;
    auto field = [&](auto get) { return mi == 0 ? get(gg.m[0]) : mi == 1 ? get(gg.m[1]) : get(gg.m[2]); };
    const uint8_t* const W = field([](const GemmMat& g) { return g.w; });
    float* const Y = field([](const GemmMat& g) { return g.y; });
    float* const P = field([](const GemmMat& g) { return g.part; });
    const int64_t ldy = field([](const GemmMat& g) { return g.ldy; });
    const int R = field([](const GemmMat& g) { return g.R; });
    const int ntile = field([](const GemmMat& g) { return g.ntile; });
    const int gps = field([](const GemmMat& g) { return g.gps; });
    const int local = bx - field([](const GemmMat& g) { return g.wg0; });
    const int split = local / ntile;
    const int n0 = (local - split * ntile) * BN, m0 = blockIdx.y * BM;
    const int64_t xrow = (int64_t)G * Q8K_BYTES;
    // super-blocks [gbeg, gend) of the K split (all of them without one); with P the sums go to
    // partial plane `split` (rows of R floats) instead of Y
    const int gbeg = split * gps, gend = gbeg + gps < G ? gbeg + gps : G;
    float* const Yo = P ? P + (int64_t)split * M * R : Y;
    const int64_t ldo = P ? (int64_t)R : ldy;

    // A operand of this lane for K step ks of super-block g: afrag[mt] + g * AG + ks * AK
    constexpr int AG = FRAG ? 8192 : Q8K_BYTES, AK = FRAG ? 1024 : 32;
    const uint8_t* afrag[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        if (FRAG) {   // fragment tile (m0 + 32 MT wm + 32 mt) / 32
            afrag[mt] = XF + ((int64_t)(blockIdx.y * (BM / 32) + MT * wm + mt) * G * 512 + lane) * 16;
        } else {      // row m, bytes 32 ks + 16 half of its quants
            int m = m0 + 32 * MT * wm + 32 * mt + l32;
            m = m < M ? m : M - 1;
            afrag[mt] = XQ + m * xrow + 4 + 16 * half;
        }
    }
    // activation row staged by this thread
    const int mr = tid % BM, xp = tid / BM;
    const uint8_t* xstage = XQ + (int64_t)(m0 + mr < M ? m0 + mr : M - 1) * xrow;
    // weight row part unpacked by this thread
    const int prow = tid % BN, pi = tid / BN;
    const int pr = n0 + prow < R ? n0 + prow : R - 1;
    const uint8_t* wrow = W + ((int64_t)(pr >> 3) * G * 8 + (pr & 7)) * BS;   // block (pr, g) = wrow + g*8*BS

    float yacc[2][16];                      // tile t = mt * NT + nt
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int a = 0; a < 16; a++) yacc[t][a] = 0.0f;

    // ---- prologue: super-block 0 staged, super-block 1's raw bytes in registers
    RawW<TYPE, PPR> raw;
    RawX<XP> rx;
    v4i afr[MT][8];
    load_raw(raw, wrow + (int64_t)gbeg * 8 * BS, pi);
    load_x(rx, xstage + (int64_t)gbeg * Q8K_BYTES, xp);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
            afr[mt][ks] = __builtin_bit_cast(v4i, ld16_a4(afrag[mt] + (int64_t)gbeg * AG + ks * AK));
    unpack(raw, pi, prow, LB0);
    stage_x<TYPE>(rx, mr, xp, LB0);
    {
        const int g1 = gbeg + 1 < gend ? gbeg + 1 : gbeg;
        load_raw(raw, wrow + (int64_t)g1 * 8 * BS, pi);
        load_x(rx, xstage + (int64_t)g1 * Q8K_BYTES, xp);
    }
    __syncthreads();

    int nrow0[NT];                          // this lane's B rows (weight rows within the tile)
#pragma unroll
    for (int nt = 0; nt < NT; nt++) nrow0[nt] = wn * NE + 32 * nt + l32;
    auto step = [&](auto cur_c, int g) {
        constexpr int cur = decltype(cur_c)::value;
        GemmBuf<BN, BM>& Lc = cur ? LB1 : LB0;   // read this step
        GemmBuf<BN, BM>& Ln = cur ? LB0 : LB1;   // filled for the next step
        const int gn = g + 1 < gend ? g + 1 : gend - 1;
        const int g2 = g + 2 < gend ? g + 2 : gend - 1;
        unpack(raw, pi, prow, Ln);
        stage_x<TYPE>(rx, mr, xp, Ln);
        load_raw(raw, wrow + (int64_t)g2 * 8 * BS, pi);
        load_x(rx, xstage + (int64_t)g2 * Q8K_BYTES, xp);

        // Q6_K: the wave's MFMA sweeps at raised issue priority, so the other wave of the SIMD runs its
        // (heavier) unpack and epilogue in the MFMAs' shadow (4096x12288 at M = 2048 / 512: 303 / 90.1
        // -> 294 / 87.5 us; for Q4_K, whose unpack is interleaved into the hi sweep, it was slower)
        if constexpr (TYPE == TYPE_Q6_K) __builtin_amdgcn_s_setprio(3);
        v16i acc[2];
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            v4i b[NT];
#pragma unroll
            for (int nt = 0; nt < NT; nt++) b[nt] = *reinterpret_cast<const v4i*>(Lc.wh + swz(nrow0[nt], 2 * ks + half));
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    acc[mt * NT + nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr[mt][ks], b[nt],
                                                                             ks == 0 ? v16i{} : acc[mt * NT + nt], 0, 0, 0);
        }
        __builtin_amdgcn_iglp_opt(1);
        __builtin_amdgcn_sched_barrier(0);

        auto epilogue = [&](int mt, int nt) {
            const int t = mt * NT + nt;
            f32x4 dxv[4];
#pragma unroll
            for (int q = 0; q < 4; q++)
                dxv[q] = *reinterpret_cast<const f32x4*>(&Lc.dx[32 * MT * wm + 32 * mt + 8 * q + 4 * half]);
            const int ml = 32 * MT * wm + 32 * mt + l32;
            const float dn = Lc.d[nrow0[nt]];
            if (TYPE == TYPE_Q4_K) {
                const float dmn = Lc.dm[nrow0[nt]];
                const v8h bm = __builtin_bit_cast(v8h, *reinterpret_cast<const u32x4*>(&Lc.wmin[nrow0[nt] * 8 + 4 * half]));
                const v8h am = __builtin_bit_cast(v8h, *reinterpret_cast<const u32x4*>(&Lc.xmin[ml * 8 + 4 * half]));
                const v16f cm = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, v16f{}, 0, 0, 0);   // -I2
#pragma unroll
                for (int a = 0; a < 16; a++) {
                    const float tt = __builtin_fmaf(dmn, cm[a], __fmul_rn(dn, (float)acc[t][a]));
                    yacc[t][a] = __builtin_fmaf(dxv[a >> 2][a & 3], tt, yacc[t][a]);
                }
            } else {
#pragma unroll
                for (int a = 0; a < 16; a++)
                    yacc[t][a] = __builtin_fmaf(dxv[a >> 2][a & 3], __fmul_rn(dn, (float)acc[t][a]), yacc[t][a]);
            }
        };

#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int a = 0; a < 16; a++) acc[t][a] <<= SHIFT;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            v4i b[NT];
#pragma unroll
            for (int nt = 0; nt < NT; nt++) b[nt] = *reinterpret_cast<const v4i*>(Lc.wl + swz(nrow0[nt], 2 * ks + half));
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
                    acc[mt * NT + nt] = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr[mt][ks], b[nt], acc[mt * NT + nt], 0, 0, 0);
                afr[mt][ks] = __builtin_bit_cast(v4i, ld16_a4(afrag[mt] + (int64_t)gn * AG + ks * AK));
            }
        }
        if constexpr (TYPE == TYPE_Q6_K) __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++) epilogue(mt, nt);
        __syncthreads();
    };
    for (int g = gbeg; g < gend; g += 2) {
        step(std::integral_constant<int, 0>{}, g);
        if (g + 1 < gend) step(std::integral_constant<int, 1>{}, g + 1);
    }

#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int n = n0 + nrow0[nt];
#pragma unroll
            for (int a = 0; a < 16; a++) {
                const int m = m0 + 32 * MT * wm + 32 * mt + (a >> 2) * 8 + half * 4 + (a & 3);
                if (m < M && n < R) Yo[(int64_t)m * ldo + n] = yacc[mt * NT + nt][a];
            }
        }
}


// Fragment-order copy of the activation quants (layout above); rows M .. 256*ceil(M/256)-1 are
// zero.  One workgroup per (32-row tile, super-block), 32 bytes per thread.
__global__ void __launch_bounds__(256)
k_q8k_frag(const uint8_t* __restrict__ XQ, int M, int G, uint8_t* __restrict__ XF) {
    const int mt = blockIdx.x, g = blockIdx.y;
    uint8_t* out = XF + ((int64_t)mt * G + g) * 8192;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int t = threadIdx.x + 256 * j;            // 16-byte slot: ks = t / 64, lane = t % 64
        const int ks = t >> 6, lane = t & 63;
        const int row = 32 * mt + (lane & 31);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (row < M) v = ld16_a4(XQ + ((int64_t)row * G + g) * Q8K_BYTES + 4 + 32 * ks + 16 * (lane >> 5));
        *reinterpret_cast<u32x4*>(out + 16 * t) = v;
    }
}

// Partial planes y_s[m][r] of the K split, added in order s = 0 .. S-1: y = ((y_0 + y_1) + y_2) + ...
// One launch for every split matrix of a call: workgroups [blk0[j], blk0[j+1]) serve matrix j, one
// thread per 4 consecutive outputs of a row.
struct ReduceMat {
    const float* part;
    float* y;
    int64_t ldy;
    int R, S, blk0;
};
struct ReduceGroup {
    ReduceMat m[3];
    int n;
};

__global__ void __launch_bounds__(256)
k_gemm_reduce(ReduceGroup rg, int M) {
    const int bx = blockIdx.x;
    const int j = rg.n > 1 && bx >= rg.m[1].blk0 ? (rg.n > 2 && bx >= rg.m[2].blk0 ? 2 : 1) : 0;
    auto field = [&](auto get) { return j == 0 ? get(rg.m[0]) : j == 1 ? get(rg.m[1]) : get(rg.m[2]); };
    const float* const P = field([](const ReduceMat& g) { return g.part; });
    float* const Y = field([](const ReduceMat& g) { return g.y; });
    const int64_t ldy = field([](const ReduceMat& g) { return g.ldy; });
    const int R = field([](const ReduceMat& g) { return g.R; });
    const int S = field([](const ReduceMat& g) { return g.S; });
    const int r4 = R >> 2;
    const int64_t i = (int64_t)(bx - field([](const ReduceMat& g) { return g.blk0; })) * 256 + threadIdx.x;
    if (i >= (int64_t)M * r4) return;
    const int64_t pstride = (int64_t)M * R;
    const int m = (int)(i / r4), r = (int)(i - (int64_t)m * r4) * 4;
    const float* p = P + (int64_t)m * R + r;
    f32x4 a = *reinterpret_cast<const f32x4*>(p);
    for (int s = 1; s < S; s++) {
        const f32x4 b = *reinterpret_cast<const f32x4*>(p + s * pstride);
        a = f32x4{__fadd_rn(a.x, b.x), __fadd_rn(a.y, b.y), __fadd_rn(a.z, b.z), __fadd_rn(a.w, b.w)};
    }
    *reinterpret_cast<f32x4_a4*>(Y + (int64_t)m * ldy + r) = a;
}

// Tiles of the launch below: 64 weight rows x 128 tokens.
constexpr int GM_TN = 64, GM_TM = 128;
// Workgroups that fill the GPU: two per CU of the 256 on an MI355X (fixed, so the split and the
// workspace size do not depend on the device).  Measured (us, unsplit -> split): 4096x12288 Q6_K
// at M = 32 / 64 / 128 / 256 / 512: 91.7 / 93.4 / 98.4 / 99.9 / 103.2 -> 34.6 / 35.9 / 38.1 /
// 57.8 / 96.1; 12288x4096 Q4_K at M = 32 / 64: 33.6 / 33.5 -> 31.5 / 33.0.
constexpr int GM_FILL = 512;
constexpr int GM_SPLIT_MIN = 4;     // super-blocks per split, at least
#ifndef KQ_GEMM_SPLIT_MAX
#define KQ_GEMM_SPLIT_MAX 8
#endif
constexpr int GM_SPLIT_MAX = KQ_GEMM_SPLIT_MAX;

// Super-blocks per split (gps) and splits (S) for a GEMM of R rows, C columns, M tokens.
static void gemm_split(int R, int C, int M, int& S, int& gps) {
    const int G = C / QK;
    const int64_t tiles = (int64_t)((R + GM_TN - 1) / GM_TN) * ((M + GM_TM - 1) / GM_TM);
    S = 1;
    if (tiles < GM_FILL) {
        int64_t want = GM_FILL / tiles;              // all S x tiles workgroups resident at once
        // a 2- or 3-way split (the grid already covers more than half the CUs) of a short K saves
        // less than adding the partial sums costs (12288x4096, M = 128: 36.6 against 34.6 us)
        if (want < 4 && G < 32) want = 1;
        want = want < GM_SPLIT_MAX ? want : GM_SPLIT_MAX;
        const int most = G / GM_SPLIT_MIN;
        S = (int)(want < most ? want : most);
        if (S < 1) S = 1;
    }
    gps = (G + S - 1) / S;
    S = (G + gps - 1) / gps;        // no empty split
}

static size_t frag_bytes(int C, int M) { return (size_t)((M + GM_BMAX - 1) / GM_BMAX) * GM_BMAX * (size_t)C; }

// Workspace of a call over n matrices sharing the activations: the fragment copy (256-byte
// aligned), then the partial planes of each matrix that splits K, back to back (multiples of 32
// bytes: R is a multiple of 8).  For one matrix this is kq_gemm_q8k_workspace.
size_t gemm_q8k_group_workspace(int n, const int* R, int C, int M) {
    size_t total = (frag_bytes(C, M) + 255) / 256 * 256;
    for (int i = 0; i < n; i++) {
        int S, gps;
        gemm_split(R[i], C, M, S, gps);
        if (S > 1) total += (size_t)S * M * R[i] * sizeof(float);
    }
    return total;
}

size_t gemm_q8k_workspace(int R, int C, int M) { return gemm_q8k_group_workspace(1, &R, C, M); }

template <int TYPE, int BN, int WN, int WM, int MT>
static void launch_tile(const GemmGroup& gg, int wgs, int G, const uint8_t* xq, const uint8_t* xf, int M,
                        const int* S, hipStream_t s) {
    constexpr int BM = 32 * MT * WM;
    static_assert(BN == GM_TN && BM == GM_TM, "the split rule assumes these tiles");
    dim3 grid(wgs, (M + BM - 1) / BM), block(64 * WN * WM);
    if (xf)
        hipLaunchKernelGGL((k_gemm_q8k<TYPE, BN, WN, WM, true, MT>), grid, block, 0, s, gg, G, xq, xf, M);
    else
        hipLaunchKernelGGL((k_gemm_q8k<TYPE, BN, WN, WM, false, MT>), grid, block, 0, s, gg, G, xq, xf, M);
    // one reduce launch for the matrices that split K
    ReduceGroup rg{};
    int blks = 0;
    for (int i = 0; i < gg.n; i++) {
        const GemmMat& mt = gg.m[i];
        if (!mt.part) continue;
        ReduceMat& rm = rg.m[rg.n++];
        rm.part = mt.part;
        rm.y = mt.y;
        rm.ldy = mt.ldy;
        rm.R = mt.R;
        rm.S = S[i];
        rm.blk0 = blks;
        blks += (int)(((int64_t)M * (mt.R / 4) + 255) / 256);
    }
    if (rg.n) hipLaunchKernelGGL(k_gemm_reduce, dim3(blks), dim3(256), 0, s, rg, M);
}

template <int TYPE>
static void launch_type(const GemmGroup& gg, int wgs, int G, const uint8_t* xq, const uint8_t* xf, int M,
                        const int* S, hipStream_t s) {
    // 128 tokens x 64 weight rows per workgroup of 4 waves (80 KB of LDS, at most 256 VGPRs), so two
    // workgroups share a CU and each SIMD holds two waves: one wave's unpack and epilogue run under
    // the other's MFMAs.  Each wave takes 32 tokens x all 64 rows (MT = 1): half the A-operand
    // loads of 64 tokens x 32 rows (MT = 2), for twice the B reads from LDS; 12288x4096 Q4_K at
    // M = 2048 / 512 / 256: 285 / 76.8 / 49.3 -> 270 / 73.8 / 45.7 us, 4096x12288 Q6_K 311 / 91.2
    // -> 300 / 88.1 us.  (Measured against 128 x 128 tiles, one wave per SIMD, 4-8 waves per
    // workgroup: 289-317 against 331-379 us at M = 2048.)
    launch_tile<TYPE, 64, 1, 4, 1>(gg, wgs, G, xq, xf, M, S, s);
}

// ------------------------------------------------------------------ the no-allocation form
// Workspace of kq_gemm_q8k_static: a file-scope device array, one copy per device, held until the
// process ends.  Its name is a host-side stand-in in host code; kernels get the device address that
// hipGetSymbolAddress returns, looked up once per device (with that device current) on the first
// call there.  Every call on a device shares that device's copy.
static __device__ __align__(256) uint8_t scratch[KQ_GEMM_STATIC_SCRATCH_BYTES];

constexpr int SCRATCH_DEVICES = 64;
static std::atomic<uint8_t*> g_scratch[SCRATCH_DEVICES];
static std::mutex g_scratch_mu;

int gemm_static_scratch(uint8_t** out, const char* fn) {
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(KQ_ERR_HIP, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
    if (dev < 0 || dev >= SCRATCH_DEVICES)
        return fail(KQ_ERR_ARG, "%s: device %d beyond the %d the library tracks", fn, dev, SCRATCH_DEVICES);
    uint8_t* p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (!p) {
            void* addr = nullptr;
            const hipError_t r = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
            if (r != hipSuccess || !addr)
                return fail(KQ_ERR_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev,
                            hipGetErrorString(r));
            p = static_cast<uint8_t*>(addr);
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return KQ_OK;
}

void launch_gemm_q8k_group(int n, const uint8_t* const* w, const int* R, int C, const int* type, const uint8_t* xq,
                           int M, float* const* y, const int64_t* ldy, uint8_t* ws, hipStream_t s, bool frag_ready) {
    const int G = C / QK;
    if (ws && !frag_ready) {   // one fragment copy serves every matrix of the call
        dim3 fgrid((M + GM_BMAX - 1) / GM_BMAX * (GM_BMAX / 32), G);
        hipLaunchKernelGGL(k_q8k_frag, fgrid, dim3(256), 0, s, xq, M, G, ws);
    }
    // each matrix's split and partial planes, as a call of its own would take them
    int S[3], gps[3];
    float* part[3];
    size_t off = (frag_bytes(C, M) + 255) / 256 * 256;
    for (int i = 0; i < n; i++) {
        S[i] = 1;
        gps[i] = G;
        part[i] = nullptr;
        if (ws) {
            gemm_split(R[i], C, M, S[i], gps[i]);
            if (S[i] > 1) {
                part[i] = reinterpret_cast<float*>(ws + off);
                off += (size_t)S[i] * M * R[i] * sizeof(float);
            } else {
                gps[i] = G;
            }
        }
    }
    // one launch per weight type, the matrices of that type in call order
    for (int ty : {TYPE_Q4_K, TYPE_Q6_K}) {
        GemmGroup gg{};
        int Sg[3];
        int wgs = 0;
        for (int i = 0; i < n; i++) {
            if (type[i] != ty) continue;
            GemmMat& mt = gg.m[gg.n];
            mt.w = w[i];
            mt.y = y[i];
            mt.part = part[i];
            mt.ldy = ldy[i];
            mt.R = R[i];
            mt.ntile = (R[i] + GM_TN - 1) / GM_TN;
            mt.gps = gps[i];
            mt.wg0 = wgs;
            Sg[gg.n] = S[i];
            wgs += mt.ntile * S[i];
            gg.n++;
        }
        if (!gg.n) continue;
        if (ty == TYPE_Q4_K) launch_type<TYPE_Q4_K>(gg, wgs, G, xq, ws, M, Sg, s);
        else launch_type<TYPE_Q6_K>(gg, wgs, G, xq, ws, M, Sg, s);
    }
}

static size_t q8k_rows_bytes(int C, int M) { return ((size_t)M * (C / QK) * Q8K_BYTES + 255) / 256 * 256; }

size_t gemm_f32_group_workspace(int n, const int* R, int C, int M) {
    return q8k_rows_bytes(C, M) + gemm_q8k_group_workspace(n, R, C, M);
}

void launch_gemm_f32_group(int n, const uint8_t* const* w, const int* R, int C, const int* type, const float* x,
                           int64_t ldx, int M, float* const* y, const int64_t* ldy, uint8_t* ws, hipStream_t s) {
    uint8_t* xq = ws;
    uint8_t* gws = ws + q8k_rows_bytes(C, M);
    launch_q8k_quantize_frag(x, ldx, C, M, (M + GM_BMAX - 1) / GM_BMAX * GM_BMAX, xq, gws, s);
    launch_gemm_q8k_group(n, w, R, C, type, xq, M, y, ldy, gws, s, true);
}

void launch_gemm_q8k(const uint8_t* w, int R, int C, int type, const uint8_t* xq, int M, float* y, int64_t ldy,
                     uint8_t* ws, hipStream_t s) {
    launch_gemm_q8k_group(1, &w, &R, C, &type, xq, M, &y, &ldy, ws, s);
}

}  // namespace kq
