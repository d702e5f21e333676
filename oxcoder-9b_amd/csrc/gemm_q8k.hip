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

// Kernel entry of the GEMM launches: every field of the three matrix records (and the other scalar
// arguments) read in one batch of loads with one wait, each passing through an empty instruction
// with the workgroup index, so that the matrix picked by that index takes its fields by selects over
// values already in registers.  Left to the compiler, the prologue made four dependent round trips
// of ~0.3 us to the kernel arguments (the field of the selected matrix was reloaded from a computed
// address).  Pointers pass as integers and come back as global pointers (kq_global).
#define KQ_GEMM_ARGS(gg)                                                                              \
    int bx = blockIdx.x;                                                                              \
    int64_t w0_ = (int64_t)(gg).m[0].w, w1_ = (int64_t)(gg).m[1].w, w2_ = (int64_t)(gg).m[2].w;      \
    int64_t y0_ = (int64_t)(gg).m[0].y, y1_ = (int64_t)(gg).m[1].y, y2_ = (int64_t)(gg).m[2].y;      \
    int64_t p0_ = (int64_t)(gg).m[0].part, p1_ = (int64_t)(gg).m[1].part, p2_ = (int64_t)(gg).m[2].part; \
    int64_t l0_ = (gg).m[0].ldy, l1_ = (gg).m[1].ldy, l2_ = (gg).m[2].ldy;                           \
    int R0_ = (gg).m[0].R, R1_ = (gg).m[1].R, R2_ = (gg).m[2].R;                                      \
    int nt0_ = (gg).m[0].ntile, nt1_ = (gg).m[1].ntile, nt2_ = (gg).m[2].ntile;                       \
    int gp0_ = (gg).m[0].gps, gp1_ = (gg).m[1].gps, gp2_ = (gg).m[2].gps;                             \
    int wg1_ = (gg).m[1].wg0, wg2_ = (gg).m[2].wg0, nmat = (gg).n;                                    \
    asm volatile("" : "+s"(bx), "+s"(w0_), "+s"(w1_), "+s"(w2_), "+s"(y0_), "+s"(y1_), "+s"(y2_), "+s"(p0_), \
                 "+s"(p1_), "+s"(p2_), "+s"(l0_), "+s"(l1_), "+s"(l2_), "+s"(R0_), "+s"(R1_), "+s"(R2_),      \
                 "+s"(nt0_), "+s"(nt1_), "+s"(nt2_), "+s"(gp0_), "+s"(gp1_), "+s"(gp2_), "+s"(wg1_), "+s"(wg2_), \
                 "+s"(nmat) : "s"(G), "s"(XQ), "s"(XF), "s"(M));                                     \
    __builtin_amdgcn_sched_barrier(0)

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
    KQ_GEMM_ARGS(gg);
    const int mi = nmat > 1 && bx >= wg1_ ? (nmat > 2 && bx >= wg2_ ? 2 : 1) : 0;
    auto pick = [&](auto a, auto b, auto c) { return mi == 0 ? a : mi == 1 ? b : c; };
    const uint8_t* const W = kq_global<const uint8_t>(pick(w0_, w1_, w2_));
    float* const Y = kq_global<float>(pick(y0_, y1_, y2_));
    float* const P = kq_global<float>(pick(p0_, p1_, p2_));
    const int64_t ldy = pick(l0_, l1_, l2_);
    const int R = pick(R0_, R1_, R2_);
    const int ntile = pick(nt0_, nt1_, nt2_);
    const int gps = pick(gp0_, gp1_, gp2_);
    const int local = bx - pick(0, wg1_, wg2_);
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

// ------------------------------------------------------------------ pipelined kernel
// A workgroup of 8 waves (512 threads, one workgroup per CU) owns 256 tokens x 64 weight rows;
// wave w takes tokens 32w..32w+31 against all 64 rows (two 32x32 MFMA tiles sharing the A
// operand).  The 8 waves share one unpack of the weight planes per super-block (each thread
// unpacks an eighth of a row: 32 codes), so each unpacked plane byte serves 256 tokens.
//
// Epilogue pipelining.  The fp32 epilogue of super-block g-1 (convert, scale, min term,
// accumulate: 4 VALU instructions per output and lane) runs while the MFMAs of super-block g are
// in flight, from the previous super-block's integer accumulators (acc_prev) and its scales in
// LDS.  Each wave therefore issues an even mix of MFMA and VALU work instead of alternating
// MFMA-only sweeps with VALU-only epilogues.  Weight planes are double-buffered (the next
// super-block is unpacked during this one); the scale arrays are triple-buffered, since the
// epilogue of g-1 still reads them while the unpack of g+1 writes.  One barrier per super-block.
constexpr int GP_BM = 256, GP_BN = 64, GP_THREADS = 512;
#ifndef KQ_GP_AHEAD
#define KQ_GP_AHEAD 2       // B operands are read this many int8 MFMAs ahead of their use
#endif

// Plane rows are padded to 272 B (68 dwords): consecutive rows start 4 banks apart, so the 16-byte
// reads of 16 consecutive rows fall on distinct banks, and every address is the row's base plus an
// immediate offset (no per-chunk address registers, as an XOR swizzle would need).
constexpr int GP_ROW = 272;
__device__ __forceinline__ int prw(int r, int c) { return r * GP_ROW + c * 16; }
struct PlaneBuf {                   // one super-block's weight planes: 64 rows of 256 B each
    int8_t wh[GP_BN * GP_ROW];
    int8_t wl[GP_BN * GP_ROW];
};
// Min-term operand rows are padded to 12 dwords: the 16-byte reads of 16 consecutive rows then
// cover distinct banks (a stride of 8 dwords made every other read collide).
constexpr int GP_MROW = 12;
struct ScaleBuf {                   // one super-block's scales
    uint32_t wmin[GP_BN * GP_MROW]; // Q4_K: row n = 16 f16 [-64 m_0..7, -m_0..7] (+ padding)
    uint32_t xmin[GP_BM * GP_MROW]; // Q4_K: token m = 16 f16 [B_0..7 >> 6, B_0..7 & 63] (+ padding)
    float d[GP_BN], dm[GP_BN], dx[GP_BM];
};

// Raw bytes of one eighth of a weight row (part pi = 0..7) for one super-block.
//   Q4_K: qs bytes 32p + 16cc .. +15 (p = pi >> 1, cc = pi & 1): elements 64p + 16cc + 0..15 (low
//         nibbles, sub-block 2p) and 64p + 32 + 16cc + 0..15 (high nibbles, sub-block 2p+1).
//   Q6_K: half h = pi >> 2, slice jj = (pi >> 1) & 1, c = pi & 1: elements 128h + 32k + 16jj + 0..15
//         for k = c and c + 2 (ql bytes 64h + 32c + 16jj, low / high nibble; qh bytes 32h + 16jj,
//         bits 2k; scales 8h + 2k + jj).
template <int TYPE> struct RawP;
template <> struct RawP<TYPE_Q4_K> { u32x4 hdr, q; };
template <> struct RawP<TYPE_Q6_K> {
    Chunk20 ql, qh;
    u32x2 sc;
    uint32_t sce, dw, sh;
};

// Raw buffer loads: a descriptor over the whole buffer in scalar registers, a per-lane byte offset
// that stays the same for every super-block, a scalar per-super-block offset, and the field offset as
// an immediate, so the loop does no 64-bit address arithmetic.  Word 3 of the descriptor is the one
// every gfx950 raw buffer here uses (32-bit data format); loads past num_records return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bld16(__amdgpu_buffer_rsrc_t r, int v, int s) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, v, s, 0));
}
__device__ __forceinline__ u32x2 bld8(__amdgpu_buffer_rsrc_t r, int v, int s) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, v, s, 0));
}
__device__ __forceinline__ uint32_t bld4(__amdgpu_buffer_rsrc_t r, int v, int s) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, v, s, 0);
}

// Lane offsets of one part's fields within its weight block (add the super-block's g * 8 * BS as
// the scalar offset).  Q6_K: a block of row r starts at 2 (r & 1) (mod 4) in the tile column, so
// every field is read from the dword at or below it and funnel-shifted by sh = 2 (r & 1); the bytes
// read past a block (at most 2, only when sh = 0) belong to the next row of the tile column.
template <int TYPE> struct PartOff;
template <> struct PartOff<TYPE_Q4_K> {
    int hdr, q;
    __device__ __forceinline__ PartOff(int blk, int pi, int) : hdr(blk), q(blk + 16 + 16 * pi) {}
};
template <> struct PartOff<TYPE_Q6_K> {
    int ql, qh, sc, base;
    uint32_t sh;
    __device__ __forceinline__ PartOff(int blk, int pi, int row) {
        const int h = pi >> 2, jj = (pi >> 1) & 1, c = pi & 1;
        sh = 2u * (uint32_t)(row & 1);
        base = blk - (int)sh;
        ql = base + 64 * h + 32 * c + 16 * jj;
        qh = base + 128 + 32 * h + 16 * jj;
        sc = base + 192 + 8 * h;
    }
};

__device__ __forceinline__ void load_rawp(RawP<TYPE_Q4_K>& r, __amdgpu_buffer_rsrc_t wr, const PartOff<TYPE_Q4_K>& o,
                                          int soff) {
    r.hdr = bld16(wr, o.hdr, soff);
    r.q = bld16(wr, o.q, soff);
}
__device__ __forceinline__ void load_rawp(RawP<TYPE_Q6_K>& r, __amdgpu_buffer_rsrc_t wr, const PartOff<TYPE_Q6_K>& o,
                                          int soff) {
    r.sh = o.sh;
    r.ql = Chunk20{bld16(wr, o.ql, soff), bld4(wr, o.ql + 16, soff)};
    r.qh = Chunk20{bld16(wr, o.qh, soff), bld4(wr, o.qh + 16, soff)};
    r.sc = bld8(wr, o.sc, soff);
    r.sce = bld4(wr, o.sc + 8, soff);
    r.dw = bld4(wr, o.base + 208, soff);
}

// Activation side of the pipelined kernel: two threads per token row, part xp holding bsums
// 8xp .. 8xp+7 and the row's d.
__device__ __forceinline__ void load_xp(RawX<2>& r, __amdgpu_buffer_rsrc_t xr, int vrow, int xp, int soff) {
    const u32x4 v = bld16(xr, vrow + 260 + 16 * xp, soff);
    r.bs[0] = v.x; r.bs[1] = v.y; r.bs[2] = v.z; r.bs[3] = v.w;
    r.d = bld4(xr, vrow, soff);
}

// The unpack of one part, in chunks that the step spreads over its MFMA slots.
template <int TYPE> struct UnpackP;
template <> struct UnpackP<TYPE_Q4_K> {
    static constexpr int NCHUNK = 3;
    uint32_t alo, blo, ahi, bhi;
    // chunk 0: scales and mins of sub-blocks 2p, 2p+1, the min operands, d and dmin; chunk 1: the
    // low nibbles (sub-block 2p) into both planes; chunk 2: the high nibbles (sub-block 2p+1)
    template <int C>
    __device__ __forceinline__ void chunk(const RawP<TYPE_Q4_K>& r, int pi, int row, PlaneBuf& Lp, ScaleBuf& Ls) {
        const int p = pi >> 1, cc = pi & 1;
        if constexpr (C == 0) {
            const ScMin sm = q4k_scmin_pair(r.hdr.y, r.hdr.z, r.hdr.w, p);
            alo = (sm.sc_lo >> 3) * 0x10001u;
            blo = (sm.sc_lo & 7u) * 0x10001u;
            ahi = (sm.sc_hi >> 3) * 0x10001u;
            bhi = (sm.sc_hi & 7u) * 0x10001u;
            // both halves (cc) of a sub-block pair store the same min operands, every part the same d
            const float mlo = (float)sm.m_lo, mhi = (float)sm.m_hi;
            Ls.wmin[row * GP_MROW + p] = pk_f16(-64.0f * mlo, -64.0f * mhi);
            Ls.wmin[row * GP_MROW + 4 + p] = pk_f16(-mlo, -mhi);
            Ls.d[row] = f16_lo(r.hdr.x);
            Ls.dm[row] = f16_hi(r.hdr.x);
        } else {
            const uint32_t w[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
            const uint32_t a = C == 1 ? alo : ahi, b = C == 1 ? blo : bhi;
            uint32_t hp[4], lp[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t q = (C == 1 ? w[i] : w[i] >> 4) & 0x0f0f0f0fu;
                hp[i] = mul_u8x4(q, a);
                lp[i] = mul_u8x4(q, b);
            }
            const int ch = 4 * p + 2 * (C - 1) + cc;           // elements 64p + 32(C-1) + 16cc + 0..15
            st16(Lp.wh + prw(row, ch), hp[0], hp[1], hp[2], hp[3]);
            st16(Lp.wl + prw(row, ch), lp[0], lp[1], lp[2], lp[3]);
        }
    }
};
template <> struct UnpackP<TYPE_Q6_K> {
    static constexpr int NCHUNK = 9;
    uint32_t Lw[4], Hw[4];
    uint32_t s2[2], c2[2];
    uint32_t hb[4], lb[4];
    // chunk 0: the funnel shifts, the two slices' scales, d; chunk 1 + 4kk + i: dword i of slice
    // k = c + 2kk; chunks 4 and 8 store the slice's two 16-byte plane pieces
    template <int C>
    __device__ __forceinline__ void chunk(const RawP<TYPE_Q6_K>& r, int pi, int row, PlaneBuf& Lp, ScaleBuf& Ls) {
        const int h = pi >> 2, jj = (pi >> 1) & 1, c = pi & 1;
        const uint32_t sh = r.sh;
        if constexpr (C == 0) {
            const uint32_t s0 = __builtin_amdgcn_alignbyte(r.sc.y, r.sc.x, sh);   // scales 8h .. 8h+3
            const uint32_t s1 = __builtin_amdgcn_alignbyte(r.sce, r.sc.y, sh);    // scales 8h+4 .. 8h+7
            Lw[0] = __builtin_amdgcn_alignbyte(r.ql.v.y, r.ql.v.x, sh);
            Lw[1] = __builtin_amdgcn_alignbyte(r.ql.v.z, r.ql.v.y, sh);
            Lw[2] = __builtin_amdgcn_alignbyte(r.ql.v.w, r.ql.v.z, sh);
            Lw[3] = __builtin_amdgcn_alignbyte(r.ql.e, r.ql.v.w, sh);
            Hw[0] = __builtin_amdgcn_alignbyte(r.qh.v.y, r.qh.v.x, sh);
            Hw[1] = __builtin_amdgcn_alignbyte(r.qh.v.z, r.qh.v.y, sh);
            Hw[2] = __builtin_amdgcn_alignbyte(r.qh.v.w, r.qh.v.z, sh);
            Hw[3] = __builtin_amdgcn_alignbyte(r.qh.e, r.qh.v.w, sh);
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {      // scale 8h + 2k + jj, k = c + 2kk: byte 2c + jj of s0 / s1
                const int sc = (int)(int8_t)(uint8_t)((kk ? s1 : s0) >> (8 * (2 * c + jj)));
                s2[kk] = (uint32_t)(sc & 0xffff) * 0x10001u;
                c2[kk] = (uint32_t)((128 - 32 * sc) & 0xffff) * 0x10001u;
            }
            Ls.d[row] = f16_lo(r.dw >> (8 * sh));         // same value from every part of the row
        } else {
            constexpr int kk = (C - 1) >> 2, i = (C - 1) & 3;
            const int k = c + 2 * kk;
            const uint32_t lq = (Lw[i] >> (4 * kk)) & 0x0f0f0f0fu;
            const uint32_t hq = ((Hw[i] >> (2 * k)) & 0x03030303u) << 4;
            const uint32_t q = lq | hq;                                          // 6-bit codes, 4 bytes
            const uint32_t e = __builtin_amdgcn_perm(0u, q, 0x0c020c00u);        // bytes 0, 2 -> 16-bit lanes
            const uint32_t o = __builtin_amdgcn_perm(0u, q, 0x0c030c01u);        // bytes 1, 3
            const s16x2 sv = __builtin_bit_cast(s16x2, s2[kk]), cv = __builtin_bit_cast(s16x2, c2[kk]);
            const uint32_t ve = __builtin_bit_cast(uint32_t, (s16x2)(__builtin_bit_cast(s16x2, e) * sv + cv));
            const uint32_t vo = __builtin_bit_cast(uint32_t, (s16x2)(__builtin_bit_cast(s16x2, o) * sv + cv));
            hb[i] = __builtin_amdgcn_perm(vo, ve, 0x07030501u);                  // high bytes, element order
            lb[i] = __builtin_amdgcn_perm(vo, ve, 0x06020400u) ^ 0x80808080u;
            if constexpr (i == 3) {
                const int ch = 8 * h + 2 * k + jj;
                st16(Lp.wh + prw(row, ch), hb[0], hb[1], hb[2], hb[3]);
                st16(Lp.wl + prw(row, ch), lb[0], lb[1], lb[2], lb[3]);
            }
        }
    }
};

// Activation side: two threads per token row (xp = 0, 1), each holding four of the eight Q4_K
// sub-block sums B_s (bsums 8xp .. 8xp+7) and the row's d.
__device__ __forceinline__ void stage_xp(const RawX<2>& r, int mr, int xp, bool q4, ScaleBuf& Ls) {
    if (q4) {
        int B[4];
#pragma unroll
        for (int i = 0; i < 4; i++) B[i] = (int)(int16_t)(r.bs[i] & 0xffffu) + (int)(int16_t)(r.bs[i] >> 16);
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
            const int dw = mr * GP_MROW + (4 * xp + i) / 2;
            Ls.xmin[dw] = pk_f16((float)(B[i] >> 6), (float)(B[i + 1] >> 6));
            Ls.xmin[dw + 4] = pk_f16((float)(B[i] & 63), (float)(B[i + 1] & 63));
        }
    }
    Ls.dx[mr] = __builtin_bit_cast(float, r.d);
}

// The step's slot program: one MFMA per slot, in this order, and the slot of every other piece of
// work.  MFMA codes: 0..15 the high-plane sweep (tile t, K step ks: 8t + ks), 16..31 the low-plane
// sweep (16 + 8t + ks), 32 / 33 the min-term MFMA of the tile 0 / tile 1 epilogue (Q4_K).
//
// Epilogues are staggered by tile: tile 0's sums are complete once its low-plane sweep ends, so
// its epilogue (E[0], from this super-block's scales) runs under tile 1's low-plane MFMAs of the
// same step; tile 1's epilogue (E[1]) runs in the next step, from the previous super-block's sums
// and scales.  Only one tile's sums are pending across a barrier.
//
// Constraints the slots keep: a tile's shift after its last high-plane MFMA (two slots of latency)
// and before its first low-plane MFMA; a min-term MFMA after its operand reads (ER) and before the
// epilogue that uses it; tile 0's epilogue after its last low-plane MFMA; the raw loads of
// super-block g+2 after the unpack has consumed g+1's; each A operand reloaded after its last use.
template <int TYPE> struct GpSched;
template <> struct GpSched<TYPE_Q4_K> {
    static constexpr int NSLOT = 34;
    static constexpr int mf[NSLOT] = {0, 1, 2, 3, 33, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 16, 17,
                                      18, 19, 14, 15, 32, 20, 21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31};
    static constexpr int U[3] = {0, 1, 2};
    static constexpr int RAW = 3, XS = 3;
    static constexpr int ER[2] = {17, 0};
    static constexpr int E[2][8] = {{27, 28, 29, 30, 31, 32, 33, 33}, {6, 7, 8, 9, 10, 11, 12, 13}};
    static constexpr int SH[2][2] = {{11, 12}, {22, 23}};
    static constexpr int A[8] = {26, 27, 28, 29, 30, 31, 32, 33};
};
template <> struct GpSched<TYPE_Q6_K> {
    static constexpr int NSLOT = 32;
    static constexpr int mf[NSLOT] = {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 16, 17,
                                      18, 19, 14, 15, 20, 21, 22, 23, 24, 25, 26, 27, 28, 29, 30, 31};
    static constexpr int U[9] = {0, 1, 2, 3, 4, 5, 6, 7, 8};
    static constexpr int RAW = 8, XS = 8;
    static constexpr int ER[2] = {20, 9};
    static constexpr int E[2][8] = {{25, 26, 27, 28, 29, 30, 31, 31}, {11, 12, 13, 14, 15, 16, 17, 18}};
    static constexpr int SH[2][2] = {{10, 11}, {21, 22}};
    static constexpr int A[8] = {24, 25, 26, 27, 28, 29, 30, 31};
};
// position of slot s among the int8 MFMAs (codes < 32), and the slot of position p
template <class SC> __host__ __device__ constexpr int gp_pos(int s) {
    int p = 0;
    for (int j = 0; j < s; j++) p += SC::mf[j] < 32;
    return p;
}
template <class SC> __host__ __device__ constexpr int gp_code_at(int p) {
    for (int j = 0; j < SC::NSLOT; j++)
        if (SC::mf[j] < 32 && gp_pos<SC>(j) == p) return SC::mf[j];
    return -1;
}

template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

template <int TYPE, bool FRAG>
__global__ void __launch_bounds__(GP_THREADS)
k_gemm_q8k_p(GemmGroup gg, int G, const uint8_t* __restrict__ XQ, const uint8_t* __restrict__ XF, int M) {
    constexpr int BS = TYPE == TYPE_Q4_K ? Q4K_BYTES : Q6K_BYTES;
    constexpr int SHIFT = TYPE == TYPE_Q4_K ? 3 : 8;
    __shared__ __attribute__((aligned(16))) PlaneBuf LP0;
    __shared__ __attribute__((aligned(16))) PlaneBuf LP1;
    __shared__ __attribute__((aligned(16))) ScaleBuf LS0;
    __shared__ __attribute__((aligned(16))) ScaleBuf LS1;
    __shared__ __attribute__((aligned(16))) ScaleBuf LS2;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int half = lane >> 5, l32 = lane & 31;
    KQ_GEMM_ARGS(gg);
    const int mi = nmat > 1 && bx >= wg1_ ? (nmat > 2 && bx >= wg2_ ? 2 : 1) : 0;
    auto pick = [&](auto a, auto b, auto c) { return mi == 0 ? a : mi == 1 ? b : c; };
    const uint8_t* const W = kq_global<const uint8_t>(pick(w0_, w1_, w2_));
    float* const Y = kq_global<float>(pick(y0_, y1_, y2_));
    float* const P = kq_global<float>(pick(p0_, p1_, p2_));
    const int64_t ldy = pick(l0_, l1_, l2_);
    const int R = pick(R0_, R1_, R2_);
    const int ntile = pick(nt0_, nt1_, nt2_);
    const int gps = pick(gp0_, gp1_, gp2_);
    const int local = bx - pick(0, wg1_, wg2_);
    const int split = local / ntile;
    const int n0 = (local - split * ntile) * GP_BN, m0 = blockIdx.y * GP_BM;
    const int64_t xrow = (int64_t)G * Q8K_BYTES;
    const int gbeg = split * gps, gend = gbeg + gps < G ? gbeg + gps : G;
    float* const Yo = P ? P + (int64_t)split * M * R : Y;
    const int64_t ldo = P ? (int64_t)R : ldy;

    // A operand of this lane for K step ks of super-block g: byte aoff + (ks & 4) * AK of the A buffer,
    // plus g * AG (scalar) and (ks & 3) * AK (immediate)
    constexpr int AG = FRAG ? 8192 : Q8K_BYTES, AK = FRAG ? 1024 : 32;
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(XQ, (uint32_t)M * (uint32_t)xrow);
    const __amdgpu_buffer_rsrc_t ar = FRAG ? buf_rsrc(XF, (uint32_t)((M + GP_BM - 1) / GP_BM * GP_BM) * (uint32_t)G * QK) : xr;
    int aoff;
    if (FRAG) {
        aoff = ((blockIdx.y * (GP_BM / 32) + wave) * G * 512 + lane) * 16;
    } else {
        int m = m0 + 32 * wave + l32;
        m = m < M ? m : M - 1;
        aoff = m * (int)xrow + 4 + 16 * half;
    }
    const int aoff4 = aoff + 4 * AK;
    auto load_a = [&](int ks, int g) {
        return __builtin_bit_cast(v4i, bld16(ar, (ks < 4 ? aoff : aoff4) + (ks & 3) * AK, g * AG));
    };
    // activation row staged by this thread (two threads per row)
    const int mr = tid & (GP_BM - 1), xp = tid >> 8;
    const int xoff = (m0 + mr < M ? m0 + mr : M - 1) * (int)xrow;
    // weight row part unpacked by this thread: wave w unpacks rows 8w..8w+7 (one tile column),
    // eight lanes per row.  The two rows of a 16-lane group are 4 (Q6_K) or 2 (Q4_K) rows apart, so
    // their plane stores (chunk sets offset by that many 16-byte chunks) fall on distinct banks.
    const int pj = lane >> 3;
    const int prow = 8 * wave + (TYPE == TYPE_Q6_K ? ((pj & 1) << 2 | pj >> 1) : ((pj & 1) << 1 | (pj & 4) | (pj >> 1 & 1))),
              pi = lane & 7;
    const int pr = n0 + prow < R ? n0 + prow : R - 1;
    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(W, (uint32_t)R * (uint32_t)G * BS);
    const PartOff<TYPE> po(((pr >> 3) * G * 8 + (pr & 7)) * BS, pi, pr);

    float yacc[2][16];
    // integer sums: tile 0's are consumed within their step; tile 1's are pending into the next
    // step, so they have one set per step parity (a step writes its own while the epilogue reads
    // the other; no copy between steps)
    v16i acc0, acc1s[2];
    acc1s[1] = v16i{};
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int a = 0; a < 16; a++) yacc[t][a] = 0.0f;
    // the first step's pending epilogue reads LS2: zero scales make it add nothing
    for (int i = tid; i < (int)(sizeof(ScaleBuf) / 4); i += GP_THREADS) reinterpret_cast<uint32_t*>(&LS2)[i] = 0u;

    RawP<TYPE> raw;
    RawX<2> rx;
    UnpackP<TYPE> up;
    v4i afr[8];
    load_rawp(raw, wr, po, gbeg * 8 * BS);
    load_xp(rx, xr, xoff, xp, gbeg * Q8K_BYTES);
#pragma unroll
    for (int ks = 0; ks < 8; ks++) afr[ks] = load_a(ks, gbeg);
    static_for<0, UnpackP<TYPE>::NCHUNK>([&](auto c) { up.template chunk<decltype(c)::value>(raw, pi, prow, LP0, LS0); });
    stage_xp(rx, mr, xp, TYPE == TYPE_Q4_K, LS0);
    {
        const int g1 = gbeg + 1 < gend ? gbeg + 1 : gbeg;
        load_rawp(raw, wr, po, g1 * 8 * BS);
        load_xp(rx, xr, xoff, xp, g1 * Q8K_BYTES);
    }
    __syncthreads();

    const int nrow[2] = {l32, 32 + l32};     // this lane's B rows (weight rows within the tile)

    // per pending tile: its d (and dmin), the tokens' dx and (Q4_K) the min term -I2
    float ep_d[2], ep_dm[2];
    f32x4 ep_dx[2][4];
    v16f ep_cm[2];
    v8h ep_am[2], ep_bm[2];
    auto epi_read = [&](const ScaleBuf& S, int nt) {
        ep_d[nt] = S.d[nrow[nt]];
        if constexpr (TYPE == TYPE_Q4_K) {
            ep_dm[nt] = S.dm[nrow[nt]];
            ep_bm[nt] = __builtin_bit_cast(v8h, *reinterpret_cast<const u32x4*>(&S.wmin[nrow[nt] * GP_MROW + 4 * half]));
            ep_am[nt] = __builtin_bit_cast(v8h, *reinterpret_cast<const u32x4*>(&S.xmin[(32 * wave + l32) * GP_MROW + 4 * half]));
        }
    };
    // two outputs (2c, 2c+1) of pending tile nt, from its integer sums a
    auto epi_part = [&](int nt, int c, const v16i& a) {
#pragma unroll
        for (int e = 2 * c; e < 2 * c + 2; e++) {
            const float v = __fmul_rn(ep_d[nt], (float)a[e]);
            if constexpr (TYPE == TYPE_Q4_K)
                yacc[nt][e] = __builtin_fmaf(ep_dx[nt][e >> 2][e & 3], __builtin_fmaf(ep_dm[nt], ep_cm[nt][e], v), yacc[nt][e]);
            else
                yacc[nt][e] = __builtin_fmaf(ep_dx[nt][e >> 2][e & 3], v, yacc[nt][e]);
        }
    };

    using SC = GpSched<TYPE>;
    auto step = [&](auto p2_c, auto p3_c, int g) {
        constexpr int p2 = decltype(p2_c)::value, p3 = decltype(p3_c)::value;
        PlaneBuf& Lc = p2 ? LP1 : LP0;                  // planes of g (read)
        PlaneBuf& Ln = p2 ? LP0 : LP1;                  // planes of g+1 (written)
        ScaleBuf& Sn = p3 == 0 ? LS1 : p3 == 1 ? LS2 : LS0;   // scales of g+1 (written)
        ScaleBuf& Sp = p3 == 0 ? LS2 : p3 == 1 ? LS0 : LS1;   // scales of g-1 (tile 1 epilogue)
        ScaleBuf& Sc = p3 == 0 ? LS0 : p3 == 1 ? LS1 : LS2;   // scales of g (tile 0 epilogue)
        const int gn = g + 1 < gend ? g + 1 : gend - 1;
        const int g2 = g + 2 < gend ? g + 2 : gend - 1;

        v16i& acc1 = acc1s[p2];                         // tile 1's sums of g
        const v16i& acc1p = acc1s[p2 ^ 1];              // tile 1's sums of g-1 (epilogue pending)
        constexpr int NB = KQ_GP_AHEAD + 1;
        v4i bb[NB];                                     // B operands, read KQ_GP_AHEAD int8 MFMAs ahead
        auto read_b = [&](int code, v4i& b) {
            const int t = (code >> 3) & 1, ks = code & 7;
            const int8_t* base = code < 16 ? Lc.wh : Lc.wl;
            b = *reinterpret_cast<const v4i*>(base + prw(nrow[t], 2 * ks + half));
        };
        static_for<0, KQ_GP_AHEAD>([&](auto k) {
            constexpr int code = gp_code_at<SC>(decltype(k)::value);
            read_b(code, bb[decltype(k)::value]);
        });

        static_for<0, SC::NSLOT>([&](auto S) {
            constexpr int s = decltype(S)::value;
            // work chunks of this slot
            static_for<0, UnpackP<TYPE>::NCHUNK>([&](auto c) {
                if constexpr (SC::U[decltype(c)::value] == s) up.template chunk<decltype(c)::value>(raw, pi, prow, Ln, Sn);
            });
            if constexpr (SC::XS == s) stage_xp(rx, mr, xp, TYPE == TYPE_Q4_K, Sn);
            if constexpr (SC::RAW == s) {
                load_rawp(raw, wr, po, g2 * 8 * BS);
                load_xp(rx, xr, xoff, xp, g2 * Q8K_BYTES);
            }
            static_for<0, 2>([&](auto t) {
                constexpr int nt = decltype(t)::value;
                v16i& acc = nt == 0 ? acc0 : acc1;
                if constexpr (SC::ER[nt] == s) epi_read(nt == 0 ? Sc : Sp, nt);
                // the tokens' dx, one 4-vector per two chunks, read one chunk ahead of its first use (all
                // 16 held at once cost 12 registers more and made the Q4_K form spill)
                static_for<0, 4>([&](auto q) {
                    constexpr int qq = decltype(q)::value;
                    constexpr int at = qq == 0 ? SC::ER[nt] : SC::E[nt][2 * qq - 1];
                    if constexpr (at == s)
                        ep_dx[nt][qq] = *reinterpret_cast<const f32x4*>(&(nt == 0 ? Sc : Sp).dx[32 * wave + 8 * qq + 4 * half]);
                });
                static_for<0, 8>([&](auto c) {
                    if constexpr (SC::E[nt][decltype(c)::value] == s)
                        epi_part(nt, decltype(c)::value, nt == 0 ? acc0 : acc1p);
                });
                if constexpr (SC::SH[nt][0] == s) {
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[e] <<= SHIFT;
                }
                if constexpr (SC::SH[nt][1] == s) {
#pragma unroll
                    for (int e = 8; e < 16; e++) acc[e] <<= SHIFT;
                }
            });
            // the slot's MFMA
            constexpr int code = SC::mf[s];
            if constexpr (code < 32) {
                constexpr int t = (code >> 3) & 1, ks = code & 7, pos = gp_pos<SC>(s);
                const bool first = code < 16 && ks == 0;
                v16i& acc = t == 0 ? acc0 : acc1;
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(afr[ks], bb[pos % NB], first ? v16i{} : acc, 0, 0, 0);
                constexpr int nxt = gp_code_at<SC>(pos + KQ_GP_AHEAD);
                if constexpr (nxt >= 0) read_b(nxt, bb[(pos + KQ_GP_AHEAD) % NB]);
            } else if constexpr (TYPE == TYPE_Q4_K) {
                ep_cm[code - 32] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ep_am[code - 32], ep_bm[code - 32], v16f{}, 0, 0, 0);
            }
            static_for<0, 8>([&](auto k) {
                constexpr int ks = decltype(k)::value;
                if constexpr (SC::A[ks] == s)
                    afr[ks] = load_a(ks, gn);
            });
            __builtin_amdgcn_sched_barrier(0);
        });
        __syncthreads();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    for (int g = gbeg; g < gend; g += 6) {
        step(I0{}, I0{}, g);
        if (g + 1 < gend) step(I1{}, I1{}, g + 1);
        if (g + 2 < gend) step(I0{}, I2{}, g + 2);
        if (g + 3 < gend) step(I1{}, I0{}, g + 3);
        if (g + 4 < gend) step(I0{}, I1{}, g + 4);
        if (g + 5 < gend) step(I1{}, I2{}, g + 5);
    }
    // tile 1's epilogue of the last super-block
    {
        const int p3 = (gend - 1 - gbeg) % 3;
        const ScaleBuf& S = p3 == 0 ? LS0 : p3 == 1 ? LS1 : LS2;
        auto last = [&](const v16i& a) {
            epi_read(S, 1);
#pragma unroll
            for (int q = 0; q < 4; q++) ep_dx[1][q] = *reinterpret_cast<const f32x4*>(&S.dx[32 * wave + 8 * q + 4 * half]);
            if constexpr (TYPE == TYPE_Q4_K)
                ep_cm[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ep_am[1], ep_bm[1], v16f{}, 0, 0, 0);
#pragma unroll
            for (int c = 0; c < 8; c++) epi_part(1, c, a);
        };
        if ((gend - 1 - gbeg) & 1) last(acc1s[1]);
        else last(acc1s[0]);
    }

#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const int n = n0 + nrow[nt];
#pragma unroll
        for (int a = 0; a < 16; a++) {
            const int m = m0 + 32 * wave + (a >> 2) * 8 + half * 4 + (a & 3);
            if (m < M && n < R) Yo[(int64_t)m * ldo + n] = yacc[nt][a];
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
    // every argument in one batch of loads (one wait; see KQ_GEMM_ARGS)
    int bx = blockIdx.x;
    int64_t p0_ = (int64_t)rg.m[0].part, p1_ = (int64_t)rg.m[1].part, p2_ = (int64_t)rg.m[2].part;
    int64_t y0_ = (int64_t)rg.m[0].y, y1_ = (int64_t)rg.m[1].y, y2_ = (int64_t)rg.m[2].y;
    int64_t l0_ = rg.m[0].ldy, l1_ = rg.m[1].ldy, l2_ = rg.m[2].ldy;
    int R0_ = rg.m[0].R, R1_ = rg.m[1].R, R2_ = rg.m[2].R, S0_ = rg.m[0].S, S1_ = rg.m[1].S, S2_ = rg.m[2].S;
    int b1_ = rg.m[1].blk0, b2_ = rg.m[2].blk0, nmat = rg.n;
    asm volatile("" : "+s"(bx), "+s"(p0_), "+s"(p1_), "+s"(p2_), "+s"(y0_), "+s"(y1_), "+s"(y2_), "+s"(l0_),
                 "+s"(l1_), "+s"(l2_), "+s"(R0_), "+s"(R1_), "+s"(R2_), "+s"(S0_), "+s"(S1_), "+s"(S2_), "+s"(b1_),
                 "+s"(b2_), "+s"(nmat) : "s"(M));
    __builtin_amdgcn_sched_barrier(0);
    const int j = nmat > 1 && bx >= b1_ ? (nmat > 2 && bx >= b2_ ? 2 : 1) : 0;
    auto pick = [&](auto a, auto b, auto c) { return j == 0 ? a : j == 1 ? b : c; };
    const float* const P = kq_global<const float>(pick(p0_, p1_, p2_));
    float* const Y = kq_global<float>(pick(y0_, y1_, y2_));
    const int64_t ldy = pick(l0_, l1_, l2_);
    const int R = pick(R0_, R1_, R2_);
    const int S = pick(S0_, S1_, S2_);
    const int r4 = R >> 2;
    const int64_t i = (int64_t)(bx - pick(0, b1_, b2_)) * 256 + threadIdx.x;
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

// Tiles of the K-split rule: 64 weight rows x 128 tokens, and the workgroups that fill the GPU: two
// per CU of the 256 on an MI355X (fixed, so the split and the workspace size do not depend on the
// device or on the kernel a call runs).  The pipelined kernel's 64 x 256 tiles at one workgroup per
// CU give the same S whenever M is a multiple of 256.  Measured (two-wave kernel, us, unsplit ->
// split): 4096x12288 Q6_K at M = 32 / 64 / 128 / 256 / 512: 91.7 / 93.4 / 98.4 / 99.9 / 103.2 ->
// 34.6 / 35.9 / 38.1 / 57.8 / 96.1; 12288x4096 Q4_K at M = 32 / 64: 33.6 / 33.5 -> 31.5 / 33.0.
constexpr int GM_TN = 64, GM_TM = 128;
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

// One reduce launch for the matrices of a group that split K.
static void launch_reduce(const GemmGroup& gg, int M, const int* S, hipStream_t s) {
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

// Which kernel runs a launch.  The pipelined kernel (256 tokens x 64 rows, one 8-wave workgroup per
// CU) serves Q6_K from 129 tokens: its shared unpack halves the heavy Q6_K plane arithmetic per
// output (4096x12288 at M = 256 / 512 / 2048: 53.6 / 89.1 / 298 -> 47.1 / 77.2 / 259 us).  Q4_K
// stays on the two-wave kernel, which the pipelined one does not beat for it (12288x4096 at M = 256
// / 512 / 2048: 46.0 / 73.9 / 269-277 against 44.9 / 85.0 / 276 us).  The pipelined kernel's raw
// buffer descriptors address at most 2^31 bytes per buffer.
static bool use_pipelined(int type, int R, int C, int M) {
    const int64_t G = C / QK;
    return type == TYPE_Q6_K && M > 128 && (int64_t)R * G * Q6K_BYTES < (int64_t(1) << 31) &&
           (int64_t)((M + GP_BM - 1) / GP_BM * GP_BM) * G * Q8K_BYTES < (int64_t(1) << 31);
}

template <int TYPE>
static void launch_type(const GemmGroup& gg, int wgs, int G, const uint8_t* xq, const uint8_t* xf, int M,
                        const int* S, bool pipelined, hipStream_t s) {
    if constexpr (TYPE == TYPE_Q6_K) {          // (the Q4_K form is not dispatched: see use_pipelined)
        if (pipelined) {
            dim3 grid(wgs, (M + GP_BM - 1) / GP_BM), block(GP_THREADS);
            if (xf)
                hipLaunchKernelGGL((k_gemm_q8k_p<TYPE, true>), grid, block, 0, s, gg, G, xq, xf, M);
            else
                hipLaunchKernelGGL((k_gemm_q8k_p<TYPE, false>), grid, block, 0, s, gg, G, xq, xf, M);
            launch_reduce(gg, M, S, s);
            return;
        }
    }
    {
        // 128 tokens x 64 weight rows per workgroup of 4 waves (80 KB of LDS, at most 256 VGPRs), so
        // two workgroups share a CU and each SIMD holds two waves: one wave's unpack and epilogue run
        // under the other's MFMAs.  Each wave takes 32 tokens x all 64 rows (MT = 1): half the A-operand
        // loads of 64 tokens x 32 rows (MT = 2), for twice the B reads from LDS; 12288x4096 Q4_K at
        // M = 2048 / 512 / 256: 285 / 76.8 / 49.3 -> 270 / 73.8 / 45.7 us, 4096x12288 Q6_K 311 / 91.2
        // -> 300 / 88.1 us.
        dim3 grid(wgs, (M + GM_TM - 1) / GM_TM), block(256);
        if (xf)
            hipLaunchKernelGGL((k_gemm_q8k<TYPE, GM_TN, 1, 4, true, 1>), grid, block, 0, s, gg, G, xq, xf, M);
        else
            hipLaunchKernelGGL((k_gemm_q8k<TYPE, GM_TN, 1, 4, false, 1>), grid, block, 0, s, gg, G, xq, xf, M);
    }
    launch_reduce(gg, M, S, s);
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
        bool pipelined = true;
        for (int i = 0; i < gg.n; i++) pipelined = pipelined && use_pipelined(ty, gg.m[i].R, C, M);
        if (ty == TYPE_Q4_K) launch_type<TYPE_Q4_K>(gg, wgs, G, xq, ws, M, Sg, pipelined, s);
        else launch_type<TYPE_Q6_K>(gg, wgs, G, xq, ws, M, Sg, pipelined, s);
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
