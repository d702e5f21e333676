// Device-side helpers shared by the gfx950 kernels of libkq.
//
// Formats (GGML block layouts, as decoded by scripts/kindi_q4/kindi/q4kernels.h:12-33):
//   Q4_K  144 B / 256 weights: f16 d @0, f16 dmin @2, 12 B packed 6-bit scales/mins @4, 128 B nibbles @16
//   Q6_K  210 B / 256 weights: 128 B low nibbles @0, 64 B 2-bit highs @128, 16 int8 scales @192, f16 d @208
//   Q8_K  292 B / 256 values : f32 d @0, 256 int8 @4, 16 int16 sums of 16 consecutive quants @260
// Weights use the Kindi 8-row interleave [R/8][G][8][block] (q4pack.py:151-160, q4kernels.h:8-10):
// one "tile column" is the 8 blocks of rows 8t..8t+7 at super-block column g, 1152 B (Q4_K) or
// 1680 B (Q6_K), both multiples of 16 B.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kq {

constexpr int QK = 256;
constexpr int Q4K_BYTES = 144;
constexpr int Q6K_BYTES = 210;
constexpr int Q8K_BYTES = 292;
constexpr int TYPE_Q4_K = 12;
constexpr int TYPE_Q6_K = 14;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Same vector with 4-byte alignment: global_load_dwordx4 only needs dword alignment.
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef u32x2 u32x2_a4 __attribute__((aligned(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef f32x4 f32x4_a4 __attribute__((aligned(4)));

__device__ __forceinline__ u32x4 ld16(const uint8_t* p) {            // p 16-byte aligned
    return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ u32x4 ld16_a4(const uint8_t* p) {         // p 4-byte aligned
    return *reinterpret_cast<const u32x4_a4*>(p);
}
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) {          // p 4-byte aligned
    return *reinterpret_cast<const uint32_t*>(p);
}

// 16 bytes at a 2-byte aligned address, read as dword-aligned loads and funnel-shifted.
// Reads the dword-aligned span [p & ~3, (p & ~3) + 20): callers guarantee it lies in the buffer.
__device__ __forceinline__ u32x4 ld16_a2(const uint8_t* p) {
    const uint32_t sh = uint32_t(reinterpret_cast<uintptr_t>(p) & 3);
    const uint8_t* q = p - sh;     // pointer arithmetic keeps the global address space
    const u32x4 v = ld16_a4(q);
    const uint32_t e = ld4(q + 16);
    u32x4 r;
    r.x = __builtin_amdgcn_alignbyte(v.y, v.x, sh);
    r.y = __builtin_amdgcn_alignbyte(v.z, v.y, sh);
    r.z = __builtin_amdgcn_alignbyte(v.w, v.z, sh);
    r.w = __builtin_amdgcn_alignbyte(e, v.w, sh);
    return r;
}

__device__ __forceinline__ float f16_lo(uint32_t u) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xffffu));
}
__device__ __forceinline__ float f16_hi(uint32_t u) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {  // signed int8 x4 dot, no clamp
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Byte k (0..3) of a dword.
__device__ __forceinline__ uint32_t byte_of(uint32_t w, int k) { return (w >> (8 * k)) & 0xffu; }

// Q4_K: 6-bit scales and mins of sub-blocks 2p and 2p+1 from the 12 scale bytes held in
// dwords s0 = bytes 0..3, s1 = 4..7, s2 = 8..11 (q4kernels.h:17-18):
//   k < 4 : sc = s[k] & 63,                      m = s[k+4] & 63
//   k >= 4: sc = (s[k+4] & 15) | (s[k-4]>>6)<<4, m = (s[k+4] >> 4) | (s[k]>>6)<<4
// Rearranged per dword: scale bytes of k=0..3 are s0 & 0x3f3f3f3f, of k=4..7 are
// (s2 & 0x0f0f0f0f) | ((s0 >> 2) & 0x30303030); mins of k=0..3 are s1 & 0x3f3f3f3f, of k=4..7
// are ((s2 >> 4) & 0x0f0f0f0f) | ((s1 >> 2) & 0x30303030).
struct ScMin { uint32_t sc_lo, sc_hi, m_lo, m_hi; };
__device__ __forceinline__ ScMin q4k_scmin_pair(uint32_t s0, uint32_t s1, uint32_t s2, int p) {
    // both candidates are formed and one is selected, so the code has no divergent branch
    const uint32_t sc_a = s0 & 0x3f3f3f3fu, m_a = s1 & 0x3f3f3f3fu;
    const uint32_t sc_b = (s2 & 0x0f0f0f0fu) | ((s0 >> 2) & 0x30303030u);
    const uint32_t m_b = ((s2 >> 4) & 0x0f0f0f0fu) | ((s1 >> 2) & 0x30303030u);
    const bool hi = p >= 2;
    const uint32_t scw = hi ? sc_b : sc_a, mw = hi ? m_b : m_a;
    const int sh = 16 * (p & 1);   // sub-blocks 2p, 2p+1 are bytes (2p)&3, (2p)&3 + 1
    ScMin r;
    r.sc_lo = (scw >> sh) & 0xffu;
    r.sc_hi = (scw >> (sh + 8)) & 0xffu;
    r.m_lo = (mw >> sh) & 0xffu;
    r.m_hi = (mw >> (sh + 8)) & 0xffu;
    return r;
}

// Wave-level helpers.  The lane order of every fp32 reduction below is part of the numerical
// contract of the GEMV kernels (batched results must equal single-token ones bit for bit), so
// all kernels use these and only these.  Each step adds a lane's value to its partner's in a
// butterfly; fp32 addition is commutative, so both partners hold the same bits afterwards.
constexpr int DPP_QUAD_XOR1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141; // lane j of each 8 <- lane 7-j
constexpr int DPP_ROW_MIRROR = 0x140;      // lane j of each 16 <- lane 15-j

// Partner values across 16- and 32-lane distances with the gfx950 permlane swaps (VALU, no LDS
// round trip).  With both operands v, v_permlane16_swap returns rows (0, 0, 2, 2) of v in one
// result and rows (1, 1, 3, 3) in the other; v_permlane32_swap returns halves (0, 0) and (1, 1).
// Lane i therefore holds {v[i], v[i ^ 16]} (resp. {v[i], v[i ^ 32]}) in the two results, in an
// order that depends on i; fp32 addition and fmax are commutative, so the butterfly sum or max of
// the pair has the same bits in either order.
struct LanePair { uint32_t a, b; };
__device__ __forceinline__ LanePair xor16_pair(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return LanePair{r[0], r[1]};
}
__device__ __forceinline__ LanePair xor32_pair(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return LanePair{r[0], r[1]};
}
__device__ __forceinline__ float xor16_sum(float v) {
    const LanePair r = xor16_pair(__builtin_bit_cast(uint32_t, v));
    return __fadd_rn(__builtin_bit_cast(float, r.a), __builtin_bit_cast(float, r.b));
}
__device__ __forceinline__ float xor32_sum(float v) {
    const LanePair r = xor32_pair(__builtin_bit_cast(uint32_t, v));
    return __fadd_rn(__builtin_bit_cast(float, r.a), __builtin_bit_cast(float, r.b));
}
__device__ __forceinline__ float xor16_max(float v) {
    const LanePair r = xor16_pair(__builtin_bit_cast(uint32_t, v));
    return __builtin_fmaxf(__builtin_bit_cast(float, r.a), __builtin_bit_cast(float, r.b));
}
__device__ __forceinline__ float xor32_max(float v) {
    const LanePair r = xor32_pair(__builtin_bit_cast(uint32_t, v));
    return __builtin_fmaxf(__builtin_bit_cast(float, r.a), __builtin_bit_cast(float, r.b));
}

// An empty instruction that takes every listed kernel-argument value in scalar registers: the loads
// that produce them are all issued ahead of it, and its wait is the kernel prologue's only one.  Left
// to the compiler, each argument load sinks to its first use, and a prologue whose addresses depend on
// earlier arguments (grid and block size, a matrix table indexed by the wave's matrix) makes several
// dependent round trips of ~0.3 us to the kernel arguments before its first data load.  Each value
// keeps a use besides the later ones, so selects over them are not folded back into an indexed load,
// and pointers keep their global address space (as outputs of the instruction they would not).  The
// scheduling barrier keeps later work from being hoisted above it (and waiting on part of the batch).
#define KQ_ARGS_READY(...)                                                                            \
    do {                                                                                              \
        asm volatile("" ::__VA_ARGS__);                                                               \
        __builtin_amdgcn_sched_barrier(0);                                                            \
    } while (0)

// A pointer that passed through an empty instruction as an integer, as a global pointer again: the
// cast through the global address space lets loads through it be global (not flat) loads.
template <class T>
__device__ __forceinline__ T* kq_global(int64_t v) {
    typedef __attribute__((address_space(1))) T GT;
    return (T*)(GT*)(uintptr_t)v;
}

// bound_ctrl set (lanes whose source lies outside the row read 0): every control used here is a quad
// permutation, a row mirror, or a row shift whose out-of-row lanes are never used, so the value is the
// same, and the compiler can fold the move into the instruction that consumes it (one v_max_f32_dpp or
// v_add_u32_dpp instead of a v_mov_b32_dpp and the operation).
template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Sum over the 4 lanes of a quad (lanes 4j..4j+3), exact for int32.
__device__ __forceinline__ int quad_sum_i32(int v) {
    v += dpp<DPP_QUAD_XOR1>(v);
    return v + dpp<DPP_QUAD_XOR2>(v);
}
// Pairwise tree over the 16 super-block slots held by lane bits 2..5 (slot = lane >> 2), for a
// value that is uniform within each quad: ((s0+s1)+(s2+s3)) + ... in natural slot order.
// Within a 16-lane row the mirrors pair quad 0 with 1 and 2 with 3, then the two halves; then
// the rows (lane ^ 16) and the halves of the wave (lane ^ 32).
__device__ __forceinline__ float slot_tree_f32(float v) {
    v = __fadd_rn(v, dppf<DPP_ROW_HALF_MIRROR>(v));
    v = __fadd_rn(v, dppf<DPP_ROW_MIRROR>(v));
    v = xor16_sum(v);
    return xor32_sum(v);
}

}  // namespace kq
