// Argmax over the outputs of a grid, in one pass: each workgroup reduces its candidates and folds
// them into one 64-bit key with an atomic max; the workgroup that finishes last (a ticket counter)
// decodes the key.  Nothing ever waits for another workgroup.
//
// Rule of the reference's k_argmax (scripts/kindi_q4/kindi/kindi.cu:637-661): the largest value,
// the smallest index among equal largest values; a value is taken only when strictly greater than
// the best so far, starting from (-1e30, index 0), so NaN is never chosen and an input with no
// value above -1e30 gives index 0.  The combine below is that rule as a total order on non-NaN
// pairs, so the result does not depend on how the candidates are grouped.
#pragma once
#include "kq_device.h"

namespace kq {

constexpr size_t ARGMAX_WS_BYTES = 256;             // key and ticket counter (and room to grow)

struct ArgBest {
    float v;
    int i;
};

__device__ __forceinline__ ArgBest arg_init() { return ArgBest{-1e30f, 0}; }

// Candidate value v at index i (the scan step of the rule).
__device__ __forceinline__ void arg_take(ArgBest& b, float v, int i) {
    if (v > b.v || (v == b.v && i < b.i)) { b.v = v; b.i = i; }
}

__device__ __forceinline__ ArgBest arg_combine(ArgBest a, ArgBest c) {
    return (c.v > a.v || (c.v == a.v && c.i < a.i)) ? c : a;
}

__device__ __forceinline__ ArgBest arg_shfl_xor(ArgBest b, int m) {
    return ArgBest{__shfl_xor(b.v, m, 64), __shfl_xor(b.i, m, 64)};
}

// Wave-level reduction; every lane returns the wave's best.
__device__ __forceinline__ ArgBest arg_wave_reduce(ArgBest b) {
#pragma unroll
    for (int m = 32; m; m >>= 1) b = arg_combine(b, arg_shfl_xor(b, m));
    return b;
}

// Candidate as one 64-bit key whose unsigned order is the rule's order: the value's bits made
// order-preserving (-0 counted as +0, so equal values tie), then ~index so that the smaller index
// of equal values is the larger key.  Every candidate is above -1e30 or is (-1e30, 0), so every
// key is above 0, the value an all-zero workspace holds.
__device__ __forceinline__ unsigned long long arg_key(ArgBest b) {
    const uint32_t u = __builtin_bit_cast(uint32_t, __fadd_rn(b.v, 0.0f));
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)o << 32) | (unsigned long long)(0xffffffffu - (uint32_t)b.i);
}

// Workgroup-level finish: `mine` is each wave's best (every lane holds it).  Thread 0 folds the
// workgroup's best into the key with one device-scope atomic max, then takes a ticket; the
// workgroup with the last ticket reads the key, writes the index to *out and zeroes key and
// counter for the next call.  The ticket is taken only once the max has returned, so a ticket
// holder's candidate is in the key; device-scope atomics act on one coherent copy, and no cache
// write-back fence is needed.  Every thread of the workgroup must call it.
// ws: [0, 8) key, [8, 12) ticket counter; both zero before the first call.
__device__ __forceinline__ void arg_grid_finish(ArgBest mine, uint8_t* ws, int* out) {
    __shared__ float sv[16];
    __shared__ int si[16];
    unsigned long long* key = reinterpret_cast<unsigned long long*>(ws);
    unsigned int* ticket = reinterpret_cast<unsigned int*>(ws + 8);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (lane == 0) { sv[wave] = mine.v; si[wave] = mine.i; }
    __syncthreads();
    if (threadIdx.x != 0) return;
    ArgBest b = arg_init();
    for (int k = 0; k < nw; k++) b = arg_combine(b, ArgBest{sv[k], si[k]});
    atomicMax(key, arg_key(b));
    __builtin_amdgcn_s_waitcnt(0x0f70);                      // vmcnt(0): the max has completed
    if (atomicAdd(ticket, 1u) != gridDim.x - 1) return;
    const unsigned long long k = atomicAdd(key, 0ull);       // coherent read of the final key
    *out = (int)(0xffffffffu - (uint32_t)(k & 0xffffffffu));
    atomicExch(key, 0ull);
    atomicExch(ticket, 0u);
}

}  // namespace kq
