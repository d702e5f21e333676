// Argmax over the outputs of a grid, in one pass: each workgroup reduces its candidates and folds
// them into a 64-bit key with an atomic max; the last workgroup to finish (a ticket counter) decodes
// the keys.  Nothing ever waits for another workgroup.  Workgroup w folds into key w mod 64 (each
// key on its own cache line), so no key sees more than a few atomics per call (same-address
// device-scope atomics serialize), and the last workgroup reads the 64 keys at once: three
// dependent atomic round trips on the way out (max, ticket, key reads), as with a single key.
//
#pragma once
#include "kq_device.h"

namespace kq {

constexpr int ARG_SLOTS = 64;                       // keys
constexpr int ARG_LINE = 128;                       // bytes between keys: one cache line each
constexpr size_t ARGMAX_WS_BYTES = (size_t)(ARG_SLOTS + 1) * ARG_LINE;   // + the ticket counter's line

struct ArgBest {
    float v;
    int i;
};

__device__ __forceinline__ ArgBest arg_init() { return ArgBest{-1e30f, 0}; }

// Candidate value v at index i (the scan step of the rule).
__device__ __forceinline__ void arg_take(ArgBest& b, float v, int i) {
    if (v > b.v || (v == b.v && i < b.i)) { b.v = v; b.i = i; }
}

// The scan step for candidates that arrive in increasing index order (a lane's outputs in a GEMV
// stream): an equal value never replaces the best, so the smaller index of equal values is kept and
// the tie test is not needed.
__device__ __forceinline__ void arg_take_ascending(ArgBest& b, float v, int i) {
    if (v > b.v) { b.v = v; b.i = i; }
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
// workgroup's best into key (w mod 64) with one device-scope atomic max, then takes a ticket; in
// the workgroup with the last ticket the 64 lanes of wave 0 read one key each, the wave takes the
// largest, writes its index to *out and zeroes the keys and the counter for the next call.  A ticket is taken only once the max has
// returned, so the last ticket holder sees every candidate; device-scope atomics act on one
// coherent copy, and no cache write-back fence is needed.  Every thread of the workgroup must call
// it.  ws: keys at lines 0..63 ([0, 8) of each), the ticket counter at line 64; zero before the
// first call, and left zero by every call.
__device__ __forceinline__ unsigned long long arg_wave_max_u64(unsigned long long k) {
#pragma unroll
    for (int m = 32; m; m >>= 1) {
        const unsigned long long o = ((unsigned long long)(uint32_t)__shfl_xor((int)(k >> 32), m, 64) << 32) |
                                     (uint32_t)__shfl_xor((int)(uint32_t)k, m, 64);
        k = o > k ? o : k;
    }
    return k;
}

__device__ __forceinline__ void arg_grid_finish(ArgBest mine, uint8_t* ws, int* out) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (lane == 0) { sv[wave] = mine.v; si[wave] = mine.i; }
    __syncthreads();
    if (wave != 0) return;
    const unsigned int nwg = gridDim.x;
    const unsigned int nkey = nwg < (unsigned)ARG_SLOTS ? nwg : (unsigned)ARG_SLOTS;
    auto key = [&](unsigned int s) { return reinterpret_cast<unsigned long long*>(ws + (size_t)s * ARG_LINE); };
    unsigned int* ticket = reinterpret_cast<unsigned int*>(ws + (size_t)ARG_SLOTS * ARG_LINE);
    int last = 0;
    if (lane == 0) {
        ArgBest b = arg_init();
        for (int k = 0; k < nw; k++) b = arg_combine(b, ArgBest{sv[k], si[k]});
        atomicMax(key(blockIdx.x % nkey), arg_key(b));
        __builtin_amdgcn_s_waitcnt(0x0f70);                  // vmcnt(0): the max has completed
        last = atomicAdd(ticket, 1u) == nwg - 1;
    }
    if (!__shfl(last, 0, 64)) return;
    // the last workgroup: lane s reads key s (all in flight at once), the wave takes the largest
    const unsigned long long k = (unsigned)lane < nkey ? atomicAdd(key(lane), 0ull) : 0ull;
    const unsigned long long best = arg_wave_max_u64(k);
    if ((unsigned)lane < nkey) atomicExch(key(lane), 0ull);
    if (lane == 0) {
        *out = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
        atomicExch(ticket, 0u);
    }
}

}  // namespace kq
