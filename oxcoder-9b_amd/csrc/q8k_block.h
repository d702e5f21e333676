// Q8_K quantization of one 256-value block by one wave (64 lanes, 4 consecutive values per lane),
// shared by the stand-alone quantizer and the fused producers (RMSNorm, SwiGLU).
//
// Semantics (GGML quantize_row_q8_K_ref): max = signed value of the first element with the
// largest |x|; iscale = -127/max; q = min(127, round-half-even(iscale*x)); d = 1/iscale;
// bsums[k] = sum of q[16k..16k+15]; an all-zero block gives d = 0, q = 0, bsums = 0.
// Division is IEEE, so d and the quants match the CPU bit for bit.
#pragma once
#include "kq_device.h"

namespace kq {

// e: this lane's values 4*lane .. 4*lane+3 of the block; ob: the block's 292 output bytes.
// Every lane of the wave must call it (cross-lane reductions).  Returns the lane's four quants
// (qs bytes 4*lane .. 4*lane+3, as stored).
__device__ __forceinline__ uint32_t q8k_block_store(const float (&e)[4], int lane, uint8_t* __restrict__ ob) {
    // max |x| over the block: butterfly max (exact, order-free); NaN never wins (v_max returns
    // the other operand), matching the strict "ax > amax" scan of the reference definition.
    float amax = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(e[0]), __builtin_fabsf(e[1])),
                                 __builtin_fmaxf(__builtin_fabsf(e[2]), __builtin_fabsf(e[3])));
    amax = __builtin_fmaxf(amax, dppf<DPP_QUAD_XOR1>(amax));
    amax = __builtin_fmaxf(amax, dppf<DPP_QUAD_XOR2>(amax));
    amax = __builtin_fmaxf(amax, dppf<DPP_ROW_HALF_MIRROR>(amax));
    amax = __builtin_fmaxf(amax, dppf<DPP_ROW_MIRROR>(amax));
    amax = xor16_max(amax);
    amax = xor32_max(amax);
    // signed value of the first element with |x| == amax: lowest lane holding one, lowest k in it
    float first = 0.0f;
    bool has = false;
#pragma unroll
    for (int k = 3; k >= 0; k--)
        if (__builtin_fabsf(e[k]) == amax) { first = e[k]; has = true; }
    const uint64_t holders = __ballot(has);
    const int src = holders ? __builtin_ctzll(holders) : 0;
    const float vmax = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, first), src));

    uint32_t packed = 0;
    int s4 = 0;
    float d = 0.0f;
    if (amax != 0.0f) {
        const float iscale = -127.0f / vmax;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float t = __fmul_rn(iscale, e[k]);
            int q = (int)__builtin_rintf(t);
            q = q < 127 ? q : 127;
            s4 += q;
            packed |= (uint32_t)(q & 0xff) << (8 * k);
        }
        d = 1.0f / iscale;
    }
    // 16-value sums: lanes 4j..4j+3 hold values 16j..16j+15.
    s4 = quad_sum_i32(s4);
    // Pack two adjacent sums (lanes 8k and 8k+4 hold sums 2k, 2k+1) into one dword for the store:
    // lane 8k reads lane 8k+7 through the half-row mirror.
    const int s_next = dpp<DPP_ROW_HALF_MIRROR>(s4);

    *reinterpret_cast<uint32_t*>(ob + 4 + 4 * lane) = packed;
    if (lane == 0) *reinterpret_cast<float*>(ob) = d;
    if ((lane & 7) == 0) {
        const uint32_t pair = ((uint32_t)s4 & 0xffffu) | ((uint32_t)s_next << 16);
        *reinterpret_cast<uint32_t*>(ob + 260 + 4 * (lane >> 3)) = pair;
    }
    return packed;
}

// NB blocks quantized by one wave at once (e[b]: this lane's values 4*lane .. 4*lane+3 of block b,
// ob[b]: its 292 output bytes): the bytes of q8k_block_store on each block, with the blocks'
// dependent steps (cross-lane maximum, first-maximum pick, divisions, sums) issued side by side in
// one straight-line sequence; an all-zero block takes iscale = 0 by a select (every quant 0, d 0),
// not a branch.
template <int NB>
__device__ __forceinline__ void q8k_blocks_store(const float (&e)[NB][4], int lane, uint8_t* const (&ob)[NB]) {
    float amax[NB];
#pragma unroll
    for (int b = 0; b < NB; b++)
        amax[b] = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(e[b][0]), __builtin_fabsf(e[b][1])),
                                  __builtin_fmaxf(__builtin_fabsf(e[b][2]), __builtin_fabsf(e[b][3])));
#pragma unroll
    for (int b = 0; b < NB; b++) amax[b] = __builtin_fmaxf(amax[b], dppf<DPP_QUAD_XOR1>(amax[b]));
#pragma unroll
    for (int b = 0; b < NB; b++) amax[b] = __builtin_fmaxf(amax[b], dppf<DPP_QUAD_XOR2>(amax[b]));
#pragma unroll
    for (int b = 0; b < NB; b++) amax[b] = __builtin_fmaxf(amax[b], dppf<DPP_ROW_HALF_MIRROR>(amax[b]));
#pragma unroll
    for (int b = 0; b < NB; b++) amax[b] = __builtin_fmaxf(amax[b], dppf<DPP_ROW_MIRROR>(amax[b]));
#pragma unroll
    for (int b = 0; b < NB; b++) amax[b] = xor16_max(amax[b]);
#pragma unroll
    for (int b = 0; b < NB; b++) amax[b] = xor32_max(amax[b]);
    float iscale[NB], d[NB];
    bool nz[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        float first = 0.0f;
        bool has = false;
#pragma unroll
        for (int k = 3; k >= 0; k--)
            if (__builtin_fabsf(e[b][k]) == amax[b]) { first = e[b][k]; has = true; }
        const uint64_t holders = __ballot(has);
        const int src = holders ? __builtin_ctzll(holders) : 0;
        const float vmax = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, first), src));
        nz[b] = amax[b] != 0.0f;
        iscale[b] = nz[b] ? -127.0f / vmax : 0.0f;
        d[b] = nz[b] ? 1.0f / iscale[b] : 0.0f;
    }
    uint32_t packed[NB];
    int s4[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        packed[b] = 0;
        s4[b] = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            int q = (int)__builtin_rintf(__fmul_rn(iscale[b], e[b][k]));
            q = !nz[b] ? 0 : q < 127 ? q : 127;
            s4[b] += q;
            packed[b] |= (uint32_t)(q & 0xff) << (8 * k);
        }
    }
    uint32_t pair[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        s4[b] = quad_sum_i32(s4[b]);
        const int s_next = dpp<DPP_ROW_HALF_MIRROR>(s4[b]);
        pair[b] = ((uint32_t)s4[b] & 0xffffu) | ((uint32_t)s_next << 16);
    }
#pragma unroll
    for (int b = 0; b < NB; b++) *reinterpret_cast<uint32_t*>(ob[b] + 4 + 4 * lane) = packed[b];
    if (lane == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++) *reinterpret_cast<float*>(ob[b]) = d[b];
    }
    if ((lane & 7) == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++) *reinterpret_cast<uint32_t*>(ob[b] + 260 + 4 * (lane >> 3)) = pair[b];
    }
}

}  // namespace kq
