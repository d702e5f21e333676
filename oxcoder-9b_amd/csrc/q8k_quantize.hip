// Q8_K activation quantizer for gfx950: one wave per 256-value block, 4 values per lane
// (block quantization in q8k_block.h).
#include "kq_device.h"
#include "kq_internal.h"
#include "q8k_block.h"

namespace kq {

__global__ void __launch_bounds__(256)
k_q8k_quantize(const float* __restrict__ x, int64_t ldx, int G, int nblocks, uint8_t* __restrict__ xq) {
    // every argument load issued before the first wait (one round trip to the arguments, not two)
    const int nthr = blockDim.x;
    KQ_ARGS_READY("s"(x), "s"(ldx), "s"(G), "s"(nblocks), "s"(xq), "s"(nthr));
    const int lane = threadIdx.x & 63;
    const int blk = blockIdx.x * (nthr >> 6) + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const int n = blk / G, g = blk - n * G;
    const f32x4 v = *reinterpret_cast<const f32x4_a4*>(x + (int64_t)n * ldx + (int64_t)g * QK + 4 * lane);
    const float e[4] = {v.x, v.y, v.z, v.w};
    q8k_block_store(e, lane, xq + (int64_t)blk * Q8K_BYTES);
}

// The same, also writing the quants in the prefill GEMM's fragment order (gemm_q8k.hip: xf[m/32][g][ks][l][16 B]
// = qs bytes 32ks + 16(l/32) .. +15 of row 32(m/32) + l%32): lane `lane` holds qs bytes 4 lane .. 4 lane + 3,
// i.e. K step lane/8, half (lane%8)/4, bytes 4(lane%4) of its 16.  Blocks of rows M .. Mpad-1 write zeros
// to the fragment copy only, as the stand-alone fragment copy does.
__global__ void __launch_bounds__(256)
k_q8k_quantize_frag(const float* __restrict__ x, int64_t ldx, int G, int M, int nblocks, uint8_t* __restrict__ xq,
                    uint8_t* __restrict__ xf) {
    const int nthr = blockDim.x;
    KQ_ARGS_READY("s"(x), "s"(ldx), "s"(G), "s"(M), "s"(nblocks), "s"(xq), "s"(xf), "s"(nthr));
    const int lane = threadIdx.x & 63;
    const int blk = blockIdx.x * (nthr >> 6) + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const int n = blk / G, g = blk - n * G;
    uint8_t* fo = xf + (((int64_t)(n >> 5) * G + g) * 8 + (lane >> 3)) * 1024 +
                  ((n & 31) + 32 * ((lane & 7) >> 2)) * 16 + 4 * (lane & 3);
    if (n >= M) {
        *reinterpret_cast<uint32_t*>(fo) = 0u;
        return;
    }
    const f32x4 v = *reinterpret_cast<const f32x4_a4*>(x + (int64_t)n * ldx + (int64_t)g * QK + 4 * lane);
    const float e[4] = {v.x, v.y, v.z, v.w};
    *reinterpret_cast<uint32_t*>(fo) = q8k_block_store(e, lane, xq + (int64_t)blk * Q8K_BYTES);
}

void launch_q8k_quantize_frag(const float* x, int64_t ldx, int C, int M, int Mpad, uint8_t* xq, uint8_t* xf,
                              hipStream_t s) {
    const int G = C / QK;
    const int nblocks = Mpad * G;
    const int wpb = 4;
    dim3 grid((nblocks + wpb - 1) / wpb), block(64 * wpb);
    hipLaunchKernelGGL(k_q8k_quantize_frag, grid, block, 0, s, x, ldx, G, M, nblocks, xq, xf);
}

void launch_q8k_quantize(const float* x, int64_t ldx, int C, int N, uint8_t* xq, hipStream_t s) {
    const int G = C / QK;
    const int nblocks = N * G;
    const int wpb = 4;
    dim3 grid((nblocks + wpb - 1) / wpb), block(64 * wpb);
    hipLaunchKernelGGL(k_q8k_quantize, grid, block, 0, s, x, ldx, G, nblocks, xq);
}

}  // namespace kq
