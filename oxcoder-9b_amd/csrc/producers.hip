// Producers of the GEMV inputs for gfx950: RMSNorm and SwiGLU that write the Q8_K activation
// blocks directly (and, optionally, the fp32 values), so no separate quantizer pass re-reads them.
//
// k_rms_q8k follows the Q4 engine's q4_rms (scripts/kindi_q4/kindi/q4.cu:39-46): optional residual
// add into h, sum of squares in double with the same order (256 strided per-thread sums, then the
// shared-memory tree), s = 1 / sqrtf((float)(sum / D) + 1e-6f), xn = (h * s) * w.  The square of a
// float is exact in double and every double addition and the float steps are IEEE, so h, s and xn
// are bit-identical to that kernel's.  The CPU engine's rmsfold (kcpu4.c:123-139) adds the squares
// in sequence instead; the two orders give the same float s except when the double sum lies within
// a few double ulps of a float rounding boundary.
//
// k_swiglu_q8k follows q4_silu (q4.cu:36-38) and the CPU engine's FFN (kcpu4.c:77, 292):
// y = (g / (1 + exp(-g))) * u.  exp is kq_expf below, a binary32 exp built from IEEE single
// operations in a fixed order (Cody-Waite reduction by ln 2, degree-7 Taylor polynomial in Horner
// form, exact scaling by 2^n), so the oracle's C copy of the same steps gives the same bits; it is
// within 2 ulp of the exact exp, as CUDA's and glibc's expf are.
#include "kq_device.h"
#include "kq_internal.h"
#include "q8k_block.h"

namespace kq {

// 2^k as a float for k in [-126, 127].
__device__ __forceinline__ float pow2i(int k) { return __builtin_bit_cast(float, (uint32_t)(k + 127) << 23); }

__device__ __forceinline__ float kq_expf(float x) {
    if (x != x) return x + x;                           // NaN
    if (x > 0x1.62e42ep+6f) return __builtin_inff();    // above the largest x with exp(x) finite
    if (x < -0x1.9fe368p+6f) return 0.0f;               // exp(x) < 2^-150 rounds to zero
    const float n = __builtin_rintf(__fmul_rn(x, 0x1.715476p+0f));            // round(x / ln 2)
    // ln 2 = 0x1.62e4p-1 (15 significant bits: n * it is exact) + 0x1.7f7d1cp-20
    const float r = __fsub_rn(__fsub_rn(x, __fmul_rn(n, 0x1.62e4p-1f)), __fmul_rn(n, 0x1.7f7d1cp-20f));
    float p = 0x1.a01a02p-13f;                                  // 1/7!
    p = __fadd_rn(__fmul_rn(p, r), 0x1.6c16c2p-10f);            // 1/6!
    p = __fadd_rn(__fmul_rn(p, r), 0x1.111112p-7f);             // 1/5!
    p = __fadd_rn(__fmul_rn(p, r), 0x1.555556p-5f);             // 1/4!
    p = __fadd_rn(__fmul_rn(p, r), 0x1.555556p-3f);             // 1/3!
    p = __fadd_rn(__fmul_rn(p, r), 0x1p-1f);                    // 1/2!
    p = __fadd_rn(__fmul_rn(p, r), 1.0f);
    p = __fadd_rn(__fmul_rn(p, r), 1.0f);
    int k = (int)n;                                             // -150 .. 128
    if (k > 127) { p = __fmul_rn(p, 2.0f); k -= 1; }
    if (k < -126) return __fmul_rn(__fmul_rn(p, pow2i(k + 64)), 0x1p-64f);   // subnormal: one rounding
    return __fmul_rn(p, pow2i(k));
}

__device__ __forceinline__ float silu_mul(float g, float u) {
    return __fmul_rn(__fdiv_rn(g, __fadd_rn(1.0f, kq_expf(-g))), u);
}

// Lane t + N's value of v in lane t, for the lanes t < N of a halving step within a wave: the gfx950
// permlane swaps for N = 32, 16 (the second result holds rows 1 and 3, halves 1), DPP row_shl for
// N = 8 .. 1 (lane t <- lane t + N within its row of 16).  Lanes t >= N receive values no step uses.
template <int N>
__device__ __forceinline__ double lane_plus(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)u, hi = (uint32_t)(u >> 32);
    uint32_t a, b;
    if constexpr (N == 32) {
        a = xor32_pair(lo).b;
        b = xor32_pair(hi).b;
    } else if constexpr (N == 16) {
        a = xor16_pair(lo).b;
        b = xor16_pair(hi).b;
    } else {
        a = (uint32_t)dpp<0x100 + N>((int)lo);
        b = (uint32_t)dpp<0x100 + N>((int)hi);
    }
    return __builtin_bit_cast(double, ((uint64_t)b << 32) | a);
}

// One workgroup per row: 16 waves, or 8 when J > 32 (16 would leave 128 VGPRs per thread for the J
// row values and spill).  Threads 0..255 do the first pass (J >= D/256 row elements each, a
// compile-time count, so every load is unconditional: elements past D re-read element D-1 and are
// not used); every wave then quantizes 256-value blocks (D/256 of them, one per wave up to
// D = 4096), so the blocks' dependent cross-lane steps run side by side instead of one after
// another in a few waves.  Every global load of the row (h, residual, and the w values of pass 2)
// is issued up front, so the kernel waits for memory once.  Dynamic LDS holds the row (D floats)
// between the two passes.
template <int J> constexpr int rms_waves() { return J <= 32 ? 16 : 8; }
template <int J>
__global__ void __launch_bounds__(64 * rms_waves<J>())
k_rms_q8k(float* h, const float* res, int add, const float* __restrict__ w, int D, int64_t ld, float* xn,
          uint8_t* __restrict__ xq) {
    constexpr int RMS_WAVES = rms_waves<J>();
    constexpr int B = (J + RMS_WAVES - 1) / RMS_WAVES;   // Q8_K blocks per wave, at most
    extern __shared__ float hrow[];            // D floats
    __shared__ double sums[128];
    __shared__ double sums64[64];
    __shared__ float s_sh;
    const int t = threadIdx.x, row = blockIdx.x;
    const int lane = t & 63, wv = t >> 6;
    const int G = D / QK;
    float* hr = h + (int64_t)row * ld;
    const float* rr = res + (int64_t)row * ld;
    const bool first = t < 256;                // a thread of the first pass
    auto at = [&](int k) { const int i = t + 256 * k; return i < D ? i : D - 1; };

    float v[J];
    if (first) {
#pragma unroll
        for (int k = 0; k < J; k++) v[k] = hr[at(k)];
        if (add) {
            float r[J];
#pragma unroll
            for (int k = 0; k < J; k++) r[k] = rr[at(k)];
#pragma unroll
            for (int k = 0; k < J; k++) v[k] = __fadd_rn(v[k], r[k]);
        }
    }
    f32x4 wq[B];                               // pass 2 operands: w of blocks wv, wv + RMS_WAVES, ...
#pragma unroll
    for (int b = 0; b < B; b++) {
        const int g = wv + RMS_WAVES * b < G ? wv + RMS_WAVES * b : G - 1;
        wq[b] = *reinterpret_cast<const f32x4_a4*>(w + g * QK + 4 * lane);
    }

    // pass 1: thread t's partial sum over i = t, t + 256, ... in sequence (q4.cu:41).  The updated
    // h goes to LDS now and to memory at the end, so no barrier below waits for global stores.
    double sum = 0.0;
    if (first) {
#pragma unroll
        for (int k = 0; k < J; k++) {
            if (t + 256 * k < D) {
                hrow[t + 256 * k] = v[k];
                sum = __dadd_rn(sum, __dmul_rn((double)v[k], (double)v[k]));
            }
        }
    }
    // the halving tree of q4.cu:42-43: sums[t] += sums[t + n] for n = 128, 64, ..., 1; the n = 64
    // level has its own array (no barrier between its stores and the n = 128 reads), and n = 32 .. 1
    // run in wave 0's registers
    if (t >= 128 && t < 256) sums[t - 128] = sum;
    __syncthreads();
    if (t < 128) {
        sum = __dadd_rn(sum, sums[t]);                           // n = 128
        if (t >= 64) sums64[t - 64] = sum;
    }
    __syncthreads();
    if (t < 64) {
        sum = __dadd_rn(sum, sums64[t]);                         // n = 64
        sum = __dadd_rn(sum, lane_plus<32>(sum));                // lane t += lane t + n
        sum = __dadd_rn(sum, lane_plus<16>(sum));
        sum = __dadd_rn(sum, lane_plus<8>(sum));
        sum = __dadd_rn(sum, lane_plus<4>(sum));
        sum = __dadd_rn(sum, lane_plus<2>(sum));
        sum = __dadd_rn(sum, lane_plus<1>(sum));
        if (t == 0) {
            // sqrtf correctly rounded: the double square root of a float, rounded to float, is
            // (53 >= 2*24 + 2 bits), while v_sqrt_f32 alone is not
            // sum / D; for D = 2^k the product with 2^-k is the same double, without a division
            const double mean = (D & (D - 1)) == 0
                ? __dmul_rn(sum, __builtin_bit_cast(double, (uint64_t)(1023 - __builtin_ctz((unsigned)D)) << 52))
                : __ddiv_rn(sum, (double)D);
            const float ms = __fadd_rn((float)mean, 1e-6f);
            s_sh = __fdiv_rn(1.0f, (float)__dsqrt_rn((double)ms));
        }
    }
    __syncthreads();
    const float s = s_sh;

    // pass 2: Q8_K blocks; wave wv takes blocks wv, wv + RMS_WAVES, ...; lane l the values 4l .. 4l+3.
    // xn may be h itself: the values come from LDS.
    float* xr = xn ? xn + (int64_t)row * ld : nullptr;
#pragma unroll
    for (int b = 0; b < B; b++) {
        const int g = wv + RMS_WAVES * b;
        if (g >= G) break;
        const int i0 = g * QK + 4 * lane;
        const f32x4 hv = *reinterpret_cast<const f32x4*>(hrow + i0);
        float e[4];
        e[0] = __fmul_rn(__fmul_rn(hv.x, s), wq[b].x);
        e[1] = __fmul_rn(__fmul_rn(hv.y, s), wq[b].y);
        e[2] = __fmul_rn(__fmul_rn(hv.z, s), wq[b].z);
        e[3] = __fmul_rn(__fmul_rn(hv.w, s), wq[b].w);
        if (xr) *reinterpret_cast<f32x4_a4*>(xr + i0) = f32x4{e[0], e[1], e[2], e[3]};
        q8k_block_store(e, lane, xq + ((int64_t)row * G + g) * Q8K_BYTES);
    }
    // h += residual, written back; when xn is h itself the normalised values written above are
    // the row's final contents (as when q4_rms writes h and then xn over it)
    if (first && add && xn != h) {
#pragma unroll
        for (int k = 0; k < J; k++)
            if (t + 256 * k < D) hr[t + 256 * k] = v[k];
    }
}

// One wave per 256-value block.
__global__ void __launch_bounds__(256)
k_swiglu_q8k(const float* __restrict__ gate, const float* __restrict__ up, int G, int64_t ld, int nblocks,
             float* __restrict__ y, uint8_t* __restrict__ xq) {
    const int nthr = blockDim.x;
    KQ_ARGS_READY("s"(gate), "s"(up), "s"(G), "s"(ld), "s"(nblocks), "s"(y), "s"(xq), "s"(nthr));
    const int lane = threadIdx.x & 63;
    const int blk = blockIdx.x * (nthr >> 6) + (threadIdx.x >> 6);
    if (blk >= nblocks) return;
    const int n = blk / G, g = blk - n * G;
    const int64_t i0 = (int64_t)n * ld + (int64_t)g * QK + 4 * lane;
    const f32x4 gv = *reinterpret_cast<const f32x4_a4*>(gate + i0);
    const f32x4 uv = *reinterpret_cast<const f32x4_a4*>(up + i0);
    float e[4];
    e[0] = silu_mul(gv.x, uv.x);
    e[1] = silu_mul(gv.y, uv.y);
    e[2] = silu_mul(gv.z, uv.z);
    e[3] = silu_mul(gv.w, uv.w);
    if (y) *reinterpret_cast<f32x4_a4*>(y + i0) = f32x4{e[0], e[1], e[2], e[3]};
    q8k_block_store(e, lane, xq + (int64_t)blk * Q8K_BYTES);
}

void launch_rms_q8k(float* h, const float* res, int add, const float* w, int D, int N, int64_t ld, float* xn,
                    uint8_t* xq, hipStream_t s) {
    const size_t lds = (size_t)D * sizeof(float);
    const int j = (D + 255) / 256;             // row elements per thread: 1 .. 64 (D <= 16384)
    const dim3 grid(N);
    const float* r = res ? res : h;
#define KQ_RMS_LAUNCH(JJ) \
    hipLaunchKernelGGL(k_rms_q8k<JJ>, grid, dim3(64 * rms_waves<JJ>()), lds, s, h, r, add, w, D, ld, xn, xq)
    if (j <= 4) KQ_RMS_LAUNCH(4);
    else if (j <= 8) KQ_RMS_LAUNCH(8);
    else if (j <= 16) KQ_RMS_LAUNCH(16);
    else if (j <= 32) KQ_RMS_LAUNCH(32);
    else if (j <= 48) KQ_RMS_LAUNCH(48);
    else KQ_RMS_LAUNCH(64);
#undef KQ_RMS_LAUNCH
}

void launch_swiglu_q8k(const float* gate, const float* up, int n, int N, int64_t ld, float* y, uint8_t* xq,
                       hipStream_t s) {
    const int G = n / QK, nblocks = N * G, wpb = 4;
    hipLaunchKernelGGL(k_swiglu_q8k, dim3((nblocks + wpb - 1) / wpb), dim3(64 * wpb), 0, s, gate, up, G, ld,
                       nblocks, y, xq);
}

}  // namespace kq
