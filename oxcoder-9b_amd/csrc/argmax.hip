// Argmax of a float vector for gfx950 (greedy decoding over the logits), one launch: a grid of
// workgroups scans the vector, the last one to finish reduces their partials (argmax_block.h).
#include "argmax_block.h"
#include "kq_internal.h"

namespace kq {

__global__ void __launch_bounds__(256) k_argmax(const float* __restrict__ y, int n, uint8_t* ws, int* out) {
    ArgBest b = arg_init();
    const int stride = gridDim.x * blockDim.x;
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    for (; i + 3 * stride < n; i += 4 * stride) {          // four loads in flight per thread
        const float v0 = y[i], v1 = y[i + stride], v2 = y[i + 2 * stride], v3 = y[i + 3 * stride];
        arg_take(b, v0, i);
        arg_take(b, v1, i + stride);
        arg_take(b, v2, i + 2 * stride);
        arg_take(b, v3, i + 3 * stride);
    }
    for (; i < n; i += stride) arg_take(b, y[i], i);
    arg_grid_finish(arg_wave_reduce(b), ws, out);
}

size_t argmax_workspace_bytes() { return ARGMAX_WS_BYTES; }

#ifndef KQ_ARGMAX_PER_THREAD
#define KQ_ARGMAX_PER_THREAD 16
#endif
void launch_argmax(const float* y, int n, uint8_t* ws, int* out, hipStream_t s) {
    constexpr int per = KQ_ARGMAX_PER_THREAD;               // values per thread, about
    int nwg = (n + 256 * per - 1) / (256 * per);
    nwg = nwg < 1 ? 1 : (nwg > 2 * device_cus() ? 2 * device_cus() : nwg);
    hipLaunchKernelGGL(k_argmax, dim3(nwg), dim3(256), 0, s, y, n, ws, out);
}

}  // namespace kq
