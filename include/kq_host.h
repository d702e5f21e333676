/*
 * kq_host.h -- C ABI of libkqhost.so: host-side preparation of synthetic quantized weights.
 *
 * The reference has no Q4_K/Q6_K quantizer: Kindi only reads pre-quantized GGUF tensors and
 * repacks them (scripts/kindi_q4/kindi/q4pack.py:110-180).  These functions produce GGML-format
 * blocks from fp32 matrices so the products can be exercised on seeded synthetic weights.  The
 * quantizer is this repository's own (deterministic, simple min/max scale search, documented
 * below); the block bytes it emits are ordinary Q4_K/Q6_K blocks that any GGML decoder reads.
 */
#ifndef KQ_HOST_H
#define KQ_HOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * w: R rows of C floats (row-major), C % 256 == 0.  out: R*(C/256) blocks in row order
 * [R][C/256][block] (the GGUF order, before the Kindi repack).
 *
 * Q4_K, per 256-block: for each 32-element sub-block, lo = min(0, min x), scale = (max x - lo)/15,
 * mn = -lo; d = fp16(max scale / 63), dmin = fp16(max mn / 63); sc = rint(scale/d), m = rint(mn/dmin)
 * clamped to 0..63; q = rint((x + dmin*m) / (d*sc)) clamped to 0..15 (0 where d*sc == 0).
 * Q6_K, per 256-block: for each 16-element sub-block, s = max|x| / 31; d = fp16(max s / 127);
 * sc = rint(s/d) clamped to -128..127; q = rint(x / (d*sc)) clamped to -32..31, stored as q+32.
 * Rounding is round-half-even; fp16 conversion is round-to-nearest-even.  Returns 0, or -1 on a
 * bad argument.
 */
int kq_host_quantize_q4k(const float* w, int64_t R, int C, uint8_t* out);
int kq_host_quantize_q6k(const float* w, int64_t R, int C, uint8_t* out);

/* Kindi repack [R][G][bs] -> [R/8][G][8][bs] (q4pack.py:155) and its inverse; R % 8 == 0. */
int kq_host_tile(const uint8_t* in, int64_t R, int C, int type, uint8_t* out);
int kq_host_untile(const uint8_t* in, int64_t R, int C, int type, uint8_t* out);

#ifdef __cplusplus
}
#endif

#endif /* KQ_HOST_H */
