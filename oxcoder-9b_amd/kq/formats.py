"""Block formats and the Kindi 8-row repack (host side, numpy).

Q4_K (type 12) and Q6_K (type 14) are GGML's super-block formats as Kindi decodes them
(scripts/kindi_q4/kindi/q4kernels.h:12-33, q4pack.py:52-76); Q8_K is GGML's block_q8_K.
The Kindi pack stores a matrix as [R/8][C/256][8][block] (q4pack.py:151-160).
"""
import numpy as np

QK = 256
Q4_K = 12
Q6_K = 14
BLOCK = {Q4_K: 144, Q6_K: 210}          # q4pack.py:18
Q8K_BYTES = 292
PAGE = 16384                            # q4pack.py:19: tensors start on 16 KiB boundaries
TYPE_NAMES = {Q4_K: "Q4_K", Q6_K: "Q6_K"}


def check_shape(R, C, ty):
    """The packed-tensor constraints of q4pack.py:97-103 and :131 (raises ValueError)."""
    if ty not in BLOCK:
        raise ValueError("Invalid tensor type %r" % (ty,))
    if R <= 0 or C <= 0 or R % 8 or C % QK:
        raise ValueError("Invalid packed tensor dimensions %dx%d" % (R, C))


def tensor_bytes(R, C, ty):
    check_shape(R, C, ty)
    return R * (C // QK) * BLOCK[ty]


def q8k_bytes(N, C):
    return N * (C // QK) * Q8K_BYTES


def tile(raw, R, C, ty):
    """GGUF row order [R][G][bs] -> Kindi layout [R/8][G][8][bs] (q4pack.py:155)."""
    check_shape(R, C, ty)
    G, bs = C // QK, BLOCK[ty]
    a = np.asarray(raw, np.uint8).reshape(R // 8, 8, G, bs)
    return np.ascontiguousarray(a.transpose(0, 2, 1, 3)).reshape(-1)


def untile(packed, R, C, ty):
    """Inverse of tile (q4pack.py:156 checks this round trip during conversion)."""
    check_shape(R, C, ty)
    G, bs = C // QK, BLOCK[ty]
    a = np.asarray(packed, np.uint8).reshape(R // 8, G, 8, bs)
    return np.ascontiguousarray(a.transpose(0, 2, 1, 3)).reshape(-1)


def block_offset(R, C, ty, row, g):
    """Byte offset of block (row, g) in the Kindi layout (q4kernels.h:8-10)."""
    G = C // QK
    return (((row // 8) * G + g) * 8 + row % 8) * BLOCK[ty]
