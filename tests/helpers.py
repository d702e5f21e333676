"""Shared test inputs and checks."""
import numpy as np


def reference_unit_inputs():
    """Inputs of the reference test tests/kindi_q4/test_quant.py:12-30, regenerated in order."""
    BLOCK = {12: 144, 14: 210}
    rng = np.random.default_rng(35)
    out = {}
    for ty in (12, 14):
        rows, cols = 16, 512
        raw = rng.integers(0, 256, (rows, cols // 256, BLOCK[ty]), dtype=np.uint8)
        for offset in ([0, 2] if ty == 12 else [208]):
            raw[:, :, offset:offset + 2] = np.array([0.013], dtype="<f2").view(np.uint8)
        tile = raw.reshape(rows // 8, 8, cols // 256, BLOCK[ty]).transpose(0, 2, 1, 3).copy().reshape(-1)
        x = rng.normal(size=cols).astype(np.float32)
        out[ty] = (tile, x, rows, cols)
    return out

