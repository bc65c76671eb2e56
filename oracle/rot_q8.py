"""float32 op-by-op restatement of the row rotation + int8 rot_q8.

Test infrastructure only (see oracle/__init__.py).

Follows the reference kernel kernels/ops.metal:272-334 (helpers :19-47,
parameters kernels/params.h:25-29, launcher h3metal/ops.py:214-222), every step
one IEEE-rounded float32 numpy operation:

  input     x[m, :D]; swiglu (mode 1): x[m, :D] * (g / (1 + exp(-g))),
            g = x[m, D:2D]                                        ops.metal:270, 291-292
  rotate    per 256-column block: butterfly stages over the column
            bits 0..7 in increasing order, (a + b, a - b) with a the
            lower column, then * 0.0625                            ops.metal:19-47, 294
  int8      scale = amax/127 over the whole row (1 if amax == 0);
            code = rint(v * (1 / scale))                           ops.metal:304-327
  OUT_HR    the rotated row rounded to float16 instead             ops.metal:297-306

Pinning status: the rotation is pinned by closed forms in tests/test_oracle.py
(the Sylvester Hadamard matrix product the reference's own test uses,
tests/test_ops.py:9-18; orthonormality, one-hot inputs, involution), the int8
step by its round trip and the amax = 0 case. The swiglu gate uses numpy's
float32 exp: the reference's Metal exp and the gfx950 library exp may differ
from it in the last bit, so swiglu codes are compared within one code (parity
unpinned at the exp's last ulp).
"""

from __future__ import annotations

import numpy as np

from .prepass import fwht_f32

F32 = np.float32
RB = 256


def silu_gated_f32(x: np.ndarray, D: int) -> np.ndarray:
    """value * silu(gate) in the reference's order: v * (g / (1 + exp(-g))) (ops.metal:270, 292)."""
    v = x[:, :D].astype(F32)
    g = x[:, D:2 * D].astype(F32)
    return (v * (g / (F32(1) + np.exp(-g)))).astype(F32)


def rotate_rows_f32(v: np.ndarray) -> np.ndarray:
    """Every 256-column block times the 256-point Walsh-Hadamard matrix over 16 (ops.metal:19-47)."""
    M, D = v.shape
    r = fwht_f32(v.astype(F32).reshape(M, D // RB, RB)).reshape(M, D)
    return (r * F32(0.0625)).astype(F32)


def rot_q8(x: np.ndarray, D: int, swiglu: bool = False):
    """(codes int8 [M][D], scales float32 [M], rotated float32 [M][D]) of rot_q8 on rows x."""
    v = silu_gated_f32(x, D) if swiglu else x[:, :D].astype(F32)
    r = rotate_rows_f32(v)
    amax = np.abs(r).max(-1)
    scale = np.where(amax > 0, amax / F32(127), F32(1)).astype(F32)
    rs = (F32(1) / scale).astype(F32)
    codes = np.rint(r * rs[:, None]).astype(np.int8)
    return codes, scale, r
