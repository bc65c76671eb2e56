"""Restatement of the projection product gemm (weight formats q8, h8, f16, bf16).

Test infrastructure only (see oracle/__init__.py).

Follows the reference kernel kernels/gemm.metal (WFMT 1: :1-40 formats, :118-261 product and epilogue;
parameters kernels/params.h:7-16; launcher h3metal/ops.py:124-174):

  acc[m][n] = sum_k a[m][k] * w[n][k]               exact integer product (int64 here)
  v         = float(acc) * sa[m] * sw[n]             float32, left to right   gemm.metal:237-238
  v        += bias[n]                                 (HAS_BIAS)               gemm.metal:249-251
  EPI 0     out = OUT_T(v)                                                     gemm.metal:255-256
  EPI 1     x  += gate[rtype[m]][n] * v              (x float32)              gemm.metal:257-259

h8 / f16 / bf16 (gemm.metal WFMT 6 / 4 / 5): acc = sum_k a[m][k] * w[n][k] accumulated in float32 by the
matrix unit (exact products; summation order unspecified), v = acc * sw[n] (h8) or acc, then the same bias and
epilogues. The restatement sums in float64; parity for these formats is the reference's own tolerance
(tests/test_gemm.py:20-84: max error below 2e-3 of the largest output, 1e-2 for bfloat outputs).

Pinning status: the integer product is exact (checked against brute-force Python integer sums); the float
epilogue is one rounding per step in this order, checked against float64 closed forms within float32 rounding
and on hand-made values where every step is exact.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def int_product(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Exact a @ w^T of int8 codes, a [M][K], w [N][K] -> int64 [M][N]. Computed in float64, which is exact
    while |acc| < 2^53 (K * 127^2 < 2^53 for any K below 5e11)."""
    acc = a.astype(np.float64) @ w.astype(np.float64).T
    return acc.astype(np.int64)


def epilogue(acc: np.ndarray, sa: np.ndarray, sw: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """float32 v = float(acc) * sa[m] * sw[n] (+ bias[n]), one rounding per operation, in the reference's order."""
    v = acc.astype(F32) * sa.astype(F32)[:, None]
    v = (v * sw.astype(F32)[None, :]).astype(F32)
    if bias is not None:
        v = (v + bias.astype(F32)[None, :]).astype(F32)
    return v


def residual(x: np.ndarray, v: np.ndarray, gate: np.ndarray, rtype: np.ndarray) -> np.ndarray:
    """EPI 1: x + gate[rtype[m]][n] * v in float32 (the product rounded, then the sum)."""
    g = gate.astype(F32)[rtype.astype(np.int64)]
    return (x.astype(F32) + (g * v).astype(F32)).astype(F32)


def float_product(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """a @ w^T in float64 for half / bfloat-valued (or int8 code) operands given as float arrays."""
    return a.astype(np.float64) @ w.astype(np.float64).T
