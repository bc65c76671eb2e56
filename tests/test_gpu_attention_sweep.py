"""A seeded sweep of attention shapes through ops.attention against float64 attention of the same (dequantised
or rounded) inputs (the reference's tests/test_attention.py:9-21 convention), at the north-star tolerance:
random head counts (up to 600 one-tile heads, so that the tail split, the XCD order and the reversed key order
of later rounds all occur), GQA ratios, ragged query and key counts, int8 (rotation-free per-row codes with
outlier channels) and bf16 / f16 inputs, and all three output types. Every case prints its parameters before
it runs."""

import numpy as np
import pytest

from h3metal_amd import ops
from oracle import attention as oa
from oracle.bf16 import from_bf16, to_bf16

pytestmark = pytest.mark.gpu

NS_MAX, NS_MEAN = 2e-2, 1e-3
D = 128


def case(seed):
    rng = np.random.default_rng(1000 + seed)
    big = seed % 4 == 3  # many short heads: more workgroups than CUs
    if big:
        H = int(rng.integers(257, 601))
        Lq, L = int(rng.integers(1, 257)), int(rng.integers(1, 400))
    else:
        H = int(rng.integers(1, 41))
        Lq, L = int(rng.integers(1, 700)), int(rng.integers(1, 1100))
    ratios = [r for r in (1, 2, 3, 4, 8) if H % r == 0]
    KVH = H // int(rng.choice(ratios))
    path = ["int8", "bf16", "f16"][seed % 3]
    out_dt = ["bf16", "f16", "f32"][(seed // 3) % 3]
    return rng, H, KVH, Lq, L, path, out_dt


def padded(gpu, arr, rows, dtype):
    full = np.zeros((arr.shape[0], rows) + arr.shape[2:], arr.dtype)
    full[:, :arr.shape[1]] = arr
    t = gpu.empty(full.shape, dtype)
    t.write(full)
    return t


@pytest.mark.parametrize("seed", range(24))
def test_random_shape_against_float64(gpu, seed):
    rng, H, KVH, Lq, L, path, out_dt = case(seed)
    print(f"[sweep] seed={seed} H={H} KVH={KVH} Lq={Lq} L={L} path={path} out={out_dt}", flush=True)
    q_rows, k_rows = (Lq + 63) // 64 * 64, (L + 31) // 32 * 32
    xq = rng.standard_normal((H, Lq, D)).astype(np.float32)
    xk = rng.standard_normal((KVH, L, D)).astype(np.float32)
    xv = rng.standard_normal((KVH, L, D)).astype(np.float32)
    vb = to_bf16(xv) if path != "f16" else None
    extra = {}
    if path == "int8":
        xq[..., :2] *= 8  # outlier channels
        xk[..., 3:5] *= 8
        qs = np.abs(xq).max(-1) / 127
        ks = np.abs(xk).max(-1) / 127
        qi = np.rint(xq / qs[..., None]).astype(np.int8)
        ki = np.rint(xk / ks[..., None]).astype(np.int8)
        qs, ks = qs.astype(np.float32), ks.astype(np.float32)
        Q, K = padded(gpu, qi, q_rows, "i8"), padded(gpu, ki, k_rows, "i8")
        V = padded(gpu, vb, k_rows, "bf16")
        extra = dict(q_scale=padded(gpu, qs, q_rows, "f32"), k_scale=padded(gpu, ks, k_rows, "f32"))
        qr, kr, vr = qi * qs[..., None].astype(np.float64), ki * ks[..., None].astype(np.float64), from_bf16(vb)
    elif path == "bf16":
        qb, kb = to_bf16(xq), to_bf16(xk)
        Q, K, V = padded(gpu, qb, q_rows, "bf16"), padded(gpu, kb, k_rows, "bf16"), padded(gpu, vb, k_rows, "bf16")
        qr, kr, vr = from_bf16(qb), from_bf16(kb), from_bf16(vb)
    else:
        qh, kh, vh = xq.astype(np.float16), xk.astype(np.float16), xv.astype(np.float16)
        Q, K, V = padded(gpu, qh, q_rows, "f16"), padded(gpu, kh, k_rows, "f16"), padded(gpu, vh, k_rows, "f16")
        qr, kr, vr = qh, kh, vh
    O = gpu.empty((q_rows, H * D), out_dt)
    ops.attention(gpu, Q, K, V, O, Lq=Lq, L=L, H=H, KVH=KVH, D=D, q_rows=q_rows, k_rows=k_rows, scale=D ** -0.5,
                  **extra)
    gpu.wait()
    o = O.numpy()[:Lq]
    got = from_bf16(o) if out_dt == "bf16" else o.astype(np.float64)
    ref = oa.ref_attention(qr, kr, vr, D ** -0.5)
    err = np.abs(got.astype(np.float64) - ref)
    assert np.isfinite(got).all()
    assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean())
