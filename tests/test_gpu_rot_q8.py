"""rot_q8 (the attention output's consumer, reference kernels/ops.metal:272-334, launcher h3metal/ops.py:214-222)
against the float32 oracle: codes and scales bit-exact without the swiglu gate, within one code with it (the exp's
last bit is library-specific); the reference's own tolerance test (tests/test_ops.py:54-78) at its shape; and the
attention -> rot_q8 chain of h3metal/dit.py:204-209."""

import numpy as np
import pytest

from h3metal_amd import ops
from h3metal_amd.gpu import GpuError
from oracle import rot_q8 as orq
from oracle.bf16 import from_bf16, to_bf16

pytestmark = pytest.mark.gpu


def host_rows(rng, M, W, dt, scale=2.0):
    """Rows in the input dtype and their exact float32 values."""
    x = (rng.standard_normal((M, W)) * scale).astype(np.float32)
    if dt == "bf16":
        b = to_bf16(x)
        return b, from_bf16(b)
    if dt == "f16":
        h = x.astype(np.float16)
        return h, h.astype(np.float32)
    return x, x


def run_rot(gpu, xh, dt, M, D, *, swiglu=False, x_stride=None, out_hr=False):
    print(f"[rot_q8] M={M} D={D} in={dt} swiglu={swiglu} x_stride={x_stride} out_hr={out_hr}", flush=True)
    X = gpu.upload(xh, dt)
    out = gpu.empty((M, D), "f16" if out_hr else "i8")
    sa = None if out_hr else gpu.empty((M,), "f32")
    ops.rot_q8(gpu, X, out, sa, M, D, swiglu=swiglu, x_stride=x_stride, out_hr=out_hr)
    gpu.wait()
    return out.numpy(), (None if out_hr else sa.numpy())


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("M,D", [(1, 256), (19, 1024), (37, 4096), (5, 5376), (3, 14336)])
def test_codes_and_scales_bit_exact(gpu, dt, M, D):
    rng = np.random.default_rng(M * 7 + D)
    xh, xf = host_rows(rng, M, D, dt)
    codes, sa = run_rot(gpu, xh, dt, M, D)
    wc, ws, _ = orq.rot_q8(xf, D)
    assert np.array_equal(sa.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(codes, wc)


@pytest.mark.parametrize("mag", [2e-37, 1e-36, 1e-33, 1e-20, 1.0, 1e4])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_tiny_and_large_rows_bit_exact(gpu, mag, dt):
    """Rows from 2e-37 (rotated values partly subnormal, 1 / scale near the float range's top) to 1e4: codes and
    scales bit for bit."""
    rng = np.random.default_rng(int(-np.log10(mag) * 10) + 500)
    M, D = 8, 1024
    x = (rng.standard_normal((M, D)) * mag).astype(np.float32)
    xh = to_bf16(x) if dt == "bf16" else x
    xf = from_bf16(xh) if dt == "bf16" else xh
    codes, sa = run_rot(gpu, xh, dt, M, D)
    wc, ws, _ = orq.rot_q8(xf, D)
    assert np.isfinite(ws).all() and np.isfinite(1 / ws).all()
    assert np.array_equal(sa.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(codes, wc)


@pytest.mark.parametrize("seed", range(12))
def test_random_shape_sweep_bit_exact(gpu, seed):
    """A seeded sweep: widths of 1 to 56 Hadamard blocks of 256, up to 3000 rows, three input types, some rows
    with outlier channels or all zeros: codes and scales bit for bit."""
    rng = np.random.default_rng(4000 + seed)
    dt = ["bf16", "f16", "f32"][seed % 3]
    D = 256 * int(rng.integers(1, 57))
    M = int(rng.integers(1, 3001))
    x = (rng.standard_normal((M, D)) * 2).astype(np.float32)
    x[rng.integers(0, M, 3)[:, None], rng.integers(0, D, 4)[None, :]] *= 50  # outliers
    x[rng.integers(0, M)] = 0
    xh = to_bf16(x) if dt == "bf16" else x.astype(np.float16) if dt == "f16" else x
    xf = from_bf16(xh) if dt == "bf16" else xh.astype(np.float32)
    codes, sa = run_rot(gpu, xh, dt, M, D)
    wc, ws, _ = orq.rot_q8(xf, D)
    assert np.array_equal(sa.view(np.uint32), ws.view(np.uint32))
    assert np.array_equal(codes, wc)


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_rotated_half_output_exact(gpu, dt):
    rng = np.random.default_rng(11)
    M, D = 13, 2048
    xh, xf = host_rows(rng, M, D, dt)
    oh, _ = run_rot(gpu, xh, dt, M, D, out_hr=True)
    _, _, r = orq.rot_q8(xf, D)
    assert np.array_equal(oh.view(np.uint16), r.astype(np.float16).view(np.uint16))


def test_swiglu_within_one_code(gpu):
    rng = np.random.default_rng(12)
    M, D = 21, 3072
    xh, xf = host_rows(rng, M, 2 * D, "bf16")
    codes, sa = run_rot(gpu, xh, "bf16", M, D, swiglu=True)
    wc, ws, _ = orq.rot_q8(xf, D, swiglu=True)
    np.testing.assert_allclose(sa, ws, rtol=2e-6, atol=0)
    assert np.abs(codes.astype(np.int32) - wc.astype(np.int32)).max() <= 1
    assert (codes != wc).mean() < 1e-3


def test_reference_tolerance_case(gpu):
    """tests/test_ops.py::test_rot at its own shape (M=19, D=14336, swiglu, bf16 input): dequantised rows within
    0.6/127 of the float64 rotation (relative to the row maximum), the rotated half output within 2e-3."""
    rng = np.random.default_rng(2)
    M, D = 19, 14336
    xin = (rng.standard_normal((M, 2 * D)) * 2).astype(np.float32)
    xb = to_bf16(xin)
    xf = from_bf16(xb).astype(np.float64)
    g = xf[:, D:]
    y = xf[:, :D] * g / (1 + np.exp(-g))
    H = np.array([[1.0]])
    while H.shape[0] < 256:
        H = np.block([[H, H], [H, -H]])
    r = (y.reshape(M, D // 256, 256) @ (H / 16.0).T).reshape(M, D)
    codes, sa = run_rot(gpu, xb, "bf16", M, D, swiglu=True)
    err = np.abs(codes.astype(np.float64) * sa[:, None] - r).max() / np.abs(r).max()
    assert err < 0.6 / 127
    oh, _ = run_rot(gpu, xb, "bf16", M, D, swiglu=True, out_hr=True)
    e2 = np.abs(oh.astype(np.float64) - r).max() / np.abs(r).max()
    assert e2 < 2e-3


def test_zero_rows_and_strided_view(gpu):
    """Zero rows get scale 1 and zero codes; rows read through a view with a wider stride (the gated columns of
    a wider buffer, h3metal/flux2.py:477) match the dense rows."""
    rng = np.random.default_rng(13)
    M, D, W = 9, 512, 4 * 512
    wide = (rng.standard_normal((M, W)) * 2).astype(np.float32)
    wide[4] = 0
    wb = to_bf16(wide)
    X = gpu.upload(wb, "bf16")
    view = X.view((M, W - 3 * D), "bf16", offset_elems=3 * D)
    out = gpu.empty((M, D), "i8")
    sa = gpu.empty((M,), "f32")
    ops.rot_q8(gpu, view, out, sa, M, D, x_stride=W)
    gpu.wait()
    wc, ws, _ = orq.rot_q8(from_bf16(wb)[:, 3 * D:4 * D], D)
    assert np.array_equal(out.numpy(), wc) and np.array_equal(sa.numpy().view(np.uint32), ws.view(np.uint32))
    assert sa.numpy()[4] == 1 and not out.numpy()[4].any()


def test_errors(gpu):
    X = gpu.empty((4, 512), "bf16")
    out = gpu.empty((4, 512), "i8")
    sa = gpu.empty((4,), "f32")
    with pytest.raises(ValueError):
        ops.rot_q8(gpu, X, out, sa, 4, 300)
    small = gpu.empty((3, 512), "i8")
    with pytest.raises(GpuError):
        ops.rot_q8(gpu, X, small, sa, 4, 512)
    with pytest.raises(GpuError):  # swiglu needs 2D columns per row
        ops.rot_q8(gpu, X, out, sa, 4, 512, swiglu=True)


def test_attention_output_chain(gpu):
    """h3metal/dit.py:204-209: the attention output O [S][H*hd] bf16 goes straight into rot_q8 with D = H*hd.
    The codes of the GPU's own O match the oracle bit for bit."""
    rng = np.random.default_rng(14)
    H, S, hd = 8, 384, 128
    q, k, v = (to_bf16(rng.standard_normal((H, S, hd)).astype(np.float32)) for _ in range(3))
    Q, K, V = (gpu.upload(t, "bf16") for t in (q, k, v))
    O = gpu.empty((S, H * hd), "bf16")
    ops.attention(gpu, Q, K, V, O, Lq=S, L=S, H=H, KVH=H, D=hd, q_rows=S, k_rows=S, scale=hd ** -0.5)
    a8 = gpu.empty((S, H * hd), "i8")
    sa = gpu.empty((S,), "f32")
    ops.rot_q8(gpu, O, a8, sa, S, H * hd)
    gpu.wait()
    o = from_bf16(O.numpy())
    wc, ws, _ = orq.rot_q8(o, H * hd)
    assert np.array_equal(a8.numpy(), wc) and np.array_equal(sa.numpy().view(np.uint32), ws.view(np.uint32))
