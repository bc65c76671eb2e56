"""The HIP runtime behind gpu.py (csrc/capi.hip): buffers, the launch table, dispatch validation, timing.
Mirrors the reference runtime's behaviour (src/capi.mm): zero-filled buffers, NULL pipeline + message for an
unknown kernel, dispatch errors as GpuError, wait returning GPU seconds."""

import numpy as np
import pytest

from h3metal_amd import ops
from h3metal_amd.gpu import GpuError, pack

pytestmark = pytest.mark.gpu


def test_device_is_gfx950(gpu):
    assert "gfx950" in gpu.device
    assert gpu.max_buffer > 200 * 2 ** 30  # 288 GB HBM3E class device


def test_buffers_zero_filled_and_roundtrip(gpu):
    t = gpu.empty((1000, 3), "f32")
    assert (t.numpy() == 0).all()
    a = np.arange(3000, dtype=np.float32).reshape(1000, 3)
    t.write(a)
    assert np.array_equal(t.numpy(), a)
    v = t.view((10, 3), offset_elems=30)
    assert np.array_equal(v.numpy(), a[10:20])
    with pytest.raises(GpuError):
        v.write(np.zeros((2000,), np.float32))


def test_unknown_kernel_and_macros(gpu):
    with pytest.raises(GpuError, match="unknown kernel module"):
        gpu.kernel("nope", "gemm")
    with pytest.raises(GpuError, match="unknown function"):
        gpu.kernel("attention", "nope")
    with pytest.raises(GpuError, match="HD 80"):
        gpu.kernel("attention", "attention", HD=80)
    with pytest.raises(GpuError, match="unknown macro"):
        gpu.kernel("attention", "attention", FOO=1)
    with pytest.raises(GpuError, match="QKROT needs QK8"):
        gpu.kernel("ops", "qk_norm_rope", QKROT=1)
    # the reference's file names and tuning macros are accepted
    k = gpu.kernel("attention.metal", "attention", HD=128, WM=10, BK=32, DB=1, PVORDER=1, VX=1, QK8=1, O_T="bfloat")
    assert k.max_threads == 768  # the three-group kernel's workgroup
    assert gpu.kernel("attention", "attention", HD=128, QK8=1, O_T="bfloat", GROUPS=2).max_threads == 512
    assert gpu.kernel("attention", "attention", HD=128, QK8=1, O_T="bfloat", CAUSAL=1).max_threads == 512


def test_dispatch_validation(gpu):
    H, S, D = 2, 64, 128
    Q = gpu.empty((H, S, D), "f16")
    small = gpu.empty((H, S // 2, D), "f16")
    O = gpu.empty((S, H * D), "f16")
    with pytest.raises(GpuError, match="k needs"):
        ops.attention(gpu, Q, small, Q, O, Lq=S, L=S, H=H, KVH=H, D=D, q_rows=S, k_rows=S, scale=0.1)
    with pytest.raises(GpuError, match="bad shape"):
        ops.attention(gpu, Q, Q, Q, O, Lq=S, L=S + 1, H=H, KVH=H, D=D, q_rows=S, k_rows=S, scale=0.1)
    with pytest.raises(GpuError, match="out needs"):
        ops.attention(gpu, Q, Q, Q, gpu.empty((S - 1, H * D), "f16"), Lq=S, L=S, H=H, KVH=H, D=D, q_rows=S,
                      k_rows=S, scale=0.1)
    k = gpu.kernel("attention", "attention", HD=128)
    with pytest.raises(GpuError, match="parameter block"):
        gpu.launch(k, None, None, [Q, Q, Q, O], pack("3i", 1, 2, 3))
    with pytest.raises(GpuError, match="not bound"):
        gpu.launch(k, None, None, [Q, None, Q, O], pack("7if3i", S, S, H, H, S, S, H * D, 0.1, 0, H, 0))
    gpu.wait()


def test_wait_time_and_profile(gpu):
    H, S, D = 4, 1024, 128
    rng = np.random.default_rng(0)
    Q = gpu.upload(rng.standard_normal((H, S, D)).astype(np.float16))
    O = gpu.empty((S, H * D), "f16")
    gpu.wait()
    gpu.profile(True)
    for _ in range(3):
        ops.attention(gpu, Q, Q, Q, O, Lq=S, L=S, H=H, KVH=H, D=D, q_rows=S, k_rows=S, scale=D ** -0.5)
    dt = gpu.wait()
    prof = gpu.profile_take()
    gpu.profile(False)
    assert dt > 0 and len(prof) == 3
    assert all(t > 0 for _, t in prof) and sum(t for _, t in prof) <= dt * 1.01
    assert prof[0][0].startswith("attention:attention(")
