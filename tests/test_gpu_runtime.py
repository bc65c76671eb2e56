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
    assert k.max_threads == 256  # the wave-pipelined kernel's workgroup
    assert gpu.kernel("attention", "attention", HD=128, O_T="bfloat").max_threads == 256
    assert gpu.kernel("attention", "attention", HD=128, QK8=1, O_T="bfloat", GROUPS=1).max_threads == 256
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


def test_profile_names_with_static_launches_and_copies(gpu):
    """In profile mode every timed operation (h3_dispatch launches, device copies) gets its name back in order;
    launches through the allocation-free entry point are not timed and take no name."""
    H, S, D = 2, 512, 128
    rng = np.random.default_rng(1)
    Q = gpu.upload(rng.standard_normal((H, S, D)).astype(np.float16))
    O = gpu.empty((S, H * D), "f16")
    C = gpu.empty((S, H * D), "f16")
    k = gpu.kernel("attention", "attention", HD=D)
    params = pack("7if3i", S, S, H, H, S, S, H * D, D ** -0.5 * ops.LOG2E, 0, H, 0)
    gpu.wait()
    gpu.profile(True)
    gpu.launch(k, None, None, [Q, Q, Q, O], params)
    gpu.launch(k, None, None, [Q, Q, Q, O], params, no_alloc=True)
    O.copy_to(C)
    gpu.launch(k, None, None, [Q, Q, Q, O], params, no_alloc=True)
    gpu.launch(k, None, None, [Q, Q, Q, O], params)
    gpu.wait()
    prof = gpu.profile_take()
    gpu.profile(False)
    assert [n for n, _ in prof] == [k.name, "h3_buffer_copy", k.name]
    assert all(t > 0 for _, t in prof)
    assert gpu.names == []
    assert np.array_equal(C.numpy(), O.numpy())


def test_device_copy(gpu):
    """h3_buffer_copy moves bytes between (views of) device buffers in order with the stream; bad ranges are
    refused."""
    from h3metal_amd.gpu import GpuError
    rng = np.random.default_rng(2)
    a = rng.integers(0, 255, 10000).astype(np.uint8)
    A = gpu.upload(a, "u8")
    B = gpu.empty((12000,), "u8")
    A.view((5000,), offset_elems=1000).copy_to(B.view((5000,), offset_elems=7000))
    got = B.numpy()
    assert np.array_equal(got[7000:12000], a[1000:6000]) and not got[:7000].any()
    with pytest.raises(GpuError, match="outside"):
        A.copy_to(B.view((4000,), offset_elems=8000))


@pytest.mark.parametrize("nbytes,src_off,dst_off", [(150_000_013, 0, 16), (1 << 20, 16, 32), (4099, 3, 0),
                                                    (15, 0, 0)])
def test_device_copy_sizes(gpu, nbytes, src_off, dst_off):
    """h3_buffer_copy at large, aligned, misaligned and tiny sizes: the destination range equals the source and
    the bytes around it stay untouched."""
    rng = np.random.default_rng(nbytes)
    a = rng.integers(0, 256, nbytes + src_off, dtype=np.uint8)
    A = gpu.upload(a, "u8")
    B = gpu.upload(np.full(nbytes + dst_off + 64, 0xA5, np.uint8), "u8")
    print(f"[copy] bytes={nbytes} src_off={src_off} dst_off={dst_off}", flush=True)
    A.view((nbytes,), offset_elems=src_off).copy_to(B.view((nbytes,), offset_elems=dst_off))
    got = B.numpy()
    assert np.array_equal(got[dst_off:dst_off + nbytes], a[src_off:])
    assert (got[:dst_off] == 0xA5).all() and (got[dst_off + nbytes:] == 0xA5).all()


def test_misaligned_views_refused(gpu):
    """Q/K/V rows are read 16 bytes at a time and O written 4 elements at a time: a view whose base breaks
    that is refused on the host, not run."""
    H, S, D = 2, 64, 128
    Q = gpu.empty((H * S * D + 8,), "f16")
    O = gpu.empty((S, H * D + 4), "f16")
    good = Q.view((H, S, D))
    bad = Q.view((H, S, D), offset_elems=4)  # 8 bytes in
    with pytest.raises(GpuError, match="16-byte aligned"):
        ops.attention(gpu, bad, good, good, O.view((S, H * D)), Lq=S, L=S, H=H, KVH=H, D=D, q_rows=S, k_rows=S,
                      scale=0.1)
    with pytest.raises(GpuError, match="aligned to 4 elements"):
        ops.attention(gpu, good, good, good, O.view((S, H * D), offset_elems=1), Lq=S, L=S, H=H, KVH=H, D=D,
                      q_rows=S, k_rows=S, scale=0.1)
    ops.attention(gpu, good, good, good, O.view((S, H * D)), Lq=S, L=S, H=H, KVH=H, D=D, q_rows=S, k_rows=S,
                  scale=0.1)
    gpu.wait()


def _int8_attention(gpu, H, S, out=None):
    """int8 attention over zero-filled inputs (unit scales): every score 0, so the output is the mean of V."""
    D = 128
    Q = gpu.empty((H, S, D), "i8")
    V = gpu.empty((H, S, D), "bf16")
    sc = gpu.upload(np.ones((H, S), np.float32))
    O = out if out is not None else gpu.empty((S, H * D), "bf16")
    return lambda: ops.attention(gpu, Q, Q, V, O, Lq=S, L=S, H=H, KVH=H, D=D, q_rows=S, k_rows=S,
                                 scale=D ** -0.5, q_scale=sc, k_scale=sc)


def test_dispatch_neither_allocates_nor_waits(gpu):
    """The scratch memory of the attention tail split is reserved when the context opens: a dispatch at a new
    shape that splits its last round of tiles neither grows it nor waits for the queued work."""
    import time
    heavy = _int8_attention(gpu, 32, 16896)
    warm = _int8_attention(gpu, 2, 4096)  # 22 tiles of 384 rows: a split last round
    fresh = _int8_attention(gpu, 3, 4096)  # 33 tiles: a split of another size
    heavy()
    warm()
    gpu.wait()
    ws0 = gpu.workspace_bytes
    assert ws0 > 0
    t0 = time.perf_counter()
    for _ in range(3):
        heavy()
    queued = time.perf_counter()
    fresh()
    dt = time.perf_counter() - queued
    gpu_s = gpu.wait()
    assert gpu.workspace_bytes == ws0
    assert gpu_s > 5e-3, gpu_s  # three config-4-sized calls were still running during the dispatch
    assert dt < 0.25 * gpu_s, (dt, gpu_s, queued - t0)


def test_h8_gemm_reserves_its_scratch_outside_the_dispatch(gpu):
    """The h8 GEMM's widened weights need N * K * 2 bytes of scratch: the launcher grows the reservation by an
    explicit call, and a dispatch that finds too little fails with the size it needs."""
    N, K, M = 4096, 16384, 256
    w = gpu.empty((N, K), "i8")
    sw = gpu.upload(np.ones(N, np.float32))
    a = gpu.empty((M, K), "f16")
    out = gpu.empty((M, N), "f16")
    need = N * K * 2
    if gpu.workspace_bytes < need:
        k = gpu.kernel("gemm", "gemm", WFMT=6, EPI=0, OUT_T="half", TM=64, TN=128, NSG=4, G=128, HAS_BIAS=0, SWZ=1)
        with pytest.raises(GpuError, match="bytes of scratch"):
            gpu.launch(k, None, None, [a, w, sw, None, out, None, None, None],
                       pack("8i", M, N, K, K, N, K, K // 128, N), params_index=8)
    ops.gemm(gpu, a, ops.QWeight("h8", w, sw, N, K), out, M)
    gpu.wait()
    assert gpu.workspace_bytes >= need
    assert (out.numpy() == 0).all()
