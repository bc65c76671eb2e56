"""The int8 projection product (ops.gemm, weight format q8; reference kernels/gemm.metal, h3metal/ops.py:124-174)
against the oracle: int32 products exact and the float32 epilogue bit for bit (f32 outputs and the residual
form), 16-bit outputs equal to the rounded oracle; the reference's own tolerance checks (tests/test_gemm.py:20-84)
on its shapes, K split over dispatches, partial tiles, and the config-4 projection shapes on sampled rows."""

import numpy as np
import pytest

from h3metal_amd import ops
from h3metal_amd.gpu import GpuError
from oracle import gemm as og
from oracle.bf16 import from_bf16, to_bf16

pytestmark = pytest.mark.gpu


def make(rng, M, N, K, m_pad=None, bias=False):
    m_pad = m_pad or M
    a = rng.integers(-127, 128, size=(m_pad, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.01, size=m_pad).astype(np.float32)
    q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    sw = rng.uniform(0.001, 0.01, size=N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    return a, sa, q, sw, b


def run(gpu, a, sa, q, sw, b, M, out_dtype="f32", tile=(64, 128, 4), no_alloc=False):
    N, K = q.shape
    print(f"[gemm] M={M} N={N} K={K} out={out_dtype} bias={b is not None}", flush=True)
    wt = ops.QWeight("q8", gpu.upload(q), gpu.upload(sw), N, K, bias=gpu.upload(b) if b is not None else None)
    m_pad = (M + tile[0] - 1) // tile[0] * tile[0]
    A = gpu.upload(np.pad(a, ((0, max(0, m_pad - a.shape[0])), (0, 0))))
    SA = gpu.upload(np.pad(sa, (0, max(0, m_pad - sa.shape[0]))))
    out = gpu.empty((m_pad, N), out_dtype)
    ops.gemm(gpu, A, wt, out, M, sa=SA, tile=tile, no_alloc=no_alloc)
    gpu.wait()
    return out.numpy()[:M]


@pytest.mark.parametrize("M,N,K,bias", [(200, 256, 512, False), (300, 640, 384, True), (64, 1024, 128, True),
                                        (1, 256, 256, False), (513, 512, 1280, False),
                                        (70, 256, 64, True), (130, 512, 192, False)])
def test_f32_outputs_bit_exact(gpu, M, N, K, bias):
    rng = np.random.default_rng(M + N + K)
    a, sa, q, sw, b = make(rng, M, N, K, bias=bias)
    got = run(gpu, a, sa, q, sw, b, M)
    want = og.epilogue(og.int_product(a[:M], q), sa[:M], sw, b)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("out_dtype", ["f16", "bf16"])
def test_16bit_outputs_are_the_rounded_oracle(gpu, out_dtype):
    rng = np.random.default_rng(41)
    M, N, K = 250, 512, 768
    a, sa, q, sw, b = make(rng, M, N, K, bias=True)
    got = run(gpu, a, sa, q, sw, b, M, out_dtype=out_dtype)
    v = og.epilogue(og.int_product(a, q), sa, sw, b)
    if out_dtype == "bf16":
        assert np.array_equal(got, to_bf16(v))
    else:
        assert np.array_equal(got.view(np.uint16), v.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("N,out_dtype", [(200, "f16"), (198, "bf16"), (198, "f32"), (260, "f32")])
def test_ragged_columns_element_path(gpu, N, out_dtype):
    """Column counts that are not a multiple of the 16-byte vector (and partial column tiles): the kernel's
    per-element output path, bit-exact."""
    rng = np.random.default_rng(N)
    M, K = 70, 192
    a, sa, q, sw, b = make(rng, M, N, K, bias=True)
    got = run(gpu, a, sa, q, sw, b, M, out_dtype=out_dtype, tile=(64, 2, 4))
    v = og.epilogue(og.int_product(a[:M], q), sa[:M], sw, b)
    if out_dtype == "f32":
        assert np.array_equal(got.view(np.uint32), v.view(np.uint32))
    elif out_dtype == "bf16":
        assert np.array_equal(got, to_bf16(v))
    else:
        assert np.array_equal(got.view(np.uint16), v.astype(np.float16).view(np.uint16))


def test_residual_ragged_columns_and_strided_output(gpu):
    """epi 1 with N = 198 into a residual buffer with a wider row stride (c_stride 203): element path; the
    columns past N are left alone."""
    rng = np.random.default_rng(5)
    M, N, K, CS = 128, 198, 256, 203
    a, sa, q, sw, b = make(rng, M, N, K, bias=True)
    x0 = rng.standard_normal((M, CS)).astype(np.float32)
    types = rng.integers(0, 2, size=M).astype(np.uint8)
    gates = rng.standard_normal((2, N)).astype(np.float32)
    wt = ops.QWeight("q8", gpu.upload(q), gpu.upload(sw), N, K, bias=gpu.upload(b))
    X = gpu.upload(x0)
    ops.gemm(gpu, gpu.upload(a), wt, X, M, sa=gpu.upload(sa), epi=1, rtype=gpu.upload(types),
             gate=gpu.upload(gates), c_stride=CS, tile=(64, 2, 4))
    gpu.wait()
    v = og.epilogue(og.int_product(a, q), sa, sw, b)
    want = x0.copy()
    want[:, :N] = og.residual(x0[:, :N], v, gates, types)
    assert np.array_equal(X.numpy().view(np.uint32), want.view(np.uint32))


def test_residual_epilogue_bit_exact_and_k_split(gpu):
    """epi 1: X += gate[rtype] * v, exact in one dispatch; with K split over 4 dispatches (the reference's ksplit),
    each slice's product is added in turn, which the oracle reproduces slice by slice."""
    rng = np.random.default_rng(42)
    M, N, K = 256, 512, 2048
    a, sa, q, sw, b = make(rng, M, N, K, bias=True)
    x0 = rng.standard_normal((M, N)).astype(np.float32)
    types = rng.integers(0, 3, size=M).astype(np.uint8)
    gates = rng.standard_normal((3, N)).astype(np.float32)
    wt = ops.QWeight("q8", gpu.upload(q), gpu.upload(sw), N, K, bias=gpu.upload(b))
    A, SA, RT, GT = gpu.upload(a), gpu.upload(sa), gpu.upload(types), gpu.upload(gates)
    for ksplit in (1, 4):
        X = gpu.upload(x0)
        ops.gemm(gpu, A, wt, X, M, sa=SA, epi=1, rtype=RT, gate=GT, ksplit=ksplit, tile=(64, 256, 8))
        gpu.wait()
        want = x0
        kp = K // ksplit
        for i in range(ksplit):
            sl = slice(i * kp, (i + 1) * kp)
            v = og.epilogue(og.int_product(a[:, sl], q[:, sl]), sa, sw, b if i == 0 else None)
            want = og.residual(want, v, gates, types)
        assert np.array_equal(X.numpy().view(np.uint32), want.view(np.uint32)), ksplit


@pytest.mark.parametrize("case", [dict(), dict(out_dtype="bf16"), dict(epi=1, K=2048, ksplit=4, tile=(64, 256, 8)),
                                  dict(N=1024, tile=(32, 512, 8)), dict(epi=1, N=1024, K=2048, ksplit=4,
                                                                          tile=(32, 512, 8))])
def test_reference_check_cases(gpu, case):
    """check() of tests/test_gemm.py:20-84 for the q8 format: max relative error against float64 below 2e-3
    (1e-2 for bf16 outputs)."""
    c = dict(M=200, N=256, K=512, epi=0, out_dtype="f16", tile=(64, 128, 4), ksplit=1)
    c.update(case)
    rng = np.random.default_rng(0)
    m_pad = (c["M"] + 127) // 128 * 128
    a = rng.integers(-127, 128, size=(m_pad, c["K"]), dtype=np.int8)
    sa = rng.uniform(0.001, 0.01, size=m_pad).astype(np.float32)
    q = rng.integers(-127, 128, size=(c["N"], c["K"]), dtype=np.int8)
    sw = rng.uniform(0.001, 0.01, size=c["N"]).astype(np.float32)
    wt = ops.QWeight("q8", gpu.upload(q), gpu.upload(sw), c["N"], c["K"])
    ref = (a.astype(np.float64) @ q.T.astype(np.float64)) * sa[:, None] * sw[None, :]
    A, SA = gpu.upload(a), gpu.upload(sa)
    if c["epi"] == 0:
        out = gpu.empty((m_pad, c["N"]), c["out_dtype"])
        ops.gemm(gpu, A, wt, out, c["M"], sa=SA, tile=c["tile"])
        gpu.wait()
        got = out.numpy()[:c["M"]]
        got = from_bf16(got).astype(np.float64) if c["out_dtype"] == "bf16" else got.astype(np.float64)
    else:
        x0 = rng.standard_normal((m_pad, c["N"])).astype(np.float32)
        X = gpu.upload(x0)
        types = rng.integers(0, 3, size=m_pad).astype(np.uint8)
        gates = rng.standard_normal((3, c["N"])).astype(np.float32)
        ops.gemm(gpu, A, wt, X, c["M"], sa=SA, epi=1, rtype=gpu.upload(types), gate=gpu.upload(gates),
                 tile=c["tile"], ksplit=c["ksplit"])
        gpu.wait()
        got = X.numpy()[:c["M"]].astype(np.float64)
        ref = x0.astype(np.float64) + gates[types] * ref
    ref = ref[:c["M"]]
    err = np.abs(got - ref).max() / (np.abs(ref).max() + 1e-12)
    assert err < (2e-3 if c["out_dtype"] != "bf16" else 1e-2), err


def test_config4_projection_shapes_sampled(gpu):
    """The qkv projection of a config-4 block (M = 16896 rows, K = 4096, N = 3 * 4096, bf16 out) on the full
    shape; 96 sampled rows against the oracle, bit for bit."""
    rng = np.random.default_rng(43)
    M, N, K = 16896, 12288, 4096
    a = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.01, size=M).astype(np.float32)
    q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    sw = rng.uniform(0.001, 0.01, size=N).astype(np.float32)
    got = run(gpu, a, sa, q, sw, None, M, out_dtype="bf16", tile=(128, 256, 8))
    rows = np.sort(rng.choice(M, 96, replace=False))
    v = og.epilogue(og.int_product(a[rows], q), sa[rows], sw)
    assert np.array_equal(got[rows], to_bf16(v))


@pytest.mark.parametrize("mode", ["f32", "bf16", "epi1"])
@pytest.mark.parametrize("no_alloc", [False, True])
def test_last_round_rows_on_small_tiles(gpu, mode, no_alloc):
    """260 tiles of 256 x 256 on 256 CUs: the last row of tiles (rows 16384..16447) runs as a second launch of
    128 x 128 tiles on the sub-problem of those rows; every row bit for bit (f32, the residual form) or equal to
    the rounded oracle (bf16), the rows of both launches alike; through h3_dispatch and through the
    allocation-free entry point h3_dispatch_static."""
    rng = np.random.default_rng(46)
    M, N, K = 16448, 1024, 128
    a, sa, q, sw, b = make(rng, M, N, K, bias=True)
    v = og.epilogue(og.int_product(a, q), sa, sw, b)
    if mode == "epi1":
        x0 = rng.standard_normal((M, N)).astype(np.float32)
        types = rng.integers(0, 3, size=M).astype(np.uint8)
        gates = rng.standard_normal((3, N)).astype(np.float32)
        wt = ops.QWeight("q8", gpu.upload(q), gpu.upload(sw), N, K, bias=gpu.upload(b))
        X = gpu.upload(x0)
        print(f"[gemm] tail rows M={M} N={N} K={K} epi=1 no_alloc={no_alloc}", flush=True)
        ops.gemm(gpu, gpu.upload(a), wt, X, M, sa=gpu.upload(sa), epi=1, rtype=gpu.upload(types),
                 gate=gpu.upload(gates), tile=(64, 256, 8), no_alloc=no_alloc)
        gpu.wait()
        want = og.residual(x0, v, gates, types)
        assert np.array_equal(X.numpy().view(np.uint32), want.view(np.uint32))
        return
    got = run(gpu, a, sa, q, sw, b, M, out_dtype=mode, no_alloc=no_alloc)
    if mode == "f32":
        assert np.array_equal(got.view(np.uint32), v.view(np.uint32))
    else:
        assert np.array_equal(got, to_bf16(v))


def test_config4_output_projection_sampled(gpu):
    """The output projection of a config-4 block (M = 16896, N = K = 4096) into the float residual: 1056 tiles,
    of which the last two rows of tiles run on 128 x 128 tiles; 48 sampled rows of each part bit for bit."""
    rng = np.random.default_rng(47)
    M, N, K = 16896, 4096, 4096
    a = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    sa = rng.uniform(0.001, 0.01, size=M).astype(np.float32)
    q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    sw = rng.uniform(0.001, 0.01, size=N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    x0 = rng.standard_normal((M, N)).astype(np.float32)
    types = rng.integers(0, 3, size=M).astype(np.uint8)
    gates = rng.standard_normal((3, N)).astype(np.float32)
    wt = ops.QWeight("q8", gpu.upload(q), gpu.upload(sw), N, K, bias=gpu.upload(b))
    X = gpu.upload(x0)
    print(f"[gemm] output projection M={M} N={N} K={K} epi=1", flush=True)
    ops.gemm(gpu, gpu.upload(a), wt, X, M, sa=gpu.upload(sa), epi=1, rtype=gpu.upload(types),
             gate=gpu.upload(gates), tile=(64, 256, 8))
    gpu.wait()
    rows = np.sort(np.concatenate([rng.choice(16384, 48, replace=False), 16384 + rng.choice(512, 48, replace=False)]))
    v = og.epilogue(og.int_product(a[rows], q), sa[rows], sw, b)
    want = og.residual(x0[rows], v, gates, types[rows])
    assert np.array_equal(X.numpy()[rows].view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("seed", range(16))
def test_random_shape_sweep_bit_exact(gpu, seed):
    """A seeded sweep of shapes (M up to 9000 rows, so that some grids pass 256 tiles and take the small-tile
    tail launch; ragged N; K a multiple of 64), both epilogues, three output types, with and without bias:
    f32 and the residual form bit for bit, 16-bit outputs equal to the rounded oracle."""
    rng = np.random.default_rng(2000 + seed)
    M = int(rng.integers(1, 9001))
    N = int(rng.choice([int(rng.integers(1, 700)), 256 * int(rng.integers(1, 17))]))
    K = 64 * int(rng.integers(1, 9))
    bias = bool(seed % 2)
    mode = ["f32", "bf16", "f16", "epi1"][seed % 4]
    print(f"[gemm sweep] seed={seed} M={M} N={N} K={K} bias={bias} mode={mode}", flush=True)
    m_pad = (M + 63) // 64 * 64
    tn = next(t for t in (256, 128, 64, 32, 16, 8, 4, 2, 1) if N % t == 0)  # the launcher's tile check
    a, sa, q, sw, b = make(rng, M, N, K, m_pad=m_pad, bias=bias)
    v = og.epilogue(og.int_product(a[:M], q), sa[:M], sw, b)
    if mode == "epi1":
        x0 = rng.standard_normal((m_pad, N)).astype(np.float32)
        types = rng.integers(0, 3, size=m_pad).astype(np.uint8)
        gates = rng.standard_normal((3, N)).astype(np.float32)
        wt = ops.QWeight("q8", gpu.upload(q), gpu.upload(sw), N, K, bias=gpu.upload(b) if bias else None)
        X = gpu.upload(x0)
        ops.gemm(gpu, gpu.upload(a), wt, X, M, sa=gpu.upload(sa), epi=1, rtype=gpu.upload(types),
                 gate=gpu.upload(gates), tile=(64, tn, 8))
        gpu.wait()
        want = og.residual(x0[:M], v, gates, types[:M])
        assert np.array_equal(X.numpy()[:M].view(np.uint32), want.view(np.uint32))
        return
    got = run(gpu, a, sa, q, sw, b, M, out_dtype=mode, tile=(64, tn, 4))
    if mode == "f32":
        assert np.array_equal(got.view(np.uint32), v.view(np.uint32))
    elif mode == "bf16":
        assert np.array_equal(got, to_bf16(v))
    else:
        assert np.array_equal(got.view(np.uint16), v.astype(np.float16).view(np.uint16))


def test_refusals(gpu):
    rng = np.random.default_rng(44)
    a, sa, q, sw, _ = make(rng, 64, 256, 256)
    wt = ops.QWeight("q8", gpu.upload(q), gpu.upload(sw), 256, 256)
    A, SA, out = gpu.upload(a), gpu.upload(sa), gpu.empty((64, 256), "f16")
    with pytest.raises(ValueError):  # the reference refuses tile widths that do not divide N
        ops.gemm(gpu, A, wt, out, 64, sa=SA, tile=(32, 512, 8))
    with pytest.raises(NotImplementedError):
        ops.gemm(gpu, A, ops.QWeight("q4", wt.w, wt.sw, 256, 256), out, 64, sa=SA)
    with pytest.raises(GpuError):  # K must be a multiple of 64
        ops.gemm(gpu, A, ops.QWeight("q8", wt.w, wt.sw, 256, 200, ws=256), out, 64, sa=SA, a_stride=256)
    with pytest.raises(GpuError):  # the output does not hold M padded rows
        ops.gemm(gpu, A, wt, gpu.empty((32, 256), "f16"), 64, sa=SA)

def float_case(gpu, fmt, rng, M, N, K, bias):
    """Device operands of an h8 / f16 / bf16 product and its float64 value (before bias and epilogue)."""
    af = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    if fmt == "bf16":
        ab = to_bf16(af)
        a_dev, a_val = gpu.upload(ab, "bf16"), from_bf16(ab)
    else:
        ah = af.astype(np.float16)
        a_dev, a_val = gpu.upload(ah), ah.astype(np.float32)
    if fmt == "h8":
        q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
        sw = rng.uniform(0.001, 0.01, size=N).astype(np.float32)
        wt = ops.QWeight("h8", gpu.upload(q), gpu.upload(sw), N, K, bias=gpu.upload(b) if bias else None)
        v = og.float_product(a_val, q) * sw[None, :].astype(np.float64)
    else:
        wf = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
        if fmt == "bf16":
            wb = to_bf16(wf)
            w_dev, w_val = gpu.upload(wb, "bf16"), from_bf16(wb)
        else:
            wh = wf.astype(np.float16)
            w_dev, w_val = gpu.upload(wh), wh.astype(np.float32)
        wt = ops.QWeight(fmt, w_dev, None, N, K, bias=gpu.upload(b) if bias else None)
        v = og.float_product(a_val, w_val)
    if bias:
        v = v + b[None, :].astype(np.float64)
    return a_dev, wt, v


@pytest.mark.parametrize("fmt", ["h8", "f16", "bf16"])
@pytest.mark.parametrize("M,N,K,out_dtype,bias", [(200, 256, 512, "f16", False), (300, 640, 384, "f32", True),
                                                  (70, 198, 96, "bf16", True), (513, 512, 1280, "f32", False)])
def test_float_formats_reference_tolerance(gpu, fmt, M, N, K, out_dtype, bias):
    """h8 / f16 / bf16 products (WFMT 6 / 4 / 5) within the reference's check() tolerance (tests/test_gemm.py:
    20-84): max error below 2e-3 of the largest output, 1e-2 for bfloat outputs; ragged N and a K of three
    32-element steps included."""
    rng = np.random.default_rng(M + N + K + len(fmt))
    print(f"[gemm {fmt}] M={M} N={N} K={K} out={out_dtype} bias={bias}", flush=True)
    A, wt, v = float_case(gpu, fmt, rng, M, N, K, bias)
    out = gpu.empty((M, N), out_dtype)
    ops.gemm(gpu, A, wt, out, M, tile=(1, 2, 4))
    gpu.wait()
    got = out.numpy()
    got = from_bf16(got).astype(np.float64) if out_dtype == "bf16" else got.astype(np.float64)
    err = np.abs(got - v).max() / np.abs(v).max()
    assert err < (2e-3 if out_dtype != "bf16" else 1e-2), err


@pytest.mark.parametrize("fmt", ["h8", "f16", "bf16"])
def test_float_formats_residual_and_k_split(gpu, fmt):
    """epi 1 with row types and gates; h8 also with K split over dispatches (the reference allows it for h8)."""
    rng = np.random.default_rng(7)
    M, N, K = 256, 512, 1024
    A, wt, v = float_case(gpu, fmt, rng, M, N, K, True)
    x0 = rng.standard_normal((M, N)).astype(np.float32)
    types = rng.integers(0, 3, size=M).astype(np.uint8)
    gates = rng.standard_normal((3, N)).astype(np.float32)
    want = x0.astype(np.float64) + gates[types].astype(np.float64) * v
    for ksplit in ((1, 4) if fmt == "h8" else (1,)):
        X = gpu.upload(x0)
        ops.gemm(gpu, A, wt, X, M, epi=1, rtype=gpu.upload(types), gate=gpu.upload(gates), ksplit=ksplit,
                 tile=(64, 256, 8))
        gpu.wait()
        err = np.abs(X.numpy().astype(np.float64) - want).max() / np.abs(want).max()
        assert err < 2e-3, (fmt, ksplit, err)


def test_rotated_half_output_into_h8_projection(gpu):
    """The text encoder's chain (h3metal/te.py:195-196): rot_q8 with out_hr (rotated rows in half precision)
    feeding an h8 projection; against float64 of the rotated rows."""
    from oracle import rot_q8 as orq
    rng = np.random.default_rng(8)
    M, D, N = 96, 1024, 512
    xb = to_bf16((rng.standard_normal((M, D)) * 2).astype(np.float32))
    X = gpu.upload(xb, "bf16")
    hr = gpu.empty((M, D), "f16")
    ops.rot_q8(gpu, X, hr, None, M, D, out_hr=True)
    q = rng.integers(-127, 128, size=(N, D), dtype=np.int8)
    sw = rng.uniform(0.001, 0.01, size=N).astype(np.float32)
    wt = ops.QWeight("h8", gpu.upload(q), gpu.upload(sw), N, D)
    out = gpu.empty((M, N), "f32")
    ops.gemm(gpu, hr, wt, out, M, tile=(1, 2, 4))
    gpu.wait()
    _, _, r = orq.rot_q8(from_bf16(xb), D)
    want = og.float_product(r.astype(np.float16).astype(np.float32), q) * sw[None, :].astype(np.float64)
    err = np.abs(out.numpy() - want).max() / np.abs(want).max()
    assert err < 2e-3, err


def test_float_format_refusals(gpu):
    rng = np.random.default_rng(9)
    A, wt, _ = float_case(gpu, "f16", rng, 64, 256, 256, False)
    out = gpu.empty((64, 256), "f16")
    with pytest.raises(ValueError):  # f16 weights take half activations
        ops.gemm(gpu, gpu.upload(np.zeros((64, 256), np.int8)), wt, out, 64, tile=(1, 2, 4))
    with pytest.raises(ValueError):  # the reference splits K only for integer-weight formats
        ops.gemm(gpu, A, wt, gpu.empty((64, 256), "f32"), 64, epi=1, rtype=gpu.upload(np.zeros(64, np.uint8)),
                 gate=gpu.upload(np.ones((1, 256), np.float32)), ksplit=2, tile=(1, 2, 4))
    with pytest.raises(GpuError):  # K must be a multiple of 32 for 16-bit operands
        ops.gemm(gpu, A, ops.QWeight("f16", wt.w, None, 256, 200, ws=256), out, 64, a_stride=256, tile=(1, 2, 4))
