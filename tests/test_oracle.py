"""Pins the CPU oracle without retyping its formulas (CPU only).

The reference ships no golden vectors and its kernels (Metal) cannot run here,
so every oracle function is checked against what the mathematics fixes:
closed forms, invariants, special cases and brute force on small inputs, each
chosen so that a plausible slip (a dropped sign, a wrong stage order or
index, a transposed operand) fails.
"""

import os

import numpy as np
import pytest

from oracle import attention as oa
from oracle import prepass as op
from oracle.bf16 import from_bf16, to_bf16

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def sylvester(n):
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


# -- rotation ------------------------------------------------------------------------------------------------------

def test_fwht_matches_sylvester_matrix():
    """The butterfly network equals the Sylvester Hadamard matrix product (H symmetric, so row/column order and
    the (a+b, a-b) orientation are both fixed by this)."""
    rng = np.random.default_rng(0)
    for n in (4, 64, 128):
        x = rng.standard_normal((7, n)).astype(np.float32)
        got = op.fwht_f32(x).astype(np.float64)
        want = x.astype(np.float64) @ sylvester(n).T
        np.testing.assert_allclose(got, want, rtol=0, atol=1e-4 * np.abs(want).max())


def test_fwht_one_hot_gives_hadamard_rows():
    n = 128
    eye = np.eye(n, dtype=np.float32)
    assert np.array_equal(op.fwht_f32(eye), sylvester(n).astype(np.float32))


def test_fwht_integer_inputs_exact():
    """Small integers: every butterfly sum is exact in float32, so the result equals the integer matrix product
    bit for bit."""
    rng = np.random.default_rng(1)
    x = rng.integers(-1000, 1000, (50, 128))
    want = x @ sylvester(128).astype(np.int64).T
    assert np.array_equal(op.fwht_f32(x.astype(np.float32)), want.astype(np.float32))


def test_hash_signs_closed_form():
    """popcount((c * 0x2545F491) mod 2^32) parity, evaluated with Python integers, for a few channels by hand."""
    s = op.hash_signs(128)
    for c in (0, 1, 2, 3, 5, 64, 127):
        par = bin((c * 0x2545F491) & 0xFFFFFFFF).count("1") & 1
        assert s[c] == (-1 if par else 1)
    assert s[0] == 1  # c = 0: popcount 0
    assert bin(0x2545F491).count("1") % 2 == 0 and s[1] == 1  # the multiplier itself has 14 set bits
    assert 0 < (s < 0).sum() < 128


def test_rotation_orthonormal_and_preserves_dot():
    """R = diag(signs) H / sqrt(n) is orthonormal: R R^T = I, and (R q).(R k) = q.k (the reason the rotation
    leaves attention unchanged, ops.metal:420-423)."""
    n = 128
    R = op.rotate_f32(np.eye(n, dtype=np.float32)).astype(np.float64)  # rows = images of unit vectors
    np.testing.assert_allclose(R @ R.T, np.eye(n), atol=1e-6)
    rng = np.random.default_rng(2)
    q, k = rng.standard_normal((2, 20, n)).astype(np.float32)
    dq = (op.rotate_f32(q).astype(np.float64) * op.rotate_f32(k)).sum(-1)
    np.testing.assert_allclose(dq, (q.astype(np.float64) * k).sum(-1), rtol=1e-5, atol=1e-4)


def test_rotation_sign_order_pinned_by_one_hot_rows():
    """The signs act on the INPUT channels, before the butterflies (kernels/ops.metal:424-428 flips channel c,
    then :430-446 transform): the image of the unit vector e_c is s_c * H[c, :] / sqrt(n), with H the Sylvester
    Hadamard matrix H[c, j] = (-1)^popcount(c & j) and s_c = -1 where popcount(c * 0x2545F491 mod 2^32) is odd,
    both evaluated here with Python integers. The other order (signs on the outputs, H diag(s)) gives
    s_j * H[c, j] instead and must fail this check."""
    n = 128
    inv = 1.0 / np.sqrt(np.float64(n))
    sign = [(-1.0 if bin((c * 0x2545F491) & 0xFFFFFFFF).count("1") & 1 else 1.0) for c in range(n)]
    H = np.array([[(-1.0) ** bin(c & j).count("1") for j in range(n)] for c in range(n)])
    want = np.array([sign[c] * H[c] for c in range(n)]) * inv
    swapped = H * np.array(sign)[None, :] * inv
    got = op.rotate_f32(np.eye(n, dtype=np.float32)).astype(np.float64)
    np.testing.assert_array_equal(got, want.astype(np.float32).astype(np.float64))
    assert not np.allclose(got, swapped)  # the plausible slip is distinguishable


def test_rotation_spreads_outlier_channel():
    """A one-hot row becomes +-1/sqrt(n) in every channel: amax drops by sqrt(n)."""
    x = np.zeros((1, 128), np.float32)
    x[0, 37] = 20.0
    r = op.rotate_f32(x)
    np.testing.assert_allclose(np.abs(r), 20.0 / np.sqrt(128), rtol=1e-6)


def test_inv_sqrt_constant_correctly_rounded():
    c = op.inv_sqrt_f32(128)
    exact = 1 / np.sqrt(np.longdouble(128))
    up, down = np.nextafter(c, np.float32(1)), np.nextafter(c, np.float32(0))
    assert abs(np.longdouble(c) - exact) <= abs(np.longdouble(up) - exact)
    assert abs(np.longdouble(c) - exact) <= abs(np.longdouble(down) - exact)


# -- int8 ----------------------------------------------------------------------------------------------------------

def test_quant_special_cases():
    codes, sc = op.quant_i8(np.zeros((2, 128), np.float32))
    assert (codes == 0).all() and (sc == 1).all()  # amax == 0 -> scale 1
    x = np.array([[127.0, -63.5, 0.5, 1.5, 2.5, -2.5] + [0] * 122], np.float32)
    codes, sc = op.quant_i8(x)
    assert sc[0] == np.float32(1)
    assert list(codes[0, :6]) == [127, -64, 0, 2, 2, -2]  # rint is half to even


def test_quant_roundtrip_bounds():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((100, 128)) * rng.uniform(0.01, 100, (100, 1))).astype(np.float32)
    codes, sc = op.quant_i8(x)
    assert np.abs(codes).max() == 127 and (np.abs(codes).max(1) == 127).all()
    err = np.abs(codes * sc[:, None].astype(np.float64) - x)
    assert (err <= sc[:, None] * 0.5 * (1 + 1e-5)).all()


# -- norm / rope ---------------------------------------------------------------------------------------------------

def test_rms_norm_against_float64():
    rng = np.random.default_rng(4)
    v = (rng.standard_normal((30, 128)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    got = op.rms_norm_f32(v, w, 1e-6).astype(np.float64)
    vd = v.astype(np.float64)
    want = vd / np.sqrt((vd ** 2).mean(-1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-6)
    # unit weight and a row of equal entries c: the result is sign(c) * 1 / sqrt(1 + eps / c^2)
    one = op.rms_norm_f32(np.full((1, 128), 2.0, np.float32), np.ones(128, np.float32), 0.0)
    assert (one == 1.0).all()


def test_rope_rotation_of_pairs():
    """Each pair (i, i + rot/2) is rotated by its angle: norms are kept, angle 0 is identity, and angle pi/2 maps
    (a, b) to (-b, a)."""
    rng = np.random.default_rng(5)
    v = rng.standard_normal((3, 128)).astype(np.float32)
    rot, h = 96, 48
    ang = rng.uniform(0, 6.28, (3, h))
    got = op.rope_f32(v, np.cos(ang), np.sin(ang), rot).astype(np.float64)
    np.testing.assert_allclose(got[:, :h] ** 2 + got[:, h:rot] ** 2,
                               v[:, :h].astype(np.float64) ** 2 + v[:, h:rot] ** 2, rtol=1e-5)
    assert np.array_equal(got[:, rot:], v[:, rot:])
    quarter = op.rope_f32(v, np.zeros((3, h)), np.ones((3, h)), rot)
    assert np.array_equal(quarter[:, :h], -v[:, h:rot]) and np.array_equal(quarter[:, h:rot], v[:, :h])
    assert np.array_equal(op.rope_f32(v, np.ones((3, h)), np.zeros((3, h)), rot), v)


def test_qk_norm_rope_layout_and_sequences():
    """Head-major output placement with batched sequences (seq_len): row m goes to sequence m // seq_len, row
    m % seq_len; V is copied through."""
    rng = np.random.default_rng(6)
    M, Hq, Hk, Hv, hd, seq_len = 10, 2, 1, 1, 64, 4
    x = rng.standard_normal((M, (Hq + Hk + Hv) * hd)).astype(np.float32)
    out = op.qk_norm_rope(x, Hq=Hq, Hk=Hk, Hv=Hv, hd=hd, out_rows=5, rot=0, eps=1e-6, norm=False,
                          seq_len=seq_len)
    nseq = 3
    assert out["Q"].shape == (nseq * Hq, 5, hd) and out["V"].shape == (nseq * Hv, 5, hd)
    for m in range(M):
        sq, r = divmod(m, seq_len)
        assert np.array_equal(out["Q"][sq * Hq + 1, r], x[m, hd:2 * hd])
        assert np.array_equal(out["K"][sq * Hk, r], x[m, 2 * hd:3 * hd])
        assert np.array_equal(out["V"][sq * Hv, r], x[m, 3 * hd:])
    assert (out["Q"][2 * Hq:, 2:] == 0).all()  # rows beyond the last (short) sequence stay empty


# -- attention -----------------------------------------------------------------------------------------------------

def test_int_scores_brute_force():
    rng = np.random.default_rng(7)
    qi = rng.integers(-127, 128, (2, 5, 32)).astype(np.int8)
    ki = rng.integers(-127, 128, (1, 6, 32)).astype(np.int8)
    s = oa.int_scores(qi, ki, H_per_kv=2)
    for h in range(2):
        for i in range(5):
            for j in range(6):
                assert s[h, i, j] == sum(int(a) * int(b) for a, b in zip(qi[h, i], ki[0, j]))
    worst = oa.int_scores(np.full((1, 1, 128), -127, np.int8), np.full((1, 1, 128), -127, np.int8))
    assert worst[0, 0, 0] == 128 * 127 * 127 < 2 ** 31


def test_ref_attention_brute_force_loops():
    rng = np.random.default_rng(8)
    H, KVH, Lq, L, D = 4, 2, 5, 7, 8
    q, k, v = rng.standard_normal((H, Lq, D)), rng.standard_normal((KVH, L + 2, D)), rng.standard_normal((KVH, L + 2, D))
    out = oa.ref_attention(q, k, v, 0.3, L=L, causal=True, off=1, seq_heads=2, seq_rows=6)
    assert out.shape == (6 + Lq, 2 * D)
    for h in range(H):
        kh = h // 2
        for i in range(Lq):
            js = [j for j in range(L) if j <= i + 1]
            s = np.array([0.3 * sum(q[h, i, d] * k[kh, j, d] for d in range(D)) for j in js])
            p = np.exp(s - s.max())
            p /= p.sum()
            want = sum(pj * v[kh, j] for pj, j in zip(p, js))
            np.testing.assert_allclose(out[(h // 2) * 6 + i, (h % 2) * D:(h % 2 + 1) * D], want, rtol=1e-12)


def test_ref_attention_invariants():
    rng = np.random.default_rng(9)
    v = rng.standard_normal((1, 9, 4))
    # identical keys: uniform weights, the output is the mean of V
    out = oa.ref_attention(rng.standard_normal((1, 3, 4)), np.ones((1, 9, 4)), v, 1.0)
    np.testing.assert_allclose(out, np.repeat(v[0].mean(0, keepdims=True), 3, 0), rtol=1e-12)
    # one key far above the rest: its value row
    q = np.ones((1, 1, 4))
    k = np.zeros((1, 9, 4))
    k[0, 4] = 100.0
    np.testing.assert_allclose(oa.ref_attention(q, k, v, 1.0)[0], v[0, 4], rtol=1e-12)


def test_f32_chunked_baseline_agrees():
    rng = np.random.default_rng(10)
    q, k, v = rng.standard_normal((3, 300, 64)).astype(np.float32)
    got = oa.attention_f32_chunked(q, k, v, 0.125, chunk=128)
    want = oa.ref_attention(q[None], k[None], v[None], 0.125)
    np.testing.assert_allclose(got, want, atol=2e-5)


def test_bf16_conversion():
    x = np.array([1.0, 1.00390625, 1.0078125, 1.005859375, -3.140625, 65504.0, 1e-30], np.float32)
    b = to_bf16(x)
    assert from_bf16(b)[0] == 1.0 and from_bf16(b)[1] == 1.0  # tie rounds to even (1.0)
    assert from_bf16(b)[2] == np.float32(1.0078125)
    assert from_bf16(b)[3] == np.float32(1.0078125)  # above the tie rounds up
    assert from_bf16(b)[4] == np.float32(-3.140625)
    assert np.array_equal(to_bf16(from_bf16(b)), b)


# -- committed golden fixtures -------------------------------------------------------------------------------------

def test_golden_prepass_fixture_reproduces():
    """The committed pre-pass fixture (tests/golden/make_golden.py) is reproduced by the current oracle."""
    f = np.load(os.path.join(GOLDEN, "prepass_rot_int8.npz"))
    x = from_bf16(f["qkv_bf16"])
    H, hd = int(f["H"]), int(f["hd"])
    out = op.qk_norm_rope(x, Hq=H, Hk=H, Hv=H, hd=hd, out_rows=int(f["out_rows"]), rot=0, eps=1e-6, norm=False,
                          q8=True, qk_rot=True)
    assert np.array_equal(out["Q"], f["Q"]) and np.array_equal(out["K"], f["K"])
    assert np.array_equal(out["qs"].view(np.uint32), f["qs"].view(np.uint32))
    assert np.array_equal(out["ks"].view(np.uint32), f["ks"].view(np.uint32))


def test_golden_scores_fixture_reproduces():
    f = np.load(os.path.join(GOLDEN, "scores_int8.npz"))
    assert np.array_equal(oa.int_scores(f["Q"], f["K"]), f["S"])


# -- rot_q8 (the attention output's consumer) ------------------------------------------------------------------------

def test_rot_rows_matches_reference_test_formula():
    """The reference's own check (tests/test_ops.py:9-18): x.reshape(M, D/256, 256) @ H^T / sqrt(256) with the
    Sylvester matrix, in float64."""
    from oracle import rot_q8 as orq
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((9, 1024)) * 2).astype(np.float32)
    want = (x.astype(np.float64).reshape(9, 4, 256) @ sylvester(256).T / 16.0).reshape(9, 1024)
    got = orq.rotate_rows_f32(x).astype(np.float64)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6 * np.abs(want).max())


def test_rot_rows_blocks_independent_and_one_hot():
    """A one-hot column c of block b yields +-1/16 exactly in block b only, with the signs of Sylvester row
    c % 256 (a block mix-up or a wrong stage order fails)."""
    from oracle import rot_q8 as orq
    D = 768
    for c in (0, 1, 37, 255, 256 + 130, 512 + 7):
        x = np.zeros((1, D), np.float32)
        x[0, c] = 1.0
        r = orq.rotate_rows_f32(x)[0]
        b = c // 256
        assert np.all(r[:b * 256] == 0) and np.all(r[(b + 1) * 256:] == 0)
        assert np.array_equal(r[b * 256:(b + 1) * 256], (sylvester(256)[c % 256] / 16).astype(np.float32))


def test_rot_rows_integer_exact_and_involution():
    """Integer rows: every butterfly sum is exact, so the result is the integer matrix product / 16 bit for bit;
    the rotation is orthonormal and symmetric, so applying it twice returns the row."""
    from oracle import rot_q8 as orq
    rng = np.random.default_rng(6)
    x = rng.integers(-500, 500, (5, 512))
    want = (x.reshape(5, 2, 256) @ sylvester(256).astype(np.int64).T).reshape(5, 512) / 16.0
    assert np.array_equal(orq.rotate_rows_f32(x.astype(np.float32)), want.astype(np.float32))
    y = rng.standard_normal((5, 512)).astype(np.float32)
    np.testing.assert_allclose(orq.rotate_rows_f32(orq.rotate_rows_f32(y)), y, rtol=0, atol=1e-5)


def test_rot_q8_int8_step():
    """Row scale = amax/127 of the rotated row: the largest entry codes to +-127, every code dequantises within
    half a step, a zero row gets scale 1 and zero codes; swiglu with zero gates is the zero row."""
    from oracle import rot_q8 as orq
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((6, 512)) * 3).astype(np.float32)
    x[2] = 0
    codes, scale, r = orq.rot_q8(x, 512)
    assert scale[2] == 1 and not codes[2].any()
    for m in (0, 1, 3, 4, 5):
        j = np.abs(r[m]).argmax()
        assert abs(int(codes[m, j])) == 127
        assert np.abs(codes[m].astype(np.float64) * scale[m] - r[m]).max() <= 0.5 * scale[m] * (1 + 1e-6)
    xs = np.concatenate([x, np.zeros_like(x)], 1)
    c2, s2, _ = orq.rot_q8(xs, 512, swiglu=True)
    assert np.all(s2 == 1) and not c2.any()


def test_silu_gate_against_float64():
    from oracle import rot_q8 as orq
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((4, 512)) * 4).astype(np.float32)
    v, g = x[:, :256].astype(np.float64), x[:, 256:].astype(np.float64)
    want = v * g / (1 + np.exp(-g))
    np.testing.assert_allclose(orq.silu_gated_f32(x, 256), want, rtol=3e-6, atol=1e-6)


# -- gemm (the int8 projections) --------------------------------------------------------------------------------------

def test_gemm_int_product_brute_force():
    from oracle import gemm as og
    rng = np.random.default_rng(9)
    a = rng.integers(-127, 128, (5, 70), dtype=np.int8)
    w = rng.integers(-127, 128, (3, 70), dtype=np.int8)
    got = og.int_product(a, w)
    for m in range(5):
        for n in range(3):
            assert got[m, n] == sum(int(a[m, k]) * int(w[n, k]) for k in range(70))
    big = np.full((1, 4096), -127, np.int8)
    assert og.int_product(big, big)[0, 0] == 4096 * 127 * 127


def test_gemm_epilogue_order_and_exact_cases():
    """Values where every step is exact give the exact result; random values agree with float64 within float32
    rounding of three operations; the residual form adds gate[type] * v."""
    from oracle import gemm as og
    acc = np.array([[3, -5], [1024, 7]], np.int64)
    sa, sw, bias = np.array([0.5, 2.0], np.float32), np.array([0.25, 4.0], np.float32), np.array([1.0, -1.0], np.float32)
    v = og.epilogue(acc, sa, sw, bias)
    assert np.array_equal(v, np.array([[3 * 0.5 * 0.25 + 1, -5 * 0.5 * 4 - 1], [1024 * 2 * 0.25 + 1, 7 * 2 * 4 - 1]],
                                      np.float32))
    rng = np.random.default_rng(10)
    acc = rng.integers(-2 ** 26, 2 ** 26, (20, 30))
    sa, sw = rng.uniform(1e-3, 1e-2, 20).astype(np.float32), rng.uniform(1e-3, 1e-2, 30).astype(np.float32)
    want = acc.astype(np.float64) * sa[:, None].astype(np.float64) * sw[None, :].astype(np.float64)
    np.testing.assert_allclose(og.epilogue(acc, sa, sw), want, rtol=4e-7, atol=0)
    x = rng.standard_normal((20, 30)).astype(np.float32)
    gate = rng.standard_normal((3, 30)).astype(np.float32)
    rt = rng.integers(0, 3, 20).astype(np.uint8)
    vv = og.epilogue(acc, sa, sw)
    got = og.residual(x, vv, gate, rt)
    np.testing.assert_allclose(got, x.astype(np.float64) + gate[rt].astype(np.float64) * vv, rtol=1e-6, atol=1e-6)
    assert got[0, 0] == np.float32(x[0, 0] + np.float32(gate[rt[0], 0] * vv[0, 0]))


def test_gemm_float_product_brute_force():
    """float_product against Python sums of exactly representable half values (small integers and halves), so
    every product and partial sum is exact in float64."""
    from oracle import gemm as og
    rng = np.random.default_rng(6)
    a = (rng.integers(-64, 65, size=(5, 40)) / 2.0).astype(np.float16)
    w = rng.integers(-127, 128, size=(7, 40), dtype=np.int8)
    got = og.float_product(a.astype(np.float32), w)
    want = np.array([[sum(float(a[i, k]) * int(w[j, k]) for k in range(40)) for j in range(7)] for i in range(5)])
    assert np.array_equal(got, want)
