"""The gfx950 attention kernels against the CPU oracle.

* int32 score accumulators of the int8 path: bit-exact against exact integer products (through attention's own
  MFMA path and LDS staging: ops.attention_scores).
* Outputs: the reference's own cases (tests/test_attention.py: check :23-56 with half inputs, check_q8 :60-114
  with int8 scores, temp/ramp stresses, GQA, causal, D=64) with its tolerance 5e-3 max-abs against float64;
  the north-star tolerance (2e-2 max-abs, 1e-3 mean-abs against fp32/float64) for the bf16 paths and the
  benchmark configs.
"""

import numpy as np
import pytest

from h3metal_amd import ops
from oracle import attention as oa
from oracle import prepass as op
from oracle.bf16 import from_bf16, to_bf16

pytestmark = pytest.mark.gpu

NS_MAX, NS_MEAN = 2e-2, 1e-3


def q8(x):
    """Per-row symmetric int8 of tests/test_attention.py:74-76."""
    s = np.abs(x).max(-1, keepdims=True) / 127
    return np.rint(x / s).astype(np.int8), s[..., 0].astype(np.float32)


def padded(gpu, arr, rows, dtype):
    t = gpu.empty((arr.shape[0], rows) + arr.shape[2:], dtype)
    full = np.zeros((arr.shape[0], rows) + arr.shape[2:], arr.dtype)
    full[:, :arr.shape[1]] = arr
    t.write(full)
    return t


def run_attention(gpu, q, k, v, *, dtype, Lq, L, H, KVH, D, scale, causal=False, off=0, qs=None, ks=None,
                  out_dt="f16", q_rows=None, k_rows=None, seq_heads=None, seq_rows=0, out_rows=None, **variant):
    q_rows = q_rows or (Lq + 63) // 64 * 64
    k_rows = k_rows or (L + 31) // 32 * 32
    print(f"[attention] Lq={Lq} L={L} H={H} KVH={KVH} D={D} dtype={dtype} causal={causal} q8={qs is not None} "
          f"out={out_dt}", flush=True)
    qdt = "i8" if qs is not None else dtype
    Q, K, V = padded(gpu, q, q_rows, qdt), padded(gpu, k, k_rows, qdt), padded(gpu, v, k_rows, dtype)
    sh = seq_heads or H
    rows = out_rows or q_rows
    O = gpu.empty((rows, sh * D), out_dt)
    extra = {}
    if qs is not None:
        extra = dict(q_scale=padded(gpu, qs, q_rows, "f32"), k_scale=padded(gpu, ks, k_rows, "f32"))
    ops.attention(gpu, Q, K, V, O, Lq=Lq, L=L, H=H, KVH=KVH, D=D, q_rows=q_rows, k_rows=k_rows, scale=scale,
                  causal=causal, causal_off=off, seq_heads=seq_heads, seq_rows=seq_rows, **extra, **variant)
    gpu.wait()
    o = O.numpy()
    return from_bf16(o) if out_dt == "bf16" else o.astype(np.float64)


# -- int32 / fp32 score accumulators -------------------------------------------------------------------------------

@pytest.mark.parametrize("Lq,L,H,KVH,D", [(100, 100, 2, 2, 128), (77, 300, 3, 3, 128), (64, 64, 4, 1, 64),
                                          (300, 1037, 2, 1, 128), (1, 5, 1, 1, 128), (700, 449, 2, 2, 128)])
def test_int32_scores_bit_exact(gpu, Lq, L, H, KVH, D):
    """int32 score accumulators of the kernel that runs equal the exact integer products (int8: D=128 the
    wave-pipelined kernel, D=64 the two-group one)."""
    rng = np.random.default_rng(Lq + L)
    qi = rng.integers(-127, 128, (H, Lq, D)).astype(np.int8)
    ki = rng.integers(-127, 128, (KVH, L, D)).astype(np.int8)
    qi[0, 0] = -127  # extreme magnitudes: 128 * 127^2 must not overflow or round
    ki[0, 0] = -127
    q_rows, k_rows = (Lq + 63) // 64 * 64, (L + 31) // 32 * 32
    Q, K = padded(gpu, qi, q_rows, "i8"), padded(gpu, ki, k_rows, "i8")
    V = gpu.empty((KVH, k_rows, D), "bf16")
    qs, ks = gpu.upload(np.ones((H, q_rows), np.float32)), gpu.upload(np.ones((KVH, k_rows), np.float32))
    S = gpu.empty((H, Lq, L), "i32")
    print(f"[scores] Lq={Lq} L={L} H={H} KVH={KVH} D={D}", flush=True)
    ops.attention_scores(gpu, Q, K, V, S, Lq=Lq, L=L, H=H, KVH=KVH, D=D, q_rows=q_rows, k_rows=k_rows,
                         q_scale=qs, k_scale=ks)
    gpu.wait()
    want = oa.int_scores(qi, ki, H_per_kv=H // KVH)
    got = S.numpy()
    assert np.array_equal(got, want), f"{(got != want).sum()} int32 scores differ"


def test_int32_scores_golden_fixture(gpu):
    import os
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "scores_int8.npz"))
    qi, ki, want = f["Q"], f["K"], f["S"]
    H, Lq, D = qi.shape
    L = ki.shape[1]
    Q, K = padded(gpu, qi, 64, "i8"), padded(gpu, ki, 64, "i8")
    S = gpu.empty((H, Lq, L), "i32")
    ops.attention_scores(gpu, Q, K, gpu.empty((H, 64, D), "bf16"), S, Lq=Lq, L=L, H=H, KVH=H, D=D, q_rows=64,
                         k_rows=64, q_scale=gpu.upload(np.ones((H, 64), np.float32)),
                         k_scale=gpu.upload(np.ones((H, 64), np.float32)))
    gpu.wait()
    assert np.array_equal(S.numpy(), want)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
def test_float_scores(gpu, dtype):
    """16-bit inputs: products are exact in fp32 and the 128-term sums are accumulated in fp32."""
    rng = np.random.default_rng(5)
    H, Lq, L, D = 2, 70, 130, 128
    q = rng.standard_normal((H, Lq, D)).astype(np.float32)
    k = rng.standard_normal((H, L, D)).astype(np.float32)
    if dtype == "bf16":
        qh, kh, qf, kf = to_bf16(q), to_bf16(k), from_bf16(to_bf16(q)), from_bf16(to_bf16(k))
    else:
        qh, kh = q.astype(np.float16), k.astype(np.float16)
        qf, kf = qh.astype(np.float32), kh.astype(np.float32)
    Q, K = padded(gpu, qh, 128, dtype), padded(gpu, kh, 160, dtype)
    S = gpu.empty((H, Lq, L), "f32")
    ops.attention_scores(gpu, Q, K, gpu.empty((H, 160, D), dtype), S, Lq=Lq, L=L, H=H, KVH=H, D=D, q_rows=128,
                         k_rows=160)
    gpu.wait()
    want = np.einsum("hqd,hkd->hqk", qf.astype(np.float64), kf.astype(np.float64))
    np.testing.assert_allclose(S.numpy(), want, rtol=0, atol=1e-3)


# -- outputs: the reference's tests/test_attention.py cases --------------------------------------------------------

CHECK_CASES = [(100, 100, 2, 2, 128, False), (77, 300, 3, 3, 128, False), (64, 64, 4, 1, 64, False),
               (130, 130, 8, 2, 128, True), (1000, 1037, 2, 2, 128, False)]


@pytest.mark.parametrize("Lq,L,H,KVH,D,causal", CHECK_CASES)
def test_half_path_reference_cases(gpu, Lq, L, H, KVH, D, causal):
    """check() of tests/test_attention.py:23-42: half Q/K/V ~N(0,1), seed 0, max-abs < 5e-3 vs float64."""
    rng = np.random.default_rng(0)
    q = rng.standard_normal((H, Lq, D)).astype(np.float16)
    k = rng.standard_normal((KVH, L, D)).astype(np.float16)
    v = rng.standard_normal((KVH, L, D)).astype(np.float16)
    got = run_attention(gpu, q, k, v, dtype="f16", Lq=Lq, L=L, H=H, KVH=KVH, D=D, scale=D ** -0.5, causal=causal)
    ref = oa.ref_attention(q, k, v, D ** -0.5, causal=causal)
    err = np.abs(got[:Lq] - ref).max()
    assert err < 5e-3, err


Q8_CASES = [dict(Lq=100, L=100, H=2, KVH=2, D=128), dict(Lq=300, L=1037, H=3, KVH=3, D=128),
            dict(Lq=130, L=130, H=8, KVH=2, D=128, causal=True), dict(Lq=64, L=64, H=4, KVH=4, D=64),
            dict(Lq=300, L=1037, H=3, KVH=3, D=128, temp=6.0),
            dict(Lq=257, L=4100, H=2, KVH=2, D=128, temp=8.0, ramp=4.0),
            dict(Lq=200, L=200, H=2, KVH=2, D=128, causal=True, temp=5.0, ramp=3.0)]


@pytest.mark.parametrize("case", Q8_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
@pytest.mark.parametrize("vdt", ["f16", "bf16"])
def test_int8_path_reference_cases(gpu, case, vdt):
    """check_q8() of tests/test_attention.py:60-114: int8 scores against float64 attention of the dequantised
    inputs; max-abs < 5e-3 with half V (the reference's bound), the north-star bound with bf16 V."""
    c = dict(case)
    Lq, L, H, KVH, D = c["Lq"], c["L"], c["H"], c["KVH"], c["D"]
    causal, temp, ramp = c.get("causal", False), c.get("temp", 1.0), c.get("ramp", 0.0)
    rng = np.random.default_rng(0)
    q = rng.standard_normal((H, Lq, D)).astype(np.float32) * temp
    k = rng.standard_normal((KVH, L, D)).astype(np.float32)
    if ramp:
        k *= (1 + ramp * np.arange(L) / L)[None, :, None].astype(np.float32)
    v = rng.standard_normal((KVH, L, D)).astype(np.float16)
    qi, qs = q8(q)
    ki, ks = q8(k)
    vh = v if vdt == "f16" else to_bf16(v.astype(np.float32))
    vf = v.astype(np.float64) if vdt == "f16" else from_bf16(vh).astype(np.float64)
    got = run_attention(gpu, qi, ki, vh, dtype=vdt, Lq=Lq, L=L, H=H, KVH=KVH, D=D, scale=D ** -0.5, causal=causal,
                        qs=qs, ks=ks, q_rows=(Lq + 255) // 256 * 256)
    ref = oa.ref_attention(qi * qs[..., None].astype(np.float64), ki * ks[..., None].astype(np.float64), vf,
                           D ** -0.5, causal=causal)
    err = np.abs(got[:Lq] - ref)
    if vdt == "f16":
        assert err.max() < 5e-3, err.max()
    else:
        assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean())


@pytest.mark.parametrize("out_dt", ["bf16", "f32"])
def test_bf16_path_and_output_types(gpu, out_dt):
    rng = np.random.default_rng(21)
    H, Lq, L, D = 3, 333, 500, 128
    q, k, v = (to_bf16(rng.standard_normal((H, n, D)).astype(np.float32)) for n in (Lq, L, L))
    got = run_attention(gpu, q, k, v, dtype="bf16", Lq=Lq, L=L, H=H, KVH=H, D=D, scale=D ** -0.5, out_dt=out_dt)
    ref = oa.ref_attention(from_bf16(q), from_bf16(k), from_bf16(v), D ** -0.5)
    err = np.abs(got[:Lq] - ref)
    assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean())
    if out_dt == "f32":
        assert err.max() < 5e-3


def test_batched_sequences_output_placement(gpu):
    """seq_heads / seq_rows (attention.metal:384-385; the VAE's batched tiles, vae.py:206-207): 6 heads as 3
    sequences of 2 heads, each sequence's rows seq_rows apart."""
    rng = np.random.default_rng(22)
    H, sh, Lq, D, seq_rows = 6, 2, 40, 64, 48
    q, k, v = (rng.standard_normal((H, Lq, D)).astype(np.float16) for _ in range(3))
    got = run_attention(gpu, q, k, v, dtype="f16", Lq=Lq, L=Lq, H=H, KVH=H, D=D, scale=D ** -0.5, seq_heads=sh,
                        seq_rows=seq_rows, out_rows=3 * seq_rows)
    ref = oa.ref_attention(q, k, v, D ** -0.5, seq_heads=sh, seq_rows=seq_rows)
    for s in range(3):
        blk = slice(s * seq_rows, s * seq_rows + Lq)
        assert np.abs(got[blk] - ref[blk]).max() < 5e-3
    assert (got[Lq:seq_rows] == 0).all()  # rows between sequences untouched


def test_causal_offset(gpu):
    rng = np.random.default_rng(23)
    H, Lq, L, D, off = 2, 90, 150, 128, 60
    q, k, v = (rng.standard_normal((H, n, D)).astype(np.float16) for n in (Lq, L, L))
    got = run_attention(gpu, q, k, v, dtype="f16", Lq=Lq, L=L, H=H, KVH=H, D=D, scale=D ** -0.5, causal=True,
                        off=off)
    ref = oa.ref_attention(q, k, v, D ** -0.5, causal=True, off=off)
    assert np.abs(got[:Lq] - ref).max() < 5e-3


# -- benchmark configs ------------------------------------------------------------------------------------------------

def test_config1_plumbing(gpu):
    """Config 1: B=1, H=4, S=256, D=128, fp32 N(0,1), scale 1/sqrt(128), no mask, vs the numpy reference of the
    fp32 inputs (the kernel takes them as bf16)."""
    rng = np.random.default_rng(0)
    H, S, D = 4, 256, 128
    q, k, v = (rng.standard_normal((H, S, D)).astype(np.float32) for _ in range(3))
    got = run_attention(gpu, to_bf16(q), to_bf16(k), to_bf16(v), dtype="bf16", Lq=S, L=S, H=H, KVH=H, D=D,
                        scale=D ** -0.5, out_dt="f32")
    ref = oa.ref_attention(q, k, v, D ** -0.5)
    err = np.abs(got[:S] - ref)
    assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean())


def axial_rope_tables(n_txt, grid, hd, theta=10000.0):
    """2D axial RoPE angles per row for the bf16 FLUX-shaped config: text rows angle 0; image rows rotate half of
    the rotated pairs by the row coordinate and half by the column coordinate (flux2.py:396-401)."""
    half = hd // 2
    per_axis = half // 2
    freqs = theta ** (-np.arange(per_axis) / per_axis)
    rows = np.zeros((n_txt + grid * grid, half))
    yy, xx = np.divmod(np.arange(grid * grid), grid)
    rows[n_txt:, :per_axis] = yy[:, None] * freqs
    rows[n_txt:, per_axis:] = xx[:, None] * freqs
    return np.cos(rows).astype(np.float32), np.sin(rows).astype(np.float32)


def test_config2_flux_joint_bf16(gpu):
    """Config 2 (FLUX.2-klein-4B joint attention): H=24, D=128, S=4608 (512 text + 64x64 image), bf16 N(0,1),
    per-head RMSNorm on Q/K and 2D axial RoPE through qk_norm_rope, unquantised bf16 attention. Checked on a
    seeded sample of query rows against float64 attention of the kernel's own bf16 Q/K/V."""
    rng = np.random.default_rng(2)
    H, D, n_txt, grid = 24, 128, 512, 64
    S = n_txt + grid * grid
    x = to_bf16(rng.standard_normal((S, 3 * H * D)).astype(np.float32))
    cs, sn = axial_rope_tables(n_txt, grid, D)
    g = gpu
    X = g.upload(x, "bf16")
    Q, K, V = (g.empty((H, S, D), "bf16") for _ in range(3))
    ones = g.upload(np.ones(D, np.float32))
    ops.qk_norm_rope(g, X, ones, ones, g.upload(cs), g.upload(sn), Q, K, V, M=S, Hq=H, Hk=H, Hv=H, hd=D,
                     out_rows=S, rot=D, eps=1e-6, norm=True)
    O = g.empty((S, H * D), "bf16")
    ops.attention(g, Q, K, V, O, Lq=S, L=S, H=H, KVH=H, D=D, q_rows=S, k_rows=S, scale=D ** -0.5)
    g.wait()
    qh, kh, vh = (from_bf16(t.numpy()).astype(np.float64) for t in (Q, K, V))
    # the pre-pass output itself against the float32 oracle (bf16 rounding of the oracle's result)
    rows = np.sort(rng.choice(S, 256, replace=False))
    want = op.qk_norm_rope(from_bf16(x[rows]), Hq=H, Hk=H, Hv=H, hd=D, out_rows=len(rows), rot=D, eps=1e-6,
                           norm=True, wq=np.ones(D, np.float32), wk=np.ones(D, np.float32), cs=cs[rows], sn=sn[rows])
    assert np.array_equal(Q.numpy()[:, rows], to_bf16(want["Q"]))
    got = from_bf16(O.numpy()).astype(np.float64)
    ref = oa.ref_attention(qh[:, rows], kh, vh, D ** -0.5)
    err = np.abs(got[rows] - ref)
    assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean())


def test_config3_zimage_key_padding(gpu):
    """Config 3 (Z-Image-Turbo): H=30, D=128, 4096 image rows then text padded to 512 with only the first
    L_txt ~ U[32, 512] valid: the boolean key mask is keys >= 4096 + L_txt (the kernel's L). The padded key rows
    hold N(0,1) data here, which the mask must ignore."""
    rng = np.random.default_rng(3)
    H, D, n_img = 30, 128, 4096
    L_txt = int(rng.integers(32, 513))
    S = n_img + 512
    L = n_img + L_txt
    q, k, v = (to_bf16(rng.standard_normal((H, S, D)).astype(np.float32)) for _ in range(3))
    Q, K, V = (gpu.upload(t, "bf16") for t in (q, k, v))
    O = gpu.empty((S, H * D), "bf16")
    ops.attention(gpu, Q, K, V, O, Lq=S, L=L, H=H, KVH=H, D=D, q_rows=S, k_rows=S, scale=D ** -0.5)
    gpu.wait()
    rows = np.sort(rng.choice(S, 192, replace=False))
    ref = oa.ref_attention(from_bf16(q[:, rows]), from_bf16(k), from_bf16(v), D ** -0.5, L=L)
    err = np.abs(from_bf16(O.numpy())[rows] - ref)
    assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean(), L_txt)


def test_config4_int32_scores_and_output_at_full_key_length(gpu):
    """The config-4 key count (L = 16896) through the scores hook, which runs ops.attention's own kernel
    (same tiles, LDS staging, tail split of the last round of tiles, P V and output): int32 scores of every
    (query, key) pair of two heads bit-exact against exact integer products, and the output of the same launch
    against float64 attention of the dequantised inputs."""
    rng = np.random.default_rng(44)
    H, D, Lq, L = 2, 128, 300, 16896
    xq = rng.standard_normal((H, Lq, D)).astype(np.float32)
    xk = rng.standard_normal((H, L, D)).astype(np.float32)
    xq[:, :, :4] *= 20
    xk[:, :, 5:9] *= 20
    qi, qsc = op.quant_i8(op.rotate_f32(xq))
    ki, ksc = op.quant_i8(op.rotate_f32(xk))
    qi[0, 0] = -127
    ki[0, 0] = -127  # the extreme product 128 * 127^2
    vb = to_bf16(rng.standard_normal((H, L, D)).astype(np.float32))
    Q, K, V = gpu.upload(qi, "i8"), gpu.upload(ki, "i8"), gpu.upload(vb, "bf16")
    qs, ks = gpu.upload(qsc), gpu.upload(ksc)
    S = gpu.empty((H, Lq, L), "i32")
    O = gpu.empty((Lq, H * D), "bf16")
    print(f"[scores] full key length Lq={Lq} L={L} H={H} (split last round)", flush=True)
    ops.attention_scores(gpu, Q, K, V, S, Lq=Lq, L=L, H=H, KVH=H, D=D, q_rows=Lq, k_rows=L, q_scale=qs,
                         k_scale=ks, out=O, scale=D ** -0.5)
    gpu.wait()
    want = oa.int_scores(qi, ki)
    got = S.numpy()
    assert np.array_equal(got, want), f"{(got != want).sum()} int32 scores differ"
    ref = oa.ref_attention(qi * qsc[..., None].astype(np.float64), ki * ksc[..., None].astype(np.float64),
                           from_bf16(vb), D ** -0.5)
    err = np.abs(from_bf16(O.numpy()).astype(np.float64) - ref)
    assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean())


def test_int32_scores_and_output_in_reversed_rounds(gpu):
    """Enough workgroups that every other round of an XCD's workgroups takes its key blocks in the order
    L-2, ..., 0, L-1 (520 one-tile heads: the rounds after the first 256 workgroups run reversed), with a ragged
    last block (L = 300: 5 blocks, the last with 44 keys) and GQA (8 key/value heads): the int32 scores of every
    head bit-exact against exact integer products (the scores hook writes each at its key index, so a block
    mapped to the wrong keys fails), and the output of sampled heads against float64 attention."""
    rng = np.random.default_rng(45)
    H, KVH, D, Lq, L = 520, 8, 128, 256, 300
    qi = rng.integers(-127, 128, (H, Lq, D)).astype(np.int8)
    ki = rng.integers(-127, 128, (KVH, L, D)).astype(np.int8)
    qsc = rng.uniform(1e-3, 2e-3, (H, Lq)).astype(np.float32)
    ksc = rng.uniform(1e-3, 2e-3, (KVH, L)).astype(np.float32)
    vb = to_bf16(rng.standard_normal((KVH, L, D)).astype(np.float32))
    Q, K, V = gpu.upload(qi, "i8"), gpu.upload(ki, "i8"), gpu.upload(vb, "bf16")
    qs, ks = gpu.upload(qsc), gpu.upload(ksc)
    S = gpu.empty((H, Lq, L), "i32")
    O = gpu.empty((Lq, H * D), "bf16")
    print(f"[scores] reversed rounds H={H} KVH={KVH} Lq={Lq} L={L}", flush=True)
    ops.attention_scores(gpu, Q, K, V, S, Lq=Lq, L=L, H=H, KVH=KVH, D=D, q_rows=Lq, k_rows=L, q_scale=qs,
                         k_scale=ks, out=O, scale=D ** -0.5)
    gpu.wait()
    g = H // KVH
    kf = ki.astype(np.float64)
    want = np.einsum("hqd,hkd->hqk", qi.astype(np.float64), np.repeat(kf, g, axis=0), optimize=True)
    got = S.numpy()
    assert np.array_equal(got, want.astype(np.int32)), f"{(got != want).sum()} int32 scores differ"
    heads = [0, 31, 32, 63, 100, 300, 519]
    kd = ki * ksc[..., None].astype(np.float64)
    ref = oa.ref_attention(qi[heads] * qsc[heads][..., None].astype(np.float64), kd[[h // g for h in heads]],
                           from_bf16(vb)[[h // g for h in heads]], D ** -0.5)
    out = from_bf16(O.numpy()).astype(np.float64).reshape(Lq, H, D)[:, heads].reshape(Lq, len(heads) * D)
    err = np.abs(out - ref)
    assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean())


def test_config4_int8_rotated_full_size(gpu):
    """Config 4 at full size: H=32, D=128, S=16896, outlier channels x20, rotation + int8 pre-pass, int8
    attention with bf16 V. On a seeded sample of query rows:
    * against float64 attention of the dequantised int8 inputs (the reference's check_q8 convention,
      tests/test_attention.py:89): the north-star tolerance, 2e-2 max-abs and 1e-3 mean-abs;
    * against fp32 attention of the unquantised bf16 Q/K (heads 0 and 1): the int8 rounding itself moves the
      output by far more than that tolerance at this outlier recipe (the oracle's dequantised attention is
      ~0.07 relative L2 / ~0.5 max-abs away from it), so the bound is that the GPU output is no further from the
      unquantised attention than the oracle's dequantised attention is (within 2%), and that the rotation cuts
      the plain int8 error to below 0.6x (the reference's criterion, tests/test_qk_rotation.py:64)."""
    rng = np.random.default_rng(4)
    H, D, S = 32, 128, 16896
    x = rng.standard_normal((S, 3, H, D)).astype(np.float32)
    for part in (0, 1):
        for h in range(H):
            x[:, part, h, rng.choice(D, 4, replace=False)] *= 20
    xb = to_bf16(x.reshape(S, 3 * H * D))
    X = gpu.upload(xb, "bf16")
    Q, K = gpu.empty((H, S, D), "i8"), gpu.empty((H, S, D), "i8")
    V = gpu.empty((H, S, D), "bf16")
    qs, ks = gpu.empty((H, S), "f32"), gpu.empty((H, S), "f32")
    ops.qk_norm_rope(gpu, X, None, None, None, None, Q, K, V, M=S, Hq=H, Hk=H, Hv=H, hd=D, out_rows=S, rot=0,
                     eps=1e-6, norm=False, q_scale=qs, k_scale=ks, qk_rot=True)
    O = gpu.empty((S, H * D), "bf16")
    ops.attention(gpu, Q, K, V, O, Lq=S, L=S, H=H, KVH=H, D=D, q_rows=S, k_rows=S, scale=D ** -0.5, q_scale=qs,
                  k_scale=ks)
    gpu.wait()
    qi, ki, qsh, ksh, vh = Q.numpy(), K.numpy(), qs.numpy(), ks.numpy(), from_bf16(V.numpy())
    rows = np.sort(rng.choice(S, 128, replace=False))
    qd = qi[:, rows] * qsh[:, rows, None].astype(np.float64)
    kd = ki * ksh[..., None].astype(np.float64)
    ref = oa.ref_attention(qd, kd, vh, D ** -0.5)
    got = from_bf16(O.numpy()).astype(np.float64)[rows]
    err = np.abs(got - ref)
    assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean())
    # the unquantised reference: fp32 attention of the bf16 Q/K (heads 0, 1)
    xf = from_bf16(xb).reshape(S, 3, H, D)
    for h in (0, 1):
        qf, kf = xf[:, 0, h].astype(np.float64), xf[:, 1, h].astype(np.float64)
        fp = oa.ref_attention(qf[rows][None], kf[None], vh[h][None], D ** -0.5)
        mine = got[:, h * D:(h + 1) * D]
        deq = ref[:, h * D:(h + 1) * D]
        pi, ps = op.quant_i8(xf[:, 0, h])
        pk, pks = op.quant_i8(xf[:, 1, h])
        plain = oa.ref_attention((pi[rows] * ps[rows, None].astype(np.float64))[None],
                                 (pk * pks[:, None].astype(np.float64))[None], vh[h][None], D ** -0.5)
        rel = lambda a: np.linalg.norm(a - fp) / np.linalg.norm(fp)  # noqa: E731
        print(f"[config4 head {h}] vs unquantised: gpu rel-L2 {rel(mine):.4f} max {np.abs(mine - fp).max():.3f}; "
              f"oracle int8 {rel(deq):.4f}; plain int8 {rel(plain):.4f}", flush=True)
        assert rel(mine) <= 1.02 * rel(deq) + 1e-3
        assert rel(mine) < 0.6 * rel(plain)


def test_config5_int8_rotated_full_size(gpu):
    """Config 5 at full size (H=32, D=128, S=66048, the config-4 recipe): pre-pass and int8 attention over all rows
    and keys; a seeded sample of query rows against float64 attention of the dequantised int8 inputs, head by
    head."""
    rng = np.random.default_rng(5)
    H, D, S = 32, 128, 66048
    X = gpu.empty((S, 3 * H * D), "bf16")
    out_ch = [rng.choice(D, 4, replace=False) for _ in range(2 * H)]
    for r0 in range(0, S, 4096):  # generated in row chunks to bound host memory
        n = min(4096, S - r0)
        x = rng.standard_normal((n, 3, H, D), dtype=np.float32)
        for part in (0, 1):
            for h in range(H):
                x[:, part, h, out_ch[part * H + h]] *= 20
        X.write(to_bf16(x.reshape(n, -1)), offset_elems=r0 * 3 * H * D)
    Q, K = gpu.empty((H, S, D), "i8"), gpu.empty((H, S, D), "i8")
    V = gpu.empty((H, S, D), "bf16")
    qs, ks = gpu.empty((H, S), "f32"), gpu.empty((H, S), "f32")
    print("[config5] pre-pass + attention", flush=True)
    ops.qk_norm_rope(gpu, X, None, None, None, None, Q, K, V, M=S, Hq=H, Hk=H, Hv=H, hd=D, out_rows=S, rot=0,
                     eps=1e-6, norm=False, q_scale=qs, k_scale=ks, qk_rot=True)
    O = gpu.empty((S, H * D), "bf16")
    ops.attention(gpu, Q, K, V, O, Lq=S, L=S, H=H, KVH=H, D=D, q_rows=S, k_rows=S, scale=D ** -0.5, q_scale=qs,
                  k_scale=ks)
    gpu.wait()
    qi, ki, qsh, ksh, vb = Q.numpy(), K.numpy(), qs.numpy(), ks.numpy(), V.numpy()
    got = from_bf16(O.numpy()).astype(np.float64)
    rows = np.sort(rng.choice(S, 48, replace=False))
    ref = np.zeros((len(rows), H * D))
    for h in range(H):
        qd = (qi[h, rows] * qsh[h, rows, None].astype(np.float64))[None]
        kd = (ki[h] * ksh[h, :, None].astype(np.float64))[None]
        ref[:, h * D:(h + 1) * D] = oa.ref_attention(qd, kd, from_bf16(vb[h])[None], D ** -0.5)
    err = np.abs(got[rows] - ref)
    assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean())


# -- other callers' variants -------------------------------------------------------------------------------------------

@pytest.mark.parametrize("dtype,H,KVH,causal", [("f16", 4, 2, False), ("f16", 4, 4, True), ("bf16", 3, 3, False)])
def test_head_dim_96(gpu, dtype, H, KVH, causal):
    """Head dim 96, the vision tower's padded head dim (h3metal/vision.py:34, 121-130): computed on 128-wide
    MFMA tiles with the missing channels read as zeros."""
    rng = np.random.default_rng(31)
    Lq, L, D = 150, 220, 96
    q = rng.standard_normal((H, Lq, D)).astype(np.float32)
    k, v = (rng.standard_normal((KVH, L, D)).astype(np.float32) for _ in range(2))
    if dtype == "bf16":
        qh, kh, vh = to_bf16(q), to_bf16(k), to_bf16(v)
        qf, kf, vf = from_bf16(qh), from_bf16(kh), from_bf16(vh)
    else:
        qh, kh, vh = q.astype(np.float16), k.astype(np.float16), v.astype(np.float16)
        qf, kf, vf = qh, kh, vh
    got = run_attention(gpu, qh, kh, vh, dtype=dtype, Lq=Lq, L=L, H=H, KVH=KVH, D=D, scale=D ** -0.5,
                        causal=causal)
    ref = oa.ref_attention(qf, kf, vf, D ** -0.5, causal=causal)
    err = np.abs(got[:Lq] - ref)
    assert err.max() < (5e-3 if dtype == "f16" else NS_MAX) and err.mean() < NS_MEAN, (err.max(), err.mean())


def test_head_dim_96_vision_padding(gpu):
    """vision.py pads head dim 72 to 96 with zero channels: the output's padded channels stay exactly zero and the
    real ones equal attention over the 72 real channels with scale 72^-0.5."""
    rng = np.random.default_rng(32)
    H, N, hd, hdp = 2, 100, 72, 96
    q, k, v = (np.zeros((H, N, hdp), np.float16) for _ in range(3))
    for t in (q, k, v):
        t[..., :hd] = rng.standard_normal((H, N, hd)).astype(np.float16)
    got = run_attention(gpu, q, k, v, dtype="f16", Lq=N, L=N, H=H, KVH=H, D=hdp, scale=hd ** -0.5)
    got = got[:N].reshape(N, H, hdp)
    assert (got[..., hd:] == 0).all()
    ref = oa.ref_attention(q[..., :hd], k[..., :hd], v[..., :hd], hd ** -0.5).reshape(N, H, hd)
    assert np.abs(got[..., :hd] - ref).max() < 5e-3


def test_int8_head_dim_96_scores_and_output(gpu):
    rng = np.random.default_rng(33)
    H, Lq, L, D = 2, 130, 190, 96
    qi, qs = q8(rng.standard_normal((H, Lq, D)).astype(np.float32))
    ki, ks = q8(rng.standard_normal((H, L, D)).astype(np.float32))
    Q, K = padded(gpu, qi, 192, "i8"), padded(gpu, ki, 192, "i8")
    S = gpu.empty((H, Lq, L), "i32")
    ops.attention_scores(gpu, Q, K, gpu.empty((H, 192, D), "bf16"), S, Lq=Lq, L=L, H=H, KVH=H, D=D, q_rows=192,
                         k_rows=192, q_scale=padded(gpu, qs, 192, "f32"), k_scale=padded(gpu, ks, 192, "f32"))
    gpu.wait()
    assert np.array_equal(S.numpy(), oa.int_scores(qi, ki))
    v = to_bf16(rng.standard_normal((H, L, D)).astype(np.float32))
    got = run_attention(gpu, qi, ki, v, dtype="bf16", Lq=Lq, L=L, H=H, KVH=H, D=D, scale=D ** -0.5, qs=qs, ks=ks)
    ref = oa.ref_attention(qi * qs[..., None].astype(np.float64), ki * ks[..., None].astype(np.float64),
                           from_bf16(v), D ** -0.5)
    err = np.abs(got[:Lq] - ref)
    assert err.max() < NS_MAX and err.mean() < NS_MEAN


def test_te_n_valid_split_dispatch(gpu):
    """h3metal/te.py:186-194: with n_valid < T, a causal call over the first n_valid rows and keys, then a
    non-causal call for rows n_valid..T-1 through a Q view and an output row view, attending to the n_valid keys;
    GQA with Hq = 8, Hkv = 2, half inputs and output."""
    rng = np.random.default_rng(34)
    Hq, Hkv, T, n_valid, hd = 8, 2, 200, 130, 128
    Tp = 256
    q = rng.standard_normal((Hq, T, hd)).astype(np.float16)
    k, v = (rng.standard_normal((Hkv, T, hd)).astype(np.float16) for _ in range(2))
    Q, K, V = padded(gpu, q, Tp, "f16"), padded(gpu, k, Tp, "f16"), padded(gpu, v, Tp, "f16")
    o = gpu.empty((Tp, Hq * hd), "f16")
    ops.attention(gpu, Q, K, V, o, Lq=n_valid, L=n_valid, H=Hq, KVH=Hkv, D=hd, q_rows=Tp, k_rows=Tp,
                  scale=hd ** -0.5, causal=True, wm=8, bk=32)
    ops.attention(gpu, Q.view(Q.shape, offset_elems=n_valid * hd), K, V, o.row(n_valid, T - n_valid),
                  Lq=T - n_valid, L=n_valid, H=Hq, KVH=Hkv, D=hd, q_rows=Tp, k_rows=Tp, scale=hd ** -0.5,
                  causal=False, wm=8, bk=32)
    gpu.wait()
    got = o.numpy().astype(np.float64)
    ref_a = oa.ref_attention(q[:, :n_valid], k[:, :n_valid], v[:, :n_valid], hd ** -0.5, causal=True)
    ref_b = oa.ref_attention(q[:, n_valid:], k[:, :n_valid], v[:, :n_valid], hd ** -0.5)
    assert np.abs(got[:n_valid] - ref_a).max() < 5e-3
    assert np.abs(got[n_valid:T] - ref_b).max() < 5e-3
    assert (got[T:] == 0).all()


@pytest.mark.parametrize("q8_path", [False, True])
def test_tail_split_matches_whole_tiles(gpu, q8_path):
    """The last, partly filled round of workgroups is cut along the keys and merged (online-softmax merge of
    per-chunk O, m, l). Same inputs with SPLIT=0 (every tile whole): outputs agree to rounding, and both meet
    the tolerance against float64. Here 2 heads x 2 query blocks = 4 tiles on 256 CUs: every tile is split."""
    rng = np.random.default_rng(35)
    H, Lq, L, D = 2, 300, 1037, 128
    if q8_path:
        qi, qs = q8(rng.standard_normal((H, Lq, D)).astype(np.float32))
        ki, ks = q8(rng.standard_normal((H, L, D)).astype(np.float32))
        q, k, extra = qi, ki, dict(q_scale=padded(gpu, qs, 512, "f32"), k_scale=padded(gpu, ks, 1056, "f32"))
        qdt, ref_q, ref_k = "i8", qi * qs[..., None].astype(np.float64), ki * ks[..., None].astype(np.float64)
    else:
        q = to_bf16(rng.standard_normal((H, Lq, D)).astype(np.float32))
        k = to_bf16(rng.standard_normal((H, L, D)).astype(np.float32))
        extra, qdt, ref_q, ref_k = {}, "bf16", from_bf16(q), from_bf16(k)
    v = to_bf16(rng.standard_normal((H, L, D)).astype(np.float32))
    Q, K, V = padded(gpu, q, 512, qdt), padded(gpu, k, 1056, qdt), padded(gpu, v, 1056, "bf16")
    outs = []
    for split in (1, 0):
        O = gpu.empty((512, H * D), "f32")
        ops.attention(gpu, Q, K, V, O, Lq=Lq, L=L, H=H, KVH=H, D=D, q_rows=512, k_rows=1056, scale=D ** -0.5,
                      SPLIT=split, **extra)
        gpu.wait()
        outs.append(O.numpy().astype(np.float64))
    ref = oa.ref_attention(ref_q, ref_k, from_bf16(v), D ** -0.5)
    for o in outs:
        err = np.abs(o[:Lq] - ref)
        assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean())
    assert np.abs(outs[0] - outs[1]).max() < 2e-3
    assert (outs[0][Lq:] == 0).all()


@pytest.mark.parametrize("H,KVH,Lq,L,seq", [(4, 4, 1000, 1500, None), (6, 2, 777, 2049, None), (4, 4, 300, 700, 2)])
def test_int8_split_and_whole_tiles_agree(gpu, H, KVH, Lq, L, seq):
    """int8 scores at D=128 without a causal mask (the wave-pipelined kernel), the default GROUPS=0 and the
    explicit GROUPS=1, with the tail split and without (SPLIT=0). Same inputs through all,
    with and without the tail split: every output meets the tolerance against float64 and the kernels agree to
    rounding. Ragged L (a partly masked last key block), GQA, several 256-row query blocks per head and batched
    sequences (seq_heads) included."""
    rng = np.random.default_rng(H * 1000 + L)
    D = 128
    qr, kr = -(-Lq // 512) * 512, -(-L // 64) * 64 + 64
    qi, qs = q8(rng.standard_normal((H, Lq, D)).astype(np.float32))
    ki, ks = q8(rng.standard_normal((KVH, L, D)).astype(np.float32))
    v = to_bf16(rng.standard_normal((KVH, L, D)).astype(np.float32))
    Q, K, V = padded(gpu, qi, qr, "i8"), padded(gpu, ki, kr, "i8"), padded(gpu, v, kr, "bf16")
    extra = dict(q_scale=padded(gpu, qs, qr, "f32"), k_scale=padded(gpu, ks, kr, "f32"))
    seq_heads = seq or H
    nseq = H // seq_heads
    outs = []
    for groups, split in ((0, 1), (1, 1), (1, 0)):
        print(f"[attention] groups={groups} split={split} H={H} KVH={KVH} Lq={Lq} L={L} seq={seq}", flush=True)
        O = gpu.empty((nseq * qr, seq_heads * D), "f32")
        ops.attention(gpu, Q, K, V, O, Lq=Lq, L=L, H=H, KVH=KVH, D=D, q_rows=qr, k_rows=kr, scale=D ** -0.5,
                      seq_heads=seq_heads, seq_rows=qr, GROUPS=groups, SPLIT=split, **extra)
        gpu.wait()
        outs.append(O.numpy().astype(np.float64))
    rq = qi * qs[..., None].astype(np.float64)
    rk = ki * ks[..., None].astype(np.float64)
    ref = oa.ref_attention(rq, rk, from_bf16(v), D ** -0.5)  # [Lq][H * D]
    for o in outs:
        got = np.concatenate([o[s * qr:s * qr + Lq, :] for s in range(nseq)], axis=1)
        err = np.abs(got - ref)
        assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean())
    for o in outs[:-1]:
        assert np.abs(o - outs[-1]).max() < 2e-3


def test_groups_macro_refused(gpu):
    """GROUPS accepts 0 and 1 only (the values 2-4 selected kernels that are retired; checked on the host when the
    pipeline is made)."""
    from h3metal_amd.gpu import GpuError
    for g in (2, 3, 4, 5):
        with pytest.raises(GpuError, match="GROUPS must be 0 or 1"):
            gpu.kernel("attention", "attention", HD=128, QK8=1, IN_T="bfloat", O_T="bfloat", GROUPS=g)


@pytest.mark.parametrize("Lq,L", [(1, 1), (5, 63), (384, 64), (385, 65), (17, 129), (700, 191), (64, 31), (65, 33),
                                  (257, 97), (200, 160)])
def test_int8_kernel_edges(gpu, Lq, L):
    """Edge shapes through the wave-pipelined kernel (int8, D=128, no causal mask): one query or one key, key counts
    around the 64-key block and its 32-key tiles
    (the last block's rows past L load as zeros and are masked), query counts around the 64-row pairs and the
    256-row tiles. Checked against float64 within the north-star tolerance."""
    rng = np.random.default_rng(Lq * 1000 + L)
    H, D = 2, 128
    qr, kr = -(-Lq // 384) * 384, -(-L // 64) * 64
    qi, qs = q8(rng.standard_normal((H, Lq, D)).astype(np.float32))
    ki, ks = q8(rng.standard_normal((H, L, D)).astype(np.float32))
    v = to_bf16(rng.standard_normal((H, L, D)).astype(np.float32))
    Q, K, V = padded(gpu, qi, qr, "i8"), padded(gpu, ki, kr, "i8"), padded(gpu, v, kr, "bf16")
    O = gpu.empty((qr, H * D), "f32")
    print(f"[attention] edge Lq={Lq} L={L}", flush=True)
    ops.attention(gpu, Q, K, V, O, Lq=Lq, L=L, H=H, KVH=H, D=D, q_rows=qr, k_rows=kr, scale=D ** -0.5,
                  q_scale=padded(gpu, qs, qr, "f32"), k_scale=padded(gpu, ks, kr, "f32"))
    gpu.wait()
    got = O.numpy().astype(np.float64)
    ref = oa.ref_attention(qi * qs[..., None].astype(np.float64), ki * ks[..., None].astype(np.float64),
                           from_bf16(v), D ** -0.5)
    err = np.abs(got[:Lq] - ref)
    assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean())
    assert (got[Lq:] == 0).all()


def test_key_count_beyond_32bit_offsets_refused(gpu):
    """The wave kernel addresses K/V rows with 32-bit byte offsets: a key count whose V bytes (plus the blocks
    the pipeline stages past the end) pass 4 GiB is refused before anything is launched."""
    from h3metal_amd.gpu import GpuError
    D, L = 128, (1 << 32) // 256 - 255  # (L + 256) * 256 bytes > 2^32
    k_rows = (L + 31) // 32 * 32
    Q, K, V = gpu.empty((1, 64, D), "i8"), gpu.empty((1, k_rows, D), "i8"), gpu.empty((1, k_rows, D), "bf16")
    qs, ks = gpu.empty((1, 64), "f32"), gpu.empty((1, k_rows), "f32")
    O = gpu.empty((64, D), "bf16")
    print(f"[attention] refusal L={L}", flush=True)
    with pytest.raises(GpuError, match="32-bit"):
        ops.attention(gpu, Q, K, V, O, Lq=1, L=L, H=1, KVH=1, D=D, q_rows=64, k_rows=k_rows, scale=D ** -0.5,
                      q_scale=qs, k_scale=ks)


@pytest.mark.parametrize("path", ["int8", "bf16", "f16"])
def test_scores_rising_far_above_the_first_block(gpu, path):
    """Key scores that rise by ~100 log2 units from the first keys to the last (a ramp on one channel shared by
    every query), so that each row's reference maximum is passed by more than the accepted growth several times
    (2^30 per block with bf16 P, 2^15 with f16 P): the recomputed blocks and the rescaled O and l against float64
    attention, at the north-star tolerance."""
    rng = np.random.default_rng(77)
    H, Lq, L, D = 2, 130, 1100, 128
    q = rng.standard_normal((H, Lq, D)).astype(np.float32)
    k = rng.standard_normal((H, L, D)).astype(np.float32)
    v = rng.standard_normal((H, L, D)).astype(np.float32)
    q[..., 0] = 8.0
    k[..., 0] = np.linspace(-50.0, 50.0, L, dtype=np.float32)
    if path == "int8":
        qi, qs = q8(q)
        ki, ks = q8(k)
        vb = to_bf16(v)
        got = run_attention(gpu, qi, ki, vb, dtype="bf16", Lq=Lq, L=L, H=H, KVH=H, D=D, scale=D ** -0.5, qs=qs,
                            ks=ks, out_dt="f32")
        ref = oa.ref_attention(qi * qs[..., None].astype(np.float64), ki * ks[..., None].astype(np.float64),
                               from_bf16(vb), D ** -0.5)
    elif path == "bf16":
        qb, kb, vb = to_bf16(q), to_bf16(k), to_bf16(v)
        got = run_attention(gpu, qb, kb, vb, dtype="bf16", Lq=Lq, L=L, H=H, KVH=H, D=D, scale=D ** -0.5,
                            out_dt="f32")
        ref = oa.ref_attention(from_bf16(qb), from_bf16(kb), from_bf16(vb), D ** -0.5)
    else:
        qh, kh, vh = q.astype(np.float16), k.astype(np.float16), v.astype(np.float16)
        got = run_attention(gpu, qh, kh, vh, dtype="f16", Lq=Lq, L=L, H=H, KVH=H, D=D, scale=D ** -0.5,
                            out_dt="f32")
        ref = oa.ref_attention(qh, kh, vh, D ** -0.5)
    got = got[:Lq]
    err = np.abs(got - ref)
    assert np.isfinite(got).all()
    assert err.max() < NS_MAX and err.mean() < NS_MEAN, (err.max(), err.mean())
