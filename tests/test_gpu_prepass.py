"""The fused pre-pass kernel (ops.qk_norm_rope) against the float32 oracle: int8 codes and scales bit-exact,
16-bit outputs exact up to the output rounding. Mirrors the reference's tests/test_ops.py::test_qk (:80-111) and
tests/test_qk_rotation.py, plus the benchmark config-4 recipe at full size on sampled rows."""

import os

import numpy as np
import pytest

from h3metal_amd import ops
from oracle import prepass as op
from oracle import attention as oa
from oracle.bf16 import from_bf16, to_bf16

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def run_prepass(gpu, x_host, in_dt, *, M, Hq, Hk, Hv, hd, out_rows, rot=0, norm=False, eps=1e-6, q8=True,
                qk_rot=True, seq_len=None, wq=None, wk=None, cs=None, sn=None, qk_dt="f16", v_dt="bf16"):
    print(f"[prepass] M={M} H={Hq}/{Hk}/{Hv} hd={hd} in={in_dt} rot={rot} norm={norm} q8={q8} qk_rot={qk_rot} "
          f"seq_len={seq_len}", flush=True)
    X = gpu.upload(x_host, in_dt)
    nseq = -(-M // (seq_len or M))
    qdt = "i8" if q8 else qk_dt
    Q = gpu.empty((nseq * Hq, out_rows, hd), qdt)
    K = gpu.empty((nseq * Hk, out_rows, hd), qdt)
    V = gpu.empty((nseq * Hv, out_rows, hd), v_dt)
    qs = gpu.empty((nseq * Hq, out_rows), "f32") if q8 else None
    ks = gpu.empty((nseq * Hk, out_rows), "f32") if q8 else None
    up = lambda a: gpu.upload(np.asarray(a, np.float32)) if a is not None else None  # noqa: E731
    ops.qk_norm_rope(gpu, X, up(wq), up(wk), up(cs), up(sn), Q, K, V, M=M, Hq=Hq, Hk=Hk, Hv=Hv, hd=hd,
                     out_rows=out_rows, rot=rot, eps=eps, norm=norm, seq_len=seq_len, q_scale=qs, k_scale=ks,
                     qk_rot=qk_rot)
    gpu.wait()
    res = {"Q": Q.numpy(), "K": K.numpy(), "V": V.numpy()}
    if q8:
        res["qs"], res["ks"] = qs.numpy(), ks.numpy()
    return res


def as_float(arr, dt):
    return from_bf16(arr) if dt == "bf16" else arr.astype(np.float32)


def outlier_rows(rng, S, H, hd, n_out=4, mult=20.0):
    x = rng.standard_normal((S, 3, H, hd)).astype(np.float32)
    for part in (0, 1):
        for h in range(H):
            x[:, part, h, rng.choice(hd, n_out, replace=False)] *= mult
    return x.reshape(S, 3 * H * hd)


ROT_CHOICES = {128: [0, 8, 24, 40, 64, 96, 128], 64: [0, 4, 12, 24, 32, 48, 64]}  # both lane layouts


@pytest.mark.parametrize("seed", range(16))
def test_random_shape_sweep_bit_exact(gpu, seed):
    """A seeded sweep of pre-pass shapes: head dim 64 / 128, Q/K/V head counts chosen independently, ragged row
    counts, batched sequences (seq_len) or one, RMS norm on or off, RoPE widths of both lane layouts, the
    rotation on or off, bf16 / f16 / f32 input: int8 codes and scales bit for bit, V equal to its bf16 rounding."""
    rng = np.random.default_rng(3000 + seed)
    hd = [128, 64][seed % 2]
    rot = int(rng.choice(ROT_CHOICES[hd]))
    in_dt = ["bf16", "f16", "f32"][seed % 3]
    norm, qk_rot = bool(rng.integers(0, 2)), bool(seed % 4 != 1)
    Hq, Hk, Hv = (int(x) for x in rng.integers(1, 9, 3))
    M = int(rng.integers(1, 700))
    seq_len = int(rng.integers(1, M + 1)) if seed % 3 == 2 else None
    out_rows = ((seq_len or M) + 63) // 64 * 64 + int(rng.integers(0, 2)) * 64
    x = (rng.standard_normal((M, (Hq + Hk + Hv) * hd)) * 2).astype(np.float32)
    x[:, rng.choice(x.shape[1], 5, replace=False)] *= 20  # a few outlier channels
    xh = to_bf16(x) if in_dt == "bf16" else x.astype(np.float16) if in_dt == "f16" else x
    wq, wk = rng.uniform(0.5, 1.5, (2, hd)).astype(np.float32)
    ang = rng.uniform(0, 6.28, (M, max(rot // 2, 1)))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    kw = dict(wq=wq, wk=wk) if norm else {}
    if rot:
        kw.update(cs=cs, sn=sn)
    got = run_prepass(gpu, xh, in_dt, M=M, Hq=Hq, Hk=Hk, Hv=Hv, hd=hd, out_rows=out_rows, rot=rot, norm=norm,
                      eps=1e-6, qk_rot=qk_rot, seq_len=seq_len, **kw)
    want = op.qk_norm_rope(as_float(xh, in_dt), Hq=Hq, Hk=Hk, Hv=Hv, hd=hd, out_rows=out_rows, rot=rot, eps=1e-6,
                           norm=norm, seq_len=seq_len, q8=True, qk_rot=qk_rot, **kw)
    for n in ("Q", "K"):
        assert np.array_equal(got[n], want[n]), n
    for n in ("qs", "ks"):
        assert np.array_equal(got[n].view(np.uint32), want[n].view(np.uint32)), n
    assert np.array_equal(got["V"].view(np.uint16), to_bf16(want["V"]))


def test_golden_fixture_bit_exact(gpu):
    f = np.load(os.path.join(GOLDEN, "prepass_rot_int8.npz"))
    H, hd, out_rows = int(f["H"]), int(f["hd"]), int(f["out_rows"])
    M = f["qkv_bf16"].shape[0]
    got = run_prepass(gpu, f["qkv_bf16"], "bf16", M=M, Hq=H, Hk=H, Hv=H, hd=hd, out_rows=out_rows)
    assert np.array_equal(got["Q"], f["Q"]) and np.array_equal(got["K"], f["K"])
    assert np.array_equal(got["qs"].view(np.uint32), f["qs"].view(np.uint32))
    assert np.array_equal(got["ks"].view(np.uint32), f["ks"].view(np.uint32))
    assert np.array_equal(got["V"][:, :M], f["qkv_bf16"].reshape(M, 3, H, hd)[:, 2].transpose(1, 0, 2))


@pytest.mark.parametrize("in_dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("qk_rot", [True, False])
@pytest.mark.parametrize("hd", [128, 64])
def test_int8_bit_exact(gpu, in_dt, qk_rot, hd):
    rng = np.random.default_rng(11)
    M, H = 97, 3
    x = outlier_rows(rng, M, H, hd)
    xh = to_bf16(x) if in_dt == "bf16" else x.astype(np.float16 if in_dt == "f16" else np.float32)
    got = run_prepass(gpu, xh, in_dt, M=M, Hq=H, Hk=H, Hv=H, hd=hd, out_rows=128, qk_rot=qk_rot)
    want = op.qk_norm_rope(as_float(xh, in_dt), Hq=H, Hk=H, Hv=H, hd=hd, out_rows=128, rot=0, eps=1e-6,
                           norm=False, q8=True, qk_rot=qk_rot)
    for n in ("Q", "K"):
        assert np.array_equal(got[n], want[n]), f"{n} codes differ at {np.argwhere(got[n] != want[n])[:5]}"
    for n in ("qs", "ks"):
        assert np.array_equal(got[n].view(np.uint32), want[n].view(np.uint32)), n


def test_int8_norm_rope_rotation_bit_exact(gpu):
    """The whole DiT recipe (dit.py:204-206): RMS norm, RoPE on 96 channels, rotation, int8."""
    rng = np.random.default_rng(12)
    M, H, hd, rot = 150, 4, 128, 96
    x = to_bf16((rng.standard_normal((M, 3 * H * hd)) * 2).astype(np.float32))
    wq, wk = rng.uniform(0.5, 1.5, (2, hd)).astype(np.float32)
    ang = rng.uniform(0, 6.28, (M, rot // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    got = run_prepass(gpu, x, "bf16", M=M, Hq=H, Hk=H, Hv=H, hd=hd, out_rows=256, rot=rot, norm=True, eps=1e-6,
                      wq=wq, wk=wk, cs=cs, sn=sn)
    want = op.qk_norm_rope(from_bf16(x), Hq=H, Hk=H, Hv=H, hd=hd, out_rows=256, rot=rot, eps=1e-6, norm=True,
                           wq=wq, wk=wk, cs=cs, sn=sn, q8=True, qk_rot=True)
    for n in ("Q", "K"):
        assert np.array_equal(got[n], want[n]), n
    for n in ("qs", "ks"):
        assert np.array_equal(got[n].view(np.uint32), want[n].view(np.uint32)), n


@pytest.mark.parametrize("hd,rot", [(128, 40), (64, 24), (64, 32), (128, 128)])
def test_norm_rope_both_lane_layouts_bit_exact(gpu, hd, rot):
    """8 channels per lane when rot/2 is a multiple of 8, else hd/32 per lane (the rotary pairs must stay
    lane-aligned): both layouts against the oracle, whose norm sum follows the same lane order."""
    rng = np.random.default_rng(hd + rot)
    M, H = 37, 3
    x = to_bf16((rng.standard_normal((M, 3 * H * hd)) * 2).astype(np.float32))
    wq, wk = rng.uniform(0.5, 1.5, (2, hd)).astype(np.float32)
    ang = rng.uniform(0, 6.28, (M, rot // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    got = run_prepass(gpu, x, "bf16", M=M, Hq=H, Hk=H, Hv=H, hd=hd, out_rows=64, rot=rot, norm=True, eps=1e-6,
                      wq=wq, wk=wk, cs=cs, sn=sn)
    want = op.qk_norm_rope(from_bf16(x), Hq=H, Hk=H, Hv=H, hd=hd, out_rows=64, rot=rot, eps=1e-6, norm=True,
                           wq=wq, wk=wk, cs=cs, sn=sn, q8=True, qk_rot=True)
    for n in ("Q", "K"):
        assert np.array_equal(got[n], want[n]), n
    for n in ("qs", "ks"):
        assert np.array_equal(got[n].view(np.uint32), want[n].view(np.uint32)), n


def test_half_outputs_like_reference_test_qk(gpu):
    """tests/test_ops.py::test_qk (:80-111): M=21, 56 heads each, hd=128, rot=96, norm, half outputs, against a
    float64 computation with the reference's tolerance; and exactly against the float32 oracle."""
    rng = np.random.default_rng(3)
    M, Hq, Hk, Hv, hd, rot = 21, 56, 56, 56, 128, 96
    S = Hq + Hk + Hv
    x = to_bf16((rng.standard_normal((M, S * hd)) * 2).astype(np.float32))
    xf = from_bf16(x).astype(np.float64)
    wq, wk = rng.uniform(0.5, 1.5, (2, hd)).astype(np.float32)
    ang = rng.uniform(0, 6.28, (M, rot // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    got = run_prepass(gpu, x, "bf16", M=M, Hq=Hq, Hk=Hk, Hv=Hv, hd=hd, out_rows=32, rot=rot, norm=True, eps=1e-5,
                      wq=wq, wk=wk, cs=cs, sn=sn, q8=False, qk_rot=False, qk_dt="f16", v_dt="f16")

    def ref(hh, w):
        v = hh / np.sqrt((hh ** 2).mean(-1, keepdims=True) + 1e-5) * w
        r = rot // 2
        x1, x2 = v[..., :r].copy(), v[..., r:2 * r].copy()
        v = v.copy()
        v[..., :r] = x1 * cs[:, None, :] - x2 * sn[:, None, :]
        v[..., r:2 * r] = x2 * cs[:, None, :] + x1 * sn[:, None, :]
        return v
    xs = xf.reshape(M, S, hd)
    q_ref, k_ref, v_ref = ref(xs[:, :Hq], wq), ref(xs[:, Hq:Hq + Hk], wk), xs[:, Hq + Hk:]
    eq = np.abs(got["Q"][:, :M].transpose(1, 0, 2) - q_ref).max()
    ek = np.abs(got["K"][:, :M].transpose(1, 0, 2) - k_ref).max()
    ev = np.abs(got["V"][:, :M].transpose(1, 0, 2) - v_ref).max()
    assert max(eq, ek) < 5e-3 * max(1, np.abs(q_ref).max()) and ev < 2e-2
    want = op.qk_norm_rope(from_bf16(x), Hq=Hq, Hk=Hk, Hv=Hv, hd=hd, out_rows=32, rot=rot, eps=1e-5, norm=True,
                           wq=wq, wk=wk, cs=cs, sn=sn)
    assert np.array_equal(got["Q"], want["Q"].astype(np.float16))
    assert np.array_equal(got["K"], want["K"].astype(np.float16))


def test_batched_sequences(gpu):
    """seq_len batching (ops.metal:381,448): rows of several sequences, heads per sequence, rotary tables per
    row of a sequence."""
    rng = np.random.default_rng(13)
    M, H, hd, rot, seq_len = 70, 2, 128, 32, 32
    x = to_bf16(rng.standard_normal((M, 3 * H * hd)).astype(np.float32))
    ang = rng.uniform(0, 6.28, (seq_len, rot // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    ones = np.ones(hd, np.float32)
    got = run_prepass(gpu, x, "bf16", M=M, Hq=H, Hk=H, Hv=H, hd=hd, out_rows=32, rot=rot, norm=True, seq_len=seq_len,
                      wq=ones, wk=ones, cs=cs, sn=sn)
    want = op.qk_norm_rope(from_bf16(x), Hq=H, Hk=H, Hv=H, hd=hd, out_rows=32, rot=rot, eps=1e-6, norm=True,
                           wq=ones, wk=ones, cs=cs, sn=sn, seq_len=seq_len, q8=True, qk_rot=True)
    for n in ("Q", "K", "qs", "ks"):
        assert np.array_equal(got[n], want[n]), n
    assert np.array_equal(got["V"].view(np.uint16), to_bf16(want["V"]))


def test_zero_rows_scale_one(gpu):
    x = np.zeros((5, 3 * 128), np.uint16)
    got = run_prepass(gpu, x, "bf16", M=5, Hq=1, Hk=1, Hv=1, hd=128, out_rows=8)
    assert (got["Q"] == 0).all() and (got["qs"][:, :5] == 1).all() and (got["ks"][:, :5] == 1).all()


@pytest.mark.parametrize("mag", [1e-40, 1e-38, 1e-36, 1e-30, 3e-20, 1e4])
def test_tiny_and_large_rows_bit_exact(gpu, mag):
    """Rows whose scale is subnormal or whose reciprocal is out of range (amax below ~2^-119) take the exact
    division for every value; ordinary magnitudes at both ends stay bit-exact too (f32 input, so the tiny
    values are representable)."""
    rng = np.random.default_rng(int(-np.log10(mag)) + 50)
    M, H = 9, 2
    x = (rng.standard_normal((M, 3 * H * 128)) * mag).astype(np.float32)
    got = run_prepass(gpu, x, "f32", M=M, Hq=H, Hk=H, Hv=H, hd=128, out_rows=16)
    want = op.qk_norm_rope(x, Hq=H, Hk=H, Hv=H, hd=128, out_rows=16, rot=0, eps=1e-6, norm=False, q8=True,
                           qk_rot=True)
    for n in ("Q", "K"):
        assert np.array_equal(got[n], want[n]), (n, mag, np.argwhere(got[n] != want[n])[:5])
    for n in ("qs", "ks"):
        assert np.array_equal(got[n].view(np.uint32), want[n].view(np.uint32)), (n, mag)


def test_config4_full_size_sampled_rows(gpu):
    """Benchmark config 4 at full size (H=32, S=16896): the kernel runs over all rows; the oracle checks a seeded
    sample of 512 rows bit for bit (the pre-pass is row-independent), and every row satisfies the int8
    invariants (max |code| = 127 for non-zero rows, dequantised rows within half a step of the rotated input's
    norm-preserving image)."""
    rng = np.random.default_rng(14)
    H, S, hd = 32, 16896, 128
    x = to_bf16(outlier_rows(rng, S, H, hd))
    got = run_prepass(gpu, x, "bf16", M=S, Hq=H, Hk=H, Hv=H, hd=hd, out_rows=S)
    rows = np.sort(rng.choice(S, 512, replace=False))
    want = op.qk_norm_rope(from_bf16(x[rows]), Hq=H, Hk=H, Hv=H, hd=hd, out_rows=len(rows), rot=0, eps=1e-6,
                           norm=False, q8=True, qk_rot=True)
    for n, s in (("Q", "qs"), ("K", "ks")):
        assert np.array_equal(got[n][:, rows], want[n]), n
        assert np.array_equal(got[s][:, rows].view(np.uint32), want[s].view(np.uint32)), s
        assert (np.abs(got[n]).max(-1) == 127).all()
    # norm preservation of the rotation, checked through the dequantised codes on every row of head 0
    xf = from_bf16(x).reshape(S, 3, H, hd)
    deq = got["Q"][0].astype(np.float64) * got["qs"][0][:, None]
    n_in = np.linalg.norm(xf[:, 0, 0].astype(np.float64), axis=-1)
    assert np.allclose(np.linalg.norm(deq, axis=-1), n_in, rtol=0.02)


def test_rotation_reduces_int8_attention_error(gpu):
    """tests/test_qk_rotation.py (:1-68): rows dominated by a few loud channels; with the rotation the int8
    attention's relative error is below 0.6x the plain one."""
    rng = np.random.default_rng(0)
    H, S, hd, rot = 4, 1000, 128, 96
    base = rng.standard_normal((3, H, S, hd))
    loud = rng.choice(hd, 8, replace=False)
    base[:2, :, :, loud] = base[:2, :, :, loud] * 12 + 20 * rng.standard_normal((2, H, 1, 8))
    q, k, v = base
    qkv = np.concatenate([q.transpose(1, 0, 2).reshape(S, -1), k.transpose(1, 0, 2).reshape(S, -1),
                          v.transpose(1, 0, 2).reshape(S, -1)], 1).astype(np.float16)
    q, k, v = (a.astype(np.float16).astype(np.float64) for a in (q, k, v))
    pos = np.arange(S)[:, None] / 10000 ** (np.arange(rot // 2)[None] / (rot // 2))
    cs, sn = np.cos(pos).astype(np.float32), np.sin(pos).astype(np.float32)
    hr = rot // 2
    rq, rk = q.copy(), k.copy()
    for a in (rq, rk):
        a1, a2 = a[..., :hr].copy(), a[..., hr:rot].copy()
        a[..., :hr], a[..., hr:rot] = a1 * cs - a2 * sn, a2 * cs + a1 * sn
    ref = oa.ref_attention(rq, rk, v, hd ** -0.5).reshape(S, H, hd).transpose(1, 0, 2)
    Sp = -(-S // 64) * 64
    errs = {}
    for qk_rot in (False, True):
        pre = run_prepass(gpu, qkv, "f16", M=S, Hq=H, Hk=H, Hv=H, hd=hd, out_rows=Sp, rot=rot, norm=False,
                          qk_rot=qk_rot, cs=cs, sn=sn, v_dt="f16")
        Q, K = gpu.upload(pre["Q"]), gpu.upload(pre["K"])
        V = gpu.upload(pre["V"])
        qs, ks = gpu.upload(pre["qs"]), gpu.upload(pre["ks"])
        o = gpu.empty((Sp, H * hd), "f16")
        ops.attention(gpu, Q, K, V, o, Lq=S, L=S, H=H, KVH=H, D=hd, q_rows=Sp, k_rows=Sp, scale=hd ** -0.5, wm=10,
                      bk=32, DB=1, PVORDER=1, VX=1, q_scale=qs, k_scale=ks)
        gpu.wait()
        got = o.numpy()[:S].astype(np.float64).reshape(S, H, hd).transpose(1, 0, 2)
        errs[qk_rot] = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    print("relative errors", errs)
    assert errs[True] < 0.6 * errs[False], errs


def test_per_stream_row_offset_views(gpu):
    """FLUX.2's double-stream blocks (h3metal/flux2.py:417-426) run the pre-pass once per stream, text rows then
    image rows, each writing into the shared Q/K/V and scale buffers through views offset by r0 rows, with the
    rotary tables' rows r0 .. r0 + M. Two calls must equal the oracle over all rows."""
    rng = np.random.default_rng(15)
    H, hd, T, Mi, rot = 3, 128, 40, 88, 128
    S = T + Mi
    Sp = 256
    x = to_bf16((rng.standard_normal((S, 3 * H * hd)) * 1.5).astype(np.float32))
    wq, wk = rng.uniform(0.5, 1.5, (2, hd)).astype(np.float32)
    ang = rng.uniform(0, 6.28, (S, rot // 2))
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    Q, K = gpu.empty((H, Sp, hd), "i8"), gpu.empty((H, Sp, hd), "i8")
    V = gpu.empty((H, Sp, hd), "bf16")
    qs, ks = gpu.empty((H, Sp), "f32"), gpu.empty((H, Sp), "f32")
    Wq, Wk, Cs, Sn = gpu.upload(wq), gpu.upload(wk), gpu.upload(cs), gpu.upload(sn)
    for r0, M in ((0, T), (T, Mi)):  # two streams, separate source tensors
        src = gpu.upload(x[r0:r0 + M], "bf16")
        ops.qk_norm_rope(gpu, src, Wq, Wk, Cs.row(r0, M), Sn.row(r0, M), Q.view(Q.shape, offset_elems=r0 * hd),
                         K.view(K.shape, offset_elems=r0 * hd), V.view(V.shape, offset_elems=r0 * hd), M=M, Hq=H, Hk=H,
                         Hv=H, hd=hd, out_rows=Sp, rot=rot, eps=1e-6, in_stride=3 * H * hd,
                         q_scale=qs.view(qs.shape, offset_elems=r0), k_scale=ks.view(ks.shape, offset_elems=r0),
                         qk_rot=True)
    gpu.wait()
    want = op.qk_norm_rope(from_bf16(x), Hq=H, Hk=H, Hv=H, hd=hd, out_rows=Sp, rot=rot, eps=1e-6, norm=True, wq=wq,
                           wk=wk, cs=cs, sn=sn, q8=True, qk_rot=True)
    assert np.array_equal(Q.numpy(), want["Q"]) and np.array_equal(K.numpy(), want["K"])
    assert np.array_equal(qs.numpy().view(np.uint32), want["qs"].view(np.uint32))
    assert np.array_equal(ks.numpy().view(np.uint32), want["ks"].view(np.uint32))
    assert np.array_equal(V.numpy(), to_bf16(want["V"]))
