"""float32 op-by-op restatement of the queries/keys pre-pass qk_norm_rope.

Test infrastructure only (see oracle/__init__.py).

Follows the reference kernel kernels/ops.metal:365-468 (parameters :344-349,
launcher h3metal/ops.py:225-239) step by step, every step one IEEE-rounded
float32 numpy operation, in the order the gfx950 kernel performs it:

  load          float(in)                                         ops.metal:385-389
  RMS norm      ss = per-lane running sum of v*v (8 channels/lane when
                rot/2 is a multiple of 8, else hd/32), then an xor
                butterfly over the slot's lanes (halving strides);
                v = (v * (1 / sqrt(ss / HDIM + eps))) * w          ops.metal:394-402
  RoPE          v_c c_c - v_{c+h} s_c ; v_{c+h} c_c + v_c s_c      ops.metal:403-419
  signs         v_c = -v_c if popcount(c * 0x2545F491) is odd       ops.metal:424-428
  FWHT          stages over channel bits 0..6 in increasing order,
                (a + b, a - b) with a the lower channel             ops.metal:430-443
  normalise     v * fl32(1/sqrt(HDIM))                               ops.metal:444-446
  int8          scale = amax/127 (1 if amax == 0); rint(v / scale)  ops.metal:450-458

Pinning status: the rotation, signs and int8 steps are pinned by closed forms
and invariants in tests/test_oracle.py (Hadamard matrix product, orthonormality,
one-hot inputs, amax/127 round trip); the order of signs and transform by the
one-hot images s_c * H[c, :] / sqrt(n), which the swapped order fails. The order of the RMS-norm sum is this
build's (Metal's simd_sum order is unspecified), so the norm's last-ulp
behaviour is pinned against the gfx950 kernel and against float64 within
tolerance only, not against the reference (parity unpinned at the last ulp).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
SIGN_MULT = 0x2545F491


def hash_signs(hdim: int) -> np.ndarray:
    """+1/-1 per channel: -1 where popcount((c * 0x2545F491) mod 2^32) is odd (ops.metal:427)."""
    c = np.arange(hdim, dtype=np.uint64)
    prod = (c * np.uint64(SIGN_MULT)) & np.uint64(0xFFFFFFFF)
    bits = np.array([bin(int(x)).count("1") & 1 for x in prod])
    return np.where(bits == 1, F32(-1), F32(1)).astype(F32)


def inv_sqrt_f32(n: int) -> np.float32:
    """The correctly rounded float32 of 1/sqrt(n)."""
    return F32(1.0 / np.sqrt(np.float64(n)))


def fwht_f32(v: np.ndarray) -> np.ndarray:
    """Unnormalised Walsh-Hadamard transform over the last axis, stages in increasing bit order, float32."""
    v = np.ascontiguousarray(v, dtype=F32)
    n = v.shape[-1]
    lead = v.shape[:-1]
    s = 1
    while s < n:
        x = v.reshape(lead + (n // (2 * s), 2, s))
        a, b = x[..., 0, :], x[..., 1, :]
        v = np.stack([a + b, a - b], axis=-2).reshape(lead + (n,))
        s *= 2
    return v


def rotate_f32(v: np.ndarray) -> np.ndarray:
    """The QKROT rotation: signs, FWHT, times fl32(1/sqrt(n)) (ops.metal:420-446)."""
    n = v.shape[-1]
    return fwht_f32(v.astype(F32) * hash_signs(n)) * inv_sqrt_f32(n)


def quant_i8(v: np.ndarray):
    """Per-row symmetric int8 (ops.metal:450-458): returns (codes int8, scale float32)."""
    v = v.astype(F32)
    amax = np.abs(v).max(-1)
    scale = np.where(amax > 0, amax / F32(127), F32(1)).astype(F32)
    codes = np.rint(v / scale[..., None]).astype(np.int8)
    return codes, scale


def lanes_per_slot(hd: int, rot: int) -> int:
    """The gfx950 kernel's lane group per (row, head): 8 channels per lane (hd/8 lanes) when the rotary pairs
    (c, c + rot/2) stay lane-aligned, i.e. rot/2 is a multiple of 8; else 32 lanes (hd/32 channels each)."""
    return hd // 8 if (rot // 2) % 8 == 0 else 32


def rms_norm_f32(v: np.ndarray, w: np.ndarray, eps: float, lanes: int = 32) -> np.ndarray:
    """RMS norm in the gfx950 kernel's order: per-lane partial sums over hd/lanes consecutive channels, then an
    xor butterfly over the `lanes` lanes (strides lanes/2 .. 1)."""
    v = v.astype(F32)
    hd = v.shape[-1]
    per = hd // lanes
    grp = v.reshape(v.shape[:-1] + (lanes, per))
    ss = grp[..., 0] * grp[..., 0]
    for i in range(1, per):
        ss = ss + grp[..., i] * grp[..., i]
    idx = np.arange(lanes)
    s = lanes // 2
    while s >= 1:
        ss = ss + ss[..., idx ^ s]
        s //= 2
    tot = ss[..., 0]
    inv = F32(1) / np.sqrt(tot / F32(hd) + F32(eps))
    return (v * inv[..., None]) * w.astype(F32)


def rope_f32(v: np.ndarray, cs: np.ndarray, sn: np.ndarray, rot: int) -> np.ndarray:
    """Half-split rotary embedding of the first `rot` channels; cs, sn broadcast against v[..., :rot//2]."""
    h = rot // 2
    out = v.astype(F32).copy()
    a, b = v[..., :h].astype(F32), v[..., h:rot].astype(F32)
    c, s = cs.astype(F32), sn.astype(F32)
    out[..., :h] = a * c - b * s
    out[..., h:rot] = b * c + a * s
    return out


def qk_norm_rope(x: np.ndarray, *, Hq: int, Hk: int, Hv: int, hd: int, out_rows: int, rot: int, eps: float,
                 norm: bool = True, wq=None, wk=None, cs=None, sn=None, seq_len: int | None = None,
                 q8: bool = False, qk_rot: bool = False):
    """The whole pre-pass on float32 input rows x [M][(Hq+Hk+Hv)*hd] (already the float value of the
    bf16/f16/f32 input). Returns dict with Q, K, V float32 [nseq*H][out_rows][hd] (zeros in unwritten rows)
    and, with q8, Q/K int8 codes plus qs/ks [nseq*H][out_rows] (scale 0 in unwritten rows)."""
    M = x.shape[0]
    seq_len = seq_len or M
    nseq = -(-M // seq_len) if M else 0
    slots = Hq + Hk + Hv
    xs = x.astype(F32).reshape(M, slots, hd)
    out = {}
    m = np.arange(M)
    sq, r = m // seq_len, m % seq_len

    def prep(v, w):
        if norm:
            v = rms_norm_f32(v, w, eps, lanes_per_slot(hd, rot))
        if rot:
            v = rope_f32(v, cs[r][:, None, :], sn[r][:, None, :], rot)
        if q8 and qk_rot:
            v = rotate_f32(v)
        return v

    for name, lo, nh, w in (("Q", 0, Hq, wq), ("K", Hq, Hk, wk)):
        v = prep(xs[:, lo:lo + nh], w)
        if q8:
            codes, sc = quant_i8(v)
            C = np.zeros((nseq * nh, out_rows, hd), np.int8)
            S = np.zeros((nseq * nh, out_rows), F32)
            for h in range(nh):
                C[sq * nh + h, r] = codes[:, h]
                S[sq * nh + h, r] = sc[:, h]
            out[name], out[name.lower() + "s"] = C, S
        else:
            T = np.zeros((nseq * nh, out_rows, hd), F32)
            for h in range(nh):
                T[sq * nh + h, r] = v[:, h]
            out[name] = T
    V = np.zeros((nseq * Hv, out_rows, hd), F32)
    for h in range(Hv):
        V[sq * Hv + h, r] = xs[:, Hq + Hk + h]
    out["V"] = V
    return out
