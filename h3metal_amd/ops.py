"""Launchers of the attention path: one Python function per GPU operation.

Drop-in for the launchers of the reference's h3metal/ops.py on the DiT
attention path, with the same arguments, buffer layouts, parameter blocks and
return value (None; results are valid after `gpu.wait()`):

  attention     <- h3metal/ops.py:177-191
  qk_norm_rope  <- h3metal/ops.py:225-239
  rot_q8        <- h3metal/ops.py:214-222 (the consumer of the attention output, h3metal/dit.py:209)
  QWeight, gemm <- h3metal/ops.py:19-34, 124-174 (the projections around attention; weight formats q8, h8,
                   f16, bf16)
  pad_rows      <- h3metal/ops.py:116-117

Element types come from the tensors, as in the reference (`OUT_DT`,
ops.py:17). The gfx950 kernels additionally accept bf16 Q/K/V (the reference's
attention inputs are half), passed to the kernel as the IN_T / QK_T / V_T
specialisations.
"""

from __future__ import annotations

from dataclasses import dataclass, replace

from .gpu import Gpu, Tensor, pack

OUT_DT = {"f16": "half", "bf16": "bfloat", "f32": "float"}
FMT_ID = {"q8": 1, "q4": 2, "q4g": 3, "f16": 4, "bf16": 5, "h8": 6, "h4": 7, "h4g": 8}  # h3metal/ops.py:15
GEMM_ACT = {"q8": "i8", "h8": "f16", "f16": "f16", "bf16": "bf16"}  # the formats built here and their activations
LOG2E = 1.4426950408889634


def pad_rows(m: int, tile: int = 128) -> int:
    return (m + tile - 1) // tile * tile


def attention(gpu: Gpu, q: Tensor, k: Tensor, v: Tensor, out: Tensor, *, Lq: int, L: int, H: int, KVH: int,
              D: int, q_rows: int, k_rows: int, scale: float, causal: bool = False, causal_off: int = 0,
              wm: int = 8, bk: int = 32, seq_heads: int | None = None, seq_rows: int = 0,
              q_scale: Tensor | None = None, k_scale: Tensor | None = None, **variant):
    """Per query head h: softmax over keys of (scale * q_i . k_j), the weights applied to the rows of v; with
    q_scale / k_scale the scores are int8 products dequantised by the two scales.

    q [H][q_rows][D], k and v [KVH][k_rows][D]; out rows (h // seq_heads) * seq_rows + i, columns
    (h % seq_heads) * D, row stride seq_heads * D. wm, bk and the reference's variant flags (DB, PVORDER, VX, KPAD,
    TG, SLACK) are tuning hints of the Metal kernel: accepted, and the gfx950 kernel uses its own tiles."""
    variant.pop("TG", None)
    q8 = q_scale is not None
    if q8 != (k_scale is not None):
        raise ValueError("attention: q_scale and k_scale go together")
    if q8 and (q.dtype != "i8" or k.dtype != "i8"):
        raise ValueError(f"attention: int8 scores need i8 q and k, got {q.dtype}, {k.dtype}")
    if not q8 and (q.dtype != k.dtype or q.dtype != v.dtype or q.dtype not in ("f16", "bf16")):
        raise ValueError(f"attention: q, k, v must all be f16 or all bf16, got {q.dtype}, {k.dtype}, {v.dtype}")
    if v.dtype not in ("f16", "bf16"):
        raise ValueError(f"attention: v must be f16 or bf16, got {v.dtype}")
    kern = gpu.kernel("attention", "attention", HD=D, WM=wm, BK=bk, CAUSAL=int(causal), O_T=OUT_DT[out.dtype],
                      QK8=int(q8), IN_T=OUT_DT[v.dtype], **variant)
    sh = seq_heads or H
    params = pack("7if3i", Lq, L, H, KVH, q_rows, k_rows, sh * D, scale * LOG2E, causal_off, sh, seq_rows)
    gpu.launch(kern, None, None, [q, k, v, out, None, q_scale, k_scale], params, params_index=4)


def attention_scores(gpu: Gpu, q: Tensor, k: Tensor, v: Tensor, scores: Tensor, *, Lq: int, L: int, H: int,
                     KVH: int, D: int, q_rows: int, k_rows: int, q_scale: Tensor | None = None,
                     k_scale: Tensor | None = None, out: Tensor | None = None, scale: float = 1.0, **variant):
    """Test hook (no reference counterpart): attention as ops.attention runs it, plus the raw score accumulators
    of its MFMAs, scores[h][i][j] = q_i . k_j (int32 for int8 inputs, f32 otherwise) for keys j < L. At D = 128
    without a causal mask the kernel that runs is ops.attention's own (same tiles, staging, tail split and
    P V), which then also writes `out` ([Lq][H * D] rows, as ops.attention with seq_heads = H). GROUPS=1 / 3
    select the wave-pipelined / paired kernel the same way; GROUPS=2 the two-group kernel, which writes the
    scores only."""
    q8 = q_scale is not None
    vt = v.dtype if v.dtype in ("f16", "bf16") else "bf16"
    if out is None:
        out = gpu.empty((Lq, H * D), vt)
    kern = gpu.kernel("attention", "attention_scores", HD=D, QK8=int(q8), IN_T=OUT_DT[vt], O_T=OUT_DT[out.dtype],
                      **variant)
    params = pack("7if3i", Lq, L, H, KVH, q_rows, k_rows, H * D, scale * LOG2E, 0, H, 0)
    gpu.launch(kern, None, None, [q, k, v, out, None, q_scale, k_scale, scores], params, params_index=4)


def qk_norm_rope(gpu: Gpu, qkv: Tensor, wq: Tensor | None, wk: Tensor | None, cos: Tensor | None,
                 sin: Tensor | None, Q: Tensor, K: Tensor, V: Tensor, *, M: int, Hq: int, Hk: int, Hv: int,
                 hd: int, out_rows: int, rot: int, eps: float, norm: bool = True, in_stride: int | None = None,
                 seq_len: int | None = None, q_scale: Tensor | None = None, k_scale: Tensor | None = None,
                 qk_rot: bool = False):
    """Per-head RMS norm and rotary embedding of queries and keys, split into head-major Q, K, V.

    qk_rot (with int8 outputs): queries and keys rotated by the same orthonormal Walsh-Hadamard matrix with
    fixed signs before their int8 rounding; their products, and attention, are unchanged, the rounding loses
    less. Q, K [heads][out_rows][hd] (i8 with q_scale / k_scale [heads][out_rows], else f16 / bf16), V likewise
    (f16 / bf16)."""
    q8 = int(q_scale is not None)
    if q8 and (Q.dtype != "i8" or K.dtype != "i8" or k_scale is None):
        raise ValueError("qk_norm_rope: int8 outputs need i8 Q and K and both scale tensors")
    qk_t = "half" if q8 else OUT_DT[Q.dtype]
    k = gpu.kernel("ops", "qk_norm_rope", NSG=8, HDIM=hd, IN_T=OUT_DT[qkv.dtype], QK8=q8,
                   QKROT=int(qk_rot and q8), QK_T=qk_t, V_T=OUT_DT[V.dtype])
    slots = Hq + Hk + Hv
    params = pack("8ifi", M, Hq, Hk, Hv, in_stride or slots * hd, out_rows, rot, int(norm), eps, seq_len or M)
    gpu.launch(k, None, None, [qkv, wq, wk, cos, sin, Q, K, V, None, q_scale, k_scale], params, params_index=8)


def _rows_kernel_cfg(D: int):
    """(NSG, MAXB) specialisation of the row kernels, chosen as in h3metal/ops.py:193-197: a row has D / 256
    rotation blocks, spread over at most 8 groups, each taking a ceiling share (NSG * MAXB * 256 >= D)."""
    blocks = D // 256
    groups = min(blocks, 8)
    return groups, (blocks + groups - 1) // groups


def rot_q8(gpu: Gpu, x: Tensor, out: Tensor, sa: Tensor | None, M: int, D: int, *, swiglu: bool = False,
           x_stride: int | None = None, out_hr: bool = False):
    """Rotates each row of x (or value * silu(gate), value in columns 0..D-1 and gate in D..2D-1 when swiglu)
    and rounds it to int8 codes with one float scale per row; out_hr keeps the rotated rows as half instead.
    The rotation multiplies every 256-column block by the
    orthonormal 256-point Walsh-Hadamard matrix. x [M][x_stride] (f16 / bf16 / f32), out [M][D] i8 (f16 with
    out_hr), sa [M] f32."""
    if D < 256 or D % 256:
        raise ValueError(f"rot_q8: D must be a positive multiple of 256, got {D}")
    nsg, maxb = _rows_kernel_cfg(D)
    k = gpu.kernel("ops", "rot_q8", NSG=nsg, MAXB=maxb, IN_T=OUT_DT[x.dtype], OUT_HR=int(out_hr))
    params = pack("4i", M, D, x_stride or (2 * D if swiglu else D), 1 if swiglu else 0)
    gpu.launch(k, None, None, [x, out, sa], params)


@dataclass
class QWeight:
    """A linear layer's weight on the GPU: W[N][K] in one of the reference's formats (h3metal/ops.py:19-34).
    This build runs "q8" and "h8" (int8 codes W[N][K] row-major, one float scale per output row sw[N]; int8 or
    half activations) and "f16" / "bf16" (W[N][K] half / bfloat, no scales)."""
    fmt: str
    w: Tensor
    sw: Tensor | None
    N: int
    K: int
    G: int = 128
    bias: Tensor | None = None
    ws: int | None = None  # row stride of the codes in elements, when it differs from K (a slice of K)
    low: object | None = None  # a low-rank term (LoRA): not built here

    @property
    def w_stride(self) -> int:
        return self.ws or self.K


def gemm(gpu: Gpu, a: Tensor, wt: QWeight, out: Tensor, M: int, *, sa: Tensor | None = None, epi: int = 0,
         rtype: Tensor | None = None, gate: Tensor | None = None, g_stride: int = 0, c_stride: int | None = None,
         a_stride: int | None = None, tile=(64, 128, 4), swz: int = 1, ksplit: int = 1, no_alloc: bool = False,
         _low=None):
    """out = A x W^T (epi 0), or out += gate[rtype] * (A x W^T) (epi 1, out float), plus bias[n]:
      q8:  A int8 [M][K] with row scales sa, W int8 codes, v = sa[m] * sw[n] * (a_m . w_n)
      h8:  A half, W int8 codes, v = sw[n] * (a_m . w_n)
      f16 / bf16: A and W half / bfloat, v = a_m . w_n

    ksplit: accumulate over that many consecutive slices of K in separate dispatches (epi 1 only), as the
    reference does. tile / swz are the Metal kernel's tile choices: checked as the reference checks them (the
    tile width must divide N) and otherwise unused (the gfx950 kernel uses 256 x 256 tiles and covers any N).
    no_alloc: dispatch through the allocation-free entry point (h3_dispatch_static); the h8 format's widened
    weights then live in its fixed scratch array."""
    if wt.fmt not in GEMM_ACT:
        raise NotImplementedError(f"gemm: weight format {wt.fmt!r} is not built (q8, h8, f16, bf16)")
    if a.dtype != GEMM_ACT[wt.fmt]:
        raise ValueError(f"gemm: format {wt.fmt} takes {GEMM_ACT[wt.fmt]} activations, got {a.dtype}")
    if wt.low is not None or _low is not None:
        raise NotImplementedError("gemm: low-rank (LoRA) terms are not built")
    if ksplit > 1:
        if epi != 1 or wt.fmt not in ("q8", "h8") or wt.K % (ksplit * 256):
            raise ValueError(f"cannot split K of a {wt.fmt} product (epi {epi}, K {wt.K}) {ksplit} ways")
        kp = wt.K // ksplit
        for i in range(ksplit):
            part = replace(wt, w=wt.w.view((wt.N, kp), offset_elems=i * kp), K=kp, ws=wt.w_stride,
                           bias=wt.bias if i == 0 else None)
            gemm(gpu, a.view((a.shape[0], kp), offset_elems=i * kp), part, out, M, sa=sa, epi=1, rtype=rtype,
                 gate=gate, g_stride=g_stride, c_stride=c_stride, a_stride=a_stride or wt.K, tile=tile, swz=swz,
                 no_alloc=no_alloc)
        return
    tm, tn, nsg = tile
    if wt.N % tn:
        raise ValueError(f"gemm tile {tile}: {tn} columns do not divide the product's {wt.N}")
    if wt.fmt == "q8" and sa is None:
        raise ValueError("gemm: int8 activations need their row scales sa")
    out_t = OUT_DT[out.dtype] if epi == 0 else "float"
    k = gpu.kernel("gemm", "gemm", WFMT=FMT_ID[wt.fmt], EPI=epi, OUT_T=out_t, TM=tm, TN=tn, NSG=nsg, G=wt.G,
                   HAS_BIAS=int(wt.bias is not None), SWZ=swz)
    if wt.fmt == "h8":
        gpu.reserve_workspace(wt.N * wt.K * 2)  # the widened weights; grows (and waits) only the first time
    m_pad = (M + tm - 1) // tm * tm
    params = pack("8i", m_pad, wt.N, wt.K, a_stride or wt.K, c_stride or wt.N, wt.w_stride, wt.K // wt.G,
                  g_stride or wt.N)
    gpu.launch(k, None, None, [a, wt.w, wt.sw, sa, out, wt.bias, rtype, gate], params, params_index=8,
               no_alloc=no_alloc)
