"""Host-side logic on the CPU: the C-ABI library loads and exports every symbol include/h3hip.h declares, the
Python launchers pack the reference's parameter blocks and buffer orders (h3metal/ops.py:177-191, 225-239), and
the runtime fails cleanly without a GPU. No kernel runs here."""

import ctypes
import os
import re
import struct

import numpy as np
import pytest

from h3metal_amd import gpu as G
from h3metal_amd import ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "h3hip.h")).read()
    text = re.sub(r"//.*", "", text)
    return sorted(set(re.findall(r"\b(h3_\w+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(G._find_library())
    names = header_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), n
    # and gpu.py binds exactly those
    assert sorted(G.SIGNATURES) == names


def test_open_without_gpu_fails_cleanly():
    if os.path.exists("/dev/kfd") and os.environ.get("HIP_VISIBLE_DEVICES", "") != "-1":
        pytest.skip("a GPU may be present")
    with pytest.raises(G.GpuError, match="device"):
        G.Gpu()


class FakeGpu:
    """Records what a launcher asks the runtime for."""

    def __init__(self):
        self.kernels, self.launches = [], []

    def kernel(self, file, fn, **macros):
        self.kernels.append((file, fn, macros))
        return (file, fn, tuple(sorted(macros.items())))

    def launch(self, k, grid, threads, args, params=b"", params_index=None, tg_mem=0, no_alloc=False):
        self.launches.append((k, args, params, params_index))


def T(shape, dtype):
    return G.Tensor(G.Buffer(0, 0), 0, tuple(shape), dtype)


def test_attention_launcher_packs_reference_params():
    g = FakeGpu()
    q, k = T((32, 256, 128), "i8"), T((32, 256, 128), "i8")
    v, o = T((32, 256, 128), "bf16"), T((256, 32 * 128), "bf16")
    qs, ks = T((32, 256), "f32"), T((32, 256), "f32")
    ops.attention(g, q, k, v, o, Lq=250, L=249, H=32, KVH=32, D=128, q_rows=256, k_rows=256, scale=128 ** -0.5,
                  wm=10, bk=32, DB=1, PVORDER=1, VX=1, TG=3, q_scale=qs, k_scale=ks)
    (file, fn, macros), = g.kernels
    assert (file, fn) == ("attention", "attention")
    assert macros["QK8"] == 1 and macros["O_T"] == "bfloat" and macros["HD"] == 128 and "TG" not in macros
    (_, args, params, pi), = g.launches
    assert pi == 4 and args[4] is None and args[5] is qs and args[6] is ks and args[:4] == [q, k, v, o]
    vals = struct.unpack("<7if3i", params)
    assert vals[:7] == (250, 249, 32, 32, 256, 256, 32 * 128) and vals[8:] == (0, 32, 0)
    assert abs(vals[7] - 128 ** -0.5 * 1.4426950408889634) < 1e-7  # scale in log2 units (ops.py:188)


def test_attention_launcher_rejects_mixed_types():
    g = FakeGpu()
    with pytest.raises(ValueError):
        ops.attention(g, T((1, 64, 128), "f16"), T((1, 64, 128), "bf16"), T((1, 64, 128), "f16"),
                      T((64, 128), "f16"), Lq=64, L=64, H=1, KVH=1, D=128, q_rows=64, k_rows=64, scale=0.1)
    with pytest.raises(ValueError):
        ops.attention(g, T((1, 64, 128), "i8"), T((1, 64, 128), "i8"), T((1, 64, 128), "f16"),
                      T((64, 128), "f16"), Lq=64, L=64, H=1, KVH=1, D=128, q_rows=64, k_rows=64, scale=0.1,
                      q_scale=T((1, 64), "f32"))


def test_qk_norm_rope_launcher_packs_reference_params():
    g = FakeGpu()
    qkv = T((100, 3 * 4 * 128), "bf16")
    Q, K, V = T((4, 128, 128), "i8"), T((4, 128, 128), "i8"), T((4, 128, 128), "bf16")
    qs, ks = T((4, 128), "f32"), T((4, 128), "f32")
    ops.qk_norm_rope(g, qkv, None, None, None, None, Q, K, V, M=100, Hq=4, Hk=4, Hv=4, hd=128, out_rows=128,
                     rot=96, eps=1e-6, norm=False, q_scale=qs, k_scale=ks, qk_rot=True)
    (file, fn, macros), = g.kernels
    assert (file, fn) == ("ops", "qk_norm_rope") and macros["QK8"] == 1 and macros["QKROT"] == 1
    assert macros["IN_T"] == "bfloat" and macros["V_T"] == "bfloat" and macros["HDIM"] == 128
    (_, args, params, pi), = g.launches
    assert pi == 8 and len(args) == 11 and args[8] is None and args[9] is qs and args[10] is ks
    vals = struct.unpack("<8ifi", params)
    assert vals[:8] == (100, 4, 4, 4, 12 * 128, 128, 96, 0) and vals[9] == 100
    # qk_rot without int8 outputs is ignored, as in the reference (QKROT=int(qk_rot and q8), ops.py:233)
    g2 = FakeGpu()
    ops.qk_norm_rope(g2, qkv, None, None, None, None, T((4, 128, 128), "f16"), T((4, 128, 128), "f16"), V, M=100,
                     Hq=4, Hk=4, Hv=4, hd=128, out_rows=128, rot=0, eps=1e-6, qk_rot=True)
    assert g2.kernels[0][2]["QKROT"] == 0 and g2.kernels[0][2]["QK_T"] == "half"


def test_rot_q8_launcher_packs_reference_params():
    """h3metal/ops.py:214-222: NSG/MAXB from the row length, IN_T from the input, pack("4i", M, D, x_stride,
    mode) with x_stride defaulting to 2D under swiglu; buffers [x, out, sa]."""
    g = FakeGpu()
    x, out, sa = T((19, 2 * 14336), "bf16"), T((19, 14336), "i8"), T((19,), "f32")
    ops.rot_q8(g, x, out, sa, 19, 14336, swiglu=True)
    ops.rot_q8(g, T((7, 4096), "f16"), T((7, 4096), "f16"), None, 7, 1024, x_stride=4096, out_hr=True)
    (f1, n1, m1), (f2, n2, m2) = g.kernels
    assert (f1, n1) == ("ops", "rot_q8") and m1 == {"NSG": 8, "MAXB": 7, "IN_T": "bfloat", "OUT_HR": 0}
    assert m2 == {"NSG": 4, "MAXB": 1, "IN_T": "half", "OUT_HR": 1}
    (_, a1, p1, i1), (_, a2, p2, i2) = g.launches
    assert a1 == [x, out, sa] and struct.unpack("<4i", p1) == (19, 14336, 2 * 14336, 1)
    assert a2[2] is None and struct.unpack("<4i", p2) == (7, 1024, 4096, 0)
    with pytest.raises(ValueError):
        ops.rot_q8(g, x, out, sa, 19, 1000)


def test_gemm_launcher_packs_reference_params():
    """h3metal/ops.py:124-174: macros WFMT/EPI/OUT_T/HAS_BIAS (+ the tile hints), pack("8i", m_pad, N, K, a_stride,
    c_stride, w_stride, K // G, g_stride), buffers [a, w, sw, sa, out, bias, rtype, gate], params index 8; K split
    into consecutive slices for the residual form."""
    g = FakeGpu()
    a, w, sw, sa = T((256, 4096), "i8"), T((12288, 4096), "i8"), T((12288,), "f32"), T((256,), "f32")
    out = T((256, 12288), "bf16")
    wt = ops.QWeight("q8", w, sw, 12288, 4096)
    ops.gemm(g, a, wt, out, 200, sa=sa)
    (f, n, m), = g.kernels
    assert (f, n) == ("gemm", "gemm") and m["WFMT"] == 1 and m["EPI"] == 0 and m["OUT_T"] == "bfloat"
    assert m["HAS_BIAS"] == 0
    (_, args, params, pi), = g.launches
    assert pi == 8 and args[:5] == [a, w, sw, sa, out] and args[5:] == [None, None, None]
    assert struct.unpack("<8i", params) == (256, 12288, 4096, 4096, 12288, 4096, 32, 12288)
    g2 = FakeGpu()
    x, rt, gate = T((256, 12288), "f32"), T((256,), "u8"), T((3, 12288), "f32")
    ops.gemm(g2, a, wt, x, 256, sa=sa, epi=1, rtype=rt, gate=gate, ksplit=4, tile=(64, 256, 8))
    assert len(g2.launches) == 4 and all(k[2]["EPI"] == 1 and k[2]["OUT_T"] == "float" for k in g2.kernels)
    offs = [args[1].offset for (_, args, _, _) in g2.launches]
    assert offs == [0, 1024, 2048, 3072]  # W slices of K / 4 columns
    assert all(struct.unpack("<8i", p)[2:4] == (1024, 4096) for (_, _, p, _) in g2.launches)  # K slice, a_stride
    with pytest.raises(ValueError):
        ops.gemm(g, a, wt, out, 200, sa=sa, tile=(32, 5000, 8))
    with pytest.raises(NotImplementedError):
        ops.gemm(g, a, ops.QWeight("q4g", w, sw, 12288, 4096), out, 200, sa=sa)


def test_pack_and_pad_rows():
    assert len(G.pack("7if3i", *range(7), 1.0, 0, 1, 2)) == 44  # sizeof(AttnParams), csrc/h3hip_internal.h
    assert len(G.pack("8ifi", *range(8), 1e-6, 5)) == 40         # sizeof(QkRopeParams)
    assert ops.pad_rows(16684) == 16768 and ops.pad_rows(16896) == 16896 and ops.pad_rows(1, 64) == 64


def test_tensor_views():
    t = T((10, 4), "f16")
    r = t.row(3, 2)
    assert r.offset == 3 * 4 * 2 and r.shape == (2, 4)
    v = t.view((5, 8), "i8", offset_elems=4)
    assert v.offset == 8 and v.dtype == "i8" and v.nbytes == 40


def test_lds_swizzles_cover_all_banks():
    """The LDS layouts of csrc/attention.hip (kswz, voff), restated: each is a permutation of a row's 16-byte
    pieces, and every read pass of the score MFMA's K operand (16 lanes of 16 bytes) and of the transposing V
    read (32 lanes of 8 bytes) touches each of the 64 four-byte banks exactly once."""
    def kswz(key, RB, NP):
        return (key // (256 // RB)) % NP

    def voff(key, pc, D):
        R = max(256 // (D * 2), 1)
        u = (pc >> 1) ^ (2 * ((key & 3) // R))
        return key * D * 2 + u * 32 + (pc & 1) * 16

    for D, RB in ((128, 128), (128, 256), (64, 64), (64, 128)):
        NP, VP = RB // 16, D * 2 // 16
        for key in range(64):
            assert sorted(p ^ kswz(key, RB, NP) for p in range(NP)) == list(range(NP))
            assert sorted(voff(key, pc, D) - key * D * 2 for pc in range(VP)) == [16 * i for i in range(VP)]
        for c in range(NP // 2):
            for h in (0, 1):
                for g in (0, 1):
                    banks = []
                    for a in range(16 * g, 16 * g + 16):
                        key = 16 * (a >> 4) + 8 * ((a >> 2) & 1) + 4 * ((a >> 3) & 1) + (a & 3)
                        addr = key * RB + (((2 * c + h) ^ kswz(key, RB, NP)) * 16)
                        banks += [(addr // 4 + i) % 64 for i in range(4)]
                    assert sorted(banks) == list(range(64))
        for db in range(D // 32):
            for h in (0, 1):
                banks = []
                for lane in range(32 * h, 32 * h + 32):
                    l16, l32 = lane & 15, lane & 31
                    addr = voff(8 * h + (l16 >> 2), (db * 32 + (l32 & 16)) // 8, D) + (l16 & 3) * 8
                    banks += [(addr // 4 + i) % 64 for i in range(2)]
                assert sorted(banks) == list(range(64))


def test_three_group_lds_direct_staging_layout():
    """The three-group attention kernel (csrc/attention.hip, attention3_kernel) stages K and V with LDS-direct
    loads: lane i of a load instruction writes LDS bytes m0 + 16 i .. + 15, so each lane must fetch the global
    piece that belongs at that swizzled position. Restated here: over a block's load instructions the written
    LDS bytes cover the K (8 KB) and V (16 KB) ring slots exactly once, and the piece that lands at each position
    is the one the operand reads (kswz / voff placement) expect there."""
    RB, D = 128, 128

    def kswz(key):
        return (key // 2) % 8

    def voff(key, pc):
        return key * 256 + ((pc >> 1) ^ (2 * (key & 3))) * 32 + (pc & 1) * 16

    # K: group 0, wave wl, round r: LDS chunk c = 4 r + wl of 1 KB
    k_written = {}
    for wl in range(4):
        for r in range(2):
            c = r * 4 + wl
            for lane in range(64):
                o = c * 1024 + 16 * lane
                row, slot = o >> 7, (o >> 4) & 7
                goff = row * RB + (slot ^ kswz(row)) * 16
                assert o not in k_written
                k_written[o] = goff
    assert sorted(k_written) == [16 * i for i in range(512)]
    for key in range(64):  # the read side: piece p of row key sits at key * RB + (p ^ kswz(key)) * 16
        for p in range(8):
            assert k_written[key * RB + ((p ^ kswz(key)) * 16)] == key * RB + p * 16
    # V: groups 1 and 2 (half = group - 1), wave wl, round r
    v_written = {}
    for half in range(2):
        for wl in range(4):
            for r in range(2):
                c = r * 4 + wl
                for lane in range(64):
                    o = half * 8192 + c * 1024 + 16 * lane
                    row, uu, sub = o >> 8, (o & 255) >> 5, (o >> 4) & 1
                    goff = row * (D * 2) + (2 * (uu ^ (2 * (row & 3))) + sub) * 16
                    assert o not in v_written
                    v_written[o] = goff
    assert sorted(v_written) == [16 * i for i in range(1024)]
    for key in range(64):
        for pc in range(16):
            assert v_written[voff(key, pc)] == key * (D * 2) + pc * 16
