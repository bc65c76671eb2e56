"""h3_dispatch_static, the entry point that allocates nothing (its scratch is a fixed 32 MiB array in the
library, one per GPU), against h3_dispatch on the same inputs: two attention calls in a row with a tail split
(the second one smaller), checked bit for bit against h3_dispatch's output and the int32 scores against exact
integer products; an h8 GEMM whose widened weights fit, bit for bit, and one whose weights do not, refused."""

import numpy as np
import pytest

from h3metal_amd import ops
from h3metal_amd.gpu import GpuError, pack
from oracle import attention as oa

pytestmark = pytest.mark.gpu

D = 128


def _inputs(gpu, H, S, seed):
    rng = np.random.default_rng(seed)
    qi = rng.integers(-127, 128, (H, S, D)).astype(np.int8)
    ki = rng.integers(-127, 128, (H, S, D)).astype(np.int8)
    v = rng.standard_normal((H, S, D)).astype(np.float32)
    vb = (v.view(np.uint32) >> 16).astype(np.uint16)
    qs = rng.uniform(1e-3, 2e-3, (H, S)).astype(np.float32)
    ks = rng.uniform(1e-3, 2e-3, (H, S)).astype(np.float32)
    T = dict(q=gpu.upload(qi, "i8"), k=gpu.upload(ki, "i8"), v=gpu.upload(vb, "bf16"), qs=gpu.upload(qs),
             ks=gpu.upload(ks))
    return T, qi, ki


def _attention(gpu, T, H, S, no_alloc, scores=None):
    O = gpu.empty((S, H * D), "bf16")
    if scores is None:
        k = gpu.kernel("attention", "attention", HD=D, QK8=1, IN_T="bfloat", O_T="bfloat")
        bufs = [T["q"], T["k"], T["v"], O, None, T["qs"], T["ks"]]
    else:
        k = gpu.kernel("attention", "attention_scores", HD=D, QK8=1, IN_T="bfloat", O_T="bfloat")
        bufs = [T["q"], T["k"], T["v"], O, None, T["qs"], T["ks"], scores]
    params = pack("7if3i", S, S, H, H, S, S, H * D, D ** -0.5 * ops.LOG2E, 0, H, 0)
    gpu.launch(k, None, None, bufs, params, params_index=4, no_alloc=no_alloc)
    gpu.wait()
    return O.numpy()


@pytest.mark.parametrize("H,S", [(1, 1024), (1, 700)])  # the second call smaller than the first
def test_static_attention_matches_dispatch(gpu, H, S):
    """Both entry points split the last round of tiles the same way at these shapes (the static scratch holds
    the split), so the outputs agree bit for bit; the scores hook through the static entry point gives exact
    int32 products."""
    T, qi, ki = _inputs(gpu, H, S, S)
    print(f"[no-alloc] attention H={H} S={S}", flush=True)
    want = _attention(gpu, T, H, S, no_alloc=False)
    got = _attention(gpu, T, H, S, no_alloc=True)
    assert np.array_equal(got, want)
    again = _attention(gpu, T, H, S, no_alloc=True)  # the array keeps the last call's contents: no effect
    assert np.array_equal(again, want)
    Sc = gpu.empty((H, S, S), "i32")
    out = _attention(gpu, T, H, S, no_alloc=True, scores=Sc)
    assert np.array_equal(Sc.numpy(), oa.int_scores(qi, ki))
    assert np.array_equal(out, want)


def test_static_h8_gemm(gpu):
    """The h8 GEMM's widened weights live in the static scratch: a product that fits matches h3_dispatch bit for
    bit; one that needs more than the 32 MiB is refused with the size it needs, although the context's own
    workspace (grown to 48 MiB) runs it through h3_dispatch."""
    rng = np.random.default_rng(3)
    M, N, K = 64, 256, 512
    a = gpu.upload(rng.standard_normal((M, K)).astype(np.float16))
    w = gpu.upload(rng.integers(-127, 128, (N, K)).astype(np.int8), "i8")
    sw = gpu.upload(rng.uniform(1e-3, 1e-2, N).astype(np.float32))
    k = gpu.kernel("gemm", "gemm", WFMT=6, EPI=0, OUT_T="half", TM=64, TN=128, NSG=4, G=128, HAS_BIAS=0, SWZ=1)

    def run(no_alloc, n, kk, wt, out):
        gpu.launch(k, None, None, [a, wt, sw, None, out, None, None, None],
                   pack("8i", M, n, kk, kk, n, kk, kk // 128, n), params_index=8, no_alloc=no_alloc)
        gpu.wait()
        return out.numpy()
    ws = gpu.workspace_bytes
    want = run(False, N, K, w, gpu.empty((M, N), "f16"))
    got = run(True, N, K, w, gpu.empty((M, N), "f16"))
    assert np.array_equal(got, want)
    # 40 MiB of widened weights: more than the 32 MiB static array, less than a context workspace of 48 MiB. The
    # ordinary entry point runs it; the allocation-free one refuses it (it never uses the context's workspace).
    gpu.reserve_workspace(48 << 20)
    ws = gpu.workspace_bytes
    assert ws >= 48 << 20
    Nb, Kb = 4096, 5120
    wb = gpu.upload(rng.integers(-127, 128, (Nb, Kb)).astype(np.int8), "i8")
    ab = gpu.upload(rng.standard_normal((M, Kb)).astype(np.float16))
    swb = gpu.upload(rng.uniform(1e-3, 1e-2, Nb).astype(np.float32))
    ob = gpu.empty((M, Nb), "f16")
    bufs = [ab, wb, swb, None, ob, None, None, None]
    params = pack("8i", M, Nb, Kb, Kb, Nb, Kb, Kb // 128, Nb)
    gpu.launch(k, None, None, bufs, params, params_index=8)
    gpu.wait()
    assert np.isfinite(ob.numpy().astype(np.float32)).all() and np.abs(ob.numpy().astype(np.float32)).max() > 0
    with pytest.raises(GpuError, match="bytes of scratch"):
        gpu.launch(k, None, None, bufs, params, params_index=8, no_alloc=True)
    assert gpu.workspace_bytes == ws  # the static calls neither used nor grew the context's workspace
