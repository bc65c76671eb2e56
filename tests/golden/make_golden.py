"""Writes the small golden fixtures of tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

The reference ships no golden vectors for this path (its kernels are Metal
code that cannot run here), so these fixtures freeze the oracle's output on
seeded inputs of the benchmark config-4 recipe (N(0,1) with 4 of 128 channels
per head x20, bf16) at a small size. tests/test_oracle.py checks that the
oracle still reproduces them; the GPU tests compare the HIP kernels with them.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import attention as oa  # noqa: E402
from oracle import prepass as op  # noqa: E402
from oracle.bf16 import from_bf16, to_bf16  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def outlier_qkv(rng, S, H, hd):
    """Fused rows [S][3*H*hd]: Q, K with 4 seeded channels per head scaled x20; V plain."""
    x = rng.standard_normal((S, 3, H, hd)).astype(np.float32)
    for part in (0, 1):
        for h in range(H):
            ch = rng.choice(hd, 4, replace=False)
            x[:, part, h, ch] *= 20
    return x.reshape(S, 3 * H * hd)


def main():
    rng = np.random.default_rng(1234)
    H, S, hd, out_rows = 2, 40, 128, 64
    qkv = to_bf16(outlier_qkv(rng, S, H, hd))
    out = op.qk_norm_rope(from_bf16(qkv), Hq=H, Hk=H, Hv=H, hd=hd, out_rows=out_rows, rot=0, eps=1e-6,
                          norm=False, q8=True, qk_rot=True)
    np.savez_compressed(os.path.join(HERE, "prepass_rot_int8.npz"), qkv_bf16=qkv, H=H, hd=hd, out_rows=out_rows,
                        Q=out["Q"], K=out["K"], qs=out["qs"], ks=out["ks"])
    S_int = oa.int_scores(out["Q"][:, :S], out["K"][:, :S])
    np.savez_compressed(os.path.join(HERE, "scores_int8.npz"), Q=out["Q"][:, :S], K=out["K"][:, :S], S=S_int)
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
