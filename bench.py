"""Attention throughput on one MI355X: the headline metric (attention TFLOP/s and % of the int8 MFMA peak at
H=32, D=128, S=16896; ms per call).

    python bench.py [--gpus 1] [--steps 20] [--warmup 10] [--config c4] [--no-cpu] [--extra c2,c3,c5]

A step is one attention call over the whole workload (all heads, all query rows) with its inputs resident in
HBM. The default workload is benchmark config 4: B=1, H=32, D=128, S=16896 (512 text + 16384 image rows), Q/K bf16
~N(0,1) with 4 of 128 channels per head x20, rotated and quantised to int8 by the fused pre-pass (timed
separately, reported under "prepass"), V bf16 ~N(0,1), int8 QK^T + bf16 P V. The attention output's consumer,
rot_q8 (256-block Hadamard + per-row int8 of O), is timed on the call's own output and reported under "rot_q8";
the int8 projections around attention (qkv, output) at the config's S and H*D under "gemm_q8". FLOPs follow the reference's
convention 4*H*Sq*Sk_valid*D (bench/attn_bench.py:27). The timed region is bracketed by stream
synchronisations; GPU time comes from HIP events on the library's stream (h3_wait), per-launch durations from
per-dispatch event pairs (profile mode). The other benchmark configs (--extra: configs 2, 3 and 5 by default) are
timed the same way in the same run and reported as extra keys of the line; the plain-copy yardstick of the
streaming kernels is the library's own device copy. One JSON line is printed.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK = {"int8": 5.0e15, "bf16": 2.5e15}  # MI355X dense MFMA peaks (ops/s)
HBM_PEAK = 8.0e12

CONFIGS = {
    # name: (H, D, S, L (valid keys), path)
    "c1": (4, 128, 256, 256, "bf16"),
    "c2": (24, 128, 4608, 4608, "bf16"),
    "c3": (30, 128, 4608, None, "bf16"),
    "c4": (32, 128, 16896, 16896, "int8"),
    "c5": (32, 128, 66048, 66048, "int8"),
}


def to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), rounded to nearest even; the synthetic inputs are finite."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def from_bf16(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def make_inputs(gpu, cfg, rng):
    """Device-resident inputs of one config. Returns (kwargs for ops.attention, prepass closure or None, L)."""
    from h3metal_amd import ops
    H, D, S, L, path = CONFIGS[cfg]
    if L is None:  # config 3: 4096 image rows, text padded to 512 with L_txt ~ U[32, 512] valid
        L = 4096 + int(rng.integers(32, 513))
    if path == "int8":
        X = gpu.empty((S, 3 * H * D), "bf16")
        chunk = 2048
        for r0 in range(0, S, chunk):  # generate in row chunks to bound host memory
            n = min(chunk, S - r0)
            x = rng.standard_normal((n, 3, H, D), dtype=np.float32)
            if r0 == 0:
                out_ch = [rng.choice(D, 4, replace=False) for _ in range(2 * H)]
            for part in (0, 1):
                for h in range(H):
                    x[:, part, h, out_ch[part * H + h]] *= 20
            X.write(to_bf16(x.reshape(n, -1)), offset_elems=r0 * 3 * H * D)
        Q, K = gpu.empty((H, S, D), "i8"), gpu.empty((H, S, D), "i8")
        V = gpu.empty((H, S, D), "bf16")
        qs, ks = gpu.empty((H, S), "f32"), gpu.empty((H, S), "f32")

        def prepass():
            ops.qk_norm_rope(gpu, X, None, None, None, None, Q, K, V, M=S, Hq=H, Hk=H, Hv=H, hd=D, out_rows=S,
                             rot=0, eps=1e-6, norm=False, q_scale=qs, k_scale=ks, qk_rot=True)
        prepass()
        gpu.wait()
        kw = dict(q=Q, k=K, v=V, q_scale=qs, k_scale=ks)
        return kw, prepass, L
    Q, K, V = (gpu.empty((H, S, D), "bf16") for _ in range(3))
    for t in (Q, K, V):
        for h in range(H):
            t.write(to_bf16(rng.standard_normal((S, D), dtype=np.float32)), offset_elems=h * S * D)
    return dict(q=Q, k=K, v=V), None, L


def head_inputs(kw, cfg, h, L):
    """Head h of the run's own device inputs as float32 host arrays: the int8 Q/K codes times their scales
    (what the GPU's scores dequantise to) or the bf16 Q/K, and the bf16 V."""
    H, D, S, _, _ = CONFIGS[cfg]

    def rows(t, n):
        return t.view((n, D), offset_elems=h * S * D).numpy()
    if "q_scale" in kw:
        q = rows(kw["q"], S).astype(np.float32) * kw["q_scale"].view((S,), offset_elems=h * S).numpy()[:, None]
        k = rows(kw["k"], L).astype(np.float32) * kw["k_scale"].view((L,), offset_elems=h * S).numpy()[:, None]
    else:
        q, k = from_bf16(rows(kw["q"], S)), from_bf16(rows(kw["k"], L))
    return q, k, from_bf16(rows(kw["v"], L))


def cpu_baseline(kw, cfg, L, budget_s=20.0):
    """The oracle's float32 numpy attention (query-chunked) on this run's own inputs, one head at a time at the
    config's full size, timed on this host and extrapolated linearly in H to the whole call. Heads are timed
    until ~budget_s seconds are spent."""
    from oracle.attention import attention_f32_chunked
    H, D, S, _, _ = CONFIGS[cfg]
    times = []
    t_start = time.perf_counter()
    while len(times) < H and (not times or time.perf_counter() - t_start < budget_s):
        q, k, v = head_inputs(kw, cfg, len(times), L)
        t0 = time.perf_counter()
        attention_f32_chunked(q, k, v, D ** -0.5, chunk=512)
        times.append(time.perf_counter() - t0)
    per_head = float(np.median(times))
    total = per_head * H
    threads = None
    try:
        from threadpoolctl import threadpool_info
        info = threadpool_info()
        threads = max((i.get("num_threads") or 0) for i in info) if info else None
    except Exception:  # noqa: BLE001
        pass
    return {"value": round(4.0 * H * S * L * D / total / 1e12, 4), "unit": "TFLOP/s",
            "cores": threads or 1, "host_cpus": os.cpu_count(), "kind": "port",
            "sample": f"heads 0..{len(times) - 1} of {H} of this run's own inputs "
                      f"({'dequantised int8 Q/K' if 'q_scale' in kw else 'bf16 Q/K'} + bf16 V as float32) at "
                      f"full size (Sq={S}, Sk={L}, D={D}), float32 numpy "
                      f"(BLAS sgemm + exp, 512-row query chunks), median head time {per_head:.3f} s, "
                      f"extrapolated x{H} heads = {total:.2f} s per call"}


def copy_rates(gpu, sizes, reps=10):
    """Bytes per second of a plain device-to-device copy moving the same traffic as each of `sizes` (n / 2 read,
    n / 2 written), through the library's own copy (h3_buffer_copy on its stream, timed per copy by HIP events):
    the HBM rate a streaming kernel of that size can reach on this part."""
    out = []
    for nb in sizes:
        n = int(nb) // 2
        src, dst = gpu.empty((n,), "u8"), gpu.empty((n,), "u8")
        for _ in range(3):
            src.copy_to(dst)
        gpu.wait()
        gpu.profile(True)
        for _ in range(reps):
            src.copy_to(dst)
        gpu.wait()
        t = float(np.mean([s for _, s in gpu.profile_take()]))
        gpu.profile(False)
        out.append(2 * n / t)
        del src, dst
    return out


def extra_config(gpu, cfg, steps, warmup):
    """ms per attention call, TFLOP/s and fraction of the MFMA peak of its score type at one more benchmark config
    (timed like the headline: HIP events on the library's stream over `steps` calls after `warmup`)."""
    from h3metal_amd import ops
    H, D, S, _, path = CONFIGS[cfg]
    kw, _, L = make_inputs(gpu, cfg, np.random.default_rng(1))
    O = gpu.empty((S, H * D), "bf16")

    def step():
        ops.attention(gpu, kw["q"], kw["k"], kw["v"], O, Lq=S, L=L, H=H, KVH=H, D=D, q_rows=S, k_rows=S,
                      scale=D ** -0.5, q_scale=kw.get("q_scale"), k_scale=kw.get("k_scale"))
    for _ in range(warmup):
        step()
    gpu.wait()
    for _ in range(steps):
        step()
    sec = gpu.wait() / steps
    flops = 4.0 * H * S * L * D
    peak = PEAK["int8" if path == "int8" else "bf16"]
    return {"workload": f"B=1 H={H} D={D} Sq={S} Sk_valid={L}, "
                        f"{'Hadamard-rotated int8 Q/K + bf16 V' if path == 'int8' else 'bf16 Q/K/V'}",
            "ms": round(sec * 1e3, 4), "TFLOP/s": round(flops / sec / 1e12, 1),
            "frac_peak": round(flops / sec / peak, 4), "peak": f"{'int8' if path == 'int8' else 'bf16'} "
                                                              f"{peak / 1e12:.0f} TFLOP/s", "steps": steps}


def traffic(kernel, cfg="c4"):
    """HBM bytes per launch of `kernel` at `cfg`, from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE runs
    (profiles/hbm_traffic_c4.md: the counters scaled by what they read for a plain copy of known size); None for
    other configs or when the profile is absent."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_{cfg}.json")
    if not os.path.exists(path) or CONFIGS_ARG.get("config") != cfg:
        return None
    with open(path) as f:
        d = json.load(f)
    return int(d[kernel]["traffic_bytes"]) if kernel in d else None


CONFIGS_ARG = {}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c4", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--extra", default="c2,c3,c5",
                    help="other configs timed in the same run and reported as extra keys ('' for none)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (to scale rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    CONFIGS_ARG["config"] = args.config
    if args.calibrate_copy:
        from h3metal_amd.gpu import Gpu
        gpu = Gpu()
        n = args.calibrate_copy * 2 ** 20
        src, dst = gpu.empty((n,), "u8"), gpu.empty((n,), "u8")
        src.copy_to(dst)
        gpu.wait()
        gpu.close()
        print(json.dumps({"calibrate_copy_bytes": n}))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs the attention path on a single MI355X (no multi-GPU "
              f"path), so --gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)

    from h3metal_amd import ops
    from h3metal_amd.gpu import Gpu

    H, D, S, _, path = CONFIGS[args.config]
    gpu = Gpu()
    rng = np.random.default_rng(0)
    kw, prepass, L = make_inputs(gpu, args.config, rng)
    O = gpu.empty((S, H * D), "bf16")


    def step():
        ops.attention(gpu, kw["q"], kw["k"], kw["v"], O, Lq=S, L=L, H=H, KVH=H, D=D, q_rows=S, k_rows=S,
                      scale=D ** -0.5, q_scale=kw.get("q_scale"), k_scale=kw.get("k_scale"))

    for _ in range(args.warmup):
        step()
    gpu.wait()
    # timed region: the stream is drained on both sides; GPU time from HIP events on the library's stream
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    gpu_s = gpu.wait()
    wall_s = time.perf_counter() - t0
    # per-launch durations (event pair per dispatch) for the roofline
    gpu.profile(True)
    for _ in range(args.steps):
        step()
    gpu.wait()
    launches = [t for _, t in gpu.profile_take()]
    gpu.profile(False)
    per_launch = float(np.mean(launches))
    flops = 4.0 * H * S * L * D
    ms = gpu_s / args.steps * 1e3
    value = flops / (gpu_s / args.steps) / 1e12
    peak = PEAK["int8" if path == "int8" else "bf16"]
    achieved = flops / per_launch
    out = {
        "metric": "attention TFLOP/s (% of MI355X MFMA peak) at H=32,D=128,S=16896; ms/call",
        "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 QK^T (int32 acc) + bf16 PV (fp32 acc)" if path == "int8" else "bf16 (fp32 acc)",
        "data": "synthetic (seeded N(0,1); config-4 outlier recipe)",
        "config": {"workload": f"{args.config}: B=1 H={H} D={D} Sq={S} Sk_valid={L}, non-causal, "
                               f"{'Hadamard-rotated int8 Q/K + bf16 V' if path == 'int8' else 'bf16 Q/K/V'}",
                   "global_batch": 1, "seq_len": S, "parallelism": "single GPU"},
        "pct_of_peak": round(100 * value * 1e12 / peak, 2),
        "wall_ms_per_step": round(wall_s / args.steps * 1e3, 4),
        "roofline": {"bound": "mfma", "achieved": round(achieved / 1e12, 2), "peak": peak / 1e12,
                     "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": traffic("attention_call"),
                     "kernel": "attention_wave_kernel (" +
                               ("int8 QK, bf16 PV" if path == "int8" else "bf16") + ") + attention_merge",
                     "per_launch_ms": round(per_launch * 1e3, 4)},
    }
    if prepass is not None:
        gpu.profile(True)
        for _ in range(args.steps):
            prepass()
        gpu.wait()
        pt = float(np.mean([t for _, t in gpu.profile_take()]))
        gpu.profile(False)
        # algorithmic bytes: read Q, K, V bf16; write Q, K int8, V bf16, one fp32 scale per Q/K row
        nbytes = S * 3 * H * D * 2 + 2 * S * H * D + S * H * D * 2 + 2 * S * H * 4
        out["prepass"] = {"ms": round(pt * 1e3, 4), "bytes": nbytes, "GB/s": round(nbytes / pt / 1e9, 1),
                          "frac_hbm": round(nbytes / pt / HBM_PEAK, 4), "traffic": traffic("qk_norm_rope_kernel")}
    # the attention output's consumer (h3metal/dit.py:209): rot_q8 of O [S][H*D] bf16 -> int8 + row scales
    a8, sa = gpu.empty((S, H * D), "i8"), gpu.empty((S,), "f32")
    ops.rot_q8(gpu, O, a8, sa, S, H * D)
    gpu.profile(True)
    for _ in range(args.steps):
        ops.rot_q8(gpu, O, a8, sa, S, H * D)
    gpu.wait()
    rt = float(np.mean([t for _, t in gpu.profile_take()]))
    gpu.profile(False)
    rbytes = S * H * D * 2 + S * H * D + S * 4
    out["rot_q8"] = {"ms": round(rt * 1e3, 4), "bytes": rbytes, "GB/s": round(rbytes / rt / 1e9, 1),
                     "frac_hbm": round(rbytes / rt / HBM_PEAK, 4), "traffic": traffic("rot_q8_kernel")}
    # the int8 projections around attention (h3metal/dit.py:200-215): qkv = A [S][H*D] x W^T [3*H*D] (bf16 out) and
    # the output projection added into the float residual stream (epi 1); random int8 codes and scales
    dm = H * D
    grng = np.random.default_rng(1)
    A8 = gpu.upload(grng.integers(-127, 128, size=(S, dm), dtype=np.int8))
    SA = gpu.upload(grng.uniform(1e-3, 1e-2, S).astype(np.float32))
    wq = ops.QWeight("q8", gpu.upload(grng.integers(-127, 128, size=(3 * dm, dm), dtype=np.int8)),
                     gpu.upload(grng.uniform(1e-3, 1e-2, 3 * dm).astype(np.float32)), 3 * dm, dm)
    wo = ops.QWeight("q8", gpu.upload(grng.integers(-127, 128, size=(dm, dm), dtype=np.int8)),
                     gpu.upload(grng.uniform(1e-3, 1e-2, dm).astype(np.float32)), dm, dm)
    QKV, X = gpu.empty((S, 3 * dm), "bf16"), gpu.empty((S, dm), "f32")
    RT, GT = gpu.empty((S,), "u8"), gpu.upload(np.ones((1, dm), np.float32))
    gl = {}
    for name, fn, n_out in (("qkv", lambda: ops.gemm(gpu, A8, wq, QKV, S, sa=SA), 3 * dm),
                            ("out", lambda: ops.gemm(gpu, A8, wo, X, S, sa=SA, epi=1, rtype=RT, gate=GT), dm)):
        fn()
        gpu.profile(True)
        for _ in range(args.steps):
            fn()
        gpu.wait()
        gt = float(np.mean([t for _, t in gpu.profile_take()]))
        gpu.profile(False)
        ops_n = 2.0 * S * n_out * dm
        gl[name] = {"M": S, "N": n_out, "K": dm, "ms": round(gt * 1e3, 4), "TOPS": round(ops_n / gt / 1e12, 1),
                    "frac_int8_peak": round(ops_n / gt / PEAK["int8"], 4)}
    out["gemm_q8"] = gl
    # the plain-copy HBM rate at the streaming kernels' traffic sizes: what a kernel that only moves these bytes
    # reaches on this part
    for key in ("prepass", "rot_q8"):
        if key in out:
            cr = copy_rates(gpu, [out[key]["bytes"]])[0]
            out[key]["copy_GB/s"] = round(cr / 1e9, 1)
            out[key]["frac_copy"] = round(out[key]["GB/s"] * 1e9 / cr, 4)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(kw, args.config, L, args.cpu_budget)
    # the other benchmark configs, timed in the same run (the headline stays the --config one)
    del kw, O, A8, QKV, X  # the headline workload's buffers
    for cfg in [c for c in args.extra.split(",") if c and c != args.config]:
        out[cfg] = extra_config(gpu, cfg, steps=4 if cfg == "c5" else args.steps, warmup=2 if cfg == "c5" else 5)
    gpu.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
