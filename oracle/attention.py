"""Reference attention on the CPU: float64 softmax attention and exact integer scores.

Test infrastructure only (see oracle/__init__.py).

ref_attention follows the reference's own oracle tests/test_attention.py:9-21
(per-head float64 softmax attention, grouped-query heads h // (H // KVH),
causal mask j > i + off) extended with the kernel's key-length mask (keys >= L,
kernels/attention.metal:234-246) and its output placement (rows
(h // seq_heads) * seq_rows + i, columns (h % seq_heads) * D,
attention.metal:384-385). The int8 path is compared, as the reference's
check_q8 does (tests/test_attention.py:89), against this float attention of
the DEQUANTISED int8 inputs codes * scale.

int_scores is the exact integer product of int8 codes (int64 accumulation;
|q . k| <= 128 * 127^2 < 2^31), the value the int32 MFMA accumulators must equal.

attention_f32_chunked is the same attention in float32 with query-row chunks
(as the reference's tests/ref/reference.py:162-170 chunks to bound memory):
the CPU baseline timed by bench.py.

Pinning: tests/test_oracle.py checks ref_attention against brute-force
per-row loops, softmax invariants (rows of P sum to 1; uniform keys give the
mean of V; a one-hot dominant key returns its value row) and int_scores
against Python integer dot products.
"""

from __future__ import annotations

import numpy as np


def ref_attention(q, k, v, scale, *, L=None, causal=False, off=0, seq_heads=None, seq_rows=0, out=None):
    """q [H][Lq][D], k, v [KVH][>=L][D] (any real dtype) -> out [rows][seq_heads*D] float64."""
    H, Lq, D = q.shape
    KVH = k.shape[0]
    L = k.shape[1] if L is None else L
    sh = seq_heads or H
    nseq = (H - 1) // sh + 1
    rows = (nseq - 1) * seq_rows + Lq
    if out is None:
        out = np.zeros((rows, sh * D))
    for h in range(H):
        kh = h // (H // KVH)
        s = q[h].astype(np.float64) @ k[kh, :L].T.astype(np.float64) * scale
        if causal:
            i = np.arange(Lq)[:, None]
            j = np.arange(L)[None, :]
            s = np.where(j > i + off, -np.inf, s)
        s -= s.max(1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(1, keepdims=True)
        seq = h // sh
        out[seq * seq_rows:seq * seq_rows + Lq, (h % sh) * D:(h % sh + 1) * D] = p @ v[kh, :L].astype(np.float64)
    return out


def int_scores(qi, ki, Lq=None, L=None, H_per_kv=1):
    """Exact q . k of int8 codes: qi [H][>=Lq][D], ki [KVH][>=L][D] -> int64 [H][Lq][L]."""
    H = qi.shape[0]
    Lq = qi.shape[1] if Lq is None else Lq
    L = ki.shape[1] if L is None else L
    out = np.empty((H, Lq, L), np.int64)
    for h in range(H):
        out[h] = qi[h, :Lq].astype(np.int64) @ ki[h // H_per_kv, :L].astype(np.int64).T
    return out


def attention_f32_chunked(q, k, v, scale, chunk=1024):
    """float32 softmax attention of one head: q [Lq][D], k, v [L][D] -> [Lq][D] (the CPU baseline)."""
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    out = np.empty((q.shape[0], v.shape[1]), np.float32)
    kt = np.ascontiguousarray(k.T)
    for i in range(0, q.shape[0], chunk):
        s = (q[i:i + chunk] @ kt) * np.float32(scale)
        s -= s.max(1, keepdims=True)
        np.exp(s, out=s)
        den = s.sum(1, keepdims=True)
        out[i:i + chunk] = (s @ v) / den
    return out
