"""Algorithmic work of the prefill path, used to express measured times as rooflines.

FLOPs count only the two contractions (QK^T and PV, 2 flops per multiply-add each);
exp, scaling and the count multiply are not counted.

* Dense causal: every row i attends keys 0..i, so 4 * D * sum_i (i + 1) per (batch, head)
  = 2 * D * N * (N + 1) * B * Hq.
* Delta (hybrid): per (batch, query head, 128-row query block) the reference schedule
  (deltaFlashAttention.py:58-113) processes the packed anchors of the safe blocks --
  only real anchors (index < c) count -- for every valid row, plus the dense keys
  ds..i for row i:  4 * D * sum [ R * A + sum_i max(0, i - ds + 1) ].
* Compression bytes per (batch, kv head): read K (N * D * 2), read the V anchor rows
  (c * D * 2), write K-hat and V-hat (2 * c * D * 2), write timestamps and counts (8c).
"""
from __future__ import annotations

from typing import Dict

import numpy as np

BLOCK = 128


def hybrid_schedule(ts: np.ndarray, P: int, n_k: int, n_q: int, window: int):
    """(n_safe, last, ds) per (batch, kv head, query block) from the packed timestamps.

    ts: [B, Hkv, >=P] int.  Block maxima treat lanes at or beyond P as n_k + 1 and the
    safe prefix ends at the first block whose maximum is >= start_m - window.
    """
    ts = np.asarray(ts, dtype=np.int64)[:, :, :P]
    B, H = ts.shape[:2]
    nblk = (P + BLOCK - 1) // BLOCK
    padded = np.full((B, H, max(nblk, 1) * BLOCK), n_k + 1, dtype=np.int64)
    padded[:, :, :P] = ts
    bmax = padded.reshape(B, H, -1, BLOCK).max(-1)[:, :, :nblk]
    pmax = np.maximum.accumulate(bmax, axis=-1) if nblk else bmax
    nqb = (n_q + BLOCK - 1) // BLOCK
    thr = np.arange(nqb) * BLOCK - window
    n_safe = (pmax[:, :, None, :] < thr[None, None, :, None]).sum(-1) if nblk else np.zeros((B, H, nqb), np.int64)
    idx = np.clip(n_safe - 1, 0, max(nblk - 1, 0))
    last = np.where(n_safe > 0, np.take_along_axis(bmax, idx, axis=-1) if nblk else -1, -1)
    ds = np.maximum(0, ((last + 1) // BLOCK) * BLOCK)
    return n_safe, last, ds


def dense_flops(B: int, Hq: int, N: int, D: int, causal: bool = True) -> float:
    if causal:
        return 2.0 * D * N * (N + 1) * B * Hq
    return 4.0 * D * N * N * B * Hq


def hybrid_flops(ts: np.ndarray, anchor_counts: np.ndarray, P: int, n: int, Hq: int, D: int,
                 window: int) -> Dict[str, float]:
    """Algorithmic and executed FLOPs of the hybrid kernel for one layer (causal, Nq = Nk = n)."""
    n_safe, last, ds = hybrid_schedule(ts, P, n, n, window)
    B, Hkv, nqb = n_safe.shape
    G = Hq // Hkv
    c = np.asarray(anchor_counts, dtype=np.int64).reshape(B, Hkv, 1)
    real_anchors = np.minimum(n_safe * BLOCK, c)                    # A(qb)
    rows = np.minimum(BLOCK, n - np.arange(nqb) * BLOCK)[None, None]  # R(qb)
    start = np.arange(nqb)[None, None] * BLOCK
    # sum over rows i in [start, start + R) of (i - ds + 1)  (ds <= start always)
    first = start - ds + 1
    dense_pairs = rows * first + rows * (rows - 1) // 2
    pairs = (rows * real_anchors + dense_pairs).sum() * G
    alg = 4.0 * D * float(pairs)
    exe_pairs = (n_safe * BLOCK * BLOCK).sum() * G + ((start + BLOCK - ds) * BLOCK).sum() * G
    return {"algorithmic": alg, "executed_tiles": 4.0 * D * float(exe_pairs),
            "mean_n_safe": float(n_safe.mean()), "mean_dense_keys": float((start + BLOCK - ds).mean())}


def compression_bytes(N: int, D: int, anchor_counts: np.ndarray) -> float:
    c = np.asarray(anchor_counts, dtype=np.float64)
    return float((N * D * 2 + c * D * 2 + 2 * c * D * 2 + 8 * c).sum())
