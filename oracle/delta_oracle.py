"""CPU restatement of the DeltaAttention prefill math -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module (as the checker / the timed CPU baseline).  Every function cites
the reference file:line it restates (paths are relative to the reference
repository Emruur/DeltaAttention).

Shapes follow the reference: K, V are [B, Hkv, N, D]; Q and the output are
[B, Hq, N, D] with query head h reading KV head g = h // (Hq // Hkv), which is
the layout ``repeat_kv`` materialises (modeling_llama.py:223-232).

Deliberate definition (the reference's own is not reproducible): the
reference's Euclidean selection reduces ``diff * diff`` with Triton's
``tl.sum`` whose bf16 reduction order is internal to the Triton GPU backend
(tritonModules.py:56-58).  This build *defines* the selection distance as
fp32 arithmetic on the (exactly up-cast) key values, reduced by a perfect
pairwise tree over the head dimension zero-padded to 128 slots:
``t[j] = t[2j] + t[2j+1]`` level by level.  The HIP kernel computes exactly
this tree, so selection is bit-exact between the two.
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import numpy as np

BLOCK_M = 128  # logical query block of the hybrid kernel (modeling_llama.py:328)
BLOCK_N = 128  # logical key / packed-anchor block (modeling_llama.py:329)

__all__ = [
    "BLOCK_M", "BLOCK_N", "chunking", "tree_sum", "select_delta", "select_periodic",
    "index_map", "pack", "hybrid_schedule", "hybrid_attention", "hybrid_bruteforce",
    "dense_attention", "dense_bruteforce", "decode_update", "decode_attention",
    "to_bf16", "bf16_round", "f16_round",
]


# --------------------------------------------------------------------------------------
# bf16 helpers (round-to-nearest-even, as torch's .to(torch.bfloat16))
# --------------------------------------------------------------------------------------
def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even); returns float32."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    nan = np.isnan(a)
    if nan.any():
        out = np.where(nan, a, out)
    return out.reshape(np.shape(x))


to_bf16 = bf16_round


# --------------------------------------------------------------------------------------
# Stage 1: selection
# --------------------------------------------------------------------------------------
def chunking(seq_len: int, chunk_size: int = 0, divide_to: int = 0) -> Tuple[int, int]:
    """Chunk size and chunk count (modeling_llama.py:602-610)."""
    if seq_len <= 0:
        raise ValueError("seq_len must be positive")
    if chunk_size > 0:
        cs = min(chunk_size, seq_len)
        nc = max(1, (seq_len + cs - 1) // cs)
    else:
        parts = 1 if divide_to == 0 else divide_to
        cs = (seq_len + parts - 1) // parts
        nc = parts
    return cs, nc


def _tree_width(d: int) -> int:
    w = 128
    while w < d:
        w *= 2
    return w


def f16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest IEEE binary16 (ties to even, beyond 65504 to
    infinity); returns float32."""
    with np.errstate(over="ignore"):
        return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round16(x: np.ndarray, arith: str) -> np.ndarray:
    """x rounded to the 16-bit type named by ``arith`` ("bf16", "fp16"); "fp32" keeps it."""
    if arith == "bf16":
        return bf16_round(x)
    if arith == "fp16":
        return f16_round(x)
    return np.asarray(x, dtype=np.float32)


def tree_sum(x: np.ndarray, arith: str = "fp32") -> np.ndarray:
    """Perfect pairwise fp32 tree sum over the last axis, zero-padded to 128 slots
    (or the next power of two above 128).  This is the build's fixed reduction
    order for the selection distance (see module docstring).  With ``arith`` "bf16" /
    "fp16" every addition is rounded to that type."""
    x = np.asarray(x, dtype=np.float32)
    d = x.shape[-1]
    w = _tree_width(d)
    t = np.zeros(x.shape[:-1] + (w,), dtype=np.float32)
    t[..., :d] = x
    while t.shape[-1] > 1:
        t = round16(t[..., 0::2] + t[..., 1::2], arith)
    return t[..., 0]


def select_threshold(threshold: float, metric: str) -> np.float32:
    """Threshold as the kernel sees it: tau^2 for Euclidean, tau for cosine, passed as
    an fp32 kernel scalar (modeling_llama.py:639-642)."""
    use_cos = metric == "cosine"
    t = float(threshold) if use_cos else float(threshold) ** 2
    return np.float32(t)


def select_delta(k: np.ndarray, threshold: float, chunk_size: int = 512, divide_to: int = 0,
                 metric: str = "euclidean", arith: str = "fp32") -> Tuple[np.ndarray, np.ndarray]:
    """Delta-mode anchor selection (tritonModules.py:7-69, launch modeling_llama.py:634-653).

    Returns keep [B,H,N] int32 and chunk_counts [B,H,nc] int32.  Only the exact string
    "cosine" selects the cosine metric (modeling_llama.py:639-640); every other string is
    Euclidean.  ``arith`` "bf16" / "fp16" rounds the Euclidean distance's differences,
    squares and tree additions to that type, as the reference's Triton code computes
    curr - ref, diff * diff and tl.sum on 16-bit keys (tritonModules.py:55-58; the cosine
    branch upcasts to fp32 there, :48-54, and stays fp32 here).  Pure numpy loop; use
    ``select_oracle_c.select_delta`` for large inputs.
    """
    k32 = np.asarray(k, dtype=np.float32)
    B, H, N, D = k32.shape
    cs, nc = chunking(N, chunk_size, divide_to)
    use_cos = metric == "cosine"
    thr = select_threshold(threshold, metric)
    eps = np.float32(1e-8)
    keep = np.zeros((B, H, N), dtype=np.int32)
    counts = np.zeros((B, H, nc), dtype=np.int32)
    for b in range(B):
        for h in range(H):
            for c in range(nc):
                s = c * cs
                if s >= N:                      # tritonModules.py:34-35
                    continue
                e = min(s + cs, N)              # tritonModules.py:32
                keep[b, h, s] = 1               # tritonModules.py:41
                a = k32[b, h, s]
                a_norm = np.sqrt(tree_sum(a * a) + eps) if use_cos else None
                cnt = 1
                for i in range(s + 1, e):       # tritonModules.py:44
                    x = k32[b, h, i]
                    if use_cos:                 # tritonModules.py:48-54
                        dot = tree_sum(x * a)
                        nx = np.sqrt(tree_sum(x * x) + eps)
                        sim = np.float32(dot / np.float32(nx * a_norm))
                        kp = bool(sim < thr)
                    else:                       # tritonModules.py:55-58
                        diff = round16(x - a, arith)
                        kp = bool(tree_sum(round16(diff * diff, arith), arith) > thr)
                    if kp:                      # tritonModules.py:60-63
                        keep[b, h, i] = 1
                        a = x
                        if use_cos:
                            a_norm = np.sqrt(tree_sum(a * a) + eps)
                        cnt += 1
                counts[b, h, c] = cnt           # tritonModules.py:68-69
    return keep, counts


def select_periodic(batch: int, heads: int, seq_len: int, target_keep_rate: float) -> np.ndarray:
    """Periodic anchors pos % period == 0, period = max(1, round(1/rate)) with Python's
    banker's rounding (modeling_llama.py:626-632)."""
    period = max(1, round(1.0 / target_keep_rate))
    row = (np.arange(seq_len) % period == 0).astype(np.int32)
    return np.broadcast_to(row, (batch, heads, seq_len)).copy()


# --------------------------------------------------------------------------------------
# Stage 2: index, pack, counts
# --------------------------------------------------------------------------------------
def index_map(keep: np.ndarray) -> np.ndarray:
    """index_map = cumsum(keep) - 1 as int32 (modeling_llama.py:655)."""
    return (np.cumsum(np.asarray(keep, dtype=np.int64), axis=-1) - 1).astype(np.int32)


def pack(k: np.ndarray, v: np.ndarray, keep: np.ndarray) -> Dict[str, np.ndarray]:
    """Pack anchors into zero-padded K-hat, V-hat, timestamps and run-length counts.

    Restates modeling_llama.py:655-685 and tritonModules.py:72-132: P is the maximum
    anchor count over (batch, kv-head) (:656); K-hat/V-hat/ts are zero tensors of length
    P (:658-660) receiving row i at index_map[i] for every kept i, with ts = i
    (tritonModules.py:131-132); counts[index_map[i]] += 1 over every position i
    (:683-685), i.e. the run length of each anchor; padding stays 0.
    """
    keep = np.asarray(keep, dtype=np.int32)
    B, H, N = keep.shape
    if np.any(keep[..., 0] == 0):
        raise ValueError("position 0 must be an anchor (index_map would be -1)")
    c = keep.sum(axis=-1).astype(np.int32)
    P = int(c.max())
    D = k.shape[-1]
    kp = np.zeros((B, H, P, D), dtype=k.dtype)
    vp = np.zeros((B, H, P, D), dtype=v.dtype)
    ts = np.zeros((B, H, P), dtype=np.int32)
    cnt = np.zeros((B, H, P), dtype=np.int32)
    im = index_map(keep)
    for b in range(B):
        for h in range(H):
            pos = np.nonzero(keep[b, h])[0]
            n = pos.size
            kp[b, h, :n] = k[b, h, pos]
            vp[b, h, :n] = v[b, h, pos]
            ts[b, h, :n] = pos
            np.add.at(cnt[b, h], im[b, h], 1)
    return {"k_packed": kp, "v_packed": vp, "timestamps": ts, "counts": cnt,
            "anchor_counts": c, "P": P, "index_map": im}


# --------------------------------------------------------------------------------------
# Stage 3: hybrid attention schedule and kernels
# --------------------------------------------------------------------------------------
def hybrid_schedule(ts: np.ndarray, P: int, n_k: int, n_q: int, window: int
                    ) -> Tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """Per (batch, head, query block) Phase-1 length and Phase-2 range.

    Restates deltaFlashAttention.py:58-111: Phase 1 walks packed blocks of BLOCK_N anchors
    while ``start_n < P``; lanes at or beyond P read timestamp ``seq_len_k + 1`` (:70);
    the loop stops at the first block whose maximum timestamp is ``>= start_m - W``
    (:73-74); ``last`` is the maximum of the last accepted block (:101).  Phase 2 covers
    ``[max(0, ((last + 1) // BLOCK_N) * BLOCK_N), min(seq_len_k, start_m + BLOCK_M))``
    (:108-113).

    Returns (n_safe, last, dense_start, dense_hi), each [B, H, n_query_blocks] int64.
    """
    ts = np.asarray(ts, dtype=np.int64)
    B, H = ts.shape[:2]
    nqb = (n_q + BLOCK_M - 1) // BLOCK_M
    nblk = (P + BLOCK_N - 1) // BLOCK_N
    padded = np.full((B, H, nblk * BLOCK_N), n_k + 1, dtype=np.int64)
    padded[:, :, :P] = ts[:, :, :P]
    bmax = padded.reshape(B, H, nblk, BLOCK_N).max(axis=-1) if nblk else np.zeros((B, H, 0), np.int64)
    pmax = np.maximum.accumulate(bmax, axis=-1) if nblk else bmax
    n_safe = np.zeros((B, H, nqb), dtype=np.int64)
    last = np.full((B, H, nqb), -1, dtype=np.int64)
    for qb in range(nqb):
        thr = qb * BLOCK_M - window
        ns = (pmax < thr).sum(axis=-1)           # prefix maxima are non-decreasing
        n_safe[:, :, qb] = ns
        if nblk:
            idx = np.clip(ns - 1, 0, nblk - 1)
            lv = np.take_along_axis(bmax, idx[..., None], axis=-1)[..., 0]
            last[:, :, qb] = np.where(ns > 0, lv, -1)
    ds = np.maximum(0, ((last + 1) // BLOCK_N) * BLOCK_N)
    dh = np.minimum(n_k, np.arange(nqb) * BLOCK_M + BLOCK_M)[None, None, :].repeat(B, 0).repeat(H, 1)
    return n_safe, last, ds, dh


def _online_update(state, s, weights, vals, round_p):
    m, l, acc = state
    m_new = np.maximum(m, s.max(axis=1))
    with np.errstate(invalid="ignore"):
        p = np.exp(s - m_new[:, None]).astype(np.float32)
        alpha = np.exp(m - m_new).astype(np.float32)
    if weights is not None:
        p = (p * weights[None, :]).astype(np.float32)
    l = l * alpha + p.sum(axis=1, dtype=np.float32)
    pv = bf16_round(p) if round_p else p
    acc = acc * alpha[:, None] + pv @ vals
    return m_new, l.astype(np.float32), acc.astype(np.float32)


def hybrid_attention(q, k, v, kp, vp, ts, counts, window: int, scale: Optional[float] = None,
                     variant: str = "hybrid", no_count: bool = False, q_blocks=None,
                     heads=None, round_p: bool = False) -> np.ndarray:
    """Two-phase compressed flash prefill on the logical 128x128 schedule.

    variant "hybrid" restates hybrid_compressed_flash_kernel (deltaFlashAttention.py:9-146),
    "sanity" restates hybrid_compressed_flash_kernel_sanity (:149-259: Phase 1 decides
    ``last`` but adds nothing) and "pure_phase1" restates pure_phase1_flash_kernel
    (:262-357: every packed block, lane valid iff count > 0 and ts <= row, no Phase 2,
    rows with l == 0 give 0).  ``no_count`` sets every count, padding included, to 1
    (modeling_llama.py:323-324).  Counts are fp32 (:321).  fp32 online softmax; with
    ``round_p`` the weights are rounded to bf16 before P.V as the bf16 kernel does (:98).

    q [B,Hq,Nq,D]; k,v [B,Hkv,Nk,D]; kp,vp [B,Hkv,P,D]; ts,counts [B,Hkv,P].
    Returns float32 [B,Hq,Nq,D]; query blocks / heads not requested are NaN.
    """
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    kp = np.asarray(kp, dtype=np.float32)
    vp = np.asarray(vp, dtype=np.float32)
    B, Hq, Nq, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    P = kp.shape[2]
    if scale is None:
        scale = D ** -0.5
    scale = np.float32(scale)
    cnt = np.asarray(counts, dtype=np.float32)
    if no_count:
        cnt = np.ones_like(cnt)
    n_safe, last, ds, dh = hybrid_schedule(ts, P, Nk, Nq, window)
    nqb = (Nq + BLOCK_M - 1) // BLOCK_M
    q_blocks = range(nqb) if q_blocks is None else q_blocks
    heads = range(Hq) if heads is None else heads
    out = np.full((B, Hq, Nq, D), np.nan, dtype=np.float32)
    tsi = np.asarray(ts, dtype=np.int64)
    for b in range(B):
        for h in heads:
            g = h // G
            for qb in q_blocks:
                start_m = qb * BLOCK_M
                rows = start_m + np.arange(BLOCK_M)
                qblk = np.zeros((BLOCK_M, D), np.float32)
                nr = min(BLOCK_M, Nq - start_m)
                qblk[:nr] = q[b, h, start_m:start_m + nr]
                state = (np.full(BLOCK_M, -np.inf, np.float32), np.zeros(BLOCK_M, np.float32),
                         np.zeros((BLOCK_M, D), np.float32))
                if variant == "pure_phase1":
                    for jb in range((P + BLOCK_N - 1) // BLOCK_N):
                        idx = jb * BLOCK_N + np.arange(BLOCK_N)
                        inb = idx < P
                        safe_idx = np.where(inb, idx, 0)
                        c = np.where(inb, cnt[b, g, safe_idx], 0.0).astype(np.float32)
                        t = np.where(inb, tsi[b, g, safe_idx], Nk + 1)
                        kv_ok = (c > 0) & inb
                        ok = (t[None, :] <= rows[:, None]) & kv_ok[None, :]
                        kb = np.where(inb[:, None], kp[b, g, safe_idx], 0.0)
                        vb = np.where(inb[:, None], vp[b, g, safe_idx], 0.0)
                        s = (qblk @ kb.T) * scale
                        s = np.where(ok, s, -np.inf).astype(np.float32)
                        state = _online_update(state, s, c, vb, round_p)
                    m, l, acc = state
                    l_safe = np.where(l > 0, l, np.float32(1.0))
                    res = acc / l_safe[:, None]
                else:
                    for jb in range(int(n_safe[b, g, qb])):
                        idx = jb * BLOCK_N + np.arange(BLOCK_N)  # safe blocks lie inside [0, P)
                        if variant == "hybrid":
                            s = ((qblk @ kp[b, g, idx].T) * scale).astype(np.float32)
                            state = _online_update(state, s, cnt[b, g, idx], vp[b, g, idx], round_p)
                    for kn in range(int(ds[b, g, qb]), int(dh[b, g, qb]), BLOCK_N):
                        j = kn + np.arange(BLOCK_N)
                        inb = j < Nk
                        jj = np.where(inb, j, 0)
                        kb = np.where(inb[:, None], k[b, g, jj], 0.0)
                        vb = np.where(inb[:, None], v[b, g, jj], 0.0)
                        s = ((qblk @ kb.T) * scale).astype(np.float32)
                        ok = (rows[:, None] >= j[None, :]) & inb[None, :]
                        s = np.where(ok, s, -np.inf).astype(np.float32)
                        state = _online_update(state, s, None, vb, round_p)
                    m, l, acc = state
                    res = acc / l[:, None]
                out[b, h, start_m:start_m + nr] = res[:nr]
    return out


def hybrid_bruteforce(q, k, v, kp, vp, ts, counts, window: int, scale: Optional[float] = None,
                      variant: str = "hybrid", no_count: bool = False, q_blocks=None,
                      heads=None) -> np.ndarray:
    """Independent fp64 formulation: per query row an explicit weighted key multiset.

    hybrid: packed anchors [0, 128*n_safe) weighted by counts, plus dense keys
    [ds, row] (both phases, so tokens in [ds, last] are counted twice); sanity: only the
    dense keys; pure_phase1: anchors with count > 0 and ts <= row weighted by counts.
    out_row = sum_j w_j exp(s_j) v_j / sum_j w_j exp(s_j) with s_j = q.k_j * scale.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    kp = np.asarray(kp, dtype=np.float64)
    vp = np.asarray(vp, dtype=np.float64)
    B, Hq, Nq, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    P = kp.shape[2]
    scale = D ** -0.5 if scale is None else float(scale)
    cnt = np.asarray(counts, dtype=np.float64)
    if no_count:
        cnt = np.ones_like(cnt)
    tsi = np.asarray(ts, dtype=np.int64)
    n_safe, last, ds, dh = hybrid_schedule(ts, P, Nk, Nq, window)
    nqb = (Nq + BLOCK_M - 1) // BLOCK_M
    q_blocks = range(nqb) if q_blocks is None else q_blocks
    heads = range(Hq) if heads is None else heads
    out = np.full((B, Hq, Nq, D), np.nan, dtype=np.float64)
    for b in range(B):
        for h in heads:
            g = h // G
            for qb in q_blocks:
                for i in range(qb * BLOCK_M, min(Nq, qb * BLOCK_M + BLOCK_M)):
                    keys, vals, w = [], [], []
                    if variant == "pure_phase1":
                        sel = (cnt[b, g] > 0) & (tsi[b, g] <= i)
                        keys.append(kp[b, g, sel]); vals.append(vp[b, g, sel]); w.append(cnt[b, g, sel])
                    else:
                        if variant == "hybrid":
                            na = int(n_safe[b, g, qb]) * BLOCK_N
                            keys.append(kp[b, g, :na]); vals.append(vp[b, g, :na]); w.append(cnt[b, g, :na])
                        lo, hi = int(ds[b, g, qb]), min(i + 1, Nk)
                        keys.append(k[b, g, lo:hi]); vals.append(v[b, g, lo:hi]); w.append(np.ones(max(0, hi - lo)))
                    K_ = np.concatenate(keys) if keys else np.zeros((0, D))
                    V_ = np.concatenate(vals) if vals else np.zeros((0, D))
                    W_ = np.concatenate(w) if w else np.zeros(0)
                    if K_.shape[0] == 0 or not np.any(W_ > 0):
                        out[b, h, i] = 0.0
                        continue
                    s = K_ @ q[b, h, i] * scale
                    s = s - s[W_ > 0].max()
                    e = W_ * np.exp(s)
                    out[b, h, i] = (e @ V_) / e.sum()
    return out


def dense_attention(q, k, v, causal: bool = True, scale: Optional[float] = None,
                    q_blocks=None, heads=None) -> np.ndarray:
    """Dense flash prefill (flashAttention.py:5-91): causal rows attend keys j <= i in the
    128-block loop ``hi = min(N, (pid + 1) * 128)``; out-of-range keys get no weight.
    Exact (non-online) fp32 softmax per 128-row block; K/V heads are shared by groups of
    Hq // Hkv query heads (the reference passes repeat_kv-expanded K/V, :94-130)."""
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    B, Hq, Nq, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    scale = np.float32(D ** -0.5 if scale is None else scale)
    nqb = (Nq + BLOCK_M - 1) // BLOCK_M
    q_blocks = range(nqb) if q_blocks is None else q_blocks
    heads = range(Hq) if heads is None else heads
    out = np.full((B, Hq, Nq, D), np.nan, dtype=np.float32)
    for b in range(B):
        for h in heads:
            g = h // G
            for qb in q_blocks:
                r0 = qb * BLOCK_M
                r1 = min(Nq, r0 + BLOCK_M)
                hi = min(Nk, r1) if causal else Nk
                s = (q[b, h, r0:r1] @ k[b, g, :hi].T) * scale
                if causal:
                    rows = np.arange(r0, r1)[:, None]
                    s = np.where(np.arange(hi)[None, :] <= rows, s, -np.inf)
                s = s - s.max(axis=1, keepdims=True)
                e = np.exp(s)
                out[b, h, r0:r1] = (e @ v[b, g, :hi]) / e.sum(axis=1, keepdims=True)
    return out


def dense_bruteforce(q, k, v, causal: bool = True, scale: Optional[float] = None) -> np.ndarray:
    """Textbook fp64 softmax(Q K^T * scale + causal mask) V with shared K/V heads."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, Hq, Nq, D = q.shape
    G = Hq // k.shape[1]
    scale = D ** -0.5 if scale is None else float(scale)
    kk = np.repeat(k, G, axis=1)
    vv = np.repeat(v, G, axis=1)
    s = np.einsum("bhid,bhjd->bhij", q, kk) * scale
    if causal:
        mask = np.arange(kk.shape[2])[None, :] <= np.arange(Nq)[:, None]
        s = np.where(mask, s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    return np.einsum("bhij,bhjd->bhid", e, vv) / e.sum(axis=-1, keepdims=True)


# --------------------------------------------------------------------------------------
# Delta decoding (deltaDecoding.py)
# --------------------------------------------------------------------------------------
def decode_update(state: Dict[str, np.ndarray], new_k: np.ndarray, new_v: np.ndarray,
                  threshold: float, metric: str = "euclidean") -> None:
    """One decode step of fused_hybrid_decode_update_kernel (deltaDecoding.py:9-104) plus
    the host-side tracker updates of HybridCompressedCache.update (:181-227), in place.

    state: k_packed/v_packed [B,H,cap,D], counts/timestamps [B,H,cap] int32,
    lengths [B*H] int32, k_exact/v_exact [B,H,W,D], plus python ints exact_len,
    total_len, window.  new_k/new_v [B,H,1,D].  The merge test is fp32 with the same
    fixed tree reduction as the selection: Euclidean merges iff dist^2 <= tau^2
    (:74-76), cosine merges iff cos >= tau (:67-72).
    """
    use_cos = metric == "cosine"
    thr = select_threshold(threshold, metric)
    eps = np.float32(1e-8)
    W = state["window"]
    el, tl = state["exact_len"], state["total_len"]
    kx, vx = state["k_exact"], state["v_exact"]
    kp, vp = state["k_packed"], state["v_packed"]
    cnt, tss, lens = state["counts"], state["timestamps"], state["lengths"]
    B, H = kx.shape[:2]
    widx = el % W                                   # :35
    for b in range(B):
        for h in range(H):
            pid = b * H + h
            if el >= W:                             # :54
                ek = kx[b, h, widx].copy()
                ev = vx[b, h, widx].copy()
                plen = int(lens[pid])
                merge = False
                if plen > 0:                        # :61-77
                    lk = kp[b, h, plen - 1].astype(np.float32)
                    e32 = ek.astype(np.float32)
                    if use_cos:
                        dot = tree_sum(e32 * lk)
                        ne = np.sqrt(tree_sum(e32 * e32) + eps)
                        nl = np.sqrt(tree_sum(lk * lk) + eps)
                        merge = bool(np.float32(dot / np.float32(ne * nl)) >= thr)
                    else:
                        d = e32 - lk
                        merge = bool(tree_sum(d * d) <= thr)
                if merge:                           # :78-82
                    cnt[b, h, plen - 1] += 1
                else:                               # :83-96
                    kp[b, h, plen] = ek
                    vp[b, h, plen] = ev
                    cnt[b, h, plen] = 1
                    tss[b, h, plen] = tl - W
                    lens[pid] = plen + 1
            kx[b, h, widx] = new_k[b, h, 0]         # :101-104
            vx[b, h, widx] = new_v[b, h, 0]
    state["exact_len"] = el + 1                      # :224-225
    state["total_len"] = tl + 1


def decode_attention(q: np.ndarray, state: Dict[str, np.ndarray], scale: Optional[float] = None,
                     round_p: bool = False) -> np.ndarray:
    """fused_hybrid_decode_kernel (deltaDecoding.py:236-362): one query per head attends
    the packed cache of its KV head with score + log(count) over the head's own packed
    length (:297-325), then the first min(exact_len, W) ring slots with no causal mask
    (:330-349, exact_len clamp at modeling_llama.py:476-479).  q [B,Hq,D] -> [B,Hq,D]."""
    q = np.asarray(q, dtype=np.float32)
    B, Hq, D = q.shape
    kp = state["k_packed"].astype(np.float32)
    vp = state["v_packed"].astype(np.float32)
    kx = state["k_exact"].astype(np.float32)
    vx = state["v_exact"].astype(np.float32)
    H = kp.shape[1]
    G = Hq // H
    scale = np.float32(D ** -0.5 if scale is None else scale)
    el = min(state["exact_len"], state["window"])
    out = np.zeros((B, Hq, D), dtype=np.float32)
    for b in range(B):
        for h in range(Hq):
            g = h // G
            pl = int(state["lengths"][b * H + g])
            c = state["counts"][b, g, :pl].astype(np.float32)
            with np.errstate(divide="ignore"):
                s1 = (kp[b, g, :pl] @ q[b, h]) * scale + np.log(c)
            s2 = (kx[b, g, :el] @ q[b, h]) * scale
            s = np.concatenate([s1, s2]).astype(np.float32)
            vals = np.concatenate([vp[b, g, :pl], vx[b, g, :el]])
            m = s.max()
            p = np.exp(s - m).astype(np.float32)
            pv = bf16_round(p) if round_p else p
            out[b, h] = (pv @ vals) / p.sum()
    return out
