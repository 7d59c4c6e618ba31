"""Blockwise torch-CPU restatement of the reference's attention math -- TEST INFRASTRUCTURE.

This is the CPU baseline that ``bench.py`` times on the GPU box's host cores (and that
``tests/test_oracle.py`` pins against ``delta_oracle``).  It restates the reference's
PyTorch attention with torch's fused CPU attention, so that 32K-token layers run in full
without an [N, N] score matrix; nothing in the product package imports it.

* ``dense_attention``: ``eager_attention_forward`` (modeling_llama.py:235-276) --
  ``Q K^T * scaling`` plus the causal mask, softmax in fp32, times V -- through torch's
  fused CPU ``scaled_dot_product_attention`` (the same math without the [N, N] score
  matrix; the G query heads of a KV head share its keys, repeat_kv at
  modeling_llama.py:223-232, via ``enable_gqa``).
* ``hybrid_attention``: the two-phase compressed prefill (deltaFlashAttention.py:9-146)
  per logical 128-row query block.  The block's keys are the packed anchors of its
  ``n_safe`` safe blocks, each weighted by its count (modeling_llama.py:321), and the
  exact keys ``[ds, row]`` under the causal mask (:108-136; tokens in ``[ds, last]``
  count twice, as in the reference).  The softmax over that weighted multiset is taken
  exactly in fp32, with the weights as an additive log-count mask (the reference's
  online softmax computes the same quantity; only its rounding points differ).  The
  schedule comes from ``delta_oracle.hybrid_schedule``.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

from .delta_oracle import BLOCK_M, BLOCK_N, hybrid_schedule


def _as_cpu_f32(x) -> torch.Tensor:
    t = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.asarray(x))
    return t.detach().to("cpu", torch.float32).contiguous()


def dense_attention(q, k, v, causal: bool = True, scale: Optional[float] = None) -> torch.Tensor:
    """q [B, Hq, N, D], k / v [B, Hkv, N, D] -> float32 [B, Hq, N, D]."""
    q, k, v = _as_cpu_f32(q), _as_cpu_f32(k), _as_cpu_f32(v)
    scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    return F.scaled_dot_product_attention(q, k, v, is_causal=causal, scale=scale, enable_gqa=True)


def hybrid_attention(q, k, v, k_packed, v_packed, timestamps, counts, window: int,
                     scale: Optional[float] = None) -> torch.Tensor:
    """The hybrid variant with counts as weights; shapes as delta_oracle.hybrid_attention
    (k_packed / v_packed / timestamps / counts hold P rows per KV head)."""
    q, k, v = _as_cpu_f32(q), _as_cpu_f32(k), _as_cpu_f32(v)
    kp, vp = _as_cpu_f32(k_packed), _as_cpu_f32(v_packed)
    cnt = _as_cpu_f32(counts)
    B, Hq, Nq, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    G = Hq // Hkv
    P = kp.shape[2]
    scale = D ** -0.5 if scale is None else float(scale)
    n_safe, _, ds, dh = hybrid_schedule(np.asarray(timestamps), P, Nk, Nq, window)
    logw = torch.where(cnt > 0, torch.log(cnt.clamp_min(1e-30)), torch.full_like(cnt, float("-inf")))
    out = torch.empty((B, Hq, Nq, D), dtype=torch.float32)
    nqb = (Nq + BLOCK_M - 1) // BLOCK_M
    for b in range(B):
        for g in range(Hkv):
            for qb in range(nqb):
                r0, r1 = qb * BLOCK_M, min(Nq, qb * BLOCK_M + BLOCK_M)
                na = int(n_safe[b, g, qb]) * BLOCK_N  # safe blocks lie inside [0, P)
                lo, hi = int(ds[b, g, qb]), int(dh[b, g, qb])
                keys = torch.cat([kp[b, g, :na], k[b, g, lo:hi]])[None, None]
                vals = torch.cat([vp[b, g, :na], v[b, g, lo:hi]])[None, None]
                causal = torch.zeros((r1 - r0, hi - lo)).masked_fill_(
                    torch.arange(lo, hi)[None, :] > torch.arange(r0, r1)[:, None], float("-inf"))
                mask = torch.cat([logw[b, g, :na][None, :].expand(r1 - r0, na), causal], dim=1)
                out[b, g * G:(g + 1) * G, r0:r1] = F.scaled_dot_product_attention(
                    q[b, g * G:(g + 1) * G, r0:r1][None], keys, vals, attn_mask=mask[None, None],
                    scale=scale, enable_gqa=True)[0]
    return out
