"""Seeded synthetic attention-layer inputs and threshold calibration.

Keys follow an AR(1) process along the sequence, k_t = rho * k_{t-1} + sigma * eps_t
(k_0 = eps_0, stationary variance ~1 for rho = 0.9, sigma = 0.44), so adjacent keys
are similar as in real post-RoPE keys; queries and values are N(0, 1).  RoPE
(rotate-half, inv_freq = base^(-2i/D), emb = cat(freqs, freqs)) is applied to Q and
K after generation, as modeling_llama.py:157-204 does.  The keys come from numpy's
PCG64 generator on the CPU so that every machine builds the same tensor; Q and V may
be drawn on the GPU for the large configurations.
"""
from __future__ import annotations

from typing import Optional, Tuple

import numpy as np
import torch


def ar1_keys(batch: int, heads: int, seq_len: int, head_dim: int, rho=0.9, sigma=0.44,
             seed: int = 0) -> torch.Tensor:
    """float32 [B, H, N, D] AR(1) keys (rho may be a per-head array of length B*H)."""
    from scipy.signal import lfilter

    rng = np.random.default_rng(seed)
    rho_arr = np.broadcast_to(np.asarray(rho, dtype=np.float64), (batch * heads,))
    out = np.empty((batch * heads, seq_len, head_dim), dtype=np.float32)
    for i in range(batch * heads):
        eps = rng.standard_normal((seq_len, head_dim), dtype=np.float32)
        eps[0] /= sigma  # k_0 = eps_0
        out[i] = lfilter([sigma], [1.0, -float(rho_arr[i])], eps, axis=0).astype(np.float32)
    return torch.from_numpy(out).view(batch, heads, seq_len, head_dim)


def rope_cos_sin(seq_len: int, head_dim: int, base: float, device=None) -> Tuple[torch.Tensor, torch.Tensor]:
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.int64, device=device)
                               .float() / head_dim))
    pos = torch.arange(seq_len, device=device, dtype=torch.float32)
    freqs = torch.outer(pos, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def apply_rope(x: torch.Tensor, base: float) -> torch.Tensor:
    """Rotate-half RoPE over the sequence axis (dim 2) in float32."""
    N, D = x.shape[2], x.shape[3]
    cos, sin = rope_cos_sin(N, D, base, device=x.device)
    x = x.float()
    x1, x2 = x[..., : D // 2], x[..., D // 2:]
    rot = torch.cat((-x2, x1), dim=-1)
    return x * cos + rot * sin


def make_layer_inputs(batch: int, q_heads: int, kv_heads: int, seq_len: int, head_dim: int,
                      rho=0.9, sigma: float = 0.44, rope_base: float = 500000.0, seed: int = 0,
                      dtype: torch.dtype = torch.bfloat16, device: str = "cpu",
                      qv_on_device: bool = False):
    """(q [B,Hq,N,D], k [B,Hkv,N,D], v [B,Hkv,N,D]) of the given dtype on ``device``."""
    k = ar1_keys(batch, kv_heads, seq_len, head_dim, rho, sigma, seed)
    k = apply_rope(k.to(device), rope_base).to(dtype)
    if qv_on_device:
        gen = torch.Generator(device=device).manual_seed(seed + 1)
        q = torch.randn((batch, q_heads, seq_len, head_dim), generator=gen, device=device)
        v = torch.randn((batch, kv_heads, seq_len, head_dim), generator=gen, device=device)
    else:
        gen = torch.Generator().manual_seed(seed + 1)
        q = torch.randn((batch, q_heads, seq_len, head_dim), generator=gen)
        v = torch.randn((batch, kv_heads, seq_len, head_dim), generator=gen)
        q, v = q.to(device), v.to(device)
    q = apply_rope(q, rope_base).to(dtype)
    return q, k, v.to(dtype)


def calibrate_threshold(k: torch.Tensor, ratio: float, chunk_size: int = 512,
                        metric: str = "euclidean", iters: int = 40,
                        lo: float = 0.0, hi: Optional[float] = None,
                        arith: str = "native") -> Tuple[float, float]:
    """Smallest Euclidean tau whose realised keep rate is <= 1/ratio, by bisection with
    the GPU selection kernel in the given arithmetic.  Returns (tau, realised ratio
    N*H / sum c)."""
    from . import ops

    target = 1.0 / ratio
    total = k.shape[0] * k.shape[1] * k.shape[2]

    def keep_rate(tau):
        _, cc = ops.select(k, tau, chunk_size, 0, metric, arith=arith)
        return float(cc.sum().item()) / total

    if hi is None:
        hi = 1.0
        while keep_rate(hi) > target:
            hi *= 2.0
    for _ in range(iters):
        mid = 0.5 * (lo + hi)
        if keep_rate(mid) > target:
            lo = mid
        else:
            hi = mid
    return hi, 1.0 / keep_rate(hi)
