"""The delta-attention prefill path of modeling_llama.py's LlamaAttention, on the
native kernels.

* ``forward_hybrid_flash`` / ``forward_hybrid_flash_sanity`` / ``forward_pure_phase1``
  restate the kernel wrappers (modeling_llama.py:306-451): same arguments, same
  conversions (timestamps to int32, counts to fp32, ``globVR.no_count``), output shaped
  like q.  K/V and the packed tensors may be per query head (repeat_kv-expanded, as the
  reference passes them) or per KV head (read directly, no expansion).
* ``delta_prefill_attention`` restates PATH 1 of LlamaAttention.forward
  (modeling_llama.py:600-773) between RoPE and o_proj: chunking, the three packing
  modes, index/pack/counts, the sparsity bookkeeping, the variant dispatch, the stage
  timings and the prefill -> HybridCompressedCache hand-off.  P stays on the device
  for the attention; only the bookkeeping and the hand-off read it back, as the
  reference does (:656, :695).
* ``dense_prefill_attention`` restates PATH 2 (modeling_llama.py:778-803), and
  ``delta_decode_handoff`` its ``delta_decode`` tail (:805-879): delta selection and
  packing of the prefill keys into the HybridCompressedCache for compressed decoding.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import globVR, ops, timing

__all__ = ["forward_hybrid_flash", "forward_hybrid_flash_sanity", "forward_pure_phase1",
           "delta_prefill_attention", "dense_prefill_attention", "delta_decode_handoff",
           "keep_mask"]


def _wrapper(variant, q, k_dense, v_dense, k_packed, v_packed, packed_timestamps, packed_counts,
             dense_window_size, scaling=None):
    q = q.contiguous()
    k_dense, v_dense = k_dense.contiguous(), v_dense.contiguous()
    k_packed, v_packed = k_packed.contiguous(), v_packed.contiguous()
    packed_timestamps = packed_timestamps.contiguous().to(torch.int32)
    packed_counts = packed_counts.contiguous().to(torch.float32)
    no_count = variant != "sanity" and bool(getattr(globVR, "no_count", False))
    return ops.hybrid_prefill(q, k_dense, v_dense, k_packed, v_packed, packed_timestamps,
                              packed_counts, window=dense_window_size, scale=scaling,
                              variant=variant, no_count=no_count)


def forward_hybrid_flash(q, k_dense, v_dense, k_packed, v_packed, packed_timestamps,
                         packed_counts, dense_window_size, scaling=None):
    """modeling_llama.py:306-354 (two-phase hybrid kernel)."""
    return _wrapper("hybrid", q, k_dense, v_dense, k_packed, v_packed, packed_timestamps,
                    packed_counts, dense_window_size, scaling)


def forward_hybrid_flash_sanity(q, k_dense, v_dense, k_packed, v_packed, packed_timestamps,
                                packed_counts, dense_window_size, scaling=None):
    """modeling_llama.py:356-401 (Phase 1 decides the window start, adds nothing)."""
    return _wrapper("sanity", q, k_dense, v_dense, k_packed, v_packed, packed_timestamps,
                    packed_counts, dense_window_size, scaling)


def forward_pure_phase1(q, k_dense, v_dense, k_packed, v_packed, packed_timestamps,
                        packed_counts, dense_window_size, scaling=None):
    """modeling_llama.py:403-451 (packed history only)."""
    return _wrapper("pure_phase1", q, k_dense, v_dense, k_packed, v_packed, packed_timestamps,
                    packed_counts, dense_window_size, scaling)


def keep_mask(key_states: torch.Tensor):
    """Anchor mask of the configured packing mode (modeling_llama.py:602-653).

    Returns (keep [B, Hkv, N] int32, per-head anchor counts [B, Hkv] int32 on device).
    """
    B, H, N, _ = key_states.shape
    mode = getattr(globVR, "packing_mode", "delta")
    if mode == "random":                                            # :620-624
        rate = getattr(globVR, "target_keep_rate", 0.5)
        keep = (torch.rand(B, H, N, device=key_states.device) < rate).to(torch.int32)
        keep[:, :, 0] = 1
        return keep, keep.sum(dim=-1, dtype=torch.int32)
    if mode == "periodic":                                          # :626-632
        rate = getattr(globVR, "target_keep_rate", 0.5)
        period = max(1, round(1.0 / rate))
        pos = torch.arange(N, device=key_states.device)
        keep = (pos % period == 0).to(torch.int32).expand(B, H, N).contiguous()
        return keep, keep.sum(dim=-1, dtype=torch.int32)
    fixed = getattr(globVR, "chunk_size", 0)                        # :602-610
    divide_to = getattr(globVR, "divide_to", 0)
    keep, chunk_counts = ops.select(key_states, getattr(globVR, "row_delta_threshold", 0.0),
                                    chunk_size=fixed if fixed > 0 else 0,
                                    divide_to=0 if fixed > 0 else divide_to,
                                    metric=getattr(globVR, "row_similarity_metric", "euclidean"),
                                    arith=getattr(globVR, "row_delta_arith", "native"))
    return keep, chunk_counts.sum(dim=-1, dtype=torch.int32)


def delta_prefill_attention(query_states: torch.Tensor, key_states: torch.Tensor,
                            value_states: torch.Tensor, layer_idx: int = 0,
                            past_key_value=None, scaling: Optional[float] = None,
                            track_sparsity: bool = True,
                            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """PATH 1 attention: q [B, Hq, N, D], post-RoPE k/v [B, Hkv, N, D] -> [B, Hq, N, D].

    ``out``, if given, is a [B, Hq, N, D] view (any strides with a contiguous head dim)
    the kernel writes into."""
    q_len = key_states.shape[2]
    ev = timing.start_event()
    keep, active = keep_mask(key_states)
    packed = ops.pack(keep, key_states, value_states)               # :655-685, P on device
    timing.stop_event("time_get_row_delta", ev)
    if track_sparsity:                                              # :694-698
        kept = int(active.sum().item())
        total = keep.numel()
        layer_spars = 1.0 - kept / total if total > 0 else 0.0
        globVR.spars = layer_spars if globVR.spars == 0.0 else (globVR.spars + layer_spars) / 2
    ev = timing.start_event()
    window = getattr(globVR, "dense_window_size", 128)              # :716
    if getattr(globVR, "pure_phase1", False):
        variant = "pure_phase1"
    elif getattr(globVR, "sanity", False):
        variant = "sanity"
    else:
        variant = "hybrid"
    out = ops.hybrid_prefill(query_states, key_states, value_states, packed.k_packed,
                             packed.v_packed, packed.timestamps, packed.counts, window=window,
                             scale=scaling, variant=variant,
                             no_count=variant != "sanity" and bool(getattr(globVR, "no_count", False)),
                             num_packed_dev=packed.num_packed, out=out)
    timing.stop_event("time_delta_mm_pattern", ev)
    if past_key_value is not None and hasattr(past_key_value, "initialize_from_prefill"):
        _handoff(past_key_value, layer_idx, packed, key_states, value_states)   # :762-773
    return out


def _handoff(cache, layer_idx, packed, key_states, value_states):
    """initialize_from_prefill with the P packed rows of every head and the last
    min(N, W) prefill tokens (modeling_llama.py:762-773, 869-879)."""
    q_len = key_states.shape[2]
    p = packed.trimmed()
    tail = min(q_len, cache.exact_window_size)
    cache.initialize_from_prefill(
        layer_idx=layer_idx, k_packed=p.k_packed, v_packed=p.v_packed, counts=p.counts,
        timestamps=p.timestamps, k_exact=key_states[:, :, -tail:, :],
        v_exact=value_states[:, :, -tail:, :], original_q_len=q_len)


def delta_decode_handoff(key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
                         past_key_value) -> None:
    """PATH 2's ``delta_decode`` tail (modeling_llama.py:805-879): after a dense prefill,
    delta-select and pack the post-RoPE keys with the globVR chunking, metric and
    threshold (always delta mode, whatever ``packing_mode`` says, as the reference
    launches chunked_eval_kernel directly), then hand the packed history and the exact
    tail to the cache."""
    fixed = getattr(globVR, "chunk_size", 0)                        # :809-816
    divide_to = getattr(globVR, "divide_to", 0)
    keep, _ = ops.select(key_states, getattr(globVR, "row_delta_threshold", 0.0),
                         chunk_size=fixed if fixed > 0 else 0,
                         divide_to=0 if fixed > 0 else divide_to,
                         metric=getattr(globVR, "row_similarity_metric", "euclidean"),
                         arith=getattr(globVR, "row_delta_arith", "native"))
    packed = ops.pack(keep, key_states, value_states)               # :836-866
    _handoff(past_key_value, layer_idx, packed, key_states, value_states)   # :868-879


def dense_prefill_attention(query_states, key_states, value_states, scaling=None, out=None):
    """PATH 2 (modeling_llama.py:778-803): dense causal flash prefill, GQA-native."""
    ev = timing.start_event()
    out = ops.dense_prefill(query_states, key_states, value_states, causal=True, scale=scaling,
                            out=out)
    timing.stop_event("time_triton_flash_attention", ev)
    return out
