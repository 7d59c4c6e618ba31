"""The modeling swap: Llama attention through this build, inside transformers.

The reference rewrites ``LlamaAttention.forward`` (modeling_llama.py:520-954): after the
projections and RoPE (:600) it runs PATH 1 -- anchor selection, packing and the hybrid
prefill (:600-773) -- or PATH 2, the dense flash prefill (:778-803), then ``o_proj``.
transformers routes exactly that step through its attention interface, so the swap
registers two implementations with it:

* ``"deltaattention"``: PATH 1, :func:`attention.delta_prefill_attention` (the globVR
  knobs select the packing mode, threshold, window and variant);
* ``"deltaattention_dense"``: PATH 2, :func:`attention.dense_prefill_attention`.

Both receive the post-RoPE key/value states with the KV heads not repeated (the native
path skips ``repeat_kv``, modeling_llama.py:223-232, 701-708) and write the output
straight into the [B, N, Hq, D] layout that ``o_proj`` reads.  Causality is applied
inside the kernels, so the matching mask functions build no mask.  This is the prefill
path; decoding goes through ``deltaDecoding.HybridCompressedCache``.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import attention, timing

DELTA = "deltaattention"
DENSE = "deltaattention_dense"

_registered = False
# CUDA event pairs around every attention call since the last reset (attention share)
_events: list = []


def _out_view(query: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    B, H, N, D = query.shape
    out = torch.empty(B, N, H, D, dtype=query.dtype, device=query.device)
    return out, out.transpose(1, 2)


def _check(query, key, attention_mask):
    if query.shape[2] != key.shape[2]:
        raise NotImplementedError(
            "the deltaattention implementations are prefill paths (query length == key "
            "length); decode through deltaDecoding.HybridCompressedCache")


def _timed(fn, on_gpu: bool):
    if not on_gpu:  # the ops refuse host tensors themselves
        return fn()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    r = fn()
    e1.record()
    _events.append((e0, e1))
    return r


def delta_attention_forward(module, query, key, value, attention_mask, scaling=None,
                            dropout=0.0, **kwargs):
    """transformers attention function for PATH 1 (modeling_llama.py:600-773)."""
    _check(query, key, attention_mask)
    out, view = _out_view(query)
    layer_idx = getattr(module, "layer_idx", 0)
    _timed(lambda: attention.delta_prefill_attention(query, key, value, layer_idx=layer_idx,
                                                     scaling=scaling, track_sparsity=False,
                                                     out=view), query.is_cuda)
    return out, None


def dense_attention_forward(module, query, key, value, attention_mask, scaling=None,
                            dropout=0.0, **kwargs):
    """transformers attention function for PATH 2 (modeling_llama.py:778-803)."""
    _check(query, key, attention_mask)
    out, view = _out_view(query)
    _timed(lambda: attention.dense_prefill_attention(query, key, value, scaling=scaling, out=view),
           query.is_cuda)
    return out, None


def _no_mask(*args, **kwargs):
    return None


def register() -> None:
    """Register both implementations (and their mask functions) with transformers."""
    global _registered
    if _registered:
        return
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface
    AttentionInterface.register(DELTA, delta_attention_forward)
    AttentionInterface.register(DENSE, dense_attention_forward)
    AttentionMaskInterface.register(DELTA, _no_mask)
    AttentionMaskInterface.register(DENSE, _no_mask)
    _registered = True


def reset_attention_time() -> None:
    _events.clear()


def attention_time_ms() -> float:
    """Summed duration of the attention calls since the last reset (synchronises)."""
    if not _events:
        return 0.0
    _events[-1][1].synchronize()
    return float(sum(a.elapsed_time(b) for a, b in _events))


def llama3_8b_config(attn_implementation: str = DELTA, num_layers: int = 32):
    """Llama-3-8B shape (the end-to-end prefill configuration): hidden 4096, FFN 14336, 32 heads / 8 KV heads,
    vocab 128256, RoPE base 5e5."""
    from transformers import LlamaConfig
    cfg = LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336,
                      num_hidden_layers=num_layers, num_attention_heads=32,
                      num_key_value_heads=8, max_position_embeddings=131072,
                      rope_theta=500000.0, rms_norm_eps=1e-5, tie_word_embeddings=False,
                      initializer_range=0.02)
    cfg._attn_implementation = attn_implementation
    return cfg


def random_llama(cfg, device: torch.device, seed: int = 0):
    """A randomly initialised LlamaForCausalLM in bf16 on ``device`` (weights ~ N(0, 0.02);
    nothing is downloaded)."""
    from transformers import LlamaForCausalLM
    register()
    torch.manual_seed(seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = LlamaForCausalLM(cfg)
    finally:
        torch.set_default_dtype(prev)
    return model.eval()


def set_implementation(model, name: str) -> None:
    """Switch the attention implementation of a built model (PATH 1 <-> PATH 2)."""
    register()
    model.config._attn_implementation = name
    for m in model.modules():
        if hasattr(m, "config") and m.config is not None:
            m.config._attn_implementation = name
