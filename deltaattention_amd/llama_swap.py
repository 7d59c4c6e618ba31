"""The modeling swap: Llama attention through this build, inside transformers.

The reference rewrites ``LlamaAttention.forward`` (modeling_llama.py:520-954): after the
projections and RoPE (:600) it runs PATH 1 -- anchor selection, packing and the hybrid
prefill (:600-773) -- or PATH 2, the dense flash prefill (:778-803), then ``o_proj``;
with a ``HybridCompressedCache`` the prefill hands its packed history to the cache
(:761-773, and PATH 2's ``delta_decode`` packing at :805-879) and every later token runs
PATH 3, the compressed decode: ``cache.update`` then the fused decode attention
(:565-567, :453-518 dispatched at :883-897).

Two layers of the swap:

* :func:`register` adds two transformers attention implementations,
  ``"deltaattention"`` (PATH 1, :func:`attention.delta_prefill_attention`) and
  ``"deltaattention_dense"`` (PATH 2, :func:`attention.dense_prefill_attention`).  They
  are prefill paths: they receive the post-RoPE key/value states with the KV heads not
  repeated (the native path skips ``repeat_kv``, modeling_llama.py:223-232, 701-708) and
  write straight into the [B, N, Hq, D] layout that ``o_proj`` reads.  Causality is
  applied inside the kernels, so the matching mask functions build no mask.  A call that
  continues a sequence (positions not starting at 0) is refused: these functions do not
  see the cache.
* :func:`install` replaces ``forward`` of every ``LlamaAttention`` of a model with
  :func:`delta_llama_attention_forward`, the reference's whole forward: PATH 1 / PATH 2
  prefill by the configured implementation, the prefill -> cache hand-off, and PATH 3
  decode over the compressed cache.  Without a ``HybridCompressedCache`` it runs the
  stock flow through the registered implementation.
"""
from __future__ import annotations

import types
from typing import Optional

import torch

from . import attention, globVR, timing

DELTA = "deltaattention"
DENSE = "deltaattention_dense"

_registered = False
# CUDA event pairs around every attention call since the last reset (attention share)
_events: list = []


def _out_view(query: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    B, H, N, D = query.shape
    out = torch.empty(B, N, H, D, dtype=query.dtype, device=query.device)
    return out, out.transpose(1, 2)


def _check(query, key, kwargs):
    if query.shape[2] != key.shape[2]:
        raise NotImplementedError(
            "the deltaattention implementations are prefill paths (query length == key "
            "length); decode through deltaDecoding.HybridCompressedCache with "
            "llama_swap.install(model)")
    pos = kwargs.get("position_ids")
    if isinstance(pos, torch.Tensor) and pos.numel() > 0 and int(pos.reshape(-1)[0]) != 0:
        # a continuation whose cache returned only the new tokens (a HybridCompressedCache
        # under the stock forward): prefill attention over them alone would be wrong
        raise NotImplementedError(
            "the deltaattention implementations see no cache: continuing a sequence "
            "(positions from %d) needs llama_swap.install(model), which runs the "
            "compressed-cache decode" % int(pos.reshape(-1)[0]))


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


def _track_sparsity() -> bool:
    return bool(getattr(globVR, "track_sparsity", True))


def delta_attention_forward(module, query, key, value, attention_mask, scaling=None,
                            dropout=0.0, **kwargs):
    """transformers attention function for PATH 1 (modeling_llama.py:600-773)."""
    _check(query, key, kwargs)
    out, view = _out_view(query)
    layer_idx = getattr(module, "layer_idx", 0)
    _timed(lambda: attention.delta_prefill_attention(query, key, value, layer_idx=layer_idx,
                                                     scaling=scaling,
                                                     track_sparsity=_track_sparsity(),
                                                     out=view), query.is_cuda)
    return out, None


def dense_attention_forward(module, query, key, value, attention_mask, scaling=None,
                            dropout=0.0, **kwargs):
    """transformers attention function for PATH 2 (modeling_llama.py:778-803)."""
    _check(query, key, kwargs)
    out, view = _out_view(query)
    _timed(lambda: attention.dense_prefill_attention(query, key, value, scaling=scaling, out=view),
           query.is_cuda)
    return out, None


def _is_compressed_cache(cache) -> bool:
    from .deltaDecoding import HybridCompressedCache
    return isinstance(cache, HybridCompressedCache)


def _kv_size_sample(cache) -> None:
    """Layer-0 KV-size tracker of the decode steps (modeling_llama.py:572-595): every
    ``kv_log_interval`` tokens, the memory saved against an uncompressed cache."""
    total_len = cache.total_seq_lens[0]
    interval = getattr(globVR, "kv_log_interval", 10)
    if total_len > 0 and total_len % interval == 0:
        exact_len = min(cache.exact_seq_lens[0], cache.exact_window_size)
        avg_packed = cache.packed_lengths[0].float().mean().item()
        savings = (1 - (exact_len + avg_packed) / total_len) * 100
        if not hasattr(globVR, "kv_compression_samples"):
            globVR.kv_compression_samples = []
        globVR.kv_compression_samples.append(savings)


def delta_llama_attention_forward(self, hidden_states: torch.Tensor,
                                  position_embeddings=None, attention_mask=None,
                                  past_key_values=None, **kwargs):
    """``LlamaAttention.forward`` of the reference (modeling_llama.py:520-954) on the HIP
    ops.  Prefill (more than one token) runs PATH 1 or PATH 2 by the model's attention
    implementation (``"deltaattention"`` / ``"deltaattention_dense"``); with a
    HybridCompressedCache the prefill hands its packed history and exact tail to the
    cache (PATH 1 :761-773; PATH 2 when ``globVR.delta_decode`` is set, :805-879) and a
    single-token step runs PATH 3: ``cache.update`` (merge or append of the evicted
    token, ring write, :565-567) then the compressed decode attention (:453-518).  Any
    other cache (or none) takes the stock flow: ``update`` then the registered
    attention implementation.  Returns (attn_output, None)."""
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb
    from . import deltaDecoding

    cache = past_key_values if past_key_values is not None else kwargs.pop("past_key_value", None)
    input_shape = hidden_states.shape[:-1]
    hidden_shape = (*input_shape, -1, self.head_dim)
    is_prefill = hidden_states.shape[1] > 1
    ev_total = timing.start_event()                                  # :540-543

    query_states = self.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    key_states = self.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    value_states = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
    cos, sin = position_embeddings
    query_states, key_states = apply_rotary_pos_emb(query_states, key_states, cos, sin)

    if not _is_compressed_cache(cache):
        if cache is not None:
            key_states, value_states = cache.update(key_states, value_states, self.layer_idx)
        fn = {DELTA: delta_attention_forward, DENSE: dense_attention_forward}.get(
            self.config._attn_implementation)
        if fn is None:  # any other implementation, as transformers dispatches it
            from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
            from transformers.models.llama.modeling_llama import eager_attention_forward
            fn = ALL_ATTENTION_FUNCTIONS.get_interface(self.config._attn_implementation,
                                                       eager_attention_forward)
        attn_output, _ = fn(self, query_states, key_states, value_states, attention_mask,
                            dropout=0.0, scaling=self.scaling, **kwargs)
    elif is_prefill:
        # the cache's update passes prefill tokens through (deltaDecoding.py:183-184)
        B, H, N, D = query_states.shape
        attn_output, view = _out_view(query_states)
        if self.config._attn_implementation == DENSE:                # PATH 2
            _timed(lambda: attention.dense_prefill_attention(
                query_states, key_states, value_states, scaling=self.scaling, out=view),
                query_states.is_cuda)
            if getattr(globVR, "delta_decode", False):               # :805-879
                attention.delta_decode_handoff(key_states, value_states, self.layer_idx, cache)
        else:                                                        # PATH 1
            _timed(lambda: attention.delta_prefill_attention(
                query_states, key_states, value_states, layer_idx=self.layer_idx,
                past_key_value=cache, scaling=self.scaling,
                track_sparsity=_track_sparsity(), out=view), query_states.is_cuda)
    else:                                                            # PATH 3
        if cache.get_seq_length(self.layer_idx) == 0:
            raise RuntimeError("compressed decode needs a prefill hand-off first: this layer's "
                               "HybridCompressedCache is empty")
        if not timing.enabled():
            # update (:565-567) and the decode attention (:453-518) in one library call
            out = cache.decode_step(query_states, key_states, value_states, self.layer_idx,
                                    scaling=self.scaling)            # [B, Hq, 1, D]
            if self.layer_idx == 0:
                _kv_size_sample(cache)
        else:
            ev = timing.start_event()
            cache.update(key_states, value_states, self.layer_idx)   # :565-567
            timing.stop_event("time_delta_decode_cache_update", ev)
            if self.layer_idx == 0:
                _kv_size_sample(cache)
            ev_dec = timing.start_event()
            out = deltaDecoding.decode_attention(query_states, cache, self.layer_idx,
                                                 scaling=self.scaling)  # [B, Hq, 1, D]
            timing.stop_event("time_delta_decode_attn_calc", ev_dec)
            timing.stop_event("time_delta_decode_inner_total", ev_dec)
        attn_output = out.transpose(1, 2)

    attn_output = attn_output.reshape(*input_shape, -1).contiguous()
    attn_output = self.o_proj(attn_output)
    timing.stop_event("time_prefill_forward_total" if is_prefill else "time_decode_forward_total",
                      ev_total)                                      # :946-952
    return attn_output, None


def install(model) -> int:
    """Route every LlamaAttention of ``model`` through :func:`delta_llama_attention_forward`
    (registers the two implementations too).  Returns the number of modules swapped."""
    from transformers.models.llama.modeling_llama import LlamaAttention
    register()
    n = 0
    for m in model.modules():
        if isinstance(m, LlamaAttention):
            m.forward = types.MethodType(delta_llama_attention_forward, m)
            n += 1
    return n


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


def random_llama(cfg, device: torch.device, seed: int = 0, dtype: torch.dtype = torch.bfloat16):
    """A randomly initialised LlamaForCausalLM in ``dtype`` (bf16 by default) on ``device``
    (weights ~ N(0, 0.02); nothing is downloaded)."""
    from transformers import LlamaForCausalLM
    register()
    torch.manual_seed(seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(dtype)
    try:
        with torch.device(device):
            model = LlamaForCausalLM(cfg)
    finally:
        torch.set_default_dtype(prev)
    install(model)
    return model.eval()


def set_implementation(model, name: str) -> None:
    """Switch the attention implementation of a built model (PATH 1 <-> PATH 2)."""
    register()
    model.config._attn_implementation = name
    for m in model.modules():
        if hasattr(m, "config") and m.config is not None:
            m.config._attn_implementation = name
