"""The modeling swap (llama_swap): a small Llama through the HIP attention path inside
transformers, against transformers' own fp32 eager attention on the same weights."""
import copy

import numpy as np
import pytest
import torch

from conftest import announce

pytestmark = pytest.mark.gpu


def _tiny_llama(impl, seed=0):
    from deltaattention_amd import llama_swap
    cfg = llama_swap.llama3_8b_config(impl, num_layers=2)
    cfg.vocab_size = 512
    cfg.hidden_size = 1024
    cfg.intermediate_size = 2048
    cfg.num_attention_heads = 8
    cfg.num_key_value_heads = 2
    cfg.head_dim = 128
    return llama_swap.random_llama(cfg, torch.device("cuda:0"), seed=seed)


def _logits(model, ids):
    with torch.no_grad():
        return model(ids, use_cache=False).logits.float()


def test_dense_swap_matches_eager_fp32(gpu):
    from deltaattention_amd import llama_swap
    announce("llama swap: dense path vs transformers eager fp32, 2 layers, N=640")
    model = _tiny_llama(llama_swap.DENSE)
    ids = torch.randint(0, 512, (1, 640), generator=torch.Generator().manual_seed(1)).cuda()
    ours = _logits(model, ids)
    ref_model = copy.deepcopy(model).float()
    ref_model.config._attn_implementation = "eager"
    for m in ref_model.modules():
        if hasattr(m, "config") and m.config is not None:
            m.config._attn_implementation = "eager"
    ref = _logits(ref_model, ids)
    err = (ours - ref).abs()
    scale = ref.abs().mean()
    print(f"dense swap: max-abs {err.max():.3e} mean-abs {err.mean():.3e} (|ref| mean {scale:.3e})")
    assert torch.isfinite(ours).all()
    assert err.mean() <= 0.02 * scale      # bf16 weights/activations vs fp32 throughout
    assert err.max() <= 0.25 * ref.abs().max()


def test_delta_swap_keep_all_equals_dense(gpu):
    """Periodic packing with period 1 keeps every key with count 1: the hybrid prefill
    then computes dense causal attention, and the two paths must agree."""
    from deltaattention_amd import globVR, llama_swap
    announce("llama swap: delta path (keep all) vs dense path, 2 layers, N=640")
    model = _tiny_llama(llama_swap.DELTA)
    ids = torch.randint(0, 512, (1, 640), generator=torch.Generator().manual_seed(2)).cuda()
    saved = (globVR.packing_mode, globVR.target_keep_rate)
    try:
        globVR.packing_mode = "periodic"
        globVR.target_keep_rate = 1.0
        delta = _logits(model, ids)
    finally:
        globVR.packing_mode, globVR.target_keep_rate = saved
    llama_swap.set_implementation(model, llama_swap.DENSE)
    dense = _logits(model, ids)
    err = (delta - dense).abs()
    print(f"delta(keep all) vs dense: max-abs {err.max():.3e} mean-abs {err.mean():.3e}")
    assert err.max() <= 2e-2 * max(1.0, float(dense.abs().max()))
    assert err.mean() <= 1e-3 * max(1.0, float(dense.abs().mean()) * 10)


def _spy_layer0(monkeypatch):
    """Record layer 0's prefill key/value states, its decode-step keys/values and its
    decode queries and attention outputs, while the real calls run."""
    from deltaattention_amd import attention, deltaDecoding
    from deltaattention_amd.deltaDecoding import HybridCompressedCache
    rec = {"prefill": None, "kv": [], "attn": []}
    real_prefill = attention.delta_prefill_attention
    real_handoff = attention.delta_decode_handoff
    real_update = HybridCompressedCache.update
    real_decode = deltaDecoding.decode_attention

    def prefill(q, k, v, layer_idx=0, **kw):
        if layer_idx == 0:
            rec["prefill"] = (k.detach().clone(), v.detach().clone())
        return real_prefill(q, k, v, layer_idx=layer_idx, **kw)

    def handoff(k, v, layer_idx, cache):
        if layer_idx == 0:
            rec["prefill"] = (k.detach().clone(), v.detach().clone())
        return real_handoff(k, v, layer_idx, cache)

    def update(self, k, v, layer_idx, cache_kwargs=None):
        if layer_idx == 0 and k.shape[2] == 1:
            rec["kv"].append((k.detach().clone(), v.detach().clone()))
        return real_update(self, k, v, layer_idx, cache_kwargs)

    def decode(q, cache, layer_idx, scaling=None):
        out = real_decode(q, cache, layer_idx, scaling=scaling)
        if layer_idx == 0:
            rec["attn"].append((q.detach().clone(), out.detach().clone()))
        return out

    real_step = HybridCompressedCache.decode_step

    def step(self, q, k, v, layer_idx, scaling=None):
        out = real_step(self, q, k, v, layer_idx, scaling=scaling)
        if layer_idx == 0:
            rec["kv"].append((k.detach().clone(), v.detach().clone()))
            rec["attn"].append((q.detach().clone(), out.detach().clone()))
        return out

    monkeypatch.setattr(attention, "delta_prefill_attention", prefill)
    monkeypatch.setattr(attention, "delta_decode_handoff", handoff)
    monkeypatch.setattr(HybridCompressedCache, "update", update)
    monkeypatch.setattr(deltaDecoding, "decode_attention", decode)
    monkeypatch.setattr(HybridCompressedCache, "decode_step", step)
    return rec


def _assert_cache_equals(cache, st, what):
    n = int(st["lengths"].max())
    assert np.array_equal(cache.packed_lengths[0].cpu().numpy(), st["lengths"]), what
    assert np.array_equal(cache.packed_counts[0, :, :, :n].cpu().numpy(), st["counts"][:, :, :n]), what
    assert np.array_equal(cache.packed_timestamps[0, :, :, :n].cpu().numpy(), st["timestamps"][:, :, :n]), what
    assert np.array_equal(cache.k_packed[0, :, :, :n].float().cpu().numpy(), st["k_packed"][:, :, :n]), what
    assert np.array_equal(cache.v_packed[0, :, :, :n].float().cpu().numpy(), st["v_packed"][:, :, :n]), what
    assert np.array_equal(cache.k_exact[0].float().cpu().numpy(), st["k_exact"]), what
    assert np.array_equal(cache.v_exact[0].float().cpu().numpy(), st["v_exact"]), what


@pytest.mark.parametrize("impl,timed,dtype", [("deltaattention", True, torch.bfloat16),
                                              ("deltaattention_dense", True, torch.bfloat16),
                                              ("deltaattention", False, torch.bfloat16),
                                              ("deltaattention", False, torch.float32)],
                         ids=["path1", "path2", "path1-fused-step", "path1-step-fp32"])
def test_model_prefill_then_decode_compressed_cache(gpu, monkeypatch, impl, timed, dtype):
    """A 2-layer Llama-3-8B-shaped model (hidden 4096, 32 query / 8 KV heads, head_dim
    128; vocab cut to 1024) prefills 2048 tokens into a HybridCompressedCache through
    llama_swap.install's forward and decodes 64 tokens one at a time.  PATH 1 hands its
    packed history to the cache (modeling_llama.py:761-773); PATH 2 packs after the dense
    prefill when delta_decode is set (:805-879); every later token runs PATH 3: update,
    then the compressed decode attention (:565-567, :453-518, :883-897), as two calls
    under stage timing and as one HybridCompressedCache.decode_step without.  Layer 0 is
    replayed in the oracle from the keys and queries it saw: the cache after the hand-off
    and after the last step is bit-exact, and every step's decode attention is within
    tolerance.  "path1-step-fp32" runs the same model in fp32 (fp32 prefill kernels, fp32
    cache, selection in fp32)."""
    from oracle import delta_oracle as O
    from oracle import select_oracle_c as OC
    from test_gpu_dropin import _oracle_cache_from_prefill
    from deltaattention_amd import globVR, llama_swap, timing
    from deltaattention_amd.deltaDecoding import HybridCompressedCache
    N, steps, W, tau = 2048, 64, 64, 20.5   # random-init keys: adjacent dist^2 ~ 420 +- 52
    cfg = llama_swap.llama3_8b_config(impl, num_layers=2)
    cfg.vocab_size = 1024
    model = llama_swap.random_llama(cfg, gpu, seed=3, dtype=dtype)
    for name, val in (("packing_mode", "delta"), ("chunk_size", 512), ("row_delta_threshold", tau),
                      ("row_similarity_metric", "euclidean"), ("delta_decode", True),
                      ("dense_window_size", 128), ("time_internal", timed), ("kv_log_interval", 16),
                      ("sanity", False), ("pure_phase1", False), ("no_count", False)):
        monkeypatch.setattr(globVR, name, val, raising=False)
    timing.reset()
    rec = _spy_layer0(monkeypatch)
    cache = HybridCompressedCache(cfg, 1, dtype=dtype, exact_window_size=W,
                                  initial_capacity=256, device="cuda")
    ids = torch.randint(0, cfg.vocab_size, (1, N + steps), generator=torch.Generator().manual_seed(4)).cuda()
    announce(f"model swap {impl}: prefill N={N} into HybridCompressedCache")
    with torch.no_grad():
        h = model.model(input_ids=ids[:, :N], past_key_values=cache, use_cache=True).last_hidden_state
    assert torch.isfinite(h).all()
    assert cache.get_seq_length(0) == N and cache.get_seq_length(1) == N
    k0, v0 = (t.float().cpu().numpy() for t in rec["prefill"])
    # the selection's native arithmetic: bf16 keys in bf16, fp32 keys in fp32
    keep, _ = OC.select_delta(k0, tau, 512, arith="bf16" if dtype == torch.bfloat16 else "fp32")
    p = O.pack(k0, v0, keep)
    st = _oracle_cache_from_prefill(p, k0, v0, W, cache.capacity + steps)
    _assert_cache_equals(cache, st, "after the prefill hand-off")
    print(f"{impl}: P={p['P']} anchors of {N} per head (max)", flush=True)
    announce(f"model swap {impl}: {steps} decode steps")
    worst = 0.0
    with torch.no_grad():
        for t in range(steps):
            h = model.model(input_ids=ids[:, N + t:N + t + 1], past_key_values=cache,
                            use_cache=True).last_hidden_state
            assert h.shape == (1, 1, cfg.hidden_size) and torch.isfinite(h).all()
            kt, vt = (x.float().cpu().numpy() for x in rec["kv"][t])
            O.decode_update(st, kt, vt, tau)
            q, out = rec["attn"][t]
            want = O.decode_attention(q[:, :, 0].float().cpu().numpy(), st, scale=128 ** -0.5)
            err = np.abs(out[:, :, 0].float().cpu().numpy() - want)
            worst = max(worst, float(err.max()))
            assert err.max() <= 2e-2 and err.mean() <= 1e-3, (t, err.max(), err.mean())
    assert cache.get_seq_length(0) == N + steps
    _assert_cache_equals(cache, st, "after the decode steps")
    appended = int((st["lengths"] - p["P"]).sum())     # evicted tokens that became anchors
    print(f"{impl}: {steps} steps, worst max-abs {worst:.3e}, packed length "
          f"{int(st['lengths'].max())}, appended {appended} of {8 * steps} evictions", flush=True)
    assert 0 < appended < 8 * steps     # the threshold both merges and appends
    assert len(rec["kv"]) == len(rec["attn"]) == steps
    if timed:
        timing.resolve_latency_events()
        stats = globVR.latency_stats
        for key in ("time_prefill_forward_total", "time_decode_forward_total",
                    "time_delta_decode_cache_update", "time_delta_decode_attn_calc"):
            assert stats.get(key, {}).get("calls", 0) > 0, key
    assert len(globVR.kv_compression_samples) >= steps // 16
    timing.reset()
