"""Control flow of the modeling swap on the CPU, with the native calls replaced by
recorders (no GPU): which path each forward takes, what reaches the compressed cache, and
that the registered prefill implementations refuse a continuation they cannot serve."""
import types

import pytest
import torch

pytest.importorskip("transformers")


def _tiny_model(impl):
    from transformers import LlamaConfig, LlamaForCausalLM
    from deltaattention_amd import llama_swap
    llama_swap.register()
    cfg = LlamaConfig(vocab_size=64, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                      max_position_embeddings=256)
    cfg._attn_implementation = impl
    torch.manual_seed(0)
    model = LlamaForCausalLM(cfg).eval()
    assert llama_swap.install(model) == 2
    return cfg, model


def _stub(monkeypatch):
    """Replace the native entry points the forward reaches with recorders that produce
    outputs of the right shape (zeros) and perform the cache hand-off bookkeeping."""
    from deltaattention_amd import attention, deltaDecoding
    from deltaattention_amd.deltaDecoding import HybridCompressedCache
    calls = []

    def prefill(q, k, v, layer_idx=0, past_key_value=None, scaling=None, track_sparsity=True, out=None):
        calls.append(("prefill", layer_idx, past_key_value is not None, tuple(q.shape), tuple(k.shape)))
        out.zero_()
        if past_key_value is not None:
            n = k.shape[2]
            tail = min(n, past_key_value.exact_window_size)
            ts = torch.arange(n, dtype=torch.int32).expand(k.shape[0], k.shape[1], n)
            past_key_value.initialize_from_prefill(layer_idx, k, v, torch.ones_like(ts), ts,
                                                   k[:, :, -tail:], v[:, :, -tail:], n)
        return out

    def dense(q, k, v, scaling=None, out=None):
        calls.append(("dense", tuple(q.shape)))
        return out.zero_()

    def handoff(k, v, layer_idx, cache):
        calls.append(("handoff", layer_idx))
        n = k.shape[2]
        tail = min(n, cache.exact_window_size)
        ts = torch.arange(n, dtype=torch.int32).expand(k.shape[0], k.shape[1], n)
        cache.initialize_from_prefill(layer_idx, k, v, torch.ones_like(ts), ts, k[:, :, -tail:],
                                      v[:, :, -tail:], n)

    def update(self, k, v, layer_idx, cache_kwargs=None):
        if k.shape[2] > 1:
            return k, v
        calls.append(("update", layer_idx, tuple(k.shape)))
        self.exact_seq_lens[layer_idx] += 1
        self.total_seq_lens[layer_idx] += 1
        return k, v

    def decode(q, cache, layer_idx, scaling=None):
        calls.append(("decode", layer_idx, tuple(q.shape), cache.get_seq_length(layer_idx)))
        return torch.zeros_like(q)

    monkeypatch.setattr(attention, "delta_prefill_attention", prefill)
    monkeypatch.setattr(attention, "dense_prefill_attention", dense)
    monkeypatch.setattr(attention, "delta_decode_handoff", handoff)
    monkeypatch.setattr(HybridCompressedCache, "update", update)
    def step(self, q, k, v, layer_idx, scaling=None):   # decode_step = update + attention
        update(self, k, v, layer_idx)
        return decode(q, self, layer_idx, scaling)

    monkeypatch.setattr(deltaDecoding, "decode_attention", decode)
    monkeypatch.setattr(HybridCompressedCache, "decode_step", step)
    return calls


@pytest.mark.parametrize("impl", ["deltaattention", "deltaattention_dense"])
def test_prefill_hands_off_and_decode_runs_path3(monkeypatch, impl):
    from deltaattention_amd import globVR
    from deltaattention_amd.deltaDecoding import HybridCompressedCache
    monkeypatch.setattr(globVR, "delta_decode", True, raising=False)
    monkeypatch.setattr(globVR, "time_internal", False, raising=False)
    monkeypatch.setattr(globVR, "kv_log_interval", 4, raising=False)
    monkeypatch.setattr(globVR, "kv_compression_samples", [], raising=False)
    cfg, model = _tiny_model(impl)
    calls = _stub(monkeypatch)
    cache = HybridCompressedCache(cfg, 1, dtype=torch.float32, exact_window_size=4,
                                  initial_capacity=16, device="cpu")
    ids = torch.randint(0, 64, (1, 13))
    with torch.no_grad():
        model.model(input_ids=ids[:, :10], past_key_values=cache, use_cache=True)
        assert [cache.get_seq_length(i) for i in range(2)] == [10, 10]
        assert cache.max_packed_len == [10, 10] and cache.exact_seq_lens == [4, 4]
        for t in range(10, 13):
            out = model.model(input_ids=ids[:, t:t + 1], past_key_values=cache, use_cache=True)
            assert out.last_hidden_state.shape == (1, 1, 128)
    if impl == "deltaattention":
        assert calls[:2] == [("prefill", 0, True, (1, 4, 10, 32), (1, 2, 10, 32)),
                             ("prefill", 1, True, (1, 4, 10, 32), (1, 2, 10, 32))]
    else:
        assert calls[:4] == [("dense", (1, 4, 10, 32)), ("handoff", 0),
                             ("dense", (1, 4, 10, 32)), ("handoff", 1)]
    dec = [c for c in calls if c[0] in ("update", "decode")]
    # every decode token and layer: update, then attention over the updated cache
    assert dec == [x for t in range(3) for layer in range(2)
                   for x in (("update", layer, (1, 2, 1, 32)), ("decode", layer, (1, 4, 1, 32), 11 + t))]
    assert globVR.kv_compression_samples == [pytest.approx((1 - (4 + 10) / 12) * 100)]


def test_decode_before_any_prefill_is_refused(monkeypatch):
    from deltaattention_amd.deltaDecoding import HybridCompressedCache
    cfg, model = _tiny_model("deltaattention")
    _stub(monkeypatch)
    cache = HybridCompressedCache(cfg, 1, dtype=torch.float32, exact_window_size=4,
                                  initial_capacity=16, device="cpu")
    with torch.no_grad(), pytest.raises(RuntimeError, match="prefill hand-off"):
        model.model(input_ids=torch.zeros((1, 1), dtype=torch.long), past_key_values=cache,
                    use_cache=True)


def test_registered_implementation_refuses_a_continuation():
    """Under transformers' own forward the attention function cannot see the cache: a
    HybridCompressedCache hands it only the new token, so a continuation (positions not
    starting at 0) must raise instead of attending to that token alone."""
    from deltaattention_amd import llama_swap
    module = types.SimpleNamespace(layer_idx=0)
    q = torch.zeros(1, 4, 1, 32)
    k = torch.zeros(1, 2, 1, 32)
    with pytest.raises(NotImplementedError, match="install"):
        llama_swap.delta_attention_forward(module, q, k, k, None, position_ids=torch.tensor([[7]]))
    with pytest.raises(NotImplementedError, match="install"):
        llama_swap.dense_attention_forward(module, q, k, k, None, position_ids=torch.tensor([[7]]))
    with pytest.raises(NotImplementedError, match="query length"):
        llama_swap.delta_attention_forward(module, q, torch.zeros(1, 2, 5, 32), k, None)


def test_without_compressed_cache_the_registered_path_runs(monkeypatch):
    cfg, model = _tiny_model("deltaattention")
    calls = _stub(monkeypatch)
    with torch.no_grad():
        model.model(input_ids=torch.randint(0, 64, (1, 6)), use_cache=False)
    assert [c[0] for c in calls] == ["prefill", "prefill"]
    assert all(c[2] is False for c in calls)     # no cache reaches the prefill


def test_other_implementations_dispatch_as_transformers_does():
    """A model switched to "eager" after install keeps transformers' own attention."""
    from deltaattention_amd import llama_swap
    cfg, model = _tiny_model("deltaattention")
    ids = torch.randint(0, 64, (1, 9))
    llama_swap.set_implementation(model, "eager")
    with torch.no_grad():
        ours = model(ids, use_cache=False).logits
    from transformers import LlamaForCausalLM
    ref = LlamaForCausalLM(cfg).eval()
    ref.load_state_dict(model.state_dict())
    ref.config._attn_implementation = "eager"
    with torch.no_grad():
        want = ref(ids, use_cache=False).logits
    assert torch.allclose(ours, want, atol=1e-5)
