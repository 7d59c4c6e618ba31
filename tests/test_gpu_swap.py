"""The modeling swap (llama_swap): a small Llama through the HIP attention path inside
transformers, against transformers' own fp32 eager attention on the same weights."""
import copy

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
