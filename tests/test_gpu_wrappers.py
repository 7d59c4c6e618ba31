"""The reference-named wrappers (modeling_llama.py:306-451) on the GPU against the oracle:
attention.forward_hybrid_flash / forward_hybrid_flash_sanity / forward_pure_phase1, called
the way the reference calls them (K, V and the packed tensors repeat_kv-expanded to the
query heads, counts int32 converted to fp32 inside) and with the KV heads not expanded,
with globVR.no_count off and on (the sanity wrapper ignores it, as the reference's does).
"""
import numpy as np
import pytest
import torch

from conftest import announce, oracle_arith
from oracle import delta_oracle as O
from oracle import select_oracle_c as OC

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 1e-3


def _repeat_kv(x, n):
    """modeling_llama.py:223-232 on [B, H, ...] tensors (3-D or 4-D)."""
    return x.repeat_interleave(n, dim=1).contiguous()


@pytest.fixture(scope="module")
def layer(gpu):
    from deltaattention_amd import ops, synth
    q, k, v = synth.make_layer_inputs(1, 8, 2, 2048, 128, seed=31, rope_base=10000.0)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    keep, _ = ops.select(kg, 10.0, 512)
    p = ops.pack(keep, kg, vg).trimmed()
    kf, vf = k.float().numpy(), v.float().numpy()
    okeep, _ = OC.select_delta(kf, 10.0, 512, arith=oracle_arith(kg))
    ref = O.pack(kf, vf, okeep)
    assert p.k_packed.shape[2] == ref["P"]
    return dict(q=qg, k=kg, v=vg, p=p, qf=q.float().numpy(), kf=kf, vf=vf, ref=ref)


@pytest.mark.parametrize("no_count", [False, True], ids=["counts", "no_count"])
@pytest.mark.parametrize("expanded", [True, False], ids=["repeat_kv", "kv_heads"])
@pytest.mark.parametrize("variant", ["hybrid", "sanity", "pure_phase1"])
def test_reference_wrappers(gpu, layer, monkeypatch, variant, expanded, no_count):
    from deltaattention_amd import attention, globVR
    monkeypatch.setattr(globVR, "no_count", no_count, raising=False)
    fn = {"hybrid": attention.forward_hybrid_flash,
          "sanity": attention.forward_hybrid_flash_sanity,
          "pure_phase1": attention.forward_pure_phase1}[variant]
    L, p = layer, layer["p"]
    G = 4
    args = [L["k"], L["v"], p.k_packed, p.v_packed, p.timestamps, p.counts]
    if expanded:
        args = [_repeat_kv(a, G) for a in args]
    announce(f"wrapper {variant} {'expanded' if expanded else 'kv heads'} no_count={no_count}")
    out = fn(L["q"], *args, 128)
    assert out.shape == L["q"].shape and out.dtype == L["q"].dtype
    r = L["ref"]
    want = O.hybrid_attention(L["qf"], L["kf"], L["vf"], r["k_packed"], r["v_packed"], r["timestamps"],
                              r["counts"], 128, variant=variant,
                              no_count=no_count and variant != "sanity")
    err = np.abs(out.float().cpu().numpy() - want)
    print(f"{variant} expanded={expanded} no_count={no_count}: max-abs {err.max():.3e} "
          f"mean-abs {err.mean():.3e}", flush=True)
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS


@pytest.mark.parametrize("variant", ["hybrid", "sanity", "pure_phase1", "dense"])
def test_reference_wrappers_fp32(gpu, variant):
    """The same wrappers and the dense drop-in (flashAttention.triton_flash_attention,
    flashAttention.py:94-130) on fp32 tensors, which the reference's kernels take as they
    take 16-bit ones: the selection runs in fp32, the output is fp32, within 1e-5 of the
    fp32 oracle."""
    from deltaattention_amd import attention, flashAttention, ops, synth
    q, k, v = synth.make_layer_inputs(1, 8, 2, 1536, 128, seed=37, rope_base=10000.0, dtype=torch.float32)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    qf, kf, vf = q.numpy(), k.numpy(), v.numpy()
    announce(f"fp32 wrapper {variant}")
    if variant == "dense":
        out = flashAttention.triton_flash_attention(qg, _repeat_kv(kg, 4), _repeat_kv(vg, 4))
        want = O.dense_attention(qf, kf, vf, True)
    else:
        keep, _ = ops.select(kg, 10.0, 512)
        p = ops.pack(keep, kg, vg).trimmed()
        okeep, _ = OC.select_delta(kf, 10.0, 512, arith="fp32")
        ref = O.pack(kf, vf, okeep)
        assert np.array_equal(keep.cpu().numpy(), okeep) and p.k_packed.shape[2] == ref["P"]
        fn = {"hybrid": attention.forward_hybrid_flash, "sanity": attention.forward_hybrid_flash_sanity,
              "pure_phase1": attention.forward_pure_phase1}[variant]
        out = fn(qg, kg, vg, p.k_packed, p.v_packed, p.timestamps, p.counts, 128)
        want = O.hybrid_attention(qf, kf, vf, ref["k_packed"], ref["v_packed"], ref["timestamps"], ref["counts"],
                                  128, variant=variant)
    assert out.dtype == torch.float32 and out.shape == qg.shape
    err = np.abs(out.cpu().numpy() - want)
    print(f"fp32 {variant}: max-abs {err.max():.3e} mean-abs {err.mean():.3e}", flush=True)
    assert err.max() <= 1e-5 and err.mean() <= 1e-6
