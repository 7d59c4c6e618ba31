"""Randomized decode parity: 8 configurations drawn with a fixed seed (batch, KV heads,
GQA group, prefill length, window, steps, metric, threshold, 16-bit type, initial cache
capacity), each a prefill hand-off followed by decode steps that alternate between
cache.update + decode_attention and the one-call cache.decode_step.  The cache state is
bit-exact against the oracle (deltaDecoding.py:9-104, 181-233) and the attention within
max-abs 2e-2 (bf16) / 5e-3 (fp16) of it (deltaDecoding.py:236-362).

The same flow at head dimensions below 128 (the reference's decode kernels mask the
head dimension to BLOCK_D, deltaDecoding.py:20,28-29,255-268; config 0 has d = 64) and
at GQA groups above 8, which the attention scores in sub-groups of at most 8 heads."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from conftest import announce, oracle_arith
from oracle import delta_oracle as O
from oracle import select_oracle_c as OC
import test_gpu_dropin as T

pytestmark = pytest.mark.gpu


def _cases(n=8, seed=11):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        metric = "cosine" if rng.random() < 0.4 else "euclidean"
        out.append(dict(
            B=int(rng.choice([1, 1, 2])), Hkv=int(rng.choice([1, 2, 3])), G=int(rng.choice([1, 2, 4, 8])),
            N=int(rng.integers(130, 2000)), W=int(rng.choice([16, 50, 128])), steps=int(rng.integers(20, 120)),
            metric=metric, tau=float(rng.uniform(0.8, 0.97)) if metric == "cosine" else float(rng.uniform(7.0, 13.0)),
            fp16=bool(rng.random() < 0.4), cap0=int(rng.choice([16, 64, 512])),
            seed=int(rng.integers(0, 1000)), pattern=int(rng.integers(0, 1 << 30))))
    return out


CASES = _cases()


def _id(c):
    return (f"B{c['B']}-Hkv{c['Hkv']}-G{c['G']}-N{c['N']}-W{c['W']}-T{c['steps']}-{c['metric'][:3]}-"
            f"{'f16' if c['fp16'] else 'bf16'}-cap{c['cap0']}")


# (B, Hkv, G, D, N, W, steps, metric, tau at D = 128, fp16): config 0's shape (8 KV heads,
# no GQA, d = 64), d = 96 under GQA 4, and groups of 9, 12 and 16 query heads (sub-groups
# of 5 + 4 with one repeated slot, 6 + 6 and 8 + 8)
DIM_CASES = [
    dict(B=1, Hkv=8, G=1, D=64, N=1500, W=128, steps=40, metric="euclidean", tau=9.0, fp16=False),
    dict(B=2, Hkv=2, G=4, D=96, N=900, W=50, steps=60, metric="cosine", tau=0.9, fp16=True),
    dict(B=1, Hkv=2, G=4, D=96, N=1200, W=128, steps=50, metric="euclidean", tau=10.0, fp16=False),
    dict(B=1, Hkv=1, G=12, D=64, N=700, W=16, steps=40, metric="euclidean", tau=8.0, fp16=False),
    dict(B=1, Hkv=2, G=16, D=128, N=800, W=128, steps=30, metric="cosine", tau=0.75, fp16=False),
    dict(B=2, Hkv=1, G=9, D=96, N=600, W=50, steps=30, metric="euclidean", tau=11.0, fp16=True),
]
for _i, _c in enumerate(DIM_CASES):
    _c.update(cap0=64, seed=100 + _i, pattern=7919 * (_i + 1))


def _dim_id(c):
    return f"D{c['D']}-G{c['G']}-Hkv{c['Hkv']}-B{c['B']}-{c['metric'][:3]}-{'f16' if c['fp16'] else 'bf16'}"


# fp32 caches (the reference's decode kernels take the cache's own type, deltaDecoding.py:
# 101-104, 303-325): config 0's model is fp32 (8 KV heads, d = 64, no GQA), then GQA 4 at
# d = 128 with the cosine test and a group of 12 (two sub-groups of 6)
FP32_CASES = [
    dict(B=1, Hkv=8, G=1, D=64, N=2048, W=128, steps=40, metric="euclidean", tau=9.0, fp16=False),
    dict(B=2, Hkv=2, G=4, D=128, N=900, W=50, steps=60, metric="cosine", tau=0.9, fp16=False),
    dict(B=1, Hkv=1, G=12, D=96, N=700, W=16, steps=40, metric="euclidean", tau=10.0, fp16=False),
]
for _i, _c in enumerate(FP32_CASES):
    _c.update(cap0=64, seed=200 + _i, pattern=104729 * (_i + 1), fp32=True)


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_random_decode_vs_oracle(gpu, c):
    _run_case(gpu, c, _id(c))


@pytest.mark.parametrize("c", DIM_CASES, ids=[_dim_id(c) for c in DIM_CASES])
def test_decode_head_dims_and_large_groups(gpu, c):
    # the Euclidean threshold scales with the distance, i.e. with sqrt(D)
    c = dict(c, tau=c["tau"] * (c["D"] / 128) ** 0.5 if c["metric"] == "euclidean" else c["tau"])
    _run_case(gpu, c, _dim_id(c))


@pytest.mark.parametrize("c", FP32_CASES, ids=[_dim_id(c).replace("bf16", "fp32") for c in FP32_CASES])
def test_decode_fp32_cache(gpu, c):
    """fp32 prefill, hand-off and decode: the cache state bit-exact against the oracle, the
    attention (fp32 P.V, unrounded as in the reference on fp32 tensors) within max-abs 1e-4
    of it, through both the one-call step and update + attention."""
    c = dict(c, tau=c["tau"] * (c["D"] / 128) ** 0.5 if c["metric"] == "euclidean" else c["tau"])
    _run_case(gpu, c, _dim_id(c).replace("bf16", "fp32"))


def _run_case(gpu, c, name):
    from deltaattention_amd import attention, globVR, synth
    from deltaattention_amd.deltaDecoding import HybridCompressedCache, decode_attention
    B, Hkv, N, W, steps = c["B"], c["Hkv"], c["N"], c["W"], c["steps"]
    D = c.get("D", 128)
    Hq = c["G"] * Hkv
    dtype = torch.float32 if c.get("fp32") else (torch.float16 if c["fp16"] else torch.bfloat16)
    announce(f"decode {name} tau={c['tau']:.3f}")
    q, k, v = (t.to(dtype) for t in synth.make_layer_inputs(B, Hq, Hkv, N + steps, D, seed=c["seed"],
                                                              rope_base=10000.0))
    cfg = SimpleNamespace(hidden_size=Hq * D, num_attention_heads=Hq, num_key_value_heads=Hkv,
                          num_hidden_layers=1, head_dim=D)
    saved = dict(vars(globVR))
    try:
        globVR.packing_mode, globVR.chunk_size = "delta", 512
        globVR.row_delta_threshold, globVR.row_similarity_metric = c["tau"], c["metric"]
        globVR.time_internal = False
        cache = HybridCompressedCache(cfg, B, dtype=dtype, exact_window_size=W, initial_capacity=c["cap0"])
        qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
        attention.delta_prefill_attention(qg[:, :, :N], kg[:, :, :N], vg[:, :, :N], 0, cache)
        kf, vf = k.float().numpy(), v.float().numpy()
        keep, _ = OC.select_delta(kf[:, :, :N], c["tau"], 512, 0, c["metric"], arith=oracle_arith(k))
        p = O.pack(kf[:, :, :N], vf[:, :, :N], keep)
        st = T._oracle_cache_from_prefill(p, kf[:, :, :N], vf[:, :, :N], W, cache.capacity + 4096)
        fused = np.random.default_rng(c["pattern"]).random(steps) < 0.5
        worst = 0.0
        for t in range(steps):
            sl = slice(N + t, N + t + 1)
            if fused[t]:
                out = cache.decode_step(qg[:, :, sl], kg[:, :, sl], vg[:, :, sl], 0)
            else:
                cache.update(kg[:, :, sl], vg[:, :, sl], 0)
                out = decode_attention(qg[:, :, sl], cache, 0)
            O.decode_update(st, kf[:, :, sl], vf[:, :, sl], c["tau"], c["metric"])
            if t % 17 == 0 or t == steps - 1:
                ref = O.decode_attention(q.float().numpy()[:, :, N + t], st)
                worst = max(worst, float(np.abs(out[:, :, 0].float().cpu().numpy() - ref).max()))
        n = int(cache.packed_lengths[0].max().item())
        assert (cache.packed_lengths[0].cpu().numpy() == st["lengths"]).all()
        assert (cache.packed_counts[0, :, :, :n].cpu().numpy() == st["counts"][:, :, :n]).all()
        assert (cache.packed_timestamps[0, :, :, :n].cpu().numpy() == st["timestamps"][:, :, :n]).all()
        assert torch.equal(cache.k_packed[0, :, :, :n].float().cpu(), torch.from_numpy(st["k_packed"][:, :, :n]))
        assert torch.equal(cache.v_packed[0, :, :, :n].float().cpu(), torch.from_numpy(st["v_packed"][:, :, :n]))
        assert torch.equal(cache.k_exact[0].float().cpu(), torch.from_numpy(st["k_exact"]))
        assert cache.get_seq_length(0) == N + steps
        print(f"{name}: attention max-abs {worst:.3e}, packed {n} of {N + steps}", flush=True)
        assert worst <= (1e-4 if c.get("fp32") else 5e-3 if c["fp16"] else 2e-2)
    finally:
        for name, val in saved.items():
            setattr(globVR, name, val)
