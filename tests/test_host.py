"""Host-side logic: chunking, the schedule and FLOP accounting, synthetic inputs."""
import numpy as np
import pytest
import torch

from deltaattention_amd import metrics, ops, synth
from oracle import delta_oracle as O


@pytest.mark.parametrize("n,cs,dt", [(1050, 100, 0), (300, 512, 0), (10, 0, 4), (3, 0, 5), (7, 0, 0)])
def test_chunking_matches_oracle(n, cs, dt):
    assert ops.chunking(n, cs, dt) == O.chunking(n, cs, dt)


def test_metrics_schedule_matches_oracle():
    rng = np.random.default_rng(2)
    N = 2000
    keep = (rng.random((2, 3, N)) < 0.25).astype(np.int32)
    keep[..., 0] = 1
    keep[1, 2, 700:] = 0       # a short head -> fully padded blocks
    k = rng.standard_normal((2, 3, N, 8)).astype(np.float32)
    p = O.pack(k, k, keep)
    for W in (0, 128, 400):
        a = metrics.hybrid_schedule(p["timestamps"], p["P"], N, N, W)
        b = O.hybrid_schedule(p["timestamps"], p["P"], N, N, W)
        for x, y in zip(a, b[:3]):
            assert (np.asarray(x) == y).all()


def test_hybrid_flops_counts_pairs():
    """The algorithmic pair count equals the brute-force weighted-key count (real anchors
    only, plus dense keys ds..i per row)."""
    rng = np.random.default_rng(4)
    N, Hq, Hkv = 900, 4, 2
    keep = (rng.random((1, Hkv, N)) < 0.3).astype(np.int32)
    keep[..., 0] = 1
    k = rng.standard_normal((1, Hkv, N, 8)).astype(np.float32)
    p = O.pack(k, k, keep)
    W = 128
    fl = metrics.hybrid_flops(p["timestamps"], p["anchor_counts"], p["P"], N, Hq, 128, W)
    n_safe, last, ds, _ = O.hybrid_schedule(p["timestamps"], p["P"], N, N, W)
    pairs = 0
    for g in range(Hkv):
        for qb in range((N + 127) // 128):
            a = min(int(n_safe[0, g, qb]) * 128, int(p["anchor_counts"][0, g]))
            for i in range(qb * 128, min(N, qb * 128 + 128)):
                pairs += a + max(0, i - int(ds[0, g, qb]) + 1)
    assert fl["algorithmic"] == 4.0 * 128 * pairs * (Hq // Hkv)
    assert metrics.dense_flops(1, 32, 32768, 128) == pytest.approx(8.796e12, rel=1e-3)


def test_synth_is_deterministic_and_ar1():
    a = synth.ar1_keys(1, 2, 4000, 16, seed=3)
    b = synth.ar1_keys(1, 2, 4000, 16, seed=3)
    assert torch.equal(a, b)
    x = a.numpy()
    assert abs(x.var() - 1.0) < 0.15
    r = (x[:, :, 1:] * x[:, :, :-1]).mean() / x.var()
    assert abs(r - 0.9) < 0.03
    q, k, v = synth.make_layer_inputs(1, 4, 2, 256, 128, seed=1)
    assert q.dtype == torch.bfloat16 and k.shape == (1, 2, 256, 128) and q.shape == (1, 4, 256, 128)


def test_llama_swap_routes_attention_to_this_build():
    """The registered transformers attention implementations reach the native ops (on
    CPU tensors those refuse with 'no CPU path': there is no fallback)."""
    torch = pytest.importorskip("torch")
    pytest.importorskip("transformers")
    from transformers import AttentionInterface
    from deltaattention_amd import llama_swap
    llama_swap.register()
    assert llama_swap.DELTA in AttentionInterface._global_mapping
    assert llama_swap.DENSE in AttentionInterface._global_mapping
    for impl in (llama_swap.DELTA, llama_swap.DENSE):
        cfg = llama_swap.llama3_8b_config(impl, num_layers=1)
        cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size = 64, 256, 512
        cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim = 2, 1, 128
        model = llama_swap.random_llama(cfg, torch.device("cpu"))
        with pytest.raises(ValueError, match="no CPU path"):
            with torch.no_grad():
                model(torch.zeros(1, 8, dtype=torch.long), use_cache=False)


def test_dtype_code_accepts_one_data_type():
    import torch
    from deltaattention_amd._native import DA_BF16, DA_F16, DA_F32, dtype_code
    a = torch.zeros(2, dtype=torch.bfloat16)
    h = torch.zeros(2, dtype=torch.float16)
    f = torch.zeros(2, dtype=torch.float32)
    assert dtype_code(a, a, None) == DA_BF16
    assert dtype_code(h, h) == DA_F16
    assert dtype_code(f, f) == DA_F32
    with pytest.raises(TypeError):
        dtype_code(a, h)
    with pytest.raises(TypeError):
        dtype_code(f, a)
    with pytest.raises(TypeError):
        dtype_code(torch.zeros(2, dtype=torch.float64))


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N with N > 1 exits with status 2 and one JSON line saying why
    (one GPU per box; the path would shard by KV head)."""
    import json
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    rec = json.loads(r.stdout.strip().splitlines()[-1])
    assert rec["n_gpus"] == 2 and "one GPU" in rec["error"]
