"""The reference-named modules, called the way modeling_llama.py calls them, and the
decode path against the oracle's state machine."""
import numpy as np
import pytest
import torch

from conftest import announce, oracle_arith
from oracle import delta_oracle as O
from oracle import select_oracle_c as OC

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-2, 1e-3


def _inputs(B, Hq, Hkv, N, seed):
    from deltaattention_amd import synth
    return synth.make_layer_inputs(B, Hq, Hkv, N, 128, seed=seed, rope_base=10000.0)


def _close(got, want, what):
    got = np.asarray(got, dtype=np.float32)
    err = np.abs(got - np.asarray(want, dtype=np.float32))
    print(f"{what}: max-abs {err.max():.3e} mean-abs {err.mean():.3e}", flush=True)
    assert np.isfinite(got).all()
    assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS, (what, err.max(), err.mean())


def _expand(t, G):
    """repeat_kv (modeling_llama.py:223-232)."""
    B, H, N = t.shape[:3]
    return t[:, :, None].expand(B, H, G, *t.shape[2:]).reshape(B, H * G, *t.shape[2:])


def test_flash_wrappers(gpu):
    from deltaattention_amd.flashAttention import _attn_fwd_flat, triton_flash_attention
    q, k, v = _inputs(1, 8, 2, 600, 1)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    announce("triton_flash_attention GQA + expanded, _attn_fwd_flat launch")
    a = triton_flash_attention(qg, kg, vg)
    b = triton_flash_attention(qg, _expand(kg, 4), _expand(vg, 4))
    out = torch.empty_like(qg)
    ke, ve = _expand(kg, 4).contiguous(), _expand(vg, 4).contiguous()
    _attn_fwd_flat[(5, 8, 1)](qg, ke, ve, 128 ** -0.5, out, *qg.stride(), *ke.stride(), *ve.stride(),
                              *out.stride(), 1, 8, 600, HEAD_DIM=128, BLOCK_M=128, BLOCK_N=128,
                              IS_CAUSAL=True, num_warps=8, num_stages=3)
    ref = O.dense_attention(q.float().numpy(), k.float().numpy(), v.float().numpy())
    for t, name in ((a, "gqa"), (b, "expanded"), (out, "kernel object")):
        _close(t.float().cpu().numpy(), ref, f"flash {name}")


def test_select_and_pack_kernel_objects(gpu):
    """chunked_eval_kernel / parallel_scatter_pack_kv_kernel launched as in
    modeling_llama.py:634-685."""
    from deltaattention_amd.tritonModules import chunked_eval_kernel, parallel_scatter_pack_kv_kernel
    q, k, v = _inputs(1, 4, 2, 1100, 2)
    kg, vg = k.to(gpu), v.to(gpu)
    bsz, H, q_len, D = kg.shape
    chunk_size, num_chunks = 512, 3
    keep_mask = torch.zeros((bsz, H, q_len), dtype=torch.int32, device=gpu)
    chunk_counts = torch.zeros((bsz, H, num_chunks), dtype=torch.int32, device=gpu)
    announce("chunked_eval_kernel object")
    chunked_eval_kernel[(bsz * H, num_chunks)](
        kg, keep_mask, chunk_counts, 9.0 ** 2, *kg.stride(), *keep_mask.stride(),
        *chunk_counts.stride(), q_len, D, chunk_size, num_heads=H, BLOCK_D=128, USE_COSINE=False)
    ok, occ = OC.select_delta(k.float().numpy(), 9.0, 512, arith=oracle_arith(k))
    assert (keep_mask.cpu().numpy() == ok).all() and (chunk_counts.cpu().numpy() == occ).all()
    index_map = (torch.cumsum(keep_mask, dim=-1) - 1).to(torch.int32)
    P = int(chunk_counts.sum(-1).max().item())
    k_packed = torch.zeros((bsz, H, P, D), device=gpu, dtype=kg.dtype)
    v_packed = torch.zeros_like(k_packed)
    ts = torch.zeros((bsz, H, P), device=gpu, dtype=torch.int32)
    announce("parallel_scatter_pack_kv_kernel object")
    parallel_scatter_pack_kv_kernel[(bsz * H, (q_len + 63) // 64)](
        kg, vg, k_packed, v_packed, ts, keep_mask, index_map, *kg.stride(), *vg.stride(),
        *k_packed.stride(), *v_packed.stride(), *ts.stride(), *keep_mask.stride(),
        *index_map.stride(), q_len, D, H, BLOCK_S=64, BLOCK_D=128)
    ref = O.pack(k.float().numpy(), v.float().numpy(), ok)
    assert (ts.cpu().numpy() == ref["timestamps"]).all()
    assert torch.equal(k_packed.float().cpu(), torch.from_numpy(ref["k_packed"]))
    assert torch.equal(v_packed.float().cpu(), torch.from_numpy(ref["v_packed"]))


@pytest.mark.parametrize("variant", ["hybrid", "sanity", "pure_phase1"])
def test_hybrid_kernel_objects_on_expanded_inputs(gpu, variant):
    """hybrid kernels launched as modeling_llama.py:334-353 on repeat_kv-expanded tensors
    equal the GQA-native path and the oracle."""
    from deltaattention_amd import deltaFlashAttention as dfa
    from deltaattention_amd import ops
    q, k, v = _inputs(1, 8, 2, 1300, 3)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    keep, _ = ops.select(kg, 9.0, 512)
    pk = ops.pack(keep, kg, vg).trimmed()
    G = 4
    ke, ve = _expand(kg, G).contiguous(), _expand(vg, G).contiguous()
    kpe, vpe = _expand(pk.k_packed, G).contiguous(), _expand(pk.v_packed, G).contiguous()
    tse = _expand(pk.timestamps, G).contiguous()
    cne = _expand(pk.counts, G).contiguous().float()
    out = torch.empty_like(qg)
    kern = {"hybrid": dfa.hybrid_compressed_flash_kernel,
            "sanity": dfa.hybrid_compressed_flash_kernel_sanity,
            "pure_phase1": dfa.pure_phase1_flash_kernel}[variant]
    announce(f"{variant} kernel object, expanded inputs")
    kern[(11, 8, 1)](qg, ke, ve, kpe, vpe, tse, cne, out, *qg.stride(), *ke.stride(), *ve.stride(),
                     *kpe.stride(), *vpe.stride(), *tse.stride(), *cne.stride(), *out.stride(),
                     128 ** -0.5, 1300, 1300, kpe.shape[2], 128, 8, 128,
                     BLOCK_M=128, BLOCK_N=128, BLOCK_D=128, num_warps=8, num_stages=1)
    native = ops.hybrid_prefill(qg, kg, vg, pk.k_packed, pk.v_packed, pk.timestamps, pk.counts,
                                window=128, variant=variant)
    # The expanded inputs run the per-head kernel (exact running max, weights multiplied
    # after exp2), the GQA-native call the grouped kernel (lazy running max, weights as
    # key biases): P is rounded to bf16 at different reference points, so the two agree
    # to that rounding -- the bar the oracle applies to each of them.
    _close(out.float().cpu().numpy(), native.float().cpu().numpy(), f"{variant} object vs native")
    kf, vf = k.float().numpy(), v.float().numpy()
    p = O.pack(kf, vf, keep.cpu().numpy())
    ref = O.hybrid_attention(q.float().numpy(), kf, vf, p["k_packed"], p["v_packed"],
                             p["timestamps"], p["counts"], 128, variant=variant)
    _close(out.float().cpu().numpy(), ref, f"{variant} object")


@pytest.mark.parametrize("mode", ["delta", "periodic"])
def test_delta_prefill_attention_glue(gpu, mode):
    """PATH 1 (modeling_llama.py:600-749) with the globVR knobs of eval_speedup.set_row_delta."""
    from deltaattention_amd import attention, globVR
    q, k, v = _inputs(1, 8, 2, 1500, 4)
    saved = dict(vars(globVR))
    try:
        globVR.packing_mode = mode
        globVR.row_delta_threshold = 9.0
        globVR.row_similarity_metric = "euclidian"
        globVR.chunk_size = 512
        globVR.target_keep_rate = 0.3
        globVR.dense_window_size = 128
        globVR.time_internal = False
        announce(f"delta_prefill_attention mode={mode}")
        out = attention.delta_prefill_attention(q.to(gpu), k.to(gpu), v.to(gpu))
        kf, vf = k.float().numpy(), v.float().numpy()
        keep = OC.select_delta(kf, 9.0, 512, arith=oracle_arith(k))[0] if mode == "delta" else O.select_periodic(1, 2, 1500, 0.3)
        p = O.pack(kf, vf, keep)
        ref = O.hybrid_attention(q.float().numpy(), kf, vf, p["k_packed"], p["v_packed"],
                                 p["timestamps"], p["counts"], 128)
        _close(out.float().cpu().numpy(), ref, f"glue {mode}")
        assert 0.0 < globVR.spars < 1.0
    finally:
        for name, val in saved.items():
            setattr(globVR, name, val)


def _oracle_cache_from_prefill(p, k, v, W, cap):
    B, H, N, D = k.shape
    P = p["P"]
    st = O_decode_state(B, H, D, cap, W)
    st["k_packed"][:, :, :P] = p["k_packed"]
    st["v_packed"][:, :, :P] = p["v_packed"]
    st["counts"][:, :, :P] = p["counts"]
    st["timestamps"][:, :, :P] = p["timestamps"]
    st["lengths"][:] = P
    e = min(N, W)
    st["k_exact"][:, :, :e] = k[:, :, -e:]
    st["v_exact"][:, :, :e] = v[:, :, -e:]
    st["exact_len"], st["total_len"] = e, N
    return st


def O_decode_state(B, H, D, cap, W):
    return {"k_packed": np.zeros((B, H, cap, D), np.float32), "v_packed": np.zeros((B, H, cap, D), np.float32),
            "counts": np.zeros((B, H, cap), np.int32), "timestamps": np.zeros((B, H, cap), np.int32),
            "lengths": np.zeros(B * H, np.int32), "k_exact": np.zeros((B, H, W, D), np.float32),
            "v_exact": np.zeros((B, H, W, D), np.float32), "exact_len": 0, "total_len": 0, "window": W}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("metric,tau", [("euclidean", 9.5), ("cosine", 0.9)])
def test_decode_cache_matches_oracle(gpu, metric, tau, dtype):
    """Prefill hand-off then 80 decode steps: cache state bit-exact and attention within
    tolerance against the oracle (deltaDecoding.py:9-362, modeling_llama.py:453-518)."""
    from types import SimpleNamespace
    from deltaattention_amd import attention, globVR, synth
    from deltaattention_amd.deltaDecoding import HybridCompressedCache, decode_attention
    B, Hq, Hkv, N, W, steps = 1, 8, 2, 700, 50, 80
    q, k, v = (t.to(dtype) for t in _inputs(B, Hq, Hkv, N + steps, 5))
    cfg = SimpleNamespace(hidden_size=Hq * 128, num_attention_heads=Hq, num_key_value_heads=Hkv,
                          num_hidden_layers=1, head_dim=128)
    saved = dict(vars(globVR))
    try:
        globVR.packing_mode, globVR.chunk_size = "delta", 512
        globVR.row_delta_threshold, globVR.row_similarity_metric = tau, metric
        globVR.time_internal = False
        cache = HybridCompressedCache(cfg, B, dtype=dtype, exact_window_size=W,
                                      initial_capacity=64)
        qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
        announce(f"decode {metric}: prefill hand-off")
        attention.delta_prefill_attention(qg[:, :, :N], kg[:, :, :N], vg[:, :, :N], 0, cache)
        kf, vf = k.float().numpy(), v.float().numpy()
        keep, _ = OC.select_delta(kf[:, :, :N], tau, 512, 0, metric, arith=oracle_arith(k))
        p = O.pack(kf[:, :, :N], vf[:, :, :N], keep)
        st = _oracle_cache_from_prefill(p, kf[:, :, :N], vf[:, :, :N], W, cache.capacity + 4096)
        outs = []
        for t in range(steps):
            if t == 0:
                announce(f"decode {metric} {dtype}: {steps} update+attention steps")
            cache.update(kg[:, :, N + t:N + t + 1], vg[:, :, N + t:N + t + 1], 0)
            outs.append(decode_attention(qg[:, :, N + t:N + t + 1], cache, 0))
            O.decode_update(st, kf[:, :, N + t:N + t + 1], vf[:, :, N + t:N + t + 1], tau, metric)
            if t in (0, steps - 1):
                ref = O.decode_attention(q.float().numpy()[:, :, N + t], st)
                _close(outs[-1][:, :, 0].float().cpu().numpy(), ref, f"decode attn step {t}")
        n = int(cache.packed_lengths[0].max().item())
        assert (cache.packed_lengths[0].cpu().numpy() == st["lengths"]).all()
        assert (cache.packed_counts[0, :, :, :n].cpu().numpy() == st["counts"][:, :, :n]).all()
        assert (cache.packed_timestamps[0, :, :, :n].cpu().numpy() == st["timestamps"][:, :, :n]).all()
        assert torch.equal(cache.k_packed[0, :, :, :n].float().cpu(), torch.from_numpy(st["k_packed"][:, :, :n]))
        assert torch.equal(cache.k_exact[0].float().cpu(), torch.from_numpy(st["k_exact"]))
        assert cache.get_seq_length(0) == N + steps
        merged = int(st["counts"].sum()) - N
        print(f"decode {metric}: evicted {steps} tokens, packed length {n}, merged-in {merged}")
    finally:
        for name, val in saved.items():
            setattr(globVR, name, val)


def _misaligned(t):
    """A copy of t whose data starts 8 bytes past a 16-byte boundary: da_decode_step then
    takes its unfused path (update kernel, then attention)."""
    buf = torch.empty(t.numel() + 4, dtype=t.dtype, device=t.device)
    out = buf[4:].view(t.shape)
    out.copy_(t)
    assert out.data_ptr() % 16 == 8
    return out


def _decode_twins(gpu, dtype, Hq, Hkv, steps, cap0, grow, seed=11, W=16):
    """Two caches fed the same tokens: cache a by cache.update + decode_attention, cache b
    by cache.decode_step.  Even steps hand decode_step 16-byte aligned key/value rows (the
    fused launch pair: the update folded into the attention); odd steps misaligned ones (the
    unfused path, which must equal the two calls bit for bit).  The fused path's output
    is bit-identical for every KV head whose step merged, dropped or evicted nothing, and
    differs only in rounding where it appended: the evicted token then sits at the end of
    its key list instead of after the packed anchors, so the slice sums add the same terms
    in another order (bar: max-abs 1e-2 bf16, 2e-3 fp16).  The cache state must be
    bit-identical.  grow=False holds the capacity (the host
    tracker is kept below it), so a full cache drops evicted tokens that do not merge
    (deltaDecoding.py:83-96)."""
    from types import SimpleNamespace
    from deltaattention_amd.deltaDecoding import HybridCompressedCache, decode_attention
    B = 2
    q, k, v = (t.to(dtype) for t in _inputs(B, Hq, Hkv, steps, seed))
    cfg = SimpleNamespace(hidden_size=Hq * 128, num_attention_heads=Hq, num_key_value_heads=Hkv,
                          num_hidden_layers=2, head_dim=128)
    a = HybridCompressedCache(cfg, B, dtype=dtype, exact_window_size=W, initial_capacity=cap0)
    b = HybridCompressedCache(cfg, B, dtype=dtype, exact_window_size=W, initial_capacity=cap0)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    bar = 1e-2 if dtype == torch.bfloat16 else 2e-3
    worst, exact_heads = 0.0, 0
    for t in range(steps):
        if not grow:
            a.max_packed_len[1] = b.max_packed_len[1] = -steps
        qt, kt, vt = qg[:, :, t:t + 1], kg[:, :, t:t + 1], vg[:, :, t:t + 1]
        a.update(kt, vt, 1)
        want = decode_attention(qt, a, 1, scaling=0.07)
        if t % 2:
            got = b.decode_step(qt, _misaligned(kt), _misaligned(vt), 1, scaling=0.07)
            assert torch.equal(got, want), t
        else:
            before = b.packed_lengths[1].clone()
            got = b.decode_step(qt, kt, vt, 1, scaling=0.07)
            err = float((got.float() - want.float()).abs().max())
            worst = max(worst, err)
            assert err <= bar, (t, err)
            appended = (b.packed_lengths[1] != before).reshape(B, Hkv)
            same = ~appended.repeat_interleave(Hq // Hkv, dim=1)   # [B, Hq]
            assert torch.equal(got[same], want[same]), t
            exact_heads += int(same.sum())
        assert got.shape == want.shape == (B, Hq, 1, 128)
    assert (b.exact_seq_lens, b.total_seq_lens) == (a.exact_seq_lens, a.total_seq_lens)
    for name in ("packed_lengths", "packed_counts", "packed_timestamps", "k_packed",
                 "v_packed", "k_exact", "v_exact"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    assert 0 < exact_heads < B * Hq * ((steps + 1) // 2)
    return a, b, worst


@pytest.mark.parametrize("metric,tau,dtype,Hq,Hkv", [
    ("euclidean", 9.5, torch.bfloat16, 8, 2),
    ("cosine", 0.9, torch.bfloat16, 8, 2),
    ("euclidean", 9.5, torch.float16, 16, 2),   # fp16 cache, GQA group 8
], ids=["euclidean-bf16-G4", "cosine-bf16-G4", "euclidean-fp16-G8"])
def test_decode_step_equals_update_then_attention(gpu, metric, tau, dtype, Hq, Hkv):
    """HybridCompressedCache.decode_step (one da_decode_step call per token) against
    cache.update + decode_attention on a twin cache, through ring fill, eviction into the
    packed cache and a capacity growth (initial capacity 8) that rebuilds the cached
    argument block: the cache state bit-identical after 96 tokens, the unfused path's
    outputs bit-identical and the fused path's within rounding."""
    from deltaattention_amd import globVR
    B, W, steps = 2, 16, 96
    saved = dict(vars(globVR))
    try:
        globVR.row_delta_threshold, globVR.row_similarity_metric = tau, metric
        announce(f"decode_step {metric}: {steps} steps on layer 1, Hq={Hq} Hkv={Hkv} W={W}")
        a, b, worst = _decode_twins(gpu, dtype, Hq, Hkv, steps, 8, True)
        assert b.capacity == a.capacity > 8
        n = int(a.packed_lengths[1].max().item())
        assert 0 < n < B * Hkv * (steps - W)
        merged = int(a.packed_counts[1].sum().item()) - int(a.packed_lengths[1].sum().item())
        assert merged > 0   # both decisions occur
        x = torch.zeros((B, Hq, 1, 128), dtype=dtype, device=gpu)
        with pytest.raises(ValueError):   # one KV head where the cache has Hkv
            b.decode_step(x, x[:, :1], x[:, :1], 1)
        print(f"decode_step {metric}: packed length {n}, merged {merged}, fused max-abs {worst:.3e}",
              flush=True)
    finally:
        for name, val in saved.items():
            setattr(globVR, name, val)


@pytest.mark.parametrize("W", [1, 3])
def test_decode_step_small_rings(gpu, W):
    """Rings of one and three slots: from the second token (W = 1) or the fourth on, every
    step evicts, and the new token's slot rotates through the ring while the packed list
    grows past capacity 8 (a rebuilt argument block)."""
    from deltaattention_amd import globVR
    saved = dict(vars(globVR))
    try:
        globVR.row_delta_threshold, globVR.row_similarity_metric = 9.5, "euclidean"
        announce(f"decode_step with a ring of {W}")
        a, b, worst = _decode_twins(gpu, torch.bfloat16, 8, 2, 40, 8, True, W=W)
        assert a.capacity > 8
        print(f"decode_step W={W}: packed length {int(a.packed_lengths[1].max())}, fused max-abs {worst:.3e}",
              flush=True)
    finally:
        for name, val in saved.items():
            setattr(globVR, name, val)


def test_decode_step_full_cache_drops_like_update(gpu):
    """A packed cache held at capacity 8: evicted tokens that do not merge are dropped
    (deltaDecoding.py:83-96), in the fused step as in the update kernel; the dropped
    token gets no weight in the fused attention (count 0)."""
    from deltaattention_amd import globVR
    saved = dict(vars(globVR))
    try:
        globVR.row_delta_threshold, globVR.row_similarity_metric = 9.5, "euclidean"
        announce("decode_step at capacity 8: drops")
        a, b, worst = _decode_twins(gpu, torch.bfloat16, 8, 2, 64, 8, False)
        assert a.capacity == 8
        assert (a.packed_lengths[1] == 8).all()
        kept = int(a.packed_counts[1].sum().item())
        assert kept < 2 * 2 * (64 - 16)     # some evicted tokens were dropped
        print(f"decode_step full cache: {kept} of {2 * 2 * (64 - 16)} evicted tokens kept, "
              f"fused max-abs {worst:.3e}", flush=True)
    finally:
        for name, val in saved.items():
            setattr(globVR, name, val)


@pytest.mark.parametrize("B,Hq,Hkv,cap,W,exact,dtype", [
    (1, 32, 8, 40000, 128, 128, torch.bfloat16),   # dense-like length: 600+ slices per head
    (1, 32, 8, 40000, 128, 128, torch.float16),
    (2, 8, 8, 3000, 128, 77, torch.bfloat16),      # G = 1
    (1, 16, 2, 20000, 64, 0, torch.bfloat16),      # G = 8, empty ring
    (1, 12, 4, 1000, 128, 5, torch.bfloat16),      # G = 3, one head with no anchors
], ids=["G4-40k-bf16", "G4-40k-fp16", "G1-B2", "G8-ring0", "G3-empty-head"])
def test_decode_attention_kernel_vs_oracle(gpu, B, Hq, Hkv, cap, W, exact, dtype):
    """da_decode_attention on a synthetic cache against the oracle (deltaDecoding.py:236-362):
    per-head packed lengths, counts with zero-count padding slots, key norms spread so that
    the maximum moves between slices, and the slice merge over up to 600+ slices."""
    from deltaattention_amd.deltaDecoding import _decode_attention_launch
    D = 128
    rng = np.random.default_rng(B * 1000 + Hq * 10 + Hkv)
    lens = rng.integers(cap // 2, cap + 1, size=B * Hkv).astype(np.int32)
    if Hkv == 4:
        lens[1] = 0
    kp = rng.standard_normal((B, Hkv, cap, D)).astype(np.float32)
    kp *= rng.uniform(0.3, 2.5, size=(B, Hkv, cap, 1)).astype(np.float32)
    vp = rng.standard_normal((B, Hkv, cap, D)).astype(np.float32)
    cnt = rng.integers(1, 9, size=(B, Hkv, cap)).astype(np.int32)
    cnt[rng.random((B, Hkv, cap)) < 0.05] = 0
    kx = rng.standard_normal((B, Hkv, W, D)).astype(np.float32)
    vx = rng.standard_normal((B, Hkv, W, D)).astype(np.float32)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dtype)
    kp_t, vp_t, kx_t, vx_t, q_t = t(kp), t(vp), t(kx), t(vx), t(q)
    st = {"k_packed": kp_t.float().numpy(), "v_packed": vp_t.float().numpy(), "counts": cnt,
          "lengths": lens, "k_exact": kx_t.float().numpy(), "v_exact": vx_t.float().numpy(),
          "exact_len": exact, "window": W}
    want = O.decode_attention(q_t.float().numpy(), st)
    g = lambda x: x.to(gpu)
    kp_g, vp_g, kx_g, vx_g, q_g = g(kp_t), g(vp_t), g(kx_t), g(vx_t), g(q_t)
    cnt_g, lens_g = g(torch.from_numpy(cnt)), g(torch.from_numpy(lens))
    out = torch.empty((B, Hq, D), dtype=dtype, device=gpu)
    announce(f"da_decode_attention B={B} Hq={Hq} Hkv={Hkv} cap={cap} W={W} exact={exact} {dtype}")
    _decode_attention_launch(q_g, Hq * D, D, kp_g, vp_g, (Hkv * cap * D, cap * D, D), cnt_g,
                             (Hkv * cap, cap), lens_g, kx_g, vx_g, (Hkv * W * D, W * D, D), W,
                             exact, D ** -0.5, out, Hq * D, D, B, Hq, Hkv, D, "decode attention")
    torch.cuda.synchronize()
    _close(out.float().cpu().numpy(), want, f"decode attention G={Hq // Hkv} cap={cap}")
