"""GPU parity on each BASELINE configuration's own workload, against the CPU oracle.

Every configuration runs the HIP path at its real shape and sizes:

* config 0: one layer, Hq = Hkv = 8, head_dim 64 (native, not padded), N = 2048, RoPE base
  1e4, r = 4 -- the whole output is compared;
* config 1: the benchmarked layer (B = 1, Hq = 32, Hkv = 8, D = 128, N = 32768, r = 4,
  the bench's own seeded inputs) -- selection and packing bit-exact at full size, the
  hybrid and dense outputs on query blocks spread from the first to the last;
* config 2: the same layer at N = 131072 for r in {2, 4, 8}, and at N = 262144 for r = 4
  (the reference's longest point);
* config 3: a Llama-3-8B-shaped model (4 layers) prefilling 65536 tokens through the
  transformers swap with periodic anchors (r = 4); every layer's attention is compared;
* config 4: a ragged batch of 8 sequences of 4096..32768 tokens with rho ~ U[0.6, 0.95]
  per (sequence, KV head), each sequence compared as a B = 1 prefill.

With Hkv = 8 and a GQA group of 4, configs 1-4 run the ping-pong kernel's XCD-aware grid
mapping (8 (batch, KV head) units), the launch behind every benchmarked number.

Bars: selection, keep masks, counts, timestamps and the packed rows are bit-exact;
attention outputs (bf16) are within max-abs 2e-2 and mean-abs 1e-3 of the fp32 oracle on
the same bf16 inputs (the tolerance BASELINE.json's north star states).
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


def _close(got, want, what):
    got = np.asarray(got, dtype=np.float32)
    want = np.asarray(want, dtype=np.float32)
    assert got.shape == want.shape
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - want)
    mx, mean = float(err.max()), float(err.mean())
    print(f"{what}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{what}: max-abs {mx:.3e}, mean-abs {mean:.3e}"


def _spread(nqb, n):
    """n query-block indexes from the first to the last."""
    return sorted(set(np.linspace(0, nqb - 1, n).round().astype(int).tolist()))


def _rows(blocks, N):
    return np.concatenate([np.arange(b * 128, min(N, b * 128 + 128)) for b in blocks])


def _check_select_pack(kg, vg, tau, keep, packed, what):
    """Keep mask, chunk counts and every packed tensor bit-exact against the oracle."""
    kf, vf = kg.float().cpu().numpy(), vg.float().cpu().numpy()
    ref_keep, _ = OC.select_delta(kf, tau, 512, arith=oracle_arith(kg))
    got_keep = keep.cpu().numpy()
    assert np.array_equal(got_keep, ref_keep), f"{what}: keep differs at {np.argwhere(got_keep != ref_keep)[:5]}"
    ref = O.pack(kf, vf, ref_keep)
    P = int(packed.num_packed.item())
    assert P == ref["P"], f"{what}: P {P} != {ref['P']}"
    assert np.array_equal(packed.anchor_counts.cpu().numpy(), ref["anchor_counts"])
    assert np.array_equal(packed.timestamps[:, :, :P].cpu().numpy(), ref["timestamps"])
    assert np.array_equal(packed.counts[:, :, :P].cpu().numpy(), ref["counts"])
    assert np.array_equal(packed.k_packed[:, :, :P].float().cpu().numpy(), ref["k_packed"])
    assert np.array_equal(packed.v_packed[:, :, :P].float().cpu().numpy(), ref["v_packed"])
    print(f"{what}: P={P} realised r={kf.shape[1] * kf.shape[2] / ref['anchor_counts'].sum():.3f}",
          flush=True)
    return kf, vf, ref


def _layer(N, seed, dev, rho=0.9, rope_base=500000.0, D=128, Hq=32, Hkv=8):
    """The bench's inputs: AR(1) keys from the CPU generator, Q and V drawn on the GPU."""
    from deltaattention_amd import synth
    q, k, v = synth.make_layer_inputs(1, Hq, Hkv, N, D, rho=rho, rope_base=rope_base, seed=seed,
                                      device=dev, qv_on_device=True)
    torch.cuda.synchronize()
    return q, k, v


def _layer_parity(q, k, v, tau, n_blocks, what, W=128):
    """delta_prefill (the bench's step) and dense_prefill on one layer, against the oracle
    on ``n_blocks`` query blocks spread over the sequence, all query heads."""
    from deltaattention_amd import ops
    N = q.shape[2]
    announce(f"{what}: delta_prefill N={N} tau={tau:.4f}")
    out, packed = ops.delta_prefill(q, k, v, tau, 512, window=W, return_packed=True)
    keep, _ = ops.select(k, tau, 512)
    torch.cuda.synchronize()
    kf, vf, ref = _check_select_pack(k, v, tau, keep, packed, what)
    blocks = _spread((N + 127) // 128, n_blocks)
    rows = _rows(blocks, N)
    qf = q.float().cpu().numpy()
    want = O.hybrid_attention(qf, kf, vf, ref["k_packed"], ref["v_packed"], ref["timestamps"],
                              ref["counts"], W, q_blocks=blocks)
    _close(out[:, :, rows].float().cpu().numpy(), want[:, :, rows], f"{what} hybrid blocks {blocks}")
    del out, want
    announce(f"{what}: dense_prefill N={N}")
    dense = ops.dense_prefill(q, k, v)
    want = O.dense_attention(qf, kf, vf, True, q_blocks=blocks)
    _close(dense[:, :, rows].float().cpu().numpy(), want[:, :, rows], f"{what} dense blocks {blocks}")


# --------------------------------------------------------------------------------------
# config 0: head_dim 64, Hq = Hkv = 8, N = 2048, RoPE base 1e4
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("variant", ["hybrid", "sanity", "pure_phase1"])
def test_config0_head_dim_64(gpu, variant):
    from deltaattention_amd import ops, synth
    N, D = 2048, 64
    q, k, v = _layer(N, 0, gpu, rope_base=10000.0, D=D, Hq=8, Hkv=8)
    tau, r_real = synth.calibrate_threshold(k, 4.0)
    announce(f"config0 D=64 N={N} {variant} tau={tau:.4f} r={r_real:.3f}")
    out, packed = ops.delta_prefill(q, k, v, tau, 512, window=128, variant=variant,
                                    return_packed=True)
    keep, _ = ops.select(k, tau, 512)
    kf, vf, ref = _check_select_pack(k, v, tau, keep, packed, "config0")
    want = O.hybrid_attention(q.float().cpu().numpy(), kf, vf, ref["k_packed"], ref["v_packed"],
                              ref["timestamps"], ref["counts"], 128, variant=variant)
    _close(out.float().cpu().numpy(), want, f"config0 D=64 {variant}")
    # the same inputs zero-padded to 128 dims run the D = 128 path: identical values
    pad = lambda t: torch.nn.functional.pad(t, (0, 128 - D))
    out128 = ops.hybrid_prefill(pad(q), pad(k), pad(v), pad(packed.k_packed), pad(packed.v_packed),
                                packed.timestamps, packed.counts, window=128, scale=D ** -0.5,
                                variant=variant, num_packed_dev=packed.num_packed)
    assert torch.equal(out128[..., :D], out)
    assert not out128[..., D:].any()


def test_config0_dense_head_dim_64(gpu):
    from deltaattention_amd import ops
    q, k, v = _layer(2048, 0, gpu, rope_base=10000.0, D=64, Hq=8, Hkv=8)
    announce("config0 dense D=64")
    out = ops.dense_prefill(q, k, v)
    want = O.dense_attention(q.float().cpu().numpy(), k.float().cpu().numpy(),
                             v.float().cpu().numpy(), True)
    _close(out.float().cpu().numpy(), want, "config0 dense D=64")


# fp32 tensors: the oracle's fp32 arithmetic without 16-bit rounding of p; the two
# differ only by fp32 summation order and the key-bias formulation of the weights
FP32_MAX_ABS = 1e-5
FP32_MEAN_ABS = 1e-6


def _close32(got, want, what):
    got = np.asarray(got, dtype=np.float32)
    err = np.abs(got - np.asarray(want, dtype=np.float32))
    mx, mean = float(err.max()), float(err.mean())
    print(f"{what}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    assert mx <= FP32_MAX_ABS and mean <= FP32_MEAN_ABS, f"{what}: max-abs {mx:.3e}, mean-abs {mean:.3e}"


@pytest.mark.parametrize("variant", ["hybrid", "sanity", "pure_phase1", "dense"])
def test_config0_fp32(gpu, variant):
    """Config 0 as BASELINE.json states it, fp32 end to end: fp32 Q, K, V (no 16-bit
    rounding of the inputs), the selection in fp32 (the keys' own arithmetic) bit-exact,
    packing bit-exact, and attention within 1e-5 of the fp32 oracle."""
    from deltaattention_amd import ops, synth
    N, D = 2048, 64
    q, k, v = synth.make_layer_inputs(1, 8, 8, N, D, rope_base=10000.0, seed=0, dtype=torch.float32,
                                      device=gpu, qv_on_device=True)
    qf, kf, vf = q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()
    if variant == "dense":
        announce("config0 fp32 dense")
        _close32(ops.dense_prefill(q, k, v).cpu().numpy(), O.dense_attention(qf, kf, vf, True), "config0 fp32 dense")
        return
    tau, r_real = synth.calibrate_threshold(k, 4.0)
    announce(f"config0 fp32 {variant} tau={tau:.4f} r={r_real:.3f}")
    out, packed = ops.delta_prefill(q, k, v, tau, 512, window=128, variant=variant, return_packed=True)
    keep, _ = ops.select(k, tau, 512)
    _, _, ref = _check_select_pack(k, v, tau, keep, packed, "config0 fp32")
    want = O.hybrid_attention(qf, kf, vf, ref["k_packed"], ref["v_packed"], ref["timestamps"], ref["counts"], 128,
                              variant=variant)
    _close32(out.cpu().numpy(), want, f"config0 fp32 {variant}")


def test_fp32_ragged_batch_and_dims(gpu):
    """fp32 through the varlen entry points (each sequence equal to its own B = 1 run),
    and at head dims 96 and 128 with GQA, against the fp32 oracle."""
    from deltaattention_amd import ops, synth
    for D, Hq, Hkv in ((96, 8, 2), (128, 8, 4)):
        q, k, v = synth.make_layer_inputs(1, Hq, Hkv, 1500, D, rope_base=10000.0, seed=D, dtype=torch.float32,
                                          device=gpu, qv_on_device=True)
        tau = 8.0 * (D / 128) ** 0.5
        announce(f"fp32 D={D} Hq={Hq} Hkv={Hkv}")
        out, packed = ops.delta_prefill(q, k, v, tau, 512, window=128, return_packed=True)
        kf, vf = k.cpu().numpy(), v.cpu().numpy()
        keep, _ = OC.select_delta(kf, tau, 512, arith="fp32")
        p = O.pack(kf, vf, keep)
        P = int(packed.num_packed.item())
        assert P == p["P"] and np.array_equal(packed.k_packed[:, :, :P].cpu().numpy(), p["k_packed"])
        want = O.hybrid_attention(q.cpu().numpy(), kf, vf, p["k_packed"], p["v_packed"], p["timestamps"],
                                  p["counts"], 128)
        _close32(out.cpu().numpy(), want, f"fp32 D={D} hybrid")
    # a ragged batch: [T, H, D] tensors, every sequence bitwise equal to its B = 1 run
    lens = [700, 1300, 64]
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    qs, ks, vs = [], [], []
    for i, n in enumerate(lens):
        q, k, v = synth.make_layer_inputs(1, 8, 2, n, 64, rope_base=10000.0, seed=50 + i, dtype=torch.float32,
                                          device=gpu, qv_on_device=True)
        qs.append(q); ks.append(k); vs.append(v)
    tok = lambda ts: torch.cat([t[0].transpose(0, 1) for t in ts]).contiguous()  # [T, H, D]
    announce(f"fp32 varlen lens {lens}")
    out = ops.delta_prefill_varlen(tok(qs), tok(ks), tok(vs), torch.tensor(cu, dtype=torch.int32, device=gpu),
                                   6.0, 512)
    for i, n in enumerate(lens):
        one = ops.delta_prefill(qs[i], ks[i], vs[i], 6.0, 512)
        assert torch.equal(out[cu[i]:cu[i + 1]].transpose(0, 1), one[0]), f"sequence {i}"


@pytest.mark.parametrize("D", [32, 80, 96])
def test_other_head_dims(gpu, D):
    """Head dims below 128 (multiples of 8) on the GQA-4 grouped kernel and the per-head
    kernel, against the oracle."""
    from deltaattention_amd import ops
    for Hq, Hkv in ((8, 2), (6, 3)):
        q, k, v = _layer(1500, D, gpu, rope_base=10000.0, D=D, Hq=Hq, Hkv=Hkv)
        announce(f"head_dim {D} Hq={Hq} Hkv={Hkv}")
        out, packed = ops.delta_prefill(q, k, v, 8.0 * (D / 128) ** 0.5, 512, window=128,
                                        return_packed=True)
        kf, vf = k.float().cpu().numpy(), v.float().cpu().numpy()
        keep, _ = OC.select_delta(kf, 8.0 * (D / 128) ** 0.5, 512, arith=oracle_arith(k))
        p = O.pack(kf, vf, keep)
        want = O.hybrid_attention(q.float().cpu().numpy(), kf, vf, p["k_packed"], p["v_packed"],
                                  p["timestamps"], p["counts"], 128)
        _close(out.float().cpu().numpy(), want, f"D={D} Hq={Hq} Hkv={Hkv} hybrid")
        dense = ops.dense_prefill(q, k, v)
        want = O.dense_attention(q.float().cpu().numpy(), kf, vf, True)
        _close(dense.float().cpu().numpy(), want, f"D={D} Hq={Hq} Hkv={Hkv} dense")


# --------------------------------------------------------------------------------------
# config 1: the benchmarked layer (N = 32768, r = 4, seed 0)
# --------------------------------------------------------------------------------------
def test_config1_layer(gpu):
    from deltaattention_amd import synth
    q, k, v = _layer(32768, 0, gpu)
    tau, r_real = synth.calibrate_threshold(k, 4.0)
    _layer_parity(q, k, v, tau, 8, f"config1 r={r_real:.3f}")


# --------------------------------------------------------------------------------------
# config 2: N = 131072, r in {2, 4, 8}
# --------------------------------------------------------------------------------------
@pytest.fixture(scope="module")
def config2_inputs(gpu):
    announce("config2 inputs N=131072")
    return _layer(131072, 0, gpu)


@pytest.mark.parametrize("ratio", [2.0, 4.0, 8.0])
def test_config2_layer(gpu, config2_inputs, ratio):
    from deltaattention_amd import synth
    q, k, v = config2_inputs
    tau, r_real = synth.calibrate_threshold(k, ratio)
    _layer_parity(q, k, v, tau, 6, f"config2 r={ratio:g} (realised {r_real:.3f})")


# --------------------------------------------------------------------------------------
# the reference's longest point (eval_speedup.py:28, the paper's 262K): the config-2 layer
# at N = 262144, r = 4 -- selection and packing bit-exact at full size, attention on query
# blocks from the first to the last
# --------------------------------------------------------------------------------------
def test_layer_262k(gpu):
    from deltaattention_amd import synth
    announce("262K inputs N=262144")
    q, k, v = _layer(262144, 0, gpu)
    tau, r_real = synth.calibrate_threshold(k, 4.0)
    _layer_parity(q, k, v, tau, 4, f"N=262144 r=4 (realised {r_real:.3f})")


# --------------------------------------------------------------------------------------
# config 3: Llama-3-8B-shaped prefill of 65536 tokens through the transformers swap
# --------------------------------------------------------------------------------------
def test_config3_model_layers(gpu, monkeypatch):
    """A 4-layer Llama-3-8B-shaped model prefills 65536 tokens through the swap (periodic
    anchors, r = 4); every layer's attention output is compared with the oracle on its own
    inputs (the layer's post-RoPE q, k, v as the swap passed them)."""
    pytest.importorskip("transformers")
    from deltaattention_amd import attention, globVR, llama_swap
    N, L = 65536, 4
    captured = {}
    real = attention.delta_prefill_attention

    def spy(query_states, key_states, value_states, layer_idx=0, **kw):
        out = real(query_states, key_states, value_states, layer_idx=layer_idx, **kw)
        if layer_idx not in captured:
            captured[layer_idx] = (query_states.detach().clone(), key_states.detach().clone(),
                                   value_states.detach().clone(), out.detach().clone())
        return out

    monkeypatch.setattr(attention, "delta_prefill_attention", spy)
    monkeypatch.setattr(globVR, "packing_mode", "periodic", raising=False)
    monkeypatch.setattr(globVR, "target_keep_rate", 0.25, raising=False)
    monkeypatch.setattr(globVR, "dense_window_size", 128, raising=False)
    cfg = llama_swap.llama3_8b_config(llama_swap.DELTA, num_layers=L)
    model = llama_swap.random_llama(cfg, gpu, seed=0)
    ids = torch.randint(0, cfg.vocab_size, (1, N), generator=torch.Generator().manual_seed(0)).to(gpu)
    announce(f"config3 {L}-layer Llama-3-8B shape, N={N}, periodic r=4")
    with torch.no_grad():
        hidden = model.model(input_ids=ids).last_hidden_state
    torch.cuda.synchronize()
    assert torch.isfinite(hidden).all()
    del model, hidden
    torch.cuda.empty_cache()
    assert sorted(captured) == list(range(L))
    keep = O.select_periodic(1, 8, N, 0.25)
    blocks = _spread(N // 128, 6)
    rows = _rows(blocks, N)
    for layer in range(L):
        q, k, v, out = captured.pop(layer)
        assert q.shape == (1, 32, N, 128) and k.shape == (1, 8, N, 128)
        kf, vf = k.float().cpu().numpy(), v.float().cpu().numpy()
        ref = O.pack(kf, vf, keep)
        want = O.hybrid_attention(q.float().cpu().numpy(), kf, vf, ref["k_packed"], ref["v_packed"],
                                  ref["timestamps"], ref["counts"], 128, q_blocks=blocks)
        _close(out[:, :, rows].float().cpu().numpy(), want[:, :, rows], f"config3 layer {layer} blocks {blocks}")
        del q, k, v, out, kf, vf, ref, want


# --------------------------------------------------------------------------------------
# config 4: ragged batch of 8 sequences, N_b ~ U[4096, 32768], rho ~ U[0.6, 0.95]
# --------------------------------------------------------------------------------------
def _config4_batch(dev, seed=0):
    """The bench's config-4 batch: packed [tokens, heads, 128] tensors and cu_seqlens."""
    from deltaattention_amd import synth
    rng = np.random.default_rng(seed)
    lens = rng.integers(4096, 32768, size=8, endpoint=True).tolist()
    qs, ks, vs = [], [], []
    for i, n in enumerate(lens):
        rho = rng.uniform(0.6, 0.95, size=8)
        q, k, v = synth.make_layer_inputs(1, 32, 8, n, 128, rho=rho, rope_base=500000.0,
                                          seed=seed * 100 + i, device=dev, qv_on_device=True)
        qs.append(q[0].permute(1, 0, 2))
        ks.append(k[0].permute(1, 0, 2))
        vs.append(v[0].permute(1, 0, 2))
    q, k, v = torch.cat(qs).contiguous(), torch.cat(ks).contiguous(), torch.cat(vs).contiguous()
    cu = [0] + np.cumsum(lens).tolist()
    return q, k, v, cu, lens


def test_config4_varlen(gpu):
    from deltaattention_amd import ops, synth
    q, k, v, cu, lens = _config4_batch(gpu)
    tau, r_real = synth.calibrate_threshold(k.permute(1, 0, 2).unsqueeze(0), 4.0)
    announce(f"config4 varlen lens={lens} tau={tau:.4f}")
    out = ops.delta_prefill_varlen(q, k, v, cu, tau, 512, window=128)
    dense = ops.dense_prefill_varlen(q, k, v, cu)
    torch.cuda.synchronize()
    for i, (s, e) in enumerate(zip(cu[:-1], cu[1:])):
        n = e - s
        sl = lambda x: x[s:e].permute(1, 0, 2).unsqueeze(0)
        kf, vf = sl(k).float().cpu().numpy(), sl(v).float().cpu().numpy()
        keep, _ = OC.select_delta(kf, tau, 512, arith=oracle_arith(k))
        ref = O.pack(kf, vf, keep)
        blocks = _spread((n + 127) // 128, 3)
        rows = _rows(blocks, n)
        qf = sl(q).float().cpu().numpy()
        want = O.hybrid_attention(qf, kf, vf, ref["k_packed"], ref["v_packed"], ref["timestamps"],
                                  ref["counts"], 128, q_blocks=blocks)
        got = sl(out)[:, :, rows].float().cpu().numpy()
        _close(got, want[:, :, rows], f"config4 seq {i} (N={n}, P={ref['P']}) hybrid")
        want = O.dense_attention(qf, kf, vf, True, q_blocks=blocks)
        _close(sl(dense)[:, :, rows].float().cpu().numpy(), want[:, :, rows],
               f"config4 seq {i} (N={n}) dense")
