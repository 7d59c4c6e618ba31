"""GPU parity of the HIP kernels against the CPU oracle and the reference's golden vectors.

Bars: selection and indexing are bit-exact; attention outputs (bf16) are within
max-abs 2e-2 and mean-abs 1e-3 of the fp32 oracle on the same bf16 inputs.
"""
import os

import numpy as np
import pytest
import torch

from conftest import announce, oracle_arith
from oracle import delta_oracle as O
from oracle import select_oracle_c as OC

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 1e-3
HERE = os.path.dirname(os.path.abspath(__file__))


def _bf16_inputs(B, Hq, Hkv, N, D, seed, rho=0.9):
    from deltaattention_amd import synth
    q, k, v = synth.make_layer_inputs(B, Hq, Hkv, N, D, rho=rho, seed=seed, rope_base=10000.0)
    return q, k, v


def _close(got, want, what):
    got = np.asarray(got, dtype=np.float32)
    want = np.asarray(want, dtype=np.float32)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - want)
    mx, mean = float(err.max()), float(err.mean())
    print(f"{what}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, f"{what}: max-abs {mx:.3e}, mean-abs {mean:.3e}"


# --------------------------------------------------------------------------------------
# selection + packing: bit-exact
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("metric,tau,chunk,divide_to", [
    ("euclidean", 9.0, 512, 0),
    ("euclidian", 7.5, 100, 0),      # any non-"cosine" string is Euclidean
    ("cosine", 0.85, 512, 0),
    ("euclidean", 8.0, 0, 3),        # divide_to chunking
    ("euclidean", 0.0, 64, 0),       # tau 0: every distinct row is kept
])
def test_select_bitexact(gpu, metric, tau, chunk, divide_to):
    from deltaattention_amd import ops
    q, k, v = _bf16_inputs(2, 2, 2, 3000, 128, seed=11)
    announce(f"select {metric} tau={tau} chunk={chunk} divide_to={divide_to} N=3000")
    keep, cc = ops.select(k.to(gpu), tau, chunk, divide_to, metric)
    torch.cuda.synchronize()
    ok, occ = OC.select_delta(k.float().numpy(), tau, chunk, divide_to, metric, arith=oracle_arith(k))
    keep_h = keep.cpu().numpy()
    cc_h = cc.cpu().numpy()
    assert (cc_h == occ).all(), "chunk counts differ"
    assert (keep_h == ok).all(), f"keep differs at {np.argwhere(keep_h != ok)[:5]}"


def test_select_bitexact_config1_shape(gpu):
    """Config-1 key shape (8 KV heads x 32768 x 128, bf16), chunk 512."""
    from deltaattention_amd import ops, synth
    k = synth.make_layer_inputs(1, 8, 8, 32768, 128, seed=1)[1]
    for tau in (8.0, 11.0):
        announce(f"select config1 N=32768 tau={tau}")
        keep, cc = ops.select(k.to(gpu), tau, 512)
        ok, occ = OC.select_delta(k.float().numpy(), tau, 512, arith=oracle_arith(k))
        assert (cc.cpu().numpy() == occ).all()
        assert (keep.cpu().numpy() == ok).all()


@pytest.mark.parametrize("H,N,chunk,tau,metric,arith", [
    (1, 3000, 1, 9.0, "euclidean", "fp32"),       # one-row chunks
    (2, 3000, 33, 9.0, "euclidean", "fp32"),      # a one-row last batch
    (2, 3000, 512, 1e6, "euclidean", "fp32"),     # one anchor per chunk
    (2, 3000, 512, 0.999, "cosine", "fp32"),      # nearly every row kept
    (2, 5000, 8193, 9.0, "euclidean", "fp32"),
    (1, 20000, 10000, 9.0, "euclidean", "fp32"),
    (8, 32768, 256, 10.3, "euclidean", "fp32"),   # 1024 chunks
    (8, 32768, 128, 0.9, "cosine", "fp32"),       # 2048 chunks
    (8, 32768, 256, 10.3, "euclidean", "native"),
    # from 2048 chunks on, one wave walks two chunks (one per 32-lane half)
    (8, 131072, 512, 10.33, "euclidean", "fp32"),  # the config-2 grid
    (8, 131072, 512, 10.33, "euclidean", "native"),
    (8, 32768, 128, 1e6, "euclidean", "fp32"),
    (64, 16000, 512, 9.0, "euclidean", "fp32"),     # a 128-row last chunk
    (9, 32768, 129, 9.0, "euclidean", "fp32"),      # 2295 chunks: the last wave's second half is empty
])
def test_select_chunk_shapes(gpu, H, N, chunk, tau, metric, arith):
    """Selection against the sequential oracle over chunk lengths from 1 to 10000 rows,
    grids of 2 to 2295 chunks (one chunk per wave below 2048, two from there on) and
    thresholds that keep one row per chunk or nearly every row."""
    from deltaattention_amd import ops, synth
    k = synth.make_layer_inputs(1, H, H, N, 128, seed=21, rope_base=500000.0)[1]
    announce(f"select H={H} N={N} chunk={chunk} tau={tau} {metric} {arith}")
    keep, cc = ops.select(k.to(gpu), tau, chunk, 0, metric, arith=arith)
    ok, occ = OC.select_delta(k.float().numpy(), tau, chunk, 0, metric,
                              arith="bf16" if arith == "native" else "fp32")
    assert np.array_equal(cc.cpu().numpy(), occ), "chunk counts differ"
    keep_h = keep.cpu().numpy()
    assert np.array_equal(keep_h, ok), f"keep differs at {np.argwhere(keep_h != ok)[:5]}"


@pytest.mark.parametrize("D,dtype", [(64, torch.bfloat16), (128, torch.float16), (66, torch.bfloat16)],
                         ids=["D64", "fp16", "D66-one-per-wave"])
def test_select_pair_grid_dims(gpu, D, dtype):
    """2048 chunks with head_dim 64 (lanes past D hold nothing) and fp16 keys walk two
    chunks per wave; head_dim 66 (not a multiple of 4) keeps one chunk per wave."""
    from deltaattention_amd import ops, synth
    k = synth.make_layer_inputs(1, 64, 64, 16384, D, seed=23, rope_base=500000.0)[1].to(dtype)
    for tau, metric in ((9.0, "euclidean"), (0.9, "cosine")):
        announce(f"select pair grid D={D} {dtype} {metric}")
        keep, cc = ops.select(k.to(gpu), tau, 512, 0, metric)
        ok, occ = OC.select_delta(k.float().numpy(), tau, 512, 0, metric, arith=oracle_arith(k))
        assert np.array_equal(cc.cpu().numpy(), occ), "chunk counts differ"
        assert np.array_equal(keep.cpu().numpy(), ok)


@pytest.mark.parametrize("dtype,oracle_arith", [(torch.bfloat16, "bf16"), (torch.float16, "fp16")])
def test_select_native_arith_bitexact(gpu, dtype, oracle_arith):
    """arith="native": the Euclidean distance in the keys' 16-bit arithmetic, bit-exact
    against the oracle's 16-bit mode, at N=3000 (chunk 512 and divide_to) and at the
    config-1 key shape; the two definitions differ on some rows."""
    from deltaattention_amd import ops, synth
    k = _bf16_inputs(2, 2, 2, 3000, 128, seed=12)[1].to(dtype)
    kc = synth.make_layer_inputs(1, 8, 8, 32768, 128, seed=0)[1].to(dtype)
    for kk, tau, chunk, div in ((k, 9.0, 512, 0), (k, 8.0, 0, 3), (kc, 10.3327, 512, 0)):
        announce(f"select native arith {dtype} N={kk.shape[2]} tau={tau}")
        keep, cc = ops.select(kk.to(gpu), tau, chunk, div, arith="native")
        ok, occ = OC.select_delta(kk.float().numpy(), tau, chunk, div, arith=oracle_arith)
        assert np.array_equal(cc.cpu().numpy(), occ)
        assert np.array_equal(keep.cpu().numpy(), ok)
    k32, _ = OC.select_delta(kc.float().numpy(), 10.3327, 512, arith="fp32")
    assert not np.array_equal(k32, ok)


@pytest.mark.parametrize("scale,tau", [(2e-3, 0.015), (40.0, 250.0)], ids=["subnormal-squares", "near-fp16-max"])
@pytest.mark.parametrize("H", [4, 64], ids=["one-chunk-per-wave", "two-chunks-per-wave"])
def test_select_fp16_native_extremes(gpu, scale, tau, H):
    """fp16 keys in the keys' own arithmetic at the edges of the format, bit-exact against
    the oracle's fp16 rounding (pinned against torch, subnormals included): keys scaled
    so that the squared differences are fp16 subnormals (spacing 6e-8) with the threshold
    among them, and keys whose distances reach the fp16 maximum (65504, spacing 32; sums
    past it are inf, kept) with tau^2 = 62500 just below it.  Both walk layouts."""
    from deltaattention_amd import ops, synth
    N = 16384 if H == 64 else 4096   # 64 heads x 32 chunks: the pair walk's 2048 chunks
    k = (synth.make_layer_inputs(1, H, H, N, 128, seed=29, rope_base=10000.0)[1].float() * scale).to(torch.float16)
    assert torch.isfinite(k).all()
    announce(f"select fp16 extremes scale={scale} tau={tau} H={H} N={N}")
    keep, cc = ops.select(k.to(gpu), tau, 512, 0, arith="native")
    ok, occ = OC.select_delta(k.float().numpy(), tau, 512, 0, arith="fp16")
    assert np.array_equal(cc.cpu().numpy(), occ), "chunk counts differ"
    assert np.array_equal(keep.cpu().numpy(), ok)
    kept = int(ok.sum())
    print(f"fp16 extremes scale={scale}: kept {kept} of {ok.size}", flush=True)
    assert 0.02 * ok.size < kept < 0.98 * ok.size   # the threshold splits the rows


@pytest.mark.parametrize("N,tau", [(3000, 10.0), (777, 7.0), (4096, 0.0)])
def test_pack_exact(gpu, N, tau):
    from deltaattention_amd import ops
    q, k, v = _bf16_inputs(1, 4, 3, N, 128, seed=5)
    announce(f"pack N={N} tau={tau}")
    kg, vg = k.to(gpu), v.to(gpu)
    keep, _ = ops.select(kg, tau, 512)
    packed = ops.pack(keep, kg, vg)
    torch.cuda.synchronize()
    ref = O.pack(k.float().numpy(), v.float().numpy(), keep.cpu().numpy())
    P = int(packed.num_packed.item())
    assert P == ref["P"]
    assert (packed.anchor_counts.cpu().numpy() == ref["anchor_counts"]).all()
    assert (packed.timestamps[:, :, :P].cpu().numpy() == ref["timestamps"]).all()
    assert (packed.counts[:, :, :P].cpu().numpy() == ref["counts"]).all()
    assert torch.equal(packed.k_packed[:, :, :P].float().cpu(), torch.from_numpy(ref["k_packed"]))
    assert torch.equal(packed.v_packed[:, :, :P].float().cpu(), torch.from_numpy(ref["v_packed"]))


@pytest.mark.parametrize("D,pad", [(128, 2), (66, 0)], ids=["offset-rows", "D66"])
def test_pack_exact_4byte_rows(gpu, D, pad):
    """The 4-byte row copy of the scatter: key/value rows that are 4-byte but not 16-byte
    aligned (views at a 2-element offset in rows of D + 4), and a head dimension that is
    not a multiple of 8."""
    from deltaattention_amd import ops
    N = 2000
    q, k, v = _bf16_inputs(1, 4, 3, N, D, seed=6)
    announce(f"pack 4-byte rows D={D} pad={pad}")
    if pad:
        kb = torch.zeros((1, 3, N, D + 4), dtype=k.dtype)
        vb = torch.zeros((1, 3, N, D + 4), dtype=v.dtype)
        kb[..., pad:pad + D], vb[..., pad:pad + D] = k, v
        kg, vg = kb.to(gpu)[..., pad:pad + D], vb.to(gpu)[..., pad:pad + D]
    else:
        kg, vg = k.to(gpu), v.to(gpu)
    keep, _ = ops.select(kg.contiguous(), 8.0 * (D / 128) ** 0.5, 512)
    packed = ops.pack(keep, kg, vg)
    torch.cuda.synchronize()
    ref = O.pack(k.float().numpy(), v.float().numpy(), keep.cpu().numpy())
    P = int(packed.num_packed.item())
    assert P == ref["P"]
    assert (packed.timestamps[:, :, :P].cpu().numpy() == ref["timestamps"]).all()
    assert (packed.counts[:, :, :P].cpu().numpy() == ref["counts"]).all()
    assert torch.equal(packed.k_packed[:, :, :P].float().cpu(), torch.from_numpy(ref["k_packed"]))
    assert torch.equal(packed.v_packed[:, :, :P].float().cpu(), torch.from_numpy(ref["v_packed"]))


def test_pack_periodic_and_exact_capacity(gpu):
    """Periodic keep mask (modeling_llama.py:626-632) packed into buffers of exactly P rows."""
    from deltaattention_amd import ops
    q, k, v = _bf16_inputs(1, 2, 2, 1000, 128, seed=6)
    keep = torch.from_numpy(O.select_periodic(1, 2, 1000, 0.3))
    ref = O.pack(k.float().numpy(), v.float().numpy(), keep.numpy())
    announce("pack periodic capacity=P")
    packed = ops.pack(keep.to(gpu), k.to(gpu), v.to(gpu), capacity=ref["P"])
    assert (packed.counts.cpu().numpy() == ref["counts"]).all()
    assert (packed.timestamps.cpu().numpy() == ref["timestamps"]).all()
    assert torch.equal(packed.k_packed.float().cpu(), torch.from_numpy(ref["k_packed"]))


# --------------------------------------------------------------------------------------
# dense flash prefill
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("B,Hq,Hkv,N,causal", [
    (1, 8, 2, 700, True),
    (2, 4, 4, 513, True),
    (1, 6, 3, 384, True),
    (1, 4, 1, 300, False),
])
def test_dense_vs_oracle(gpu, B, Hq, Hkv, N, causal):
    from deltaattention_amd import ops
    q, k, v = _bf16_inputs(B, Hq, Hkv, N, 128, seed=3)
    announce(f"dense B={B} Hq={Hq} Hkv={Hkv} N={N} causal={causal}")
    out = ops.dense_prefill(q.to(gpu), k.to(gpu), v.to(gpu), causal=causal)
    ref = O.dense_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal)
    _close(out.float().cpu().numpy(), ref, f"dense N={N}")


def _ramp_inputs(B, Hq, Hkv, N, D, seed, top):
    """bf16 inputs whose scaled scores follow a ramp over the keys: from 0 to `top` for a
    query along the ramp direction (top < 0: falling), plus unit noise.  A rising ramp
    moves each row's maximum in most tiles, so the kernels' rescale path runs often; a
    falling one leaves late keys with p far below 2^-126."""
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(D, generator=g)
    u = u / u.norm()
    scale = D ** -0.5
    qn = 8.0
    q = torch.randn(B, Hq, N, D, generator=g) * 0.5 + qn * u
    ramp = torch.linspace(0.0, 1.0, N).view(1, 1, N, 1) * (top / (scale * qn))
    k = torch.randn(B, Hkv, N, D, generator=g) + ramp * u
    v = torch.randn(B, Hkv, N, D, generator=g)
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


@pytest.mark.parametrize("top", [200.0, 60.0, -200.0], ids=["rise200", "rise60", "fall200"])
def test_dense_rescale_stress_vs_oracle(gpu, top):
    """Scores that climb across the keys make the running maximum move in most tiles
    (the grouped kernel's exact path and O rescale), and falling ones drive p to zero."""
    from deltaattention_amd import ops
    q, k, v = _ramp_inputs(1, 8, 2, 2048, 128, seed=11, top=top)
    announce(f"dense rescale stress top={top}")
    out = ops.dense_prefill(q.to(gpu), k.to(gpu), v.to(gpu), causal=True)
    ref = O.dense_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), True)
    _close(out.float().cpu().numpy(), ref, f"dense ramp {top}")


@pytest.mark.parametrize("top,tau,variant", [
    (200.0, 1e6, "hybrid"), (60.0, 16.0, "hybrid"), (200.0, 16.0, "sanity"),
    (-200.0, 1e6, "hybrid"), (60.0, 16.0, "pure_phase1")])
def test_delta_rescale_stress_vs_oracle(gpu, top, tau, variant):
    from deltaattention_amd import ops
    q, k, v = _ramp_inputs(1, 8, 2, 2048, 128, seed=12, top=top)
    announce(f"delta rescale stress top={top} tau={tau} {variant}")
    out = ops.delta_prefill(q.to(gpu), k.to(gpu), v.to(gpu), tau, 512, window=128, variant=variant)
    kf, vf = k.float().numpy(), v.float().numpy()
    keep, _ = OC.select_delta(kf, tau, 512, arith=oracle_arith(k))
    p = O.pack(kf, vf, keep)
    ref = O.hybrid_attention(q.float().numpy(), kf, vf, p["k_packed"], p["v_packed"],
                             p["timestamps"], p["counts"], 128, variant=variant)
    _close(out.float().cpu().numpy(), ref, f"delta ramp {top} {variant}")


# --------------------------------------------------------------------------------------
# hybrid prefill against the reference's own outputs (golden vectors, D=32 zero-padded)
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("case", ["A", "B", "C", "D"])
@pytest.mark.parametrize("variant", ["hybrid", "sanity", "pure_phase1"])
@pytest.mark.parametrize("native", [True, False], ids=["d32", "d32-padded"])
def test_hybrid_golden(gpu, case, variant, native):
    """The golden inputs are bf16-exact with D=32.  "d32" runs head_dim 32 natively (the
    kernels zero-fill dims 32..127, like the reference's BLOCK_D masking); "d32-padded"
    zero-pads D to 128 on the host, which leaves every score unchanged (scale 32**-0.5),
    and compares the first 32 output dims.  Both against the reference's interpreter
    outputs."""
    from deltaattention_amd import ops
    z = np.load(os.path.join(HERE, "golden", "hybrid_golden.npz"))
    g = lambda n: z[f"{case}/{n}"]
    q, k, v, keep = g("q"), g("k"), g("v"), g("keep")
    W, no_count = int(g("window")), bool(g("no_count"))
    D = q.shape[-1]
    width = D if native else 128
    pad = lambda a: torch.from_numpy(np.pad(a, [(0, 0)] * 3 + [(0, width - D)])).to(torch.bfloat16).to(gpu)
    qg, kg, vg = pad(q), pad(k), pad(v)
    announce(f"golden case {case} {variant} {'native D' if native else 'padded to 128'}")
    packed = ops.pack(torch.from_numpy(keep).to(gpu), kg, vg)
    out = ops.hybrid_prefill(qg, kg, vg, packed.k_packed, packed.v_packed, packed.timestamps,
                             packed.counts, window=W, scale=D ** -0.5, variant=variant,
                             no_count=no_count, num_packed_dev=packed.num_packed)
    got = out.float().cpu().numpy()
    assert np.all(got[..., D:] == 0)
    _close(got[..., :D], g(f"out_{variant}"), f"golden {case}/{variant}")


# --------------------------------------------------------------------------------------
# end-to-end delta prefill against the oracle
# --------------------------------------------------------------------------------------
@pytest.mark.parametrize("B,Hq,Hkv,N,tau,W,variant,no_count", [
    (1, 8, 2, 2048, 10.0, 128, "hybrid", False),
    (1, 4, 4, 1500, 9.0, 0, "hybrid", False),
    (1, 4, 2, 1100, 8.0, 300, "hybrid", True),
    (2, 8, 2, 1024, 10.0, 128, "sanity", False),
    (1, 4, 2, 900, 9.0, 128, "pure_phase1", False),
    (1, 8, 2, 3000, 12.0, 128, "hybrid", False),
    (1, 2, 1, 2048, 1e6, 128, "hybrid", False),   # only chunk starts are anchors
    # GQA group of 4 (the grouped kernel), counts of 512: the largest key biases
    (1, 8, 2, 2048, 1e6, 128, "hybrid", False),
    (1, 8, 2, 2048, 1e6, 128, "pure_phase1", False),
    (1, 8, 2, 2048, 1e6, 128, "hybrid", True),
    (1, 8, 2, 1, 10.0, 128, "hybrid", False),      # one token
    (2, 8, 2, 77, 9.0, 128, "hybrid", False),      # shorter than the window and one block
    (1, 4, 2, 77, 9.0, 128, "pure_phase1", False),
])
def test_delta_prefill_vs_oracle(gpu, B, Hq, Hkv, N, tau, W, variant, no_count):
    from deltaattention_amd import ops
    q, k, v = _bf16_inputs(B, Hq, Hkv, N, 128, seed=N + Hq)
    announce(f"delta_prefill B={B} Hq={Hq} Hkv={Hkv} N={N} tau={tau} W={W} {variant} nc={no_count}")
    out = ops.delta_prefill(q.to(gpu), k.to(gpu), v.to(gpu), tau, 512, window=W, variant=variant,
                            no_count=no_count)
    kf, vf = k.float().numpy(), v.float().numpy()
    keep, _ = OC.select_delta(kf, tau, 512, arith=oracle_arith(k))
    p = O.pack(kf, vf, keep)
    ref = O.hybrid_attention(q.float().numpy(), kf, vf, p["k_packed"], p["v_packed"],
                             p["timestamps"], p["counts"], W, variant=variant, no_count=no_count)
    _close(out.float().cpu().numpy(), ref, f"delta {variant} N={N}")


def test_hybrid_float_counts_matches_int(gpu):
    from deltaattention_amd import ops
    q, k, v = _bf16_inputs(1, 4, 1, 1024, 128, seed=9)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    announce("hybrid fp32 counts vs int32 counts")
    keep, _ = ops.select(kg, 10.0, 512)
    pk = ops.pack(keep, kg, vg).trimmed()
    a = ops.hybrid_prefill(qg, kg, vg, pk.k_packed, pk.v_packed, pk.timestamps, pk.counts)
    b = ops.hybrid_prefill(qg, kg, vg, pk.k_packed, pk.v_packed, pk.timestamps, pk.counts.float())
    assert torch.equal(a, b)


@pytest.mark.parametrize("N,Hq", [(40960, 4), (70000, 4), (70000, 2)])
def test_keep_all_hybrid_equals_dense_full_size(gpu, N, Hq):
    """tau = 0 keeps every distinct key with count 1, so the hybrid prefill covers every
    key once and must agree with dense causal attention.  At these sizes the packed
    blocks number 320 and 547 (more than one 256-block pass of the Phase-1 count); a
    GQA group of 2 runs the per-head kernel, a group of 4 the grouped one."""
    from deltaattention_amd import ops
    q, k, v = _bf16_inputs(1, Hq, 1, N, 128, seed=5)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    announce(f"keep-all hybrid vs dense N={N} Hq={Hq}")
    keep, counts = ops.select(kg, 0.0, 512)
    assert int(keep.sum()) == N
    pk = ops.pack(keep, kg, vg)
    hyb = ops.hybrid_prefill(qg, kg, vg, pk.k_packed, pk.v_packed, pk.timestamps, pk.counts,
                             window=128, num_packed_dev=pk.num_packed)
    dense = ops.dense_prefill(qg, kg, vg)
    _close(hyb.float().cpu().numpy(), dense.float().cpu().numpy(), f"keep-all N={N}")


@pytest.mark.parametrize("Hq", [4, 2])
def test_phase1_extent_full_size(gpu, Hq):
    """Q = 0 makes every score 0, so each output row is the count-weighted mean of the
    V rows it sees: weight 2 for the packed keys of Phase 1, 1 for the exact keys of
    Phase 2.  With every key kept (timestamps 0..N-1) the Phase-1 extent of a 128-row
    query block has the closed form L = 128 * #{b : 128 b + 127 < start_m - W}
    (deltaFlashAttention.py:58-80), so the expected output is exact: V[:, 0] marks the
    keys at or beyond 32768, V[:, 1] is 1.  N = 70000 gives 547 packed blocks, more than
    one 256-block pass of the count; a wrong extent moves thousands of keys between
    weights 2 and 1."""
    from deltaattention_amd import ops
    N, W, D = 70000, 128, 128
    announce(f"phase-1 extent, closed form, N={N} Hq={Hq}")
    q = torch.zeros((1, Hq, N, D), dtype=torch.bfloat16, device=gpu)
    k = torch.randn((1, 1, N, D), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(gpu)
    v = torch.zeros((1, 1, N, D), dtype=torch.bfloat16)
    v[0, 0, 32768:, 0] = 1.0
    v[0, 0, :, 1] = 1.0
    v = v.to(gpu)
    keep = torch.ones((1, 1, N), dtype=torch.int32, device=gpu)
    pk = ops.pack(keep, k, v)
    out = ops.hybrid_prefill(q, k, v, pk.k_packed, pk.v_packed, pk.timestamps, pk.counts * 2,
                             window=W, num_packed_dev=pk.num_packed)
    got = out[0, :, :, :2].float().cpu().numpy()
    i = np.arange(N, dtype=np.int64)
    start_m = (i // 128) * 128
    n_safe = np.maximum(0, -(-(start_m - W - 127) // 128))   # ceil, clipped at 0
    L = 128 * n_safe
    late = lambda a, b: np.maximum(0, b - np.maximum(a, 32768))   # keys in [a, b) at >= 32768
    num = 2.0 * late(0, L) + late(L, i + 1)
    den = 2.0 * L + (i + 1 - L)
    want0 = num / den
    assert np.all(got[..., 1] == 1.0)
    err = np.abs(got[..., 0] - want0[None, :])
    print(f"phase-1 extent: max-abs {err.max():.3e}", flush=True)
    assert err.max() <= 4e-3   # bf16 rounding of values in [0, 1]


# --------------------------------------------------------------------------------------
# fp16 inputs: the same kernels on the other 16-bit type (P rounded to fp16 before P.V,
# as the reference rounds p to V's type, deltaFlashAttention.py:98, 137)
# --------------------------------------------------------------------------------------
def _f16_inputs(B, Hq, Hkv, N, D, seed):
    q, k, v = _bf16_inputs(B, Hq, Hkv, N, D, seed)
    return q.half(), k.half(), v.half()


@pytest.mark.parametrize("metric,tau", [("euclidean", 9.0), ("cosine", 0.85)])
def test_select_bitexact_fp16(gpu, metric, tau):
    from deltaattention_amd import ops
    _, k, _ = _f16_inputs(2, 4, 2, 1500, 128, seed=21)
    announce(f"select fp16 {metric} tau={tau}")
    keep, counts = ops.select(k.to(gpu), tau, 512, 0, metric)
    ref_keep, ref_counts = OC.select_delta(k.float().numpy(), tau, 512, 0, metric, arith=oracle_arith(k))
    assert np.array_equal(keep.cpu().numpy(), ref_keep)
    assert np.array_equal(counts.cpu().numpy(), ref_counts)


@pytest.mark.parametrize("B,Hq,Hkv,N,tau,W,variant", [
    (1, 8, 2, 2048, 10.0, 128, "hybrid"),
    (1, 4, 2, 1100, 8.0, 300, "hybrid"),
    (2, 8, 2, 1024, 10.0, 128, "sanity"),
    (1, 8, 2, 2048, 1e6, 128, "pure_phase1"),
])
def test_delta_prefill_fp16_vs_oracle(gpu, B, Hq, Hkv, N, tau, W, variant):
    from deltaattention_amd import ops
    q, k, v = _f16_inputs(B, Hq, Hkv, N, 128, seed=N + 7)
    announce(f"delta_prefill fp16 B={B} Hq={Hq} Hkv={Hkv} N={N} {variant}")
    out = ops.delta_prefill(q.to(gpu), k.to(gpu), v.to(gpu), tau, 512, window=W, variant=variant)
    assert out.dtype == torch.float16
    kf, vf = k.float().numpy(), v.float().numpy()
    keep, _ = OC.select_delta(kf, tau, 512, arith=oracle_arith(k))
    p = O.pack(kf, vf, keep)
    ref = O.hybrid_attention(q.float().numpy(), kf, vf, p["k_packed"], p["v_packed"],
                             p["timestamps"], p["counts"], W, variant=variant)
    _close(out.float().cpu().numpy(), ref, f"delta fp16 {variant} N={N}")


@pytest.mark.parametrize("B,Hq,Hkv,N", [(1, 8, 2, 700), (1, 6, 3, 384)])
def test_dense_fp16_vs_oracle(gpu, B, Hq, Hkv, N):
    from deltaattention_amd import ops
    q, k, v = _f16_inputs(B, Hq, Hkv, N, 128, seed=4)
    announce(f"dense fp16 B={B} Hq={Hq} Hkv={Hkv} N={N}")
    out = ops.dense_prefill(q.to(gpu), k.to(gpu), v.to(gpu))
    assert out.dtype == torch.float16
    ref = O.dense_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), True)
    _close(out.float().cpu().numpy(), ref, f"dense fp16 N={N}")


def test_keep_all_fp16_hybrid_equals_dense(gpu):
    from deltaattention_amd import ops
    q, k, v = _f16_inputs(1, 4, 1, 40960, 128, seed=5)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    announce("keep-all fp16 hybrid vs dense N=40960")
    keep, _ = ops.select(kg, 0.0, 512)
    pk = ops.pack(keep, kg, vg)
    hyb = ops.hybrid_prefill(qg, kg, vg, pk.k_packed, pk.v_packed, pk.timestamps, pk.counts,
                             window=128, num_packed_dev=pk.num_packed)
    dense = ops.dense_prefill(qg, kg, vg)
    _close(hyb.float().cpu().numpy(), dense.float().cpu().numpy(), "keep-all fp16")


def test_mixed_dtypes_are_rejected(gpu):
    from deltaattention_amd import ops
    q, k, v = _bf16_inputs(1, 4, 1, 256, 128, seed=1)
    with pytest.raises(TypeError):
        ops.dense_prefill(q.to(gpu), k.half().to(gpu), v.to(gpu))


# --------------------------------------------------------------------------------------
# key / value rows 2^22 + 8 elements apart: byte pitch 2^23 + 16, past the signed 24-bit
# range of the staging's row-offset product (an unsigned product is exact up to 2^24)
# --------------------------------------------------------------------------------------
def test_attention_with_sequence_stride_past_2_pow_22(gpu):
    from deltaattention_amd import ops
    B, Hq, Hkv, N, D, W = 1, 4, 1, 160, 128, 32
    stride = (1 << 22) + 8
    q, k, v = _bf16_inputs(B, Hq, Hkv, N, D, seed=23)
    announce(f"dense + hybrid, K/V/K^/V^ sequence stride {stride} elements, N={N} Hq={Hq}")

    def spread(t):
        # [B, 1, N, D] rows placed `stride` elements apart in one large buffer
        buf = torch.zeros(N * stride, dtype=t.dtype, device=gpu)
        view = buf.as_strided((B, Hkv, N, D), (N * stride, N * stride, stride, 1))
        view.copy_(t.to(gpu))
        return view, buf

    kd, kbuf = spread(k)
    vd, vbuf = spread(v)
    qd = q.to(gpu)
    out = ops.dense_prefill(qd, kd, vd, causal=True)
    torch.cuda.synchronize()
    want = O.dense_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), True)
    _close(out.float().cpu().numpy(), want, "dense, stride 2^22+8")

    tau = 9.0
    keep, _ = ops.select(kd, tau, 64)
    packed = ops.pack(keep, kd, vd)
    P = int(packed.num_packed.item())
    kp, kpbuf = spread(packed.k_packed[:, :, :N].float().cpu().to(torch.bfloat16))
    vp, vpbuf = spread(packed.v_packed[:, :, :N].float().cpu().to(torch.bfloat16))
    out_h = ops.hybrid_prefill(qd, kd, vd, kp, vp, packed.timestamps, packed.counts, window=W,
                               num_packed_dev=packed.num_packed)
    torch.cuda.synchronize()
    kf, vf = k.float().numpy(), v.float().numpy()
    okeep, _ = OC.select_delta(kf, tau, 64, arith=oracle_arith(k))
    p = O.pack(kf, vf, okeep)
    assert p["P"] == P
    want_h = O.hybrid_attention(q.float().numpy(), kf, vf, p["k_packed"], p["v_packed"], p["timestamps"],
                                p["counts"], W)
    _close(out_h.float().cpu().numpy(), want_h, "hybrid, stride 2^22+8")
    del kbuf, vbuf, kpbuf, vpbuf
