"""Ragged batched prefill (config 4 semantics): a packed [tokens, heads, 128] batch with
cu_seqlens, where each sequence is exactly a B = 1 delta prefill.  The reference has no
varlen API, so parity is each sequence run on its own as B = 1."""
import numpy as np
import pytest
import torch

from conftest import announce, oracle_arith
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu

LENS = [300, 5, 1537, 1000, 64]   # ragged, a tiny one, one not a multiple of 64/128


def _batch(lens, hq=8, hkv=2, d=128, seed=3):
    from deltaattention_amd import synth
    qs, ks, vs = [], [], []
    for i, n in enumerate(lens):
        if n == 0:
            for lst, h in ((qs, hq), (ks, hkv), (vs, hkv)):
                lst.append(torch.zeros((0, h, d), dtype=torch.bfloat16, device="cuda"))
            continue
        rho = np.random.default_rng(seed + i).uniform(0.6, 0.95, size=hkv)  # per head
        q, k, v = synth.make_layer_inputs(1, hq, hkv, n, d, rho=rho, seed=seed + i,
                                          device="cuda")
        qs.append(q[0].permute(1, 0, 2))
        ks.append(k[0].permute(1, 0, 2))
        vs.append(v[0].permute(1, 0, 2))
    cu = np.concatenate([[0], np.cumsum(lens)]).tolist()
    return torch.cat(qs).contiguous(), torch.cat(ks).contiguous(), torch.cat(vs).contiguous(), cu


def test_varlen_delta_equals_per_sequence_runs(gpu):
    from deltaattention_amd import ops
    announce(f"varlen delta prefill vs per-sequence B=1 runs, lens {LENS}")
    q, k, v, cu = _batch(LENS)
    tau = 9.0
    out = ops.delta_prefill_varlen(q, k, v, cu, tau, 512, window=128)
    for s, e in zip(cu[:-1], cu[1:]):
        qb = q[s:e].permute(1, 0, 2).unsqueeze(0).contiguous()
        kb = k[s:e].permute(1, 0, 2).unsqueeze(0).contiguous()
        vb = v[s:e].permute(1, 0, 2).unsqueeze(0).contiguous()
        ref = ops.delta_prefill(qb, kb, vb, tau, 512, window=128)
        got = out[s:e].permute(1, 0, 2).unsqueeze(0)
        assert torch.equal(got, ref), f"sequence [{s}, {e})"


def test_varlen_delta_matches_oracle(gpu):
    from deltaattention_amd import ops
    announce(f"varlen delta prefill vs oracle per sequence, lens {LENS}")
    q, k, v, cu = _batch(LENS)
    tau = 9.0
    out = ops.delta_prefill_varlen(q, k, v, cu, tau, 512, window=128).float().cpu().numpy()
    worst = 0.0
    for s, e in zip(cu[:-1], cu[1:]):
        qb = q[s:e].permute(1, 0, 2)[None].float().cpu().numpy()
        kb = k[s:e].permute(1, 0, 2)[None].float().cpu().numpy()
        vb = v[s:e].permute(1, 0, 2)[None].float().cpu().numpy()
        keep, _ = O.select_delta(kb, tau, 512, arith=oracle_arith(k))
        p = O.pack(kb, vb, keep)
        ref = O.hybrid_attention(qb, kb, vb, p["k_packed"], p["v_packed"], p["timestamps"],
                                 p["counts"], 128)
        got = out[s:e].transpose(1, 0, 2)[None]
        err = np.abs(got - ref)
        worst = max(worst, float(err.max()))
        assert err.max() <= 2e-2 and err.mean() <= 1e-3, f"sequence [{s}, {e}): {err.max()}"
    print(f"varlen vs oracle: worst max-abs {worst:.3e}")


def test_varlen_dense_matches_per_sequence_dense(gpu):
    from deltaattention_amd import ops
    announce(f"varlen dense prefill vs per-sequence dense, lens {LENS}")
    q, k, v, cu = _batch(LENS)
    out = ops.dense_prefill_varlen(q, k, v, cu)
    for s, e in zip(cu[:-1], cu[1:]):
        qb = q[s:e].permute(1, 0, 2).unsqueeze(0).contiguous()
        kb = k[s:e].permute(1, 0, 2).unsqueeze(0).contiguous()
        vb = v[s:e].permute(1, 0, 2).unsqueeze(0).contiguous()
        ref = ops.dense_prefill(qb, kb, vb)
        assert torch.equal(out[s:e].permute(1, 0, 2).unsqueeze(0), ref)


def test_varlen_rejects_bad_cu_seqlens(gpu):
    from deltaattention_amd import ops
    q, k, v, cu = _batch([64, 64])
    with pytest.raises(ValueError, match="cu_seqlens"):
        ops.delta_prefill_varlen(q, k, v, [0, 100, 64], 9.0)
    with pytest.raises(ValueError, match="cu_seqlens"):
        ops.dense_prefill_varlen(q, k, v, [0, 64])


LENS2 = [1000, 0, 700, 1, 2100, 129]   # an empty sequence and a one-token one


def _per_seq(x, s, e):
    return x[s:e].permute(1, 0, 2).unsqueeze(0).contiguous()


@pytest.mark.parametrize("chunk,divide_to", [(512, 0), (0, 3)])
def test_varlen_select_pack_bitexact(gpu, chunk, divide_to):
    """select_varlen and pack_varlen against the oracle run on each sequence alone:
    keep rows, chunk counts, anchor counts, P_b, timestamps, counts and packed rows
    bit-exact, zero padding up to P_b included."""
    from deltaattention_amd import ops
    from oracle import select_oracle_c as OC
    q, k, v, cu = _batch(LENS2, hq=8, hkv=2)
    tau = 9.0
    announce(f"varlen select+pack lens {LENS2} chunk={chunk} divide_to={divide_to}")
    keep, cc = ops.select_varlen(k, cu, tau, chunk, divide_to)
    packed = ops.pack_varlen(keep, k, v, cu)
    torch.cuda.synchronize()
    keep_h, cc_h = keep.cpu().numpy(), cc.cpu().numpy()
    P_h = packed.num_packed.cpu().numpy()
    for b, (s, e) in enumerate(zip(cu[:-1], cu[1:])):
        n = e - s
        if n == 0:
            assert P_h[b] == 0 and (cc_h[b] == 0).all()
            continue
        kf = _per_seq(k, s, e).float().cpu().numpy()
        vf = _per_seq(v, s, e).float().cpu().numpy()
        okeep, occ = OC.select_delta(kf, tau, chunk, divide_to, arith=oracle_arith(k))
        assert np.array_equal(keep_h[:, s:e], okeep[0]), f"keep of sequence {b}"
        assert np.array_equal(cc_h[b, :, :occ.shape[-1]], occ[0]) and (cc_h[b, :, occ.shape[-1]:] == 0).all()
        ref = O.pack(kf, vf, okeep)
        P = ref["P"]
        assert P_h[b] == P
        assert np.array_equal(packed.anchor_counts[b].cpu().numpy(), ref["anchor_counts"][0])
        assert np.array_equal(packed.timestamps[:, s:s + P].cpu().numpy(), ref["timestamps"][0])
        assert np.array_equal(packed.counts[:, s:s + P].cpu().numpy(), ref["counts"][0])
        assert np.array_equal(packed.k_packed[s:s + P].permute(1, 0, 2).float().cpu().numpy(), ref["k_packed"][0])
        assert np.array_equal(packed.v_packed[s:s + P].permute(1, 0, 2).float().cpu().numpy(), ref["v_packed"][0])


@pytest.mark.parametrize("chunk,divide_to", [(512, 0), (0, 32)])
def test_varlen_select_pair_grid(gpu, chunk, divide_to):
    """A ragged batch whose grid reaches 2048 chunks (8 sequences x 8 KV heads x 32 chunks,
    by chunk size or by divide_to) takes the two-chunks-per-wave walk; halves past a
    sequence's last chunk write a zero count.  Keep rows and chunk counts against the
    oracle on each sequence alone."""
    from deltaattention_amd import ops
    from oracle import select_oracle_c as OC
    lens = [16384, 9000, 300, 12000, 5, 16384, 7000, 1]
    q, k, v, cu = _batch(lens, hq=8, hkv=8)
    tau = 9.0
    announce(f"varlen select pair grid lens {lens} chunk={chunk} divide_to={divide_to}")
    keep, cc = ops.select_varlen(k, cu, tau, chunk, divide_to)
    torch.cuda.synchronize()
    keep_h, cc_h = keep.cpu().numpy(), cc.cpu().numpy()
    assert cc_h.shape[-1] * cc_h.shape[0] * cc_h.shape[1] >= 2048
    for b, (s, e) in enumerate(zip(cu[:-1], cu[1:])):
        kf = _per_seq(k, s, e).float().cpu().numpy()
        okeep, occ = OC.select_delta(kf, tau, chunk, divide_to, arith=oracle_arith(k))
        assert np.array_equal(keep_h[:, s:e], okeep[0]), f"keep of sequence {b}"
        assert np.array_equal(cc_h[b, :, :occ.shape[-1]], occ[0]) and (cc_h[b, :, occ.shape[-1]:] == 0).all()


@pytest.mark.parametrize("hq,hkv", [(8, 2), (6, 3)], ids=["gqa4-grouped", "gqa2-per-head"])
@pytest.mark.parametrize("variant", ["hybrid", "sanity", "pure_phase1"])
def test_varlen_variants_equal_per_sequence_runs(gpu, hq, hkv, variant):
    """One varlen launch equals B = 1 launches sequence by sequence, bit for bit, for every
    variant and for both attention kernels (GQA group a multiple of 4 or not); the empty
    sequence leaves its (zero) rows untouched.  cu_seqlens is passed as a device tensor
    with max_seqlen."""
    from deltaattention_amd import ops
    q, k, v, cu = _batch(LENS2, hq=hq, hkv=hkv)
    tau = 9.0
    announce(f"varlen {variant} Hq={hq} Hkv={hkv} lens {LENS2}")
    cu_dev = torch.tensor(cu, dtype=torch.int32, device=gpu)
    out = ops.delta_prefill_varlen(q, k, v, cu_dev, tau, 512, window=128, variant=variant,
                                   max_seqlen=max(LENS2))
    dense = ops.dense_prefill_varlen(q, k, v, cu_dev, max_seqlen=max(LENS2))
    for s, e in zip(cu[:-1], cu[1:]):
        if e == s:
            continue
        ref = ops.delta_prefill(_per_seq(q, s, e), _per_seq(k, s, e), _per_seq(v, s, e), tau, 512,
                                window=128, variant=variant)
        assert torch.equal(_per_seq(out, s, e), ref), f"{variant} sequence [{s}, {e})"
        ref = ops.dense_prefill(_per_seq(q, s, e), _per_seq(k, s, e), _per_seq(v, s, e))
        assert torch.equal(_per_seq(dense, s, e), ref), f"dense sequence [{s}, {e})"
