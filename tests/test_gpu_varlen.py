"""Ragged batched prefill (config 4 semantics): a packed [tokens, heads, 128] batch with
cu_seqlens, where each sequence is exactly a B = 1 delta prefill.  The reference has no
varlen API, so parity is each sequence run on its own as B = 1."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu

LENS = [300, 5, 1537, 1000, 64]   # ragged, a tiny one, one not a multiple of 64/128


def _batch(lens, hq=8, hkv=2, d=128, seed=3):
    from deltaattention_amd import synth
    qs, ks, vs = [], [], []
    for i, n in enumerate(lens):
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
        keep, _ = O.select_delta(kb, tau, 512)
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
