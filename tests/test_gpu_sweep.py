"""Randomized GPU parity over the knobs together: 24 configurations drawn with a fixed
seed (GQA group, KV heads, batch, length, head dim, 16-bit type, metric, 16-bit
arithmetic, chunk size, threshold, window, variant, no_count), each run through
select -> pack -> hybrid prefill on the GPU and through the oracle on the CPU.

Bars: keep masks, chunk counts, P, timestamps and counts bit-exact; attention within
max-abs 2e-2 (bf16) / 5e-3 (fp16) and mean-abs 1e-3 of the fp32 oracle."""
import numpy as np
import pytest
import torch

from conftest import announce
from oracle import delta_oracle as O
from oracle import select_oracle_c as OC

pytestmark = pytest.mark.gpu


def _cases(n=24, seed=7):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        G = int(rng.choice([1, 2, 3, 4, 8]))
        Hkv = int(rng.choice([1, 2, 3]))
        metric = "cosine" if rng.random() < 0.25 else "euclidean"
        D = int(rng.choice([64, 80, 96, 128, 128, 128]))
        out.append(dict(
            B=int(rng.choice([1, 2])), Hq=G * Hkv, Hkv=Hkv, N=int(rng.integers(64, 3500)), D=D,
            fp16=bool(rng.random() < 0.25), metric=metric,
            native=bool(metric == "euclidean" and rng.random() < 0.3),
            chunk=int(rng.choice([512, 512, 256, 100, 1000])),
            tau=float(rng.uniform(0.7, 0.98)) if metric == "cosine"
            else float(rng.uniform(4.0, 14.0) * (D / 128) ** 0.5),
            W=int(rng.choice([0, 64, 128, 128, 300])),
            variant=str(rng.choice(["hybrid", "hybrid", "sanity", "pure_phase1"])),
            no_count=bool(rng.random() < 0.2), seed=int(rng.integers(0, 1 << 30))))
    return out


CASES = _cases()


def _id(c):
    return (f"B{c['B']}-Hq{c['Hq']}-Hkv{c['Hkv']}-N{c['N']}-D{c['D']}-{'f16' if c['fp16'] else 'bf16'}-"
            f"{c['metric'][:3]}{'-n16' if c['native'] else ''}-c{c['chunk']}-W{c['W']}-{c['variant']}"
            f"{'-nc' if c['no_count'] else ''}")


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_random_knobs_vs_oracle(gpu, c):
    from deltaattention_amd import ops, synth
    dtype = torch.float16 if c["fp16"] else torch.bfloat16
    announce(f"sweep {_id(c)} tau={c['tau']:.3f}")
    q, k, v = synth.make_layer_inputs(c["B"], c["Hq"], c["Hkv"], c["N"], c["D"], seed=c["seed"],
                                      rope_base=10000.0)
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    qg, kg, vg = q.to(gpu), k.to(gpu), v.to(gpu)
    arith = "native" if c["native"] else "fp32"
    keep, cc = ops.select(kg, c["tau"], c["chunk"], 0, c["metric"], arith=arith)
    o_arith = ("fp16" if c["fp16"] else "bf16") if c["native"] else "fp32"
    ok, occ = OC.select_delta(k.float().numpy(), c["tau"], c["chunk"], 0, c["metric"], arith=o_arith)
    assert np.array_equal(cc.cpu().numpy(), occ), "chunk counts differ"
    assert np.array_equal(keep.cpu().numpy(), ok), "keep differs"
    packed = ops.pack(keep, kg, vg)
    out = ops.hybrid_prefill(qg, kg, vg, packed.k_packed, packed.v_packed, packed.timestamps,
                             packed.counts, window=c["W"], variant=c["variant"],
                             no_count=c["no_count"], num_packed_dev=packed.num_packed)
    kf, vf = k.float().numpy(), v.float().numpy()
    p = O.pack(kf, vf, ok)
    P = int(packed.num_packed.item())
    assert P == p["P"]
    assert np.array_equal(packed.timestamps[:, :, :P].cpu().numpy(), p["timestamps"])
    assert np.array_equal(packed.counts[:, :, :P].cpu().numpy(), p["counts"])
    ref = O.hybrid_attention(q.float().numpy(), kf, vf, p["k_packed"], p["v_packed"], p["timestamps"],
                             p["counts"], c["W"], variant=c["variant"], no_count=c["no_count"])
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    mx, mean = float(err.max()), float(err.mean())
    print(f"{_id(c)}: max-abs {mx:.3e} mean-abs {mean:.3e}", flush=True)
    assert mx <= (5e-3 if c["fp16"] else 2e-2) and mean <= 1e-3, f"max-abs {mx:.3e} mean-abs {mean:.3e}"
