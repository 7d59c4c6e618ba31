"""The two selection definitions: fp32 distance (the default) and the keys' own 16-bit
arithmetic (``arith="native"``), which rounds every difference, square and tree addition
as the reference's Triton code does on bf16 / fp16 keys (tritonModules.py:55-58).

Pins of the 16-bit mode: the numpy and C restatements agree bit for bit; a closed-form
pair of keys whose fp32 and bf16 distances straddle the threshold; and an independent
implementation in torch's own bf16 / fp16 tensor arithmetic (curr - ref, diff * diff and
pairwise sums on 16-bit tensors, as the reference writes them) gives the same decisions.
The last test measures, on the config-1 keys, how far the two definitions lead apart.
"""
import numpy as np
import pytest

from oracle import delta_oracle as O
from oracle import select_oracle_c as OC

torch = pytest.importorskip("torch")


def _keys(seed, H, N, D=128, dtype=torch.bfloat16):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((1, H, N, D)).astype(np.float32)
    # a slowly varying walk: adjacent keys close to each other, so decisions are near tau
    k = np.cumsum(k * 0.3, axis=2) / np.sqrt(1 + np.arange(N) * 0.09)[None, None, :, None]
    return torch.from_numpy(k.astype(np.float32)).to(dtype).float().numpy()


@pytest.mark.parametrize("arith,dtype", [("bf16", torch.bfloat16), ("fp16", torch.float16)])
def test_numpy_and_c_agree_in_16bit_arithmetic(arith, dtype):
    k = _keys(1, 2, 700, dtype=dtype)
    for tau in (3.0, 5.5, 8.0):
        a = O.select_delta(k, tau, 256, arith=arith)
        b = OC.select_delta(k, tau, 256, arith=arith)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_bf16_distance_closed_form():
    """Anchor 0, next key 1.0078125 (bf16-exact) in dimension 0: the fp32 distance is
    1.0078125^2 = 1.015686035..., its bf16 rounding 1.015625.  A threshold between them
    keeps the key in fp32 and merges it in bf16."""
    k = np.zeros((1, 1, 2, 128), np.float32)
    k[0, 0, 1, 0] = 1.0078125
    tau = float(np.sqrt(1.01566))
    for impl in (O.select_delta, OC.select_delta):
        assert impl(k, tau, 512, arith="fp32")[0][0, 0].tolist() == [1, 1]
        assert impl(k, tau, 512, arith="bf16")[0][0, 0].tolist() == [1, 0]


def _torch_reference_select(k16, tau, chunk):
    """The reference's selection loop written with torch 16-bit tensor arithmetic: diff and
    its square are 16-bit tensor ops, the sum a pairwise tree of 16-bit additions over
    the head dimension zero-padded to 128; the decision compares with tau^2 in fp32."""
    H, N, D = k16.shape
    thr = np.float32(tau * tau)
    keep = np.zeros((H, N), np.int32)
    for h in range(H):
        for s in range(0, N, chunk):
            e = min(s + chunk, N)
            a = k16[h, s]
            keep[h, s] = 1
            for i in range(s + 1, e):
                diff = k16[h, i] - a
                t = torch.zeros(128, dtype=k16.dtype)
                t[:D] = diff * diff
                while t.numel() > 1:
                    t = t[0::2] + t[1::2]
                if float(t[0]) > thr:
                    keep[h, i] = 1
                    a = k16[h, i]
    return keep


@pytest.mark.parametrize("arith,dtype", [("bf16", torch.bfloat16), ("fp16", torch.float16)])
def test_16bit_mode_matches_torch_16bit_arithmetic(arith, dtype):
    k = _keys(2, 2, 300, dtype=dtype)
    k16 = torch.from_numpy(k[0]).to(dtype)
    for tau in (2.5, 4.0):
        want = _torch_reference_select(k16, tau, 128)
        got, _ = OC.select_delta(k, tau, 128, arith=arith)
        assert np.array_equal(got[0], want), (arith, tau)


def test_f16_round_matches_torch():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(100000) * np.exp2(rng.integers(-30, 18, 100000))).astype(np.float32)
    got = O.f16_round(x)
    want = torch.from_numpy(x).to(torch.float16).float().numpy()
    assert np.array_equal(got, want)


def test_definition_gap_on_config1_keys():
    """Config-1 keys (8 KV heads x 32768, AR(1) rho = 0.9 + RoPE base 5e5, bf16) at the
    thresholds calibrated to r = 2, 4, 8: the fraction of positions whose decision differs
    between the fp32 and the bf16 definitions, and the realised ratios."""
    from deltaattention_amd import synth
    k = synth.ar1_keys(1, 8, 32768, 128, 0.9, 0.44, seed=0)
    k = synth.apply_rope(k, 500000.0).to(torch.bfloat16).float().numpy()
    for tau in (6.6807, 10.3327, 12.9053):
        a, ca = OC.select_delta(k, tau, 512, arith="fp32")
        b, cb = OC.select_delta(k, tau, 512, arith="bf16")
        flips = float((a != b).mean())
        ra, rb = a.size / a.sum(), b.size / b.sum()
        print(f"tau {tau}: flip rate {flips:.3%}, realised r {ra:.4f} (fp32) vs {rb:.4f} (bf16), "
              f"chunks with a difference {(ca != cb).mean():.1%}")
        assert flips < 0.05
        assert abs(ra / rb - 1) < 0.01
