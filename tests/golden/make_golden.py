"""Write golden vectors for the hybrid prefill kernels from the reference itself.

Run in the build container only (``python tests/golden/make_golden.py``): it imports
the reference's ``deltaFlashAttention.py`` from /root/reference with
``TRITON_INTERPRET=1`` so Triton executes the kernels on CPU tensors, and saves the
inputs (q, k, v and the keep mask; the packed tensors are re-derived with the
oracle's ``pack``, which integer closed forms pin) and the outputs as
``tests/golden/hybrid_golden.npz``.  Nothing under
/root/reference is copied; the fixture is data (inputs + outputs).

Why these functions: the hybrid kernel's double counting of tokens in [ds, last] and
its padding-block quirk (fully zero-padded packed blocks have timestamp 0 and reset
Phase 2 to key 0, deltaFlashAttention.py:66-109) are behaviours that only the
reference's code fixes; no closed form or invariant pins them.  The same holds for
the Phase-2 start of the sanity variant.  The interpreter pins the control flow and
fp32 math, not GPU rounding.

Launch parameters follow the reference wrappers (modeling_llama.py:306-451):
BLOCK_M = BLOCK_N = 128, BLOCK_D = next_pow2(D), counts as fp32, K/V/packed tensors
expanded to the query heads as repeat_kv does (modeling_llama.py:701-708).
"""
from __future__ import annotations

import os
import sys

os.environ["TRITON_INTERPRET"] = "1"

import numpy as np  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
REF = "/root/reference"


def _bf16(x):
    """Inputs are rounded to bf16-representable fp32 values so that the bf16 HIP kernels
    consume exactly the inputs the reference saw."""
    from oracle import delta_oracle as O
    return O.bf16_round(np.asarray(x, dtype=np.float32))


def _normal(rng, shape):
    return _bf16(rng.standard_normal(shape))


def _ar1_keys(rng, B, H, N, D, rho=0.9, sigma=0.44):
    e = rng.standard_normal((B, H, N, D)).astype(np.float64)
    k = np.empty_like(e)
    k[:, :, 0] = e[:, :, 0]
    for t in range(1, N):
        k[:, :, t] = rho * k[:, :, t - 1] + sigma * e[:, :, t]
    return _bf16(k)


def _pack_from_keep(k, v, keep):
    from oracle import delta_oracle as O
    return O.pack(k, v, keep)


def make_cases():
    from oracle import delta_oracle as O
    rng = np.random.default_rng(1234)
    cases = []

    # A: realistic delta selection, N not a multiple of 128, W = 128; Phase 1 runs for
    # query blocks 4-7 with 1-2 packed blocks (double counting of [ds, last]).
    B, Hq, Hkv, N, D = 1, 4, 2, 1000, 32
    k = _ar1_keys(rng, B, Hkv, N, D)
    v = _normal(rng, (B, Hkv, N, D))
    q = _normal(rng, (B, Hq, N, D))
    keep, _ = O.select_delta(k, 3.6, 512, 0, "euclidean")
    cases.append(("A", q, k, v, keep, 128, False))

    # B: constructed keep masks that trigger the padding-block quirk: head 0 keeps every
    # 3rd position of [0, 300) (100 anchors), head 1 keeps 400 random positions, so P = 400
    # and head 0 has fully padded blocks [128, 256) and [256, 384) with timestamp 0.
    N = 640
    k = _ar1_keys(rng, B, Hkv, N, D)
    v = _normal(rng, (B, Hkv, N, D))
    q = _normal(rng, (B, Hq, N, D))
    keep = np.zeros((B, Hkv, N), np.int32)
    keep[0, 0, 0:300:3] = 1
    sel = np.sort(rng.choice(np.arange(1, N), size=399, replace=False))
    keep[0, 1, 0] = 1
    keep[0, 1, sel] = 1
    cases.append(("B", q, k, v, keep, 128, False))

    # C: random keep masks of different density per head, W = 0, no_count.
    N = 512
    k = _ar1_keys(rng, B, Hkv, N, D)
    v = _normal(rng, (B, Hkv, N, D))
    q = _normal(rng, (B, Hq, N, D))
    keep = np.zeros((B, Hkv, N), np.int32)
    keep[0, 0] = (rng.random(N) < 0.30)
    keep[0, 1] = (rng.random(N) < 0.55)
    keep[..., 0] = 1
    cases.append(("C", q, k, v, keep, 0, True))

    # D: W larger than the sequence (=> dense), GQA group 4.
    Hq, Hkv, N = 4, 1, 384
    k = _ar1_keys(rng, B, Hkv, N, D)
    v = _normal(rng, (B, Hkv, N, D))
    q = _normal(rng, (B, Hq, N, D))
    keep, _ = O.select_delta(k, 4.2, 128, 0, "euclidean")
    cases.append(("D", q, k, v, keep, 1000, False))
    return cases


def run_reference(q, k, v, kp, vp, ts, cnt, W, no_count, variant):
    import torch
    import triton
    sys.path.insert(0, REF)
    import deltaFlashAttention as dfa  # the reference module, interpreted on CPU

    B, Hq, N, D = q.shape
    G = Hq // k.shape[1]
    ex = lambda a: torch.from_numpy(np.ascontiguousarray(np.repeat(a, G, axis=1)))
    qt = torch.from_numpy(q)
    kd, vd, kpt, vpt = ex(k), ex(v), ex(kp), ex(vp)
    tst = ex(ts).to(torch.int32)
    ct = ex(cnt).to(torch.float32)
    if no_count:
        ct = torch.ones_like(ct)
    out = torch.empty_like(qt)
    kern = {"hybrid": dfa.hybrid_compressed_flash_kernel,
            "sanity": dfa.hybrid_compressed_flash_kernel_sanity,
            "pure_phase1": dfa.pure_phase1_flash_kernel}[variant]
    grid = (triton.cdiv(N, 128), B * Hq, 1)
    kern[grid](
        qt, kd, vd, kpt, vpt, tst, ct, out,
        *qt.stride(), *kd.stride(), *vd.stride(), *kpt.stride(), *vpt.stride(),
        *tst.stride(), *ct.stride(), *out.stride(),
        D ** -0.5, N, kd.shape[2], kpt.shape[2], D, Hq, W,
        BLOCK_M=128, BLOCK_N=128, BLOCK_D=triton.next_power_of_2(D),
        num_warps=8, num_stages=1)
    return out.numpy().copy()


def main():
    blobs = {}
    for name, q, k, v, keep, W, no_count in make_cases():
        p = _pack_from_keep(k, v, keep)
        blobs[f"{name}/q"] = q
        blobs[f"{name}/k"] = k
        blobs[f"{name}/v"] = v
        blobs[f"{name}/keep"] = keep
        blobs[f"{name}/window"] = np.int64(W)
        blobs[f"{name}/no_count"] = np.int64(no_count)
        for variant in ("hybrid", "sanity", "pure_phase1"):
            o = run_reference(q, k, v, p["k_packed"], p["v_packed"], p["timestamps"],
                              p["counts"], W, no_count, variant)
            blobs[f"{name}/out_{variant}"] = o
            print(name, variant, "P", p["P"], "c", p["anchor_counts"].ravel(), "nan", int(np.isnan(o).sum()),
                  flush=True)
    path = os.path.join(HERE, "hybrid_golden.npz")
    np.savez_compressed(path, **blobs)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
