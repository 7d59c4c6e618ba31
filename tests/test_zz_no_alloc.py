"""da_decode_attention_noalloc: decode attention with its scratch in a static device
array instead of a caller workspace.  Its output must equal da_decode_attention's on the
same cache (the same kernels run on the same inputs), call after call, including a
second, smaller call that reuses the array the first one filled; both are also checked
against the CPU oracle of deltaDecoding.py:236-362."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import announce
from oracle import delta_oracle as O

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_ABS = 1e-3


def _cache(B, Hq, Hkv, cap, W, exact, dtype, seed):
    D = 128
    rng = np.random.default_rng(seed)
    lens = rng.integers(cap // 2, cap + 1, size=B * Hkv).astype(np.int32)
    kp = rng.standard_normal((B, Hkv, cap, D)).astype(np.float32)
    kp *= rng.uniform(0.3, 2.5, size=(B, Hkv, cap, 1)).astype(np.float32)
    vp = rng.standard_normal((B, Hkv, cap, D)).astype(np.float32)
    cnt = rng.integers(1, 9, size=(B, Hkv, cap)).astype(np.int32)
    cnt[rng.random((B, Hkv, cap)) < 0.05] = 0
    kx = rng.standard_normal((B, Hkv, W, D)).astype(np.float32)
    vx = rng.standard_normal((B, Hkv, W, D)).astype(np.float32)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dtype)
    return dict(q=t(q), kp=t(kp), vp=t(vp), kx=t(kx), vx=t(vx), cnt=torch.from_numpy(cnt),
                lens=torch.from_numpy(lens), B=B, Hq=Hq, Hkv=Hkv, cap=cap, W=W, exact=exact, D=D)


def _run(c, gpu, noalloc):
    from deltaattention_amd import _native
    lib = _native.lib()
    g = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in c.items()}
    B, Hq, Hkv, cap, W, D = c["B"], c["Hq"], c["Hkv"], c["cap"], c["W"], c["D"]
    out = torch.full((B, Hq, D), float("nan"), dtype=c["q"].dtype, device=gpu)
    dt = _native.dtype_code(g["q"])
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [g["q"].data_ptr(), dt, B, Hq, Hkv, D, Hq * D, D, g["kp"].data_ptr(), g["vp"].data_ptr(),
            Hkv * cap * D, cap * D, D, g["cnt"].data_ptr(), Hkv * cap, cap, g["lens"].data_ptr(),
            cap, g["kx"].data_ptr(), g["vx"].data_ptr(), Hkv * W * D, W * D, D, W, c["exact"],
            ctypes.c_float(D ** -0.5), out.data_ptr(), Hq * D, D]
    if noalloc:
        rc = lib.da_decode_attention_noalloc(*args, stream)
        _native.check(rc, "da_decode_attention_noalloc")
    else:
        ws_bytes = lib.da_decode_workspace_size(B, Hq, cap, W)
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=gpu)
        rc = lib.da_decode_attention(*args, ws.data_ptr(), ws_bytes, stream)
        _native.check(rc, "da_decode_attention")
    torch.cuda.synchronize()
    return out.cpu()


def _oracle(c):
    st = {"k_packed": c["kp"].float().numpy(), "v_packed": c["vp"].float().numpy(),
          "counts": c["cnt"].numpy(), "lengths": c["lens"].numpy(),
          "k_exact": c["kx"].float().numpy(), "v_exact": c["vx"].float().numpy(),
          "exact_len": c["exact"], "window": c["W"]}
    return O.decode_attention(c["q"].float().numpy(), st)


def test_noalloc_matches_workspace_entry_point(gpu):
    cases = [
        ("large", _cache(1, 32, 8, 20000, 128, 128, torch.bfloat16, seed=1)),
        ("smaller", _cache(2, 8, 2, 3000, 64, 17, torch.bfloat16, seed=2)),
    ]
    for name, c in cases:
        announce(f"da_decode_attention_noalloc {name}: B={c['B']} Hq={c['Hq']} Hkv={c['Hkv']} "
                 f"cap={c['cap']} W={c['W']}")
        got = _run(c, gpu, noalloc=True)
        want = _run(c, gpu, noalloc=False)
        assert torch.equal(got, want), f"{name}: no-alloc output differs from da_decode_attention"
        err = np.abs(got.float().numpy() - _oracle(c))
        print(f"{name}: max-abs {err.max():.3e} mean-abs {err.mean():.3e}", flush=True)
        assert err.max() <= MAX_ABS and err.mean() <= MEAN_ABS


def test_noalloc_rejects_caches_beyond_the_scratch(gpu):
    """The size check runs on the host before any launch."""
    from deltaattention_amd import _native
    lib = _native.lib()
    B, Hq, Hkv, D, W = 1, 32, 8, 128, 128
    cap = 200000
    assert lib.da_decode_workspace_size(B, Hq, cap, W) > _native.DA_DECODE_SCRATCH_BYTES
    fake = torch.empty(16, dtype=torch.bfloat16, device=gpu)
    p = fake.data_ptr()
    rc = lib.da_decode_attention_noalloc(p, 1, B, Hq, Hkv, D, Hq * D, D, p, p, Hkv * cap * D,
                                         cap * D, D, p, Hkv * cap, cap, p, cap, p, p,
                                         Hkv * W * D, W * D, D, W, 0, ctypes.c_float(0.1), p,
                                         Hq * D, D, None)
    assert rc == -2
    assert b"static maximum" in lib.da_last_error()
