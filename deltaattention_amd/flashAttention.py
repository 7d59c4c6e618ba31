"""Dense flash prefill with the reference's names (flashAttention.py).

``triton_flash_attention`` and the kernel object ``_attn_fwd_flat`` run the gfx950
dense kernel of libdeltaattn.so (the uncompressed control of the delta path).
"""
from __future__ import annotations

import ctypes

import torch

from . import ops
from ._launch import HALF, KernelLauncher, tensor, unit_stride
from ._native import check, dtype_code, lib, strides_array

__all__ = ["triton_flash_attention", "_attn_fwd_flat"]


class _AttnFwdFlat(KernelLauncher):
    """Drop-in for ``_attn_fwd_flat[grid](...)`` (flashAttention.py:5-91).

    Q, K, V, Out are [Z, H, N_CTX, HEAD_DIM] with H heads each (K/V already expanded as
    the reference's wrapper passes them); causal rows attend keys j <= i.
    """

    NAME = "_attn_fwd_flat"
    PARAMS = ("Q", "K", "V", "sm_scale", "Out",
              "stride_qz", "stride_qh", "stride_qm", "stride_qk",
              "stride_kz", "stride_kh", "stride_kn", "stride_kk",
              "stride_vz", "stride_vh", "stride_vk", "stride_vn",
              "stride_oz", "stride_oh", "stride_om", "stride_on",
              "Z", "H", "N_CTX", "HEAD_DIM", "BLOCK_M", "BLOCK_N", "IS_CAUSAL")

    def launch(self, grid, a):
        q = tensor(a, "Q", HALF)
        k = tensor(a, "K", HALF)
        v = tensor(a, "V", HALF)
        o = tensor(a, "Out", HALF)
        unit_stride(a, "stride_qk", "stride_kk", "stride_vn", "stride_on")
        Z, H, N, D = int(a["Z"]), int(a["H"]), int(a["N_CTX"]), int(a["HEAD_DIM"])
        st = strides_array([a["stride_qz"], a["stride_qh"], a["stride_qm"],
                            a["stride_kz"], a["stride_kh"], a["stride_kn"],
                            a["stride_vz"], a["stride_vh"], a["stride_vk"],
                            0, 0, 0, 0, 0, 0,
                            a["stride_oz"], a["stride_oh"], a["stride_om"]] + [0] * 6)
        rc = lib().da_dense_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dtype_code(q, k, v, o),
                                    Z, H, H, N, N, D, st, 1 if a["IS_CAUSAL"] else 0,
                                    ctypes.c_float(float(a["sm_scale"])),
                                    ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        check(rc, "_attn_fwd_flat")


_attn_fwd_flat = _AttnFwdFlat()


def triton_flash_attention(q, k, v, causal=True, sm_scale=None):
    """Dense causal (or full) attention, out = softmax(q k^T * scale) v per head.

    Same contract as flashAttention.py:94-130 (inputs made contiguous, default scale
    head_dim ** -0.5, output shaped like q).  K/V may carry either the query heads
    (repeat_kv-expanded, as the reference passes them) or fewer KV heads that divide
    them, which the kernel indexes directly.
    """
    batch_size, num_heads, q_len, head_dim = q.shape
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    if sm_scale is None:
        sm_scale = 1.0 / (head_dim ** 0.5)
    return ops.dense_prefill(q, k, v, causal=causal, scale=sm_scale)
