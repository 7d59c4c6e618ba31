"""Anchor selection and packing with the reference's kernel names (tritonModules.py).

``chunked_eval_kernel[grid](...)`` and ``parallel_scatter_pack_kv_kernel[grid](...)``
take the reference's arguments and run the gfx950 kernels of libdeltaattn.so.
"""
from __future__ import annotations

import ctypes

import torch

from ._launch import HALF, KernelLauncher, tensor, unit_stride
from ._native import check, dtype_code, lib

__all__ = ["chunked_eval_kernel", "parallel_scatter_pack_kv_kernel"]


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


class _ChunkedEval(KernelLauncher):
    """Drop-in for ``chunked_eval_kernel[(B*H, num_chunks)](...)`` (tritonModules.py:7-69).

    ``threshold_sq`` is tau^2 for Euclidean and tau for cosine, as the caller passes it
    (modeling_llama.py:641-642).  keep_mask [B,H,N] and chunk_counts [B,H,nc] must be
    contiguous int32.
    """

    NAME = "chunked_eval_kernel"
    PARAMS = ("in_ptr", "keep_mask_ptr", "chunk_counts_ptr", "threshold_sq",
              "stride_in_b", "stride_in_h", "stride_in_s", "stride_in_d",
              "stride_km_b", "stride_km_h", "stride_km_s",
              "stride_cc_b", "stride_cc_h", "stride_cc_c",
              "seq_len", "head_dim", "chunk_size", "num_heads", "BLOCK_D", "USE_COSINE")

    def launch(self, grid, a):
        k = tensor(a, "in_ptr", HALF)
        keep = tensor(a, "keep_mask_ptr", torch.int32)
        cc = tensor(a, "chunk_counts_ptr", torch.int32)
        unit_stride(a, "stride_in_d")
        H, N, D = int(a["num_heads"]), int(a["seq_len"]), int(a["head_dim"])
        if grid[0] % H:
            raise ValueError("grid[0] must be batch * num_heads")
        B, nc = grid[0] // H, grid[1]
        if (int(a["stride_km_s"]), int(a["stride_km_h"]), int(a["stride_km_b"])) != (1, N, H * N):
            raise ValueError("keep_mask must be a contiguous [B, H, N] tensor")
        if (int(a["stride_cc_c"]), int(a["stride_cc_h"]), int(a["stride_cc_b"])) != (1, nc, H * nc):
            raise ValueError("chunk_counts must be a contiguous [B, H, num_chunks] tensor")
        rc = lib().da_select(k.data_ptr(), dtype_code(k), B, H, N, D, int(a["stride_in_b"]),
                             int(a["stride_in_h"]), int(a["stride_in_s"]),
                             ctypes.c_float(float(a["threshold_sq"])), _flags(bool(a["USE_COSINE"])),
                             int(a["chunk_size"]), nc, keep.data_ptr(), cc.data_ptr(), _stream())
        check(rc, "chunked_eval_kernel")


def _flags(use_cosine: bool) -> int:
    """da_select flags: the cosine test, or the Euclidean distance in the keys' 16-bit
    arithmetic as the replaced kernel computes it (tritonModules.py:55-58; the default,
    globVR.row_delta_arith == "native") or in fp32 (globVR.row_delta_arith == "fp32")."""
    from . import globVR
    from ._native import DA_SELECT_ARITH16, DA_SELECT_COSINE
    if use_cosine:
        return DA_SELECT_COSINE
    return DA_SELECT_ARITH16 if getattr(globVR, "row_delta_arith", "native") == "native" else 0


class _ScatterPack(KernelLauncher):
    """Drop-in for ``parallel_scatter_pack_kv_kernel[(B*H, cdiv(N, BLOCK_S))](...)``
    (tritonModules.py:72-132).

    Writes K-hat, V-hat and the timestamps of every anchor at its packed index; the
    packed tensors must be contiguous [B, H, P, D] / [B, H, P].  The index map argument
    is accepted for signature compatibility: packed indices are recomputed from the keep
    mask (they equal cumsum(keep) - 1 by definition, modeling_llama.py:655).  Rows past
    a head's anchors are zero, as in the reference's zero-initialised tensors.
    """

    NAME = "parallel_scatter_pack_kv_kernel"
    PARAMS = ("k_in_ptr", "v_in_ptr", "k_packed_ptr", "v_packed_ptr", "pt_ptr",
              "keep_mask_ptr", "index_map_ptr",
              "stride_kb", "stride_kh", "stride_ks", "stride_kd",
              "stride_vb", "stride_vh", "stride_vs", "stride_vd",
              "stride_kpb", "stride_kph", "stride_kpa", "stride_kpd",
              "stride_vpb", "stride_vph", "stride_vpa", "stride_vpd",
              "stride_ptb", "stride_pth", "stride_pta",
              "stride_km_b", "stride_km_h", "stride_km_s",
              "stride_im_b", "stride_im_h", "stride_im_s",
              "seq_len", "head_dim", "num_heads", "BLOCK_S", "BLOCK_D")

    def launch(self, grid, a):
        k = tensor(a, "k_in_ptr", HALF)
        v = tensor(a, "v_in_ptr", HALF)
        kp = tensor(a, "k_packed_ptr", HALF)
        vp = tensor(a, "v_packed_ptr", HALF)
        ts = tensor(a, "pt_ptr", torch.int32)
        keep = tensor(a, "keep_mask_ptr")
        unit_stride(a, "stride_kd", "stride_vd", "stride_kpd", "stride_vpd")
        H, N, D = int(a["num_heads"]), int(a["seq_len"]), int(a["head_dim"])
        if grid[0] % H:
            raise ValueError("grid[0] must be batch * num_heads")
        B = grid[0] // H
        for t, name in ((kp, "k_packed"), (vp, "v_packed"), (ts, "packed_timestamps")):
            if not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous")
        P = kp.shape[2]
        if keep.dtype != torch.int32 or not keep.is_contiguous():
            keep = keep.to(torch.int32).contiguous()
        counts = torch.empty((B, H, P), dtype=torch.int32, device=k.device)
        ac = torch.empty((B, H), dtype=torch.int32, device=k.device)
        num = torch.empty((1,), dtype=torch.int32, device=k.device)
        ws_bytes = lib().da_pack_workspace_size(B, H, N)
        ws = torch.empty((max(1, ws_bytes),), dtype=torch.uint8, device=k.device)
        rc = lib().da_pack(keep.data_ptr(), k.data_ptr(), v.data_ptr(), dtype_code(k, v, kp, vp), B, H, N, D,
                           int(a["stride_kb"]), int(a["stride_kh"]), int(a["stride_ks"]),
                           int(a["stride_vb"]), int(a["stride_vh"]), int(a["stride_vs"]), P,
                           kp.data_ptr(), vp.data_ptr(), ts.data_ptr(), counts.data_ptr(),
                           ac.data_ptr(), num.data_ptr(), ws.data_ptr(), ws_bytes, _stream())
        check(rc, "parallel_scatter_pack_kv_kernel")


chunked_eval_kernel = _ChunkedEval()
parallel_scatter_pack_kv_kernel = _ScatterPack()
