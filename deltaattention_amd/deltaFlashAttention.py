"""Two-phase compressed flash prefill kernels with the reference's names
(deltaFlashAttention.py).

``hybrid_compressed_flash_kernel``, ``hybrid_compressed_flash_kernel_sanity`` and
``pure_phase1_flash_kernel`` accept the reference's ``kernel[grid](...)`` launch and run
the gfx950 kernel of libdeltaattn.so.  The inputs are the per-query-head tensors the
reference's wrappers pass (repeat_kv-expanded), so every head is its own KV head here;
``ops.hybrid_prefill`` is the GQA-native entry that reads each KV head once.
"""
from __future__ import annotations

import ctypes

import torch

from ._launch import HALF, KernelLauncher, tensor, unit_stride
from ._native import DA_F32, DA_I32, DA_VARIANT, check, dtype_code, lib, strides_array

__all__ = ["hybrid_compressed_flash_kernel", "hybrid_compressed_flash_kernel_sanity",
           "pure_phase1_flash_kernel"]

_PARAMS = ("Q", "K_dense", "V_dense", "K_packed", "V_packed", "Packed_Timestamps",
           "Packed_Counts", "Out",
           "stride_qb", "stride_qh", "stride_qm", "stride_qd",
           "stride_kdb", "stride_kdh", "stride_kdn", "stride_kdd",
           "stride_vdb", "stride_vdh", "stride_vdn", "stride_vdd",
           "stride_kpb", "stride_kph", "stride_kpn", "stride_kpd",
           "stride_vpb", "stride_vph", "stride_vpn", "stride_vpd",
           "stride_ptb", "stride_pth", "stride_ptn",
           "stride_pcb", "stride_pch", "stride_pcn",
           "stride_ob", "stride_oh", "stride_om", "stride_od",
           "sm_scale", "seq_len_q", "seq_len_k", "num_packed_keys", "head_dim", "num_heads",
           "denseWindowSize", "BLOCK_M", "BLOCK_N", "BLOCK_D")


class _HybridKernel(KernelLauncher):
    PARAMS = _PARAMS

    def __init__(self, name: str, variant: str):
        self.NAME = name
        self.variant = variant

    def launch(self, grid, a):
        if int(a["BLOCK_M"]) != 128 or int(a["BLOCK_N"]) != 128:
            raise NotImplementedError(
                f"{self.NAME}: the schedule is defined on 128x128 logical blocks "
                "(BLOCK_M = BLOCK_N = 128, modeling_llama.py:328-329)")
        q = tensor(a, "Q", HALF)
        kd = tensor(a, "K_dense", HALF)
        vd = tensor(a, "V_dense", HALF)
        kp = tensor(a, "K_packed", HALF)
        vp = tensor(a, "V_packed", HALF)
        ts = tensor(a, "Packed_Timestamps", torch.int32)
        cnt = tensor(a, "Packed_Counts")
        out = tensor(a, "Out", HALF)
        if cnt.dtype not in (torch.float32, torch.int32):
            raise TypeError("Packed_Counts must be float32 or int32")
        unit_stride(a, "stride_qd", "stride_kdd", "stride_vdd", "stride_kpd", "stride_vpd",
                    "stride_od", "stride_ptn", "stride_pcn")
        H = int(a["num_heads"])
        if grid[1] % H:
            raise ValueError("grid[1] must be batch * num_heads")
        B = grid[1] // H
        st = strides_array([a[n] for n in (
            "stride_qb", "stride_qh", "stride_qm", "stride_kdb", "stride_kdh", "stride_kdn",
            "stride_vdb", "stride_vdh", "stride_vdn", "stride_kpb", "stride_kph", "stride_kpn",
            "stride_vpb", "stride_vph", "stride_vpn", "stride_ob", "stride_oh", "stride_om",
            "stride_ptb", "stride_pth", "stride_ptn", "stride_pcb", "stride_pch", "stride_pcn")])
        P = int(a["num_packed_keys"])
        nq, nk, D = int(a["seq_len_q"]), int(a["seq_len_k"]), int(a["head_dim"])
        ws_bytes = lib().da_hybrid_workspace_size(B, H, max(P, 1))
        ws = torch.empty((max(1, ws_bytes),), dtype=torch.uint8, device=q.device)
        rc = lib().da_hybrid_prefill(
            q.data_ptr(), kd.data_ptr(), vd.data_ptr(), kp.data_ptr(), vp.data_ptr(),
            ts.data_ptr(), cnt.data_ptr(), DA_F32 if cnt.dtype == torch.float32 else DA_I32,
            out.data_ptr(), dtype_code(q, kd, vd, kp, vp, out), B, H, H, nq, nk, D, st, P, None, int(a["denseWindowSize"]),
            ctypes.c_float(float(a["sm_scale"])), DA_VARIANT[self.variant], 0, ws.data_ptr(),
            ws_bytes, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        check(rc, self.NAME)


hybrid_compressed_flash_kernel = _HybridKernel("hybrid_compressed_flash_kernel", "hybrid")
hybrid_compressed_flash_kernel_sanity = _HybridKernel("hybrid_compressed_flash_kernel_sanity", "sanity")
pure_phase1_flash_kernel = _HybridKernel("pure_phase1_flash_kernel", "pure_phase1")
