"""Compressed KV cache and decode kernels with the reference's names (deltaDecoding.py).

``HybridCompressedCache`` keeps the reference's layout and host-side trackers
(deltaDecoding.py:111-233): per layer a packed anchor cache [L, B, Hkv, cap, D] with
counts / timestamps / lengths, and an exact ring [L, B, Hkv, W, D].  The decode update
and decode attention run the gfx950 kernels of libdeltaattn.so; the kernel objects
``fused_hybrid_decode_update_kernel`` and ``fused_hybrid_decode_kernel`` accept the
reference's ``kernel[grid](...)`` launch.  bf16 caches only.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import globVR
from ._launch import HALF, KernelLauncher, tensor, unit_stride
from ._native import DecodeStep, check, dtype_code, lib

try:  # transformers' Cache base (the reference subclasses it, deltaDecoding.py:2, 111)
    from transformers import Cache as _CacheBase
except Exception:  # pragma: no cover - transformers is optional for the kernels
    _CacheBase = object

__all__ = ["HybridCompressedCache", "fused_hybrid_decode_update_kernel",
           "fused_hybrid_decode_kernel", "decode_attention"]


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _raw_stream(device: torch.device) -> int:
    """The current stream's handle without building a torch Stream object."""
    get = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if get is None:  # pragma: no cover - older torch
        return torch.cuda.current_stream(device).cuda_stream
    return get(device.index if device.index is not None else torch.cuda.current_device())


def _metric_threshold():
    """(threshold as the kernel sees it, use_cosine) from the globVR knobs
    (deltaDecoding.py:192-195)."""
    metric = getattr(globVR, "row_similarity_metric", "euclidean")
    use_cos = metric == "cosine"
    raw = getattr(globVR, "row_delta_threshold", 0.0)
    return (raw if use_cos else raw ** 2), use_cos


class _DecodeUpdate(KernelLauncher):
    """Drop-in for ``fused_hybrid_decode_update_kernel[(B*H,)](...)`` (deltaDecoding.py:9-104)."""

    NAME = "fused_hybrid_decode_update_kernel"
    PARAMS = ("new_k_ptr", "new_v_ptr", "k_exact_ptr", "v_exact_ptr", "k_packed_ptr",
              "v_packed_ptr", "packed_counts_ptr", "packed_timestamps_ptr", "packed_lengths_ptr",
              "exact_seq_len", "total_seq_len", "threshold_sq", "exact_window_size",
              "stride_new_b", "stride_new_h", "stride_new_s", "stride_new_d",
              "stride_exact_b", "stride_exact_h", "stride_exact_s", "stride_exact_d",
              "stride_pack_b", "stride_pack_h", "stride_pack_s", "stride_pack_d",
              "stride_pc_b", "stride_pc_h", "stride_pc_s",
              "num_heads", "head_dim", "BLOCK_D", "USE_COSINE")

    def launch(self, grid, a):
        nk = tensor(a, "new_k_ptr", HALF)
        nv = tensor(a, "new_v_ptr", HALF)
        kx = tensor(a, "k_exact_ptr", HALF)
        vx = tensor(a, "v_exact_ptr", HALF)
        kp = tensor(a, "k_packed_ptr", HALF)
        vp = tensor(a, "v_packed_ptr", HALF)
        cnt = tensor(a, "packed_counts_ptr", torch.int32)
        ts = tensor(a, "packed_timestamps_ptr", torch.int32)
        lens = tensor(a, "packed_lengths_ptr", torch.int32)
        unit_stride(a, "stride_new_d", "stride_exact_d", "stride_pack_d", "stride_pc_s")
        H = int(a["num_heads"])
        if grid[0] % H:
            raise ValueError("grid[0] must be batch * num_heads")
        B = grid[0] // H
        rc = lib().da_decode_update(
            nk.data_ptr(), nv.data_ptr(), dtype_code(nk, nv, kx, vx, kp, vp), B, H, int(a["head_dim"]),
            int(a["stride_new_b"]), int(a["stride_new_h"]), kx.data_ptr(), vx.data_ptr(),
            int(a["stride_exact_b"]), int(a["stride_exact_h"]), int(a["stride_exact_s"]),
            kp.data_ptr(), vp.data_ptr(), int(a["stride_pack_b"]), int(a["stride_pack_h"]),
            int(a["stride_pack_s"]), cnt.data_ptr(), ts.data_ptr(), int(a["stride_pc_b"]),
            int(a["stride_pc_h"]), lens.data_ptr(), kp.shape[-2], int(a["exact_seq_len"]),
            int(a["total_seq_len"]), int(a["exact_window_size"]),
            ctypes.c_float(float(a["threshold_sq"])), 1 if a["USE_COSINE"] else 0, _stream())
        check(rc, self.NAME)


class _DecodeAttention(KernelLauncher):
    """Drop-in for ``fused_hybrid_decode_kernel[(B, Hq)](...)`` (deltaDecoding.py:236-362)."""

    NAME = "fused_hybrid_decode_kernel"
    PARAMS = ("Q", "K_packed", "V_packed", "Packed_Counts", "Packed_Lengths", "K_exact", "V_exact",
              "Out", "stride_qb", "stride_qh", "stride_qd",
              "stride_kpb", "stride_kph", "stride_kpn", "stride_kpd",
              "stride_vpb", "stride_vph", "stride_vpn", "stride_vpd",
              "stride_cb", "stride_ch", "stride_cn", "stride_lb", "stride_lh",
              "stride_keb", "stride_keh", "stride_ken", "stride_ked",
              "stride_veb", "stride_veh", "stride_ven", "stride_ved",
              "stride_ob", "stride_oh", "stride_od", "sm_scale", "exact_len", "num_kv_groups",
              "head_dim", "BLOCK_M", "BLOCK_N", "BLOCK_D")

    def launch(self, grid, a):
        q = tensor(a, "Q", HALF)
        kp = tensor(a, "K_packed", HALF)
        vp = tensor(a, "V_packed", HALF)
        cnt = tensor(a, "Packed_Counts", torch.int32)
        lens = tensor(a, "Packed_Lengths", torch.int32)
        kx = tensor(a, "K_exact", HALF)
        vx = tensor(a, "V_exact", HALF)
        out = tensor(a, "Out", HALF)
        unit_stride(a, "stride_qd", "stride_kpd", "stride_vpd", "stride_cn", "stride_ked",
                    "stride_ved", "stride_od", "stride_lh")
        if (int(a["stride_kpb"]), int(a["stride_kph"]), int(a["stride_kpn"])) != \
                (int(a["stride_vpb"]), int(a["stride_vph"]), int(a["stride_vpn"])) or \
                (int(a["stride_keb"]), int(a["stride_keh"]), int(a["stride_ken"])) != \
                (int(a["stride_veb"]), int(a["stride_veh"]), int(a["stride_ven"])):
            raise ValueError("packed K/V and exact K/V must share strides")
        B, Hq = grid[0], grid[1]
        G = int(a["num_kv_groups"])
        Hkv = Hq // G
        if int(a["stride_lb"]) != Hkv:
            raise ValueError("Packed_Lengths must be a contiguous [B, Hkv] view")
        _decode_attention_launch(q, int(a["stride_qb"]), int(a["stride_qh"]), kp, vp,
                                 (int(a["stride_kpb"]), int(a["stride_kph"]), int(a["stride_kpn"])),
                                 cnt, (int(a["stride_cb"]), int(a["stride_ch"])), lens, kx, vx,
                                 (int(a["stride_keb"]), int(a["stride_keh"]), int(a["stride_ken"])),
                                 kx.shape[-2], int(a["exact_len"]), float(a["sm_scale"]), out,
                                 int(a["stride_ob"]), int(a["stride_oh"]), B, Hq, Hkv,
                                 int(a["head_dim"]), self.NAME)


def _decode_attention_launch(q, sq_b, sq_h, kp, vp, sp, cnt, sc, lens, kx, vx, sx, window,
                             exact_len, scale, out, so_b, so_h, B, Hq, Hkv, D, what):
    capacity = kp.shape[-2]
    ws_bytes = lib().da_decode_workspace_size(B, Hq, capacity, window)
    ws = torch.empty((max(1, ws_bytes),), dtype=torch.uint8, device=q.device)
    rc = lib().da_decode_attention(
        q.data_ptr(), dtype_code(q, kp, vp, kx, vx, out), B, Hq, Hkv, D, sq_b, sq_h, kp.data_ptr(), vp.data_ptr(),
        sp[0], sp[1], sp[2], cnt.data_ptr(), sc[0], sc[1], lens.data_ptr(), capacity,
        kx.data_ptr(), vx.data_ptr(), sx[0], sx[1], sx[2], window, exact_len,
        ctypes.c_float(scale), out.data_ptr(), so_b, so_h, ws.data_ptr(), ws_bytes, _stream())
    check(rc, what)


fused_hybrid_decode_update_kernel = _DecodeUpdate()
fused_hybrid_decode_kernel = _DecodeAttention()


class HybridCompressedCache(_CacheBase):
    """Packed-anchor + exact-ring KV cache (deltaDecoding.py:111-233).

    Same constructor, fields and methods as the reference.  With the transformers
    version installed here the base class needs an explicit empty layer list.
    """

    def __init__(self, config, batch_size, dtype=torch.float16, exact_window_size=50,
                 initial_capacity=1024, device="cuda"):
        if _CacheBase is not object:
            try:
                super().__init__(layers=[])
            except TypeError:
                super().__init__()
        self.exact_window_size = exact_window_size
        self.head_dim = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
        self.n_kv_heads = config.num_key_value_heads
        self.bsz = batch_size
        self.dtype = dtype
        self.device = torch.device(device)
        self.num_layers = config.num_hidden_layers
        self.capacity = initial_capacity
        L, B, H, D, W = self.num_layers, self.bsz, self.n_kv_heads, self.head_dim, exact_window_size
        self.k_packed = torch.zeros((L, B, H, self.capacity, D), device=self.device, dtype=dtype)
        self.v_packed = torch.zeros_like(self.k_packed)
        self.packed_counts = torch.zeros((L, B, H, self.capacity), device=self.device, dtype=torch.int32)
        self.packed_timestamps = torch.zeros((L, B, H, self.capacity), device=self.device, dtype=torch.int32)
        self.packed_lengths = torch.zeros((L, B * H), device=self.device, dtype=torch.int32)
        self.k_exact = torch.zeros((L, B, H, W, D), device=self.device, dtype=dtype)
        self.v_exact = torch.zeros_like(self.k_exact)
        # host trackers (no GPU synchronisation in the common case)
        self.exact_seq_lens = [0 for _ in range(L)]
        self.max_packed_len = [0 for _ in range(L)]
        self.total_seq_lens = [0 for _ in range(L)]
        self._plans = {}  # layer -> (DaDecodeStep block, workspace) for decode_step

    def _expand_capacity(self, target_capacity):
        """Grow to max(2 * capacity, target) keeping contents (deltaDecoding.py:138-157)."""
        new_capacity = max(self.capacity * 2, target_capacity)
        L, B, H, D = self.num_layers, self.bsz, self.n_kv_heads, self.head_dim
        new_k = torch.zeros((L, B, H, new_capacity, D), device=self.device, dtype=self.dtype)
        new_v = torch.zeros_like(new_k)
        new_c = torch.zeros((L, B, H, new_capacity), device=self.device, dtype=torch.int32)
        new_t = torch.zeros((L, B, H, new_capacity), device=self.device, dtype=torch.int32)
        old = self.k_packed.shape[3]
        if old > 0:
            new_k[:, :, :, :old] = self.k_packed
            new_v[:, :, :, :old] = self.v_packed
            new_c[:, :, :, :old] = self.packed_counts
            new_t[:, :, :, :old] = self.packed_timestamps
        self.k_packed, self.v_packed = new_k, new_v
        self.packed_counts, self.packed_timestamps = new_c, new_t
        self.capacity = new_capacity
        self._plans = {}

    def initialize_from_prefill(self, layer_idx, k_packed, v_packed, counts, timestamps, k_exact,
                                v_exact, original_q_len):
        """Prefill hand-off (deltaDecoding.py:159-179): every packed row (P of them,
        padding included) goes to the packed cache with length P for every head, and the
        last min(N, W) prefill tokens go to the ring."""
        p_len = k_packed.shape[2]
        self.max_packed_len[layer_idx] = p_len
        if p_len > self.capacity:
            self._expand_capacity(p_len + 1024)
        self.k_packed[layer_idx, :, :, :p_len] = k_packed
        self.v_packed[layer_idx, :, :, :p_len] = v_packed
        self.packed_counts[layer_idx, :, :, :p_len] = counts
        self.packed_timestamps[layer_idx, :, :, :p_len] = timestamps
        self.packed_lengths[layer_idx, :] = p_len
        e_len = k_exact.shape[2]
        self.k_exact[layer_idx, :, :, :e_len] = k_exact
        self.v_exact[layer_idx, :, :, :e_len] = v_exact
        self.exact_seq_lens[layer_idx] = e_len
        self.total_seq_lens[layer_idx] = original_q_len

    def update(self, key_states, value_states, layer_idx, cache_kwargs=None):
        """One decode token (deltaDecoding.py:181-227); prefill calls pass through."""
        if key_states.shape[2] > 1:
            return key_states, value_states
        if self.max_packed_len[layer_idx] + 1 >= self.capacity:
            self._expand_capacity(self.capacity + 1024)
        threshold, use_cos = _metric_threshold()
        kp, vp = self.k_packed[layer_idx], self.v_packed[layer_idx]
        kx, vx = self.k_exact[layer_idx], self.v_exact[layer_idx]
        cnt, ts = self.packed_counts[layer_idx], self.packed_timestamps[layer_idx]
        key_states = key_states if key_states.stride(-1) == 1 else key_states.contiguous()
        value_states = value_states if value_states.stride(-1) == 1 else value_states.contiguous()
        if key_states.stride()[:2] != value_states.stride()[:2]:
            value_states = value_states.contiguous()
            key_states = key_states.contiguous()
        rc = lib().da_decode_update(
            key_states.data_ptr(), value_states.data_ptr(), dtype_code(key_states, value_states, kx, vx, kp, vp), self.bsz, self.n_kv_heads,
            self.head_dim, key_states.stride(0), key_states.stride(1), kx.data_ptr(), vx.data_ptr(),
            kx.stride(0), kx.stride(1), kx.stride(2), kp.data_ptr(), vp.data_ptr(), kp.stride(0),
            kp.stride(1), kp.stride(2), cnt.data_ptr(), ts.data_ptr(), cnt.stride(0), cnt.stride(1),
            self.packed_lengths[layer_idx].data_ptr(), self.capacity,
            self.exact_seq_lens[layer_idx], self.total_seq_lens[layer_idx], self.exact_window_size,
            ctypes.c_float(float(threshold)), 1 if use_cos else 0, _stream())
        check(rc, "HybridCompressedCache.update")
        if self.exact_seq_lens[layer_idx] >= self.exact_window_size:
            self.max_packed_len[layer_idx] += 1
            if self.total_seq_lens[layer_idx] % 256 == 0:  # reconcile with the device (:219-221)
                self.max_packed_len[layer_idx] = int(self.packed_lengths[layer_idx].max().item())
        self.exact_seq_lens[layer_idx] += 1
        self.total_seq_lens[layer_idx] += 1
        return key_states, value_states

    def _plan(self, layer_idx, Hq):
        """The layer's DaDecodeStep block with the cache fields filled in, and its
        workspace; keyed by the cache tensors' addresses, so a block is never used after
        the tensors move (capacity growth, or a caller replacing them)."""
        key = (layer_idx, Hq, self.k_packed.data_ptr(), self.k_exact.data_ptr())
        plan = self._plans.get(key)
        if plan is not None:
            return plan
        st = DecodeStep()
        kp, vp = self.k_packed[layer_idx], self.v_packed[layer_idx]
        kx, vx = self.k_exact[layer_idx], self.v_exact[layer_idx]
        cnt, ts = self.packed_counts[layer_idx], self.packed_timestamps[layer_idx]
        st.k_exact, st.v_exact = kx.data_ptr(), vx.data_ptr()
        st.sx_b, st.sx_h, st.sx_s = kx.stride(0), kx.stride(1), kx.stride(2)
        st.k_packed, st.v_packed = kp.data_ptr(), vp.data_ptr()
        st.sp_b, st.sp_h, st.sp_s = kp.stride(0), kp.stride(1), kp.stride(2)
        st.counts, st.timestamps = cnt.data_ptr(), ts.data_ptr()
        st.sc_b, st.sc_h = cnt.stride(0), cnt.stride(1)
        st.lengths = self.packed_lengths[layer_idx].data_ptr()
        st.capacity = self.capacity
        st.window = self.exact_window_size
        st.dtype = dtype_code(kp, vp, kx, vx)
        st.B, st.Hq, st.Hkv, st.D = self.bsz, Hq, self.n_kv_heads, self.head_dim
        ws_bytes = lib().da_decode_workspace_size(self.bsz, Hq, self.capacity, self.exact_window_size)
        ws = torch.empty((max(1, ws_bytes),), dtype=torch.uint8, device=self.device)
        st.workspace, st.workspace_bytes = ws.data_ptr(), ws_bytes
        plan = (st, ws, ctypes.byref(st))
        self._plans[key] = plan
        return plan

    def decode_step(self, query_states, key_states, value_states, layer_idx, scaling=None):
        """One decode token of one layer in one library call: ``update`` and
        ``decode_attention`` (modeling_llama.py:565-567 then :453-518) fused into
        ``da_decode_step``, with the layer's argument block built once.  q [B, Hq, 1, D],
        key/value [B, Hkv, 1, D] -> [B, Hq, 1, D].  The cache state is that of the two calls
        in sequence, bit for bit; so is the output of every KV head whose evicted token
        merged or was dropped, while one that appended gets the same terms summed in
        another order (the new anchor is scored at the end of its key list)."""
        if self.max_packed_len[layer_idx] + 1 >= self.capacity:
            self._expand_capacity(self.capacity + 1024)
        B, Hq, _, D = query_states.shape
        want = (self.bsz, self.n_kv_heads, 1, self.head_dim)
        if (B, D) != (self.bsz, self.head_dim) or query_states.shape[2] != 1 \
                or tuple(key_states.shape) != want or tuple(value_states.shape) != want:
            raise ValueError(f"decode_step: expected q [{self.bsz}, Hq, 1, {self.head_dim}] and "
                             f"key/value {list(want)}, got {list(query_states.shape)}, "
                             f"{list(key_states.shape)}, {list(value_states.shape)}")
        st, ws, ref = self._plan(layer_idx, Hq)
        q = query_states.squeeze(2)
        if q.stride(-1) != 1:
            q = q.contiguous()
        k = key_states if key_states.stride(-1) == 1 else key_states.contiguous()
        v = value_states if value_states.stride(-1) == 1 else value_states.contiguous()
        if k.stride()[:2] != v.stride()[:2]:
            k, v = k.contiguous(), v.contiguous()
        if dtype_code(q, k, v) != st.dtype:
            raise TypeError("decode_step: query, key and value must have the cache's dtype")
        out = torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
        threshold, use_cos = _metric_threshold()
        st.new_k, st.new_v, st.sn_b, st.sn_h = k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1)
        st.q, st.sq_b, st.sq_h = q.data_ptr(), q.stride(0), q.stride(1)
        st.out, st.so_b, st.so_h = out.data_ptr(), out.stride(0), out.stride(1)
        st.exact_seq_len = self.exact_seq_lens[layer_idx]
        st.total_seq_len = self.total_seq_lens[layer_idx]
        st.threshold = float(threshold)
        st.use_cosine = 1 if use_cos else 0
        st.scale = D ** -0.5 if scaling is None else float(scaling)
        check(lib().da_decode_step(ref, _raw_stream(q.device)), "HybridCompressedCache.decode_step")
        if self.exact_seq_lens[layer_idx] >= self.exact_window_size:
            self.max_packed_len[layer_idx] += 1
            if self.total_seq_lens[layer_idx] % 256 == 0:  # reconcile with the device (:219-221)
                self.max_packed_len[layer_idx] = int(self.packed_lengths[layer_idx].max().item())
        self.exact_seq_lens[layer_idx] += 1
        self.total_seq_lens[layer_idx] += 1
        return out.unsqueeze(2)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.total_seq_lens[layer_idx]

    def get_max_length(self):
        return None

    def get_max_cache_shape(self, layer_idx: int = 0):
        return None


def decode_attention(q: torch.Tensor, cache: HybridCompressedCache, layer_idx: int,
                     scaling: Optional[float] = None) -> torch.Tensor:
    """q [B, Hq, 1, D] -> [B, Hq, 1, D] over the layer's compressed cache; restates
    LlamaAttention._forward_fused_hybrid_decode (modeling_llama.py:453-518)."""
    B, Hq, _, D = q.shape
    q2 = q.squeeze(2).contiguous()
    kp, vp = cache.k_packed[layer_idx], cache.v_packed[layer_idx]
    kx, vx = cache.k_exact[layer_idx], cache.v_exact[layer_idx]
    cnt = cache.packed_counts[layer_idx]
    lens = cache.packed_lengths[layer_idx]
    exact_len = min(cache.exact_seq_lens[layer_idx], cache.exact_window_size)
    out = torch.empty_like(q2)
    scale = D ** -0.5 if scaling is None else scaling
    _decode_attention_launch(q2, q2.stride(0), q2.stride(1), kp, vp,
                             (kp.stride(0), kp.stride(1), kp.stride(2)), cnt,
                             (cnt.stride(0), cnt.stride(1)), lens, kx, vx,
                             (kx.stride(0), kx.stride(1), kx.stride(2)), cache.exact_window_size,
                             exact_len, scale, out, out.stride(0), out.stride(1), B, Hq,
                             cache.n_kv_heads, D, "decode_attention")
    return out.unsqueeze(2)
