"""Native DeltaAttention prefill operations on torch tensors (ROCm, gfx950).

Every operation calls libdeltaattn.so through its C ABI on the current HIP stream;
tensors only provide device memory and streams.  There is no CPU fallback.

Layouts follow the reference: K, V are [B, Hkv, N, D] (post-RoPE keys), Q and the
output are [B, Hq, N, D]; query head h uses KV head h // (Hq // Hkv), which is what
``repeat_kv`` materialises in the reference (modeling_llama.py:223-232) -- here it is
never materialised.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _native
from ._native import DA_F32, DA_I32, DA_VARIANT, check, dtype_code, lib, strides_array

__all__ = ["PackedKV", "chunking", "select", "pack", "hybrid_prefill", "dense_prefill",
           "delta_prefill", "VarlenBatch", "varlen_batch", "PackedVarlen", "select_varlen",
           "pack_varlen", "hybrid_prefill_varlen", "delta_prefill_varlen", "dense_prefill_varlen"]


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require_device(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise ValueError("deltaattention_amd operations take GPU tensors "
                             f"(got a tensor on {t.device}); there is no CPU path")


def _data_dtype(*ts: torch.Tensor) -> int:
    """The library's code of the one data dtype (bf16, fp16 or fp32) the tensors share."""
    return dtype_code(*ts)


def _last_dim_contig(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def chunking(seq_len: int, chunk_size: int = 0, divide_to: int = 0) -> Tuple[int, int]:
    """(chunk size, chunk count) as modeling_llama.py:602-610 computes them."""
    if seq_len <= 0:
        raise ValueError("seq_len must be positive")
    if chunk_size > 0:
        cs = min(chunk_size, seq_len)
        return cs, max(1, (seq_len + cs - 1) // cs)
    parts = 1 if divide_to == 0 else divide_to
    return (seq_len + parts - 1) // parts, parts


SELECT_ARITH = ("fp32", "native")


def _select_flags(metric: str, arith: str) -> int:
    if arith not in SELECT_ARITH:
        raise ValueError(f"arith must be one of {SELECT_ARITH}, got {arith!r}")
    if metric == "cosine":
        return _native.DA_SELECT_COSINE
    return _native.DA_SELECT_ARITH16 if arith == "native" else 0


def select(k: torch.Tensor, threshold: float, chunk_size: int = 512, divide_to: int = 0,
           metric: str = "euclidean", keep: Optional[torch.Tensor] = None,
           chunk_counts: Optional[torch.Tensor] = None,
           arith: str = "native") -> Tuple[torch.Tensor, torch.Tensor]:
    """Delta-mode anchor selection (tritonModules.py:7-69 via modeling_llama.py:634-653).

    ``metric == "cosine"`` selects the cosine test (keep iff cos < threshold); every
    other string is Euclidean (keep iff ||k - anchor||^2 > threshold^2), exactly as
    modeling_llama.py:639-642.  The default ``arith="native"`` evaluates the Euclidean
    distance in the keys' own 16-bit arithmetic (every difference, square and tree
    addition rounded, as the reference's Triton code does on bf16 / fp16 keys,
    tritonModules.py:55-58); "fp32" keeps them in fp32.  Both reduce over the same fixed
    tree.
    Returns keep [B, Hkv, N] int32 and chunk counts [B, Hkv, num_chunks] int32.
    """
    _require_device(k)
    dt = _data_dtype(k)
    k = _last_dim_contig(k)
    B, H, N, D = k.shape
    cs, nc = chunking(N, chunk_size, divide_to)
    use_cos = metric == "cosine"
    thr = float(threshold) if use_cos else float(threshold) ** 2
    if keep is None:  # the chunks tile [0, N): the kernel writes every flag
        keep = torch.empty((B, H, N), dtype=torch.int32, device=k.device)
    if chunk_counts is None:
        chunk_counts = torch.empty((B, H, nc), dtype=torch.int32, device=k.device)
    rc = lib().da_select(k.data_ptr(), dt, B, H, N, D, k.stride(0), k.stride(1), k.stride(2),
                         ctypes.c_float(thr), _select_flags(metric, arith), cs, nc, keep.data_ptr(),
                         chunk_counts.data_ptr(), _stream())
    check(rc, "da_select")
    return keep, chunk_counts


@dataclass
class PackedKV:
    """Packed anchors of every (batch, kv head).

    k_packed/v_packed [B, Hkv, capacity, D], timestamps/counts [B, Hkv, capacity] int32;
    rows [0, c) hold the anchors of a head, rows [c, P) are zero padding, rows at or
    beyond P are not defined.  anchor_counts [B, Hkv] int32 holds c, num_packed [1]
    int32 holds P = max c on the device (no host synchronisation).
    """
    k_packed: torch.Tensor
    v_packed: torch.Tensor
    timestamps: torch.Tensor
    counts: torch.Tensor
    anchor_counts: torch.Tensor
    num_packed: torch.Tensor

    @property
    def capacity(self) -> int:
        return self.k_packed.shape[2]

    def trimmed(self) -> "PackedKV":
        """Views cut to P rows (reads P back to the host, as modeling_llama.py:656)."""
        P = int(self.num_packed.item())
        return PackedKV(self.k_packed[:, :, :P], self.v_packed[:, :, :P],
                        self.timestamps[:, :, :P], self.counts[:, :, :P],
                        self.anchor_counts, self.num_packed)


def pack(keep: torch.Tensor, k: torch.Tensor, v: torch.Tensor, capacity: Optional[int] = None,
         out: Optional[PackedKV] = None) -> PackedKV:
    """Index + pack + counts (modeling_llama.py:655-685, tritonModules.py:72-132).

    ``capacity`` (rows per head of the outputs) defaults to N, which always holds every
    anchor, so nothing waits for P on the host.
    """
    _require_device(keep, k, v)
    dt = _data_dtype(k, v)
    k, v = _last_dim_contig(k), _last_dim_contig(v)
    keep = keep.contiguous()
    if keep.dtype != torch.int32:
        keep = keep.to(torch.int32)
    B, H, N, D = k.shape
    if capacity is None:
        capacity = N if out is None else out.capacity
    dev = k.device
    if out is None:
        out = PackedKV(
            torch.empty((B, H, capacity, D), dtype=k.dtype, device=dev),
            torch.empty((B, H, capacity, D), dtype=v.dtype, device=dev),
            torch.empty((B, H, capacity), dtype=torch.int32, device=dev),
            torch.empty((B, H, capacity), dtype=torch.int32, device=dev),
            torch.empty((B, H), dtype=torch.int32, device=dev),
            torch.empty((1,), dtype=torch.int32, device=dev))
    for t in (out.k_packed, out.v_packed, out.timestamps, out.counts):
        if not t.is_contiguous():
            raise ValueError("packed outputs must be contiguous")
    ws_bytes = lib().da_pack_workspace_size(B, H, N)
    ws = torch.empty((max(1, ws_bytes),), dtype=torch.uint8, device=dev)
    rc = lib().da_pack(keep.data_ptr(), k.data_ptr(), v.data_ptr(), dt, B, H, N, D,
                       k.stride(0), k.stride(1), k.stride(2), v.stride(0), v.stride(1),
                       v.stride(2), out.capacity, out.k_packed.data_ptr(), out.v_packed.data_ptr(),
                       out.timestamps.data_ptr(), out.counts.data_ptr(),
                       out.anchor_counts.data_ptr(), out.num_packed.data_ptr(), ws.data_ptr(),
                       ws_bytes, _stream())
    check(rc, "da_pack")
    return out


def _attn_strides(q, k, v, out, kp=None, vp=None, ts=None, cnt=None):
    vals = [0] * 24
    for base, t in ((0, q), (3, k), (6, v), (9, kp), (12, vp), (15, out)):
        if t is not None:
            vals[base:base + 3] = [t.stride(0), t.stride(1), t.stride(2)]
    for base, t in ((18, ts), (21, cnt)):
        if t is not None:
            vals[base:base + 3] = [t.stride(0), t.stride(1), t.stride(2)]
    return strides_array(vals)


def hybrid_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_packed: torch.Tensor,
                   v_packed: torch.Tensor, timestamps: torch.Tensor, counts: torch.Tensor,
                   window: int = 128, scale: Optional[float] = None, variant: str = "hybrid",
                   no_count: bool = False, num_packed_dev: Optional[torch.Tensor] = None,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Two-phase compressed prefill (deltaFlashAttention.py:9-357) with GQA indexing.

    k_packed etc. hold P = k_packed.shape[2] rows per head (or, when ``num_packed_dev``
    is given, that many of them); counts may be int32 or float32.
    """
    if variant not in DA_VARIANT:
        raise ValueError(f"variant must be one of {sorted(DA_VARIANT)}")
    _require_device(q, k, v, k_packed, v_packed, timestamps, counts)
    dt = _data_dtype(q, k, v, k_packed, v_packed)
    q, k, v = _last_dim_contig(q), _last_dim_contig(k), _last_dim_contig(v)
    k_packed, v_packed = _last_dim_contig(k_packed), _last_dim_contig(v_packed)
    timestamps = _last_dim_contig(timestamps)
    counts = _last_dim_contig(counts)
    if timestamps.dtype != torch.int32:
        timestamps = timestamps.to(torch.int32)
    if counts.dtype not in (torch.int32, torch.float32):
        counts = counts.to(torch.float32)
    B, Hq, Nq, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    P = k_packed.shape[2]
    if scale is None:
        scale = D ** -0.5
    if out is None:
        out = torch.empty_like(q)
    dtype_code(q, out)
    ws_bytes = lib().da_hybrid_workspace_size(B, Hkv, max(P, 1))
    ws = torch.empty((max(1, ws_bytes),), dtype=torch.uint8, device=q.device)
    st = _attn_strides(q, k, v, out, k_packed, v_packed, timestamps, counts)
    rc = lib().da_hybrid_prefill(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), k_packed.data_ptr(), v_packed.data_ptr(),
        timestamps.data_ptr(), counts.data_ptr(),
        DA_F32 if counts.dtype == torch.float32 else DA_I32, out.data_ptr(), dt,
        B, Hq, Hkv, Nq, Nk, D, st, P, _ptr(num_packed_dev), int(window), ctypes.c_float(scale),
        DA_VARIANT[variant], 1 if no_count else 0, ws.data_ptr(), ws_bytes, _stream())
    check(rc, "da_hybrid_prefill")
    return out


def dense_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = True,
                  scale: Optional[float] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Dense flash prefill (flashAttention.py:5-130) with GQA indexing."""
    _require_device(q, k, v)
    dt = _data_dtype(q, k, v)
    q, k, v = _last_dim_contig(q), _last_dim_contig(k), _last_dim_contig(v)
    B, Hq, Nq, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    if scale is None:
        scale = D ** -0.5
    if out is None:
        out = torch.empty_like(q)
    dtype_code(q, out)
    st = _attn_strides(q, k, v, out)
    rc = lib().da_dense_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), dt,
                                B, Hq, Hkv, Nq, Nk, D, st, 1 if causal else 0,
                                ctypes.c_float(scale), _stream())
    check(rc, "da_dense_prefill")
    return out


def delta_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, threshold: float,
                  chunk_size: int = 512, divide_to: int = 0, metric: str = "euclidean",
                  window: int = 128, scale: Optional[float] = None, variant: str = "hybrid",
                  no_count: bool = False, keep: Optional[torch.Tensor] = None,
                  return_packed: bool = False, out: Optional[torch.Tensor] = None,
                  arith: str = "native"):
    """select -> pack -> hybrid prefill with P kept on the device (no host sync).

    Restates PATH 1 of LlamaAttention.forward (modeling_llama.py:600-749) for the delta
    packing mode; pass ``keep`` to use a mask from another packing mode.
    """
    if keep is None:
        keep, _ = select(k, threshold, chunk_size, divide_to, metric, arith=arith)
    packed = pack(keep, k, v)
    out = hybrid_prefill(q, k, v, packed.k_packed, packed.v_packed, packed.timestamps,
                         packed.counts, window=window, scale=scale, variant=variant,
                         no_count=no_count, num_packed_dev=packed.num_packed, out=out)
    return (out, packed) if return_packed else out


def _seq_bounds(cu_seqlens, total: int):
    """Host list of (start, end) per sequence from cu_seqlens [B + 1]."""
    if isinstance(cu_seqlens, torch.Tensor):
        cu = cu_seqlens.detach().to("cpu", torch.int64).tolist()
    else:
        cu = [int(x) for x in cu_seqlens]
    if len(cu) < 2 or cu[0] != 0 or cu[-1] != total or any(b < a for a, b in zip(cu, cu[1:])):
        raise ValueError(f"cu_seqlens must rise from 0 to the token count {total}, got {cu}")
    return list(zip(cu[:-1], cu[1:]))


@dataclass
class VarlenBatch:
    """A ragged batch: cu_seqlens on the device (int32 [B + 1]), B and the longest length."""
    cu: torch.Tensor
    batch: int
    max_seqlen: int


def varlen_batch(cu_seqlens, total: int, device, max_seqlen: Optional[int] = None) -> VarlenBatch:
    """cu_seqlens (host list / tensor, or a device int32 tensor) -> VarlenBatch.  Host values
    are validated (rising from 0 to ``total``); for a device tensor without ``max_seqlen``
    the lengths are read back once (one synchronisation)."""
    if isinstance(cu_seqlens, VarlenBatch):
        return cu_seqlens
    if isinstance(cu_seqlens, torch.Tensor) and cu_seqlens.device.type == "cuda":
        cu = cu_seqlens if cu_seqlens.dtype == torch.int32 else cu_seqlens.to(torch.int32)
        cu = cu.contiguous()
        if max_seqlen is None:
            bounds = _seq_bounds(cu, total)
            max_seqlen = max(e - s for s, e in bounds)
        return VarlenBatch(cu, cu.numel() - 1, int(max_seqlen))
    bounds = _seq_bounds(cu_seqlens, total)
    host = [0] + [e for _, e in bounds]
    return VarlenBatch(torch.tensor(host, dtype=torch.int32, device=device), len(bounds),
                       max(1, max(e - s for s, e in bounds)))


def _check_varlen(q, k, v):
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("varlen tensors are [tokens, heads, head_dim]")
    if q.shape[0] != k.shape[0] or k.shape != v.shape:
        raise ValueError("q, k and v must hold the same tokens; k and v the same heads")


def select_varlen(k: torch.Tensor, cu_seqlens, threshold: float, chunk_size: int = 512,
                  divide_to: int = 0, metric: str = "euclidean", arith: str = "native",
                  max_seqlen: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Delta-mode selection of every sequence of a ragged batch in one launch: k [T, Hkv, D]
    -> keep [Hkv, T] int32, chunk counts [B, Hkv, max_chunks] int32.  Each sequence is
    chunked by the reference's rule on its own length (modeling_llama.py:602-610)."""
    _require_device(k)
    dt = _data_dtype(k)
    k = _last_dim_contig(k)
    T, H, D = k.shape
    vb = varlen_batch(cu_seqlens, T, k.device, max_seqlen)
    nc = max(1, -(-vb.max_seqlen // chunk_size)) if chunk_size > 0 else max(1, divide_to)
    use_cos = metric == "cosine"
    thr = float(threshold) if use_cos else float(threshold) ** 2
    keep = torch.zeros((H, T), dtype=torch.int32, device=k.device)
    counts = torch.empty((vb.batch, H, nc), dtype=torch.int32, device=k.device)
    rc = lib().da_select_varlen(k.data_ptr(), dt, vb.batch, H, T, D, k.stride(0), k.stride(1),
                                vb.cu.data_ptr(), vb.max_seqlen, ctypes.c_float(thr),
                                _select_flags(metric, arith), chunk_size, divide_to,
                                keep.data_ptr(), counts.data_ptr(), nc, _stream())
    check(rc, "da_select_varlen")
    return keep, counts


@dataclass
class PackedVarlen:
    """Packed anchors of a ragged batch: k_packed / v_packed [T, Hkv, D] (row j of sequence b
    at token cu[b] + j), timestamps / counts [Hkv, T] likewise, anchor_counts [B, Hkv] and
    num_packed [B] (P_b) on the device; rows [c_bg, P_b) are zero, rows beyond undefined."""
    k_packed: torch.Tensor
    v_packed: torch.Tensor
    timestamps: torch.Tensor
    counts: torch.Tensor
    anchor_counts: torch.Tensor
    num_packed: torch.Tensor


def pack_varlen(keep: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens,
                max_seqlen: Optional[int] = None) -> PackedVarlen:
    """Index + pack + counts of every sequence of a ragged batch in one pass
    (modeling_llama.py:655-685 per sequence)."""
    _require_device(keep, k, v)
    dt = _data_dtype(k, v)
    k, v = _last_dim_contig(k), _last_dim_contig(v)
    T, H, D = k.shape
    vb = varlen_batch(cu_seqlens, T, k.device, max_seqlen)
    keep = keep.contiguous()
    if keep.shape != (H, T) or keep.dtype != torch.int32:
        raise ValueError("keep must be an int32 [Hkv, T] tensor (as select_varlen returns it)")
    dev = k.device
    out = PackedVarlen(torch.empty((T, H, D), dtype=k.dtype, device=dev),
                       torch.empty((T, H, D), dtype=v.dtype, device=dev),
                       torch.empty((H, T), dtype=torch.int32, device=dev),
                       torch.empty((H, T), dtype=torch.int32, device=dev),
                       torch.empty((vb.batch, H), dtype=torch.int32, device=dev),
                       torch.empty((vb.batch,), dtype=torch.int32, device=dev))
    ws_bytes = lib().da_pack_varlen_workspace_size(vb.batch, H, vb.max_seqlen)
    ws = torch.empty((max(1, ws_bytes),), dtype=torch.uint8, device=dev)
    rc = lib().da_pack_varlen(keep.data_ptr(), k.data_ptr(), v.data_ptr(), dt, vb.batch, H, T, D,
                              k.stride(0), k.stride(1), v.stride(0), v.stride(1), vb.cu.data_ptr(),
                              vb.max_seqlen, out.k_packed.data_ptr(), out.v_packed.data_ptr(),
                              out.timestamps.data_ptr(), out.counts.data_ptr(),
                              out.anchor_counts.data_ptr(), out.num_packed.data_ptr(), ws.data_ptr(),
                              ws_bytes, _stream())
    check(rc, "da_pack_varlen")
    return out


def _varlen_strides(q, k, v, out, kp=None, vp=None, ts=None, cnt=None):
    """The 24-entry stride array with (0, head, token) per token-major tensor and
    (0, head, 1) for the head-major timestamps / counts."""
    vals = [0] * 24
    for base, t in ((0, q), (3, k), (6, v), (9, kp), (12, vp), (15, out)):
        if t is not None:
            vals[base:base + 3] = [0, t.stride(1), t.stride(0)]
    for base, t in ((18, ts), (21, cnt)):
        if t is not None:
            vals[base:base + 3] = [0, t.stride(0), t.stride(1)]
    return strides_array(vals)


def hybrid_prefill_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, packed: PackedVarlen,
                          cu_seqlens, window: int = 128, scale: Optional[float] = None,
                          variant: str = "hybrid", no_count: bool = False,
                          max_seqlen: Optional[int] = None,
                          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Two-phase compressed prefill of a ragged batch in one launch: every sequence gets
    the schedule and result of a B = 1 hybrid prefill of its own length."""
    if variant not in DA_VARIANT:
        raise ValueError(f"variant must be one of {sorted(DA_VARIANT)}")
    _check_varlen(q, k, v)
    _require_device(q, k, v, packed.k_packed)
    dt = _data_dtype(q, k, v, packed.k_packed, packed.v_packed)
    q, k, v = _last_dim_contig(q), _last_dim_contig(k), _last_dim_contig(v)
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    vb = varlen_batch(cu_seqlens, T, q.device, max_seqlen)
    if scale is None:
        scale = D ** -0.5
    if out is None:
        out = torch.empty_like(q)
    dtype_code(q, out)
    ws_bytes = lib().da_hybrid_varlen_workspace_size(vb.batch, Hkv, vb.max_seqlen)
    ws = torch.empty((max(1, ws_bytes),), dtype=torch.uint8, device=q.device)
    st = _varlen_strides(q, k, v, out, packed.k_packed, packed.v_packed, packed.timestamps,
                         packed.counts)
    rc = lib().da_hybrid_prefill_varlen(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), packed.k_packed.data_ptr(),
        packed.v_packed.data_ptr(), packed.timestamps.data_ptr(), packed.counts.data_ptr(),
        DA_F32 if packed.counts.dtype == torch.float32 else DA_I32, out.data_ptr(), dt,
        vb.batch, Hq, Hkv, T, D, st, vb.cu.data_ptr(), vb.max_seqlen,
        packed.num_packed.data_ptr(), int(window), ctypes.c_float(scale), DA_VARIANT[variant],
        1 if no_count else 0, ws.data_ptr(), ws_bytes, _stream())
    check(rc, "da_hybrid_prefill_varlen")
    return out


def delta_prefill_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens,
                         threshold: float, chunk_size: int = 512, divide_to: int = 0,
                         metric: str = "euclidean", window: int = 128,
                         scale: Optional[float] = None, variant: str = "hybrid",
                         no_count: bool = False, arith: str = "native",
                         max_seqlen: Optional[int] = None, return_packed: bool = False):
    """Delta prefill of a packed ragged batch: q [T, Hq, D], k, v [T, Hkv, D] with the
    sequences at cu_seqlens -> out [T, Hq, D].

    The reference has no varlen API; each sequence is exactly a B = 1 delta prefill with
    its own chunking, anchors, P and schedule.  Three launches cover the whole batch
    (select, pack, hybrid prefill; plus the schedule pre-pass), with every per-sequence
    quantity on the device."""
    _check_varlen(q, k, v)
    vb = varlen_batch(cu_seqlens, q.shape[0], q.device, max_seqlen)
    keep, _ = select_varlen(k, vb, threshold, chunk_size, divide_to, metric, arith)
    packed = pack_varlen(keep, k, v, vb)
    out = hybrid_prefill_varlen(q, k, v, packed, vb, window, scale, variant, no_count)
    return (out, packed) if return_packed else out


def dense_prefill_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens,
                         causal: bool = True, scale: Optional[float] = None,
                         max_seqlen: Optional[int] = None,
                         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Dense flash prefill of a packed ragged batch in one launch (the control of
    delta_prefill_varlen)."""
    _check_varlen(q, k, v)
    _require_device(q, k, v)
    dt = _data_dtype(q, k, v)
    q, k, v = _last_dim_contig(q), _last_dim_contig(k), _last_dim_contig(v)
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    vb = varlen_batch(cu_seqlens, T, q.device, max_seqlen)
    if scale is None:
        scale = D ** -0.5
    if out is None:
        out = torch.empty_like(q)
    dtype_code(q, out)
    st = _varlen_strides(q, k, v, out)
    rc = lib().da_dense_prefill_varlen(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), dt,
                                       vb.batch, Hq, Hkv, T, D, st, vb.cu.data_ptr(), vb.max_seqlen,
                                       1 if causal else 0, ctypes.c_float(scale), _stream())
    check(rc, "da_dense_prefill_varlen")
    return out
