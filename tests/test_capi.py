"""The C ABI (include/deltaattn.h): the library loads, exports every declared symbol, and
rejects bad arguments before touching the GPU."""
import ctypes
import os
import re

import pytest

from deltaattention_amd import _native

HERE = os.path.dirname(os.path.abspath(__file__))
HEADER = os.path.join(os.path.dirname(HERE), "include", "deltaattn.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(da_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    assert declared_symbols() == sorted([
        "da_last_error", "da_version", "da_select", "da_pack_workspace_size", "da_pack",
        "da_hybrid_workspace_size", "da_hybrid_prefill", "da_dense_prefill",
        "da_decode_update", "da_decode_workspace_size", "da_decode_attention",
        "da_decode_attention_noalloc", "da_select_varlen", "da_pack_varlen_workspace_size",
        "da_pack_varlen", "da_hybrid_varlen_workspace_size", "da_hybrid_prefill_varlen",
        "da_dense_prefill_varlen", "da_decode_step"])


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name
        assert name in _native.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.da_version() == 1


def _err():
    return _native.lib().da_last_error().decode()


def test_select_rejects_null_and_dtype():
    lib = _native.lib()
    f = ctypes.c_float(1.0)
    assert lib.da_select(None, 1, 1, 1, 8, 128, 0, 0, 0, f, 0, 8, 1, None, None, None) == -1
    assert "null" in _err()
    fake = ctypes.c_void_p(1 << 20)
    # keys are bf16, fp16 or fp32: int32 (DA_I32 = 3) is refused
    assert lib.da_select(fake, 3, 1, 1, 8, 128, 0, 0, 128, f, 0, 8, 1, fake, fake, None) == -2
    assert "bf16, fp16 or fp32" in _err()
    # fp32 rows are read 8 bytes per lane: odd strides are refused
    assert lib.da_select(fake, 4, 1, 1, 8, 128, 0, 0, 129, f, 0, 8, 1, fake, fake, None) == -1
    assert lib.da_select(fake, 1, 1, 1, 8, 130, 0, 0, 130, f, 0, 8, 1, fake, fake, None) == -2
    assert "head_dim" in _err()
    assert lib.da_select(fake, 1, 1, 1, 8, 128, 0, 0, 129, f, 0, 8, 1, fake, fake, None) == -1
    assert lib.da_select(fake, 1, 1, 1, 8, 128, 0, 0, 128, f, 0, 0, 1, fake, fake, None) == -1
    # flags: DA_SELECT_COSINE | DA_SELECT_ARITH16 only
    assert lib.da_select(fake, 1, 1, 1, 8, 128, 0, 0, 128, f, 4, 8, 1, fake, fake, None) == -1
    assert "flags" in _err()


def test_pack_rejects_small_workspace():
    lib = _native.lib()
    fake = ctypes.c_void_p(1 << 20)
    need = lib.da_pack_workspace_size(1, 8, 32768)
    assert need == 2 * 8 * 512 * 4
    rc = lib.da_pack(fake, fake, fake, 1, 1, 8, 32768, 128, 0, 0, 128, 0, 0, 128, 32768, fake, fake,
                     fake, fake, fake, fake, fake, need - 4, None)
    assert rc == -4 and "workspace" in _err()


def test_attention_rejects_bad_shapes():
    lib = _native.lib()
    fake = ctypes.c_void_p(1 << 20)
    st = _native.strides_array([0] * 24)
    f = ctypes.c_float(0.088)
    # head_dim must be a multiple of 8 in [8, 128]
    for D in (60, 136, 0):
        assert lib.da_dense_prefill(fake, fake, fake, fake, 1, 1, 4, 2, 64, 64, D, st, 1, f, None) == -2
        assert "head_dim" in _err()
    # Hq not a multiple of Hkv
    assert lib.da_dense_prefill(fake, fake, fake, fake, 1, 1, 6, 4, 64, 64, 128, st, 1, f, None) == -1
    # negative scale
    assert lib.da_dense_prefill(fake, fake, fake, fake, 1, 1, 4, 2, 64, 64, 128, st, 1,
                                ctypes.c_float(-1.0), None) == -1
    # negative window / unknown variant / missing workspace
    args = [fake] * 7
    assert lib.da_hybrid_prefill(*args, 3, fake, 1, 1, 4, 2, 64, 64, 128, st, 10, None, -1,
                                 f, 0, 0, fake, 1 << 20, None) == -1
    assert lib.da_hybrid_prefill(*args, 3, fake, 1, 1, 4, 2, 64, 64, 128, st, 10, None, 0,
                                 f, 7, 0, fake, 1 << 20, None) == -1
    # (batch, head, sequence) strides of q, k, v, k_packed, v_packed, out, timestamps, counts
    rows = [8192, 8192, 128]
    st2 = _native.strides_array(rows * 6 + [0, 0, 1, 0, 0, 1])
    assert lib.da_hybrid_prefill(*args, 3, fake, 1, 1, 4, 2, 64, 64, 128, st2, 10, None, 0,
                                 f, 0, 0, None, 0, None) == -4
    # key/value rows that overlap (sequence stride below head_dim) are refused
    st3 = _native.strides_array(rows * 3 + [8192, 8192, 64] + rows * 2 + [0, 0, 1, 0, 0, 1])
    assert lib.da_hybrid_prefill(*args, 3, fake, 1, 1, 4, 2, 64, 64, 128, st3, 10, None, 0,
                                 f, 0, 0, fake, 1 << 20, None) == -1
    assert b"sequence strides" in lib.da_last_error()
    # sequence strides from 2^23 elements on are refused (the kernel's per-row byte offset
    # is a 24-bit product); 2^23 - 8 is accepted and reaches the workspace check
    big = [0, 0, 1 << 23]
    st4 = _native.strides_array(rows + big + rows * 4 + [0, 0, 1, 0, 0, 1])
    assert lib.da_hybrid_prefill(*args, 3, fake, 1, 1, 4, 2, 64, 64, 128, st4, 10, None, 0,
                                 f, 0, 0, fake, 1 << 20, None) == -1
    assert b"sequence strides" in lib.da_last_error()
    st5 = _native.strides_array(rows + [0, 0, (1 << 23) - 8] + rows * 4 + [0, 0, 1, 0, 0, 1])
    assert lib.da_hybrid_prefill(*args, 3, fake, 1, 1, 4, 2, 64, 64, 128, st5, 10, None, 0,
                                 f, 0, 0, None, 0, None) == -4


def test_decode_rejects_misaligned_values():
    """Value rows are read 4 bytes per lane: misaligned v_packed / v_exact are refused."""
    lib = _native.lib()
    a = ctypes.c_void_p(1 << 20)
    odd = ctypes.c_void_p((1 << 20) + 2)
    f = ctypes.c_float(0.088)
    D, cap, W = 128, 64, 16
    st_p, st_x = (8 * cap * D, cap * D, D), (8 * W * D, W * D, D)
    for vp, vx in ((odd, a), (a, odd)):
        for fn, tail in ((lib.da_decode_attention, [a, 1 << 30, None]),
                         (lib.da_decode_attention_noalloc, [None])):
            rc = fn(a, 1, 1, 32, 8, D, 32 * D, D, a, vp, *st_p, a, 8 * cap, cap, a, cap, a, vx,
                    *st_x, W, 0, f, a, 32 * D, D, *tail)
            assert rc == -1 and "value rows" in _err()


def test_decode_shape_limits():
    """Decode attention takes bf16, fp16 or fp32 caches, head dims that are multiples of 8 up
    to 128 and GQA groups up to 64; other shapes are refused as unsupported before any launch (the accepted ones
    reach the workspace check)."""
    lib = _native.lib()
    a = ctypes.c_void_p(1 << 20)
    f = ctypes.c_float(0.1)
    cap, W = 64, 16

    def call(Hq, Hkv, D, ws=None, ws_bytes=0, dtype=1):
        st_p, st_x = (Hkv * cap * D, cap * D, D), (Hkv * W * D, W * D, D)
        return lib.da_decode_attention(a, dtype, 1, Hq, Hkv, D, Hq * D, D, a, a, *st_p, a, Hkv * cap, cap, a,
                                       cap, a, a, *st_x, W, 0, f, a, Hq * D, D, ws, ws_bytes, None)

    # the decode cache is bf16, fp16 or fp32: int32 (DA_I32 = 3) is refused as unsupported,
    # fp32 (DA_F32 = 4) reaches the workspace check
    assert call(8, 8, 64, dtype=3) == -2 and "bf16, fp16 or fp32" in _err()
    assert call(8, 8, 64, dtype=4) == -4 and "workspace" in _err()

    for D in (4, 100, 136):
        assert call(8, 8, D) == -2 and "head_dim" in _err(), D
    assert call(65, 1, 64) == -2 and "GQA group" in _err()
    for Hq, Hkv, D in ((8, 8, 64), (8, 2, 96), (16, 1, 128), (64, 1, 8), (9, 1, 96)):
        assert call(Hq, Hkv, D) == -4 and "workspace" in _err(), (Hq, Hkv, D)


def test_varlen_entry_points_reject_bad_arguments():
    lib = _native.lib()
    fake = ctypes.c_void_p(1 << 20)
    f = ctypes.c_float(1.0)
    # null cu_seqlens, max_seqlen beyond the token count, max_chunks too small
    assert lib.da_select_varlen(fake, 1, 2, 8, 1000, 128, 1024, 128, None, 600, f, 0, 512, 0,
                                fake, fake, 2, None) == -1
    assert lib.da_select_varlen(fake, 1, 2, 8, 1000, 128, 1024, 128, fake, 1001, f, 0, 512, 0,
                                fake, fake, 2, None) == -1
    assert lib.da_select_varlen(fake, 1, 2, 8, 1000, 128, 1024, 128, fake, 600, f, 0, 512, 0,
                                fake, fake, 1, None) == -1
    assert "max_chunks" in _err()
    need = lib.da_pack_varlen_workspace_size(2, 8, 600)
    assert need == 2 * 2 * 8 * 10 * 4
    assert lib.da_pack_varlen(fake, fake, fake, 1, 2, 8, 1000, 128, 1024, 128, 1024, 128, fake, 600,
                              fake, fake, fake, fake, fake, fake, fake, need - 4, None) == -4
    st = _native.strides_array([0, 128, 4096] + [0, 128, 1024] * 2 + [0, 128, 1024] * 2 +
                               [0, 128, 4096] + [0, 1000, 1] * 2)
    assert lib.da_hybrid_varlen_workspace_size(2, 8, 600) == lib.da_hybrid_workspace_size(2, 8, 600)
    assert lib.da_hybrid_prefill_varlen(fake, fake, fake, fake, fake, fake, fake, 3, fake, 1, 2, 32, 8,
                                        1000, 128, st, None, 600, fake, 128, f, 0, 0, fake, 1 << 30,
                                        None) == -1
    assert lib.da_dense_prefill_varlen(fake, fake, fake, fake, 1, 2, 32, 8, 1000, 128, st, fake, 0, 1,
                                       f, None) == -1


def test_workspace_sizes():
    lib = _native.lib()

    def r256(x):
        return (x + 255) // 256 * 256

    def hybrid_ws(B, H, P):
        nblk = max(1, (P + 127) // 128)
        wcap = 128 * nblk
        # schedule, fp32 weights, timestamps, 64 zeros, 8 work-queue counters (each region
        # 256-byte aligned)
        return r256(B * H * 2 * nblk * 4) + 2 * r256(B * H * wcap * 4) + 256 + 256

    assert lib.da_hybrid_workspace_size(1, 8, 8192) == hybrid_ws(1, 8, 8192)
    assert lib.da_hybrid_workspace_size(2, 8, 1) == hybrid_ws(2, 8, 1)
    assert lib.da_hybrid_workspace_size(1, 8, 8192) == 4096 + 2 * 8 * 8192 * 4 + 512


def test_ops_refuse_cpu_tensors():
    torch = pytest.importorskip("torch")
    from deltaattention_amd import ops
    k = torch.zeros(1, 1, 16, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="no CPU path"):
        ops.select(k, 1.0)
    with pytest.raises(ValueError, match="no CPU path"):
        ops.dense_prefill(k, k, k)


def test_decode_step_block_matches_header_and_checks_workspace():
    """The ctypes DecodeStep mirrors DaDecodeStep field for field, and the entry point
    reads the block at those offsets: a valid block with no workspace is refused with
    DA_ERR_WORKSPACE before anything is launched."""
    text = open(HEADER).read()
    body = re.search(r"typedef struct DaDecodeStep \{(.*?)\} DaDecodeStep;", text, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    names = re.findall(r"\**\s*(\w+)\s*[,;]", body)
    assert names == [f for f, _ in _native.DecodeStep._fields_]
    lib = _native.lib()
    assert lib.da_decode_step(None, None) == -1 and "null" in _err()
    a = 1 << 20
    D, cap, W, Hq, Hkv = 128, 64, 16, 32, 8
    st = _native.DecodeStep(
        new_k=a, new_v=a, sn_b=Hkv * D, sn_h=D, q=a, sq_b=Hq * D, sq_h=D, out=a, so_b=Hq * D,
        so_h=D, k_exact=a, v_exact=a, sx_b=Hkv * W * D, sx_h=W * D, sx_s=D, k_packed=a,
        v_packed=a, sp_b=Hkv * cap * D, sp_h=cap * D, sp_s=D,
        counts=a, timestamps=a, sc_b=Hkv * cap, sc_h=cap, lengths=a, capacity=cap, exact_seq_len=3,
        total_seq_len=3, window=W, threshold=1.0, use_cosine=0, scale=0.088, dtype=_native.DA_BF16, B=1,
        Hq=Hq, Hkv=Hkv, D=D, workspace=None, workspace_bytes=0)
    assert lib.da_decode_step(ctypes.byref(st), None) == -4 and "workspace" in _err()
    st.Hq = 30    # not a multiple of Hkv: the attention checks run first
    assert lib.da_decode_step(ctypes.byref(st), None) == -1
