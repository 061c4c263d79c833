"""C-ABI library (CPU): it loads, exports every declared symbol, and rejects
out-of-contract arguments on the host before any launch."""

import ctypes
import os
import re

import pytest
import torch

from unum_ops_amd import _lib
from unum_ops_amd.infllm_v2 import infllmv2_attn_stage1, max_pooling_1d_varlen
from unum_ops_amd.sparse_kernel_extension import get_block_table

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "unum_ops_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(unum_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_bound_symbols():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.unum_abi_version() == _lib.ABI_VERSION
    assert lib.unum_last_error() == b""


def _null():
    return ctypes.c_void_p(0)


def test_block_table_rejects_bad_sizes():
    lib = _lib.load()
    n = _null()
    st = lib.unum_get_block_table(n, 1, 1, 1, n, 1, n, n, 1, n, 1, n, -1, 1, 1, 1, 1, 2, n)
    assert st == _lib.UNUM_ERR_INVALID_ARGUMENT
    assert b"negative size" in lib.unum_last_error()
    # empty problem: nothing to launch, success
    assert lib.unum_get_block_table(n, 1, 1, 1, n, 1, n, n, 1, n, 1, n, 2, 0, 4, 1, 1, 2, n) == 0
    # token_pos_in_bs of the wrong length
    st = lib.unum_get_block_table(n, 1, 1, 1, n, 1, n, n, 3, n, 1, n, 2, 4, 4, 1, 8, 2, n)
    assert st == _lib.UNUM_ERR_INVALID_ARGUMENT and b"token_pos_in_bs" in lib.unum_last_error()


def test_maxpool_rejects_bad_arguments():
    lib = _lib.load()
    n = _null()
    st = lib.unum_max_pooling_1d_varlen(n, 10, 0, n, n, n, n, 1, 2, 1, 4, 1, 64, 0, 1, 1, n)
    assert st == _lib.UNUM_ERR_INVALID_ARGUMENT and b"block_size" in lib.unum_last_error()
    # row stride beyond the input: 2 heads * 8 tokens * stride 4 > 40 elements
    x = ctypes.c_void_p(16)
    st = lib.unum_max_pooling_1d_varlen(x, 40, 0, x, x, x, x, 2, 8, 1, 4, 2, 64, 16, 1, 1, n)
    assert st == _lib.UNUM_ERR_INVALID_ARGUMENT and b"exceeds" in lib.unum_last_error()
    st = lib.unum_max_pooling_1d_varlen(x, 64, 7, x, x, x, x, 2, 8, 1, 4, 2, 64, 16, 1, 1, n)
    assert st == _lib.UNUM_ERR_UNSUPPORTED
    # more heads than the grid's y dimension holds (the head is blockIdx.y)
    st = lib.unum_max_pooling_1d_varlen(x, 70000, 0, x, x, x, x, 70000, 1, 1, 1, 1, 64, 16, 1, 1, n)
    assert st == _lib.UNUM_ERR_INVALID_ARGUMENT and b"too many rows" in lib.unum_last_error()
    st = lib.unum_max_pooling_1d_varlen_topk(x, 280000, x, x, x, n, x, 70000, 1, 1, 4, 1, 64, 16,
                                             1, 1, 1, n)
    assert st == _lib.UNUM_ERR_INVALID_ARGUMENT and b"too many rows" in lib.unum_last_error()


def test_stage1_rejects_bad_arguments():
    lib = _lib.load()
    n = _null()
    st = lib.unum_infllmv2_attn_stage1(n, 1, 1, n, 1, 1, n, n, n, 0, 1, 4, 4, 30, 4, 128,
                                       10, 128, 0.1, 1, n, 0, n)
    assert st == _lib.UNUM_ERR_INVALID_ARGUMENT and b"not a multiple" in lib.unum_last_error()
    st = lib.unum_infllmv2_attn_stage1(n, 1, 1, n, 1, 1, n, n, n, 0, 1, 4, 4, 32, 2, 128,
                                       300, 256, 0.1, 1, n, 0, n)
    assert st == _lib.UNUM_ERR_INVALID_ARGUMENT and b"max_seqlen_k" in lib.unum_last_error()
    x = ctypes.c_void_p(16)
    st = lib.unum_infllmv2_attn_stage1(x, 1, 1, x, 1, 1, x, x, x, 5, 1, 4, 4, 32, 2, 128,
                                       10, 128, 0.1, 1, n, 0, n)
    assert st == _lib.UNUM_ERR_UNSUPPORTED
    assert lib.unum_infllmv2_attn_stage1_workspace_size(4, 32768, 32, 2, 128, 511) >= 0


def test_stage1_maxpool_rejects_bad_arguments():
    lib = _lib.load()
    n = _null()
    # q, strides, k, strides, cu_q, cu_k, scores, pooled, B, Tq, Tk, Hq, Hkv, D,
    # max_seqlen_k, out_cols, scale, causal, num_blocks, local, init, workspace, bytes, stream
    st = lib.unum_infllmv2_attn_stage1_maxpool(n, 1, 1, n, 1, 1, n, n, n, n, 1, 4, 4, 32, 2, 128,
                                               600, 640, 0.1, 1, -1, 1, 1, n, 0, n)
    assert st == _lib.UNUM_ERR_INVALID_ARGUMENT and b"num_blocks" in lib.unum_last_error()
    st = lib.unum_infllmv2_attn_stage1_maxpool(n, 1, 1, n, 1, 1, n, n, n, n, 1, 4, 4, 32, 2, 128,
                                               700, 640, 0.1, 1, 16, 1, 1, n, 0, n)
    assert st == _lib.UNUM_ERR_INVALID_ARGUMENT and b"max_seqlen_k" in lib.unum_last_error()
    # nothing to do: success without touching any pointer
    assert lib.unum_infllmv2_attn_stage1_maxpool(n, 1, 1, n, 1, 1, n, n, n, n, 1, 0, 4, 32, 2,
                                                 128, 600, 640, 0.1, 1, 16, 1, 1, n, 0, n) == 0


def test_check_maps_status_to_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.UNUM_ERR_INVALID_ARGUMENT, "op")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.UNUM_ERR_UNSUPPORTED, "op")
    with pytest.raises(RuntimeError):
        _lib.check(_lib.UNUM_ERR_LAUNCH, "op")
    _lib.check(_lib.UNUM_OK, "op")


def test_ops_refuse_cpu_tensors():
    """No CPU fallback: host tensors raise instead of running anything."""
    cu = torch.tensor([0, 4], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="HIP device"):
        infllmv2_attn_stage1(torch.zeros(4, 32, 128, dtype=torch.bfloat16),
                             torch.zeros(4, 2, 128, dtype=torch.bfloat16), None, cu, cu)
    with pytest.raises(RuntimeError, match="HIP device"):
        max_pooling_1d_varlen(torch.zeros(2, 4, 8), cu, cu, torch.zeros(1, dtype=torch.int32),
                              128, 128, 1, 1)
    with pytest.raises(RuntimeError, match="HIP device"):
        get_block_table(torch.zeros(2, 1, 4, dtype=torch.int32), torch.zeros(1, 8, dtype=torch.int32),
                        torch.zeros(1, dtype=torch.int32), torch.ones(1, dtype=torch.int32),
                        torch.ones(1, dtype=torch.int32))


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setenv("UNUM_OPS_AMD_LIB", str(tmp_path / "absent.so"))
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.load()


def test_split_workspace_bound():
    # Without a device the plan counts 256 CUs (an MI355X): the split
    # workspace stays below 12 KiB + 288 bytes per CU (3.07 MiB), inside the
    # 4 MiB array of the no-allocation entry, at the worst shapes found (one
    # kv head, 8 sequences, ~23K tokens over 2047 keys: 2.97 MiB).
    lib = _lib.load()
    worst = 0
    for Hkv in (1, 2):
        for B, tqs in ((1, (1, 3, 16, 300, 20000, 24021, 30000, 40000)),
                       (8, (8, 17, 128, 2400, 22939)), (256, (256, 513, 4096, 76800))):
            for Tq in tqs:
                for max_k in (513, 2047, 8447, 131071, 131072):
                    worst = max(worst, lib.unum_infllmv2_attn_stage1_workspace_size(
                        B, Tq, 16 * Hkv, Hkv, 128, max_k))
    assert 5 << 19 < worst < (12 * 1024 + 288) * 256 < 4 << 20, worst


def test_stage1_checks_the_launch_device():
    # Past validation the stage-1 entries resolve the launch device (the
    # current one, which the stream must belong to) before any launch: with
    # no device here they fail with a status and a message, launching nothing.
    if torch.cuda.is_available():
        pytest.skip("needs a host without a GPU")
    lib = _lib.load()
    fake = ctypes.c_void_p(256)
    st = lib.unum_infllmv2_attn_stage1(fake, 4096, 128, fake, 256, 128, fake, fake, fake,
                                       _lib.UNUM_DTYPE_F32, 1, 16, 16, 32, 2, 128, 16, 128,
                                       0.08, 1, None, 0, None)
    assert st == _lib.UNUM_ERR_LAUNCH and b"device" in lib.unum_last_error()
