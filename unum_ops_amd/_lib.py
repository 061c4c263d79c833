"""ctypes binding of the gfx950 C-ABI library (``include/unum_ops_amd.h``).

The library is loaded lazily on first use, after ``torch`` (so the process
has a single HIP runtime: torch's).  There is no fallback: if the library is
missing or fails to load, every op raises ``RuntimeError``.
"""

import contextlib
import ctypes
import os
import threading

import torch  # noqa: F401  -- must precede the library: it provides the HIP runtime

from .build import LIB_PATH

UNUM_OK = 0
UNUM_ERR_INVALID_ARGUMENT = -1
UNUM_ERR_UNSUPPORTED = -2
UNUM_ERR_WORKSPACE = -3
UNUM_ERR_LAUNCH = -4

UNUM_DTYPE_F32 = 0
UNUM_DTYPE_BF16 = 1
UNUM_DTYPE_F16 = 2

ABI_VERSION = 2

# Every symbol declared in include/unum_ops_amd.h with (restype, argtypes).
_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
SIGNATURES = {
    "unum_last_error": (ctypes.c_char_p, []),
    "unum_abi_version": (ctypes.c_int, []),
    "unum_infllmv2_attn_stage1": (ctypes.c_int, [
        _p, _i64, _i64,            # q, q_stride_t, q_stride_h
        _p, _i64, _i64,            # k, k_stride_t, k_stride_h
        _p, _p,                    # cu_seqlens_q, cu_seqlens_k
        _p, _i32,                  # out, out_dtype
        _i64, _i64, _i64,          # B, Tq, Tk
        _i64, _i64, _i64,          # Hq, Hkv, D
        _i64, _i64,                # max_seqlen_k, out_cols
        ctypes.c_float, _i32,      # scale, causal
        _p, _i64,                  # workspace, workspace_bytes
        _p,                        # stream
    ]),
    "unum_infllmv2_attn_stage1_workspace_size": (_i64, [_i64] * 6),
    "unum_infllmv2_attn_stage1_noalloc": (ctypes.c_int, [
        _p, _i64, _i64,            # q, q_stride_t, q_stride_h
        _p, _i64, _i64,            # k, k_stride_t, k_stride_h
        _p, _p,                    # cu_seqlens_q, cu_seqlens_k
        _p, _i32,                  # out, out_dtype
        _i64, _i64, _i64,          # B, Tq, Tk
        _i64, _i64, _i64,          # Hq, Hkv, D
        _i64, _i64,                # max_seqlen_k, out_cols
        ctypes.c_float, _i32,      # scale, causal
        _p,                        # stream
    ]),
    "unum_infllmv2_attn_stage1_maxpool": (ctypes.c_int, [
        _p, _i64, _i64,            # q, q_stride_t, q_stride_h
        _p, _i64, _i64,            # k, k_stride_t, k_stride_h
        _p, _p,                    # cu_seqlens_q, cu_seqlens_k
        _p, _p,                    # scores (may be NULL), pooled
        _i64, _i64, _i64,          # B, Tq, Tk
        _i64, _i64, _i64,          # Hq, Hkv, D
        _i64, _i64,                # max_seqlen_k, out_cols
        ctypes.c_float, _i32,      # scale, causal
        _i64, _i32, _i32,          # num_blocks, local_blocks, init_blocks
        _p, _i64,                  # workspace, workspace_bytes
        _p,                        # stream
    ]),
    "unum_max_pooling_1d_varlen": (ctypes.c_int, [
        _p, _i64, _i32,            # input, input_numel, dtype
        _p, _p, _p,                # cu_seqlens_q, cu_seqlens_k, cache_lens
        _p,                        # out
        _i64, _i64, _i64,          # H, Tq, B
        _i64, _i64,                # flat_stride, num_blocks
        _i32, _i32, _i32, _i32,    # block_size, stride, local_blocks, init_blocks
        _p,                        # stream
    ]),
    "unum_max_pooling_1d_varlen_topk": (ctypes.c_int, [
        _p, _i64,                  # input, input_numel
        _p, _p, _p,                # cu_seqlens_q, cu_seqlens_k, cache_lens
        _p, _p,                    # pooled (may be NULL), topk_idx
        _i64, _i64, _i64,          # H, Tq, B
        _i64, _i64,                # flat_stride, num_blocks
        _i32, _i32, _i32, _i32,    # block_size, stride, local_blocks, init_blocks
        _i32,                      # topk
        _p,                        # stream
    ]),
    "unum_topk_blocks": (ctypes.c_int, [
        _p, _i64, _i64, _i64,      # pooled, rows, row_stride, num_blocks
        _p, _i32,                  # topk_idx, topk
        _p,                        # stream
    ]),
    "unum_compress_keys": (ctypes.c_int, [
        _p, _i64, _i64,            # k, k_stride_t, k_stride_h
        _p, _p, _p, _i64,          # cu_seqlens_raw, cu_seqlens_comp, unit_prefix, n_units
        _p,                        # out
        _i64, _i64, _i64, _i64, _i64,  # B, T_raw, T_comp, H, D
        _i32, _i32, _i32,          # kernel_size, stride, windows_per_unit
        _p,                        # stream
    ]),
    "unum_sparse_paged_attention": (ctypes.c_int, [
        _p, _i64, _i64,            # q, q_stride_t, q_stride_h
        _p, _p, _i64, _i64,        # key_cache, value_cache, kv_row_stride, n_rows
        _p, _i64, _i64, _i64,      # topk_idx + strides (h, t, k)
        _p, _i64,                  # block_table, row stride
        _p,                        # slots (may be NULL)
        _p, _p, _i64,              # token_to_bs, token_pos_in_bs, numel
        _p, _i64,                  # seqlen_q, numel
        _p, _i32,                  # out, out_dtype
        _i64, _i64, _i64, _i64, _i64, _i64, _i64,  # T, Hq, Hkv, D, K, B, L
        ctypes.c_float,            # scale
        _p,                        # stream
    ]),
    "unum_sparse_gather_calibrate": (ctypes.c_int, [
        _p, _p, _i64, _i64,        # key_cache, value_cache, kv_row_stride, n_rows
        _p, _i64, _i64, _i64,      # topk_idx + strides (h, t, k)
        _p, _i64,                  # block_table, row stride
        _p,                        # slots (may be NULL)
        _p, _p, _i64,              # token_to_bs, token_pos_in_bs, numel
        _p, _i64,                  # seqlen_q, numel
        _p,                        # out (u32 [T, Hkv, 64])
        _i64, _i64, _i64, _i64, _i64,  # T, Hkv, K, B, L
        _p,                        # stream
    ]),
    "unum_get_block_table": (ctypes.c_int, [
        _p, _i64, _i64, _i64,      # topk_idx + strides (h, t, k)
        _p, _i64,                  # block_table, row stride
        _p,                        # token_to_bs
        _p, _i64,                  # token_pos_in_bs, numel
        _p, _i64,                  # seqlen_q, numel
        _p,                        # out
        _i64, _i64, _i64, _i64, _i64,  # H, T, K, B, L
        _i32,                      # head_group
        _p,                        # stream
    ]),
}

_lock = threading.Lock()
_lib = None


def library_path():
    return os.environ.get("UNUM_OPS_AMD_LIB", LIB_PATH)


def load():
    """Load and bind the library (idempotent). Raises RuntimeError if absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"unum_ops_amd: native library not found at {path}; build it with "
                "`python -m unum_ops_amd.build` (there is no CPU fallback)")
        lib = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.unum_abi_version() != ABI_VERSION:
            raise RuntimeError(f"unum_ops_amd: ABI version {lib.unum_abi_version()} != {ABI_VERSION}")
        _lib = lib
        return lib


def check(status, what):
    """Turn a C status into an exception carrying the library's message."""
    if status == UNUM_OK:
        return
    msg = load().unum_last_error().decode(errors="replace")
    if status in (UNUM_ERR_INVALID_ARGUMENT, UNUM_ERR_WORKSPACE):
        raise ValueError(f"{what}: {msg}")
    if status == UNUM_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (status {status})")


# torch's own raw-stream query (what its kernel launchers call): a plain int,
# without building a Stream object per call.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device):
    """Raw hipStream_t of torch's current stream on ``device`` (an int; the
    entry points take it as ``void*``)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t):
    """A tensor's device address for a ``void*`` argument (None: NULL)."""
    return t.data_ptr() if t is not None else None


def device_guard(device):
    """``torch.cuda.device(device)``, or nothing when it is already current."""
    if device.index is None or device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)
