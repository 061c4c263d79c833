"""Key compression: raw keys -> the compressed keys stage 1 scores against.

The reference's stage 1 (``infllmv2_attn_stage1_triton_v2.py:153-228``) takes
compressed keys as input and the repository has no code that makes them; its
benchmark configurations define them as mean-pooled windows of 32 raw keys,
16 apart.  ``compress_keys`` computes exactly that on the GPU, packed varlen
like the other ops: window ``j`` of sequence ``b`` is the mean of raw keys
``16j .. 16j+31`` of the sequence, and a sequence of ``L`` tokens has
``(L - 32) // 16 + 1`` windows (none if ``L < 32``).
"""

import torch

from . import _lib
from ._common import require_gpu

KERNEL, STRIDE = 32, 16


def compressed_lengths(lengths, kernel_size=KERNEL, stride=STRIDE):
    """Windows per sequence for int64 ``lengths``."""
    return torch.where(lengths >= kernel_size, (lengths - kernel_size) // stride + 1,
                       torch.zeros_like(lengths))


class CompressionPlan:
    """Host-side sizes of a compression: the compressed prefix sums and the
    work split, already on the device, so ``compress_keys`` needs no sync."""

    def __init__(self, cu_seqlens_k, H, D, device, kernel_size=KERNEL, stride=STRIDE):
        cu = torch.as_tensor(cu_seqlens_k).detach().to("cpu", torch.int64).reshape(-1)
        self.B = cu.numel() - 1
        if self.B < 0:
            raise ValueError("compress_keys: cu_seqlens_k must hold at least one entry")
        lengths = cu[1:] - cu[:-1]
        if (lengths < 0).any() or (self.B > 0 and cu[0] < 0):
            raise ValueError("compress_keys: cu_seqlens_k must be non-decreasing from >= 0")
        lk = compressed_lengths(lengths, kernel_size, stride)
        cu_c = torch.zeros(self.B + 1, dtype=torch.int64)
        cu_c[1:] = torch.cumsum(lk, 0)
        self.total = int(cu_c[-1]) if self.B > 0 else 0
        self.max_len = int(lk.max()) if self.B > 0 else 0
        self.raw_total = int(cu[-1]) if self.B > 0 else 0
        self.kernel_size, self.stride, self.H, self.D = kernel_size, stride, H, D
        # Windows per lane group: a group loads and sums each half-block of
        # its run of windows once, so longer runs load less; about 512 waves
        # in all measured fastest, at most 16 windows a group.  A lane takes
        # 4 elements of a token row when the row fits a wave that way, else
        # 8 (the kernel's rule), which sets the groups per wave.
        slice_elems = 4 if H * (D // 4) <= 64 else 8
        groups = 64 // max(1, H * (D // slice_elems))
        per_group = max(1, min(16, self.total // (512 * max(groups, 1))))
        self.per_unit = per_group * max(groups, 1)
        units = (lk + self.per_unit - 1) // self.per_unit
        prefix = torch.zeros(self.B + 1, dtype=torch.int64)
        prefix[1:] = torch.cumsum(units, 0)
        self.n_units = int(prefix[-1]) if self.B > 0 else 0
        self.cu_raw = cu.to(torch.int32).to(device)
        self.cu_comp = cu_c.to(torch.int32).to(device)
        self.unit_prefix = prefix.to(torch.int32).to(device)


def compress_keys(k, cu_seqlens_k, kernel_size=KERNEL, stride=STRIDE, plan=None):
    """Mean-pool raw keys ``k [T, H, D]`` (bf16) per sequence of ``cu_seqlens_k``.

    Returns ``(k_compressed [T_c, H, D] bf16, cu_seqlens_compressed int32 [B+1],
    max_seqlen_compressed)``, the first two on ``k``'s device -- the inputs
    ``infllmv2_attn_stage1`` takes as ``k``, ``cu_seqlens_k`` and
    ``max_seqlen_k``.  Sums run in fp32 in token order over 16-token halves
    of each window; the mean is rounded to bf16 (nearest-even).  Without a
    ``plan`` (a ``CompressionPlan`` of the same ``cu_seqlens_k``) the ``B+1``
    prefix sums are read back to the host to size the output -- one sync, as
    the reference's stage 1 makes for ``max_seqlen_k``.
    """
    op = "compress_keys"
    dev = require_gpu(op, k, cu_seqlens_k)
    if k.dim() != 3:
        raise ValueError(f"{op}: k must be [total_tokens, H, D]")
    if kernel_size != 2 * stride or stride != STRIDE:
        raise NotImplementedError(f"{op}: kernel_size={kernel_size} stride={stride} "
                                  f"(supported: {KERNEL} / {STRIDE})")
    if k.dtype != torch.bfloat16:
        raise TypeError(f"{op}: k must be bfloat16, got {k.dtype}")
    T, H, D = k.shape
    if D % 8 != 0 or H * (D // 8) > 64:
        raise NotImplementedError(f"{op}: H*D/8 = {H * D // 8} must be at most 64 (D % 8 == 0)")
    if k.stride(-1) != 1 or k.stride(0) % 8 or k.stride(1) % 8 or k.data_ptr() % 16:
        k = k.contiguous()
    if plan is None:
        plan = CompressionPlan(cu_seqlens_k, H, D, dev, kernel_size, stride)
    elif (plan.H, plan.D, plan.kernel_size, plan.stride) != (H, D, kernel_size, stride):
        raise ValueError(f"{op}: the plan was made for another shape")
    if plan.raw_total > T:
        raise ValueError(f"{op}: cu_seqlens_k ends at {plan.raw_total} > {T} key rows")
    out = torch.empty(plan.total, H, D, dtype=torch.bfloat16, device=dev)
    if plan.total == 0:
        return out, plan.cu_comp, plan.max_len
    lib = _lib.load()
    with _lib.device_guard(dev):
        st = lib.unum_compress_keys(
            _lib.ptr(k), k.stride(0), k.stride(1), _lib.ptr(plan.cu_raw), _lib.ptr(plan.cu_comp),
            _lib.ptr(plan.unit_prefix), plan.n_units, _lib.ptr(out), plan.B, T, plan.total, H, D,
            kernel_size, stride, plan.per_unit, _lib.stream_ptr(dev))
    _lib.check(st, op)
    return out, plan.cu_comp, plan.max_len


__all__ = ["compress_keys", "compressed_lengths", "CompressionPlan"]
