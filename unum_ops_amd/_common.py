"""Argument plumbing shared by the op wrappers (device checks, int32 views)."""

import torch


def require_gpu(op, *tensors):
    """All tensors on one HIP device; the path has no CPU implementation."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{op}: expected torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise RuntimeError(
                f"{op}: tensors must be on a HIP device (got {t.device}); "
                "unum_ops_amd runs only on gfx950 GPUs and has no CPU fallback")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{op}: tensors on different devices ({dev} vs {t.device})")
    return dev


def as_i32(t, name, op):
    """Contiguous int32 view/copy of an integer index tensor."""
    if t.dtype.is_floating_point or t.dtype == torch.bool:
        raise TypeError(f"{op}: {name} must be an integer tensor, got {t.dtype}")
    if t.dtype != torch.int32:
        t = t.to(torch.int32)
    return t.contiguous()


def as_int(x, name, op):
    """Python int from an int or a one-element tensor (the reference's callers pass both)."""
    if isinstance(x, torch.Tensor):
        if x.numel() != 1:
            raise ValueError(f"{op}: {name} must be a scalar")
        return int(x.item())
    return int(x)
