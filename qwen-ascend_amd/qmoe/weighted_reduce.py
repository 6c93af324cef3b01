"""BF16 product rounding followed by ordered fp32 accumulation (the MoE combine).

Drop-in for ``fnx/weighted_reduce.py:10-42`` modes 1/2 (kernel
``kernels/reduce/reduce.cpp:27-56``):
out[t, :] = bf16(sum_{g in order} bf16(x[row, :] * w[t, g])) with
row = inverse[t*G + g] (``inverse`` given) or t*G + g. Any width and group
count; ``mean=True`` (the hyper-connection mixer mode) is not part of the MoE
path and returns None so the caller falls back, as the reference does for
shapes its kernel does not take.
"""
import torch

from . import _lib


def reduce(values, weights, *, inverse=None, mean=False, order=0):
    if mean or order != 0:
        return None
    if weights.dim() != 2:
        return None
    batch, groups = weights.shape
    width = values.shape[-1]
    x = values.reshape(-1, width)
    if values.dtype != torch.bfloat16 or weights.dtype != torch.bfloat16 or x.stride(1) != 1:
        return None
    if x.device != weights.device or x.device.type != "cuda":
        return None
    if inverse is None and x.shape[0] < batch * groups:
        return None
    if inverse is not None and (inverse.dtype != torch.int64 or not inverse.is_contiguous()
                                or inverse.numel() != batch * groups or inverse.device != x.device):
        return None
    w = weights.float().contiguous()
    output = torch.empty((batch, width), dtype=torch.bfloat16, device=x.device)
    rc = _lib.lib().qmoe_weighted_reduce(x.data_ptr(), w.data_ptr(), _lib.ptr(inverse), output.data_ptr(),
                                         batch, groups, width, x.stride(0), x.shape[0], _lib.stream_of(x))
    if rc:
        raise RuntimeError(f"weighted reduction launch rejected: {rc}")
    return output
