"""Shared-expert merge with the reference's intermediate bf16 rounding.

Drop-in for ``fnx/post_ops.py:36-39`` ``moe_merge`` (kernel
``kernels/post_ops/post_ops.cpp:72-94``):
out = bf16(e + bf16(s * bf16(sigmoid(g)))), one gate value per row of e.
The hyper-connection mixer ops of that module are not on the MoE path.
"""
import torch

from . import _lib


def moe_merge(experts, shared, gate):
    tensors = (experts, shared, gate)
    if (shared.shape != experts.shape or experts.dim() < 1 or experts.device.type != "cuda"
            or any(t.dtype != torch.bfloat16 or not t.is_contiguous() or t.device != experts.device
                   for t in tensors)):
        return None
    width = experts.shape[-1]
    rows = experts.numel() // width
    if gate.numel() != rows:
        return None
    out = torch.empty_like(experts)
    rc = _lib.lib().qmoe_moe_merge(experts.data_ptr(), shared.data_ptr(), gate.data_ptr(), out.data_ptr(),
                                   rows, width, _lib.stream_of(experts))
    if rc:
        raise RuntimeError(f"decode postprocessing launch rejected: {rc}")
    return out
