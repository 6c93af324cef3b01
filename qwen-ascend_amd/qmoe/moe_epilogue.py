"""Decode MoE combine over the Cartesian down output, with the reference's rounding.

Drop-in for ``fnx/moe_epilogue.py:6-21`` (kernel
``kernels/moe_epilogue/epilogue.cpp:4-43``): r = bf16(sum_j bf16(y_jj * w_j))
over the diagonal blocks of ``cartesian [k, k*H]``, then
out = bf16(r + bf16(shared * bf16(sigmoid(gate)))). Shape-generic in k and H;
``shared``/``gate`` may both be None (no shared expert: out = r). Returns None
for non-bf16, non-contiguous or mixed-device inputs.
"""
import torch

from . import _lib


def merge(cartesian, weights, shared, gate):
    tensors = tuple(t for t in (cartesian, weights, shared, gate) if t is not None)
    if cartesian.dim() != 2 or (shared is None) != (gate is None):
        return None
    k = cartesian.shape[0]
    if k < 1 or cartesian.shape[1] % k or weights.numel() != k:
        return None
    H = cartesian.shape[1] // k
    if (cartesian.device.type != "cuda"
            or any(t.dtype != torch.bfloat16 or not t.is_contiguous() or t.device != cartesian.device
                   for t in tensors)
            or (shared is not None and (shared.numel() != H or gate.numel() != 1))):
        return None
    out = torch.empty((1, H), dtype=torch.bfloat16, device=cartesian.device)
    rc = _lib.lib().qmoe_moe_epilogue(cartesian.data_ptr(), weights.data_ptr(), _lib.ptr(shared),
                                      _lib.ptr(gate), out.data_ptr(), k, H, _lib.stream_of(cartesian))
    if rc:
        raise RuntimeError(f"MoE epilogue launch rejected: {rc}")
    return out
