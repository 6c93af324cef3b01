"""Gather selected expert-major W4 weights/scales into a K-major concatenation.

Drop-in for ``fnx/expert_gather.py:9-31`` (kernel
``kernels/expert_gather/gather.cpp:4-27``): ``ow[k, j*N/8 + c] = w4[ids[j], k, c]``
and ``os[g, j*N + n] = S[ids[j], g, n]``. Shape-generic (any K, G, N with
N % 32 == 0 and any number of ids); returns None, like the reference, when the
projection is not expert-major with cached scales or the tensors are not
contiguous device tensors of the expected dtypes.
"""
import torch

from . import _lib


def gather(projection, ids):
    if (not projection.expert_major or projection._scales is None or ids.dim() != 1
            or ids.dtype != torch.int64 or not ids.is_contiguous()):
        return None
    w, s = projection.w4, projection._scales
    if (w.dtype != torch.int32 or s.dtype != torch.bfloat16 or not w.is_contiguous() or not s.is_contiguous()
            or w.device != s.device or w.device != ids.device or w.device.type != "cuda"
            or projection.N % 32):
        return None
    k = ids.numel()
    ow = torch.empty((projection.K, k * projection.N // 8), dtype=torch.int32, device=w.device)
    oscale = torch.empty((projection.G, k * projection.N), dtype=torch.bfloat16, device=w.device)
    rc = _lib.lib().qmoe_expert_gather(w.data_ptr(), s.data_ptr(), ids.data_ptr(), ow.data_ptr(),
                                       oscale.data_ptr(), projection.K, projection.G, projection.N,
                                       projection.E, k, _lib.stream_of(w))
    if rc:
        raise RuntimeError(f"expert gather launch rejected: {rc}")
    return ow, oscale
