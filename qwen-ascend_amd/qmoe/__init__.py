"""qmoe: MI355X (gfx950) W4A16 MoE expert path with the reference's call signatures.

Host code is Python on PyTorch-ROCm; compute is hand-written HIP in
libqmoe.so, reached through a C ABI (include/qmoe.h) with ctypes.
"""
from . import _lib  # noqa: F401
from . import artifact  # noqa: F401
from . import shared  # noqa: F401
from .dense import DenseW8  # noqa: F401
from .engine import ExpW4, decode_status, moe_decode, moe_experts, moe_prefill  # noqa: F401
from .ops import grouped_matmul, route_group, router_topk, swiglu, weight_quant_batchmatmul  # noqa: F401

__all__ = ["artifact", "shared", "DenseW8", "ExpW4", "decode_status", "moe_decode", "moe_experts", "moe_prefill", "grouped_matmul", "route_group",
           "router_topk", "swiglu", "weight_quant_batchmatmul"]
