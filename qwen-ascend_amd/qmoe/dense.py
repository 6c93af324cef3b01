"""W8A16 dense projections: the reference's ``DenseW8`` container
(``fnx/engine.py:297-384``) on the HIP W8A16 kernels.

Same constructor, attributes (``w8t, sc, gs, K, N, chunks``) and methods
(``make_chunks``, ``deq_w``, ``__call__``, ``merge``): int8 weights stay
resident, the per-group dequantisation happens inside the GEMM
(``qmoe_w8a16_gemv`` for up to four rows, ``qmoe_w8a16_gemm_mfma`` above),
reached through :func:`qmoe.weight_quant_batchmatmul` exactly as the
reference reaches ``torch_npu.npu_weight_quant_batchmatmul``.
"""
from __future__ import annotations

import torch

from .ops import weight_quant_batchmatmul

BF16 = torch.bfloat16


class DenseW8:
    """Dense int8 weights with bf16 group scales: y = x @ (q * S).

    q: int8 [N, Kp] (per output row, possibly padded past K); s: [N, G'] group
    scales (gs = Kp // G'); K: the unpadded reduction length. Kept as
    w8t int8 [K, N] and sc bf16 [K/gs, N], the operator's layout
    (``fnx/engine.py:318-328``).
    """

    __slots__ = ("w8t", "sc", "gs", "K", "N", "chunks")

    def __init__(self, q, s, K=None):
        gs = q.shape[-1] // s.shape[-1]
        kk = q.shape[-1] if K is None else K
        if kk % gs:
            raise ValueError(f"DenseW8: K={kk} is not a multiple of gs={gs}")
        g = kk // gs
        self.w8t = q[:, :kk].t().contiguous()
        self.sc = s[:, :g].t().contiguous().to(BF16)
        self.gs = gs
        self.K = kk
        self.N = self.w8t.shape[1]
        self.chunks = None

    def make_chunks(self, chunk_n):
        """Pre-split along N into contiguous pieces (``fnx/engine.py:330-349``;
        the reference needs it for the operator's N <= 65535 limit, which these
        kernels do not have; kept so callers that chunk keep working)."""
        parts = []
        off = 0
        for w, s in zip(torch.split(self.w8t, chunk_n, dim=1), torch.split(self.sc, chunk_n, dim=1)):
            n0 = off
            off += w.shape[1]
            parts.append((w.contiguous(), s.contiguous(), n0, off))
        self.chunks = parts
        self.w8t = None
        self.sc = None

    def deq_w(self):
        """bf16 dequantised weights [N, K] (``fnx/engine.py:351-356``: the
        product rounded to bf16, for callers that pre-dequantise)."""
        if self.chunks is not None:
            raise RuntimeError("DenseW8 is split into chunks; dequantise before make_chunks")
        w = self.w8t.to(BF16) * self.sc.repeat_interleave(self.gs, dim=0)
        return w.t().contiguous()

    def __call__(self, x):
        sh = x.shape
        if x.dtype != BF16:
            x = x.to(BF16)
        x2 = x if x.dim() == 2 else x.reshape(-1, sh[-1])
        if self.chunks is None:
            y = weight_quant_batchmatmul(x2, self.w8t, self.sc, antiquant_group_size=self.gs)
        else:
            y = torch.empty(x2.shape[0], self.N, dtype=BF16, device=x2.device)
            for w, s, n0, n1 in self.chunks:
                y[:, n0:n1] = weight_quant_batchmatmul(x2, w, s, antiquant_group_size=self.gs)
        return y if x.dim() <= 2 else y.view(*sh[:-1], self.N)

    @staticmethod
    def merge(parts):
        """Concatenate projections that read the same input along N
        (``fnx/engine.py:369-384``): one call computes them all."""
        assert parts and all(p is not None for p in parts)
        gs = parts[0].gs
        assert all(p.gs == gs and p.K == parts[0].K for p in parts), "group size / K differ"
        o = DenseW8.__new__(DenseW8)
        o.w8t = torch.cat([p.w8t for p in parts], dim=1)
        o.sc = torch.cat([p.sc for p in parts], dim=1)
        o.gs, o.K, o.N = gs, parts[0].K, o.w8t.shape[1]
        o.chunks = None
        return o
