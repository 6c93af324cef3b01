"""W8A16 dense projections on the HIP W8A16 kernels.

:class:`DenseW8` has the interface of the reference's container
(``fnx/engine.py:297-384``): the constructor ``(q, s, K=None)``, the attributes
``w8t, sc, gs, K, N, chunks`` and the methods ``make_chunks``, ``deq_w``,
``__call__`` and ``merge``. The layout is the operator's: int8 weights
``[K, N]`` stay resident and the per-group dequantisation happens inside the
GEMM (``qmoe_w8a16_gemv`` for up to four rows, ``qmoe_w8a16_gemm_mfma``
above), reached through :func:`qmoe.weight_quant_batchmatmul`.

The HIP kernels have no limit on N, so one launch always covers the whole
projection: ``make_chunks`` only records column ranges (views of the
resident weight) for callers that iterate over them, and ``deq_w`` keeps
working after it.
"""
from __future__ import annotations

import torch

from .ops import weight_quant_batchmatmul

BF16 = torch.bfloat16


def _operator_layout(q, s, K):
    """(w8t int8 [K, N], sc bf16 [K/gs, N], gs) from per-output-row int8
    weights q [N, Kp] and group scales s [N, Gp] (columns past K are padding)."""
    if q.dim() != 2 or s.dim() != 2 or q.shape[0] != s.shape[0]:
        raise ValueError("DenseW8 takes q [N, Kp] and s [N, Gp] with the same N")
    if q.dtype != torch.int8:
        raise ValueError("DenseW8 weights must be int8")
    padded_k, padded_g = q.shape[1], s.shape[1]
    gs = padded_k // padded_g
    k = padded_k if K is None else int(K)
    if gs < 1 or k > padded_k or k % gs:
        raise ValueError(f"DenseW8: K={k} is not a multiple of gs={gs}")
    groups = k // gs
    w8t = q.narrow(1, 0, k).transpose(0, 1).contiguous()
    sc = s.narrow(1, 0, groups).to(BF16).transpose(0, 1).contiguous()
    return w8t, sc, gs


class DenseW8:
    """Dense int8 weights with bf16 group scales: y = x @ (q * S).

    q: int8 [N, Kp] (per output row, possibly padded past K); s: [N, Gp]
    group scales (gs = Kp // Gp); K: the unpadded reduction length.
    """

    __slots__ = ("w8t", "sc", "gs", "K", "N", "chunks")

    def __init__(self, q, s, K=None):
        self._adopt(*_operator_layout(q, s, K))

    def _adopt(self, w8t, sc, gs):
        self.w8t, self.sc, self.gs = w8t, sc, int(gs)
        self.K, self.N = w8t.shape
        if sc.shape != (self.K // self.gs, self.N):
            raise ValueError("scales must be [K/gs, N]")
        self.chunks = None

    def make_chunks(self, chunk_n):
        """Record column ranges of ``chunk_n`` columns as (weights, scales, n0,
        n1) views. The reference pre-splits to respect its operator's
        N <= 65535 limit (``fnx/engine.py:330-349``); the HIP kernels have
        none, so calls still run as one launch over the resident weight."""
        step = int(chunk_n)
        if step < 1:
            raise ValueError("chunk_n must be positive")
        self.chunks = [(self.w8t[:, n0:min(n0 + step, self.N)], self.sc[:, n0:min(n0 + step, self.N)],
                        n0, min(n0 + step, self.N)) for n0 in range(0, self.N, step)]

    def deq_w(self):
        """bf16 dequantised weights [N, K]: bf16(q * S[k // gs]), the rounding
        of the reference's bf16 multiply (``fnx/engine.py:351-356``; an int8
        times a bf16 is exact in fp32)."""
        groups = self.K // self.gs
        w = self.w8t.view(groups, self.gs, self.N).to(torch.float32) * self.sc.to(torch.float32).unsqueeze(1)
        return w.reshape(self.K, self.N).to(BF16).transpose(0, 1).contiguous()

    def __call__(self, x):
        lead = x.shape[:-1]
        rows = x.reshape(-1, x.shape[-1])
        if rows.dtype != BF16:
            rows = rows.to(BF16)
        y = weight_quant_batchmatmul(rows, self.w8t, self.sc, antiquant_group_size=self.gs)
        return y if x.dim() <= 2 else y.reshape(*lead, self.N)

    @staticmethod
    def merge(parts):
        """One projection whose columns are those of ``parts`` in order, for
        projections that read the same input (``fnx/engine.py:369-384``)."""
        parts = list(parts)
        if not parts or any(p is None for p in parts):
            raise ValueError("merge needs at least one projection")
        first = parts[0]
        for p in parts[1:]:
            if p.K != first.K or p.gs != first.gs:
                raise ValueError("merged projections must share K and the group size")
        merged = DenseW8.__new__(DenseW8)
        merged._adopt(torch.cat([p.w8t for p in parts], dim=1), torch.cat([p.sc for p in parts], dim=1), first.gs)
        return merged
