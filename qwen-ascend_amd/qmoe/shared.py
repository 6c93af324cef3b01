"""Shared expert and router projection of the MoE block, and the whole block.

The step before the experts in ``FnLayer._moe`` (``fnx/engine.py:1786-1802``,
fused form ``sh_gw``: the four projections that read x concatenated into one
weight, ``fnx/engine.py:1226-1241``):

    gu     = F.linear(x, sh_gu)            # [b, 2MI + 1 + E]: gate | up | gate2 | router
    sh     = F.linear(F.silu(gu[:, :MI]) * gu[:, MI:2MI], sh_down)
    gate2  = gu[:, 2MI:2MI+1];  logits = gu[:, 2MI+1:]

One to four rows run the hand-written bf16 GEMVs of libqmoe.so (the shared
SwiGLU is computed inside the second one); larger batches run the two
projections on the hand-written bf16 MFMA GEMM with the SwiGLU and gate
kernels of libqmoe.so. :func:`moe_block` chains this with the expert block: at decode
the sigmoid-gated shared merge is fused into the experts' epilogue
(``fnx/engine.py:1790-1791, 1884-1891``); for larger batches the shared
output is gated first, ``sh = sigmoid(gate2) * sh`` (``fnx/engine.py:1793``),
and added after the ordered slot reduction (``fnx/engine.py:1853``).
"""
from __future__ import annotations

import torch

from . import _lib
from .engine import DECODE_MAX_TOKENS, moe_decode, moe_prefill

BF16 = torch.bfloat16


def _check_bf16_2d(t, what):
    if t.dtype != BF16 or t.dim() != 2:
        raise RuntimeError(f"{what} must be a 2-D bf16 tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"{what} must be a device tensor")


def linear(x, w):
    """``F.linear(x, w)`` for bf16 x [M, K] and w [N, K] (the reference's
    ``_fl``, ``fnx/engine.py:256``): fp32 accumulation, bf16 out. Up to four
    rows run the HIP GEMV, more rows the HIP MFMA GEMM (``qmoe_bf16_gemm``)."""
    _check_bf16_2d(x, "x")
    _check_bf16_2d(w, "w")
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise RuntimeError(f"x {tuple(x.shape)} and w {tuple(w.shape)} do not match")
    if M > DECODE_MAX_TOKENS:
        return _gemm(x, w)
    return _gemv(x, w, N)


def _gemm(x, w, ldy=None):
    """HIP MFMA GEMM into rows ldy >= N apart; returns the [M, N] view."""
    M, K = x.shape
    N = w.shape[0]
    ldy = N if ldy is None else ldy
    x = x if (x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0) else x.contiguous()
    w = w.contiguous()
    y = torch.empty((M, ldy), dtype=BF16, device=x.device)
    _lib.check(_lib.lib().qmoe_bf16_gemm(x.data_ptr(), x.stride(0), w.data_ptr(), y.data_ptr(), ldy, M, K, N,
                                         _lib.stream_of(x)), "bf16 GEMM")
    return y[:, :N]


def _gemv(x, w, ldy):
    """HIP GEMV into rows ldy >= N apart (a padded stride keeps later
    16-byte reads of the rows aligned); returns the [M, N] view."""
    M, K = x.shape
    N = w.shape[0]
    x, w = x.contiguous(), w.contiguous()
    y = torch.empty((M, ldy), dtype=BF16, device=x.device)
    if M:
        rc = _lib.lib().qmoe_bf16_gemv(x.data_ptr(), K, w.data_ptr(), y.data_ptr(), ldy, M, K, N,
                                       _lib.stream_of(x))
        _lib.check(rc, "bf16 linear")
    return y[:, :N]


def swiglu_bf16(gu, MI):
    """``F.silu(gu[:, :MI]) * gu[:, MI:2MI]`` on bf16 (two roundings,
    ``fnx/engine.py:1788``) -> [rows, MI]."""
    _check_bf16_2d(gu, "gu")
    gu = gu if gu.stride(1) == 1 else gu.contiguous()
    rows = gu.shape[0]
    act = torch.empty((rows, MI), dtype=BF16, device=gu.device)
    rc = _lib.lib().qmoe_swiglu_bf16(gu.data_ptr(), gu.stride(0), act.data_ptr(), rows, MI, _lib.stream_of(gu))
    _lib.check(rc, "swiglu_bf16")
    return act


def gate_shared(sh, gate2):
    """``torch.sigmoid(gate2) * sh`` on bf16 (``fnx/engine.py:1793``):
    bf16(bf16(sigmoid(g)) * sh) with g [rows, 1] broadcast over sh [rows, H]."""
    _check_bf16_2d(sh, "sh")
    sh = sh.contiguous()
    rows, H = sh.shape
    out = torch.empty_like(sh)
    rc = _lib.lib().qmoe_shared_gate(sh.data_ptr(), gate2.data_ptr(), gate2.stride(0), out.data_ptr(), rows, H,
                                     _lib.stream_of(sh))
    _lib.check(rc, "shared_gate")
    return out


def shared_router(x2, sh_gu, sh_down, MI):
    """Shared expert (ungated) and router logits of ``fnx/engine.py:1786-1796``.

    x2 bf16 [b, H]; sh_gu bf16 [2MI + 1 + E, H] (gate, up, gate2 and router
    rows); sh_down bf16 [H, MI]. Returns (sh [b, H], gate2 [b, 1],
    logits [b, E]); gate2 is a view of the fused projection. Up to four rows
    the GEMV writes the logits into rows of their own (16-byte aligned, as
    the one-token decode kernel reads them); above, logits is a view too."""
    _check_bf16_2d(x2, "x2")
    _check_bf16_2d(sh_gu, "sh_gu")
    _check_bf16_2d(sh_down, "sh_down")
    b, H = x2.shape
    if sh_gu.shape[1] != H or sh_gu.shape[0] <= 2 * MI + 1 or sh_down.shape != (H, MI):
        raise RuntimeError("sh_gu must be [2MI+1+E, H] and sh_down [H, MI]")
    N, split = sh_gu.shape[0], 2 * MI + 1
    if b > DECODE_MAX_TOKENS:
        gu = _gemm(x2, sh_gu, (N + 7) // 8 * 8)
        sh = linear(swiglu_bf16(gu, MI), sh_down)
        return sh, gu[:, 2 * MI:split], gu[:, split:]
    # gate | up | gate2 into gu, the router columns into logits; the shared
    # SwiGLU is read straight from gu by the down GEMV
    ld = (split + 7) // 8 * 8
    x2, sh_gu = x2.contiguous(), sh_gu.contiguous()
    gu = torch.empty((b, ld), dtype=BF16, device=x2.device)
    logits = torch.empty((b, N - split), dtype=BF16, device=x2.device)
    sh = torch.empty((b, H), dtype=BF16, device=x2.device)
    if b:
        L, st = _lib.lib(), _lib.stream_of(x2)
        _lib.check(L.qmoe_bf16_gemv_split(x2.data_ptr(), H, sh_gu.data_ptr(), gu.data_ptr(), ld, logits.data_ptr(),
                                          N - split, split, b, H, N, st), "shared/router projection")
        _lib.check(L.qmoe_bf16_gemv_swiglu(gu.data_ptr(), ld, sh_down.contiguous().data_ptr(), sh.data_ptr(), H, b,
                                           MI, H, st), "shared down")
    return sh, gu[:, 2 * MI:split], logits


def moe_block(x2, sh_gu, sh_down, exp_gu, exp_dn, topk):
    """The whole MoE block of ``FnLayer._moe`` for ``ExpW4`` experts
    (``fnx/engine.py:1782-1891``): shared expert and router, then the routed
    experts with the top-k combine and the shared merge. x2 bf16 [b, H] ->
    bf16 [b, H]."""
    MI = exp_dn.K
    sh, gate2, logits = shared_router(x2, sh_gu, sh_down, MI)
    if x2.shape[0] <= DECODE_MAX_TOKENS:
        return moe_decode(x2, logits.contiguous(), exp_gu, exp_dn, topk, shared=sh,
                          shared_gate=gate2.contiguous())[0]
    return moe_prefill(x2, logits.contiguous(), exp_gu, exp_dn, topk, shared=gate_shared(sh, gate2))
