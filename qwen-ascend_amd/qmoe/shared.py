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
    """HIP MFMA GEMM into rows ldy >= N apart; returns the [M, N] view.

    The kernel reads 16-byte pieces of 32-wide K chunks: operands that start
    off a 16-byte boundary are copied to fresh (aligned) tensors, and a K that
    is not a multiple of 32 is zero-padded (extra zero products leave every
    fp32 sum unchanged)."""
    M, K = x.shape
    N = w.shape[0]
    ldy = N if ldy is None else ldy
    if K % 32:
        Kp = (K + 31) // 32 * 32
        xp = torch.zeros((M, Kp), dtype=BF16, device=x.device)
        wp = torch.zeros((N, Kp), dtype=BF16, device=w.device)
        xp[:, :K] = x
        wp[:, :K] = w
        x, w, K = xp, wp, Kp
    if not (x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0):
        x = x.clone(memory_format=torch.contiguous_format)   # a fresh allocation is 16-byte aligned
    w = w.contiguous()
    if w.data_ptr() % 16:
        w = w.clone()
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


def _check_block_args(x2, sh_gu, sh_down, MI):
    _check_bf16_2d(x2, "x2")
    _check_bf16_2d(sh_gu, "sh_gu")
    _check_bf16_2d(sh_down, "sh_down")
    H = x2.shape[1]
    if sh_gu.shape[1] != H or sh_gu.shape[0] <= 2 * MI + 1 or sh_down.shape != (H, MI):
        raise RuntimeError("sh_gu must be [2MI+1+E, H] and sh_down [H, MI]")


def _project(x2, sh_gu, MI):
    """Up to four rows: the fused projection as gu bf16 [b, ld] (gate | up |
    gate2, rows 16-byte aligned) and logits bf16 [b, E] in rows of their own
    (one GEMV launch)."""
    b, H = x2.shape
    N, split = sh_gu.shape[0], 2 * MI + 1
    ld = (split + 7) // 8 * 8
    x2, sh_gu = x2.contiguous(), sh_gu.contiguous()
    gu = torch.empty((b, ld), dtype=BF16, device=x2.device)
    logits = torch.empty((b, N - split), dtype=BF16, device=x2.device)
    if b:
        _lib.check(_lib.lib().qmoe_bf16_gemv_split(x2.data_ptr(), H, sh_gu.data_ptr(), gu.data_ptr(), ld,
                                                   logits.data_ptr(), N - split, split, b, H, N, _lib.stream_of(x2)),
                   "shared/router projection")
    return gu, logits


def _shared_down(gu, sh_down, MI, H):
    """sh = F.linear(F.silu(gu[:, :MI]) * gu[:, MI:2MI], sh_down) for up to
    four rows, the SwiGLU read straight from gu by the down GEMV."""
    b = gu.shape[0]
    sh = torch.empty((b, H), dtype=BF16, device=gu.device)
    if b:
        _lib.check(_lib.lib().qmoe_bf16_gemv_swiglu(gu.data_ptr(), gu.stride(0), sh_down.contiguous().data_ptr(),
                                                    sh.data_ptr(), H, b, MI, H, _lib.stream_of(gu)), "shared down")
    return sh


def shared_router(x2, sh_gu, sh_down, MI):
    """Shared expert (ungated) and router logits of ``fnx/engine.py:1786-1796``.

    x2 bf16 [b, H]; sh_gu bf16 [2MI + 1 + E, H] (gate, up, gate2 and router
    rows); sh_down bf16 [H, MI]. Returns (sh [b, H], gate2 [b, 1],
    logits [b, E]); gate2 is a view of the fused projection. Up to four rows
    the GEMV writes the logits into rows of their own (16-byte aligned, as
    the one-token decode kernel reads them); above, logits is a view too."""
    _check_block_args(x2, sh_gu, sh_down, MI)
    b, H = x2.shape
    N, split = sh_gu.shape[0], 2 * MI + 1
    if b > DECODE_MAX_TOKENS:
        gu = _gemm(x2, sh_gu, (N + 7) // 8 * 8)
        sh = linear(swiglu_bf16(gu, MI), sh_down)
        return sh, gu[:, 2 * MI:split], gu[:, split:]
    gu, logits = _project(x2, sh_gu, MI)
    return _shared_down(gu, sh_down, MI, H), gu[:, 2 * MI:split], logits


def _block_one_token(x2, gu, logits, sh_down, exp_gu, exp_dn, topk, MI, tiles):
    """One token: the experts and the shared expert's down projection in one
    launch (``qmoe_moe_block_decode``); None for shapes that launch does not
    take."""
    from .engine import _check_pair, _first_call_check, _tiles_for
    _check_pair(x2, exp_gu, exp_dn)
    H, dev = x2.shape[1], x2.device
    L = _lib.lib()
    ncnt = L.qmoe_moe_decode_counters(1, topk, H, MI)
    if ncnt < 0 or logits.shape != (1, exp_gu.E):
        return None
    gu_t, dn_t = _tiles_for(exp_gu, exp_dn, tiles)
    out = torch.empty((1, H), dtype=BF16, device=dev)
    idx = torch.empty((1, topk), dtype=torch.int64, device=dev)
    w = torch.empty((1, topk), dtype=BF16, device=dev)
    cnt = _lib.counters(dev, ncnt)
    x2 = x2.contiguous()
    rc = L.qmoe_moe_block_decode(x2.data_ptr(), logits.data_ptr(), exp_gu.w4.data_ptr(), exp_gu._scales.data_ptr(),
                                 exp_dn.w4.data_ptr(), exp_dn._scales.data_ptr(), _lib.ptr(gu_t), _lib.ptr(dn_t),
                                 gu.data_ptr(), sh_down.contiguous().data_ptr(), out.data_ptr(), idx.data_ptr(),
                                 w.data_ptr(), exp_gu.E, topk, H, MI, exp_gu.gs, exp_dn.gs, cnt.data_ptr(),
                                 _lib.stream_of(x2))
    if rc == _lib.EINVAL:
        return None
    _lib.check(rc, "moe_block_decode")
    _first_call_check(cnt, "moe_block")
    return out


def moe_block(x2, sh_gu, sh_down, exp_gu, exp_dn, topk, tiles=None):
    """The whole MoE block of ``FnLayer._moe`` for ``ExpW4`` experts
    (``fnx/engine.py:1782-1891``): shared expert and router, then the routed
    experts with the top-k combine and the shared merge. x2 bf16 [b, H] ->
    bf16 [b, H]. One token runs in two launches where it can (the
    projection, then the experts with the shared down projection beside
    them), else three; the bits are the same. ``tiles`` chooses the decode
    weights as in :func:`qmoe.engine.moe_decode` (None: the experts' decode
    tiles if they were built, True: build them, False: the int4pack only)."""
    MI = exp_dn.K
    _check_block_args(x2, sh_gu, sh_down, MI)
    b, H = x2.shape
    if b > DECODE_MAX_TOKENS:
        sh, gate2, logits = shared_router(x2, sh_gu, sh_down, MI)
        return moe_prefill(x2, logits.contiguous(), exp_gu, exp_dn, topk, shared=gate_shared(sh, gate2))
    gu, logits = _project(x2, sh_gu, MI)
    if b == 1:
        out = _block_one_token(x2, gu, logits, sh_down, exp_gu, exp_dn, topk, MI, tiles)
        if out is not None:
            return out
    sh = _shared_down(gu, sh_down, MI, H)
    return moe_decode(x2, logits, exp_gu, exp_dn, topk, shared=sh, shared_gate=gu[:, 2 * MI:2 * MI + 1].contiguous(),
                      tiles=tiles)[0]
