"""Expert containers and the MoE expert block on MI355X.

:class:`ExpW4` mirrors the reference container (``fnx/engine.py:619-753``):
same constructor, attributes (``w4, s8t, base, _scales, K, N, E, G, gs,
expert_major``) and methods (``apply``, ``apply_diag``, ``apply_grouped``,
``_wcat``, ``_scat``), so ``FnLayer._moe`` can call it unchanged. The
production flag set of the reference (``FNX_W4_SCALE_CACHE=1``,
``FNX_EXPERT_GATHER=1``, ``FNX_MOE_GROUP=1``, ...) is the only behaviour: the
bf16 scale cache is always built and there is no flag matrix.

:func:`moe_experts` is the fused expert block of ``FnLayer._moe``
(``fnx/engine.py:1803-1891``) from router logits to the combined output:
one to four tokens run the decode kernels (router, de-duplicated expert
GEMVs, SwiGLU, down GEMV and the top-k combine fused into its epilogue);
larger batches run the grouped prefill path (GPU routing histogram, stable
expert-major permutation, MFMA grouped GEMMs, weighted scatter, ordered
slot reduction).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .ops import grouped_matmul, route_group, router_topk, weight_quant_batchmatmul

BF16 = torch.bfloat16
DECODE_MAX_TOKENS = 4


class ExpW4:
    """Per-group W4A16 expert weights (int4pack) with a bf16 scale cache.

    w4: int32 [K, E, N/8] (K-major artifact) or [E, K, N/8] (``expert_major``);
    s8t: int8 [G, E, N]; base: bf16 [E, N]. The scale cache
    ``_scales = bf16(s8t^T * base)`` is expert-major [E, G, N]
    (``fnx/engine.py:653-659``). Use :meth:`from_scales` when bf16 scales
    are given directly.
    """

    __slots__ = ("w4", "s8t", "base", "K", "N", "E", "G", "gs", "expert_major", "_scales")

    def __init__(self, w4, s8t, base, gs, expert_major=False):
        self.w4 = w4
        self.expert_major = expert_major
        self.K, self.E = (w4.shape[1], w4.shape[0]) if expert_major else (w4.shape[0], w4.shape[1])
        self.N = w4.shape[2] * 8
        self.G = s8t.shape[0] if s8t is not None else None
        self.gs = gs
        self._scales = None
        self.s8t = s8t
        self.base = base
        if s8t is not None:
            self._scales = (s8t.permute(1, 0, 2).to(BF16) * base[:, None, :]).contiguous()
            self.s8t = self.base = None
        if self.G is not None and self.G * gs != self.K:
            raise ValueError(f"G {self.G} x gs {gs} != K {self.K}")

    @classmethod
    def from_scales(cls, w4_em, scales_em):
        """Expert-major int4pack [E, K, N/8] + bf16 scales [E, G, N]."""
        self = cls.__new__(cls)
        self.w4 = w4_em
        self.expert_major = True
        self.E, self.K = w4_em.shape[0], w4_em.shape[1]
        self.N = w4_em.shape[2] * 8
        self.G = scales_em.shape[1]
        if self.K % self.G:
            raise ValueError("K must be a multiple of the scale group count")
        self.gs = self.K // self.G
        self._scales = scales_em
        self.s8t = self.base = None
        return self

    def _wcat(self, ids):
        if self.expert_major:
            p = self.w4.index_select(0, ids).permute(1, 0, 2).contiguous()
            return p.reshape(self.K, -1)
        p = torch.index_select(self.w4, 1, ids)
        return p.reshape(self.K, p.shape[1] * (self.N // 8))

    def _scat(self, ids):
        return self._scales.index_select(0, ids).transpose(0, 1).contiguous().view(self.G, -1)

    def apply(self, x, ids):
        """x [M,K] bf16, ids [k] -> [M, k*N]: the k experts concatenated along N."""
        if self.expert_major:
            from .expert_gather import gather
            selected = gather(self, ids)
            if selected is not None:
                weights, scales = selected
                return weight_quant_batchmatmul(x, weights, scales, antiquant_group_size=self.gs)
        return weight_quant_batchmatmul(x, self._wcat(ids), self._scat(ids), antiquant_group_size=self.gs)

    def apply_diag(self, x, ids):
        """Row j of x [k,K] times expert ids[j] -> [k, N] (no Cartesian product)."""
        k = x.shape[0]
        if ids.numel() != k:
            raise ValueError("one expert id per activation row")
        if not self.expert_major:
            y = self.apply(x, ids)
            idx = torch.arange(k, device=x.device)
            return y.view(k, k, self.N)[idx, idx]
        ends = torch.arange(1, k + 1, dtype=torch.int64, device=x.device)
        return grouped_matmul([x], [self.w4.index_select(0, ids)],
                              antiquant_scale=[self._scales.index_select(0, ids)],
                              group_list=ends, split_item=3, group_type=0, output_dtype=BF16)[0]

    def apply_grouped(self, x, group_ends, host_ends=None):
        """Rows sorted by expert, one grouped GEMM (``fnx/engine.py:723-753``)."""
        if not self.expert_major:
            raise RuntimeError("grouped prefill requires the expert-major artifact")
        return grouped_matmul([x], [self.w4], antiquant_scale=[self._scales], group_list=group_ends,
                              split_item=3, group_type=0, output_dtype=BF16)[0]


def _check_pair(x, exp_gu, exp_dn):
    if not (exp_gu.expert_major and exp_dn.expert_major):
        raise RuntimeError("the fused expert block needs expert-major weights")
    if x.dtype != BF16 or x.dim() != 2 or x.shape[1] != exp_gu.K:
        raise RuntimeError("x must be bf16 [b, H]")
    if exp_gu.N % 2 or exp_dn.K != exp_gu.N // 2 or exp_dn.N != exp_gu.K or exp_gu.E != exp_dn.E:
        raise RuntimeError("gate_up [E,H,2MI] / down [E,MI,H] shapes do not match")


def _decode_intermediates(ws, B, k, H, MI):
    """Views of the decode workspace after a call: per (token, slot) the SwiGLU
    row and the weighted product (bf16 [B, k, MI] and [B, k, H])."""
    L = _lib.lib()
    o = [ctypes.c_size_t() for _ in range(3)]
    _lib.check(L.qmoe_moe_decode_layout(B, k, H, MI, *[ctypes.byref(v) for v in o]), "decode layout")
    off_plan, off_act, off_prod = (v.value for v in o)
    plan = ws[off_plan:off_plan + 705 * 4].view(torch.int32).cpu()
    umax = 64
    utok = plan[1 + 2 * umax:1 + 2 * umax + 4 * umax].view(umax, 4)
    uslot = plan[1 + 6 * umax:1 + 6 * umax + 4 * umax].view(umax, 4)
    umult = plan[1 + umax:1 + 2 * umax]
    act_all = ws[off_act:off_act + B * k * 4 * MI * 2].view(BF16).view(B * k, 4, MI)
    act = torch.empty((B, k, MI), dtype=BF16, device=ws.device)
    for u in range(int(plan[0])):
        for m in range(int(umult[u])):
            act[int(utok[u, m]), int(uslot[u, m])] = act_all[u, m]
    prod = ws[off_prod:off_prod + B * k * H * 4].view(torch.float32).view(B, k, H).to(BF16)
    return act, prod


def moe_decode(x, logits, exp_gu, exp_dn, topk, shared=None, shared_gate=None, return_intermediates=False):
    """Fused decode expert block for 1..4 tokens.

    x bf16 [B, H]; logits bf16 [B, E]. Returns (out bf16 [B, H], idx int64
    [B, topk], w bf16 [B, topk]). With ``shared``/``shared_gate`` (bf16 [B, H]
    / [B, 1]) the shared-expert merge of ``fnx/engine.py:1874-1891`` is
    applied in the same epilogue.
    """
    _check_pair(x, exp_gu, exp_dn)
    B, H = x.shape
    if not 1 <= B <= DECODE_MAX_TOKENS:
        raise RuntimeError(f"decode path takes 1..{DECODE_MAX_TOKENS} tokens")
    if logits.shape != (B, exp_gu.E) or logits.dtype != BF16:
        raise RuntimeError("logits must be bf16 [B, E]")
    if (shared is None) != (shared_gate is None):
        raise RuntimeError("shared and shared_gate go together")
    x, logits = x.contiguous(), logits.contiguous()
    dev = x.device
    MI = exp_dn.K
    out = torch.empty((B, H), dtype=BF16, device=dev)
    idx = torch.empty((B, topk), dtype=torch.int64, device=dev)
    w = torch.empty((B, topk), dtype=BF16, device=dev)
    L = _lib.lib()
    ws = _lib.workspace(dev, L.qmoe_moe_decode_workspace(B, topk, H, MI))
    ncnt = L.qmoe_moe_decode_counters(B, topk, H, MI)
    if ncnt < 0:
        raise RuntimeError("moe_decode: shape too large for the decode counters")
    cnt = _lib.counters(dev, ncnt)
    sh = shared.contiguous() if shared is not None else None
    sg = shared_gate.contiguous() if shared_gate is not None else None
    rc = L.qmoe_moe_decode(x.data_ptr(), logits.data_ptr(), exp_gu.w4.data_ptr(), exp_gu._scales.data_ptr(),
                           exp_dn.w4.data_ptr(), exp_dn._scales.data_ptr(), _lib.ptr(sh), _lib.ptr(sg),
                           out.data_ptr(), idx.data_ptr(), w.data_ptr(), B, exp_gu.E, topk, H, MI, exp_gu.gs,
                           exp_dn.gs, ws.data_ptr(), ws.numel(), cnt.data_ptr(), _lib.stream_of(x))
    _lib.check(rc, "moe_decode")
    if return_intermediates:
        return out, idx, w, _decode_intermediates(ws, B, topk, H, MI)
    return out, idx, w


def moe_decode_gate_up(x, logits, exp_gu, topk, MI):
    """The first of the two launches of the decode block in its two-launch form
    (router + gate_up + SwiGLU; :func:`moe_decode` itself is one launch), for
    callers that time or interleave the halves; returns the workspace it
    filled (its act rows are what ``qmoe_moe_decode_down`` reads)."""
    B, H = x.shape
    L = _lib.lib()
    ws = _lib.workspace(x.device, L.qmoe_moe_decode_workspace(B, topk, H, MI))
    idx = torch.empty((B, topk), dtype=torch.int64, device=x.device)
    w = torch.empty((B, topk), dtype=BF16, device=x.device)
    rc = L.qmoe_moe_decode_gate_up(x.data_ptr(), logits.data_ptr(), exp_gu.w4.data_ptr(), exp_gu._scales.data_ptr(),
                                   idx.data_ptr(), w.data_ptr(), B, exp_gu.E, topk, H, MI, exp_gu.gs, ws.data_ptr(),
                                   ws.numel(), _lib.counters(x.device).data_ptr(), _lib.stream_of(x))
    _lib.check(rc, "moe_decode_gate_up")
    return ws


def moe_prefill(x, logits, exp_gu, exp_dn, topk, shared=None, return_routing=False, return_intermediates=False):
    """Grouped prefill expert block for any number of tokens.

    Router on the GPU, routing histogram + stable expert-major permutation,
    gate_up grouped GEMM over rows gathered through the permutation with the
    SwiGLU epilogue, down grouped GEMM with the routing weight folded into its
    epilogue, ordered slot reduction, and ``+ shared`` (bf16 add,
    ``fnx/engine.py:1853``) when given. Returns out bf16 [T, H], plus the
    routing tensors (idx, w, counts, ends, order, inverse) when
    ``return_routing``, plus (act [T*k, MI] in expert-major row order, prod
    [T*k, H] token-major) when ``return_intermediates``.
    """
    _check_pair(x, exp_gu, exp_dn)
    T, H = x.shape
    if logits.shape != (T, exp_gu.E) or logits.dtype != BF16:
        raise RuntimeError("logits must be bf16 [T, E]")
    x = x.contiguous()
    dev = x.device
    MI = exp_dn.K
    E = exp_gu.E
    idx, w = router_topk(logits, topk)
    counts, ends, order, inverse, tiles, mt = route_group(idx, E, with_tiles=True)
    out = torch.empty((T, H), dtype=BF16, device=dev)
    L = _lib.lib()
    ws = _lib.workspace(dev, L.qmoe_moe_prefill_workspace(T, topk, H, MI))
    sh = shared.contiguous() if shared is not None else None
    rc = L.qmoe_moe_experts_grouped(
        x.data_ptr(), T, H, MI, E, topk, w.data_ptr(), order.data_ptr(), exp_gu.w4.data_ptr(),
        exp_gu._scales.data_ptr(), exp_gu.gs, exp_dn.w4.data_ptr(), exp_dn._scales.data_ptr(), exp_dn.gs,
        tiles[:mt].data_ptr(), tiles[mt:2 * mt].data_ptr(), tiles[2 * mt:3 * mt].data_ptr(),
        tiles[3 * mt:].data_ptr(), mt, _lib.ptr(sh), out.data_ptr(), ws.data_ptr(), ws.numel(),
        _lib.stream_of(x))
    _lib.check(rc, "moe_prefill")
    res = [out]
    if return_routing:
        res.append((idx, w, counts, ends, order, inverse))
    if return_intermediates:
        R = T * topk
        o = (ctypes.c_size_t(), ctypes.c_size_t())
        _lib.check(L.qmoe_moe_prefill_layout(T, topk, H, MI, *(ctypes.byref(v) for v in o)), "prefill layout")
        off_act, off_prod = (v.value for v in o)
        res.append((ws[off_act:off_act + R * MI * 2].view(BF16).view(R, MI),
                    ws[off_prod:off_prod + R * H * 2].view(BF16).view(R, H)))
    return res[0] if len(res) == 1 else tuple(res)


def moe_experts(x2, logits, exp_gu, exp_dn, topk, shared=None, shared_gate=None):
    """Expert block of ``FnLayer._moe``: decode kernels for <= 4 tokens, grouped
    prefill otherwise. ``shared_gate`` (decode) applies the sigmoid-gated
    shared merge; for prefill pass the already gated ``shared`` output."""
    if x2.shape[0] <= DECODE_MAX_TOKENS:
        return moe_decode(x2, logits, exp_gu, exp_dn, topk, shared, shared_gate)[0]
    if shared_gate is not None:
        raise RuntimeError("prefill takes the already gated shared-expert output")
    return moe_prefill(x2, logits, exp_gu, exp_dn, topk, shared)
