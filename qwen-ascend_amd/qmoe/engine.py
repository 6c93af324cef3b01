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
import os

import torch

from . import _lib
from .ops import grouped_matmul, route_group, router_topk, weight_quant_batchmatmul

BF16 = torch.bfloat16
DECODE_MAX_TOKENS = 4
_CHECK_DECODE = os.environ.get("QMOE_DECODE_CHECK", "0") == "1"


class ExpW4:
    """Per-group W4A16 expert weights (int4pack) with a bf16 scale cache.

    Interface of the reference container (``fnx/engine.py:619-753``): the
    constructor ``(w4, s8t, base, gs, expert_major=False)``, the attributes
    ``w4, s8t, base, _scales, K, N, E, G, gs, expert_major`` and the methods
    ``apply``, ``apply_diag``, ``apply_grouped``, ``_wcat`` and ``_scat``, so
    ``FnLayer._moe`` calls it unchanged.

    Storage: ``w4`` is int32 int4pack ``[K, E, N/8]`` (K-major artifact) or
    ``[E, K, N/8]`` (``expert_major``); the scale cache ``_scales`` is bf16
    ``[E, G, N]`` in both cases, composed on the GPU from ``s8t`` int8
    ``[G, E, N]`` and ``base`` bf16 ``[E, N]`` (``qmoe_scale_cache``), after
    which ``s8t``/``base`` are dropped as the reference's cached mode does.
    Every method runs HIP kernels: the selection of k experts is one gather
    launch for either layout, the diagonal down projection is a grouped GEMM
    over one-row tiles that reads the experts in place, and the grouped
    prefill GEMM reads all experts in place.
    """

    __slots__ = ("_w4", "s8t", "base", "K", "N", "E", "G", "gs", "expert_major", "_scales", "_dtile",
                 "_dtile_failed")

    def __init__(self, w4, s8t, base, gs, expert_major=False):
        if w4.dtype != torch.int32 or w4.dim() != 3:
            raise ValueError("w4 must be int32 int4pack [K, E, N/8] or [E, K, N/8]")
        self._dtile = None
        self._dtile_failed = False
        self._w4 = w4
        self.expert_major = bool(expert_major)
        outer, inner, words = w4.shape
        self.E, self.K = (outer, inner) if self.expert_major else (inner, outer)
        self.N = 8 * words
        self.gs = int(gs)
        if self.gs <= 0 or self.K % self.gs:
            raise ValueError(f"K {self.K} is not a multiple of the group size {self.gs}")
        self.G = self.K // self.gs
        self.s8t = self.base = None
        self._scales = None
        self._dtile = None
        self._dtile_failed = False
        if s8t is not None:
            if tuple(s8t.shape) != (self.G, self.E, self.N) or tuple(base.shape) != (self.E, self.N):
                raise ValueError("s8t must be [G, E, N] and base [E, N]")
            self._scales = _compose_scales(s8t, base)

    @classmethod
    def from_scales(cls, w4_em, scales_em):
        """Expert-major int4pack [E, K, N/8] with bf16 scales [E, G, N] given directly."""
        E, K = w4_em.shape[0], w4_em.shape[1]
        G = scales_em.shape[1]
        if scales_em.dim() != 3 or scales_em.shape[0] != E or K % G:
            raise ValueError("scales must be [E, G, N] with G dividing K")
        obj = cls(w4_em, None, None, K // G, expert_major=True)
        obj._scales = scales_em
        return obj

    @property
    def w4(self):
        return self._w4

    @w4.setter
    def w4(self, t):
        """Rebinding the weights drops their decode tiles (built again on request)."""
        self._w4 = t
        self._dtile = None
        self._dtile_failed = False

    def cached_decode_tiles(self, kind):
        """The decode tiles built earlier by :meth:`decode_tiles`, or None: tiles
        are never built here. Tiles of a ``w4`` that was rebound, moved or
        changed in place since (tensor version) are dropped, not returned."""
        t = self._dtile
        if t is None:
            return None
        if t[0] != kind:
            raise ValueError(f"decode tiles of these weights were built as {t[0]!r}")
        w = self._w4
        if t[2] != (w.data_ptr(), w.untyped_storage().data_ptr(), w._version):
            self._dtile = None
            return None
        return t[1]

    def decode_tiles(self, kind):
        """Build (once) and return the decode-tile copy of these expert-major
        weights: the order in which the one-token decode launch's workgroups
        read them (``qmoe_decode_tiles_gate_up`` / ``_down``), kind
        ``"gate_up"`` for ``[E, H, 2MI/8]`` weights (tiled for this
        container's group size) or ``"down"`` for ``[E, MI, H/8]``.

        Opt-in: the decode reads them only once they exist (build them at
        load time, outside graph capture). They are a second copy the size of
        ``w4``: 0.75 GiB per 512-expert layer at H2048/MI512 and 1.17 GiB at
        the reference model's H2560/MI640, for 11.25 against 11.8 us per
        one-token layer. None for shapes that launch does not take (H not a
        multiple of 256, MI not of 128), for K-major weights, under graph
        capture, and when the device has no memory for the copy (the decode
        then reads ``w4``). After an in-place update of ``w4`` they are built
        again on the next request; a graph captured before keeps reading the
        old copy and must be captured again."""
        if kind not in ("gate_up", "down"):
            raise ValueError("kind is 'gate_up' or 'down'")
        t = self.cached_decode_tiles(kind)
        if t is not None or self._dtile_failed:
            return t
        if not self.expert_major:
            return None
        H, MI = (self.K, self.N // 2) if kind == "gate_up" else (self.N, self.K)
        if H < 256 or H % 256 or MI < 128 or MI % 128 or torch.cuda.is_current_stream_capturing():
            return None
        w = self._w4
        try:
            t = torch.empty_like(w)
        except torch.OutOfMemoryError:
            self._dtile_failed = True
            return None
        L, st = _lib.lib(), _lib.stream_of(w)
        if kind == "gate_up":
            rc = L.qmoe_decode_tiles_gate_up(w.data_ptr(), t.data_ptr(), self.E, H, MI, self.gs, st)
        else:
            rc = L.qmoe_decode_tiles_down(w.data_ptr(), t.data_ptr(), self.E, H, MI, st)
        _lib.check(rc, "decode tiles")
        self._dtile = (kind, t, (w.data_ptr(), w.untyped_storage().data_ptr(), w._version))
        return t

    # ---- selection of k experts (the operator's K-major concatenation)
    def _select(self, ids):
        """(weights int32 [K, k*N/8], scales bf16 [G, k*N]) of experts ids, in ids order."""
        ids = ids.reshape(-1).to(torch.int64).contiguous()
        k = ids.numel()
        dev = self.w4.device
        ow = torch.empty((self.K, k * self.N // 8), dtype=torch.int32, device=dev)
        osc = torch.empty((self.G, k * self.N), dtype=BF16, device=dev)
        entry = "qmoe_expert_gather" if self.expert_major else "qmoe_expert_gather_kmajor"
        _lib.check(getattr(_lib.lib(), entry)(self.w4.data_ptr(), self._scales.data_ptr(), ids.data_ptr(),
                                              ow.data_ptr(), osc.data_ptr(), self.K, self.G, self.N, self.E, k,
                                              _lib.stream_of(self.w4)), "expert selection")
        return ow, osc

    def _wcat(self, ids):
        return self._select(ids)[0]

    def _scat(self, ids):
        return self._select(ids)[1]

    def apply(self, x, ids):
        """x [M, K] bf16, ids [k] -> [M, k*N]: every row against the k experts
        concatenated along N (one W4A16 GEMM)."""
        ow, osc = self._select(ids)
        return weight_quant_batchmatmul(x, ow, osc, antiquant_group_size=self.gs)

    def apply_diag(self, x, ids):
        """Row j of x [k, K] against expert ids[j] only -> [k, N].

        Expert-major: a grouped GEMM whose k one-row tiles name the experts
        directly (no weight copy, no Cartesian product). K-major: the
        Cartesian product and its diagonal blocks."""
        k = x.shape[0]
        if ids.numel() != k:
            raise ValueError("apply_diag takes one expert id per activation row")
        if not self.expert_major:
            full = self.apply(x, ids).view(k, k, self.N)
            return torch.diagonal(full, dim1=0, dim2=1).t().contiguous()
        if x.dtype != BF16 or x.dim() != 2 or x.shape[1] != self.K:
            raise RuntimeError("x must be bf16 [k, K]")
        ids = ids.reshape(-1).to(torch.int64).contiguous()
        x = x.contiguous()
        dev = x.device
        L = _lib.lib()
        st = _lib.stream_of(x)
        tiles = torch.empty((3 * k + 1,), dtype=torch.int32, device=dev)
        te, tr0, trows, tcnt = tiles[:k], tiles[k:2 * k], tiles[2 * k:3 * k], tiles[3 * k:]
        _lib.check(L.qmoe_tiles_from_ids(ids.data_ptr(), k, self.E, te.data_ptr(), tr0.data_ptr(), trows.data_ptr(),
                                         tcnt.data_ptr(), st), "apply_diag tiles")
        y = torch.empty((k, self.N), dtype=BF16, device=dev)
        ws = _lib.workspace(dev, L.qmoe_grouped_gemm_workspace(k, self.K))
        _lib.check(L.qmoe_grouped_gemm(x.data_ptr(), k, self.K, self.N, self.E, self.gs, self.w4.data_ptr(),
                                       self._scales.data_ptr(), te.data_ptr(), tr0.data_ptr(), trows.data_ptr(),
                                       tcnt.data_ptr(), k, y.data_ptr(), ws.data_ptr(), ws.numel(), st),
                   "apply_diag")
        return y

    def apply_grouped(self, x, group_ends, host_ends=None):
        """Rows sorted by expert (``group_ends`` inclusive cumsum) through one
        grouped GEMM over all experts in place. ``host_ends`` is accepted for
        the reference's signature; the GPU kernel needs no workspace bound,
        so it is not used."""
        if not self.expert_major:
            raise RuntimeError("grouped prefill requires the expert-major artifact")
        return grouped_matmul([x], [self.w4], antiquant_scale=[self._scales], group_list=group_ends,
                              split_item=3, group_type=0, output_dtype=BF16)[0]


def _compose_scales(s8t, base):
    """bf16 [E, G, N] scale cache of an (s8t [G, E, N], base [E, N]) artifact."""
    G, E, N = s8t.shape
    if s8t.dtype != torch.int8 or base.dtype != BF16:
        raise ValueError("s8t must be int8 and base bfloat16")
    if s8t.device.type != "cuda" or base.device != s8t.device:
        raise RuntimeError("the ExpW4 scale cache is built by a HIP kernel: s8t and base must be device tensors")
    s8t, base = s8t.contiguous(), base.contiguous()
    out = torch.empty((E, G, N), dtype=BF16, device=s8t.device)
    _lib.check(_lib.lib().qmoe_scale_cache(s8t.data_ptr(), base.data_ptr(), out.data_ptr(), G, E, N,
                                           _lib.stream_of(s8t)), "scale cache")
    return out


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


def moe_decode(x, logits, exp_gu, exp_dn, topk, shared=None, shared_gate=None, return_intermediates=False,
               counters=None, tiles=None):
    """Fused decode expert block for 1..4 tokens (one launch).

    x bf16 [B, H]; logits bf16 [B, E]. Returns (out bf16 [B, H], idx int64
    [B, topk], w bf16 [B, topk]). With ``shared``/``shared_gate`` (bf16 [B, H]
    / [B, 1]) the shared-expert merge of ``fnx/engine.py:1874-1891`` is
    applied in the same epilogue. ``counters`` is the per-device array by
    default; calls overlapping on another stream pass their own
    (``_lib.new_counters``). With ``return_intermediates`` the launch also
    writes inspection copies (act rows and weighted products) to a workspace.
    With ``QMOE_DECODE_CHECK=1`` in the environment every call synchronises
    and raises if one of its bounded waits timed out; without it the first
    eager call on each counters array does so once. ``tiles``: None reads the
    experts' decode tiles where they have been built (``ExpW4.decode_tiles``),
    True builds them first (outside graph capture; a second copy of the
    weights), False reads ``w4`` only; one token or, up to 512 experts,
    several read the tiles, and the bits are the same either way.
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
    ncnt = L.qmoe_moe_decode_counters(B, topk, H, MI)
    if ncnt < 0:
        raise RuntimeError("moe_decode: shape too large for the decode counters")
    if counters is None:
        cnt = _lib.counters(dev, ncnt)
    else:
        if counters.dtype != torch.int32 or counters.numel() < ncnt or counters.device != dev:
            raise RuntimeError(f"counters must be int32 with at least {ncnt} slots on {dev}")
        cnt = counters
    ws = _lib.workspace(dev, L.qmoe_moe_decode_workspace(B, topk, H, MI)) if return_intermediates else None
    sh = shared.contiguous() if shared is not None else None
    sg = shared_gate.contiguous() if shared_gate is not None else None
    gu_t, dn_t = _tiles_for(exp_gu, exp_dn, tiles) if (B == 1 or exp_gu.E <= 512) else (None, None)
    args = (out.data_ptr(), idx.data_ptr(), w.data_ptr(), B, exp_gu.E, topk, H, MI, exp_gu.gs, exp_dn.gs,
            _lib.ptr(ws), 0 if ws is None else ws.numel(), cnt.data_ptr(), _lib.stream_of(x))
    if gu_t is not None and dn_t is not None:
        rc = L.qmoe_moe_decode_tiled(x.data_ptr(), logits.data_ptr(), exp_gu.w4.data_ptr(),
                                     exp_gu._scales.data_ptr(), exp_dn.w4.data_ptr(), exp_dn._scales.data_ptr(),
                                     gu_t.data_ptr(), dn_t.data_ptr(), _lib.ptr(sh), _lib.ptr(sg), *args)
    else:
        rc = L.qmoe_moe_decode(x.data_ptr(), logits.data_ptr(), exp_gu.w4.data_ptr(), exp_gu._scales.data_ptr(),
                               exp_dn.w4.data_ptr(), exp_dn._scales.data_ptr(), _lib.ptr(sh), _lib.ptr(sg), *args)
    _lib.check(rc, "moe_decode")
    _first_call_check(cnt, "moe_decode")
    if return_intermediates:
        return out, idx, w, _decode_intermediates(ws, B, topk, H, MI)
    return out, idx, w


def _tiles_for(exp_gu, exp_dn, tiles):
    """(gate_up tiles, down tiles) for a decode call, both or neither: built on
    request (tiles=True), the ones built earlier (None), none (False)."""
    if tiles is False:
        return None, None
    get = (lambda e, kind: e.decode_tiles(kind)) if tiles else (lambda e, kind: e.cached_decode_tiles(kind))
    gu_t = get(exp_gu, "gate_up")
    dn_t = get(exp_dn, "down") if gu_t is not None else None
    return (gu_t, dn_t) if dn_t is not None else (None, None)


_CHECKED_COUNTERS: set = set()


def _first_call_check(cnt, what):
    """Error flag of a counters array after its first eager decode call (once
    per array; every call with QMOE_DECODE_CHECK=1): a bounded wait that timed
    out means that call's output is wrong. One synchronisation per array."""
    key = (cnt.data_ptr(), cnt.numel())
    if not _CHECK_DECODE and key in _CHECKED_COUNTERS:
        return
    if torch.cuda.is_current_stream_capturing():
        return
    _CHECKED_COUNTERS.add(key)
    if _lib.decode_status(cnt):
        raise RuntimeError(f"{what}: a bounded wait timed out; this call's output is wrong")


def decode_status(device=None, counters=None, clear=True):
    """1 if a decode call on this device's counters array (or on ``counters``)
    had a bounded wait time out since the flag was last cleared, else 0.
    Synchronises; call outside graph capture."""
    if counters is None:
        dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        counters = _lib.counters(dev)
    return _lib.decode_status(counters, clear)


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
