"""Drop-in replacements for the Ascend-only operators on the MoE expert path.

* :func:`weight_quant_batchmatmul` — ``torch_npu.npu_weight_quant_batchmatmul``
  (per-group W4A16, ``fnx/engine.py:698-701``).
* :func:`grouped_matmul` — ``torch_npu.npu_grouped_matmul`` with
  ``split_item=3, group_type=0`` (``fnx/engine.py:712-716, 744-753``).
* :func:`swiglu` — ``npu_swiglu(gu.float(), dim=-1).to(torch.bfloat16)``
  (``fnx/engine.py:1827, 1866``).
* :func:`router_topk`, :func:`route_group` — the router and grouping glue of
  ``FnLayer._moe`` (``fnx/engine.py:1810-1823, 1832-1843``) on the GPU.

All launch HIP kernels from libqmoe.so on the current stream, allocate only
through torch, and never synchronise, so they can be captured in a graph.
"""
from __future__ import annotations

import torch

from . import _lib

BF16 = torch.bfloat16


def _cuda(*ts):
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("qmoe ops take device tensors")


def _same_device(*ts):
    dev = ts[0].device
    for t in ts[1:]:
        if t is not None and t.device != dev:
            raise RuntimeError("all tensors must be on the same device")


def weight_quant_batchmatmul(x, weight, antiquant_scale, antiquant_offset=None, quant_scale=None,
                             quant_offset=None, bias=None, antiquant_group_size=0):
    """y[M,N] = bf16(x[M,K] @ dequant(weight, antiquant_scale)) with fp32 accumulation.

    weight: int4pack int32 [K, N/8] (nibble j of word c = column 8c+j, low
    first, two's complement), or int8 [K, N] (the W8A16 form the dense
    projections use, ``fnx/engine.py:358-364``); antiquant_scale: bf16
    [K/gs, N]; x: 2-D bf16.
    Same argument order as ``torch_npu.npu_weight_quant_batchmatmul``; the
    symmetric per-group form is the one the reference uses
    (``fnx/engine.py:698-701``), so offsets, quant scales and bias must be
    None, and the scale dtype must equal x's (``…第37轮实测记录.md:19-30``).
    """
    if antiquant_offset is not None or quant_scale is not None or quant_offset is not None or bias is not None:
        raise RuntimeError("only symmetric per-group W4A16 (no offset/quant/bias) is supported")
    if x.dim() != 2:
        raise RuntimeError("x must be 2-D [M, K]")
    if x.dtype != BF16 or antiquant_scale.dtype != x.dtype:
        raise RuntimeError("x and antiquant_scale must both be bfloat16")
    if weight.dtype not in (torch.int32, torch.int8) or weight.dim() != 2:
        raise RuntimeError("weight must be int4pack int32 [K, N/8] or int8 [K, N]")
    _cuda(x, weight, antiquant_scale)
    _same_device(x, weight, antiquant_scale)
    M, K = x.shape
    if weight.dtype == torch.int8:
        return _w8a16(x, weight, antiquant_scale, int(antiquant_group_size))
    N = weight.shape[1] * 8
    gs = int(antiquant_group_size)
    if weight.shape[0] != K or gs <= 0 or K % gs or antiquant_scale.shape != (K // gs, N):
        raise RuntimeError(f"shape mismatch: x {tuple(x.shape)} weight {tuple(weight.shape)} "
                           f"scale {tuple(antiquant_scale.shape)} gs {gs}")
    x = x.contiguous()
    weight = weight.contiguous()
    antiquant_scale = antiquant_scale.contiguous()
    y = torch.empty((M, N), dtype=BF16, device=x.device)
    if M == 0:
        return y
    L = _lib.lib()
    st = _lib.stream_of(x)
    if M <= 4:
        ncnt = L.qmoe_w4a16_gemm_counters(M, K, N)
        if ncnt < 0:
            raise RuntimeError("weight_quant_batchmatmul: shape too large for the counters array")
        rc = L.qmoe_w4a16_gemv(x.data_ptr(), weight.data_ptr(), antiquant_scale.data_ptr(), y.data_ptr(),
                               M, K, N, gs, None, 0, _lib.counters(x.device, ncnt).data_ptr(), st)
    else:
        ws = _lib.workspace(x.device, L.qmoe_w4a16_gemm_mfma_workspace(M, K))
        rc = L.qmoe_w4a16_gemm_mfma(x.data_ptr(), weight.data_ptr(), antiquant_scale.data_ptr(), y.data_ptr(),
                                    M, K, N, gs, ws.data_ptr(), ws.numel(), st)
    _lib.check(rc, "weight_quant_batchmatmul")
    return y


def _w8a16(x, weight, scale, gs):
    """The int8 weight form of :func:`weight_quant_batchmatmul`."""
    M, K = x.shape
    N = weight.shape[1]
    if weight.shape[0] != K or gs <= 0 or K % gs or scale.shape != (K // gs, N):
        raise RuntimeError(f"shape mismatch: x {tuple(x.shape)} weight {tuple(weight.shape)} "
                           f"scale {tuple(scale.shape)} gs {gs}")
    x, weight, scale = x.contiguous(), weight.contiguous(), scale.contiguous()
    y = torch.empty((M, N), dtype=BF16, device=x.device)
    if M == 0:
        return y
    L = _lib.lib()
    st = _lib.stream_of(x)
    if M <= 4:
        ws = _lib.workspace(x.device, L.qmoe_w8a16_gemv_workspace(M, K, N))
        rc = L.qmoe_w8a16_gemv(x.data_ptr(), weight.data_ptr(), scale.data_ptr(), y.data_ptr(), M, K, N, gs,
                               ws.data_ptr(), ws.numel(), _lib.counters(x.device).data_ptr(), st)
    else:
        rc = L.qmoe_w8a16_gemm_mfma(x.data_ptr(), weight.data_ptr(), scale.data_ptr(), y.data_ptr(), M, K, N, gs,
                                    st)
    _lib.check(rc, "weight_quant_batchmatmul (int8)")
    return y


def _tile_table(R, E, device):
    L = _lib.lib()
    bm = L.qmoe_gemm_tile_rows()
    mt = L.qmoe_max_row_tiles(R, E, bm)
    tiles = torch.empty((3 * mt + 1,), dtype=torch.int32, device=device)
    return bm, mt, tiles


def grouped_matmul(x, weight, *, bias=None, scale=None, offset=None, antiquant_scale=None,
                   antiquant_offset=None, per_token_scale=None, group_list=None, activation_input=None,
                   activation_quant_scale=None, activation_quant_offset=None, split_item=0, group_type=None,
                   group_list_type=0, act_type=0, output_dtype=None, tuning_config=None):
    """Expert-major grouped W4A16 GEMM, the reference's GroupedMatmulV5 call.

    ``x=[rows [R,K] bf16]``, ``weight=[int4pack int32 [E,K,N/8]]``,
    ``antiquant_scale=[bf16 [E,G,N]]``, ``group_list`` = int64 [E] inclusive
    cumulative row counts (``group_list_type=0``), ``split_item=3``,
    ``group_type=0`` -> ``[y [R,N] bf16]``. Rows of expert e are
    ``[group_list[e-1], group_list[e])``; empty experts are allowed and rows
    past ``group_list[-1]`` are left unwritten. Any contiguous tensor is
    accepted (no storage-offset restriction).
    """
    unsupported = (bias, scale, offset, antiquant_offset, per_token_scale, activation_input,
                   activation_quant_scale, activation_quant_offset)
    if any(u is not None for u in unsupported) or act_type:
        raise RuntimeError("only the W4A16 antiquant form of grouped_matmul is supported")
    if split_item != 3 or group_type != 0 or group_list_type != 0:
        raise RuntimeError("supported: split_item=3, group_type=0, group_list_type=0")
    if output_dtype not in (None, BF16):
        raise RuntimeError("output_dtype must be bfloat16")
    if len(x) != 1 or len(weight) != 1 or antiquant_scale is None or len(antiquant_scale) != 1:
        raise RuntimeError("x, weight and antiquant_scale must be one-element lists")
    xt, w, s = x[0], weight[0], antiquant_scale[0]
    if xt.dim() != 2 or xt.dtype != BF16 or w.dtype != torch.int32 or w.dim() != 3 or s.dtype != BF16:
        raise RuntimeError("expect x [R,K] bf16, weight [E,K,N/8] int32, antiquant_scale [E,G,N] bf16")
    gl = group_list
    if gl is None or gl.dtype != torch.int64 or gl.dim() != 1 or gl.numel() != w.shape[0]:
        raise RuntimeError("group_list must be int64 [E]")
    _cuda(xt, w, s, gl)
    _same_device(xt, w, s, gl)
    R, K = xt.shape
    E, Kw, nw = w.shape
    N = nw * 8
    if Kw != K or s.shape[0] != E or s.shape[2] != N or K % s.shape[1]:
        raise RuntimeError("shape mismatch between x, weight and antiquant_scale")
    gs = K // s.shape[1]
    xt, w, s, gl = xt.contiguous(), w.contiguous(), s.contiguous(), gl.contiguous()
    y = torch.empty((R, N), dtype=BF16, device=xt.device)
    if R == 0:
        return [y]
    L = _lib.lib()
    st = _lib.stream_of(xt)
    bm, mt, tiles = _tile_table(R, E, xt.device)
    te, tr0, trows, tcount = tiles[:mt], tiles[mt:2 * mt], tiles[2 * mt:3 * mt], tiles[3 * mt:]
    _lib.check(L.qmoe_tiles_from_ends(gl.data_ptr(), E, R, bm, te.data_ptr(), tr0.data_ptr(),
                                      trows.data_ptr(), tcount.data_ptr(), st), "grouped_matmul tiles")
    ws = _lib.workspace(xt.device, L.qmoe_grouped_gemm_workspace(R, K))
    _lib.check(L.qmoe_grouped_gemm(xt.data_ptr(), R, K, N, E, gs, w.data_ptr(), s.data_ptr(), te.data_ptr(),
                                   tr0.data_ptr(), trows.data_ptr(), tcount.data_ptr(), mt, y.data_ptr(),
                                   ws.data_ptr(), ws.numel(), st), "grouped_matmul")
    return [y]


def swiglu(gu):
    """act = bf16(silu(fp32 g) * fp32 u) for gu = [g | u] bf16 [..., 2*MI].

    Replaces ``torch_npu.npu_swiglu(gu.float(), dim=-1).to(torch.bfloat16)``
    and its torch twin (``fnx/engine.py:1827-1829, 1866-1868``).
    """
    if gu.dtype != BF16 or gu.shape[-1] % 2:
        raise RuntimeError("swiglu expects bf16 [..., 2*MI]")
    _cuda(gu)
    gu = gu.contiguous()
    mi = gu.shape[-1] // 2
    rows = gu.numel() // gu.shape[-1]
    act = torch.empty(gu.shape[:-1] + (mi,), dtype=BF16, device=gu.device)
    _lib.check(_lib.lib().qmoe_swiglu(gu.data_ptr(), act.data_ptr(), rows, mi, _lib.stream_of(gu)), "swiglu")
    return act


def router_topk(logits, k):
    """(idx int64 [T,k], w bf16 [T,k]) = top-k of softmax(fp32 logits), renormalised.

    ``fnx/engine.py:1810-1813``. Ties in logits go to the lower expert id.
    """
    if logits.dim() != 2 or logits.dtype != BF16:
        raise RuntimeError("logits must be bf16 [T, E]")
    _cuda(logits)
    logits = logits.contiguous()
    T, E = logits.shape
    idx = torch.empty((T, k), dtype=torch.int64, device=logits.device)
    w = torch.empty((T, k), dtype=BF16, device=logits.device)
    if T:
        _lib.check(_lib.lib().qmoe_router_topk(logits.data_ptr(), idx.data_ptr(), w.data_ptr(), T, E, k,
                                               _lib.stream_of(logits)), "router_topk")
    return idx, w


def route_group(idx, E, with_tiles=False):
    """Expert-major grouping of routed ids (``fnx/engine.py:1816-1823, 1832-1843``).

    Returns (counts, ends, order, inverse) int64 — ends is the inclusive
    cumsum (``group_list``), order the stable expert-major permutation of the
    flat ids, inverse[order[p]] = p. With ``with_tiles`` also the grouped
    GEMM row-tile table (tile tensor, max tiles).
    """
    if idx.dtype != torch.int64:
        raise RuntimeError("ids must be int64")
    _cuda(idx)
    ids = idx.contiguous().view(-1)
    R = ids.numel()
    dev = ids.device
    counts = torch.empty((E,), dtype=torch.int64, device=dev)
    ends = torch.empty((E,), dtype=torch.int64, device=dev)
    order = torch.empty((R,), dtype=torch.int64, device=dev)
    inverse = torch.empty((R,), dtype=torch.int64, device=dev)
    L = _lib.lib()
    bm, mt, tiles = _tile_table(R, E, dev)
    ws = _lib.workspace(dev, L.qmoe_route_group_workspace(R, E))
    te, tr0, trows, tcount = tiles[:mt], tiles[mt:2 * mt], tiles[2 * mt:3 * mt], tiles[3 * mt:]
    _lib.check(L.qmoe_route_group(ids.data_ptr(), R, E, counts.data_ptr(), ends.data_ptr(), order.data_ptr(),
                                  inverse.data_ptr(), bm, te.data_ptr(), tr0.data_ptr(), trows.data_ptr(),
                                  tcount.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(ids)),
               "route_group")
    if with_tiles:
        return counts, ends, order, inverse, tiles, mt
    return counts, ends, order, inverse
