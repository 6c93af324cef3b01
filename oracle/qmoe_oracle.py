"""CPU oracle for the W4A16 MoE expert path — TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the arithmetic of xyzhou613-dev/qwen-ascend's
quantized-MoE expert path so the HIP kernels can be checked against it. It is
never shipped or called by the product path: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import it,
and only as the checker (or, for the bench, as the timed CPU port).

Every function cites the reference file:line it follows. bf16 values are held
as ``uint16`` bit patterns (``*_bits``) or as float32 arrays that are exactly
representable in bf16. Rounding to bf16 is round-to-nearest-even, the rounding
``torch.Tensor.to(torch.bfloat16)`` and the AscendC ``CAST_RINT`` casts use.

Parity pinning (what checks each function besides re-typing it) lives in
``tests/test_oracle.py``; every function here is pinned by at least one
known-answer vector, closed form, invariant or brute-force check there.
"""
from __future__ import annotations

import numpy as np

# --------------------------------------------------------------------------
# bf16 <-> fp32
# --------------------------------------------------------------------------


def f32_to_bf16_bits(a) -> np.ndarray:
    """Round float32 values to bf16 (nearest-even), return uint16 bit patterns.

    Same rounding as ``torch.Tensor.to(torch.bfloat16)`` used throughout
    ``fnx/engine.py`` (e.g. 1812, 1827) and ``Cast(..., CAST_RINT)`` in
    ``kernels/reduce/reduce.cpp:51``. NaN stays NaN (quiet bit forced).
    """
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16))
    out = r.astype(np.uint16)
    nan = np.isnan(a)
    if nan.any():
        out[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return out


def bf16_bits_to_f32(b) -> np.ndarray:
    """Widen bf16 bit patterns (uint16/int16) to float32 exactly."""
    b = np.ascontiguousarray(b).view(np.uint16)
    return (b.astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(a) -> np.ndarray:
    """float32 -> nearest bf16 value, returned as float32."""
    return bf16_bits_to_f32(f32_to_bf16_bits(a))


# --------------------------------------------------------------------------
# int4pack (the W4A16 weight container) and the LQP v2o layout
# --------------------------------------------------------------------------


def pack_int4(q) -> np.ndarray:
    """Signed int4 values [..., K, N] (-8..7) -> int4pack int32 [..., K, N/8].

    Packs along the LAST axis N: nibble j (bits 4j..4j+3, low nibble first) of
    word m holds element 8m+j, two's complement. Follows the packer in
    ``ops/scripts/r37_w4a16_semantics.py:69-76`` (``(v & 0xF) << 4j`` over
    ``u[..., j::8]``) and the container of ``npu_convert_weight_to_int4pack``
    as used by ``tools/repack_w4a16.py:70`` ([K,N] -> [K,N/8]).
    """
    q = np.asarray(q)
    if q.shape[-1] % 8:
        raise ValueError("last axis must be a multiple of 8")
    if q.size and (q.min() < -8 or q.max() > 7):
        raise ValueError("int4 values must lie in [-8, 7]")
    u = (q.astype(np.int64) & 0xF).astype(np.uint32)
    out = np.zeros(q.shape[:-1] + (q.shape[-1] // 8,), dtype=np.uint32)
    for j in range(8):
        out |= u[..., j::8] << np.uint32(4 * j)
    return out.view(np.int32)


def unpack_int4(w) -> np.ndarray:
    """int4pack int32 [..., K, N/8] -> int8 [..., K, N] in -8..7.

    Inverse of :func:`pack_int4`; the read side matches the byte addressing
    of the reference's direct K-major kernel,
    ``experiments/r156-moe-kmajor/w4_kmajor.cpp:30,33`` (byte k*N/2 + n/2,
    ``int4b_t`` low nibble = even n).
    """
    w = np.ascontiguousarray(w).view(np.uint32)
    out = np.empty(w.shape[:-1] + (w.shape[-1] * 8,), dtype=np.int8)
    for j in range(8):
        nib = ((w >> np.uint32(4 * j)) & np.uint32(0xF)).astype(np.int16)
        out[..., j::8] = ((nib ^ 8) - 8).astype(np.int8)
    return out


def pack_v2o(q) -> np.ndarray:
    """int8 [E, N, K] (-8..7) -> LQP v2o offset-binary uint8 [E, N, K/2].

    Per 128-wide K segment s, byte 64s+j holds W[128s+j] in the low nibble and
    W[128s+64+j] in the high nibble, each stored as value+8.
    ``tools/repack_v2.py:39-54`` (``pack_v2_ob``); layout described in
    ``tools/layout_v2_check.py:4-9``.
    """
    q = np.asarray(q)
    E, N, K = q.shape
    if K % 128:
        raise ValueError("K must be a multiple of 128 for v2o")
    v = q.reshape(E, N, K // 128, 2, 64).astype(np.int16) + 8
    if v.size and (v.min() < 0 or v.max() > 15):
        raise ValueError("int4 values must lie in [-8, 7]")
    lo = v[:, :, :, 0, :].astype(np.uint8)
    hi = v[:, :, :, 1, :].astype(np.uint8)
    return (lo | (hi << np.uint8(4))).reshape(E, N, K // 2)


def unpack_v2o(p) -> np.ndarray:
    """LQP v2o uint8 [E, N, K/2] -> int8 [E, N, K]; ``tools/repack_w4a16.py:41-55``."""
    p = np.asarray(p, dtype=np.uint8)
    E, N, half = p.shape
    K = half * 2
    s = K // 128
    b = p.astype(np.int16)
    out = np.empty((E, N, s, 2, 64), dtype=np.int8)
    out[..., 0, :] = ((b & 15) - 8).reshape(E, N, s, 64)
    out[..., 1, :] = ((b >> 4) - 8).reshape(E, N, s, 64)
    return out.reshape(E, N, K)


def compose_scales(s8t, base_bits) -> np.ndarray:
    """LQP scale pair -> expert-major bf16 scales [E, G, N] (bit patterns).

    ``_scales = bf16(s8t.permute(1,0,2).to(bf16) * base[:, None, :])``,
    ``fnx/engine.py:653-659``. s8t is int8 [G, E, N]; base is bf16 [E, N].
    int8 -> bf16 is exact, so this is one bf16 rounding of the fp32 product.
    """
    s8 = np.asarray(s8t, dtype=np.int8).transpose(1, 0, 2).astype(np.float32)
    base = bf16_bits_to_f32(base_bits)[:, None, :]
    return f32_to_bf16_bits(s8 * base)


def lqp_to_em(v2o, s8, base_fp16):
    """LQP v2o artifact -> expert-major int4pack + composed bf16 scales.

    The chain ``tools/repack_w4a16.py:58-76`` (unpack v2o, transpose to
    [K,N], int4pack along N, s8 -> s8t, base fp16 -> bf16) followed by
    ``tools/repack_w4_em.py:16`` ([K,E,N/8] -> [E,K,N/8]) and the scale cache
    ``fnx/engine.py:653-659``. Inputs: v2o uint8 [E,N,K/2], s8 int8 [E,N,G],
    base fp16 [E,N]. Returns (w4 int32 [E,K,N/8], s8t int8 [G,E,N],
    base bf16 bits [E,N], scales bf16 bits [E,G,N]).
    """
    q = unpack_v2o(v2o)                                   # [E,N,K]
    w4 = pack_int4(np.ascontiguousarray(q.transpose(0, 2, 1)))   # [E,K,N/8]
    s8t = np.ascontiguousarray(np.asarray(s8, dtype=np.int8).transpose(2, 0, 1))
    base_bits = f32_to_bf16_bits(np.asarray(base_fp16, dtype=np.float16).astype(np.float32))
    return w4, s8t, base_bits, compose_scales(s8t, base_bits)


# --------------------------------------------------------------------------
# Per-expert loops
# --------------------------------------------------------------------------

_WORKERS = 1


def set_workers(n: int) -> int:
    """Threads over which the per-expert loops below run (default 1). Each
    expert's rows are computed on their own and written to rows no other
    expert touches, so results do not depend on n (numpy releases the GIL in
    its array loops, and BLAS is held to one thread per call meanwhile).
    Returns the previous value."""
    global _WORKERS
    prev, _WORKERS = _WORKERS, max(1, int(n))
    return prev


def _each_expert(fn, experts):
    """fn(e) for every expert e (independent calls with disjoint outputs)."""
    experts = [int(e) for e in experts]
    if _WORKERS <= 1 or len(experts) < 2:
        for e in experts:
            fn(e)
        return
    from concurrent.futures import ThreadPoolExecutor
    try:
        from threadpoolctl import threadpool_limits
        limit = threadpool_limits(1)
    except ImportError:  # pragma: no cover - threadpoolctl ships with the image
        limit = None
    try:
        with ThreadPoolExecutor(_WORKERS) as ex:
            for _ in ex.map(fn, experts):
                pass
    finally:
        if limit is not None:
            limit.restore_original_limits()


# --------------------------------------------------------------------------
# W4A16 GEMM (npu_weight_quant_batchmatmul) and grouped GEMM (GroupedMatmulV5)
# --------------------------------------------------------------------------


def dequant(w4, scale_bits, gs) -> np.ndarray:
    """int4pack [K, N/8] + bf16 scales [G, N] -> exact fp32 weights [K, N].

    W[k, n] = q[k, n] * S[k // gs, n]: per-group, per-column, symmetric, no
    zero point (``fnx/engine.py:247-252`` ``deq``; operator contract in
    ``docs/Qwen3.8-Flash-Next-第37轮实测记录.md:19-30``). q has <= 4 significant
    bits and S 8, so the fp32 product is exact (no bf16 rounding of weights).
    """
    q = unpack_int4(w4).astype(np.float32)
    K = q.shape[0]
    s = bf16_bits_to_f32(scale_bits)
    if s.shape[0] * gs != K:
        raise ValueError(f"scale groups {s.shape[0]} x gs {gs} != K {K}")
    return q * np.repeat(s, gs, axis=0)


def w4a16_gemm(x_bits, w4, scale_bits, gs) -> np.ndarray:
    """y[M,N] = bf16(sum_k x[m,k] * q[k,n] * S[k//gs, n]), fp32 accumulation.

    The semantics of ``torch_npu.npu_weight_quant_batchmatmul(x, W, S,
    antiquant_group_size=gs)`` at ``fnx/engine.py:698-701``: x bf16 [M,K],
    W int4pack [K,N/8], S bf16 [G,N]; one bf16 rounding of the fp32 result.
    Returns bf16 bit patterns [M, N].
    """
    x = bf16_bits_to_f32(x_bits)
    w = dequant(w4, scale_bits, gs)
    return f32_to_bf16_bits(np.matmul(x, w, dtype=np.float32))


def grouped_gemm(x_bits, w4_em, scale_em_bits, ends) -> np.ndarray:
    """Expert-major grouped W4A16 GEMM (``npu_grouped_matmul``, group_type 0).

    ``fnx/engine.py:749-753``: rows [ends[e-1], ends[e]) of x use expert e's
    weights w4_em[e] (int4pack [K, N/8]) and scales[e] ([G, N]); ``ends`` is
    the inclusive cumulative count (``group_list``); empty experts are
    allowed. Rows past ends[-1] are not written by the operator; here they
    are returned as zeros. Returns bf16 bits [R, N].
    """
    x = bf16_bits_to_f32(x_bits)
    R, K = x.shape
    E = w4_em.shape[0]
    N = w4_em.shape[2] * 8
    G = scale_em_bits.shape[1]
    gs = K // G
    out = np.zeros((R, N), dtype=np.uint16)
    ends = np.asarray(ends, dtype=np.int64)
    begins = np.concatenate([[0], ends[:-1]])

    def one(e):
        begin, end = int(begins[e]), int(ends[e])
        if end > begin:
            w = dequant(w4_em[e], scale_em_bits[e], gs)
            out[begin:end] = f32_to_bf16_bits(np.matmul(x[begin:end], w, dtype=np.float32))

    _each_expert(one, range(E))
    return out


def w4a16_gemm_exact(x_bits, w4, scale_bits, gs):
    """float64 value of the W4A16 product before its bf16 rounding, and the
    sum of absolute products sum_k |x q S| (the scale of any fp32
    accumulation error). Reference point of the rounding-window checks."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    w = dequant(w4, scale_bits, gs).astype(np.float64)
    return x @ w, np.abs(x) @ np.abs(w)


def grouped_gemm_exact(x_bits, w4_em, scale_em_bits, ends):
    """float64 pre-rounding values of :func:`grouped_gemm` and their absolute
    product sums (rows past ends[-1] = 0)."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    R = x.shape[0]
    N = w4_em.shape[2] * 8
    gs = x.shape[1] // scale_em_bits.shape[1]
    out = np.zeros((R, N), dtype=np.float64)
    mag = np.zeros((R, N), dtype=np.float64)
    ends = np.asarray(ends, dtype=np.int64)
    begins = np.concatenate([[0], ends[:-1]])

    def one(e):
        begin, end = int(begins[e]), int(ends[e])
        if end > begin:
            w = dequant(w4_em[e], scale_em_bits[e], gs).astype(np.float64)
            out[begin:end] = x[begin:end] @ w
            mag[begin:end] = np.abs(x[begin:end]) @ np.abs(w)

    _each_expert(one, range(w4_em.shape[0]))
    return out, mag


REL_WINDOW = 2.0 ** -15      # relative to the value
ACC_WINDOW = 2.0 ** -20      # relative to the sum of absolute terms


def bf16_interval(exact, abs_sum=None):
    """Admissible bf16 results of a value computed by fp32 accumulation.

    Returns (lo, hi) bit arrays: the nearest-even roundings of exact -/+ d,
    d = 2^-15 |exact| + 2^-20 sum|terms|. With products of random sign the
    partial sums of an fp32 accumulation stay near sum|terms| / sqrt(K), so
    its rounding error has a spread of about 2^-25 sum|terms| whatever the
    (blocked) order; d is ~32 times that. Away from a rounding boundary
    lo == hi and the result must equal the rounding of the exact value.
    """
    e = np.asarray(exact, dtype=np.float64)
    d = np.abs(e) * REL_WINDOW
    if abs_sum is not None:
        d = d + np.asarray(abs_sum, dtype=np.float64) * ACC_WINDOW
    return f32_to_bf16_bits((e - d).astype(np.float32)), f32_to_bf16_bits((e + d).astype(np.float32))


def swiglu_interval(g_exact, g_abs, u_exact, u_abs):
    """Admissible SwiGLU outputs given exact gate/up values: the extremes of
    bf16(silu(g_b) * u_b) over the admissible bf16 g_b, u_b (corners of the
    intervals), widened by the relative window of the final rounding."""
    g_lo, g_hi = (bf16_bits_to_f32(b).astype(np.float64) for b in bf16_interval(g_exact, g_abs))
    u_lo, u_hi = (bf16_bits_to_f32(b).astype(np.float64) for b in bf16_interval(u_exact, u_abs))
    vals = []
    with np.errstate(over="ignore", invalid="ignore"):
        for g in (g_lo, g_hi):
            sg = g / (1.0 + np.exp(-g))
            for u in (u_lo, u_hi):
                vals.append(sg * u)
    v = np.stack(vals)
    lo, hi = v.min(axis=0), v.max(axis=0)
    return (f32_to_bf16_bits((lo - np.abs(lo) * REL_WINDOW).astype(np.float32)),
            f32_to_bf16_bits((hi + np.abs(hi) * REL_WINDOW).astype(np.float32)))


def router_weights_exact(logits_bits, idx):
    """float64 renormalised softmax weights of the selected experts."""
    l = bf16_bits_to_f32(np.asarray(logits_bits).view(np.uint16)).astype(np.float64)
    e = np.exp(l - l.max(axis=1, keepdims=True))
    p = e / e.sum(axis=1, keepdims=True)
    pk = np.take_along_axis(p, np.asarray(idx), axis=1)
    return pk / pk.sum(axis=1, keepdims=True)


# --------------------------------------------------------------------------
# W8A16 dense projections (DenseW8, fnx/engine.py:297-384)
# --------------------------------------------------------------------------


def dense_w8_from_qs(q, s, K=None):
    """``DenseW8.__init__`` (``fnx/engine.py:318-328``): per-row int8 weights
    q [N, Kp] with fp16 group scales s [N, G'] (gs = Kp // G') -> the operator's
    containers w8t int8 [K, N] = q[:, :K]^T and sc bf16 bits [K/gs, N] =
    bf16(s[:, :K/gs]^T). Returns (w8t, sc_bits, gs)."""
    q = np.asarray(q, dtype=np.int8)
    s = np.asarray(s, dtype=np.float16)
    gs = q.shape[-1] // s.shape[-1]
    kk = q.shape[-1] if K is None else K
    if kk % gs:
        raise ValueError(f"K={kk} is not a multiple of gs={gs}")
    w8t = np.ascontiguousarray(q[:, :kk].T)
    sc = f32_to_bf16_bits(np.ascontiguousarray(s[:, :kk // gs].T).astype(np.float32))
    return w8t, sc, gs


def w8a16_gemm(x_bits, w8t, scale_bits, gs) -> np.ndarray:
    """``npu_weight_quant_batchmatmul(x, w8t, sc, antiquant_group_size=gs)``
    with int8 weights (``fnx/engine.py:358-364``): y[M,N] = bf16(sum_k x[m,k] *
    q[k,n] * S[k//gs, n]), fp32 accumulation; q [K, N] int8, S bf16 [K/gs, N].
    q (8 bits) * S (8 bits) is exact in fp32, as are the products with x."""
    x = bf16_bits_to_f32(x_bits)
    w = np.asarray(w8t, dtype=np.int8).astype(np.float32) * np.repeat(bf16_bits_to_f32(scale_bits), gs, axis=0)
    return f32_to_bf16_bits(np.matmul(x, w, dtype=np.float32))


def w8a16_gemm_exact(x_bits, w8t, scale_bits, gs):
    """float64 value of :func:`w8a16_gemm` before rounding, and sum_k |x q S|."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    w = np.asarray(w8t, dtype=np.int8).astype(np.float64) * np.repeat(
        bf16_bits_to_f32(scale_bits).astype(np.float64), gs, axis=0)
    return x @ w, np.abs(x) @ np.abs(w)


# --------------------------------------------------------------------------
# Dense bf16 projections: shared expert and router (fnx/engine.py:1786-1802)
# --------------------------------------------------------------------------


def linear(x_bits, w_bits) -> np.ndarray:
    """``F.linear(x, w)`` on bf16 tensors (the reference's ``_fl``,
    ``fnx/engine.py:256``): y[M,N] = bf16(sum_k x[m,k] * w[n,k]) with fp32
    accumulation; x [M,K], w [N,K] (the ``Raw`` container, ``fnx/engine.py:387``)."""
    x = bf16_bits_to_f32(x_bits)
    w = bf16_bits_to_f32(w_bits)
    return f32_to_bf16_bits(np.matmul(x, w.T, dtype=np.float32))


def linear_exact(x_bits, w_bits):
    """float64 value of :func:`linear` before its rounding, and sum_k |x w|."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    w = bf16_bits_to_f32(w_bits).astype(np.float64)
    return x @ w.T, np.abs(x) @ np.abs(w).T


def silu_bf16(g_bits) -> np.ndarray:
    """``F.silu`` of a bf16 tensor: silu in fp32, one rounding to bf16."""
    g = bf16_bits_to_f32(g_bits)
    with np.errstate(over="ignore"):
        return f32_to_bf16_bits(g / (np.float32(1.0) + np.exp(-g)))


def swiglu_bf16(gu_bits, MI) -> np.ndarray:
    """``F.silu(gu[:, :MI]) * gu[:, MI:2*MI]`` on bf16 tensors
    (``fnx/engine.py:1788``): bf16(bf16(silu(g)) * u), two roundings, unlike
    the fp32 ``npu_swiglu`` form of :func:`swiglu`."""
    gu = np.asarray(gu_bits).view(np.uint16)
    s = bf16_bits_to_f32(silu_bf16(gu[:, :MI]))
    return f32_to_bf16_bits(s * bf16_bits_to_f32(gu[:, MI:2 * MI]))


def shared_gate(sh_bits, gate_bits) -> np.ndarray:
    """``torch.sigmoid(g) * sh`` on bf16 tensors (``fnx/engine.py:1793``):
    bf16(bf16(sigmoid(g)) * sh), g [M, 1] broadcast over sh [M, H]."""
    sg = sigmoid_bf16(np.asarray(gate_bits).view(np.uint16).reshape(-1, 1))   # bf16 values as fp32
    return f32_to_bf16_bits(sg * bf16_bits_to_f32(sh_bits))


def shared_router(x_bits, sh_gu_bits, sh_down_bits, MI):
    """Shared expert + router projection of ``FnLayer._moe`` in its fused form
    (``sh_gw``, ``fnx/engine.py:1786-1796``; the weight merge is
    ``fnx/engine.py:1226-1241``): one projection x -> [gate MI | up MI |
    gate2 1 | router E], the shared SwiGLU and down projection. Returns
    (gu [M, 2MI+1+E], act [M, MI], sh [M, H], shared_gate [M, 1],
    logits [M, E]), all bf16 bits; ``sh`` is not yet gated."""
    gu = linear(x_bits, sh_gu_bits)
    act = swiglu_bf16(gu, MI)
    sh = linear(act, sh_down_bits)
    return gu, act, sh, gu[:, 2 * MI:2 * MI + 1], gu[:, 2 * MI + 1:]


# --------------------------------------------------------------------------
# Router and grouping glue
# --------------------------------------------------------------------------


def bf16_order_key(bits) -> np.ndarray:
    """Monotone uint32 key of bf16 values: a < b  <=>  key(a) < key(b).

    -0 and +0 map to different keys (as do the two zeros of any float
    compare-by-bits order); ties only occur for identical bit patterns.
    """
    b = np.asarray(bits).view(np.uint16).astype(np.uint32)
    neg = (b & 0x8000) != 0
    return np.where(neg, (~b) & 0xFFFF, b | 0x8000).astype(np.uint32)


def router(logits_bits, k):
    """Softmax router: ``fnx/engine.py:1810-1813``.

    probs = softmax(fp32(logits)) (max-subtracted, fp32 sum in index order);
    the k experts with the largest logits are selected, ordered by logit
    descending and, on equal logits, by lower expert id; their probabilities
    are renormalised by their fp32 sum (taken in rank order) and rounded to
    bf16. Selecting on logits equals selecting on probs (softmax is monotone);
    the tie rule is this build's definition (the NPU ``topk`` tie order is
    closed). Returns (idx int64 [T,k], w bf16 bits [T,k]).
    """
    lb = np.asarray(logits_bits).view(np.uint16)
    T, E = lb.shape
    l = bf16_bits_to_f32(lb)
    key = bf16_order_key(lb).astype(np.int64)
    # sort by (-key, index): stable argsort on -key keeps lower index first
    idx = np.argsort(-key, axis=1, kind="stable")[:, :k].astype(np.int64)
    m = l.max(axis=1, keepdims=True)
    e = np.exp(l - m, dtype=np.float32)
    z = np.zeros((T, 1), dtype=np.float32)
    for j in range(E):
        z[:, 0] = z[:, 0] + e[:, j]
    p = (e / z).astype(np.float32)
    pk = np.take_along_axis(p, idx, axis=1)
    s = np.zeros((T, 1), dtype=np.float32)
    for j in range(k):
        s[:, 0] = s[:, 0] + pk[:, j]
    return idx, f32_to_bf16_bits(pk / s)


def group_routing(idx, E):
    """Expert-major grouping: ``fnx/engine.py:1816-1823, 1832-1843``.

    ids = idx.flatten(); counts = bincount(ids, E); ends = cumsum(counts)
    (int64, the ``group_list``); order = stable argsort of ids (within an
    expert, ascending flat index t*k+slot — the reference's
    ``argsort(ids.float())`` at 1820 is not stable; this build defines the
    stable order); inverse[order[p]] = p (1840-1842).
    Returns (counts, ends, order, inverse), all int64.
    """
    ids = np.asarray(idx, dtype=np.int64).reshape(-1)
    counts = np.bincount(ids, minlength=E).astype(np.int64)
    ends = np.cumsum(counts).astype(np.int64)
    order = np.argsort(ids, kind="stable").astype(np.int64)
    inverse = np.empty_like(order)
    inverse[order] = np.arange(order.size, dtype=np.int64)
    return counts, ends, order, inverse


def swiglu(gu_bits) -> np.ndarray:
    """act = bf16(silu(fp32 g) * fp32 u), g = first half, u = second half.

    ``npu_swiglu(gu.float(), dim=-1).to(bf16)`` at ``fnx/engine.py:1827,1866``
    with the pure-torch twin ``(F.silu(gu[:, :MI].float()) *
    gu[:, MI:].float()).to(bf16)`` at 1829/1868. silu(g) = g / (1 + exp(-g)).
    """
    gu = bf16_bits_to_f32(gu_bits)
    mi = gu.shape[-1] // 2
    g = gu[..., :mi]
    u = gu[..., mi:]
    with np.errstate(over="ignore"):
        silu = (g / (np.float32(1) + np.exp(-g, dtype=np.float32))).astype(np.float32)
    return f32_to_bf16_bits(silu * u)


# --------------------------------------------------------------------------
# Combine glue: weighted reduce, decode epilogue, shared merge, gather
# --------------------------------------------------------------------------


def weighted_reduce(values_bits, weights_bits, inverse=None) -> np.ndarray:
    """MoE combine with bf16 product rounding and ordered fp32 accumulation.

    ``kernels/reduce/reduce.cpp:27-56`` modes 1/2 (wrapper
    ``fnx/weighted_reduce.py:10-42``): out[t,:] = bf16(sum_{g=0..G-1, in
    order} fp32(bf16(fp32(x[row,:]) * fp32(w[t,g])))) with row = inverse[t*G+g]
    (mode 2) or t*G+g (mode 1). values: bf16 [rows, W]; weights: bf16 [B, G].
    """
    x = bf16_bits_to_f32(np.asarray(values_bits).reshape(-1, np.shape(values_bits)[-1]))
    w = bf16_bits_to_f32(weights_bits)
    B, G = w.shape
    rows = np.arange(B * G) if inverse is None else np.asarray(inverse, dtype=np.int64)
    acc = np.zeros((B, x.shape[1]), dtype=np.float32)
    for g in range(G):
        r = rows.reshape(B, G)[:, g]
        acc = acc + round_bf16(x[r] * w[:, g:g + 1])
    return f32_to_bf16_bits(acc)


def sigmoid_bf16(g_bits) -> np.ndarray:
    """bf16(1 / (1 + exp(-fp32 g))) — ``kernels/moe_epilogue/epilogue.cpp:33-35``."""
    g = bf16_bits_to_f32(g_bits)
    with np.errstate(over="ignore"):
        return round_bf16(np.float32(1) / (np.float32(1) + np.exp(-g, dtype=np.float32)))


def moe_merge(experts_bits, shared_bits, gate_bits) -> np.ndarray:
    """out = bf16(e + bf16(s * bf16(sigmoid(g)))) — ``kernels/post_ops/post_ops.cpp:72-94``.

    ``gate`` holds one value per token (row).
    """
    e = bf16_bits_to_f32(experts_bits)
    s = bf16_bits_to_f32(shared_bits)
    g = sigmoid_bf16(np.asarray(gate_bits).reshape(-1)).reshape(-1, 1)
    e2 = e.reshape(g.shape[0], -1)
    s2 = s.reshape(g.shape[0], -1)
    return f32_to_bf16_bits(e2 + round_bf16(s2 * g)).reshape(np.shape(experts_bits))


def moe_epilogue(cartesian_bits, weights_bits, shared_bits, gate_bits) -> np.ndarray:
    """Decode fused combine: ``kernels/moe_epilogue/epilogue.cpp:17-39``.

    cartesian [k, k*H] holds the down output of every activation row j
    against every selected expert; only diagonal block (j, j) is used:
    r = bf16(sum_{j in order} fp32(bf16(y_jj * w_j))), then
    out = bf16(r + bf16(shared * bf16(sigmoid(gate)))). Returns [1, H].
    """
    c = np.asarray(cartesian_bits).view(np.uint16)
    k = c.shape[0]
    H = c.shape[1] // k
    diag = np.stack([c[j, j * H:(j + 1) * H] for j in range(k)])        # [k, H]
    r = weighted_reduce(diag, np.asarray(weights_bits).reshape(1, k))
    return moe_merge(r, np.asarray(shared_bits).reshape(1, H), gate_bits)


def expert_gather(w4_em, scale_em_bits, ids):
    """Selected experts, expert-major -> K-major concatenation.

    ``kernels/expert_gather/gather.cpp:8-21`` (wrapper
    ``fnx/expert_gather.py:9-31``): ow[k, j*N/8 + c] = w4[ids[j], k, c],
    os[g, j*N + n] = S[ids[j], g, n]. Returns (ow int32 [K, k*N/8],
    os bf16 bits [G, k*N]).
    """
    ids = np.asarray(ids, dtype=np.int64)
    w = np.asarray(w4_em)[ids]                       # [k, K, N/8]
    s = np.asarray(scale_em_bits).view(np.uint16)[ids]   # [k, G, N]
    ow = np.ascontiguousarray(w.transpose(1, 0, 2)).reshape(w.shape[1], -1)
    os_ = np.ascontiguousarray(s.transpose(1, 0, 2)).reshape(s.shape[1], -1)
    return ow, os_


# --------------------------------------------------------------------------
# Whole MoE expert block (decode b == 1 and grouped prefill b > 1)
# --------------------------------------------------------------------------


def moe_decode(x_bits, logits_bits, gu_w4, gu_s, dn_w4, dn_s, k, shared_bits=None, gate_bits=None):
    """One-token MoE expert block, ``fnx/engine.py:1859-1891`` (r152 flags).

    gate_up of the k selected experts on x (``ExpW4.apply``, 1861), SwiGLU
    (1866), down of activation row j with expert j (the diagonal of the
    Cartesian product, 1873 / ``apply_diag`` 703-721), ordered bf16-product
    combine (``moe_epilogue`` 1874 or ``weighted_reduce`` 1884), then the
    optional shared-expert merge (1887-1891). Expert tensors are expert-major:
    gu_w4 int32 [E, H, 2MI/8], gu_s bf16 [E, G1, 2MI], dn_w4 [E, MI, H/8],
    dn_s [E, G2, H]. Returns a dict of bit-pattern arrays.
    """
    x = np.asarray(x_bits).view(np.uint16).reshape(1, -1)
    idx, w = router(np.asarray(logits_bits).view(np.uint16).reshape(1, -1), k)
    H = x.shape[1]
    g1 = gu_s.shape[1]
    g2 = dn_s.shape[1]
    gu = np.stack([w4a16_gemm(x, gu_w4[e], gu_s[e], H // g1)[0] for e in idx[0]])   # [k, 2MI]
    act = swiglu(gu)                                                              # [k, MI]
    mi = act.shape[1]
    y = np.stack([w4a16_gemm(act[j:j + 1], dn_w4[e], dn_s[e], mi // g2)[0]
                  for j, e in enumerate(idx[0])])                                  # [k, H]
    out = weighted_reduce(y, w)
    prod = f32_to_bf16_bits(bf16_bits_to_f32(y) * bf16_bits_to_f32(w).reshape(-1, 1))
    mag = combine_magnitude(prod, len(idx[0]))
    if shared_bits is not None:
        out = moe_merge(out, np.asarray(shared_bits).reshape(1, H), gate_bits)
        mag = np.maximum(mag, np.abs(bf16_bits_to_f32(out)))
    return {"idx": idx, "w": w, "gu": gu, "act": act, "y": y, "prod": prod, "mag": mag, "out": out}


def moe_prefill(x_bits, logits_bits, gu_w4, gu_s, dn_w4, dn_s, k, shared_bits=None):
    """Grouped prefill MoE, ``fnx/engine.py:1815-1853`` (r152 flags).

    Router, expert-major grouping with a stable order, row gather
    ``x.index_select(0, order // k)`` (1825), grouped gate_up GEMM, SwiGLU,
    grouped down GEMM, inverse permutation and the mode-2 weighted reduce
    (1846), plus ``+ sh`` (1853, a bf16 add) when a shared-expert output is
    given. Returns a dict of arrays.
    """
    x = np.asarray(x_bits).view(np.uint16)
    T = x.shape[0]
    E = gu_w4.shape[0]
    idx, w = router(np.asarray(logits_bits).view(np.uint16), k)
    counts, ends, order, inverse = group_routing(idx, E)
    rows = x[order // k]
    gu = grouped_gemm(rows, gu_w4, gu_s, ends)
    act = swiglu(gu)
    yd = grouped_gemm(act, dn_w4, dn_s, ends)
    out = weighted_reduce(yd, w, inverse=inverse)
    wf = bf16_bits_to_f32(w).reshape(-1)
    prod = f32_to_bf16_bits(bf16_bits_to_f32(yd[inverse]) * wf[:, None])
    mag = combine_magnitude(prod, k)
    if shared_bits is not None:
        out = f32_to_bf16_bits(bf16_bits_to_f32(out) + bf16_bits_to_f32(shared_bits))
    return {"idx": idx, "w": w, "counts": counts, "ends": ends, "order": order,
            "inverse": inverse, "gu": gu, "act": act, "yd": yd, "mag": mag, "out": out, "T": T}


# --------------------------------------------------------------------------
# Element-wise admissible outputs of the whole expert block
# --------------------------------------------------------------------------


def _round_bounds(lo, hi, abs_sum=None):
    """bf16 values reachable by rounding (nearest even) any fp32 result of an
    accumulation whose exact value lies in [lo, hi]: the windows of
    :func:`bf16_interval` applied at both ends. Returns float64 arrays."""
    lo_b = bf16_interval(lo, abs_sum)[0]
    hi_b = bf16_interval(hi, abs_sum)[1]
    return bf16_bits_to_f32(lo_b).astype(np.float64), bf16_bits_to_f32(hi_b).astype(np.float64)


def moe_output_interval(x_bits, idx, logits_bits, gu_w4, gu_s, dn_w4, dn_s, shared_bits=None, gate_bits=None):
    """Element-wise bounds [lo, hi] (bf16 bits [T, H]) on the combined output
    of the expert block over every admissible rounding of its intermediates.

    The reference's chain (``fnx/engine.py:1815-1891``) rounds to bf16 at gate/
    up, act, down output, each weighted product and the slot sum. Two fp32
    accumulations of the same exact value in different orders may round to
    neighbouring bf16 values when it lies near a boundary, and such a flip
    propagates. Here every rounding takes every value it admissibly can:
    gate/up and the router weights within :func:`bf16_interval` of their
    float64 values, act by :func:`swiglu_interval`, the down output over the
    act box by interval arithmetic (exact float64 bounds of a linear map), the
    weighted product at the corners of (y, w), the ordered fp32 slot sum
    widened by its rounding error, then the shared-expert terms: ``+ sh``
    (prefill, a bf16 add) or the sigmoid-gated merge of
    ``kernels/post_ops/post_ops.cpp:72-94`` (decode, ``gate_bits`` [T]).
    Any output outside [lo, hi] comes from a wrong operand, index, scale,
    sign or rounding point, not from summation order.
    x_bits bf16 [T, H]; idx int64 [T, k] (the routing); logits bf16 [T, E].
    """
    x = bf16_bits_to_f32(np.asarray(x_bits).view(np.uint16)).astype(np.float64)
    idx = np.asarray(idx, dtype=np.int64)
    T, k = idx.shape
    H = x.shape[1]
    MI = dn_w4.shape[1]
    g1, g2 = gu_s.shape[1], dn_s.shape[1]
    wex = router_weights_exact(logits_bits, idx)
    w_lo, w_hi = (bf16_bits_to_f32(b).astype(np.float64) for b in bf16_interval(wex))
    p_lo = np.zeros((T, k, H))
    p_hi = np.zeros((T, k, H))
    flat = idx.reshape(-1)
    order = np.argsort(flat, kind="stable")
    uniq, first = np.unique(flat[order], return_index=True)
    spans = dict(zip(uniq.tolist(), zip(first.tolist(), np.append(first[1:], flat.size).tolist())))

    def one(e):
        a, b = spans[e]
        tt, jj = np.divmod(order[a:b], k)
        cu = dequant(gu_w4[e], gu_s[e], H // g1).astype(np.float64)
        ge, ga = x[tt] @ cu, np.abs(x[tt]) @ np.abs(cu)
        a_lo, a_hi = (bf16_bits_to_f32(b).astype(np.float64)
                      for b in swiglu_interval(ge[:, :MI], ga[:, :MI], ge[:, MI:], ga[:, MI:]))
        cd = dequant(dn_w4[e], dn_s[e], MI // g2).astype(np.float64)
        cp, cn = np.maximum(cd, 0.0), np.minimum(cd, 0.0)
        y_lo = a_lo @ cp + a_hi @ cn
        y_hi = a_hi @ cp + a_lo @ cn
        yab = np.maximum(np.abs(a_lo), np.abs(a_hi)) @ np.abs(cd)
        yb_lo, yb_hi = _round_bounds(y_lo, y_hi, yab)
        wl, wh = w_lo[tt, jj][:, None], w_hi[tt, jj][:, None]
        corners = np.stack([yb_lo * wl, yb_lo * wh, yb_hi * wl, yb_hi * wh])
        plo, phi = _round_bounds(corners.min(axis=0), corners.max(axis=0))
        p_lo[tt, jj] = plo
        p_hi[tt, jj] = phi

    _each_expert(one, uniq)
    eps = k * 2.0 ** -24 * np.maximum(np.abs(p_lo), np.abs(p_hi)).sum(axis=1)
    r_lo, r_hi = _round_bounds(p_lo.sum(axis=1) - eps, p_hi.sum(axis=1) + eps)
    if shared_bits is not None:
        sh = bf16_bits_to_f32(np.asarray(shared_bits).view(np.uint16)).reshape(T, H).astype(np.float64)
        if gate_bits is None:
            r_lo, r_hi = _round_bounds(r_lo + sh, r_hi + sh)
        else:
            g = bf16_bits_to_f32(np.asarray(gate_bits).view(np.uint16)).reshape(T, 1).astype(np.float64)
            sg_lo, sg_hi = (bf16_bits_to_f32(b).astype(np.float64) for b in bf16_interval(1.0 / (1.0 + np.exp(-g))))
            t_lo, t_hi = _round_bounds(np.minimum(sh * sg_lo, sh * sg_hi), np.maximum(sh * sg_lo, sh * sg_hi))
            r_lo, r_hi = _round_bounds(r_lo + t_lo, r_hi + t_hi)
    return f32_to_bf16_bits(r_lo.astype(np.float32)), f32_to_bf16_bits(r_hi.astype(np.float32))


# --------------------------------------------------------------------------
# Parity metrics
# --------------------------------------------------------------------------


def compare(got_bits, ref_bits, mag=None):
    """Return (rel_l2, max_abs, n_beyond) between two bf16 arrays.

    n_beyond counts elements whose difference exceeds 1e-2 plus one bf16
    step (2^-7) of the larger of |ref| and ``mag``: the allowance for a value
    that two fp32 accumulations in different orders place on opposite sides
    of a bf16 rounding boundary. ``mag`` is the magnitude of the largest term
    entering the element's last sum (e.g. the largest weighted expert
    product of a combined MoE output), since a one-step flip of that term
    survives the sum unchanged.
    """
    g = bf16_bits_to_f32(got_bits).astype(np.float64)
    r = bf16_bits_to_f32(ref_bits).astype(np.float64)
    d = np.abs(g - r)
    denom = np.sqrt((r * r).sum())
    rel = float(np.sqrt((d * d).sum()) / denom) if denom > 0 else float(np.sqrt((d * d).sum()))
    scale = np.abs(r) if mag is None else np.maximum(np.abs(r), np.broadcast_to(np.abs(mag), r.shape))
    beyond = int((d > 1e-2 + scale * 2.0 ** -7).sum())
    return rel, float(d.max()) if d.size else 0.0, beyond


def combine_magnitude(prod_bits, k):
    """Largest |term| of each combined output element: prod bf16 [T*k, H] -> [T, H]."""
    p = np.abs(bf16_bits_to_f32(prod_bits)).reshape(-1, k, np.shape(prod_bits)[-1])
    return p.max(axis=1)
