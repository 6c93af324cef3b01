"""Pins the CPU oracle (CPU only).

Each oracle function is checked against something it does not itself
contain: known-answer vectors derived from the reference's own statements,
an independent implementation (torch's bf16 casts and ops, byte-level
decoding, the reference's index_select/permute formulation), brute force on
tiny shapes, or invariants the reference tests assert. Several checks are
chosen so a plausible slip (nibble order, pack axis, scale indexing, sign,
summation order, tie rule) fails them.
"""
import math

import numpy as np
import pytest
import torch

from oracle import qmoe_oracle as O

rng = np.random.default_rng(1234)


def tbits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)


# ------------------------------------------------------------------ bf16


def test_bf16_rounding_matches_torch():
    specials = np.array([0.0, -0.0, 1.0, -1.0, 1.00390625, 1.01171875, 3.4e38, -3.4e38, 1e-40, -1e-40,
                         np.inf, -np.inf, 65504.0, 2.0 ** -133, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8],
                        dtype=np.float32)
    vals = np.concatenate([specials, rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000)])
    vals = vals.astype(np.float32)
    ref = tbits(torch.from_numpy(vals).to(torch.bfloat16))
    assert np.array_equal(O.f32_to_bf16_bits(vals), ref)
    # round half to even on exact ties
    assert O.f32_to_bf16_bits(np.float32(1.0 + 2 ** -8)) == 0x3F80
    assert O.f32_to_bf16_bits(np.float32(1.0 + 3 * 2 ** -8)) == 0x3F82
    nan = O.f32_to_bf16_bits(np.array([np.nan], dtype=np.float32))
    assert np.isnan(O.bf16_bits_to_f32(nan))[0]


# ------------------------------------------------------------------ int4pack


def test_int4pack_known_answers():
    # values -8..-1 along N pack low nibble first into one word
    q = np.arange(-8, 0, dtype=np.int8).reshape(1, 8)
    assert O.pack_int4(q).view(np.uint32)[0, 0] == 0xFEDCBA98
    q = np.arange(0, 8, dtype=np.int8).reshape(1, 8)
    assert O.pack_int4(q).view(np.uint32)[0, 0] == 0x76543210
    # column 8c+j lives in word c, nibble j; pack runs along the last axis (N)
    q = np.zeros((2, 16), dtype=np.int8)
    q[1, 9] = -3
    w = O.pack_int4(q).view(np.uint32)
    assert w.shape == (2, 2) and w[1, 1] == (0xD << 4) and w[0].sum() == 0 and w[1, 0] == 0


def test_int4pack_matches_reference_byte_addressing():
    # r156 kernel: byte k*N/2 + n/2 of the row-major int4pack, low nibble = even n
    K, N = 16, 64
    q = rng.integers(-8, 8, size=(K, N)).astype(np.int8)
    w = O.pack_int4(q)
    b = w.view(np.uint8).reshape(K, N // 2)
    lo = ((b & 0xF).astype(np.int16) ^ 8) - 8
    hi = ((b >> 4).astype(np.int16) ^ 8) - 8
    dec = np.empty((K, N), dtype=np.int16)
    dec[:, 0::2] = lo
    dec[:, 1::2] = hi
    assert np.array_equal(dec, q)
    assert np.array_equal(O.unpack_int4(w), q)


def test_int4pack_rejects_out_of_range():
    with pytest.raises(ValueError):
        O.pack_int4(np.full((1, 8), 8, dtype=np.int8))


# ------------------------------------------------------------------ LQP v2o


def test_v2o_layout_and_round_trip():
    E, N, K = 2, 3, 256
    q = rng.integers(-8, 8, size=(E, N, K)).astype(np.int8)
    p = O.pack_v2o(q)
    assert p.shape == (E, N, K // 2)
    # tools/layout_v2_check.py:4-9: byte 64s+j = W[128s+j] (low) | W[128s+64+j] (high), offset-binary
    for s in range(K // 128):
        for j in (0, 17, 63):
            byte = int(p[1, 2, 64 * s + j])
            assert (byte & 15) - 8 == q[1, 2, 128 * s + j]
            assert (byte >> 4) - 8 == q[1, 2, 128 * s + 64 + j]
    assert np.array_equal(O.unpack_v2o(p), q)


def test_lqp_to_expert_major_chain():
    E, N, K, gs = 3, 16, 128, 64
    q = rng.integers(-8, 8, size=(E, N, K)).astype(np.int8)
    s8 = rng.integers(-127, 128, size=(E, N, K // gs)).astype(np.int8)
    base = (rng.random((E, N)) * 0.01).astype(np.float16)
    w4, s8t, base_bits, sc = O.lqp_to_em(O.pack_v2o(q), s8, base)
    assert w4.shape == (E, K, N // 8) and s8t.shape == (K // gs, E, N)
    # expert-major int4pack element [e, k, n] is the original W[e, n, k]
    assert np.array_equal(O.unpack_int4(w4), q.transpose(0, 2, 1))
    # K-major artifact [K, E, N/8] and expert-major differ by permute(1,0,2) only (tools/repack_w4_em.py:19)
    kmajor = np.ascontiguousarray(w4.transpose(1, 0, 2))
    assert np.array_equal(kmajor.transpose(1, 0, 2), w4)
    # scale cache = bf16(bf16(s8) * bf16(base)) computed by torch the way fnx/engine.py:657 does
    ref = (torch.from_numpy(s8t).permute(1, 0, 2).to(torch.bfloat16)
           * torch.from_numpy(base.astype(np.float32)).to(torch.bfloat16)[:, None, :])
    assert np.array_equal(sc, tbits(ref))


# ------------------------------------------------------------------ GEMMs


def _brute_w4a16(xf, q, s, gs):
    # float64 triple loop over an independently decoded weight
    M, K = xf.shape
    N = q.shape[1]
    y = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                acc += float(xf[m, k]) * float(q[k, n]) * float(s[k // gs, n])
            y[m, n] = acc
    return y


def test_w4a16_gemm_brute_force():
    M, K, N, gs = 2, 64, 16, 32
    q = rng.integers(-8, 8, size=(K, N)).astype(np.int8)
    # strongly non-uniform scales: a swapped group/column index changes the result
    s = O.f32_to_bf16_bits((np.arange(K // gs)[:, None] + 1) * (np.arange(N)[None, :] + 1) * 0.01)
    x = O.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    y = O.bf16_bits_to_f32(O.w4a16_gemm(x, O.pack_int4(q), s, gs)).astype(np.float64)
    ref = _brute_w4a16(O.bf16_bits_to_f32(x), q, O.bf16_bits_to_f32(s), gs)
    assert np.all(np.abs(y - ref) <= np.abs(ref) * 2 ** -8 + 1e-6)
    # and matches the reference's torch dequant formulation (fnx/engine.py:247-252) in fp32
    wt = torch.from_numpy(q.astype(np.float32)) * torch.from_numpy(np.repeat(O.bf16_bits_to_f32(s), gs, 0))
    yt = (torch.from_numpy(O.bf16_bits_to_f32(x)) @ wt).to(torch.bfloat16)
    assert np.mean(tbits(yt) == O.w4a16_gemm(x, O.pack_int4(q), s, gs)) > 0.99


def test_grouped_gemm_equals_per_row_selection():
    E, K, N, gs = 5, 64, 32, 32
    w4 = np.stack([O.pack_int4(rng.integers(-8, 8, size=(K, N)).astype(np.int8)) for _ in range(E)])
    sc = O.f32_to_bf16_bits(np.abs(rng.standard_normal((E, K // gs, N))).astype(np.float32) * 0.02)
    counts = np.array([3, 0, 1, 0, 4])          # empty experts included
    ends = np.cumsum(counts)
    R = int(ends[-1])
    x = O.f32_to_bf16_bits(rng.standard_normal((R, K)).astype(np.float32))
    y = O.grouped_gemm(x, w4, sc, ends)
    e_of_row = np.repeat(np.arange(E), counts)
    for p in range(R):
        assert np.array_equal(y[p], O.w4a16_gemm(x[p:p + 1], w4[e_of_row[p]], sc[e_of_row[p]], gs)[0])


# ------------------------------------------------------------------ router / grouping


def test_router_brute_force_and_ties():
    T, E, k = 6, 40, 10
    logits = O.f32_to_bf16_bits(rng.standard_normal((T, E)).astype(np.float32))
    logits[0, 5] = logits[0, 30] = logits[0, 7] = 0x4100     # three-way tie at 8.0, the max
    logits[1, :] = 0x3F80                                      # all equal
    idx, w = O.router(logits, k)
    lf = O.bf16_bits_to_f32(logits).astype(np.float64)
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-lf[t, e], e))[:k]
        assert list(idx[t]) == order
        p = np.exp(lf[t] - lf[t].max())
        p /= p.sum()
        ref = p[order] / p[order].sum()
        assert np.allclose(O.bf16_bits_to_f32(w[t]), ref, rtol=2 ** -7, atol=0)
    assert list(idx[0][:3]) == [5, 7, 30]
    assert list(idx[1]) == list(range(k))


def test_router_negative_and_signed_zero_order():
    logits = O.f32_to_bf16_bits(np.array([[-0.0, 0.0, -1.0, -2.0, 1e-30, -1e-30]], dtype=np.float32))
    idx, _ = O.router(logits, 6)
    # +tiny > +0 > -0 > -tiny > -1 > -2 under the bf16 order key
    assert list(idx[0]) == [4, 1, 0, 5, 2, 3]


def test_group_routing_brute_force():
    T, k, E = 37, 10, 64
    idx = rng.integers(0, E, size=(T, k))
    idx[:, 0] = 3                                   # a popular expert
    counts, ends, order, inverse = O.group_routing(idx, E)
    flat = idx.reshape(-1)
    assert np.array_equal(counts, [int((flat == e).sum()) for e in range(E)])
    assert np.array_equal(ends, np.cumsum(counts))
    ref_order = [f for e in range(E) for f in range(flat.size) if flat[f] == e]
    assert list(order) == ref_order
    assert np.array_equal(order[inverse], np.arange(flat.size))
    assert np.array_equal(inverse[order], np.arange(flat.size))


# ------------------------------------------------------------------ element-wise glue


def test_swiglu_against_torch_twin():
    gu = O.f32_to_bf16_bits(rng.standard_normal((64, 256)).astype(np.float32) * 4)
    t = from_bits(gu)
    # the reference's pure-torch twin, fnx/engine.py:1829
    ref = (torch.nn.functional.silu(t[:, :128].float()) * t[:, 128:].float()).to(torch.bfloat16)
    got = O.swiglu(gu)
    # exp implementations may differ in the last fp32 bit; allow rare one-step flips
    assert np.mean(got == tbits(ref)) > 0.995
    d = np.abs(O.bf16_bits_to_f32(got) - ref.float().numpy())
    assert np.all(d <= np.abs(ref.float().numpy()) * 2 ** -7 + 1e-30)


def test_weighted_reduce_cancellation_vectors():
    # tests/r118_weighted_reduce.py:38-41: only a sequential fp32 order gives these sums
    H = 4
    v = np.zeros((1, 10, H), dtype=np.float32)
    v[0, :4, 0] = [1e8, 1, -1e8, 1]
    v[0, :4, 1] = [1e8, -1e8, 1, 1]
    v[0, :, 2] = np.arange(10) * 0.5
    vb = O.f32_to_bf16_bits(v).reshape(10, H)
    w = O.f32_to_bf16_bits(np.ones((1, 10), dtype=np.float32))
    out = O.bf16_bits_to_f32(O.weighted_reduce(vb, w))
    assert out[0, 0] == 1.0 and out[0, 1] == 2.0 and out[0, 2] == 22.5
    # the pairwise order a vectorised sum might use gives 0 in column 0
    b = O.bf16_bits_to_f32(vb)[:4, 0]
    assert np.float32((b[0] + b[1]) + (b[2] + b[3])) == 0.0


def test_weighted_reduce_product_rounding_and_inverse():
    B, G, W = 7, 10, 64
    vals = O.f32_to_bf16_bits(rng.standard_normal((B * G, W)).astype(np.float32))
    w = O.f32_to_bf16_bits(rng.random((B, G)).astype(np.float32))
    # the reference's fallback composition in torch bf16 (fnx/engine.py:1851):
    # bf16 products, one fp32-accumulated sum
    ref = (from_bits(vals).view(B, G, W) * from_bits(w).unsqueeze(-1)).float().sum(1).to(torch.bfloat16)
    got = O.weighted_reduce(vals, w)
    assert np.mean(got == tbits(ref)) > 0.99
    # mode 2 (inverse gather) == mode 1 on the restored rows == scatter (tests/r100_moe_exact.py:17)
    perm = rng.permutation(B * G)
    src = vals[perm]                              # row p of src holds flat row perm[p]
    inverse = np.empty_like(perm)
    inverse[perm] = np.arange(B * G)
    assert np.array_equal(O.weighted_reduce(src, w, inverse=inverse), got)


def test_moe_merge_and_epilogue():
    H, k = 32, 10
    e = O.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
    s = O.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
    g0 = O.f32_to_bf16_bits(np.zeros(1, dtype=np.float32))
    # sigmoid(0) = 0.5 exactly: out = bf16(e + bf16(s / 2)) = bf16(e + s/2)
    out = O.moe_merge(e, s, g0)
    assert np.array_equal(out, O.f32_to_bf16_bits(O.bf16_bits_to_f32(e) + O.bf16_bits_to_f32(s) * 0.5))
    # torch formulation of kernels/post_ops/post_ops.cpp:72-94
    g = O.f32_to_bf16_bits(np.array([0.7], dtype=np.float32))
    te, ts, tg = from_bits(e), from_bits(s), from_bits(g)
    ref = (te.float() + (ts.float() * torch.sigmoid(tg.float()).to(torch.bfloat16).float()).to(torch.bfloat16).float()).to(torch.bfloat16)
    assert np.array_equal(O.moe_merge(e, s, g), tbits(ref))
    # epilogue reads only the diagonal blocks of the Cartesian product
    cart = np.full((k, k * H), 0x7FC0, dtype=np.uint16)       # NaN everywhere ...
    diag = O.f32_to_bf16_bits(rng.standard_normal((k, H)).astype(np.float32))
    for j in range(k):
        cart[j, j * H:(j + 1) * H] = diag[j]                  # ... except block (j, j)
    w = O.f32_to_bf16_bits(rng.random((1, k)).astype(np.float32))
    out = O.moe_epilogue(cart, w, s, g)
    assert not np.isnan(O.bf16_bits_to_f32(out)).any()
    # fused epilogue == reduce then merge (docs/r141-moe-epilogue.md:41)
    assert np.array_equal(out, O.moe_merge(O.weighted_reduce(diag, w), s, g))


def test_expert_gather_matches_reference_wcat():
    E, K, N, G = 6, 32, 64, 2
    w4 = rng.integers(-2**31, 2**31, size=(E, K, N // 8), dtype=np.int64).astype(np.int32)
    sc = rng.integers(0, 2**16, size=(E, G, N), dtype=np.int64).astype(np.uint16)
    ids = np.array([4, 0, 4, 2])
    ow, os_ = O.expert_gather(w4, sc, ids)
    # fnx/engine.py:661-664 / 677-679 formulation
    tw = torch.from_numpy(w4).index_select(0, torch.from_numpy(ids)).permute(1, 0, 2).contiguous().reshape(K, -1)
    ts = torch.from_numpy(sc.view(np.int16)).index_select(0, torch.from_numpy(ids)).transpose(0, 1).contiguous().view(G, -1)
    assert np.array_equal(ow, tw.numpy()) and np.array_equal(os_, ts.numpy().view(np.uint16))


# ------------------------------------------------------------------ whole block


def _layer(E, H, MI, gs, seed):
    r = np.random.default_rng(seed)
    return (r.integers(0, 2**32, size=(E, H, 2 * MI // 8), dtype=np.uint32).view(np.int32),
            O.f32_to_bf16_bits(np.abs(r.standard_normal((E, H // gs, 2 * MI))).astype(np.float32) * 0.02),
            r.integers(0, 2**32, size=(E, MI, H // 8), dtype=np.uint32).view(np.int32),
            O.f32_to_bf16_bits(np.abs(r.standard_normal((E, MI // gs, H))).astype(np.float32) * 0.02))


def test_decode_equals_prefill_for_one_token():
    E, H, MI, gs, k = 16, 64, 32, 32, 4
    gw, gsc, dw, dsc = _layer(E, H, MI, gs, 5)
    x = O.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
    lg = O.f32_to_bf16_bits(rng.standard_normal((1, E)).astype(np.float32))
    d = O.moe_decode(x, lg, gw, gsc, dw, dsc, k)
    p = O.moe_prefill(x, lg, gw, gsc, dw, dsc, k)
    assert np.array_equal(d["out"], p["out"])
    assert np.array_equal(d["idx"], p["idx"])


def test_prefill_inverse_gather_equals_scatter():
    E, H, MI, gs, k, T = 8, 64, 32, 32, 3, 9
    gw, gsc, dw, dsc = _layer(E, H, MI, gs, 7)
    x = O.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    lg = O.f32_to_bf16_bits(rng.standard_normal((T, E)).astype(np.float32))
    p = O.moe_prefill(x, lg, gw, gsc, dw, dsc, k)
    # scatter path of fnx/engine.py:1848-1852: restored = index_copy(order, yd), then (restored*w).sum(1)
    restored = np.empty_like(p["yd"])
    restored[p["order"]] = p["yd"]
    assert np.array_equal(O.weighted_reduce(restored, p["w"]), p["out"])
    # per-token loop through w4a16_gemm agrees with the grouped formulation
    for t in range(T):
        ys = []
        for j, e in enumerate(p["idx"][t]):
            gu = O.w4a16_gemm(x[t:t + 1], gw[e], gsc[e], gs)
            ys.append(O.w4a16_gemm(O.swiglu(gu), dw[e], dsc[e], gs)[0])
        assert np.array_equal(O.weighted_reduce(np.stack(ys), p["w"][t:t + 1])[0], p["out"][t])


def test_compare_metric():
    a = O.f32_to_bf16_bits(np.array([1.0, 2.0, 100.0], dtype=np.float32))
    b = O.f32_to_bf16_bits(np.array([1.0, 2.0, 100.5], dtype=np.float32))
    rel, mx, beyond = O.compare(b, a)
    assert math.isclose(mx, 0.5) and beyond == 0          # one bf16 step at 100 is 0.5
    c = O.f32_to_bf16_bits(np.array([1.0, 2.0, 102.0], dtype=np.float32))
    assert O.compare(c, a)[2] == 1


# ------------------------------------------------------------------ shared expert / router projection


def _near_boundary(v_f64, got_bits, ref_bits):
    """Positions where two bf16 roundings differ must sit on a rounding
    boundary of v (fp32 exp implementations may differ in the last place)."""
    diff = np.asarray(got_bits) != np.asarray(ref_bits)
    if diff.any():
        lo, hi = O.bf16_interval(v_f64)
        assert np.all(lo[diff] != hi[diff]), "differs away from a rounding boundary"
    return diff.mean()


def test_linear_known_answer_and_brute_force():
    # known answer: [1, 2] . [[3, 4], [0.5, -1]]^T = [11, -1.5]
    x = O.f32_to_bf16_bits(np.array([[1.0, 2.0]], np.float32))
    w = O.f32_to_bf16_bits(np.array([[3.0, 4.0], [0.5, -1.0]], np.float32))
    assert np.array_equal(O.bf16_bits_to_f32(O.linear(x, w)), np.array([[11.0, -1.5]], np.float32))
    # float64 brute force of the exact value; the fp32 result rounds it admissibly
    xb = O.f32_to_bf16_bits(rng.standard_normal((3, 37)).astype(np.float32))
    wb = O.f32_to_bf16_bits(rng.standard_normal((5, 37)).astype(np.float32))
    ex, ab = O.linear_exact(xb, wb)
    xf, wf = O.bf16_bits_to_f32(xb).astype(np.float64), O.bf16_bits_to_f32(wb).astype(np.float64)
    for m in range(3):
        for n in range(5):
            terms = [xf[m, k] * wf[n, k] for k in range(37)]
            assert ex[m, n] == pytest.approx(sum(terms), rel=1e-15, abs=1e-15)
            assert ab[m, n] == pytest.approx(sum(abs(t) for t in terms), rel=1e-15)
    lo, hi = O.bf16_interval(ex, ab)
    y = O.bf16_bits_to_f32(O.linear(xb, wb)).astype(np.float64)
    assert np.all((y >= O.bf16_bits_to_f32(lo)) & (y <= O.bf16_bits_to_f32(hi)))
    # against torch's own F.linear in float64 on the same bf16 inputs (the reference's _fl)
    t = torch.nn.functional.linear(torch.from_numpy(xf), torch.from_numpy(wf)).numpy()
    assert np.allclose(t, ex, rtol=1e-12, atol=1e-12)


def test_swiglu_bf16_matches_torch_bf16_ops():
    """fnx/engine.py:1788 is F.silu(g) * u on bf16 tensors: torch's own CPU
    bf16 arithmetic is the independent check (two roundings)."""
    MI = 257
    gu = O.f32_to_bf16_bits((rng.standard_normal((6, 2 * MI)) * 4).astype(np.float32))
    t = torch.from_numpy(gu.view(np.int16)).view(torch.bfloat16)
    ref = (torch.nn.functional.silu(t[:, :MI]) * t[:, MI:]).contiguous().view(torch.int16).numpy().view(np.uint16)
    got = O.swiglu_bf16(gu, MI)
    g = O.bf16_bits_to_f32(gu[:, :MI]).astype(np.float64)
    frac = _near_boundary(g / (1 + np.exp(-g)), got, ref)
    assert frac < 0.01
    # the fp32 npu_swiglu form rounds once and differs from the bf16 form somewhere
    assert not np.array_equal(O.swiglu(gu), got)


def test_shared_gate_matches_torch_bf16_ops():
    """fnx/engine.py:1793: torch.sigmoid(g) * sh on bf16 tensors."""
    g = O.f32_to_bf16_bits((rng.standard_normal((9, 1)) * 3).astype(np.float32))
    sh = O.f32_to_bf16_bits(rng.standard_normal((9, 40)).astype(np.float32))
    tg = torch.from_numpy(g.view(np.int16)).view(torch.bfloat16)
    ts = torch.from_numpy(sh.view(np.int16)).view(torch.bfloat16)
    ref = (torch.sigmoid(tg) * ts).contiguous().view(torch.int16).numpy().view(np.uint16)
    got = O.shared_gate(sh, g)
    gf = O.bf16_bits_to_f32(g).astype(np.float64)
    sig = np.broadcast_to(1 / (1 + np.exp(-gf)), sh.shape)
    _near_boundary(sig, got, ref)


def test_shared_router_layout():
    """The fused projection's column blocks (fnx/engine.py:1226-1241 merge
    order gate, up, gate2, router): each block of gu is the linear of x with
    the matching rows, and logits/gate2 are its last E+1 columns."""
    H, MI, E = 16, 8, 5
    x = O.f32_to_bf16_bits(rng.standard_normal((2, H)).astype(np.float32))
    parts = [O.f32_to_bf16_bits(rng.standard_normal((n, H)).astype(np.float32) * 0.1) for n in (MI, MI, 1, E)]
    sh_gu = np.concatenate(parts, axis=0)
    sh_down = O.f32_to_bf16_bits(rng.standard_normal((H, MI)).astype(np.float32) * 0.1)
    gu, act, sh, g2, lg = O.shared_router(x, sh_gu, sh_down, MI)
    assert np.array_equal(gu[:, :MI], O.linear(x, parts[0]))
    assert np.array_equal(gu[:, MI:2 * MI], O.linear(x, parts[1]))
    assert np.array_equal(g2, O.linear(x, parts[2]))
    assert np.array_equal(lg, O.linear(x, parts[3]))
    assert np.array_equal(act, O.swiglu_bf16(np.concatenate([gu[:, :MI], gu[:, MI:2 * MI]], axis=1), MI))
    assert np.array_equal(sh, O.linear(act, sh_down))


# ------------------------------------------------------------------ W8A16 (DenseW8)


def test_w8a16_known_answer_and_brute_force():
    # x = [1, -2], q = [[3, -128], [127, 1]], S = [[0.5, 2]] (gs = 2): y = [(3 - 254) * 0.5, (-128 - 2) * 2]
    x = O.f32_to_bf16_bits(np.array([[1.0, -2.0]], np.float32))
    q = np.array([[3, -128], [127, 1]], np.int8)
    S = O.f32_to_bf16_bits(np.array([[0.5, 2.0]], np.float32))
    y = O.bf16_bits_to_f32(O.w8a16_gemm(x, q, S, 2))
    assert np.array_equal(y, np.array([[-125.5, -260.0]], np.float32))
    xb = O.f32_to_bf16_bits(rng.standard_normal((2, 24)).astype(np.float32))
    qb = rng.integers(-128, 128, size=(24, 6)).astype(np.int8)
    Sb = O.f32_to_bf16_bits(np.abs(rng.standard_normal((3, 6))).astype(np.float32) * 0.01)
    ex, ab = O.w8a16_gemm_exact(xb, qb, Sb, 8)
    xf, Sf = O.bf16_bits_to_f32(xb).astype(np.float64), O.bf16_bits_to_f32(Sb).astype(np.float64)
    for m in range(2):
        for n in range(6):
            terms = [xf[m, k] * float(qb[k, n]) * Sf[k // 8, n] for k in range(24)]
            assert ex[m, n] == pytest.approx(sum(terms), rel=1e-14, abs=1e-14)
            assert ab[m, n] == pytest.approx(sum(abs(t) for t in terms), rel=1e-14)


def test_dense_w8_container_matches_reference_formula():
    """fnx/engine.py:318-328 with torch: w8t = q[:, :K].t(), sc = s[:, :K/gs].t().to(bf16)."""
    N, Kp, K, gs = 12, 136, 128, 8
    q = rng.integers(-128, 128, size=(N, Kp)).astype(np.int8)
    s = (rng.random((N, Kp // gs)) * 0.01).astype(np.float16)
    w8t, sc, g = O.dense_w8_from_qs(q, s, K)
    tq, ts = torch.from_numpy(q), torch.from_numpy(s)
    assert g == gs
    assert np.array_equal(w8t, tq[:, :K].t().contiguous().numpy())
    assert np.array_equal(sc, tbits(ts[:, :K // gs].t().contiguous().to(torch.bfloat16)))
    with pytest.raises(ValueError):
        O.dense_w8_from_qs(q, s, K=130)


# ------------------------------------------------------------------ float64 checkers used by the GPU tests


def test_w4a16_gemm_exact_brute_force():
    """The float64 reference point of the GPU rounding checks against a triple
    loop over independently decoded weights, with non-uniform scales so a
    swapped group or column index fails; the absolute sums likewise."""
    M, K, N, gs = 3, 96, 24, 32
    q = rng.integers(-8, 8, size=(K, N)).astype(np.int8)
    s = O.f32_to_bf16_bits((np.arange(K // gs)[:, None] + 1) * (np.arange(N)[None, :] + 2) * 0.01)
    x = O.f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    ex, ab = O.w4a16_gemm_exact(x, O.pack_int4(q), s, gs)
    xf, sf = O.bf16_bits_to_f32(x), O.bf16_bits_to_f32(s)
    assert np.allclose(ex, _brute_w4a16(xf, q, sf, gs), rtol=1e-13, atol=1e-13)
    brute_abs = _brute_w4a16(np.abs(xf), np.abs(q.astype(np.int64)), sf, gs)
    assert np.allclose(ab, brute_abs, rtol=1e-13, atol=1e-13)
    # the fp32 GEMM rounds the exact value admissibly
    lo, hi = O.bf16_interval(ex, ab)
    y = O.w4a16_gemm(x, O.pack_int4(q), s, gs)
    yv, lov, hiv = (O.bf16_bits_to_f32(b) for b in (y, lo, hi))
    assert np.all((yv >= lov) & (yv <= hiv))


def test_grouped_gemm_exact_equals_per_row():
    E, K, N, gs = 4, 64, 16, 32
    w4 = np.stack([O.pack_int4(rng.integers(-8, 8, size=(K, N)).astype(np.int8)) for _ in range(E)])
    sc = O.f32_to_bf16_bits(np.abs(rng.standard_normal((E, K // gs, N))).astype(np.float32) * 0.02)
    counts = np.array([2, 0, 3, 1])
    ends = np.cumsum(counts)
    x = O.f32_to_bf16_bits(rng.standard_normal((int(ends[-1]) + 2, K)).astype(np.float32))  # 2 rows past the end
    ex, ab = O.grouped_gemm_exact(x, w4, sc, ends)
    e_of_row = np.repeat(np.arange(E), counts)
    for p in range(int(ends[-1])):
        e1, a1 = O.w4a16_gemm_exact(x[p:p + 1], w4[e_of_row[p]], sc[e_of_row[p]], gs)
        assert np.array_equal(ex[p], e1[0]) and np.array_equal(ab[p], a1[0])
    assert np.all(ex[int(ends[-1]):] == 0) and np.all(ab[int(ends[-1]):] == 0)


def test_router_weights_exact_brute_force():
    T, E, k = 3, 24, 5
    logits = O.f32_to_bf16_bits(rng.standard_normal((T, E)).astype(np.float32) * 3)
    idx, _ = O.router(logits, k)
    got = O.router_weights_exact(logits, idx)
    lf = O.bf16_bits_to_f32(logits)
    for t in range(T):
        z = sum(math.exp(float(v)) for v in lf[t])
        p = [math.exp(float(lf[t, e])) / z for e in idx[t]]
        for j in range(k):
            assert got[t, j] == pytest.approx(p[j] / sum(p), rel=1e-12)
    # a plausible slip (weights not renormalised over the selection) is caught
    assert not np.allclose(got[0].sum(), 1.0 - 1e-3)
    assert np.allclose(got.sum(axis=1), 1.0)


def test_bf16_interval_and_swiglu_interval():
    """bf16_interval is one value away from a rounding boundary and contains
    the nearest-even rounding; swiglu_interval contains the SwiGLU of every
    admissible gate/up rounding and rejects swapped halves."""
    v = rng.standard_normal(4000) * 10
    lo, hi = O.bf16_interval(v)
    r = O.f32_to_bf16_bits(v.astype(np.float32))
    assert np.all(O.bf16_bits_to_f32(lo) <= O.bf16_bits_to_f32(r))
    assert np.all(O.bf16_bits_to_f32(r) <= O.bf16_bits_to_f32(hi))
    assert np.mean(lo != hi) < 0.03                     # two-valued only near a boundary (~1%)
    # a value exactly half-way between two bf16 neighbours is two-valued
    mid = (float(O.bf16_bits_to_f32(np.array([0x3F80], np.uint16))[0]) +
           float(O.bf16_bits_to_f32(np.array([0x3F81], np.uint16))[0])) / 2
    l2, h2 = O.bf16_interval(np.array([mid]))
    assert (int(l2[0]), int(h2[0])) == (0x3F80, 0x3F81)
    g = rng.standard_normal(2000) * 4
    u = rng.standard_normal(2000) * 4
    slo, shi = O.swiglu_interval(g, np.abs(g), u, np.abs(u))
    gb, ub = O.f32_to_bf16_bits(g.astype(np.float32)), O.f32_to_bf16_bits(u.astype(np.float32))
    act = O.swiglu(np.concatenate([gb, ub])[None, :])
    av = O.bf16_bits_to_f32(act[0])
    assert np.all((av >= O.bf16_bits_to_f32(slo)) & (av <= O.bf16_bits_to_f32(shi)))
    swapped = O.bf16_bits_to_f32(O.swiglu(np.concatenate([ub, gb])[None, :])[0])
    outside = (swapped < O.bf16_bits_to_f32(slo)) | (swapped > O.bf16_bits_to_f32(shi))
    assert np.mean(outside) > 0.5


# ------------------------------------------------------------------ element-wise output bounds


def _tiny_layer(E=8, H=64, MI=32, gs=32, seed=5):
    r = np.random.default_rng(seed)
    gu_w = np.stack([O.pack_int4(r.integers(-8, 8, size=(H, 2 * MI)).astype(np.int8)) for _ in range(E)])
    dn_w = np.stack([O.pack_int4(r.integers(-8, 8, size=(MI, H)).astype(np.int8)) for _ in range(E)])
    gu_s = O.f32_to_bf16_bits(np.abs(r.standard_normal((E, H // gs, 2 * MI))).astype(np.float32) * 0.05)
    dn_s = O.f32_to_bf16_bits(np.abs(r.standard_normal((E, MI // gs, H))).astype(np.float32) * 0.05)
    return gu_w, gu_s, dn_w, dn_s


def _f32_gemm_in_order(x, w, order):
    """fp32 accumulation of x @ w with the k terms added in the given order."""
    acc = np.zeros((x.shape[0], w.shape[1]), dtype=np.float32)
    for kk in order:
        acc = acc + (x[:, kk:kk + 1] * w[kk:kk + 1, :]).astype(np.float32)
    return acc


def _block_any_order(x_bits, lg, k, lay, rs):
    """The expert block with every GEMM accumulated in a random order."""
    gu_w, gu_s, dn_w, dn_s = lay
    idx, w = O.router(lg, k)
    T, H = x_bits.shape
    MI = dn_w.shape[1]
    out = np.zeros((T, H), dtype=np.float32)
    for t in range(T):
        acc = np.zeros(H, dtype=np.float32)
        for j in range(k):
            e = idx[t, j]
            cu = O.dequant(gu_w[e], gu_s[e], H // gu_s.shape[1])
            gu = O.f32_to_bf16_bits(_f32_gemm_in_order(O.bf16_bits_to_f32(x_bits[t:t + 1]), cu, rs.permutation(H)))
            act = O.swiglu(gu)
            cd = O.dequant(dn_w[e], dn_s[e], MI // dn_s.shape[1])
            y = O.round_bf16(_f32_gemm_in_order(O.bf16_bits_to_f32(act), cd, rs.permutation(MI)))[0]
            acc = acc + O.round_bf16(y * O.bf16_bits_to_f32(w[t, j]))
        out[t] = acc
    return O.f32_to_bf16_bits(out)


def _inside(got_bits, lo, hi):
    g, l, h = (O.bf16_bits_to_f32(np.asarray(b).view(np.uint16)) for b in (got_bits, lo, hi))
    return (g >= l) & (g <= h)


def test_output_interval_contains_every_summation_order():
    """Soundness: the block computed with every GEMM summed in random orders
    (the only freedom two correct implementations have) always lands inside
    the bounds, and so do the oracle's decode and prefill outputs."""
    lay = _tiny_layer()
    E, k, T = 8, 3, 4
    r = np.random.default_rng(11)
    x = O.f32_to_bf16_bits(r.standard_normal((T, 64)).astype(np.float32) * 2)
    lg = O.f32_to_bf16_bits(r.standard_normal((T, E)).astype(np.float32))
    idx, _ = O.router(lg, k)
    lo, hi = O.moe_output_interval(x, idx, lg, *lay)
    ref = O.moe_prefill(x, lg, *lay, k)
    assert np.all(_inside(ref["out"], lo, hi))
    rs = np.random.default_rng(3)
    for _ in range(12):
        assert np.all(_inside(_block_any_order(x, lg, k, lay, rs), lo, hi))
    # the decode form with the sigmoid-gated shared merge, token by token
    sh = O.f32_to_bf16_bits(r.standard_normal((T, 64)).astype(np.float32))
    gate = O.f32_to_bf16_bits(r.standard_normal(T).astype(np.float32))
    lo2, hi2 = O.moe_output_interval(x, idx, lg, *lay, shared_bits=sh, gate_bits=gate)
    for t in range(T):
        d = O.moe_decode(x[t], lg[t], *lay, k, shared_bits=sh[t:t + 1], gate_bits=gate[t])
        assert np.all(_inside(d["out"], lo2[t:t + 1], hi2[t:t + 1]))
    # and the bounds are tight: one value away from rounding boundaries
    assert np.mean(lo != hi) < 0.5


def test_output_interval_rejects_planted_mistakes():
    """A dropped routing weight, swapped gate/up halves or a wrong expert put
    most outputs outside the bounds."""
    gu_w, gu_s, dn_w, dn_s = lay = _tiny_layer(seed=6)
    E, k, T = 8, 3, 4
    r = np.random.default_rng(12)
    x = O.f32_to_bf16_bits(r.standard_normal((T, 64)).astype(np.float32) * 2)
    lg = O.f32_to_bf16_bits(r.standard_normal((T, E)).astype(np.float32))
    idx, w = O.router(lg, k)
    lo, hi = O.moe_output_interval(x, idx, lg, *lay)
    ones = O.f32_to_bf16_bits(np.ones_like(O.bf16_bits_to_f32(w)))
    # no routing weight
    bad = O.moe_prefill(x, lg, *lay, k)
    unweighted = O.weighted_reduce(O.f32_to_bf16_bits(O.bf16_bits_to_f32(bad["yd"])[bad["inverse"]]), ones)
    assert np.mean(_inside(unweighted, lo, hi)) < 0.2
    # gate and up halves swapped
    swapped_gu = np.concatenate([gu_s[:, :, 32:], gu_s[:, :, :32]], axis=2)
    swapped_w = np.stack([O.pack_int4(np.concatenate([O.unpack_int4(m)[:, 32:], O.unpack_int4(m)[:, :32]], axis=1))
                          for m in gu_w])
    sw = O.moe_prefill(x, lg, swapped_w, swapped_gu, dn_w, dn_s, k)["out"]
    assert np.mean(_inside(sw, lo, hi)) < 0.2
    # slot 0 of every token on the next expert
    idx2 = idx.copy()
    idx2[:, 0] = (idx2[:, 0] + 1) % E
    lo2, hi2 = O.moe_output_interval(x, idx2, lg, *lay)
    assert np.mean(_inside(O.moe_prefill(x, lg, *lay, k)["out"], lo2, hi2)) < 0.2


def test_expert_threads_do_not_change_results():
    """The per-expert loops give the same arrays on one thread and on several
    (each expert writes only its own rows)."""
    r = np.random.default_rng(77)
    E, H, MI, gs, k, T = 12, 128, 64, 32, 3, 40
    gu_w = r.integers(0, 2**32, size=(E, H, 2 * MI // 8), dtype=np.uint32).view(np.int32)
    gu_s = O.f32_to_bf16_bits(np.abs(r.standard_normal((E, H // gs, 2 * MI))).astype(np.float32) * 0.02)
    dn_w = r.integers(0, 2**32, size=(E, MI, H // 8), dtype=np.uint32).view(np.int32)
    dn_s = O.f32_to_bf16_bits(np.abs(r.standard_normal((E, MI // gs, H))).astype(np.float32) * 0.02)
    x = O.f32_to_bf16_bits(r.standard_normal((T, H)).astype(np.float32))
    lg = O.f32_to_bf16_bits(r.standard_normal((T, E)).astype(np.float32))

    def run():
        ref = O.moe_prefill(x, lg, gu_w, gu_s, dn_w, dn_s, k)
        ex = O.grouped_gemm_exact(x[ref["order"] // k], gu_w, gu_s, ref["ends"])
        return ref, ex, O.moe_output_interval(x, ref["idx"], lg, gu_w, gu_s, dn_w, dn_s)

    prev = O.set_workers(1)
    try:
        a = run()
        O.set_workers(4)
        b = run()
    finally:
        O.set_workers(prev)
    for key in ("gu", "act", "yd", "out", "mag"):
        assert np.array_equal(a[0][key], b[0][key]), key
    for u, v in zip(a[1] + a[2], b[1] + b[2]):
        assert np.array_equal(u, v)
