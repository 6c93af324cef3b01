"""The reference's own MoE call sequences run unmodified through qmoe.

``FnLayer._moe`` (fnx/engine.py:1782-1930) calls the expert container and the
glue modules in two ways on the W4A16 path:

* decode, b == 1 (1859-1891): ``exp_gu.apply(x2, idx[0])`` -> ``npu_swiglu`` ->
  the Cartesian ``exp_dn.apply(act, idx[0])`` -> ``moe_epilogue.merge``, or
  ``exp_dn.apply_diag`` -> ``weighted_reduce.reduce`` -> ``post_ops.moe_merge``;
* grouped prefill, b > 1 (1815-1853): ``apply_grouped`` x2 around the SwiGLU,
  then ``weighted_reduce.reduce(yd, w, inverse=inverse)`` and ``+ sh``.

Here the same sequences run against :class:`qmoe.ExpW4` built with the
reference's constructor ``(w4, s8t, base, gs, expert_major)`` in both artifact
layouts, and are compared stage by stage with the oracle, with each other and
with the fused kernels (``moe_decode`` / ``moe_prefill`` / ``moe_experts``).
"""
import numpy as np
import pytest
import torch

from gpu_util import bf16_normal, int4_words, log
from oracle import qmoe_oracle as O
from parity import assert_block_output, assert_bf16_equal, assert_equal_off_boundary, assert_in_interval, bits, to_dev


def artifact_layer(E, H, MI, gs, seed):
    """One layer in the W4A16 artifact form: expert-major int4pack words, s8t
    int8 [G, E, N], base bf16 [E, N] (tools/repack_w4a16.py:13-15), and the
    oracle's composed scales [E, G, N]."""
    r = np.random.default_rng(seed)
    lay = {}
    for name, (K, N) in (("gu", (H, 2 * MI)), ("dn", (MI, H))):
        w = int4_words((E, K, N // 8), seed + len(name) + K)
        s8t = r.integers(-127, 128, size=(K // gs, E, N)).astype(np.int8)
        base = O.f32_to_bf16_bits((r.random((E, N)) * 4e-4 + 1e-4).astype(np.float32))
        lay[name] = dict(w=w, s8t=s8t, base=base, s=O.compose_scales(s8t, base))
    return lay


def containers(lay, gs, device, expert_major):
    from qmoe import ExpW4
    out = []
    for name in ("gu", "dn"):
        p = lay[name]
        w = p["w"] if expert_major else np.ascontiguousarray(p["w"].transpose(1, 0, 2))
        out.append(ExpW4(to_dev(w, device), to_dev(p["s8t"], device), to_dev(p["base"], device), gs,
                         expert_major=expert_major))
    return out


def decode_cartesian(x2, logits, exp_gu, exp_dn, k, sh, gate):
    """fnx/engine.py:1859-1876 with the production flags (epilogue path)."""
    from qmoe import router_topk, swiglu
    from qmoe.moe_epilogue import merge
    idx, w = router_topk(logits, k)
    y = exp_gu.apply(x2, idx[0]).view(k, -1)
    act = swiglu(y)
    cartesian = exp_dn.apply(act, idx[0])
    return merge(cartesian, w, sh, gate), dict(idx=idx, w=w, y=y, act=act, cartesian=cartesian)


def decode_diag(x2, logits, exp_gu, exp_dn, k, sh, gate):
    """fnx/engine.py:1877-1891: apply_diag, weighted_reduce.reduce, post_ops.moe_merge."""
    from qmoe import router_topk, swiglu
    from qmoe.post_ops import moe_merge
    from qmoe.weighted_reduce import reduce
    idx, w = router_topk(logits, k)
    act = swiglu(exp_gu.apply(x2, idx[0]).view(k, -1))
    y2 = exp_dn.apply_diag(act, idx[0])
    reduced = reduce(y2, w)
    return moe_merge(reduced, sh, gate.reshape(1)), dict(y2=y2, reduced=reduced, act=act)


def prefill_grouped(x2, logits, exp_gu, exp_dn, k, sh):
    """fnx/engine.py:1815-1853 with FNX_MOE_GROUP=1, FNX_MOE_INVERSE=1, FNX_MOE_REDUCE=1
    (the routing glue through qmoe.route_group: a stable expert-major order)."""
    from qmoe import route_group, router_topk, swiglu
    from qmoe.weighted_reduce import reduce
    idx, w = router_topk(logits, k)
    counts, ends, order, inverse = route_group(idx, exp_gu.E)
    rows = x2.index_select(0, order // k)
    gu = exp_gu.apply_grouped(rows, ends)
    act = swiglu(gu)
    yd = exp_dn.apply_grouped(act, ends)
    y = reduce(yd, w, inverse=inverse)
    return y + sh, dict(idx=idx, w=w, order=order, ends=ends, gu=gu, act=act, yd=yd)


@pytest.mark.gpu
def test_container_selection_both_layouts(device):
    """_scales, _wcat and _scat of both layouts against the oracle's scale
    composition and gather (fnx/engine.py:653-689)."""
    E, H, MI, gs = 64, 512, 128, 64
    log("ExpW4 selection, both layouts")
    lay = artifact_layer(E, H, MI, gs, 3)
    ids = np.array([3, 17, 61, 0, 63, 40, 41, 2], dtype=np.int64)
    idd = to_dev(ids, device)
    for em in (True, False):
        gu, dn = containers(lay, gs, device, em)
        for exp, p in ((gu, lay["gu"]), (dn, lay["dn"])):
            assert (exp.K, exp.N, exp.E, exp.G, exp.gs, exp.expert_major) == \
                (p["w"].shape[1], p["w"].shape[2] * 8, E, p["w"].shape[1] // gs, gs, em)
            assert exp.s8t is None and exp.base is None
            assert np.array_equal(bits(exp._scales), p["s"])
            ow, osc = O.expert_gather(p["w"], p["s"], ids)
            assert np.array_equal(exp._wcat(idd).cpu().numpy(), ow)
            assert np.array_equal(bits(exp._scat(idd)), osc)
    gu_km, _ = containers(lay, gs, device, False)
    with pytest.raises(RuntimeError):
        gu_km.apply_grouped(torch.zeros((4, H), dtype=torch.bfloat16, device=device),
                            torch.full((E,), 4, dtype=torch.int64, device=device))


@pytest.mark.gpu
@pytest.mark.parametrize("E,H,MI,gs,k", [(512, 2048, 512, 128, 10), (64, 512, 128, 64, 8)])
def test_decode_sequences(device, E, H, MI, gs, k):
    from qmoe import moe_decode, moe_experts
    log(f"_moe decode sequences E={E} H={H} MI={MI} k={k}")
    lay = artifact_layer(E, H, MI, gs, E + H)
    x = bf16_normal((1, H), 7)
    lg = bf16_normal((1, E), 8)
    sh = bf16_normal((1, H), 9)
    gate = bf16_normal((1, 1), 10)
    xd, lgd, shd, gd = (to_dev(a, device) for a in (x, lg, sh, gate))
    ref = O.moe_decode(x[0], lg[0], lay["gu"]["w"], lay["gu"]["s"], lay["dn"]["w"], lay["dn"]["s"], k,
                       shared_bits=sh, gate_bits=gate[0])
    bounds = O.moe_output_interval(x, ref["idx"], lg, lay["gu"]["w"], lay["gu"]["s"], lay["dn"]["w"], lay["dn"]["s"],
                                   shared_bits=sh, gate_bits=gate[0])
    results = {}
    for em in (True, False):
        gu, dn = containers(lay, gs, device, em)
        out, st = decode_cartesian(xd, lgd, gu, dn, k, shd, gd)
        out2, st2 = decode_diag(xd, lgd, gu, dn, k, shd, gd)
        torch.cuda.synchronize()
        tag = "expert-major" if em else "K-major"
        assert np.array_equal(st["idx"][0].cpu().numpy(), ref["idx"][0])
        # stage 1: gate_up of the k selected experts (concatenated along N)
        y = bits(st["y"])
        for j, e in enumerate(ref["idx"][0]):
            ex, ab = O.w4a16_gemm_exact(x, lay["gu"]["w"][e], lay["gu"]["s"][e], gs)
            assert_in_interval(y[j:j + 1], *O.bf16_interval(ex, ab), f"{tag} gate_up expert {j}")
        # stage 2: SwiGLU of the GPU's own gate_up rows
        yf = O.bf16_bits_to_f32(y).astype(np.float64)
        exact = yf[:, :MI] / (1.0 + np.exp(-yf[:, :MI])) * yf[:, MI:]
        act = bits(st["act"])
        assert_equal_off_boundary(act, O.swiglu(y), exact, f"{tag} swiglu")
        # stage 3: the diagonal blocks of the Cartesian down projection, and apply_diag
        cart = bits(st["cartesian"]).reshape(k, k, H)
        diag = np.stack([cart[j, j] for j in range(k)])
        y2 = bits(st2["y2"])
        for j, e in enumerate(ref["idx"][0]):
            ex, ab = O.w4a16_gemm_exact(act[j:j + 1], lay["dn"]["w"][e], lay["dn"]["s"][e], gs)
            lo, hi = O.bf16_interval(ex, ab)
            assert_in_interval(diag[j:j + 1], lo, hi, f"{tag} cartesian diagonal {j}")
            assert_in_interval(y2[j:j + 1], lo, hi, f"{tag} apply_diag row {j}")
        # stage 4: the epilogue is reduce + merge, bit for bit, on the same rows
        from qmoe.post_ops import moe_merge
        from qmoe.weighted_reduce import reduce
        w = st["w"]
        via_glue = moe_merge(reduce(to_dev(diag, device), w), shd, gd.reshape(1))
        torch.cuda.synchronize()
        assert_bf16_equal(out, bits(via_glue), f"{tag} epilogue == reduce + moe_merge")
        assert_bf16_equal(st2["reduced"], O.weighted_reduce(y2, bits(w)), f"{tag} reduce of apply_diag rows")
        # end to end, both sequences
        assert_block_output(out, ref["out"], bounds, f"{tag} cartesian sequence end-to-end", mag=ref["mag"])
        assert_block_output(out2, ref["out"], bounds, f"{tag} diag sequence end-to-end", mag=ref["mag"])
        results[em] = (bits(out), bits(out2))
    # the two layouts hold the same words: same bits
    assert np.array_equal(results[True][0], results[False][0])
    assert np.array_equal(results[True][1], results[False][1])
    # the fused decode block and the dispatcher, on the same container
    gu, dn = containers(lay, gs, device, True)
    fused = moe_decode(xd, lgd, gu, dn, k, shd, gd)[0]
    disp = moe_experts(xd, lgd, gu, dn, k, shd, gd)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), disp.view(torch.int16))
    assert_block_output(fused, ref["out"], bounds, "fused decode end-to-end", mag=ref["mag"])
    assert_block_output(fused, results[True][0], bounds, "fused decode vs the reference's sequence")


@pytest.mark.gpu
@pytest.mark.parametrize("T,E,H,MI,gs,k", [(64, 64, 512, 128, 64, 8), (300, 512, 2048, 512, 128, 10)])
def test_prefill_sequence(device, T, E, H, MI, gs, k):
    from qmoe import moe_experts, moe_prefill
    log(f"_moe grouped prefill sequence T={T} E={E} H={H}")
    lay = artifact_layer(E, H, MI, gs, T + E)
    x = bf16_normal((T, H), 11)
    lg = bf16_normal((T, E), 12)
    sh = bf16_normal((T, H), 13)
    xd, lgd, shd = (to_dev(a, device) for a in (x, lg, sh))
    gu, dn = containers(lay, gs, device, True)
    out, st = prefill_grouped(xd, lgd, gu, dn, k, shd)
    fused = moe_prefill(xd, lgd, gu, dn, k, shd)
    disp = moe_experts(xd, lgd, gu, dn, k, shd)
    torch.cuda.synchronize()
    ref = O.moe_prefill(x, lg, lay["gu"]["w"], lay["gu"]["s"], lay["dn"]["w"], lay["dn"]["s"], k, shared_bits=sh)
    assert np.array_equal(st["idx"].cpu().numpy(), ref["idx"])
    assert np.array_equal(st["order"].cpu().numpy(), ref["order"])
    assert np.array_equal(st["ends"].cpu().numpy(), ref["ends"])
    # stage-wise: the grouped gate_up, SwiGLU of the GPU's rows, grouped down
    gub = bits(st["gu"])
    ge, ga = O.grouped_gemm_exact(x[ref["order"] // k], lay["gu"]["w"], lay["gu"]["s"], ref["ends"])
    assert_in_interval(gub, *O.bf16_interval(ge, ga), "prefill gate_up")
    gf = O.bf16_bits_to_f32(gub).astype(np.float64)
    act = bits(st["act"])
    assert_equal_off_boundary(act, O.swiglu(gub), gf[:, :MI] / (1.0 + np.exp(-gf[:, :MI])) * gf[:, MI:],
                              "prefill swiglu")
    ye, ya = O.grouped_gemm_exact(act, lay["dn"]["w"], lay["dn"]["s"], ref["ends"])
    assert_in_interval(bits(st["yd"]), *O.bf16_interval(ye, ya), "prefill down")
    # the fused prefill block keeps the same rounding points: the same bits
    assert_bf16_equal(fused, bits(out), "fused prefill == the reference's sequence")
    assert torch.equal(fused.view(torch.int16), disp.view(torch.int16))
    bounds = O.moe_output_interval(x, ref["idx"], lg, lay["gu"]["w"], lay["gu"]["s"], lay["dn"]["w"], lay["dn"]["s"],
                                   shared_bits=sh)
    assert_block_output(out, ref["out"], bounds, "prefill sequence end-to-end", mag=ref["mag"])
