"""Fused MoE expert block (decode and grouped prefill) vs the oracle."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_normal, check_expert_rows, layer, layer_dev, log, prod_interval
from oracle import qmoe_oracle as O
from parity import assert_block_output, assert_bf16_equal, assert_in_interval, assert_rounds_exactly, bits, to_dev


@pytest.mark.gpu
@pytest.mark.parametrize("B,E,H,MI,gs,k", [
    (1, 512, 2048, 512, 128, 10),    # the decode workload: 512 experts, top-10
    (4, 512, 2048, 512, 128, 10),    # batch-4 decode step of the 48-layer workload (one layer)
    (2, 64, 256, 128, 64, 8),
    (3, 16, 512, 96, 32, 4),         # MI not a multiple of 128
    (1, 640, 512, 128, 64, 8),       # one token, more than 512 experts (routing through the shared plan)
    (1, 64, 352, 64, 32, 16),        # k = 16; H not a multiple of 64 (a partial last column tile)
    (2, 128, 768, 256, 64, 6),       # two tokens; H a multiple of 256 but not of 2048
    (4, 256, 512, 128, 64, 16),      # four tokens x top-16: 64 (token, slot) pairs, the most a call holds
    (3, 64, 352, 64, 32, 8),         # several tokens, H not a multiple of 256 (a partial wide down tile)
    (3, 640, 512, 128, 64, 8),       # more than 512 experts: the shared plan and the four-row kernel
    (2, 1024, 256, 128, 64, 4),      # the two-row kernel
])
def test_moe_decode(device, B, E, H, MI, gs, k):
    from qmoe import moe_decode
    log(f"moe_decode B={B} E={E} H={H} MI={MI} gs={gs} k={k}")
    lay = layer(E, H, MI, gs, 100 * B + E)
    gu, dn = layer_dev(lay, device)
    x = bf16_normal((B, H), 1)
    lg = bf16_normal((B, E), 2)
    out, idx, w, (act, prod) = moe_decode(to_dev(x, device), to_dev(lg, device), gu, dn, k,
                                          return_intermediates=True)
    torch.cuda.synchronize()
    ab, pb, ob = bits(act), bits(prod), bits(out)
    for t in range(B):
        ref = O.moe_decode(x[t], lg[t], lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"], k)
        assert np.array_equal(idx[t].cpu().numpy(), ref["idx"][0])
        assert_rounds_exactly(w[t:t + 1], O.router_weights_exact(lg[t:t + 1], ref["idx"]), None, "router weights")
        check_expert_rows(np.repeat(x[t:t + 1], k, 0), ref["idx"][0], ref["w"][0], ab[t], pb[t], lay, gs, gs,
                          f"decode token {t}")
        ones = O.f32_to_bf16_bits(np.ones((1, k), np.float32))
        assert_bf16_equal(ob[t:t + 1], O.weighted_reduce(pb[t], ones), f"decode token {t} slot sum")
        bounds = O.moe_output_interval(x[t:t + 1], ref["idx"], lg[t:t + 1], lay["gu_w"], lay["gu_s"], lay["dn_w"],
                                       lay["dn_s"])
        assert_block_output(ob[t:t + 1], ref["out"], bounds, f"decode token {t} end-to-end", mag=ref["mag"])


@pytest.mark.gpu
def test_moe_decode_shared_experts_and_merge(device):
    """Tokens with identical logits share all their experts (multiplicity 2..4 rows
    per expert), and the shared-expert merge runs in the same epilogue."""
    from qmoe import moe_decode
    log("moe_decode shared experts + merge")
    E, H, MI, gs, k, B = 32, 512, 128, 64, 6, 4
    lay = layer(E, H, MI, gs, 77)
    gu, dn = layer_dev(lay, device)
    x = bf16_normal((B, H), 5)
    lg = bf16_normal((B, E), 6)
    lg[1] = lg[0]
    lg[3] = lg[0]
    sh = bf16_normal((B, H), 7)
    sg = bf16_normal((B, 1), 8)
    out, idx, w, (act, prod) = moe_decode(to_dev(x, device), to_dev(lg, device), gu, dn, k, to_dev(sh, device),
                                          to_dev(sg, device), return_intermediates=True)
    torch.cuda.synchronize()
    ab, pb, ob = bits(act), bits(prod), bits(out)
    ones = O.f32_to_bf16_bits(np.ones((1, k), np.float32))
    for t in range(B):
        ref = O.moe_decode(x[t], lg[t], lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"], k,
                           shared_bits=sh[t:t + 1], gate_bits=sg[t])
        assert np.array_equal(idx[t].cpu().numpy(), ref["idx"][0])
        check_expert_rows(np.repeat(x[t:t + 1], k, 0), ref["idx"][0], ref["w"][0], ab[t], pb[t], lay, gs, gs,
                          f"decode+merge token {t}")
        merged = O.moe_merge(O.weighted_reduce(pb[t], ones), sh[t:t + 1], sg[t])
        assert_bf16_equal(ob[t:t + 1], merged, f"decode+merge token {t} merge")
        bounds = O.moe_output_interval(x[t:t + 1], ref["idx"], lg[t:t + 1], lay["gu_w"], lay["gu_s"], lay["dn_w"],
                                       lay["dn_s"], shared_bits=sh[t:t + 1], gate_bits=sg[t])
        assert_block_output(ob[t:t + 1], ref["out"], bounds, f"decode+merge token {t} end-to-end", mag=ref["mag"])


@pytest.mark.gpu
@pytest.mark.parametrize("T,E,H,MI,gs,k,zipf", [
    (9, 8, 256, 64, 64, 3, None),
    (64, 64, 512, 128, 128, 10, 1.1),
    (512, 512, 2048, 512, 128, 10, 1.1),   # the 512-token Zipf prefill workload
])
def test_moe_prefill(device, T, E, H, MI, gs, k, zipf):
    from qmoe import moe_prefill
    from qmoe.workload import zipf_logits
    log(f"moe_prefill T={T} E={E} H={H} MI={MI} gs={gs} k={k} zipf={zipf}")
    lay = layer(E, H, MI, gs, 7 * T + E)
    gu, dn = layer_dev(lay, device)
    x = bf16_normal((T, H), 3)
    lg = zipf_logits(T, E, zipf, 4) if zipf else bf16_normal((T, E), 4)
    out, (idx, w, counts, ends, order, inverse), (act, prod) = moe_prefill(
        to_dev(x, device), to_dev(lg, device), gu, dn, k, return_routing=True, return_intermediates=True)
    torch.cuda.synchronize()
    ref = O.moe_prefill(x, lg, lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"], k)
    assert np.array_equal(idx.cpu().numpy(), ref["idx"])
    assert np.array_equal(counts.cpu().numpy(), ref["counts"])
    assert np.array_equal(ends.cpu().numpy(), ref["ends"])
    assert np.array_equal(order.cpu().numpy(), ref["order"])
    assert np.array_equal(inverse.cpu().numpy(), ref["inverse"])
    assert_rounds_exactly(w, O.router_weights_exact(lg, ref["idx"]), None, "router weights")
    ab, pb, ob = bits(act), bits(prod), bits(out)
    # stage 1: gate_up + SwiGLU on the permuted rows, from the true inputs
    ge, ga = O.grouped_gemm_exact(x[ref["order"] // k], lay["gu_w"], lay["gu_s"], ref["ends"])
    assert_in_interval(ab, *O.swiglu_interval(ge[:, :MI], ga[:, :MI], ge[:, MI:], ga[:, MI:]), f"prefill T={T} act")
    # stage 2: down + routing weight from the GPU's act, scattered token-major
    ye, ya = O.grouped_gemm_exact(ab, lay["dn_w"], lay["dn_s"], ref["ends"])
    lo, hi = prod_interval(ye, ya, ref["w"].reshape(-1)[ref["order"]])
    flo, fhi = np.empty_like(lo), np.empty_like(hi)
    flo[ref["order"]] = lo
    fhi[ref["order"]] = hi
    assert_in_interval(pb, flo, fhi, f"prefill T={T} prod")
    # stage 3: ordered slot sum of the GPU products
    ones = O.f32_to_bf16_bits(np.ones((T, k), np.float32))
    assert_bf16_equal(ob, O.weighted_reduce(pb, ones), f"prefill T={T} slot sum")
    bounds = O.moe_output_interval(x, ref["idx"], lg, lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"])
    assert_block_output(out, ref["out"], bounds, f"prefill T={T} end-to-end", mag=ref["mag"])


@pytest.mark.gpu
@pytest.mark.timeout(900)
@pytest.mark.parametrize("T,H,MI", [
    (4096, 3072, 768),    # the 4096-token prefill workload
    (8192, 2560, 640),    # the reference's production chunk (FNX_CHUNK=8192) at its model's expert shapes
])
def test_moe_prefill_full_size(device, T, H, MI):
    """Large prefill chunks, 512 experts top-10, g64, uniform routing, as
    tests/r100_moe_exact.py:13-27 checks whole _moe outputs at T=8192:
    routing in full; every token's output against the oracle's grouped path
    (rel-L2 over the whole output, every element inside its propagated
    bounds); a token sample stage by stage; token-permutation invariance
    (scripts/prod_pipeline.sh:38)."""
    import os
    from qmoe import moe_prefill
    E, gs, k = 512, 64, 10
    log(f"moe_prefill full T={T} H={H} MI={MI}: generating the layer")
    lay = layer(E, H, MI, gs, 4000)
    gu, dn = layer_dev(lay, device)
    x = bf16_normal((T, H), 4001)
    lg = bf16_normal((T, E), 4002)
    xd, lgd = to_dev(x, device), to_dev(lg, device)
    out, (idx, w, counts, ends, order, inverse), (act, prod) = moe_prefill(
        xd, lgd, gu, dn, k, return_routing=True, return_intermediates=True)
    torch.cuda.synchronize()
    prev = O.set_workers(min(16, len(os.sched_getaffinity(0))))
    try:
        log(f"moe_prefill full T={T}: oracle output")
        ref = O.moe_prefill(x, lg, lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"], k)
        assert np.array_equal(idx.cpu().numpy(), ref["idx"])
        assert np.array_equal(counts.cpu().numpy(), ref["counts"]) and np.array_equal(ends.cpu().numpy(), ref["ends"])
        assert np.array_equal(order.cpu().numpy(), ref["order"])
        assert np.array_equal(inverse.cpu().numpy(), ref["inverse"])
        assert_rounds_exactly(w, O.router_weights_exact(lg, ref["idx"]), None, "router weights")
        log(f"moe_prefill full T={T}: oracle bounds of every output element")
        bounds = O.moe_output_interval(x, ref["idx"], lg, lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"])
    finally:
        O.set_workers(prev)
    assert_block_output(out, ref["out"], bounds, f"prefill T={T} H={H} MI={MI} end-to-end, all tokens",
                        mag=ref["mag"])
    ab, pb, ob = bits(act), bits(prod), bits(out)
    ones = O.f32_to_bf16_bits(np.ones((1, k), np.float32))
    ri = ref["inverse"]
    for t in (0, 1, 777, T - 1):
        rows = ri[t * k:(t + 1) * k]                       # expert-major positions of the token's slots
        check_expert_rows(np.repeat(x[t:t + 1], k, 0), ref["idx"][t], ref["w"][t], ab[rows], pb[t * k:(t + 1) * k],
                          lay, gs, gs, f"prefill token {t}")
        assert_bf16_equal(ob[t:t + 1], O.weighted_reduce(pb[t * k:(t + 1) * k], ones), f"prefill token {t} sum")
    # permuting tokens permutes outputs bit for bit (rows are independent)
    p = torch.randperm(T, generator=torch.Generator().manual_seed(9)).to(device)
    out_p = moe_prefill(xd[p].contiguous(), lgd[p].contiguous(), gu, dn, k)
    torch.cuda.synchronize()
    assert torch.equal(out_p.view(torch.int16), out[p].view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("B,E", [(1, 64), (3, 640)])
def test_moe_decode_single_launch_matches_two_launches(device, B, E):
    """The one-launch decode (down workgroups waiting on the gate_up ones) gives
    the same bits as the two separate launches, over repeated calls, and leaves
    every counter (ready and arrival counters, error flag) at zero; the epoch
    slot counts the array's one-launch calls. (Several tokens over at
    most 512 experts take the per-pair one-row launch, whose down tiles sum in
    another order than the separate launches' multi-row tiles: those are
    checked against the oracle instead.)"""
    import ctypes
    from qmoe import _lib, moe_decode
    H, MI, gs, k = 1024, 256, 128, 8
    log(f"moe_decode single launch vs two launches B={B}")
    lay = layer(E, H, MI, gs, 500 + B)
    gu, dn = layer_dev(lay, device)
    L = _lib.lib()
    ncnt = L.qmoe_moe_decode_counters(B, k, H, MI)
    cnt = _lib.counters(device, ncnt)
    for rep in range(3):
        x = to_dev(bf16_normal((B, H), 10 + rep), device)
        lg = to_dev(bf16_normal((B, E), 20 + rep), device)
        out1, idx1, w1 = moe_decode(x, lg, gu, dn, k)
        ws = torch.empty(L.qmoe_moe_decode_workspace(B, k, H, MI), dtype=torch.uint8, device=device)
        out2 = torch.empty_like(out1)
        idx2 = torch.empty_like(idx1)
        w2 = torch.empty_like(w1)
        st = _lib.stream_of(x)
        _lib.check(L.qmoe_moe_decode_gate_up(x.data_ptr(), lg.data_ptr(), gu.w4.data_ptr(), gu._scales.data_ptr(),
                                             idx2.data_ptr(), w2.data_ptr(), B, E, k, H, MI, gs, ws.data_ptr(),
                                             ws.numel(), cnt.data_ptr(), st), "gate_up")
        _lib.check(L.qmoe_moe_decode_down(dn.w4.data_ptr(), dn._scales.data_ptr(), None, None, out2.data_ptr(), B, k,
                                          H, MI, gs, ws.data_ptr(), ws.numel(), cnt.data_ptr(), st), "down")
        torch.cuda.synchronize()
        assert torch.equal(idx1, idx2) and torch.equal(w1.view(torch.int16), w2.view(torch.int16))
        assert torch.equal(out1.view(torch.int16), out2.view(torch.int16)), f"rep {rep}"
        assert int(cnt[_lib.DECODE_ERROR_SLOT]) == 0, f"wait timed out in rep {rep}"
        assert int(cnt[:_lib.DECODE_EPOCH_SLOT].abs().sum()) == 0, f"counters not re-armed after rep {rep}"
