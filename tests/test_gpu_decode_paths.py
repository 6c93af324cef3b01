"""Decode paths the headline tests do not reach, and the decode kernel's state.

* Tokens that share experts on the de-duplicated kernels (more than 512
  experts): the multi-row gate_up and down tiles, the plan's token/slot
  scatter and the ballot de-duplication, in the one-launch and the
  two-launch form.
* Graph capture: the decode block, the prefill block and the per-op drop-ins
  captured once and replayed with fresh inputs must give the eager bits
  (the reference's own gates: tests/r100_moe_exact.py:18-27,
  tests/r118_weighted_reduce.py:67-72, fnx/model.py:261-268).
* Two streams with separate counters arrays run decodes concurrently and
  give the serial bits (epoch, mailbox and error flag live in the array).
"""
import numpy as np
import pytest
import torch

from gpu_util import bf16_normal, check_expert_rows, layer, layer_dev, log
from oracle import qmoe_oracle as O
from parity import assert_block_output, assert_bf16_equal, bits, to_dev


def _shared_logits(B, E, seed, case):
    lg = bf16_normal((B, E), seed)
    if case == "copies":          # tokens 1 and 3 route exactly as token 0: multiplicity 3
        lg[1] = lg[0]
        lg[3 % B] = lg[0]
    elif case == "identical":     # every token the same: multiplicity B
        lg[:] = lg[0]
    elif case == "partial":       # token 1 shares all but its three best experts with token 0
        lg[1] = lg[0]
        top = np.argsort(-O.bf16_bits_to_f32(lg[0]), kind="stable")[:3]
        lg[1, top] = O.f32_to_bf16_bits(np.full(3, -30.0, np.float32))
    return lg


@pytest.mark.gpu
@pytest.mark.parametrize("B,E,H,MI,gs,k,case", [
    (4, 640, 512, 128, 64, 8, "copies"),
    (2, 640, 512, 128, 64, 8, "identical"),
    (3, 768, 1024, 256, 128, 10, "partial"),
    (4, 1024, 512, 128, 64, 16, "identical"),    # 16 unique experts, each with four rows
    (4, 640, 2048, 512, 128, 10, "partial"),     # the decode layer's expert shapes
])
def test_decode_shared_experts_deduplicated(device, B, E, H, MI, gs, k, case):
    import ctypes
    from qmoe import _lib, moe_decode
    log(f"decode de-dup B={B} E={E} H={H} MI={MI} k={k} case={case}")
    lay = layer(E, H, MI, gs, 31 * B + E)
    gu, dn = layer_dev(lay, device)
    x = bf16_normal((B, H), 40 + B)
    lg = _shared_logits(B, E, 41 + B, case)
    ridx = [O.router(lg[t:t + 1], k)[0][0] for t in range(B)]
    distinct = len(set(np.concatenate(ridx).tolist()))
    assert distinct < B * k, "the case must route several tokens to one expert"
    xd, lgd = to_dev(x, device), to_dev(lg, device)
    out, idx, w, (act, prod) = moe_decode(xd, lgd, gu, dn, k, return_intermediates=True)
    torch.cuda.synchronize()
    # the plan the launch built: distinct experts and their multiplicities
    L = _lib.lib()
    offs = [ctypes.c_size_t() for _ in range(3)]
    _lib.check(L.qmoe_moe_decode_layout(B, k, H, MI, *[ctypes.byref(v) for v in offs]), "layout")
    ab, pb, ob = bits(act), bits(prod), bits(out)
    for t in range(B):
        ref = O.moe_decode(x[t], lg[t], lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"], k)
        assert np.array_equal(idx[t].cpu().numpy(), ref["idx"][0])
        check_expert_rows(np.repeat(x[t:t + 1], k, 0), ref["idx"][0], ref["w"][0], ab[t], pb[t], lay, gs, gs,
                          f"de-dup token {t}")
        ones = O.f32_to_bf16_bits(np.ones((1, k), np.float32))
        assert_bf16_equal(ob[t:t + 1], O.weighted_reduce(pb[t], ones), f"de-dup token {t} slot sum")
        bounds = O.moe_output_interval(x[t:t + 1], ref["idx"], lg[t:t + 1], lay["gu_w"], lay["gu_s"], lay["dn_w"],
                                       lay["dn_s"])
        assert_block_output(ob[t:t + 1], ref["out"], bounds, f"de-dup token {t} end-to-end", mag=ref["mag"])
    # tokens with identical logits and inputs give identical rows
    if case in ("copies", "identical"):
        x2 = x.copy()
        x2[:] = x[0]
        out2 = moe_decode(to_dev(x2, device), lgd, gu, dn, k)[0]
        torch.cuda.synchronize()
        o2 = bits(out2)
        for t in range(1, B):
            if case == "identical" or t in (1, 3 % B):
                assert np.array_equal(o2[t], o2[0])
    # the two-launch form gives the same bits
    ws = torch.empty(L.qmoe_moe_decode_workspace(B, k, H, MI), dtype=torch.uint8, device=device)
    cnt = _lib.counters(device)
    out3 = torch.empty_like(out)
    idx3 = torch.empty_like(idx)
    w3 = torch.empty_like(w)
    st = _lib.stream_of(xd)
    _lib.check(L.qmoe_moe_decode_gate_up(xd.data_ptr(), lgd.data_ptr(), gu.w4.data_ptr(), gu._scales.data_ptr(),
                                         idx3.data_ptr(), w3.data_ptr(), B, E, k, H, MI, gs, ws.data_ptr(),
                                         ws.numel(), cnt.data_ptr(), st), "gate_up")
    _lib.check(L.qmoe_moe_decode_down(dn.w4.data_ptr(), dn._scales.data_ptr(), None, None, out3.data_ptr(), B, k,
                                      H, MI, gs, ws.data_ptr(), ws.numel(), cnt.data_ptr(), st), "down")
    torch.cuda.synchronize()
    assert torch.equal(idx3, idx) and torch.equal(w3.view(torch.int16), w.view(torch.int16))
    assert torch.equal(out3.view(torch.int16), out.view(torch.int16))
    plan = ws[int(offs[0].value):int(offs[0].value) + 705 * 4].view(torch.int32).cpu().numpy()
    nunique, umult = int(plan[0]), plan[1 + 64:1 + 128]
    assert nunique == distinct and int(umult[:nunique].max()) >= 2 and int(umult[:nunique].sum()) == B * k
    assert int(cnt[:_lib.DECODE_EPOCH_SLOT].abs().sum()) == 0, "counters not re-armed"


def _device_layer(E, H, MI, gs, seed, device):
    """A random expert-major layer generated on the device (graph tests compare
    GPU runs with each other, so no host copy is needed)."""
    from qmoe import ExpW4
    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def words(*shape):
        return torch.randint(-2**31, 2**31 - 1, shape, generator=g, device=device, dtype=torch.int64).to(torch.int32)

    def sc(*shape):
        return (torch.randn(shape, generator=g, device=device).abs() * 0.02).to(torch.bfloat16)

    return (ExpW4.from_scales(words(E, H, 2 * MI // 8), sc(E, H // gs, 2 * MI)),
            ExpW4.from_scales(words(E, MI, H // 8), sc(E, MI // gs, H)))


def _replay_matches_eager(fn, inputs, fresh, what):
    """Capture fn(*inputs) once, then for each set of fresh inputs copy them in,
    replay three times with eager work and synchronisations in between, and
    compare every replay with an eager call on the same inputs, bit for bit."""
    fn(*inputs)                                  # eager warm-up (workspaces, counters)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_out = fn(*inputs)
    static_out = static_out if isinstance(static_out, (tuple, list)) else (static_out,)
    for rep, vals in enumerate(fresh):
        for dst, src in zip(inputs, vals):
            dst.copy_(src)
        eager = fn(*vals)
        eager = eager if isinstance(eager, (tuple, list)) else (eager,)
        torch.cuda.synchronize()
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(zip(static_out, eager)):
                assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                                   b.view(torch.int16) if b.dtype == torch.bfloat16 else b), \
                    f"{what}: replay output {i} differs from eager (inputs {rep})"
    del g


@pytest.mark.gpu
@pytest.mark.parametrize("B", [1, 4])
def test_decode_graph_replay(device, B):
    from qmoe import decode_status, moe_decode
    E, H, MI, gs, k = 512, 2048, 512, 128, 10
    log(f"decode graph replay B={B}")
    gu, dn = _device_layer(E, H, MI, gs, 300 + B, device)
    x = torch.randn(B, H, device=device).to(torch.bfloat16)
    lg = torch.randn(B, E, device=device).to(torch.bfloat16)
    fresh = [(torch.randn(B, H, device=device).to(torch.bfloat16), torch.randn(B, E, device=device).to(torch.bfloat16))
             for _ in range(3)]
    _replay_matches_eager(lambda a, b: moe_decode(a, b, gu, dn, k), [x, lg], fresh, f"moe_decode B={B}")
    assert decode_status(device) == 0


@pytest.mark.gpu
def test_prefill_graph_replay(device):
    from qmoe import moe_prefill
    from qmoe.workload import zipf_logits
    E, H, MI, gs, k, T = 512, 2048, 512, 128, 10, 512
    log("prefill graph replay T=512 zipf")
    gu, dn = _device_layer(E, H, MI, gs, 400, device)
    x = torch.randn(T, H, device=device).to(torch.bfloat16)
    lg = to_dev(zipf_logits(T, E, 1.1, 5), device)
    fresh = [(torch.randn(T, H, device=device).to(torch.bfloat16), to_dev(zipf_logits(T, E, 1.1, 6 + i), device))
             for i in range(3)]
    _replay_matches_eager(lambda a, b: moe_prefill(a, b, gu, dn, k), [x, lg], fresh, "moe_prefill")


@pytest.mark.gpu
def test_grouped_matmul_and_weighted_reduce_graph_replay(device):
    from qmoe import grouped_matmul
    from qmoe.weighted_reduce import reduce
    E, K, N, gs, R = 64, 1024, 512, 64, 700
    log("grouped_matmul / weighted_reduce graph replay")
    gu, _ = _device_layer(E, K, N // 2, gs, 500, device)

    def counts_to_ends(seed):
        c = torch.randint(0, 2 * R // E, (E,), generator=torch.Generator().manual_seed(seed))
        c[0] += R - int(c.sum()) if int(c.sum()) < R else 0
        return torch.cumsum(c, 0).clamp(max=R).to(device)

    x = torch.randn(R, K, device=device).to(torch.bfloat16)
    ends = counts_to_ends(1)
    fresh = [(torch.randn(R, K, device=device).to(torch.bfloat16), counts_to_ends(2 + i)) for i in range(3)]

    def gmm(a, e):
        return grouped_matmul([a], [gu.w4], antiquant_scale=[gu._scales], group_list=e, split_item=3,
                              group_type=0)[0]
    _replay_matches_eager(gmm, [x, ends], fresh, "grouped_matmul")

    T, kk, W = 300, 10, 2048
    vals = torch.randn(T * kk, W, device=device).to(torch.bfloat16)
    wts = torch.rand(T, kk, device=device).to(torch.bfloat16)
    inv = torch.randperm(T * kk, device=device)
    fresh = [(torch.randn(T * kk, W, device=device).to(torch.bfloat16), torch.rand(T, kk, device=device).to(torch.bfloat16),
              torch.randperm(T * kk, device=device)) for _ in range(3)]
    _replay_matches_eager(lambda v, w, i: reduce(v, w, inverse=i), [vals, wts, inv], fresh, "weighted_reduce")


@pytest.mark.gpu
def test_decode_two_streams(device):
    """Decodes issued concurrently on two streams, each with its own counters
    array, give the serial results bit for bit and leave both flags clear."""
    from qmoe import _lib, decode_status, moe_decode
    E, H, MI, gs, k, n = 512, 2048, 512, 128, 10, 6
    log("decode on two streams")
    gu, dn = _device_layer(E, H, MI, gs, 600, device)
    xs = [torch.randn(1, H, device=device).to(torch.bfloat16) for _ in range(n)]
    lgs = [torch.randn(1, E, device=device).to(torch.bfloat16) for _ in range(n)]
    serial = [moe_decode(a, b, gu, dn, k)[0] for a, b in zip(xs, lgs)]
    torch.cuda.synchronize()
    cnts = [_lib.new_counters(device, _lib.lib().qmoe_moe_decode_counters(1, k, H, MI)) for _ in range(2)]
    streams = [torch.cuda.Stream(device=device) for _ in range(2)]
    outs = [None] * n
    for i in range(n):                     # interleaved issue: calls of the two streams overlap
        s = i % 2
        with torch.cuda.stream(streams[s]):
            outs[i] = moe_decode(xs[i], lgs[i], gu, dn, k, counters=cnts[s])[0]
    torch.cuda.synchronize()
    for i in range(n):
        assert torch.equal(outs[i].view(torch.int16), serial[i].view(torch.int16)), f"call {i}"
    for c in cnts:
        assert decode_status(counters=c) == 0
        assert int(c[:_lib.DECODE_EPOCH_SLOT].abs().sum()) == 0
        assert int(c[_lib.DECODE_EPOCH_SLOT]) == n // 2   # each array's own launch count


@pytest.mark.gpu
def test_decode_one_token_gate_up_group_not_multiple_of_16(device):
    """One token on the XCD-group launch with a gate_up group size of 24 (its
    K-slices then hold 8 rows per lane, so a lane's rows stay in one scale
    group) and a down group size of 32: routing, stage-wise rounding, the slot
    sum, the end-to-end bound and the two-launch form's bits."""
    import ctypes
    from gpu_util import int4_words, scales
    from qmoe import _lib, moe_decode
    H, MI, E, k, gs_gu, gs_dn = 768, 256, 64, 8, 24, 32
    log(f"decode one token gs_gu={gs_gu} gs_dn={gs_dn}")
    lay = dict(gu_w=int4_words((E, H, 2 * MI // 8), 71), gu_s=scales((E, H // gs_gu, 2 * MI), 72),
               dn_w=int4_words((E, MI, H // 8), 73), dn_s=scales((E, MI // gs_dn, H), 74))
    gu, dn = layer_dev(lay, device)
    x = bf16_normal((1, H), 75)
    lg = bf16_normal((1, E), 76)
    xd, lgd = to_dev(x, device), to_dev(lg, device)
    out, idx, w, (act, prod) = moe_decode(xd, lgd, gu, dn, k, return_intermediates=True)
    torch.cuda.synchronize()
    ab, pb, ob = bits(act), bits(prod), bits(out)
    ref = O.moe_decode(x[0], lg[0], lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"], k)
    assert np.array_equal(idx[0].cpu().numpy(), ref["idx"][0])
    check_expert_rows(np.repeat(x, k, 0), ref["idx"][0], ref["w"][0], ab[0], pb[0], lay, gs_gu, gs_dn, "gs24 token")
    ones = O.f32_to_bf16_bits(np.ones((1, k), np.float32))
    assert_bf16_equal(ob, O.weighted_reduce(pb[0], ones), "gs24 slot sum")
    bounds = O.moe_output_interval(x, ref["idx"], lg, lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"])
    assert_block_output(ob, ref["out"], bounds, "gs24 end-to-end", mag=ref["mag"])
    L = _lib.lib()
    ws = torch.empty(L.qmoe_moe_decode_workspace(1, k, H, MI), dtype=torch.uint8, device=device)
    cnt = _lib.counters(device)
    out2, idx2, w2 = torch.empty_like(out), torch.empty_like(idx), torch.empty_like(w)
    st = _lib.stream_of(xd)
    _lib.check(L.qmoe_moe_decode_gate_up(xd.data_ptr(), lgd.data_ptr(), gu.w4.data_ptr(), gu._scales.data_ptr(),
                                         idx2.data_ptr(), w2.data_ptr(), 1, E, k, H, MI, gs_gu, ws.data_ptr(),
                                         ws.numel(), cnt.data_ptr(), st), "gate_up")
    _lib.check(L.qmoe_moe_decode_down(dn.w4.data_ptr(), dn._scales.data_ptr(), None, None, out2.data_ptr(), 1, k,
                                      H, MI, gs_dn, ws.data_ptr(), ws.numel(), cnt.data_ptr(), st), "down")
    torch.cuda.synchronize()
    assert torch.equal(out2.view(torch.int16), out.view(torch.int16))
    assert _lib.decode_status(cnt) == 0


def _tile_index_gate_up(H, MI, gs_gu):
    """(row, word) of every word of one expert's gate_up decode tiles, in tile
    order: tile s * t1 + m, word p * 256 + t = the p-th row word of thread t
    (K-slice s of 128 rows, act tile m; p = h * GR + i, rows 128 s + h * 8 GR +
    (t / 32) * GR + i; word of lane chunk t % 32: the gate words of tile m,
    then its up words)."""
    GR = 16 if gs_gu % 16 == 0 else 8
    t1 = MI // 128
    s, m, p, t = np.meshgrid(np.arange(H // 128), np.arange(t1), np.arange(16), np.arange(256), indexing="ij")
    h, i = p // GR, p % GR
    row = 128 * s + h * 8 * GR + (t // 32) * GR + i
    cc = t % 32
    col = np.where(cc < 16, 16 * m + cc, MI // 8 + 16 * m + (cc - 16))
    return row.reshape(-1), col.reshape(-1)


def _tile_index_down(H, MI):
    """(row, word) of one expert's down decode tiles: tile m * t2 + c, word
    p * 256 + t = row 128 m + (t / 32) * 16 + p, word 32 c + t % 32."""
    m, c, p, t = np.meshgrid(np.arange(MI // 128), np.arange(H // 256), np.arange(16), np.arange(256), indexing="ij")
    return (128 * m + (t // 32) * 16 + p).reshape(-1), (32 * c + t % 32).reshape(-1)


@pytest.mark.gpu
@pytest.mark.parametrize("E,H,MI,gs_gu,gs_dn,k", [
    (512, 2048, 512, 128, 128, 10),   # the headline layer
    (64, 768, 256, 24, 32, 8),        # gate_up group 24: 8 rows per lane, two halves per K-slice
    (32, 512, 384, 64, 64, 6),        # an odd act-tile count (no line pairs)
])
def test_decode_tiles(device, E, H, MI, gs_gu, gs_dn, k):
    """Decode tiles: the layout against its restatement on the host (for a
    few experts), and the decode reading them (one token on the XCD-group
    launch, four on the per-pair launch) against the decode reading w4: the
    same out, idx and w bits, error flag clear."""
    from qmoe import _lib, moe_decode
    log(f"decode tiles E={E} H={H} MI={MI} gs={gs_gu}/{gs_dn}")
    from gpu_util import int4_words, scales
    lay = dict(gu_w=int4_words((E, H, 2 * MI // 8), 81), gu_s=scales((E, H // gs_gu, 2 * MI), 82),
               dn_w=int4_words((E, MI, H // 8), 83), dn_s=scales((E, MI // gs_dn, H), 84))
    gu, dn = layer_dev(lay, device)
    gu_t, dn_t = gu.decode_tiles("gate_up"), dn.decode_tiles("down")
    assert gu_t is not None and dn_t is not None
    torch.cuda.synchronize()
    rg, cg = _tile_index_gate_up(H, MI, gs_gu)
    rd, cd = _tile_index_down(H, MI)
    for e in sorted({0, E // 2, E - 1}):
        assert np.array_equal(gu_t[e].cpu().numpy().reshape(-1), lay["gu_w"][e][rg, cg]), f"gate_up tiles of expert {e}"
        assert np.array_equal(dn_t[e].cpu().numpy().reshape(-1), lay["dn_w"][e][rd, cd]), f"down tiles of expert {e}"
    cnt = _lib.counters(device)
    for seed, B in ((85, 1), (86, 1), (87, 4)):   # four tokens: the per-pair launch reads the same tiles
        x, lg = to_dev(bf16_normal((B, H), seed), device), to_dev(bf16_normal((B, E), seed + 10), device)
        a = moe_decode(x, lg, gu, dn, k, tiles=False)
        b = moe_decode(x, lg, gu, dn, k, tiles=True)
        torch.cuda.synchronize()
        for u, v, what in zip(a, b, ("out", "idx", "w")):
            assert torch.equal(u.view(torch.int16) if u.dtype == torch.bfloat16 else u,
                               v.view(torch.int16) if v.dtype == torch.bfloat16 else v), f"{what} differs with tiles"
    # weights changed in place: the tiles are built again, not read stale
    gu.w4.bitwise_xor_(0x11111111)
    dn.w4.bitwise_xor_(0x01010101)
    x, lg = to_dev(bf16_normal((1, H), 88), device), to_dev(bf16_normal((1, E), 98), device)
    a = moe_decode(x, lg, gu, dn, k, tiles=False)[0]
    b = moe_decode(x, lg, gu, dn, k, tiles=True)[0]
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)), "tiles stale after an in-place change of w4"
    assert _lib.decode_status(cnt) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("b,tiles", [(1, True), (1, False), (64, None)])
def test_moe_block_graph_replay(device, b, tiles):
    """The whole MoE block (shared/router projection + experts) captured once
    and replayed with fresh tokens: one token in its two-launch form (from
    decode tiles and from the int4pack container), 64 tokens through the
    prefill path (the reference captures the whole layer: fnx/model.py:261-286)."""
    from qmoe import decode_status
    from qmoe.shared import moe_block
    E, H, MI, gs, k = 512, 2048, 512, 128, 10
    log(f"moe_block graph replay b={b} tiles={tiles}")
    gu, dn = _device_layer(E, H, MI, gs, 800 + b, device)
    if tiles:
        gu.decode_tiles("gate_up")
        dn.decode_tiles("down")
    g = torch.Generator(device=device)
    g.manual_seed(801)
    sh_gu = (torch.randn((2 * MI + 1 + E, H), generator=g, device=device) * 0.03).to(torch.bfloat16)
    sh_dn = (torch.randn((H, MI), generator=g, device=device) * 0.03).to(torch.bfloat16)
    x = torch.randn(b, H, device=device).to(torch.bfloat16)
    fresh = [(torch.randn(b, H, device=device).to(torch.bfloat16),) for _ in range(3)]
    _replay_matches_eager(lambda a: moe_block(a, sh_gu, sh_dn, gu, dn, k, tiles=tiles), [x], fresh,
                          f"moe_block b={b}")
    assert decode_status(device) == 0


@pytest.mark.gpu
def test_prefill_graph_replay_production_chunk(device):
    """The reference's production prefill chunk (FNX_CHUNK=8192 tokens,
    scripts/prod_pipeline.sh:38) at its model's expert shapes (512 experts,
    H2560/MI640, g64, top-10) captured and replayed with fresh tokens, as
    tests/r100_moe_exact.py:13-27 gates it."""
    from qmoe import moe_prefill
    E, H, MI, gs, k, T = 512, 2560, 640, 64, 10, 8192
    log("prefill graph replay T=8192 H2560/MI640")
    gu, dn = _device_layer(E, H, MI, gs, 900, device)
    x = torch.randn(T, H, device=device).to(torch.bfloat16)
    lg = torch.randn(T, E, device=device).to(torch.bfloat16)
    fresh = [(torch.randn(T, H, device=device).to(torch.bfloat16), torch.randn(T, E, device=device).to(torch.bfloat16))
             for _ in range(3)]
    _replay_matches_eager(lambda a, c: moe_prefill(a, c, gu, dn, k), [x, lg], fresh, "moe_prefill T=8192")
