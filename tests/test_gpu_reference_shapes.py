"""The expert block at the shapes the drop-in really serves, and the launch
forms that depend on them.

``FnLayer._moe`` calls the experts with H2560, E512, top-10, MI640
(``fnx/engine.py:23,40-42``) and group size 64 (``fnx/load.py:74``). There
the one-token XCD-group launch has 5 act tiles per slot (an odd count: no
line pairs) and 20 K-slices per group, the four-token per-pair launch runs
its 512-row K-slices at g64, and the one-token block's shared-down
workgroups read 2 pieces of the projection row per lane (4 at MI 2048).
Each case is checked stage by stage against the oracle and end to end
against its propagated bounds, and the decode error flag must stay clear.
The same cases run with the workgroup-placement check switched off, which
sends one token to the device-coherent per-pair launch.
"""
import numpy as np
import pytest
import torch

from gpu_util import bf16_normal, check_expert_rows, layer, layer_dev, log
from oracle import qmoe_oracle as O
from parity import assert_bf16_equal, assert_block_output, bits, to_dev

REF_SHAPE = dict(E=512, H=2560, MI=640, gs=64, k=10)


@pytest.fixture(scope="module")
def ref_layer(device):
    s = REF_SHAPE
    log(f"reference-shape layer E={s['E']} H={s['H']} MI={s['MI']} gs={s['gs']}")
    lay = layer(s["E"], s["H"], s["MI"], s["gs"], 2560)
    return lay, layer_dev(lay, device)


@pytest.fixture
def placement_off(device):
    """The device's workgroup-placement verdict forced to 'fails' for one test."""
    from qmoe import _lib
    _lib.xcd_placement(device, 1)
    yield
    _lib.xcd_placement(device, 2)
    assert _lib.xcd_placement(device) in (0, 1)


def _check_decode(lay, x, lg, out, idx, w, act, prod, k, gs, what):
    ab, pb, ob = bits(act), bits(prod), bits(out)
    ones = O.f32_to_bf16_bits(np.ones((1, k), np.float32))
    for t in range(x.shape[0]):
        ref = O.moe_decode(x[t], lg[t], lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"], k)
        assert np.array_equal(idx[t].cpu().numpy(), ref["idx"][0])
        check_expert_rows(np.repeat(x[t:t + 1], k, 0), ref["idx"][0], ref["w"][0], ab[t], pb[t], lay, gs, gs,
                          f"{what} token {t}")
        assert_bf16_equal(ob[t:t + 1], O.weighted_reduce(pb[t], ones), f"{what} token {t} slot sum")
        bounds = O.moe_output_interval(x[t:t + 1], ref["idx"], lg[t:t + 1], lay["gu_w"], lay["gu_s"], lay["dn_w"],
                                       lay["dn_s"])
        assert_block_output(ob[t:t + 1], ref["out"], bounds, f"{what} token {t} end-to-end", mag=ref["mag"])


@pytest.mark.gpu
@pytest.mark.parametrize("B,tiles", [(1, False), (1, True), (4, False), (4, True)])
def test_decode_reference_shape(device, ref_layer, B, tiles):
    """One token on the XCD-group launch (5 act tiles per slot), four on the
    per-pair launch with 512-row K-slices, from the int4pack container and
    from decode tiles."""
    from qmoe import _lib, moe_decode
    lay, (gu, dn) = ref_layer
    k, gs, H, E = REF_SHAPE["k"], REF_SHAPE["gs"], REF_SHAPE["H"], REF_SHAPE["E"]
    log(f"decode reference shape B={B} tiles={tiles}")
    x = bf16_normal((B, H), 2561 + B)
    lg = bf16_normal((B, E), 2571 + B)
    out, idx, w, (act, prod) = moe_decode(to_dev(x, device), to_dev(lg, device), gu, dn, k,
                                          return_intermediates=True, tiles=tiles)
    torch.cuda.synchronize()
    _check_decode(lay, x, lg, out, idx, w, act, prod, k, gs, f"ref-shape B={B} tiles={tiles}")
    assert _lib.decode_status(_lib.counters(device)) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("B", [1, 4])
def test_decode_reference_shape_placement_off(device, ref_layer, placement_off, B):
    """With the placement check failing, one token runs the device-coherent
    per-pair launch: the same oracle checks hold."""
    from qmoe import _lib, moe_decode
    lay, (gu, dn) = ref_layer
    k, gs, H, E = REF_SHAPE["k"], REF_SHAPE["gs"], REF_SHAPE["H"], REF_SHAPE["E"]
    assert _lib.xcd_placement(device) == 0
    log(f"decode reference shape B={B}, placement check off")
    x = bf16_normal((B, H), 2581 + B)
    lg = bf16_normal((B, E), 2591 + B)
    out, idx, w, (act, prod) = moe_decode(to_dev(x, device), to_dev(lg, device), gu, dn, k,
                                          return_intermediates=True)
    torch.cuda.synchronize()
    _check_decode(lay, x, lg, out, idx, w, act, prod, k, gs, f"placement-off B={B}")
    assert _lib.decode_status(_lib.counters(device)) == 0


@pytest.mark.gpu
def test_projection_placement_off_same_bits(device):
    """The one-row GEMV gives the same bits with its slice partials stored
    device-coherent (placement check failing) as through one XCD's L2."""
    from qmoe import _lib, weight_quant_batchmatmul
    from gpu_util import int4_words, scales
    K, N, gs = 2560, 1280, 64
    log("projection, placement check on and off")
    w = to_dev(int4_words((K, N // 8), 31), device)
    s = to_dev(scales((K // gs, N), 32), device)
    x = to_dev(bf16_normal((1, K), 33), device)
    a = weight_quant_batchmatmul(x, w, s, antiquant_group_size=gs)
    torch.cuda.synchronize()
    _lib.xcd_placement(device, 1)
    try:
        b = weight_quant_batchmatmul(x, w, s, antiquant_group_size=gs)
        torch.cuda.synchronize()
    finally:
        _lib.xcd_placement(device, 2)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    ref_e, ref_a = O.w4a16_gemm_exact(bits(x), w.cpu().numpy(), bits(s), gs)
    from parity import assert_rounds_exactly
    assert_rounds_exactly(a, ref_e, ref_a, "projection 2560x1280 g64")


def _block_weights(E, H, MI, device, seed):
    sh_gu = to_dev(bf16_normal((2 * MI + 1 + E, H), seed, 0.04), device)
    sh_down = to_dev(bf16_normal((H, MI), seed + 1, 0.04), device)
    return sh_gu, sh_down


@pytest.mark.gpu
@pytest.mark.parametrize("E,H,MI,gs,k", [
    (512, 2560, 640, 64, 10),    # the reference model's shape: 2 projection pieces per lane
    (64, 1024, 1024, 64, 8),     # 2 pieces per lane, 8 act tiles
    (64, 512, 2048, 128, 8),     # the largest MI the one-launch block takes: 4 pieces per lane
])
def test_moe_block_one_token_shapes(device, E, H, MI, gs, k):
    """One token: the block in two launches gives the three-launch form's bits
    and lies inside the oracle's end-to-end bounds (fed the GPU's shared
    output and router logits)."""
    from qmoe import _lib, moe_decode
    from qmoe.shared import moe_block, shared_router
    log(f"moe_block one token E={E} H={H} MI={MI} gs={gs}")
    lay = layer(E, H, MI, gs, 700 + MI)
    gu_e, dn_e = layer_dev(lay, device)
    sh_gu, sh_down = _block_weights(E, H, MI, device, 710 + MI)
    for seed, tiles in ((720, False), (721, True)):
        x = bf16_normal((1, H), seed)
        xd = to_dev(x, device)
        fused = moe_block(xd, sh_gu, sh_down, gu_e, dn_e, k, tiles=tiles)
        sh, gate2, logits = shared_router(xd, sh_gu, sh_down, MI)
        three = moe_decode(xd, logits, gu_e, dn_e, k, shared=sh, shared_gate=gate2.contiguous(), tiles=tiles)[0]
        torch.cuda.synchronize()
        assert torch.equal(fused.view(torch.int16), three.view(torch.int16)), f"seed {seed}"
        sh_b, g2_b, lg_b = bits(sh), np.ascontiguousarray(bits(gate2)), np.ascontiguousarray(bits(logits))
        ref = O.moe_decode(x[0], lg_b[0], lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"], k,
                           shared_bits=sh_b, gate_bits=g2_b[0])
        bounds = O.moe_output_interval(x, ref["idx"], lg_b, lay["gu_w"], lay["gu_s"], lay["dn_w"], lay["dn_s"],
                                       shared_bits=sh_b, gate_bits=g2_b[0])
        assert_block_output(fused, ref["out"], bounds, f"moe_block MI={MI} tiles={tiles}", mag=ref["mag"])
    assert _lib.decode_status(_lib.counters(device)) == 0


@pytest.mark.gpu
def test_moe_block_one_token_placement_off(device, placement_off):
    """Placement check failing: the one-launch block is refused and the block
    runs its three launches, with their bits."""
    from qmoe import _lib, moe_decode
    from qmoe.shared import _block_one_token, _project, moe_block, shared_router
    E, H, MI, gs, k = 64, 512, 256, 64, 8
    log("moe_block one token, placement check off")
    lay = layer(E, H, MI, gs, 731)
    gu_e, dn_e = layer_dev(lay, device)
    sh_gu, sh_down = _block_weights(E, H, MI, device, 732)
    xd = to_dev(bf16_normal((1, H), 733), device)
    gu, logits = _project(xd, sh_gu, MI)
    assert _block_one_token(xd, gu, logits, sh_down, gu_e, dn_e, k, MI, None) is None
    a = moe_block(xd, sh_gu, sh_down, gu_e, dn_e, k)
    sh, gate2, lg = shared_router(xd, sh_gu, sh_down, MI)
    b = moe_decode(xd, lg, gu_e, dn_e, k, shared=sh, shared_gate=gate2.contiguous())[0]
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert _lib.decode_status(_lib.counters(device)) == 0


@pytest.mark.gpu
def test_decode_tiles_follow_rebound_weights(device):
    """Tiles are opt-in: built only on request, read once built, dropped when
    w4 is rebound to another tensor (no stale tiles)."""
    from qmoe import moe_decode
    from gpu_util import int4_words
    E, H, MI, gs, k = 64, 512, 256, 64, 8
    log("decode tiles opt-in and rebinding")
    lay = layer(E, H, MI, gs, 741)
    gu, dn = layer_dev(lay, device)
    x, lg = to_dev(bf16_normal((1, H), 742), device), to_dev(bf16_normal((1, E), 743), device)
    moe_decode(x, lg, gu, dn, k)
    assert gu.cached_decode_tiles("gate_up") is None and dn.cached_decode_tiles("down") is None
    a = moe_decode(x, lg, gu, dn, k, tiles=True)[0]
    assert gu.cached_decode_tiles("gate_up") is not None and dn.cached_decode_tiles("down") is not None
    b = moe_decode(x, lg, gu, dn, k)[0]                      # reads the tiles built above
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    gu.w4 = to_dev(int4_words(tuple(gu.w4.shape), 744), device)
    assert gu.cached_decode_tiles("gate_up") is None
    c = moe_decode(x, lg, gu, dn, k, tiles=False)[0]
    d = moe_decode(x, lg, gu, dn, k, tiles=True)[0]
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int16), d.view(torch.int16)), "tiles of the old weights were read"
