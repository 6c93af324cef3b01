"""Expert weight artifacts: LQP v2o -> int4pack conversion, scale composition,
the W4A16 (-em) safetensors loader, and decode on converted weights."""
import numpy as np
import pytest
import torch

from gpu_util import log
from oracle import qmoe_oracle as O
from parity import bits

rng = np.random.default_rng(77)


def lqp_layer(E, H, MI, gs, seed):
    """Synthetic LQP tensors of one layer (host): per projection v2o uint8
    [E, N, K/2], s8 int8 [E, N, G], base fp16 [E, N], plus the int4 values."""
    r = np.random.default_rng(seed)
    out = {}
    for proj, (K, N) in (("gate_up_proj", (H, 2 * MI)), ("down_proj", (MI, H))):
        q = r.integers(-8, 8, size=(E, N, K)).astype(np.int8)
        s8 = r.integers(-127, 128, size=(E, N, K // gs)).astype(np.int8)
        base = (r.random((E, N)) * 4e-4 + 1e-4).astype(np.float16)
        out[proj] = dict(q=q, v2o=O.pack_v2o(q), s8=s8, base=base)
    return out


def save_lqp(path, lay):
    from safetensors.torch import save_file
    t = {}
    for proj, d in lay.items():
        t[f"mlp.experts.{proj}.v2o"] = torch.from_numpy(d["v2o"])
        t[f"mlp.experts.{proj}.s8"] = torch.from_numpy(d["s8"])
        t[f"mlp.experts.{proj}.base"] = torch.from_numpy(d["base"])
    save_file(t, str(path))


# ---------------------------------------------------------------- host side


def test_layer_path_convention(tmp_path):
    from qmoe.artifact import layer_path
    assert str(layer_path("/m/X-w4a16", 7, expert_major=False)) == "/m/X-w4a16/L07.w4.safetensors"
    assert str(layer_path("/m/X-w4a16/", 12, expert_major=True)) == "/m/X-w4a16-em/L12.w4.safetensors"


def test_exp_w4_scale_cache_needs_device():
    """The scale cache is composed by a HIP kernel: host tensors are refused
    loudly instead of being composed on the CPU."""
    from qmoe import ExpW4
    w4 = torch.zeros((4, 256, 16), dtype=torch.int32)
    s8t = torch.zeros((4, 4, 128), dtype=torch.int8)
    base = torch.zeros((4, 128), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="device"):
        ExpW4(w4, s8t, base, 64, expert_major=True)


@pytest.mark.gpu
@pytest.mark.parametrize("em", [False, True])
def test_load_layer_w4(tmp_path, em, device):
    """fnx/load.py:56-77: the loader builds ExpW4 with the artifact's layout and
    gs = K / G, and its scale cache (qmoe_scale_cache) is the oracle's."""
    from safetensors.torch import save_file
    from qmoe.artifact import load_layer_w4
    E, H, MI, gs = 4, 256, 128, 64
    lay = lqp_layer(E, H, MI, gs, 5)
    d = tmp_path / ("X-em" if em else "X")
    d.mkdir()
    t, ref = {}, {}
    for proj, p in lay.items():
        w4, s8t, base_bits, sc = O.lqp_to_em(p["v2o"], p["s8"], p["base"])
        if not em:
            w4 = np.ascontiguousarray(w4.transpose(1, 0, 2))       # the K-major artifact
        t[f"mlp.experts.{proj}.w4"] = torch.from_numpy(w4)
        t[f"mlp.experts.{proj}.s8t"] = torch.from_numpy(s8t)
        t[f"mlp.experts.{proj}.base"] = torch.from_numpy(base_bits.view(np.int16)).view(torch.bfloat16)
        ref[proj] = (w4, sc)
    save_file(t, str(d / "L03.w4.safetensors"))
    got = load_layer_w4(d / "L03.w4.safetensors", device)
    assert sorted(got) == ["mlp.experts.down_proj", "mlp.experts.gate_up_proj"]
    for proj, (w4, sc) in ref.items():
        e = got[f"mlp.experts.{proj}"]
        assert e.expert_major == em and e.E == E and e.gs == gs
        assert np.array_equal(e.w4.cpu().numpy(), w4)
        assert np.array_equal(bits(e._scales), sc)


# ---------------------------------------------------------------- kernels


@pytest.mark.gpu
@pytest.mark.parametrize("E,N,K", [(3, 264, 256), (2, 1024, 2048), (5, 40, 128), (1, 2048, 512)])
@pytest.mark.parametrize("em", [True, False])
def test_lqp_to_int4pack(device, E, N, K, em):
    from qmoe.artifact import lqp_to_int4pack
    log(f"lqp_to_int4pack E={E} N={N} K={K} expert_major={em}")
    q = rng.integers(-8, 8, size=(E, N, K)).astype(np.int8)
    v2o = O.pack_v2o(q)
    w4 = lqp_to_int4pack(torch.from_numpy(v2o).to(device), expert_major=em)
    torch.cuda.synchronize()
    ref = O.pack_int4(np.ascontiguousarray(q.transpose(0, 2, 1)))   # [E, K, N/8]
    if not em:
        ref = np.ascontiguousarray(ref.transpose(1, 0, 2))
    assert np.array_equal(w4.cpu().numpy(), ref)


@pytest.mark.gpu
@pytest.mark.parametrize("E,N,G", [(3, 264, 4), (512, 1024, 16), (2, 5, 1)])
def test_lqp_scales(device, E, N, G):
    from qmoe.artifact import lqp_scales
    log(f"lqp_scales E={E} N={N} G={G}")
    s8 = rng.integers(-128, 128, size=(E, N, G)).astype(np.int8)
    base = (rng.standard_normal((E, N)) * 3e-3).astype(np.float16)
    base[0, 0] = np.float16(65504.0)          # largest fp16: rounds up in bf16
    base[-1, -1] = np.float16(6e-8)           # fp16 subnormal
    s8t, base_bf, sc = lqp_scales(torch.from_numpy(s8).to(device), torch.from_numpy(base).to(device))
    torch.cuda.synchronize()
    r_s8t = np.ascontiguousarray(s8.transpose(2, 0, 1))                       # tools/repack_w4a16.py:71
    r_base = O.f32_to_bf16_bits(base.astype(np.float32))                      # :72
    r_sc = O.compose_scales(r_s8t, r_base)                                    # fnx/engine.py:653-659
    assert np.array_equal(s8t.cpu().numpy(), r_s8t)
    assert np.array_equal(bits(base_bf), r_base)
    assert np.array_equal(bits(sc), r_sc)


@pytest.mark.gpu
def test_repack_load_decode(device, tmp_path):
    """LQP file -> repack on the GPU -> W4A16 -em file -> loader -> one-token
    decode, equal bit for bit to the decode on weights built by the oracle's
    conversion chain; the K-major file loads to the same words."""
    from qmoe import ExpW4, moe_decode
    from qmoe.artifact import exp_w4_from_lqp, load_layer_w4, repack_lqp_layer
    from parity import to_dev
    E, H, MI, gs, k = 64, 512, 256, 64, 8
    log(f"repack+load+decode E={E} H={H} MI={MI}")
    lay = lqp_layer(E, H, MI, gs, 9)
    src = tmp_path / "L00.safetensors"
    save_lqp(src, lay)
    (tmp_path / "w4-em").mkdir()
    (tmp_path / "w4").mkdir()
    repack_lqp_layer(src, tmp_path / "w4-em" / "L00.w4.safetensors", device, expert_major=True)
    repack_lqp_layer(src, tmp_path / "w4" / "L00.w4.safetensors", device, expert_major=False)
    em = load_layer_w4(tmp_path / "w4-em" / "L00.w4.safetensors", device)
    km = load_layer_w4(tmp_path / "w4" / "L00.w4.safetensors", device)
    ref = {}
    for proj, p in lay.items():
        w4, _, _, sc = O.lqp_to_em(p["v2o"], p["s8"], p["base"])
        ref[proj] = ExpW4.from_scales(to_dev(w4, device), to_dev(sc, device))
        got = em[f"mlp.experts.{proj}"]
        assert np.array_equal(got.w4.cpu().numpy(), w4)
        assert np.array_equal(bits(got._scales), sc)
        kg = km[f"mlp.experts.{proj}"]
        assert not kg.expert_major and np.array_equal(kg.w4.permute(1, 0, 2).cpu().numpy(), w4)
        direct = exp_w4_from_lqp(*(torch.from_numpy(p[n]).to(device) for n in ("v2o", "s8", "base")))
        assert np.array_equal(direct.w4.cpu().numpy(), w4) and np.array_equal(bits(direct._scales), sc)
    x = to_dev(O.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32)), device)
    lg = to_dev(O.f32_to_bf16_bits(rng.standard_normal((1, E)).astype(np.float32)), device)
    out_a = moe_decode(x, lg, em["mlp.experts.gate_up_proj"], em["mlp.experts.down_proj"], k)[0]
    out_b = moe_decode(x, lg, ref["gate_up_proj"], ref["down_proj"], k)[0]
    torch.cuda.synchronize()
    assert np.array_equal(bits(out_a), bits(out_b))
