"""Glue kernels: gather, weighted reduce, decode epilogue, shared merge, SwiGLU."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_normal, int4_words, log, scales
from oracle import qmoe_oracle as O
from parity import assert_bf16_equal, assert_equal_off_boundary, bits, to_dev


@pytest.mark.gpu
@pytest.mark.parametrize("K,G,N,E,ids", [(2560, 40, 1280, 512, [3, 17, 61, 200, 255, 256, 400, 401, 510, 511]),
                                         (640, 10, 2560, 512, [7, 343, 105, 212, 243, 254, 403, 168, 302, 67]),
                                         (2048, 16, 1024, 64, [5, 5, 0, 63])])
def test_expert_gather(device, K, G, N, E, ids):
    from qmoe import ExpW4
    from qmoe.expert_gather import gather
    log(f"gather K={K} N={N}")
    w = int4_words((E, K, N // 8), K)
    s = scales((E, G, N), K + 1)
    proj = ExpW4.from_scales(to_dev(w, device), to_dev(s, device))
    ow, os_ = gather(proj, torch.tensor(ids, dtype=torch.int64, device=device))
    torch.cuda.synchronize()
    rw, rs = O.expert_gather(w, s, np.array(ids))
    assert np.array_equal(ow.cpu().numpy(), rw)
    assert np.array_equal(bits(os_), rs)


@pytest.mark.gpu
@pytest.mark.parametrize("B,W,G", [(1, 2560, 10), (128, 2048, 10), (512, 3072, 10), (3, 100, 10), (4, 2048, 20),
                                   (64, 2560, 1)])
def test_weighted_reduce(device, B, W, G):
    """8-aligned widths with up to 16 groups take the vectorised kernel, the
    rest (W = 100, G = 20) the one-column-per-thread one; both bit-exact."""
    from qmoe.weighted_reduce import reduce
    log(f"weighted_reduce B={B} W={W} G={G}")
    vals = bf16_normal((B * G, W), B + W, 0.1)
    wts = O.f32_to_bf16_bits(np.random.default_rng(B).random((B, G)).astype(np.float32))
    out1 = reduce(to_dev(vals, device), to_dev(wts, device))
    perm = np.random.default_rng(W).permutation(B * G)
    inverse = np.empty_like(perm)
    inverse[perm] = np.arange(B * G)
    out2 = reduce(to_dev(vals[perm], device), to_dev(wts, device), inverse=to_dev(inverse.astype(np.int64), device))
    torch.cuda.synchronize()
    ref = O.weighted_reduce(vals, wts)
    assert_bf16_equal(out1, ref, "mode 1")
    assert_bf16_equal(out2, ref, "mode 2")


@pytest.mark.gpu
def test_weighted_reduce_cancellation_vectors(device):
    from qmoe.weighted_reduce import reduce
    log("weighted_reduce cancellation")
    v = np.zeros((10, 2560), dtype=np.float32)
    v[:4, 0] = [1e8, 1, -1e8, 1]
    v[:4, 1] = [1e8, -1e8, 1, 1]
    out = reduce(to_dev(O.f32_to_bf16_bits(v), device), torch.ones((1, 10), dtype=torch.bfloat16, device=device))
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    assert o[0, 0] == 1.0 and o[0, 1] == 2.0


@pytest.mark.gpu
@pytest.mark.parametrize("k,H,with_shared", [(10, 2560, True), (10, 2048, False), (4, 96, True)])
def test_moe_epilogue(device, k, H, with_shared):
    from qmoe.moe_epilogue import merge
    log(f"moe_epilogue k={k} H={H}")
    cart = bf16_normal((k, k * H), H, 3.0)
    w = O.f32_to_bf16_bits(np.random.default_rng(k).random((1, k)).astype(np.float32))
    sh = bf16_normal((1, H), H + 1) if with_shared else None
    g = bf16_normal((1, 1), H + 2) if with_shared else None
    out = merge(to_dev(cart, device), to_dev(w, device), to_dev(sh, device) if with_shared else None,
                to_dev(g, device) if with_shared else None)
    torch.cuda.synchronize()
    if with_shared:
        ref = O.moe_epilogue(cart, w, sh, g)
    else:
        diag = np.stack([cart[j, j * H:(j + 1) * H] for j in range(k)])
        ref = O.weighted_reduce(diag, w)
    if not with_shared:
        assert_bf16_equal(out, ref, "epilogue (no shared expert)")
        return
    # the sigmoid's exp() may round differently in fp32 on the two sides: the
    # output must be the oracle's for the gate's bf16 sigmoid, or for its
    # neighbour when the float64 sigmoid lies on a bf16 rounding boundary
    diag = np.stack([cart[j, j * H:(j + 1) * H] for j in range(k)])
    r = O.bf16_bits_to_f32(O.weighted_reduce(diag, w))
    got = bits(out)
    cands = [merge_with_sigmoid(r, sh, sg) for sg in sigmoid_candidates(g)]
    assert np.array_equal(got, ref) or (len(cands) == 2 and any(np.array_equal(got, c) for c in cands)), \
        "epilogue differs from the oracle and the sigmoid is not on a rounding boundary"


def sigmoid_candidates(g_bits):
    """bf16 sigmoid values admissible for the gate (two only on a boundary)."""
    gv = O.bf16_bits_to_f32(g_bits).astype(np.float64).reshape(-1)
    lo, hi = O.bf16_interval(1.0 / (1.0 + np.exp(-gv)))
    return [O.bf16_bits_to_f32(lo)] if np.all(lo == hi) else [O.bf16_bits_to_f32(lo), O.bf16_bits_to_f32(hi)]


def merge_with_sigmoid(r, sh_bits, sg):
    """bf16(r + bf16(sh * sg)) for bf16 values r, sh and a bf16 sigmoid sg (exact products in fp32)."""
    return O.f32_to_bf16_bits(r + O.round_bf16(O.bf16_bits_to_f32(sh_bits) * sg.reshape(-1, 1)))


@pytest.mark.gpu
@pytest.mark.parametrize("W,MI", [(2560, 768), (100, 100)])
def test_moe_merge_and_swiglu(device, W, MI):
    """8-aligned widths take the 16-byte kernels, the others the one-element ones."""
    from qmoe import swiglu
    from qmoe.post_ops import moe_merge
    log(f"moe_merge / swiglu W={W} MI={MI}")
    e = bf16_normal((3, W), 1)
    s = bf16_normal((3, W), 2)
    g = bf16_normal((3, 1), 3)
    out = moe_merge(to_dev(e, device), to_dev(s, device), to_dev(g, device))
    gu = bf16_normal((257, 2 * MI), 4, 4.0)
    act = swiglu(to_dev(gu, device))
    torch.cuda.synchronize()
    # merge: per row, the oracle's bits, or (sigmoid on a boundary) its neighbour's
    got = bits(out)
    ref = O.moe_merge(e, s, g)
    er = O.bf16_bits_to_f32(e)
    for t in range(3):
        if np.array_equal(got[t], ref[t]):
            continue
        cands = sigmoid_candidates(g[t])
        assert len(cands) == 2, f"moe_merge row {t} differs away from a sigmoid rounding boundary"
        assert any(np.array_equal(got[t], merge_with_sigmoid(er[t:t + 1], s[t:t + 1], c)[0]) for c in cands)
    # swiglu (fp32 npu form): bit-equal except where silu(g) * u sits on a rounding boundary
    gf = O.bf16_bits_to_f32(gu).astype(np.float64)
    mi = gu.shape[1] // 2
    exact = gf[:, :mi] / (1.0 + np.exp(-gf[:, :mi])) * gf[:, mi:]
    assert_equal_off_boundary(act, O.swiglu(gu), exact, "swiglu")
