"""W8A16 GEMM (the int8 form of npu_weight_quant_batchmatmul) and the DenseW8
container: stage-wise rounding exactness against the oracle."""
import numpy as np
import pytest
import torch

from gpu_util import bf16_normal, log
from oracle import qmoe_oracle as O
from parity import assert_in_interval, bits, to_dev

rng = np.random.default_rng(88)


def w8_case(M, K, N, gs, seed):
    r = np.random.default_rng(seed)
    x = bf16_normal((M, K), seed)
    q = r.integers(-128, 128, size=(K, N)).astype(np.int8)
    S = O.f32_to_bf16_bits(np.abs(r.standard_normal((K // gs, N))).astype(np.float32) * 0.003)
    return x, q, S


def check(y_bits, x, q, S, gs, what):
    ex, ab = O.w8a16_gemm_exact(x, q, S, gs)
    lo, hi = O.bf16_interval(ex, ab)
    assert_in_interval(y_bits, lo, hi, what)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 64, 300])
@pytest.mark.parametrize("K,N,gs", [(2560, 1024, 128), (2048, 4096, 128), (640, 2560, 64), (96, 48, 32),
                                    (4096, 160, 256), (64, 16, 32)])
def test_w8a16_gemm(device, M, K, N, gs):
    from qmoe import weight_quant_batchmatmul
    log(f"w8a16 M={M} K={K} N={N} gs={gs}")
    x, q, S = w8_case(M, K, N, gs, M * 7 + K + N)
    y = weight_quant_batchmatmul(to_dev(x, device), to_dev(q, device), to_dev(S, device), antiquant_group_size=gs)
    torch.cuda.synchronize()
    check(bits(y), x, q, S, gs, f"w8a16 M={M}")


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,N,gs", [(512, 2048, 8192, 128), (520, 1024, 6544, 64), (1000, 512, 4160, 128)])
def test_w8a16_gemm_wide_tiles(device, M, K, N, gs):
    """Grids of at least 256 128 x 128 tiles (the 8-wave tile), with partial
    row and column tiles."""
    from qmoe import weight_quant_batchmatmul
    log(f"w8a16 wide M={M} K={K} N={N} gs={gs}")
    x, q, S = w8_case(M, K, N, gs, M + 3 * K + N)
    y = weight_quant_batchmatmul(to_dev(x, device), to_dev(q, device), to_dev(S, device), antiquant_group_size=gs)
    torch.cuda.synchronize()
    check(bits(y), x, q, S, gs, f"w8a16 wide M={M} N={N}")


@pytest.mark.gpu
def test_w8a16_small_group_gemv(device):
    """gs = 8 (a 4-row run per thread stays in one group) on the GEMV path."""
    from qmoe import weight_quant_batchmatmul
    x, q, S = w8_case(2, 512, 256, 8, 5)
    y = weight_quant_batchmatmul(to_dev(x, device), to_dev(q, device), to_dev(S, device), antiquant_group_size=8)
    torch.cuda.synchronize()
    check(bits(y), x, q, S, 8, "w8a16 gs8")


@pytest.mark.gpu
def test_dense_w8_container(device):
    """DenseW8 (fnx/engine.py:297-384): padded K, 3-D input, chunks, merge."""
    from qmoe import DenseW8
    N, Kp, K, gs = 512, 2560 + 128, 2560, 128
    q = rng.integers(-128, 128, size=(N, Kp)).astype(np.int8)
    s = (np.abs(rng.standard_normal((N, Kp // gs))) * 0.004).astype(np.float16)
    d = DenseW8(torch.from_numpy(q).to(device), torch.from_numpy(s).to(device), K=K)
    assert (d.K, d.N, d.gs) == (K, N, gs)
    w8t, sc, _ = O.dense_w8_from_qs(q, s, K)
    assert np.array_equal(d.w8t.cpu().numpy(), w8t) and np.array_equal(bits(d.sc), sc)
    for M in (1, 4, 37):
        x = bf16_normal((M, 1, K), 90 + M)                                # [b, 1, H] as the layer passes it
        y = d(to_dev(x, device))
        torch.cuda.synchronize()
        assert tuple(y.shape) == (M, 1, N)
        check(bits(y).reshape(M, N), x.reshape(M, K), w8t, sc, gs, f"DenseW8 M={M}")
    # merge two projections that read the same x, then chunk along N: same words
    d2 = DenseW8(torch.from_numpy(q[:256]).to(device), torch.from_numpy(s[:256]).to(device), K=K)
    m = DenseW8.merge([d, d2])
    x = to_dev(bf16_normal((3, K), 95), device)
    ym = m(x)
    ya, yb = d(x), d2(x)
    m.make_chunks(320)
    yc = m(x)
    torch.cuda.synchronize()
    assert np.array_equal(bits(ym), np.concatenate([bits(ya), bits(yb)], axis=1))
    assert np.array_equal(bits(yc), bits(ym))
